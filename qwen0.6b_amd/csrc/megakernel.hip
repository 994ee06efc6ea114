// Qwen3-0.6B batch-1 decode engine for MI355X (gfx950): one cooperative,
// persistent kernel runs whole token steps (embedding, 28 layers, final norm,
// tied lm_head, argmax) and, in generate mode, feeds each argmax back as the
// next step's input without returning to the host.
//
// Design (from measurements on MI355X):
//  * one 512-thread workgroup per CU; workgroup w runs on XCD w % 8, and the
//    work partition (qwen_layout.h) keeps each kv head's QKV rows, attention
//    splits, softmax combine, o_proj and a 384-row slice of the MLP inside one
//    XCD. Per layer only two steps cross XCDs: the sums of the 8 per-XCD
//    o_proj and down partials into the residual stream (each workgroup reads
//    its 32 rows from the 8 XCDs);
//  * no grid barrier: every hand-off is an exchange buffer of 8-byte slots
//    carrying payload + step tag, written with device-scope stores and polled
//    with device-scope loads (one-way latency 0.3-0.5 us; a fence-based flag
//    costs 1-2 us more);
//  * waves 0-3 compute: each polls a quarter of a stage's input, the quarters
//    meet in LDS, and each wave computes a quarter of the stage's rows and
//    stores its own results. They hold no outstanding weight loads, so a poll
//    never waits behind a prefetch;
//  * waves 4-7 stream every stage's weights and K/V rows with LDS-DMA
//    (global_load_lds_dwordx4) into a 128 KB ring of 1 KB lines, up to 128
//    lines ahead of the compute waves; a compute wave reads its lines into
//    registers (and frees them) while it waits for its input, so only the
//    arithmetic follows the input's arrival. In the lm_head the loader waves
//    compute rows alongside the compute waves, and the last fifth of the
//    vocabulary is claimed at run time by groups of 8 workgroups (one per XCD);
//  * the residual stream stays fp32 inside the workgroup that owns its rows;
//    only the all-gathered copies are fp16;
//  * every wait is bounded by a wall-clock deadline; a missed deadline sets a
//    status word and all waves leave, so a broken exchange cannot hang the GPU.
//
// Reference behaviour followed: Tools/megakernel/megakernel.cu:763-920 (op
// order), 242-291 (QKV), 308-553 (q/k norm, RoPE, KV write, attention),
// 558-709 (o_proj, post-norm, SiLU*up, down), 893-919 (final norm),
// 1001-1144 (lm_head + argmax), 1150-1314 (launchers).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <type_traits>
#include <cstring>
#include <mutex>

#include "qwen_layout.h"
#include "qwen_megakernel.h"

using namespace ql;

typedef unsigned int u32;
typedef unsigned long long u64;
typedef u32 v4u __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr float RMS_EPS = 1e-6f;
constexpr u32 ST_TIMEOUT = 1u;
constexpr u32 ST_BAD_TOKEN = 2u;
// XCC id of the executing wave: s_getreg of hardware register 20 (XCC_ID), bits [3:0]
__device__ __forceinline__ u32 xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20); }
constexpr int DMA_DEPTH = 16;  // LDS-DMA lines a loader wave keeps in flight
// optional device timestamps (wall clock) per workgroup and stage of one token
constexpr int TRACE_EVENTS = 6;
enum TraceEvent : int {
  TR_POLL = 0,   // compute wave 0 starts waiting for the stage input
  TR_INPUT = 1,  // compute wave 0 has the stage input
  TR_SYNC = 2,   // attention: the wave's partial is in LDS (before the merge barrier);
                 // lm_head stage: compute wave 0 finished its lm_head rows
  TR_STORE = 3,  // compute wave 0 stored its results (and they were acknowledged)
  TR_LINES = 4,  // layer stages: compute wave 0 has the stage's ring lines;
                 // lm_head stage: compute wave 0 has the argmax partials of all workgroups
  TR_MERGE = 5,  // attention: compute wave 0 passed the barrier before the split merge;
                 // lm_head stage: loader wave 0 finished its lm_head rows
};
QL_HD int trace_stages(int L) { return NSTAGE * L + 1; }

struct KParams {
  const _Float16* embed;
  const LDGLayerWeight* layers;
  const _Float16* final_norm;
  const _Float16* lm_head;
  const _Float16* cos_t;
  const _Float16* sin_t;
  _Float16* k_cache;
  _Float16* v_cache;
  _Float16* hidden_out;    // [1024] fp16
  float* norm_out;         // [1024] fp32
  int* out_tokens;         // [num_steps]
  const int* forced;       // nullable [num_steps]
  float* logits_out;       // nullable [num_steps][VOCAB]
  float* hidden_steps;     // nullable [num_steps][HIDDEN]
  const _Float16* in_vec;  // MODE_LMHEAD / MODE_MLP input [1024]
  float* out_vec;          // MODE_MLP output [1024]
  u64* ws;                 // exchange slots
  u32* status;             // status word (device scope)
  u64 deadline;            // wall-clock ticks a single wait may take
  u64* trace;              // nullable [NWG][trace_stages(L)][TRACE_EVENTS]
  int trace_token;         // token index whose stages are traced
  int* out_count;          // nullable: steps run (the generation stops after eos)
  int eos;                 // stop after the first step whose argmax is this id (-1: never)
  int mode, num_layers, first_token, start_pos, num_steps, max_seq;
  float attn_scale;
  u32 epoch0;
  // the sampling build of the kernel: every next token is the argmax of logit / temperature +
  // Gumbel noise (seed, position) instead of the logit's (temperature sampling, on the device)
  float temperature;
  u64 seed;
  int sample;              // host side: launch the sampling build
  // the sampling builds with top_k >= 1: the token is drawn from the top-k (then top-p, when
  // top_p < 1) tokens of the step's logits instead of from all of them; top_k = VOCAB: top-p
  // alone. 1 <= top_k <= TOPK_MAX: the `sampled` build (draw_topk); larger: `dsampled`
  // (draw_dist); top_k = 0: `tsampled` (temperature alone)
  int top_k;
  float top_p;
};
constexpr int TOPK_MAX = 128;  // largest top_k of the `sampled` build

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): 10 rounds of two 32x32 -> 64 multiplies
// with the published multipliers and key increments; returns the first output word
__device__ __forceinline__ u32 philox_x0(u32 c0, u32 c1, u32 c2, u32 c3, u32 k0, u32 k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const u64 p0 = (u64)0xD2511F53u * c0, p1 = (u64)0xCD9E8D57u * c2;
    const u32 n0 = (u32)(p1 >> 32) ^ c1 ^ k0, n2 = (u32)(p0 >> 32) ^ c3 ^ k1;
    c0 = n0;
    c1 = (u32)p1;
    c2 = n2;
    c3 = (u32)p0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

// Gumbel(0, 1) noise of token j at `step` (the position of the step's input token) under `seed`:
// g = -log(-log(u)) with u = (top 23 bits of Philox of counter (j, step, 0, 0), key (seed low,
// seed high), + 0.5) / 2^23, every step exact in fp32, so u lies in [2^-24, 1 - 2^-24] (24 bits
// would round the largest value up to 1.0 and give g = +inf)
__device__ __forceinline__ float gumbel(u64 seed, u32 step, u32 j) {
  const u32 x = philox_x0(j, step, 0u, 0u, (u32)seed, (u32)(seed >> 32));
  const float u = ((float)(x >> 9) + 0.5f) * (1.0f / 8388608.0f);
  return -logf(-logf(u));
}

// order-preserving key: larger floats give larger keys; NaN gives 0 (below -inf)
__device__ __forceinline__ u32 fkey(float v) {
  if (v != v) return 0u;
  const u32 b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(u32 k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// unnormalised probability exp((l - M) / T) in units of 2^-40; 0 for NaN (M is the largest
// logit, so the value is at most 2^40 and a vocabulary's sum fits 64 bits)
__device__ __forceinline__ u64 mass(float l, float M, float T) {
  if (l != l) return 0;
  return (u64)(expf((l - M) / T) * 1099511627776.0f);
}

// (key << 32 | ~index): the larger of two is the larger key, then the lower index
__device__ __forceinline__ u64 pack_best(u32 key, int idx) { return ((u64)key << 32) | (u64)(0xffffffffu - (u32)idx); }
__device__ __forceinline__ int best_index(u64 b) { return (int)(0xffffffffu - (u32)b); }

// ------------------------------------------------------------------------------------
// device code: the production kernel, and a copy that records per-stage timestamps

namespace fast {
constexpr bool kTrace = false;
constexpr bool kSample = false;
constexpr bool kTopK = false;
constexpr bool kDist = false;
#include "decode_body.inc"
}  // namespace fast

namespace traced {
constexpr bool kTrace = true;
constexpr bool kSample = false;
constexpr bool kTopK = false;
constexpr bool kDist = false;
#include "decode_body.inc"
}  // namespace traced

namespace sampled {
constexpr bool kTrace = false;
constexpr bool kSample = true;
constexpr bool kTopK = true;
constexpr bool kDist = false;
#include "decode_body.inc"
}  // namespace sampled

// top_k > TOPK_MAX and top-p alone: the sampling build whose draw splits the selections over
// every workgroup's slice when the published entries cannot decide them (draw_dist)
namespace dsampled {
constexpr bool kTrace = false;
constexpr bool kSample = true;
constexpr bool kTopK = true;
constexpr bool kDist = true;
#include "decode_body.inc"
}  // namespace dsampled

// temperature alone: the sampling build without the top-k draw, whose code would otherwise
// share (and reshape) this kernel's register allocation
namespace tsampled {
constexpr bool kTrace = false;
constexpr bool kSample = true;
constexpr bool kTopK = false;
constexpr bool kDist = false;
#include "decode_body.inc"
}  // namespace tsampled

// the batched prefill kernel (namespace pf)
#include "prefill_body.inc"

// the token sampler (namespace smp)
#include "sample_body.inc"

// one workgroup per CU, as the decode kernel: each records the XCC it runs on
__global__ void __launch_bounds__(BLOCK, 1) qwen_placement_probe(u32* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// the prefill kernel's geometry (two 256-thread workgroups per CU): each records its XCC
__global__ void __launch_bounds__(pf::NT, pf::WG_PER_CU) qwen_placement_probe_pf(u32* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// zeroes n 8-byte words (a kernel, not hipMemsetAsync: callers may capture the stream)
__global__ void qwen_zero_words(u64* p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0;
}

// Exchange workspace of qwen_generate_nosync_noalloc: the same layout as the workspace the
// other entry points allocate (slots, status line, lm_head pool counters), as module memory,
// one copy per device. Host code never uses this name as an address: it uses the pointer
// hipGetSymbolAddress returns for the current device (DeviceState::fixed).
static_assert(WORKSPACE_BYTES % 256 == 0, "whole 256-byte lines");
static __device__ __align__(256) unsigned char scratch[WORKSPACE_BYTES];

// ------------------------------------------------------------------------------------
// host side

namespace {

constexpr int MAX_DEVICES = 16;
constexpr u64 DEFAULT_WAIT_US = 500000;

// one exchange workspace (WORKSPACE_BYTES) and the token epoch its tags continue from
struct Workspace {
  u64* ws = nullptr;
  u32* status = nullptr;
  u32 epoch = 1;
};

struct DeviceState {
  bool init = false;
  int err = QWEN_OK;
  Workspace heap;                 // hipMalloc'd on first use by the allocating entry points
  Workspace fixed;                // the `scratch` array of this device (no allocation)
  LDGLayerWeight* tab = nullptr;  // the isolated MLP block's one-layer pointer table
  char* pf = nullptr;             // prefill activations (PF_BYTES), on first use
  char* smp = nullptr;            // the sampler's work area (SMP_BYTES), allocated on first use
  u32 smp_parity = 0;             // sampler launches so far (selects the work area copy)
  u64 clk_khz = 100000;
  u64 deadline = 0;
  u64* trace = nullptr;
  long long trace_elems = 0;
  int trace_token = -1;
};

std::mutex g_mu;
DeviceState g_dev[MAX_DEVICES];
// What the library allocates (workspaces, the MLP block's pointer table, the prefill and
// sampler buffers) is held until the process ends and released with it; no exit handler
// calls into the HIP runtime.

int zero_words(void* p, long bytes, hipStream_t s) {
  hipLaunchKernelGGL(qwen_zero_words, dim3(NWG), dim3(256), 0, s, (u64*)p, bytes / 8);
  return hipGetLastError() == hipSuccess ? QWEN_OK : QWEN_ERR_LAUNCH;
}

// Every workgroup w of the decode launch (256 x 512) and of the prefill launch (512 x 256) must
// run on XCD w % 8: the decode's work partition and XCD-local exchange stores, and the prefill's
// per-XCD barrier (one L2 write-back and invalidate per XCD) rely on it. Checked once per device
// and geometry with a probe launch that writes into `buf` (n words).
int check_placement(const void* probe, int n, int threads, u32* buf, hipStream_t s) {
  void* args[] = {&buf};
  if (hipLaunchCooperativeKernel(probe, dim3(n), dim3(threads), args, 0, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return QWEN_ERR_LAUNCH;
  static u32 xcc[2 * NWG];
  if (n > 2 * NWG || hipMemcpy(xcc, buf, sizeof(u32) * n, hipMemcpyDeviceToHost) != hipSuccess)
    return QWEN_ERR_LAUNCH;
  for (int w = 0; w < n; ++w)
    if ((int)(xcc[w] & 15) != xcd_of(w)) {
      fprintf(stderr, "qwen_megakernel: workgroup %d of %d runs on XCC %u, the kernel needs XCC %d\n", w, n,
              xcc[w] & 15, xcd_of(w));
      return QWEN_ERR_DEVICE;
    }
  return QWEN_OK;
}

// Device checks and the fixed workspace, once per device; allocates nothing. (Caller holds g_mu.)
int device_state(DeviceState** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return QWEN_ERR_DEVICE;
  DeviceState& st = g_dev[dev];
  if (!st.init) {
    st.init = true;
    st.err = QWEN_ERR_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return st.err;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || prop.multiProcessorCount != NWG || !prop.cooperativeLaunch) {
      fprintf(stderr, "qwen_megakernel: needs a 256-CU gfx950 device with cooperative launch (got %s, %d CUs)\n",
              prop.gcnArchName, prop.multiProcessorCount);
      return st.err;
    }
    // every build of the decode kernel must fit one workgroup per CU
    const void* builds[] = {(const void*)fast::qwen_decode_kernel, (const void*)traced::qwen_decode_kernel,
                            (const void*)sampled::qwen_decode_kernel, (const void*)tsampled::qwen_decode_kernel};
    for (const void* k : builds) {
      int occ = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, BLOCK, 0) != hipSuccess || occ < 1) return st.err;
    }
    int clk_khz = 0;
    if (hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || clk_khz <= 0)
      clk_khz = 100000;
    st.clk_khz = (u64)clk_khz;
    st.deadline = st.clk_khz * DEFAULT_WAIT_US / 1000;  // 0.5 s per single wait
    // this device's copy of `scratch`: its address, never the host-side name
    void* fixed = nullptr;
    if (hipGetSymbolAddress(&fixed, HIP_SYMBOL(scratch)) != hipSuccess || fixed == nullptr) {
      st.err = QWEN_ERR_LAUNCH;
      return st.err;
    }
    st.err = check_placement((const void*)qwen_placement_probe, NWG, BLOCK, (u32*)fixed, nullptr);
    if (st.err != QWEN_OK) return st.err;
    if (zero_words(fixed, WORKSPACE_BYTES, nullptr) != QWEN_OK || hipDeviceSynchronize() != hipSuccess) {
      st.err = QWEN_ERR_LAUNCH;
      return st.err;
    }
    st.fixed.ws = (u64*)fixed;
    st.fixed.status = (u32*)((char*)fixed + TOTAL_SLOTS * 8);
    st.err = QWEN_OK;
  }
  if (st.err != QWEN_OK) return st.err;
  *out = &st;
  return QWEN_OK;
}

// The allocating entry points' workspace, on first use. (Caller holds g_mu.)
int heap_workspace(DeviceState* st) {
  if (st->heap.ws) return QWEN_OK;
  void* p = nullptr;
  if (hipMalloc(&p, WORKSPACE_BYTES) != hipSuccess) return QWEN_ERR_LAUNCH;
  if (hipMemset(p, 0, WORKSPACE_BYTES) != hipSuccess) {
    (void)hipFree(p);
    return QWEN_ERR_LAUNCH;
  }
  st->heap.ws = (u64*)p;
  st->heap.status = (u32*)((char*)p + TOTAL_SLOTS * 8);
  return QWEN_OK;
}

// launches the decode kernel on the heap workspace, or (fixed = true) on the device's
// `scratch` array, in which case nothing is allocated
int launch(KParams& P, hipStream_t stream, bool fixed = false) {
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  if (!fixed && (rc = heap_workspace(st)) != QWEN_OK) return rc;
  Workspace& w = fixed ? st->fixed : st->heap;
  // a trace buffer must hold every stage of every workgroup of this launch's layers
  if (st->trace && (long long)NWG * trace_stages(P.num_layers) * TRACE_EVENTS > st->trace_elems) return QWEN_ERR_ARG;
  // the traced build is the greedy kernel: a sampled launch while tracing would return argmax ids
  if (st->trace && P.sample) return QWEN_ERR_ARG;
  P.ws = w.ws;
  P.status = w.status;
  P.deadline = st->deadline;
  P.trace = st->trace;
  P.trace_token = st->trace_token;
  P.epoch0 = w.epoch;
  // epochs are 24-bit in the tag; wrap back to 1 (never 0: a zeroed slot is never "ready")
  u64 next = (u64)w.epoch + (u64)P.num_steps + 1;
  if (next >= (1u << 24)) {
    if (zero_words(w.ws, TOTAL_SLOTS * 8, stream) != QWEN_OK) return QWEN_ERR_LAUNCH;
    P.epoch0 = 1;
    next = 1 + (u64)P.num_steps + 1;
  }
  w.epoch = (u32)next;
  void* args[] = {&P};
  const void* kernel = P.trace    ? (const void*)traced::qwen_decode_kernel
                       : P.sample ? (P.top_k > TOPK_MAX ? (const void*)dsampled::qwen_decode_kernel
                                    : P.top_k > 0      ? (const void*)sampled::qwen_decode_kernel
                                                       : (const void*)tsampled::qwen_decode_kernel)
                                  : (const void*)fast::qwen_decode_kernel;
  if (hipLaunchCooperativeKernel(kernel, dim3(NWG), dim3(BLOCK), args, 0, stream) != hipSuccess)
    return QWEN_ERR_LAUNCH;
  return QWEN_OK;
}

// prefill activations for up to MAX_SEQ_LIMIT positions: residual X fp32 [n, 1024], q and the
// attention output fp16 [n, 2048] each, SiLU * up fp16 [n, 3072], the next RMSNorm's gained input
// fp16 [n, 1024] and its block sums of squares fp32 [n, 32], then the barrier counters and
// the split attention items' arrival counters (zeroed before every launch), the timestamps and
// the split items' partial results
constexpr long PF_X = 0;
constexpr long PF_Q = PF_X + (long)MAX_SEQ_LIMIT * HIDDEN * 4;
constexpr long PF_AO = PF_Q + (long)MAX_SEQ_LIMIT * QSZ * 2;
constexpr long PF_IM = PF_AO + (long)MAX_SEQ_LIMIT * QSZ * 2;
constexpr long PF_XN = PF_IM + (long)MAX_SEQ_LIMIT * INTER * 2;
constexpr long PF_SSQ = PF_XN + (long)MAX_SEQ_LIMIT * HIDDEN * 2;
constexpr long PF_BAR = PF_SSQ + (long)MAX_SEQ_LIMIT * 32 * 4;
constexpr int PF_NTS = 1 + 1 + 5 * MAX_LAYERS;  // launch start, then every grid barrier
constexpr long PF_BAR_LINES = 4096;              // barrier words: 8 XCDs x 64 arrivals, then 8 leaders
constexpr long PF_ACNT = PF_BAR + PF_BAR_LINES;
constexpr long PF_BAR_BYTES = PF_BAR_LINES + 4L * pf::MAX_QB * NKV;
constexpr long PF_TS = PF_BAR + PF_BAR_BYTES;
constexpr long PF_PART = (PF_TS + 8L * ((PF_NTS + 31) / 32 * 32) + 255) / 256 * 256;
constexpr long PF_BYTES = PF_PART + 4L * pf::MAX_PSLOTS * NKV * pf::PART_FLOATS;
static_assert(PF_BAR_BYTES % 4 == 0 && PF_PART % 256 == 0, "prefill workspace alignment");
static_assert(4L * (64 + 1) * NXCD <= PF_BAR_LINES, "the barrier words fit their lines");

// The attention work of a prefill of n positions from position start: query block b (positions
// start + 32 b ..) reads key blocks 0 .. nkb(b) - 1 (64 keys each, causal), in chunks of
// pf::KCHUNK key blocks; a block with more than one chunk is split into units (the kernel merges their partial
// results). Units are sorted longest first (ties: later query block first, then chunk order),
// the order in which the kernel deals them out.
static int prefill_units(int n, int start, pf::PParams& P) {
  const int nqb = (n + pf::QR - 1) / pf::QR;
  if (nqb > pf::MAX_QB) return QWEN_ERR_ARG;
  struct U {
    int cost, b, c, s;
  } u[pf::MAX_UNITS];
  int nu = 0, slot = 0;
  for (int b = 0; b < nqb; ++b) {
    const int qmax = (pf::QR * b + pf::QR < n ? pf::QR * b + pf::QR : n) - 1 + start;
    const int nkb = qmax / pf::QB + 1;
    const int sb = (nkb + pf::KCHUNK - 1) / pf::KCHUNK;
    if (sb > pf::MAX_CHUNKS || nu + sb > pf::MAX_UNITS) return QWEN_ERR_ARG;
    P.pslot[b] = (unsigned char)(sb > 1 ? slot : 0);
    if (sb > 1) slot += sb;
    for (int c = 0; c < sb; ++c) {
      const int left = nkb - pf::KCHUNK * c;
      u[nu++] = {left < pf::KCHUNK ? left : pf::KCHUNK, b, c, sb};
    }
  }
  if (slot > pf::MAX_PSLOTS) return QWEN_ERR_ARG;
  std::sort(u, u + nu, [](const U& x, const U& y) {
    if (x.cost != y.cost) return x.cost > y.cost;
    if (x.b != y.b) return x.b > y.b;
    return x.c < y.c;
  });
  for (int i = 0; i < nu; ++i) P.unit[i] = (unsigned short)(u[i].b | u[i].c << 6 | (u[i].s - 1) << 8);
  P.nunits = nu;
  return QWEN_OK;
}

// sampler buffer: the sampler's work area (two copies, chosen by launch parity)
constexpr long SMP_WORK = 0;
constexpr long SMP_BYTES = (smp::WORK_BYTES + 255) / 256 * 256;

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// temperature, top_k and top_p as the sampler reads them (NaN refused)
bool sample_args_ok(float temperature, int top_k, float top_p) {
  return temperature == temperature && top_k >= 0 && top_p == top_p;
}

// the decode kernel's top_k for a draw with these arguments (checked by sample_args_ok):
// temperature <= 0 is the argmax (1); no top-k (0 or >= VOCAB) is VOCAB with top_p < 1 (top-p
// alone) and 0 without (temperature alone)
int device_top_k(float temperature, int top_k, float top_p) {
  if (!(temperature > 0.f)) return 1;
  if (top_k == 0 || top_k >= VOCAB) return top_p < 1.f ? VOCAB : 0;
  return top_k;
}

// the device's sampler buffer (allocated and cleared on first use); caller holds g_mu
int sampler_buffer(DeviceState* st, hipStream_t stream) {
  if (st->smp) return QWEN_OK;
  int rc = heap_workspace(st);  // the status word the sampler reports to
  if (rc != QWEN_OK) return rc;
  void* p = nullptr;
  if (hipMalloc(&p, SMP_BYTES) != hipSuccess) return QWEN_ERR_LAUNCH;
  if (zero_words(p, SMP_BYTES, stream) != QWEN_OK) {
    (void)hipFree(p);
    return QWEN_ERR_LAUNCH;
  }
  st->smp = (char*)p;
  return QWEN_OK;
}

// one sampler launch on the device's work area; caller holds g_mu
int launch_sampler(DeviceState* st, smp::SParams& S, hipStream_t stream) {
  S.work = (u64*)(st->smp + SMP_WORK);
  S.parity = st->smp_parity++;
  S.status = st->heap.status;
  S.deadline = st->deadline;
  void* args[] = {&S};
  if (hipLaunchCooperativeKernel((const void*)smp::qwen_sample_kernel, dim3(smp::NB), dim3(smp::NT), args, 0,
                                 stream) != hipSuccess)
    return QWEN_ERR_LAUNCH;
  return QWEN_OK;
}

int fill_decode(KParams& P, const void* embed, const LDGLayerWeight* lw, const void* fnorm, const void* lm_head,
                const void* cos_t, const void* sin_t, void* kc, void* vc, void* hidden, void* norm_out,
                int num_layers, int start, int steps, int max_seq, float scale) {
  if (!embed || !lw || !fnorm || !lm_head || !cos_t || !sin_t || !kc || !vc || !hidden || !norm_out) return QWEN_ERR_ARG;
  if (!aligned16(lw) || !aligned16(embed) || !aligned16(lm_head) || !aligned16(kc) || !aligned16(vc) ||
      !aligned16(cos_t) || !aligned16(sin_t) || !aligned16(hidden) || !aligned16(norm_out) || !aligned16(fnorm))
    return QWEN_ERR_ARG;
  // max_seq must keep every ring line of 4 positions inside the cache
  if (num_layers < 1 || num_layers > MAX_LAYERS || steps < 1 || start < 0 || max_seq < 4 || (max_seq & 3) != 0 ||
      (long)start + steps > (long)max_seq || max_seq > MAX_SEQ_LIMIT)
    return QWEN_ERR_ARG;
  memset(&P, 0, sizeof(P));
  P.eos = -1;
  P.embed = (const _Float16*)embed;
  P.layers = lw;
  P.final_norm = (const _Float16*)fnorm;
  P.lm_head = (const _Float16*)lm_head;
  P.cos_t = (const _Float16*)cos_t;
  P.sin_t = (const _Float16*)sin_t;
  P.k_cache = (_Float16*)kc;
  P.v_cache = (_Float16*)vc;
  P.hidden_out = (_Float16*)hidden;
  P.norm_out = (float*)norm_out;
  P.mode = MODE_DECODE;
  P.num_layers = num_layers;
  P.start_pos = start;
  P.num_steps = steps;
  P.max_seq = max_seq;
  P.attn_scale = scale;
  return QWEN_OK;
}

}  // namespace

extern "C" int launch_ldg_decode_direct(int input_token_id, int* output_token_id, const void* embed_weight,
                                        const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                        const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                        void* k_cache, void* v_cache, void* hidden_buffer, void*, void*, void*,
                                        void*, void*, void*, void*, void* g_normalized, void*, void*,
                                        int num_layers, int position, int max_seq_len, float attn_scale,
                                        hipStream_t stream) {
  KParams P;
  int rc = fill_decode(P, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table,
                       k_cache, v_cache, hidden_buffer, g_normalized, num_layers, position, 1, max_seq_len,
                       attn_scale);
  if (rc != QWEN_OK) return rc;
  if (!output_token_id || input_token_id < 0 || input_token_id >= VOCAB) return QWEN_ERR_ARG;
  P.first_token = input_token_id;
  P.out_tokens = output_token_id;
  return launch(P, stream);
}

extern "C" int launch_ldg_decode_persistent(int input_token_id, int* output_token_id, const void* embed_weight,
                                            const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                            const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                            void* k_cache, void* v_cache, void* hidden_buffer, void* a, void* b,
                                            void* c, void* d, void* e, void* f, void* g, void* g_normalized, void* h,
                                            void* i, int num_layers, int position, int cache_len, int max_seq_len,
                                            float attn_scale, hipStream_t stream) {
  (void)cache_len;  // unused by the reference too: its kernel reads the position (megakernel.cu:1211-1230)
  return launch_ldg_decode_direct(input_token_id, output_token_id, embed_weight, layer_weights, final_norm_weight,
                                  lm_head_weight, cos_table, sin_table, k_cache, v_cache, hidden_buffer, a, b, c, d,
                                  e, f, g, g_normalized, h, i, num_layers, position, max_seq_len, attn_scale, stream);
}

extern "C" int qwen_generate_ex(int first_token_id, int num_steps, const int* forced_tokens, const void* embed_weight,
                                const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                void* k_cache, void* v_cache, void* hidden_buffer, void* g_normalized,
                                int* output_log, float* logits_out, float* hidden_steps, int num_layers,
                                int start_position, int max_seq_len, float attn_scale, hipStream_t stream) {
  KParams P;
  int rc = fill_decode(P, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table,
                       k_cache, v_cache, hidden_buffer, g_normalized, num_layers, start_position, num_steps,
                       max_seq_len, attn_scale);
  if (rc != QWEN_OK) return rc;
  if (!output_log || first_token_id < 0 || first_token_id >= VOCAB) return QWEN_ERR_ARG;
  if ((logits_out && !aligned16(logits_out)) || (hidden_steps && !aligned16(hidden_steps))) return QWEN_ERR_ARG;
  P.first_token = first_token_id;
  P.out_tokens = output_log;
  P.forced = forced_tokens;
  P.logits_out = logits_out;
  P.hidden_steps = hidden_steps;
  return launch(P, stream);
}

extern "C" int qwen_generate_until(int first_token_id, int num_steps, int eos_token_id, const void* embed_weight,
                                   const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                   const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                   void* k_cache, void* v_cache, void* hidden_buffer, void* g_normalized,
                                   int* output_log, int* out_count, int num_layers, int start_position,
                                   int max_seq_len, float attn_scale, hipStream_t stream) {
  KParams P;
  int rc = fill_decode(P, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table,
                       k_cache, v_cache, hidden_buffer, g_normalized, num_layers, start_position, num_steps,
                       max_seq_len, attn_scale);
  if (rc != QWEN_OK) return rc;
  if (!output_log || !out_count || first_token_id < 0 || first_token_id >= VOCAB || eos_token_id < 0 ||
      eos_token_id >= VOCAB)
    return QWEN_ERR_ARG;
  P.first_token = first_token_id;
  P.out_tokens = output_log;
  P.out_count = out_count;
  P.eos = eos_token_id;
  return launch(P, stream);
}

extern "C" int launch_ldg_generate_nosync(int first_token_id, int num_steps, const void* embed_weight,
                                          const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                          const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                          void* k_cache, void* v_cache, void* hidden_buffer, void*, void*, void*,
                                          void*, void*, void*, void*, void* g_normalized, void*, void*,
                                          int* output_log, int num_layers, int start_position, int max_seq_len,
                                          float attn_scale, hipStream_t stream) {
  return qwen_generate_ex(first_token_id, num_steps, nullptr, embed_weight, layer_weights, final_norm_weight,
                          lm_head_weight, cos_table, sin_table, k_cache, v_cache, hidden_buffer, g_normalized,
                          output_log, nullptr, nullptr, num_layers, start_position, max_seq_len, attn_scale, stream);
}

// launch_ldg_generate_nosync on the device's fixed `scratch` workspace: no allocation in this
// call or in its first-use set-up on a device. The workspace need does not depend on the
// arguments; their limits are those of launch_ldg_generate_nosync (QWEN_ERR_ARG beyond them,
// and on a stream that is being captured).
extern "C" int qwen_generate_nosync_noalloc(int first_token_id, int num_steps, const void* embed_weight,
                                            const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                            const void* lm_head_weight, const void* cos_table,
                                            const void* sin_table, void* k_cache, void* v_cache,
                                            void* hidden_buffer, void*, void*, void*, void*, void*, void*, void*,
                                            void* g_normalized, void*, void*, int* output_log, int num_layers,
                                            int start_position, int max_seq_len, float attn_scale,
                                            hipStream_t stream) {
  KParams P;
  int rc = fill_decode(P, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table,
                       k_cache, v_cache, hidden_buffer, g_normalized, num_layers, start_position, num_steps,
                       max_seq_len, attn_scale);
  if (rc != QWEN_OK) return rc;
  if (!output_log || first_token_id < 0 || first_token_id >= VOCAB) return QWEN_ERR_ARG;
  // Not for stream capture: the tags' token epochs are kernel arguments, so a replayed graph
  // would reuse them against slots that already carry them, and a device's first call
  // synchronises with the host (placement probe).
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return QWEN_ERR_ARG;
  P.first_token = first_token_id;
  P.out_tokens = output_log;
  return launch(P, stream, /*fixed=*/true);
}

extern "C" int qwen_prefill(const int* ids, int n, const void* embed_weight, const LDGLayerWeight* layer_weights,
                            const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                            void* hidden_buffer, int num_layers, int start_position, int max_seq_len,
                            float attn_scale, hipStream_t stream) {
  if (!ids || !embed_weight || !layer_weights || !cos_table || !sin_table || !k_cache || !v_cache || !hidden_buffer)
    return QWEN_ERR_ARG;
  if (!aligned16(embed_weight) || !aligned16(layer_weights) || !aligned16(cos_table) || !aligned16(sin_table) ||
      !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(hidden_buffer))
    return QWEN_ERR_ARG;
  if (n < 1 || num_layers < 1 || num_layers > MAX_LAYERS || start_position < 0 || max_seq_len < 4 ||
      (max_seq_len & 3) != 0 || max_seq_len > MAX_SEQ_LIMIT || (long)start_position + n > (long)max_seq_len)
    return QWEN_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  if ((rc = heap_workspace(st)) != QWEN_OK) return rc;
  if (!st->pf) {
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)pf::qwen_prefill_kernel, pf::NT, 0) !=
            hipSuccess || occ < pf::WG_PER_CU)
      return QWEN_ERR_DEVICE;
    void* p = nullptr;
    if (hipMalloc(&p, PF_BYTES) != hipSuccess) return QWEN_ERR_LAUNCH;
    if ((rc = check_placement((const void*)qwen_placement_probe_pf, pf::NWG_PF, pf::NT, (u32*)p, stream)) != QWEN_OK) {
      (void)hipFree(p);
      return rc;
    }
    st->pf = (char*)p;
  }
  pf::PParams P;
  memset(&P, 0, sizeof(P));
  P.ids = ids;
  P.embed = (const _Float16*)embed_weight;
  P.layers = layer_weights;
  P.cos_t = (const _Float16*)cos_table;
  P.sin_t = (const _Float16*)sin_table;
  P.kc = (_Float16*)k_cache;
  P.vc = (_Float16*)v_cache;
  P.hidden_out = (_Float16*)hidden_buffer;
  P.X = (float*)(st->pf + PF_X);
  P.Q = (_Float16*)(st->pf + PF_Q);
  P.AO = (_Float16*)(st->pf + PF_AO);
  P.IM = (_Float16*)(st->pf + PF_IM);
  P.XN = (_Float16*)(st->pf + PF_XN);
  P.SSQ = (float*)(st->pf + PF_SSQ);
  P.bar = (u32*)(st->pf + PF_BAR);
  P.acnt = (u32*)(st->pf + PF_ACNT);
  P.ts = (u64*)(st->pf + PF_TS);
  P.part = (float*)(st->pf + PF_PART);
  P.status = st->heap.status;
  P.deadline = st->deadline;
  P.n = n;
  P.start = start_position;
  P.num_layers = num_layers;
  P.max_seq = max_seq_len;
  P.attn_scale = attn_scale;
  if ((rc = prefill_units(n, start_position, P)) != QWEN_OK) return rc;
  if (zero_words(P.bar, PF_BAR_BYTES, stream) != QWEN_OK) return QWEN_ERR_LAUNCH;
  void* args[] = {&P};
  if (hipLaunchCooperativeKernel((const void*)pf::qwen_prefill_kernel, dim3(pf::NWG_PF), dim3(pf::NT), args, 0, stream) !=
      hipSuccess)
    return QWEN_ERR_LAUNCH;
  return QWEN_OK;
}

extern "C" int qwen_prefill_timestamps(unsigned long long* out, int max_entries) {
  if (!out || max_entries < 1) return QWEN_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  const int n = max_entries < PF_NTS ? max_entries : PF_NTS;
  if (!st->pf) {
    memset(out, 0, sizeof(unsigned long long) * n);
    return QWEN_OK;
  }
  if (hipDeviceSynchronize() != hipSuccess) return QWEN_ERR_LAUNCH;
  if (hipMemcpy(out, st->pf + PF_TS, sizeof(unsigned long long) * n, hipMemcpyDeviceToHost) != hipSuccess)
    return QWEN_ERR_LAUNCH;
  return QWEN_OK;
}

extern "C" int qwen_sample(const float* logits, int n, float temperature, int top_k, float top_p,
                           unsigned long long seed, unsigned int step, int* out_token, hipStream_t stream) {
  if (!logits || !out_token || n < 1 || n > smp::MAX_N || !sample_args_ok(temperature, top_k, top_p))
    return QWEN_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK || (rc = sampler_buffer(st, stream)) != QWEN_OK) return rc;
  smp::SParams S;
  memset(&S, 0, sizeof(S));
  S.logits = logits;
  S.n = n;
  S.temperature = temperature;
  S.top_k = top_k;
  S.top_p = top_p;
  S.seed = seed;
  S.step = step;
  S.out_token = out_token;
  return launch_sampler(st, S, stream);
}

extern "C" int qwen_generate_sampled(int first_token_id, int num_steps, int eos_token_id, const void* embed_weight,
                                     const LDGLayerWeight* layer_weights, const void* final_norm_weight,
                                     const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                     void* k_cache, void* v_cache, void* hidden_buffer, void* g_normalized,
                                     int* output_log, int* out_count, int num_layers, int start_position,
                                     int max_seq_len, float attn_scale, float temperature, int top_k, float top_p,
                                     unsigned long long seed, hipStream_t stream) {
  KParams P;
  // the whole range is checked before anything is launched
  int rc = fill_decode(P, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table,
                       k_cache, v_cache, hidden_buffer, g_normalized, num_layers, start_position, num_steps,
                       max_seq_len, attn_scale);
  if (rc != QWEN_OK) return rc;
  if (!output_log || first_token_id < 0 || first_token_id >= VOCAB || eos_token_id < -1 || eos_token_id >= VOCAB ||
      !sample_args_ok(temperature, top_k, top_p))
    return QWEN_ERR_ARG;
  // one launch of num_steps steps, every token drawn inside the decode kernel (eos checked on the
  // device as in qwen_generate_until): temperature <= 0 is the argmax (top_k 1); temperature
  // alone runs the `tsampled` build, top-k (then top-p) and top-p alone the `sampled` /
  // `dsampled` builds
  P.first_token = first_token_id;
  P.out_tokens = output_log;
  P.out_count = out_count;
  P.eos = eos_token_id;
  P.temperature = temperature;
  P.seed = seed;
  P.sample = 1;
  P.top_k = device_top_k(temperature, top_k, top_p);
  P.top_p = top_p;
  return launch(P, stream);
}

extern "C" int qwen_lm_head_argmax(const void* hidden_f16, const void* weight, int* out_token, float* logits_out,
                                   hipStream_t stream) {
  if (!hidden_f16 || !weight || !out_token || !aligned16(hidden_f16) || !aligned16(weight)) return QWEN_ERR_ARG;
  if (logits_out && !aligned16(logits_out)) return QWEN_ERR_ARG;
  KParams P;
  memset(&P, 0, sizeof(P));
  P.eos = -1;
  P.lm_head = (const _Float16*)weight;
  P.in_vec = (const _Float16*)hidden_f16;
  P.out_tokens = out_token;
  P.logits_out = logits_out;
  P.mode = MODE_LMHEAD;
  P.num_layers = 1;
  P.num_steps = 1;
  P.max_seq = MAX_SEQ_LIMIT;
  return launch(P, stream);
}

extern "C" int qwen_lm_head_sample(const void* hidden_f16, const void* weight, float temperature, int top_k,
                                   float top_p, unsigned long long seed, int position, int* out_token,
                                   float* logits_out, hipStream_t stream) {
  if (!hidden_f16 || !weight || !out_token || !aligned16(hidden_f16) || !aligned16(weight)) return QWEN_ERR_ARG;
  if (logits_out && !aligned16(logits_out)) return QWEN_ERR_ARG;
  if (!(temperature > 0.f) || !sample_args_ok(temperature, top_k, top_p) || position < 0) return QWEN_ERR_ARG;
  KParams P;
  memset(&P, 0, sizeof(P));
  P.eos = -1;
  P.lm_head = (const _Float16*)weight;
  P.in_vec = (const _Float16*)hidden_f16;
  P.out_tokens = out_token;
  P.logits_out = logits_out;
  P.mode = MODE_LMHEAD;
  P.num_layers = 1;
  P.num_steps = 1;
  P.start_pos = position;
  P.max_seq = MAX_SEQ_LIMIT;
  P.temperature = temperature;
  P.seed = seed;
  P.sample = 1;
  P.top_k = device_top_k(temperature, top_k, top_p);
  P.top_p = top_p;
  return launch(P, stream);
}

extern "C" int qwen_mlp_block(const void* x_f16, const void* post_norm_weight, const void* gate_weight,
                              const void* up_weight, const void* down_weight, float* y_out, hipStream_t stream) {
  if (!x_f16 || !post_norm_weight || !gate_weight || !up_weight || !down_weight || !y_out) return QWEN_ERR_ARG;
  if (!aligned16(x_f16) || !aligned16(post_norm_weight) || !aligned16(gate_weight) || !aligned16(up_weight) ||
      !aligned16(down_weight) || !aligned16(y_out))
    return QWEN_ERR_ARG;
  // the kernel reads the layer pointer table from device memory
  LDGLayerWeight h;
  memset(&h, 0, sizeof(h));
  h.post_attn_layernorm_weight = post_norm_weight;
  h.gate_proj_weight = gate_weight;
  h.up_proj_weight = up_weight;
  h.down_proj_weight = down_weight;
  LDGLayerWeight* tab = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc != QWEN_OK) return rc;
    if (!st->tab && hipMalloc(&st->tab, sizeof(LDGLayerWeight)) != hipSuccess) return QWEN_ERR_LAUNCH;
    tab = st->tab;
  }
  if (hipMemcpyAsync(tab, &h, sizeof(h), hipMemcpyHostToDevice, stream) != hipSuccess) return QWEN_ERR_LAUNCH;
  if (hipStreamSynchronize(stream) != hipSuccess) return QWEN_ERR_LAUNCH;
  KParams P;
  memset(&P, 0, sizeof(P));
  P.eos = -1;
  P.layers = tab;
  P.in_vec = (const _Float16*)x_f16;
  P.out_vec = y_out;
  P.mode = MODE_MLP;
  P.num_layers = 1;
  P.num_steps = 1;
  P.max_seq = MAX_SEQ_LIMIT;
  return launch(P, stream);
}

namespace {

// status word of one workspace: 0, or the error it reports (the workspace is then cleared
// and its epochs restart)
int take_status(Workspace& w) {
  if (!w.ws) return QWEN_OK;
  u32 s = 0;
  if (hipMemcpy(&s, w.status, sizeof(s), hipMemcpyDeviceToHost) != hipSuccess) return QWEN_ERR_LAUNCH;
  if (s == 0) return QWEN_OK;
  // a failed launch leaves slots in an unknown state: start clean
  if (zero_words(w.ws, WORKSPACE_BYTES, nullptr) != QWEN_OK || hipDeviceSynchronize() != hipSuccess)
    return QWEN_ERR_LAUNCH;
  w.epoch = 1;
  return (s & ST_BAD_TOKEN) ? QWEN_ERR_BAD_TOKEN : QWEN_ERR_TIMEOUT;
}

}  // namespace

extern "C" int qwen_last_error(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return QWEN_ERR_DEVICE;
  DeviceState& st = g_dev[dev];
  if (!st.init) return QWEN_OK;
  if (st.err != QWEN_OK) return st.err;
  if (hipDeviceSynchronize() != hipSuccess) return QWEN_ERR_LAUNCH;
  const int a = take_status(st.heap);
  const int b = take_status(st.fixed);
  // a failed sampler launch can leave its work area (histograms, barrier words) dirty
  if (a != QWEN_OK && st.smp &&
      (zero_words(st.smp + SMP_WORK, smp::WORK_BYTES / 8 * 8, nullptr) != QWEN_OK || hipDeviceSynchronize() != hipSuccess))
    return QWEN_ERR_LAUNCH;
  return a != QWEN_OK ? a : b;
}

extern "C" int qwen_set_wait_deadline_us(long long us) {
  if (us < 0) return QWEN_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  st->deadline = st->clk_khz * (us == 0 ? DEFAULT_WAIT_US : (u64)us) / 1000;
  if (st->deadline == 0) st->deadline = 1;
  return QWEN_OK;
}

extern "C" int qwen_abi_version(void) { return QWEN_ABI_VERSION; }

extern "C" int qwen_set_trace(unsigned long long* buf, long long elems, int token) {
  if (buf && elems <= 0) return QWEN_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  st->trace = buf;
  st->trace_elems = buf ? elems : 0;
  st->trace_token = buf ? token : -1;
  return QWEN_OK;
}

extern "C" int qwen_trace_events(void) { return TRACE_EVENTS; }
