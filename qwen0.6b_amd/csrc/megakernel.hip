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
//    lines ahead of the compute waves; in the lm_head they compute rows
//    alongside the compute waves;
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
};

// ------------------------------------------------------------------------------------
// small device helpers

__device__ __forceinline__ v4u ld_nt(const void* p) { return __builtin_nontemporal_load((const v4u*)p); }

// 8 fp16 weights (one 16-byte load) dotted with 8 fp32 activations
__device__ __forceinline__ float dot8(v4u w, const float (&a)[8]) {
  h8 h = __builtin_bit_cast(h8, w);
  float s = fmaf((float)h[0], a[0], 0.0f);  // one v_fma_mix (see gain_act)
  s = fmaf((float)h[1], a[1], s);
  s = fmaf((float)h[2], a[2], s);
  s = fmaf((float)h[3], a[3], s);
  s = fmaf((float)h[4], a[4], s);
  s = fmaf((float)h[5], a[5], s);
  s = fmaf((float)h[6], a[6], s);
  s = fmaf((float)h[7], a[7], s);
  return s;
}

// 8 fp16 weights dotted with 8 fp16 activations (v_dot2_f32_f16: exact products, fp32 sums).
// The whole 16 bytes are reinterpreted once and split by swizzle: bit-casting a single
// element expression such as `w.y` compiles to the `.x` element with this toolchain.
__device__ __forceinline__ float dot8h(v4u w, v4u a) {
  const h8 wh = __builtin_bit_cast(h8, w), ah = __builtin_bit_cast(h8, a);
  float s = __builtin_amdgcn_fdot2(wh.s01, ah.s01, 0.f, false);
  s = __builtin_amdgcn_fdot2(wh.s23, ah.s23, s, false);
  s = __builtin_amdgcn_fdot2(wh.s45, ah.s45, s, false);
  s = __builtin_amdgcn_fdot2(wh.s67, ah.s67, s, false);
  return s;
}

// ---- cross-lane reductions ---------------------------------------------------------
// A wave is 4 rows of 16 lanes. Within a row: DPP row_ror (folded into v_add/v_max).
// Across rows: gfx950 v_permlane16_swap (rows 0<->1, 2<->3) and v_permlane32_swap
// (lanes 0-31 <-> 32-63). pack16/pack32 add two registers' partner rows and pack
// the two results into one register, so R rows reduce in about R + 4 instructions.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int ROR8 = 0x128, ROR4 = 0x124, ROR2 = 0x122, ROR1 = 0x121;
// max of two non-NaN values as one v_max_f32: fmaxf adds two canonicalizing ops for
// values that come out of lane permutes (this kernel runs in IEEE mode)
__device__ __forceinline__ float fmax2(float a, float b) {
  float r;
  asm("v_max_f32_e32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// every lane: sum of its 16-lane row
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<ROR8>(v);
  v += dpp<ROR4>(v);
  v += dpp<ROR2>(v);
  v += dpp<ROR1>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmax2(v, dpp<ROR8>(v));
  v = fmax2(v, dpp<ROR4>(v));
  v = fmax2(v, dpp<ROR2>(v));
  v = fmax2(v, dpp<ROR1>(v));
  return v;
}
// rows of the result: 0 = a.r0 + a.r1, 1 = b.r0 + b.r1, 2 = a.r2 + a.r3, 3 = b.r2 + b.r3
__device__ __forceinline__ float pack16(float a, float b) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// lanes 0-31 of the result: a.lo + a.hi; lanes 32-63: b.lo + b.hi
__device__ __forceinline__ float pack32(float a, float b) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max16x(float v) {  // max of partner rows (0<->1, 2<->3)
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max32x(float v) {  // max of the two 32-lane halves
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// every lane: sum over the whole wave
__device__ __forceinline__ float wave_sum(float v) { return row16_sum(pack16(pack32(v, v), pack32(v, v))); }
// every lane: sum over its 32-lane half
__device__ __forceinline__ float half_sum(float v) { return row16_sum(pack16(v, v)); }
// every lane: sum over the 4 lanes {l, l^16, l^32, l^48} (same position in every row)
__device__ __forceinline__ float rows4_sum(float v) {
  const float t = pack16(v, v);
  return pack32(t, t);
}
__device__ __forceinline__ float rows4_max(float v) { return max32x(max16x(v)); }
// 4 row partials -> full sums: lanes 0-15 hold a, 16-31 c, 32-47 b, 48-63 d
__device__ __forceinline__ float reduce4(float a, float b, float c, float d) {
  return row16_sum(pack16(pack32(a, b), pack32(c, d)));
}
// 6 row partials -> full sums: p holds (a, b, d, e) and q holds (c, c, f, f) in rows 0..3
__device__ __forceinline__ void reduce6(const float (&v)[6], float& p, float& q) {
  const float x1 = pack32(v[0], v[3]), x2 = pack32(v[1], v[4]), x3 = pack32(v[2], v[5]);
  p = row16_sum(pack16(x1, x2));
  q = row16_sum(pack16(x3, x3));
}
// 8 row partials -> full sums: y0 rows 0..3 = (v0, v2, v1, v3), y1 rows 0..3 = (v4, v6, v5, v7)
__device__ __forceinline__ void reduce8(const float (&v)[8], float& y0, float& y1) {
  y0 = row16_sum(pack16(pack32(v[0], v[1]), pack32(v[2], v[3])));
  y1 = row16_sum(pack16(pack32(v[4], v[5]), pack32(v[6], v[7])));
}
// row (0..7 of reduce8's inputs) whose total lane `lane` holds in y0; y1 holds row + 4
__device__ __forceinline__ int reduce8_row(int lane) { return (lane >> 4) == 1 ? 2 : ((lane >> 4) == 2 ? 1 : (lane >> 4)); }
// (value, index) arg-max over the whole wave, lowest index on ties; every lane gets the result
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  better(v, i, dpp<ROR8>(v), dpp_i<ROR8>(i));
  better(v, i, dpp<ROR4>(v), dpp_i<ROR4>(i));
  better(v, i, dpp<ROR2>(v), dpp_i<ROR2>(i));
  better(v, i, dpp<ROR1>(v), dpp_i<ROR1>(i));
  auto rv = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  auto ri = __builtin_amdgcn_permlane16_swap((unsigned)i, (unsigned)i, false, false);
  v = __uint_as_float(rv[0]);
  i = (int)ri[0];
  better(v, i, __uint_as_float(rv[1]), (int)ri[1]);
  rv = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  ri = __builtin_amdgcn_permlane32_swap((unsigned)i, (unsigned)i, false, false);
  v = __uint_as_float(rv[0]);
  i = (int)ri[0];
  better(v, i, __uint_as_float(rv[1]), (int)ri[1]);
}
__device__ __forceinline__ float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ u32 pack_h2(float a, float b) {
  h2 h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(u32, h);
}
__device__ __forceinline__ float lo_h(u32 p) { return (float)__builtin_bit_cast(h2, p)[0]; }
__device__ __forceinline__ float hi_h(u32 p) { return (float)__builtin_bit_cast(h2, p)[1]; }

// a slot read by workgroups on other XCDs: device-scope (sc1) store
__device__ __forceinline__ void ll_store(u64* ws, long slot, u32 payload, u32 tag) {
  __hip_atomic_store(ws + slot, ((u64)tag << 32) | (u64)payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// a slot read only by workgroups of the writer's XCD: a plain 8-byte store lands in
// the XCD's L2, where the readers' device-scope loads find it (measured on MI355X:
// a 32-workgroup all-gather of 1024 values takes 1.1 us per round this way, 1.5 us
// with device-scope stores)
__device__ __forceinline__ void ll_store_xcd(u64* ws, long slot, u32 payload, u32 tag) {
  __hip_atomic_store(ws + slot, ((u64)tag << 32) | (u64)payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(const u64* ws) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)ws, 0, 0x7fffffff, 0x00020000);
}
// one 16-byte device-scope (sc1) load of two slots at byte offset voff + soff
__device__ __forceinline__ v4u ld_pair(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 16);
}

__device__ __forceinline__ u32 lds_ld(const u32* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_st(u32* p, u32 v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local"); }
__device__ __forceinline__ void lds_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local"); }

// LDS-DMA: 16 bytes per lane from global memory to LDS byte address lds + 16 lane.
// Issued through inline assembly so the compiler adds no vmcnt wait before the
// wave's later LDS accesses; the loader tracks completion with explicit vmcnt waits.
__device__ __forceinline__ void dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(lds), "v"(g) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ------------------------------------------------------------------------------------
// workgroup shared state

struct Shared {
  v4u ring[RING_LINES][LINE_BYTES / 16];  // 128 KB weight / K-V line ring (must stay first: LDS offset 0)
  float wbuf[NCW][2 * HD];          // per-wave scratch: the roped fp16 q0 | q1 | k | v of attention
  float xs[HIDDEN];                // QKV / gate-up input vector, gathered from the four waves' quarters
  float xss[2][NCW];               // the quarters' sums of squares (alternating)
  float apart[NCW][2][PART_PER_HEAD];  // per-wave attention partials (m, l, acc)
  float resid[HROWS];              // fp32 residual x, rows [32 i, 32 i + 32) (wave c: rows 8 c .. 8 c + 7)
  float actres[HROWS];             // fp32 post-attention residual, same rows and owners
  float xfin[HIDDEN];              // lm_head input (fp32)
  float lmv[NCW + NLW];            // per-wave lm_head best value
  int lmi[NCW + NLW];              // per-wave lm_head best row
  float argv[NCW];                 // per-wave best of the global argmax
  int argi[NCW];
  u32 sync;                        // compute-wave barrier arrivals (monotonic)
  u32 done_upto[NLW];              // loader wave q: smallest line (== q mod 4) not yet in the ring
  u32 cons[NCW];                   // compute wave c: ring lines below this are no longer read
  u32 xfin_cnt;                    // quarters of xfin stored (monotonic)
  u32 lm_cnt;                      // lm_head partials stored (monotonic)
  u32 lm_next[2];                  // next lm_head chunk of the workgroup (by phase parity)
  u32 lm_pool_done[2];             // the pool ran out (by phase parity)
  u32 abort;
  // the layer pointer table, copied from global memory at start: reading it from
  // LDS keeps the loader waves' vmcnt free of anything but their own DMAs
  LDGLayerWeight lw[MAX_LAYERS];
};

struct Ctl {
  const KParams* P;
  Shared* S;
  __amdgpu_buffer_rsrc_t r;
  bool ok;
  u64 deadline;
};

// t0 == 0: the wait's clock starts at its 16th spin (a poll's first sweeps pay no clock read)
__device__ __forceinline__ bool give_up(Ctl& C, u64& t0, int& spins) {
  ++spins;
  if ((spins & 15) == 0) {
    if (lds_ld(&C.S->abort)) return true;
    const u64 now = wall_clock64();
    if (t0 == 0) t0 = now;
    if (now - t0 > C.deadline) {
      __hip_atomic_fetch_or(C.P->status, ST_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      lds_st(&C.S->abort, 1u);
      return true;
    }
  }
  if ((spins & 255) == 0 && __hip_atomic_load(C.P->status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
    lds_st(&C.S->abort, 1u);
    return true;
  }
  return false;
}

// Polls K slot pairs per lane until both slots of every pair carry `tag`. Pair k
// of this lane is at byte voff[k] + soff of the workspace (soff wave-uniform).
// Lanes with active == false take no part. `first` runs once, after the first
// sweep's loads are issued (the ring check of the stage hides behind their latency).
struct NoPre {
  __device__ void operator()() const {}
};
template <int K, typename Pre = NoPre>
__device__ __forceinline__ void poll(Ctl& C, u32 tag, const int (&voff)[K], int soff, bool active, v4u (&out)[K],
                                     Pre first = Pre()) {
#pragma unroll
  for (int k = 0; k < K; ++k) out[k] = v4u{0, 0, 0, 0};
  if (!C.ok) {
    first();
    return;
  }
  // first sweep: every active lane loads all its pairs (most polls end here)
  asm volatile("" ::: "memory");
  if (active) {
#pragma unroll
    for (int k = 0; k < K; ++k) out[k] = ld_pair(C.r, voff[k], soff);
  }
  first();
  bool done[K];
  bool all = true;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    done[k] = !active || ((out[k].y == tag) && (out[k].w == tag));
    all = all && done[k];
  }
  if (__all(all)) return;
  // later sweeps reload only the pairs still missing
  u64 t0 = 0;
  int spins = 0;
  for (;;) {
    if (give_up(C, t0, spins)) {
      C.ok = false;
      return;
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (!done[k]) out[k] = ld_pair(C.r, voff[k], soff);
    all = true;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (!done[k]) done[k] = (out[k].y == tag) && (out[k].w == tag);
      all = all && done[k];
    }
    if (__all(all)) return;
  }
}

// spins until *p >= v (LDS), bounded
__device__ __forceinline__ void lds_wait_ge(Ctl& C, const u32* p, u32 v) {
  if (!C.ok) return;
  if (lds_ld(p) >= v) {
    lds_acquire();
    return;
  }
  u64 t0 = wall_clock64();
  int spins = 0;
  while (lds_ld(p) < v) {
    if (give_up(C, t0, spins)) {
      C.ok = false;
      return;
    }

  }
  lds_acquire();
}

// Each compute wave waits for its own result stores before it starts polling the next stage's
// inputs. Polls issued while the stores are still in flight delay those stores (the consumer's
// hop grows by about 0.5 us per stage); bit s of the mask enables this after stage s.
#ifndef STORE_DRAIN_MASK
#define STORE_DRAIN_MASK 0xff
#endif
__device__ __forceinline__ void drain_stores(int stage) {
  if ((STORE_DRAIN_MASK >> stage) & 1) wait_vmcnt<0>();
}

// a uniform branch (one scalar compare per call site when tracing is off); lane 0 stores
__device__ __forceinline__ void trace_ev(const KParams& P, int token, int stage, int what) {
  if (__builtin_expect(P.trace != nullptr && token == P.trace_token, 0)) {
    const u64 now = wall_clock64();
    if (__lane_id() == 0) P.trace[((long)blockIdx.x * trace_stages(P.num_layers) + stage) * TRACE_EVENTS + what] = now;
  }
}

// A stage's lines from its first global line n0: vb = this lane's byte offset of line n0
// in the ring, and line n0 + k is at (vb + 1024 k) mod the ring size (the ring is the first
// 128 KB of LDS), one add and one and per line
__device__ __forceinline__ u32 ring_vbase(u32 n0, int lane) { return (n0 % RING_LINES) * LINE_BYTES + 16 * lane; }
__device__ __forceinline__ v4u ring_ld(const Shared* S, u32 vb, int k) {
  return *(const v4u*)((const char*)S->ring + ((vb + (u32)k * LINE_BYTES) & (RING_LINES * LINE_BYTES - 1)));
}

// ------------------------------------------------------------------------------------
// lm_head rows (every wave): 8-row chunks of the tied embedding (the workgroup's own,
// then claimed from the pool), two chunks in registers per wave, dotted with xfin (fp32)

__device__ __forceinline__ void lm_issue(const KParams& P, int g, v4u (&buf)[16]) {
  const int lane = __lane_id();
#pragma unroll
  for (int j = 0; j < LM_CHUNK; ++j) {
    const _Float16* base = P.lm_head + (long)(LM_CHUNK * g + j) * HIDDEN;
    buf[2 * j] = ld_nt(base + 8 * lane);
    buf[2 * j + 1] = ld_nt(base + 512 + 8 * lane);
  }
}

__device__ __forceinline__ void lm_consume(const KParams& P, int g, int t, const v4u (&buf)[16],
                                           const float (&a)[8], const float (&b)[8], float& best, int& bidx) {
  const int lane = __lane_id();
  float part[8];
#pragma unroll
  for (int j = 0; j < LM_CHUNK; ++j) part[j] = dot8(buf[2 * j], a) + dot8(buf[2 * j + 1], b);
  float y0, y1;
  reduce8(part, y0, y1);
  // lanes 0, 16, 32, 48 hold rows (0, 4), (2, 6), (1, 5), (3, 7); chunks arrive in no
  // particular order, so equal logits keep the lower row explicitly
  if ((lane & 15) == 0) {
    const int jr = reduce8_row(lane);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = LM_CHUNK * g + jr + 4 * h;
      const float val = h == 0 ? y0 : y1;
      if (P.logits_out) P.logits_out[(long)t * VOCAB + row] = val;
      const float vv = __builtin_isnan(val) ? -INFINITY : val;
      if (vv > best || (vv == best && row < bidx)) {
        best = vv;
        bidx = row;
      }
    }
  }
}

// next chunk of this phase's shared counter (lane 0 takes it, every lane gets it)
__device__ __forceinline__ int lm_grab(Shared* S, u32 phase) {
  u32 ch = 0;
  if (__lane_id() == 0) ch = __hip_atomic_fetch_add(&S->lm_next[phase & 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return (int)__builtin_amdgcn_readfirstlane(ch);
}

// pool counter of group G for token epoch e: (epoch << 32) + chunks claimed so far.
// Workgroup 0 sets the counters of epochs e + 2 and e + 3 during token e, when every claim
// of tokens e - 2 and e - 1 (same counters) has returned; a counter whose epoch differs
// is not in use.
__device__ __forceinline__ u64* lm_pool_ctr(const KParams& P, u32 e, int G) {
  return (u64*)((char*)P.status + 256 + ((e & 3) * LM_NGRP + G) * LM_CTR_STRIDE);
}

struct LmClaim {
  int ch;     // the workgroup's chunk counter value
  bool pool;  // a pool claim was sent
  u64 r;      // its result (lane 0)
};

// claim the wave's next chunk: the workgroup's own chunks first, then the pool (the
// device-scope add is sent now and read at lm_take, one chunk later)
__device__ __forceinline__ LmClaim lm_claim(const KParams& P, Shared* S, u32 phase, u32 epoch) {
  LmClaim c;
  c.ch = lm_grab(S, phase);
  c.pool = c.ch >= LM_STATIC && lds_ld(&S->lm_pool_done[phase & 1]) == 0u;
  c.r = 0;
  if (c.pool && __lane_id() == 0) {
    // a per-lane address keeps the atomic optimizer from rewriting the add into a
    // wave-wide one whose result is read (and waited for) right where it is sent
    __attribute__((address_space(1))) u64* ctr =
        (__attribute__((address_space(1))) u64*)lm_pool_ctr(P, epoch, blockIdx.x / LM_GROUP);
    asm volatile("" : "+v"(ctr));
    c.r = __hip_atomic_fetch_add(ctr, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return c;
}

// the claimed chunk id, or -1 when the wave is done
__device__ __forceinline__ int lm_take(Shared* S, const LmClaim& c, int w, u32 phase, u32 epoch) {
  if (c.ch < LM_STATIC) return w + NWG * c.ch;
  if (!c.pool) return -1;  // the pool ran out
  // read the claim here, not where it was sent: without the fence the compiler moves the
  // lane-0 reads up to the add itself, which then waits for every load sent before it
  u64 r = c.r;
  asm volatile("" : "+v"(r));
  const u32 lo = __builtin_amdgcn_readfirstlane((u32)r), hi = __builtin_amdgcn_readfirstlane((u32)(r >> 32));
  if (hi == epoch) {
    const int G = w / LM_GROUP;
    if (lo < (u32)lm_group_chunks(G)) return LM_STATIC * NWG + LM_NGRP * (int)lo + G;
    if (__lane_id() == 0) lds_st(&S->lm_pool_done[phase & 1], 1u);
    return -1;
  }
  // the counter is not set up for this token: the workgroup's remaining dealt chunks
  return c.ch < lm_chunks(w) ? w + NWG * c.ch : -1;
}

__device__ __forceinline__ void lm_rows(Ctl& C, const KParams& P, int v, int t, u32 phase, u32 epoch) {
  Shared* S = C.S;
  const int w = blockIdx.x, lane = __lane_id();
  // the next phase's counter and flag are idle until every wave has passed this phase's
  // xfin wait, and each wave reaches that wait only after its last claim of the previous phase
  if (v == 0 && lane == 0) {
    lds_st(&S->lm_next[(phase + 1) & 1], 0u);
    lds_st(&S->lm_pool_done[(phase + 1) & 1], 0u);
  }
  v4u A[16], B[16];
  // two chunks in flight (A, B); each buffer's next chunk is claimed right after its loads
  // are sent, so a pool claim returns behind them and is read once they are consumed
  int ga = lm_take(S, lm_claim(P, S, phase, epoch), w, phase, epoch);
  if (ga >= 0) lm_issue(P, ga, A);
  LmClaim na = lm_claim(P, S, phase, epoch);
  lds_wait_ge(C, &S->xfin_cnt, NCW * phase);
  float a[8], b[8];
  {
    const float4 p0 = *(const float4*)(S->xfin + 8 * lane), p1 = *(const float4*)(S->xfin + 8 * lane + 4);
    const float4 q0 = *(const float4*)(S->xfin + 512 + 8 * lane), q1 = *(const float4*)(S->xfin + 512 + 8 * lane + 4);
    a[0] = p0.x; a[1] = p0.y; a[2] = p0.z; a[3] = p0.w; a[4] = p1.x; a[5] = p1.y; a[6] = p1.z; a[7] = p1.w;
    b[0] = q0.x; b[1] = q0.y; b[2] = q0.z; b[3] = q0.w; b[4] = q1.x; b[5] = q1.y; b[6] = q1.z; b[7] = q1.w;
  }
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  int gb = lm_take(S, lm_claim(P, S, phase, epoch), w, phase, epoch);
  if (gb >= 0) lm_issue(P, gb, B);
  LmClaim nb = lm_claim(P, S, phase, epoch);
  for (;;) {
    if (ga >= 0) {
      lm_consume(P, ga, t, A, a, b, best, bidx);
      ga = lm_take(S, na, w, phase, epoch);
      if (ga >= 0) {
        lm_issue(P, ga, A);
        na = lm_claim(P, S, phase, epoch);
      }
    }
    if (gb >= 0) {
      lm_consume(P, gb, t, B, a, b, best, bidx);
      gb = lm_take(S, nb, w, phase, epoch);
      if (gb >= 0) {
        lm_issue(P, gb, B);
        nb = lm_claim(P, S, phase, epoch);
      }
    }
    if (ga < 0 && gb < 0) break;
  }
  wave_argmax(best, bidx);
  if (lane == 0) {
    S->lmv[v] = best;
    S->lmi[v] = bidx;
  }
  lds_release();
  if (lane == 0) __hip_atomic_fetch_add(&S->lm_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ------------------------------------------------------------------------------------
// compute waves

struct CW {
  Ctl C;
  int w, x, i, c, lane;
  u32 nsync;   // barriers passed
  u32 gl;      // global ring line index of the next stage
};

// LDS byte address of a workgroup-shared variable
__device__ __forceinline__ u32 lds_addr(const void* p) { return (u32)(size_t)(const __attribute__((address_space(3))) void*)p; }
// barrier of the 4 compute waves (monotonic LDS counter); lane 0 adds with a plain ds_add_u32
// (the compiler's atomic optimizer would first count the active lanes)
__device__ __forceinline__ void sync4(CW& W) {
  lds_release();
  if (W.lane == 0) asm volatile("ds_add_u32 %0, %1" ::"v"(lds_addr(&W.C.S->sync)), "v"(1u) : "memory");
  ++W.nsync;
  lds_wait_ge(W.C, &W.C.S->sync, NCW * W.nsync);
}

__device__ __forceinline__ u32 lines_done(const Shared* S) {
  const u32 a = lds_ld(&S->done_upto[0]), b = lds_ld(&S->done_upto[1]);
  const u32 c = lds_ld(&S->done_upto[2]), d = lds_ld(&S->done_upto[3]);
  return min(min(a, b), min(c, d));
}
// waits until every ring line below `end` is in LDS
__device__ __forceinline__ void wait_lines(CW& W, u32 end) {
  if (!W.C.ok) return;
  if (lines_done(W.C.S) >= end) {
    lds_acquire();
    return;
  }
  u64 t0 = wall_clock64();
  int spins = 0;
  while (lines_done(W.C.S) < end) {
    if (give_up(W.C, t0, spins)) {
      W.C.ok = false;
      return;
    }

  }
  lds_acquire();
}
// this wave no longer reads ring lines below `end`
__device__ __forceinline__ void release_lines(CW& W, u32 end) {
  lds_release();
  if (W.lane == 0) lds_st(&W.C.S->cons[W.c], end);
}

// Stage inputs: small ones (attention output, split partials, residual partials) go
// straight from the exchange slots into each compute wave's registers, every wave
// polling what it needs; the larger vectors (x, q|k|v, SiLU*up) are polled one quarter
// per wave and gathered in LDS behind one four-wave barrier, which keeps each XCD's
// polling traffic a quarter as large.

__device__ __forceinline__ float sumsq16(const float (&xa)[8], const float (&xb)[8]) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = fmaf(xa[e], xa[e], fmaf(xb[e], xb[e], s));
  return s;
}
// the lane's values x[8 lane, +8) and x[512 + 8 lane, +8) of a 1024-value H2 vector in
// slots [base_slot, base_slot + 512); returns the whole vector's sum of squares. Each wave
// polls one quarter (1 KB): polling the whole 4 KB from all 128 waves of an XCD costs
// 2.5x as long per hand-off (measured 1.10 vs 0.43 us per all-gather round)
template <typename Pre>
__device__ __forceinline__ float poll_x1024(CW& W, u32 tag, long base_slot, float (&xa)[8], float (&xb)[8], Pre first) {
  // wave c polls quarter c (slots [128 c, +128): lane -> values 256 c + 4 lane .. +4) into the
  // workgroup's vector; after the four-wave barrier every wave reads its lanes' 16 values
  Shared* S = W.C.S;
  const int lane = W.lane, p = W.nsync & 1;
  const int voff[1] = {16 * lane};
  v4u v[1];
  poll<1>(W.C, tag, voff, (int)((base_slot + 128 * W.c) * 8), true, v, first);
  const float a = lo_h(v[0].x), b = hi_h(v[0].x), cc = lo_h(v[0].z), d = hi_h(v[0].z);
  *(float4*)(S->xs + 256 * W.c + 4 * lane) = make_float4(a, b, cc, d);
  const float q = wave_sum(a * a + b * b + cc * cc + d * d);
  if (lane == 0) S->xss[p][W.c] = q;
  sync4(W);
  const float4 p0 = *(const float4*)(S->xs + 8 * lane), p1 = *(const float4*)(S->xs + 8 * lane + 4);
  const float4 q0 = *(const float4*)(S->xs + 512 + 8 * lane), q1 = *(const float4*)(S->xs + 512 + 8 * lane + 4);
  xa[0] = p0.x; xa[1] = p0.y; xa[2] = p0.z; xa[3] = p0.w; xa[4] = p1.x; xa[5] = p1.y; xa[6] = p1.z; xa[7] = p1.w;
  xb[0] = q0.x; xb[1] = q0.y; xb[2] = q0.z; xb[3] = q0.w; xb[4] = q1.x; xb[5] = q1.y; xb[6] = q1.z; xb[7] = q1.w;
  return (S->xss[p][0] + S->xss[p][1]) + (S->xss[p][2] + S->xss[p][3]);
}
// the same from a 1024-value fp16 vector in global memory (embedding row, MLP input)
__device__ __forceinline__ float load_x1024(const _Float16* src, int lane, float (&xa)[8], float (&xb)[8]) {
  const h8 p = *(const h8*)(src + 8 * lane), q = *(const h8*)(src + 512 + 8 * lane);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xa[e] = (float)p[e];
    xb[e] = (float)q[e];
  }
  return wave_sum(sumsq16(xa, xb));
}
// 1 / RMS of a 1024-value vector from its sum of squares
// v_rsq_f32 for an argument >= RMS_EPS: rsqrtf adds a denormal-input path that such an
// argument never takes (same result, six instructions fewer)
__device__ __forceinline__ float rsq_normal(float v) { return __builtin_amdgcn_rsqf(v); }
__device__ __forceinline__ float rstd_of(float ss) { return rsq_normal(ss * (1.0f / HIDDEN) + RMS_EPS); }

// the lane's 16 normalised activations a = x[8 l .. 8 l + 8), b = x[512 + 8 l ..]
__device__ __forceinline__ void norm_act(const float (&xa)[8], const float (&xb)[8], float rstd, const h8& w0,
                                         const h8& w1, float (&a)[8], float (&b)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = xa[e] * rstd * (float)w0[e];
    b[e] = xb[e] * rstd * (float)w1[e];
  }
}

// the lane's 16 gain-weighted activations a = x[8 l ..] * g, b = x[512 + 8 l ..] * g; the
// RMSNorm scale rstd is applied to the row sums instead. Written as fma(x, g, +0), one
// v_fma_mix_f32 per value (a plain product costs a conversion and a multiply); it differs
// from x * g only in the sign of an exact zero, which no dot product sees
__device__ __forceinline__ void gain_act(const float (&xa)[8], const float (&xb)[8], const h8& w0, const h8& w1,
                                         float (&a)[8], float (&b)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = fmaf(xa[e], (float)w0[e], 0.0f);
    b[e] = fmaf(xb[e], (float)w1[e], 0.0f);
  }
}

// one 2 KB weight row (read from ring lines n, n + 1 into registers) dotted with (a | b)
__device__ __forceinline__ float row2k_r(const v4u& w0, const v4u& w1, const float (&a)[8], const float (&b)[8]) {
  return dot8(w0, a) + dot8(w1, b);
}

// ---- stages ----------------------------------------------------------------------------

// QKV: rows [16 i + 4 c, +4) of the kv group from the normalised residual
__device__ __forceinline__ void st_qkv(CW& W, const KParams& P, int t, int l, u32 epoch, int token) {
  Shared* S = W.C.S;
  const int lane = W.lane, par = l & 1;
  trace_ev(P, t, NSTAGE * l + S_QKV, TR_POLL);
  const u32 n0 = W.gl;  // lines n0, n0 + 1: input norm weights; then the rows
  W.gl += LINES_QKV;
  float xa[8], xb[8], ss;
  const u32 vb = ring_vbase(n0, lane);
  // the wave's ring lines (norm weights, 4 rows) are read into registers while it waits for
  // its input, so no LDS latency follows the input's arrival, and released right away
  v4u wl[LINES_NORM + 8];
  auto lines = [&] {
    wait_lines(W, W.gl);
    trace_ev(P, t, NSTAGE * l + S_QKV, TR_LINES);
    wl[0] = ring_ld(S, vb, 0);
    wl[1] = ring_ld(S, vb, 1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wl[LINES_NORM + 2 * r] = ring_ld(S, vb, LINES_NORM + 2 * (4 * W.c + r));
      wl[LINES_NORM + 2 * r + 1] = ring_ld(S, vb, LINES_NORM + 2 * (4 * W.c + r) + 1);
    }
    release_lines(W, W.gl);
  };
  if (l == 0) {
    const _Float16* row = P.embed + (long)token * HIDDEN;
    ss = load_x1024(row, lane, xa, xb);
    if (lane < 8) S->resid[8 * W.c + lane] = (float)row[HROWS * W.i + 8 * W.c + lane];
    lines();
  } else {
    ss = poll_x1024(W, tag_of(epoch, l - 1, S_DSUM), xbuf(par ^ 1, W.x, B_X), xa, xb, lines);
  }
  trace_ev(P, t, NSTAGE * l + S_QKV, TR_INPUT);
  float a[8], b[8];
  gain_act(xa, xb, __builtin_bit_cast(h8, wl[0]), __builtin_bit_cast(h8, wl[1]), a, b);
  float part[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) part[r] = row2k_r(wl[LINES_NORM + 2 * r], wl[LINES_NORM + 2 * r + 1], a, b);
  // lanes 0, 16, 32, 48 hold rows 0, 2, 1, 3
  const float rs = reduce4(part[0], part[1], part[2], part[3]) * rstd_of(ss);
  const float r0 = bcast(rs, 0), r1 = bcast(rs, 32), r2 = bcast(rs, 16), r3 = bcast(rs, 48);
  if (lane < 2)
    ll_store_xcd(P.ws, xbuf(par, W.x, B_QKV) + (QKV_PER_WG / 2) * W.i + 2 * W.c + lane,
             lane == 0 ? pack_h2(r0, r1) : pack_h2(r2, r3), tag_of(epoch, l, S_QKV));
  drain_stores(S_QKV);
  trace_ev(P, t, NSTAGE * l + S_QKV, TR_STORE);
}

// attention split i of kv head x: q/k norms, RoPE, K/V write, 16 positions per wave, merge
__device__ __forceinline__ void st_att(CW& W, const KParams& P, int t, int l, u32 epoch) {
  Shared* S = W.C.S;
  const int lane = W.lane, par = l & 1;
  const int pos = P.start_pos + t, ctx = pos + 1;
  _Float16* qr = (_Float16*)S->wbuf[W.c];  // roped q0 | q1 | k | v of the current position (fp16)
  trace_ev(P, t, NSTAGE * l + S_ATT, TR_POLL);
  // ring: line n0 = q_norm | k_norm | cos[pos] | sin[pos]; K lines n0 + 1 + m; V lines n0 + 1 + nk + m
  const int t0 = att_t0(ctx, W.i), t1 = att_t1(ctx, W.i), nk = att_nk(ctx, W.i);
  const u32 n0 = W.gl;
  W.gl += LINES_ATTMISC + 2 * nk;
  // the group's 512 q0 | q1 | k | v values: lane l (h = l / 32, dm = 2 (l % 32)) takes dims
  // dm, dm + 1 and their rotate-half partners 64 + dm, 65 + dm of q head h, and of k (h = 0)
  // or v (h = 1), so RoPE needs no other lane
  const int dm = 2 * (lane & 31), hb = 128 * (lane >> 5) + dm;
  const u32 nkl = n0 + LINES_ATTMISC;  // first K line
  const u32 vbk = ring_vbase(nkl, lane);
  // this wave's 16 positions: K lines 4c..4c+3, V lines nk + 4c ..; a wave whose lines run
  // past the split's last (m >= nk) reads that last line again (or, for an empty split, the
  // misc line), which holds finite values; those positions are masked out of the softmax
  const int j = lane >> 4, q16 = lane & 15;
  // the norm / cos / sin values and the wave's K and V lines are read into registers (and the
  // lines released) while the wave waits for its input
  h2 qn0, qn1, kn0, kn1, cv0, cv1, sv0, sv1;
  v4u kw[4], vw[4];
  float2 qlo, qhi, klo, khi;
  {  // wave c polls slots [64 c, +64) (lane % 32: values 128 c + 4 (lane % 32) .. +4) into S->xs;
     // lanes 32-63 repeat lanes 0-31 (same lines, same values), which keeps the wave unbranched
    const int voff[1] = {16 * (lane & 31)};
    v4u v[1];
    poll<1>(W.C, tag_of(epoch, l, S_QKV), voff, (int)((xbuf(par, W.x, B_QKV) + 64 * W.c) * 8), true, v,
            [&] {
      wait_lines(W, W.gl);
      trace_ev(P, t, NSTAGE * l + S_ATT, TR_LINES);
      const char* misc = (const char*)S->ring[n0 % RING_LINES];
      qn0 = *(const h2*)(misc + 2 * dm);
      qn1 = *(const h2*)(misc + 2 * (64 + dm));
      kn0 = *(const h2*)(misc + 256 + 2 * dm);
      kn1 = *(const h2*)(misc + 256 + 2 * (64 + dm));
      cv0 = *(const h2*)(misc + 512 + 2 * dm);
      cv1 = *(const h2*)(misc + 512 + 2 * (64 + dm));
      sv0 = *(const h2*)(misc + 768 + 2 * dm);
      sv1 = *(const h2*)(misc + 768 + 2 * (64 + dm));
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int mm = nk > 0 ? min(4 * W.c + bb, nk - 1) : -LINES_ATTMISC;
        kw[bb] = ring_ld(S, vbk, mm);
        vw[bb] = ring_ld(S, vbk, (nk > 0 ? nk : 0) + mm);
      }
      release_lines(W, W.gl);
    });
    *(float4*)(S->xs + 128 * W.c + 4 * (lane & 31)) =
        make_float4(lo_h(v[0].x), hi_h(v[0].x), lo_h(v[0].z), hi_h(v[0].z));
    sync4(W);
    qlo = *(const float2*)(S->xs + hb);
    qhi = *(const float2*)(S->xs + hb + 64);
    klo = *(const float2*)(S->xs + 256 + hb);
    khi = *(const float2*)(S->xs + 256 + hb + 64);
  }
  trace_ev(P, t, NSTAGE * l + S_ATT, TR_INPUT);
  // every wave computes the normed, roped q0 | q1 | k and v into its own scratch
  {
    const float qn[4] = {(float)qn0[0], (float)qn0[1], (float)qn1[0], (float)qn1[1]};
    const float kn[4] = {(float)kn0[0], (float)kn0[1], (float)kn1[0], (float)kn1[1]};
    const float cs[4] = {(float)cv0[0], (float)cv0[1], (float)cv1[0], (float)cv1[1]};
    const float sn[4] = {-(float)sv0[0], -(float)sv0[1], (float)sv1[0], (float)sv1[1]};
    const float q[4] = {qlo.x, qlo.y, qhi.x, qhi.y};
    const float k[4] = {klo.x, klo.y, khi.x, khi.y};
    const float rq = rsq_normal(half_sum(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]) * (1.0f / HD) + RMS_EPS);
    const float rk = rsq_normal(half_sum(k[0] * k[0] + k[1] * k[1] + k[2] * k[2] + k[3] * k[3]) * (1.0f / HD) + RMS_EPS);
    float qq[4], kk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qq[j] = q[j] * rq * qn[j];
      kk[j] = k[j] * rk * kn[j];
    }
    // rotate-half RoPE: out[d] = x[d] cos[d] - x[d + 64] sin[d], out[d + 64] = x[d + 64] cos[d + 64] + x[d] sin[d + 64]
    float qo[4], ko[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qo[j] = qq[j] * cs[j] + qq[j ^ 2] * sn[j];
      ko[j] = kk[j] * cs[j] + kk[j ^ 2] * sn[j];
    }
    // fp16, as the values the cache keeps (and as the reference rounds q)
    const h2 qh0 = {(_Float16)qo[0], (_Float16)qo[1]}, qh1 = {(_Float16)qo[2], (_Float16)qo[3]};
    // lanes 0-31 keep the normed, roped k; lanes 32-63 the raw v (selected per value, unbranched)
    float kx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) kx[j] = lane < 32 ? ko[j] : k[j];
    const h2 kv0 = {(_Float16)kx[0], (_Float16)kx[1]}, kv1 = {(_Float16)kx[2], (_Float16)kx[3]};
    *(h2*)(qr + hb) = qh0;
    *(h2*)(qr + hb + 64) = qh1;
    *(h2*)(qr + 256 + hb) = kv0;
    *(h2*)(qr + 256 + hb + 64) = kv1;
    // the split holding `pos` writes this position's K (roped) and V to the cache
    if (W.c == 0 && att_t0(ctx, W.i) <= pos && pos < att_t1(ctx, W.i)) {
      _Float16* row = (lane < 32 ? P.k_cache : P.v_cache) + (((long)l * NKV + W.x) * P.max_seq + pos) * HD + dm;
      *(h2*)row = kv0;
      *(h2*)(row + 64) = kv1;
    }
  }
  // the scratch was written as fp16 vectors of another type: keep the compiler from
  // moving these reads above those writes (type-based alias analysis would allow it)
  asm volatile("" ::: "memory");
  const v4u qa = *(const v4u*)(qr + 8 * q16), qb = *(const v4u*)(qr + 128 + 8 * q16);  // q heads 0, 1 (fp16)
  // the current position is not in the cache lines (the loader reads a spare row for it):
  // the wave whose 16 positions include it puts its fp16 k and v into row jp of its line
  // registers (rows are lanes 16 jp .. 16 jp + 15)
  {
    const int mp = (pos - t0) >> 2, jp = (pos - t0) & 3;
    if (pos >= t0 && pos < t1 && (mp >> 2) == W.c) {
      const v4u kn = *(const v4u*)(qr + 256 + 8 * q16), vn = *(const v4u*)(qr + 384 + 8 * q16);
#pragma unroll
      for (int bb = 0; bb < 4; ++bb)
        if (bb == (mp & 3) && j == jp) {
          kw[bb] = kn;
          vw[bb] = vn;
        }
    }
  }
  bool valid[4];
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) valid[bb] = 4 * W.c + bb < nk && t0 + 4 * (4 * W.c + bb) + j < t1;
  float sc[4][2];
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    const float s0 = row16_sum(dot8h(kw[bb], qa)) * P.attn_scale;
    const float s1 = row16_sum(dot8h(kw[bb], qb)) * P.attn_scale;
    sc[bb][0] = valid[bb] ? s0 : -INFINITY;
    sc[bb][1] = valid[bb] ? s1 : -INFINITY;
  }
  float mh[2], lh[2], acc[2][8];
  float pr[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float mx = rows4_max(fmaxf(fmaxf(sc[0][h], sc[1][h]), fmaxf(sc[2][h], sc[3][h])));
    mh[h] = mx;
    float lsum = 0.f;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      pr[h][bb] = valid[bb] ? __expf(sc[bb][h] - mx) : 0.f;
      lsum += pr[h][bb];
    }
    lh[h] = rows4_sum(lsum);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    const h8 vh = __builtin_bit_cast(h8, vw[bb]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[0][e] = fmaf(pr[0][bb], (float)vh[e], acc[0][e]);
      acc[1][e] = fmaf(pr[1][bb], (float)vh[e], acc[1][e]);
    }
  }
  // sums over the 4 rows (positions) of the 16 accumulators, transposed: row R ends up
  // with accumulators 4 R .. 4 R + 3 (head R / 2, dims 8 q16 + 4 (R % 2) + 0..3)
  float u[4];
  {
    float tt[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) tt[j] = pack32(acc[0][j], acc[1][j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = pack16(tt[j], tt[j + 4]);
  }
  float* rec = &S->apart[W.c][0][0];
  {
    const int R = lane >> 4;
    *(float4*)(rec + (R >> 1) * PART_PER_HEAD + 2 + 8 * q16 + 4 * (R & 1)) = make_float4(u[0], u[1], u[2], u[3]);
  }
  // m and l are uniform over the wave: every lane writes the same values
  *(float2*)rec = make_float2(mh[0], lh[0]);
  *(float2*)(rec + PART_PER_HEAD) = make_float2(mh[1], lh[1]);
  trace_ev(P, t, NSTAGE * l + S_ATT, TR_SYNC);
  sync4(W);
  trace_ev(P, t, NSTAGE * l + S_ATT, TR_MERGE);
  // merge the 4 wave partials: wave c writes the 64 accumulators of head c / 2, dims
  // 64 (c % 2) + lane; wave 0 lanes 0-3 also write (M, L) of both heads
  const int hm = W.c >> 1;
  float wt[NCW];
  float Mh = -INFINITY;
#pragma unroll
  for (int cc = 0; cc < NCW; ++cc) Mh = fmaxf(Mh, S->apart[cc][hm][0]);
#pragma unroll
  for (int cc = 0; cc < NCW; ++cc) {
    const float mc = S->apart[cc][hm][0];
    wt[cc] = (mc == -INFINITY) ? 0.f : __expf(mc - Mh);
  }
  {
    const int k = 2 + 64 * (W.c & 1) + lane;
    float val = 0.f;
#pragma unroll
    for (int cc = 0; cc < NCW; ++cc) val = fmaf(wt[cc], S->apart[cc][hm][k], val);
    ll_store_xcd(P.ws, xbuf(par, W.x, B_PART) + part_index(W.i, hm, k), __float_as_uint(val), tag_of(epoch, l, S_ATT));
  }
  if (W.c == 0 && lane < 4) {
    const int h = lane >> 1;
    float M = -INFINITY;
#pragma unroll
    for (int cc = 0; cc < NCW; ++cc) M = fmaxf(M, S->apart[cc][h][0]);
    float L = 0.f;
#pragma unroll
    for (int cc = 0; cc < NCW; ++cc) {
      const float mc = S->apart[cc][h][0];
      L = fmaf((mc == -INFINITY) ? 0.f : __expf(mc - M), S->apart[cc][h][1], L);
    }
    ll_store_xcd(P.ws, xbuf(par, W.x, B_PART) + part_index(W.i, h, lane & 1), __float_as_uint((lane & 1) ? L : M),
                 tag_of(epoch, l, S_ATT));
  }
  drain_stores(S_ATT);
  trace_ev(P, t, NSTAGE * l + S_ATT, TR_STORE);
}

// combine: q head 2x + i / 16; compute wave c merges dims d0 + 2 c, +1 (d0 = 8 (i % 16))
// over the 32 split partials of the kv head (lane < 32: split lane)
__device__ __forceinline__ void st_comb(CW& W, const KParams& P, int t, int l, u32 epoch) {
  const int lane = W.lane, par = l & 1;
  const int hh = W.i / 16, d = 8 * (W.i % 16) + 2 * W.c;
  const int s = lane & 31;
  const int voff[2] = {(int)(part_index(s, hh, 0) * 8), (int)(part_index(s, hh, 2 + d) * 8)};
  v4u v[2];
  trace_ev(P, t, NSTAGE * l + S_COMB, TR_POLL);
  poll<2>(W.C, tag_of(epoch, l, S_ATT), voff, (int)(xbuf(par, W.x, B_PART) * 8), lane < NSPLIT, v);
  trace_ev(P, t, NSTAGE * l + S_COMB, TR_INPUT);
  const float m = lane < NSPLIT ? __uint_as_float(v[0].x) : -INFINITY;  // lanes >= 32 hold 0
  const float M = max16x(row16_max(m));  // over lanes 0-31
  const float e = (lane < NSPLIT && m != -INFINITY) ? __expf(m - M) : 0.f;
  const float Lt = half_sum(e * __uint_as_float(v[0].z));
  const float oa = half_sum(e * __uint_as_float(v[1].x));
  const float ob = half_sum(e * __uint_as_float(v[1].z));
  const float inv = Lt > 0.f ? __builtin_amdgcn_rcpf(Lt) : 0.f;  // v_rcp_f32 (1 ulp)
  if (lane == 0)
    ll_store_xcd(P.ws, xbuf(par, W.x, B_ATTO) + 4 * W.i + W.c, pack_h2(oa * inv, ob * inv), tag_of(epoch, l, S_COMB));
  drain_stores(S_COMB);
  trace_ev(P, t, NSTAGE * l + S_COMB, TR_STORE);
}

// o_proj partial of the XCD: rows [32 i + 8 c, +8) over the XCD's 256 attention dims
__device__ __forceinline__ void st_o(CW& W, const KParams& P, int t, int l, u32 epoch) {
  Shared* S = W.C.S;
  const int lane = W.lane, par = l & 1;
  trace_ev(P, t, NSTAGE * l + S_O, TR_POLL);
  const u32 n0 = W.gl;
  W.gl += LINES_O;
  v4u a;  // attention output values [8 (lane % 32), +8), fp16 as exchanged
  // line 4c + m holds rows 8c + 2m (lanes 0-31) and 8c + 2m + 1 (lanes 32-63); read into
  // registers (and released) while the wave waits for its input
  const u32 vb = ring_vbase(n0, lane);
  v4u wl[4];
  {
    const int voff[2] = {32 * (lane & 31), 32 * (lane & 31) + 16};
    v4u v[2];
    poll<2>(W.C, tag_of(epoch, l, S_COMB), voff, (int)(xbuf(par, W.x, B_ATTO) * 8), true, v,
            [&] {
      wait_lines(W, W.gl);
      trace_ev(P, t, NSTAGE * l + S_O, TR_LINES);
#pragma unroll
      for (int m = 0; m < 4; ++m) wl[m] = ring_ld(S, vb, 4 * W.c + m);
      release_lines(W, W.gl);
    });
    a = v4u{v[0].x, v[0].z, v[1].x, v[1].z};
  }
  trace_ev(P, t, NSTAGE * l + S_O, TR_INPUT);
  float part[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) part[m] = dot8h(wl[m], a);
  // y0 rows: (line 0 lo, line 1 lo, line 0 hi, line 1 hi) = rows 8c + (0, 2, 1, 3); y1 = +4
  const float y0 = row16_sum(pack16(part[0], part[1])), y1 = row16_sum(pack16(part[2], part[3]));
  if ((lane & 15) == 0) {
    const int r = 8 * W.c + reduce8_row(lane);
    const long base = xbuf(par, W.x, B_OP) + HROWS * W.i;
    ll_store(P.ws, base + r, __float_as_uint(y0), tag_of(epoch, l, S_O));
    ll_store(P.ws, base + r + 4, __float_as_uint(y1), tag_of(epoch, l, S_O));
  }
  drain_stores(S_O);
  trace_ev(P, t, NSTAGE * l + S_O, TR_STORE);
}

// sum of the 8 per-XCD partials plus the residual: compute wave c owns rows
// [32 i + 8 c, +8) and their fp32 residual; `src` is B_OP (o_proj, producing the
// post-attention residual) or B_DP (down, producing the next layer's residual)
__device__ __forceinline__ void st_sum(CW& W, const KParams& P, int t, int l, u32 epoch, bool is_down) {
  Shared* S = W.C.S;
  const int lane = W.lane, par = l & 1;
  const int st = is_down ? S_DSUM : S_OSUM;
  const int pr = lane & 3;  // rows 8 c + 2 pr, +1
  trace_ev(P, t, NSTAGE * l + st, TR_POLL);
  // the input residual of the rows (this wave wrote it), read before the wait
  float* res = is_down ? S->actres : S->resid;
  float* out = is_down ? S->resid : S->actres;
  const float2 rv = *(const float2*)(res + 8 * W.c + 2 * pr);
  float y0, y1;
  {  // lanes 0-31: XCD lane / 4, rows 8 c + 2 pr, +1
    const long src0 = xbuf(par, 0, is_down ? B_DP : B_OP) + HROWS * W.i + 8 * W.c;
    const int voff[1] = {(int)(((long)((lane >> 2) & 7) * XCD_SLOTS + 2 * pr) * 8)};
    v4u v[1];
    poll<1>(W.C, tag_of(epoch, l, is_down ? S_DOWN : S_O), voff, (int)(src0 * 8), lane < 32, v);
    y0 = __uint_as_float(v[0].x);  // lanes 32-63 hold 0
    y1 = __uint_as_float(v[0].z);
  }
  trace_ev(P, t, NSTAGE * l + st, TR_INPUT);
  // over the 8 XCDs: lanes pr + 4 g (g = 0..3 in each 16-lane row), then rows 0 + 1
  y0 += dpp<ROR8>(y0);
  y1 += dpp<ROR8>(y1);
  y0 += dpp<ROR4>(y0);
  y1 += dpp<ROR4>(y1);
  y0 = pack16(y0, y0);
  y1 = pack16(y1, y1);
  if (lane < 4) {
    const int r = 8 * W.c + 2 * pr;
    const float s0 = y0 + rv.x, s1 = y1 + rv.y;
    *(float2*)(out + r) = make_float2(s0, s1);
    const int row = HROWS * W.i + r;
    if (P.mode == MODE_MLP) {
      if (W.x == 0) *(float2*)(P.out_vec + row) = make_float2(s0, s1);
    } else {
      ll_store_xcd(P.ws, xbuf(par, W.x, is_down ? B_X : B_ACT) + row / 2, pack_h2(s0, s1), tag_of(epoch, l, st));
      if (is_down && l == P.num_layers - 1 && W.x == 0) {  // final-layer residual
        if (P.hidden_steps) *(float2*)(P.hidden_steps + (long)t * HIDDEN + row) = make_float2(s0, s1);
        const h2 ho = {(_Float16)s0, (_Float16)s1};
        *(h2*)(P.hidden_out + row) = ho;
      }
    }
  }
  drain_stores(st);
  trace_ev(P, t, NSTAGE * l + st, TR_STORE);
}

// gate/up rows 384 x + 12 i + 3 c + {0, 1, 2} -> SiLU(gate) * up
__device__ __forceinline__ void st_gu(CW& W, const KParams& P, int t, int l, u32 epoch) {
  Shared* S = W.C.S;
  const int lane = W.lane, par = l & 1;
  trace_ev(P, t, NSTAGE * l + S_GU, TR_POLL);
  const u32 n0 = W.gl;  // lines n0, n0 + 1: post-attention norm weights; then gate rows, up rows
  W.gl += LINES_GU;
  float xa[8], xb[8], ss;
  const u32 vb = ring_vbase(n0, lane);
  constexpr int ng = LINES_NORM;
  // norm weights, then gate rows (wl[ng + 2 jj ..]) and up rows (wl[ng + 6 + 2 jj ..]),
  // read into registers (and released) while the wave waits for its input
  v4u wl[ng + 12];
  auto lines = [&] {
    wait_lines(W, W.gl);
    trace_ev(P, t, NSTAGE * l + S_GU, TR_LINES);
    wl[0] = ring_ld(S, vb, 0);
    wl[1] = ring_ld(S, vb, 1);
#pragma unroll
    for (int jj = 0; jj < 3; ++jj) {
      wl[ng + 2 * jj] = ring_ld(S, vb, ng + 2 * (3 * W.c + jj));
      wl[ng + 2 * jj + 1] = ring_ld(S, vb, ng + 2 * (3 * W.c + jj) + 1);
      wl[ng + 6 + 2 * jj] = ring_ld(S, vb, ng + 2 * GU_PER_WG + 2 * (3 * W.c + jj));
      wl[ng + 6 + 2 * jj + 1] = ring_ld(S, vb, ng + 2 * GU_PER_WG + 2 * (3 * W.c + jj) + 1);
    }
    release_lines(W, W.gl);
  };
  if (P.mode == MODE_MLP) {
    ss = load_x1024(P.in_vec, lane, xa, xb);
    if (lane < 8) S->actres[8 * W.c + lane] = (float)P.in_vec[HROWS * W.i + 8 * W.c + lane];
    lines();
  } else {
    ss = poll_x1024(W, tag_of(epoch, l, S_OSUM), xbuf(par, W.x, B_ACT), xa, xb, lines);
  }
  trace_ev(P, t, NSTAGE * l + S_GU, TR_INPUT);
  float a[8], b[8];
  gain_act(xa, xb, __builtin_bit_cast(h8, wl[0]), __builtin_bit_cast(h8, wl[1]), a, b);
  float part[6];
#pragma unroll
  for (int jj = 0; jj < 3; ++jj) {
    part[jj] = row2k_r(wl[ng + 2 * jj], wl[ng + 2 * jj + 1], a, b);              // gate
    part[3 + jj] = row2k_r(wl[ng + 6 + 2 * jj], wl[ng + 6 + 2 * jj + 1], a, b);  // up
  }
  float pq, qq;
  reduce6(part, pq, qq);  // pq rows: gate0, gate1, up0, up1; qq rows: gate2, gate2, up2, up2
  const float rstd = rstd_of(ss);
  pq *= rstd;
  qq *= rstd;
  const float g0 = bcast(pq, 0), g1 = bcast(pq, 16), u0 = bcast(pq, 32), u1 = bcast(pq, 48);
  const float g2 = bcast(qq, 0), u2 = bcast(qq, 32);
  // SiLU(g) * u with v_rcp_f32 (1 ulp) in place of an IEEE divide
  const float s0 = g0 * __builtin_amdgcn_rcpf(1.0f + __expf(-g0)) * u0;
  const float s1 = g1 * __builtin_amdgcn_rcpf(1.0f + __expf(-g1)) * u1;
  const float s2 = g2 * __builtin_amdgcn_rcpf(1.0f + __expf(-g2)) * u2;
  if (lane < 2)
    ll_store_xcd(P.ws, xbuf(par, W.x, B_INT) + int_slot(W.i, W.c, lane), lane == 0 ? pack_h2(s0, s1) : pack_h2(s2, 0.f),
             tag_of(epoch, l, S_GU));
  drain_stores(S_GU);
  trace_ev(P, t, NSTAGE * l + S_GU, TR_STORE);
}

// down partial of the XCD: rows [32 i + 8 c, +8) over the XCD's 384 inter values
__device__ __forceinline__ void st_down(CW& W, const KParams& P, int t, int l, u32 epoch) {
  Shared* S = W.C.S;
  const int lane = W.lane, par = l & 1;
  trace_ev(P, t, NSTAGE * l + S_DOWN, TR_POLL);
  const u32 n0 = W.gl;
  W.gl += LINES_DOWN;
  v4u a;
  const u32 vb = ring_vbase(n0, lane);
  v4u wl[8];  // the wave's 8 lines, read into registers (and released) while it waits for its input
  {
    // wave c polls slot pairs k = 32 c + lane (lanes < 32): workgroup k / 4, wave k % 4 ->
    // inter values 12 (k / 4) + 3 (k % 4) + {0, 1, 2} (the pair's last half is padding),
    // gathered in S->xs; lanes 0-47 then own inter values [8 lane, 8 lane + 8)
    const int voff[1] = {16 * lane};
    v4u v[1];
    poll<1>(W.C, tag_of(epoch, l, S_GU), voff, (int)((xbuf(par, W.x, B_INT) + 64 * W.c) * 8), lane < 32, v,
            [&] {
      wait_lines(W, W.gl);
      trace_ev(P, t, NSTAGE * l + S_DOWN, TR_LINES);
#pragma unroll
      for (int r = 0; r < 8; ++r) wl[r] = ring_ld(S, vb, 8 * W.c + r);
      release_lines(W, W.gl);
    });
    if (lane < 32) {
      const int k = 32 * W.c + lane;
      float* dst = S->xs + GU_PER_WG * (k >> 2) + 3 * (k & 3);
      dst[0] = lo_h(v[0].x);
      dst[1] = hi_h(v[0].x);
      dst[2] = lo_h(v[0].z);
    }
    sync4(W);
    const int o = lane < 48 ? 8 * lane : 0;
    const float4 a0 = *(const float4*)(S->xs + o), a1 = *(const float4*)(S->xs + o + 4);
    // back to the fp16 values they were exchanged as (exact); lanes 48-63 contribute nothing
    const h8 ah = {(_Float16)a0.x, (_Float16)a0.y, (_Float16)a0.z, (_Float16)a0.w,
                   (_Float16)a1.x, (_Float16)a1.y, (_Float16)a1.z, (_Float16)a1.w};
    a = lane < 48 ? __builtin_bit_cast(v4u, ah) : v4u{0, 0, 0, 0};
  }
  trace_ev(P, t, NSTAGE * l + S_DOWN, TR_INPUT);
  float part[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) part[r] = dot8h(wl[r], a);
  float y0, y1;
  reduce8(part, y0, y1);
  if ((lane & 15) == 0) {
    const int r = 8 * W.c + reduce8_row(lane);
    const long base = xbuf(par, W.x, B_DP) + HROWS * W.i;
    ll_store(P.ws, base + r, __float_as_uint(y0), tag_of(epoch, l, S_DOWN));
    ll_store(P.ws, base + r + 4, __float_as_uint(y1), tag_of(epoch, l, S_DOWN));
  }
  drain_stores(S_DOWN);
  trace_ev(P, t, NSTAGE * l + S_DOWN, TR_STORE);
}

// lm_head input: final RMSNorm of the all-gathered residual (decode) or the caller's vector
__device__ __forceinline__ void st_lm_input(CW& W, const KParams& P, int t, u32 epoch) {
  Shared* S = W.C.S;
  const int lane = W.lane, L = P.num_layers;
  if (P.mode == MODE_LMHEAD) {
    const int o = 256 * W.c + 4 * lane;
    const h4 v = *(const h4*)(P.in_vec + o);
    *(float4*)(S->xfin + o) = make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
  } else {
    // every wave normalises the whole vector and stores it (identical values)
    const h8 w0 = *(const h8*)(P.final_norm + 8 * lane), w1 = *(const h8*)(P.final_norm + 512 + 8 * lane);
    trace_ev(P, t, NSTAGE * L, TR_POLL);
    float xa[8], xb[8], a[8], b[8];
    const float ss = poll_x1024(W, tag_of(epoch, L - 1, S_DSUM), xbuf((L - 1) & 1, W.x, B_X), xa, xb, NoPre());
    trace_ev(P, t, NSTAGE * L, TR_INPUT);
    norm_act(xa, xb, rstd_of(ss), w0, w1, a, b);
    *(float4*)(S->xfin + 8 * lane) = make_float4(a[0], a[1], a[2], a[3]);
    *(float4*)(S->xfin + 8 * lane + 4) = make_float4(a[4], a[5], a[6], a[7]);
    *(float4*)(S->xfin + 512 + 8 * lane) = make_float4(b[0], b[1], b[2], b[3]);
    *(float4*)(S->xfin + 512 + 8 * lane + 4) = make_float4(b[4], b[5], b[6], b[7]);
    if (W.w == 0 && W.c == 0) {
      *(float4*)(P.norm_out + 8 * lane) = make_float4(a[0], a[1], a[2], a[3]);
      *(float4*)(P.norm_out + 8 * lane + 4) = make_float4(a[4], a[5], a[6], a[7]);
      *(float4*)(P.norm_out + 512 + 8 * lane) = make_float4(b[0], b[1], b[2], b[3]);
      *(float4*)(P.norm_out + 512 + 8 * lane + 4) = make_float4(b[4], b[5], b[6], b[7]);
    }
  }
  lds_release();
  if (lane == 0) __hip_atomic_fetch_add(&S->xfin_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void compute_wave(const KParams& P, Shared* S, int c) {
  CW W;
  W.C.P = &P;
  W.C.S = S;
  W.C.r = ws_rsrc(P.ws);
  W.C.ok = true;
  W.C.deadline = P.deadline;
  W.w = blockIdx.x;
  W.x = xcd_of(W.w);
  W.i = loc_of(W.w);
  W.c = c;
  W.lane = __lane_id();
  W.nsync = 0;
  W.gl = 0;
  const int L = P.num_layers;
  int token = P.first_token;
  u32 phase = 0;
  for (int t = 0; t < P.num_steps && W.C.ok; ++t) {
    const u32 epoch = P.epoch0 + (u32)t;
    if (P.mode == MODE_MLP) {
      st_gu(W, P, t, 0, epoch);
      st_down(W, P, t, 0, epoch);
      st_sum(W, P, t, 0, epoch, true);
      break;
    }
    if (P.mode == MODE_DECODE) {
      for (int l = 0; l < L && W.C.ok; ++l) {
        st_qkv(W, P, t, l, epoch, token);
        st_att(W, P, t, l, epoch);
        st_comb(W, P, t, l, epoch);
        st_o(W, P, t, l, epoch);
        st_sum(W, P, t, l, epoch, false);
        st_gu(W, P, t, l, epoch);
        st_down(W, P, t, l, epoch);
        st_sum(W, P, t, l, epoch, true);
      }
      if (!W.C.ok) break;
    }
    st_lm_input(W, P, t, epoch);
    ++phase;
    lm_rows(W.C, P, c, t, phase, epoch);
    trace_ev(P, t, NSTAGE * L, TR_SYNC);
    // workgroup partial -> ARG slots; every workgroup then reduces all 256
    if (c == 0) {
      lds_wait_ge(W.C, &S->lm_cnt, (NCW + NLW) * phase);
      float best = -INFINITY;
      int bidx = 0x7fffffff;
#pragma unroll
      for (int v = 0; v < NCW + NLW; ++v) better(best, bidx, S->lmv[v], S->lmi[v]);
      if (W.w == 0 && W.lane < LM_NGRP) {  // set up the pool counters of tokens epoch + 2, epoch + 3
#pragma unroll
        for (u32 d = 2; d < 4; ++d)
          __hip_atomic_store(lm_pool_ctr(P, epoch + d, W.lane), (u64)(epoch + d) << 32, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
      if (W.lane == 0) {
        const u32 tg = tag_arg(epoch);
        ll_store(P.ws, slot_arg(t & 1, 2 * W.w), __float_as_uint(best), tg);
        ll_store(P.ws, slot_arg(t & 1, 2 * W.w + 1), (u32)bidx, tg);
      }
    }
    {
      const int voff[1] = {16 * W.lane};
      v4u v[1];
      poll<1>(W.C, tag_arg(epoch), voff, (int)(slot_arg(t & 1, 128 * c) * 8), true, v);
      trace_ev(P, t, NSTAGE * L, TR_LINES);
      float best = __uint_as_float(v[0].x);
      int bidx = (int)v[0].z;
      wave_argmax(best, bidx);
      if (W.lane == 0) {
        S->argv[c] = best;
        S->argi[c] = bidx;
      }
      sync4(W);
      best = -INFINITY;
      bidx = 0x7fffffff;
#pragma unroll
      for (int cc = 0; cc < NCW; ++cc) better(best, bidx, S->argv[cc], S->argi[cc]);
      if (bidx < 0 || bidx >= VOCAB) bidx = 0;  // every logit NaN
      if (W.w == 0 && c == 0 && W.lane == 0) P.out_tokens[t] = bidx;
      trace_ev(P, t, NSTAGE * L, TR_STORE);
      // every workgroup reduced the same 256 partials, so all of them stop at the same step
      const bool stop = bidx == P.eos;
      if (P.out_count && W.w == 0 && c == 0 && W.lane == 0 && (stop || t + 1 == P.num_steps)) *P.out_count = t + 1;
      token = (P.forced && t + 1 < P.num_steps) ? P.forced[t + 1] : bidx;
      // the loader waves wait for ring space in the next step: the workgroup's abort flag
      // (set below) ends that wait, and they leave without a device-side error
      if (stop) W.C.ok = false;
      if (token < 0 || token >= VOCAB) {  // a forced id out of range: report and stop
        __hip_atomic_fetch_or(P.status, ST_BAD_TOKEN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        W.C.ok = false;
      }
    }
  }
  if (!W.C.ok) lds_st(&S->abort, 1u);
}

// ------------------------------------------------------------------------------------
// loader waves: every ring line of every stage in execution order; wave q
// handles the lines n == q (mod 4). Each stage is one or two streams of lines
// whose 16-byte piece for lane `lane` is at base + m * stride + loff: the
// weight rows a workgroup reads are contiguous per stage (QKV: 16 rows of one
// matrix; gate, up: 12 rows each) or evenly strided (o_proj: 2 rows of 512 B
// per line; down: one 768-byte row segment per line), and 4 positions of one
// kv head are 1 KB of contiguous K (or V) cache.

struct Stream {
  const char* base;  // this lane's first byte of line 0
  long stride;       // bytes between lines
  int n;             // lines
  int vlim;          // K/V streams: lane's position index 4 m + lane / 16 must be < vlim
};

__device__ __forceinline__ Stream make_stream(const KParams& P, const Shared* S, int si, int l, int x, int i, int pos,
                                              int ctx, int lane) {
  const LDGLayerWeight& lw = S->lw[l];
  const StreamGeom g = stream_geom(si, x, i, ctx, pos, lane);
  const long kv = ((long)l * NKV + x) * P.max_seq * HD;
  const void* M;
  switch (g.mat) {  // lane-uniform except for the attention-vector line
    case 0: M = lw.q_proj_weight; break;
    case 1: M = lw.k_proj_weight; break;
    case 2: M = lw.v_proj_weight; break;
    case 3: M = P.k_cache + kv; break;
    case 4: M = P.v_cache + kv; break;
    case 5: M = lw.o_proj_weight; break;
    case 6: M = lw.gate_proj_weight; break;
    case 7: M = lw.up_proj_weight; break;
    case 8: M = lw.down_proj_weight; break;
    case 9: M = lw.input_layernorm_weight; break;
    case 10: M = lw.post_attn_layernorm_weight; break;
    case 11: M = lw.q_norm_weight; break;
    case 12: M = lw.k_norm_weight; break;
    case 13: M = P.cos_t; break;
    default: M = P.sin_t; break;
  }
  Stream st;
  st.base = (const char*)((const _Float16*)M + g.elem0 + g.loff);
  st.stride = g.stride * 2;
  st.n = g.n;
  st.vlim = g.vlim;
  return st;
}

__device__ __forceinline__ u32 cons_min(const Shared* S) {
  const u32 a = lds_ld(&S->cons[0]), b = lds_ld(&S->cons[1]);
  const u32 c = lds_ld(&S->cons[2]), d = lds_ld(&S->cons[3]);
  return min(min(a, b), min(c, d));
}

__device__ __forceinline__ void loader_wave(const KParams& P, Shared* S, int q) {
  Ctl C;
  C.P = &P;
  C.S = S;
  C.r = ws_rsrc(P.ws);
  C.ok = true;
  C.deadline = P.deadline;
  const int w = blockIdx.x, x = xcd_of(w), i = loc_of(w), lane = __lane_id();
  const int L = P.num_layers;
  // lanes without a cached position read the embedding's first row instead, so every
  // DMA covers all 64 lanes and no line of an unwritten position is ever cached
  const char* spare = (const char*)P.embed + 16 * lane;
  u32 gl = 0;     // global index of the next stream's first line
  u32 avail = 0;  // lines below this may be written (compute waves released their slots)
  u32 phase = 0;
  for (int t = 0; t < P.num_steps && C.ok; ++t) {
    const int pos = P.start_pos + t, ctx = pos + 1;
    if (P.mode != MODE_LMHEAD) {
      u32 last = 0;     // last line issued
      int pending = 0;  // lines issued whose completion is not yet published
      const int nl = P.mode == MODE_MLP ? 1 : L;
      const int s0 = P.mode == MODE_MLP ? MLP_FIRST_STREAM : 0;
      for (int l = 0; l < nl && C.ok; ++l) {
        for (int si = s0; si < NSTREAM && C.ok; ++si) {
          const Stream st = make_stream(P, S, si, l, x, i, pos, ctx, lane);
          const char* src = st.base;
          int m = (int)((u32)(q - (int)gl) & 3u);
          src += (long)m * st.stride;
          for (; m < st.n; m += 4, src += 4 * st.stride) {
            const u32 n = gl + (u32)m;
            if (n >= avail) {
              avail = cons_min(S) + RING_LINES;
              if (n >= avail) {
                // publish everything issued before waiting, so the compute waves can release lines
                wait_vmcnt<0>();
                if (pending > 0) lds_st(&S->done_upto[q], last + 4);
                pending = 0;
                u64 t0 = wall_clock64();
                int spins = 0;
                while (n >= (avail = cons_min(S) + RING_LINES)) {
                  if (give_up(C, t0, spins)) {
                    C.ok = false;
                    break;
                  }
                  __builtin_amdgcn_s_sleep(1);
                }
                if (!C.ok) break;
                lds_acquire();
              }
            }
            const bool cached = 4 * m + (lane >> 4) < st.vlim;
            dma16(cached ? src : spare, __builtin_amdgcn_readfirstlane((n % RING_LINES) * LINE_BYTES));
            last = n;
            if (++pending > DMA_DEPTH) {
              // all but the newest DMA_DEPTH lines of this wave are in LDS
              wait_vmcnt<DMA_DEPTH>();
              lds_st(&S->done_upto[q], n - 4 * DMA_DEPTH + 4);
              pending = DMA_DEPTH;
            }
          }
          gl += (u32)st.n;
        }
      }
      wait_vmcnt<0>();
      if (pending > 0) lds_st(&S->done_upto[q], last + 4);
    }
    if (P.mode == MODE_MLP || !C.ok) break;
    ++phase;
    lm_rows(C, P, NCW + q, t, phase, P.epoch0 + (u32)t);
    if (q == 0) trace_ev(P, t, NSTAGE * L, TR_MERGE);
  }
  if (!C.ok) lds_st(&S->abort, 1u);
}

__global__ void __launch_bounds__(BLOCK, 1) qwen_decode_kernel(KParams P) {
  __shared__ Shared S;
  // wave index is uniform per wave; readfirstlane lets the compiler keep it (and
  // every address derived from it) in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  if (threadIdx.x == 0) {
    S.sync = 0;
    S.xfin_cnt = 0;
    S.lm_cnt = 0;
    S.lm_next[0] = 0;
    S.lm_next[1] = 0;
    S.lm_pool_done[0] = 0;
    S.lm_pool_done[1] = 0;
    S.abort = 0;
  }
  if (threadIdx.x < NLW) S.done_upto[threadIdx.x] = threadIdx.x;
  if (threadIdx.x < NCW) S.cons[threadIdx.x] = 0;
  // (the isolated lm_head workload has no layers and passes no table)
  if (P.mode != MODE_LMHEAD && threadIdx.x < P.num_layers * 12) {
    const u64* src = (const u64*)P.layers;
    ((u64*)S.lw)[threadIdx.x] = src[threadIdx.x];
  }
  __syncthreads();
  if (wave < NCW)
    compute_wave(P, &S, wave);
  else
    loader_wave(P, &S, wave - NCW);
}

// ------------------------------------------------------------------------------------
// host side

namespace {

constexpr int MAX_DEVICES = 16;

struct DeviceState {
  bool init = false;
  int err = QWEN_OK;
  u64* ws = nullptr;
  u32* status = nullptr;
  u32 epoch = 1;
  u64 deadline = 0;
  u64* trace = nullptr;
  int trace_token = -1;
};

std::mutex g_mu;
DeviceState g_dev[MAX_DEVICES];

int device_state(DeviceState** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return QWEN_ERR_DEVICE;
  DeviceState& st = g_dev[dev];
  if (!st.init) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return QWEN_ERR_DEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || prop.multiProcessorCount != NWG || !prop.cooperativeLaunch) {
      fprintf(stderr, "qwen_megakernel: needs a 256-CU gfx950 device with cooperative launch (got %s, %d CUs)\n",
              prop.gcnArchName, prop.multiProcessorCount);
      st.err = QWEN_ERR_DEVICE;
      st.init = true;
      return st.err;
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)qwen_decode_kernel, BLOCK, 0) != hipSuccess ||
        occ < 1) {
      st.err = QWEN_ERR_DEVICE;
      st.init = true;
      return st.err;
    }
    int clk_khz = 0;
    if (hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || clk_khz <= 0)
      clk_khz = 100000;
    st.deadline = (u64)clk_khz * 500;  // 0.5 s per single wait
    void* p = nullptr;
    if (hipMalloc(&p, WORKSPACE_BYTES) != hipSuccess) return QWEN_ERR_LAUNCH;
    if (hipMemset(p, 0, WORKSPACE_BYTES) != hipSuccess) return QWEN_ERR_LAUNCH;
    st.ws = (u64*)p;
    st.status = (u32*)((char*)p + TOTAL_SLOTS * 8);
    st.init = true;
  }
  if (st.err != QWEN_OK) return st.err;
  *out = &st;
  return QWEN_OK;
}

int launch(KParams& P, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  P.ws = st->ws;
  P.status = st->status;
  P.deadline = st->deadline;
  P.trace = st->trace;
  P.trace_token = st->trace_token;
  P.epoch0 = st->epoch;
  // epochs are 24-bit in the tag; wrap back to 1 (never 0: a zeroed slot is never "ready")
  u64 next = (u64)st->epoch + (u64)P.num_steps + 1;
  if (next >= (1u << 24)) {
    if (hipMemsetAsync(st->ws, 0, TOTAL_SLOTS * 8, stream) != hipSuccess) return QWEN_ERR_LAUNCH;
    P.epoch0 = 1;
    next = 1 + (u64)P.num_steps + 1;
  }
  st->epoch = (u32)next;
  void* args[] = {&P};
  if (hipLaunchCooperativeKernel((const void*)qwen_decode_kernel, dim3(NWG), dim3(BLOCK), args, 0, stream) != hipSuccess)
    return QWEN_ERR_LAUNCH;
  return QWEN_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

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
  if (cache_len != position + 1) return QWEN_ERR_ARG;
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

extern "C" int qwen_mlp_block(const void* x_f16, const void* post_norm_weight, const void* gate_weight,
                              const void* up_weight, const void* down_weight, float* y_out, hipStream_t stream) {
  if (!x_f16 || !post_norm_weight || !gate_weight || !up_weight || !down_weight || !y_out) return QWEN_ERR_ARG;
  if (!aligned16(x_f16) || !aligned16(post_norm_weight) || !aligned16(gate_weight) || !aligned16(up_weight) ||
      !aligned16(down_weight) || !aligned16(y_out))
    return QWEN_ERR_ARG;
  // the kernel reads the layer pointer table from device memory
  static LDGLayerWeight* d_tab[MAX_DEVICES] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return QWEN_ERR_DEVICE;
  LDGLayerWeight h;
  memset(&h, 0, sizeof(h));
  h.post_attn_layernorm_weight = post_norm_weight;
  h.gate_proj_weight = gate_weight;
  h.up_proj_weight = up_weight;
  h.down_proj_weight = down_weight;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!d_tab[dev] && hipMalloc(&d_tab[dev], sizeof(LDGLayerWeight)) != hipSuccess) return QWEN_ERR_LAUNCH;
  }
  if (hipMemcpyAsync(d_tab[dev], &h, sizeof(h), hipMemcpyHostToDevice, stream) != hipSuccess) return QWEN_ERR_LAUNCH;
  if (hipStreamSynchronize(stream) != hipSuccess) return QWEN_ERR_LAUNCH;
  KParams P;
  memset(&P, 0, sizeof(P));
  P.eos = -1;
  P.layers = d_tab[dev];
  P.in_vec = (const _Float16*)x_f16;
  P.out_vec = y_out;
  P.mode = MODE_MLP;
  P.num_layers = 1;
  P.num_steps = 1;
  P.max_seq = MAX_SEQ_LIMIT;
  return launch(P, stream);
}

extern "C" int qwen_last_error(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return QWEN_ERR_DEVICE;
  DeviceState& st = g_dev[dev];
  if (!st.init) return QWEN_OK;
  if (st.err != QWEN_OK) return st.err;
  if (hipDeviceSynchronize() != hipSuccess) return QWEN_ERR_LAUNCH;
  u32 s = 0;
  if (hipMemcpy(&s, st.status, sizeof(s), hipMemcpyDeviceToHost) != hipSuccess) return QWEN_ERR_LAUNCH;
  if (s == 0) return QWEN_OK;
  // a failed launch leaves slots in an unknown state: start clean
  if (hipMemset(st.ws, 0, WORKSPACE_BYTES) != hipSuccess) return QWEN_ERR_LAUNCH;
  st.epoch = 1;
  return QWEN_ERR_TIMEOUT;
}

extern "C" int qwen_abi_version(void) { return QWEN_ABI_VERSION; }

extern "C" int qwen_set_trace(unsigned long long* buf, int token) {
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState* st = nullptr;
  int rc = device_state(&st);
  if (rc != QWEN_OK) return rc;
  st->trace = buf;
  st->trace_token = buf ? token : -1;
  return QWEN_OK;
}

extern "C" int qwen_trace_events(void) { return TRACE_EVENTS; }
