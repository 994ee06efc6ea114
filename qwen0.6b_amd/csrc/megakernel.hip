// Qwen3-0.6B batch-1 decode engine for MI355X (gfx950): one cooperative,
// persistent kernel runs whole token steps (embedding, 28 layers, final norm,
// tied lm_head, argmax) and, in generate mode, feeds each argmax back as the
// next step's input without returning to the host.
//
// Design (measured on MI355X before it was written):
//  * one 576-thread workgroup per CU (256), fixed work partition (qwen_layout.h);
//  * no grid barrier: every inter-workgroup hand-off is an exchange buffer of
//    8-byte slots carrying payload + step tag, written with device-scope (sc1)
//    stores and polled with device-scope loads. A release/acquire grid barrier
//    measured 8.3 us per crossing on this part; a tagged-slot hand-off costs
//    one store->load visibility latency (~0.6 us);
//  * wave specialisation: waves 0-7 stream weights with nontemporal 16-B loads
//    issued two stages ahead into registers; wave 8 (the exchange wave) polls
//    the next stage's input, applies the vector work (RMSNorm, q/k norm, RoPE,
//    KV-cache write, split-K softmax merge, argmax) and hands it over in LDS.
//    Loads retire in order per wave, so polling from a weight-streaming wave
//    would wait behind its own prefetches; a separate wave does not;
//  * inside a workgroup, the 8 compute waves meet through LDS counters (last
//    arriver finalises), never s_barrier, so the exchange wave runs free;
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
typedef u32 v2u __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr float RMS_EPS = 1e-6f;
constexpr u32 ST_TIMEOUT = 1u;
constexpr u32 ST_BAD_TOKEN = 2u;
// optional device timestamps (wall clock) per workgroup and finalised stage of one token
constexpr int TRACE_EVENTS = 8;
enum TraceEvent : int {
  TR_POLL = 0,     // exchange wave starts waiting for the stage input
  TR_PUBLISH = 1,  // stage input handed to the compute waves
  TR_FINAL = 2,    // stage results stored
  TR_COMBINE = 3,  // attention merge stored / argmax known
  TR_CSTART = 4,   // compute wave 0 of the stage's group saw the input
  TR_CDONE = 5,    // compute wave 0 of the stage's group finished the stage
  TR_FSTART = 6,   // the finalising wave starts finalising
};

struct KParams {
  const _Float16* embed;
  const LDGLayerWeight* layers;
  const _Float16* final_norm;
  const _Float16* lm_head;
  const _Float16* cos_t;
  const _Float16* sin_t;
  _Float16* k_cache;
  _Float16* v_cache;
  _Float16* hidden_out;  // [1024] fp16
  float* norm_out;       // [1024] fp32
  int* out_tokens;       // [num_steps]
  const int* forced;     // nullable [num_steps]
  float* logits_out;     // nullable [num_steps][VOCAB]
  float* hidden_steps;   // nullable [num_steps][HIDDEN]
  const _Float16* in_vec;  // MODE_LMHEAD / MODE_MLP input [1024]
  float* out_vec;          // MODE_MLP output [1024]
  u64* ws;                 // exchange slots
  u32* status;             // status word (device scope)
  u64 deadline;            // wall-clock ticks a single wait may take
  u64* trace;              // nullable [NWG][fins per token][TRACE_EVENTS]
  int trace_token;         // token index whose stages are traced
  int mode, num_layers, first_token, start_pos, num_steps, max_seq;
  float attn_scale;
  u32 epoch0;
};

// ------------------------------------------------------------------------------------
// small device helpers

__device__ __forceinline__ v4u ld_nt(const _Float16* p) { return __builtin_nontemporal_load((const v4u*)p); }
__device__ __forceinline__ v4u ld_plain(const _Float16* p) { return *(const v4u*)p; }

__device__ __forceinline__ float dot8(v4u w, const float* a) {
  h8 h = __builtin_bit_cast(h8, w);
  float4 a0 = *(const float4*)a;
  float4 a1 = *(const float4*)(a + 4);
  float s = (float)h[0] * a0.x;
  s = fmaf((float)h[1], a0.y, s);
  s = fmaf((float)h[2], a0.z, s);
  s = fmaf((float)h[3], a0.w, s);
  s = fmaf((float)h[4], a1.x, s);
  s = fmaf((float)h[5], a1.y, s);
  s = fmaf((float)h[6], a1.z, s);
  s = fmaf((float)h[7], a1.w, s);
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
// every lane: sum of its 16-lane row
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<ROR8>(v);
  v += dpp<ROR4>(v);
  v += dpp<ROR2>(v);
  v += dpp<ROR1>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<ROR8>(v));
  v = fmaxf(v, dpp<ROR4>(v));
  v = fmaxf(v, dpp<ROR2>(v));
  v = fmaxf(v, dpp<ROR1>(v));
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
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max32x(float v) {  // max of the two 32-lane halves
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
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
// value of lane ^ 16 (the partner row at the same position)
__device__ __forceinline__ float xor16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return ((__lane_id() >> 4) & 1) ? __uint_as_float(r[0]) : __uint_as_float(r[1]);
}
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

__device__ __forceinline__ u32 pack_h2(float a, float b) {
  h2 h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(u32, h);
}
__device__ __forceinline__ float lo_h(u32 p) { return (float)__builtin_bit_cast(h2, p)[0]; }
__device__ __forceinline__ float hi_h(u32 p) { return (float)__builtin_bit_cast(h2, p)[1]; }

__device__ __forceinline__ void ll_store(u64* ws, long slot, u32 payload, u32 tag) {
  __hip_atomic_store(ws + slot, ((u64)tag << 32) | (u64)payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(const u64* ws) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)ws, 0, 0x7fffffff, 0x00020000);
}
// one 16-byte device-scope (sc1) load of two slots at byte offset voff + soff
// (voff per lane, soff wave-uniform so it travels in the instruction's soffset)
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

// ------------------------------------------------------------------------------------
// workgroup shared state

struct Shared {
  float in[2][INTER];            // stage input prepared by the exchange wave (parity of fin)
  float red[2][NCW * 260];       // per-wave partial results (parity of fin)
  float xres[HID_PER_WG];        // residual rows before attention (fp32)
  float actres[HID_PER_WG];      // residual rows after attention (fp32)
  u32 ready;                     // fin + 1 of the newest prepared input
  u32 cnt[2];                    // compute-wave arrivals at the current fin of each parity
  u32 done[2];                   // fin + 1 of the newest finalised fin of each parity
  u32 abort;
};

// ------------------------------------------------------------------------------------
// exchange-wave polling

struct Poll {
  __amdgpu_buffer_rsrc_t r;
  const KParams* P;
  Shared* S;
  bool ok;
};

__device__ __forceinline__ bool poll_give_up(Poll& pl, u64 t0, int& spins) {
  ++spins;
  if ((spins & 15) == 0 && wall_clock64() - t0 > pl.P->deadline) {
    __hip_atomic_fetch_or(pl.P->status, ST_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  if ((spins & 255) == 0) {
    if (__hip_atomic_load(pl.P->status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return true;
  }
  return false;
}

__device__ __forceinline__ void xtrace(const KParams& P, int token, u32 fin_in_token, int what) {
  if (P.trace && token == P.trace_token && __lane_id() == 0) {
    const int FT = fins_per_token(P.mode, P.num_layers);
    P.trace[((long)blockIdx.x * FT + fin_in_token) * TRACE_EVENTS + what] = wall_clock64();
  }
}

// Polls K slot pairs per lane until both slots of every pair carry `tag`. Pair k
// of this lane starts at byte voff + soff_of(k) of the workspace; soff_of(k) must be
// wave-uniform. Lanes with active == false take no part.
template <int K, typename F>
__device__ __forceinline__ void poll_pairs(Poll& pl, u32 tag, int voff, bool active, F soff_of, v4u (&out)[K]) {
  if (!pl.ok) return;
  bool done[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    done[k] = !active;
    out[k] = v4u{0, 0, 0, 0};
  }
  const u64 t0 = wall_clock64();
  int spins = 0;
  for (;;) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (!done[k]) out[k] = ld_pair(pl.r, voff, soff_of(k));
    bool all = true;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (!done[k]) done[k] = (out[k].y == tag) && (out[k].w == tag);
      all = all && done[k];
    }
    if (__all(all)) return;
    if (poll_give_up(pl, t0, spins)) {
      pl.ok = false;
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// exchange wave: wait until fin - 2 (same parity) is finalised, so in[fin % 2] is free
__device__ __forceinline__ void wait_consumed(Poll& pl, u32 fin) {
  if (!pl.ok || fin < 2) return;
  const u64 t0 = wall_clock64();
  int spins = 0;
  while (lds_ld(&pl.S->done[fin & 1]) < fin - 1) {
    if (poll_give_up(pl, t0, spins)) {
      pl.ok = false;
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  lds_acquire();
}

__device__ __forceinline__ void publish(Poll& pl, u32 fin) {
  lds_release();
  if (__lane_id() == 0) lds_st(&pl.S->ready, fin + 1);
}

// RMS of the 16 values a lane holds as x[4(lane + 64 i) + j], i < 4, j < 4
__device__ __forceinline__ float rstd_1024(const float (&x)[16]) {
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) ss = fmaf(x[k], x[k], ss);
  ss = wave_sum(ss);
  return rsqrtf(ss * (1.0f / HIDDEN) + RMS_EPS);
}

// polls a 1024-value H2 vector (512 slots from slot `base`) into x[4(lane + 64 i) + j]
__device__ __forceinline__ void poll_vec1024(Poll& pl, u32 tag, long base, float (&x)[16]) {
  v4u v[4];
  const int lane = __lane_id();
  poll_pairs<4>(pl, tag, lin_voff(lane), true, [&](int k) -> int { return (int)lin_soff(base, k); }, v);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    x[4 * k + 0] = lo_h(v[k].x);
    x[4 * k + 1] = hi_h(v[k].x);
    x[4 * k + 2] = lo_h(v[k].z);
    x[4 * k + 3] = hi_h(v[k].z);
  }
}

// the lane's 16 norm weights w[4(lane + 64k) + j]; loaded before polling so the
// load overlaps the wait instead of following it
struct NormW {
  h4 v[4];
};
__device__ __forceinline__ NormW load_norm(const _Float16* w) {
  NormW n;
  const int lane = __lane_id();
#pragma unroll
  for (int k = 0; k < 4; ++k) n.v[k] = *(const h4*)(w + 4 * (lane + 64 * k));
  return n;
}
// in[i] = x[i] * rstd * w[i] for the lane's 16 values
__device__ __forceinline__ void store_normed(float* dst, const float (&x)[16], float rstd, const NormW& wv) {
  const int lane = __lane_id();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int i = 4 * (lane + 64 * k);
    float4 o = make_float4(x[4 * k] * rstd * (float)wv.v[k][0], x[4 * k + 1] * rstd * (float)wv.v[k][1],
                           x[4 * k + 2] * rstd * (float)wv.v[k][2], x[4 * k + 3] * rstd * (float)wv.v[k][3]);
    *(float4*)(dst + i) = o;
  }
}

// ------------------------------------------------------------------------------------
// exchange wave program

__device__ void exchange_wave(const KParams& P, Shared* S) {
  const int w = blockIdx.x;
  const int lane = __lane_id();
  Poll pl{ws_rsrc(P.ws), &P, S, true};
  const int L = P.num_layers;
  const int FT = fins_per_token(P.mode, L);

  if (P.mode == MODE_MLP) {
    const LDGLayerWeight& lw = P.layers[0];
    // GU input: x -> RMSNorm * post_norm; residual rows x[4w..4w+3]
    float x[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      h4 v = *(const h4*)(P.in_vec + 4 * (lane + 64 * k));
      for (int j = 0; j < 4; ++j) x[4 * k + j] = (float)v[j];
    }
    const float rs = rstd_1024(x);
    store_normed(S->in[0], x, rs, load_norm((const _Float16*)lw.post_attn_layernorm_weight));
    if (lane < HID_PER_WG) S->actres[lane] = (float)P.in_vec[HID_PER_WG * w + lane];
    publish(pl, 0);
    // DOWN input: SiLU(gate)*up from every workgroup
    wait_consumed(pl, 1);
    v4u v[12];
    poll_pairs<12>(pl, tag_of(P.epoch0, 0, SID_INT), lin_voff(lane), true,
                   [&](int k) -> int { return (int)lin_soff(slot_int(0, 0), k); }, v);
    if (!pl.ok) { S->abort = 1; return; }
#pragma unroll
    for (int k = 0; k < 12; ++k) {
      const int i = 4 * (lane + 64 * k);
      *(float4*)(S->in[1] + i) = make_float4(lo_h(v[k].x), hi_h(v[k].x), lo_h(v[k].z), hi_h(v[k].z));
    }
    publish(pl, 1);
    return;
  }

  if (P.mode == MODE_LMHEAD) {
    float x[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      h4 v = *(const h4*)(P.in_vec + 4 * (lane + 64 * k));
      for (int j = 0; j < 4; ++j) x[4 * k + j] = (float)v[j];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      *(float4*)(S->in[0] + 4 * (lane + 64 * k)) = make_float4(x[4 * k], x[4 * k + 1], x[4 * k + 2], x[4 * k + 3]);
    publish(pl, 0);
  }

  int token = P.first_token;
  for (int t = 0; t < P.num_steps; ++t) {
    const u32 epoch = P.epoch0 + (u32)t;
    const int pos = P.start_pos + t;
    if (P.mode == MODE_DECODE) {
      const int ctx = pos + 1;
      for (int l = 0; l < L; ++l) {
        const LDGLayerWeight& lw = P.layers[l];
        const int par = l & 1;
        u32 fin = (u32)(t * FT + 5 * l);
        // ---- QKV input: residual stream -> RMSNorm * input_layernorm
        wait_consumed(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_POLL);
        const NormW w_in = load_norm((const _Float16*)lw.input_layernorm_weight);
        float x[16];
        if (l == 0) {
          const _Float16* row = P.embed + (long)token * HIDDEN;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            h4 v = *(const h4*)(row + 4 * (lane + 64 * k));
            for (int j = 0; j < 4; ++j) x[4 * k + j] = (float)v[j];
          }
          if (lane < HID_PER_WG) S->xres[lane] = (float)row[HID_PER_WG * w + lane];
        } else {
          poll_vec1024(pl, tag_of(epoch, l - 1, SID_X), slot_x(par, 0), x);
        }
        if (!pl.ok) break;
        {
          const float rs = rstd_1024(x);
          store_normed(S->in[fin & 1], x, rs, w_in);
        }
        publish(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_PUBLISH);

        // ---- attention input: raw q (2 heads), k, v of kv head g -> norms, RoPE, KV write
        ++fin;
        wait_consumed(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_POLL);
        const int g = att_kv(w), s = att_split(w);
        {
          const int d0 = 4 * (lane & 31);
          const h4 cv = *(const h4*)(P.cos_t + (long)pos * HD + d0);
          const h4 sv = *(const h4*)(P.sin_t + (long)pos * HD + d0);
          const h4 qn = *(const h4*)((const _Float16*)lw.q_norm_weight + d0);
          const h4 kn = *(const h4*)((const _Float16*)lw.k_norm_weight + d0);
          v4u vq[1], vkv[1];
          // q slots 128g + 2 lane; k slots (lane < 32) or v slots (lane >= 32)
          poll_pairs<1>(pl, tag_of(epoch, l, SID_QKV), attq_voff(lane), true,
                        [&](int) -> int { return (int)attq_soff(par, g); }, vq);
          poll_pairs<1>(pl, tag_of(epoch, l, SID_QKV), attkv_voff(lane), true,
                        [&](int) -> int { return (int)attkv_soff(par, g); }, vkv);
          if (!pl.ok) break;
          // vq: q values 4 lane .. (q head 2g for lane < 32, 2g+1 above)
          // vkv: lane < 32: k dims 4 lane.., lane >= 32: v dims 4(lane-32)..
          float q[4] = {lo_h(vq[0].x), hi_h(vq[0].x), lo_h(vq[0].z), hi_h(vq[0].z)};
          float kv[4] = {lo_h(vkv[0].x), hi_h(vkv[0].x), lo_h(vkv[0].z), hi_h(vkv[0].z)};
          // q head norms (each 32-lane half is one head)
          float ssq = q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3];
          ssq = half_sum(ssq);
          const float rq = rsqrtf(ssq * (1.0f / HD) + RMS_EPS);
          float ssk = kv[0] * kv[0] + kv[1] * kv[1] + kv[2] * kv[2] + kv[3] * kv[3];
          ssk = half_sum(ssk);  // lanes < 32: k norm; lanes >= 32: unused (v)
          const float rk = rsqrtf(ssk * (1.0f / HD) + RMS_EPS);
          float qq[4], kk[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            qq[j] = q[j] * rq * (float)qn[j];
            kk[j] = kv[j] * rk * (float)kn[j];
          }
          // rotate-half RoPE: partner dims d +- 64 live in lane ^ 16
          const bool lo_half = (lane & 31) < 16;
          float qo[4], ko[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float qp = xor16(qq[j]);
            const float kp = xor16(kk[j]);
            const float c = (float)cv[j], sgn = lo_half ? -(float)sv[j] : (float)sv[j];
            qo[j] = qq[j] * c + qp * sgn;
            ko[j] = kk[j] * c + kp * sgn;
          }
          float* in = S->in[fin & 1];
          *(float4*)(in + 4 * lane) = make_float4(qo[0], qo[1], qo[2], qo[3]);  // q0r | q1r
          if (lane < 32)
            *(float4*)(in + 256 + 4 * lane) = make_float4(ko[0], ko[1], ko[2], ko[3]);  // kr
          else
            *(float4*)(in + 384 + 4 * (lane - 32)) = make_float4(kv[0], kv[1], kv[2], kv[3]);  // vr
          // the split holding `pos` writes this position's K (roped) and V to the cache
          if (att_t0(ctx, s) <= pos && pos < att_t1(ctx, s)) {
            const long row = (((long)l * NKV + g) * P.max_seq + pos) * HD;
            if (lane < 32) {
              h4 o = {(_Float16)ko[0], (_Float16)ko[1], (_Float16)ko[2], (_Float16)ko[3]};
              __hip_atomic_store((u64*)(P.k_cache + row + d0), __builtin_bit_cast(u64, o), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
            } else {
              h4 o = {(_Float16)kv[0], (_Float16)kv[1], (_Float16)kv[2], (_Float16)kv[3]};
              __hip_atomic_store((u64*)(P.v_cache + row + d0), __builtin_bit_cast(u64, o), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
            }
          }
        }
        publish(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_PUBLISH);

        // ---- combine: q head w/16, dims [d0, d0+8) over the 32 splits of its kv head
        {
          const int h = cmb_head(w), gh = h / 2, ih = h % 2, d0 = cmb_d0(w);
          v4u v[5];
          // lane s < 32 reads split s: (m, l) and acc[d0 .. d0+8)
          poll_pairs<5>(pl, tag_of(epoch, l, SID_PART), lane < NSPLIT ? cmb_voff(lane) : 0, lane < NSPLIT,
                        [&](int k) -> int { return (int)cmb_soff(par, h, d0, k); }, v);
          if (!pl.ok) break;
          float m = -INFINITY, lsum = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          if (lane < NSPLIT) {
            m = __uint_as_float(v[0].x);
            lsum = __uint_as_float(v[0].z);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              acc[2 * k] = __uint_as_float(v[k + 1].x);
              acc[2 * k + 1] = __uint_as_float(v[k + 1].z);
            }
          }
          const float M = max16x(row16_max(m));  // over lanes 0-31 (lanes >= 32 hold -inf)
          const float e = (lane < NSPLIT && m != -INFINITY) ? __expf(m - M) : 0.f;
          float Lt = half_sum(e * lsum);
          float o[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = half_sum(e * acc[j]);
          const float inv = Lt > 0.f ? 1.0f / Lt : 0.f;
          // drain the KV-cache stores before any workgroup can depend on this step
          __builtin_amdgcn_s_waitcnt(0);
          // lane k < 4 stores dims 2k, 2k+1 (static selects: no lane-indexed array)
          const float oa = lane == 0 ? o[0] : (lane == 1 ? o[2] : (lane == 2 ? o[4] : o[6]));
          const float ob = lane == 0 ? o[1] : (lane == 1 ? o[3] : (lane == 2 ? o[5] : o[7]));
          if (lane < 4)
            ll_store(P.ws, slot_att(par, 4 * w + lane), pack_h2(oa * inv, ob * inv), tag_of(epoch, l, SID_ATT));
          xtrace(P, t, fin - (u32)(t * FT), TR_COMBINE);
        }

        // ---- o_proj input: all 2048 attention values
        ++fin;
        wait_consumed(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_POLL);
        {
          v4u v[8];
          poll_pairs<8>(pl, tag_of(epoch, l, SID_ATT), lin_voff(lane), true,
                        [&](int k) -> int { return (int)lin_soff(slot_att(par, 0), k); }, v);
          if (!pl.ok) break;
          float* in = S->in[fin & 1];
#pragma unroll
          for (int k = 0; k < 8; ++k)
            *(float4*)(in + 4 * (lane + 64 * k)) = make_float4(lo_h(v[k].x), hi_h(v[k].x), lo_h(v[k].z), hi_h(v[k].z));
        }
        publish(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_PUBLISH);

        // ---- gate/up input: post-attention residual -> RMSNorm * post_attention_layernorm
        ++fin;
        wait_consumed(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_POLL);
        {
          const NormW w_post = load_norm((const _Float16*)lw.post_attn_layernorm_weight);
          poll_vec1024(pl, tag_of(epoch, l, SID_ACT), slot_act(par, 0), x);
          if (!pl.ok) break;
          const float rs = rstd_1024(x);
          store_normed(S->in[fin & 1], x, rs, w_post);
        }
        publish(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_PUBLISH);

        // ---- down input: SiLU(gate)*up, 3072 values
        ++fin;
        wait_consumed(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_POLL);
        {
          v4u v[12];
          poll_pairs<12>(pl, tag_of(epoch, l, SID_INT), lin_voff(lane), true,
                         [&](int k) -> int { return (int)lin_soff(slot_int(par, 0), k); }, v);
          if (!pl.ok) break;
          float* in = S->in[fin & 1];
#pragma unroll
          for (int k = 0; k < 12; ++k)
            *(float4*)(in + 4 * (lane + 64 * k)) = make_float4(lo_h(v[k].x), hi_h(v[k].x), lo_h(v[k].z), hi_h(v[k].z));
        }
        publish(pl, fin);
        xtrace(P, t, fin - (u32)(t * FT), TR_PUBLISH);
      }
      if (!pl.ok) break;

      // ---- lm_head input: final residual -> RMSNorm * final_norm
      const u32 fin = (u32)(t * FT + 5 * L);
      wait_consumed(pl, fin);
      xtrace(P, t, fin - (u32)(t * FT), TR_POLL);
      const NormW w_fin = load_norm(P.final_norm);
      float x[16];
      poll_vec1024(pl, tag_of(epoch, L - 1, SID_X), slot_x(L & 1, 0), x);
      if (!pl.ok) break;
      const float rs = rstd_1024(x);
      store_normed(S->in[fin & 1], x, rs, w_fin);
      publish(pl, fin);
      xtrace(P, t, fin - (u32)(t * FT), TR_PUBLISH);
      if (w == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int i = 4 * (lane + 64 * k);
          h4 hv = {(_Float16)x[4 * k], (_Float16)x[4 * k + 1], (_Float16)x[4 * k + 2], (_Float16)x[4 * k + 3]};
          *(h4*)(P.hidden_out + i) = hv;
          const h4 wv = w_fin.v[k];
          *(float4*)(P.norm_out + i) = make_float4(x[4 * k] * rs * (float)wv[0], x[4 * k + 1] * rs * (float)wv[1],
                                                   x[4 * k + 2] * rs * (float)wv[2], x[4 * k + 3] * rs * (float)wv[3]);
          if (P.hidden_steps)
            *(float4*)(P.hidden_steps + (long)t * HIDDEN + i) = make_float4(x[4 * k], x[4 * k + 1], x[4 * k + 2], x[4 * k + 3]);
        }
      }
    }

    // ---- argmax over the 256 workgroup partials (lowest index on ties)
    {
      v4u v[4];
      poll_pairs<4>(pl, tag_arg(epoch), lin_voff(lane), true,
                    [&](int k) -> int { return (int)lin_soff(slot_arg(t & 1, 0), k); }, v);
      if (!pl.ok) break;
      float best = -INFINITY;
      int bidx = 0x7fffffff;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float val = __uint_as_float(v[k].x);
        const int idx = (int)v[k].z;
        if (val > best || (val == best && idx < bidx)) {
          best = val;
          bidx = idx;
        }
      }
      wave_argmax(best, bidx);
      if (bidx < 0 || bidx >= VOCAB) bidx = 0;  // every logit NaN
      if (w == 0 && lane == 0) P.out_tokens[t] = bidx;
      xtrace(P, t, (u32)(FT - 1), TR_COMBINE);
      token = (P.forced && t + 1 < P.num_steps) ? P.forced[t + 1] : bidx;
      if (token < 0 || token >= VOCAB) {  // a forced id out of range: report and stop
        __hip_atomic_fetch_or(P.status, ST_BAD_TOKEN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pl.ok = false;
        break;
      }
    }
  }
  if (!pl.ok) lds_st(&S->abort, 1u);
}

// ------------------------------------------------------------------------------------
// compute waves

struct Buf {
  v4u v[12];
};

__device__ __forceinline__ const LDGLayerWeight& layer_of(const KParams& P, int l) { return P.layers[l]; }

// Issues stage d's weight (or KV-cache) loads for group member m into b. Every
// path issues its loads unconditionally; rows outside the work range are
// clamped to a valid row and ignored by the compute.
__device__ __forceinline__ void prefetch(const KParams& P, const StageDesc& d, Buf& b, int w, int m, int lane) {
  switch (d.type) {
    case C_QKV: {
      const LDGLayerWeight& lw = layer_of(P, d.layer);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = QKV_PER_WG * w + 4 * m + r;
        const int mat = qkv_matrix(row);
        const _Float16* base =
            (const _Float16*)(mat == 0 ? lw.q_proj_weight : (mat == 1 ? lw.k_proj_weight : lw.v_proj_weight)) +
            (long)qkv_row_in(row) * HIDDEN;
        b.v[2 * r] = ld_nt(base + 8 * lane);
        b.v[2 * r + 1] = ld_nt(base + 512 + 8 * lane);
      }
      break;
    }
    case C_ATT: {
      const int pos = P.start_pos + d.token, ctx = pos + 1;
      const int g = att_kv(w), s = att_split(w);
      const int t0 = att_t0(ctx, s), t1 = att_t1(ctx, s);
      const int j = lane >> 4, q = lane & 15;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        int p = t0 + att_local_pos(m, j, bb);
        if (!(p < t1 && p != pos)) p = 0;  // position 0 always exists; its value is unused
        const long row = (((long)d.layer * NKV + g) * P.max_seq + p) * HD + 8 * q;
        b.v[bb] = ld_plain(P.k_cache + row);
        b.v[4 + bb] = ld_plain(P.v_cache + row);
      }
      break;
    }
    case C_OPROJ: {
      const LDGLayerWeight& lw = layer_of(P, d.layer);
      const _Float16* base = (const _Float16*)lw.o_proj_weight + (long)(HID_PER_WG * w + m) * QSZ;
#pragma unroll
      for (int k = 0; k < 4; ++k) b.v[k] = ld_nt(base + 8 * lane + 512 * k);
      break;
    }
    case C_GU: {
      const LDGLayerWeight& lw = layer_of(P, d.layer);
      // member 0,1: gate rows 6m..6m+5; member 2,3: up rows 6(m-2)..
      const _Float16* mat = (const _Float16*)(m < 2 ? lw.gate_proj_weight : lw.up_proj_weight);
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const _Float16* base = mat + (long)(INT_PER_WG * w + 6 * (m & 1) + k) * HIDDEN;
        b.v[2 * k] = ld_nt(base + 8 * lane);
        b.v[2 * k + 1] = ld_nt(base + 512 + 8 * lane);
      }
      break;
    }
    case C_DOWN: {
      const LDGLayerWeight& lw = layer_of(P, d.layer);
      const _Float16* base = (const _Float16*)lw.down_proj_weight + (long)(HID_PER_WG * w + m) * INTER;
#pragma unroll
      for (int k = 0; k < 6; ++k) b.v[k] = ld_nt(base + 8 * lane + 512 * k);
      break;
    }
    default: {  // C_LMH
      const int nrows = lm_rows(w), r0 = lm_row0(w);
#pragma unroll
      for (int i = 0; i < LM_ROWS_PER_CHUNK; ++i) {
        int lr = lm_local_row(m, d.chunk, i);
        if (lr >= nrows) lr = nrows - 1;  // clamped rows are loaded but not used
        const _Float16* base = P.lm_head + (long)(r0 + lr) * HIDDEN;
        b.v[2 * i] = ld_nt(base + 8 * lane);
        b.v[2 * i + 1] = ld_nt(base + 512 + 8 * lane);
      }
      break;
    }
  }
}

struct CState {
  float lm_best;
  int lm_idx;
};

// returns false when the workgroup aborted
__device__ __forceinline__ bool wait_ready(Shared* S, u32 fin, u64 deadline) {
  if (lds_ld(&S->ready) > fin) {
    lds_acquire();
    return true;
  }
  const u64 t0 = wall_clock64();
  int spins = 0;
  while (lds_ld(&S->ready) <= fin) {
    if (lds_ld(&S->abort)) return false;
    if ((++spins & 63) == 0 && wall_clock64() - t0 > deadline) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  lds_acquire();
  return true;
}

// One compute wave's arrival at finalised stage `fin`, which takes `n` arrivals;
// returns true in the wave that arrives last: it finalises (and resets the counter).
__device__ __forceinline__ bool arrive(Shared* S, u32 fin, u32 n) {
  lds_release();
  u32 old = 0;
  if (__lane_id() == 0) old = __hip_atomic_fetch_add(&S->cnt[fin & 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  old = __builtin_amdgcn_readfirstlane(old);
  const bool last = old == n - 1;
  if (last) {
    lds_acquire();
    if (__lane_id() == 0) lds_st(&S->cnt[fin & 1], 0u);
  }
  return last;
}

// marks `fin` finalised (all its reads of S->in and S->red are done) for the exchange wave;
// called by the finalising wave after its last LDS read and before its exchange stores
__device__ __forceinline__ void mark_done(Shared* S, u32 fin) {
  lds_release();
  if (__lane_id() == 0) lds_st(&S->done[fin & 1], fin + 1);
}

__device__ __forceinline__ void trace_mark(const KParams& P, int token, u32 fin_in_token, int what) {
  if (P.trace && token == P.trace_token && __lane_id() == 0) {
    const int FT = fins_per_token(P.mode, P.num_layers);
    P.trace[((long)blockIdx.x * FT + fin_in_token) * TRACE_EVENTS + what] = wall_clock64();
  }
}

__device__ __forceinline__ void compute(const KParams& P, Shared* S, const StageDesc& d, const Buf& b, CState& cs,
                                        int w, int m, int c, int lane) {
  const u32 fin = (u32)d.fin;
  const float* in = S->in[fin & 1];
  float* red = S->red[fin & 1];
  const u32 epoch = P.epoch0 + (u32)d.token;
  const int par = d.layer & 1;
  const u32 fin_in_token = fin - (u32)(d.token * fins_per_token(P.mode, P.num_layers));
  switch (d.type) {
    case C_QKV: {
      float part[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) part[r] = dot8(b.v[2 * r], in + 8 * lane) + dot8(b.v[2 * r + 1], in + 512 + 8 * lane);
      // lanes 0, 16, 32, 48 hold rows 0, 2, 1, 3
      const float rs = reduce4(part[0], part[1], part[2], part[3]);
      if ((lane & 15) == 0) red[4 * m + ((lane >> 4) == 1 ? 2 : ((lane >> 4) == 2 ? 1 : (lane >> 4)))] = rs;
      if (arrive(S, fin, NGW)) {
        trace_mark(P, d.token, fin_in_token, TR_FSTART);
        float v0 = 0.f, v1 = 0.f;
        if (lane < QKV_PER_WG / 2) {
          v0 = red[2 * lane];
          v1 = red[2 * lane + 1];
        }
        mark_done(S, fin);
        if (lane < QKV_PER_WG / 2)
          ll_store(P.ws, slot_qkv(par, (QKV_PER_WG / 2) * w + lane), pack_h2(v0, v1), tag_of(epoch, d.layer, SID_QKV));
        trace_mark(P, d.token, fin_in_token, TR_FINAL);
      }
      break;
    }
    case C_ATT: {
      const int pos = P.start_pos + d.token, ctx = pos + 1;
      const int g = att_kv(w), s = att_split(w);
      const int t0 = att_t0(ctx, s), t1 = att_t1(ctx, s);
      const int j = lane >> 4, q = lane & 15;
      const float* q0 = in;
      const float* q1 = in + 128;
      const float* kr = in + 256;
      const float* vr = in + 384;
      float4 qa0 = *(const float4*)(q0 + 8 * q), qb0 = *(const float4*)(q0 + 8 * q + 4);
      float4 qa1 = *(const float4*)(q1 + 8 * q), qb1 = *(const float4*)(q1 + 8 * q + 4);
      const float qv0[8] = {qa0.x, qa0.y, qa0.z, qa0.w, qb0.x, qb0.y, qb0.z, qb0.w};
      const float qv1[8] = {qa1.x, qa1.y, qa1.z, qa1.w, qb1.x, qb1.y, qb1.z, qb1.w};
      float sc[4][2];
      bool valid[4];
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int p = t0 + att_local_pos(m, j, bb);
        valid[bb] = p < t1;
        float kf[8];
        if (p == pos) {
#pragma unroll
          for (int e = 0; e < 8; ++e) kf[e] = (float)(_Float16)kr[8 * q + e];  // the cached value is fp16
        } else {
          h8 kh = __builtin_bit_cast(h8, b.v[bb]);
#pragma unroll
          for (int e = 0; e < 8; ++e) kf[e] = (float)kh[e];
        }
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s0 = fmaf(kf[e], qv0[e], s0);
          s1 = fmaf(kf[e], qv1[e], s1);
        }
        s0 = row16_sum(s0) * P.attn_scale;
        s1 = row16_sum(s1) * P.attn_scale;
        sc[bb][0] = valid[bb] ? s0 : -INFINITY;
        sc[bb][1] = valid[bb] ? s1 : -INFINITY;
      }
      float mh[2], lh[2], acc[2][8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float mx = fmaxf(fmaxf(sc[0][h], sc[1][h]), fmaxf(sc[2][h], sc[3][h]));
        mx = rows4_max(mx);
        mh[h] = mx;
        float pr[4];
        float l = 0.f;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          pr[bb] = valid[bb] ? __expf(sc[bb][h] - mx) : 0.f;
          l += pr[bb];
        }
        l = rows4_sum(l);
        lh[h] = l;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          const int p = t0 + att_local_pos(m, j, bb);
          float vf[8];
          if (p == pos) {
#pragma unroll
            for (int e = 0; e < 8; ++e) vf[e] = (float)(_Float16)vr[8 * q + e];
          } else {
            h8 vh = __builtin_bit_cast(h8, b.v[4 + bb]);
#pragma unroll
            for (int e = 0; e < 8; ++e) vf[e] = (float)vh[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(pr[bb], vf[e], acc[h][e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[h][e] = rows4_sum(acc[h][e]);
        }
      }
      float* rec = red + m * 260;
      if (lane < 16) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          *(float4*)(rec + h * 130 + 2 + 8 * q) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
          *(float4*)(rec + h * 130 + 2 + 8 * q + 4) = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
      }
      if (lane == 0) {
        rec[0] = mh[0];
        rec[1] = lh[0];
        rec[130] = mh[1];
        rec[131] = lh[1];
      }
      if (arrive(S, fin, NGW)) {
        trace_mark(P, d.token, fin_in_token, TR_FSTART);
        // merge the 4 wave partials into the workgroup partial (m, l, acc) per head
        float Mx[2], wt[2][NGW];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float M = -INFINITY;
#pragma unroll
          for (int cc = 0; cc < NGW; ++cc) M = fmaxf(M, red[cc * 260 + h * 130]);
          Mx[h] = M;
#pragma unroll
          for (int cc = 0; cc < NGW; ++cc) {
            const float mc = red[cc * 260 + h * 130];
            wt[h][cc] = (mc == -INFINITY) ? 0.f : __expf(mc - M);
          }
        }
        float vals[5];
#pragma unroll
        for (int it = 0; it < 5; ++it) {
          const int e = lane + 64 * it;
          vals[it] = 0.f;
          if (e < 260) {
            const bool h1 = e >= 130;
            const int k = h1 ? e - 130 : e;
            if (k == 0) {
              vals[it] = h1 ? Mx[1] : Mx[0];
            } else {
#pragma unroll
              for (int cc = 0; cc < NGW; ++cc)
                vals[it] = fmaf(h1 ? wt[1][cc] : wt[0][cc], red[cc * 260 + e], vals[it]);
            }
          }
        }
        mark_done(S, fin);
#pragma unroll
        for (int it = 0; it < 5; ++it) {
          const int e = lane + 64 * it;
          if (e < 260) {
            const bool h1 = e >= 130;
            ll_store(P.ws, slot_part(par, g, s, h1 ? 1 : 0, h1 ? e - 130 : e), __float_as_uint(vals[it]),
                     tag_of(epoch, d.layer, SID_PART));
          }
        }
        trace_mark(P, d.token, fin_in_token, TR_FINAL);
      }
      break;
    }
    case C_OPROJ: {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) sum += dot8(b.v[k], in + 8 * lane + 512 * k);
      sum = wave_sum(sum);
      if (lane == 0) red[m] = sum;
      if (arrive(S, fin, NGW)) {
        trace_mark(P, d.token, fin_in_token, TR_FSTART);
        float a0 = 0.f, a1 = 0.f;
        if (lane < 2) {
          const int r0 = 2 * lane;
          a0 = red[r0] + S->xres[r0];
          a1 = red[r0 + 1] + S->xres[r0 + 1];
          S->actres[r0] = a0;
          S->actres[r0 + 1] = a1;
        }
        mark_done(S, fin);
        if (lane < 2) ll_store(P.ws, slot_act(par, 2 * w + lane), pack_h2(a0, a1), tag_of(epoch, d.layer, SID_ACT));
        trace_mark(P, d.token, fin_in_token, TR_FINAL);
      }
      break;
    }
    case C_GU: {
      float part[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) part[k] = dot8(b.v[2 * k], in + 8 * lane) + dot8(b.v[2 * k + 1], in + 512 + 8 * lane);
      float pr, qr;
      reduce6(part, pr, qr);  // pr: rows 0,1,3,4 at lanes 0,16,32,48; qr: rows 2 (lane 0), 5 (lane 32)
      if ((lane & 15) == 0) red[6 * m + (lane >> 4) + ((lane >> 4) >= 2 ? 1 : 0)] = pr;
      if ((lane & 31) == 0) red[6 * m + (lane == 0 ? 2 : 5)] = qr;
      if (arrive(S, fin, NGW)) {
        trace_mark(P, d.token, fin_in_token, TR_FSTART);
        float o[2] = {0.f, 0.f};
        if (lane < INT_PER_WG / 2) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float gt = red[2 * lane + e], up = red[INT_PER_WG + 2 * lane + e];
            o[e] = gt / (1.0f + __expf(-gt)) * up;
          }
        }
        mark_done(S, fin);
        if (lane < INT_PER_WG / 2)
          ll_store(P.ws, slot_int(par, (INT_PER_WG / 2) * w + lane), pack_h2(o[0], o[1]), tag_of(epoch, d.layer, SID_INT));
        trace_mark(P, d.token, fin_in_token, TR_FINAL);
      }
      break;
    }
    case C_DOWN: {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < 6; ++k) sum += dot8(b.v[k], in + 8 * lane + 512 * k);
      sum = wave_sum(sum);
      if (lane == 0) red[m] = sum;
      if (arrive(S, fin, NGW)) {
        trace_mark(P, d.token, fin_in_token, TR_FSTART);
        float x0 = 0.f, x1 = 0.f;
        if (lane < 2) {
          const int r0 = 2 * lane;
          x0 = red[r0] + S->actres[r0];
          x1 = red[r0 + 1] + S->actres[r0 + 1];
          S->xres[r0] = x0;
          S->xres[r0 + 1] = x1;
        }
        mark_done(S, fin);
        if (lane < 2) {
          if (P.mode == MODE_MLP) {
            P.out_vec[HID_PER_WG * w + 2 * lane] = x0;
            P.out_vec[HID_PER_WG * w + 2 * lane + 1] = x1;
          } else {
            ll_store(P.ws, slot_x((d.layer + 1) & 1, 2 * w + lane), pack_h2(x0, x1), tag_of(epoch, d.layer, SID_X));
          }
        }
        trace_mark(P, d.token, fin_in_token, TR_FINAL);
      }
      break;
    }
    default: {  // C_LMH chunk: this wave's 6 rows of chunk d.chunk
      if (d.chunk < 2) {  // first chunk this wave sees in this token
        cs.lm_best = -INFINITY;
        cs.lm_idx = 0x7fffffff;
      }
      const int nrows = lm_rows(w), r0 = lm_row0(w);
      float part[LM_ROWS_PER_CHUNK];
#pragma unroll
      for (int i = 0; i < LM_ROWS_PER_CHUNK; ++i)
        part[i] = dot8(b.v[2 * i], in + 8 * lane) + dot8(b.v[2 * i + 1], in + 512 + 8 * lane);
      float pr, qr;
      reduce6(part, pr, qr);
      // lane 0: rows 0 (pr), 2 (qr); lane 16: row 1; lane 32: rows 3 (pr), 5 (qr); lane 48: row 4.
      // Each lane's rows ascend across chunks, so strict > keeps the lowest index.
      if ((lane & 15) == 0) {
        const int ip = (lane >> 4) + ((lane >> 4) >= 2 ? 1 : 0);
        const int lr = lm_local_row(m, d.chunk, ip);
        if (lr < nrows) {
          if (P.logits_out) P.logits_out[(long)d.token * VOCAB + r0 + lr] = pr;
          const float v = __builtin_isnan(pr) ? -INFINITY : pr;
          if (v > cs.lm_best) {
            cs.lm_best = v;
            cs.lm_idx = r0 + lr;
          }
        }
      }
      if ((lane & 31) == 0) {
        const int lr = lm_local_row(m, d.chunk, lane == 0 ? 2 : 5);
        if (lr < nrows) {
          if (P.logits_out) P.logits_out[(long)d.token * VOCAB + r0 + lr] = qr;
          const float v = __builtin_isnan(qr) ? -INFINITY : qr;
          if (v > cs.lm_best) {
            cs.lm_best = v;
            cs.lm_idx = r0 + lr;
          }
        }
      }
      if (d.chunk >= LM_CHUNKS - 2) {  // this wave's last chunk of the token
        float bv = cs.lm_best;
        int bi = cs.lm_idx;
        wave_argmax(bv, bi);
        if (lane == 0) {
          red[2 * c] = bv;
          red[2 * c + 1] = __int_as_float(bi);
        }
        if (arrive(S, fin, NCW)) {
          trace_mark(P, d.token, fin_in_token, TR_FSTART);
          float best = -INFINITY;
          int bidx = 0x7fffffff;
          for (int cc = 0; cc < NCW; ++cc) {
            const float v = red[2 * cc];
            const int ix = __float_as_int(red[2 * cc + 1]);
            if (v > best || (v == best && ix < bidx)) {
              best = v;
              bidx = ix;
            }
          }
          mark_done(S, fin);
          if (lane == 0) {
            const u32 tg = tag_arg(epoch);
            ll_store(P.ws, slot_arg(d.token & 1, 2 * w), __float_as_uint(best), tg);
            ll_store(P.ws, slot_arg(d.token & 1, 2 * w + 1), (u32)bidx, tg);
          }
          trace_mark(P, d.token, fin_in_token, TR_FINAL);
        }
      }
      break;
    }
  }
}

// Compute wave c of group c / 4 (member c % 4) runs the stages j with j % 2 == group.
// Its single register buffer holds stage j's weights, loaded right after it computed
// stage j - 2: the only loads in flight when it computes are the ones it needs, so the
// compiler's wait for them never waits on a later prefetch.
__device__ void compute_wave(const KParams& P, Shared* S, int c) {
  const int w = blockIdx.x;
  const int lane = __lane_id();
  const int L = P.num_layers;
  const int grp = c / NGW, m = c % NGW;
  const int total = stages_per_token(P.mode, L) * P.num_steps;
  const u64 deadline = 2 * P.deadline;
  Buf b;
  CState cs{-INFINITY, 0x7fffffff};
  if (grp < total) prefetch(P, stage_desc(P.mode, L, grp), b, w, m, lane);
  for (int j = grp; j < total; j += 2) {
    const StageDesc d = stage_desc(P.mode, L, j);
    if (!wait_ready(S, (u32)d.fin, deadline)) break;
    const u32 fin_in_token = (u32)d.fin - (u32)(d.token * fins_per_token(P.mode, L));
    if (m == 0) trace_mark(P, d.token, fin_in_token, TR_CSTART);
    compute(P, S, d, b, cs, w, m, c, lane);
    if (m == 0) trace_mark(P, d.token, fin_in_token, TR_CDONE);
    if (j + 2 < total) prefetch(P, stage_desc(P.mode, L, j + 2), b, w, m, lane);
  }
}

__global__ void __launch_bounds__(BLOCK, 1) qwen_decode_kernel(KParams P) {
  __shared__ Shared S;
  // wave index is uniform per wave; readfirstlane lets the compiler keep it (and
  // every weight address derived from it) in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  if (threadIdx.x == 0) {
    S.ready = 0;
    S.cnt[0] = 0;
    S.cnt[1] = 0;
    S.done[0] = 0;
    S.done[1] = 0;
    S.abort = 0;
  }
  __syncthreads();
  if (wave == NCW)
    exchange_wave(P, &S);
  else
    compute_wave(P, &S, wave);
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
  if (num_layers < 1 || num_layers > MAX_LAYERS || steps < 1 || start < 0 || max_seq < 1 ||
      (long)start + steps > (long)max_seq || max_seq > NSPLIT * MAX_SPLIT_POS)
    return QWEN_ERR_ARG;
  memset(&P, 0, sizeof(P));
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
  P.lm_head = (const _Float16*)weight;
  P.in_vec = (const _Float16*)hidden_f16;
  P.out_tokens = out_token;
  P.logits_out = logits_out;
  P.mode = MODE_LMHEAD;
  P.num_layers = 1;
  P.num_steps = 1;
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
  P.layers = d_tab[dev];
  P.in_vec = (const _Float16*)x_f16;
  P.out_vec = y_out;
  P.mode = MODE_MLP;
  P.num_layers = 1;
  P.num_steps = 1;
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
