// Work partition, LDS weight-ring schedule and exchange-buffer layout of the
// persistent decode kernel.
//
// Everything here is plain integer arithmetic shared by the device code and
// the host-side exhaustive bounds checker (layout_check.cpp), so every index
// the kernel forms can be verified on the CPU before a GPU runs it.
//
// Model shape: Qwen3-0.6B (Tools/megakernel/megakernel.cu:15-22,80-81).
//
// Grid: one 512-thread workgroup per CU of MI355X (256 CUs in 8 XCDs). The
// hardware places workgroup w on XCD w % 8, so w = 8 i + x names local index
// i (0..31) on XCD x. XCD x owns kv head x and everything that can be computed
// from it without leaving the XCD:
//   QKV rows   the 512 rows [q head 2x | q head 2x+1 | k head x | v head x];
//              workgroup i computes rows [16 i, 16 i + 16) of that list
//   attention  position split i of kv head x (32 splits), both q heads
//   combine    q head 2x + i / 16, dims [8 (i % 16), +8)
//   o_proj     partial over the XCD's 256 attention dims: rows [32 i, 32 i + 32)
//   gate/up    inter rows [384 x + 12 i, +12) of each of Wg, Wu
//   down       partial over the XCD's 384 inter values: rows [32 i, 32 i + 32)
// and two cross-XCD steps per layer: workgroup i of every XCD sums rows
// [32 i, 32 i + 32) of the 8 per-XCD o_proj (resp. down) partials into the
// residual stream (each XCD computes identical sums), which is then
// all-gathered inside the XCD.
// Waves 0-3 compute (each a quarter of every stage); waves 4-7 stream the
// stage weights and K/V rows into a ring of 1 KB lines in LDS.
#pragma once

#ifdef __HIPCC__
#define QL_HD __host__ __device__ __forceinline__
#else
#define QL_HD inline
#endif

namespace ql {

constexpr int HIDDEN = 1024;
constexpr int INTER = 3072;
constexpr int NQ = 16;
constexpr int NKV = 8;
constexpr int HD = 128;
constexpr int QSZ = NQ * HD;    // 2048
constexpr int KVSZ = NKV * HD;  // 1024
constexpr int VOCAB = 151936;
constexpr int MAX_LAYERS = 28;
constexpr int MAX_SEQ_LIMIT = 2048;  // largest max_seq_len the split schedule covers

constexpr int NWG = 256;
constexpr int NXCD = 8;
constexpr int NLOC = NWG / NXCD;  // 32 workgroups per XCD
constexpr int WAVE = 64;
constexpr int NCW = 4;            // compute waves
constexpr int NLW = 4;            // loader waves
constexpr int BLOCK = (NCW + NLW) * WAVE;  // 512

QL_HD int xcd_of(int w) { return w % NXCD; }
QL_HD int loc_of(int w) { return w / NXCD; }

// ---- partition ----------------------------------------------------------------------
constexpr int GRP_ROWS = 512;    // QKV rows of one kv group
constexpr int QKV_PER_WG = 16;   // 4 per compute wave
constexpr int HROWS = 32;        // o_proj / down / residual rows per workgroup, 8 per compute wave
constexpr int OCOLS = 256;       // attention dims per XCD (q heads 2x, 2x+1)
constexpr int ICOLS = 384;       // inter values per XCD
constexpr int GU_PER_WG = 12;    // gate rows (and up rows) per workgroup, 3 per compute wave
constexpr int NSPLIT = NLOC;     // attention position splits per kv head

// group row r (0..511) of kv group x -> (matrix 0/1/2 = q/k/v, row within that matrix)
QL_HD int grp_matrix(int r) { return r < 256 ? 0 : (r < 384 ? 1 : 2); }
QL_HD int grp_row_in(int x, int r) { return r < 256 ? 256 * x + r : (r < 384 ? 128 * x + r - 256 : 128 * x + r - 384); }

// attention split schedule: spans are multiples of 4 positions so a ring line holds 4 whole positions
QL_HD int att_span(int ctx) { return 4 * ((ctx + 4 * NSPLIT - 1) / (4 * NSPLIT)); }
QL_HD int att_t0(int ctx, int s) { return s * att_span(ctx); }
QL_HD int att_t1(int ctx, int s) {
  int a = att_t0(ctx, s), e = a + att_span(ctx);
  if (a > ctx) return a;
  return e < ctx ? e : ctx;
}
QL_HD int att_nk(int ctx, int s) {  // K lines (= V lines) of split s
  int a = att_t0(ctx, s), b = att_t1(ctx, s);
  return b > a ? (b - a + 3) / 4 : 0;
}

// ---- LDS weight ring ---------------------------------------------------------------
constexpr int RING_LINES = 128;
constexpr int LINE_BYTES = 1024;
// The per-layer norm weights and the per-token RoPE row travel through the ring
// too, so a compute wave never has a global load outstanding when it polls.
constexpr int LINES_NORM = 2;   // a 1024-entry fp16 norm weight vector
constexpr int LINES_QKV = LINES_NORM + 32;  // input norm, then 16 rows x 2 lines
constexpr int LINES_ATTMISC = 1;  // q_norm | k_norm | cos[pos] | sin[pos], 256 B each
constexpr int LINES_O = 16;     // 32 rows x 512 B, 2 rows per line
constexpr int LINES_GU = LINES_NORM + 48;   // post-attention norm, then 12 gate rows, 12 up rows, 2 lines each
constexpr int LINES_DOWN = 32;  // 32 rows x 768 B, one row per line (last 256 B unused)

enum StageId : int { S_QKV = 0, S_ATT = 1, S_COMB = 2, S_O = 3, S_OSUM = 4, S_GU = 5, S_DOWN = 6, S_DSUM = 7 };
constexpr int NSTAGE = 8;
enum Mode : int { MODE_DECODE = 0, MODE_LMHEAD = 1, MODE_MLP = 2 };

// ring lines of a stage; ctx = position + 1, s = attention split
QL_HD int stage_lines(int st, int ctx, int s) {
  switch (st) {
    case S_QKV: return LINES_QKV;
    case S_ATT: return LINES_ATTMISC + 2 * att_nk(ctx, s);
    case S_O: return LINES_O;
    case S_GU: return LINES_GU;
    case S_DOWN: return LINES_DOWN;
    default: return 0;
  }
}

// ---- loader streams ------------------------------------------------------------------
// The ring lines of a layer come from 10 streams, in this order: 0 input norm (2
// lines), 1 QKV rows (32), 2 attention vectors (1), 3 K (nk), 4 V (nk), 5 o_proj
// (16), 6 post-attention norm (2), 7 gate (24), 8 up (24), 9 down (32). Line m of
// a stream gives lane `lane` 8 fp16 values at element
//   elem0 + m * stride + loff
// of the lane's source array `mat`: 0..2 Wq/Wk/Wv, 3 K cache, 4 V cache, 5 Wo,
// 6 Wg, 7 Wu, 8 Wd, 9 input norm, 10 post-attention norm, 11 q_norm, 12 k_norm,
// 13 cos table, 14 sin table (cache elements counted from layer l's kv head x at
// position 0). Only the attention-vector line mixes sources: lanes 0-15 q_norm,
// 16-31 k_norm, 32-47 cos[pos], 48-63 sin[pos]. For K/V lines, lanes whose
// position index 4 m + lane / 16 is >= vlim read no cache element (they read a
// fixed spare row instead).
constexpr int NSTREAM = 10;
constexpr int MLP_FIRST_STREAM = 6;
struct StreamGeom {
  int mat;
  long elem0, stride, loff;
  int n, vlim;
};
QL_HD StreamGeom stream_geom(int si, int x, int i, int ctx, int pos, int lane) {
  StreamGeom g;
  g.vlim = 0x7fffffff;
  g.loff = 8 * lane;
  g.stride = 512;
  switch (si) {
    case 0:
    case 6:
      g.mat = si == 0 ? 9 : 10;
      g.elem0 = 0;
      g.n = LINES_NORM;
      break;
    case 1: {
      const int gr = QKV_PER_WG * i;
      g.mat = grp_matrix(gr);
      g.elem0 = (long)grp_row_in(x, gr) * HIDDEN;
      g.n = LINES_QKV - LINES_NORM;
      break;
    }
    case 2: {
      const int seg = lane >> 4;
      g.mat = 11 + seg;
      g.elem0 = seg >= 2 ? (long)pos * HD : 0;
      g.loff = 8 * (lane & 15);
      g.n = LINES_ATTMISC;
      break;
    }
    case 3:
    case 4: {
      const int t0 = att_t0(ctx, i), t1 = att_t1(ctx, i);
      g.mat = si == 3 ? 3 : 4;
      g.elem0 = (long)t0 * HD;
      g.n = att_nk(ctx, i);
      g.vlim = (t1 < pos ? t1 : pos) - t0;
      break;
    }
    case 5:
      g.mat = 5;
      g.elem0 = (long)HROWS * i * QSZ + OCOLS * x;
      g.stride = 2L * QSZ;
      g.loff = (long)(lane >> 5) * QSZ + 8 * (lane & 31);
      g.n = LINES_O;
      break;
    case 7:
    case 8:
      g.mat = si == 7 ? 6 : 7;
      g.elem0 = (long)(ICOLS * x + GU_PER_WG * i) * HIDDEN;
      g.n = 2 * GU_PER_WG;
      break;
    default:
      g.mat = 8;
      g.elem0 = (long)HROWS * i * INTER + ICOLS * x;
      g.stride = INTER;
      g.loff = 8 * (lane < 48 ? lane : lane - 48);
      g.n = LINES_DOWN;
      break;
  }
  return g;
}

// ---- LM head ------------------------------------------------------------------------
constexpr int LM_CHUNK = 8;                  // rows a wave takes per grab
static_assert(VOCAB % LM_CHUNK == 0, "whole chunks");
constexpr int LM_NCHUNK = VOCAB / LM_CHUNK;  // 18992
// The vocabulary's 8-row chunks are dealt to the workgroups in turn (chunk g to workgroup
// g mod NWG), so every workgroup streams rows from the whole table; a workgroup's 8 waves
// take its chunks 0, 1, 2, .. in turn from a shared counter. Only its first LM_STATIC
// chunks are its own. The chunks from LM_STATIC * NWG on form a pool, split over groups
// of 8 consecutive workgroups (one per XCD): the waves of a group claim its share from a
// device-scope counter once their own chunks are taken, so the group's workgroups on
// faster XCDs take more of it. (When the counters are not set up for a token, each
// workgroup takes all of its dealt chunks instead.)
QL_HD int lm_chunks(int w) { return (LM_NCHUNK - w + NWG - 1) / NWG; }
// lm_head row of workgroup w's chunk ch, slot j
QL_HD int lm_row(int w, int ch, int j) { return LM_CHUNK * (w + NWG * ch) + j; }
constexpr int LM_STATIC = 60;
static_assert(LM_STATIC * NWG <= LM_NCHUNK, "every workgroup has LM_STATIC chunks");
constexpr int LM_POOL = LM_NCHUNK - LM_STATIC * NWG;  // 3632
constexpr int LM_GROUP = NXCD;                        // workgroups per pool group
constexpr int LM_NGRP = NWG / LM_GROUP;               // 32
// claim k of group G is pool chunk LM_STATIC * NWG + LM_NGRP * k + G
QL_HD int lm_group_chunks(int G) { return (LM_POOL - G + LM_NGRP - 1) / LM_NGRP; }
// pool counters: one 128-byte line per (token epoch mod 4, group), after the status line
constexpr long LM_CTR_STRIDE = 128;
constexpr long LM_CTR_BYTES = 4L * LM_NGRP * LM_CTR_STRIDE;

// ---- exchange ("LL") buffers ---------------------------------------------------------
// A slot is 8 bytes: 32 bits of payload + a 32-bit tag, written with one 8-byte
// device-scope store and read with device-scope loads; a reader accepts a slot
// only when its tag equals the tag of the step it waits for, so data and
// "ready" travel together. H2 slots carry two fp16 values, F1 slots one fp32.
// Per-layer buffers exist twice (layer parity), ARG twice (token parity), so a
// fast workgroup never overwrites a slot a slow one has yet to read.
constexpr int X_SLOTS = HIDDEN / 2;           // 512  residual stream x, H2, per XCD
constexpr int QKV_SLOTS = GRP_ROWS / 2;       // 256  q|k|v of the kv group, H2
constexpr int PART_PER_HEAD = 2 + HD;         // m, l, acc[128]
constexpr int PART_SLOTS = NSPLIT * 2 * PART_PER_HEAD;  // 8320, F1
constexpr int ATTO_SLOTS = OCOLS / 2;         // 128  combined attention of the XCD's 2 q heads, H2
constexpr int OP_SLOTS = HIDDEN;              // 1024 o_proj partial of the XCD, F1
constexpr int ACT_SLOTS = HIDDEN / 2;         // 512  post-attention residual, H2
constexpr int INT_SLOTS = 8 * NLOC;           // 256  SiLU(gate)*up, H2, 8 slots per workgroup (12 values + pad)
constexpr int DP_SLOTS = HIDDEN;              // 1024 down partial of the XCD, F1
constexpr int ARG_SLOTS = 2 * NWG;            // 512  per-workgroup (max, index), F1

constexpr long B_X = 0;
constexpr long B_QKV = B_X + X_SLOTS;
constexpr long B_PART = B_QKV + QKV_SLOTS;
constexpr long B_ATTO = B_PART + PART_SLOTS;
constexpr long B_OP = B_ATTO + ATTO_SLOTS;
constexpr long B_ACT = B_OP + OP_SLOTS;
constexpr long B_INT = B_ACT + ACT_SLOTS;
constexpr long B_DP = B_INT + INT_SLOTS;
constexpr long XCD_SLOTS = B_DP + DP_SLOTS;   // 12032 per XCD per parity
constexpr long OFF_ARG = 2L * NXCD * XCD_SLOTS;
// Top-k sampling inside the decode kernel (its sampling build) adds two buffers, each written
// once per token (no workgroup reaches the next token's lm_head before every workgroup has
// finished this token's draw, so one copy suffices):
//  * LOGIT: the step's logits, F1, one slot per row (an lm_head chunk is one 64-byte line);
//  * SEL: the SEL_DEPTH largest entries of each slice (slice w: rows w + NWG j, SL_ROWS or
//    SL_ROWS - 1 of them), in descending (key, lower row) order, as slot pairs
//    (order-preserving key of the logit, row).
constexpr int SL_ROWS = (VOCAB + NWG - 1) / NWG;  // 594
constexpr int SL_FULL = VOCAB - (SL_ROWS - 1) * NWG;  // 128 slices hold SL_ROWS rows
constexpr int SEL_DEPTH = 8;
constexpr long OFF_LOGIT = OFF_ARG + 2L * ARG_SLOTS;
constexpr long LOGIT_SLOTS = VOCAB;
constexpr long OFF_SEL = OFF_LOGIT + LOGIT_SLOTS;
constexpr long SEL_SLOTS = 2L * NWG * SEL_DEPTH;   // 4096
// Draws split by slice (the build for top_k > TOPK_MAX and for top-p alone): every workgroup
// adds its slice's radix histogram into a global one (DHIST) with device-scope atomics, then
// announces it in a DIST round: one slot pair per workgroup per round, tagged
// tag_dist(epoch, round). Rounds also carry each slice's mass sum and Gumbel maximum, so
// every round has its own slots (a slow workgroup never finds a later round's tag in place
// of the one it waits for).
constexpr int DIST_ROUNDS = 10;  // 4 count passes, the mass total, 4 mass passes, the draw
constexpr long OFF_DIST = OFF_SEL + SEL_SLOTS;
constexpr long DIST_SLOTS = 2L * NWG * DIST_ROUNDS;  // 5120
constexpr long TOTAL_SLOTS = OFF_DIST + DIST_SLOTS;
// DHIST: per token parity, 8 passes x 256 bins of u64 (workgroup 0 clears the token's copy as
// the token starts: the token two back, which used it, has ended in every workgroup)
constexpr int DHIST_PASSES = 8;
constexpr long DHIST_BYTES = 2L * DHIST_PASSES * 256 * 8;
// after the slots: one 256-byte line of status words, the lm_head pool counters, DHIST
constexpr long WORKSPACE_BYTES = TOTAL_SLOTS * 8 + 256 + LM_CTR_BYTES + DHIST_BYTES;
// byte offset of DHIST pass `pass` of token `epoch` from the status line
QL_HD long dhist_off(unsigned epoch, int pass) {
  return 256 + LM_CTR_BYTES + ((long)(epoch & 1u) * DHIST_PASSES + pass) * 256 * 8;
}

// first slot of buffer `b` (one of B_*) of XCD x, parity par
QL_HD long xbuf(int par, int x, long b) { return ((long)par * NXCD + x) * XCD_SLOTS + b; }
QL_HD long slot_arg(int par, int k) { return OFF_ARG + (long)par * ARG_SLOTS + k; }
QL_HD long slot_logit(int row) { return OFF_LOGIT + row; }
// rows of slice w
QL_HD int slice_rows(int w) { return w < SL_FULL ? SL_ROWS : SL_ROWS - 1; }
// PART entry e (0..129) of split s, local q head hh
QL_HD long part_index(int s, int hh, int e) { return (long)(s * 2 + hh) * PART_PER_HEAD + e; }
// INT slot holding inter values 12 i + 3 c + {0, 1} (k = 0) or {2, pad} (k = 1)
QL_HD int int_slot(int i, int c, int k) { return 8 * i + 2 * c + k; }

// ---- step tags ----------------------------------------------------------------------
// tag = epoch << 8 | layer * 8 + stage id; epoch counts tokens (never 0).
QL_HD unsigned tag_of(unsigned epoch, int layer, int st) { return (epoch << 8) | (unsigned)(layer * NSTAGE + st); }
QL_HD unsigned tag_arg(unsigned epoch) { return (epoch << 8) | 255u; }
QL_HD unsigned tag_logit(unsigned epoch) { return (epoch << 8) | 254u; }
QL_HD unsigned tag_sel(unsigned epoch) { return (epoch << 8) | 253u; }
QL_HD unsigned tag_dist(unsigned epoch, int round) { return (epoch << 8) | (unsigned)(232 + round); }

// ---- prefill LDS layouts -------------------------------------------------------------
// The prefill kernel's LDS operand tiles hold each row as 16-byte chunks in a permuted order,
// so that the rows one MFMA operand read takes fall on distinct banks. Measured on MI355X
// (each pattern alone, 8 waves per CU): a 16-byte read whose 16-lane groups each touch 16
// distinct 16-byte bank units of a 256-byte window runs conflict-free; the same reads with the
// chunks in natural order run 3.5x (GEMM rows of 128 bytes) and, for the transposing 8-byte
// reads of V, 4.45x slower. layout_check verifies that property for these permutations.
// GEMM ring rows (128 bytes, 8 chunks): logical chunk q of tile row r at position q ^ pf_swz8(r)
QL_HD int pf_swz8(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
// attention key rows (256 bytes, 16 chunks): chunk q of key row r at position pf_kpos(q, r) for
// K, pf_vpos(q, r) for V (each its own inverse: the DMA lane at position p loads source chunk
// pf_kpos(p, r))
QL_HD int pf_kpos(int q, int r) { return q ^ (r & 15); }
QL_HD int pf_vpos(int q, int r) { return q ^ (2 * (r & 7)); }

// ---- 64-bit values through a 32-bit lane broadcast -----------------------------------
// `bcast` stands for the GPU's readfirstlane, which takes and returns a signed int. Each
// half of v is broadcast on its own and read back through unsigned, so a low half with
// bit 31 set is not sign-extended into the high half when the two are joined (casting the
// signed result straight to 64 bits would OR 0xffffffff into the high word).
struct U32Pair {
  unsigned lo, hi;
};
template <typename B>
QL_HD U32Pair uniform_halves(unsigned long long v, B bcast) {
  U32Pair r;
  r.lo = (unsigned)bcast((int)(unsigned)v);
  r.hi = (unsigned)bcast((int)(unsigned)(v >> 32));
  return r;
}
template <typename B>
QL_HD unsigned long long uniform_u64(unsigned long long v, B bcast) {
  const U32Pair h = uniform_halves(v, bcast);
  return ((unsigned long long)h.hi << 32) | (unsigned long long)h.lo;
}

}  // namespace ql
