// Work partition and exchange-buffer layout of the persistent decode kernel.
//
// Everything here is plain integer arithmetic shared by the device code and
// the host-side exhaustive bounds checker (layout_check.cpp), so every index
// the kernel forms can be verified on the CPU before a GPU ever runs it.
//
// Model shape: Qwen3-0.6B (Tools/megakernel/megakernel.cu:15-22,80-81).
// Grid: one 576-thread workgroup per CU of MI355X (256 CUs in 8 XCDs).
// Workgroup w owns:
//   QKV rows      [16w, 16w+16)                 of the 4096-row [Wq;Wk;Wv]
//   attention     kv head w%8, position split w/8 (32 splits per kv head)
//   combine       q head w/16, dims [8(w%16), 8(w%16)+8)
//   o_proj rows   [4w, 4w+4)       (residual rows of the same range)
//   gate/up rows  [12w, 12w+12)    of each of Wg and Wu
//   down rows     [4w, 4w+4)
//   lm_head rows  [593w + min(w,128), +593 + (w<128))  of 151936
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
constexpr int QKV_ROWS = QSZ + 2 * KVSZ;  // 4096
constexpr int VOCAB = 151936;
constexpr int MAX_LAYERS = 28;

constexpr int NWG = 256;          // workgroups = CUs
constexpr int NCW = 8;            // compute waves per workgroup
constexpr int NGW = 4;            // compute waves per group; stage j runs on group j % 2
constexpr int WAVE = 64;
constexpr int BLOCK = (NCW + 1) * WAVE;  // 8 compute waves + 1 exchange wave
constexpr int NSPLIT = NWG / NKV;  // 32 position splits per kv head
constexpr int MAX_SPLIT_POS = 64;  // positions per split at max context 2048

// ---- per-workgroup row ownership --------------------------------------------------
constexpr int QKV_PER_WG = QKV_ROWS / NWG;  // 16
constexpr int HID_PER_WG = HIDDEN / NWG;    // 4
constexpr int INT_PER_WG = INTER / NWG;     // 12
constexpr int LM_BASE = VOCAB / NWG;        // 593
constexpr int LM_EXTRA = VOCAB % NWG;       // 128
constexpr int LM_MAX_ROWS = LM_BASE + 1;    // 594
constexpr int LM_ROWS_PER_CHUNK = 6;        // rows per wave per pipeline stage
constexpr int LM_CHUNKS = (LM_MAX_ROWS + NGW * LM_ROWS_PER_CHUNK - 1) / (NGW * LM_ROWS_PER_CHUNK);  // 25

QL_HD int lm_row0(int w) { return LM_BASE * w + (w < LM_EXTRA ? w : LM_EXTRA); }
QL_HD int lm_rows(int w) { return LM_BASE + (w < LM_EXTRA ? 1 : 0); }
// local lm_head row handled by group member m (0..3), chunk k, slot i (may be >= lm_rows)
QL_HD int lm_local_row(int m, int k, int i) { return NGW * LM_ROWS_PER_CHUNK * k + LM_ROWS_PER_CHUNK * m + i; }

// QKV row r -> (matrix 0/1/2 = q/k/v, row within it)
QL_HD int qkv_matrix(int r) { return r < QSZ ? 0 : (r < QSZ + KVSZ ? 1 : 2); }
QL_HD int qkv_row_in(int r) { return r < QSZ ? r : (r < QSZ + KVSZ ? r - QSZ : r - QSZ - KVSZ); }

// attention role
QL_HD int att_kv(int w) { return w % NKV; }
QL_HD int att_split(int w) { return w / NKV; }
// positions per split for context length ctx (= position + 1)
QL_HD int att_span(int ctx) { return (ctx + NSPLIT - 1) / NSPLIT; }
QL_HD int att_t0(int ctx, int s) { return s * att_span(ctx); }
QL_HD int att_t1(int ctx, int s) {
  int e = att_t0(ctx, s) + att_span(ctx);
  return e < ctx ? e : ctx;
}
// position within the split handled by group member m (0..3), lane group j (0..3), slot b (0..3)
QL_HD int att_local_pos(int m, int j, int b) { return 16 * m + j + 4 * b; }

// combine role
QL_HD int cmb_head(int w) { return w / 16; }
QL_HD int cmb_d0(int w) { return 8 * (w % 16); }

// ---- exchange ("LL") buffers -------------------------------------------------------
// A slot is 8 bytes: 32 bits of payload + a 32-bit tag, written with one 8-byte
// device-scope store and read with device-scope loads; a reader accepts a slot
// only when its tag equals the tag of the step it waits for, so data and
// "ready" travel together. Format H2: payload = two fp16 values. Format F1:
// payload = one fp32 (or u32) value. Every buffer exists twice (layer parity
// for the per-layer buffers, token parity for ARG) so a fast workgroup never
// overwrites a slot a slow one has yet to read.
constexpr int X_SLOTS = HIDDEN / 2;         // 512   residual stream (H2)
constexpr int QKV_SLOTS = QKV_ROWS / 2;     // 2048  raw q|k|v (H2)
constexpr int PART_PER_HEAD = 2 + HD;       // m, l, acc[128] (F1)
constexpr int PART_SLOTS = NWG * 2 * PART_PER_HEAD;  // 66560
constexpr int ATT_SLOTS = QSZ / 2;          // 1024  combined attention (H2)
constexpr int ACT_SLOTS = HIDDEN / 2;       // 512   post-attention residual (H2)
constexpr int INT_SLOTS = INTER / 2;        // 1536  SiLU(gate)*up (H2)
constexpr int ARG_SLOTS = 2 * NWG;          // 512   per-WG (max, index) (F1)

constexpr long OFF_X = 0;
constexpr long OFF_QKV = OFF_X + 2L * X_SLOTS;
constexpr long OFF_PART = OFF_QKV + 2L * QKV_SLOTS;
constexpr long OFF_ATT = OFF_PART + 2L * PART_SLOTS;
constexpr long OFF_ACT = OFF_ATT + 2L * ATT_SLOTS;
constexpr long OFF_INT = OFF_ACT + 2L * ACT_SLOTS;
constexpr long OFF_ARG = OFF_INT + 2L * INT_SLOTS;
constexpr long TOTAL_SLOTS = OFF_ARG + 2L * ARG_SLOTS;
// after the slots: one 256-byte line of status words (error flags)
constexpr long WORKSPACE_BYTES = TOTAL_SLOTS * 8 + 256;

QL_HD long slot_x(int par, int k) { return OFF_X + (long)par * X_SLOTS + k; }
QL_HD long slot_qkv(int par, int k) { return OFF_QKV + (long)par * QKV_SLOTS + k; }
// partial of (kv head g, split s, local q head i), entry e in [0, 130)
QL_HD long slot_part(int par, int g, int s, int i, int e) {
  return OFF_PART + (long)par * PART_SLOTS + ((long)((g * NSPLIT + s) * 2 + i)) * PART_PER_HEAD + e;
}
QL_HD long slot_att(int par, int k) { return OFF_ATT + (long)par * ATT_SLOTS + k; }
QL_HD long slot_act(int par, int k) { return OFF_ACT + (long)par * ACT_SLOTS + k; }
QL_HD long slot_int(int par, int k) { return OFF_INT + (long)par * INT_SLOTS + k; }
QL_HD long slot_arg(int par, int k) { return OFF_ARG + (long)par * ARG_SLOTS + k; }

// QKV slots read by the attention workgroups of kv head g, as a list of 256:
// [0,128) q heads 2g and 2g+1, [128,192) k head g, [192,256) v head g.
QL_HD int att_in_slot(int g, int c) {
  return c < 128 ? 128 * g + c : (c < 192 ? QSZ / 2 + 64 * g + (c - 128) : (QSZ + KVSZ) / 2 + 64 * g + (c - 192));
}

// ---- exchange-wave poll addressing (byte offsets into the workspace) -------------
// The exchange wave reads two slots (16 B) per lane per load at byte
// voff(lane) + soff(k), with soff wave-uniform. Linear vectors: pair k of lane
// covers slots 2(lane + 64k), 2(lane + 64k) + 1.
QL_HD int lin_voff(int lane) { return 16 * lane; }
QL_HD long lin_soff(long base_slot, int k) { return base_slot * 8 + 1024L * k; }
// attention input of kv head g: load 0 = q slots, load 1 = k (lane < 32) / v (lane >= 32)
QL_HD int attq_voff(int lane) { return 16 * lane; }
QL_HD long attq_soff(int par, int g) { return slot_qkv(par, att_in_slot(g, 0)) * 8; }
QL_HD int attkv_voff(int lane) { return lane < 32 ? 16 * lane : 16 * (lane - 32) + 8 * (KVSZ / 2); }
QL_HD long attkv_soff(int par, int g) { return slot_qkv(par, QSZ / 2 + 64 * g) * 8; }
// combine of q head h (kv head h/2, local head h%2), dims [d0, d0+8): lane s < 32
// reads split s; load 0 = (m, l), loads 1..4 = acc pairs
QL_HD int cmb_voff(int lane) { return lane * 2 * PART_PER_HEAD * 8; }
QL_HD long cmb_soff(int par, int h, int d0, int k) {
  return slot_part(par, h / 2, 0, h % 2, k == 0 ? 0 : 2 + d0 + 2 * (k - 1)) * 8;
}

// ---- step tags ----------------------------------------------------------------------
// tag = epoch << 8 | stage id; epoch counts tokens (never 0), stage id names
// the buffer written within the token.
enum StageId : int { SID_QKV = 0, SID_PART = 1, SID_ATT = 2, SID_ACT = 3, SID_INT = 4, SID_X = 5 };
QL_HD unsigned tag_of(unsigned epoch, int layer, int sid) { return (epoch << 8) | (unsigned)(layer * 8 + sid); }
QL_HD unsigned tag_arg(unsigned epoch) { return (epoch << 8) | 250u; }

// ---- compute-wave stage sequence ---------------------------------------------------
enum CType : int { C_QKV = 0, C_ATT = 1, C_OPROJ = 2, C_GU = 3, C_DOWN = 4, C_LMH = 5 };
enum Mode : int { MODE_DECODE = 0, MODE_LMHEAD = 1, MODE_MLP = 2 };

struct StageDesc {
  int type;   // CType
  int layer;  // transformer layer (QKV..DOWN)
  int chunk;  // lm_head chunk (LMH)
  int token;  // token index within the launch
  int fin;    // global index of the finalised stage this stage belongs to
};

// compute stages per token and finalised stages per token
QL_HD int stages_per_token(int mode, int L) {
  return mode == MODE_DECODE ? 5 * L + LM_CHUNKS : (mode == MODE_LMHEAD ? LM_CHUNKS : 2);
}
QL_HD int fins_per_token(int mode, int L) { return mode == MODE_DECODE ? 5 * L + 1 : (mode == MODE_LMHEAD ? 1 : 2); }

QL_HD StageDesc stage_desc(int mode, int L, int i) {
  StageDesc d;
  const int st = stages_per_token(mode, L);
  d.token = i / st;
  const int r = i % st;
  const int base = d.token * fins_per_token(mode, L);
  d.layer = 0;
  d.chunk = 0;
  if (mode == MODE_DECODE) {
    if (r < 5 * L) {
      d.type = r % 5;
      d.layer = r / 5;
      d.fin = base + r;
    } else {
      d.type = C_LMH;
      d.chunk = r - 5 * L;
      d.fin = base + 5 * L;
    }
  } else if (mode == MODE_LMHEAD) {
    d.type = C_LMH;
    d.chunk = r;
    d.fin = base;
  } else {
    d.type = r == 0 ? C_GU : C_DOWN;
    d.fin = base + r;
  }
  return d;
}

}  // namespace ql
