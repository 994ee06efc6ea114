// Exhaustive CPU check of every index the decode kernel forms (qwen_layout.h):
// work partitions cover their ranges exactly once, every exchange-slot read and
// write stays inside its own buffer, poll offsets address the intended slots,
// and the stage sequence is consistent. Exit status 0 = all checks passed.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "qwen_layout.h"

using namespace ql;

static int g_fail = 0;
#define CHECK(cond, ...)                          \
  do {                                            \
    if (!(cond)) {                                \
      if (g_fail < 20) {                          \
        fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
        fprintf(stderr, __VA_ARGS__);             \
        fprintf(stderr, "\n");                    \
      }                                           \
      ++g_fail;                                   \
    }                                             \
  } while (0)

static bool in_buf(long slot, long off, long n) { return slot >= off && slot < off + n; }

int main() {
  // buffers: disjoint, in order, inside the workspace, pair-aligned
  const long offs[] = {OFF_X, OFF_QKV, OFF_PART, OFF_ATT, OFF_ACT, OFF_INT, OFF_ARG, TOTAL_SLOTS};
  const long sizes[] = {2L * X_SLOTS, 2L * QKV_SLOTS, 2L * PART_SLOTS, 2L * ATT_SLOTS,
                        2L * ACT_SLOTS, 2L * INT_SLOTS, 2L * ARG_SLOTS};
  for (int b = 0; b < 7; ++b) {
    CHECK(offs[b] + sizes[b] == offs[b + 1], "buffer %d not contiguous", b);
    CHECK(offs[b] % 2 == 0, "buffer %d base not pair aligned", b);
  }
  CHECK(TOTAL_SLOTS * 8 + 256 == WORKSPACE_BYTES, "workspace size");
  CHECK(WORKSPACE_BYTES < (1L << 31), "workspace offsets must fit the 32-bit buffer offset");
  CHECK(BLOCK == 576 && NWG * QKV_PER_WG == QKV_ROWS && NWG * HID_PER_WG == HIDDEN && NWG * INT_PER_WG == INTER,
        "partition constants");

  // QKV rows: each of the 4096 rows exactly once; matrix/row mapping in range
  {
    std::vector<int> seen(QKV_ROWS, 0);
    for (int w = 0; w < NWG; ++w)
      for (int m = 0; m < NGW; ++m)
        for (int r = 0; r < 4; ++r) {
          int row = QKV_PER_WG * w + 4 * m + r;
          CHECK(row < QKV_ROWS, "qkv row");
          seen[row]++;
          int mat = qkv_matrix(row), ri = qkv_row_in(row);
          int lim = mat == 0 ? QSZ : KVSZ;
          CHECK(ri >= 0 && ri < lim, "qkv row_in %d", row);
          CHECK((mat == 0 ? ri : (mat == 1 ? QSZ + ri : QSZ + KVSZ + ri)) == row, "qkv map %d", row);
        }
    for (int r = 0; r < QKV_ROWS; ++r) CHECK(seen[r] == 1, "qkv row %d seen %d", r, seen[r]);
    // finalize slots: slot 8w + lane holds rows 16w + 2 lane, +1
    for (int w = 0; w < NWG; ++w)
      for (int lane = 0; lane < QKV_PER_WG / 2; ++lane)
        for (int par = 0; par < 2; ++par) {
          long s = slot_qkv(par, (QKV_PER_WG / 2) * w + lane);
          CHECK(in_buf(s, OFF_QKV + par * QKV_SLOTS, QKV_SLOTS), "qkv slot");
        }
  }

  // attention input poll: load 0 / load 1 address exactly att_in_slot(g, 2(lane + 64k))
  for (int par = 0; par < 2; ++par)
    for (int g = 0; g < NKV; ++g) {
      std::vector<int> seen(256, 0);
      for (int lane = 0; lane < WAVE; ++lane) {
        long b0 = attq_voff(lane) + attq_soff(par, g);
        long b1 = attkv_voff(lane) + attkv_soff(par, g);
        CHECK(b0 % 16 == 0 && b1 % 16 == 0, "att poll alignment");
        CHECK(b0 == slot_qkv(par, att_in_slot(g, 2 * lane)) * 8, "att q poll g%d lane%d", g, lane);
        CHECK(b1 == slot_qkv(par, att_in_slot(g, 2 * (lane + 64))) * 8, "att kv poll g%d lane%d", g, lane);
        for (int k = 0; k < 2; ++k) {
          int c = 2 * (lane + 64 * k);
          seen[c]++;
          seen[c + 1]++;
          // the pair never straddles a q|k|v segment
          CHECK(att_in_slot(g, c + 1) == att_in_slot(g, c) + 1, "att pair contiguity");
        }
      }
      for (int c = 0; c < 256; ++c) CHECK(seen[c] == 1, "att input %d", c);
      // q slots hold q heads 2g, 2g+1; k slots k head g; v slots v head g
      for (int c = 0; c < 256; ++c) {
        int slot = att_in_slot(g, c), v0 = 2 * slot;  // first value index in the 4096-vector
        if (c < 128) CHECK(v0 >= 256 * g && v0 < 256 * g + 256, "q segment");
        else if (c < 192) CHECK(v0 >= QSZ + 128 * g && v0 < QSZ + 128 * g + 128, "k segment");
        else CHECK(v0 >= QSZ + KVSZ + 128 * g && v0 < QSZ + KVSZ + 128 * g + 128, "v segment");
      }
    }

  // attention positions: every position of every context exactly once, <= 64 per split
  for (int ctx = 1; ctx <= NSPLIT * MAX_SPLIT_POS; ++ctx) {
    CHECK(att_span(ctx) <= MAX_SPLIT_POS, "span ctx %d", ctx);
    std::vector<int> seen(ctx, 0);
    for (int s = 0; s < NSPLIT; ++s) {
      int t0 = att_t0(ctx, s), t1 = att_t1(ctx, s);
      for (int m = 0; m < NGW; ++m)
        for (int j = 0; j < 4; ++j)
          for (int b = 0; b < 4; ++b) {
            int lp = att_local_pos(m, j, b);
            CHECK(lp >= 0 && lp < MAX_SPLIT_POS, "local pos");
            int p = t0 + lp;
            if (p < t1) {
              CHECK(p >= 0 && p < ctx, "pos range");
              seen[p]++;
            }
          }
    }
    for (int p = 0; p < ctx; ++p) CHECK(seen[p] == 1, "ctx %d pos %d seen %d", ctx, p, seen[p]);
    // exactly one split holds the newest position
    int holders = 0;
    for (int s = 0; s < NSPLIT; ++s) holders += (att_t0(ctx, s) <= ctx - 1 && ctx - 1 < att_t1(ctx, s));
    CHECK(holders == 1, "pos holder ctx %d", ctx);
  }
  // each (kv head, split) pair is one workgroup
  {
    std::vector<int> seen(NWG, 0);
    for (int w = 0; w < NWG; ++w) seen[att_kv(w) * NSPLIT + att_split(w)]++;
    for (int i = 0; i < NWG; ++i) CHECK(seen[i] == 1, "att role %d", i);
  }
  // partial slots written by the attention finalizer stay in their buffer
  for (int par = 0; par < 2; ++par)
    for (int w = 0; w < NWG; ++w)
      for (int e = 0; e < 2 * PART_PER_HEAD; ++e) {
        int h = e >= PART_PER_HEAD, k = e - PART_PER_HEAD * h;
        long s = slot_part(par, att_kv(w), att_split(w), h, k);
        CHECK(in_buf(s, OFF_PART + par * PART_SLOTS, PART_SLOTS), "part slot");
      }

  // combine: 2048 attention outputs exactly once; poll offsets hit (m,l) and acc pairs
  {
    std::vector<int> seen(QSZ, 0);
    for (int w = 0; w < NWG; ++w) {
      int h = cmb_head(w), d0 = cmb_d0(w);
      CHECK(h < NQ && d0 + 8 <= HD, "combine role");
      for (int e = 0; e < 8; ++e) seen[h * HD + d0 + e]++;
      CHECK(8 * w == h * HD + d0, "combine output slots");
      for (int par = 0; par < 2; ++par)
        for (int lane = 0; lane < NSPLIT; ++lane)
          for (int k = 0; k < 5; ++k) {
            long b = cmb_voff(lane) + cmb_soff(par, h, d0, k);
            long expect = slot_part(par, h / 2, lane, h % 2, k == 0 ? 0 : 2 + d0 + 2 * (k - 1)) * 8;
            CHECK(b == expect && b % 16 == 0, "combine poll w%d lane%d k%d", w, lane, k);
            CHECK(in_buf(b / 8, OFF_PART + par * PART_SLOTS, PART_SLOTS) &&
                      in_buf(b / 8 + 1, OFF_PART + par * PART_SLOTS, PART_SLOTS),
                  "combine poll range");
          }
      for (int lane = 0; lane < 4; ++lane)
        CHECK(in_buf(slot_att(0, 4 * w + lane), OFF_ATT, ATT_SLOTS), "att slot");
    }
    for (int i = 0; i < QSZ; ++i) CHECK(seen[i] == 1, "combine out %d", i);
  }

  // o_proj / down rows (4 per WG, one per group member), gate/up (12 + 12 per WG, 6 per member)
  {
    std::vector<int> oseen(HIDDEN, 0), gseen(INTER, 0), useen(INTER, 0);
    for (int w = 0; w < NWG; ++w) {
      for (int m = 0; m < NGW; ++m) oseen[HID_PER_WG * w + m]++;
      for (int m = 0; m < NGW; ++m)
        for (int k = 0; k < 6; ++k) {
          int lr = 6 * m + k;
          int row = INT_PER_WG * w + (lr % INT_PER_WG);
          (lr < INT_PER_WG ? gseen : useen)[row]++;
        }
      for (int lane = 0; lane < 2; ++lane) {
        CHECK(in_buf(slot_act(1, 2 * w + lane), OFF_ACT + ACT_SLOTS, ACT_SLOTS), "act slot");
        CHECK(in_buf(slot_x(1, 2 * w + lane), OFF_X + X_SLOTS, X_SLOTS), "x slot");
      }
      for (int lane = 0; lane < INT_PER_WG / 2; ++lane)
        CHECK(in_buf(slot_int(1, (INT_PER_WG / 2) * w + lane), OFF_INT + INT_SLOTS, INT_SLOTS), "int slot");
      for (int lane = 0; lane < 2; ++lane) CHECK(in_buf(slot_arg(1, 2 * w + lane), OFF_ARG + ARG_SLOTS, ARG_SLOTS), "arg");
    }
    for (int i = 0; i < HIDDEN; ++i) CHECK(oseen[i] == 1, "o/down row %d", i);
    for (int i = 0; i < INTER; ++i) CHECK(gseen[i] == 1 && useen[i] == 1, "gate/up row %d", i);
    // activation offsets read per lane: 8 lane + 512k + 8 <= 2048 (o_proj, k < 4), <= 3072 (down, k < 6)
    for (int lane = 0; lane < WAVE; ++lane) {
      for (int k = 0; k < 4; ++k) CHECK(512 * k + 8 * lane + 8 <= QSZ, "o_proj act index");
      for (int k = 0; k < 6; ++k) CHECK(512 * k + 8 * lane + 8 <= INTER, "down act index");
    }
  }

  // linear polls: pair k of lane covers slots 2(lane+64k), +1 inside the buffer
  {
    struct V { long base; int n; const char* name; } vecs[] = {
        {slot_x(1, 0), X_SLOTS, "x"}, {slot_att(1, 0), ATT_SLOTS, "att"}, {slot_act(1, 0), ACT_SLOTS, "act"},
        {slot_int(1, 0), INT_SLOTS, "int"}, {slot_arg(1, 0), ARG_SLOTS, "arg"}};
    for (auto& v : vecs) {
      std::vector<int> seen(v.n, 0);
      const int K = v.n / 128;
      for (int lane = 0; lane < WAVE; ++lane)
        for (int k = 0; k < K; ++k) {
          long b = lin_voff(lane) + lin_soff(v.base, k);
          long s = b / 8 - v.base;
          CHECK(b % 16 == 0 && s == 2 * (lane + 64 * k), "%s poll address", v.name);
          CHECK(s >= 0 && s + 1 < v.n, "%s poll range", v.name);
          if (s >= 0 && s + 1 < v.n) {
            seen[s]++;
            seen[s + 1]++;
          }
        }
      for (int i = 0; i < v.n; ++i) CHECK(seen[i] == 1, "%s slot %d read %d", v.name, i, seen[i]);
    }
  }

  // lm_head rows: [0, VOCAB) exactly once over (w, c, chunk, i)
  {
    std::vector<int> seen(VOCAB, 0);
    CHECK(lm_row0(NWG - 1) + lm_rows(NWG - 1) == VOCAB, "lm rows end");
    for (int w = 0; w < NWG; ++w) {
      CHECK(lm_rows(w) <= LM_MAX_ROWS, "lm rows");
      for (int m = 0; m < NGW; ++m)
        for (int k = 0; k < LM_CHUNKS; ++k)
          for (int i = 0; i < LM_ROWS_PER_CHUNK; ++i) {
            int lr = lm_local_row(m, k, i);
            if (lr < lm_rows(w)) seen[lm_row0(w) + lr]++;
          }
    }
    for (int r = 0; r < VOCAB; ++r) CHECK(seen[r] == 1, "lm row %d seen %d", r, seen[r]);
  }

  // tags: distinct per (layer, stage id) and never the ARG tag; 24-bit epochs fit
  {
    std::vector<int> seen(256, 0);
    for (int l = 0; l < MAX_LAYERS; ++l)
      for (int sid = 0; sid <= SID_X; ++sid) seen[tag_of(0, l, sid)]++;
    seen[tag_arg(0)]++;
    for (int i = 0; i < 256; ++i) CHECK(seen[i] <= 1, "tag collision %d", i);
    CHECK(tag_of(1, 0, 0) != 0 && tag_arg(1) != 0, "tags of epoch >= 1 are never 0");
    CHECK((tag_of((1u << 24) - 1, 27, SID_X) >> 8) == (1u << 24) - 1, "24-bit epoch");
  }

  // stage sequence: fin non-decreasing, +1 steps, LMH chunks share one fin; types cycle
  for (int mode = 0; mode < 3; ++mode)
    for (int L = 1; L <= MAX_LAYERS; ++L) {
      if (mode != MODE_DECODE && L != 1) continue;
      const int steps = 3, total = stages_per_token(mode, L) * steps;
      int prev_fin = -1, nfin = 0;
      for (int i = 0; i < total; ++i) {
        StageDesc d = stage_desc(mode, L, i);
        CHECK(d.token == i / stages_per_token(mode, L), "token");
        CHECK(d.fin == prev_fin || d.fin == prev_fin + 1, "fin step mode%d L%d i%d", mode, L, i);
        if (d.fin != prev_fin) ++nfin;
        prev_fin = d.fin;
        CHECK(d.layer >= 0 && d.layer < L, "layer");
        CHECK(d.chunk >= 0 && d.chunk < LM_CHUNKS, "chunk");
        if (mode == MODE_DECODE && d.type != C_LMH) CHECK(d.type == (i % stages_per_token(mode, L)) % 5, "type order");
      }
      CHECK(nfin == fins_per_token(mode, L) * steps, "fin count mode%d L%d", mode, L);
    }

  if (g_fail) {
    fprintf(stderr, "layout_check: %d failures\n", g_fail);
    return 1;
  }
  printf("layout_check: all checks passed\n");
  return 0;
}
