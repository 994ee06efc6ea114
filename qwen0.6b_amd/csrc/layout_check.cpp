// Exhaustive CPU check of every index the decode kernel forms (qwen_layout.h):
// work partitions cover their ranges exactly once, every exchange-slot read and
// write stays inside its own buffer, the poll addresses (per-lane offset +
// wave-uniform base, exactly as the kernel forms them) hit the intended slots,
// ring lines stay inside their matrices, and the attention split schedule
// covers every context. Exit status 0 = all checks passed.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "qwen_layout.h"

using namespace ql;

static int g_fail = 0;
#define CHECK(cond, ...)                                     \
  do {                                                       \
    if (!(cond)) {                                           \
      if (g_fail < 20) {                                     \
        fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
        fprintf(stderr, __VA_ARGS__);                        \
        fprintf(stderr, "\n");                               \
      }                                                      \
      ++g_fail;                                              \
    }                                                        \
  } while (0)

static bool in_buf(long slot, long off, long n) { return slot >= off && slot < off + n; }

int main() {
  // ---- exchange layout: buffers contiguous, pair-aligned, inside the workspace ----
  const long offs[] = {B_X, B_QKV, B_PART, B_ATTO, B_OP, B_ACT, B_INT, B_DP, XCD_SLOTS};
  const long sizes[] = {X_SLOTS, QKV_SLOTS, PART_SLOTS, ATTO_SLOTS, OP_SLOTS, ACT_SLOTS, INT_SLOTS, DP_SLOTS};
  for (int b = 0; b < 8; ++b) {
    CHECK(offs[b] + sizes[b] == offs[b + 1], "buffer %d not contiguous", b);
    CHECK(offs[b] % 2 == 0 && sizes[b] % 2 == 0, "buffer %d not pair aligned", b);
  }
  CHECK(XCD_SLOTS % 2 == 0 && OFF_ARG % 2 == 0, "xcd / arg alignment");
  CHECK(xbuf(1, NXCD - 1, XCD_SLOTS) == OFF_ARG, "xcd buffers end at the ARG buffer");
  CHECK(OFF_ARG + 2L * ARG_SLOTS == OFF_LOGIT && OFF_LOGIT + LOGIT_SLOTS == OFF_SEL &&
            OFF_SEL + SEL_SLOTS == OFF_DIST && OFF_DIST + DIST_SLOTS == TOTAL_SLOTS, "ARG, LOGIT, SEL, DIST end");
  CHECK(OFF_DIST % 2 == 0, "DIST pairs are 16-byte aligned");
  // DIST tags sit between the stage tags and the LOGIT / SEL / ARG tags of the same epoch
  CHECK((tag_of(1, MAX_LAYERS - 1, NSTAGE - 1) & 255u) < (tag_dist(1, 0) & 255u) &&
            (tag_dist(1, DIST_ROUNDS - 1) & 255u) < (tag_sel(1) & 255u), "DIST tags are distinct");
  CHECK(dhist_off(1, DHIST_PASSES - 1) + 256 * 8 == 256 + LM_CTR_BYTES + DHIST_BYTES &&
            TOTAL_SLOTS * 8 + dhist_off(0, 0) + DHIST_BYTES == WORKSPACE_BYTES, "DHIST ends the workspace");
  CHECK(OFF_LOGIT % 2 == 0 && LOGIT_SLOTS % 2 == 0 && OFF_SEL % 2 == 0, "LOGIT / SEL pairs are 16-byte aligned");
  CHECK(OFF_LOGIT % LM_CHUNK == 0 && slot_logit(0) == OFF_LOGIT && slot_logit(VOCAB - 1) == OFF_LOGIT + VOCAB - 1,
        "an lm_head chunk's logits are one 64-byte line");
  CHECK((SL_ROWS - 1) * NWG + SL_FULL == VOCAB && SL_FULL > 0 && SL_FULL <= NWG, "slices cover the vocabulary");
  {
    long used = 0;
    for (int w = 0; w < NWG; ++w) {
      used += slice_rows(w);
      CHECK(w + (long)NWG * (slice_rows(w) - 1) < VOCAB && w + (long)NWG * slice_rows(w) >= VOCAB, "slice w's rows");
    }
    CHECK(used == VOCAB, "slice sizes sum to the vocabulary");
  }
  CHECK(TOTAL_SLOTS * 8 + 256 + LM_CTR_BYTES + DHIST_BYTES == WORKSPACE_BYTES && WORKSPACE_BYTES < (1L << 31), "workspace size");
  CHECK(BLOCK == 512 && NLOC == 32 && NXCD * NLOC == NWG, "grid constants");
  for (int w = 0; w < NWG; ++w) CHECK(8 * loc_of(w) + xcd_of(w) == w, "w = 8 i + x");

  // ---- QKV rows: over all (x, i, c, r) each row of Wq, Wk, Wv exactly once ----
  {
    std::vector<int> q(QSZ, 0), k(KVSZ, 0), v(KVSZ, 0);
    for (int x = 0; x < NXCD; ++x)
      for (int i = 0; i < NLOC; ++i)
        for (int c = 0; c < NCW; ++c)
          for (int r = 0; r < 4; ++r) {
            const int gr = QKV_PER_WG * i + 4 * c + r;
            CHECK(gr < GRP_ROWS, "group row");
            const int mat = grp_matrix(gr), row = grp_row_in(x, gr);
            if (mat == 0) {
              CHECK(row >= 0 && row < QSZ && row / HD == 2 * x + gr / HD, "q row %d", row);
              if (row >= 0 && row < QSZ) q[row]++;
            } else {
              CHECK(row >= 0 && row < KVSZ && row / HD == x, "k/v row %d", row);
              if (row >= 0 && row < KVSZ) (mat == 1 ? k : v)[row]++;
            }
            // the store slot holds group rows 2s, 2s+1 of this workgroup's 16
            const int slot = (QKV_PER_WG / 2) * i + 2 * c + r / 2;
            CHECK(2 * slot + (r & 1) == gr && slot < QKV_SLOTS, "qkv slot");
          }
    for (int r = 0; r < QSZ; ++r) CHECK(q[r] == 1, "q row %d seen %d", r, q[r]);
    for (int r = 0; r < KVSZ; ++r) CHECK(k[r] == 1 && v[r] == 1, "k/v row %d", r);
    // ring lines of the QKV stage: line m = row m / 2, half m % 2
    for (int m = 0; m < LINES_QKV - LINES_NORM; ++m) CHECK((m >> 1) < QKV_PER_WG, "qkv line");
  }

  // ---- attention input poll: wave c, lane < 32 -> slots 64 c + 2 lane, +1 = values
  //      128 c + 4 lane .. +4, gathered in LDS; every lane then reads q values [4 lane, +4)
  //      and k | v values [256 + 4 lane, +4) ----
  {
    std::vector<int> seen(GRP_ROWS, 0);
    for (int c = 0; c < NCW; ++c)
      for (int lane = 0; lane < 32; ++lane) {
        const long slot = 64 * c + (16 * lane) / 8;  // (soff + voff) / 8 relative to the buffer
        CHECK(slot % 2 == 0 && slot + 1 < QKV_SLOTS, "att poll range");
        for (int e = 0; e < 4; ++e) {
          CHECK(2 * (int)slot + e == 128 * c + 4 * lane + e, "att gather index");
          seen[2 * (int)slot + e]++;
        }
      }
    for (int e = 0; e < GRP_ROWS; ++e) CHECK(seen[e] == 1, "att input %d", e);
  }

  // ---- attention split schedule: every position of every context exactly once ----
  for (int ctx = 1; ctx <= MAX_SEQ_LIMIT; ++ctx) {
    const int pos = ctx - 1;
    std::vector<int> seen(ctx, 0);
    int holders = 0;
    for (int s = 0; s < NSPLIT; ++s) {
      const int t0 = att_t0(ctx, s), t1 = att_t1(ctx, s), nk = att_nk(ctx, s);
      CHECK(t0 % 4 == 0 && t1 >= t0 && t1 <= (ctx > t0 ? ctx : t0), "split range ctx %d s %d", ctx, s);
      CHECK(nk <= 16 && 2 * nk <= RING_LINES, "split lines ctx %d", ctx);
      CHECK(nk == 0 || (t0 + 4 * nk >= t1 && t0 + 4 * (nk - 1) < t1), "nk covers the split");
      holders += (t0 <= pos && pos < t1);
      // positions the compute waves treat as valid: m = 4c + bb < nk, p = t0 + 4m + j < t1
      for (int c = 0; c < NCW; ++c)
        for (int bb = 0; bb < 4; ++bb)
          for (int j = 0; j < 4; ++j) {
            const int m = 4 * c + bb, p = t0 + 4 * m + j;
            if (m < nk && p < t1) {
              CHECK(p >= 0 && p < ctx, "pos range");
              seen[p]++;
            }
          }
      // loader: cached positions p < min(t1, pos), inside the cache rows
      for (int m = 0; m < nk; ++m)
        for (int lane = 0; lane < WAVE; ++lane) {
          const int p = t0 + 4 * m + (lane >> 4);
          const int lim = t1 < pos ? t1 : pos;
          if (p < lim) CHECK(p >= 0 && p < pos && p < MAX_SEQ_LIMIT, "cached position");
        }
    }
    for (int p = 0; p < ctx; ++p) CHECK(seen[p] == 1, "ctx %d pos %d seen %d", ctx, p, seen[p]);
    CHECK(holders == 1, "pos holder ctx %d", ctx);
  }

  // ---- attention partial stores and the combine poll ----
  {
    for (int i = 0; i < NLOC; ++i)
      for (int c = 0; c < NCW; ++c)
        for (int it = 0; it < 2; ++it)
          for (int lane = 0; lane < WAVE; ++lane) {
            if (it == 1 && lane != 0) continue;
            const int e = 65 * c + (it == 0 ? lane : 64);
            const int h = e >= PART_PER_HEAD ? 1 : 0, k = e - PART_PER_HEAD * h;
            CHECK(e < 2 * PART_PER_HEAD && k >= 0 && k < PART_PER_HEAD, "merge entry");
            CHECK(part_index(i, h, k) < PART_SLOTS, "part slot");
          }
    std::vector<int> seen(OCOLS, 0);
    for (int i = 0; i < NLOC; ++i) {
      const int hh = i / 16, d0 = 8 * (i % 16);
      for (int e = 0; e < 8; ++e) seen[hh * HD + d0 + e]++;
      CHECK(8 * i == hh * HD + d0, "ATTO value order");
      // wave c merges dims d0 + 2 c, +1: lane s < 32 polls (m, l) and that dim pair of split s
      for (int c = 0; c < NCW; ++c) {
        for (int s = 0; s < NSPLIT; ++s)
          for (const int e : {0, 2 + d0 + 2 * c}) {
            const long slot = part_index(s, hh, e);
            CHECK(slot % 2 == 0 && slot + 1 < PART_SLOTS, "combine poll");
          }
        CHECK(4 * i + c < ATTO_SLOTS && 2 * (4 * i + c) == hh * HD + d0 + 2 * c, "atto slot");
      }
    }
    for (int e = 0; e < OCOLS; ++e) CHECK(seen[e] == 1, "combine value %d", e);
  }

  // ---- o_proj: ATTO poll (lane -> values [8 (lane % 32), +8) = slots 4 (lane % 32) .. +3,
  //      the columns its ring lines hold), ring lines, partial rows ----
  {
    std::vector<int> seen(OCOLS, 0);
    for (int lane = 0; lane < 32; ++lane)
      for (const int voff : {32 * lane, 32 * lane + 16}) {
        const int slot = voff / 8;
        CHECK(slot % 2 == 0 && slot + 1 < ATTO_SLOTS, "atto poll");
        CHECK(2 * slot >= 8 * lane && 2 * slot + 4 <= 8 * lane + 8, "atto values match the lane's columns");
        for (int e = 0; e < 4; ++e) seen[2 * slot + e]++;
      }
    for (int e = 0; e < OCOLS; ++e) CHECK(seen[e] == 1, "o input %d", e);
    std::vector<int> rows(HIDDEN * NXCD, 0);
    for (int x = 0; x < NXCD; ++x)
      for (int i = 0; i < NLOC; ++i)
        for (int m = 0; m < LINES_O; ++m)
          for (int lane = 0; lane < WAVE; ++lane) {
            const int row = HROWS * i + 2 * m + (lane >> 5), col = OCOLS * x + 8 * (lane & 31);
            CHECK(row < HIDDEN && col + 8 <= QSZ && col >= OCOLS * x && col + 8 <= OCOLS * (x + 1), "o line");
            if ((lane & 31) == 0) rows[x * HIDDEN + row]++;
          }
    for (int r = 0; r < HIDDEN * NXCD; ++r) CHECK(rows[r] == 1, "o row %d", r);
    // compute wave c: lines 4c + m; stored rows 8c + {0,2,1,3} (+4)
    for (int c = 0; c < NCW; ++c) {
      std::vector<int> rs(8, 0);
      for (int l16 = 0; l16 < 4; ++l16) {
        const int rr = (l16 == 1 ? 2 : (l16 == 2 ? 1 : l16));
        rs[rr]++;
        rs[rr + 4]++;
        // the line holding that row: (rr / 2) within the first pair of lines
        const int line_y0 = 4 * c + (l16 & 1), half = l16 >> 1;
        CHECK(2 * line_y0 + half == 8 * c + rr, "o row from y0");
        const int line_y1 = 4 * c + 2 + (l16 & 1);
        CHECK(2 * line_y1 + half == 8 * c + rr + 4, "o row from y1");
      }
      for (int r = 0; r < 8; ++r) CHECK(rs[r] == 1, "o store rows");
    }
  }

  // ---- residual sums: wave c, lane < 32 polls XCD lane / 4, rows 8 c + 2 (lane % 4), +1 ----
  for (int par = 0; par < 2; ++par)
    for (int i = 0; i < NLOC; ++i)
      for (const long B : {B_OP, B_DP}) {
        std::vector<int> seen(NXCD * HROWS, 0);
        for (int c = 0; c < NCW; ++c) {
          const long src0 = xbuf(par, 0, B) + HROWS * i + 8 * c;
          for (int lane = 0; lane < 32; ++lane) {
            const int g = (lane >> 2) & 7, pr = lane & 3, r = 8 * c + 2 * pr;
            const long slot = src0 + ((long)g * XCD_SLOTS + 2 * pr);
            CHECK(slot == xbuf(par, g, B) + HROWS * i + r && slot % 2 == 0, "peer poll address");
            CHECK(in_buf(slot, xbuf(par, g, B), HIDDEN) && in_buf(slot + 1, xbuf(par, g, B), HIDDEN), "peer range");
            // DPP row_ror 8 and 4 sum lanes pr + 4 g' of one 16-lane row; rows 0 and 1 hold g < 4 and g >= 4
            CHECK(lane / 16 == g / 4 && (lane % 16) / 4 == g % 4, "peer lane placement");
            seen[g * HROWS + r]++;
            seen[g * HROWS + r + 1]++;
          }
        }
        for (int e = 0; e < NXCD * HROWS; ++e) CHECK(seen[e] == 1, "peer row %d", e);
      }
  // residual row stores: ACT / X slots 16 i + 4 c + lane hold rows 32 i + 8 c + 2 lane, +1
  {
    std::vector<int> seen(HIDDEN, 0);
    for (int i = 0; i < NLOC; ++i)
      for (int c = 0; c < NCW; ++c)
        for (int lane = 0; lane < 4; ++lane) {
          const int slot = 16 * i + 4 * c + lane;
          CHECK(slot < X_SLOTS && 2 * slot == HROWS * i + 8 * c + 2 * lane, "x slot rows");
          seen[2 * slot]++;
          seen[2 * slot + 1]++;
        }
    for (int r = 0; r < HIDDEN; ++r) CHECK(seen[r] == 1, "x row %d", r);
    // quarter polls of a 1024-value vector: wave c, lane -> slots 128 c + 2 lane, +1 =
    // values 256 c + 4 lane .. +4, gathered in LDS; lanes then read [8 lane, +8) and [512 + 8 lane, +8)
    std::vector<int> got(HIDDEN, 0);
    for (int c = 0; c < NCW; ++c)
      for (int lane = 0; lane < WAVE; ++lane) {
        const int slot = 128 * c + 2 * lane;
        CHECK(slot + 1 < X_SLOTS, "x poll");
        for (int e = 0; e < 4; ++e) {
          CHECK(2 * slot + e == 256 * c + 4 * lane + e, "x gather index");
          got[2 * slot + e]++;
        }
      }
    for (int r = 0; r < HIDDEN; ++r) CHECK(got[r] == 1, "x value %d", r);
  }

  // ---- gate/up rows, INT slots, down input order ----
  {
    std::vector<int> g(INTER, 0);
    for (int x = 0; x < NXCD; ++x)
      for (int i = 0; i < NLOC; ++i)
        for (int m = 0; m < LINES_GU - LINES_NORM; ++m) {
          const bool up = m >= 2 * GU_PER_WG;
          const int mm = up ? m - 2 * GU_PER_WG : m;
          const int row = ICOLS * x + GU_PER_WG * i + (mm >> 1);
          CHECK(row < INTER, "gu row");
          if (!up && (mm & 1) == 0) g[row]++;
        }
    for (int r = 0; r < INTER; ++r) CHECK(g[r] == 1, "gate row %d", r);
    // compute wave c: gate rows 3c + jj at lines 2(3c + jj), up at 24 + 2(3c + jj)
    for (int c = 0; c < NCW; ++c)
      for (int jj = 0; jj < 3; ++jj) CHECK(LINES_NORM + 2 * GU_PER_WG + 2 * (3 * c + jj) + 1 < LINES_GU, "gu lines");
    // INT slots and the down poll: wave c, lane < 32 -> pair k = 32 c + lane (slots 2 k, 2 k + 1)
    // = workgroup k / 4, wave k % 4: values 12 (k / 4) + 3 (k % 4) + {0, 1, 2}, gathered in LDS
    std::vector<int> seen(ICOLS, 0);
    for (int c = 0; c < NCW; ++c)
      for (int lane = 0; lane < 32; ++lane) {
        const int k = 32 * c + lane, slot = 64 * c + 2 * lane;
        CHECK(slot == int_slot(k >> 2, k & 3, 0) && slot + 1 == int_slot(k >> 2, k & 3, 1), "int slots");
        CHECK(slot + 1 < INT_SLOTS, "int range");
        for (int e = 0; e < 3; ++e) seen[GU_PER_WG * (k >> 2) + 3 * (k & 3) + e]++;
      }
    for (int e = 0; e < ICOLS; ++e) CHECK(seen[e] == 1, "inter value %d", e);
    // down ring lines: row 32 i + m, columns 384 x + 8 ln (ln < 48)
    std::vector<int> rows(HIDDEN * NXCD, 0);
    for (int x = 0; x < NXCD; ++x)
      for (int i = 0; i < NLOC; ++i)
        for (int m = 0; m < LINES_DOWN; ++m)
          for (int lane = 0; lane < WAVE; ++lane) {
            const int ln = lane < 48 ? lane : lane - 48;
            const int row = HROWS * i + m, col = ICOLS * x + 8 * ln;
            CHECK(row < HIDDEN && col >= ICOLS * x && col + 8 <= ICOLS * (x + 1), "down line");
            if (lane == 0) rows[x * HIDDEN + row]++;
          }
    for (int r = 0; r < HIDDEN * NXCD; ++r) CHECK(rows[r] == 1, "down row %d", r);
  }

  // ---- loader streams: every line / lane element equals the per-line row-column formula ----
  {
    // element counts of the sources (K/V: one kv head of one layer)
    const int max_seq = MAX_SEQ_LIMIT;
    const long msize[15] = {(long)QSZ * HIDDEN, (long)KVSZ * HIDDEN, (long)KVSZ * HIDDEN, (long)max_seq * HD,
                            (long)max_seq * HD, (long)HIDDEN * QSZ, (long)INTER * HIDDEN, (long)INTER * HIDDEN,
                            (long)HIDDEN * INTER, HIDDEN, HIDDEN, HD, HD, (long)max_seq * HD, (long)max_seq * HD};
    const int ctxs[] = {1, 2, 3, 4, 5, 31, 127, 128, 129, 500, 1021, 1920, 1921, 2000, 2047, 2048};
    for (int ctx : ctxs) {
      const int pos = ctx - 1;
      for (int x = 0; x < NXCD; ++x)
        for (int i = 0; i < NLOC; ++i) {
          int total = 0, mlp_total = 0;
          for (int si = 0; si < NSTREAM; ++si)
            for (int lane = 0; lane < WAVE; ++lane) {
              const StreamGeom g = stream_geom(si, x, i, ctx, pos, lane);
              if (lane == 0) {
                total += g.n;
                if (si >= MLP_FIRST_STREAM) mlp_total += g.n;
              }
              for (int m = 0; m < g.n; ++m) {
                const long e = g.elem0 + m * g.stride + g.loff;
                long want = -1;
                int want_mat = -1;
                switch (si) {
                  case 0:
                  case 6:
                    want_mat = si == 0 ? 9 : 10;
                    want = 512 * m + 8 * lane;
                    break;
                  case 1: {
                    const int gr = QKV_PER_WG * i + (m >> 1);
                    want_mat = grp_matrix(gr);
                    want = (long)grp_row_in(x, gr) * HIDDEN + 512 * (m & 1) + 8 * lane;
                    break;
                  }
                  case 2:
                    want_mat = 11 + (lane >> 4);
                    want = ((lane >> 4) >= 2 ? (long)pos * HD : 0) + 8 * (lane & 15);
                    break;
                  case 3:
                  case 4: {
                    want_mat = si == 3 ? 3 : 4;
                    const int p = att_t0(ctx, i) + 4 * m + (lane >> 4);
                    const bool cached = 4 * m + (lane >> 4) < g.vlim;
                    const int lim = att_t1(ctx, i) < pos ? att_t1(ctx, i) : pos;
                    CHECK(cached == (p < lim), "K/V cached lanes ctx %d", ctx);
                    if (!cached) continue;
                    CHECK(p >= 0 && p < pos && p < max_seq, "K/V position");
                    want = (long)p * HD + 8 * (lane & 15);
                    break;
                  }
                  case 5:
                    want_mat = 5;
                    want = (long)(HROWS * i + 2 * m + (lane >> 5)) * QSZ + OCOLS * x + 8 * (lane & 31);
                    break;
                  case 7:
                  case 8:
                    want_mat = si == 7 ? 6 : 7;
                    want = (long)(ICOLS * x + GU_PER_WG * i + (m >> 1)) * HIDDEN + 512 * (m & 1) + 8 * lane;
                    break;
                  default:
                    want_mat = 8;
                    want = (long)(HROWS * i + m) * INTER + ICOLS * x + 8 * (lane < 48 ? lane : lane - 48);
                    break;
                }
                CHECK(want_mat == g.mat && e == want, "stream %d element x%d i%d m%d lane%d", si, x, i, m, lane);
                CHECK(g.mat >= 0 && g.mat < 15 && e >= 0 && e + 8 <= msize[g.mat], "stream %d in its source", si);
              }
            }
          int st_total = 0;
          for (int st = 0; st < NSTAGE; ++st) st_total += stage_lines(st, ctx, i);
          CHECK(total == st_total, "streams cover the stage lines ctx %d", ctx);
          CHECK(mlp_total == stage_lines(S_GU, ctx, i) + stage_lines(S_DOWN, ctx, i), "MLP streams");
        }
    }
    // stage-by-stage: the stream line counts add up to each stage's lines, in order
    for (int ctx : ctxs) {
      const int pos = ctx - 1;
      const int sl[NSTREAM] = {0, 0, 1, 1, 1, 3, 5, 5, 5, 6};  // stage of each stream
      int per_stage[NSTAGE] = {0};
      for (int si = 0; si < NSTREAM; ++si) per_stage[sl[si]] += stream_geom(si, 0, 5, ctx, pos, 0).n;
      for (int st = 0; st < NSTAGE; ++st) CHECK(per_stage[st] == stage_lines(st, ctx, 5), "stage %d lines", st);
    }
  }

  // ---- ring schedule: every stage fits the ring ----
  for (int ctx = 1; ctx <= MAX_SEQ_LIMIT; ++ctx)
    for (int s = 0; s < NSPLIT; ++s)
      for (int st = 0; st < NSTAGE; ++st) CHECK(stage_lines(st, ctx, s) <= RING_LINES, "stage lines");

  // ---- lm_head rows: [0, VOCAB) exactly once over (w, v, k, j) ----
  {
    std::vector<int> seen(VOCAB, 0);
    for (int w = 0; w < NWG; ++w)
      for (int ch = 0; ch < lm_chunks(w); ++ch)
        for (int j = 0; j < LM_CHUNK; ++j) {
          const int r = lm_row(w, ch, j);
          CHECK(r >= 0 && r < VOCAB, "lm row range");
          CHECK(ch == 0 || r > lm_row(w, ch - 1, LM_CHUNK - 1), "lm rows ascend");
          seen[r]++;
        }
    for (int r = 0; r < VOCAB; ++r) CHECK(seen[r] == 1, "lm row %d seen %d", r, seen[r]);
    // with the pool: the workgroups' first LM_STATIC chunks and the pool's LM_POOL chunks
    std::vector<int> seen2(LM_NCHUNK, 0);
    for (int w = 0; w < NWG; ++w)
      for (int ch = 0; ch < LM_STATIC; ++ch) {
        CHECK(ch < lm_chunks(w), "static chunk is dealt");
        seen2[w + NWG * ch]++;
      }
    CHECK(LM_GROUP * LM_NGRP == NWG && LM_NGRP <= WAVE, "pool groups");
    for (int G = 0; G < LM_NGRP; ++G)
      for (int k = 0; k < lm_group_chunks(G); ++k) {
        const int g = LM_STATIC * NWG + LM_NGRP * k + G;
        CHECK(g >= LM_STATIC * NWG && g < LM_NCHUNK, "pool chunk range");
        seen2[g]++;
      }
    for (int g = 0; g < LM_NCHUNK; ++g) CHECK(seen2[g] == 1, "lm chunk %d seen %d", g, seen2[g]);
    // ARG: workgroup w stores slots 2w, 2w + 1; quarter c polls pairs 64 c + lane
    for (int c = 0; c < NCW; ++c)
      for (int lane = 0; lane < WAVE; ++lane) {
        const int slot = 128 * c + 2 * lane;
        CHECK(slot == 2 * (64 * c + lane) && slot + 1 < ARG_SLOTS, "arg poll");
      }
  }

  // ---- tags: distinct per (layer, stage), never the ARG tag, epoch >= 1 never 0 ----
  {
    std::vector<int> seen(256, 0);
    for (int l = 0; l < MAX_LAYERS; ++l)
      for (int st = 0; st < NSTAGE; ++st) seen[tag_of(0, l, st)]++;
    seen[tag_arg(0)]++;
    for (int e = 0; e < 256; ++e) CHECK(seen[e] <= 1, "tag collision %d", e);
    CHECK(tag_of(1, 0, 0) != 0 && tag_arg(1) != 0, "tags of epoch >= 1 are never 0");
  }

  // ---- prefill LDS tiles: every operand read puts each 16-lane group on distinct bank units ----
  // (16-byte reads: the 16 units of 16 bytes of a 256-byte window; transposing 8-byte reads: the
  // 32 units of 8 bytes). The permutations are also bijections, so the LDS-DMA lane that writes
  // position p of a row (source chunk perm(p, r)) fills every chunk of the row exactly once.
  {
    auto distinct = [](const int* u, int n) {
      for (int a = 0; a < n; ++a)
        for (int b = a + 1; b < n; ++b)
          if (u[a] == u[b]) return false;
      return true;
    };
    // GEMM ring: tile rows of 128 bytes; a read takes rows base + (lane % 16) (base a multiple
    // of 16) and logical chunk c = 4 ks + lane / 16 at position c ^ pf_swz8(row)
    for (int base = 0; base < 128; base += 16)
      for (int ks = 0; ks < 2; ++ks)
        for (int g = 0; g < 4; ++g) {
          int u[16], un[16];
          for (int fr = 0; fr < 16; ++fr) {
            const int row = base + fr, c = 4 * ks + g;
            u[fr] = ((row * 128 + 16 * (c ^ pf_swz8(row))) / 16) % 16;
            un[fr] = ((row * 128 + 16 * c) / 16) % 16;
          }
          CHECK(distinct(u, 16), "gemm operand read: bank units repeat (base %d ks %d group %d)", base, ks, g);
          CHECK(!distinct(un, 16), "the natural chunk order would not conflict (the check would be vacuous)");
        }
    for (int r = 0; r < 16; ++r) {
      int p8[8], pk[16], pv[16];
      for (int q = 0; q < 8; ++q) p8[q] = q ^ pf_swz8(r);
      for (int q = 0; q < 16; ++q) {
        pk[q] = pf_kpos(q, r);
        pv[q] = pf_vpos(q, r);
        CHECK(pf_kpos(pk[q], r) == q && pf_vpos(pv[q], r) == q, "K/V chunk permutations are involutions");
      }
      CHECK(distinct(p8, 8) && distinct(pk, 16) && distinct(pv, 16), "chunk permutations are bijections (row %d)", r);
    }
    // attention K: key rows of 256 bytes; a read takes key rows 16 j + (lane % 16), logical chunk
    // 4 kk + lane / 16
    for (int j = 0; j < 4; ++j)
      for (int kk = 0; kk < 4; ++kk)
        for (int g = 0; g < 4; ++g) {
          int u[16];
          for (int fr = 0; fr < 16; ++fr) u[fr] = pf_kpos(4 * kk + g, 16 * j + fr) % 16;
          CHECK(distinct(u, 16), "attention K read: bank units repeat (j %d kk %d group %d)", j, kk, g);
        }
    // attention V^T by transposing 8-byte reads: lane i of 16-lane group fg addresses key row
    // kr + i / 4 (kr = 32 kk + 4 fg, + 16), bytes 16 ch + 8 (i % 2) with ch = pf_vpos(2 tt + (i % 4) / 2, row)
    for (int kk = 0; kk < 2; ++kk)
      for (int half = 0; half < 2; ++half)
        for (int fg = 0; fg < 4; ++fg)
          for (int tt = 0; tt < 8; ++tt) {
            int u[16], un[16];
            for (int i = 0; i < 16; ++i) {
              const int te = i >> 2, tq = i & 3, r = 32 * kk + 16 * half + 4 * fg + te;
              const int ch = pf_vpos(2 * tt + (tq >> 1), r);
              u[i] = ((r * 256 + 16 * ch + 8 * (tq & 1)) / 8) % 32;
              un[i] = ((r * 256 + 16 * (2 * tt + (tq >> 1)) + 8 * (tq & 1)) / 8) % 32;
            }
            CHECK(distinct(u, 16), "attention V^T read: bank units repeat (kk %d fg %d tt %d)", kk, fg, tt);
            CHECK(!distinct(un, 16), "V^T natural order would not conflict (the check would be vacuous)");
          }
  }

  // ---- 64-bit pointers through the 32-bit lane broadcast (readfirstlane: int -> int) ----
  // Device addresses whose low word has bit 31 set are where a signed broadcast result,
  // widened straight to 64 bits, would corrupt the high word; every such case is checked
  // here instead of relying on the allocator to hand one out on the GPU.
  {
    auto bcast = [](int x) -> int { return x; };  // host stand-in: same signature as readfirstlane
    const unsigned long long his[] = {0x0ull, 0x1ull, 0x7f12ull, 0x7fffull, 0xffffffffull};
    const unsigned long long los[] = {0x0ull, 0x1000ull, 0x7fffffffull, 0x80000000ull, 0x80001234ull,
                                      0xc0000000ull, 0xfffff000ull, 0xffffffffull};
    int widened_wrong = 0;
    for (unsigned long long hi : his)
      for (unsigned long long lo : los) {
        const unsigned long long v = (hi << 32) | lo;
        CHECK(uniform_u64(v, bcast) == v, "uniform_u64(%llx)", v);
        const U32Pair h = uniform_halves(v, bcast);
        CHECK(h.lo == (unsigned)lo && h.hi == (unsigned)hi, "uniform_halves(%llx)", v);
        // the mistake the helper avoids: the signed low half widened to 64 bits before the OR
        const unsigned long long naive =
            ((unsigned long long)(unsigned)bcast((int)(unsigned)(v >> 32)) << 32) | (unsigned long long)(long long)bcast((int)(unsigned)v);
        widened_wrong += naive != v;
      }
    // (a high word of all ones hides it: 5 low words >= 2^31 times the 4 other high words)
    CHECK(widened_wrong == 5 * 4, "the naive join fails exactly for low words >= 2^31 (%d)", widened_wrong);
  }

  if (g_fail) {
    fprintf(stderr, "layout_check: %d failures\n", g_fail);
    return 1;
  }
  printf("layout_check: all checks passed\n");
  return 0;
}
