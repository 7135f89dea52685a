// CPU check of the launch planners (mlc-vla_amd/csrc/plan.h) over sweeps of shapes, built with
// the address and undefined-behaviour sanitizers by tests/test_planners.py.  Every plan must
// cover its whole K (or key) range with no empty slice, stay within its workspace, and -- for
// the split-K tile GEMM, whose splits meet through a bounded wait -- keep the whole grid
// resident (one workgroup per CU).  Prints the number of plans checked; exits 1 on a failure.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../mlc-vla_amd/csrc/plan.h"

using namespace mlcv;

static long checked = 0;
static int failures = 0;

#define CHECK(cond, ...)                             \
  do {                                               \
    if (!(cond)) {                                   \
      if (failures++ < 20) {                         \
        std::fprintf(stderr, "FAIL %s: ", #cond);    \
        std::fprintf(stderr, __VA_ARGS__);           \
        std::fprintf(stderr, "\n");                  \
      }                                              \
    }                                                \
  } while (0)

static void check_attn() {
  for (int rows : {1, 8, 16, 50, 63, 64, 65, 400, 800, 7744, 8192})
    for (int Sp : {0, 1, 31, 32, 33, 256, 800, 968, 1018, 4096})
      for (int Ts : {0, 1, 8, 50, 64})
        for (int target : {1, 7, 64, 100, 128, 224, 256, 1000}) {
          if (Sp == 0 && Ts == 0) continue;
          int ns = -1, kps = -1;
          attn_plan(rows, Sp, Ts, target, &ns, &kps);
          ++checked;
          const int nsp = ns - (Ts > 0 ? 1 : 0);
          CHECK(ns >= 1 && ns <= 32, "rows %d Sp %d Ts %d target %d: nsplit %d", rows, Sp, Ts, target, ns);
          CHECK(kps >= ATTN_KCH && kps % ATTN_KCH == 0, "kps %d", kps);
          if (Sp > 0) {
            CHECK(nsp >= 1 && (long)nsp * kps >= Sp, "Sp %d nsp %d kps %d: keys not covered", Sp, nsp, kps);
            CHECK((long)(nsp - 1) * kps < Sp, "Sp %d nsp %d kps %d: an empty prefix split", Sp, nsp, kps);
          } else {
            CHECK(nsp == 0, "no prefix keys but %d prefix splits", nsp);
          }
          // every partial the kernels write lies inside the workspace
          for (int KV : {1, 2, 8}) {
            const int hd = 256;
            const size_t ws = attn_ws_floats(KV, rows, hd, ns);
            if (ns == 1) {
              CHECK(ws == 0, "one split needs no workspace");
              continue;
            }
            const size_t rpad = (size_t)((rows + ATTN_ROWS - 1) / ATTN_ROWS) * ATTN_ROWS;
            const size_t last_row = ((size_t)(KV - 1) * ns + (ns - 1)) * rpad + (rows - 1);
            const size_t o_end_halfs = (last_row + 1) * hd;           // fp16 O
            const size_t ml_off = (size_t)KV * ns * rpad * hd;        // floats, after O
            const size_t ml_end = ml_off + (last_row + 1) * 2;
            CHECK(o_end_halfs <= 2 * ml_off, "O partials overlap (m, l)");
            CHECK(ml_end <= ws, "rows %d ns %d KV %d: (m, l) end %zu > workspace %zu", rows, ns, KV, ml_end, ws);
          }
        }
}

static void check_skinny() {
  for (int ntiles : {1, 2, 3, 8, 16, 40, 64, 160, 256, 512, 1024})
    for (int K : {32, 96, 128, 129, 512, 1024, 2048, 4096, 16384})
      for (int mblocks : {1, 2, 4, 16})
        for (int splits : {-1, 0, 1, 2, 3, 4, 8, 9, 100}) {
          const SkPlan p = sk_plan(ntiles, K, mblocks, splits);
          ++checked;
          CHECK(p.splitk >= 1 && p.splitk <= SK_MAX_SPLIT, "splitk %d", p.splitk);
          CHECK(p.kper >= SK_KC && p.kper % SK_KC == 0, "kper %d", p.kper);
          CHECK((long)p.kper * p.splitk >= K, "K %d: %d x %d does not cover it", K, p.splitk, p.kper);
          CHECK((long)(p.splitk - 1) * p.kper < K, "K %d: %d x %d leaves an empty slice", K, p.splitk, p.kper);
          if (splits > 0) CHECK(p.splitk <= splits, "asked %d splits, got %d", splits, p.splitk);
          const size_t ws = sk_ws_floats(ntiles, mblocks, p, 4);
          CHECK((ws == 0) == (p.splitk == 1), "workspace %zu for %d splits", ws, p.splitk);
          if (p.splitk > 1)
            CHECK(ws == (size_t)ntiles * mblocks * p.splitk * 4 * 64, "workspace %zu", ws);
        }
}

static void check_tile() {
  for (int cus : {8, 80, 256, 304})
    for (int M : {1, 32, 255, 256, 257, 968, 4096})
      for (int N : {4, 256, 1024, 2048, 2560, 8192, 16384})
        for (int K : {8, 64, 200, 512, 1024, 2048, 4096, 16384})
          for (int geglu : {0, 1})
            for (int ws_given : {0, 1}) {
              TilePlanIn in{};
              in.M = M;
              in.N = N;
              in.K = K;
              in.F = N;
              in.n1 = in.n2 = geglu ? 2 * N : N;
              in.lda = K;
              in.ldb = K;
              in.ldc = N;
              in.geglu = geglu != 0;
              in.small_tiles = false;
              in.split_ws = ws_given != 0;
              in.ws_floats = (size_t)cus * TG_BM * 256;  // one 256 x 256 partial per CU
              in.sync_tiles = cus;
              in.cus = cus;
              TilePlan p{};
              if (!tile_plan(in, p)) {
                ++checked;
                CHECK(geglu ? N % 128 != 0 : (N % 4 != 0 || K % 8 != 0), "M %d N %d K %d: no 256-row plan", M, N, K);
                continue;
              }
              ++checked;
              const int tiles = p.mtiles * p.ntiles, kts = (K + TG_BK - 1) / TG_BK;
              CHECK(p.bm == TG_BM || (p.bm == 128 && (p.bn == 128 || p.bn == 64) && p.splitk == 1 && !geglu), "m tile %d", p.bm);
              CHECK((long)p.mtiles * p.bm >= M && (long)(p.mtiles - 1) * p.bm < M, "m tiles %d for M %d", p.mtiles, M);
              const long ncover = geglu ? (long)p.ntiles * (p.bn / 2) : (long)p.ntiles * p.bn;
              CHECK(ncover >= N, "n tiles %d x %d for N %d", p.ntiles, p.bn, N);
              CHECK(p.splitk >= 1 && p.kt_per >= 1, "splitk %d kt_per %d", p.splitk, p.kt_per);
              CHECK((long)p.kt_per * p.splitk >= kts && (long)(p.splitk - 1) * p.kt_per < kts,
                    "K %d: %d slices of %d k tiles", K, p.splitk, p.kt_per);
              CHECK(p.bn == 64 || p.bn == 128 || p.bn == 256, "n tile %d", p.bn);
              if (p.bn == 64) CHECK(p.splitk == 1 && 2 * tiles >= cus, "256 x 64 tiles: %d tiles, %d splits", tiles, p.splitk);
              // the 256 x 256 kernel (not GeGLU) stores split partials and meets even over one slice
              if (p.bn == 256 && !geglu) {
                CHECK(ws_given && tiles <= in.sync_tiles, "256 x 256: %d tiles, workspace %d", tiles, ws_given);
                CHECK((size_t)tiles * p.splitk * tile_part_floats(p.bn) <= in.ws_floats, "256 x 256 partials overflow");
              }
              if (p.splitk > 1) {
                CHECK(!geglu && ws_given, "split-K without a workspace or with the GeGLU epilogue");
                CHECK(tiles <= in.sync_tiles, "%d tiles, %d meeting counters", tiles, in.sync_tiles);
                CHECK((long)tile_slots(tiles) * p.splitk <= cus,
                      "M %d N %d K %d cus %d: %d slots x %d splits not resident at once", M, N, K, cus,
                      tile_slots(tiles), p.splitk);
                CHECK((size_t)tiles * p.splitk * tile_part_floats(p.bn) <= in.ws_floats, "partials overflow");
                CHECK(p.kt_per >= 4, "slices of %d k tiles", p.kt_per);
              }
            }
}

int main() {
  check_attn();
  check_skinny();
  check_tile();
  std::printf("plans checked: %ld, failures: %d\n", checked, failures);
  return failures ? 1 : 0;
}
