// Host-side launch planners: how the attention, the skinny GEMM and the prefill tile GEMM
// split their work, and the workspace each plan needs.  Plain C++ (no HIP types), so that
// the plans and their invariants are checked by a CPU build under the sanitizers
// (tests/plan_check.cpp).
#pragma once

#include <algorithm>
#include <cstddef>

namespace mlcv {

// ---- joint attention (attn_impl.h) ------------------------------------------------------
constexpr int ATTN_ROWS = 64;  // query rows per workgroup
constexpr int ATTN_KCH = 32;   // keys per chunk

// Key splits of `rows` query rows against Sp prefix keys (+ one split for Ts > 0 suffix keys):
// about target_blocks workgroups, prefix splits of whole chunks, at most 31 of them, none
// empty.  *kps: prefix keys per split.
inline void attn_plan(int rows, int Sp, int Ts, int target_blocks, int* nsplit, int* kps) {
  const int rb = (rows + ATTN_ROWS - 1) / ATTN_ROWS;
  const int chunks = (Sp + ATTN_KCH - 1) / ATTN_KCH;
  int ns = (target_blocks + rb - 1) / rb - (Ts > 0 ? 1 : 0);
  ns = std::min(ns, 31);
  ns = std::min(ns, chunks);
  ns = std::max(ns, 1);
  const int cps = chunks > 0 ? (chunks + ns - 1) / ns : 1;
  *kps = cps * ATTN_KCH;
  *nsplit = (chunks > 0 ? (chunks + cps - 1) / cps : 0) + (Ts > 0 ? 1 : 0);
}

// Split partials of a plan: fp16 O [KV][nsplit][rpad][hd] in the first KV*nsplit*rpad*hd
// floats (half of them used), then fp32 (m, l) [KV][nsplit][rpad][2].  None for one split.
inline size_t attn_ws_floats(int KV, int rows, int hd, int nsplit) {
  const int rpad = ((rows + ATTN_ROWS - 1) / ATTN_ROWS) * ATTN_ROWS;
  return nsplit > 1 ? (size_t)KV * nsplit * rpad * (hd + 2) : 0;
}

// ---- skinny GEMM (gemm_skinny.hip) ------------------------------------------------------
constexpr int SK_KC = 128;        // k per chunk
constexpr int SK_MAX_SPLIT = 8;   // K slices at most

struct SkPlan {
  int splitk, kper;  // K slices, k per slice (whole chunks)
};

// splits > 0: that many K slices (at most one per chunk); otherwise enough slices for about
// one workgroup per CU of a 256-CU part, at most SK_MAX_SPLIT.  No slice is empty.
inline SkPlan sk_plan(int ntiles, int K, int mblocks, int splits) {
  const int chunks = (K + SK_KC - 1) / SK_KC;
  int want = splits;
  if (want <= 0) {
    const int blocks = std::max(ntiles * mblocks, 1);
    want = (256 + blocks - 1) / blocks;
  }
  want = std::min(want, SK_MAX_SPLIT);
  want = std::min(want, chunks);
  want = std::max(want, 1);
  const int cps = (chunks + want - 1) / want;
  SkPlan p;
  p.kper = cps * SK_KC;
  p.splitk = (chunks + cps - 1) / cps;
  return p;
}

// fp32 partials of a split plan: [ntiles][mblocks][splitk][tr x 64]
inline size_t sk_ws_floats(int ntiles, int mblocks, const SkPlan& p, int tr) {
  return p.splitk > 1 ? (size_t)ntiles * mblocks * p.splitk * tr * 64 : 0;
}

// ---- prefill tile GEMM, 256-row tiles (gemm_tile.hip) -------------------------------------
constexpr int TG_BM = 256, TG_BK = 64, TG_NXCD = 8;

struct TilePlanIn {
  int M, N, K;
  int F;           // GeGLU: outputs (the gate rows, then F up rows)
  int n1, n2;      // weight segment boundaries in N
  int lda, ldb, ldc;
  bool geglu, small_tiles;
  bool split_ws;   // a split-K workspace and meeting counters are given
  size_t ws_floats;
  int sync_tiles;  // tiles with meeting counters
  int cus;         // compute units of the device
  bool m128 = true;  // 128 x 128 tiles allowed (tuning switch)
  bool n64m128 = true;  // 128 x 64 tiles where 128 x 128 ones fill at most half the CUs (tuning switch)
};

struct TilePlan {
  int bm, bn, splitk, kt_per;  // m tile, n tile, K slices, k tiles (of TG_BK) per slice
  int mtiles, ntiles;          // ntiles: n tiles of bn (GeGLU: of bn / 2 outputs)
};

// fp32 partials of one split of a tile: [4 waves][bn / 64 blocks][4][4][64] f4
inline size_t tile_part_floats(int bn) { return (size_t)4 * (bn / 64) * 4 * 4 * 64 * 4; }

// Launch slots of a tile grid: tiles dealt round-robin to the XCDs, rounded to whole rounds.
inline int tile_slots(int tiles) { return ((tiles + TG_NXCD - 1) / TG_NXCD) * TG_NXCD; }

// false: the shape needs the 128 x 128 kernel.  A split-K plan keeps every workgroup of the
// grid resident at once (slots x splits <= CUs, one workgroup per CU), because the splits of
// a tile meet through a bounded wait, and its partials within the workspace.
inline bool tile_plan(const TilePlanIn& a, TilePlan& p) {
  if (a.small_tiles || a.K % 8 != 0 || a.M < 1 || a.lda % 8 != 0 || a.ldb % 8 != 0 || a.ldc % 4 != 0) return false;
  p.bm = TG_BM;
  if (a.geglu) {
    if (a.F % 128 != 0) return false;
    p.bn = 256;
    p.ntiles = a.F / 128;
  } else {
    if (a.N % 4 != 0) return false;
    if ((a.n1 % 8 != 0 && a.n1 != a.N) || (a.n2 % 8 != 0 && a.n2 != a.N)) return false;
    // long K (down_proj): 256 x 256 tiles over up to 8 K slices load a third less through
    // L2 than 256 x 128 tiles over 4.  Shorter K, over the whole K, when the tiles give at
    // least half a workgroup per CU: 128 x 128 (the prefill's q/k/v at P = 968), or 128 x 64
    // where 128 x 128 would leave half the CUs idle (o_proj: 256 tiles instead of 128); else
    // 256 x 64; else 256 x 128.
    const int mt = (a.M + TG_BM - 1) / TG_BM, mt2 = (a.M + 127) / 128;
    // (the 256 x 256 kernel stores every tile's product as a split partial and meets on the
    // tile's counter, also over one slice: only where the workspace and counters hold its tiles)
    const long t256 = (long)mt * (a.N / 256);
    if (a.K >= 8192 && a.N % 256 == 0 && (a.n1 % 16 == 0 || a.n1 == a.N) && (a.n2 % 16 == 0 || a.n2 == a.N) &&
        a.split_ws && t256 <= a.sync_tiles && (size_t)t256 * tile_part_floats(256) <= a.ws_floats) {
      p.bn = 256;
    } else if (a.K < 8192 && a.m128 && 2 * mt2 * ((a.N + 127) / 128) >= a.cus && a.cus > 0) {
      p.bm = 128;
      p.bn = a.n64m128 && mt2 * ((a.N + 127) / 128) <= a.cus / 2 ? 64 : 128;
    } else if (a.K < 8192 && 2 * mt * ((a.N + 63) / 64) >= a.cus && a.cus > 0) {
      p.bn = 64;
    } else {
      p.bn = 128;
    }
    p.ntiles = (a.N + p.bn - 1) / p.bn;
  }
  p.mtiles = (a.M + p.bm - 1) / p.bm;
  const int tiles = p.mtiles * p.ntiles, kts = (a.K + TG_BK - 1) / TG_BK;
  const int slots = tile_slots(tiles);
  int S = 1;
  if (!a.geglu && p.bn != 64 && p.bm == TG_BM && a.split_ws && tiles <= a.sync_tiles && a.cus > 0) {
    // at least 4 k tiles per slice
    S = std::min({8, a.cus / slots, kts / 4});
    const size_t part = tile_part_floats(p.bn);
    while (S > 1 && (size_t)tiles * S * part > a.ws_floats) --S;
    S = std::max(S, 1);
  }
  p.kt_per = (kts + S - 1) / S;
  p.splitk = (kts + p.kt_per - 1) / p.kt_per;
  return true;
}

}  // namespace mlcv
