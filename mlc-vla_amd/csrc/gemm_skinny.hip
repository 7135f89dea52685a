// Skinny GEMM for the suffix path (M = action horizon <= 64 per block): HBM-bound
// weight streaming into MFMA 16x16x32 f16, with the adaRMS prologue and the
// residual / GeGLU / bias / SiLU / Euler epilogues fused, and q4f16_1 weights
// dequantized in registers.
//
// Mapping: D[n][m] = sum_k W[n][k] * X[m][k]: the A operand is a 16-row slab of W
// (lane l holds row l%16; per 128-k chunk one load instruction covers 64 contiguous
// bytes of each of the wave's 16 rows), the B operand is X^T read from LDS with the
// same k order.  A workgroup (4 waves) owns 64 output columns (for GeGLU: 32
// columns, i.e. their 32 gate + 32 up weight rows) and one K slice of NC*128 per
// round; K slices of one tile are reduced by the last-arriving workgroup in split
// order.
//
// Every result stays in the MFMA D layout until it is stored: lane (g, r) holds
// columns n0..n0+3 (n0 = 4g within its wave's 16) of rows r, 16+r, 32+r, 48+r.
//
// The kernel is straight-line by construction: a workgroup always computes 4 m
// tiles and NC chunks per round, loads use clamped (always valid) addresses, and K
// positions past the slice are zeroed with selects on X.  Conditional MFMAs or
// conditional loads would make the compiler shuttle the accumulators between
// register files and split the code into exec-mask blocks, which costs more than
// the work they skip: with one wave per SIMD every VALU instruction is latency.
//
// Row statistics of the adaRMS prologue are not recomputed from x: every epilogue
// that writes the residual stream x also writes, per 64-column tile, the partial
// sum of squares of each row (``rowss_out``); the consuming GEMM sums those partials
// in tile order (``rowss_in``).
//
// Split-K partials: with gridDim.x a multiple of 8 the splits of a tile run on one
// XCD (workgroups are dealt to the 8 XCDs round-robin by linear id), so partials go
// through that XCD's L2 with plain stores; otherwise they are written through to
// memory.  The last workgroup to increment the tile counter sums them.
#include "kernels.h"

namespace mlcv {

namespace {
constexpr int KC = 128;           // k per chunk (4 MFMA k-steps of 32)
constexpr int MB = 64;            // m rows per block (4 MFMA m tiles)
constexpr int MAX_SPLIT = 8;
static_assert(KC == SK_KC && MAX_SPLIT == SK_MAX_SPLIT, "the planner's chunk and split limits (plan.h)");


// pre-scaled adaRMS input: fp16(x * (1 + scale) * c) for 4 columns (c: the norm's power-of-two
// prescale, exact in fp32)
__device__ __forceinline__ void store_xu(_Float16* p, h4 x, h4 scale, float c) {
  h4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = f2h(h2f(x[e]) * (1.0f + h2f(scale[e])) * c);
  *reinterpret_cast<h4*>(p) = o;
}


// raw weight bits of one chunk for one lane: fp16 (4 x 16 B) or q4 (16 B + one scale)
template <bool Q4>
struct WRaw {
  h8 v[4];
};
template <>
struct WRaw<true> {
  u4 words;
  _Float16 s;
};

// Weights of one 128-k chunk at kc for this lane's row (lane group g), clamped into
// the row so every load is valid (the matching X entries are zero past the slice):
//   fp16: k-step j holds k = kc + 32j + 8g .. +7 (one load instruction covers 64
//         contiguous bytes of each of the wave's 16 rows);
//   q4:   the 32 nibbles at kc + 32g .. +31 (16 B) and their group scale; k-step j
//         takes dequantized elements 8j..8j+7 in the order [n0,n4,n1,n5,n2,n6,n3,n7].
template <bool Q4>
__device__ __forceinline__ void load_wraw(WRaw<Q4>& f, const SkSeg& seg, int row, int kc, int g, int K) {
  if constexpr (!Q4) {
    const _Float16* p = seg.w + (size_t)row * K;
#pragma unroll
    for (int j = 0; j < 4; ++j) f.v[j] = load_global(reinterpret_cast<const h8*>(p + min(kc + 32 * j + 8 * g, K - 8)));
  } else {
    const int k = min(kc + 32 * g, K - 32);
    f.words = load_global(reinterpret_cast<const u4*>(seg.qw + (size_t)row * (K / 8) + k / 8));
    f.s = load_global(seg.qs + (size_t)row * (K / 32) + k / 32);
  }
}

template <bool Q4>
__device__ __forceinline__ h8 wfrag(const WRaw<Q4>& f, int j) {
  if constexpr (!Q4) return f.v[j];
  else return dequant_word(f.words[j], f.s);
}

// acc[i] (this wave's owned m tiles) = sum over the NS split partials, in split order
template <int NS, int NOWN>
__device__ __forceinline__ void sum_splits(const float* base, size_t split_stride, const int* own_off, f4* acc) {
  f4 part[NS][NOWN];
#pragma unroll
  for (int q = 0; q < NS; ++q)
#pragma unroll
    for (int i = 0; i < NOWN; ++i) part[q][i] = *reinterpret_cast<const f4*>(base + q * split_stride + own_off[i]);
#pragma unroll
  for (int i = 0; i < NOWN; ++i) {
    f4 sum = part[0][i];
#pragma unroll
    for (int q = 1; q < NS; ++q) sum += part[q][i];
    acc[i] = sum;
  }
}

// One output tile of TR weight rows (SLABS = TR/16 MFMA row slabs) over one K slice.
// Wave w = (slab, kg): slab w % SLABS, k group w / SLABS takes chunks kg*CPW .. +CPW of
// every round.  The k groups of a slab are summed through LDS in k-group order; after
// that wave (slab, kg) owns m tiles kg, kg + KG, ... of its slab (split-K, epilogue).
// NORM: 0 none; 1 adaRMS applied to X per element (row scales from the row statistics);
// 2 pre-scaled X (the producer wrote fp16(x * (1 + scale)) and the shift as row M), the
// row scale and shift product applied in the epilogue.
// XM: 0 X row-major, staged through LDS; 1 fragment-major X and weights, loaded straight
// into registers (16-row tiles); 2 row-major X with M <= 16 (one m tile, lanes of rows
// past M contribute zeros) and fragment-major weights, loaded straight into registers.
// MG (fragment-major 16-row tiles): the 4 m tiles of a 64-row block are shared out over
// MG workgroups per weight slab (grid z = m block * MG + m group), each multiplying 4 / MG
// m tiles: MG times the weight reads (one XCD's L2 serves them, the groups of a slab share
// its XCD when the tile count is a multiple of 8), a 1 / MG share of X per workgroup and
// MG times the workgroups, with no exchange between them.  With the pre-scaled adaRMS
// input every group also multiplies the m tile that holds the shift row M.
template <bool Q4, int NORM, int EPI, int NC, bool TABLE, int TR, int XM, int MG = 1>
__global__ __launch_bounds__(256) void skinny_kernel(SkOp op) {
  static_assert(MG == 1 || ((MG == 2 || MG == 4) && XM == 1 && TR == 16 && NORM != 1),
                "m groups: fragment-major 16-row tiles");
  constexpr int SLABS = TR / 16;
  constexpr int KG = 4 / SLABS;      // waves per slab
  constexpr int CPW = NC / KG;       // chunks per wave per round
  constexpr int NOWN = 4 / KG;       // m tiles owned per wave after the k-group sum
  static_assert(SLABS * KG == 4 && CPW * KG == NC && CPW >= 1, "tile / chunk configuration");
  constexpr int XK = NC * KC;        // k per round
  constexpr int XLD = XK + 8;        // LDS row stride of the X slice (halfs)
  constexpr int TPR = XK / 8;        // threads per X row
  constexpr int RPP = 256 / TPR;     // X rows per load pass
  constexpr int NXL = MB / RPP;      // X loads per thread
  constexpr int TILE_F = TR * 64;    // floats of one split-K partial tile
  // 16-row tiles without the per-element prologue: every wave owns its own k range, so
  // its MFMA B fragments are loaded straight from X into registers (no LDS staging, no
  // barrier between loads and MFMAs: each MFMA waits only for its own operands)
  constexpr bool DIRECT = XM != 0;
  constexpr int XMT = XM == 2 ? 1 : 4 / MG;  // this workgroup's m tiles (direct path)
  constexpr int EXT = MG > 1 && NORM == 2 ? 1 : 0;  // + the shift row's m tile (local XMT)
  constexpr int PMT = XMT + EXT;              // m tiles loaded and multiplied by the direct path
  constexpr int RMT = XM == 2 ? 1 : MG > 1 ? PMT : 4;  // m tiles held in the k-group sums
  constexpr int RST = XM == 2 ? 1 : 4;                 // their m-tile stride in LDS
  constexpr int MROWS = MG > 1 ? 16 * XMT : MB;  // rows of X this workgroup covers
  // fragment-major tiles of several slabs: the 4 waves split K as in a 16-row tile and
  // every wave multiplies its X fragments by all the slabs' weights (X is loaded once per
  // workgroup); the 4 k-group partials of each slab are summed before the epilogue, which
  // keeps the (slab, kg) wave roles
  // (small-M row-major X, XM 2, likewise: one m tile, so its k-group sums take a quarter of the LDS)
  constexpr bool MSD = (XM == 1 || XM == 2) && SLABS > 1;
  constexpr int SW = MSD ? SLABS : 1;   // slabs per wave in the product
  constexpr int LKG = MSD ? 4 : KG;     // k groups of the product
  constexpr int LCPW = NC / LKG;        // chunks per wave per round in the product
  static_assert(!MSD || (LCPW >= 1 && LCPW * LKG == NC), "multi-slab tiles need NC >= 4");
  constexpr int XS_HALFS = DIRECT ? LKG * SLABS * RST * 64 * 8 : MB * XLD;
  __shared__ __attribute__((aligned(16))) _Float16 xs[XS_HALFS];
  __shared__ float denom[4][MB];     // NORM 1: 1 / sqrt(mean(x^2) + eps) per row, per wave;
                                     // NORM 2: each wave's partial sum of squares per row
  __shared__ f4 shiftacc[SLABS * 4]; // NORM 2: the shift row's product, per slab and lane group
  __shared__ int is_last;
  static_assert(LKG == 1 || (size_t)LKG * SLABS * RST * 64 * 4 * 4 <= sizeof(xs), "k-group sums alias the X slice");
  f4* red = reinterpret_cast<f4*>(xs);  // [LKG][SLABS][4 m tiles][64 lanes] after the last round

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int slab = w % SLABS, kg = w / SLABS;
  if (blockIdx.y >= op.splitk) {  // prefetch workgroups (grid rows past the K slices)
    if (blockIdx.z == 0) prefetch_run(op.pf, blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * op.splitk);
    return;
  }
  const int tile_id = blockIdx.x, s = blockIdx.y, mb = blockIdx.z / MG;
  const int mgi = MG > 1 ? (int)blockIdx.z % MG : 0;  // m group: m tiles XMT*mgi .. +XMT-1
  const int S = op.splitk;
  const int m0 = mb * MB + 16 * XMT * mgi;
  const int mlast = op.M - 1;
  const int mrows = min(MROWS, op.M - m0);
  const int xlast = NORM == 2 ? op.M : mlast;  // pre-scaled X carries the shift as row M

  // the segment: up to 3 from the kernel arguments, picked by selects (no branch on an
  // argument value, so every argument load issues at once), or from a device table of
  // equal-sized segments (one dependent load)
  SkSeg seg;
  if constexpr (!TABLE) {
    const SkSeg s0 = op.inl[0], s1 = op.inl[1], s2 = op.inl[2];
    const bool u1 = op.nseg > 1 && tile_id >= s1.tile0;
    const bool u2 = op.nseg > 2 && tile_id >= s2.tile0;
    seg = u2 ? s2 : (u1 ? s1 : s0);
  } else {
    seg = op.segs[tile_id / op.seg_tiles];
  }
  const int lt = tile_id - seg.tile0;
  const int K = op.K;
  const int kbeg = s * op.kper;
  const int kend = min(K, kbeg + op.kper);
  // GeGLU: a slab holds 8 gate + 8 up rows of 8 output columns (TR/2 outputs per tile)
  const int row = (EPI == EPI_GEGLU) ? (r16 < 8 ? 0 : op.geglu_F) + (TR / 2) * lt + 8 * slab + (r16 & 7)
                                     : min(TR * lt + 16 * slab + r16, seg.n - 1);
  // output columns n0..n0+3 of this lane (GeGLU: lanes g < 2 own the outputs)
  const int n0 = (EPI == EPI_GEGLU) ? (TR / 2) * lt + 8 * slab + 4 * (g & 1) : TR * lt + 16 * slab + 4 * g;
  const int ncl = max(0, min(n0, seg.n - 4));
  const bool nok = n0 < seg.n;
  const size_t ldo = (size_t)seg.ldo;
  const bool has_bias = seg.bias != nullptr;

  // ---- epilogue operands first (owned m tiles only): they do not depend on the product ----
  h4 xo[NOWN], gq = (h4){0, 0, 0, 0}, bq = (h4){0, 0, 0, 0};
  f4 x32o[NOWN];
  const _Float16* zero_h = reinterpret_cast<const _Float16*>(op.zero);
  if constexpr (EPI == EPI_GATED_RES) {
    const _Float16* xb = reinterpret_cast<const _Float16*>(seg.out);
#pragma unroll
    for (int i = 0; i < NOWN; ++i)
      xo[i] = *reinterpret_cast<const h4*>(xb + (size_t)min(m0 + 16 * (kg + i * KG) + r16, mlast) * ldo + ncl);
    gq = *reinterpret_cast<const h4*>(op.gate + ncl);
  }
  if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_SILU || EPI == EPI_VOUT || EPI == EPI_EULER) {
    bq = load_global(reinterpret_cast<const h4*>(has_bias ? seg.bias + ncl : zero_h));
  }
  if constexpr (EPI == EPI_EULER) {
#pragma unroll
    for (int i = 0; i < NOWN; ++i)
      x32o[i] = *reinterpret_cast<const f4*>(op.x32 + (size_t)min(m0 + 16 * (kg + i * KG) + r16, mlast) * ldo + ncl);
  }
  // RoPE segments: this lane's two dims d, d + 1 of the first half (rows paired (d, d + hd/2)
  // in the slab; after the lane ^ 32 exchange, lanes g < 2 take i = 0, 1 and g >= 2 i = 2, 3)
  f4 rcs = (f4){0.f, 0.f, 0.f, 0.f};  // cos d, cos d+1, sin d, sin d+1 of this lane's token
  int rope_d = 0;
  if constexpr (EPI == EPI_STORE && XM == 1) {
    if (seg.rope) {
      const int spb = op.rope_hd / 16;
      rope_d = 8 * (lt % spb) + 4 * (g & 1) + (g < 2 ? 0 : 2);
      const size_t tr0 = (size_t)min(m0 + 16 * kg + r16, mlast) * (op.rope_hd / 2) + rope_d;
      const f2 cc = load_global(reinterpret_cast<const f2*>(op.rope_cos + tr0));
      const f2 ss = load_global(reinterpret_cast<const f2*>(op.rope_sin + tr0));
      rcs = (f4){cc[0], cc[1], ss[0], ss[1]};
    }
  }
  // next adaRMS operands for the pre-scaled copy of x (STORE / GATED_RES producers)
  h4 xus = (h4){0, 0, 0, 0}, xush = xus;
  if constexpr (EPI == EPI_GATED_RES || EPI == EPI_STORE) {
    const bool has_xu = op.xu_out != nullptr;
    xus = load_global(reinterpret_cast<const h4*>(has_xu ? op.xu_scale + ncl : zero_h));
    xush = load_global(reinterpret_cast<const h4*>(has_xu ? op.xu_shift + ncl : zero_h));
  }
  const float xuc = op.xu_nsc ? *op.xu_nsc : 1.0f;

  // adaRMS row statistics: the producer's partial sums of squares per 16-column group,
  // stored [row][group]; one row per lane, every wave keeps its own copy of the row scales
  f4 rss[16];
  if constexpr (NORM == 1) {
    const float* rr = op.rowss_in + (size_t)min(m0 + lane, mlast) * op.rowss_ld;
#pragma unroll
    for (int q = 0; q < 16; ++q) rss[q] = *reinterpret_cast<const f4*>(rr + min(4 * q, op.rowss_tiles - 4));
  }
  // NORM 2: wave w sums groups 4(w + 4j) .. +3 of row `lane` once the product is done (the
  // loads stay in flight meanwhile); the epilogue adds the 4 waves
  f4 part[4];
  if constexpr (NORM == 2) {
    const float* rr = op.rowss_in + (size_t)min(m0 + lane, mlast) * op.rowss_ld;
#pragma unroll
    for (int j = 0; j < 4; ++j) part[j] = load_global(reinterpret_cast<const f4*>(rr + min(4 * (w + 4 * j), op.rowss_tiles - 4)));
  }

  f4 acc[SW][4];
#pragma unroll
  for (int sl = 0; sl < SW; ++sl)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[sl][i] = (f4){0.f, 0.f, 0.f, 0.f};
  const int lkg = MSD ? w : kg;  // this wave's k group in the product
  // chunk of a round taken by k group q as its c-th: rounds of up to 8 chunks give each k group
  // a run of LCPW; a 16-chunk round is two 8-chunk rounds in one, so that every wave sums the
  // same k ranges in the same order as with NC = 8 (bit-identical results)
  auto chunk_of = [&](int q, int c) __attribute__((always_inline)) -> int {
    if constexpr (NC <= 8) return q * LCPW + c;
    else {
      constexpr int CPV = 8 / LKG;  // chunks per k group in each 8-chunk half
      return (c / CPV) * 8 + q * CPV + c % CPV;
    }
  };

  // one round: rounds after the first run in a loop, the first is peeled so that the
  // prefetched loads above stay in flight (a loop header would wait for all of them)
  const int kk = (tid % TPR) * 8, mr = tid / TPR;
  auto round_direct = [&](const int kr) __attribute__((always_inline)) {
    // fragment-major operands: every load below is one contiguous 1 KB per wave (q4 X:
    // four 256 B runs).  This wave's X fragments (L2) first, then the weights (HBM / MALL):
    // a wave's loads return in issue order, so X issued behind the weights would wait for
    // the weights' memory latency before streaming in.  Chunk c, k step j, m tile mt
    // holds X[16 mt + r16][kc + ko .. +7], the B operand of mfma16x16x32 in the k order
    // of the weight fragments (q4: the dequantized nibble order, so the X fragment is
    // permuted after the load).
    const int KS = K >> 5, KCN = K >> 7;
    // X is the previous kernel's output: device-scope loads (sc1) read it at the memory
    // side instead of filling this XCD's L2 with lines the next launch cannot reuse
    __amdgpu_buffer_rsrc_t xr;
    if constexpr (XM == 1) xr = dev_rsrc(op.x, MB * K * 2);
    h8 xf[LCPW][4][PMT];
#pragma unroll
    for (int c = 0; c < LCPW; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kcs = kr + chunk_of(lkg, c) * KC;
        if constexpr (XM == 1) {
          const int ks = min((kcs >> 5) + (Q4 ? g : j), KS - 1);
          const int piece = Q4 ? 16 * j + r16 : lane;
#pragma unroll
          for (int mt = 0; mt < PMT; ++mt) {
            const int gmt = mt < XMT ? XMT * mgi + mt : op.M >> 4;  // 64-row block's m tile
            xf[c][j][mt] = load_dev<h8, X_AUX>(xr, ((ks * 4 + gmt) * 64 + piece) * 16);
          }
        } else {
          const int kx = min(kcs + (Q4 ? 32 * g + 8 * j : 32 * j + 8 * g), K - 8);
          xf[c][j][0] = load_global(reinterpret_cast<const h8*>(op.x + (size_t)min(r16, mlast) * op.ldx + kx));
        }
      }
    WRaw<Q4> wr[SW][LCPW];
#pragma unroll
    for (int sl = 0; sl < SW; ++sl)
#pragma unroll
      for (int c = 0; c < LCPW; ++c) {
        const int kcs = kr + chunk_of(lkg, c) * KC;
        // 16-row slab of the shuffled weights (multi-slab tiles without MSD: the wave's own slab)
        const size_t wsl = (size_t)SLABS * lt + (MSD ? sl : slab);
        if constexpr (!Q4) {
          const __amdgpu_buffer_rsrc_t rw = dev_rsrc(seg.w + wsl * KS * 512, (uint32_t)KS * 1024);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            wr[sl][c].v[j] = load_dev<h8, XM == 2 ? WROW_AUX : W_AUX>(rw, (min((kcs >> 5) + j, KS - 1) * 64 + lane) * 16);
        } else {
          const size_t blk = (wsl * KCN + min(kcs >> 7, KCN - 1)) * 64 + lane;
          wr[sl][c].words = load_global(reinterpret_cast<const u4*>(seg.qw + blk * 4));
          wr[sl][c].s = load_global(seg.qs + blk);
        }
      }
    // every load of the round in flight before the first MFMA (the scheduler would
    // otherwise interleave them and keep only a few outstanding)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < LCPW; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // k past the slice: the weight fragment is zeroed (X there is finite data of the
        // same rows, so the products vanish)
        const bool kok = kr + chunk_of(lkg, c) * KC + (Q4 ? 32 * g + 8 * j : 32 * j + 8 * g) < kend;
        h8 a[SW];
#pragma unroll
        for (int sl = 0; sl < SW; ++sl) {
          a[sl] = wfrag<Q4>(wr[sl][c], j);
#pragma unroll
          for (int e = 0; e < 8; ++e) a[sl][e] = kok ? a[sl][e] : (_Float16)0.0f;
        }
#pragma unroll
        for (int mt = 0; mt < PMT; ++mt) {
          h8 b = xf[c][j][mt];
          if constexpr (XM == 2) {
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = r16 < op.M ? b[e] : (_Float16)0.0f;
          }
          if constexpr (Q4) b = perm8(b);
#pragma unroll
          for (int sl = 0; sl < SW; ++sl) acc[sl][mt] = mfma16x16x32(a[sl], b, acc[sl][mt]);
        }
      }
  };
  auto round = [&](const int kr, const bool first) __attribute__((always_inline)) {
    // (1) the X slice [64 rows][XK]: thread -> 8 consecutive k of rows mr + RPP*i (rows
    //     past M repeat the last row; k past the slice is zeroed below)
    const int kg8 = kr + kk;
    const bool kok = kg8 < kend;
    const int kgc = min(kg8, K - 8);
    h8 v[NXL];
#pragma unroll
    for (int i = 0; i < NXL; ++i)
      v[i] = *reinterpret_cast<const h8*>(op.x + (size_t)min(m0 + mr + RPP * i, xlast) * op.ldx + kgc);
    h8 sc = (h8){0, 0, 0, 0, 0, 0, 0, 0}, sh = sc;
    if constexpr (NORM == 1) {
      sc = *reinterpret_cast<const h8*>(op.scale + kgc);
      sh = *reinterpret_cast<const h8*>(op.shift + kgc);
    }
    // (2) then this wave's weight chunks of the round
    WRaw<Q4> wr[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) load_wraw<Q4>(wr[c], seg, row, kr + (kg * CPW + c) * KC, g, K);
    if constexpr (NORM == 1) {
      if (first) {
        float ssum = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) ssum += 4 * q + e < op.rowss_tiles ? rss[q][e] : 0.f;
        const float* rr = op.rowss_in + (size_t)min(m0 + lane, mlast) * op.rowss_ld;
        for (int t = 64; t < op.rowss_tiles; ++t) ssum += rr[t];  // widths past 1024
        denom[w][lane] = 1.0f / sqrtf(ssum / (float)K + op.eps);  // read back by this wave only
      }
    }
    // (3) normalize / mask the X slice into LDS while the weights are in flight
    float a1[8], b1[8];
    if constexpr (NORM == 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a1[e] = kok ? 1.0f + h2f(sc[e]) : 0.f;
        b1[e] = kok ? h2f(sh[e]) : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < NXL; ++i) {
      const int m = mr + RPP * i;
      h8 o;
      if constexpr (NORM == 1) {
        const float rinv = denom[w][m];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f2h(fmaf(h2f(v[i][e]) * rinv, a1[e], b1[e]));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = kok ? v[i][e] : (_Float16)0.0f;
      }
      if constexpr (Q4) o = perm8(o);
      *reinterpret_cast<h8*>(&xs[m * XLD + kk]) = o;
    }
    __syncthreads();
    // (4) MFMA over this wave's chunks of the round
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h8 a = wfrag<Q4>(wr[c], j);
        const int ko = (kg * CPW + c) * KC + (Q4 ? 32 * g + 8 * j : 32 * j + 8 * g);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const h8 b = *reinterpret_cast<const h8*>(&xs[(mt * 16 + r16) * XLD + ko]);
          acc[0][mt] = mfma16x16x32(a, b, acc[0][mt]);
        }
      }
    }
    __syncthreads();
  };
  if constexpr (DIRECT) {
    round_direct(kbeg);
    for (int kr = kbeg + XK; kr < kend; kr += XK) round_direct(kr);
  } else {
    round(kbeg, true);
    for (int kr = kbeg + XK; kr < kend; kr += XK) round(kr, false);
  }

  if constexpr (NORM == 2) {
    const float* rr = op.rowss_in + (size_t)min(m0 + lane, mlast) * op.rowss_ld;
    float ssum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * (w + 4 * j) < op.rowss_tiles) ssum += ((part[j][0] + part[j][1]) + part[j][2]) + part[j][3];
    for (int t = 4 * (w + 16); t < op.rowss_tiles; t += 16)  // widths past 1024
      ssum += ((rr[t] + rr[t + 1]) + rr[t + 2]) + rr[t + 3];
    denom[w][lane] = ssum;
    if constexpr (KG == 1) __syncthreads();  // otherwise the k-group sum below has one
  }

  // ---- k groups of a slab summed in k-group order; wave keeps m tiles kg + i*KG ----------
  f4 own[NOWN];
  if constexpr (LKG == 1) {
#pragma unroll
    for (int i = 0; i < NOWN; ++i) own[i] = acc[0][i];
  } else {
    // product k group q of slab sl at red[q][sl]: MSD waves write every slab of their k group
#pragma unroll
    for (int sl = 0; sl < SW; ++sl)
#pragma unroll
      for (int mt = 0; mt < RMT; ++mt)
        red[((lkg * SLABS + (MSD ? sl : slab)) * RST + mt) * 64 + lane] = acc[sl][mt];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NOWN; ++i) {
      // with m groups, waves kg >= XMT own no m tile of the output (rows past MROWS: nothing
      // is stored); wave XMT holds the shift row's tile (pre-scaled input)
      const int mt = min(kg + i * KG, RMT - 1);
      f4 sum = red[((0 * SLABS + slab) * RST + mt) * 64 + lane];
#pragma unroll
      for (int q = 1; q < LKG; ++q) sum += red[((q * SLABS + slab) * RST + mt) * 64 + lane];
      own[i] = sum;
    }
  }

  // ---- split-K: partials of every split, summed by the last workgroup in split order ----
  // partial layout per tile: [slab][m tile][lane][4]
  int own_off[NOWN];
#pragma unroll
  for (int i = 0; i < NOWN; ++i) own_off[i] = ((slab * 4 + kg + i * KG) * 64 + lane) * 4;
  if (S > 1) {
    const int cidx = tile_id * gridDim.z + blockIdx.z;
    float* wsp = op.ws + ((size_t)cidx * S + s) * TILE_F;
    if ((gridDim.x & 7) == 0) {
#pragma unroll
      for (int i = 0; i < NOWN; ++i) *reinterpret_cast<f4*>(wsp + own_off[i]) = own[i];
    } else {
#pragma unroll
      for (int i = 0; i < NOWN; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) store_coherent(wsp + own_off[i] + e, own[i][e]);
    }
    wait_all_memory();
    __syncthreads();
    if (tid == 0) is_last = counter_add(&op.counters[cidx], 1u) == (unsigned)(S - 1);
    __syncthreads();
    if (!is_last) return;
    // XCD-local: the partials are in this XCD's L2 and this CU's L1 has never held
    // these lines in this kernel, so plain loads see them; otherwise drop stale copies
    if ((gridDim.x & 7) != 0) acquire_agent();
    const float* base = op.ws + (size_t)cidx * S * TILE_F;
    switch (S) {  // every partial of the tile in one batch of loads, summed in split order
      case 2: sum_splits<2, NOWN>(base, TILE_F, own_off, own); break;
      case 3: sum_splits<3, NOWN>(base, TILE_F, own_off, own); break;
      case 4: sum_splits<4, NOWN>(base, TILE_F, own_off, own); break;
      case 5: sum_splits<5, NOWN>(base, TILE_F, own_off, own); break;
      case 6: sum_splits<6, NOWN>(base, TILE_F, own_off, own); break;
      case 7: sum_splits<7, NOWN>(base, TILE_F, own_off, own); break;
      default: sum_splits<8, NOWN>(base, TILE_F, own_off, own); break;
    }
    if (tid == 0) counter_reset(&op.counters[cidx]);
  }

  // ---- pre-scaled adaRMS: y[m] = acc[m] / sqrt(mean(x^2) + eps) + acc[M] -----------------
  if constexpr (NORM == 2) {
    const int mtM = op.M >> 4, cM = op.M & 15;  // the shift row (M < 64: one m block)
#pragma unroll
    for (int i = 0; i < NOWN; ++i)
      if (kg + i * KG == (MG > 1 ? XMT : mtM) && r16 == cM) shiftacc[slab * 4 + g] = own[i];
    __syncthreads();
    const f4 sv = shiftacc[slab * 4 + g];
    const float nsc = op.nsc ? *op.nsc : 1.0f;
#pragma unroll
    for (int i = 0; i < NOWN; ++i) {
      const int m = 16 * (kg + i * KG) + r16;
      const float tot = ((denom[0][m] + denom[1][m]) + denom[2][m]) + denom[3][m];
      const float rinv = 1.0f / sqrtf(tot / (float)K + op.eps) / nsc;
#pragma unroll
      for (int e = 0; e < 4; ++e) own[i][e] = fmaf(own[i][e], rinv, sv[e]);
    }
  }

  // ---- epilogue in the D layout: row m0 + 16mt + r16 (owned mt), columns n0..n0+3 --------
  if constexpr (EPI == EPI_GEGLU) {
    // lanes g < 2 hold 4 gate columns, lane ^ 32 the matching 4 up columns: the pair
    // swaps halves so that each lane finishes 2 columns (g < 2: the first two)
    const bool lo = g < 2;
    const int col = n0 + (lo ? 0 : 2);
#pragma unroll
    for (int i = 0; i < NOWN; ++i) {
      const int mt = kg + i * KG;
      const float r0 = swap_halves(own[i][2], own[i][0], lo);  // = lane ^ 32's (lo ? [2] : [0])
      const float r1 = swap_halves(own[i][3], own[i][1], lo);
      const float ga = lo ? own[i][0] : r0, gb = lo ? own[i][1] : r1;
      const float ua = lo ? r0 : own[i][2], ub = lo ? r1 : own[i][3];
      h2 o;
      o[0] = hmul(f2h(gelu_tanh_hw(h2f(f2h(ga)))), f2h(ua));
      o[1] = hmul(f2h(gelu_tanh_hw(h2f(f2h(gb)))), f2h(ub));
      if (16 * mt + r16 < mrows && nok) {
        const int m = m0 + 16 * mt + r16;
        _Float16* ob = reinterpret_cast<_Float16*>(seg.out);
        *reinterpret_cast<h2*>(ob + (op.frag_out ? xf_index(m, col) : (size_t)m * ldo + col)) = o;
      }
    }
    return;
  }

  if constexpr (EPI == EPI_STORE && XM == 1) {
    if (seg.rope) {
      // the projection rounds to fp16 (the reference's q / k), RoPE in fp32 on those values
      static_assert(NOWN == 1, "RoPE epilogue: one owned m tile per wave");
      const bool lo = g < 2;
      const int HD = op.rope_hd, HALF = HD / 2;
      const int hh = lt / (HD / 16);  // head of this slab
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 t = f2h(own[0][e]);
        if (has_bias) t = hadd(t, bq[e]);
        y[e] = h2f(t);
      }
      const float r0 = swap_halves(y[2], y[0], lo);
      const float r1 = swap_halves(y[3], y[1], lo);
      const float x1a = lo ? y[0] : r0, x1b = lo ? y[1] : r1;
      const float x2a = lo ? r0 : y[2], x2b = lo ? r1 : y[3];
      const float o1a = x1a * rcs[0] - x2a * rcs[2], o1b = x1b * rcs[1] - x2b * rcs[3];
      const float o2a = x2a * rcs[0] + x1a * rcs[2], o2b = x2b * rcs[1] + x1b * rcs[3];
      const int m = m0 + 16 * kg + r16;
      if (16 * kg + r16 < mrows) {  // m < M, and a row of this m group
        if (seg.rope == 1) {
          const int kvh = hh / op.rope_grp, row = (hh % op.rope_grp) * op.M + m;
          const int ntiles = op.rope_rpad / 16, nks = (HD + 31) / 32;
          _Float16* qf = reinterpret_cast<_Float16*>(seg.out);
          const float o[2][2] = {{o1a, o1b}, {o2a, o2b}};
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            h2 hi, lo2;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              _Float16 hv, lv;
              split_f32(o[hf][e] * op.rope_scale, hv, lv);
              hi[e] = hv;
              lo2[e] = lv;
            }
            const int d = rope_d + hf * HALF;
            *reinterpret_cast<h2*>(qf + attn_qf_index(kvh, ntiles, nks, row, d, 0)) = hi;
            *reinterpret_cast<h2*>(qf + attn_qf_index(kvh, ntiles, nks, row, d, 1)) = lo2;
          }
        } else {
          float* kr = reinterpret_cast<float*>(seg.out) + (size_t)m * ldo + (size_t)hh * HD + rope_d;
          *reinterpret_cast<f2*>(kr) = (f2){o1a, o1b};
          *reinterpret_cast<f2*>(kr + HALF) = (f2){o2a, o2b};
        }
      }
      return;
    }
  }

  float ss[NOWN];  // row sums of squares of the stored x over this lane's 4 columns
#pragma unroll
  for (int i = 0; i < NOWN; ++i) {
    const int mt = kg + i * KG;
    const bool mok = 16 * mt + r16 < mrows;
    const size_t mo = (size_t)(m0 + 16 * mt + r16) * ldo + n0;
    float s2 = 0.f;
    if constexpr (EPI == EPI_GATED_RES) {
      h4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 r = hadd(xo[i][e], hmul(f2h(own[i][e]), gq[e]));
        o[e] = r;
        s2 += h2f(r) * h2f(r);
      }
      if (mok && nok) *reinterpret_cast<h4*>(reinterpret_cast<_Float16*>(seg.out) + mo) = o;
      if (op.xu_out && mok && nok)
        store_xu(op.xu_out + (op.frag_out ? xf_index(m0 + 16 * mt + r16, n0) : mo), o, xus, xuc);
    } else {
      h4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 t = f2h(own[i][e]);
        if (has_bias) t = hadd(t, bq[e]);
        if constexpr (EPI == EPI_STORE_SILU) t = f2h(silu_hw(h2f(t)));
        y[e] = t;
      }
      if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_SILU) {
        if (mok && nok) *reinterpret_cast<h4*>(reinterpret_cast<_Float16*>(seg.out) + mo) = y;
        if (EPI == EPI_STORE && op.xu_out && mok && nok)
          store_xu(op.xu_out + (op.frag_out ? xf_index(m0 + 16 * mt + r16, n0) : mo), y, xus, xuc);
#pragma unroll
        for (int e = 0; e < 4; ++e) s2 += h2f(y[e]) * h2f(y[e]);
      } else if constexpr (EPI == EPI_VOUT) {
        if (mok && nok)
          *reinterpret_cast<f4*>(reinterpret_cast<float*>(seg.out) + mo) = (f4){h2f(y[0]), h2f(y[1]), h2f(y[2]), h2f(y[3])};
      } else if constexpr (EPI == EPI_EULER) {
        f4 nx;
        h4 nh;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          nx[e] = euler_update(x32o[i][e], op.dt, h2f(y[e]));
          nh[e] = f2h(nx[e]);
        }
        if (mok && nok) {
          *reinterpret_cast<f4*>(op.x32 + mo) = nx;
          *reinterpret_cast<h4*>(op.x16 + mo) = nh;
        }
      }
    }
    ss[i] = nok ? s2 : 0.f;
  }
  if constexpr (EPI == EPI_GATED_RES || EPI == EPI_STORE) {
    // the shift row of the pre-scaled copy: one lane per 4 columns
    if (op.xu_out && kg == 0 && r16 == 0 && nok && mgi == 0)
      *reinterpret_cast<h4*>(op.xu_out + (op.frag_out ? xf_index(op.M, n0) : (size_t)op.M * ldo + n0)) = xush;
  }
  if constexpr (EPI == EPI_GATED_RES || EPI == EPI_STORE) {
    if (op.rowss_out) {
      // this slab's 16 columns: the 4 lanes of a row hold 4 columns each
      const int grp = (TR * lt + 16 * slab) / 16;
#pragma unroll
      for (int i = 0; i < NOWN; ++i) {
        float v = ss[i];
        v = xor_sum_16_32(v);
        const int mt = kg + i * KG;
        if (g == 0 && 16 * mt + r16 < mrows)
          op.rowss_out[(size_t)(m0 + 16 * mt + r16) * op.rowss_ld + grp] = v;
      }
    }
  }
}

__global__ void q4_quantize_kernel(const _Float16* __restrict__ w, uint32_t* __restrict__ qw,
                                   _Float16* __restrict__ qs, int N, int K) {
  const int groups = K / 32;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long)N * groups) return;
  const int n = (int)(gid / groups), gi = (int)(gid % groups);
  const _Float16* src = w + (size_t)n * K + gi * 32;
  float vals[32];
  float mx = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    vals[e] = h2f(src[e]);
    mx = fmaxf(mx, fabsf(vals[e]));
  }
  const _Float16 sc = f2h(__fdiv_rn(mx, 7.0f));
  const float scf = h2f(sc);
  uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    float q;
    if (scf == 0.f) {
      q = 7.f;
    } else {
      _Float16 t = f2h(__fdiv_rn(vals[e], scf));
      t = f2h(h2f(t) + 7.0f);
      q = rintf(h2f(t));
      q = fminf(fmaxf(q, 0.f), 14.f);
    }
    words[e >> 3] |= ((uint32_t)q & 0xFu) << (4 * (e & 7));
  }
  uint32_t* dst = qw + (size_t)n * (K / 8) + gi * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = words[i];
  qs[(size_t)n * groups + gi] = sc;
}

__global__ void q4_dequant_kernel(const uint32_t* __restrict__ qw, const _Float16* __restrict__ qs,
                                  _Float16* __restrict__ out, int N, int K) {
  const long wid = (long)blockIdx.x * blockDim.x + threadIdx.x;  // one word
  const int wpr = K / 8;
  if (wid >= (long)N * wpr) return;
  const int n = (int)(wid / wpr), j = (int)(wid % wpr);
  const h8 v = dequant_word(qw[wid], qs[(size_t)n * (K / 32) + j / 4]);
  _Float16* o = out + (size_t)n * K + 8 * j;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    o[p] = v[2 * p];
    o[p + 4] = v[2 * p + 1];
  }
}

// fragment-major weight copies (layout in kernels.h): one thread per 16-byte piece
__device__ __forceinline__ int wf_row(int s, int r, int geglu_F, int rope_hd) {
  if (geglu_F > 0) return r < 8 ? 8 * s + r : geglu_F + 8 * s + r - 8;
  if (rope_hd > 0) {
    const int spb = rope_hd / 16, h = s / spb, j = s % spb;
    return h * rope_hd + (r < 8 ? 8 * j + r : rope_hd / 2 + 8 * j + r - 8);
  }
  return 16 * s + r;
}

__global__ void wf_shuffle_kernel(const _Float16* __restrict__ w, _Float16* __restrict__ wf, int nslabs, int K,
                                  int geglu_F, int rope_hd) {
  const int KS = K / 32;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)nslabs * KS * 64) return;
  const int lane = (int)(i % 64);
  const long blk = i / 64;
  const int ks = (int)(blk % KS), s = (int)(blk / KS);
  const int row = wf_row(s, lane & 15, geglu_F, rope_hd);
  *reinterpret_cast<h8*>(wf + i * 8) = *reinterpret_cast<const h8*>(w + (size_t)row * K + 32 * ks + 8 * (lane >> 4));
}

__global__ void wf_shuffle_q4_kernel(const uint32_t* __restrict__ qw, const _Float16* __restrict__ qs,
                                     uint32_t* __restrict__ qwf, _Float16* __restrict__ qsf, int nslabs, int K,
                                     int geglu_F, int rope_hd) {
  const int KCN = K / 128;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)nslabs * KCN * 64) return;
  const int lane = (int)(i % 64), g = lane >> 4;
  const long blk = i / 64;
  const int c = (int)(blk % KCN), s = (int)(blk / KCN);
  const int row = wf_row(s, lane & 15, geglu_F, rope_hd);
  *reinterpret_cast<u4*>(qwf + i * 4) = *reinterpret_cast<const u4*>(qw + (size_t)row * (K / 8) + 16 * c + 4 * g);
  qsf[i] = qs[(size_t)row * (K / 32) + 4 * c + g];
}

// instantiated (tile rows, prologue, epilogue) combinations -- the ones the engine uses:
//   16: adaRMS + store (q/k/v);  32: adaRMS + GeGLU, gated residual, plain store (action_in);
//   64: everything else
template <int NORM, int EPI, bool TABLE, int TR, int XM>
constexpr bool sk_combo() {
  if (XM == 1)
    return !TABLE && ((TR == 16 && ((NORM == 2 && EPI != EPI_GATED_RES && EPI != EPI_STORE_SILU) ||
                                    (NORM == 0 && EPI == EPI_GATED_RES))) ||
                      (TR == 32 && ((NORM == 2 && EPI == EPI_GEGLU) || (NORM == 0 && EPI == EPI_GATED_RES))));
  if (XM == 2)
    return NORM == 0 && ((TR == 16 && (EPI == EPI_STORE || (EPI == EPI_STORE_SILU && !TABLE))) ||
                         ((TR == 32 || TR == 64) && TABLE && EPI == EPI_STORE));
  if (TABLE) return TR == 64 && NORM == 0 && EPI == EPI_STORE;
  if (TR == 16) return NORM == 1 && EPI == EPI_STORE;
  if (TR == 32) return (NORM == 1 && EPI == EPI_GEGLU) || (NORM == 0 && (EPI == EPI_GATED_RES || EPI == EPI_STORE));
  return TR == 64 && NORM != 2 && EPI != EPI_GATED_RES && EPI != EPI_GEGLU;
}

template <bool Q4, int NORM, int EPI, bool TABLE, int TR, int XM, int MG>
int launch_nc_mg(const SkOp& op, int nc, dim3 grid, hipStream_t st) {
  constexpr bool MSD = (XM == 1 || XM == 2) && TR > 16;  // multi-slab register-direct tiles: 4 k groups
  constexpr int KG = MSD ? 4 : 4 / (TR / 16);
  if (nc < KG) nc = KG;
  switch (nc) {
    case 1:
      if constexpr (KG <= 1) skinny_kernel<Q4, NORM, EPI, 1, TABLE, TR, XM, MG><<<grid, 256, 0, st>>>(op);
      break;
    case 2:
      if constexpr (KG <= 2) skinny_kernel<Q4, NORM, EPI, 2, TABLE, TR, XM, MG><<<grid, 256, 0, st>>>(op);
      break;
    case 4: skinny_kernel<Q4, NORM, EPI, 4, TABLE, TR, XM, MG><<<grid, 256, 0, st>>>(op); break;
    case 16:  // one m tile per wave (4 m groups): a K slice of 2048 in one round of loads
      if constexpr (MG == 4 && NORM == 0) skinny_kernel<Q4, NORM, EPI, 16, TABLE, TR, XM, MG><<<grid, 256, 0, st>>>(op);
      else skinny_kernel<Q4, NORM, EPI, 8, TABLE, TR, XM, MG><<<grid, 256, 0, st>>>(op);
      break;
    default: skinny_kernel<Q4, NORM, EPI, 8, TABLE, TR, XM, MG><<<grid, 256, 0, st>>>(op); break;
  }
  return 0;
}

template <bool Q4, int NORM, int EPI, bool TABLE, int TR, int XM>
int launch_nc(const SkOp& op, int nc, dim3 grid, hipStream_t st) {
  if constexpr (!sk_combo<NORM, EPI, TABLE, TR, XM>()) {
    MLCV_REQUIRE(false, "skinny GEMM: tile rows / prologue / epilogue combination not built");
  } else {
    if (op.mg > 1) {
      // m groups: built for the fragment-major 16-row tiles
      if constexpr (XM == 1 && TR == 16 && !TABLE) {
        if (op.mg == 2) return launch_nc_mg<Q4, NORM, EPI, TABLE, TR, XM, 2>(op, nc, grid, st);
        return launch_nc_mg<Q4, NORM, EPI, TABLE, TR, XM, 4>(op, nc, grid, st);
      } else {
        MLCV_REQUIRE(false, "skinny GEMM m groups need fragment-major 16-row tiles");
      }
    }
    return launch_nc_mg<Q4, NORM, EPI, TABLE, TR, XM, 1>(op, nc, grid, st);
  }
  return 0;
}

template <bool Q4, int NORM, int EPI, bool TABLE, int XM>
int launch_tr(const SkOp& op, int nc, dim3 grid, hipStream_t st) {
  switch (op.tr) {
    case 16: return launch_nc<Q4, NORM, EPI, TABLE, 16, XM>(op, nc, grid, st);
    case 32: return launch_nc<Q4, NORM, EPI, TABLE, 32, XM>(op, nc, grid, st);
    case 64: return launch_nc<Q4, NORM, EPI, TABLE, 64, XM>(op, nc, grid, st);
    default: MLCV_REQUIRE(false, "skinny GEMM tile rows must be 16, 32 or 64");
  }
}

template <bool Q4, int NORM, int XM>
int launch_norm(const SkOp& op, int nc, dim3 grid, hipStream_t st) {
  switch (op.epi) {
    case EPI_STORE: return launch_tr<Q4, NORM, EPI_STORE, false, XM>(op, nc, grid, st);
    case EPI_GEGLU: return launch_tr<Q4, NORM, EPI_GEGLU, false, XM>(op, nc, grid, st);
    case EPI_VOUT: return launch_tr<Q4, NORM, EPI_VOUT, false, XM>(op, nc, grid, st);
    case EPI_EULER: return launch_tr<Q4, NORM, EPI_EULER, false, XM>(op, nc, grid, st);
    default: MLCV_REQUIRE(false, "unsupported skinny GEMM prologue/epilogue combination");
  }
}

template <bool Q4, int XM>
int launch_epi(const SkOp& op, int norm, int nc, dim3 grid, hipStream_t st) {
  if (norm == 1) return launch_norm<Q4, 1, XM>(op, nc, grid, st);
  if (norm == 2) return launch_norm<Q4, 2, XM>(op, nc, grid, st);
  switch (op.epi) {
    case EPI_STORE: return launch_tr<Q4, 0, EPI_STORE, false, XM>(op, nc, grid, st);
    case EPI_STORE_SILU: return launch_tr<Q4, 0, EPI_STORE_SILU, false, XM>(op, nc, grid, st);
    case EPI_GATED_RES: return launch_tr<Q4, 0, EPI_GATED_RES, false, XM>(op, nc, grid, st);
    default: MLCV_REQUIRE(false, "unsupported skinny GEMM prologue/epilogue combination");
  }
}

template <bool Q4>
int launch_q(const SkOp& op, int norm, int nc, dim3 grid, hipStream_t st) {
  if (op.nseg > 3) {
    MLCV_REQUIRE(norm == 0 && op.epi == EPI_STORE && op.seg_tiles > 0 && op.segs && !op.frag,
                 "more than 3 weight segments need equal sizes, a plain store and no prologue");
    if (op.xrow) return launch_tr<Q4, 0, EPI_STORE, true, 2>(op, nc, grid, st);
    return launch_tr<Q4, 0, EPI_STORE, true, 0>(op, nc, grid, st);
  }
  if (op.frag) return launch_epi<Q4, 1>(op, norm, nc, grid, st);
  if (op.xrow) return launch_epi<Q4, 2>(op, norm, nc, grid, st);
  return launch_epi<Q4, 0>(op, norm, nc, grid, st);
}

}  // namespace

int sk_launch(const SkOp& op, bool q4, hipStream_t st) {
  MLCV_REQUIRE(op.K % 32 == 0 && op.K >= 32, "skinny GEMM needs K % 32 == 0");
  MLCV_REQUIRE(op.M >= 1, "skinny GEMM needs M >= 1");
  MLCV_REQUIRE(op.splitk >= 1 && op.splitk <= MAX_SPLIT, "skinny GEMM split count");
  MLCV_REQUIRE(op.kper % KC == 0 && (long)op.kper * op.splitk >= op.K, "skinny GEMM split plan");
  MLCV_REQUIRE(op.zero != nullptr, "skinny GEMM needs the zero page");
  MLCV_REQUIRE(op.splitk == 1 || (op.ws && op.counters), "skinny GEMM split-K workspace missing");
  MLCV_REQUIRE(op.scale == nullptr || (op.rowss_in && op.rowss_tiles >= 4 && op.rowss_tiles % 4 == 0 &&
                                       op.rowss_ld % 4 == 0),
               "adaRMS prologue needs the producer's row statistics (groups of 16 columns, multiple of 4)");
  MLCV_REQUIRE(op.rowss_out == nullptr || op.rowss_ld > 0, "row statistics stride");
  MLCV_REQUIRE(op.ldx % 8 == 0, "skinny GEMM needs 16-byte aligned X rows");
  MLCV_REQUIRE(op.nseg >= 1, "skinny GEMM needs a weight segment");
  for (int i = 0; i < op.nseg && i < 3; ++i) {
    MLCV_REQUIRE(op.inl[i].n % 4 == 0 && op.inl[i].ldo % 4 == 0, "skinny GEMM outputs need n % 4 == 0");
  }
  const int mblocks = (op.M + MB - 1) / MB;
  const int mg = op.mg > 1 ? op.mg : 1;
  dim3 grid(op.ntiles, op.splitk, mblocks * mg);
  MLCV_REQUIRE(!op.prescaled || (op.rowss_in && op.M < MB && op.rowss_tiles >= 4 && op.rowss_tiles % 4 == 0 &&
                                  op.rowss_ld % 4 == 0),
               "pre-scaled adaRMS needs M < 64 (row M carries the shift) and the row statistics");
  MLCV_REQUIRE(op.xu_out == nullptr || (op.M < MB && op.xu_scale && op.xu_shift &&
                                        (op.epi == EPI_GATED_RES || op.epi == EPI_STORE) && op.nseg == 1),
               "pre-scaled output needs M < 64, its scale and shift, and a STORE / GATED_RES epilogue");
  const int norm = op.prescaled ? 2 : (op.scale != nullptr ? 1 : 0);
  const int cps = op.kper / KC;
  int nc = cps >= 5 ? 8 : cps >= 3 ? 4 : cps;
  static const bool nc16 = !std::getenv("MLCV_SK_NC16") || std::atoi(std::getenv("MLCV_SK_NC16")) != 0;
  if (nc16 && cps >= 16 && op.mg == 4 && op.frag && norm == 0) nc = 16;
  const bool direct = op.frag || op.xrow;  // operands straight into registers, little LDS
  MLCV_REQUIRE(!(op.frag && op.xrow), "fragment-major and row-major X at once");
  MLCV_REQUIRE(!direct || op.tr == 16 || (op.frag && op.tr == 32) || (op.xrow && (op.tr == 32 || op.tr == 64)),
               "register-direct operands need 16-row tiles (fragment-major X: 16 or 32; small-M row-major X: "
               "16, 32 or 64)");
  MLCV_REQUIRE(!op.xrow || (op.M <= 16 && op.K % 128 == 0 && norm == 0),
               "row-major direct X needs M <= 16, K % 128 == 0 and no prologue");
  MLCV_REQUIRE(!op.frag || (op.M < MB && op.K % 128 == 0 && op.nseg <= 3),
               "fragment-major operands need M < 64, K % 128 == 0 and at most 3 segments");
  MLCV_REQUIRE(!op.frag_out || op.M < MB, "fragment-major outputs need M < 64");
  for (int i = 0; i < op.nseg && i < 3; ++i)
    MLCV_REQUIRE(op.inl[i].rope == 0 || (op.frag && op.tr == 16 && op.epi == EPI_STORE && op.rope_cos &&
                                         op.rope_sin && op.rope_hd >= 16 && op.rope_hd % 16 == 0 &&
                                         op.rope_grp >= 1 && op.rope_rpad % 64 == 0),
                 "RoPE epilogue needs fragment-major 16-row store tiles and its tables");
  MLCV_REQUIRE(mg == 1 || ((mg == 2 || mg == 4) && op.frag && op.tr == 16 && norm != 1 && op.nseg <= 3),
               "skinny GEMM m groups (2 or 4) need fragment-major 16-row tiles");
  if (!direct && nc > 4 && (long)grid.x * grid.y * grid.z > 256) nc = 4;  // keep 2 workgroups per CU (LDS)
  MLCV_REQUIRE(op.pf.nreg >= 0 && op.pf.nreg <= PF_MAX_REGIONS, "prefetch regions");
  for (int i = 0; i < op.pf.nreg; ++i)
    MLCV_REQUIRE(op.pf.r[i].slab_bytes > 0 && op.pf.r[i].slab_bytes % 64 == 0 && op.pf.r[i].nslabs >= 0,
                 "prefetch slabs must be whole 64-byte lines");
  SkOp kop = op;
  const int pf_rows = op.pf.nreg > 0 && op.pf.nblocks > 0 ? (op.pf.nblocks + op.ntiles - 1) / op.ntiles : 0;
  kop.pf.nblocks = pf_rows * op.ntiles;
  grid.y += pf_rows;
  if (q4) MLCV_TRY(launch_q<true>(kop, norm, nc, grid, st));
  else MLCV_TRY(launch_q<false>(kop, norm, nc, grid, st));
  MLCV_HIP(hipGetLastError());
  return 0;
}

int wf_shuffle_launch(const _Float16* w, _Float16* wf, int N, int K, int geglu_F, int rope_hd, hipStream_t st) {
  MLCV_REQUIRE(K % 128 == 0, "fragment-major weights need K % 128 == 0");
  MLCV_REQUIRE(geglu_F > 0 ? (N == 2 * geglu_F && geglu_F % 8 == 0) : N % 16 == 0,
               "fragment-major weights need 16-row slabs (GeGLU: F % 8 == 0)");
  MLCV_REQUIRE(rope_hd <= 0 || (geglu_F <= 0 && rope_hd % 16 == 0 && N % rope_hd == 0), "RoPE pairing shape");
  const int nslabs = geglu_F > 0 ? geglu_F / 8 : N / 16;
  const long n = (long)nslabs * (K / 32) * 64;
  wf_shuffle_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(w, wf, nslabs, K, geglu_F, rope_hd);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int wf_shuffle_q4_launch(const uint32_t* qw, const _Float16* qs, uint32_t* qwf, _Float16* qsf, int N, int K,
                         int geglu_F, int rope_hd, hipStream_t st) {
  MLCV_REQUIRE(K % 128 == 0, "fragment-major weights need K % 128 == 0");
  MLCV_REQUIRE(geglu_F > 0 ? (N == 2 * geglu_F && geglu_F % 8 == 0) : N % 16 == 0,
               "fragment-major weights need 16-row slabs (GeGLU: F % 8 == 0)");
  MLCV_REQUIRE(rope_hd <= 0 || (geglu_F <= 0 && rope_hd % 16 == 0 && N % rope_hd == 0), "RoPE pairing shape");
  const int nslabs = geglu_F > 0 ? geglu_F / 8 : N / 16;
  const long n = (long)nslabs * (K / 128) * 64;
  wf_shuffle_q4_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(qw, qs, qwf, qsf, nslabs, K, geglu_F, rope_hd);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int q4_quantize_launch(const _Float16* w, uint32_t* qw, _Float16* qs, int N, int K, hipStream_t st) {
  MLCV_REQUIRE(K % 32 == 0, "q4 quantize needs K % 32 == 0");
  const long groups = (long)N * (K / 32);
  q4_quantize_kernel<<<(unsigned)((groups + 255) / 256), 256, 0, st>>>(w, qw, qs, N, K);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int q4_dequant_launch(const uint32_t* qw, const _Float16* qs, _Float16* out, int N, int K, hipStream_t st) {
  MLCV_REQUIRE(K % 32 == 0, "q4 dequant needs K % 32 == 0");
  const long words = (long)N * (K / 8);
  q4_dequant_kernel<<<(unsigned)((words + 255) / 256), 256, 0, st>>>(qw, qs, out, N, K);
  MLCV_HIP(hipGetLastError());
  return 0;
}

namespace {
// one norm per workgroup
__global__ __launch_bounds__(256) void nscale_kernel(const _Float16* __restrict__ mod, int W1, int NM, int norm_lo,
                                                     int norms_n, float* __restrict__ out) {
  __shared__ float red[4];
  const int n = (blockIdx.x / norms_n) * NM + norm_lo + blockIdx.x % norms_n;
  const _Float16* sc = mod + (size_t)n * 3 * W1;
  float mx = 0.f;
  for (int j = threadIdx.x; j < W1; j += 256) mx = fmaxf(mx, fabsf(1.0f + h2f(sc[j])));
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float c = 1.0f;
    if (v <= 3.0e38f) {  // finite (a NaN or inf modulation leaves c = 1)
      while (v * c > 1.0f) c *= 0.5f;
    }
    out[n] = c;
  }
}
}  // namespace

int nscale_launch(const _Float16* mod, int W1, int NM, int steps, int norm_lo, int norms_n, float* out,
                  hipStream_t st) {
  MLCV_REQUIRE(steps > 0 && norms_n > 0 && W1 > 0 && norm_lo >= 0 && norm_lo + norms_n <= NM, "norm scale arguments");
  nscale_kernel<<<steps * norms_n, 256, 0, st>>>(mod, W1, NM, norm_lo, norms_n, out);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
