#include <cstdlib>
// Tiled MFMA GEMM for prefill (M = prefix length, ~1k rows): C[M,N] = A[M,K] . B[N,K]^T,
// fp16 operands, fp32 accumulation on v_mfma_f32_32x32x16_f16.
//
// Workgroup tile 128 x 128 x 64, 4 waves in 2 x 2, each wave 64 x 64 (2 x 2 MFMA
// blocks of 32 x 32).  Both operands are K-contiguous ("NT"), staged through
// double-buffered LDS with a 16-byte row pad (conflict-free 16-byte MFMA operand
// reads).  Tiles are ordered so that all M tiles of one N tile run on the same XCD
// (dispatch is round-robin over the 8 XCDs), so each weight tile is fetched into
// one L2 only.
#include "kernels.h"

#include <algorithm>

namespace mlcv {

namespace {
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;  // halfs per LDS row
constexpr int NXCD = TG_NXCD;

__device__ __forceinline__ const _Float16* brow_ptr(const TgArgs& a, int n) {
  if (n < a.n1) return a.b0 + (size_t)n * a.ldb;
  if (n < a.n2) return a.b1 + (size_t)(n - a.n1) * a.ldb;
  return a.b2 + (size_t)(n - a.n2) * a.ldb;
}

__global__ __launch_bounds__(256) void tile_gemm_kernel(TgArgs a, int mtiles, int ntiles) {
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDK];

  // XCD-aware tile order
  const int id = blockIdx.x;
  const int xcd = id % NXCD, k = id / NXCD;
  const int tm = k % mtiles;
  const int tn = xcd + NXCD * (k / mtiles);
  if (tn >= ntiles) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const bool geglu = a.epi == TG_GEGLU;
  const int m0 = tm * BM;

  // global -> register staging: 4 x 16 B of A and of B per thread
  const int lrow = tid >> 3, lk = (tid & 7) * 8;
  const _Float16* aptr[4];
  const _Float16* bptr[4];
  bool aok[4], bok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = lrow + 32 * i;
    const int m = m0 + r;
    aok[i] = m < a.M;
    aptr[i] = a.a + (size_t)(aok[i] ? m : 0) * a.lda;
    int n;
    if (geglu) {
      const int j0 = tn * 64;
      const int wnn = r / 64, bn = (r / 32) & 1, jj = r & 31;
      n = (bn ? a.F : 0) + j0 + 32 * wnn + jj;
      bok[i] = true;
      bptr[i] = a.b0 + (size_t)n * a.ldb;
    } else {
      n = tn * BN + r;
      bok[i] = n < a.N;
      bptr[i] = brow_ptr(a, bok[i] ? n : 0);
    }
  }

  h8 ra[4], rb[4];
  auto gload = [&](int kt) {
    const int kk = kt * BK + lk;
    const bool kok = kk < a.K;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = (aok[i] && kok) ? *reinterpret_cast<const h8*>(aptr[i] + kk) : (h8){0, 0, 0, 0, 0, 0, 0, 0};
      rb[i] = (bok[i] && kok) ? *reinterpret_cast<const h8*>(bptr[i] + kk) : (h8){0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<h8*>(&As[buf][(lrow + 32 * i) * LDK + lk]) = ra[i];
      *reinterpret_cast<h8*>(&Bs[buf][(lrow + 32 * i) * LDK + lk]) = rb[i];
    }
  };

  f16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int nk = (a.K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int l32 = lane & 31, lh = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      h8 av[2], bv[2];
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
        av[bm] = *reinterpret_cast<const h8*>(&As[cur][(wm * 64 + bm * 32 + l32) * LDK + ks * 16 + 8 * lh]);
#pragma unroll
      for (int bn = 0; bn < 2; ++bn)
        bv[bn] = *reinterpret_cast<const h8*>(&Bs[cur][(wn * 64 + bn * 32 + l32) * LDK + ks * 16 + 8 * lh]);
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int bn = 0; bn < 2; ++bn) acc[bm][bn] = mfma32x32x16(av[bm], bv[bn], acc[bm][bn]);
    }
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds D[8*(e/4) + 4*lh + (e%4)][l32] of each 32x32 block
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm * 64 + bm * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
      if (m >= a.M) continue;
      if (geglu) {
        const int j = tn * 64 + 32 * wn + l32;
        const _Float16 gv = f2h(acc[bm][0][e]);
        const _Float16 uv = f2h(acc[bm][1][e]);
        a.c[(size_t)m * a.ldc + j] = hmul(f2h(gelu_tanh_hw(h2f(gv))), uv);
        continue;
      }
#pragma unroll
      for (int bn = 0; bn < 2; ++bn) {
        const int n = tn * BN + wn * 64 + bn * 32 + l32;
        if (n >= a.N) continue;
        _Float16* cp = a.c + (size_t)m * a.ldc + n;
        const _Float16 y = f2h(acc[bm][bn][e]);
        if (a.epi == TG_RESIDUAL) *cp = hadd(*cp, y);
        else *cp = y;
      }
    }
  }
}

// ---- long-M GEMM: 256-row tiles, operands DMA'd straight into swizzled LDS ----------------
//
// Workgroup tile 256 (m) x BN (n) x BK (k).  4 waves in 2 x 2: wave (wm, wn) owns m rows
// [128 wm, +128) and n rows [BN/2 wn, +BN/2); 8 waves in 2 x 4: n rows [BN/4 wn, +BN/4).  A
// wave's rows are 4 x NBW blocks of 32 x 32 on v_mfma_f32_32x32x16_f16 with the weights as
// the A operand, so D[n][m] leaves each lane 4 consecutive n of one m row (8-byte stores).
// LDS: per stage A 256 x BK and B BN x BK halfs.  One global_load_lds of 16 B per lane
// moves 512 / BK rows (BK 64: 8 rows x 128 B, a row is 8 lanes, one whole line); row r's
// piece p (8 halfs) lands in slot p ^ swz(r) of the row, so the MFMA operand reads
// (consecutive lanes = consecutive rows, same piece) touch distinct 16-byte slots:
// conflict-free.  NST stages: the DMA of k tiles t + 1 .. t + NST - 2 runs while tile t is
// multiplied.
// Split-K (SPLIT): the S workgroups of a tile run on one XCD (workgroups are dealt to the 8
// XCDs round-robin by linear id); each writes its fp32 partial in the MFMA register order
// (1 KB per store), they meet (group_meet_gen: the grid is launched only when it fits on
// the CUs at once, so the meeting completes), and each reduces a share of the tile's blocks
// in split order (deterministic) before the epilogue.  Should other work hold CUs so that a
// split cannot start, the waiting workgroups give up after TgArgs::meet_polls polls: they
// write NaN and raise the error word, which the entry point reports as a failed call.
constexpr int GBM = TG_BM, GBK = TG_BK;

struct GemmPlan : TilePlan {
  float* ws;               // split-K partials [tile][split][4 waves][blocks][4][64] f4
  unsigned* sync;          // per tile: 32 words (arrivals, generation)
};

// 16 bytes per lane from a buffer into LDS at lds + 16 lane.  The builtin is only given to
// the device pass: in the host pass it makes clang drop the launch stubs of the kernels
// that use it, without a diagnostic.
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, __attribute__((address_space(3))) void* lds,
                                                int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
#endif
}

// LDS image of a row-major operand tile of BK halfs per row: one 1 KB DMA instruction holds
// RPI = 512 / BK rows, row r's 16-byte piece p sits in slot p ^ swz(r) of the row.  The
// MFMA operand read (consecutive lanes = consecutive rows, one piece) then hits distinct
// banks whether the LDS serves 128 or 256 bytes of a 16-byte read per clock (32 or 64 banks):
// BK 32 (64-byte rows) swizzles by (r / 4) mod 4; BK 64 (128-byte rows) by (r mod 8) xor
// bit 3 of r, which separates rows r and r + 8 (the same bank half at 64 banks; r mod 8
// alone made them collide: a 2-way conflict on every operand read).
template <int BK>
__device__ __forceinline__ int tile_swz(int r) { return BK == 64 ? ((r & 7) ^ ((r >> 3) & 1)) : ((r >> 2) & 3); }
template <int BK>
__device__ __forceinline__ int lds_swz(int r, int p) {
  constexpr int RPI = 512 / BK;
  return (r / RPI) * 1024 + (r % RPI) * (BK * 2) + ((p ^ tile_swz<BK>(r)) << 4);
}
// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}
// LDS barrier without a wait for outstanding global loads (the DMA of later stages)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// NWV waves: 4 in 2 x 2 (a wave owns 128 m x BN/2 n), or 8 in 2 x 4 (128 m x BN/4 n; two
// waves per SIMD, so one's LDS reads and barrier waits overlap the other's MFMAs)
// BM: m rows of the tile (256, or 128: 64 m rows per wave)
template <int BN, int BK, int NST, int EPI, bool SPLIT, int NWV = 4, int BM = GBM>
__global__ __launch_bounds__(64 * NWV) void big_gemm_kernel(TgArgs a, GemmPlan p) {
  static_assert(NWV == 4 || (NWV == 8 && BN >= 128), "8 waves need n tiles of 128 or 256");
  static_assert(BM == 256 || BM == 128, "m tiles of 256 or 128 rows");
  constexpr int WNN = NWV / 2;                  // waves along n
  constexpr int TNW = BN / WNN;                 // n rows per wave
  constexpr int NBW = TNW / 32;                 // n blocks of 32 per wave
  constexpr int TMW = BM / 2;                   // m rows per wave
  constexpr int MB = TMW / 32;                  // m blocks of 32 per wave
  constexpr int ASZ = BM * BK * 2, BSZ = BN * BK * 2;
  constexpr int STG = ASZ + BSZ;
  constexpr int RPI = 512 / BK, LPR = BK / 8;   // rows per DMA instruction, lanes per row
  __shared__ __attribute__((aligned(16))) char lds[NST * STG];
  typedef __attribute__((address_space(3))) void* lptr_t;

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, lh = lane >> 5;
  const int wm = w / WNN, wn = w % WNN;
  // tile and K slice: XCD x (id % 8) owns the consecutive tiles [x per, (x + 1) per), all
  // M tiles of an N tile together, so each weight tile is fetched into one L2; the S
  // slices of a tile share the XCD
  const int id = blockIdx.x, xcd = id % NXCD, j = id / NXCD;
  const int S = SPLIT ? p.splitk : 1;
  const int s = j % S, tl = j / S;
  const int ntile_all = p.mtiles * p.ntiles, per = (ntile_all + NXCD - 1) / NXCD;
  const int tile = xcd * per + tl;
  if (tile >= ntile_all) return;
  // split K: the generation of the tile's meeting, read now (off the meeting's critical path)
  const unsigned gen = SPLIT && tid == 0 ? group_gen(p.sync + 32 * tile) : 0u;
  const int tm = tile % p.mtiles, tn = tile / p.mtiles;
  const int m0 = tm * BM;
  const int kbeg = s * p.kt_per * GBK, nkt = (min(a.K, kbeg + p.kt_per * GBK) - kbeg + BK - 1) / BK;

  // DMA of this wave's rows: A rows [GBM/NWV w, +GBM/NWV), B rows [BN/NWV w, +BN/NWV), RPI
  // rows per instruction, as buffer loads to LDS: a 32-bit row offset per lane, the k tile in
  // the scalar offset; rows past the operand read zeros (the buffer's size)
  constexpr int NAI = BM / RPI / NWV, NBI = BN / RPI / NWV, NI = NAI + NBI;
  static_assert(NAI * RPI * NWV == BM && NBI * RPI * NWV == BN, "whole DMA instructions per wave");
  // row in the instruction and LDS slot of this lane; the piece it loads depends on the tile row
  const int lr = lane / LPR, ls = lane % LPR;
  // tile-major X (32-k tiles with TgArgs::at): whole 16-row blocks, so the buffer ends at the
  // last block's end (rows past M inside it are finite data whose products are never stored)
  const bool xt = BK == 32 && a.at != 0;
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(a.a), 0,
      (int)min(xt ? (size_t)((a.M + 15) / 16) * 16 * a.lda * 2 : (size_t)a.M * a.lda * 2, (size_t)0x7fffffff),
      0x00020000);
  int aoff[NAI], apc[NAI];
#pragma unroll
  for (int i = 0; i < NAI; ++i) {
    const int r = (NAI * w + i) * RPI + lr;
    apc[i] = ls ^ tile_swz<BK>(r);
    aoff[i] = xt ? (m0 + r - lr) / 16 * (a.K / 32) * 1024 + lr * 64 + apc[i] * 16 : ((m0 + r) * a.lda + apc[i] * 8) * 2;
  }
  // tile-major weights (32-k tiles with TgArgs::bt): block (row / 16, k / 32) is 1 KB, the lane's
  // piece at (row % 16) * 64 + 16 piece; the k tile moves the scalar offset by 1 KB per 32 k
  const bool wt = BK == 32 && a.bt != nullptr;
  const _Float16* bbase[NBI];  // per instruction (wave-uniform): segment base and bytes
  int bbytes[NBI], boff[NBI], bpc[NBI];
#pragma unroll
  for (int i = 0; i < NBI; ++i) {
    const int r0 = (NBI * w + i) * RPI;  // first B tile row of the instruction (uniform)
    const _Float16* base;
    int rows, row;
    if constexpr (EPI == TG_GEGLU) {
      // wave half wn holds 64 outputs as [gate 32, up 32, gate 32, up 32]
      const int hw = r0 / (BN / 2), blk = (r0 % (BN / 2)) / 32;
      const int jo = tn * (BN / 2) + hw * (BN / 4) + (blk >> 1) * 32 + (r0 % 32);
      base = a.b0;
      rows = 2 * a.F;
      row = ((blk & 1) ? a.F + jo : jo) + lr;
    } else {
      const int n0 = tn * BN + r0;  // segment boundaries are multiples of 8
      const int seg0 = n0 < a.n1 ? 0 : n0 < a.n2 ? a.n1 : a.n2;
      base = n0 < a.n1 ? a.b0 : n0 < a.n2 ? a.b1 : a.b2;
      rows = (n0 < a.n1 ? a.n1 : n0 < a.n2 ? a.n2 : a.N) - seg0;
      row = n0 - seg0 + lr;
    }
    bbase[i] = wt ? a.bt : base;
    bbytes[i] = (int)min((size_t)rows * a.ldb * 2, (size_t)0x7fffffff);
    bpc[i] = ls ^ tile_swz<BK>(r0 + lr);
    boff[i] = wt ? ((row - lr) / 16 * (a.K / 32) * 1024 + lr * 64 + bpc[i] * 16) : (row * a.ldb + bpc[i] * 8) * 2;
  }
  // DMA instruction i (A rows for i < NAI, then B rows) of k tile kt into a stage
  // K past the last multiple of BK: this lane's 8-half piece at k >= K gets an offset past the
  // buffer, which reads zeros (K % 8 == 0, so a piece is wholly inside or outside)
  constexpr int OOB = 0x7ffffff0;
  // live = false: the same instruction reads zeros (an offset past the buffer) into a free
  // stage, so the k loop issues its DMA unconditionally: a branch around it made the compiler
  // wait for every outstanding LDS read at the join, before the first MFMA of the tile
  auto dma1 = [&](int i, int kt, int stage, bool live = true) __attribute__((always_inline)) {
    char* sb = lds + stage * STG;
    const int ko = (kbeg + kt * BK) * 2;
    const bool kin = live && kbeg + kt * BK + (i < NAI ? apc[i] : bpc[i - NAI]) * 8 < a.K;
    if (i < NAI)
      buffer_to_lds16(rA, (lptr_t)(sb + (NAI * w + i) * 1024), kin ? aoff[i] : OOB, xt ? ko * 16 : ko);
    else
      buffer_to_lds16(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(bbase[i - NAI]), 0, bbytes[i - NAI], 0x00020000),
          (lptr_t)(sb + ASZ + (NBI * w + i - NAI) * 1024), kin ? boff[i - NAI] : OOB, wt ? ko * 16 : ko);
  };
  auto dma = [&](int kt, int stage, bool live) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NI; ++i) dma1(i, kt, stage, live);
  };

  f16v acc[NBW][MB];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[nb][mb][e] = 0.f;

  // operand fragments of k step kb (16 k): weights of the wave's n blocks, X of its m blocks
  auto ldfrag = [&](const char* sa, int kb, h8* wf, h8* xf) __attribute__((always_inline)) {
    const int pp = 2 * kb + lh;
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
      wf[nb] = *reinterpret_cast<const h8*>(sa + ASZ + lds_swz<BK>(wn * TNW + nb * 32 + l32, pp));
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xf[mb] = *reinterpret_cast<const h8*>(sa + lds_swz<BK>(wm * TMW + mb * 32 + l32, pp));
  };

  // NST-stage ring: the DMA of tiles kt+1 .. kt+NST-2 stays in flight while tile kt
  // multiplies; tile kt+NST-1 goes into the stage tile kt-1 used.  Every tile issues its NI
  // instructions (zeros past the K range), so the vmcnt counts below hold at the tail too.
  // Pipelined across tiles: before the last MFMA group of tile kt (whose fragments are in
  // registers) the wave waits for tile kt+1, crosses the barrier and reads tile kt+1's first
  // fragments, so that LDS latency hides under that group.
  static_assert(NST >= 3, "the ring keeps one tile in flight beyond the next");
  constexpr int KB = BK / 16;          // k steps per tile
  constexpr int NP = KB * NBW;         // MFMA groups of 4 per tile
  static_assert(KB % 2 == 0, "fragment buffers alternate by k step parity");
  // DMA instructions issued before the last group (tile kt+NST-1's part in flight at the wait)
  constexpr int ISSUED = [] {
    int n = 0;
    for (int i = 0; i < NI; ++i) n += (i * NP) / NI < NP - 1;
    return n;
  }();
  // late: the next k step's fragments are read after the first group of this one (NBW >= 2;
  // read before the group, the compiler waited for all of them at its first MFMA)
  constexpr bool LATE = NBW >= 2;
#pragma unroll
  for (int t = 0; t < NST - 1; ++t) dma(t, t, t < nkt);
  h8 wf[2][NBW], xf[2][MB];
  vm_wait<(NST - 2) * NI>();  // this wave's DMA of tile 0 (loads complete in issue order)
  lds_barrier();
  ldfrag(lds, 0, wf[0], xf[0]);
  for (int kt = 0; kt < nkt; ++kt) {
    const bool more = kt + NST - 1 < nkt, next = kt + 1 < nkt;
    const int knext = kt + NST - 1, snext = (kt + NST - 1) % NST;
    const char* sa = lds + (kt % NST) * STG;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (!LATE && kb + 1 < KB) ldfrag(sa, kb + 1, wf[(kb + 1) & 1], xf[(kb + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        const int piece = kb * NBW + nb;
        if (piece == NP - 1 && next) {
          // every fragment of tile kt is in registers once this wave's reads are back; after
          // the barrier no wave reads tile kt's stage, and tile kt+1 is in LDS
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
          vm_wait<(NST - 3) * NI + ISSUED>();
          lds_barrier();
          ldfrag(lds + ((kt + 1) % NST) * STG, 0, wf[0], xf[0]);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if ((i * NP) / NI == piece) dma1(i, knext, snext, more);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mfma32x32x16(wf[kb & 1][nb], xf[kb & 1][mb], acc[nb][mb]);
        __builtin_amdgcn_sched_barrier(0);
        if (LATE && nb == 0 && kb + 1 < KB) {
          ldfrag(sa, kb + 1, wf[(kb + 1) & 1], xf[(kb + 1) & 1]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  vm_wait<0>();  // the zero-filling DMA past the K range, before the epilogue

  // epilogue of one 32 x 32 block (wave role wm2 / wn2, blocks nb / mb): lane column
  // m = l32, rows n = 8 (e / 4) + 4 lh + (e % 4)
  auto store_block = [&](const f16v& v, int wm2, int wn2, int nb, int mb) __attribute__((always_inline)) {
    const int m = m0 + wm2 * TMW + mb * 32 + l32;
    if (m >= a.M) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = tn * BN + wn2 * TNW + nb * 32 + 8 * q + 4 * lh;
      if (n >= a.N) continue;
      _Float16* cp = a.c + (size_t)m * a.ldc + n;
      h4 y;
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = f2h(v[4 * q + i]);
      if constexpr (EPI == TG_RESIDUAL) {
        const h4 c0 = *reinterpret_cast<const h4*>(cp);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = hadd(c0[i], y[i]);
      }
      *reinterpret_cast<h4*>(cp) = y;
    }
  };

  if constexpr (EPI == TG_GEGLU) {
    // blocks (0, 1) and (2, 3) of the wave are gate / up of the same 32 outputs
#pragma unroll
    for (int hb = 0; hb < NBW / 2; ++hb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = m0 + wm * TMW + mb * 32 + l32;
        if (m >= a.M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int jo = tn * (BN / 2) + wn * (TNW / 2) + hb * 32 + 8 * q + 4 * lh;
          h4 y;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const _Float16 gv = f2h(acc[2 * hb][mb][4 * q + i]), uv = f2h(acc[2 * hb + 1][mb][4 * q + i]);
            y[i] = hmul(f2h(gelu_tanh_hw(h2f(gv))), uv);
          }
          const size_t ci = a.ct ? ((size_t)(m >> 4) * (a.ldc >> 5) + (jo >> 5)) * 512 + (m & 15) * 32 + (jo & 31)
                                 : (size_t)m * a.ldc + jo;
          *reinterpret_cast<h4*>(a.c + ci) = y;
        }
      }
    return;
  } else if constexpr (!SPLIT) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) store_block(acc[nb][mb], wm, wn, nb, mb);
    return;
  } else {
    // partial of this split: [wave][nb][mb][q][lane] f4
    constexpr int BLK = NBW * MB;               // blocks per wave
    constexpr size_t TILE_F4 = NWV * BLK * 4 * 64;  // f4 per split partial
    f4* part = reinterpret_cast<f4*>(p.ws) + ((size_t)tile * S + s) * TILE_F4;
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f4 v = {acc[nb][mb][4 * q], acc[nb][mb][4 * q + 1], acc[nb][mb][4 * q + 2], acc[nb][mb][4 * q + 3]};
          part[((w * BLK + nb * MB + mb) * 4 + q) * 64 + lane] = v;
        }
    int& met = *reinterpret_cast<int*>(lds);  // the stages are free after the last tile
    wait_all_memory();
    __syncthreads();
    if (tid == 0) {
      met = group_meet_gen(p.sync + 32 * tile, (unsigned)S, a.meet_polls, gen);
      if (!met && a.err) __hip_atomic_store(a.err, TG_ERR_MEET, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    // blocks u = (wave role, nb, mb) of the tile, u % S == s, one wave each
    const f4* base = reinterpret_cast<const f4*>(p.ws) + (size_t)tile * S * TILE_F4;
    for (int u = s + S * w; u < NWV * BLK; u += NWV * S) {
      const int w2 = u / BLK, b = u % BLK, nb = b / MB, mb = b % MB;
      f16v v;
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = 0.f;
      for (int sp = 0; sp < S; ++sp) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f4 x = base[(size_t)sp * TILE_F4 + ((size_t)u * 4 + q) * 64 + lane];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[4 * q + i] += x[i];
        }
      }
      if (!met) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = __builtin_nanf("");
      }
      store_block(v, w2 / WNN, w2 % WNN, nb, mb);
    }
  }
}

// 256-row tile plan; false = the shape needs the 128 x 128 kernel
bool big_plan(const TgArgs& a, GemmPlan& p) {
  TilePlanIn in{};
  in.M = a.M;
  in.N = a.N;
  in.K = a.K;
  in.F = a.F;
  in.n1 = a.n1;
  in.n2 = a.n2;
  in.lda = a.lda;
  in.ldb = a.ldb;
  in.ldc = a.ldc;
  in.geglu = a.epi == TG_GEGLU;
  in.small_tiles = a.small_tiles != 0;
  in.split_ws = a.ws && a.sync;
  in.ws_floats = a.ws_floats;
  in.sync_tiles = a.sync_tiles;
  in.cus = device_cus();
  static const bool m128 = !std::getenv("MLCV_TG_M128") || std::atoi(std::getenv("MLCV_TG_M128")) != 0;
  in.m128 = m128;  // tuning switch
  static const bool n64m128 = !std::getenv("MLCV_TG_N64M128") || std::atoi(std::getenv("MLCV_TG_N64M128")) != 0;
  in.n64m128 = n64m128;
  if (!tile_plan(in, p)) return false;
  p.ws = a.ws;
  p.sync = a.sync;
  return true;
}

__global__ void wtile_shuffle_kernel(const _Float16* __restrict__ w, _Float16* __restrict__ wt, int K, long n8) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;  // one 8-half piece of the copy
  if (i >= n8) return;
  const int KT = K / 32;
  const long blk = i / 64;  // 1 KB block (row / 16, k tile)
  const int e = (int)(i % 64), r = e / 4, q = e % 4;
  const long rb = blk / KT;
  const int kt = (int)(blk % KT);
  *reinterpret_cast<h8*>(wt + i * 8) = *reinterpret_cast<const h8*>(w + (rb * 16 + r) * (long)K + kt * 32 + 8 * q);
}

int big_launch(const TgArgs& a, const GemmPlan& p, hipStream_t st) {
  MLCV_REQUIRE(!a.bt || ((a.epi == TG_GEGLU || (a.n1 >= a.N && a.n2 >= a.N)) && a.ldb == a.K && a.K % 32 == 0),
               "tile-major weights need one segment (or GeGLU) and K-contiguous rows, K % 32 == 0");
  // the tile-major X / output layouts exist only in the 32-k tiles of 256 x 256
  const bool k32 = p.bm == 256 && (p.bn == 256 || a.epi == TG_GEGLU);
  MLCV_REQUIRE(!(a.at || a.ct) || (k32 && a.lda == a.K && a.K % 32 == 0 && (!a.ct || (a.epi == TG_GEGLU && a.ldc % 32 == 0))),
               "tile-major X / GeGLU output: only on the 256 x 256 tiles of 32 k");
  const int tiles = p.mtiles * p.ntiles;
  // the split-K kernels (every 256 x 256 product but GeGLU) store partials and meet per tile
  MLCV_REQUIRE(!((p.bm == 256 && p.bn == 256 && a.epi != TG_GEGLU) || p.splitk > 1) ||
                   (p.ws && p.sync && tiles <= a.sync_tiles),
               "split-K tile GEMM without a workspace and meeting counters for its tiles");
  const unsigned blocks = (unsigned)(((tiles + NXCD - 1) / NXCD) * NXCD * p.splitk);
  // 256 x 256 tiles: 4 stages of 32 k (128 KB), 8 waves (the prefill at P = 968: down 92 vs
  // 102 us, its split-K reduction spread over twice the waves; gate_up unchanged; 5 stages
  // (160 KB) were slower); 256 x 128: 3 stages of 64 k (144 KB); 256 x 64: 3 stages of 64 k
  if (p.bm == 128 && p.bn == 64) {
    // 128 x 64 over the whole K, 4 waves of 64 x 32, 4 stages (96 KB): the prefill's o_proj on
    // 256 workgroups instead of 128 (prefill 5.25 vs 5.33 ms, results identical); q/k/v on
    // 3-stage 128 x 64 tiles (two workgroups per CU for its 320 tiles) was slower than 128 x 128
    if (a.epi == TG_RESIDUAL) big_gemm_kernel<64, 64, 4, TG_RESIDUAL, false, 4, 128><<<blocks, 256, 0, st>>>(a, p);
    else big_gemm_kernel<64, 64, 4, TG_STORE, false, 4, 128><<<blocks, 256, 0, st>>>(a, p);
  } else if (p.bm == 128) {
    // 128 x 128 over the whole K: 4 stages of 64 k (128 KB), 8 waves of 64 x 32 (the prefill's
    // q/k/v 21.2 and o_proj 23.2 us against 256 x 64 tiles' 27 and 29 us; 8 waves against 4:
    // prefill -12 us)
    if (a.epi == TG_RESIDUAL) big_gemm_kernel<128, 64, 4, TG_RESIDUAL, false, 8, 128><<<blocks, 512, 0, st>>>(a, p);
    else big_gemm_kernel<128, 64, 4, TG_STORE, false, 8, 128><<<blocks, 512, 0, st>>>(a, p);
  } else if (a.epi == TG_GEGLU) big_gemm_kernel<256, 32, 4, TG_GEGLU, false, 8><<<blocks, 512, 0, st>>>(a, p);
  else if (p.bn == 256) {
    if (a.epi == TG_RESIDUAL) big_gemm_kernel<256, 32, 4, TG_RESIDUAL, true, 8><<<blocks, 512, 0, st>>>(a, p);
    else big_gemm_kernel<256, 32, 4, TG_STORE, true, 8><<<blocks, 512, 0, st>>>(a, p);
  } else if (p.bn == 64) {
    if (p.splitk > 1) {
      if (a.epi == TG_RESIDUAL) big_gemm_kernel<64, 64, 3, TG_RESIDUAL, true><<<blocks, 256, 0, st>>>(a, p);
      else big_gemm_kernel<64, 64, 3, TG_STORE, true><<<blocks, 256, 0, st>>>(a, p);
    } else {
      if (a.epi == TG_RESIDUAL) big_gemm_kernel<64, 64, 3, TG_RESIDUAL, false><<<blocks, 256, 0, st>>>(a, p);
      else big_gemm_kernel<64, 64, 3, TG_STORE, false><<<blocks, 256, 0, st>>>(a, p);
    }
  } else if (p.splitk > 1) {
    if (a.epi == TG_RESIDUAL) big_gemm_kernel<128, 64, 3, TG_RESIDUAL, true><<<blocks, 256, 0, st>>>(a, p);
    else big_gemm_kernel<128, 64, 3, TG_STORE, true><<<blocks, 256, 0, st>>>(a, p);
  } else {
    if (a.epi == TG_RESIDUAL) big_gemm_kernel<128, 64, 3, TG_RESIDUAL, false><<<blocks, 256, 0, st>>>(a, p);
    else big_gemm_kernel<128, 64, 3, TG_STORE, false><<<blocks, 256, 0, st>>>(a, p);
  }
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace

int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

size_t tg_sync_words() { return (size_t)std::max(device_cus(), 1) * 32; }
// one 256 x 256 fp32 partial per CU
size_t tg_ws_floats() { return (size_t)std::max(device_cus(), 1) * GBM * 256; }

int tg_launch(const TgArgs& a, hipStream_t st) {
  MLCV_REQUIRE(a.K % 8 == 0 && a.lda % 8 == 0 && a.ldb % 8 == 0, "tile GEMM needs 16-byte aligned rows");
  GemmPlan p{};
  if (big_plan(a, p)) return big_launch(a, p, st);
  int ntiles;
  if (a.epi == TG_GEGLU) {
    MLCV_REQUIRE(a.F % 64 == 0, "GeGLU tile GEMM needs mlp_dim % 64 == 0");
    ntiles = a.F / 64;
  } else {
    ntiles = (a.N + BN - 1) / BN;
  }
  const int mtiles = (a.M + BM - 1) / BM;
  const int ngroups = (ntiles + NXCD - 1) / NXCD;
  const unsigned blocks = (unsigned)(mtiles * ngroups * NXCD);
  tile_gemm_kernel<<<blocks, 256, 0, st>>>(a, mtiles, ntiles);
  MLCV_HIP(hipGetLastError());
  return 0;
}

bool tg_plan_k32(const TgArgs& a) {
  GemmPlan p{};
  return a.K % 8 == 0 && a.lda % 8 == 0 && a.ldb % 8 == 0 && big_plan(a, p) && p.bm == 256 &&
         (p.bn == 256 || a.epi == TG_GEGLU);
}

int wtile_shuffle_launch(const _Float16* w, _Float16* wt, int rows, int K, hipStream_t st) {
  MLCV_REQUIRE(w && wt && rows > 0 && rows % 16 == 0 && K > 0 && K % 32 == 0, "tile-major copy: shape");
  const long n8 = (long)rows * K / 8;
  wtile_shuffle_kernel<<<(unsigned)((n8 + 255) / 256), 256, 0, st>>>(w, wt, K, n8);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
