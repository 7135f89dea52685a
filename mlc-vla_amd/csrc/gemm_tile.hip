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

namespace mlcv {

namespace {
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;  // halfs per LDS row
constexpr int NXCD = 8;

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
        a.c[(size_t)m * a.ldc + j] = hmul(f2h(gelu_tanh(h2f(gv))), uv);
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

}  // namespace

int tg_launch(const TgArgs& a, hipStream_t st) {
  MLCV_REQUIRE(a.K % 8 == 0 && a.lda % 8 == 0 && a.ldb % 8 == 0, "tile GEMM needs 16-byte aligned rows");
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

}  // namespace mlcv
