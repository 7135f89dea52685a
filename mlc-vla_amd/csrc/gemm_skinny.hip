// Skinny GEMM for the suffix path (M = action horizon <= 64 per block): HBM-bound
// weight streaming into MFMA 16x16x32 f16, with the adaRMS prologue and the
// residual / GeGLU / bias / SiLU / Euler epilogues fused, and q4f16_1 weights
// dequantized in registers.
//
// Mapping: D[n][m] = sum_k W[n][k] * X[m][k]: the A operand is a 16-row slab of W
// (lane l streams 32 contiguous k of row l%16 per 128-k chunk, so one wave reads
// 16 rows x 256 contiguous bytes), the B operand is X^T read from LDS with the
// same k permutation.  A workgroup (4 waves) owns 64 consecutive output rows
// (for GeGLU: 32 gate rows + the matching 32 up rows) and one K slice; K slices
// are reduced by the last-arriving workgroup of a tile in a fixed order.
#include "kernels.h"

namespace mlcv {

namespace {
constexpr int KC = 128;           // k per chunk (32 per lane group)
constexpr int MB = 64;            // m rows per block
constexpr int XLD = KC + 8;       // LDS row stride of the X chunk (halfs)
constexpr int TLD = 64 + 4;       // LDS row stride of the fp32 result tile

// 8 nibbles of a word -> fp16 (q - 7) * s, ordered [n0,n4,n1,n5,n2,n6,n3,n7].
__device__ __forceinline__ h8 dequant_word(uint32_t word, _Float16 s) {
  h8 r;
  const h2 bias = {(_Float16)1031.0f, (_Float16)1031.0f};
  const h2 sc = {s, s};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t bits = ((word >> (4 * p)) & 0x000F000Fu) | 0x64006400u;  // 1024 + q in each half
    h2 v = __builtin_bit_cast(h2, bits);
    v = (v - bias) * sc;                                                // exact, then one RNE
    r[2 * p] = v[0];
    r[2 * p + 1] = v[1];
  }
  return r;
}

__device__ __forceinline__ h8 perm8(h8 v) {
  h8 r;
  r[0] = v[0]; r[1] = v[4]; r[2] = v[1]; r[3] = v[5];
  r[4] = v[2]; r[5] = v[6]; r[6] = v[3]; r[7] = v[7];
  return r;
}

template <bool Q4>
struct WFrag {
  h8 v[4];
};

template <bool Q4>
__device__ __forceinline__ void load_wfrag(WFrag<Q4>& f, const SkSeg& seg, int row, bool row_ok, int k,
                                           int kend, int K) {
  if (!row_ok || k >= kend) {
#pragma unroll
    for (int j = 0; j < 4; ++j) f.v[j] = (h8){0, 0, 0, 0, 0, 0, 0, 0};
    return;
  }
  if constexpr (!Q4) {
    const h8* p = reinterpret_cast<const h8*>(seg.w + (size_t)row * K + k);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.v[j] = p[j];
  } else {
    const u4 words = *reinterpret_cast<const u4*>(seg.qw + (size_t)row * (K / 8) + k / 8);
    const _Float16 s = seg.qs[(size_t)row * (K / 32) + k / 32];
#pragma unroll
    for (int j = 0; j < 4; ++j) f.v[j] = dequant_word(words[j], s);
  }
}

template <bool Q4, bool NORM>
__global__ __launch_bounds__(256) void skinny_kernel(SkOp op) {
  __shared__ __attribute__((aligned(16))) _Float16 xs[MB * XLD];
  __shared__ __attribute__((aligned(16))) float tile[MB * TLD];
  __shared__ float denom[MB];
  __shared__ int is_last;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int tile_id = blockIdx.x, s = blockIdx.y, mb = blockIdx.z;
  const int m0 = mb * MB;
  const int mrows = min(MB, op.M - m0);
  const int MT = (mrows + 15) >> 4;

  int si = 0;
  while (si + 1 < op.nseg && op.segs[si + 1].tile0 <= tile_id) ++si;
  const SkSeg seg = op.segs[si];
  const int lt = tile_id - seg.tile0;
  const bool geglu = op.epi == EPI_GEGLU;
  const int row = geglu ? ((w < 2) ? (32 * lt + 16 * w + r16) : (op.geglu_F + 32 * lt + 16 * (w - 2) + r16))
                        : (64 * lt + 16 * w + r16);
  const bool row_ok = geglu ? true : (row < seg.n);

  const int K = op.K;
  const int kbeg = s * op.kper;
  const int kend = min(K, kbeg + op.kper);

  if constexpr (NORM) {
    for (int m = w; m < mrows; m += 4) {
      const _Float16* xr = op.x + (size_t)(m0 + m) * op.ldx;
      float ss = 0.f;
      for (int k = lane * 8; k < K; k += 512) {
        h8 v = *reinterpret_cast<const h8*>(xr + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float f = h2f(v[e]);
          ss += f * f;
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) denom[m] = sqrtf(ss / (float)K + op.eps);
    }
    __syncthreads();
  }

  f4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = (f4){0.f, 0.f, 0.f, 0.f};

  WFrag<Q4> wcur, wnext;
  load_wfrag<Q4>(wcur, seg, row, row_ok, kbeg + 32 * g, kend, K);

  for (int kc = kbeg; kc < kend; kc += KC) {
    // stage the X chunk (64 rows x 128 k) into LDS, normalizing on the fly
    {
      const int m = tid >> 2, kk = (tid & 3) * 32;
      const int kg = kc + kk;
      h8 v[4];
      if (m < mrows && kg < kend) {
        const _Float16* xr = op.x + (size_t)(m0 + m) * op.ldx + kg;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = reinterpret_cast<const h8*>(xr)[q];
        if constexpr (NORM) {
          const float dn = denom[m];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const h8 sc = *reinterpret_cast<const h8*>(op.scale + kg + 8 * q);
            const h8 sh = *reinterpret_cast<const h8*>(op.shift + kg + 8 * q);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              float nrm = h2f(v[q][e]) / dn;
              v[q][e] = f2h(nrm * (1.0f + h2f(sc[e])) + h2f(sh[e]));
            }
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (h8){0, 0, 0, 0, 0, 0, 0, 0};
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        h8 o = Q4 ? perm8(v[q]) : v[q];
        *reinterpret_cast<h8*>(&xs[m * XLD + kk + 8 * q]) = o;
      }
    }
    const int knext = kc + KC;
    if (knext < kend) load_wfrag<Q4>(wnext, seg, row, row_ok, knext + 32 * g, kend, K);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if (mt < MT) {
          const h8 b = *reinterpret_cast<const h8*>(&xs[(mt * 16 + r16) * XLD + 32 * g + 8 * j]);
          acc[mt] = mfma16x16x32(wcur.v[j], b, acc[mt]);
        }
      }
    }
    __syncthreads();
    wcur = wnext;
  }

  // ---- result tile: tile[m][n_local] -------------------------------------
  if (gridDim.y == 1) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      if (mt < MT) *reinterpret_cast<f4*>(&tile[(mt * 16 + r16) * TLD + 16 * w + 4 * g]) = acc[mt];
    __syncthreads();
  } else {
    const int cidx = tile_id * gridDim.z + mb;
    float* wsp = op.ws + ((size_t)cidx * gridDim.y + s) * (MB * 64);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      if (mt < MT) *reinterpret_cast<f4*>(&wsp[(mt * 16 + r16) * 64 + 16 * w + 4 * g]) = acc[mt];
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      unsigned prev = atomicAdd(&op.counters[cidx], 1u);
      is_last = (prev == gridDim.y - 1);
      if (is_last) __threadfence();
    }
    __syncthreads();
    if (!is_last) return;
    const float* base = op.ws + (size_t)cidx * gridDim.y * (MB * 64);
    for (int idx = tid; idx < mrows * 64; idx += 256) {
      float sum = 0.f;
      for (int sp = 0; sp < (int)gridDim.y; ++sp) sum += base[(size_t)sp * (MB * 64) + idx];
      tile[(idx >> 6) * TLD + (idx & 63)] = sum;
    }
    if (tid == 0) op.counters[cidx] = 0u;
    __syncthreads();
  }

  // ---- epilogue -------------------------------------------------------------
  const int epi = op.epi;
  for (int idx = tid; idx < mrows * 64; idx += 256) {
    const int m = idx >> 6, nl = idx & 63;
    const float a = tile[m * TLD + nl];
    const size_t mo = (size_t)(m0 + m) * seg.ldo;
    if (epi == EPI_GEGLU) {
      if (nl >= 32) continue;
      const int j = 32 * lt + nl;
      const _Float16 gv = f2h(a);
      const _Float16 uv = f2h(tile[m * TLD + nl + 32]);
      const _Float16 gg = f2h(gelu_tanh(h2f(gv)));
      reinterpret_cast<_Float16*>(seg.out)[mo + j] = hmul(gg, uv);
      continue;
    }
    const int n = 64 * lt + nl;
    if (n >= seg.n) continue;
    _Float16 y = f2h(a);
    if (epi == EPI_GATED_RES) {
      _Float16* xo = reinterpret_cast<_Float16*>(seg.out) + mo + n;
      *xo = hadd(*xo, hmul(y, op.gate[n]));
      continue;
    }
    if (seg.bias) y = hadd(y, seg.bias[n]);
    if (epi == EPI_STORE) {
      reinterpret_cast<_Float16*>(seg.out)[mo + n] = y;
    } else if (epi == EPI_STORE_SILU) {
      reinterpret_cast<_Float16*>(seg.out)[mo + n] = f2h(silu(h2f(y)));
    } else if (epi == EPI_VOUT) {
      reinterpret_cast<float*>(seg.out)[mo + n] = h2f(y);
    } else if (epi == EPI_EULER) {
      const float nx = euler_update(op.x32[mo + n], op.dt, h2f(y));
      op.x32[mo + n] = nx;
      op.x16[mo + n] = f2h(nx);
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

}  // namespace

SkPlan sk_plan(int ntiles, int K, int mblocks) {
  // enough workgroups to cover the 256 CUs; each split keeps >= 128 of K
  const int chunks = (K + KC - 1) / KC;
  int want = (256 + ntiles * mblocks - 1) / (ntiles * mblocks);
  if (want < 1) want = 1;
  if (want > 16) want = 16;
  if (want > chunks) want = chunks;
  const int cps = (chunks + want - 1) / want;
  SkPlan p;
  p.kper = cps * KC;
  p.splitk = (chunks + cps - 1) / cps;
  return p;
}

size_t sk_ws_floats(int ntiles, int mblocks, const SkPlan& p) {
  return p.splitk > 1 ? (size_t)ntiles * mblocks * p.splitk * MB * 64 : 0;
}

int sk_launch(const SkOp& op, bool q4, hipStream_t st) {
  MLCV_REQUIRE(op.K % 32 == 0, "skinny GEMM needs K % 32 == 0");
  MLCV_REQUIRE(op.M >= 1, "skinny GEMM needs M >= 1");
  const int mblocks = (op.M + MB - 1) / MB;
  dim3 grid(op.ntiles, op.splitk, mblocks);
  const bool norm = op.scale != nullptr;
  if (q4) {
    if (norm) skinny_kernel<true, true><<<grid, 256, 0, st>>>(op);
    else skinny_kernel<true, false><<<grid, 256, 0, st>>>(op);
  } else {
    if (norm) skinny_kernel<false, true><<<grid, 256, 0, st>>>(op);
    else skinny_kernel<false, false><<<grid, 256, 0, st>>>(op);
  }
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

}  // namespace mlcv
