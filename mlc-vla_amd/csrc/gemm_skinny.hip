// Skinny GEMM for the suffix path (M = action horizon <= 64 per block): HBM-bound
// weight streaming into MFMA 16x16x32 f16, with the adaRMS prologue and the
// residual / GeGLU / bias / SiLU / Euler epilogues fused, and q4f16_1 weights
// dequantized in registers.
//
// Mapping: D[n][m] = sum_k W[n][k] * X[m][k]: the A operand is a 16-row slab of W
// (lane l holds 32 contiguous k of row l%16 per 128-k chunk, so one wave reads
// 16 rows x 256 contiguous bytes), the B operand is X^T read from LDS with the
// same k permutation.  A workgroup (4 waves) owns 64 consecutive output rows
// (for GeGLU: 32 gate rows + the matching 32 up rows) and one K slice, taken in
// rounds of 512; K slices are reduced by the last-arriving workgroup of a tile in
// a fixed order.
//
// Latency structure (each kernel moves only 4-17 MB, so one HBM round trip is a
// large part of its time): every memory phase is one batch of independent loads --
// all W chunks of a round, then the X slice, then (split-K) all partials, then the
// epilogue's operands -- never a loop of dependent loads.
//
// Row statistics of the adaRMS prologue are not recomputed from x: every epilogue
// that writes the residual stream x also writes, per 64-column tile, the partial
// sum of squares of each row (``rowss_out``); the consuming GEMM sums those partials
// in tile order (``rowss_in``).
#include "kernels.h"

namespace mlcv {

namespace {
constexpr int KC = 128;           // k per chunk (32 per lane group)
constexpr int RK = 4 * KC;        // k per round (all of it loaded at once)
constexpr int MB = 64;            // m rows per block
constexpr int XLD = RK + 8;       // LDS row stride of the X slice (halfs)
constexpr int TLD = 64 + 4;       // LDS row stride of the fp32 result tile (aliases the X slice)
constexpr int MAX_SPLIT = 16;

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

// Weights of one 128-k chunk at kc for this lane (row `row`, lane group g):
//   fp16: k-step j holds k = kc + 32j + 8g .. +7 (one load instruction covers 64
//         contiguous bytes of each of the wave's 16 rows); a k-step at or past kend is 0.
//   q4:   the 32 nibbles at kc + 32g .. +31 (16 B) and their group scale; the k-step j
//         takes dequantized elements 8j..8j+7 in the order [n0,n4,n1,n5,n2,n6,n3,n7].
// kend is a multiple of 32, so every 32-k step is either fully valid or fully invalid.
template <bool Q4>
__device__ __forceinline__ void load_wraw(WRaw<Q4>& f, const SkSeg& seg, int row, bool row_ok, int kc, int g,
                                          int kend, int K) {
  if constexpr (!Q4) {
    const _Float16* p = seg.w + (size_t)row * K + kc + 8 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      f.v[j] = (row_ok && kc + 32 * j < kend) ? *reinterpret_cast<const h8*>(p + 32 * j)
                                              : (h8){0, 0, 0, 0, 0, 0, 0, 0};
  } else {
    const int k = kc + 32 * g;
    if (!(row_ok && k < kend)) {
      f.words = (u4){0x77777777u, 0x77777777u, 0x77777777u, 0x77777777u};  // q = 7 -> 0
      f.s = (_Float16)0.0f;
      return;
    }
    f.words = *reinterpret_cast<const u4*>(seg.qw + (size_t)row * (K / 8) + k / 8);
    f.s = seg.qs[(size_t)row * (K / 32) + k / 32];
  }
}

template <bool Q4>
__device__ __forceinline__ h8 wfrag(const WRaw<Q4>& f, int j) {
  if constexpr (!Q4) return f.v[j];
  else return dequant_word(f.words[j], f.s);
}

__device__ __forceinline__ void load16h(const _Float16* p, float out[16]) {
  const h8 a = reinterpret_cast<const h8*>(p)[0];
  const h8 b = reinterpret_cast<const h8*>(p)[1];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    out[e] = h2f(a[e]);
    out[8 + e] = h2f(b[e]);
  }
}

template <bool Q4, bool NORM>
__global__ __launch_bounds__(256) void skinny_kernel(SkOp op) {
  __shared__ __attribute__((aligned(16))) _Float16 xs[MB * XLD];
  __shared__ float denom[MB];  // 1 / sqrt(mean(x^2) + eps) per row
  __shared__ int is_last;
  float* tile = reinterpret_cast<float*>(xs);  // result tile [m][n_local], reuses the X slice

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int tile_id = blockIdx.x, s = blockIdx.y, mb = blockIdx.z;
  const int m0 = mb * MB;
  const int mrows = min(MB, op.M - m0);
  const int MT = (mrows + 15) >> 4;

  int si = 0;
  SkSeg seg;
  if (op.nseg <= 3) {  // kernel arguments: no dependent global load before the weight stream
    if (op.nseg > 1 && op.inl[1].tile0 <= tile_id) si = 1;
    if (op.nseg > 2 && op.inl[2].tile0 <= tile_id) si = 2;
    seg = op.inl[si];
  } else {
    while (si + 1 < op.nseg && op.segs[si + 1].tile0 <= tile_id) ++si;
    seg = op.segs[si];
  }
  const int lt = tile_id - seg.tile0;
  const bool geglu = op.epi == EPI_GEGLU;
  const int row = geglu ? ((w < 2) ? (32 * lt + 16 * w + r16) : (op.geglu_F + 32 * lt + 16 * (w - 2) + r16))
                        : (64 * lt + 16 * w + r16);
  const bool row_ok = geglu ? true : (row < seg.n);

  const int K = op.K;
  const int kbeg = s * op.kper;
  const int kend = min(K, kbeg + op.kper);

  // adaRMS row statistics: the producer's per-tile partial sums of squares, issued first
  // and summed in tile order once the X / W loads of the first round are in flight
  float rss[16];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      rss[i] = (tid < mrows && i < op.rowss_tiles) ? op.rowss_in[(size_t)i * op.rowss_ld + m0 + tid] : 0.f;
  }

  f4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = (f4){0.f, 0.f, 0.f, 0.f};

  for (int kr = kbeg; kr < kend; kr += RK) {
    // (1) the X slice [64 rows][512 k] first (L2-resident, and vmcnt retires in order):
    //     thread -> 8 consecutive k (tid % 64) of rows tid/64 + 4i
    const int kk = (tid & 63) * 8, mr = tid >> 6;
    const int kg = kr + kk;
    const bool kok = kg < kend;
    h8 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = mr + 4 * i;
      v[i] = (kok && m < mrows) ? *reinterpret_cast<const h8*>(op.x + (size_t)(m0 + m) * op.ldx + kg)
                                : (h8){0, 0, 0, 0, 0, 0, 0, 0};
    }
    h8 sc = (h8){0, 0, 0, 0, 0, 0, 0, 0}, sh = sc;
    if constexpr (NORM) {
      if (kok) {
        sc = *reinterpret_cast<const h8*>(op.scale + kg);
        sh = *reinterpret_cast<const h8*>(op.shift + kg);
      }
    }
    // (2) then every weight chunk of this round
    WRaw<Q4> wr[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kc = kr + c * KC;
      load_wraw<Q4>(wr[c], seg, row, row_ok, kc, g, kend, K);
    }
    if (NORM && kr == kbeg) {
      if (tid < mrows) {
        float ssum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) ssum += rss[i];
        for (int grp = 16; grp < op.rowss_tiles; grp += 16)  // widths > 1024 only
          for (int i = grp; i < min(grp + 16, op.rowss_tiles); ++i) ssum += op.rowss_in[(size_t)i * op.rowss_ld + m0 + tid];
        denom[tid] = 1.0f / sqrtf(ssum / (float)K + op.eps);  // reciprocal of the rms
      }
      __syncthreads();
    }
    // (3) normalize the X slice into LDS while the weights are in flight
    {
      if constexpr (NORM) {
        float sc1[8], shf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          sc1[e] = 1.0f + h2f(sc[e]);
          shf[e] = h2f(sh[e]);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int m = mr + 4 * i;
          const float rinv = m < mrows ? denom[m] : 1.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float nrm = h2f(v[i][e]) * rinv;
            v[i][e] = (m < mrows && kok) ? f2h(nrm * sc1[e] + shf[e]) : (_Float16)0.0f;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const h8 o = Q4 ? perm8(v[i]) : v[i];
        *reinterpret_cast<h8*>(&xs[(mr + 4 * i) * XLD + kk]) = o;
      }
    }
    __syncthreads();
    // (4) MFMA over the round
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (kr + c * KC < kend) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const h8 a = wfrag<Q4>(wr[c], j);
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            if (mt < MT) {
              const int ko = Q4 ? 32 * g + 8 * j : 32 * j + 8 * g;
              const h8 b = *reinterpret_cast<const h8*>(&xs[(mt * 16 + r16) * XLD + c * KC + ko]);
              acc[mt] = mfma16x16x32(a, b, acc[mt]);
            }
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- result tile in LDS: tile[m][n_local] ---------------------------------
  if (gridDim.y == 1) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      if (mt < MT) *reinterpret_cast<f4*>(&tile[(mt * 16 + r16) * TLD + 16 * w + 4 * g]) = acc[mt];
    __syncthreads();
  } else {
    // partials through the coherent memory side, reduced by the last workgroup of the tile
    const int cidx = tile_id * gridDim.z + mb;
    float* wsp = op.ws + ((size_t)cidx * gridDim.y + s) * (MB * 64);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int mm = mt * 16 + r16;
      if (mt < MT && mm < mrows)
#pragma unroll
        for (int i = 0; i < 4; ++i) store_coherent(&wsp[mm * 64 + 16 * w + 4 * g + i], acc[mt][i]);
    }
    wait_all_memory();
    __syncthreads();
    if (tid == 0) is_last = counter_add(&op.counters[cidx], 1u) == gridDim.y - 1;
    __syncthreads();
    if (!is_last) return;
    // every other split's partial has been written through before its counter add;
    // drop any stale cached copies, then read them with plain vector loads
    if (w == 0) acquire_agent();
    __syncthreads();
    const int mm = tid >> 2, cc = (tid & 3) * 16;
    if (mm < mrows) {
      const float* base = op.ws + (size_t)cidx * gridDim.y * (MB * 64) + mm * 64 + cc;
      f4 sum[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sum[i] = (f4){0.f, 0.f, 0.f, 0.f};
      const int S = gridDim.y;
#pragma unroll
      for (int grp = 0; grp < MAX_SPLIT; grp += 8) {
        if (grp < S) {
          f4 part[8][4];
#pragma unroll
          for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              part[q][i] = (grp + q < S) ? reinterpret_cast<const f4*>(base + (size_t)(grp + q) * (MB * 64))[i]
                                         : (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] += part[q][i];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<f4*>(&tile[mm * TLD + cc + 4 * i]) = sum[i];
    }
    if (tid == 0) counter_reset(&op.counters[cidx]);
    __syncthreads();
  }

  // ---- epilogue: thread -> row m, 16 consecutive output columns ----------------
  const int m = tid >> 2, c0 = (tid & 3) * 16;
  const int epi = op.epi;
  const bool mok = m < mrows;
  float a[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = mok ? tile[m * TLD + c0 + i] : 0.f;
  const size_t mo = (size_t)(m0 + m) * seg.ldo;
  if (epi == EPI_GEGLU) {
    if (mok && c0 < 32) {
      h8 o[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const _Float16 gv = f2h(a[i]);
        const _Float16 uv = f2h(tile[m * TLD + 32 + c0 + i]);
        o[i >> 3][i & 7] = hmul(f2h(gelu_tanh(h2f(gv))), uv);
      }
      h8* dst = reinterpret_cast<h8*>(reinterpret_cast<_Float16*>(seg.out) + mo + 32 * lt + c0);
      dst[0] = o[0];
      dst[1] = o[1];
    }
    return;
  }
  const int n0 = 64 * lt + c0;
  const bool full = mok && n0 + 16 <= seg.n;
  float ss = 0.f;  // row sum of squares of the new x over these columns
  if (epi == EPI_GATED_RES) {
    if (full) {
      _Float16* xo = reinterpret_cast<_Float16*>(seg.out) + mo + n0;
      float xv[16], gv[16];
      load16h(xo, xv);
      load16h(op.gate + n0, gv);
      h8 o[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const _Float16 r = hadd(f2h(xv[i]), hmul(f2h(a[i]), f2h(gv[i])));
        o[i >> 3][i & 7] = r;
        ss += h2f(r) * h2f(r);
      }
      reinterpret_cast<h8*>(xo)[0] = o[0];
      reinterpret_cast<h8*>(xo)[1] = o[1];
    } else if (mok) {
      for (int i = 0; i < 16 && n0 + i < seg.n; ++i) {
        _Float16* xo = reinterpret_cast<_Float16*>(seg.out) + mo + n0 + i;
        const _Float16 r = hadd(*xo, hmul(f2h(a[i]), op.gate[n0 + i]));
        *xo = r;
        ss += h2f(r) * h2f(r);
      }
    }
  } else {
    float bv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) bv[i] = 0.f;
    if (seg.bias) {
      if (full) {
        load16h(seg.bias + n0, bv);
      } else if (mok) {
        for (int i = 0; i < 16 && n0 + i < seg.n; ++i) bv[i] = h2f(seg.bias[n0 + i]);
      }
    }
    _Float16 y[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      y[i] = f2h(a[i]);
      if (seg.bias) y[i] = hadd(y[i], f2h(bv[i]));
      if (epi == EPI_STORE_SILU) y[i] = f2h(silu(h2f(y[i])));
    }
    if (epi == EPI_STORE || epi == EPI_STORE_SILU) {
      _Float16* o = reinterpret_cast<_Float16*>(seg.out) + mo + n0;
      if (full) {
        h8 v0, v1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          v0[i] = y[i];
          v1[i] = y[8 + i];
        }
        reinterpret_cast<h8*>(o)[0] = v0;
        reinterpret_cast<h8*>(o)[1] = v1;
      } else if (mok) {
        for (int i = 0; i < 16 && n0 + i < seg.n; ++i) o[i] = y[i];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (mok && n0 + i < seg.n) ss += h2f(y[i]) * h2f(y[i]);
    } else if (epi == EPI_VOUT) {
      if (mok)
        for (int i = 0; i < 16 && n0 + i < seg.n; ++i) reinterpret_cast<float*>(seg.out)[mo + n0 + i] = h2f(y[i]);
    } else if (epi == EPI_EULER) {
      if (mok)
        for (int i = 0; i < 16 && n0 + i < seg.n; ++i) {
          const float nx = euler_update(op.x32[mo + n0 + i], op.dt, h2f(y[i]));
          op.x32[mo + n0 + i] = nx;
          op.x16[mo + n0 + i] = f2h(nx);
        }
    }
  }
  if (op.rowss_out) {
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    if ((tid & 3) == 0 && mok) op.rowss_out[(size_t)lt * op.rowss_ld + m0 + m] = ss;
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
  // one wave of workgroups (<= 256, one per CU); each split keeps >= 128 of K; at most 8 splits
  const int chunks = (K + KC - 1) / KC;
  const int blocks = ntiles * mblocks;
  int want = (256 + blocks - 1) / blocks;
  if (want < 1) want = 1;
  if (want > 8) want = 8;
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
  MLCV_REQUIRE(op.splitk >= 1 && op.splitk <= MAX_SPLIT, "skinny GEMM split count");
  MLCV_REQUIRE(op.scale == nullptr || (op.rowss_in && op.rowss_tiles >= 1),
               "adaRMS prologue needs the producer's row statistics");
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
