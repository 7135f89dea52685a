// SigLIP vision tower + PaliGemma multi-modal projector (siglip.py:20-120), the
// `embed_image` function (pi0_model.py:97-99): one channels-last image [S][S][C] in fp16
// -> [num_patches][projection_dim] fp16.
//
// The linears run on the tile GEMMs (fp32 accumulation, one fp16 rounding), followed by
// an elementwise pass that adds the bias in fp16 and applies GELU or the residual add.
// LayerNorm keeps its statistics in fp32 (siglip.py:20-35).  The attention follows the
// reference's cast points (siglip.py:58-70): q * scale in fp16, logits and softmax in fp32,
// probabilities rounded to fp16, P.V accumulated in fp32 and rounded to fp16.
#include "kernels.h"

#include <cmath>

namespace mlcv {

namespace {

// patches [np][kp]: row py * side + px, column (i * p + j) * C + c holds pixel
// (py * p + i, px * p + j, c) (siglip.py:97-107); columns past p * p * C are zero
__global__ void patchify_kernel(const _Float16* __restrict__ img, int size, int p, int C, int kp,
                                _Float16* __restrict__ out) {
  const int patch = blockIdx.x, side = size / p;
  const int py = patch / side, px = patch % side;
  for (int col = threadIdx.x; col < kp; col += blockDim.x) {
    _Float16 v = (_Float16)0.f;
    if (col < p * p * C) {
      const int c = col % C, j = (col / C) % p, i = col / (C * p);
      v = img[((size_t)(py * p + i) * size + (px * p + j)) * C + c];
    }
    out[(size_t)patch * kp + col] = v;
  }
}

// w [n][k] -> wp [n][kp], zero columns past k
__global__ void pad_cols_kernel(const _Float16* __restrict__ w, int k, int kp, _Float16* __restrict__ wp) {
  const int r = blockIdx.x;
  for (int c = threadIdx.x; c < kp; c += blockDim.x) wp[(size_t)r * kp + c] = c < k ? w[(size_t)r * k + c] : (_Float16)0.f;
}

enum VisEpi { VE_BIAS = 0, VE_BIAS_GELU = 1, VE_BIAS_RESIDUAL = 2, VE_BIAS_POS = 3 };

// y = fp16(y + b) on columns [0, n) of rows with stride ldy, then:
//   VE_BIAS_GELU      y = fp16(gelu_tanh(y))
//   VE_BIAS_RESIDUAL  x = fp16(x + y)            (x: the residual stream, stride ldx)
//   VE_BIAS_POS       y = fp16(y + pos[m % npos])  (position embedding, stride n)
__global__ void vis_epilogue_kernel(_Float16* __restrict__ y, int ldy, const _Float16* __restrict__ b, int n,
                                    int mode, _Float16* __restrict__ x, int ldx, const _Float16* __restrict__ pos,
                                    int npos) {
  const int m = blockIdx.x;
  for (int c = threadIdx.x; c < n; c += blockDim.x) {
    _Float16 v = hadd(y[(size_t)m * ldy + c], b[c]);
    if (mode == VE_BIAS_GELU) v = f2h(gelu_tanh(h2f(v)));
    if (mode == VE_BIAS_RESIDUAL) {
      x[(size_t)m * ldx + c] = hadd(x[(size_t)m * ldx + c], v);
      continue;
    }
    if (mode == VE_BIAS_POS) v = hadd(v, pos[(size_t)(m % npos) * n + c]);
    y[(size_t)m * ldy + c] = v;
  }
}

// LayerNorm of one row per block: mean, then variance about it, in fp32 (two passes over
// the row), out = fp16((x - mean) / sqrt(var + eps) * w + b) with w, b in fp32
__global__ __launch_bounds__(256) void layernorm_kernel(const _Float16* __restrict__ x, const _Float16* __restrict__ w,
                                                        const _Float16* __restrict__ b, int n, float eps,
                                                        _Float16* __restrict__ out) {
  __shared__ float red[4];
  __shared__ float stat[2];
  const int r = blockIdx.x, tid = threadIdx.x;
  const _Float16* xr = x + (size_t)r * n;
  float s = 0.f;
  for (int c = tid; c < n; c += 256) s += h2f(xr[c]);
  s = wave_sum(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) stat[0] = (red[0] + red[1] + red[2] + red[3]) / (float)n;
  __syncthreads();
  const float mean = stat[0];
  float q = 0.f;
  for (int c = tid; c < n; c += 256) {
    const float d = h2f(xr[c]) - mean;
    q += d * d;
  }
  q = wave_sum(q);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = q;
  __syncthreads();
  if (tid == 0) stat[1] = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
  __syncthreads();
  const float rstd = stat[1];
  for (int c = tid; c < n; c += 256)
    out[(size_t)r * n + c] = f2h((h2f(xr[c]) - mean) * rstd * h2f(w[c]) + h2f(b[c]));
}

constexpr int VA_ROWS = 64, VA_KEYS = 64, VA_LANES = 4;

// bidirectional attention of one head over T tokens: qkv [T][3 H hd] (q | k | v), out
// [T][H hd].  A block holds 64 query rows with 4 lanes per row (consecutive lanes of one
// wave), each lane taking every 4th key of the tiles that stream through LDS.  Pass 1 finds
// each row's max logit and exp sum (combined over the 4 lanes by shuffles), pass 2 forms the
// fp16 probabilities and accumulates P.V, summed over the 4 lanes at the end.
template <int HD>
__global__ __launch_bounds__(VA_ROWS* VA_LANES) void vis_attention_kernel(const _Float16* __restrict__ qkv, int T,
                                                                          int H, _Float16 qscale,
                                                                          _Float16* __restrict__ out) {
  constexpr int hd = HD;
  __shared__ float ks[VA_KEYS][HD];
  __shared__ _Float16 vs[VA_KEYS][HD];
  const int h = blockIdx.y, tid = threadIdx.x, kl = tid % VA_LANES;
  const int row = blockIdx.x * VA_ROWS + tid / VA_LANES;
  const int ld = 3 * H * hd;
  const bool ok = row < T;
  float q[HD], acc[HD];
#pragma unroll
  for (int d = 0; d < hd; ++d) {
    q[d] = h2f(hmul(qkv[(size_t)min(row, T - 1) * ld + h * hd + d], qscale));
    acc[d] = 0.f;
  }
  float mx = -INFINITY, sum = 0.f;
  for (int pass = 0; pass < 2; ++pass) {
    for (int k0 = 0; k0 < T; k0 += VA_KEYS) {
      const int nk = min(VA_KEYS, T - k0);
      __syncthreads();
      for (int i = tid; i < nk * hd; i += VA_ROWS * VA_LANES) {
        const int j = i / hd, d = i % hd;
        ks[j][d] = h2f(qkv[(size_t)(k0 + j) * ld + H * hd + h * hd + d]);
        vs[j][d] = qkv[(size_t)(k0 + j) * ld + 2 * H * hd + h * hd + d];
      }
      __syncthreads();
      for (int j = kl; j < nk; j += VA_LANES) {
        float l = 0.f;
#pragma unroll
        for (int d = 0; d < hd; ++d) l += q[d] * ks[j][d];
        if (pass == 0) {
          const float m2 = fmaxf(mx, l);
          sum = sum * expf(mx - m2) + expf(l - m2);
          mx = m2;
        } else {
          const float pr = h2f(f2h(expf(l - mx) / sum));
#pragma unroll
          for (int d = 0; d < hd; ++d) acc[d] += pr * h2f(vs[j][d]);
        }
      }
    }
    if (pass == 0) {  // the row's max and sum over its 4 lanes
#pragma unroll
      for (int o = 1; o < VA_LANES; o <<= 1) {
        const float m2 = __shfl_xor(mx, o), s2 = __shfl_xor(sum, o);
        const float m = fmaxf(mx, m2);
        sum = (mx == -INFINITY ? 0.f : sum * expf(mx - m)) + (m2 == -INFINITY ? 0.f : s2 * expf(m2 - m));
        mx = m;
      }
    }
  }
#pragma unroll
  for (int d = 0; d < hd; ++d) {
    acc[d] += __shfl_xor(acc[d], 1);
    acc[d] += __shfl_xor(acc[d], 2);
  }
  if (ok && kl == 0) {
#pragma unroll
    for (int d = 0; d < hd; ++d) out[(size_t)row * H * hd + h * hd + d] = f2h(acc[d]);
  }
}

}  // namespace

size_t vision_ws_bytes(const VisionCfg& v) {
  const size_t np = (size_t)(v.image_size / v.patch_size) * (v.image_size / v.patch_size);
  const size_t kp = ((size_t)v.patch_size * v.patch_size * v.num_channels + 7) / 8 * 8;
  const size_t halfs = np * kp + (size_t)v.hidden * kp + np * v.hidden * 4 + np * 3 * v.hidden + np * v.inter;
  return halfs * 2 + 256;
}

int embed_image_enqueue(const VisionCfg& v, const _Float16* const* prm, const _Float16* image, _Float16* out,
                        void* ws, size_t ws_bytes, float* gemm_ws, size_t gemm_ws_floats, unsigned* gemm_sync,
                        int gemm_sync_tiles, hipStream_t st) {
  MLCV_REQUIRE(v.image_size % v.patch_size == 0 && v.hidden % v.heads == 0, "vision config");
  const int hdv = v.hidden / v.heads;
  MLCV_REQUIRE(hdv == 16 || hdv == 32 || hdv == 64 || hdv == 72, "vision head_dim must be 16, 32, 64 or 72");
  MLCV_REQUIRE(v.hidden % 8 == 0 && v.inter % 8 == 0 && v.proj % 4 == 0, "vision widths must be multiples of 8");
  MLCV_REQUIRE(ws_bytes >= vision_ws_bytes(v), "vision workspace too small");
  const int side = v.image_size / v.patch_size, np = side * side, H = v.hidden, hd = H / v.heads;
  const int pdim = v.patch_size * v.patch_size * v.num_channels, kp = (pdim + 7) / 8 * 8;
  _Float16* p = reinterpret_cast<_Float16*>((reinterpret_cast<uintptr_t>(ws) + 255) & ~uintptr_t(255));
  _Float16* patches = p;
  p += (size_t)np * kp;
  _Float16* wpad = p;
  p += (size_t)H * kp;
  _Float16* x = p;
  p += (size_t)np * H;
  _Float16* hn = p;
  p += (size_t)np * H;
  _Float16* ctx = p;
  p += (size_t)np * H;
  _Float16* t = p;
  p += (size_t)np * H;
  _Float16* qkv = p;
  p += (size_t)np * 3 * H;
  _Float16* u = p;

  auto gemm = [&](const _Float16* a, int lda, const _Float16* b0, const _Float16* b1, const _Float16* b2, int n1,
                  int n2, int ldb, _Float16* c, int ldc, int M, int N, int K) {
    TgArgs g{};
    g.a = a;
    g.lda = lda;
    g.b0 = b0;
    g.b1 = b1;
    g.b2 = b2;
    g.n1 = n1;
    g.n2 = n2;
    g.ldb = ldb;
    g.c = c;
    g.ldc = ldc;
    g.M = M;
    g.N = N;
    g.K = K;
    g.epi = TG_STORE;
    g.ws = gemm_ws;
    g.ws_floats = gemm_ws_floats;
    g.sync = gemm_sync;
    g.sync_tiles = gemm_sync_tiles;
    return tg_launch(g, st);
  };
  auto epi = [&](_Float16* y, int ldy, const _Float16* b, int n, int mode, _Float16* xr, const _Float16* pos) {
    vis_epilogue_kernel<<<np, 256, 0, st>>>(y, ldy, b, n, mode, xr, H, pos, np);
    MLCV_HIP(hipGetLastError());
    return 0;
  };

  // patch embedding (+ bias) + position embedding
  patchify_kernel<<<np, 256, 0, st>>>(image, v.image_size, v.patch_size, v.num_channels, kp, patches);
  pad_cols_kernel<<<H, 256, 0, st>>>(prm[0], pdim, kp, wpad);
  MLCV_HIP(hipGetLastError());
  MLCV_TRY(gemm(patches, kp, wpad, wpad, wpad, H, H, kp, x, H, np, H, kp));
  MLCV_TRY(epi(x, H, prm[1], H, VE_BIAS_POS, nullptr, prm[2]));
  const _Float16 qscale = (_Float16)(1.0 / std::sqrt((double)hd));
  for (int L = 0; L < v.layers; ++L) {
    const _Float16* const* lp = prm + 3 + 16 * L;  // q w,b  k w,b  v w,b  o w,b  fc1 w,b  fc2 w,b  ln1 w,b  ln2 w,b
    layernorm_kernel<<<np, 256, 0, st>>>(x, lp[12], lp[13], H, v.eps, hn);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(gemm(hn, H, lp[0], lp[2], lp[4], H, 2 * H, H, qkv, 3 * H, np, 3 * H, H));
    for (int s = 0; s < 3; ++s) MLCV_TRY(epi(qkv + s * H, 3 * H, lp[1 + 2 * s], H, VE_BIAS, nullptr, nullptr));
    const dim3 ag((np + VA_ROWS - 1) / VA_ROWS, v.heads);
    constexpr int NT = VA_ROWS * VA_LANES;
    switch (hd) {
      case 16: vis_attention_kernel<16><<<ag, NT, 0, st>>>(qkv, np, v.heads, qscale, ctx); break;
      case 32: vis_attention_kernel<32><<<ag, NT, 0, st>>>(qkv, np, v.heads, qscale, ctx); break;
      case 64: vis_attention_kernel<64><<<ag, NT, 0, st>>>(qkv, np, v.heads, qscale, ctx); break;
      default: vis_attention_kernel<72><<<ag, NT, 0, st>>>(qkv, np, v.heads, qscale, ctx); break;
    }
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(gemm(ctx, H, lp[6], lp[6], lp[6], H, H, H, t, H, np, H, H));
    MLCV_TRY(epi(t, H, lp[7], H, VE_BIAS_RESIDUAL, x, nullptr));
    layernorm_kernel<<<np, 256, 0, st>>>(x, lp[14], lp[15], H, v.eps, hn);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(gemm(hn, H, lp[8], lp[8], lp[8], v.inter, v.inter, H, u, v.inter, np, v.inter, H));
    MLCV_TRY(epi(u, v.inter, lp[9], v.inter, VE_BIAS_GELU, nullptr, nullptr));
    MLCV_TRY(gemm(u, v.inter, lp[10], lp[10], lp[10], H, H, v.inter, t, H, np, H, v.inter));
    MLCV_TRY(epi(t, H, lp[11], H, VE_BIAS_RESIDUAL, x, nullptr));
  }
  const _Float16* const* tail = prm + 3 + 16 * v.layers;  // post LN w, b; projector w, b
  layernorm_kernel<<<np, 256, 0, st>>>(x, tail[0], tail[1], H, v.eps, hn);
  MLCV_HIP(hipGetLastError());
  MLCV_TRY(gemm(hn, H, tail[2], tail[2], tail[2], v.proj, v.proj, H, out, v.proj, np, v.proj, H));
  return epi(out, v.proj, tail[3], v.proj, VE_BIAS, nullptr, nullptr);
}

}  // namespace mlcv
