// SigLIP vision tower + PaliGemma multi-modal projector (siglip.py:20-120), the
// `embed_image` function (pi0_model.py:97-99): one channels-last image [S][S][C] in fp16
// -> [num_patches][projection_dim] fp16.
//
// The linears run on the tile GEMMs (fp32 accumulation, one fp16 rounding), followed by
// an elementwise pass that adds the bias in fp16 and applies GELU or the residual add.
// LayerNorm keeps its statistics in fp32 (siglip.py:20-35).  The attention follows the
// reference's cast points (siglip.py:58-70) on the MFMA attention kernel of the step: keys
// and q at fp32-level precision (q * scale stays fp32, where the reference rounds it to
// fp16), fp32 logits and softmax, fp16 probabilities, P.V accumulated in fp32.  head_dim 72
// runs padded with zeros to 128 (no logit or output changes).
#include "kernels.h"

#include <algorithm>
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
  if ((n & 7) == 0 && (ldy & 7) == 0 && (ldx & 7) == 0 &&
      ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(x) |
        reinterpret_cast<uintptr_t>(pos)) & 15) == 0) {
    // 16-byte pieces, the same arithmetic per element
    for (int c = 8 * threadIdx.x; c < n; c += 8 * blockDim.x) {
      const h8 yv = *reinterpret_cast<const h8*>(y + (size_t)m * ldy + c), bv = *reinterpret_cast<const h8*>(b + c);
      h8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = hadd(yv[e], bv[e]);
        if (mode == VE_BIAS_GELU) v[e] = f2h(gelu_tanh(h2f(v[e])));
      }
      if (mode == VE_BIAS_RESIDUAL) {
        h8* xp = reinterpret_cast<h8*>(x + (size_t)m * ldx + c);
        const h8 xv = *xp;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = hadd(xv[e], v[e]);
        *xp = v;
        continue;
      }
      if (mode == VE_BIAS_POS) {
        const h8 pv = *reinterpret_cast<const h8*>(pos + (size_t)(m % npos) * n + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = hadd(v[e], pv[e]);
      }
      *reinterpret_cast<h8*>(y + (size_t)m * ldy + c) = v;
    }
    return;
  }
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

// q, k, v of every head from the fused projection [T][3 H hd] into the attention kernel's
// layouts at head_dim hp >= hd, zero past hd: q [T][H][hp], k and v [H][T][hp]
__global__ void vis_pad_qkv_kernel(const _Float16* __restrict__ qkv, int T, int H, int hd, int hp,
                                   _Float16* __restrict__ q, _Float16* __restrict__ k, _Float16* __restrict__ v) {
  const int t = blockIdx.x, h = blockIdx.y;
  const _Float16* src = qkv + (size_t)t * 3 * H * hd + (size_t)h * hd;
  for (int d = threadIdx.x; d < hp; d += blockDim.x) {
    const bool in = d < hd;
    const _Float16 z = (_Float16)0.f;
    q[((size_t)t * H + h) * hp + d] = in ? src[d] : z;
    k[((size_t)h * T + t) * hp + d] = in ? src[H * hd + d] : z;
    v[((size_t)h * T + t) * hp + d] = in ? src[2 * H * hd + d] : z;
  }
}

// attention output [T][H][hp] -> [T][H hd]
__global__ void vis_unpad_kernel(const _Float16* __restrict__ o, int H, int hd, int hp, _Float16* __restrict__ out) {
  const int t = blockIdx.x;
  for (int i = threadIdx.x; i < H * hd; i += blockDim.x)
    out[(size_t)t * H * hd + i] = o[((size_t)t * H + i / hd) * hp + i % hd];
}

int vis_head_pad(int hd) {
  for (int hp : {16, 32, 64, 128, 256})
    if (hd <= hp) return hp;
  return 0;
}

// key splits of the attention over T tokens of H heads: one round of workgroups on the CUs
void vis_attn_plan(int T, int H, int* nsplit, int* kps) {
  const int rb = (T + 63) / 64;
  const int target = std::max(1, std::max(device_cus(), 1) / (rb * H)) * rb;
  attn_plan(T, T, 0, target, nsplit, kps);
}

}  // namespace

size_t vision_ws_bytes(const VisionCfg& v) {
  const int np = (v.image_size / v.patch_size) * (v.image_size / v.patch_size);
  const size_t kp = ((size_t)v.patch_size * v.patch_size * v.num_channels + 7) / 8 * 8;
  const int hp = vis_head_pad(v.hidden / std::max(v.heads, 1));
  int nsplit = 1, kps = 32;
  vis_attn_plan(np, v.heads, &nsplit, &kps);
  const size_t halfs = (size_t)np * kp + (size_t)v.hidden * kp + (size_t)np * v.hidden * 4 +
                       (size_t)np * 3 * v.hidden + (size_t)np * v.inter + (size_t)4 * np * v.heads * hp;
  return halfs * 2 + attn_ws_floats(v.heads, np, hp, nsplit) * 4 + 512;
}

int embed_image_enqueue(const VisionCfg& v, const _Float16* const* prm, const _Float16* image, _Float16* out,
                        void* ws, size_t ws_bytes, float* gemm_ws, size_t gemm_ws_floats, unsigned* gemm_sync,
                        int gemm_sync_tiles, unsigned* gemm_err, hipStream_t st) {
  MLCV_REQUIRE(v.image_size % v.patch_size == 0 && v.hidden % v.heads == 0, "vision config");
  MLCV_REQUIRE(vis_head_pad(v.hidden / v.heads) > 0, "vision head_dim above 256");
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
  p += (size_t)np * v.inter;
  const int hp = vis_head_pad(hd);
  _Float16* qp = p;
  p += (size_t)np * v.heads * hp;
  _Float16* kpd = p;
  p += (size_t)np * v.heads * hp;
  _Float16* vpd = p;
  p += (size_t)np * v.heads * hp;
  _Float16* op = p;
  p += (size_t)np * v.heads * hp;
  float* aws = reinterpret_cast<float*>((reinterpret_cast<uintptr_t>(p) + 255) & ~uintptr_t(255));
  // the attention: the MFMA kernel of the step and prefill at head_dim hp, no RoPE, no mask
  AttnArgs at{};
  at.q = qp;
  at.q_ld = v.heads * hp;
  at.q_scale = (float)(1.0 / std::sqrt((double)hd));
  at.Tq = np;
  at.H = v.heads;
  at.KV = v.heads;
  at.hd = hp;
  at.kp = kpd;
  at.kp_f32 = 0;
  at.vp = vpd;
  at.Sp = np;
  at.out = op;
  at.out_ld = v.heads * hp;
  vis_attn_plan(np, v.heads, &at.nsplit, &at.kps);
  at.rows = np;
  at.rpad = ((np + 63) / 64) * 64;
  at.part_o = aws;
  at.part_ml = aws + (size_t)v.heads * at.nsplit * at.rpad * hp;

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
    g.err = gemm_err;
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
  for (int L = 0; L < v.layers; ++L) {
    const _Float16* const* lp = prm + 3 + 16 * L;  // q w,b  k w,b  v w,b  o w,b  fc1 w,b  fc2 w,b  ln1 w,b  ln2 w,b
    layernorm_kernel<<<np, 256, 0, st>>>(x, lp[12], lp[13], H, v.eps, hn);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(gemm(hn, H, lp[0], lp[2], lp[4], H, 2 * H, H, qkv, 3 * H, np, 3 * H, H));
    for (int s = 0; s < 3; ++s) MLCV_TRY(epi(qkv + s * H, 3 * H, lp[1 + 2 * s], H, VE_BIAS, nullptr, nullptr));
    vis_pad_qkv_kernel<<<dim3(np, v.heads), 128, 0, st>>>(qkv, np, v.heads, hd, hp, qp, kpd, vpd);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(attn_launch(at, st));
    vis_unpad_kernel<<<np, 256, 0, st>>>(op, v.heads, hd, hp, ctx);
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
