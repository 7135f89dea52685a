// The float32 model (Pi0Config(dtype="float32"), the reference's default dtype,
// pi0_config.py:97): prefill, denoise_step_kv, denoise_loop_kv and the chunk computed in float32
// from end to end, for the small shapes the reference runs in float32 (its CPU dummy model, the
// 2-layer test model).  With dtype = float32 every cast point of the reference is the identity:
// linears are fp32 products with fp32 sums (gemma_dual.py: nn.Linear at the model dtype), RMSNorm
// and adaRMS normalise in fp32 (:60-88), RoPE rotates in fp32 (:47-57), attention takes fp32
// logits, softmax and probabilities (:97-122), GeGLU (:125-135) and the gated residual (:91-94)
// round after each op, and the Euler update is x + dt * v in fp32 (pi0_model.py:165-194).
//
// These kernels are generic and simple (one tiled FMA GEMM, one workgroup per row or per query
// row and head elsewhere): the float32 model is for parity at small shapes; the fp16 and q4f16_1
// models are the fast paths.  Elementwise kernels keep the reference's rounding order
// (floating-point contraction is off in this file; the GEMM's and the dot products' fmaf are
// explicit).
#include <cmath>
#include <memory>
#include <vector>

#include "../../include/mlcvla.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace mlcv {
namespace {

constexpr int F32_NT = 256;

// Y[m][n] = act(sum_k X[m][k] W[n][k] + b[n]) for row-major X (ldx) and W [N][K]: 64 x 64
// tiles of 256 threads (4 x 4 outputs each), k in steps of 16 through LDS, sums in k order.
// act: 0 none, 1 SiLU (x / (1 + exp(-x)))
__global__ __launch_bounds__(F32_NT) void f32_gemm_kernel(const float* __restrict__ X, int ldx,
                                                          const float* __restrict__ W, const float* __restrict__ b,
                                                          float* __restrict__ Y, int ldy, int M, int N, int K,
                                                          int act) {
  __shared__ float xs[16][64 + 4];
  __shared__ float ws[16][64 + 4];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = threadIdx.x + F32_NT * i, r = e >> 4, kk = e & 15;
      const int gk = k0 + kk;
      xs[kk][r] = (m0 + r < M && gk < K) ? X[(size_t)(m0 + r) * ldx + gk] : 0.f;
      ws[kk][r] = (n0 + r < N && gk < K) ? W[(size_t)(n0 + r) * K + gk] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk][ty * 4 + i];
        w[i] = ws[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], w[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= N) continue;
      float y = acc[i][j];
      if (b) y = y + b[n];
      if (act == 1) y = y / (1.0f + expf(-y));
      Y[(size_t)m * ldy + n] = y;
    }
  }
}

// sum over the workgroup (256 threads) of each thread's v
__device__ __forceinline__ float f32_block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  if (lane == 0) red[w] = v;
  __syncthreads();
  const float s = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return s;
}
__device__ __forceinline__ float f32_block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if (lane == 0) red[w] = v;
  __syncthreads();
  const float s = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return s;
}

// row r of x [rows][W]: xn = x / sqrt(mean(x^2) + eps), then xn * (1 + w) (Gemma RMSNorm,
// w non-null) or xn * (1 + scale) + shift (adaRMS, mod = [scale | shift | gate] of 3W)
__global__ __launch_bounds__(F32_NT) void f32_norm_kernel(const float* __restrict__ x, int W,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ mod, float eps,
                                                          float* __restrict__ out) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * W;
  float ss = 0.f;
  for (int i = threadIdx.x; i < W; i += F32_NT) ss += xr[i] * xr[i];
  const float var = f32_block_sum(ss, red) / (float)W;
  const float den = sqrtf(var + eps);
  float* o = out + (size_t)blockIdx.x * W;
  for (int i = threadIdx.x; i < W; i += F32_NT) {
    const float xn = xr[i] / den;
    o[i] = w ? xn * (1.0f + w[i]) : xn * (1.0f + mod[i]) + mod[W + i];
  }
}

// in place on columns [col0, col0 + heads * hd) of row t of buf (ld): the half-split rotation
// of each head by cos / sin [rows][hd / 2], then * scale
__global__ void f32_rope_kernel(float* buf, int ld, int col0, int heads, int hd, const float* __restrict__ cs,
                                const float* __restrict__ sn, float scale) {
  const int t = blockIdx.x, half = hd / 2;
  for (int e = threadIdx.x; e < heads * half; e += blockDim.x) {
    const int hh = e / half, i = e % half;
    float* p = buf + (size_t)t * ld + col0 + hh * hd;
    const float c = cs[(size_t)t * half + i], s = sn[(size_t)t * half + i];
    const float x1 = p[i], x2 = p[i + half];
    p[i] = (x1 * c - x2 * s) * scale;
    p[i + half] = (x2 * c + x1 * s) * scale;
  }
}

// the layer's cache slices keys / values [KV][P][hd] from k / v [P][KV * hd]
__global__ void f32_kv_write_kernel(const float* __restrict__ k, const float* __restrict__ v, int P, int KV, int hd,
                                    float* __restrict__ keys, float* __restrict__ values) {
  const size_t n = (size_t)P * KV * hd;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(e % hd), p = (int)((e / hd) % P), kh = (int)(e / ((size_t)hd * P));
    keys[e] = k[(size_t)p * KV * hd + kh * hd + d];
    values[e] = v[(size_t)p * KV * hd + kh * hd + d];
  }
}

// out[t][h hd + d] = sum_j p_j val_j[d], p = softmax over the keys j of (q_t,h . key_j + mask_j):
// keys [0, Sp) from the prefix cache kp / vp [KV][Sp][hd] with the additive mask, then keys
// [Sp, Sp + Ts) from the suffix rows ks / vs [Ts][s_ld] (mask 0).  Query head h reads kv head
// h / (H / KV).  One workgroup per (query row, head); logits in LDS.
__global__ __launch_bounds__(F32_NT) void f32_attn_kernel(const float* __restrict__ q, int q_ld, int H, int KV,
                                                          int hd, const float* __restrict__ kp,
                                                          const float* __restrict__ vp, int Sp,
                                                          const float* __restrict__ mask,
                                                          const float* __restrict__ ks,
                                                          const float* __restrict__ vs, int s_ld, int Ts,
                                                          float* __restrict__ out, int o_ld) {
  extern __shared__ float sm[];
  float* qs = sm;       // [hd]
  float* lg = sm + hd;  // [Sp + Ts]
  __shared__ float red[4];
  const int t = blockIdx.x, h = blockIdx.y, kvh = h / (H / KV), nk = Sp + Ts;
  for (int d = threadIdx.x; d < hd; d += F32_NT) qs[d] = q[(size_t)t * q_ld + h * hd + d];
  __syncthreads();
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < nk; j += F32_NT) {
    const float* kr = j < Sp ? kp + ((size_t)kvh * Sp + j) * hd : ks + (size_t)(j - Sp) * s_ld + kvh * hd;
    float s = 0.f;
    for (int d = 0; d < hd; ++d) s = fmaf(qs[d], kr[d], s);
    if (j < Sp && mask) s = s + mask[j];
    lg[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = f32_block_max(mx, red);
  float sum = 0.f;
  for (int j = threadIdx.x; j < nk; j += F32_NT) {
    const float e = expf(lg[j] - mx);
    lg[j] = e;
    sum += e;
  }
  sum = f32_block_sum(sum, red);
  for (int j = threadIdx.x; j < nk; j += F32_NT) lg[j] = lg[j] / sum;
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += F32_NT) {
    float acc = 0.f;
    for (int j = 0; j < Sp; ++j) acc = fmaf(lg[j], vp[((size_t)kvh * Sp + j) * hd + d], acc);
    for (int j = 0; j < Ts; ++j) acc = fmaf(lg[Sp + j], vs[(size_t)j * s_ld + kvh * hd + d], acc);
    out[(size_t)t * o_ld + h * hd + d] = acc;
  }
}

// h[t][i] = gelu_tanh(gu[t][i]) * gu[t][F + i]
__global__ void f32_geglu_kernel(const float* __restrict__ gu, int F, int rows, float* __restrict__ hout) {
  const size_t n = (size_t)rows * F;
  const float c = 0.7978845608028654f;  // sqrt(2 / pi)
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
    const size_t t = e / F, i = e % F;
    const float x = gu[t * 2 * F + i], u = gu[t * 2 * F + F + i];
    const float g = 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
    hout[e] = g * u;
  }
}

// x[t][i] = x[t][i] + y[t][i] (gate null) or x[t][i] + y[t][i] * gate[i]
__global__ void f32_residual_kernel(float* __restrict__ x, const float* __restrict__ y,
                                    const float* __restrict__ gate, int W, int rows) {
  const size_t n = (size_t)rows * W;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
    const float yy = gate ? y[e] * gate[e % W] : y[e];
    x[e] = x[e] + yy;
  }
}

// x = x + dt * v
__global__ void f32_euler_kernel(float* __restrict__ x, const float* __restrict__ v, float dt, int n) {
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < n; e += gridDim.x * blockDim.x) x[e] = x[e] + dt * v[e];
}

int ew_grid(size_t n) { return (int)std::min<size_t>((n + 255) / 256, 4096); }

}  // namespace

struct F32Lin {
  const float* w = nullptr;
  const float* b = nullptr;
  int N = 0, K = 0;
};
struct F32Layer {
  F32Lin q[2], k[2], v[2], o[2], gu[2], dn[2], mod_in, mod_post;
  const float* ln_in0 = nullptr;
  const float* ln_post0 = nullptr;
};

struct F32Model {
  int W0, F0, W1, F1, D, H, KV, HD, P, T, A, S;
  float eps;
  bool bound = false;
  std::vector<F32Layer> layers;
  F32Lin final_mod, ain, aout, tin, tout;
  std::vector<void*> owned;
  // prefill
  float *px, *pxn, *pq, *pk, *pv, *pattn, *po, *pgu, *ph, *pcos, *psin, *mask;
  // the chunk's own cache
  float *ckeys, *cvalues;
  // step
  float *x, *xn, *q, *k, *v, *attn, *o, *gu, *h, *cond, *tmp, *mods, *vout, *x32;
  float *scos, *ssin, *smask, *te, *xt;

  ~F32Model() {
    for (void* p : owned) (void)hipFree(p);
  }
  int alloc(float** p, size_t n) {
    MLCV_HIP(hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(n, 1) * sizeof(float)));
    owned.push_back(*p);
    MLCV_HIP(hipMemset(*p, 0, std::max<size_t>(n, 1) * sizeof(float)));
    return 0;
  }
};

namespace {

int gemm(const float* X, int ldx, const F32Lin& l, float* Y, int ldy, int M, int act, hipStream_t st,
         bool bias = true) {
  const dim3 grid((l.N + 63) / 64, (M + 63) / 64);
  f32_gemm_kernel<<<grid, F32_NT, 0, st>>>(X, ldx, l.w, bias ? l.b : nullptr, Y, ldy, M, l.N, l.K, act);
  MLCV_HIP(hipGetLastError());
  return 0;
}
int attn(const float* q, int q_ld, const F32Model& m, const float* kp, const float* vp, int Sp, const float* mask,
         const float* ks, const float* vs, int s_ld, int Ts, float* out, int rows, hipStream_t st) {
  const size_t lds = (size_t)(m.HD + Sp + Ts) * sizeof(float);
  MLCV_REQUIRE(lds <= 64 * 1024, "float32 attention: too many keys");
  f32_attn_kernel<<<dim3(rows, m.H), F32_NT, lds, st>>>(q, q_ld, m.H, m.KV, m.HD, kp, vp, Sp, mask, ks, vs, s_ld,
                                                        Ts, out, m.H * m.HD);
  MLCV_HIP(hipGetLastError());
  return 0;
}
int norm(const float* x, int W, const float* w, const float* mod, float eps, float* out, int rows, hipStream_t st) {
  f32_norm_kernel<<<rows, F32_NT, 0, st>>>(x, W, w, mod, eps, out);
  MLCV_HIP(hipGetLastError());
  return 0;
}
int residual(float* x, const float* y, const float* gate, int W, int rows, hipStream_t st) {
  f32_residual_kernel<<<ew_grid((size_t)rows * W), 256, 0, st>>>(x, y, gate, W, rows);
  MLCV_HIP(hipGetLastError());
  return 0;
}

// one velocity evaluation on x_t (the model's x) with the time embedding te (pi0_model.py:142-163)
int f32_step_on(F32Model& m, const float* keys, const float* values, const float* x_t, const float* te,
                const float* cs, const float* sn, const float* pmask, float* v_out, hipStream_t st) {
  const int T = m.T, W1 = m.W1, nq = m.H * m.HD, nkv = m.KV * m.HD, W3 = 3 * W1;
  const size_t kvs = (size_t)m.KV * m.P * m.HD;  // one layer's cache slice
  const float scale = 1.0f / std::sqrt((float)m.HD);
  MLCV_TRY(gemm(x_t, m.A, m.ain, m.x, W1, T, 0, st));
  MLCV_TRY(gemm(te, W1, m.tin, m.tmp, W1, 1, 1, st));
  MLCV_TRY(gemm(m.tmp, W1, m.tout, m.cond, W1, 1, 1, st));
  for (int L = 0; L < m.D; ++L) {
    MLCV_TRY(gemm(m.cond, W1, m.layers[L].mod_in, m.mods + (size_t)(2 * L) * W3, W3, 1, 0, st));
    MLCV_TRY(gemm(m.cond, W1, m.layers[L].mod_post, m.mods + (size_t)(2 * L + 1) * W3, W3, 1, 0, st));
  }
  MLCV_TRY(gemm(m.cond, W1, m.final_mod, m.mods + (size_t)(2 * m.D) * W3, W3, 1, 0, st));
  for (int L = 0; L < m.D; ++L) {
    const F32Layer& ly = m.layers[L];
    const float* mi = m.mods + (size_t)(2 * L) * W3;
    const float* mp = m.mods + (size_t)(2 * L + 1) * W3;
    MLCV_TRY(norm(m.x, W1, nullptr, mi, m.eps, m.xn, T, st));
    MLCV_TRY(gemm(m.xn, W1, ly.q[1], m.q, nq, T, 0, st, false));
    MLCV_TRY(gemm(m.xn, W1, ly.k[1], m.k, nkv, T, 0, st, false));
    MLCV_TRY(gemm(m.xn, W1, ly.v[1], m.v, nkv, T, 0, st, false));
    f32_rope_kernel<<<T, 256, 0, st>>>(m.q, nq, 0, m.H, m.HD, cs, sn, scale);
    f32_rope_kernel<<<T, 256, 0, st>>>(m.k, nkv, 0, m.KV, m.HD, cs, sn, 1.0f);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(attn(m.q, nq, m, keys + L * kvs, values + L * kvs, m.P, pmask, m.k, m.v, nkv, T, m.attn, T, st));
    MLCV_TRY(gemm(m.attn, nq, ly.o[1], m.o, W1, T, 0, st, false));
    MLCV_TRY(residual(m.x, m.o, mi + 2 * W1, W1, T, st));
    MLCV_TRY(norm(m.x, W1, nullptr, mp, m.eps, m.xn, T, st));
    MLCV_TRY(gemm(m.xn, W1, ly.gu[1], m.gu, 2 * m.F1, T, 0, st, false));
    f32_geglu_kernel<<<ew_grid((size_t)T * m.F1), 256, 0, st>>>(m.gu, m.F1, T, m.h);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(gemm(m.h, m.F1, ly.dn[1], m.o, W1, T, 0, st, false));
    MLCV_TRY(residual(m.x, m.o, mp + 2 * W1, W1, T, st));
  }
  MLCV_TRY(norm(m.x, W1, nullptr, m.mods + (size_t)(2 * m.D) * W3, m.eps, m.xn, T, st));
  return gemm(m.xn, W1, m.aout, v_out, m.A, T, 0, st);
}

}  // namespace

int f32_create(const ::mlcv_config& cfg, F32Model** out) {
  auto m = std::make_unique<F32Model>();
  m->W0 = cfg.vlm_width;
  m->F0 = cfg.vlm_mlp;
  m->W1 = cfg.ae_width;
  m->F1 = cfg.ae_mlp;
  m->D = cfg.depth;
  m->H = cfg.num_heads;
  m->KV = cfg.num_kv_heads;
  m->HD = cfg.head_dim;
  m->P = cfg.prefix_len;
  m->T = cfg.suffix_len;
  m->A = cfg.action_dim;
  m->S = cfg.num_steps;
  m->eps = cfg.rms_norm_eps;
  MLCV_REQUIRE(m->HD % 2 == 0 && m->H % m->KV == 0, "float32 model: head_dim even, heads a multiple of kv heads");
  MLCV_REQUIRE((size_t)(m->HD + m->P + m->T) * 4 <= 64 * 1024, "float32 model: prefix_len + suffix_len too large");
  const size_t P = m->P, T = m->T, nq = (size_t)m->H * m->HD, nkv = (size_t)m->KV * m->HD;
  const size_t kv = (size_t)m->D * nkv * P;
  F32Model& r = *m;
  for (auto [p, n] : std::initializer_list<std::pair<float**, size_t>>{
           {&r.px, P * r.W0}, {&r.pxn, P * r.W0}, {&r.pq, P * nq}, {&r.pk, P * nkv}, {&r.pv, P * nkv},
           {&r.pattn, P * nq}, {&r.po, P * r.W0}, {&r.pgu, P * 2 * r.F0}, {&r.ph, P * r.F0},
           {&r.pcos, P * r.HD / 2}, {&r.psin, P * r.HD / 2}, {&r.mask, P}, {&r.ckeys, kv}, {&r.cvalues, kv},
           {&r.x, T * r.W1}, {&r.xn, T * r.W1}, {&r.q, T * nq}, {&r.k, T * nkv}, {&r.v, T * nkv},
           {&r.attn, T * nq}, {&r.o, T * r.W1}, {&r.gu, T * 2 * r.F1}, {&r.h, T * r.F1}, {&r.cond, r.W1},
           {&r.tmp, r.W1}, {&r.mods, (size_t)(2 * r.D + 1) * 3 * r.W1}, {&r.vout, T * r.A}, {&r.x32, T * r.A},
           {&r.scos, T * r.HD / 2}, {&r.ssin, T * r.HD / 2}, {&r.smask, P}, {&r.te, (size_t)r.S * r.W1},
           {&r.xt, T * r.A}})
    MLCV_TRY(r.alloc(p, n));
  // RoPE of the prefill's positions 0..P-1: radians = pos / theta^((2/hd) i) in float64
  std::vector<float> hc(P * r.HD / 2), hs(P * r.HD / 2);
  for (size_t p = 0; p < P; ++p)
    for (int i = 0; i < r.HD / 2; ++i) {
      const double rad = (double)p / std::pow((double)cfg.rope_theta, (2.0 / r.HD) * i);
      hc[p * (r.HD / 2) + i] = (float)std::cos(rad);
      hs[p * (r.HD / 2) + i] = (float)std::sin(rad);
    }
  MLCV_HIP(hipMemcpy(r.pcos, hc.data(), hc.size() * 4, hipMemcpyHostToDevice));
  MLCV_HIP(hipMemcpy(r.psin, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
  *out = m.release();
  return 0;
}

void f32_destroy(F32Model* m) { delete m; }

int f32_bind(F32Model& m, const void* const* ptrs, int count) {
  m.bound = false;
  int idx = 0;
  auto f = [&]() { return reinterpret_cast<const float*>(ptrs[idx++]); };
  auto lin = [&](F32Lin& l, int N, int K, bool bias) {
    l.N = N;
    l.K = K;
    l.w = f();
    l.b = bias ? f() : nullptr;
  };
  const int nq = m.H * m.HD, nkv = m.KV * m.HD;
  const int widths[2] = {m.W0, m.W1}, mlps[2] = {m.F0, m.F1};
  m.layers.assign(m.D, F32Layer{});
  for (int L = 0; L < m.D; ++L) {  // the order of named_params (pi0_model.py:81-88)
    F32Layer& ly = m.layers[L];
    for (int e = 0; e < 2; ++e) {
      lin(ly.q[e], nq, widths[e], false);
      lin(ly.k[e], nkv, widths[e], false);
      lin(ly.v[e], nkv, widths[e], false);
      lin(ly.o[e], widths[e], nq, false);
    }
    for (int e = 0; e < 2; ++e) {
      lin(ly.gu[e], 2 * mlps[e], widths[e], false);
      lin(ly.dn[e], widths[e], mlps[e], false);
    }
    ly.ln_in0 = f();
    lin(ly.mod_in, 3 * m.W1, m.W1, true);
    ly.ln_post0 = f();
    lin(ly.mod_post, 3 * m.W1, m.W1, true);
  }
  idx++;  // backbone.final_norm.0.weight (not read by the M1 functions)
  lin(m.final_mod, 3 * m.W1, m.W1, true);
  lin(m.ain, m.W1, m.A, true);
  lin(m.aout, m.A, m.W1, true);
  lin(m.tin, m.W1, m.W1, true);
  lin(m.tout, m.W1, m.W1, true);
  MLCV_REQUIRE(idx == count, "internal: float32 parameter walk mismatch");
  for (int i = 0; i < count; ++i) MLCV_REQUIRE(ptrs[i] != nullptr, "null parameter pointer");
  m.bound = true;
  return 0;
}

// prefill (pi0_model.py:128-140; prefill_e0 gemma_dual.py:334-341, attn_prefill_e0 :236-253)
int f32_prefill(F32Model& m, const void* prefix_embs, const float* prefix_mask, float* keys, void* values,
                hipStream_t st) {
  MLCV_REQUIRE(m.bound, "parameters not bound");
  const int P = m.P, W0 = m.W0, nq = m.H * m.HD, nkv = m.KV * m.HD;
  const size_t kvs = (size_t)m.KV * P * m.HD;
  float* vals = reinterpret_cast<float*>(values);
  const float scale = 1.0f / std::sqrt((float)m.HD);
  MLCV_HIP(hipMemcpyAsync(m.px, prefix_embs, (size_t)P * W0 * 4, hipMemcpyDeviceToDevice, st));
  MLCV_HIP(hipMemcpyAsync(m.mask, prefix_mask, (size_t)P * 4, hipMemcpyDeviceToDevice, st));
  for (int L = 0; L < m.D; ++L) {
    const F32Layer& ly = m.layers[L];
    MLCV_TRY(norm(m.px, W0, ly.ln_in0, nullptr, m.eps, m.pxn, P, st));
    MLCV_TRY(gemm(m.pxn, W0, ly.q[0], m.pq, nq, P, 0, st, false));
    MLCV_TRY(gemm(m.pxn, W0, ly.k[0], m.pk, nkv, P, 0, st, false));
    MLCV_TRY(gemm(m.pxn, W0, ly.v[0], m.pv, nkv, P, 0, st, false));
    f32_rope_kernel<<<P, 256, 0, st>>>(m.pq, nq, 0, m.H, m.HD, m.pcos, m.psin, scale);
    f32_rope_kernel<<<P, 256, 0, st>>>(m.pk, nkv, 0, m.KV, m.HD, m.pcos, m.psin, 1.0f);
    f32_kv_write_kernel<<<ew_grid(kvs), 256, 0, st>>>(m.pk, m.pv, P, m.KV, m.HD, keys + L * kvs, vals + L * kvs);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(attn(m.pq, nq, m, keys + L * kvs, vals + L * kvs, P, m.mask, nullptr, nullptr, 0, 0, m.pattn, P, st));
    MLCV_TRY(gemm(m.pattn, nq, ly.o[0], m.po, W0, P, 0, st, false));
    MLCV_TRY(residual(m.px, m.po, nullptr, W0, P, st));
    MLCV_TRY(norm(m.px, W0, ly.ln_post0, nullptr, m.eps, m.pxn, P, st));
    MLCV_TRY(gemm(m.pxn, W0, ly.gu[0], m.pgu, 2 * m.F0, P, 0, st, false));
    f32_geglu_kernel<<<ew_grid((size_t)P * m.F0), 256, 0, st>>>(m.pgu, m.F0, P, m.ph);
    MLCV_HIP(hipGetLastError());
    MLCV_TRY(gemm(m.ph, m.F0, ly.dn[0], m.po, W0, P, 0, st, false));
    MLCV_TRY(residual(m.px, m.po, nullptr, W0, P, st));
  }
  return 0;
}

int f32_step(F32Model& m, const float* keys, const void* values, const void* x_t, const void* time_emb,
             const float* cs, const float* sn, const float* prefix_mask, float* v_out, hipStream_t st) {
  MLCV_REQUIRE(m.bound, "parameters not bound");
  return f32_step_on(m, keys, reinterpret_cast<const float*>(values), reinterpret_cast<const float*>(x_t),
                     reinterpret_cast<const float*>(time_emb), cs, sn, prefix_mask, v_out, st);
}

// N Euler steps x <- x + (-1/N) v(x), x fed to each step as the model's x (pi0_model.py:165-194)
int f32_loop(F32Model& m, const float* keys, const void* values, const float* x0, const void* time_embs,
             const float* cs, const float* sn, const float* prefix_mask, float* x_out, hipStream_t st) {
  MLCV_REQUIRE(m.bound, "parameters not bound");
  const int n = m.T * m.A;
  const float dt = (float)(-1.0 / m.S);
  MLCV_HIP(hipMemcpyAsync(m.x32, x0, (size_t)n * 4, hipMemcpyDeviceToDevice, st));
  for (int i = 0; i < m.S; ++i) {
    MLCV_TRY(f32_step_on(m, keys, reinterpret_cast<const float*>(values), m.x32,
                         reinterpret_cast<const float*>(time_embs) + (size_t)i * m.W1, cs, sn, prefix_mask, m.vout,
                         st));
    f32_euler_kernel<<<ew_grid(n), 256, 0, st>>>(m.x32, m.vout, dt, n);
    MLCV_HIP(hipGetLastError());
  }
  MLCV_HIP(hipMemcpyAsync(x_out, m.x32, (size_t)n * 4, hipMemcpyDeviceToDevice, st));
  return 0;
}

int f32_chunk(F32Model& m, const void* prefix_embs, const float* prefix_mask, const float* x0, const void* time_embs,
              const float* cs, const float* sn, float* x_out, hipStream_t st) {
  MLCV_TRY(f32_prefill(m, prefix_embs, prefix_mask, m.ckeys, m.cvalues, st));
  return f32_loop(m, m.ckeys, m.cvalues, x0, time_embs, cs, sn, m.mask, x_out, st);
}

}  // namespace mlcv
