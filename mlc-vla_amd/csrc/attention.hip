// Joint attention for the M1 path: the suffix queries (all heads of one KV head
// stacked into one row set, so the frozen prefix K/V is streamed once per row
// block) attend to [prefix K/V ; suffix K/V] with an additive prefix mask.
//
// Numerics follow the reference's cast points: q and k are roped in fp32, q is
// scaled after RoPE, logits are fp32 (QK^T on MFMA as hi*hi + hi*lo + lo*hi of an
// fp16 hi/lo split of both operands, ~2^-22 relative), softmax in fp32, the
// probabilities enter P.V as fp16 and P.V accumulates in fp32.  The softmax is the
// online (running max / running sum) form over key chunks and over key splits.
//
// MFMA mapping (16x16x32 f16): S^T[key][row] = K[key][:] . Q[row][:]  (A = K tile
// from LDS, B = Q^T held in registers), which leaves each lane with 4 consecutive
// keys of one query row -- exactly the B-operand layout of O^T[d][row] =
// V^T[d][key] . P^T[key][row], so P never leaves registers; V^T is staged in LDS.
#include "kernels.h"

namespace mlcv {

namespace {
constexpr int KCH = 32;    // keys per chunk
constexpr int ROWS = 64;   // query rows per workgroup (4 waves x 16)

template <int HD>
struct AttnSmem {
  static constexpr int KLD = HD + 8;        // halfs per K row
  static constexpr int VLD = KCH + 8;       // halfs per V^T row
  _Float16 kh[KCH * KLD];
  _Float16 kl[KCH * KLD];
  _Float16 vt[HD * VLD];
  float msk[KCH];
};

// rope for 8 consecutive dims [d0, d0+8) of one vector; pair = the dims at d0 +- half.
__device__ __forceinline__ void rope8(const _Float16* x, int d0, int half, const float* cs, const float* sn,
                                      float out[8]) {
  const bool first = d0 < half;
  const int dp = first ? d0 + half : d0 - half;
  const int dc = first ? d0 : d0 - half;
  const h8 a = *reinterpret_cast<const h8*>(x + d0);
  const h8 b = *reinterpret_cast<const h8*>(x + dp);
  const f4 c0 = *reinterpret_cast<const f4*>(cs + dc), c1 = *reinterpret_cast<const f4*>(cs + dc + 4);
  const f4 s0 = *reinterpret_cast<const f4*>(sn + dc), s1 = *reinterpret_cast<const f4*>(sn + dc + 4);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = e < 4 ? c0[e] : c1[e - 4], sv = e < 4 ? s0[e] : s1[e - 4];
    const float xa = h2f(a[e]), xb = h2f(b[e]);
    out[e] = first ? (xa * c - xb * sv) : (xa * c + xb * sv);
  }
}

// one key chunk of K (fp32, roped) and V (fp16) held in registers between the
// global loads and the LDS stores, so the next chunk's loads overlap this chunk's math
template <int HD>
struct KvRegs {
  static constexpr int NIT = (KCH * (HD / 8) + 255) / 256;
  float k[NIT][8];
  h8 v[NIT];
  float msk;
};

template <int HD>
__device__ __forceinline__ void kv_gload(KvRegs<HD>& r, const AttnArgs& a, int c0, int kend, int kvh, int tid) {
  constexpr int HALF = HD / 2;
  const float* kp32 = reinterpret_cast<const float*>(a.kp) + (size_t)kvh * a.Sp * HD;
  const _Float16* kp16 = reinterpret_cast<const _Float16*>(a.kp) + (size_t)kvh * a.Sp * HD;
  const _Float16* vpb = a.vp + (size_t)kvh * a.Sp * HD;
#pragma unroll
  for (int it = 0; it < KvRegs<HD>::NIT; ++it) {
    const int item = tid + 256 * it;
    const int jl = item / (HD / 8);
    const int d0 = (item % (HD / 8)) * 8;
    const int kj = c0 + jl;
    r.v[it] = (h8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) r.k[it][e] = 0.f;
    if (item >= KCH * (HD / 8) || kj >= kend) continue;
    if (kj < a.Sp) {
      if (a.kp_f32) {
        const f4 x0 = *reinterpret_cast<const f4*>(kp32 + (size_t)kj * HD + d0);
        const f4 x1 = *reinterpret_cast<const f4*>(kp32 + (size_t)kj * HD + d0 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r.k[it][e] = x0[e];
          r.k[it][e + 4] = x1[e];
        }
      } else {
        const h8 x = *reinterpret_cast<const h8*>(kp16 + (size_t)kj * HD + d0);
#pragma unroll
        for (int e = 0; e < 8; ++e) r.k[it][e] = h2f(x[e]);
      }
      r.v[it] = *reinterpret_cast<const h8*>(vpb + (size_t)kj * HD + d0);
    } else {
      const int ts = kj - a.Sp;
      const _Float16* kr = a.ks + (size_t)ts * a.ks_ld + (size_t)kvh * HD;
      if (!a.ks_roped && a.cos) {
        rope8(kr, d0, HALF, a.cos + (size_t)ts * HALF, a.sin + (size_t)ts * HALF, r.k[it]);
      } else {
        const h8 x = *reinterpret_cast<const h8*>(kr + d0);
#pragma unroll
        for (int e = 0; e < 8; ++e) r.k[it][e] = h2f(x[e]);
      }
      r.v[it] = *reinterpret_cast<const h8*>(a.vs + (size_t)ts * a.vs_ld + (size_t)kvh * HD + d0);
    }
  }
  r.msk = 0.f;
  if (tid < KCH) {
    const int kj = c0 + tid;
    if (kj >= kend) r.msk = -INFINITY;
    else if (kj < a.Sp) r.msk = a.mask ? a.mask[kj] : 0.f;
  }
}

template <int HD>
__device__ __forceinline__ void kv_sstore(const KvRegs<HD>& r, AttnSmem<HD>& sm, int tid) {
  constexpr int KLD = AttnSmem<HD>::KLD, VLD = AttnSmem<HD>::VLD;
#pragma unroll
  for (int it = 0; it < KvRegs<HD>::NIT; ++it) {
    const int item = tid + 256 * it;
    if (item >= KCH * (HD / 8)) continue;
    const int jl = item / (HD / 8);
    const int d0 = (item % (HD / 8)) * 8;
    h8 hi8, lo8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      _Float16 hi, lo;
      split_f32(r.k[it][e], hi, lo);
      hi8[e] = hi;
      lo8[e] = lo;
    }
    *reinterpret_cast<h8*>(&sm.kh[jl * KLD + d0]) = hi8;
    *reinterpret_cast<h8*>(&sm.kl[jl * KLD + d0]) = lo8;
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.vt[(d0 + e) * VLD + jl] = r.v[it][e];
  }
  if (tid < KCH) sm.msk[tid] = r.msk;
}

template <int HD>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) AttnSmem<HD> sm;
  constexpr int KLD = AttnSmem<HD>::KLD, VLD = AttnSmem<HD>::VLD;
  constexpr int NKS = (HD + 31) / 32;   // k-steps of 32 dims
  constexpr int NDT = HD / 16;          // output d tiles
  constexpr int HALF = HD / 2;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int kvh = blockIdx.z, split = blockIdx.y;
  const int grp = a.H / a.KV;
  const int row = blockIdx.x * ROWS + 16 * w + r16;   // this lane's query row (B-operand column)
  const bool row_ok = row < a.rows;
  const int hl = row_ok ? row / a.Tq : 0;
  const int t = row_ok ? row % a.Tq : 0;
  const int h = kvh * grp + hl;

  // ---- Q^T fragments (hi/lo) for this lane's row --------------------------
  h8 qh[NKS], ql[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d0 = 32 * ks + 8 * g;
    float v[8];
    if (row_ok && d0 < HD) {
      const _Float16* qr = a.q + (size_t)t * a.q_ld + (size_t)h * HD;
      if (a.cos) {
        rope8(qr, d0, HALF, a.cos + (size_t)t * HALF, a.sin + (size_t)t * HALF, v);
      } else {
        const h8 x = *reinterpret_cast<const h8*>(qr + d0);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = h2f(x[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= a.q_scale;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      _Float16 hi, lo;
      split_f32(v[e], hi, lo);
      qh[ks][e] = hi;
      ql[ks][e] = lo;
    }
  }

  f4 oacc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) oacc[i] = (f4){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.f;

  const int S = a.Sp + a.Ts;
  const int kbeg = split * a.kps;
  const int kend = min(S, kbeg + a.kps);
  KvRegs<HD> regs;
  if (kbeg < kend) kv_gload<HD>(regs, a, kbeg, kend, kvh, tid);

  for (int c0 = kbeg; c0 < kend; c0 += KCH) {
    kv_sstore<HD>(regs, sm, tid);
    if (c0 + KCH < kend) kv_gload<HD>(regs, a, c0 + KCH, kend, kvh, tid);
    __syncthreads();

    // ---- logits S^T for 2 key tiles of 16 --------------------------------
    float p[8];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f4 sacc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d0 = 32 * ks + 8 * g;
        h8 ah = (h8){0, 0, 0, 0, 0, 0, 0, 0}, al = ah;
        if (d0 < HD) {
          ah = *reinterpret_cast<const h8*>(&sm.kh[(16 * kt + r16) * KLD + d0]);
          al = *reinterpret_cast<const h8*>(&sm.kl[(16 * kt + r16) * KLD + d0]);
        }
        sacc = mfma16x16x32(al, qh[ks], sacc);
        sacc = mfma16x16x32(ah, ql[ks], sacc);
        sacc = mfma16x16x32(ah, qh[ks], sacc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) p[4 * kt + i] = sacc[i] + sm.msk[16 * kt + 4 * g + i];
    }
    // S^T tile layout: lane holds keys 16kt + 4g + i of row r16 -- but the MFMA
    // output row index is the A row (key) = 4g + i and the column is B col (row) = r16.
    float cmax = p[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) cmax = fmaxf(cmax, p[i]);
    cmax = xor_max_16_32(cmax);
    const float m_new = fmaxf(m_run, cmax);
    const float alpha = expf(m_run - m_new);
    float psum = 0.f;
    h8 pb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float e = expf(p[i] - m_new);
      psum += e;
      pb[i] = f2h(e);
    }
    psum = xor_sum_16_32(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // ---- O^T += V^T . P^T ----------------------------------------------------
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const _Float16* vr = &sm.vt[(16 * dt + r16) * VLD];
      const h4 v0 = *reinterpret_cast<const h4*>(vr + 4 * g);
      const h4 v1 = *reinterpret_cast<const h4*>(vr + 16 + 4 * g);
      h8 av;
      av[0] = v0[0]; av[1] = v0[1]; av[2] = v0[2]; av[3] = v0[3];
      av[4] = v1[0]; av[5] = v1[1]; av[6] = v1[2]; av[7] = v1[3];
      f4 o = oacc[dt];
      o[0] *= alpha; o[1] *= alpha; o[2] *= alpha; o[3] *= alpha;
      oacc[dt] = mfma16x16x32(av, pb, o);
    }
    __syncthreads();
  }

  if (!row_ok) return;
  if (a.nsplit == 1) {
    const float inv = 1.0f / l_run;
    _Float16* orow = a.out + (size_t)t * a.out_ld + (size_t)h * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      h4 o4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = f2h(oacc[dt][i] * inv);
      *reinterpret_cast<h4*>(orow + 16 * dt + 4 * g) = o4;
    }
  } else {
    const size_t pr = ((size_t)kvh * a.nsplit + split) * a.rpad + row;
    float* po = a.part_o + pr * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<f4*>(po + 16 * dt + 4 * g) = oacc[dt];
    if (g == 0) {
      a.part_ml[pr * 2 + 0] = m_run;
      a.part_ml[pr * 2 + 1] = l_run;
    }
  }
}

// combine the per-split partial softmax states of one row (one wave per row)
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a) {
  const int row = blockIdx.x, kvh = blockIdx.y, lane = threadIdx.x;
  const int hd = a.hd;
  const int grp = a.H / a.KV;
  const int hl = row / a.Tq, t = row % a.Tq, h = kvh * grp + hl;
  const size_t pr0 = (size_t)kvh * a.nsplit * a.rpad + row;
  // split weights w_s = exp(m_s - max) / sum_s l_s exp(m_s - max), lane s holds split s
  float m = -INFINITY, l = 0.f;
  if (lane < a.nsplit) {
    m = a.part_ml[(pr0 + (size_t)lane * a.rpad) * 2];
    l = a.part_ml[(pr0 + (size_t)lane * a.rpad) * 2 + 1];
  }
  float mmax = m;
  for (int o = 32; o > 0; o >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, o));
  const float e = lane < a.nsplit ? expf(m - mmax) : 0.f;
  const float lsum = wave_sum(l * e);
  const float wgt = e / lsum;
  float wv[16];  // all lanes take part in the shuffles (nsplit <= 16)
#pragma unroll
  for (int s = 0; s < 16; ++s) wv[s] = __shfl(wgt, s);
  _Float16* orow = a.out + (size_t)t * a.out_ld + (size_t)h * hd;
  for (int d = lane * 4; d < hd; d += 256) {
    f4 acc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      if (s >= a.nsplit) break;
      const float ws = wv[s];
      const f4 o = *reinterpret_cast<const f4*>(a.part_o + (pr0 + (size_t)s * a.rpad) * hd + d);
      acc[0] += ws * o[0];
      acc[1] += ws * o[1];
      acc[2] += ws * o[2];
      acc[3] += ws * o[3];
    }
    h4 o4;
#pragma unroll
    for (int i = 0; i < 4; ++i) o4[i] = f2h(acc[i]);
    *reinterpret_cast<h4*>(orow + d) = o4;
  }
}

// post-RoPE K (fp32) and V (fp16) of one prefill layer into the [KV][P][hd] cache slices
__global__ void kv_writer_kernel(const _Float16* __restrict__ qkv, int ld, int koff, int voff,
                                 const float* __restrict__ cosb, const float* __restrict__ sinb, int P, int KV,
                                 int hd, float* __restrict__ keys, _Float16* __restrict__ values) {
  const int half = hd / 2;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)P * KV * half;
  if (idx >= total) return;
  const int i = (int)(idx % half);
  const int kvh = (int)((idx / half) % KV);
  const int p = (int)(idx / ((long)half * KV));
  const _Float16* kr = qkv + (size_t)p * ld + koff + (size_t)kvh * hd;
  const _Float16* vr = qkv + (size_t)p * ld + voff + (size_t)kvh * hd;
  const float c = cosb[(size_t)p * half + i], s = sinb[(size_t)p * half + i];
  const float x1 = h2f(kr[i]), x2 = h2f(kr[i + half]);
  float* ko = keys + ((size_t)kvh * P + p) * hd;
  _Float16* vo = values + ((size_t)kvh * P + p) * hd;
  ko[i] = x1 * c - x2 * s;
  ko[i + half] = x2 * c + x1 * s;
  vo[i] = vr[i];
  vo[i + half] = vr[i + half];
}

// plain Gemma RMSNorm: out = fp16(x / sqrt(mean(x^2) + eps) * (1 + w)), one block per row
__global__ __launch_bounds__(256) void rmsnorm_kernel(const _Float16* __restrict__ x, const _Float16* __restrict__ w,
                                                      _Float16* __restrict__ out, int dim, float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const _Float16* xr = x + (size_t)r * dim;
  float ss = 0.f;
  for (int k = tid; k < dim; k += 256) {
    const float f = h2f(xr[k]);
    ss += f * f;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float dn = sqrtf(tot / (float)dim + eps);
  for (int k = tid; k < dim; k += 256) out[(size_t)r * dim + k] = f2h(h2f(xr[k]) / dn * (1.0f + h2f(w[k])));
}

__global__ void euler_init_kernel(const float* __restrict__ x0, float* __restrict__ x32, _Float16* __restrict__ x16,
                                  int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    x32[i] = x0[i];
    x16[i] = f2h(x0[i]);
  }
}

}  // namespace

void attn_plan(int rows, int keys, int target_blocks, int* nsplit, int* kps) {
  const int rb = (rows + ROWS - 1) / ROWS;
  const int chunks = (keys + KCH - 1) / KCH;
  int ns = (target_blocks + rb - 1) / rb;
  if (ns > 16) ns = 16;
  if (ns > chunks) ns = chunks;
  if (ns < 1) ns = 1;
  const int cps = (chunks + ns - 1) / ns;
  *kps = cps * KCH;
  *nsplit = (chunks + cps - 1) / cps;
}

size_t attn_ws_floats(int KV, int rows, int hd, int nsplit) {
  const int rpad = ((rows + ROWS - 1) / ROWS) * ROWS;
  return nsplit > 1 ? (size_t)KV * nsplit * rpad * (hd + 2) : 0;
}

int attn_launch(const AttnArgs& a, hipStream_t st) {
  MLCV_REQUIRE(a.H % a.KV == 0 && (a.KV == 1 || a.KV == a.H), "kv heads must broadcast to q heads");
  MLCV_REQUIRE(a.rows == a.Tq * (a.H / a.KV), "attention rows mismatch");
  MLCV_REQUIRE(a.kps % KCH == 0 && a.nsplit >= 1, "attention split plan");
  MLCV_REQUIRE((long)a.nsplit * a.kps >= (long)(a.Sp + a.Ts), "attention splits do not cover the keys");
  MLCV_REQUIRE(a.nsplit == 1 || (a.part_o && a.part_ml), "attention workspace missing");
  MLCV_REQUIRE(a.nsplit <= 16, "at most 16 key splits");
  dim3 grid((a.rows + ROWS - 1) / ROWS, a.nsplit, a.KV);
  switch (a.hd) {
    case 16: attn_kernel<16><<<grid, 256, 0, st>>>(a); break;
    case 32: attn_kernel<32><<<grid, 256, 0, st>>>(a); break;
    case 64: attn_kernel<64><<<grid, 256, 0, st>>>(a); break;
    case 128: attn_kernel<128><<<grid, 256, 0, st>>>(a); break;
    case 256: attn_kernel<256><<<grid, 256, 0, st>>>(a); break;
    default: MLCV_REQUIRE(false, "head_dim must be one of 16, 32, 64, 128, 256");
  }
  MLCV_HIP(hipGetLastError());
  if (a.nsplit > 1) {
    attn_combine_kernel<<<dim3(a.rows, a.KV), 64, 0, st>>>(a);
    MLCV_HIP(hipGetLastError());
  }
  return 0;
}

int kv_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin, int P,
                     int KV, int hd, float* keys, _Float16* values, hipStream_t st) {
  const long total = (long)P * KV * (hd / 2);
  kv_writer_kernel<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(qkv, ld, koff, voff, cos, sin, P, KV, hd, keys,
                                                                     values);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int rmsnorm_launch(const _Float16* x, const _Float16* w, _Float16* out, int rows, int dim, float eps,
                   hipStream_t st) {
  rmsnorm_kernel<<<rows, 256, 0, st>>>(x, w, out, dim, eps);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int euler_init_launch(const float* x0, float* x32, _Float16* x16, int n, hipStream_t st) {
  euler_init_kernel<<<(n + 255) / 256, 256, 0, st>>>(x0, x32, x16, n);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
