// Joint attention kernels (the device code is in attn_impl.h): the standalone attention and
// combine kernels, the chunk-image builder, and the prefill helpers (K/V writer, RMSNorm,
// Euler init, batched copies).
#include <algorithm>
#include <type_traits>

#ifdef MLCV_ATTN_TRACE
// timeline of the last standalone attention launch (trace build): [workgroup][stage]
__device__ unsigned long long attn_trace[1024 * 8];
#define ATTN_STAMP(k)                                                                                     \
  do {                                                                                                    \
    if (tid == 0) attn_trace[(blockIdx.x + gridDim.x * blockIdx.y) * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#endif
#include "attn_impl.h"

namespace mlcv {

namespace {

template <int HD, bool KF32, bool ROPE, bool IMG, bool QF, int NW>
__global__ __launch_bounds__(64 * NW) void attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds_raw[2 * attn_buf_bytes<HD, IMG>()];
  if (a.xgroup) {  // XCD-grouped order: column x of the grid runs on XCD x
    const int x = blockIdx.x, j = blockIdx.y, rbs = (a.rows + ROWS - 1) / ROWS;
    const int nt = (a.nsplit - x + 7) / 8 * rbs;  // tasks of splits x, x + 8, ...
    if (j < nt) {
      attn_block<HD, KF32, ROPE, IMG, QF, false, NW>(a, j % rbs, x + 8 * (j / rbs), blockIdx.z, lds_raw, threadIdx.x);
    } else if (j < nt + a.pf.nblocks / 8 && blockIdx.z == 0) {
      prefetch_ranked(a.pf, x, j - nt, a.pf.nblocks / 8);
    }
    return;
  }
  if (blockIdx.y >= a.nsplit) {  // prefetch workgroups (grid rows past the key splits)
    if (blockIdx.z == 0) prefetch_run(a.pf, blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * a.nsplit);
    return;
  }
  attn_block<HD, KF32, ROPE, IMG, QF, false, NW>(a, blockIdx.x, blockIdx.y, blockIdx.z, lds_raw, threadIdx.x);
}

// chunk images of the prefix K/V of `layers` layers: grid (chunks, KV, layers)
template <int HD, bool KF32>
__global__ __launch_bounds__(256) void attn_img_prep_kernel(const void* __restrict__ keys,
                                                            const _Float16* __restrict__ values,
                                                            const float* __restrict__ mask, int Sp, int KV,
                                                            char* __restrict__ img, size_t layer_bytes) {
  constexpr int KLD = AttnSmem<HD>::KLD;
  constexpr int IMGB = img_bytes<HD>();
  __shared__ __attribute__((aligned(16))) _Float16 sv[KCH * HD];
  const int c = blockIdx.x, kvh = blockIdx.y, layer = blockIdx.z, tid = threadIdx.x;
  const int c0 = c * KCH;
  const size_t kvbase = ((size_t)layer * KV + kvh) * Sp * HD;
  AttnSmem<HD>* im =
      reinterpret_cast<AttnSmem<HD>*>(img + layer * layer_bytes + ((size_t)kvh * gridDim.x + c) * IMGB);
  const h8 zero8 = (h8){0, 0, 0, 0, 0, 0, 0, 0};
  // K rows split hi/lo (the pad columns past HD and keys past Sp are zero)
  for (int i = tid; i < KCH * (KLD / 8); i += 256) {
    const int j = i / (KLD / 8), dq = (i % (KLD / 8)) * 8;
    h8 hi = zero8, lo = zero8;
    if (dq < HD && c0 + j < Sp) {
      float v[8];
      if constexpr (KF32) {
        const float* kp = reinterpret_cast<const float*>(keys) + kvbase + (size_t)(c0 + j) * HD + dq;
        const f4 x = *reinterpret_cast<const f4*>(kp), y = *reinterpret_cast<const f4*>(kp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = x[e];
          v[e + 4] = y[e];
        }
      } else {
        const h8 x = *reinterpret_cast<const h8*>(reinterpret_cast<const _Float16*>(keys) + kvbase +
                                                  (size_t)(c0 + j) * HD + dq);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = h2f(x[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16 hh, ll;
        split_f32(v[e], hh, ll);
        hi[e] = hh;
        lo[e] = ll;
      }
    }
    *reinterpret_cast<h8*>(&im->kh[j * KLD + dq]) = hi;
    *reinterpret_cast<h8*>(&im->kl[j * KLD + dq]) = lo;
  }
  // V: staged in LDS, written transposed vt[d][j] = V[c0 + j][d] (keys past Sp and the
  // pad slots past 32 are zero)
  for (int i = tid; i < KCH * HD / 8; i += 256) {
    const int j = i / (HD / 8), d8 = (i % (HD / 8)) * 8;
    const h8 v = c0 + j < Sp ? *reinterpret_cast<const h8*>(values + kvbase + (size_t)(c0 + j) * HD + d8) : zero8;
    *reinterpret_cast<h8*>(&sv[j * HD + d8]) = v;
  }
  __syncthreads();
  for (int i = tid; i < HD * (VLD / 4); i += 256) {  // 8-byte pieces (V^T rows are 8-byte aligned)
    const int d = i / (VLD / 4), j4 = (i % (VLD / 4)) * 4;
    h4 o = (h4){0, 0, 0, 0};
    if (j4 < KCH) {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = sv[(j4 + e) * HD + d];
    }
    *reinterpret_cast<h4*>(&im->vt[d * VLD + j4]) = o;
  }
  if (tid < KCH) im->msk[tid] = c0 + tid < Sp ? (mask ? mask[c0 + tid] : 0.f) : -INFINITY;
}

// combine the per-split partial softmax states, one wave per row
template <int MAXS>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a) {
  combine_row<MAXS, false>(a, blockIdx.y, blockIdx.x, threadIdx.x);
}

// The attention and its split combine in one launch (decode shapes: every workgroup resident
// at once).  Workgroup id runs row block b = 8 (id / 8 / nsplit) + id % 8 (over the kv heads)
// against key split (id / 8) % nsplit, so the splits of a row block are dealt to one XCD (the
// dispatch order is round-robin over the 8 XCDs).  Each split stores its partial (O_s / l_s in
// fp16, (m, l) in fp32) with device-scope stores; the splits of a row block meet at a counter
// (group_meet_gen, bounded); then workgroup `split` combines rows split, split + nsplit, ... of
// the block, one wave per row, with device-scope loads (so a workgroup placed on another XCD
// than the order gives still reads the right values).  A meeting that gives up raises *err and
// writes NaN rows instead.
template <int HD, bool KF32, int MAXS>
__global__ __launch_bounds__(256) void attn_fused_kernel(AttnArgs a, unsigned* meet, unsigned polls, unsigned* err) {
  __shared__ __attribute__((aligned(16))) char lds_raw[2 * attn_buf_bytes<HD, false>()];
  __shared__ int met;
  const int id = blockIdx.x, x = id % 8, j = id / 8;
  const int rbs = (a.rows + ROWS - 1) / ROWS;  // row blocks per kv head
  const int b = (j / a.nsplit) * 8 + x, split = j % a.nsplit;
  if (b >= rbs * a.KV) return;  // no row block on this slot: takes part in no meeting
  const int kvh = b / rbs, bx = b % rbs, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const unsigned gen = tid == 0 ? group_gen(meet + 32 * b) : 0u;
  attn_block<HD, KF32, false, false, false, true, 4>(a, bx, split, kvh, lds_raw, tid);
  wait_all_memory();  // this wave's partial stores have completed
  __syncthreads();
  if (tid == 0) {
    met = group_meet_gen(meet + 32 * b, (unsigned)a.nsplit, polls, gen) ? 1 : 0;
    if (!met && err) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  __syncthreads();
  for (int r = split + a.nsplit * w; r < ROWS; r += 4 * a.nsplit) {
    const int row = bx * ROWS + r;
    if (row >= a.rows) break;
    if (met) {
      combine_row<MAXS, true, false>(a, kvh, row, lane);  // the output is read by later launches
    } else {
      const int grp = a.H / a.KV, hl = row / a.Tq, t = row % a.Tq, h = kvh * grp + hl;
      for (int d = 4 * lane; d < a.hd; d += 256) {
        const float nan = __builtin_nanf("");
        const h4 o4 = {f2h(nan), f2h(nan), f2h(nan), f2h(nan)};
        *reinterpret_cast<h4*>(a.out + (size_t)t * a.out_ld + (size_t)h * HD + d) = o4;
      }
    }
  }
}

// q fragments of the prefill: one thread per (kv head, 16-row tile, k step of the first half
// of the head dims, lane): lane 16 g + r of k step ks takes row 16 tile + r, dims
// d = 32 ks + 8 g .. +7 and their RoPE partners d + hd/2, and writes their hi and lo halves,
// so every wave store is one whole 1 KB fragment block (attn_qf_index).  RoPE and the scale
// in fp32 as the attention's own q loader (make_q) computes them.
__device__ __forceinline__ void q_frag_item(const _Float16* __restrict__ q, int ld, const float* __restrict__ cosb,
                                            const float* __restrict__ sinb, int P, int grp, int hd, float q_scale,
                                            int KV, int ntiles, _Float16* __restrict__ qf, long idx) {
  const int half = hd / 2, nks = hd / 32, nk2 = nks / 2;
  if (idx >= (long)KV * ntiles * nk2 * 64) return;
  const int lane = (int)(idx & 63);
  const long rest = idx >> 6;
  const int ks = (int)(rest % nk2), tile = (int)((rest / nk2) % ntiles), kvh = (int)(rest / nk2 / ntiles);
  const int row = 16 * tile + (lane & 15), d = 32 * ks + 8 * (lane >> 4);
  h8 hi1, lo1, hi2, lo2;
  if (row < P * grp) {
    const int hl = row / P, t = row % P, h = kvh * grp + hl;
    const _Float16* qr = q + (size_t)t * ld + (size_t)h * hd + d;
    const h8 x1 = *reinterpret_cast<const h8*>(qr), x2 = *reinterpret_cast<const h8*>(qr + half);
    const f4* cp = reinterpret_cast<const f4*>(cosb + (size_t)t * half + d);
    const f4* sp = reinterpret_cast<const f4*>(sinb + (size_t)t * half + d);
    const f4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = h2f(x1[e]), b = h2f(x2[e]);
      const float c = e < 4 ? c0[e] : c1[e - 4], sn = e < 4 ? s0[e] : s1[e - 4];
      _Float16 hv, lv;
      split_f32((a * c - b * sn) * q_scale, hv, lv);
      hi1[e] = hv;
      lo1[e] = lv;
      split_f32((b * c + a * sn) * q_scale, hv, lv);
      hi2[e] = hv;
      lo2[e] = lv;
    }
  } else {
    hi1 = lo1 = hi2 = lo2 = (h8){0, 0, 0, 0, 0, 0, 0, 0};
  }
  *reinterpret_cast<h8*>(qf + attn_qf_index(kvh, ntiles, nks, row, d, 0)) = hi1;
  *reinterpret_cast<h8*>(qf + attn_qf_index(kvh, ntiles, nks, row, d, 1)) = lo1;
  *reinterpret_cast<h8*>(qf + attn_qf_index(kvh, ntiles, nks, row, d + half, 0)) = hi2;
  *reinterpret_cast<h8*>(qf + attn_qf_index(kvh, ntiles, nks, row, d + half, 1)) = lo2;
}
__global__ __launch_bounds__(256) void q_frag_kernel(const _Float16* __restrict__ q, int ld,
                                                     const float* __restrict__ cosb, const float* __restrict__ sinb,
                                                     int P, int grp, int hd, float q_scale, int KV, int ntiles,
                                                     _Float16* __restrict__ qf) {
  q_frag_item(q, ld, cosb, sinb, P, grp, hd, q_scale, KV, ntiles, qf, (long)blockIdx.x * blockDim.x + threadIdx.x);
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

// the same with 4 consecutive dims per thread (hd % 8 == 0, ld, koff, voff multiples of 4)
__device__ __forceinline__ void kv_writer4_item(const _Float16* __restrict__ qkv, int ld, int koff, int voff,
                                                const float* __restrict__ cosb, const float* __restrict__ sinb, int P,
                                                int KV, int hd, float* __restrict__ keys,
                                                _Float16* __restrict__ values, long idx) {
  const int half = hd / 2, q4 = half / 4;
  const long total = (long)P * KV * q4;
  if (idx >= total) return;
  const int i = (int)(idx % q4) * 4;
  const int kvh = (int)((idx / q4) % KV);
  const int p = (int)(idx / ((long)q4 * KV));
  const _Float16* kr = qkv + (size_t)p * ld + koff + (size_t)kvh * hd;
  const _Float16* vr = qkv + (size_t)p * ld + voff + (size_t)kvh * hd;
  const f4 c = *reinterpret_cast<const f4*>(cosb + (size_t)p * half + i);
  const f4 sn = *reinterpret_cast<const f4*>(sinb + (size_t)p * half + i);
  const h4 a = *reinterpret_cast<const h4*>(kr + i), b = *reinterpret_cast<const h4*>(kr + i + half);
  f4 o1, o2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x1 = h2f(a[e]), x2 = h2f(b[e]);
    o1[e] = x1 * c[e] - x2 * sn[e];
    o2[e] = x2 * c[e] + x1 * sn[e];
  }
  float* ko = keys + ((size_t)kvh * P + p) * hd;
  _Float16* vo = values + ((size_t)kvh * P + p) * hd;
  *reinterpret_cast<f4*>(ko + i) = o1;
  *reinterpret_cast<f4*>(ko + i + half) = o2;
  *reinterpret_cast<h4*>(vo + i) = *reinterpret_cast<const h4*>(vr + i);
  *reinterpret_cast<h4*>(vo + i + half) = *reinterpret_cast<const h4*>(vr + i + half);
}
__global__ void kv_writer4_kernel(const _Float16* __restrict__ qkv, int ld, int koff, int voff,
                                  const float* __restrict__ cosb, const float* __restrict__ sinb, int P, int KV, int hd,
                                  float* __restrict__ keys, _Float16* __restrict__ values) {
  kv_writer4_item(qkv, ld, koff, voff, cosb, sinb, P, KV, hd, keys, values,
                  (long)blockIdx.x * blockDim.x + threadIdx.x);
}
// one launch for both: the first kvb blocks write the K/V cache slices, the rest q's fragments
__global__ __launch_bounds__(256) void kvq_writer_kernel(const _Float16* __restrict__ qkv, int ld, int koff, int voff,
                                                         const float* __restrict__ cosb, const float* __restrict__ sinb,
                                                         int P, int H, int KV, int hd, float* __restrict__ keys,
                                                         _Float16* __restrict__ values, float q_scale, int ntiles,
                                                         _Float16* __restrict__ qf, int kvb) {
  if ((int)blockIdx.x < kvb)
    kv_writer4_item(qkv, ld, koff, voff, cosb, sinb, P, KV, hd, keys, values,
                    (long)blockIdx.x * blockDim.x + threadIdx.x);
  else
    q_frag_item(qkv, ld, cosb, sinb, P, H / KV, hd, q_scale, KV, ntiles, qf,
                (long)(blockIdx.x - kvb) * blockDim.x + threadIdx.x);
}

// plain Gemma RMSNorm: out = fp16(x / sqrt(mean(x^2) + eps) * (1 + w)), one block per row.
// Rows of at most 256 x 8 x NP halfs (dim % 8 == 0) stay in registers between the two
// passes, one 16-byte load per piece.
template <int NP>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const _Float16* __restrict__ x, const _Float16* __restrict__ w,
                                                          _Float16* __restrict__ out, int dim, float eps, int tile) {
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x, n8 = dim / 8;
  const _Float16* xr = x + (size_t)r * dim;
  h8 v[NP];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int i = tid + 256 * p;
    v[p] = i < n8 ? *reinterpret_cast<const h8*>(xr + 8 * i) : (h8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = h2f(v[p][e]);
      ss += f * f;
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float dn = sqrtf(tot / (float)dim + eps);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int i = tid + 256 * p;
    if (i >= n8) break;
    const h8 wv = *reinterpret_cast<const h8*>(w + 8 * i);
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f2h(h2f(v[p][e]) / dn * (1.0f + h2f(wv[e])));
    // tile-major: [rows / 16][dim / 32][16][32] (the 32-k tiles of the prefill GEMM)
    const size_t oi = tile ? ((size_t)(r >> 4) * (dim >> 5) + (8 * i >> 5)) * 512 + (r & 15) * 32 + (8 * i & 31)
                           : (size_t)r * dim + 8 * i;
    *reinterpret_cast<h8*>(out + oi) = o;
  }
}

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

struct CopyList {
  CopyJob j[COPY_MAX];
};
// job blockIdx.y; 16-byte pieces when both ends and the size are 16-byte aligned, bytes otherwise
__global__ void copy_list_kernel(CopyList L) {
  const CopyJob jb = L.j[blockIdx.y];
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x, nt = (size_t)gridDim.x * blockDim.x;
  if (((reinterpret_cast<uintptr_t>(jb.src) | reinterpret_cast<uintptr_t>(jb.dst) | jb.bytes) & 15) == 0) {
    const u4* s = static_cast<const u4*>(jb.src);
    u4* d = static_cast<u4*>(jb.dst);
    for (size_t i = t; i < jb.bytes / 16; i += nt) d[i] = s[i];
  } else {
    const char* s = static_cast<const char*>(jb.src);
    char* d = static_cast<char*>(jb.dst);
    for (size_t i = t; i < jb.bytes; i += nt) d[i] = s[i];
  }
}

}  // namespace

int copy_list_launch(const CopyJob* jobs, int n, hipStream_t st) {
  MLCV_REQUIRE(n >= 0 && n <= COPY_MAX, "at most 8 copies per batch");
  CopyList L{};
  size_t most = 0;
  int k = 0;
  for (int i = 0; i < n; ++i) {
    if (jobs[i].bytes == 0) continue;
    MLCV_REQUIRE(jobs[i].src && jobs[i].dst, "null copy buffer");
    L.j[k++] = jobs[i];
    most = std::max(most, jobs[i].bytes);
  }
  if (k == 0) return 0;
  const unsigned bx = (unsigned)std::min<size_t>(256, (most / 16 + 255) / 256 + 1);
  copy_list_kernel<<<dim3(bx, k), 256, 0, st>>>(L);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int attn_fused_launch(const AttnArgs& a, unsigned* meet, unsigned polls, unsigned* err, hipStream_t st) {
  MLCV_REQUIRE(a.H % a.KV == 0 && a.rows == a.Tq * (a.H / a.KV) && a.hd == 256 && !a.qf && !a.kimg && !a.cos &&
                   !a.out_frag && a.ks_roped && a.nsplit >= 2 && a.nsplit <= 32 && a.kps % KCH == 0 &&
                   a.part_o && a.part_ml && meet,
               "one-launch attention: head_dim 256, raw q, roped suffix keys, 2..32 splits, workspace");
  const int nsp = a.nsplit - (a.Ts > 0 ? 1 : 0);
  MLCV_REQUIRE((long)nsp * a.kps >= (long)a.Sp && (a.Sp > 0 || nsp == 0), "attention splits do not cover the keys");
  const int nrb = (a.rows + ROWS - 1) / ROWS * a.KV;
  const unsigned blocks = (unsigned)((nrb + 7) / 8 * a.nsplit * 8);
  MLCV_REQUIRE((int)blocks <= device_cus(), "one-launch attention: every workgroup must be resident at once");
  if (a.kp_f32) attn_fused_kernel<256, true, 32><<<blocks, 256, 0, st>>>(a, meet, polls, err);
  else attn_fused_kernel<256, false, 32><<<blocks, 256, 0, st>>>(a, meet, polls, err);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int attn_launch(const AttnArgs& a, hipStream_t st) {
  MLCV_REQUIRE(a.H % a.KV == 0 && (a.KV == 1 || a.KV == a.H), "kv heads must broadcast to q heads");
  MLCV_REQUIRE(a.rows == a.Tq * (a.H / a.KV), "attention rows mismatch");
  MLCV_REQUIRE(a.kps % KCH == 0 && a.kps > 0 && a.nsplit >= 1, "attention split plan");
  const int nsp = a.nsplit - (a.Ts > 0 ? 1 : 0);
  MLCV_REQUIRE((long)nsp * a.kps >= (long)a.Sp && (a.Sp > 0 || nsp == 0), "attention splits do not cover the keys");
  MLCV_REQUIRE(a.Ts == 0 || (a.ks && a.vs), "suffix keys missing");
  MLCV_REQUIRE(a.nsplit == 1 || (a.part_o && a.part_ml), "attention workspace missing");
  MLCV_REQUIRE(!a.out_frag || (a.Tq <= 64 && (a.H * a.hd) % 32 == 0), "fragment-major output needs Tq <= 64");
  MLCV_REQUIRE(a.nsplit <= 32, "at most 32 key splits");
  MLCV_REQUIRE(!a.kimg || a.img_chunks == (a.Sp + KCH - 1) / KCH, "chunk images do not match the prefix length");
  MLCV_REQUIRE(a.cos == nullptr || a.sin != nullptr, "rope needs cos and sin");
  MLCV_REQUIRE(a.Ts == 0 || a.cos != nullptr || a.ks_roped || a.qf, "raw suffix keys need the rope tables");
  MLCV_REQUIRE(!a.qf || ((a.Ts == 0 || a.ks32) && a.kp_f32 && a.rpad % 64 == 0),
               "fragment-order q needs the fp32 suffix keys and an fp32 prefix cache");
  MLCV_REQUIRE(a.pf.nreg >= 0 && a.pf.nreg <= PF_MAX_REGIONS, "prefetch regions");
  for (int i = 0; i < a.pf.nreg; ++i)
    MLCV_REQUIRE(a.pf.r[i].slab_bytes > 0 && a.pf.r[i].slab_bytes % 64 == 0 && a.pf.r[i].nslabs >= 0,
                 "prefetch slabs must be whole 64-byte lines");
  const int rb = (a.rows + ROWS - 1) / ROWS;
  AttnArgs ka = a;
  const int pf_rows = a.pf.nreg > 0 && a.pf.nblocks > 0 ? (a.pf.nblocks + rb - 1) / rb : 0;
  ka.pf.nblocks = pf_rows * rb;
  dim3 grid(rb, a.nsplit + pf_rows, a.KV);
  if (a.xgroup) {
    MLCV_REQUIRE(a.qf && !a.kimg, "XCD-grouped order: the 8-wave q-fragment form");
    const int pfx = a.pf.nreg > 0 && a.pf.nblocks > 0 ? (a.pf.nblocks + 7) / 8 : 0;  // per XCD
    ka.pf.nblocks = 8 * pfx;
    grid = dim3(8, (a.nsplit + 7) / 8 * rb + pfx, a.KV);
  }
// the step's form (q fragments, converted chunks) runs on 8 waves (attn_block): 868 vs 871 us
// per step; the others on 4 (the prefill's form spills at 8 waves: +20 us per prefill)
#define MLCV_ATTN_CASE(HDV)                                                                        \
  case HDV:                                                                                        \
    if (a.qf) {                                                                                    \
      if (a.kimg) attn_kernel<HDV, true, false, true, true, 4><<<grid, 256, 0, st>>>(ka);           \
      else attn_kernel<HDV, true, false, false, true, 8><<<grid, 512, 0, st>>>(ka);                 \
    } else if (a.kimg) {                                                                           \
      if (a.cos) attn_kernel<HDV, true, true, true, false, 4><<<grid, 256, 0, st>>>(ka);            \
      else attn_kernel<HDV, true, false, true, false, 4><<<grid, 256, 0, st>>>(ka);                 \
    } else if (a.kp_f32) {                                                                         \
      if (a.cos) attn_kernel<HDV, true, true, false, false, 4><<<grid, 256, 0, st>>>(ka);           \
      else attn_kernel<HDV, true, false, false, false, 4><<<grid, 256, 0, st>>>(ka);                \
    } else {                                                                                       \
      if (a.cos) attn_kernel<HDV, false, true, false, false, 4><<<grid, 256, 0, st>>>(ka);          \
      else attn_kernel<HDV, false, false, false, false, 4><<<grid, 256, 0, st>>>(ka);               \
    }                                                                                              \
    break;
  switch (a.hd) {
    MLCV_ATTN_CASE(16)
    MLCV_ATTN_CASE(32)
    MLCV_ATTN_CASE(64)
    MLCV_ATTN_CASE(128)
    MLCV_ATTN_CASE(256)
    default: MLCV_REQUIRE(false, "head_dim must be one of 16, 32, 64, 128, 256");
  }
#undef MLCV_ATTN_CASE
  MLCV_HIP(hipGetLastError());
  if (a.nsplit > 1) {
    const dim3 cg(a.rows, a.KV);
    if (a.nsplit <= 8) attn_combine_kernel<8><<<cg, 64, 0, st>>>(a);
    else if (a.nsplit <= 16) attn_combine_kernel<16><<<cg, 64, 0, st>>>(a);
    else if (a.nsplit <= 24) attn_combine_kernel<24><<<cg, 64, 0, st>>>(a);
    else attn_combine_kernel<32><<<cg, 64, 0, st>>>(a);
    MLCV_HIP(hipGetLastError());
  }
  return 0;
}

size_t attn_img_bytes(int KV, int Sp, int hd) {
  int ib = 0;
  switch (hd) {
    case 16: ib = img_bytes<16>(); break;
    case 32: ib = img_bytes<32>(); break;
    case 64: ib = img_bytes<64>(); break;
    case 128: ib = img_bytes<128>(); break;
    case 256: ib = img_bytes<256>(); break;
    default: return 0;
  }
  return (size_t)KV * ((Sp + KCH - 1) / KCH) * ib;
}

int attn_img_prep_launch(const void* keys, int k_f32, const _Float16* values, const float* mask, int layers, int KV,
                         int Sp, int hd, char* img, hipStream_t st) {
  MLCV_REQUIRE(Sp > 0 && layers > 0 && KV > 0 && img, "chunk image preparation arguments");
  const size_t lb = attn_img_bytes(KV, Sp, hd);
  MLCV_REQUIRE(lb > 0, "head_dim must be one of 16, 32, 64, 128, 256");
  dim3 grid((Sp + KCH - 1) / KCH, KV, layers);
#define MLCV_PREP_CASE(HDV)                                                                              \
  case HDV:                                                                                              \
    if (k_f32) attn_img_prep_kernel<HDV, true><<<grid, 256, 0, st>>>(keys, values, mask, Sp, KV, img, lb);  \
    else attn_img_prep_kernel<HDV, false><<<grid, 256, 0, st>>>(keys, values, mask, Sp, KV, img, lb);       \
    break;
  switch (hd) {
    MLCV_PREP_CASE(16)
    MLCV_PREP_CASE(32)
    MLCV_PREP_CASE(64)
    MLCV_PREP_CASE(128)
    MLCV_PREP_CASE(256)
    default: MLCV_REQUIRE(false, "head_dim must be one of 16, 32, 64, 128, 256");
  }
#undef MLCV_PREP_CASE
  MLCV_HIP(hipGetLastError());
  return 0;
}

int kv_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin, int P,
                     int KV, int hd, float* keys, _Float16* values, hipStream_t st) {
  const bool vec = hd % 8 == 0 && ld % 4 == 0 && koff % 4 == 0 && voff % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(keys) |
                     reinterpret_cast<uintptr_t>(values) | reinterpret_cast<uintptr_t>(cos) |
                     reinterpret_cast<uintptr_t>(sin)) & 15) == 0;
  if (vec) {
    const long total = (long)P * KV * (hd / 8);
    kv_writer4_kernel<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(qkv, ld, koff, voff, cos, sin, P, KV, hd, keys,
                                                                        values);
  } else {
    const long total = (long)P * KV * (hd / 2);
    kv_writer_kernel<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(qkv, ld, koff, voff, cos, sin, P, KV, hd, keys,
                                                                       values);
  }
  MLCV_HIP(hipGetLastError());
  return 0;
}

int kvq_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin, int P,
                      int H, int KV, int hd, float* keys, _Float16* values, float q_scale, int rpad, _Float16* qf,
                      hipStream_t st) {
  const bool vec = hd % 8 == 0 && ld % 4 == 0 && koff % 4 == 0 && voff % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(keys) |
                     reinterpret_cast<uintptr_t>(values) | reinterpret_cast<uintptr_t>(cos) |
                     reinterpret_cast<uintptr_t>(sin) | reinterpret_cast<uintptr_t>(qf)) & 15) == 0;
  if (!vec || !qf || hd % 64 != 0 || ld % 8 != 0) {  // two launches
    MLCV_TRY(kv_writer_launch(qkv, ld, koff, voff, cos, sin, P, KV, hd, keys, values, st));
    return qf ? q_frag_launch(qkv, ld, cos, sin, P, H, KV, hd, q_scale, rpad, qf, st) : 0;
  }
  MLCV_REQUIRE(P > 0 && KV > 0 && H % KV == 0 && rpad % 64 == 0 && rpad >= P * (H / KV), "q fragment shape");
  const long kvt = (long)P * KV * (hd / 8), qt = (long)KV * (rpad / 16) * (hd / 64) * 64;
  const int kvb = (int)((kvt + 255) / 256);
  kvq_writer_kernel<<<(unsigned)(kvb + (qt + 255) / 256), 256, 0, st>>>(qkv, ld, koff, voff, cos, sin, P, H, KV, hd,
                                                                          keys, values, q_scale, rpad / 16, qf, kvb);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int q_frag_launch(const _Float16* q, int ld, const float* cos, const float* sin, int P, int H, int KV, int hd,
                  float q_scale, int rpad, _Float16* qf, hipStream_t st) {
  MLCV_REQUIRE(q && cos && sin && qf && P > 0 && KV > 0 && H % KV == 0, "q fragment arguments");
  MLCV_REQUIRE(hd % 64 == 0 && ld % 8 == 0 && rpad % 64 == 0 && rpad >= P * (H / KV), "q fragment shape");
  MLCV_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(cos) | reinterpret_cast<uintptr_t>(sin) |
                 reinterpret_cast<uintptr_t>(qf)) & 15) == 0, "q fragment buffers must be 16-byte aligned");
  const long total = (long)KV * (rpad / 16) * (hd / 64) * 64;
  q_frag_kernel<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(q, ld, cos, sin, P, H / KV, hd, q_scale, KV, rpad / 16,
                                                                   qf);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int rmsnorm_launch(const _Float16* x, const _Float16* w, _Float16* out, int rows, int dim, float eps,
                   hipStream_t st, bool tile) {
  const bool vec = dim % 8 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                      reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  MLCV_REQUIRE(!tile || (vec && dim % 32 == 0 && dim <= 256 * 8 * 4), "tile-major RMSNorm output: dim % 32 == 0");
  if (vec && dim <= 256 * 8) rmsnorm_vec_kernel<1><<<rows, 256, 0, st>>>(x, w, out, dim, eps, tile ? 1 : 0);
  else if (vec && dim <= 256 * 8 * 4) rmsnorm_vec_kernel<4><<<rows, 256, 0, st>>>(x, w, out, dim, eps, tile ? 1 : 0);
  else rmsnorm_kernel<<<rows, 256, 0, st>>>(x, w, out, dim, eps);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int euler_init_launch(const float* x0, float* x32, _Float16* x16, int n, hipStream_t st) {
  euler_init_kernel<<<(n + 255) / 256, 256, 0, st>>>(x0, x32, x16, n);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv

#ifdef MLCV_ATTN_TRACE
extern "C" void* mlcv_attn_trace_ptr() {
  void* p = nullptr;
  (void)hipGetSymbolAddress(&p, HIP_SYMBOL(attn_trace));
  return p;
}
#endif
