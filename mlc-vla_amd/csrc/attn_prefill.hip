// The prefill's attention at head_dim 256 (attn_prefill_e0, gemma_dual.py:236-253,334-341): every
// prefix query row attends to every prefix key through the additive pad mask (gemma_dual.py:97-122),
// with q roped in fp32 and scaled, the logits q . k in fp32 against the roped fp32 keys of the cache,
// the softmax in fp32, the probabilities and V in fp16 with fp32 sums, the output rounded to fp16.
//
// Layout of the work (one MI355X, P = 968, 8 query heads on 1 K/V head: 7744 query rows):
// - The layer's K/V writer (pa_writer_kernel) writes, next to the fp32 key / fp16 value cache
//   slices, a per-chunk image of 32 keys exactly as the attention holds it in LDS (48 KB: K split
//   into fp16 hi + lo, and V transposed), plus q roped, scaled and split hi + lo in the MFMA
//   operand order.  Each chunk is converted once per layer instead of once per workgroup.
// - A workgroup (4 waves, one per SIMD) takes 128 query rows (32 per wave) and a range of key
//   chunks.  The chunks arrive by buffer -> LDS DMA into two buffers; a wave keeps its q (hi, lo:
//   128 registers) and its O^T accumulators (128) in registers.  Per chunk a wave runs
//   S^T = K . q^T (3 products for the fp32 logits: hi.hi, hi.lo, lo.hi) and O^T += V^T . P^T on
//   v_mfma_f32_32x32x16_f16, which moves half the LDS bytes per flop of the 16-row tiling.
// - Key splits are balanced over the chunks that hold a valid key: split s takes the valid chunks
//   of rank [n s / S, n (s + 1) / S).  Chunks whose 32 keys are all masked (<= -1e9) are skipped
//   (exact: exp of a -1e9 logit is 0 in fp32 next to any valid key); with the skip off they are
//   computed in the same splits, so the results are bit-identical.
// - The splits of a row block meet at an arrival counter: each stores its O / l in fp16 with its
//   (m, l) through to the memory side, and the last to arrive combines the splits in split order
//   (deterministic whatever the arrival order) and writes the output.  No second launch.
#include "kernels.h"

#include <type_traits>

namespace mlcv {

namespace {

constexpr int PA_HD = 256;
constexpr int PA_KCH = 32;                        // keys per chunk
constexpr int PA_ROWS = 128;                      // query rows per workgroup: 4 waves x 32
constexpr int PA_NT = 256;                        // threads per workgroup
constexpr int PA_KS = PA_HD / 16;                 // k steps of the logits
constexpr int PA_PART = PA_KCH * PA_HD * 2;       // K hi, K lo and V^T of a chunk: 16 KB each
constexpr int PA_CHUNK = 3 * PA_PART;             // 48 KB
constexpr int PA_MAXCH = 64;                      // chunks: prefix length <= 2048
constexpr int PA_MAXS = 8;                        // key splits
constexpr int PA_WAVE_PART = 8 * 2 * 64 * 8;      // halfs of one wave's fp16 partial O (32 x 256)
static_assert(PA_CHUNK / (4 * 1024) <= PA_KS, "a chunk's DMA spreads over the logits' k steps, one 1 KB block per wave each");

// ---- chunk image: byte offsets within a 48 KB chunk --------------------------------------
// K hi (lo at + PA_PART): key r's 16-byte piece p (dims 8p..8p+7) in slot p ^ (r mod 16) of its
// 512-byte row, so the 16 rows of a 16-lane operand read hit 16 distinct slots of a 256-byte bank
// line (and 8 of a 128-byte one).
__host__ __device__ __forceinline__ int pa_k_off(int r, int p) { return r * 512 + ((p ^ (r & 15)) << 4); }
// V^T row d (64 bytes, 4 pieces of 8 key positions) at 2 PA_PART + 64 d: piece p in slot
// p ^ swz(d), swz a bijection on d's bits 1..3 both for rows of equal d mod 2 (128-byte lines)
// and of equal d mod 4 (256-byte lines)
__host__ __device__ __forceinline__ int pa_v_swz(int d) { return ((d >> 2) & 1) | ((((d >> 1) ^ (d >> 3)) & 1) << 1); }
__host__ __device__ __forceinline__ int pa_v_off(int d, int p) { return 2 * PA_PART + d * 64 + ((p ^ pa_v_swz(d)) << 4); }
// the key at position q of a V^T row: the order in which a lane holds the probabilities of its
// row after the logits MFMA (lane half lh holds keys 8i + 4lh + (0..3)); the B operand of k step
// kk takes positions 16 kk + 8 lh + (0..7)
__host__ __device__ __forceinline__ int pa_v_key(int q) {
  return 16 * (q >> 4) + 8 * ((q >> 2) & 1) + 4 * ((q >> 3) & 1) + (q & 3);
}
// q fragments: (kv head, 32-row tile, k step, hi/lo) is one 1 KB block; lane 32 lh + r holds
// Q[32 tile + r][16 ks + 8 lh .. +7], the B operand of v_mfma_f32_32x32x16_f16
__host__ __device__ __forceinline__ size_t pa_qf_index(int kvh, int ntiles, int row, int d, int lo) {
  return ((((size_t)kvh * ntiles + (row >> 5)) * PA_KS + (d >> 4)) * 2 + lo) * 512 +
         ((((d >> 3) & 1) << 5) | (row & 31)) * 8 + (d & 7);
}

// ---- the layer's K/V writer ----------------------------------------------------------------
// blocks [0, ab): the K/V cache slices (roped fp32 K, fp16 V [KV][P][256]) and the K hi / lo
//   image, one thread per (key, 4 dims of the first half and their rope partners); keys past P
//   (the last chunk's padding) get zero images;
// blocks [ab, ab + vb): the V^T image, one thread per (chunk, d, 8 key positions);
// the rest: q fragments, one thread per (row, 8 dims of the first half and their partners).
// from_cache: K and V from the cache slices (keys, values) instead of the q/k/v rows, which then
// hold only q; the cache is not written.
__global__ __launch_bounds__(256) void pa_writer_kernel(const _Float16* __restrict__ qkv, int ld, int koff, int voff,
                                                        const float* __restrict__ cosb, const float* __restrict__ sinb,
                                                        int P, int H, int KV, float q_scale, float* __restrict__ keys,
                                                        _Float16* __restrict__ values, char* __restrict__ img,
                                                        _Float16* __restrict__ qf, int nch, int ntiles, int ab,
                                                        int vb, int from_cache) {
  constexpr int half = PA_HD / 2;
  const int bid = blockIdx.x;
  if (bid < ab) {
    const long idx = (long)bid * 256 + threadIdx.x;
    if (idx >= (long)nch * PA_KCH * KV * 32) return;
    const int i = (int)(idx & 31) * 4;
    const int kvh = (int)((idx >> 5) % KV);
    const int p = (int)((idx >> 5) / KV);
    char* ck = img + ((size_t)kvh * nch + p / PA_KCH) * PA_CHUNK;
    const int r = p % PA_KCH;
    h4 h1, l1, h2, l2;
    if (p < P && from_cache) {
      const float* kc = keys + ((size_t)kvh * P + p) * PA_HD;
      const f4 o1 = *reinterpret_cast<const f4*>(kc + i), o2 = *reinterpret_cast<const f4*>(kc + i + half);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 hv, lv;
        split_f32(o1[e], hv, lv);
        h1[e] = hv;
        l1[e] = lv;
        split_f32(o2[e], hv, lv);
        h2[e] = hv;
        l2[e] = lv;
      }
    } else if (p < P) {
      const _Float16* kr = qkv + (size_t)p * ld + koff + (size_t)kvh * PA_HD;
      const _Float16* vr = qkv + (size_t)p * ld + voff + (size_t)kvh * PA_HD;
      const f4 c = *reinterpret_cast<const f4*>(cosb + (size_t)p * half + i);
      const f4 sn = *reinterpret_cast<const f4*>(sinb + (size_t)p * half + i);
      const h4 a = *reinterpret_cast<const h4*>(kr + i), b = *reinterpret_cast<const h4*>(kr + i + half);
      f4 o1, o2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x1 = h2f(a[e]), x2 = h2f(b[e]);
        o1[e] = x1 * c[e] - x2 * sn[e];
        o2[e] = x2 * c[e] + x1 * sn[e];
        _Float16 hv, lv;
        split_f32(o1[e], hv, lv);
        h1[e] = hv;
        l1[e] = lv;
        split_f32(o2[e], hv, lv);
        h2[e] = hv;
        l2[e] = lv;
      }
      float* ko = keys + ((size_t)kvh * P + p) * PA_HD;
      _Float16* vo = values + ((size_t)kvh * P + p) * PA_HD;
      *reinterpret_cast<f4*>(ko + i) = o1;
      *reinterpret_cast<f4*>(ko + i + half) = o2;
      *reinterpret_cast<h4*>(vo + i) = *reinterpret_cast<const h4*>(vr + i);
      *reinterpret_cast<h4*>(vo + i + half) = *reinterpret_cast<const h4*>(vr + i + half);
    } else {
      h1 = l1 = h2 = l2 = (h4){0, 0, 0, 0};
    }
    const int i2 = i + half;
    *reinterpret_cast<h4*>(ck + pa_k_off(r, i >> 3) + (i & 7) * 2) = h1;
    *reinterpret_cast<h4*>(ck + PA_PART + pa_k_off(r, i >> 3) + (i & 7) * 2) = l1;
    *reinterpret_cast<h4*>(ck + pa_k_off(r, i2 >> 3) + (i2 & 7) * 2) = h2;
    *reinterpret_cast<h4*>(ck + PA_PART + pa_k_off(r, i2 >> 3) + (i2 & 7) * 2) = l2;
  } else if (bid < ab + vb) {
    const long idx = (long)(bid - ab) * 256 + threadIdx.x;
    if (idx >= (long)KV * nch * PA_HD * 4) return;
    const int pp = (int)(idx & 3), d = (int)((idx >> 2) & (PA_HD - 1));
    const long rest = idx >> 10;
    const int ch = (int)(rest % nch), kvh = (int)(rest / nch);
    h8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = ch * PA_KCH + pa_v_key(8 * pp + j);
      v[j] = key >= P     ? (_Float16)0
             : from_cache ? values[((size_t)kvh * P + key) * PA_HD + d]
                          : qkv[(size_t)key * ld + voff + (size_t)kvh * PA_HD + d];
    }
    *reinterpret_cast<h8*>(img + ((size_t)kvh * nch + ch) * PA_CHUNK + pa_v_off(d, pp)) = v;
  } else {
    const long idx = (long)(bid - ab - vb) * 256 + threadIdx.x;
    if (idx >= (long)KV * ntiles * 512) return;
    const int l32 = (int)(idx & 31), g = (int)((idx >> 6) & 7) * 2 + (int)((idx >> 5) & 1);
    const int tile = (int)((idx >> 9) % ntiles), kvh = (int)((idx >> 9) / ntiles);
    const int grp = H / KV, row = 32 * tile + l32, d = 8 * g;
    h8 hi1, lo1, hi2, lo2;
    if (row < P * grp) {
      const int hl = row / P, t = row % P, h = kvh * grp + hl;
      const _Float16* qr = qkv + (size_t)t * ld + (size_t)h * PA_HD + d;
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
    *reinterpret_cast<h8*>(qf + pa_qf_index(kvh, ntiles, row, d, 0)) = hi1;
    *reinterpret_cast<h8*>(qf + pa_qf_index(kvh, ntiles, row, d, 1)) = lo1;
    *reinterpret_cast<h8*>(qf + pa_qf_index(kvh, ntiles, row, d + half, 0)) = hi2;
    *reinterpret_cast<h8*>(qf + pa_qf_index(kvh, ntiles, row, d + half, 1)) = lo2;
  }
}

// ---- the attention --------------------------------------------------------------------------
__device__ __forceinline__ void pa_lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS accesses; DMA not waited
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void pa_vm_wait0() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | 0xF00);  // vmcnt(0)
  asm volatile("" ::: "memory");
}
// 16 bytes per lane from the buffer into LDS at lds + 16 lane (device pass only: in the host
// pass the builtin drops the kernel's launch stub)
__device__ __forceinline__ void pa_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
#endif
}
// the XCD this wave runs on
__device__ __forceinline__ int pa_xcc() {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return (int)(x & 7u);
}
// max / sum of a value and its copy in lane l ^ 32 (one row-swap instruction), the same in both
__device__ __forceinline__ float pa_xor32_max(float v) {
  const unsigned b = __float_as_uint(v);
  const auto s = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float pa_xor32_sum(float v) {
  const unsigned b = __float_as_uint(v);
  const auto s = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

__global__ __launch_bounds__(PA_NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void pa_attn_kernel(const PaArgs a) {
  // one LDS object: with separate objects the compiler tags each access with its object and, as
  // the chunk DMA and the chunk reads name the same one, waits for the DMA in flight (the next
  // chunk's) before every chunk's first read
  __shared__ __attribute__((aligned(16))) char lds[2 * PA_CHUNK + PA_MAXCH * PA_KCH * 4 + (PA_MAXCH + 4) * 4];
  char* sbuf = lds;                                                     // two chunk buffers
  float* smask = reinterpret_cast<float*>(lds + 2 * PA_CHUNK);          // the mask of every key
  int* slist = reinterpret_cast<int*>(lds + 2 * PA_CHUNK + PA_MAXCH * PA_KCH * 4);
  // slist: the workgroup's chunks; [PA_MAXCH] their count; [PA_MAXCH + 1] the last-arrival flag
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar DMA offsets)
  const int l32 = lane & 31, lh = lane >> 5;
  const int kvh = blockIdx.y, S = a.nsplit;
  // workgroup g runs on XCD g mod 8 (round-robin dispatch): the S splits of row block b sit on one
  // XCD, at slots S (b / 8) + s of XCD b mod 8, so they share that XCD's L2 for q
  const int gslot = (int)blockIdx.x >> 3;
  const int s = gslot % S;
  const int b = 8 * (gslot / S) + ((int)blockIdx.x & 7);
  if (b >= a.nrb) return;

  // ---- the mask in LDS, this split's chunks -------------------------------------------------
  // every load in flight before the first wait: the mask's, then q's (needed at the first chunk)
  const int nk = a.nch * PA_KCH;
  constexpr int MPT = PA_MAXCH * PA_KCH / PA_NT;  // mask values per thread
  float mv[MPT];
#pragma unroll
  for (int i = 0; i < MPT; ++i) {
    const int k = tid + PA_NT * i;
    mv[i] = k < a.P ? (a.mask ? load_global(a.mask + k) : 0.f) : -INFINITY;
  }
  // this wave's q: 32 rows x 256 dims, hi and lo
  const int ntiles = 4 * a.nrb, tile = 4 * b + w;
  h8 qh[PA_KS], ql[PA_KS];
  {
    const h8* qb = reinterpret_cast<const h8*>(a.qf + ((size_t)kvh * ntiles + tile) * PA_KS * 2 * 512) + lane;
#pragma unroll
    for (int ks = 0; ks < PA_KS; ++ks) {
      qh[ks] = load_global(qb + (2 * ks) * 64);
      ql[ks] = load_global(qb + (2 * ks + 1) * 64);
    }
  }
#pragma unroll
  for (int i = 0; i < MPT; ++i)
    if (tid + PA_NT * i < nk) smask[tid + PA_NT * i] = mv[i];
  __syncthreads();
  if (w == 0) {
    bool valid = false;
    if (lane < a.nch) {
      const f4* mk = reinterpret_cast<const f4*>(smask + lane * PA_KCH);
#pragma unroll
      for (int i = 0; i < PA_KCH / 4; ++i) {
        const f4 v = mk[i];
        valid = valid || v[0] > -1e9f || v[1] > -1e9f || v[2] > -1e9f || v[3] > -1e9f;
      }
    }
    uint64_t vm = __ballot(valid);
    const bool skip = !a.noskip && vm != 0;
    // no valid key at all: the splits cover every chunk and compute it (the softmax of the
    // masked logits, as the reference computes it)
    if (vm == 0) vm = a.nch >= 64 ? ~0ull : ((1ull << a.nch) - 1);
    const int n = __popcll(vm);
    const bool isv = (vm >> lane) & 1;
    const int rank = __popcll(vm & ((1ull << lane) - 1));
    const int t0 = (int)((long)n * s / S), t1 = (int)((long)n * (s + 1) / S);
    const uint64_t st0 = __ballot(isv && rank == t0), st1 = __ballot(isv && rank == t1);
    const int c0 = s == 0 ? 0 : (st0 ? __ffsll((unsigned long long)st0) - 1 : a.nch);
    const int c1 = s + 1 == S ? a.nch : (st1 ? __ffsll((unsigned long long)st1) - 1 : a.nch);
    const bool take = lane >= c0 && lane < c1 && (!skip || isv);
    const uint64_t tm = __ballot(take);
    if (take) slist[__popcll(tm & ((1ull << lane) - 1))] = lane;
    if (lane == 0) slist[PA_MAXCH] = __popcll(tm);
  }
  __syncthreads();
  const int nl = __builtin_amdgcn_readfirstlane(slist[PA_MAXCH]);

  // ---- chunk DMA: 48 KB = 12 x 1 KB per wave ---------------------------------------------------
  const __amdgpu_buffer_rsrc_t rimg = dev_rsrc(a.img + (size_t)kvh * a.nch * PA_CHUNK, (uint32_t)(a.nch * PA_CHUNK));
  // the first chunk; later chunks go out during the previous one's logits.  Past the list
  // (j >= nl) the same instructions read past the image (zeros) into the free buffer, so that the
  // loop issues its DMA unconditionally (a branch around it made the compiler wait for the DMA
  // before the chunk's first LDS read).
  if (nl > 0) {
    const int c = __builtin_amdgcn_readfirstlane(slist[0]);  // uniform: a scalar offset
#pragma unroll
    for (int i = 0; i < PA_CHUNK / (4 * 1024); ++i) {
      const int blk = 4 * i + w;
      pa_dma16(rimg, sbuf + blk * 1024, lane * 16, c * PA_CHUNK + blk * 1024);
    }
  }


  f16v o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  float m_run = -1e30f, l_run = 0.f;

  const int ky = lh ^ (l32 & 15);  // piece 2 ks + lh of row l32 sits in slot (2 ks) ^ ky
  const int vsw = pa_v_swz(l32);
  const int voff0 = 2 * PA_PART + l32 * 64 + ((lh ^ vsw) << 4);
  const int voff1 = 2 * PA_PART + l32 * 64 + (((2 + lh) ^ vsw) << 4);

  // chunk j's logits S^T[key][row] with the mask added: lane holds keys 8 (e / 4) + 4 lh + e % 4
  // of row l32; cmax is the row's chunk max (this lane's 16 keys and lane l ^ 32's)
  float sv[16], cmax;
  auto logits = [&](int j) __attribute__((always_inline)) {
    pa_vm_wait0();     // this wave's part of chunk j (and, at j = 0, its q)
    pa_lds_barrier();  // every wave's part has landed; every wave is done with chunk j - 1
    // chunk j + 1's DMA goes out one instruction per k step below: issued in one burst, the busy
    // memory pipeline held the wave at issue while its MFMAs idled
    const int cn = __builtin_amdgcn_readfirstlane(j + 1 < nl ? slist[j + 1] : a.nch);
    char* dnext = sbuf + ((j + 1) & 1) * PA_CHUNK;
    const char* B = sbuf + (j & 1) * PA_CHUNK;
    const int c = __builtin_amdgcn_readfirstlane(slist[j]);
    f16v acc0, acc1, acc2;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc0[e] = acc1[e] = acc2[e] = 0.f;
    const char* kb = B + l32 * 512;
    h8 kf[2][2];
    kf[0][0] = *reinterpret_cast<const h8*>(kb + (ky << 4));
    kf[0][1] = *reinterpret_cast<const h8*>(kb + PA_PART + (ky << 4));
#pragma unroll
    for (int ks = 0; ks < PA_KS; ++ks) {
      if (ks + 1 < PA_KS) {
        const int off = ((2 * (ks + 1)) ^ ky) << 4;
        kf[(ks + 1) & 1][0] = *reinterpret_cast<const h8*>(kb + off);
        kf[(ks + 1) & 1][1] = *reinterpret_cast<const h8*>(kb + PA_PART + off);
      }
      __builtin_amdgcn_sched_barrier(0);
      const h8 kh = kf[ks & 1][0], kl = kf[ks & 1][1];
      acc0 = mfma32x32x16(kh, qh[ks], acc0);
      acc1 = mfma32x32x16(kh, ql[ks], acc1);
      acc2 = mfma32x32x16(kl, qh[ks], acc2);
      if (ks < PA_CHUNK / (4 * 1024)) {
        __builtin_amdgcn_sched_barrier(0);
        pa_dma16(rimg, dnext + (4 * ks + w) * 1024, lane * 16, cn * PA_CHUNK + (4 * ks + w) * 1024);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const float* mk = smask + c * PA_KCH + 4 * lh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f4 mq = *reinterpret_cast<const f4*>(mk + 8 * i);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 4 * i + r;
        sv[e] = (acc2[e] + acc1[e]) + acc0[e] + mq[r];
      }
    }
    cmax = sv[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) cmax = fmaxf(cmax, sv[e]);
    cmax = pa_xor32_max(cmax);
  };
  // probabilities exp(s - m_new) in fp16, l, and O^T[d][row] += V^T . P^T over the chunk's two
  // 16-key steps (O already scaled to m_new)
  auto softmax_pv = [&](int j, float m_new, float alpha) __attribute__((always_inline)) {
    const char* B = sbuf + (j & 1) * PA_CHUNK;
    float psum = 0.f;
    h8 pb[2];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float ex = exp_hw(sv[e] - m_new);
      psum += ex;
      pb[e >> 3][e & 7] = f2h(ex);
    }
    psum = pa_xor32_sum(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const char* vb = B + (kk ? voff1 : voff0);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const h8 vf = *reinterpret_cast<const h8*>(vb + dt * 32 * 64);
        o[dt] = mfma32x32x16(vf, pb[kk], o[dt]);
      }
    }
  };
  // Online softmax with a lazy running max: it moves only when a chunk's max exceeds it by more
  // than 8, so p = exp(s - m_run) stays below e^8 (fp16-safe).  At the first chunk O is zero and
  // needs no rescale; a later move (rare) leaves the loop, rescales O and comes back, so that the
  // loop itself holds no multiply of the accumulators.
  int j = 0;
  while (j < nl) {
    bool moved = false;
    for (; j < nl; ++j) {
      logits(j);
      const bool grow = cmax > m_run + 8.0f;
      if (j > 0 && __any(grow)) {
        moved = true;
        break;
      }
      const float m_new = grow ? cmax : m_run;
      softmax_pv(j, m_new, exp_hw(m_run - m_new));
    }
    if (!moved) break;
    const float m_new = cmax > m_run + 8.0f ? cmax : m_run;
    const float alpha = exp_hw(m_run - m_new);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
    softmax_pv(j, m_new, alpha);
    ++j;
  }

  // ---- output ----------------------------------------------------------------------------------
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  const int grp = a.H / a.KV;
  // The wave's 32 rows x 256 dims in fp16 through LDS (the chunk buffers are free once the last
  // DMA has landed): lane value e of d tile dt is O[row l32][32 dt + 8 (e / 4) + 4 lh + e % 4];
  // written to a [32][264] half tile, then stored a row's 512 bytes per 32 lanes, not 8 bytes
  // of 32 different rows per instruction.
  constexpr int ORS = PA_HD + 8;  // halfs per staged row
  _Float16* stg = reinterpret_cast<_Float16*>(sbuf) + w * 32 * ORS;
  auto stage_out = [&](auto&& val) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = f2h(val(dt, 4 * i + r));
        *reinterpret_cast<h4*>(stg + l32 * ORS + 32 * dt + 8 * i + 4 * lh) = v;
      }
  };
  auto write_out = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int r = 2 * it + lh;
      const int row = PA_ROWS * b + 32 * w + r;
      const h8 v = *reinterpret_cast<const h8*>(stg + r * ORS + 8 * l32);
      if (row < a.rows) {
        const int hl = row / a.P, t = row % a.P;
        *reinterpret_cast<h8*>(a.out + (size_t)t * a.out_ld + (size_t)(kvh * grp + hl) * PA_HD + 8 * l32) = v;
      }
    }
  };
  if (S == 1) {
    pa_vm_wait0();  // the last (past the list) DMA into the chunk buffers
    __syncthreads();
    stage_out([&](int dt, int e) { return o[dt][e] * inv; });
    write_out();
    return;
  }
  // the split's O / l in fp16 (lane-local order) and its (m, l), through to the memory side
  h8 ph[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) ph[dt][i2][jj] = f2h(o[dt][8 * i2 + jj] * inv);
  const size_t rb_id = (size_t)kvh * a.nrb + b;
  const __amdgpu_buffer_rsrc_t rpart = dev_rsrc(a.part + rb_id * S * 4 * PA_WAVE_PART, (uint32_t)(S * 4 * PA_WAVE_PART * 2));
  const __amdgpu_buffer_rsrc_t rml = dev_rsrc(a.part_ml + rb_id * S * PA_ROWS * 2, (uint32_t)(S * PA_ROWS * 8));
  auto part_off = [&](int sp, int dt, int i2) __attribute__((always_inline)) {
    return (((sp * 4 + w) * 16 + dt * 2 + i2) * 64 + lane) * 16;
  };
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2) store_dev<h8>(rpart, part_off(s, dt, i2), ph[dt][i2]);
  if (lh == 0) store_dev<f2>(rml, ((s * PA_ROWS) + 32 * w + l32) * 8, (f2){m_run, l_run});
  wait_all_memory();  // the stores are complete before the arrival
  __syncthreads();
  if (tid == 0) {
    // arrivals in the low half of the counter; the high half counts splits that ran on another XCD
    // than the launch order places them on (then the last reads at device scope, not from its L2)
    unsigned* ctr = a.ctr + rb_id;
    const bool off = pa_xcc() != ((int)blockIdx.x & 7);
    const unsigned old = counter_add(ctr, off ? 0x10001u : 1u);
    const bool last = (old & 0xFFFFu) == (unsigned)(S - 1);
    if (last) counter_reset(ctr);
    slist[PA_MAXCH + 1] = last ? 1 | (off || (old >> 16) || a.dev_combine ? 2 : 0) : 0;
  }
  __syncthreads();
  const int fl = __builtin_amdgcn_readfirstlane(slist[PA_MAXCH + 1]);
  if (!fl) return;
  // ---- the last split of the row block: combine every split in split order ----
  // Every split's (m, l) and O / l are read back, this one's included, so the arithmetic is the
  // same whichever split arrives last.  The splits wrote them through to the memory side; with
  // every split on this XCD the reads hit its L2 (sc0: past this CU's L1), else device scope.
  float acc[8][16];
  float winv = 0.f;
  auto combine = [&](auto aux) __attribute__((always_inline)) {
    constexpr int AUX = decltype(aux)::value;
    // every split's (m, l), then the first two splits' fragments, all in flight at once; each
    // later split's fragments go out while the one before is accumulated
    f2 ml[PA_MAXS];
#pragma unroll
    for (int sp = 0; sp < PA_MAXS; ++sp)
      if (sp < S) ml[sp] = load_dev<f2, AUX>(rml, ((sp * PA_ROWS) + 32 * w + l32) * 8);
    h8 v[2][8][2];
    auto fetch = [&](int sp, int bb) __attribute__((always_inline)) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) v[bb][dt][i2] = load_dev<h8, AUX>(rpart, part_off(sp, dt, i2));
    };
    fetch(0, 0);
    if (S > 1) fetch(1, 1);
    float ll[PA_MAXS];
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < PA_MAXS; ++sp)
      if (sp < S) M = fmaxf(M, ml[sp][0]);
    float wsum = 0.f;
#pragma unroll
    for (int sp = 0; sp < PA_MAXS; ++sp) {
      if (sp < S) {
        ll[sp] = ml[sp][1] * exp_hw(ml[sp][0] - M);  // the split's weight
        wsum += ll[sp];
      }
    }
    winv = wsum > 0.f ? 1.0f / wsum : 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;
    // the splits in order, each split's 16 fragments (O / l of every d of this lane's row)
    // accumulated with the split's weight
#pragma unroll
    for (int sp = 0; sp < PA_MAXS; ++sp) {
      if (sp < S) {
        const float ws = ll[sp];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[dt][e] += ws * h2f(v[sp & 1][dt][e >> 3][e & 7]);
        if (sp + 2 < S) fetch(sp + 2, sp & 1);
      }
    }
  };
  if (fl & 2) combine(std::integral_constant<int, 16>{});
  else combine(std::integral_constant<int, 1>{});
  stage_out([&](int dt, int e) { return acc[dt][e] * winv; });
  write_out();
}

}  // namespace

bool pa_supported(int hd, int P, int H, int KV) {
  return hd == PA_HD && P > 0 && P <= PA_MAXCH * PA_KCH && KV > 0 && H % KV == 0;
}

PaPlan pa_plan(int P, int H, int KV) {
  PaPlan p{};
  p.nch = (P + PA_KCH - 1) / PA_KCH;
  p.nrb = (P * (H / KV) + PA_ROWS - 1) / PA_ROWS;
  const int cus = std::max(device_cus(), 1);
  p.nsplit = std::max(1, std::min(std::min(PA_MAXS, p.nch), cus / std::max(1, KV * p.nrb)));
  p.img_bytes = (size_t)KV * p.nch * PA_CHUNK;
  p.qf_halfs = (size_t)KV * p.nrb * PA_ROWS * PA_HD * 2;
  p.part_halfs = (size_t)KV * p.nrb * p.nsplit * 4 * PA_WAVE_PART;
  p.ml_floats = (size_t)KV * p.nrb * p.nsplit * PA_ROWS * 2;
  p.counters = (size_t)KV * p.nrb;
  return p;
}

int pa_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin, int P, int H,
                     int KV, float q_scale, float* keys, _Float16* values, const PaPlan& plan, char* img, _Float16* qf,
                     int from_cache, hipStream_t st) {
  MLCV_REQUIRE(pa_supported(PA_HD, P, H, KV) && qkv && cos && sin && keys && values && img && qf,
               "prefill attention writer arguments");
  MLCV_REQUIRE(ld % 8 == 0 && koff % 8 == 0 && voff % 8 == 0, "q/k/v row layout must be 16-byte aligned");
  MLCV_REQUIRE(((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(keys) |
                 reinterpret_cast<uintptr_t>(values) | reinterpret_cast<uintptr_t>(cos) |
                 reinterpret_cast<uintptr_t>(sin) | reinterpret_cast<uintptr_t>(img) |
                 reinterpret_cast<uintptr_t>(qf)) & 15) == 0, "prefill attention writer buffers must be 16-byte aligned");
  const int ntiles = 4 * plan.nrb;
  const long at = (long)plan.nch * PA_KCH * KV * 32, vt = (long)KV * plan.nch * PA_HD * 4, qt = (long)KV * ntiles * 512;
  const int ab = (int)((at + 255) / 256), vb = (int)((vt + 255) / 256), qb = (int)((qt + 255) / 256);
  pa_writer_kernel<<<(unsigned)(ab + vb + qb), 256, 0, st>>>(qkv, ld, koff, voff, cos, sin, P, H, KV, q_scale, keys,
                                                            values, img, qf, plan.nch, ntiles, ab, vb, from_cache);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int pa_attn_launch(const PaArgs& a, hipStream_t st) {
  MLCV_REQUIRE(pa_supported(PA_HD, a.P, a.H, a.KV), "prefill attention shape");
  MLCV_REQUIRE(a.rows == a.P * (a.H / a.KV) && a.nrb == (a.rows + PA_ROWS - 1) / PA_ROWS &&
                   a.nch == (a.P + PA_KCH - 1) / PA_KCH,
               "prefill attention plan does not match the shape");
  MLCV_REQUIRE(a.nsplit >= 1 && a.nsplit <= PA_MAXS && a.nsplit <= a.nch, "prefill attention splits");
  MLCV_REQUIRE(a.qf && a.img && a.out && a.out_ld >= a.H * PA_HD, "prefill attention buffers");
  MLCV_REQUIRE(a.nsplit == 1 || (a.part && a.part_ml && a.ctr), "prefill attention split workspace");
  const dim3 grid((unsigned)(8 * a.nsplit * ((a.nrb + 7) / 8)), (unsigned)a.KV);
  pa_attn_kernel<<<grid, PA_NT, 0, st>>>(a);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
