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
// from LDS, B = Q^T held in registers), which leaves each lane with 4 keys of one
// query row per 16-key tile -- the B-operand layout of O^T[d][row] = V^T[d][key] .
// P^T[key][row] once V^T is read in the same key order, so P never leaves registers.
//
// Work split: a workgroup owns 64 query rows and one key range.  Key splits
// 0..n-2 cover the prefix cache, the last split (when there is a suffix block) the
// suffix keys, so every workgroup runs one straight-line loader: the prefix loader
// reads the cached roped fp32 K, the suffix loader ropes the raw fp16 k on the fly.
// Keys past the range are clamped to a valid row and masked with -inf.
//
// LDS: K as hi/lo fp16 [key][d] rows (row pitch HD+8 halfs: the 16 rows one MFMA
// A read touches start on distinct banks); V transposed [d][key] with a pitch of 36
// halfs, written as packed key pairs (ds_write_b32) -- lanes of one store cover 16
// key pairs x 4 dims and a wave's MFMA reads of 16 d-rows land on disjoint banks.
//
// This header holds the attention's device code (chunk loaders, LDS layout, the per-workgroup
// body attn_block and the split combine combine_row) so that the standalone attention kernel
// and the persistent step kernel run the same code.
#pragma once

#include "kernels.h"

// cache policy of the q fragments written by the previous launch (the persistent step, which
// writes them in the same launch, always reads them at device scope)
#ifndef MLCV_ATTN_Q_AUX
#define MLCV_ATTN_Q_AUX 16
#endif
constexpr int ATTN_Q_AUX = MLCV_ATTN_Q_AUX;
// cache policy of the split combine's partial loads when the attention wrote them in an
// earlier launch (the persistent step's combine, in the same launch, reads at device scope):
// device scope; plain loads measure the same on the current kernels (813.0 vs 813.1 us)
#ifndef MLCV_COMB_AUX
#define MLCV_COMB_AUX 16
#endif
constexpr int COMB_AUX = MLCV_COMB_AUX;

// timeline stamps of the trace build of the persistent step (empty otherwise)
#ifndef ATTN_STAMP
#define ATTN_STAMP(k) \
  do {                \
  } while (0)
#endif

namespace mlcv {
namespace {
constexpr int KCH = 32;        // keys per chunk
constexpr int ROWS = 64;       // query rows per workgroup (4 waves x 16)
// halfs per V^T row (a multiple of 4, at least KCH).  18 dwords: the b32 key-pair stores of
// a half wave (two d groups 8 rows apart, 16 dwords each) start 16 banks apart, and the b64
// MFMA reads of 16 consecutive d rows cover 32 distinct banks -- neither conflicts on 32 banks
// (40 halfs: both 2-way).  Against 40: step -6 us, prefill -36 us, results bit-identical.
constexpr int VLD = KCH + 4;
static_assert(VLD % 4 == 0 && VLD >= KCH, "V^T rows hold a chunk's keys in 8-byte pieces");
constexpr int NT = 256;        // threads per workgroup (4 waves, one 16-row query tile each)
static_assert(ROWS == ATTN_ROWS && KCH == ATTN_KCH, "the planner's rows and chunk (plan.h)");

template <int HD>
struct AttnSmem {
  static constexpr int KLD = HD + 8;  // halfs per K row
  _Float16 kh[KCH * KLD];
  _Float16 kl[KCH * KLD];
  _Float16 vt[HD * VLD];
  float msk[KCH];
};

// One 32-key chunk of prefix K/V as a byte image of AttnSmem (K split hi/lo, V
// transposed, the mask), rounded up to whole passes of 256 threads x 16 bytes.  Images
// are built once per call by attn_img_prep_kernel; the attention kernel copies them into
// LDS with 16-byte loads and stores (no conversion on the critical path).
template <int HD>
constexpr int img_bytes() {
  return ((int)sizeof(AttnSmem<HD>) + NT * 16 - 1) / (NT * 16) * (NT * 16);
}

// One key chunk in registers between its global loads and its LDS stores.
//   K item (key j, dims dp..dp+7 and dp+HD/2..+7) as fp32 (the RoPE pair of the suffix
//   loader is one item); V item (keys 2jp, 2jp+1; dims d0..d0+7).  Items past the
//   chunk's item count are repeats of earlier ones (identical LDS stores).
template <int HD, int NTH = NT>
struct ChunkRegs {
  static constexpr int HALF = HD / 2;
  static constexpr int KITEMS = KCH * (HALF / 8);
  static constexpr int VITEMS = (KCH / 2) * (HD / 8);
  static constexpr int NK = (KITEMS + NTH - 1) / NTH;
  static constexpr int NV = (VITEMS + NTH - 1) / NTH;
  float k[NK][16];
  h8 v[NV][2];
  float msk;  // the mask value as loaded; keys past the range get -inf when stored (mok)
  bool mok;
};

template <int HD, int NTH>
__device__ __forceinline__ void kitem(int i, int tid, int& j, int& dp) {
  constexpr int HALF = HD / 2;
  const int it = (tid + NTH * i) % ChunkRegs<HD, NTH>::KITEMS;
  j = it / (HALF / 8);
  dp = (it % (HALF / 8)) * 8;
}
template <int HD, int NTH>
__device__ __forceinline__ void vitem(int i, int tid, int& jp, int& d0) {
  const int it = (tid + NTH * i) % ChunkRegs<HD, NTH>::VITEMS;
  jp = it % (KCH / 2);
  d0 = (it / (KCH / 2)) * 8;
}

__device__ __forceinline__ void cvt8(const h8 x, float* o) {
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = h2f(x[e]);
}
template <int AUX>
__device__ __forceinline__ void ld8f(__amdgpu_buffer_rsrc_t r, int byte_off, float* o) {
  const f4 a = load_dev<f4, AUX>(r, byte_off), b = load_dev<f4, AUX>(r, byte_off + 16);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = a[e];
    o[e + 4] = b[e];
  }
}

// prefix keys [c0, c0+32) of this split (cached, roped; fp32 or fp16), clamped below kend
template <int HD, bool KF32, int NTH>
__device__ __forceinline__ void load_prefix(ChunkRegs<HD, NTH>& r, const AttnArgs& a, int kvh, int c0, int kend, int tid) {
  constexpr int HALF = HD / 2;
  // this kv head's keys and values (element offsets below are within one head: < 2^31 bytes)
  const size_t head = (size_t)kvh * a.Sp * HD, hbytes = (size_t)a.Sp * HD;
  const __amdgpu_buffer_rsrc_t rk = dev_rsrc(static_cast<const char*>(a.kp) + head * (KF32 ? 4 : 2),
                                             (uint32_t)(hbytes * (KF32 ? 4 : 2)));
  const __amdgpu_buffer_rsrc_t rv = dev_rsrc(a.vp + head, (uint32_t)(hbytes * 2));
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD, NTH>::NK; ++i) {
    int j, dp;
    kitem<HD, NTH>(i, tid, j, dp);
    const int off = min(c0 + j, kend - 1) * HD + dp;
    if constexpr (KF32) {
      ld8f<KV_AUX>(rk, off * 4, r.k[i]);
      ld8f<KV_AUX>(rk, (off + HALF) * 4, r.k[i] + 8);
    } else {
      cvt8(load_dev<h8, KV_AUX>(rk, off * 2), r.k[i]);
      cvt8(load_dev<h8, KV_AUX>(rk, (off + HALF) * 2), r.k[i] + 8);
    }
  }
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD, NTH>::NV; ++i) {
    int jp, d0;
    vitem<HD, NTH>(i, tid, jp, d0);
    r.v[i][0] = load_dev<h8, KV_AUX>(rv, (min(c0 + 2 * jp, kend - 1) * HD + d0) * 2);
    r.v[i][1] = load_dev<h8, KV_AUX>(rv, (min(c0 + 2 * jp + 1, kend - 1) * HD + d0) * 2);
  }
  // a global-space load whose value is untouched until store time: a flat load, or
  // arithmetic on the loaded value here, would make the compiler wait for every load in
  // flight (this chunk's and the previous one's) before the loader returns
  const int kj = c0 + (tid & (KCH - 1));
  r.msk = a.mask ? load_global(a.mask + min(kj, kend - 1)) : 0.f;
  r.mok = kj < kend;
}

// Suffix keys [c0, c0+32): the raw fp16 k of the suffix rows and their rope tables stay
// in registers as loaded (no arithmetic on in-flight loads), roped at store time.
template <int HD, int NTH = NT>
struct SufRegs {
  static constexpr int NK = ChunkRegs<HD, NTH>::NK, NV = ChunkRegs<HD, NTH>::NV;
  h8 x1[NK], x2[NK];
  f4 c[NK][2], s[NK][2];
  h8 v[NV][2];
  float msk;
  bool mok;
};

template <int HD, bool ROPE, int NTH>
__device__ __forceinline__ void load_suffix(SufRegs<HD, NTH>& r, const AttnArgs& a, int kvh, int c0, int kend, int tid) {
  constexpr int HALF = HD / 2;
#pragma unroll
  for (int i = 0; i < SufRegs<HD, NTH>::NK; ++i) {
    int j, dp;
    kitem<HD, NTH>(i, tid, j, dp);
    const int ts = min(c0 + j, kend - 1);
    const _Float16* kr = a.ks + (size_t)ts * a.ks_ld + (size_t)kvh * HD + dp;
    r.x1[i] = load_global(reinterpret_cast<const h8*>(kr));
    r.x2[i] = load_global(reinterpret_cast<const h8*>(kr + HALF));
    if constexpr (ROPE) {
      const f4* cp = reinterpret_cast<const f4*>(a.cos + (size_t)ts * HALF + dp);
      const f4* sp = reinterpret_cast<const f4*>(a.sin + (size_t)ts * HALF + dp);
      r.c[i][0] = load_global(cp);
      r.c[i][1] = load_global(cp + 1);
      r.s[i][0] = load_global(sp);
      r.s[i][1] = load_global(sp + 1);
    }
  }
#pragma unroll
  for (int i = 0; i < SufRegs<HD, NTH>::NV; ++i) {
    int jp, d0;
    vitem<HD, NTH>(i, tid, jp, d0);
    const _Float16* vb = a.vs + (size_t)kvh * HD + d0;
    r.v[i][0] = load_global(reinterpret_cast<const h8*>(vb + (size_t)min(c0 + 2 * jp, kend - 1) * a.vs_ld));
    r.v[i][1] = load_global(reinterpret_cast<const h8*>(vb + (size_t)min(c0 + 2 * jp + 1, kend - 1) * a.vs_ld));
  }
  r.msk = 0.f;
  r.mok = c0 + (tid & (KCH - 1)) < kend;
}

// suffix keys handed over roped in fp32 ([Ts][ks_ld], the qkv epilogue's output) and the
// suffix v: the prefix loader's chunk layout with the suffix row strides
// AUX: the cache policy (device scope when the suffix k/v were written in the same launch)
template <int HD, int AUX, int NTH>
__device__ __forceinline__ void load_suffix32(ChunkRegs<HD, NTH>& r, const AttnArgs& a, int kvh, int c0, int kend, int tid) {
  constexpr int HALF = HD / 2;
  // the previous kernel's output: device-scope loads
  const __amdgpu_buffer_rsrc_t rk = dev_rsrc(a.ks32, (uint32_t)kend * a.ks_ld * 4);
  const __amdgpu_buffer_rsrc_t rv = dev_rsrc(a.vs, (uint32_t)kend * a.vs_ld * 2);
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD, NTH>::NK; ++i) {
    int j, dp;
    kitem<HD, NTH>(i, tid, j, dp);
    const int off = min(c0 + j, kend - 1) * a.ks_ld + kvh * HD + dp;
    ld8f<AUX>(rk, off * 4, r.k[i]);
    ld8f<AUX>(rk, (off + HALF) * 4, r.k[i] + 8);
  }
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD, NTH>::NV; ++i) {
    int jp, d0;
    vitem<HD, NTH>(i, tid, jp, d0);
    r.v[i][0] = load_dev<h8, AUX>(rv, (min(c0 + 2 * jp, kend - 1) * a.vs_ld + kvh * HD + d0) * 2);
    r.v[i][1] = load_dev<h8, AUX>(rv, (min(c0 + 2 * jp + 1, kend - 1) * a.vs_ld + kvh * HD + d0) * 2);
  }
  r.msk = 0.f;
  r.mok = c0 + (tid & (KCH - 1)) < kend;
}

// rope the suffix keys (unless handed over roped) into the fp32 chunk layout
template <int HD, bool ROPE, int NTH>
__device__ __forceinline__ void rope_suffix(const SufRegs<HD, NTH>& in, ChunkRegs<HD, NTH>& r, bool roped) {
#pragma unroll
  for (int i = 0; i < SufRegs<HD, NTH>::NK; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x1 = h2f(in.x1[i][e]), x2 = h2f(in.x2[i][e]);
      if constexpr (ROPE) {
        const float c = in.c[i][e >> 2][e & 3], sn = in.s[i][e >> 2][e & 3];
        r.k[i][e] = roped ? x1 : x1 * c - x2 * sn;
        r.k[i][8 + e] = roped ? x2 : x2 * c + x1 * sn;
      } else {
        r.k[i][e] = x1;
        r.k[i][8 + e] = x2;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < SufRegs<HD, NTH>::NV; ++i) {
    r.v[i][0] = in.v[i][0];
    r.v[i][1] = in.v[i][1];
  }
  r.msk = in.msk;
  r.mok = in.mok;
}

// Workgroup barrier for LDS hand-off: waits for this wave's LDS accesses (lgkmcnt), not for
// its outstanding global loads, whose latency the prefetches hide.  The explicit wait and the
// empty asm statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt / expcnt not waited
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int HD, int NTH>
__device__ __forceinline__ void store_chunk(const ChunkRegs<HD, NTH>& r, AttnSmem<HD>& sm, int tid) {
  constexpr int KLD = AttnSmem<HD>::KLD, HALF = HD / 2;
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD, NTH>::NK; ++i) {
    int j, dp;
    kitem<HD, NTH>(i, tid, j, dp);
#pragma unroll
    for (int hpart = 0; hpart < 2; ++hpart) {
      h8 hi8, lo8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16 hi, lo;
        split_f32(r.k[i][8 * hpart + e], hi, lo);
        hi8[e] = hi;
        lo8[e] = lo;
      }
      *reinterpret_cast<h8*>(&sm.kh[j * KLD + dp + hpart * HALF]) = hi8;
      *reinterpret_cast<h8*>(&sm.kl[j * KLD + dp + hpart * HALF]) = lo8;
    }
  }
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD, NTH>::NV; ++i) {
    int jp, d0;
    vitem<HD, NTH>(i, tid, jp, d0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const h2 pair = {r.v[i][0][e], r.v[i][1][e]};
      *reinterpret_cast<h2*>(&sm.vt[(d0 + e) * VLD + 2 * jp]) = pair;
    }
  }
  if (tid < KCH) sm.msk[tid] = r.mok ? r.msk : -INFINITY;
}

// Q^T fragments of this lane's row: roped (fp32) unless already roped, scaled, split hi/lo.
// Loaded in one batch (QRaw), converted after the caller has issued its other loads.
// (in two halves of the load pairs, so the raw values of only one half are live at a time)
template <int HD>
struct QRaw {
  static constexpr int NPT = HD >= 64 ? HD / 64 : 1;      // load pairs (dims d, d + HD/2) in all
  static constexpr int NP = NPT > 1 ? NPT / 2 : 1;        // pairs per half
  static constexpr int NHALF = NPT > 1 ? 2 : 1;
  h8 x1[NP], x2[NP];
  f4 c[NP][2], s[NP][2];
};

template <int HD, bool ROPE>
__device__ __forceinline__ void load_q(const AttnArgs& a, int t, int h, int g, QRaw<HD>& r, int half) {
  constexpr int HALF = HD / 2;
  const _Float16* qr = a.q + (size_t)t * a.q_ld + (size_t)h * HD;
#pragma unroll
  for (int pi = 0; pi < QRaw<HD>::NP; ++pi) {
    const int p = half * QRaw<HD>::NP + pi;
    // HD >= 64: pair p covers dims d = 32p + 8g and d + HD/2 (k-steps p and p + HD/64);
    // HD < 64: one k-step of 32 dims, lanes past HD load a valid row and are zeroed later
    const int d = HD >= 64 ? 32 * p + 8 * g : min(8 * g, HD - 8);
    const bool first = HD >= 64 || d < HALF;
    const int dc = first ? d : d - HALF;
    r.x1[pi] = load_global(reinterpret_cast<const h8*>(qr + d));
    r.x2[pi] = load_global(reinterpret_cast<const h8*>(qr + (first ? d + HALF : d - HALF)));
    if constexpr (ROPE) {
      const f4* cp = reinterpret_cast<const f4*>(a.cos + (size_t)t * HALF + dc);
      const f4* sp = reinterpret_cast<const f4*>(a.sin + (size_t)t * HALF + dc);
      r.c[pi][0] = load_global(cp);
      r.c[pi][1] = load_global(cp + 1);
      r.s[pi][0] = load_global(sp);
      r.s[pi][1] = load_global(sp + 1);
    }
  }
}

template <int HD, bool ROPE>
__device__ __forceinline__ void make_q(const AttnArgs& a, const QRaw<HD>& r, int g, h8* qh, h8* ql, int half) {
  constexpr int NKS = (HD + 31) / 32, HALF = HD / 2;
  auto emit = [&](int ks, const float* v) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      _Float16 hi, lo;
      split_f32(v[e] * a.q_scale, hi, lo);
      qh[ks][e] = hi;
      ql[ks][e] = lo;
    }
  };
#pragma unroll
  for (int pi = 0; pi < QRaw<HD>::NP; ++pi) {
    const int p = half * QRaw<HD>::NP + pi;
    const int d = HD >= 64 ? 32 * p + 8 * g : 8 * g;
    const bool first = HD >= 64 || d < HALF;
    float o1[8], o2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x1 = h2f(r.x1[pi][e]), x2 = h2f(r.x2[pi][e]);
      if constexpr (ROPE) {
        const float c = r.c[pi][e >> 2][e & 3], sn = r.s[pi][e >> 2][e & 3];
        o1[e] = first ? x1 * c - x2 * sn : x1 * c + x2 * sn;
        o2[e] = x2 * c + x1 * sn;
      } else {
        o1[e] = x1;
        o2[e] = x2;
      }
    }
    if constexpr (HD >= 64) {
      emit(p, o1);
      emit(p + NKS / 2, o2);
    } else {
      if (d >= HD) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o1[e] = 0.f;
      }
      emit(0, o1);
    }
  }
}

// Combine the per-split partial softmax states of one query row with one wave: every
// partial load goes out at once (split indices past nsplit repeat a valid split with
// weight 0).  Lane s holds split s's statistics and normalized weight; each weight reaches
// the other lanes by one v_readlane where it is used, so no per-split arrays of uniform
// registers stay live (at 24 or 32 splits they spilled).
// COH: the partials were stored in this launch (device-scope loads); ST_DEV: the output is
// read in this launch too (device-scope stores), otherwise by later launches (plain stores)
template <int MAXS, bool COH, bool ST_DEV = COH>
__device__ __forceinline__ void combine_row(const AttnArgs& a, int kvh, int row, int lane) {
  static_assert(MAXS <= 64, "one split per lane");
  const int hd = a.hd;
  const int grp = a.H / a.KV;
  const int hl = row / a.Tq, t = row % a.Tq, h = kvh * grp + hl;
  const size_t pr0 = (size_t)kvh * a.nsplit * a.rpad + row;
  const int ns = a.nsplit;
  const int sl = min(lane, ns - 1);
  // the partials were written by the attention kernel just before: device-scope loads
  const uint32_t nrow = (uint32_t)a.KV * ns * a.rpad;
  const __amdgpu_buffer_rsrc_t rml = dev_rsrc(a.part_ml, nrow * 8), ro = dev_rsrc(a.part_o, nrow * hd * 2);
  const float m_l = load_dev<float, COH ? 16 : COMB_AUX>(rml, (int)((pr0 + (size_t)sl * a.rpad) * 8));
  const float l_l = load_dev<float, COH ? 16 : COMB_AUX>(rml, (int)((pr0 + (size_t)sl * a.rpad) * 8 + 4));
  // the O loads of the first 256 dims go out with the m / l loads (partials: fp16 O_s / l_s)
  const int d0 = min(lane * 4, hd - 4);
  h4 o[MAXS];
#pragma unroll
  for (int s = 0; s < MAXS; ++s) o[s] = load_dev<h4, COH ? 16 : COMB_AUX>(ro, (int)(((pr0 + (size_t)min(s, ns - 1) * a.rpad) * hd + d0) * 2));
  // out = sum_s w_s l_s (O_s / l_s) / sum_s w_s l_s with w_s = exp(m_s - max)
  // max and sum over the splits: butterflies within groups of P >= MAXS lanes (the first
  // group holds every split; the other groups' results are never read)
  constexpr int P = MAXS <= 8 ? 8 : MAXS <= 16 ? 16 : MAXS <= 32 ? 32 : 64;
  const bool mine = lane < ns;
  float mmax = mine ? m_l : -INFINITY;
#pragma unroll
  for (int o2 = P / 2; o2 > 0; o2 >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, o2));
  const float w = mine ? exp_hw(m_l - mmax) * l_l : 0.f;
  float lsum = w;
#pragma unroll
  for (int o2 = P / 2; o2 > 0; o2 >>= 1) lsum += __shfl_xor(lsum, o2);
  const float wn = w * (1.0f / lsum);  // lanes past nsplit: 0
  // a trip count uniform across the wave: every lane is active at the v_readlane of each
  // weight (a lane outside a divergent loop might not hold its weight there)
  for (int db = 0; db < hd; db += 256) {
    const int d = db + lane * 4;
    if (db > 0) {  // head dims past 256
      const int dc = min(d, hd - 4);
#pragma unroll
      for (int s = 0; s < MAXS; ++s) o[s] = load_dev<h4, COH ? 16 : COMB_AUX>(ro, (int)(((pr0 + (size_t)min(s, ns - 1) * a.rpad) * hd + dc) * 2));
    }
    f4 acc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wn), s));
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += ws * h2f(o[s][i]);
    }
    h4 o4;
#pragma unroll
    for (int i = 0; i < 4; ++i) o4[i] = f2h(acc[i]);
    if (d < hd) {
      const int col = h * hd + d;
      const size_t oi = a.out_frag ? xf_index(t, col) : (size_t)t * a.out_ld + col;
      if constexpr (ST_DEV) store_dev<h4>(dev_rsrc(a.out, 0x7FFFFFF0), (int)(oi * 2), o4);
      else *reinterpret_cast<h4*>(a.out + oi) = o4;
    }
  }
}

// Chunks stream through two LDS buffers with two chunks of loads in flight in registers.
// IMG: prefix splits copy prebuilt chunk images; otherwise (and for the suffix split)
// the chunk is converted in registers (hi/lo split, V transposed, suffix RoPE).
// QF: q arrives roped, scaled and split in fragment order (a.qf) and the suffix k roped in
// fp32 (a.ks32), both from the qkv epilogue.
template <int HD, bool IMG>
constexpr int attn_buf_bytes() {
  return IMG ? img_bytes<HD>() : ((int)sizeof(AttnSmem<HD>) + 15) / 16 * 16;
}

// One workgroup's share of the joint attention: row block bx (64 query rows) of kv head kvh
// against key split `split`, with the two chunk buffers in lds_raw (2 * attn_buf_bytes).
// COH: the partials and outputs are written with device-scope stores (written through to
// the memory side), for a consumer in the same launch on another XCD.
// tid: this thread's index in the workgroup (threadIdx.x; the persistent step passes a copy
// the compiler cannot hoist)
// NW: waves per workgroup.  4: wave w computes query tile w over every chunk.  8: the two waves
// of query tile w & 3 take alternate chunks (wave w >> 2 == chunk parity), so both LDS buffers
// are computed at once and each SIMD runs two waves, whose LDS reads and softmax hide each
// other's latency; their online-softmax states merge through LDS at the end.
template <int HD, bool KF32, bool ROPE, bool IMG, bool QF, bool COH, int NW = 4>
__device__ __forceinline__ void attn_block(const AttnArgs& a, const int bx, const int split, const int kvh,
                                           char* lds_raw, const int tid) {
  static_assert(NW == 4 || (NW == 8 && !IMG), "8 waves read converted chunks, not images");
  constexpr int NTH = 64 * NW;  // threads of the workgroup
  constexpr int BUFB = attn_buf_bytes<HD, IMG>();
  constexpr int IMGB = img_bytes<HD>();
  constexpr int KLD = AttnSmem<HD>::KLD;
  constexpr int NKS = (HD + 31) / 32;  // k-steps of 32 dims
  constexpr int NDT = HD / 16;         // output d tiles

  const int lane = tid & 63, w = tid >> 6;
  const int rt = w & 3;   // this wave's 16-row query tile
  const int cp = w >> 2;  // 8 waves: the parity of the chunks this wave computes
  const int g = lane >> 4, r16 = lane & 15;
  const int grp = a.H / a.KV;
  const int row = bx * ROWS + 16 * rt + r16;  // this lane's query row (B-operand column)
  const bool row_ok = row < a.rows;
  const int rowc = min(row, a.rows - 1);
  const int hl = rowc / a.Tq, t = rowc % a.Tq;
  const int h = kvh * grp + hl;
  const int nsp = a.nsplit - (a.Ts > 0 ? 1 : 0);     // prefix splits; the last split is the suffix
  const bool suffix = split >= nsp;
  const int kbeg = suffix ? 0 : split * a.kps;
  const int kend = suffix ? a.Ts : min(a.Sp, kbeg + a.kps);
  const int nch = (kend - kbeg + KCH - 1) / KCH;

  h8 qh[NKS], ql[NKS];
  f4 oacc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) oacc[i] = (f4){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.f;

  // logits, online softmax and O^T += V^T . P^T for one chunk resident in LDS.  A chunk whose
  // 32 keys are all masked (<= -1e9, padding -inf) is skipped: for a row with any valid key its
  // probabilities are exp(s - 1e9 - m) = 0 in fp32, so it changes neither l nor O (before the
  // row's first valid chunk, its state is scaled by exp(-1e9 - m) = 0), and the results are
  // bit-identical to computing it (GPU test at 800 of 968 prefix keys valid).
  auto chunk_math = [&](const AttnSmem<HD>& sk) __attribute__((always_inline)) {
    if (!a.noskip && __all(sk.msk[lane & (KCH - 1)] <= -1e9f)) return;
    // ---- logits S^T for the 2 key tiles of 16: 6 independent accumulation chains --
    f4 acc3[2][3];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc3[kt][j] = (f4){0.f, 0.f, 0.f, 0.f};
    // K fragments of k step ks + 1 are read from LDS while step ks multiplies
    h8 kf[2][2][2];  // [buffer][key tile][hi, lo]
    auto ldk = [&](int ks, int b) __attribute__((always_inline)) {
      const int d0 = 32 * ks + 8 * g;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        kf[b][kt][0] = *reinterpret_cast<const h8*>(&sk.kh[(16 * kt + r16) * KLD + d0]);
        kf[b][kt][1] = *reinterpret_cast<const h8*>(&sk.kl[(16 * kt + r16) * KLD + d0]);
        if constexpr (HD < 32) {
          if (d0 >= HD) kf[b][kt][0] = kf[b][kt][1] = (h8){0, 0, 0, 0, 0, 0, 0, 0};
        }
      }
    };
    ldk(0, 0);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (ks + 1 < NKS) ldk(ks + 1, (ks + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead (the scheduler would sink them)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const h8 ah = kf[ks & 1][kt][0], al = kf[ks & 1][kt][1];
        acc3[kt][0] = mfma16x16x32(al, qh[ks], acc3[kt][0]);
        acc3[kt][1] = mfma16x16x32(ah, ql[ks], acc3[kt][1]);
        acc3[kt][2] = mfma16x16x32(ah, qh[ks], acc3[kt][2]);
      }
    }
    // lane holds keys 16kt + 4g + i of row r16
    float p[8];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p[4 * kt + i] = (acc3[kt][0][i] + acc3[kt][1][i]) + acc3[kt][2][i] + sk.msk[16 * kt + 4 * g + i];
    // ---- online softmax over this chunk (row r16: lanes r16, +16, +32, +48) --------
    float cmax = p[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) cmax = fmaxf(cmax, p[i]);
    cmax = xor_max_16_32(cmax);
    // lazy running max: it moves only when a chunk's max exceeds it by more than 8, so
    // p = exp(s - m_run) stays below e^8 (fp16-safe) and most chunks skip the rescale of
    // the accumulators (the result is the same softmax: m_run, l_run and O agree)
    const bool grow = cmax > m_run + 8.0f;
    const float m_new = grow ? cmax : m_run;
    const float alpha = exp_hw(m_run - m_new);
    const bool rescale = __any(grow);
    float psum = 0.f;
    h8 pb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float e = exp_hw(p[i] - m_new);
      psum += e;
      pb[i] = f2h(e);
    }
    psum = xor_sum_16_32(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    if (rescale) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
    }
    // ---- O^T += V^T . P^T (V^T read in the key order of P: 4g..4g+3, 16+4g..16+4g+3) --
    // V^T fragments read two d tiles ahead of their MFMA
    h4 vf[3][2];
    auto ldv = [&](int dt, int b) __attribute__((always_inline)) {
      const _Float16* vr = &sk.vt[(16 * dt + r16) * VLD];
      vf[b][0] = *reinterpret_cast<const h4*>(vr + 4 * g);
      vf[b][1] = *reinterpret_cast<const h4*>(vr + 16 + 4 * g);
    };
    ldv(0, 0);
    if (NDT > 1) ldv(1, 1);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      if (dt + 2 < NDT) ldv(dt + 2, (dt + 2) % 3);
      __builtin_amdgcn_sched_barrier(0);
      const h4 v0 = vf[dt % 3][0], v1 = vf[dt % 3][1];
      const h8 av = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      oacc[dt] = mfma16x16x32(av, pb, oacc[dt]);
    }
  };

  auto buf = [&](int b) -> const AttnSmem<HD>& { return *reinterpret_cast<const AttnSmem<HD>*>(lds_raw + b * BUFB); };
  auto wbuf = [&](int b) -> AttnSmem<HD>& { return *reinterpret_cast<AttnSmem<HD>*>(lds_raw + b * BUFB); };

  // Chunk c is computed from buffer c & 1.  Register stage R0 / R1 carries chunk c + 2
  // (loaded two chunks ahead) until buffer c & 1 is free again after chunk c.
  //   load(c, R): issue the loads of chunk c;  store(R, b): write it into buffer b.
  auto pipeline = [&](auto& R0, auto& R1, auto&& load, auto&& store) __attribute__((always_inline)) {
    load(0, R0);
    if (nch > 1) load(1, R1);
    if constexpr (QF) {
      // q fragments from the q/k/v epilogue of the previous kernel: device-scope loads
      const __amdgpu_buffer_rsrc_t rq = dev_rsrc(a.qf, (uint32_t)a.KV * a.rpad * NKS * 128);
      const int tile = kvh * (a.rpad / 16) + (bx * ROWS + 16 * rt) / 16;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int qb = (((tile * NKS + ks) * 2) * 512 + lane * 8) * 2;
        qh[ks] = load_dev<h8, COH ? 16 : ATTN_Q_AUX>(rq, qb);
        ql[ks] = load_dev<h8, COH ? 16 : ATTN_Q_AUX>(rq, qb + 1024);
      }
    } else {
      QRaw<HD> qa, qb;
      load_q<HD, ROPE>(a, t, h, g, qa, 0);
      if constexpr (QRaw<HD>::NHALF > 1) load_q<HD, ROPE>(a, t, h, g, qb, 1);
      __builtin_amdgcn_sched_barrier(0);
      make_q<HD, ROPE>(a, qa, g, qh, ql, 0);
      if constexpr (QRaw<HD>::NHALF > 1) make_q<HD, ROPE>(a, qb, g, qh, ql, 1);
    }
    store(R0, 0);
    if (nch > 1) store(R1, 1);
    lds_barrier();
    ATTN_STAMP(1);
    if constexpr (NW == 8) {
      // chunks c and c + 1 at once, one per wave group; the next pair's loads in flight
      for (int c = 0; c < nch; c += 2) {
        if (c + 2 < nch) load(c + 2, R0);
        if (c + 3 < nch) load(c + 3, R1);
        if (c + cp < nch) chunk_math(buf(cp));
        lds_barrier();
        if (c + 2 < nch) {
          store(R0, 0);
          if (c + 3 < nch) store(R1, 1);
          lds_barrier();
        }
      }
      return;
    }
    if (nch > 2) load(2, R0);
    if (nch > 3) load(3, R1);
    for (int c = 0; c < nch; c += 2) {
      chunk_math(buf(0));
      lds_barrier();
      if (c + 2 < nch) {
        store(R0, 0);
        if (c + 4 < nch) load(c + 4, R0);
      }
      if (c + 1 < nch) {
        chunk_math(buf(1));
        lds_barrier();
        if (c + 3 < nch) {
          store(R1, 1);
          if (c + 5 < nch) load(c + 5, R1);
        }
      }
    }
  };
  ATTN_STAMP(0);
  if (QF && suffix) {
    ChunkRegs<HD, NTH> R0, R1;
    pipeline(
        R0, R1,
        [&](int c, ChunkRegs<HD, NTH>& R) {
          load_suffix32<HD, COH ? 16 : ATTN_Q_AUX, NTH>(R, a, kvh, c * KCH, kend, tid);
        },
        [&](const ChunkRegs<HD, NTH>& R, int b) { store_chunk<HD, NTH>(R, wbuf(b), tid); });
  } else if (suffix) {
    SufRegs<HD, NTH> R0, R1;
    pipeline(
        R0, R1, [&](int c, SufRegs<HD, NTH>& R) { load_suffix<HD, ROPE, NTH>(R, a, kvh, c * KCH, kend, tid); },
        [&](const SufRegs<HD, NTH>& R, int b) {
          ChunkRegs<HD, NTH> k32;
          rope_suffix<HD, ROPE, NTH>(R, k32, a.ks_roped != 0);
          store_chunk<HD, NTH>(k32, wbuf(b), tid);
        });
  } else if constexpr (IMG) {
    constexpr int NI = IMGB / (NT * 16);
    struct ImgRegs {
      u4 v[NI];
    };
    const char* ib = a.kimg + ((size_t)kvh * a.img_chunks + kbeg / KCH) * IMGB;
    ImgRegs R0, R1;
    pipeline(
        R0, R1,
        [&](int c, ImgRegs& R) {
#pragma unroll
          for (int i = 0; i < NI; ++i)
            R.v[i] = load_global(reinterpret_cast<const u4*>(ib + (size_t)c * IMGB + (size_t)(i * NT + tid) * 16));
        },
        [&](const ImgRegs& R, int b) {
#pragma unroll
          for (int i = 0; i < NI; ++i) *reinterpret_cast<u4*>(lds_raw + b * BUFB + (i * NT + tid) * 16) = R.v[i];
        });
  } else {
    ChunkRegs<HD, NTH> R0, R1;
    pipeline(
        R0, R1,
        [&](int c, ChunkRegs<HD, NTH>& R) { load_prefix<HD, KF32, NTH>(R, a, kvh, kbeg + c * KCH, kend, tid); },
        [&](const ChunkRegs<HD, NTH>& R, int b) { store_chunk<HD, NTH>(R, wbuf(b), tid); });
  }

  if constexpr (NW == 8) {
    // the odd-chunk wave of each query tile hands (O, m, l) to the even-chunk wave through LDS
    // (the chunk buffers are free after the loop's last barrier); that wave merges the two
    // online-softmax states and writes the tile
    f4* mo = reinterpret_cast<f4*>(lds_raw) + (size_t)rt * (NDT + 1) * 64;
    static_assert(4 * (NDT + 1) * 64 * 16 <= 2 * BUFB, "merge area");
    if (cp == 1) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) mo[dt * 64 + lane] = oacc[dt];
      mo[NDT * 64 + lane] = (f4){m_run, l_run, 0.f, 0.f};
    }
    lds_barrier();
    if (cp == 0) {
      const f4 ml = mo[NDT * 64 + lane];
      const float m_new = fmaxf(m_run, ml[0]);
      const float a0 = exp_hw(m_run - m_new), a1 = exp_hw(ml[0] - m_new);
      l_run = l_run * a0 + ml[1] * a1;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] = oacc[dt] * a0 + mo[dt * 64 + lane] * a1;
      m_run = m_new;
    }
    lds_barrier();  // every merge read is done before the partial rows are staged over it
    if (cp == 1) return;
  }

  ATTN_STAMP(2);
  if (a.nsplit > 1) {
    // the split's output normalized by its own softmax sum (a convex combination of V
    // rows, so fp16 holds it), with (m, l) in fp32 for the combine.  The wave's 16 rows go
    // through its own LDS rows (free after the last chunk's barrier) so that every store
    // writes two whole rows of the partial (1 KB contiguous) instead of 16 pieces of 32 B.
    constexpr int PLD = HD + 8;  // halfs per LDS row
    _Float16* pl = reinterpret_cast<_Float16*>(lds_raw) + (size_t)rt * 16 * PLD;
    const float linv = l_run > 0.f ? 1.0f / l_run : 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      h4 o4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = f2h(oacc[dt][i] * linv);
      *reinterpret_cast<h4*>(pl + r16 * PLD + 16 * dt + 4 * g) = o4;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    constexpr int LPR = HD / 8;           // 8-half pieces per row
    constexpr int ITEMS = 16 * LPR;       // pieces of the wave's 16 rows, 64 per store
    const size_t pr0 = ((size_t)kvh * a.nsplit + split) * a.rpad + bx * ROWS + 16 * rt;
    _Float16* po = reinterpret_cast<_Float16*>(a.part_o);
    const __amdgpu_buffer_rsrc_t rpo = dev_rsrc(po, 0x7FFFFFF0), rpml = dev_rsrc(a.part_ml, 0x7FFFFFF0);
#pragma unroll
    for (int it = 0; it < (ITEMS + 63) / 64; ++it) {
      const int idx = 64 * it + lane, rr = idx / LPR, cc = (idx % LPR) * 8;
      if (idx < ITEMS && bx * ROWS + 16 * rt + rr < a.rows) {
        const h8 v = *reinterpret_cast<const h8*>(pl + rr * PLD + cc);
        if constexpr (COH) store_dev<h8>(rpo, (int)(((pr0 + rr) * HD + cc) * 2), v);
        else *reinterpret_cast<h8*>(po + (pr0 + rr) * HD + cc) = v;
      }
    }
    if (g == 0 && row_ok) {
      const size_t pr = ((size_t)kvh * a.nsplit + split) * a.rpad + row;
      if constexpr (COH) {
        store_dev<f2>(rpml, (int)(pr * 8), (f2){m_run, l_run});
      } else {
        a.part_ml[pr * 2 + 0] = m_run;
        a.part_ml[pr * 2 + 1] = l_run;
      }
    }
    ATTN_STAMP(3);
    return;
  }
  if (!row_ok) return;
  {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;  // 0: every key of the row masked (all skipped)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      h4 o4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = f2h(oacc[dt][i] * inv);
      const int col = h * HD + 16 * dt + 4 * g;
      const size_t oi = a.out_frag ? xf_index(t, col) : (size_t)t * a.out_ld + col;
      if constexpr (COH) store_dev<h4>(dev_rsrc(a.out, 0x7FFFFFF0), (int)(oi * 2), o4);
      else *reinterpret_cast<h4*>(a.out + oi) = o4;
    }
  }
}

}  // namespace
}  // namespace mlcv
