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
// A read touches start on distinct banks); V transposed [d][key] with a pitch of 40
// halfs, written as packed key pairs (ds_write_b32) -- lanes of one store cover 16
// key pairs x 4 dims and a wave's MFMA reads of 16 d-rows land on disjoint banks.
#include <type_traits>

#include "kernels.h"

namespace mlcv {

namespace {
constexpr int KCH = 32;        // keys per chunk
constexpr int ROWS = 64;       // query rows per workgroup (4 waves x 16)
constexpr int VLD = KCH + 8;   // halfs per V^T row
constexpr int NT = 256;        // threads per workgroup (4 waves, one 16-row query tile each)

__device__ const float kZeroF = 0.0f;

template <int HD>
struct AttnSmem {
  static constexpr int KLD = HD + 8;  // halfs per K row
  _Float16 kh[KCH * KLD];
  _Float16 kl[KCH * KLD];
  _Float16 vt[HD * VLD];
  float msk[KCH];
};

// One key chunk in registers between its global loads and its LDS stores.
//   K item (key j, dims dp..dp+7 and dp+HD/2..+7) as fp32 (the RoPE pair of the suffix
//   loader is one item); V item (keys 2jp, 2jp+1; dims d0..d0+7).  Items past the
//   chunk's item count are repeats of earlier ones (identical LDS stores).
template <int HD>
struct ChunkRegs {
  static constexpr int HALF = HD / 2;
  static constexpr int KITEMS = KCH * (HALF / 8);
  static constexpr int VITEMS = (KCH / 2) * (HD / 8);
  static constexpr int NK = (KITEMS + NT - 1) / NT;
  static constexpr int NV = (VITEMS + NT - 1) / NT;
  float k[NK][16];
  h8 v[NV][2];
  float msk;
};

template <int HD>
__device__ __forceinline__ void kitem(int i, int tid, int& j, int& dp) {
  constexpr int HALF = HD / 2;
  const int it = (tid + NT * i) % ChunkRegs<HD>::KITEMS;
  j = it / (HALF / 8);
  dp = (it % (HALF / 8)) * 8;
}
template <int HD>
__device__ __forceinline__ void vitem(int i, int tid, int& jp, int& d0) {
  const int it = (tid + NT * i) % ChunkRegs<HD>::VITEMS;
  jp = it % (KCH / 2);
  d0 = (it / (KCH / 2)) * 8;
}

__device__ __forceinline__ void cvt8(const h8 x, float* o) {
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = h2f(x[e]);
}
__device__ __forceinline__ void ld8f(const float* p, float* o) {
  const f4 a = load_global(reinterpret_cast<const f4*>(p)), b = load_global(reinterpret_cast<const f4*>(p + 4));
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = a[e];
    o[e + 4] = b[e];
  }
}

// prefix keys [c0, c0+32) of this split (cached, roped; fp32 or fp16), clamped below kend
template <int HD, bool KF32>
__device__ __forceinline__ void load_prefix(ChunkRegs<HD>& r, const AttnArgs& a, int kvh, int c0, int kend, int tid) {
  constexpr int HALF = HD / 2;
  const size_t base = (size_t)kvh * a.Sp * HD;
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD>::NK; ++i) {
    int j, dp;
    kitem<HD>(i, tid, j, dp);
    const size_t off = base + (size_t)min(c0 + j, kend - 1) * HD + dp;
    if constexpr (KF32) {
      const float* kp = reinterpret_cast<const float*>(a.kp);
      ld8f(kp + off, r.k[i]);
      ld8f(kp + off + HALF, r.k[i] + 8);
    } else {
      const _Float16* kp = reinterpret_cast<const _Float16*>(a.kp);
      cvt8(load_global(reinterpret_cast<const h8*>(kp + off)), r.k[i]);
      cvt8(load_global(reinterpret_cast<const h8*>(kp + off + HALF)), r.k[i] + 8);
    }
  }
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD>::NV; ++i) {
    int jp, d0;
    vitem<HD>(i, tid, jp, d0);
    const _Float16* vb = a.vp + base + d0;
    r.v[i][0] = load_global(reinterpret_cast<const h8*>(vb + (size_t)min(c0 + 2 * jp, kend - 1) * HD));
    r.v[i][1] = load_global(reinterpret_cast<const h8*>(vb + (size_t)min(c0 + 2 * jp + 1, kend - 1) * HD));
  }
  const int kj = c0 + (tid & (KCH - 1));
  const float* mp = a.mask ? a.mask : &kZeroF;
  const float mv = mp[a.mask ? min(kj, kend - 1) : 0];
  r.msk = kj < kend ? mv : -INFINITY;
}

// Suffix keys [c0, c0+32): the raw fp16 k of the suffix rows and their rope tables stay
// in registers as loaded (no arithmetic on in-flight loads), roped at store time.
template <int HD>
struct SufRegs {
  static constexpr int NK = ChunkRegs<HD>::NK, NV = ChunkRegs<HD>::NV;
  h8 x1[NK], x2[NK];
  f4 c[NK][2], s[NK][2];
  h8 v[NV][2];
  float msk;
};

template <int HD, bool ROPE>
__device__ __forceinline__ void load_suffix(SufRegs<HD>& r, const AttnArgs& a, int kvh, int c0, int kend, int tid) {
  constexpr int HALF = HD / 2;
#pragma unroll
  for (int i = 0; i < SufRegs<HD>::NK; ++i) {
    int j, dp;
    kitem<HD>(i, tid, j, dp);
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
  for (int i = 0; i < SufRegs<HD>::NV; ++i) {
    int jp, d0;
    vitem<HD>(i, tid, jp, d0);
    const _Float16* vb = a.vs + (size_t)kvh * HD + d0;
    r.v[i][0] = load_global(reinterpret_cast<const h8*>(vb + (size_t)min(c0 + 2 * jp, kend - 1) * a.vs_ld));
    r.v[i][1] = load_global(reinterpret_cast<const h8*>(vb + (size_t)min(c0 + 2 * jp + 1, kend - 1) * a.vs_ld));
  }
  r.msk = c0 + (tid & (KCH - 1)) < kend ? 0.f : -INFINITY;
}

// rope the suffix keys (unless handed over roped) into the fp32 chunk layout
template <int HD, bool ROPE>
__device__ __forceinline__ void rope_suffix(const SufRegs<HD>& in, ChunkRegs<HD>& r, bool roped) {
#pragma unroll
  for (int i = 0; i < SufRegs<HD>::NK; ++i) {
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
  for (int i = 0; i < SufRegs<HD>::NV; ++i) {
    r.v[i][0] = in.v[i][0];
    r.v[i][1] = in.v[i][1];
  }
  r.msk = in.msk;
}

template <int HD>
__device__ __forceinline__ void store_chunk(const ChunkRegs<HD>& r, AttnSmem<HD>& sm, int tid) {
  constexpr int KLD = AttnSmem<HD>::KLD, HALF = HD / 2;
#pragma unroll
  for (int i = 0; i < ChunkRegs<HD>::NK; ++i) {
    int j, dp;
    kitem<HD>(i, tid, j, dp);
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
  for (int i = 0; i < ChunkRegs<HD>::NV; ++i) {
    int jp, d0;
    vitem<HD>(i, tid, jp, d0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const h2 pair = {r.v[i][0][e], r.v[i][1][e]};
      *reinterpret_cast<h2*>(&sm.vt[(d0 + e) * VLD + 2 * jp]) = pair;
    }
  }
  if (tid < KCH) sm.msk[tid] = r.msk;
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

template <int HD, bool KF32, bool ROPE>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) AttnSmem<HD> sm;
  constexpr int KLD = AttnSmem<HD>::KLD;
  constexpr int NKS = (HD + 31) / 32;  // k-steps of 32 dims
  constexpr int NDT = HD / 16;         // output d tiles

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int kvh = blockIdx.z, split = blockIdx.y;
  const int grp = a.H / a.KV;
  const int row = blockIdx.x * ROWS + 16 * w + r16;   // this lane's query row (B-operand column)
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

  auto body = [&](auto suffix_tag) {
    constexpr bool SUF = decltype(suffix_tag)::value;
    using Regs = typename std::conditional<SUF, SufRegs<HD>, ChunkRegs<HD>>::type;
    Regs regs;
    auto load = [&](int c0) {
      if constexpr (SUF) load_suffix<HD, ROPE>(regs, a, kvh, c0, kend, tid);
      else load_prefix<HD, KF32>(regs, a, kvh, c0, kend, tid);
    };
    auto store = [&]() {
      if constexpr (SUF) {
        ChunkRegs<HD> k32;
        rope_suffix<HD, ROPE>(regs, k32, a.ks_roped != 0);
        store_chunk<HD>(k32, sm, tid);
      } else {
        store_chunk<HD>(regs, sm, tid);
      }
    };
    // Q and the first chunk go out as one batch of loads: Q half 0, the chunk, Q half 1
    QRaw<HD> qa, qb;
    load_q<HD, ROPE>(a, t, h, g, qa, 0);
    load(kbeg);
    if constexpr (QRaw<HD>::NHALF > 1) load_q<HD, ROPE>(a, t, h, g, qb, 1);
    __builtin_amdgcn_sched_barrier(0);
    make_q<HD, ROPE>(a, qa, g, qh, ql, 0);
    if constexpr (QRaw<HD>::NHALF > 1) make_q<HD, ROPE>(a, qb, g, qh, ql, 1);
    for (int c = 0; c < nch; ++c) {
      store();
      __syncthreads();
      load(kbeg + min(c + 1, nch - 1) * KCH);  // next chunk (the last one again at the end)
      __builtin_amdgcn_sched_barrier(0);       // keep the prefetch ahead of this chunk's MFMAs

      // ---- logits S^T for the 2 key tiles of 16: 6 independent accumulation chains --
      f4 acc3[2][3];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc3[kt][j] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d0 = 32 * ks + 8 * g;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          h8 ah = *reinterpret_cast<const h8*>(&sm.kh[(16 * kt + r16) * KLD + d0]);
          h8 al = *reinterpret_cast<const h8*>(&sm.kl[(16 * kt + r16) * KLD + d0]);
          if constexpr (HD < 32) {
            if (d0 >= HD) ah = al = (h8){0, 0, 0, 0, 0, 0, 0, 0};
          }
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
          p[4 * kt + i] = (acc3[kt][0][i] + acc3[kt][1][i]) + acc3[kt][2][i] + sm.msk[16 * kt + 4 * g + i];
      // ---- online softmax over this chunk (row r16: lanes r16, +16, +32, +48) --------
      float cmax = p[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) cmax = fmaxf(cmax, p[i]);
      cmax = xor_max_16_32(cmax);
      const float m_new = fmaxf(m_run, cmax);
      const float alpha = exp_hw(m_run - m_new);
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

      // ---- O^T += V^T . P^T (V^T read in the key order of P: 4g..4g+3, 16+4g..16+4g+3) --
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const _Float16* vr = &sm.vt[(16 * dt + r16) * VLD];
        const h4 v0 = *reinterpret_cast<const h4*>(vr + 4 * g);
        const h4 v1 = *reinterpret_cast<const h4*>(vr + 16 + 4 * g);
        const h8 av = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        f4 o = oacc[dt];
        o[0] *= alpha;
        o[1] *= alpha;
        o[2] *= alpha;
        o[3] *= alpha;
        oacc[dt] = mfma16x16x32(av, pb, o);
      }
      __syncthreads();
    }
  };
  if (suffix) body(std::true_type{});
  else body(std::false_type{});

  if (!row_ok) return;
  if (a.nsplit == 1) {
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      h4 o4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = f2h(oacc[dt][i] * inv);
      const int col = h * HD + 16 * dt + 4 * g;
      *reinterpret_cast<h4*>(a.out + (a.out_frag ? xf_index(t, col) : (size_t)t * a.out_ld + col)) = o4;
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

// combine the per-split partial softmax states of one row (one wave per row); every
// load goes out at once (split indices past nsplit repeat a valid split with weight 0)
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a) {
  constexpr int MAXS = 32;
  const int row = blockIdx.x, kvh = blockIdx.y, lane = threadIdx.x;
  const int hd = a.hd;
  const int grp = a.H / a.KV;
  const int hl = row / a.Tq, t = row % a.Tq, h = kvh * grp + hl;
  const size_t pr0 = (size_t)kvh * a.nsplit * a.rpad + row;
  const int ns = a.nsplit;
  const int sl = min(lane, ns - 1);
  const float m_l = a.part_ml[(pr0 + (size_t)sl * a.rpad) * 2];
  const float l_l = a.part_ml[(pr0 + (size_t)sl * a.rpad) * 2 + 1];
  // the O loads of the first 256 dims go out with the m / l loads
  const int d0 = min(lane * 4, hd - 4);
  f4 o[MAXS];
#pragma unroll
  for (int s = 0; s < MAXS; ++s)
    o[s] = *reinterpret_cast<const f4*>(a.part_o + (pr0 + (size_t)min(s, ns - 1) * a.rpad) * hd + d0);
  // split weights w_s = exp(m_s - max) / sum_s l_s exp(m_s - max), lane s holds split s
  // (computed by all 64 lanes: the shuffles below need every lane active)
  const float m = lane < ns ? m_l : -INFINITY;
  float mmax = m;
  for (int off = 32; off > 0; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
  const float e = lane < ns ? exp_hw(m - mmax) : 0.f;
  const float lsum = wave_sum(l_l * e);
  const float wgt = e / lsum;
  float wv[MAXS];
#pragma unroll
  for (int s = 0; s < MAXS; ++s) wv[s] = __shfl(wgt, s);
  for (int d = lane * 4; d < hd; d += 256) {
    if (d != d0) {  // head dims past 256
#pragma unroll
      for (int s = 0; s < MAXS; ++s)
        o[s] = *reinterpret_cast<const f4*>(a.part_o + (pr0 + (size_t)min(s, ns - 1) * a.rpad) * hd + d);
    }
    f4 acc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < MAXS; ++s) acc += wv[s] * o[s];
    h4 o4;
#pragma unroll
    for (int i = 0; i < 4; ++i) o4[i] = f2h(acc[i]);
    const int col = h * hd + d;
    *reinterpret_cast<h4*>(a.out + (a.out_frag ? xf_index(t, col) : (size_t)t * a.out_ld + col)) = o4;
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

void attn_plan(int rows, int Sp, int Ts, int target_blocks, int* nsplit, int* kps) {
  // prefix splits of whole 32-key chunks, plus one split for the suffix block
  const int rb = (rows + ROWS - 1) / ROWS;
  const int chunks = (Sp + KCH - 1) / KCH;
  int ns = (target_blocks + rb - 1) / rb - (Ts > 0 ? 1 : 0);
  if (ns > 31) ns = 31;
  if (ns > chunks) ns = chunks;
  if (ns < 1) ns = 1;
  const int cps = chunks > 0 ? (chunks + ns - 1) / ns : 1;
  *kps = cps * KCH;
  *nsplit = (chunks > 0 ? (chunks + cps - 1) / cps : 0) + (Ts > 0 ? 1 : 0);
}

size_t attn_ws_floats(int KV, int rows, int hd, int nsplit) {
  const int rpad = ((rows + ROWS - 1) / ROWS) * ROWS;
  return nsplit > 1 ? (size_t)KV * nsplit * rpad * (hd + 2) : 0;
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
  MLCV_REQUIRE(a.cos == nullptr || a.sin != nullptr, "rope needs cos and sin");
  MLCV_REQUIRE(a.Ts == 0 || a.cos != nullptr || a.ks_roped, "raw suffix keys need the rope tables");
  dim3 grid((a.rows + ROWS - 1) / ROWS, a.nsplit, a.KV);
#define MLCV_ATTN_CASE(HDV)                                                            \
  case HDV:                                                                            \
    if (a.kp_f32) {                                                                    \
      if (a.cos) attn_kernel<HDV, true, true><<<grid, 256, 0, st>>>(a);                \
      else attn_kernel<HDV, true, false><<<grid, 256, 0, st>>>(a);                     \
    } else {                                                                           \
      if (a.cos) attn_kernel<HDV, false, true><<<grid, 256, 0, st>>>(a);               \
      else attn_kernel<HDV, false, false><<<grid, 256, 0, st>>>(a);                    \
    }                                                                                  \
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
