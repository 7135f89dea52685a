// Persistent step kernel: one launch of one workgroup per CU runs a whole denoise_step_kv
// (pi0_model.py:142-163 with decode_e1 / attn_decode_e1, gemma_dual.py:255-275,343-351,
// 417-433) once the adaRMS modulations are known.
//
// The step is a chain of about 110 dependent phases (action_in; per layer q/k/v, attention,
// split combine, o_proj, gate_up, down; the head), each only a few microseconds of HBM time.
// As separate kernels every phase pays a launch and a cold start (its weights from HBM after
// its inputs are ready).  Here every workgroup owns fixed tasks of every phase and
//   1. publishes its progress word once its tasks of a phase are stored,
//   2. issues the weight loads of its next task,
//   3. waits until every workgroup has published the previous phase,
//   4. loads its activations and multiplies, with the weights already in registers.
// Data crossing workgroups is written with device-scope stores (through this XCD's L2 to the
// memory side) and read with device-scope loads, and every buffer is written once per launch,
// so no cache maintenance is needed.  Waits are bounded: a wait that gives up sets the error
// word and every workgroup leaves the kernel (mlcv_sync reports it and resets the words).
//
// GEMM tasks are the fragment-major skinny tiles of gemm_skinny.hip in a fixed shape: SW
// 16-row weight slabs, one K slice split over the 4 waves in equal k ranges, the 4 partial
// sums added through LDS in wave order; wave w then owns m tile w.  Split-K tasks meet at a
// per-tile arrival counter, and the last to arrive adds the partials in split order.
#include <type_traits>

#include "attn_impl.h"

namespace mlcv {

#ifdef MLCV_PK_TRACE
// phase timeline of the last launch for the trace build: [phase][workgroup][start, waited,
// done, published] in s_memrealtime ticks (100 MHz)
__device__ unsigned long long pk_trace[256 * 512 * 4];
__shared__ int pk_trace_ph;
#define PK_STAMP(k)                                                                                   \
  do {                                                                                                \
    if (pk_tid() == 0)                                                                             \
      pk_trace[((size_t)pk_trace_ph * 512 + blockIdx.x) * 4 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define PK_STAMP(k) \
  do {              \
  } while (0)
#endif

namespace {

constexpr int PK_THREADS = 256;
constexpr int PK_KPW = 8;  // k steps of 32 per wave at most (K slice <= 1024)

template <int HD>
constexpr int pk_smem_bytes() {
  constexpr int attn = 2 * attn_buf_bytes<HD, false>();
  constexpr int gemm = 4 * 2 * 4 * 64 * 16 + 4 * 64 * 4 + 2 * 4 * 16;
  return attn > gemm ? attn : gemm;
}
constexpr int PK_RED_OFF = 0;                           // f4 [4 k groups][SW][4 m tiles][64]
constexpr int PK_DENOM_OFF = 4 * 2 * 4 * 64 * 16;       // float [4 waves][64 rows]
constexpr int PK_SHIFT_OFF = PK_DENOM_OFF + 4 * 64 * 4;  // f4 [SW][4 lane groups]

struct PkShared {
  int flag;
  int is_last;
};

// The kernel's arguments and the weight table are read in the constant address space
// (scalar loads through the constant cache) without copying them anywhere.
typedef __attribute__((address_space(4))) const PkArgs CPk;
typedef __attribute__((address_space(4))) const PkLin CPkLin;

// This thread's index, through a copy the compiler cannot see through: values computed from
// it (lane offsets of the fragment loads, ...) are then recomputed in each phase instead of
// being hoisted to the top of the kernel and held (or spilled) across all phases.
__device__ __forceinline__ int pk_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ int pk_bid() {
  int b = blockIdx.x;
  asm volatile("" : "+s"(b));
  return b;
}

// ---- synchronisation ----------------------------------------------------------------
__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every wave's stores are complete, then the workgroup meets: s_barrier (__syncthreads) alone
// does not wait for outstanding global stores on this part, so each wave first waits for its
// own.  Every store another workgroup reads is a device-scope (write-through) store, visible
// device-wide once complete, so the word that announces them needs no L2 write-back (a release
// fence there, buffer_wbl2, cost about 300 us per step) and is stored relaxed.
__device__ __forceinline__ void pk_stores_done() {
  wait_all_memory();
  __syncthreads();
}

// every store of this workgroup's tasks is complete; then the progress word
__device__ __forceinline__ void pk_publish(CPk& p, unsigned value) {
  pk_stores_done();
  if (pk_tid() == 0) __hip_atomic_store(p.prog + pk_bid(), value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every workgroup's progress word has reached `target` (wrapping compare).  Wave 0
// polls; the other waves keep their loads in flight at an LDS-only barrier.  false: the
// error word is set (this wait gave up, or another workgroup's did).
__device__ __forceinline__ bool pk_wait(CPk& p, unsigned target, PkShared& sh) {
  if (pk_tid() < 64) {
    const int lane = pk_tid();
    bool ok = false, failed = false;
    for (unsigned it = 0; it < p.spin; ++it) {  // spin == 0: give up without polling
      unsigned v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = lane + 64 * j < p.G ? ld_agent(p.prog + lane + 64 * j) : target;
      const unsigned e = ld_agent(p.err);
      bool done = true;
#pragma unroll
      for (int j = 0; j < 8; ++j) done = done && (int)(v[j] - target) >= 0;
      if (__all(done)) {
        ok = true;
        break;
      }
      if (e != 0) {
        failed = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (!ok && !failed) {  // this wait gave up: every workgroup leaves at its next wait
        __hip_atomic_fetch_or(p.err, PK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      sh.flag = ok ? 1 : 0;
    }
  }
  lds_barrier();
  const bool ok = sh.flag != 0;
  lds_barrier();  // the flag is read by every wave before wave 0 can write it again
  PK_STAMP(1);
  return ok;
}

// Wait until the counter word has reached `target` (wrapping compare); wave 0 polls.  false:
// the error word is set (this wait gave up, or another workgroup's did).
__device__ __forceinline__ bool pk_wait_count(CPk& p, const unsigned* ctr, unsigned target, PkShared& sh) {
  if (pk_tid() < 64) {
    bool ok = false, failed = false;
    for (unsigned it = 0; it < p.spin; ++it) {
      const unsigned v = ld_agent(ctr), e = ld_agent(p.err);
      if ((int)(v - target) >= 0) {
        ok = true;
        break;
      }
      if (e != 0) {
        failed = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (pk_tid() == 0) {
      if (!ok && !failed) {
        __hip_atomic_fetch_or(p.err, PK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      sh.flag = ok ? 1 : 0;
    }
  }
  lds_barrier();
  const bool ok = sh.flag != 0;
  lds_barrier();
  return ok;
}

// ---- GEMM tasks -----------------------------------------------------------------------
template <bool Q4, int SW>
struct WRegs {
  h8 v[SW][PK_KPW];
};
template <int SW>
struct WRegs<true, SW> {
  u4 q[SW][PK_KPW / 4];
  _Float16 s[SW][PK_KPW / 4];
};

// weights of SW consecutive 16-row slabs from slab0 of a K-wide matrix, k steps
// kbase .. kbase + kpw - 1 (q4: whole 128-k chunks, kpw % 4 == 0)
// KP > 0: kpw == KP is known at compile time (straight-line code); KP == 0: kpw at run time
template <bool Q4, int SW, int KP>
__device__ __forceinline__ void pk_load_w(WRegs<Q4, SW>& r, CPkLin& L, int slab0, int K, int kbase, int kpw) {
  if constexpr (KP > 0) kpw = KP;
  const int lane = pk_tid() & 63;
  if constexpr (!Q4) {
    const int KS = K >> 5;
#pragma unroll
    for (int sl = 0; sl < SW; ++sl) {
      const __amdgpu_buffer_rsrc_t rw = dev_rsrc(L.w + (size_t)(slab0 + sl) * KS * 512, (uint32_t)KS * 1024);
#pragma unroll
      for (int j = 0; j < PK_KPW; ++j)
        if (j < kpw) r.v[sl][j] = load_dev<h8, W_AUX>(rw, ((kbase + j) * 64 + lane) * 16);
    }
  } else {
    const int KCN = K >> 7;
#pragma unroll
    for (int sl = 0; sl < SW; ++sl)
#pragma unroll
      for (int c = 0; c < PK_KPW / 4; ++c)
        if (4 * c < kpw) {
          const size_t blk = ((size_t)(slab0 + sl) * KCN + (kbase >> 2) + c) * 64 + lane;
          r.q[sl][c] = load_global(reinterpret_cast<const u4*>(L.qw + blk * 4));
          r.s[sl][c] = load_global(L.qs + blk);
        }
  }
}

// X fragments (fragment-major [64][K]) of this wave's k steps for the 4 m tiles; rows past
// xlast read zeros from past the buffer (no memory access).  q4: the weights' k order.
// X is written by another workgroup of the launch (write-through) and read after its
// progress word with device-scope loads.  (Plain loads, shared through this XCD's L2, were
// measured to return a stale line now and then even with an L2 invalidate at the start of
// the launch: a chunk graph then differed from prefill + loop in the last bits.)
constexpr int PK_X_AUX = 16;
template <bool Q4, int KP>
__device__ __forceinline__ void pk_load_x(h8 (&xf)[PK_KPW][4], const _Float16* x, int K, int kbase, int kpw,
                                          int xlast) {
  if constexpr (KP > 0) kpw = KP;
  const int lane = pk_tid() & 63, g = lane >> 4, r16 = lane & 15;
  const __amdgpu_buffer_rsrc_t rx = dev_rsrc(x, (uint32_t)(64 * K * 2));
#pragma unroll
  for (int j = 0; j < PK_KPW; ++j)
    if (j < kpw) {
      const int ks = Q4 ? kbase + 4 * (j >> 2) + g : kbase + j;
      const int piece = Q4 ? 16 * (j & 3) + r16 : lane;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int off = 16 * mt + r16 <= xlast ? ((ks * 4 + mt) * 64 + piece) * 16 : 0x7FFFFF00;
        xf[j][mt] = load_dev<h8, PK_X_AUX>(rx, off);
      }
    }
}

template <bool Q4, int SW, int KP>
__device__ __forceinline__ void pk_mma(const WRegs<Q4, SW>& wr, const h8 (&xf)[PK_KPW][4], int kpw, f4 (&acc)[SW][4]) {
  if constexpr (KP > 0) kpw = KP;
#pragma unroll
  for (int sl = 0; sl < SW; ++sl)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[sl][mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < PK_KPW; ++j)
    if (j < kpw) {
      h8 a[SW];
#pragma unroll
      for (int sl = 0; sl < SW; ++sl) {
        if constexpr (Q4) a[sl] = dequant_word(wr.q[sl][j >> 2][j & 3], wr.s[sl][j >> 2]);
        else a[sl] = wr.v[sl][j];
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        h8 b = xf[j][mt];
        if constexpr (Q4) b = perm8(b);
#pragma unroll
        for (int sl = 0; sl < SW; ++sl) acc[sl][mt] = mfma16x16x32(a[sl], b, acc[sl][mt]);
      }
    }
}

// the 4 waves' k-range sums added in wave order; wave w keeps m tile w
template <int SW>
__device__ __forceinline__ void pk_kgroup_sum(const f4 (&acc)[SW][4], f4 (&own)[SW], char* smem) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6;
  f4* red = reinterpret_cast<f4*>(smem + PK_RED_OFF);
#pragma unroll
  for (int sl = 0; sl < SW; ++sl)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) red[((w * SW + sl) * 4 + mt) * 64 + lane] = acc[sl][mt];
  lds_barrier();
#pragma unroll
  for (int sl = 0; sl < SW; ++sl) {
    f4 s = red[((0 * SW + sl) * 4 + w) * 64 + lane];
#pragma unroll
    for (int q = 1; q < 4; ++q) s += red[((q * SW + sl) * 4 + w) * 64 + lane];
    own[sl] = s;
  }
}

// adaRMS on the pre-scaled product: this lane's quarter of the row sums of squares of row
// `lane` (issued before the product, added in the epilogue)
__device__ __forceinline__ float pk_rowss_quarter(const float* rss, int W1, int T) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6;
  const int ng = W1 >> 4, q = ng >> 2;  // partials per row / per wave (even: W1 % 128 == 0)
  const int row = min(lane, T - 1);
  const __amdgpu_buffer_rsrc_t rr = dev_rsrc(rss, (uint32_t)(T * ng * 4));
  f2 v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = 2 * i < q ? load_dev<f2>(rr, (row * ng + w * q + 2 * i) * 4) : (f2){0.f, 0.f};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += v[i][0] + v[i][1];
  return s;
}

// y = acc * rinv(m) / nscale + acc[shift row T]: the normalized adaRMS input times W^T.
// part = this wave's pk_rowss_quarter; own = m tile w after the k-group sum.
template <int SW>
__device__ __forceinline__ void pk_norm2(f4 (&own)[SW], float part, CPk& p, float nsc, char* smem) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  float* denom = reinterpret_cast<float*>(smem + PK_DENOM_OFF);
  f4* shiftacc = reinterpret_cast<f4*>(smem + PK_SHIFT_OFF);
  denom[w * 64 + lane] = part;
  if (w == (p.T >> 4) && r16 == (p.T & 15)) {
#pragma unroll
    for (int sl = 0; sl < SW; ++sl) shiftacc[sl * 4 + g] = own[sl];
  }
  lds_barrier();
  const int m = 16 * w + r16;
  const float tot = ((denom[m] + denom[64 + m]) + denom[128 + m]) + denom[192 + m];
  const float rinv = 1.0f / sqrtf(tot / (float)p.W1 + p.eps) / nsc;
#pragma unroll
  for (int sl = 0; sl < SW; ++sl) {
    const f4 sv = shiftacc[sl * 4 + g];
#pragma unroll
    for (int e = 0; e < 4; ++e) own[sl][e] = fmaf(own[sl][e], rinv, sv[e]);
  }
  lds_barrier();  // denom / shiftacc are free again
}

// split-K meeting: this task's partial (m tile w of its single slab) is stored, the last of
// the tile's S tasks to arrive adds all S partials in split order.  false: not the last.
__device__ __forceinline__ bool pk_splitk(f4& own, float* ws, unsigned* cnt, int tile, int s, int S, PkShared& sh) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6;
  if (S == 1) return true;
  const __amdgpu_buffer_rsrc_t rw = dev_rsrc(ws, 0x7FFFFF00);
  store_dev<f4>(rw, ((((tile * S + s) * 4 + w) * 64) + lane) * 16, own);
  pk_stores_done();  // every wave's partial store is complete
  if (pk_tid() == 0) {
    const unsigned old = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.is_last = (int)((old & (unsigned)(S - 1)) == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!sh.is_last) return false;
  f4 parts[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    if (q < S) parts[q] = load_dev<f4>(rw, ((((tile * S + q) * 4 + w) * 64) + lane) * 16);
  f4 sum = parts[0];
#pragma unroll
  for (int q = 1; q < 8; ++q)
    if (q < S) sum += parts[q];
  own = sum;
  return true;
}

// power-of-two prescale of norm n's pre-scaled input (computed by nscale_launch)
__device__ __forceinline__ float pk_nsc(CPk& p, int n) { return load_global(p.nscale + n); }

// ---- epilogues that produce the residual stream -----------------------------------------
// x_new = fp16(x_old + fp16(fp16(acc) * gate)) (gate == null: y = fp16(fp16(acc) + bias)),
// row m = 16 w + r16, columns col .. col + 3; also the row sums of squares per 16 columns
// (rss_out[m][col / 16]) and the next norm's pre-scaled input (fragment-major, shift row T).
struct ResOut {
  _Float16* x;
  float* rss;
  _Float16* u;
  const _Float16* mod;  // the next norm's [scale | shift | gate]
  float nsc;
};
__device__ __forceinline__ void pk_residual_epilogue(CPk& p, f4 acc, int col, const h4 xo, const h4 gq,
                                                     bool gated, const h4 bq, const ResOut& o, const h4 sc,
                                                     const h4 shf) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  const int m = 16 * w + r16;
  h4 xn;
  float s2 = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const _Float16 y = f2h(acc[e]);
    xn[e] = gated ? hadd(xo[e], hmul(y, gq[e])) : hadd(y, bq[e]);
    s2 += h2f(xn[e]) * h2f(xn[e]);
  }
  s2 = xor_sum_16_32(s2);  // the 16 columns of this slab: lanes g = 0..3 of row m
  const __amdgpu_buffer_rsrc_t rx = dev_rsrc(o.x, 0x7FFFFF00), rs = dev_rsrc(o.rss, 0x7FFFFF00),
                               ru = dev_rsrc(o.u, 0x7FFFFF00);
  if (m < p.T) {
    store_dev<h4>(rx, (m * p.W1 + col) * 2, xn);
    if (g == 0) store_dev<float>(rs, (m * (p.W1 >> 4) + (col >> 4)) * 4, s2);
    h4 u;
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = f2h(h2f(xn[e]) * (1.0f + h2f(sc[e])) * o.nsc);
    store_dev<h4>(ru, (int)xf_index(m, col) * 2, u);
  } else if (m == p.T) {
    store_dev<h4>(ru, (int)xf_index(m, col) * 2, shf);
  }
}

// ---- phases ---------------------------------------------------------------------------
// Phase order of one launch: 0 action_in; 1 + 6 L + j for layer L with j = 0 q/k/v,
// 1 attention, 2 combine, 3 o_proj, 4 gate_up, 5 down; 1 + 6 D the head.  Every phase
// function issues the weight loads of its first task, waits for the previous phase (all
// progress words >= target) and runs its tasks; false: a wait gave up.
enum : int { PH_AIN = 0, PH_QKV, PH_ATTN, PH_COMB, PH_OPROJ, PH_GATEUP, PH_DOWN, PH_HEAD };

// Read the arguments through a pointer the compiler cannot see through, once per phase:
// their loads then stay inside the phase instead of being hoisted to the top of the kernel
// and held in registers across every phase.
__device__ __forceinline__ CPk* launder(CPk* q) {
  asm volatile("" : "+s"(q));
  return q;
}

__device__ __forceinline__ void phase_ain(CPk& p) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  const int m = 16 * w + r16, W1 = p.W1, T = p.T;
  const _Float16* m0 = p.modp;  // norm 0: the input norm of layer 0
  const float nsc = pk_nsc(p, 0);
  for (int t = pk_bid(); t < W1 / 16; t += p.G) {
    f4 acc = (f4){0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < p.A / 32; ++ks) {
      const h8 a = load_global(reinterpret_cast<const h8*>(p.ain_w + (size_t)(16 * t + r16) * p.A + 32 * ks + 8 * g));
      const h8 x = m < T ? load_global(reinterpret_cast<const h8*>(p.xin + (size_t)m * p.A + 32 * ks + 8 * g))
                         : (h8){0, 0, 0, 0, 0, 0, 0, 0};
      acc = mfma16x16x32(a, x, acc);
    }
    const int col = 16 * t + 4 * g;
    const h4 bq = p.ain_b ? load_global(reinterpret_cast<const h4*>(p.ain_b + col)) : (h4){0, 0, 0, 0};
    const h4 sc = load_global(reinterpret_cast<const h4*>(m0 + col));
    const h4 shf = load_global(reinterpret_cast<const h4*>(m0 + W1 + col));
    const ResOut o{p.xres, p.rres, p.ures, m0, nsc};
    pk_residual_epilogue(p, acc, col, (h4){0, 0, 0, 0}, (h4){0, 0, 0, 0}, false, bq, o, sc, shf);
  }
}

template <int HD, bool Q4, int KP>
__device__ __forceinline__ bool phase_qkv(CPk& p, int L, unsigned target, PkShared& sh, char* smem) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  const int m = 16 * w + r16, T = p.T, W1 = p.W1, mc = min(m, T - 1);
  CPkLin* lw = ((CPkLin*)p.lw) + (size_t)L * PK_NLIN;
  const int nqt = p.nq / 16, nkt = p.nkv / 16, n = nqt + 2 * nkt, kpw = W1 / 128;
  const float nsc = pk_nsc(p, 2 * L);
  const _Float16* xu = p.ures + L * p.s_u;
  const float* rs = p.rres + L * p.s_r;
  auto seg_of = [&](int tt, int& li, int& slab) {
    li = tt < nqt ? PK_Q : tt < nqt + nkt ? PK_K : PK_V;
    slab = tt < nqt ? tt : tt < nqt + nkt ? tt - nqt : tt - nqt - nkt;
  };
  WRegs<Q4, 1> wr;
  int t = pk_bid();
  if (t < n) {
    int li, slab;
    seg_of(t, li, slab);
    pk_load_w<Q4, 1, KP>(wr, lw[li], slab, W1, w * kpw, kpw);
  }
  if (!pk_wait(p, target, sh)) return false;
  const float qscale = 1.0f / sqrtf((float)HD);
  for (; t < n; t += p.G) {
    int li, slab;
    seg_of(t, li, slab);
    if (t != (int)pk_bid()) pk_load_w<Q4, 1, KP>(wr, lw[li], slab, W1, w * kpw, kpw);
    h8 xf[PK_KPW][4];
    pk_load_x<Q4, KP>(xf, xu, W1, w * kpw, kpw, T);
    const float part_ss = pk_rowss_quarter(rs, W1, T);
    // RoPE tables of this lane's token and dims (q and k slabs pair rows d, d + HD/2)
    constexpr int spb = HD / 16;
    const int rope_d = 8 * (slab % spb) + 4 * (g & 1) + (g < 2 ? 0 : 2);
    const f2 cc = load_global(reinterpret_cast<const f2*>(p.cos + (size_t)mc * (HD / 2) + rope_d));
    const f2 ss = load_global(reinterpret_cast<const f2*>(p.sin + (size_t)mc * (HD / 2) + rope_d));
    f4 acc[1][4], own[1];
    pk_mma<Q4, 1, KP>(wr, xf, kpw, acc);
    pk_kgroup_sum<1>(acc, own, smem);
    pk_norm2<1>(own, part_ss, p, nsc, smem);
    CPkLin& lin = lw[li];
    const int col = 16 * slab + 4 * g;  // v: 4 consecutive columns of this lane
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      _Float16 tt = f2h(own[0][e]);
      if (lin.bias) tt = hadd(tt, lin.bias[col + e]);
      y[e] = h2f(tt);
    }
    if (li == PK_V) {  // uniform per task
      if (m < T) {
        const h4 v4 = {f2h(y[0]), f2h(y[1]), f2h(y[2]), f2h(y[3])};
        store_dev<h4>(dev_rsrc(p.vs + L * p.s_k, 0x7FFFFF00), (m * p.nkv + col) * 2, v4);
      }
      continue;
    }
    // the projection rounds to fp16 (the reference's q / k), RoPE in fp32 on those values;
    // lane ^ 32 holds the partner dims (d + HD/2 for lanes g < 2, d - HD/2 otherwise)
    const bool lo = g < 2;
    const float r0 = swap_halves(y[2], y[0], lo);
    const float r1 = swap_halves(y[3], y[1], lo);
    const float x1a = lo ? y[0] : r0, x1b = lo ? y[1] : r1;
    const float x2a = lo ? r0 : y[2], x2b = lo ? r1 : y[3];
    const float o1a = x1a * cc[0] - x2a * ss[0], o1b = x1b * cc[1] - x2b * ss[1];
    const float o2a = x2a * cc[0] + x1a * ss[0], o2b = x2b * cc[1] + x1b * ss[1];
    const int hh = slab / spb;  // head of this slab
    if (m < T && li == PK_Q) {
      const int grp = p.H / p.KV;
      const int kvh = hh / grp, row = (hh % grp) * T + m;
      const int ntiles = p.rpad / 16, nks = HD / 32;
      const __amdgpu_buffer_rsrc_t rq = dev_rsrc(p.qf + L * p.s_qf, 0x7FFFFF00);
      const float o[2][2] = {{o1a, o1b}, {o2a, o2b}};
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        h2 hi, lo2;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          _Float16 hv, lv;
          split_f32(o[hf][e] * qscale, hv, lv);
          hi[e] = hv;
          lo2[e] = lv;
        }
        const int d = rope_d + hf * (HD / 2);
        store_dev<h2>(rq, (int)attn_qf_index(kvh, ntiles, nks, row, d, 0) * 2, hi);
        store_dev<h2>(rq, (int)attn_qf_index(kvh, ntiles, nks, row, d, 1) * 2, lo2);
      }
    } else if (m < T) {
      const __amdgpu_buffer_rsrc_t rk = dev_rsrc(p.k32 + L * p.s_k, 0x7FFFFF00);
      const int kb = m * p.nkv + hh * HD + rope_d;
      store_dev<f2>(rk, kb * 4, (f2){o1a, o1b});
      store_dev<f2>(rk, (kb + HD / 2) * 4, (f2){o2a, o2b});
    }
  }
  return true;
}

__device__ __forceinline__ AttnArgs pk_attn_args(CPk& p, int L) {
  AttnArgs a{};
  a.Tq = p.T;
  a.H = p.H;
  a.KV = p.KV;
  a.hd = p.HD;
  a.kp = p.keys + (size_t)L * p.KV * p.P * p.HD;
  a.kp_f32 = 1;
  a.vp = p.values + (size_t)L * p.KV * p.P * p.HD;
  a.Sp = p.P;
  a.mask = p.mask;
  a.ks32 = p.k32 + L * p.s_k;
  a.ks_ld = p.nkv;
  a.vs = p.vs + L * p.s_k;
  a.vs_ld = p.nkv;
  a.Ts = p.T;
  a.qf = p.qf + L * p.s_qf;
  a.out = p.attn + L * p.s_attn;
  a.out_ld = p.nq;
  a.out_frag = 1;
  a.noskip = p.noskip;
  a.nsplit = p.nsplit;
  a.kps = p.kps;
  a.rows = p.rows;
  a.rpad = p.rpad;
  a.part_o = p.part + L * p.s_part;
  a.part_ml = a.part_o + (size_t)p.KV * p.nsplit * p.rpad * p.HD;  // the layout of attn_ws_floats
  return a;
}

// Workgroups without a task in the attention or combine phase pull weights of the later phases
// of this layer into the L2 of their XCD (the consumer of GEMM task t runs on workgroup t, XCD
// t % 8; L2 keeps its lines for the rest of the launch) and into the memory-side cache: one
// 4-byte load per 128-byte line, 8 in flight per thread.  idle0: the first idle workgroup;
// regions: task t's weights are task_bytes at base + (t - t0) * task_bytes for t in [t0, t1).
struct PfReg {
  const char* base;
  unsigned task_bytes;
  int t0, t1;
};
__device__ __forceinline__ void pk_touch(CPk& p, const PfReg* regs, int nreg, int idle0) {
  const int b = pk_bid(), x = b & 7, tid = pk_tid();
  const int f = idle0 + ((x - idle0) & 7);  // the first idle workgroup on this XCD
  if (b < f || f >= p.G) return;
  const int rank = (b - f) >> 3, nrank = (p.G - 1 - f) / 8 + 1;
  const int stride = nrank * PK_THREADS;
  unsigned acc = 0;
  for (int ri = 0; ri < nreg; ++ri) {
    const PfReg R = regs[ri];
    const int tf = R.t0 + ((x - R.t0) & 7);  // this XCD's first task of the region
    if (tf >= R.t1) continue;
    const int ntask = (R.t1 - 1 - tf) / 8 + 1;
    const int lpt = (int)(R.task_bytes >> 7);
    const int total = ntask * lpt;
    for (int l0 = rank * PK_THREADS + tid; l0 < total; l0 += 8 * stride) {
      unsigned v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int l = min(l0 + k * stride, total - 1);
        const int j = l / lpt, off = l - j * lpt;
        v[k] = load_global(reinterpret_cast<const unsigned*>(R.base + (size_t)(tf + 8 * j - R.t0) * R.task_bytes +
                                                             (size_t)off * 128));
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) acc ^= v[k];
    }
  }
  if (p.sink) p.sink[tid] = acc;  // keeps the loads (the sink is null)
}

// the o_proj, gate_up and down weights of layer L (fp16 slabs, or q4 blocks and scales)
template <bool Q4>
__device__ __forceinline__ int pk_layer_regions(CPk& p, int L, PfReg* r) {
  CPkLin* lw = (CPkLin*)p.lw + (size_t)L * PK_NLIN;
  const int n_o = (p.W1 / 16) * p.so, n_d = (p.W1 / 16) * p.sd, n_gu = p.F1 / (8 * p.gu_sw);
  const unsigned ko = p.nq / p.so, kd = p.F1 / p.sd, kg = p.W1 * p.gu_sw;  // k columns x slabs per task
  int n = 0;
  if constexpr (!Q4) {
    r[n++] = PfReg{(const char*)lw[PK_O].w, ko * 32, 0, n_o};   // 16 rows x k halfs per task
    r[n++] = PfReg{(const char*)lw[PK_GU].w, kg * 32, 0, n_gu};
    r[n++] = PfReg{(const char*)lw[PK_DN].w, kd * 32, 0, n_d};
  } else {
    r[n++] = PfReg{(const char*)lw[PK_O].qw, ko * 8, 0, n_o};   // 16 rows x k nibbles
    r[n++] = PfReg{(const char*)lw[PK_GU].qw, kg * 8, 0, n_gu};
    r[n++] = PfReg{(const char*)lw[PK_DN].qw, kd * 8, 0, n_d};
    r[n++] = PfReg{(const char*)lw[PK_O].qs, ko, 0, n_o};      // 16 rows x k / 32 scales
    r[n++] = PfReg{(const char*)lw[PK_GU].qs, kg, 0, n_gu};
    r[n++] = PfReg{(const char*)lw[PK_DN].qs, kd, 0, n_d};
  }
  return n;
}

__device__ __forceinline__ void pk_combine_row(const AttnArgs& a, int nsplit, int kvh, int row, int lane) {
  if (nsplit <= 8) combine_row<8, true>(a, kvh, row, lane);
  else if (nsplit <= 16) combine_row<16, true>(a, kvh, row, lane);
  else if (nsplit <= 24) combine_row<24, true>(a, kvh, row, lane);
  else combine_row<32, true>(a, kvh, row, lane);
}

// Joint attention of layer L.  With merge_comb (every task on its own workgroup), the key
// splits of a row block meet at the block's arrival counter once their partials are stored
// (each split adds 1; the counter is 0 at launch start: layer L's o_proj phase of the previous
// launch reset it), and split s then combines rows s * rps .. (s + 1) * rps - 1 of the block, one
// row per wave.
template <int HD, bool Q4>
__device__ __forceinline__ bool phase_attn(CPk& p, int L, unsigned target, PkShared& sh, char* smem) {
  if (!pk_wait(p, target, sh)) return false;
  const AttnArgs a = pk_attn_args(p, L);
  const int rb = p.rpad / 64, n = rb * p.nsplit * p.KV;
  const int rps = (64 + p.nsplit - 1) / p.nsplit;
  for (int t = pk_bid(); t < n; t += p.G) {
    const int rbi = t % rb, rest = t / rb, split = rest % p.nsplit, kvh = rest / p.nsplit;
    attn_block<HD, true, false, false, true, true>(a, rbi, split, kvh, smem, pk_tid());
    pk_stores_done();  // the partial stores are complete; the chunk buffers are free again
    if (p.merge_comb && p.nsplit > 1) {
      unsigned* ctr = p.cntm + ((size_t)L * p.KV + kvh) * rb + rbi;
      if (pk_tid() == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (!pk_wait_count(p, ctr, (unsigned)p.nsplit, sh)) return false;
      const int lane = pk_tid() & 63, w = pk_tid() >> 6;
      for (int r = split * rps + w; r < min(64, (split + 1) * rps); r += 4) {
        const int row = rbi * 64 + r;
        if (row < p.rows) pk_combine_row(a, p.nsplit, kvh, row, lane);
      }
    }
  }
  if (p.prefetch && n < p.G) {
    PfReg r[6];
    const int nr = pk_layer_regions<Q4>(p, L, r);
    pk_touch(p, r, nr, n);
  }
  return true;
}

__device__ __forceinline__ bool phase_comb(CPk& p, int L, unsigned target, PkShared& sh) {
  if (!pk_wait(p, target, sh)) return false;
  const int lane = pk_tid() & 63, w = pk_tid() >> 6;
  const AttnArgs a = pk_attn_args(p, L);
  const int n = (p.KV * p.rows + 3) / 4;
  for (int t = pk_bid(); t < n; t += p.G) {
    const int rr = 4 * t + w;
    if (rr < p.KV * p.rows) {
      const int kvh = rr / p.rows, row = rr % p.rows;
      pk_combine_row(a, p.nsplit, kvh, row, lane);
    }
  }
  return true;
}

// o_proj (down = false: K = nq over so slices, X = the attention output, residual x_in)
// or down (K = F1 over sd slices, X = the GeGLU output, residual x_mid), + gated residual,
// the residual's row statistics and the next norm's pre-scaled input
template <bool Q4, int KP>
__device__ __forceinline__ bool phase_res(CPk& p, int L, bool down, unsigned target, PkShared& sh,
                                          char* smem) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  const int m = 16 * w + r16, T = p.T, W1 = p.W1, mc = min(m, T - 1), D = p.D;
  const size_t W3 = (size_t)3 * W1;
  const int S = down ? p.sd : p.so, K = down ? p.F1 : p.nq;
  const int kslice = K / S / 32, kpw = kslice / 4, n = (W1 / 16) * S;
  CPkLin& lin = ((CPkLin*)p.lw)[(size_t)L * PK_NLIN + (down ? PK_DN : PK_O)];
  const _Float16* gate_mod = p.modp + (size_t)(down ? 2 * L + 1 : 2 * L) * W3;
  const int nn = down ? (L + 1 < D ? 2 * (L + 1) : 2 * D) : 2 * L + 1;  // the next norm
  const _Float16* mod_next = p.modp + (size_t)nn * W3;
  const _Float16* xold = down ? p.xmid + L * p.s_x : p.xres + L * p.s_x;
  const _Float16* X = down ? p.h + L * p.s_h : p.attn + L * p.s_attn;
  const ResOut o = down ? ResOut{p.xres + (L + 1) * p.s_x, p.rres + (L + 1) * p.s_r, p.ures + (L + 1) * p.s_u,
                                 mod_next, pk_nsc(p, nn)}
                        : ResOut{p.xmid + L * p.s_x, p.rmid + L * p.s_r, p.umid + L * p.s_u, mod_next,
                                 pk_nsc(p, nn)};
  float* ws = down ? p.skd + L * p.s_skd : p.sko + L * p.s_sko;
  unsigned* cnt = (down ? p.cntd : p.cnto) + (size_t)L * (W1 / 16);
  WRegs<Q4, 1> wr;
  h4 xo, gq, sc, shf;
  // the residual x_old is complete before this phase's wait (o_proj: the q/k/v phase waited
  // for it; down: gate_up waited for o_proj); the gate and the next norm are inputs
  auto operands = [&](int tt) {
    const int col = 16 * (tt / S) + 4 * g;
    xo = load_dev<h4>(dev_rsrc(xold, 0x7FFFFF00), (mc * W1 + col) * 2);
    gq = load_global(reinterpret_cast<const h4*>(gate_mod + 2 * W1 + col));
    sc = load_global(reinterpret_cast<const h4*>(mod_next + col));
    shf = load_global(reinterpret_cast<const h4*>(mod_next + W1 + col));
  };
  int t = pk_bid();
  if (t < n) pk_load_w<Q4, 1, KP>(wr, lin, t / S, K, (t % S) * kslice + w * kpw, kpw);
  if (!pk_wait(p, target, sh)) return false;
  if (!down && p.merge_comb && p.nsplit > 1) {
    // every workgroup has left layer L's attention phase (this wait): its row-block counters
    // go back to 0 for the next launch, whose combiners wait for exactly nsplit arrivals
    const int nc = p.KV * (p.rpad / 64);
    if (pk_tid() == 0)
      for (int c = pk_bid(); c < nc; c += p.G)
        __hip_atomic_store(p.cntm + (size_t)L * nc + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  for (; t < n; t += p.G) {
    const int tile = t / S, s = t % S;
    const int kbase = s * kslice + w * kpw;
    if (t != (int)pk_bid()) pk_load_w<Q4, 1, KP>(wr, lin, tile, K, kbase, kpw);
    h8 xf[PK_KPW][4];
    pk_load_x<Q4, KP>(xf, X, K, kbase, kpw, T - 1);
    operands(t);  // behind X: wave 0's poll above did not wait for them
    f4 acc[1][4], own[1];
    pk_mma<Q4, 1, KP>(wr, xf, kpw, acc);
    pk_kgroup_sum<1>(acc, own, smem);
    if (!pk_splitk(own[0], ws, cnt, tile, s, S, sh)) continue;
    pk_residual_epilogue(p, own[0], 16 * tile + 4 * g, xo, gq, true, (h4){0, 0, 0, 0}, o, sc, shf);
  }
  return true;
}

template <bool Q4, int SW, int KP>
__device__ __forceinline__ bool phase_gateup(CPk& p, int L, unsigned target, PkShared& sh, char* smem) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  const int m = 16 * w + r16, T = p.T, W1 = p.W1, kpw = W1 / 128;
  const int n = p.F1 / (8 * SW);
  const float nsc = pk_nsc(p, 2 * L + 1);
  const _Float16* xu = p.umid + L * p.s_u;
  const float* rs = p.rmid + L * p.s_r;
  CPkLin& lin = ((CPkLin*)p.lw)[(size_t)L * PK_NLIN + PK_GU];
  WRegs<Q4, SW> wr;
  int t = pk_bid();
  if (t < n) pk_load_w<Q4, SW, KP>(wr, lin, SW * t, W1, w * kpw, kpw);
  if (!pk_wait(p, target, sh)) return false;
  const __amdgpu_buffer_rsrc_t rh = dev_rsrc(p.h + L * p.s_h, 0x7FFFFF00);
  for (; t < n; t += p.G) {
    if (t != (int)pk_bid()) pk_load_w<Q4, SW, KP>(wr, lin, SW * t, W1, w * kpw, kpw);
    h8 xf[PK_KPW][4];
    pk_load_x<Q4, KP>(xf, xu, W1, w * kpw, kpw, T);
    const float part_ss = pk_rowss_quarter(rs, W1, T);
    f4 acc[SW][4], own[SW];
    pk_mma<Q4, SW, KP>(wr, xf, kpw, acc);
    pk_kgroup_sum<SW>(acc, own, smem);
    pk_norm2<SW>(own, part_ss, p, nsc, smem);
    // lanes g < 2 hold 4 gate columns, lane ^ 32 the matching up columns: each lane
    // finishes 2 outputs of its slab
    const bool lo = g < 2;
#pragma unroll
    for (int sl = 0; sl < SW; ++sl) {
      const float r0 = swap_halves(own[sl][2], own[sl][0], lo);
      const float r1 = swap_halves(own[sl][3], own[sl][1], lo);
      const float ga = lo ? own[sl][0] : r0, gb = lo ? own[sl][1] : r1;
      const float ua = lo ? r0 : own[sl][2], ub = lo ? r1 : own[sl][3];
      h2 o;
      o[0] = hmul(f2h(gelu_tanh_hw(h2f(f2h(ga)))), f2h(ua));
      o[1] = hmul(f2h(gelu_tanh_hw(h2f(f2h(gb)))), f2h(ub));
      const int col = 8 * (SW * t + sl) + 4 * (g & 1) + (lo ? 0 : 2);
      if (m < T) store_dev<h2>(rh, (int)xf_index(m, col) * 2, o);
    }
  }
  return true;
}

template <bool Q4, int KP>
__device__ __forceinline__ bool phase_head(CPk& p, unsigned target, PkShared& sh, char* smem) {
  const int lane = pk_tid() & 63, w = pk_tid() >> 6, g = lane >> 4, r16 = lane & 15;
  const int m = 16 * w + r16, T = p.T, W1 = p.W1, D = p.D, kpw = W1 / 128;
  const float nsc = pk_nsc(p, 2 * D);
  const _Float16* xu = p.ures + D * p.s_u;
  const float* rs = p.rres + D * p.s_r;
  const int n = p.A / 16;
  WRegs<Q4, 1> wr;
  int t = pk_bid();
  if (t < n) pk_load_w<Q4, 1, KP>(wr, p.aout, t, W1, w * kpw, kpw);
  if (!pk_wait(p, target, sh)) return false;
  for (; t < n; t += p.G) {
    if (t != (int)pk_bid()) pk_load_w<Q4, 1, KP>(wr, p.aout, t, W1, w * kpw, kpw);
    h8 xf[PK_KPW][4];
    pk_load_x<Q4, KP>(xf, xu, W1, w * kpw, kpw, T);
    const float part_ss = pk_rowss_quarter(rs, W1, T);
    f4 acc[1][4], own[1];
    pk_mma<Q4, 1, KP>(wr, xf, kpw, acc);
    pk_kgroup_sum<1>(acc, own, smem);
    pk_norm2<1>(own, part_ss, p, nsc, smem);
    const int col = 16 * t + 4 * g;
    const h4 bq = p.aout.bias ? load_global(reinterpret_cast<const h4*>(p.aout.bias + col)) : (h4){0, 0, 0, 0};
    if (m < T) {
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = h2f(hadd(f2h(own[0][e]), bq[e]));
      if (p.euler) {
        f4 x = *reinterpret_cast<const f4*>(p.x32 + (size_t)m * p.A + col);
        h4 xh;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = euler_update(x[e], p.dt, y[e]);
          xh[e] = f2h(x[e]);
        }
        *reinterpret_cast<f4*>(p.x32 + (size_t)m * p.A + col) = x;
        *reinterpret_cast<h4*>(p.x16 + (size_t)m * p.A + col) = xh;
      } else {
        *reinterpret_cast<f4*>(p.vout + (size_t)m * p.A + col) = (f4){y[0], y[1], y[2], y[3]};
      }
    }
  }
  return true;
}

// ---- the kernel ----------------------------------------------------------------------
template <int HD, bool Q4>
__global__ __launch_bounds__(PK_THREADS) void pstep_kernel(PkArgs args) {
  __shared__ __attribute__((aligned(16))) char smem[pk_smem_bytes<HD>()];
  __shared__ PkShared sh;
  (void)args;  // read in place: the only argument, at offset 0 of the kernarg segment
  CPk* ka = (CPk*)__builtin_amdgcn_kernarg_segment_ptr();
  const unsigned base = ld_agent(ka->prog + pk_bid());
  const int ppl = ka->merge_comb ? 5 : 6;  // phases per layer
  const int nph = 2 + ppl * ka->D;
  for (int ph = 0; ph < nph; ++ph) {
    CPk& p = *launder(ka);
    const unsigned target = base + (unsigned)ph;  // every workgroup has published phase ph - 1
    const int L = (ph - 1) / ppl, j = (ph - 1) % ppl;
    const int type = ph == 0 ? PH_AIN : ph == nph - 1 ? PH_HEAD : ppl == 6 || j < 2 ? 1 + j : 2 + j;
    bool ok = true;
#ifdef MLCV_PK_TRACE
    if (pk_tid() == 0) pk_trace_ph = ph;
#endif
    PK_STAMP(0);
    // the pi0.5 shapes (8 k steps per wave in every GEMM) take the straight-line code
    const bool k8 = p.W1 == 1024;
    switch (type) {
      case PH_AIN: phase_ain(p); break;
      case PH_QKV:
        ok = k8 ? phase_qkv<HD, Q4, 8>(p, L, target, sh, smem) : phase_qkv<HD, Q4, 0>(p, L, target, sh, smem);
        break;
      case PH_ATTN: ok = phase_attn<HD, Q4>(p, L, target, sh, smem); break;
      case PH_COMB: ok = phase_comb(p, L, target, sh); break;
      case PH_OPROJ:
        ok = p.nq / p.so == 1024  ? phase_res<Q4, 8>(p, L, false, target, sh, smem)
             : p.nq / p.so == 512 ? phase_res<Q4, 4>(p, L, false, target, sh, smem)
                                  : phase_res<Q4, 0>(p, L, false, target, sh, smem);
        break;
      case PH_GATEUP:
        if (p.gu_sw == 2)
          ok = k8 ? phase_gateup<Q4, 2, 8>(p, L, target, sh, smem) : phase_gateup<Q4, 2, 0>(p, L, target, sh, smem);
        else
          ok = phase_gateup<Q4, 1, 0>(p, L, target, sh, smem);
        break;
      case PH_DOWN:
        ok = p.F1 / p.sd == 1024 ? phase_res<Q4, 8>(p, L, true, target, sh, smem)
                                 : phase_res<Q4, 0>(p, L, true, target, sh, smem);
        break;
      default: ok = k8 ? phase_head<Q4, 8>(p, target, sh, smem) : phase_head<Q4, 0>(p, target, sh, smem); break;
    }
    if (!ok) return;
    PK_STAMP(2);
    pk_publish(p, base + (unsigned)ph + 1u);
    PK_STAMP(3);
  }
}

}  // namespace

bool pk_head_dim_ok(int hd) { return hd == 64 || hd == 128 || hd == 256; }

#ifdef MLCV_PK_TRACE
}  // namespace mlcv
extern "C" void* mlcv_pk_trace_ptr() {
  void* p = nullptr;
  (void)hipGetSymbolAddress(&p, HIP_SYMBOL(mlcv::pk_trace));
  return p;
}
namespace mlcv {
#endif

int pk_launch(const PkArgs& p, bool q4, hipStream_t st) {
  MLCV_REQUIRE(p.T >= 1 && p.T < 64, "persistent step: 1 <= T < 64");
  MLCV_REQUIRE(p.W1 % 128 == 0 && p.W1 / 128 <= PK_KPW && p.F1 % 128 == 0 && p.nq % 128 == 0, "persistent step widths");
  MLCV_REQUIRE(p.A % 32 == 0 && p.nkv % 16 == 0, "persistent step: action_dim % 32, kv width % 16");
  MLCV_REQUIRE(p.so >= 1 && (p.so & (p.so - 1)) == 0 && p.so <= 8 && p.sd >= 1 && (p.sd & (p.sd - 1)) == 0 &&
                   p.sd <= 8,
               "split-K slices must be powers of two up to 8");
  const int kpw_o = p.nq / p.so / 128, kpw_d = p.F1 / p.sd / 128;
  MLCV_REQUIRE(p.nq % (p.so * 128) == 0 && p.F1 % (p.sd * 128) == 0 && kpw_o >= 1 && kpw_o <= PK_KPW && kpw_d >= 1 &&
                   kpw_d <= PK_KPW,
               "split-K slices must hold 128 to 1024 columns of K per wave");
  MLCV_REQUIRE(!q4 || ((p.W1 / 128) % 4 == 0 && kpw_o % 4 == 0 && kpw_d % 4 == 0),
               "q4 persistent step: whole 128-k chunks per wave");
  MLCV_REQUIRE(p.gu_sw == 1 || p.gu_sw == 2, "gate_up slabs per task");
  MLCV_REQUIRE(p.F1 % (8 * p.gu_sw) == 0, "gate_up tiles");
  MLCV_REQUIRE(p.G >= 1 && p.G <= 512, "persistent step: 1..512 workgroups");
  MLCV_REQUIRE(p.nsplit >= 1 && p.nsplit <= 32 && p.rpad % 64 == 0 && p.rows == p.T * (p.H / p.KV),
               "persistent step attention plan");
  MLCV_REQUIRE(p.prog && p.err && p.lw && p.modp && p.nscale, "persistent step buffers");
  MLCV_REQUIRE(!p.merge_comb || (p.cntm && (p.rpad / 64) * p.nsplit * p.KV <= p.G),
               "merged combine: every attention task on its own workgroup");
  MLCV_REQUIRE(pk_head_dim_ok(p.HD), "persistent step head_dim");
#define MLCV_PK_CASE(HDV)                                                        \
  case HDV:                                                                      \
    if (q4) pstep_kernel<HDV, true><<<p.G, PK_THREADS, 0, st>>>(p);             \
    else pstep_kernel<HDV, false><<<p.G, PK_THREADS, 0, st>>>(p);               \
    break;
  switch (p.HD) {
    MLCV_PK_CASE(64)
    MLCV_PK_CASE(128)
    MLCV_PK_CASE(256)
    default: MLCV_REQUIRE(false, "persistent step head_dim");
  }
#undef MLCV_PK_CASE
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
