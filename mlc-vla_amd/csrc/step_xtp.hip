// XCD tensor-parallel denoise step: the decoder layers of denoise_step_kv (pi0_model.py:142-163;
// decode_suffix / decode_e1 gemma_dual.py:343-351,417-433; attn_decode_e1 + _sdpa :97-122,
// 255-275; adaRMS :60-88; GeGLU :125-135; gated residual :91-94) as two launches per layer.
//
// At T = 50 every op of a layer is a few microseconds of latency chains over little data, and
// every edge between ops is all-to-all.  MI355X has 8 XCDs of 32 CUs, each with its own L2: a
// barrier among the 32 workgroups of one XCD (flags in that L2) costs about 0.5 us, a barrier
// across XCDs (flags and data written through to the memory side) 3-4 us, a kernel boundary in
// a graph about 1.7 us.  So the layer runs tensor-parallel over the XCDs, Megatron style:
//   XCD x owns query head x: its q rows, its attention over all keys, and columns
//   [256 x, 256 x + 256) of o_proj's K (a row-parallel partial of o_proj's output);
//   it computes the shared k and v itself (all 8 XCDs read the same 1 MB of k/v weights);
//   XCD x owns MLP columns [512 x, 512 x + 512): their gate/up rows and down's K slice.
// The two cross-XCD sums of a layer (o_proj's and down's 8 partials) fall on the launch
// boundaries: the next launch starts with every XCD adding the 8 partials of residual
// columns [32 s, 32 s + 32) in workgroup s, so each XCD holds its own copy of the residual
// stream.  All other edges are barriers inside one XCD.
//
//   launch A (layer L): [action_in | down partials -> x] . q/k/v . attention . combine . o_proj
//   launch B (layer L): [o_proj partials -> x_mid] . gate_up + GeGLU . down
//   final:              [down partials -> x] in the launch chain's layout (its head runs next)
//
// A workgroup is 8 waves.  Waves 0-3 carry the critical path: the barrier polls, activation
// loads, MFMA, epilogue stores.  Waves 4-7 stream: they move the weights of the coming stage into
// LDS with buffer-to-LDS DMA, and (launch A, waves 6-7) build the attention's key chunk (K split
// hi/lo, V transposed) before the attention's inputs are ready.  The split matters: a wave's
// memory operations complete in issue order against one counter, so a wave that polls a flag or
// waits for its own stores would also wait for every weight load it issued before; and the
// q/k/v weights (needed at barrier 1) and the key chunk (needed at barrier 2) are in different
// waves, so barrier 1 waits for the first only.
//
// Each launch starts bound by the memory side (the weights of its first stage, 5-6 TB/s over all
// CUs); the rest is a chain of L2 round trips and barriers.  Loads that pull the next launch's
// weights into L2 during that chain delay the chain's own loads on the same CU (they share its
// vector memory path) by about as much as they save the next launch, so there are none.
//
// Intra-XCD data is written with plain stores (L2) and read with device-scope loads (which miss
// the CU's L1 and hit the XCD's L2); barrier words are plain stores polled with device-scope loads.
// Every barrier wait is bounded; a wait that gives up sets the error word and the workgroup leaves.
#include "attn_impl.h"

namespace mlcv {

#ifdef MLCV_XT_TRACE
// timeline of the last step for the trace build: [launch 2 L + (MLP half)][workgroup][stamp] in
// s_memrealtime ticks (100 MHz); stamps 0-10 by thread 0 (compute), 11-15 by thread 256 (stream)
__device__ unsigned long long xt_trace[64 * 256 * 16];
#define XT_STAMP(launch, k, who)                                                                           \
  do {                                                                                                     \
    if (threadIdx.x == (who))                                                                              \
      xt_trace[((size_t)(launch) * 256 + blockIdx.x) * 16 + (k)] = __builtin_amdgcn_s_memrealtime();       \
  } while (0)
#else
#define XT_STAMP(launch, k, who) \
  do {                           \
  } while (0)
#endif

namespace {

constexpr int XT_NX = 8;        // XCDs
constexpr int XT_NS = 32;       // workgroups (CUs) per XCD
constexpr int XT_NT = 512;      // threads: 4 compute waves + 4 stream waves
constexpr int XT_NC = 256;      // compute threads
constexpr int XT_W = 1024;      // action expert width
constexpr int XT_F = 4096;      // MLP width
constexpr int XT_HD = 256;      // head dim
constexpr int XT_FX = XT_F / XT_NX;  // MLP columns per XCD
constexpr int XT_RSS = XT_W / 16;    // row-sum partials per row (16 columns each)
constexpr int XT_KCH = KCH;          // keys per workgroup: one chunk
static_assert(XT_W / XT_NS == 32, "32 residual columns per workgroup");

typedef __attribute__((address_space(3))) void* lptr_t;
// cache policy of the loads of data another workgroup of this XCD wrote earlier in the same launch
// (plain: each such buffer is written before any workgroup of the launch reads it, and read once
// per workgroup, so no CU's L1 holds a stale line; 25-40 us per step faster than device scope)
#ifndef MLCV_XT_LOC_AUX
#define MLCV_XT_LOC_AUX 0
#endif
constexpr int LOC = MLCV_XT_LOC_AUX;
// the weight table read through the constant address space: scalar loads, so the buffer
// descriptors built from it stay uniform (a vector load would wrap every DMA in a loop)
typedef __attribute__((address_space(4))) const PkLin CPkLinX;
__device__ __forceinline__ const _Float16* xt_weights(const XtArgs& a, int L, int which) {
  return ((CPkLinX*)a.lw)[(size_t)L * PK_NLIN + which].w;
}
// q4f16_1 models (quant.py:176-193, 301-325): per 16-row slab and 128-k chunk, a 1 KB block of
// nibbles (lane l: row l & 15, the 32 k of quantization group l >> 4 of the chunk, as the
// fragment-major shuffle packs them) and a 128-byte block of the 64 lanes' fp16 scales
__device__ __forceinline__ const uint32_t* xt_qw(const XtArgs& a, int L, int which) {
  return ((CPkLinX*)a.lw)[(size_t)L * PK_NLIN + which].qw;
}
__device__ __forceinline__ const _Float16* xt_qs(const XtArgs& a, int L, int which) {
  return ((CPkLinX*)a.lw)[(size_t)L * PK_NLIN + which].qs;
}

// ---- LDS layouts (bytes) --------------------------------------------------------------
constexpr int XT_KVB = ((int)sizeof(AttnSmem<XT_HD>) + 255) / 256 * 256;
constexpr int XT_PLD = XT_HD + 8;                 // halfs per staged partial row
// launch A
constexpr int XA_W = 0;                           // q/k/v weights: 2 slabs x 32 KB
constexpr int XA_STAGE = 0;                       // after q/k/v: attention partial rows, 4 waves x 16
constexpr int XA_WO = 36864;                      // o_proj weights: 2 slabs x 8 KB (during the attention)
constexpr int XA_KV = 65536;                      // the key chunk
constexpr int XA_RED = XA_KV + XT_KVB;            // k-group sums [4 waves][2 slabs][4 m tiles][64] f4
constexpr int XA_DEN = XA_RED + 4 * 2 * 4 * 64 * 16;
constexpr int XA_BYTES = XA_DEN + 4 * 64 * 4;
static_assert(XA_STAGE + 4 * 16 * XT_PLD * 2 <= XA_WO && XA_WO + 16384 <= XA_KV, "launch A LDS");
static_assert(XA_BYTES <= 160 * 1024, "launch A LDS");
// q4: nibble blocks (1 KB per slab and 128-k chunk) at the same offsets, their scales after them
constexpr int XA_WSC = XA_W + 16384;              // q/k/v: 2 slabs x 8 chunks; scales 2 KB
constexpr int XA_WOSC = XA_WO + 4096;             // o_proj: 2 slabs x 2 chunks; scales 512 B
// launch B
constexpr int XB_GU = 0;                          // gate_up weights: 2 slabs x 32 KB
constexpr int XB_DN = 65536;                      // down weights: 2 slabs x 16 KB
constexpr int XB_RED = XB_DN + 32768;
constexpr int XB_DEN = XB_RED + 4 * 2 * 4 * 64 * 16;
constexpr int XB_BYTES = XB_DEN + 4 * 64 * 4;
static_assert(XB_BYTES <= 160 * 1024, "launch B LDS");
constexpr int XB_GUSC = XB_GU + 16384;            // q4 gate_up: 2 slabs x 8 chunks; scales 2 KB
constexpr int XB_DNSC = XB_DN + 8192;             // q4 down: 2 slabs x 4 chunks; scales 1 KB
static_assert(XA_WSC + 2048 <= XA_WO && XA_WOSC + 512 <= XA_KV && XB_GUSC + 2048 <= XB_DN && XB_DNSC + 1024 <= XB_RED,
              "q4 LDS");
// q4 with the stream waves unpacking (MLCV_XT_Q4_UNPACK, default on): the nibble blocks and scales
// land in a staging area and the stream waves write the fp16 slab layout of the fp16 product, so
// the compute waves run the same product as for fp16 weights.  Staging: launch A, the k-group sum
// area (free until the q/k/v product ends): 2 slabs x 8 chunks of 1 KB, then their 2 KB of scales;
// launch B, past its fp16 layout: up to 2 slabs x 8 chunks and 2 KB of scales
#ifndef MLCV_XT_Q4_UNPACK
#define MLCV_XT_Q4_UNPACK 3
#endif
// bit 0: launch A's q/k/v; bit 1: launch B's gate_up and down
constexpr bool XT_UNPACK_A = (MLCV_XT_Q4_UNPACK & 1) != 0, XT_UNPACK = (MLCV_XT_Q4_UNPACK & 2) != 0;
constexpr int XA_ST = XA_RED, XA_STSC = XA_ST + 16384;
constexpr int XB_ST = XB_BYTES, XB_STSC = XB_ST + 16384, XB_BYTES_Q4 = XB_STSC + 2048;
static_assert(XA_STSC + 2048 <= XA_RED + 4 * 2 * 4 * 64 * 16 && XB_BYTES_Q4 <= 160 * 1024, "q4 staging LDS");

struct XtSh {
  unsigned base;  // this workgroup's barrier word at launch start (equal across the XCD)
  int ok;
};

// thread index / XCD through copies the compiler cannot hoist or fold
__device__ __forceinline__ int xt_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int xt_xcd() {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return (int)(x & 7u);
}
__device__ __forceinline__ unsigned xt_ld_agent(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// every wave of the workgroup: its LDS accesses done, then s_barrier
__device__ __forceinline__ void xt_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
template <int N>
__device__ __forceinline__ void xt_vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
  asm volatile("" ::: "memory");
}

// Barrier k of the XCD's 32 workgroups, first half: the compute waves' stores are complete,
// the workgroup meets, thread 0 raises its word to base + k.
__device__ __forceinline__ void xt_arrive(const XtArgs& a, int h, int s, bool comp, unsigned k, const XtSh& sh) {
  if (comp) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);
  }
  xt_sync();
  if (xt_tid() == 0) {
    const __amdgpu_buffer_rsrc_t rf = dev_rsrc(a.flags, XT_NX * XT_NS * 4);
    __builtin_amdgcn_raw_buffer_store_b32(sh.base + k, rf, (h * XT_NS + s) * 4, 0, 0);
  }
}
// second half: wave 0 polls the 32 words of this XCD (and the error word); every wave meets.
// false: the wait gave up (or another workgroup's did), the workgroup must leave.
__device__ __forceinline__ bool xt_wait(const XtArgs& a, int h, unsigned k, XtSh& sh) {
  if (xt_tid() < 64) {
    const int lane = xt_tid();
    const unsigned target = sh.base + k;
    bool ok = false, failed = false;
    for (unsigned it = 0; it < a.spin; ++it) {
      const unsigned v = lane < XT_NS ? xt_ld_agent(a.flags + h * XT_NS + lane) : target;
      const unsigned e = xt_ld_agent(a.err);
      if (__all((int)(v - target) >= 0)) {
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
      if (!ok && !failed) __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.ok = ok ? 1 : 0;
    }
  }
  xt_sync();
  return sh.ok != 0;
}

// ---- stream waves: weight blocks into LDS -------------------------------------------------
// 1 KB block `blk` of a fragment-major weight run (64 lanes x 16 B) into LDS at dst
__device__ __forceinline__ void xt_dma(__amdgpu_buffer_rsrc_t r, int blk, char* dst, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)dst, 16, blk * 1024 + lane * 16, 0, 0, 0);
#endif
}

// 256 bytes (64 lanes x 4 B) at byte `off` of the run into LDS at dst: two chunks' q4 scales
__device__ __forceinline__ void xt_dma4(__amdgpu_buffer_rsrc_t r, int off, char* dst, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)dst, 4, off + lane * 4, 0, 0, 0);
#endif
}
// the q4 blocks of `nch` consecutive chunks from chunk c0 of 16-row slab `slab` of a matrix of
// kcn chunks per slab, into LDS slot `slot` of an area of `lch` chunks per slab (nibbles at wq,
// scales at wsc); stream wave v of nv takes every nv-th 1 KB block and 256-byte scale piece
__device__ __forceinline__ void xt_dma_q4(const uint32_t* qw, const _Float16* qs, int slab, int kcn, int c0, int nch,
                                          char* wq, char* wsc, int slot, int lch, int v, int nv, int lane) {
  const size_t b0 = (size_t)slab * kcn + c0;  // first block of the run
  const __amdgpu_buffer_rsrc_t rq = dev_rsrc(qw + b0 * 256, nch * 1024);
  const __amdgpu_buffer_rsrc_t rs = dev_rsrc(qs + b0 * 64, nch * 128);
  for (int c = v; c < nch; c += nv) xt_dma(rq, c, wq + (slot * lch + c) * 1024, lane);
  for (int c = 2 * v; c < nch; c += 2 * nv) xt_dma4(rs, c * 128, wsc + (slot * lch + c) * 128, lane);
}

// q4 blocks for the stream waves' unpacking: `nch` chunks from chunk c0 of 16-row slab `slab` (kcn
// chunks per slab) into staging slot sl (nibble blocks at wq + (sl nch + c) KB, scales at wsc +
// (sl nch + c) 128 B).  Chunk pair p of the slot (2 nibble blocks and their 256 bytes of scales,
// one 4-byte-per-lane DMA) belongs to stream wave (sl nch / 2 + p) mod nv, which also unpacks it.
__device__ __forceinline__ void xt_dma_q4_pairs(const uint32_t* qw, const _Float16* qs, int slab, int kcn, int c0,
                                                int nch, char* wq, char* wsc, int sl, int v, int nv, int lane) {
  const size_t b0 = (size_t)slab * kcn + c0;
  const __amdgpu_buffer_rsrc_t rq = dev_rsrc(qw + b0 * 256, nch * 1024);
  const __amdgpu_buffer_rsrc_t rs = dev_rsrc(qs + b0 * 64, nch * 128);
  for (int p = 0; p < nch / 2; ++p) {
    if ((sl * (nch / 2) + p) % nv != v) continue;
    xt_dma(rq, 2 * p, wq + (sl * nch + 2 * p) * 1024, lane);
    xt_dma(rq, 2 * p + 1, wq + (sl * nch + 2 * p + 1) * 1024, lane);
    xt_dma4(rs, 2 * p * 128, wsc + (sl * nch + 2 * p) * 128, lane);
  }
}
// 8 consecutive weights of one q4 word in k order: (n - 7) * scale in fp16 (quant.py:176-193), the
// same two fp16 roundings as dequant_word (only the element order differs)
__device__ __forceinline__ h8 dequant_word_nat(uint32_t word, _Float16 s) {
  h8 r;
  const h2 bias = {(_Float16)1031.0f, (_Float16)1031.0f};
  const h2 sc = {s, s};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t bits = ((word >> (8 * p)) & 0xFu) | (((word >> (8 * p + 4)) & 0xFu) << 16) | 0x64006400u;
    h2 v = __builtin_bit_cast(h2, bits);
    v = (v - bias) * sc;
    r[2 * p] = v[0];
    r[2 * p + 1] = v[1];
  }
  return r;
}
// this stream wave's chunk pairs of staging slot sl into the fp16 slab layout of xt_mma (block
// (sl, k step kw) at wl + (sl WKS + kw) KB, lane 16 g + r holding W[r][32 kw + 8 g .. +7]); q4 lane
// 16 gq + r holds row r's quantization group gq of the chunk, word j its k 8 j .. 8 j + 7
__device__ __forceinline__ void xt_unpack_q4_pairs(const char* wq, const char* wsc, int nch, char* wl, int WKS, int sl,
                                                   int v, int nv, int lane) {
  const int r = lane & 15, gq = lane >> 4;
  for (int p = 0; p < nch / 2; ++p) {
    if ((sl * (nch / 2) + p) % nv != v) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = 2 * p + i, kw = 4 * c + gq;
      const u4 q = *reinterpret_cast<const u4*>(wq + ((sl * nch + c) * 64 + lane) * 16);
      const _Float16 sc = *reinterpret_cast<const _Float16*>(wsc + ((sl * nch + c) * 64 + lane) * 2);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<h8*>(wl + ((sl * WKS + kw) * 64 + 16 * j + r) * 16) = dequant_word_nat(q[j], sc);
    }
  }
}

// ---- compute waves: the skinny GEMM pieces ---------------------------------------------------
// this wave's X fragments (fragment-major [64][K], device-scope loads): k steps ks0 .. ks0 + KPW - 1
// of the 4 m tiles; rows past xlast read zeros (an offset past the buffer)
// q4 (ks0 a multiple of 4): the weights' k order, k step kk of chunk kk / 4 taking 32-k block
// ks0 + 4 (kk / 4) + g of the lane's group g and its 8-k piece kk & 3 (perm8 before the MFMA)
template <int KPW, bool Q4 = false>
__device__ __forceinline__ void xt_load_x(h8 (&xf)[KPW][4], const _Float16* x, int K, int ks0, int xlast, int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const __amdgpu_buffer_rsrc_t rx = dev_rsrc(x, (uint32_t)(64 * K * 2));
#pragma unroll
  for (int kk = 0; kk < KPW; ++kk)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int ks = Q4 ? ks0 + 4 * (kk >> 2) + g : ks0 + kk, piece = Q4 ? 16 * (kk & 3) + r16 : lane;
      const int off = 16 * mt + r16 <= xlast ? ((ks * 4 + mt) * 64 + piece) * 16 : 0x7FFFFF00;
      xf[kk][mt] = load_dev<h8, LOC>(rx, off);
    }
}
// acc[sl][mt] = sum over this wave's k steps of W(sl, k) X(k, mt); W block (slab sl, k step kw)
// in LDS at wl + (sl * WKS + kw) * 1024 (the DMA's layout); slabs past nsl are not multiplied
template <int KPW>
__device__ __forceinline__ void xt_mma(f4 (&acc)[2][4], const h8 (&xf)[KPW][4], const char* wl, int WKS, int kw0,
                                       int nsl, int lane) {
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[sl][mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < KPW; ++kk) {
    const h8 a0 = *reinterpret_cast<const h8*>(wl + ((0 * WKS + kw0 + kk) * 64 + lane) * 16);
    const h8 a1 = *reinterpret_cast<const h8*>(wl + ((1 * WKS + kw0 + kk) * 64 + lane) * 16);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      acc[0][mt] = mfma16x16x32(a0, xf[kk][mt], acc[0][mt]);
      if (nsl > 1) acc[1][mt] = mfma16x16x32(a1, xf[kk][mt], acc[1][mt]);
    }
  }
}
// q4: the same product from q4 blocks in LDS (nibbles at wq, scales at wsc, lch chunks per slab):
// chunks c0 .. c0 + KPW / 4 - 1 of slab SL0 (and of slab SL0 + 1 when nsl > 1); the other
// slab's sums stay 0
template <int KPW, int SL0 = 0>
__device__ __forceinline__ void xt_mma_q4(f4 (&acc)[2][4], const h8 (&xf)[KPW][4], const char* wq, const char* wsc,
                                          int lch, int c0, int nsl, int lane) {
  static_assert(KPW % 4 == 0 && (SL0 == 0 || SL0 == 1), "whole 128-k chunks");
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[sl][mt] = (f4){0.f, 0.f, 0.f, 0.f};
  const bool two = SL0 == 0 && nsl > 1;
#pragma unroll
  for (int c = 0; c < KPW / 4; ++c) {
    u4 q[2] = {};
    _Float16 sc[2] = {};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i == 1 && !two) continue;
      const int blk = (SL0 + i) * lch + c0 + c;
      q[i] = *reinterpret_cast<const u4*>(wq + (blk * 64 + lane) * 16);
      sc[i] = *reinterpret_cast<const _Float16*>(wsc + (blk * 64 + lane) * 2);
    }
#pragma unroll
    for (int word = 0; word < 4; ++word) {
      const h8 a0 = dequant_word(q[0][word], sc[0]);
      const h8 a1 = two ? dequant_word(q[1][word], sc[1]) : a0;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const h8 b = perm8(xf[4 * c + word][mt]);
        acc[SL0][mt] = mfma16x16x32(a0, b, acc[SL0][mt]);
        if constexpr (SL0 == 0)
          if (two) acc[1][mt] = mfma16x16x32(a1, b, acc[1][mt]);
      }
    }
  }
}

__device__ __forceinline__ void xt_red_store(const f4 (&acc)[2][4], char* red, int w, int lane) {
  f4* r = reinterpret_cast<f4*>(red);
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) r[((w * 2 + sl) * 4 + mt) * 64 + lane] = acc[sl][mt];
}
// the 4 waves' k ranges of slab sl, m tile mt, lane ln, added in wave order
__device__ __forceinline__ f4 xt_red_sum(const char* red, int sl, int mt, int ln) {
  const f4* r = reinterpret_cast<const f4*>(red);
  f4 s = r[((0 * 2 + sl) * 4 + mt) * 64 + ln];
#pragma unroll
  for (int q = 1; q < 4; ++q) s += r[((q * 2 + sl) * 4 + mt) * 64 + ln];
  return s;
}
// adaRMS on the pre-scaled product: this wave's quarter of the row sums of squares of row `lane`
__device__ __forceinline__ float xt_rss_quarter(const float* rss, int T, int w, int lane) {
  const int row = min(lane, T - 1);
  const __amdgpu_buffer_rsrc_t rr = dev_rsrc(rss, (uint32_t)(T * XT_RSS * 4));
  f4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = load_dev<f4, LOC>(rr, (row * XT_RSS + 16 * w + 4 * i) * 4);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s += ((v[i][0] + v[i][1]) + v[i][2]) + v[i][3];
  return s;
}
// 1 / sqrt(mean(x^2) + eps) / nscale of row m from the 4 waves' quarters
__device__ __forceinline__ float xt_rinv(const char* den, int m, float eps, float nsc) {
  const float* d = reinterpret_cast<const float*>(den);
  const float tot = ((d[m] + d[64 + m]) + d[128 + m]) + d[192 + m];
  return 1.0f / sqrtf(tot / (float)XT_W + eps) / nsc;
}

// ---- the residual stream: one workgroup's 32 columns ----------------------------------------
// x = x_old + fp16(fp16(sum of the 8 XCDs' partials) * gate) (the gated residual after
// o_proj / down), or (action_in) x = fp16(fp16(x_t W^T) + b); then the row sums of squares per
// 16 columns and the next adaRMS's pre-scaled input fp16(x (1 + scale) c), its shift in row T.
// Compute thread = (row m, 8 columns).
// The cross-XCD partials of o_proj and down in fp16 (1) or fp32 (0).  The reference rounds these
// projections to fp16 (their output dtype), so each XCD's share, a sum over a quarter or an eighth
// of K, fits too; the 8 are added in fp32 before the one rounding of the sum.  fp16 halves the
// 13 MB that the 256 workgroups read at the start of every launch: 40 us per step.
#ifndef MLCV_XT_P16
#define MLCV_XT_P16 1
#endif
constexpr bool XT_P16 = MLCV_XT_P16 != 0;
// the attention's split partials written through this XCD's L2 (clean lines: the launch's end has
// less to write back) instead of plain stores
#ifndef MLCV_XT_AP_WT
#define MLCV_XT_AP_WT 1
#endif
constexpr bool XT_AP_WT = MLCV_XT_AP_WT != 0;
// this lane's 4 columns (n .. n + 3) of row m of the partial block of (XCD h, slot s)
// the cross-XCD partials written through too (tuning switch; measured 660 vs 655 us per step: they
// are the launch's last stores, so their acknowledgements end the launch later)
#ifndef MLCV_XT_PART_WT
#define MLCV_XT_PART_WT 0
#endif
__device__ __forceinline__ void xt_store_part(float* part, int h, int s, int T, int m, int n, f4 v) {
  const size_t i = (((size_t)h * XT_NS + s) * T + m) * 32 + n;
  if constexpr (XT_P16) {
    const h4 hv = (h4){f2h(v[0]), f2h(v[1]), f2h(v[2]), f2h(v[3])};
    if constexpr (MLCV_XT_PART_WT != 0) store_dev<h4>(dev_rsrc(part, 0x7FFFFFF0), (int)(i * 2), hv);
    else *reinterpret_cast<h4*>(reinterpret_cast<_Float16*>(part) + i) = hv;
  } else {
    *reinterpret_cast<f4*>(part + i) = v;
  }
}

struct XtRed {
  const float* part;      // [8][32][T][32], or null: action_in
  const _Float16* xold;   // [T][W1]
  const _Float16* gate;   // [W1]
  const _Float16* mnext;  // the next norm's [scale | shift]
  float nsc;
  _Float16* x;            // [T][W1]
  float* rss;             // [T][W1/16]
  _Float16* u;            // [64][W1] fragment-major
};
__device__ __forceinline__ void xt_reduce(const XtArgs& a, const XtRed& r, int s, int tid) {
  const int T = a.T, m = tid >> 2, c8 = tid & 3, n = 32 * s + 8 * c8;
  if (m > T) return;
  if (m == T) {  // the next norm's shift, as the pre-scaled input's row T
    *reinterpret_cast<h8*>(r.u + xf_index(T, n)) = load_global(reinterpret_cast<const h8*>(r.mnext + XT_W + n));
    return;
  }
  const h8 sc = load_global(reinterpret_cast<const h8*>(r.mnext + n));
  h8 xn;
  if (r.part) {
    constexpr int EB = XT_P16 ? 2 : 4;  // bytes per partial element
    const __amdgpu_buffer_rsrc_t rp = dev_rsrc(r.part, (uint32_t)(XT_NX * XT_NS * T * 32 * EB));
    f4 p[XT_NX][2];
#pragma unroll
    for (int hx = 0; hx < XT_NX; ++hx) {
      const int off = (((hx * XT_NS + s) * T + m) * 32 + 8 * c8) * EB;
      if constexpr (XT_P16) {
        const h8 q = load_dev<h8, 16>(rp, off);
        p[hx][0] = (f4){h2f(q[0]), h2f(q[1]), h2f(q[2]), h2f(q[3])};
        p[hx][1] = (f4){h2f(q[4]), h2f(q[5]), h2f(q[6]), h2f(q[7])};
      } else {
        p[hx][0] = load_dev<f4, 16>(rp, off);
        p[hx][1] = load_dev<f4, 16>(rp, off + 16);
      }
    }
    const h8 xo = load_dev<h8, 16>(dev_rsrc(r.xold, (uint32_t)(T * XT_W * 2)), (m * XT_W + n) * 2);
    const h8 g = load_global(reinterpret_cast<const h8*>(r.gate + n));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = p[0][e >> 2][e & 3];
#pragma unroll
      for (int hx = 1; hx < XT_NX; ++hx) acc += p[hx][e >> 2][e & 3];
      xn[e] = hadd(xo[e], hmul(f2h(acc), g[e]));
    }
  } else {
    const int A = a.A;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    for (int k = 0; k < A; k += 8) {
      const h8 xv = load_global(reinterpret_cast<const h8*>(a.xin + (size_t)m * A + k));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const h8 wv = load_global(reinterpret_cast<const h8*>(a.ain_w + (size_t)(n + e) * A + k));
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[e] = fmaf(h2f(xv[j]), h2f(wv[j]), acc[e]);
      }
    }
    const h8 b = a.ain_b ? load_global(reinterpret_cast<const h8*>(a.ain_b + n)) : (h8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) xn[e] = a.ain_b ? hadd(f2h(acc[e]), b[e]) : f2h(acc[e]);
  }
  float s2 = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s2 += h2f(xn[e]) * h2f(xn[e]);
  s2 += __shfl_xor(s2, 1);  // the 16 columns of this group: threads c8 and c8 ^ 1
  *reinterpret_cast<h8*>(r.x + (size_t)m * XT_W + n) = xn;
  if ((c8 & 1) == 0) r.rss[m * XT_RSS + 2 * s + (c8 >> 1)] = s2;
  h8 uu;
#pragma unroll
  for (int e = 0; e < 8; ++e) uu[e] = f2h(h2f(xn[e]) * (1.0f + h2f(sc[e])) * r.nsc);
  *reinterpret_cast<h8*>(r.u + xf_index(m, n)) = uu;
}

// The partial path of xt_reduce split at a workgroup barrier: every load issued before it, the
// arithmetic and stores after.  Launch A's stream waves start their DMA at that barrier, so the
// reduce's few loads are ahead of the 112 KB per CU of weights and keys in the memory system.
struct XtRedLd {
  h8 q[XT_NX];  // the 8 XCDs' partials (fp16) of this thread's 8 columns
  h8 xo, g, sc, sh;
};
__device__ __forceinline__ void xt_red_issue(const XtArgs& a, const XtRed& r, int s, int tid, XtRedLd& l) {
  static_assert(XT_P16, "the ordered reduce reads fp16 partials");
  const int T = a.T, m = tid >> 2, c8 = tid & 3, n = 32 * s + 8 * c8;
  const bool row = m < T;  // other rows read zeros without a fetch (offsets past the buffers)
  const __amdgpu_buffer_rsrc_t rp = dev_rsrc(r.part, (uint32_t)(XT_NX * XT_NS * T * 32 * 2));
#pragma unroll
  for (int hx = 0; hx < XT_NX; ++hx)
    l.q[hx] = load_dev<h8, 16>(rp, row ? (((hx * XT_NS + s) * T + m) * 32 + 8 * c8) * 2 : 0x7FFFFF00);
  l.xo = load_dev<h8, 16>(dev_rsrc(r.xold, (uint32_t)(T * XT_W * 2)), row ? (m * XT_W + n) * 2 : 0x7FFFFF00);
  l.g = load_global(reinterpret_cast<const h8*>(r.gate + n));
  l.sc = load_global(reinterpret_cast<const h8*>(r.mnext + n));
  l.sh = load_global(reinterpret_cast<const h8*>(r.mnext + XT_W + n));
}
// same arithmetic, order and stores as xt_reduce's partial path
__device__ __forceinline__ void xt_red_finish(const XtArgs& a, const XtRed& r, int s, int tid, const XtRedLd& l) {
  const int T = a.T, m = tid >> 2, c8 = tid & 3, n = 32 * s + 8 * c8;
  if (m == T) *reinterpret_cast<h8*>(r.u + xf_index(T, n)) = l.sh;
  if (m >= T) return;
  h8 xn;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float acc = h2f(l.q[0][e]);
#pragma unroll
    for (int hx = 1; hx < XT_NX; ++hx) acc += h2f(l.q[hx][e]);
    xn[e] = hadd(l.xo[e], hmul(f2h(acc), l.g[e]));
  }
  float s2 = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s2 += h2f(xn[e]) * h2f(xn[e]);
  s2 += __shfl_xor(s2, 1);
  *reinterpret_cast<h8*>(r.x + (size_t)m * XT_W + n) = xn;
  if ((c8 & 1) == 0) r.rss[m * XT_RSS + 2 * s + (c8 >> 1)] = s2;
  h8 uu;
#pragma unroll
  for (int e = 0; e < 8; ++e) uu[e] = f2h(h2f(xn[e]) * (1.0f + h2f(l.sc[e])) * r.nsc);
  *reinterpret_cast<h8*>(r.u + xf_index(m, n)) = uu;
}
// s_barrier of all 8 waves with no wait on any counter (the loads before it stay in flight)
__device__ __forceinline__ void xt_bar_raw() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ size_t xt_tw(const XtArgs& a, int L, int h) { return ((size_t)L * a.ls * XT_NX + h) * a.T * XT_W; }
__device__ __forceinline__ const _Float16* xt_mod(const XtArgs& a, int norm) { return a.modp + (size_t)norm * 3 * XT_W; }

// ---- attention key chunk ---------------------------------------------------------------------
// The 32 key slots of workgroup s.  Slots [0, nh) hold prefix keys [nh s, nh s + nh); slots
// [nh, nh + nt) hold keys [32 nh + nt s, + nt) of the tail [32 nh, P + T) (the last prefix keys,
// then the suffix); later slots, and keys past P + T, are padding (masked with -inf).  nt is the
// least count with 32 (nh + nt) >= P + T, nh = min(P / 32, 32 - nt), so the head keys are all
// prefix keys and every workgroup holds at most nt of the suffix keys (2 at T = 50): the keys
// computed in this launch reach each workgroup in one small load after barrier 2, instead of 50
// of them reaching two workgroups.  Any partition of the keys gives the same attention; only the
// order of the fp32 sums in the combine follows it.
struct XtKeys {
  int s, nh, nt;
  __device__ __forceinline__ int key(int j) const {
    return j < nh ? nh * s + j : (j < nh + nt ? 32 * nh + nt * s + (j - nh) : 0x3FFFFFFF);
  }
  __device__ __forceinline__ bool has_suffix(int P, int T) const {
    const int t0 = 32 * nh + nt * s;
    return t0 + nt > P && t0 < P + T;
  }
};
__device__ __forceinline__ XtKeys xt_keys(int P, int T, int s) {
  XtKeys k;
  k.s = s;
  for (k.nt = 1; k.nt < XT_KCH; ++k.nt) {  // ends: at nh + nt = 32, 32 (nh + nt) = 1024 >= P + T
    k.nh = min(P / XT_KCH, XT_KCH - k.nt);
    if (XT_KCH * (k.nh + k.nt) >= P + T) break;
  }
  return k;
}

// Key slots of `ck` into chunk registers (stream thread lt of NTH): prefix keys from the cache,
// suffix keys (when ready) from this XCD's k / v of the layer, padding clamped to a valid key and
// masked with -inf.  Before the suffix is ready its slots hold a prefix key as a placeholder
// (mask 0): xt_store_suffix overwrites them once it is.
template <int NTH>
__device__ __forceinline__ void xt_load_chunk(ChunkRegs<XT_HD, NTH>& R, const XtArgs& a, int L, int h, const XtKeys& ck,
                                              bool suffix_ready, int lt) {
  constexpr int HALF = XT_HD / 2;
  const int P = a.P, T = a.T;
  const __amdgpu_buffer_rsrc_t rk = dev_rsrc(a.keys + (size_t)L * P * XT_HD, (uint32_t)(P * XT_HD * 4));
  const __amdgpu_buffer_rsrc_t rv = dev_rsrc(a.values + (size_t)L * P * XT_HD, (uint32_t)(P * XT_HD * 2));
  const __amdgpu_buffer_rsrc_t sk = dev_rsrc(a.k32 + ((size_t)L * a.ls * XT_NX + h) * T * XT_HD, (uint32_t)(T * XT_HD * 4));
  const __amdgpu_buffer_rsrc_t sv = dev_rsrc(a.v + ((size_t)L * a.ls * XT_NX + h) * T * XT_HD, (uint32_t)(T * XT_HD * 2));
#pragma unroll
  for (int i = 0; i < ChunkRegs<XT_HD, NTH>::NK; ++i) {
    int j, dp;
    kitem<XT_HD, NTH>(i, lt, j, dp);
    const int kj = ck.key(j);
    if (suffix_ready && kj >= P && kj < P + T) {
      const int off = (kj - P) * XT_HD + dp;
      ld8f<16>(sk, off * 4, R.k[i]);
      ld8f<16>(sk, (off + HALF) * 4, R.k[i] + 8);
    } else {
      const int off = min(kj, P - 1) * XT_HD + dp;
      ld8f<KV_AUX>(rk, off * 4, R.k[i]);
      ld8f<KV_AUX>(rk, (off + HALF) * 4, R.k[i] + 8);
    }
  }
#pragma unroll
  for (int i = 0; i < ChunkRegs<XT_HD, NTH>::NV; ++i) {
    int jp, d0;
    vitem<XT_HD, NTH>(i, lt, jp, d0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int kj = ck.key(2 * jp + q);
      if (suffix_ready && kj >= P && kj < P + T)
        R.v[i][q] = load_dev<h8, 16>(sv, ((kj - P) * XT_HD + d0) * 2);
      else
        R.v[i][q] = load_dev<h8, KV_AUX>(rv, (min(kj, P - 1) * XT_HD + d0) * 2);
    }
  }
  const int km = ck.key(lt & (KCH - 1));
  R.msk = km < P ? load_global(a.mask + km) : 0.f;
  R.mok = km < P + T;
}

// The suffix keys among this workgroup's slots, once the layer's k / v are ready: their K rows
// (split hi/lo) and their V^T key pairs over the placeholders the first load left (stream thread
// lt of 256; a V pair holding one prefix and one suffix key is rewritten whole).
__device__ __forceinline__ void xt_store_suffix(const XtArgs& a, int L, int h, const XtKeys& ck, AttnSmem<XT_HD>& sm, int lt) {
  constexpr int HALF = XT_HD / 2, KLD = AttnSmem<XT_HD>::KLD;
  constexpr int NK = ChunkRegs<XT_HD, 256>::NK, NV = ChunkRegs<XT_HD, 256>::NV;
  const int P = a.P, T = a.T;
  const _Float16* pv = a.values + (size_t)L * P * XT_HD;
  const _Float16* sv = a.v + ((size_t)L * a.ls * XT_NX + h) * T * XT_HD;
  const __amdgpu_buffer_rsrc_t sk = dev_rsrc(a.k32 + ((size_t)L * a.ls * XT_NX + h) * T * XT_HD, (uint32_t)(T * XT_HD * 4));
  auto is_suf = [&](int kj) { return kj >= P && kj < P + T; };
  float kr[NK][16];
  h8 vr[NV][2];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    int j, dp;
    kitem<XT_HD, 256>(i, lt, j, dp);
    const int kj = ck.key(j);
    if (is_suf(kj)) {
      const int off = (kj - P) * XT_HD + dp;
      ld8f<LOC>(sk, off * 4, kr[i]);
      ld8f<LOC>(sk, (off + HALF) * 4, kr[i] + 8);
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    int jp, d0;
    vitem<XT_HD, 256>(i, lt, jp, d0);
    const int k0 = ck.key(2 * jp), k1 = ck.key(2 * jp + 1);
    if (is_suf(k0) || is_suf(k1)) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {  // one load per key: its source picked per lane
        const int kj = q ? k1 : k0;
        const _Float16* src = is_suf(kj) ? sv + (size_t)(kj - P) * XT_HD + d0 : pv + (size_t)min(kj, P - 1) * XT_HD + d0;
        vr[i][q] = load_global(reinterpret_cast<const h8*>(src));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    int j, dp;
    kitem<XT_HD, 256>(i, lt, j, dp);
    if (!is_suf(ck.key(j))) continue;
#pragma unroll
    for (int hp = 0; hp < 2; ++hp) {
      h8 hi8, lo8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16 hi, lo;
        split_f32(kr[i][8 * hp + e], hi, lo);
        hi8[e] = hi;
        lo8[e] = lo;
      }
      *reinterpret_cast<h8*>(&sm.kh[j * KLD + dp + hp * HALF]) = hi8;
      *reinterpret_cast<h8*>(&sm.kl[j * KLD + dp + hp * HALF]) = lo8;
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    int jp, d0;
    vitem<XT_HD, 256>(i, lt, jp, d0);
    if (!(is_suf(ck.key(2 * jp)) || is_suf(ck.key(2 * jp + 1)))) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const h2 pair = {vr[i][0][e], vr[i][1][e]};
      *reinterpret_cast<h2*>(&sm.vt[(d0 + e) * VLD + 2 * jp]) = pair;
    }
  }
}

// ---- launch A: layer L's attention half -----------------------------------------------------
template <bool FIRST, bool Q4>
__global__ __launch_bounds__(XT_NT) void xt_attn_kernel(const XtArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[XA_BYTES];
  __shared__ XtSh sh;
  const int tid = xt_tid();
  const bool comp = tid < XT_NC;
  const int w = (tid >> 6) & 3, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int h = xt_xcd(), s = blockIdx.x >> 3, L = a.L, T = a.T, P = a.P;
  const int v = __builtin_amdgcn_readfirstlane(tid >> 6) - 4;  // stream wave 0-3 (negative: compute)
  const XtKeys ck = xt_keys(P, T, s);  // this workgroup's keys of [prefix ; suffix]
  const bool has_suffix = ck.has_suffix(P, T);
  const int nsl = s + XT_NS < 48 ? 2 : 1;  // q/k/v slabs: j = s, s + 32 of [q_h | k | v] (16 each)
  AttnSmem<XT_HD>& kv = *reinterpret_cast<AttnSmem<XT_HD>*>(lds + XA_KV);
  if (tid == 0) sh.base = xt_ld_agent(a.flags + h * XT_NS + s);
  XT_STAMP(2 * L, 0, 0);

  // ---- 1. residual stream entering layer L | q/k/v weights (waves 4, 5), the key chunk (6, 7) --
  XtRed r;
  r.part = FIRST ? nullptr : a.dpart;
  r.xold = FIRST ? nullptr : a.xm + xt_tw(a, L - 1, h);
  r.gate = FIRST ? nullptr : xt_mod(a, 2 * L - 1) + 2 * XT_W;
  r.mnext = xt_mod(a, 2 * L);
  r.nsc = load_global(a.nscale + 2 * L);
  r.x = a.x + xt_tw(a, L, h);
  r.rss = a.rss + (size_t)h * T * XT_RSS;
  r.u = a.u + (size_t)h * 64 * XT_W;
  XtRedLd rl;
  if (!FIRST) {  // the reduce's loads first, then the stream waves' 112 KB
    if (comp) xt_red_issue(a, r, s, tid, rl);
    xt_bar_raw();
  }
  ChunkRegs<XT_HD, 128> R;  // waves 6, 7: the key chunk, stored to LDS after barrier 1
  if (comp) {
    if (FIRST) xt_reduce(a, r, s, tid);
    else xt_red_finish(a, r, s, tid, rl);
  } else if (v < 2) {
    for (int sl = 0; sl < nsl; ++sl) {
      const int j = s + XT_NS * sl;
      const int which = j < 16 ? PK_Q : j < 32 ? PK_K : PK_V, slab = j < 16 ? 16 * h + j : j < 32 ? j - 16 : j - 32;
      if constexpr (Q4 && XT_UNPACK_A) {
        xt_dma_q4_pairs(xt_qw(a, L, which), xt_qs(a, L, which), slab, XT_W / 128, 0, XT_W / 128, lds + XA_ST,
                        lds + XA_STSC, sl, v, 2, lane);
      } else if constexpr (Q4) {
        xt_dma_q4(xt_qw(a, L, which), xt_qs(a, L, which), slab, XT_W / 128, 0, XT_W / 128, lds + XA_W, lds + XA_WSC,
                  sl, XT_W / 128, v, 2, lane);
      } else {
        const __amdgpu_buffer_rsrc_t rw = dev_rsrc(xt_weights(a, L, which) + (size_t)slab * 32 * 512, 32 * 1024);
#pragma unroll
        for (int i = 0; i < 16; ++i) xt_dma(rw, v + 2 * i, lds + XA_W + (sl * 32 + v + 2 * i) * 1024, lane);
      }
    }
  } else {
    xt_load_chunk<128>(R, a, L, h, ck, false, tid - XT_NC - 128);
  }
  XT_STAMP(2 * L, 1, 0);
  xt_arrive(a, h, s, comp, 1, sh);
  if (v == 0 || v == 1) xt_vm_wait<0>();  // the q/k/v blocks have landed (this wave issued only those)
  if constexpr (Q4 && XT_UNPACK_A) {
    // the compute waves wait here for the blocks anyway: all 8 waves unpack them, one chunk
    // pair each, into the fp16 slab layout (barrier 1's s_barrier publishes the LDS writes)
    xt_sync();
    const int w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int sl = 0; sl < nsl; ++sl) xt_unpack_q4_pairs(lds + XA_ST, lds + XA_STSC, XT_W / 128, lds + XA_W, 32, sl, w8, 8, lane);
  }
  XT_STAMP(2 * L, 11, XT_NC);
  if (!xt_wait(a, h, 1, sh)) return;
  if (v >= 2) store_chunk<XT_HD, 128>(R, kv, tid - XT_NC - 128);  // nothing reads the chunk before barrier 2
  XT_STAMP(2 * L, 2, 0);

  // ---- 2. adaRMS + q/k/v (RoPE, q hi/lo in the attention's fragment order) ------------------
  f4 acc[2][4];
  if (comp) {
    h8 xf[8][4];
    xt_load_x<8, Q4 && !XT_UNPACK_A>(xf, a.u + (size_t)h * 64 * XT_W, XT_W, 8 * w, T, lane);
    const float part = xt_rss_quarter(a.rss + (size_t)h * T * XT_RSS, T, w, lane);
    if constexpr (Q4 && !XT_UNPACK_A) xt_mma_q4<8>(acc, xf, lds + XA_W, lds + XA_WSC, XT_W / 128, 2 * w, nsl, lane);
    else xt_mma<8>(acc, xf, lds + XA_W, 32, 8 * w, nsl, lane);
    xt_red_store(acc, lds + XA_RED, w, lane);
    reinterpret_cast<float*>(lds + XA_DEN)[w * 64 + lane] = part;
  }
  XT_STAMP(2 * L, 3, 0);
  xt_sync();
  if (comp) {
    const int m = 16 * w + r16, mc = min(m, T - 1);
    const float rinv = xt_rinv(lds + XA_DEN, m, a.eps, load_global(a.nscale + 2 * L));
    for (int sl = 0; sl < nsl; ++sl) {
      const int j = s + XT_NS * sl;
      const f4 own = xt_red_sum(lds + XA_RED, sl, w, lane);
      const f4 sv = xt_red_sum(lds + XA_RED, sl, T >> 4, 16 * g + (T & 15));
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = h2f(f2h(fmaf(own[e], rinv, sv[e])));  // the projection in fp16
      if (j >= 32) {  // v: 4 consecutive columns
        if (m < T) {
          const h4 v4 = {f2h(y[0]), f2h(y[1]), f2h(y[2]), f2h(y[3])};
          *reinterpret_cast<h4*>(a.v + ((size_t)L * a.ls * XT_NX + h) * T * XT_HD + (size_t)m * XT_HD + 16 * (j - 32) + 4 * g) = v4;
        }
        continue;
      }
      // q / k: RoPE in fp32 on the fp16 projection; rows (d, d + 128) paired in the slab,
      // lane ^ 32 holds the partner dims
      const int rope_d = 8 * (j & 15) + 4 * (g & 1) + (g < 2 ? 0 : 2);
      const f2 cc = load_global(reinterpret_cast<const f2*>(a.cos + (size_t)mc * (XT_HD / 2) + rope_d));
      const f2 ss = load_global(reinterpret_cast<const f2*>(a.sin + (size_t)mc * (XT_HD / 2) + rope_d));
      const bool lo = g < 2;
      const float r0 = swap_halves(y[2], y[0], lo);
      const float r1 = swap_halves(y[3], y[1], lo);
      const float x1a = lo ? y[0] : r0, x1b = lo ? y[1] : r1;
      const float x2a = lo ? r0 : y[2], x2b = lo ? r1 : y[3];
      const float o1a = x1a * cc[0] - x2a * ss[0], o1b = x1b * cc[1] - x2b * ss[1];
      const float o2a = x2a * cc[0] + x1a * ss[0], o2b = x2b * cc[1] + x1b * ss[1];
      if (m >= T) continue;
      if (j < 16) {
        _Float16* qf = a.qf + ((size_t)L * a.ls * XT_NX + h) * XT_QF;
        const float o[2][2] = {{o1a, o1b}, {o2a, o2b}};
        const float qscale = 1.0f / sqrtf((float)XT_HD);
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
          const int d = rope_d + hf * (XT_HD / 2);
          *reinterpret_cast<h2*>(qf + attn_qf_index(0, 4, XT_HD / 32, m, d, 0)) = hi;
          *reinterpret_cast<h2*>(qf + attn_qf_index(0, 4, XT_HD / 32, m, d, 1)) = lo2;
        }
      } else {
        float* kr = a.k32 + ((size_t)L * a.ls * XT_NX + h) * T * XT_HD + (size_t)m * XT_HD + rope_d;
        *reinterpret_cast<f2*>(kr) = (f2){o1a, o1b};
        *reinterpret_cast<f2*>(kr + XT_HD / 2) = (f2){o2a, o2b};
      }
    }
  }
  XT_STAMP(2 * L, 4, 0);
  xt_arrive(a, h, s, comp, 2, sh);
  if (!xt_wait(a, h, 2, sh)) return;
  XT_STAMP(2 * L, 5, 0);

  // ---- 3. attention of head h over this workgroup's 32 key slots: one split of 32 --------------
  h8 qh[8], ql[8];
  if (comp) {
    const __amdgpu_buffer_rsrc_t rq = dev_rsrc(a.qf + ((size_t)L * a.ls * XT_NX + h) * XT_QF, XT_QF * 2);
    const bool qrow = 16 * w + r16 < T;  // rows past T: zeros without a fetch
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int qb = (((w * 8 + ks) * 2) * 512 + lane * 8) * 2;
      qh[ks] = load_dev<h8, LOC>(rq, qrow ? qb : 0x7FFFFF00);
      ql[ks] = load_dev<h8, LOC>(rq, qrow ? qb + 1024 : 0x7FFFFF00);
    }
  } else {
    XT_STAMP(2 * L, 14, XT_NC);
    if (has_suffix) xt_store_suffix(a, L, h, ck, kv, tid - XT_NC);  // this workgroup holds suffix keys
    XT_STAMP(2 * L, 15, XT_NC);
  }
  xt_sync();
  XT_STAMP(2 * L, 13, 0);
  if (!comp) {  // o_proj weights (slabs 2s, 2s + 1, k steps [8h, 8h + 8)) into LDS, during the attention
    if constexpr (Q4) {
      for (int sl = 0; sl < 2; ++sl)  // chunks [2h, 2h + 2) of the 16 per slab
        xt_dma_q4(xt_qw(a, L, PK_O), xt_qs(a, L, PK_O), 2 * s + sl, 2 * XT_W / 128, 2 * h, 2, lds + XA_WO,
                  lds + XA_WOSC, sl, 2, v, 4, lane);
    } else {
      const _Float16* wo = xt_weights(a, L, PK_O);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = v + 4 * i, sl = b >> 3, kk = b & 7;
        xt_dma(dev_rsrc(wo + ((size_t)(2 * s + sl) * 64 + 8 * h) * 512, 8 * 1024), kk, lds + XA_WO + b * 1024, lane);
      }
    }
  }
  if (comp) {
    // a chunk whose keys are all masked (<= -1e9: exp underflows to 0 for every row that has a
    // valid key, and every row has the suffix keys) contributes nothing: skip it, exactly
    const bool skip = !a.noskip && __all(kv.msk[lane & (KCH - 1)] <= -1e9f);
    const int m = 16 * w + r16;  // this lane's query row (token)
    float* aml = a.aml + ((size_t)h * XT_NS + s) * 64 * 2;
    if (skip) {
      if (g == 0 && m < T) *reinterpret_cast<f2*>(aml + m * 2) = (f2){-1e30f, 0.f};
    } else {
      constexpr int NKS = XT_HD / 32, NDT = XT_HD / 16, KLD = AttnSmem<XT_HD>::KLD;
      // S^T[key][row] = K . Q^T as hi.hi + hi.lo + lo.hi (fp32-level logits)
      f4 acc3[2][3];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int q = 0; q < 3; ++q) acc3[kt][q] = (f4){0.f, 0.f, 0.f, 0.f};
      h8 kf[2][2][2];
      auto ldk = [&](int ks, int b) __attribute__((always_inline)) {
        const int d0 = 32 * ks + 8 * g;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          kf[b][kt][0] = *reinterpret_cast<const h8*>(&kv.kh[(16 * kt + r16) * KLD + d0]);
          kf[b][kt][1] = *reinterpret_cast<const h8*>(&kv.kl[(16 * kt + r16) * KLD + d0]);
        }
      };
      ldk(0, 0);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        if (ks + 1 < NKS) ldk(ks + 1, (ks + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const h8 ah = kf[ks & 1][kt][0], al = kf[ks & 1][kt][1];
          acc3[kt][0] = mfma16x16x32(al, qh[ks], acc3[kt][0]);
          acc3[kt][1] = mfma16x16x32(ah, ql[ks], acc3[kt][1]);
          acc3[kt][2] = mfma16x16x32(ah, qh[ks], acc3[kt][2]);
        }
      }
      // lane holds keys 16 kt + 4 g + i of row r16; softmax over the chunk in fp32
      float p[8];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p[4 * kt + i] = (acc3[kt][0][i] + acc3[kt][1][i]) + acc3[kt][2][i] + kv.msk[16 * kt + 4 * g + i];
      float cmax = p[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) cmax = fmaxf(cmax, p[i]);
      cmax = xor_max_16_32(cmax);
      const float mrow = cmax > -1e30f ? cmax : -1e30f;
      float psum = 0.f;
      h8 pb;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = exp_hw(p[i] - mrow);
        psum += e;
        pb[i] = f2h(e);
      }
      const float lrow = xor_sum_16_32(psum);
      // O^T += V^T . P^T, the V^T fragments read two d tiles ahead
      f4 oacc[NDT];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] = (f4){0.f, 0.f, 0.f, 0.f};
      h4 vf[3][2];
      auto ldv = [&](int dt, int b) __attribute__((always_inline)) {
        const _Float16* vr = &kv.vt[(16 * dt + r16) * VLD];
        vf[b][0] = *reinterpret_cast<const h4*>(vr + 4 * g);
        vf[b][1] = *reinterpret_cast<const h4*>(vr + 16 + 4 * g);
      };
      ldv(0, 0);
      ldv(1, 1);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        if (dt + 2 < NDT) ldv(dt + 2, (dt + 2) % 3);
        __builtin_amdgcn_sched_barrier(0);
        const h4 v0 = vf[dt % 3][0], v1 = vf[dt % 3][1];
        const h8 av = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        oacc[dt] = mfma16x16x32(av, pb, oacc[dt]);
      }
      // the split's output normalized by its own sum (fp16), staged through this wave's LDS rows
      // so that each store writes whole rows
      _Float16* pl = reinterpret_cast<_Float16*>(lds + XA_STAGE) + (size_t)w * 16 * XT_PLD;
      const float linv = lrow > 0.f ? 1.0f / lrow : 0.f;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        h4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = f2h(oacc[dt][i] * linv);
        *reinterpret_cast<h4*>(pl + r16 * XT_PLD + 16 * dt + 4 * g) = o4;
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_wave_barrier();
      _Float16* po = a.ap + (((size_t)h * XT_NS + s) * 64 + 16 * w) * XT_HD;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int idx = 64 * it + lane, rr = idx >> 5, cc = (idx & 31) * 8;
        if (16 * w + rr < T) {
          const h8 pv = *reinterpret_cast<const h8*>(pl + rr * XT_PLD + cc);
          if constexpr (XT_AP_WT) store_dev<h8>(dev_rsrc(po, 16 * XT_HD * 2), (rr * XT_HD + cc) * 2, pv);
          else *reinterpret_cast<h8*>(po + rr * XT_HD + cc) = pv;
        }
      }
      if (g == 0 && m < T) {
        if constexpr (XT_AP_WT) store_dev<f2>(dev_rsrc(aml, 64 * 8), m * 8, (f2){mrow, lrow});
        else *reinterpret_cast<f2*>(aml + m * 2) = (f2){mrow, lrow};
      }
    }
  }
  XT_STAMP(2 * L, 6, 0);
  xt_arrive(a, h, s, comp, 3, sh);
  if (!xt_wait(a, h, 3, sh)) return;
  XT_STAMP(2 * L, 7, 0);

  // ---- 4. combine the 32 splits of rows s and s + 32 (one wave per row) ---------------------
  if (comp && w < 2 && s + XT_NS * w < T) {
    const int t = s + XT_NS * w, sp = lane & 31;
    const __amdgpu_buffer_rsrc_t rml = dev_rsrc(a.aml + (size_t)h * XT_NS * 64 * 2, XT_NS * 64 * 2 * 4);
    const __amdgpu_buffer_rsrc_t ro = dev_rsrc(a.ap + (size_t)h * XT_NS * 64 * XT_HD, XT_NS * 64 * XT_HD * 2);
    const f2 ml = load_dev<f2, LOC>(rml, (sp * 64 + t) * 8);
    h4 o[XT_NS];
#pragma unroll
    for (int q = 0; q < XT_NS; ++q) o[q] = load_dev<h4, LOC>(ro, ((q * 64 + t) * XT_HD + 4 * lane) * 2);
    const bool mine = lane < XT_NS;
    float mmax = mine ? ml[0] : -INFINITY;
#pragma unroll
    for (int o2 = 16; o2 > 0; o2 >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, o2));
    const float wgt = mine ? exp_hw(ml[0] - mmax) * ml[1] : 0.f;
    float lsum = wgt;
#pragma unroll
    for (int o2 = 16; o2 > 0; o2 >>= 1) lsum += __shfl_xor(lsum, o2);
    const float wn = wgt * (1.0f / lsum);
    f4 acc4 = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < XT_NS; ++q) {
      const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wn), q));
#pragma unroll
      for (int i = 0; i < 4; ++i) acc4[i] += ws != 0.f ? ws * h2f(o[q][i]) : 0.f;  // skipped splits: no O
    }
    h4 o4;
#pragma unroll
    for (int i = 0; i < 4; ++i) o4[i] = f2h(acc4[i]);
    *reinterpret_cast<h4*>(a.attn + ((size_t)L * a.ls * XT_NX + h) * 64 * XT_HD + xf_index(t, 4 * lane)) = o4;
  }
  XT_STAMP(2 * L, 8, 0);
  xt_arrive(a, h, s, comp, 4, sh);
  if (!comp) xt_vm_wait<0>();  // the o_proj blocks have landed
  XT_STAMP(2 * L, 12, XT_NC);
  if (!xt_wait(a, h, 4, sh)) return;
  XT_STAMP(2 * L, 9, 0);

  // ---- 5. o_proj, row-parallel: this XCD's 256 columns of K, outputs [32 s, 32 s + 32) ------
  if (comp) {
    const _Float16* ab = a.attn + ((size_t)L * a.ls * XT_NX + h) * 64 * XT_HD;
    if constexpr (Q4) {  // 2 slabs x 2 chunks: wave w takes slab w >> 1, chunk w & 1
      h8 xf[4][4];
      xt_load_x<4, true>(xf, ab, XT_HD, 4 * (w & 1), T - 1, lane);
      if (w < 2) xt_mma_q4<4, 0>(acc, xf, lds + XA_WO, lds + XA_WOSC, 2, w & 1, 1, lane);
      else xt_mma_q4<4, 1>(acc, xf, lds + XA_WO, lds + XA_WOSC, 2, w & 1, 1, lane);
    } else {
      h8 xf[2][4];
      xt_load_x<2>(xf, ab, XT_HD, 2 * w, T - 1, lane);
      xt_mma<2>(acc, xf, lds + XA_WO, 8, 2 * w, 2, lane);
    }
    xt_red_store(acc, lds + XA_RED, w, lane);
  }
  xt_sync();
  if (comp) {
    const int m = 16 * w + r16;
    if (m < T) {
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
        xt_store_part(a.opart, h, s, T, m, 16 * sl + 4 * g, xt_red_sum(lds + XA_RED, sl, w, lane));
    }
  }
  XT_STAMP(2 * L, 10, 0);
}

// ---- launch B: layer L's MLP half ----------------------------------------------------------
template <bool Q4>
__global__ __launch_bounds__(XT_NT) void xt_mlp_kernel(const XtArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[Q4 && XT_UNPACK ? XB_BYTES_Q4 : XB_BYTES];
  __shared__ XtSh sh;
  const int tid = xt_tid();
  const bool comp = tid < XT_NC;
  const int w = (tid >> 6) & 3, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int h = xt_xcd(), s = blockIdx.x >> 3, L = a.L, T = a.T;
  if (tid == 0) sh.base = xt_ld_agent(a.flags + h * XT_NS + s);
  XT_STAMP(2 * L + 1, 0, 0);

  // ---- 1. residual stream after the attention | gate_up and down weights ---------------------
  if (comp) {
    XtRed r;
    r.part = a.opart;
    r.xold = a.x + xt_tw(a, L, h);
    r.gate = xt_mod(a, 2 * L) + 2 * XT_W;
    r.mnext = xt_mod(a, 2 * L + 1);
    r.nsc = load_global(a.nscale + 2 * L + 1);
    r.x = a.xm + xt_tw(a, L, h);
    r.rss = a.rss + (size_t)h * T * XT_RSS;
    r.u = a.u + (size_t)h * 64 * XT_W;
    xt_reduce(a, r, s, tid);
  } else {
    const int lt = tid - XT_NC, v = __builtin_amdgcn_readfirstlane(lt >> 6);
    // gate_up slabs 64 h + 2 s, + 1 (8 gate + 8 up rows each): 64 contiguous blocks
    if constexpr (Q4 && XT_UNPACK) {
      for (int sl = 0; sl < 2; ++sl)
        xt_dma_q4_pairs(xt_qw(a, L, PK_GU), xt_qs(a, L, PK_GU), XT_FX / 8 * h + 2 * s + sl, XT_W / 128, 0, XT_W / 128,
                        lds + XB_ST, lds + XB_STSC, sl, v, 4, lane);
    } else if constexpr (Q4) {
      for (int sl = 0; sl < 2; ++sl)
        xt_dma_q4(xt_qw(a, L, PK_GU), xt_qs(a, L, PK_GU), XT_FX / 8 * h + 2 * s + sl, XT_W / 128, 0, XT_W / 128,
                  lds + XB_GU, lds + XB_GUSC, sl, XT_W / 128, v, 4, lane);
    } else {
      const __amdgpu_buffer_rsrc_t rg = dev_rsrc(xt_weights(a, L, PK_GU) + (size_t)(XT_FX / 8 * h + 2 * s) * 32 * 512, 64 * 1024);
#pragma unroll
      for (int i = 0; i < 16; ++i) xt_dma(rg, v + 4 * i, lds + XB_GU + (v + 4 * i) * 1024, lane);
    }
  }
  XT_STAMP(2 * L + 1, 1, 0);
  xt_arrive(a, h, s, comp, 1, sh);
  if (!comp) xt_vm_wait<0>();  // the gate_up blocks have landed
  if constexpr (Q4 && XT_UNPACK) {  // all 8 waves unpack them, one chunk pair each
    xt_sync();
    const int w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int sl = 0; sl < 2; ++sl) xt_unpack_q4_pairs(lds + XB_ST, lds + XB_STSC, XT_W / 128, lds + XB_GU, 32, sl, w8, 8, lane);
  }
  XT_STAMP(2 * L + 1, 11, XT_NC);
  if (!xt_wait(a, h, 1, sh)) return;
  XT_STAMP(2 * L + 1, 2, 0);

  // ---- 2. adaRMS (post) + gate_up + GeGLU: MLP columns [512 h + 16 s, + 16) ------------------
  // The activations (this XCD's L2) land first; only then do the stream waves start the down
  // weights, so that the two do not share the CU's load path.
  f4 acc[2][4];
  h8 xf[8][4];
  float part = 0.f;
  if (comp) {
    xt_load_x<8, Q4 && !XT_UNPACK>(xf, a.u + (size_t)h * 64 * XT_W, XT_W, 8 * w, T, lane);
    part = xt_rss_quarter(a.rss + (size_t)h * T * XT_RSS, T, w, lane);
    xt_vm_wait<0>();
  }
  xt_sync();
  if (!comp) {  // down slabs 2 s, 2 s + 1, k steps [16 h, 16 h + 16)
    const int lt = tid - XT_NC, v = __builtin_amdgcn_readfirstlane(lt >> 6);
    if constexpr (Q4 && XT_UNPACK) {  // chunks [4h, 4h + 4) of the 32 per slab, into the staging area
      for (int sl = 0; sl < 2; ++sl)
        xt_dma_q4_pairs(xt_qw(a, L, PK_DN), xt_qs(a, L, PK_DN), 2 * s + sl, XT_F / 128, 4 * h, 4, lds + XB_ST,
                        lds + XB_STSC, sl, v, 4, lane);
    } else if constexpr (Q4) {
      for (int sl = 0; sl < 2; ++sl)  // chunks [4h, 4h + 4) of the 32 per slab
        xt_dma_q4(xt_qw(a, L, PK_DN), xt_qs(a, L, PK_DN), 2 * s + sl, XT_F / 128, 4 * h, 4, lds + XB_DN, lds + XB_DNSC,
                  sl, 4, v, 4, lane);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int b = v + 4 * i, sl = b >> 4, kk = b & 15;
        xt_dma(dev_rsrc(xt_weights(a, L, PK_DN) + ((size_t)(2 * s + sl) * 128 + 16 * h) * 512, 16 * 1024), kk,
               lds + XB_DN + b * 1024, lane);
      }
    }
  }
  if (comp) {
    if constexpr (Q4 && !XT_UNPACK) xt_mma_q4<8>(acc, xf, lds + XB_GU, lds + XB_GUSC, XT_W / 128, 2 * w, 2, lane);
    else xt_mma<8>(acc, xf, lds + XB_GU, 32, 8 * w, 2, lane);
    xt_red_store(acc, lds + XB_RED, w, lane);
    reinterpret_cast<float*>(lds + XB_DEN)[w * 64 + lane] = part;
  }
  XT_STAMP(2 * L + 1, 3, 0);
  xt_sync();
  if (comp) {
    const int m = 16 * w + r16;
    const float rinv = xt_rinv(lds + XB_DEN, m, a.eps, load_global(a.nscale + 2 * L + 1));
    _Float16* hb = a.h + ((size_t)L * a.ls * XT_NX + h) * 64 * XT_FX;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const f4 own = xt_red_sum(lds + XB_RED, sl, w, lane);
      const f4 sv = xt_red_sum(lds + XB_RED, sl, T >> 4, 16 * g + (T & 15));
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = fmaf(own[e], rinv, sv[e]);
      // lanes g < 2 hold 4 gate columns, lane ^ 32 the matching 4 up columns
      const bool lo = g < 2;
      const float r0 = swap_halves(y[2], y[0], lo);
      const float r1 = swap_halves(y[3], y[1], lo);
      const float ga = lo ? y[0] : r0, gb = lo ? y[1] : r1;
      const float ua = lo ? r0 : y[2], ub = lo ? r1 : y[3];
      h2 o;
      o[0] = hmul(f2h(gelu_tanh_hw(h2f(f2h(ga)))), f2h(ua));
      o[1] = hmul(f2h(gelu_tanh_hw(h2f(f2h(gb)))), f2h(ub));
      const int col = 8 * (2 * s + sl) + 4 * (g & 1) + (lo ? 0 : 2);
      if (m < T) *reinterpret_cast<h2*>(hb + xf_index(m, col)) = o;
    }
  }
  XT_STAMP(2 * L + 1, 4, 0);
  xt_arrive(a, h, s, comp, 2, sh);
  if (!comp) {
    xt_vm_wait<0>();  // the down blocks have landed
    if constexpr (Q4 && XT_UNPACK) {
      const int v = __builtin_amdgcn_readfirstlane((tid - XT_NC) >> 6);
      for (int sl = 0; sl < 2; ++sl) xt_unpack_q4_pairs(lds + XB_ST, lds + XB_STSC, 4, lds + XB_DN, 16, sl, v, 4, lane);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    }
  }
  XT_STAMP(2 * L + 1, 12, XT_NC);
  if (!xt_wait(a, h, 2, sh)) return;
  XT_STAMP(2 * L + 1, 5, 0);

  // ---- 3. down, row-parallel: this XCD's 512 columns of K, outputs [32 s, 32 s + 32) ---------
  h8 xd[4][4];
  if (comp) xt_load_x<4, Q4 && !XT_UNPACK>(xd, a.h + ((size_t)L * a.ls * XT_NX + h) * 64 * XT_FX, XT_FX, 4 * w, T - 1, lane);
  if (comp) {
    if constexpr (Q4 && !XT_UNPACK) xt_mma_q4<4>(acc, xd, lds + XB_DN, lds + XB_DNSC, 4, w, 2, lane);
    else xt_mma<4>(acc, xd, lds + XB_DN, 16, 4 * w, 2, lane);
    xt_red_store(acc, lds + XB_RED, w, lane);
  }
  xt_sync();
  if (comp) {
    const int m = 16 * w + r16;
    if (m < T) {
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
        xt_store_part(a.dpart, h, s, T, m, 16 * sl + 4 * g, xt_red_sum(lds + XB_RED, sl, w, lane));
    }
  }
  XT_STAMP(2 * L + 1, 6, 0);
}

// ---- the head: last layer's down partials -> residual stream -> final adaRMS -> action_out_proj ----
// decode_e1's final norm (gemma_dual.py:417-433), action_out_proj (pi0_model.py:142-163) and, in the
// loop, the Euler update (pi0_model.py:165-194).  One workgroup per token row m:
//   - the row's residual stream: the 8 XCDs' partials summed in XCD order, then the gated residual,
//     as every layer's reduce does (stored into x16 in the launch chain's layout);
//   - its adaRMS in the reference's order: fp32 statistics, x / sqrt(mean(x^2) + eps), times
//     (1 + scale), plus shift, each op rounded in fp32, one rounding to fp16;
//   - the A outputs of action_out_proj: fp32 sums over K (8 lanes per output, 128 k each), one
//     rounding to fp16, the fp16 bias add; then the velocity in fp32, or the Euler update.
__global__ __launch_bounds__(256) void xt_head_kernel(const XtArgs a) {
  __shared__ float red[4];
  __shared__ __attribute__((aligned(16))) _Float16 xs[XT_W];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int D = a.D, T = a.T, A = a.A, n = 4 * tid;  // this thread's columns n .. n + 3
  const int s = n >> 5, cc = n & 31;                 // residual column slice and offset in it
  f4 p[XT_NX];
#pragma unroll
  for (int hx = 0; hx < XT_NX; ++hx) {
    const size_t off = (((size_t)hx * XT_NS + s) * T + m) * 32 + cc;
    if constexpr (XT_P16) {
      const h4 q = load_global(reinterpret_cast<const h4*>(reinterpret_cast<const _Float16*>(a.dpart) + off));
      p[hx] = (f4){h2f(q[0]), h2f(q[1]), h2f(q[2]), h2f(q[3])};
    } else {
      p[hx] = load_global(reinterpret_cast<const f4*>(a.dpart + off));
    }
  }
  const h4 xo = load_global(reinterpret_cast<const h4*>(a.xm + xt_tw(a, D - 1, 0) + (size_t)m * XT_W + n));
  const h4 g = load_global(reinterpret_cast<const h4*>(xt_mod(a, 2 * D - 1) + 2 * XT_W + n));
  const _Float16* fin = xt_mod(a, 2 * D);
  const h4 sc = load_global(reinterpret_cast<const h4*>(fin + n));
  const h4 sh = load_global(reinterpret_cast<const h4*>(fin + XT_W + n));
  h4 x;
  float s2 = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float acc = p[0][e];
#pragma unroll
    for (int hx = 1; hx < XT_NX; ++hx) acc += p[hx][e];
    x[e] = hadd(xo[e], hmul(f2h(acc), g[e]));
    s2 += h2f(x[e]) * h2f(x[e]);
  }
  if (a.x16) *reinterpret_cast<h4*>(a.x16 + (size_t)m * XT_W + n) = x;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s2 += __shfl_xor(s2, o);
  if (lane == 0) red[w] = s2;
  __syncthreads();
  const float tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float den = __fsqrt_rn(__fadd_rn(__fdiv_rn(tot, (float)XT_W), a.eps));
  h4 xn;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float nv = __fdiv_rn(h2f(x[e]), den);
    xn[e] = f2h(__fadd_rn(__fmul_rn(nv, __fadd_rn(1.0f, h2f(sc[e]))), h2f(sh[e])));
  }
  *reinterpret_cast<h4*>(xs + n) = xn;
  __syncthreads();
  // action_out_proj: output j on lanes 8 (tid >> 3) .. +7, lane part k range [128 part, +128)
  const int part = tid & 7;
  for (int j = tid >> 3; j < A; j += 32) {
    const _Float16* wr = a.aout_w + (size_t)j * XT_W + 128 * part;
    float acc = 0.f;
#pragma unroll 4
    for (int k = 0; k < 128; k += 8) {
      const h8 wv = load_global(reinterpret_cast<const h8*>(wr + k));
      const h8 xv = *reinterpret_cast<const h8*>(xs + 128 * part + k);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(h2f(xv[e]), h2f(wv[e]), acc);
    }
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 4);
    if (part == 0) {
      _Float16 y = f2h(acc);
      if (a.aout_b) y = hadd(y, a.aout_b[j]);
      const float v = h2f(y);
      const size_t o = (size_t)m * A + j;
      if (a.euler) {
        const float nx = euler_update(a.x32[o], a.dt, v);
        a.x32[o] = nx;
        a.xnext[o] = f2h(nx);
      } else {
        a.vout[o] = v;
        if (a.vout_user) a.vout_user[o] = v;
      }
    }
  }
}

}  // namespace

#ifdef MLCV_XT_TRACE
}  // namespace mlcv
extern "C" void* mlcv_xt_trace_ptr() {
  void* p = nullptr;
  (void)hipGetSymbolAddress(&p, HIP_SYMBOL(mlcv::xt_trace));
  return p;
}
namespace mlcv {
#endif

bool xt_shape_ok(int W1, int F1, int H, int KV, int HD, int T, int P, int A) {
  return W1 == XT_W && F1 == XT_F && H == XT_NX && KV == 1 && HD == XT_HD && T >= 1 && T < 64 && P >= XT_KCH &&
         P + T <= XT_NS * XT_KCH && A >= 8 && A % 8 == 0;
}

static int xt_check(const XtArgs& a) {
  MLCV_REQUIRE(a.lw && a.modp && a.nscale && a.keys && a.values && a.mask && a.cos && a.sin && a.xin && a.ain_w,
               "XCD step: inputs");
  MLCV_REQUIRE(a.x && a.xm && a.qf && a.k32 && a.v && a.attn && a.h && a.u && a.rss && a.ap && a.aml && a.opart &&
                   a.dpart && a.flags && a.err,
               "XCD step: buffers");
  MLCV_REQUIRE(xt_shape_ok(XT_W, XT_F, XT_NX, 1, XT_HD, a.T, a.P, a.A), "XCD step: shape");
  MLCV_REQUIRE(a.L >= 0 && a.L < a.D, "XCD step: layer");
  return 0;
}

int xt_attn_launch(const XtArgs& a, hipStream_t st) {
  MLCV_TRY(xt_check(a));
  if (a.q4) {
    if (a.L == 0) xt_attn_kernel<true, true><<<XT_NX * XT_NS, XT_NT, 0, st>>>(a);
    else xt_attn_kernel<false, true><<<XT_NX * XT_NS, XT_NT, 0, st>>>(a);
  } else {
    if (a.L == 0) xt_attn_kernel<true, false><<<XT_NX * XT_NS, XT_NT, 0, st>>>(a);
    else xt_attn_kernel<false, false><<<XT_NX * XT_NS, XT_NT, 0, st>>>(a);
  }
  MLCV_HIP(hipGetLastError());
  return 0;
}

int xt_mlp_launch(const XtArgs& a, hipStream_t st) {
  MLCV_TRY(xt_check(a));
  if (a.q4) xt_mlp_kernel<true><<<XT_NX * XT_NS, XT_NT, 0, st>>>(a);
  else xt_mlp_kernel<false><<<XT_NX * XT_NS, XT_NT, 0, st>>>(a);
  MLCV_HIP(hipGetLastError());
  return 0;
}

int xt_head_launch(const XtArgs& a, hipStream_t st) {
  MLCV_REQUIRE(a.dpart && a.xm && a.modp && a.aout_w && (a.euler ? a.x32 && a.xnext : a.vout != nullptr),
               "XCD step: head buffers");
  MLCV_REQUIRE(a.T >= 1 && a.T < 64 && a.D >= 1 && a.A >= 1, "XCD step: head shape");
  xt_head_kernel<<<a.T, 256, 0, st>>>(a);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
