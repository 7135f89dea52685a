// Shared device/host helpers for the gfx950 pi0.5 denoise library.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <string>

namespace mlcv {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// ---- error reporting (host) ------------------------------------------------
void set_error(const std::string& msg);
const char* get_error();

#define MLCV_HIP(expr)                                                               \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess) {                                                          \
      ::mlcv::set_error(std::string(#expr) + " failed: " + hipGetErrorString(_e) +   \
                        " (" __FILE__ ":" + std::to_string(__LINE__) + ")");         \
      return -1;                                                                     \
    }                                                                                \
  } while (0)

#define MLCV_REQUIRE(cond, msg)                                                      \
  do {                                                                               \
    if (!(cond)) {                                                                   \
      ::mlcv::set_error(std::string("invalid argument: ") + (msg));                  \
      return -2;                                                                     \
    }                                                                                \
  } while (0)

#define MLCV_TRY(expr)                                                               \
  do {                                                                               \
    int _r = (expr);                                                                 \
    if (_r != 0) return _r;                                                          \
  } while (0)

// ---- device numerics helpers ----------------------------------------------
// Fragment-major activation layout for the skinny GEMMs (rows m < 64, K % 32 == 0,
// 64 x K halfs): the B operand of mfma16x16x32 f16 for k step ks and m tile mt is one
// contiguous 1 KB block, lane 16 g + r holding X[16 mt + r][32 ks + 8 g .. +7].  A wave
// then loads each fragment with one fully coalesced instruction.
__host__ __device__ __forceinline__ size_t xf_index(int m, int k) {
  return ((size_t)((k >> 5) * 4 + (m >> 4)) * 64 + ((((k >> 3) & 3) << 4) | (m & 15))) * 8 + (k & 7);
}

// Attention query fragments (q roped and scaled, split fp16 hi + lo): the B operand of
// mfma16x16x32 for (kv head, 16-row tile, k step, hi/lo) is one contiguous 1 KB block,
// lane 16 g + r holding Q[row 16 tile + r][32 ks + 8 g .. +7]; row = (q head within the kv
// group) * Tq + token, tiles = rows padded to 64 / 16.
__host__ __device__ __forceinline__ size_t attn_qf_index(int kvh, int ntiles, int nks, int row, int d, int lo) {
  return ((((size_t)kvh * ntiles + (row >> 4)) * nks + (d >> 5)) * 2 + lo) * 512 +
         ((((d >> 3) & 3) << 4) | (row & 15)) * 8 + (d & 7);
}

// Load through a global-address-space pointer: a pointer the compiler cannot trace to
// global memory becomes a flat load, which forces a full vmcnt(0) wait at its first use.
template <class T>
__device__ __forceinline__ T load_global(const T* p) {
  typedef const __attribute__((address_space(1))) T gT;
  return *(gT*)p;
}

// Buffer loads with explicit cache-policy bits (AUX: 16 = device scope, sc1).  Device-scope
// loads of data the previous kernel wrote read it at the memory side instead of missing in
// this XCD's L2 and filling it with lines no later launch reuses.  Offsets are in bytes;
// past `bytes` the load returns zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}
template <class T, int AUX = 16>
__device__ __forceinline__ T load_dev(__amdgpu_buffer_rsrc_t r, int byte_off) {
  static_assert(sizeof(T) == 16 || sizeof(T) == 8 || sizeof(T) == 4, "4, 8 or 16 bytes");
  if constexpr (sizeof(T) == 16) return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, AUX));
  else if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, AUX));
  else return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, AUX));
}
// Buffer stores with explicit cache-policy bits: AUX 16 (device scope, sc1) writes through
// this XCD's L2 to the memory side, so that a workgroup on another XCD of the same launch
// reads the value with a device-scope load once it has seen the writer's progress flag.
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
template <class T, int AUX = 16>
__device__ __forceinline__ void store_dev(__amdgpu_buffer_rsrc_t r, int byte_off, T v) {
  static_assert(sizeof(T) == 16 || sizeof(T) == 8 || sizeof(T) == 4, "4, 8 or 16 bytes");
  if constexpr (sizeof(T) == 16) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, byte_off, 0, AUX);
  else if constexpr (sizeof(T) == 8) __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, v), r, byte_off, 0, AUX);
  else __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, byte_off, 0, AUX);
}
// cache policy of the streamed operands (measured on the step at P=968, T=50):
// prefix keys and values (written by an earlier launch): plain loads, 9 us per step and
// 40 us per prefill faster than device-scope ones on the current kernels;
// weights (layer GEMMs, and the row-major time-MLP / modulation GEMVs): non-temporal (2),
// 54 us per step faster than plain loads on the current kernels
#ifndef MLCV_KV_AUX
#define MLCV_KV_AUX 0
#endif
#ifndef MLCV_W_AUX
#define MLCV_W_AUX 2
#endif
#ifndef MLCV_WROW_AUX
#define MLCV_WROW_AUX 2
#endif
// the fragment-major activations of the layer GEMMs (the previous launch's output): device
// scope; plain loads measure the same on the current kernels (812.0 vs 812.1 us per step)
#ifndef MLCV_X_AUX
#define MLCV_X_AUX 16
#endif
constexpr int KV_AUX = MLCV_KV_AUX, W_AUX = MLCV_W_AUX, WROW_AUX = MLCV_WROW_AUX, X_AUX = MLCV_X_AUX;

// fp16 <-> fp32 with IEEE round-to-nearest-even (v_cvt_f16_f32 / v_cvt_f32_f16).
__device__ __forceinline__ float h2f(_Float16 h) { return (float)h; }
__device__ __forceinline__ _Float16 f2h(float f) { return (_Float16)f; }

// model-dtype (fp16) arithmetic: one rounding per operation.
__device__ __forceinline__ _Float16 hadd(_Float16 a, _Float16 b) { return f2h(h2f(a) + h2f(b)); }
__device__ __forceinline__ _Float16 hmul(_Float16 a, _Float16 b) { return f2h(h2f(a) * h2f(b)); }

// x + dt * v with two roundings (product, then sum), never contracted into an fma:
// the same arithmetic as the float32 host Euler update.
__device__ __forceinline__ float euler_update(float x, float dt, float v) {
#pragma clang fp contract(off)
  const float p = dt * v;
  return x + p;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// The same two functions from the hardware exp2 / reciprocal (about 2 ulp of float32,
// far below the fp16 rounding their results get): 0.5 x (1 + tanh(u)) = x / (1 + e^(-2u))
// and x / (1 + e^(-x)).  Saturate correctly: e^(+big) = inf gives x * 0, e^(-big) = 0 gives x.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float gelu_tanh_hw(float x) {
  const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return x * __builtin_amdgcn_rcpf(1.0f + exp_hw(-2.0f * u));
}
__device__ __forceinline__ float silu_hw(float x) { return x * __builtin_amdgcn_rcpf(1.0f + exp_hw(-x)); }

// wave-level reductions over lanes l, l^16, l^32 (the 4 row groups of a 16x16 MFMA tile),
// on the gfx950 row-swap instructions instead of the LDS crossbar: swapping two copies of
// v pairs every lane with its xor-16 (xor-32) partner, so max / sum of the two results is
// the reduction step in every lane
__device__ __forceinline__ float xor_max_16_32(float v) {
  const unsigned b = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const unsigned c = __float_as_uint(v);
  const auto s = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float xor_sum_16_32(float v) {
  const unsigned b = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const unsigned c = __float_as_uint(v);
  const auto s = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
// lanes l < 32 receive hi_src of lane l + 32, lanes l >= 32 lo_src of lane l - 32 (the
// xor-32 exchange where the two halves send different values), one row-swap instruction
__device__ __forceinline__ float swap_halves(float lo_src, float hi_src, bool lo_lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(hi_src), __float_as_uint(lo_src), false, false);
  return __uint_as_float(lo_lane ? r[1] : r[0]);
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// 16x16x16 f16: lane l holds A[l%16][4(l/16)+i], B[4(l/16)+i][l%16], D[4(l/16)+i][l%16]
__device__ __forceinline__ f4 mfma16x16x16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16v mfma32x32x16(h8 a, h8 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Cross-workgroup hand-off without cache maintenance: data written with agent-scope
// stores (write-through to the coherent memory side), a full s_waitcnt before the
// agent-scope counter RMW, and agent-scope loads on the reading side.  This avoids the
// L2 writeback + invalidate that a device-scope fence costs on a multi-XCD part.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }
// agent-scope acquire: invalidate possibly stale cached lines before plain loads of data
// another workgroup wrote through with store_coherent (no writeback of this XCD's L2)
__device__ __forceinline__ void acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
__device__ __forceinline__ unsigned counter_add(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void counter_reset(unsigned* p) {
  __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Meeting point of the n workgroups of one group (one thread of each calls it once, after
// its stores have completed).  ctr[0] counts the arrivals of the current meeting, ctr[1]
// is its generation: the last to arrive resets the count and advances the generation, the
// others poll the generation.  The count is zero after every meeting, so launches with a
// different n may reuse the counters; meetings over the same counters must be ordered.
// The poll is bounded: false after `limit` polls (the group did not meet).
// `gen` is the generation read by group_gen at the start of the launch (the meetings of
// earlier launches over these counters have completed by then), so that read is off the
// meeting's critical path; the wait below completes it before this arrival counts.
__device__ __forceinline__ unsigned group_gen(const unsigned* ctr) {
  return __hip_atomic_load(ctr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool group_meet_gen(unsigned* ctr, unsigned n, unsigned limit, unsigned gen) {
  wait_all_memory();  // the generation is read before this arrival can complete the meeting
  if (counter_add(ctr, 1u) == n - 1) {
    counter_add(ctr + 1, 1u);  // releases the others first; nothing reads the count again here
    counter_reset(ctr);
    return true;
  }
  for (unsigned i = 0; i < limit; ++i) {
    if (__hip_atomic_load(ctr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != gen) return true;
    __builtin_amdgcn_s_sleep(2);
  }
  return false;
}

// q4f16_1 in registers: the 8 nibbles of a word -> fp16 (q - 7) * s, ordered
// [n0,n4,n1,n5,n2,n6,n3,n7] (0x6400 | q is 1024 + q in fp16, so (v - 1031) * s is exact
// before its one rounding); perm8 puts 8 consecutive X values in that order.
__device__ __forceinline__ h8 dequant_word(uint32_t word, _Float16 s) {
  h8 r;
  const h2 bias = {(_Float16)1031.0f, (_Float16)1031.0f};
  const h2 sc = {s, s};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t bits = ((word >> (4 * p)) & 0x000F000Fu) | 0x64006400u;
    h2 v = __builtin_bit_cast(h2, bits);
    v = (v - bias) * sc;
    r[2 * p] = v[0];
    r[2 * p + 1] = v[1];
  }
  return r;
}
__device__ __forceinline__ h8 perm8(h8 v) {
  h8 r;
  r[0] = v[0]; r[1] = v[4]; r[2] = v[1]; r[3] = v[5];
  r[4] = v[2]; r[5] = v[6]; r[6] = v[3]; r[7] = v[7];
  return r;
}

// Split an fp32 value into fp16 hi + lo with hi + lo ~= x to ~2^-22 relative
// (absolute floor: fp16 subnormal spacing 2^-24 on the lo part).
__device__ __forceinline__ void split_f32(float x, _Float16& hi, _Float16& lo) {
  hi = f2h(x);
  lo = f2h(x - h2f(hi));
}

}  // namespace mlcv
