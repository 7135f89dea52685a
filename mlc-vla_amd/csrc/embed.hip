// Language-token embedding of the prefix (Pi0Model.embed_language, pi0_model.py:101-104):
// out[t][:] = fp16(table[ids[t]][:] * fp16(sqrt(width))).  The scale is a constant of the
// table's dtype, so the product of two fp16 values is rounded once to fp16.
#include "kernels.h"

#include <cmath>

namespace mlcv {

namespace {

// one block per token; ids outside [0, vocab) are clamped into the table
// vec: 16-byte pieces (width % 8 == 0 and 16-byte aligned table and output)
__global__ __launch_bounds__(256) void embed_rows_kernel(const int32_t* __restrict__ ids,
                                                         const _Float16* __restrict__ table, int vocab, int width,
                                                         _Float16 scale, _Float16* __restrict__ out, int vec) {
  const int t = blockIdx.x;
  const int id = min(max(ids[t], 0), vocab - 1);
  const _Float16* row = table + (size_t)id * width;
  _Float16* o = out + (size_t)t * width;
  if (vec) {
    for (int i = threadIdx.x; i < width / 8; i += blockDim.x) {
      const h8 v = *reinterpret_cast<const h8*>(row + 8 * i);
      h8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = hmul(v[e], scale);
      *reinterpret_cast<h8*>(o + 8 * i) = r;
    }
  } else {
    for (int i = threadIdx.x; i < width; i += blockDim.x) o[i] = hmul(row[i], scale);
  }
}

}  // namespace

int embed_language_launch(const int32_t* ids, int n, const _Float16* table, int vocab, int width, _Float16* out,
                          hipStream_t st) {
  MLCV_REQUIRE(ids && table && out && n > 0 && vocab > 0 && width > 0, "embedding arguments");
  const int vec = (width & 7) == 0 && ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const _Float16 scale = (_Float16)std::sqrt((double)width);  // the constant in the table's dtype
  embed_rows_kernel<<<n, 256, 0, st>>>(ids, table, vocab, width, scale, out, vec);
  MLCV_HIP(hipGetLastError());
  return 0;
}

}  // namespace mlcv
