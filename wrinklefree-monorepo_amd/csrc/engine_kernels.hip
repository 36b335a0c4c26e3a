// The native engine's own small kernels (embedding rows, bf16 conversion at load, the decode step's commit,
// the hidden-state restore) and their launches; the engine itself (engine.hip) is host code.
#include <algorithm>

#include "engine_kernels.h"
#include "wfb_common.h"

namespace wfb {
namespace {

// out[r, :] = table[ids[r], :] (bf16 rows of h elements, h % 8 == 0).  Ids are checked on the host
// (prompt) or come from the argmax (decode); the clamp keeps every read inside the table regardless.
// One workgroup per row.
__global__ void embed_rows_kernel(const uint16_t* __restrict__ table, int64_t vocab, int h,
                                  const int64_t* __restrict__ ids, uint16_t* __restrict__ out) {
  int64_t id = ids[blockIdx.x];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const uint4* src = reinterpret_cast<const uint4*>(table + id * h);
  uint4* dst = reinterpret_cast<uint4*>(out + (int64_t)blockIdx.x * h);
  for (int i = threadIdx.x; i < h / 8; i += blockDim.x) dst[i] = src[i];
}

// dst = bf16(src) for a float32 / float16 / bfloat16 source (SGLBITNT dtype ids 1 / 2 / 3);
// round to nearest even, as torch's conversion.
__global__ void to_bf16_kernel(const void* __restrict__ src, int dtype_id, int64_t n, uint16_t* __restrict__ dst) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (dtype_id == 3) {
      dst[i] = reinterpret_cast<const uint16_t*>(src)[i];
    } else {
      const float v = dtype_id == 1 ? reinterpret_cast<const float*>(src)[i]
                                    : f16_bits_to_f32(reinterpret_cast<const uint16_t*>(src)[i]);
      dst[i] = f32_to_bf16_rne(v);
    }
  }
}

// End of a decode step: ctl = {token, position, count}.  The hidden state after the step (the token run
// through every layer) goes to ring slot count % ring, the token to tokens[count] (when count < cap) and
// to *last; then position and count advance.  One workgroup.
__global__ void commit_kernel(int64_t* __restrict__ ctl, int32_t* __restrict__ tokens, int64_t cap,
                              int32_t* __restrict__ last, const uint16_t* __restrict__ x, uint16_t* __restrict__ ring,
                              int nring, int h) {
  const int64_t count = ctl[2];
  const uint4* src = reinterpret_cast<const uint4*>(x);
  uint4* dst = reinterpret_cast<uint4*>(ring + (count % nring) * h);
  for (int i = threadIdx.x; i < h / 8; i += blockDim.x) dst[i] = src[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    const int32_t tok = (int32_t)ctl[0];
    if (count >= 0 && count < cap) tokens[count] = tok;
    *last = tok;
    ctl[1] = ctl[1] + 1;
    ctl[2] = count + 1;
  }
}

// dst = src (h bf16 elements, h % 8 == 0): a ring slot back to the hidden state.
__global__ void copy_row_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int h) {
  for (int i = threadIdx.x; i < h / 8; i += blockDim.x)
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
}

}  // namespace

hipError_t launch_embed_rows(const uint16_t* table, int64_t vocab, int h, const int64_t* ids, int64_t rows,
                             uint16_t* out, hipStream_t s) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, table, vocab, h, ids, out);
  return hipGetLastError();
}

hipError_t launch_to_bf16(const void* src, int dtype_id, int64_t n, uint16_t* dst, hipStream_t s) {
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dtype_id, n, dst);
  return hipGetLastError();
}

hipError_t launch_commit(int64_t* ctl, int32_t* tokens, int64_t cap, int32_t* last, const uint16_t* x, uint16_t* ring,
                         int nring, int h, hipStream_t s) {
  hipLaunchKernelGGL(commit_kernel, dim3(1), dim3(256), 0, s, ctl, tokens, cap, last, x, ring, nring, h);
  return hipGetLastError();
}

hipError_t launch_copy_row(const uint16_t* src, uint16_t* dst, int h, hipStream_t s) {
  hipLaunchKernelGGL(copy_row_kernel, dim3(1), dim3(256), 0, s, src, dst, h);
  return hipGetLastError();
}

}  // namespace wfb
