// The native engine's own small kernels (embedding rows, float conversion at load, the decode step's commit,
// the hidden-state restore) and their launches; the engine itself (engine.hip) is host code.
#include <algorithm>

#include "engine_kernels.h"
#include "wfb_common.h"

namespace wfb {
namespace {

// out[r, :] = table[ids[r], :] (rows of `chunks` 16-byte pieces).  Ids are checked on the host (prompt) or
// come from the argmax (decode); the clamp keeps every read inside the table regardless.  One workgroup per row.
__global__ void embed_rows_kernel(const uint4* __restrict__ table, int64_t vocab, int chunks,
                                  const int64_t* __restrict__ ids, uint4* __restrict__ out) {
  int64_t id = ids[blockIdx.x];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const uint4* src = table + id * chunks;
  uint4* dst = out + (int64_t)blockIdx.x * chunks;
  for (int i = threadIdx.x; i < chunks; i += blockDim.x) dst[i] = src[i];
}

// dst = float32 / float16 / bfloat16 source (SGLBITNT dtype ids 1 / 2 / 3) as bf16 (round to nearest even, as
// torch's conversion) or as fp32 (exact).
__global__ void to_float_kernel(const void* __restrict__ src, int dtype_id, int64_t n, void* __restrict__ dst,
                                int out_dt) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float v;
    if (dtype_id == 3) {
      const uint16_t b = reinterpret_cast<const uint16_t*>(src)[i];
      if (out_dt == WFB_BF16) {
        reinterpret_cast<uint16_t*>(dst)[i] = b;
        continue;
      }
      v = bf16_bits_to_f32(b);
    } else {
      v = dtype_id == 1 ? reinterpret_cast<const float*>(src)[i]
                        : f16_bits_to_f32(reinterpret_cast<const uint16_t*>(src)[i]);
    }
    if (out_dt == WFB_F32) reinterpret_cast<float*>(dst)[i] = v;
    else reinterpret_cast<uint16_t*>(dst)[i] = f32_to_bf16_rne(v);
  }
}

// End of a decode step: ctl = {token, position, count}.  The hidden state after the step (the token run
// through every layer, `chunks` 16-byte pieces) goes to ring slot count % ring, the token to tokens[count]
// (when count < cap) and to *last; then position and count advance.  One workgroup.
__global__ void commit_kernel(int64_t* __restrict__ ctl, int32_t* __restrict__ tokens, int64_t cap,
                              int32_t* __restrict__ last, const uint4* __restrict__ x, uint4* __restrict__ ring,
                              int nring, int chunks) {
  const int64_t count = ctl[2];
  uint4* dst = ring + (count % nring) * chunks;
  for (int i = threadIdx.x; i < chunks; i += blockDim.x) dst[i] = x[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    const int32_t tok = (int32_t)ctl[0];
    if (count >= 0 && count < cap) tokens[count] = tok;
    *last = tok;
    ctl[1] = ctl[1] + 1;
    ctl[2] = count + 1;
  }
}

// dst = src (`chunks` 16-byte pieces): a ring slot back to the hidden state.
__global__ void copy_row_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, int chunks) {
  for (int i = threadIdx.x; i < chunks; i += blockDim.x) dst[i] = src[i];
}

}  // namespace

hipError_t launch_embed_rows(const void* table, int64_t vocab, int h, int es, const int64_t* ids, int64_t rows,
                             void* out, hipStream_t s) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, static_cast<const uint4*>(table), vocab,
                     h * es / 16, ids, static_cast<uint4*>(out));
  return hipGetLastError();
}

hipError_t launch_to_float(const void* src, int dtype_id, int64_t n, void* dst, int out_dt, hipStream_t s) {
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(to_float_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dtype_id, n, dst, out_dt);
  return hipGetLastError();
}

hipError_t launch_commit(int64_t* ctl, int32_t* tokens, int64_t cap, int32_t* last, const void* x, void* ring,
                         int nring, int h, int es, hipStream_t s) {
  hipLaunchKernelGGL(commit_kernel, dim3(1), dim3(256), 0, s, ctl, tokens, cap, last, static_cast<const uint4*>(x),
                     static_cast<uint4*>(ring), nring, h * es / 16);
  return hipGetLastError();
}

hipError_t launch_copy_row(const void* src, void* dst, int h, int es, hipStream_t s) {
  hipLaunchKernelGGL(copy_row_kernel, dim3(1), dim3(256), 0, s, static_cast<const uint4*>(src), static_cast<uint4*>(dst),
                     h * es / 16);
  return hipGetLastError();
}

}  // namespace wfb
