// Load-time format conversion on the device: HF "offline" ternary layout -> I2_S.
//
// Source layout (packages/inference/scripts/quantize_dlm_to_offline.py:27-98, the layout of the HF
// BitNet integration): uint8 [NB, K] with NB = ceil(N/4); byte (j, k) holds column k of rows j, j + NB,
// j + 2NB and j + 3NB in bits 1:0, 3:2, 5:4 and 7:6, code = w + 1.  The reference converter
// (packages/inference/scripts/convert_to_sglkernel.py:221-246) unpacks all 4*NB rows and repacks
// w * weight_scale with pack_ternary_sglkernel, which keeps every code (|w| / mean|w| >= 1 rounds and
// clamps back to +-1) and sets the scale to mean(|w * weight_scale|) = weight_scale * nnz / (4*NB*K).
// Code 3 (never written) unpacks to +2 there and clamps to +1; it is mapped to +1 here too.
//
// One thread per output dword (bytes j0..j0+3 of one 128-weight I2_S block): each output byte gathers
// the codes of columns 128b + 32f + j (f = 0..3) of its row from the source byte row r % NB, shifted
// by 2*(r / NB).  Columns past K (up to k_pad) are zero weights.  Every workgroup also counts the
// non-zero weights it wrote (exact integer partials, summed by the scale kernel).
#include "wfb_common.h"

namespace wfb {

namespace {

__device__ __forceinline__ uint32_t code_at(const uint8_t* src, int64_t srow, int64_t k, int64_t kk, int sh) {
  if (kk >= k) return 1u;
  const uint32_t c = (src[srow * k + kk] >> sh) & 3u;
  return c == 3u ? 2u : c;
}

__global__ __launch_bounds__(256) void convert_hf_kernel(const uint8_t* __restrict__ src, int64_t nb, int64_t n,
                                                         int64_t k, int64_t k_pad, uint32_t* __restrict__ qw,
                                                         int64_t* __restrict__ part_nnz, bool vec4) {
  __shared__ int red[4];
  const int64_t per_row = k_pad / 16;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int nnz = 0;
  if (idx < n * per_row) {
    const int64_t r = idx / per_row, p = idx % per_row;
    const int64_t b = p / 8;
    const int j0 = 4 * (int)(p % 8);
    const int64_t srow = r % nb;
    const int sh = 2 * (int)(r / nb);
    uint32_t out = 0;
    if (vec4) {
      // the 4 source bytes j0..j0+3 of each field f are one dword (K % 4 == 0): 4 loads in flight,
      // bounded at the source row's end (dwords past it read as 0; their columns take code 1 below)
      const buf_t rb = make_buf(src + srow * k, (uint32_t)k);
      uint32_t w4[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) w4[f] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rb, (int)(128 * b + 32 * f + j0), 0, 0);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        uint32_t byte = 0;
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          uint32_t c = (w4[f] >> (8 * jj + sh)) & 3u;
          c = 128 * b + 32 * f + j0 + jj < k ? (c == 3u ? 2u : c) : 1u;
          byte |= c << (6 - 2 * f);
          nnz += c != 1u;
        }
        out |= byte << (8 * jj);
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        uint32_t byte = 0;
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const uint32_t c = code_at(src, srow, k, 128 * b + 32 * f + j0 + jj, sh);
          byte |= c << (6 - 2 * f);
          nnz += c != 1u;
        }
        out |= byte << (8 * jj);
      }
    }
    qw[idx] = out;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) nnz += __shfl_xor(nnz, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = nnz;
  __syncthreads();
  if (threadIdx.x == 0) part_nnz[blockIdx.x] = (int64_t)red[0] + red[1] + red[2] + red[3];
}

// Sums the partial counts, adds the non-zeros of the padding rows n .. 4*NB-1 (they count in the
// reference's mean too), and writes the scale.
__global__ __launch_bounds__(256) void convert_scale_kernel(const int64_t* __restrict__ part_nnz, int64_t nparts,
                                                            const uint8_t* __restrict__ src, int64_t nb, int64_t n,
                                                            int64_t k, const void* __restrict__ ws_dev, int ws_dt,
                                                            float ws_host, int mode, float* __restrict__ scale_out) {
  __shared__ int64_t red[256];
  int64_t acc = 0;
  for (int64_t i = threadIdx.x; i < nparts; i += 256) acc += part_nnz[i];
  for (int64_t i = threadIdx.x; i < (4 * nb - n) * k; i += 256) {
    const int64_t r = n + i / k, kk = i % k;
    acc += code_at(src, r % nb, k, kk, 2 * (int)(r / nb)) != 1u;
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float ws = ws_host;
    if (ws_dev) ws = ws_dt == WFB_F32 ? reinterpret_cast<const float*>(ws_dev)[0]
                                      : bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(ws_dev)[0]);
    float s = ws;
    if (mode == WFB_SCALE_REFERENCE) {
      s = (float)((double)ws * ((double)red[0] / ((double)(4 * nb) * (double)k)));
      if ((double)s < 1e-8) s = 1.0f;
    }
    scale_out[0] = s;
  }
}

}  // namespace

hipError_t launch_convert_hf_offline(const uint8_t* src, int64_t nb, int64_t n, int64_t k, int64_t k_pad,
                                     const void* ws_dev, int ws_dt, float ws_host, int mode, uint8_t* qw,
                                     float* scale_out, int64_t* parts, hipStream_t s) {
  const int64_t total = n * (k_pad / 16);
  const int64_t blocks = (total + 255) / 256;
  // dword source loads when every source row starts 4-byte aligned and its bytes fit a buffer range
  const bool vec4 = k % 4 == 0 && (uintptr_t)src % 4 == 0 && k < (int64_t)1 << 31;
  hipLaunchKernelGGL(convert_hf_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, nb, n, k, k_pad,
                     reinterpret_cast<uint32_t*>(qw), parts, vec4);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(convert_scale_kernel, dim3(1), dim3(256), 0, s, parts, blocks, src, nb, n, k, ws_dev, ws_dt,
                     ws_host, mode, scale_out);
  return hipGetLastError();
}

}  // namespace wfb
