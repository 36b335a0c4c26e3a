// Launches of the native engine's small kernels (engine_kernels.hip), host declarations only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wfb {

// out[r, :] = table[ids[r], :] for r < rows (bf16 rows of h elements, h % 8 == 0; ids clamped to the table).
hipError_t launch_embed_rows(const uint16_t* table, int64_t vocab, int h, const int64_t* ids, int64_t rows,
                             uint16_t* out, hipStream_t s);
// dst = bf16(src) (round to nearest even) for SGLBITNT float dtypes 1 (f32), 2 (f16), 3 (bf16).
hipError_t launch_to_bf16(const void* src, int dtype_id, int64_t n, uint16_t* dst, hipStream_t s);
// End of a decode step, ctl = {token, position, count}: hidden x to ring slot count % nring, the token to
// tokens[count] (count < cap) and *last, position and count + 1.
hipError_t launch_commit(int64_t* ctl, int32_t* tokens, int64_t cap, int32_t* last, const uint16_t* x, uint16_t* ring,
                         int nring, int h, hipStream_t s);
// dst = src, h bf16 elements (h % 8 == 0).
hipError_t launch_copy_row(const uint16_t* src, uint16_t* dst, int h, hipStream_t s);

}  // namespace wfb
