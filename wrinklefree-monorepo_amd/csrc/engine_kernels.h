// Launches of the native engine's small kernels (engine_kernels.hip), host declarations only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wfb {

// out[r, :] = table[ids[r], :] for r < rows (rows of h elements of es bytes, es = 2 or 4, h % 8 == 0; ids
// clamped to the table).
hipError_t launch_embed_rows(const void* table, int64_t vocab, int h, int es, const int64_t* ids, int64_t rows,
                             void* out, hipStream_t s);
// dst = src converted to out_dt (WFB_BF16: round to nearest even; WFB_F32: exact) for SGLBITNT float dtypes
// 1 (f32), 2 (f16), 3 (bf16).
hipError_t launch_to_float(const void* src, int dtype_id, int64_t n, void* dst, int out_dt, hipStream_t s);
// End of a decode step, ctl = {token, position, count}: hidden x (h elements of es bytes) to ring slot
// count % nring, the token to tokens[count] (count < cap) and *last, position and count + 1.
hipError_t launch_commit(int64_t* ctl, int32_t* tokens, int64_t cap, int32_t* last, const void* x, void* ring,
                         int nring, int h, int es, hipStream_t s);
// dst = src, h elements of es bytes (h % 8 == 0).
hipError_t launch_copy_row(const void* src, void* dst, int h, int es, hipStream_t s);

}  // namespace wfb
