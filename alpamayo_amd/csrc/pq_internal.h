// Launchers shared between the library's translation units (not exported).
#ifndef PQ_INTERNAL_H
#define PQ_INTERNAL_H

#include "pq_common.h"

#define PQ_HIDDEN __attribute__((visibility("hidden")))

namespace pq {

// Rows per launch of the split rotation (and rows the rotated GEMM accepts).
constexpr int kSplitMaxRows = 16;

// Rotation of m <= kSplitMaxRows rows with one wave per 128-channel group:
// xr [m][h] rotated values (fp16 when flags has PQ_RQ_MATERIALIZE_FP16, else
// fp32) and gmax [m][h/128] the absmax of each row's group.
PQ_HIDDEN void launch_rotate_split(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                                   const float* scales, void* xr, float* gmax, int m, int h, int krot, unsigned flags,
                                   hipStream_t stream);

// Decode GEMM whose A operand is quantized in the kernel from launch_rotate_split's
// output: token scale = max over the row's gmax / 127.  Returns false when m or
// the LDS image of A (m x (k + 16) bytes) is out of range.
PQ_HIDDEN bool gemm_rotated_supported(int64_t m, int64_t k);
PQ_HIDDEN void launch_gemm_rotated(const void* xr, bool xr_fp16, const float* gmax, const uint8_t* wpack,
                                   const uint32_t* wmeta, const void* bias, int bias_dtype, void* y, int y_dtype,
                                   int m, int n, int k, hipStream_t stream);

}  // namespace pq

#endif
