// Launchers shared between the library's translation units (not exported).
#ifndef PQ_INTERNAL_H
#define PQ_INTERNAL_H

#include "pq_common.h"

#define PQ_HIDDEN __attribute__((visibility("hidden")))

namespace pq {

// Linears that share one input run as a group: one rotation launch and one
// GEMM launch over the members' concatenated output columns.
constexpr int kMaxGroup = 4;

// One member of a GEMM group: its A operand (int8 rows xq + token scales xs,
// or rotated rows xr + per-group maxima gmax), its packed weights, its bias
// and its output y [m][n].  The partials instances of the kernels (the
// parity entry points) write, instead of y, the member's int32 partials
// [m][k/128][n] and, when the kernel quantizes A itself, the int8 image of A
// it multiplies (a_out [m][k]) and the token scales of its epilogue
// (as_out [m]).
struct GemmMember {
  const int8_t* xq;
  const float* xs;
  const void* xr;
  const float* gmax;
  const uint8_t* wpack;
  const uint32_t* wmeta;
  const void* bias;
  void* y;
  int n;
  int32_t* partials;
  int8_t* a_out;
  float* as_out;
};
struct GemmGroup {
  GemmMember mem[kMaxGroup];
  int count;
  int first[kMaxGroup + 1];   // first workgroup tile of each member; set by the launchers
};

// One member of a rotation group (grid.y = member): its rotation operands,
// its outputs -- out / out_scale = xr / gmax for the split rotation, xq /
// xscale for the row rotate+quant -- and an optional fp16 copy of the
// rotated rows (xrot, row kernel only).
struct RotMember {
  const uint32_t* rot_idx;
  const float* rot_cs;
  const float* scales;
  void* out;
  float* out_scale;
  void* xrot;
};
struct RotGroup {
  RotMember mem[kMaxGroup];
  int count;
};

// Per-token int8 quantization of a split rotation's output (launch_quant_split):
// xr [m][k] (fp16 or fp32) and gmax [m][k/128] in, xq [m][k] and xscale [m] out.
struct QuantMember {
  const void* xr;
  const float* gmax;
  int8_t* xq;
  float* xscale;
};
struct QuantGroup {
  QuantMember mem[kMaxGroup];
  int count;
};

// Rows per launch of the split rotation (and rows the rotated GEMM accepts).
constexpr int kSplitMaxRows = 16;

// Optional RMSNorm prologue of a group's rotation (a decoder layer's norm in
// front of q/k/v or gate/up):  s = x + res (rounded to x's dtype; s = x when
// res is null),  h = round(w * round(s * rsqrt(mean_k(s^2) + eps))), both
// roundings to x's dtype, mean and rsqrt in float32.  The members rotate h;
// h and s are also written when h_out / s_out are set ([m][k], x's dtype).
// w: [k] in x's dtype.
//
// mode generalizes the prologue (PQ_PRO_*): RMSNORM as above; ADD rotates
// s = x + res (rounded to x's dtype) and writes it to s_out when set; SWIGLU
// rotates h = round(round(silu(x)) * res) (silu in float32: x / (1 + exp(-x)))
// and writes it to h_out when set.
struct NormArgs {
  const void* res;
  const void* w;
  void* h_out;
  void* s_out;
  float eps;
  int mode;
};

// Rotation of m <= kSplitMaxRows rows with one wave per 128-channel group,
// for every member of the group: xr [m][h] rotated values (fp16 when flags
// has PQ_RQ_MATERIALIZE_FP16, else fp32) and gmax [m][h/128] the absmax of
// each row's group.
// rows_per_wave > 0 spreads the m rows over ceil(m / rows_per_wave) waves
// per group (each wave then holds at most rows_per_wave rows); 0 keeps all
// m <= kSplitMaxRows rows in one wave.
PQ_HIDDEN void launch_rotate_split(const void* x, int x_dtype, const RotGroup& grp, int m, int h, int krot,
                                   unsigned flags, hipStream_t stream, const NormArgs* norm = nullptr,
                                   int rows_per_wave = 0);
// Token scales (absmax / 127 over each row's group maxima) and int8 codes of
// a split rotation's rows; the same values the rotated decode GEMM derives in
// its prologue.  mat16: xr holds fp16 (else fp32).
PQ_HIDDEN void launch_quant_split(const QuantGroup& grp, int m, int h, bool mat16, hipStream_t stream);
// Rotation + per-token int8 quant of whole rows for every member of the group.
PQ_HIDDEN void launch_rotate_quant_group(const void* x, int x_dtype, const RotGroup& grp, int64_t rows, int h,
                                         int krot, unsigned flags, hipStream_t stream,
                                         const NormArgs* norm = nullptr);

// Decode GEMM whose A operand is quantized in the kernel from launch_rotate_split's
// output: token scale = max over the row's gmax / 127.  Returns false when m or
// the LDS image of A (m x (k + 16) bytes) is out of range.
PQ_HIDDEN bool gemm_rotated_supported(int64_t m, int64_t k);
// The GEMM of a group (count >= 1 members, same m and k).  aq selects the A
// operand: 0 = xq/xs (any m), 1 / 2 = fp16 / fp32 xr plus gmax quantized in
// the kernel (gemm_rotated_supported(m, k)).
PQ_HIDDEN void launch_gemm_group(GemmGroup grp, int aq, int bias_dtype, int y_dtype, int m, int k,
                                 hipStream_t stream);
// launch_gemm_group's kernels, with the same configuration and tiling, in
// their partials form: each member's int32 partials (and, for aq != 0, its
// A image and token scales) go to the member's partials / a_out / as_out.
PQ_HIDDEN void launch_gemm_group_partials(GemmGroup grp, int aq, int m, int k, hipStream_t stream);

}  // namespace pq

#endif
