/*
 * paroquant_hip.h -- C ABI of libparoquant_hip.so, the MI355X (gfx950)
 * implementation of the ParoQuant W4A8 linear path.
 *
 * Conventions (shared by every entry point):
 *   - plain pointers and sizes; every device buffer is allocated by the
 *     caller; no entry point allocates device memory or synchronises;
 *   - work is enqueued on the `stream` argument (a hipStream_t, passed as
 *     void* so the header needs no HIP include; NULL = default stream);
 *   - the return value is a pq_status; on failure pq_last_error() returns a
 *     thread-local message describing the first failing check.  Arguments
 *     are validated on the host before anything is launched;
 *   - inputs are never written.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   pq_rotate            torch.ops.rotation.rotate
 *                        kernels/paroquant_kernels/src/rotation.cu:456-493, 576-584
 *   pq_rotation_pack     load-time packing of Rotation's buffers (host)
 *                        src/alpamayo_r1/utils/quantization/rotation_linear.py:26-43
 *   pq_rotate_quant_i8   rotation.rotate (fp16) followed by vLLM's per-token
 *                        int8 quant inside apply_awq_marlin_linear
 *                        src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:59-65, 319-333
 *   pq_quant_i8          the per-token int8 quant alone (same call site)
 *   pq_w4a8_gemm         the Marlin int4 x int8 GEMM (same call site, launch #4)
 *   pq_w4a8_prepack      MarlinW4A8Linear.load_from_awq's repack of AWQ
 *                        buffers (paroquant_marlin_w4a8.py:274-312)
 *   pq_w4a8_linear       the whole linear of a converted layer:
 *                        BF16RotateLinearWrapper -> RotateLinearInt4 ->
 *                        rotation::rotate -> MarlinW4A8Linear.forward
 *                        (paroquant_marlin_w4a8.py:59-65, 314-333;
 *                        rotation_linear.py:120-124)
 *   pq_rotate_backward   RotateTensorFunc.backward
 *                        kernels/paroquant_kernels/interface.py:30-93
 *   pq_rotate_mxfp4      rotation::rotate_and_quant (rotation.cu:62-111),
 *                        in the OCP MXFP4 format instead of NVFP4
 *   pq_w4a16_gemm        torch.ops.awq.gemv / torch.ops.awq.gemm behind
 *                        WQLinear.forward (qmodule.py:207-232)
 *   pq_w4a16_prepack     the weight preparation those kernels need
 *   pq_w4a16_linear      RotateLinearInt4.forward with a WQLinear:
 *                        rotation::rotate -> WQLinear.forward
 *                        (rotation_linear.py:136-139)
 *   pq_w4a16_linear_group  the same for linears sharing their input
 *                        (no counterpart)
 */
#ifndef PAROQUANT_HIP_H
#define PAROQUANT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PQ_ABI_VERSION 1

enum pq_status {
  PQ_OK = 0,
  PQ_ERR_ARG = 1,          /* bad pointer, size, alignment or shape */
  PQ_ERR_UNSUPPORTED = 2,  /* valid but not implemented (dtype, krot, group) */
  PQ_ERR_HIP = 3,          /* a HIP runtime call failed */
  PQ_ERR_WORKSPACE = 4     /* workspace missing or too small */
};

enum pq_dtype { PQ_F32 = 0, PQ_F16 = 1, PQ_BF16 = 2 };

/* flags of pq_rotate_quant_i8 */
#define PQ_RQ_INPUT_FP16 1u        /* round the input to fp16 first (the bf16->fp16 wrapper cast) */
#define PQ_RQ_MATERIALIZE_FP16 2u  /* round rotated values to fp16 before quantizing */

/* Prologue of pq_w4a8_linear_group_fused: what the members rotate, from x and x2. */
#define PQ_PRO_RMSNORM 1  /* h = RMSNorm(x + x2) (x2 may be NULL), as pq_w4a8_linear_group_rmsnorm */
#define PQ_PRO_ADD 2      /* s = x + x2 (the residual add of a decoder layer) */
#define PQ_PRO_SWIGLU 3   /* h = silu(x) * x2 (x = gate, x2 = up: a gated MLP's down_proj input) */

int pq_abi_version(void);
const char* pq_last_error(void);

/* y = R_{krot-1} ... R_0 (scales * x) per group, the rotation::rotate op.
 * x, y: [rows, h] of `dtype`; idx_ij: int16 [krot, h] group-local pair
 * indices (pair t of group g = idx[r, g*G+2t], idx[r, g*G+2t+1]); theta:
 * [krot, h/2] of `dtype`; scales: [h] of `dtype` or NULL.
 * krot in {1, 2, 4, 8, 16}; group_size in {64, 128}; h % group_size == 0.
 * Each layer must pair every channel of a group exactly once.
 * Reference: rotation.cu:116-225 (launcher), 456-493 (dispatch). */
int pq_rotate(const void* x, void* y, const int16_t* idx_ij, const void* theta,
              const void* scales, int64_t rows, int64_t h, int krot, int group_size,
              int dtype, void* stream);

/* Bytes of workspace pq_rotate_backward needs: per-workgroup partial sums,
 * min(ceil(rows / 16), 64) * (krot * h/2 + h) * 4 bytes (0 for rows = 0). */
size_t pq_rotate_backward_workspace_size(int64_t rows, int64_t h, int krot);

/* Gradients of pq_rotate's y = R_{krot-1} ... R_0 (scales * x) given grad_y:
 * grad_x [rows, h], grad_theta [krot, h/2] (summed over rows) and, when
 * scales is not NULL, grad_scales [h] (summed over rows), all of `dtype`
 * like x, grad_y, theta and scales; arguments and rules as for pq_rotate.
 * The layers are recomputed from x in float32 (each layer's outputs kept),
 * then walked backwards: the angle gradient of a pair is
 * sum_rows g_a' * b' - g_b' * a' at the layer's outputs (a', b') and
 * gradients (g_a', g_b'), and the gradient passes through the transposed
 * rotation; grad_x = scales * g_t and grad_scales = sum_rows x * g_t at
 * t = scales * x.  Sums are float32 in a fixed order (deterministic).
 * workspace: pq_rotate_backward_workspace_size bytes, 16-byte aligned.
 * Reference: RotateTensorFunc.backward (kernels/paroquant_kernels/
 * interface.py:30-93), which gives the same gradients by inverting y one
 * layer at a time with rotation::rotate. */
int pq_rotate_backward(const void* x, const void* grad_y, void* grad_x, void* grad_theta, void* grad_scales,
                       const int16_t* idx_ij, const void* theta, const void* scales, int64_t rows, int64_t h,
                       int krot, int group_size, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Fused rotation + OCP MXFP4 quantization: the rotation of pq_rotate (same
 * arguments and rules), then, per row and per block of 32 channels of the
 * float32 result v, the shared exponent e = floor(log2(max|v|)) - 2 clamped
 * to [-127, 127] and the E2M1 code of each v / 2^e (round to nearest even,
 * saturating at +-6, sign kept).  q_out: uint8 [rows, h/2], element 2i in
 * the low nibble of byte i, 4-byte aligned; scale_out: uint8 [rows, h/32],
 * the E8M0 byte e + 127, or 0xFF for a block holding a NaN.
 * Reference: rotation::rotate_and_quant (rotation.cu:62-111, 230-315, 587),
 * which writes NVFP4 (16-element blocks, FP8 scales, a global scale); this
 * entry point is its counterpart in the MX format gfx950 multiplies natively. */
int pq_rotate_mxfp4(const void* x, uint8_t* q_out, uint8_t* scale_out, const int16_t* idx_ij, const void* theta,
                    const void* scales, int64_t rows, int64_t h, int krot, int group_size, int dtype, void* stream);

/* pq_rotate (out_mode PQ_ROWS_SAME: out [rows, h] in x_dtype) or
 * pq_rotate_mxfp4 (PQ_ROWS_MXFP4: out = codes [rows, h/2], mx_scales
 * [rows, h/32]) on packed rotation operands (pq_rotation_pack, group 128,
 * cos/sin of each angle evaluated in float64 and rounded to float32) and
 * float32 channel scales (or NULL): the register-chain kernel of the fused
 * linear, whole rows per workgroup.  The results equal pq_rotate's /
 * pq_rotate_mxfp4's on the pairs and angles the operands were packed from.
 * h % 128 == 0, h <= 16384, krot in 1..16; x, out, rot_idx, rot_cs 16-byte
 * aligned.  Reference: rotation::rotate (rotation.cu:456-493) and the fused
 * rotate_and_quant (rotation.cu:62-111), in the MX format for the latter. */
int pq_rotate_rows(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs, const float* scales,
                   void* out, uint8_t* mx_scales, int64_t rows, int64_t h, int krot, int out_mode, void* stream);

/* out_mode of pq_rotate_rows */
#define PQ_ROWS_SAME 0   /* rotated rows in x's dtype (rotation::rotate) */
#define PQ_ROWS_MXFP4 1  /* OCP MXFP4 codes + E8M0 scales (rotation::rotate_and_quant_mxfp4) */

/* Packs rotation parameters (host memory, host code; no GPU involved) into
 * the operand layout of the fused kernels, G = h/128, KP = 8 for krot <= 8,
 * else 16:
 *   rot_idx [G][64][KP/2] uint32  per lane: word 0 = Af | Bf << 8 | init << 16,
 *                                 byte 4 + r = src | flag << 7 (layer r)
 *   rot_cs  [G][64][KP][2] float  (cos, +-sin) of the lane's pair in layer r
 * The kernels rotate a group with one wave in registers: lane l starts with
 * channels l and l+64 in slots (a, b) (swapped if init), fetches before each
 * layer slot a of lane `src` with one cross-lane read (into slot a if flag,
 * else slot b, its old slot b going to the other slot), applies
 * a' = fma(a, c, b*s), b' = fma(b, c, -(a*s)), and ends with channels Af, Bf
 * in slots a, b.  Input: pairs int16 [krot][h] group-local (pair t of group
 * g = pairs[r][g*128+2t], +1) and cos_sin float [krot][h/2][2] (the pair's
 * angle in theta's layout).  krot in 1..16.  Fails with PQ_ERR_ARG unless
 * every layer pairs each channel of each 128-group exactly once.
 * Reference: the parameters of Rotation (rotation_linear.py:26-43). */
int pq_rotation_pack(const int16_t* pairs, const float* cos_sin, int64_t h, int krot, uint32_t* rot_idx,
                     float* rot_cs);

/* Fused rotation + channel scale + per-token absmax + int8 quantization.
 * x: [rows, h] of x_dtype; rot_idx / rot_cs: packed parameters
 * (pq_rotation_pack) of krot layers; scales: float32 [h] or NULL.
 * Outputs xq int8 [rows, h], xscale float32 [rows] (absmax/127), and, when
 * xrot is not NULL, the rotated activations as fp16 [rows, h].
 * flags: PQ_RQ_* bits.  krot in 1..16, h % 128 == 0, h <= 16384.
 * Reference: rotation.cu:15-60 + paroquant_marlin_w4a8.py:319-333. */
int pq_rotate_quant_i8(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                       const float* scales, int8_t* xq, float* xscale, void* xrot,
                       int64_t rows, int64_t h, int krot, unsigned flags, void* stream);

/* Per-token int8 quantization of x [rows, h] (x_dtype) -> xq, xscale.
 * Reference: vLLM scaled_int8_quant as called at paroquant_marlin_w4a8.py:319-333. */
int pq_quant_i8(const void* x, int x_dtype, int8_t* xq, float* xscale, int64_t rows, int64_t h,
                void* stream);

/* Bytes of workspace pq_w4a8_gemm needs for this shape.  No kernel of this
 * version exchanges data between workgroups, so this is 0 and the workspace
 * arguments of pq_w4a8_gemm are ignored; they stay in the ABI for kernels
 * that may need one (a non-zero size would come with its own rules). */
size_t pq_w4a8_workspace_size(int64_t m, int64_t n, int64_t k, int group_size);

/* y[m, n] = xscale[m] * sum_g s[g, n] * sum_{k in g} (q[k, n] - z[g, n]) * xq[m, k]
 *           (+ bias[n]),  written as y_dtype.
 * xq: int8 [m, k]; xscale: float32 [m]; wpack/wmeta: the prepacked weights
 * (pq_w4a8_prepack); bias: [n] of bias_dtype or NULL.
 * group_size == 128, k % 128 == 0, n % 16 == 0.
 * Reference: apply_awq_marlin_linear, paroquant_marlin_w4a8.py:314-333. */
int pq_w4a8_gemm(const int8_t* xq, const float* xscale, const uint8_t* wpack, const uint32_t* wmeta,
                 const void* bias, int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n,
                 int64_t k, int group_size, void* workspace, size_t workspace_bytes, void* stream);

/* Debug/parity variant: the exact per-group int32 partials
 * partials[m, g, n] = sum_{k in g} (q[k, n] - z[g, n]) * xq[m, k].
 * Same kernels as pq_w4a8_gemm up to the epilogue.  Reference: the int32
 * accumulators of the Marlin W4A8 GEMM (paroquant_marlin_w4a8.py:319-333). */
int pq_w4a8_gemm_partials(const int8_t* xq, const uint8_t* wpack, const uint32_t* wmeta,
                          int32_t* partials, int64_t m, int64_t n, int64_t k, int group_size,
                          void* stream);

/* Repack AWQ buffers into the kernel layout.
 * awq_qweight: int32 [k, n/8]; awq_scales: fp16 bits [k/128, n];
 * awq_qzeros: int32 [k/128, n/8] (nibble order 0,2,4,6,1,3,5,7).
 * wpack: uint8 [n/16, k/128, 64, 16] (n*k/2 bytes); wmeta: uint32 [n/16, k/128, 16].
 * Reference: MarlinW4A8Linear.load_from_awq, paroquant_marlin_w4a8.py:274-312. */
int pq_w4a8_prepack(const int32_t* awq_qweight, const uint16_t* awq_scales,
                    const int32_t* awq_qzeros, uint8_t* wpack, uint32_t* wmeta, int64_t k,
                    int64_t n, int group_size, void* stream);

/* Bytes of scratch pq_w4a8_linear needs between its kernels.  Size it with
 * this function rather than a formula of your own; the rule it follows is:
 *   split pair (m*k <= 8192, or k >= 8192 and m <= 2): the rotated rows and
 *     per-group maxima, m*k*4 rounded up to 256 plus 4*m*(k/128) bytes;
 *   three launches (k a multiple of 128 in [4096, 16384], beyond the split
 *     pair, up to m = 32): both of those plus the int8 activations and
 *     their scales (m*k rounded up to 256, plus 4*m);
 *   otherwise (the row rotate+quant kernel): the int8 activations and their
 *     scales only, m*k rounded up to 256 plus 4*m bytes.
 * The scratch is written before it is read; its content does not matter. */
size_t pq_w4a8_linear_workspace_size(int64_t m, int64_t n, int64_t k, int krot);

/* y = W4A8 GEMM of the per-token int8 quantization of the rotation of x:
 * x [m, k] (x_dtype) -> y [m, n] (y_dtype), rotation operands as for
 * pq_rotate_quant_i8, weights as for pq_w4a8_gemm, flags PQ_RQ_*.
 * k <= 16384.  Same results as pq_rotate_quant_i8 followed by pq_w4a8_gemm.
 * Reference: paroquant_marlin_w4a8.py:59-65, 314-333; rotation_linear.py:120-124. */
int pq_w4a8_linear(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs, const float* scales,
                   const uint8_t* wpack, const uint32_t* wmeta, const void* bias, int bias_dtype, void* y,
                   int y_dtype, int64_t m, int64_t n, int64_t k, int krot, unsigned flags, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Bytes of the library's fixed scratch array used by pq_w4a8_linear_noalloc
 * (one array per GPU, held until the process ends). */
#define PQ_NOALLOC_SCRATCH_BYTES (16u << 20)

/* pq_w4a8_linear without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The scratch between its kernels is a
 * fixed array of PQ_NOALLOC_SCRATCH_BYTES per GPU inside the library (its
 * address is looked up once per device, on the first call made with that
 * device current); the call itself allocates nothing.  Same kernels and same
 * results as pq_w4a8_linear.  Fails with PQ_ERR_WORKSPACE, before touching
 * the GPU, when pq_w4a8_linear_workspace_size(m, n, k, krot) exceeds
 * PQ_NOALLOC_SCRATCH_BYTES (e.g. more than about 16.7M int8 activations on
 * the row path: m = 3072 at k = 4096 fits, at k = 12288 it does not).
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents (the kernels write it before reading it; nothing needs to start at
 * zero): calls that overlap in time on one GPU -- on different streams, or
 * from different threads -- race and must be serialized by the caller.
 * No counterpart in the reference; it exists for the callers above. */
int pq_w4a8_linear_noalloc(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                           const float* scales, const uint8_t* wpack, const uint32_t* wmeta, const void* bias,
                           int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n, int64_t k, int krot,
                           unsigned flags, void* stream);

/* One linear of a group that shares its input x (pq_w4a8_linear_group). */
typedef struct pq_linear_member {
  const uint32_t* rot_idx; /* this linear's rotation operands (pq_rotation_pack) */
  const float* rot_cs;
  const float* scales;     /* channel scales [k] or NULL */
  const uint8_t* wpack;    /* its weights (pq_w4a8_prepack) */
  const uint32_t* wmeta;
  const void* bias;        /* [n] in bias_dtype, or NULL */
  void* y;                 /* [m, n] in y_dtype */
  int64_t n;               /* output features, a positive multiple of 16 */
} pq_linear_member;

/* 1 when pq_w4a8_linear (and the group entry points) run m tokens of k
 * features through the split rotation (waves per 128-channel group, spread
 * over the chip): with a GEMM that quantizes A itself (m*k <= 8192,
 * or k >= 8192 and m <= 2), or for rows of 4096 channels or more (k a
 * multiple of 128 in [4096, 16384], up to 64 tokens) with a token-scale +
 * int8 kernel and the
 * GEMM on int8 A.  0 when they run the row rotate+quant kernel plus the
 * GEMM.  Callers use it to decide whether an elementwise step is cheaper
 * fused into the rotation launch (it is on the split path) or as a separate
 * kernel.  No counterpart in the reference. */
int pq_w4a8_linear_split_path(int64_t m, int64_t k);

/* Bytes of workspace pq_w4a8_linear_group needs for count members sharing an
 * [m, k] input: count times what pq_w4a8_linear needs for one (it does not
 * depend on n). */
size_t pq_w4a8_linear_group_workspace_size(int64_t m, int64_t k, int count);

/* count (1..4) W4A8 linears over the same input x [m, k] (x_dtype), each with
 * its own rotation and weights: member i writes its y [m, n_i].  Same results
 * as pq_w4a8_linear per member, in two launches for the whole group -- one
 * rotation (+ quant) launch and one GEMM over the concatenated columns.
 * All members share k, krot, flags, bias_dtype and y_dtype.  No counterpart
 * in the reference, whose ParoQuant loading runs q/k/v and gate/up as
 * separate linears (paroquant_marlin_w4a8.py:455-460); it replaces, for one
 * input, the calls BF16RotateLinearWrapper.forward makes per linear
 * (paroquant_marlin_w4a8.py:59-65). */
int pq_w4a8_linear_group(const void* x, int x_dtype, const pq_linear_member* members, int count, int bias_dtype,
                         int y_dtype, int64_t m, int64_t k, int krot, unsigned flags, void* workspace,
                         size_t workspace_bytes, void* stream);

/* pq_w4a8_linear_group behind a decoder layer's RMSNorm, in the same two
 * launches: the members read h instead of x, where
 *   s = x + residual (rounded to x's dtype; s = x when residual is NULL),
 *   h = round(w * round(s * rsqrt(mean(s^2) + eps))),
 * both roundings to x's dtype, mean and rsqrt in float32.  The float32 sum of
 * squares runs in one fixed order on every path, so a row's h does not depend
 * on m or on the other rows of the call.  norm_weight: [k] in x's dtype.  When set, h_out and sum_out ([m, k], x's dtype) receive h
 * and s (sum_out needs a residual).  residual must be 16-byte aligned.
 * Reference: Qwen3VLTextRMSNorm.forward (src/alpamayo_r1/models/qwen3_vl/
 * modeling_qwen3_vl.py:354-359) in front of the ParoQuant linears that read
 * its output (q/k/v after input_layernorm, gate/up after
 * post_attention_layernorm; paroquant_marlin_w4a8.py:59-65 per linear).
 * No counterpart of the fusion itself in the reference. */
int pq_w4a8_linear_group_rmsnorm(const void* x, const void* residual, const void* norm_weight, float eps,
                                 void* h_out, void* sum_out, int x_dtype, const pq_linear_member* members,
                                 int count, int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot,
                                 unsigned flags, void* workspace, size_t workspace_bytes, void* stream);

/* ---- W4A16 (fp16 activations, no activation quant) ---- */

/* Repack WQLinear weights for pq_w4a16_gemm: awq_qweight int32 [k, n/8] (the
 * codes in AWQ order, as unpack_wqlinear_qweight + pack_awq_int32 give them,
 * paroquant_marlin_w4a8.py:95-164), scales and scaled_zeros fp16 [k/128, n]
 * (the first k/128 rows of WQLinear's buffers).  wpack: the same layout as
 * pq_w4a8_prepack's; wmeta: uint32 [n/16, k/128, 16] = s | sz << 16.
 * Reference: the WQLinear buffers read by torch.ops.awq.gemv / gemm
 * (qmodule.py:113-147, 207-232). */
int pq_w4a16_prepack(const int32_t* awq_qweight, const uint16_t* scales, const uint16_t* scaled_zeros,
                     uint8_t* wpack, uint32_t* wmeta, int64_t k, int64_t n, int group_size, void* stream);

/* y[m, n] = sum_k x[m, k] * w[k, n] (+ bias[n]), written as y_dtype, with
 * w = fp16(q * s + sz) (one rounding) and float32 accumulation.  x: fp16
 * [m, k], 16-byte aligned; wpack/wmeta from pq_w4a16_prepack; bias: [n] of
 * bias_dtype or NULL.  group_size == 128, k % 128 == 0, n % 16 == 0.
 * Reference: WQLinear.forward (qmodule.py:207-232): torch.ops.awq.gemv for
 * fewer than 8 rows, torch.ops.awq.gemm otherwise, then + bias; weight
 * semantics of dequant_wqlinear (paroquant_marlin_w4a8.py:216-224). */
int pq_w4a16_gemm(const void* x, const uint8_t* wpack, const uint32_t* wmeta, const void* bias, int bias_dtype,
                  void* y, int y_dtype, int64_t m, int64_t n, int64_t k, int group_size, void* stream);

/* Bytes of scratch pq_w4a16_linear needs between its two kernels: the
 * rotated fp16 rows, 2*m*k rounded up to 256, plus, when m <= 16,
 * 4*m*(k/128) bytes of group maxima, the sum rounded up to 256.  Its content
 * does not matter. */
size_t pq_w4a16_linear_workspace_size(int64_t m, int64_t k);

/* y = pq_w4a16_gemm of the rotation of x, rounded to fp16: x [m, k]
 * (x_dtype f32/f16/bf16), rotation operands as for pq_w4a8_linear,
 * flags 0 or PQ_RQ_INPUT_FP16 (round x to fp16 first).  Two launches.
 * Reference: RotateLinearInt4.forward with a WQLinear qlinear
 * (rotation_linear.py:136-139): rotation::rotate (rotation.cu:456-493),
 * then WQLinear.forward (qmodule.py:207-232). */
int pq_w4a16_linear(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs, const float* scales,
                    const uint8_t* wpack, const uint32_t* wmeta, const void* bias, int bias_dtype, void* y,
                    int y_dtype, int64_t m, int64_t n, int64_t k, int krot, unsigned flags, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Bytes of workspace pq_w4a16_linear_group needs for count members sharing
 * an [m, k] input: count times what pq_w4a16_linear needs for one; 0 for a
 * count outside 1..4. */
size_t pq_w4a16_linear_group_workspace_size(int64_t m, int64_t k, int count);

/* pq_w4a16_linear for count (1..4) linears that read the same x (q/k/v,
 * gate/up): one rotation launch over all members and, for m <= 16, one GEMM
 * launch over their concatenated columns (for larger m, one GEMM launch per
 * member).  Each member's y is what pq_w4a16_linear gives for it.  Members
 * as for pq_w4a8_linear_group.  No counterpart in the reference (its
 * linears run one by one, rotation_linear.py:136-139 each). */
int pq_w4a16_linear_group(const void* x, int x_dtype, const pq_linear_member* members, int count,
                          int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot, unsigned flags,
                          void* workspace, size_t workspace_bytes, void* stream);

/* pq_w4a8_linear_group behind a decoder layer's elementwise step, chosen by
 * mode (PQ_PRO_*), in the same two launches; the members read
 *   PQ_PRO_RMSNORM: h = RMSNorm(x + x2) exactly as pq_w4a8_linear_group_rmsnorm
 *                   (x2 = residual, may be NULL; norm_weight, eps as there);
 *   PQ_PRO_ADD:     s = x + x2 (rounded to x's dtype; x2 required);
 *   PQ_PRO_SWIGLU:  h = round(round(silu(x)) * x2), silu(x) = x / (1 + exp(-x))
 *                   in float32 (x = gate, x2 = up, both [m, k]).
 * h_out ([m, k], x's dtype, RMSNORM / SWIGLU) and sum_out (s, RMSNORM with
 * x2 / ADD) are written when non-NULL; x2 16-byte aligned.  norm_weight and
 * eps are read for RMSNORM only.
 * Reference: the Qwen3-VL decoder layer around its linears
 * (src/alpamayo_r1/models/qwen3_vl/modeling_qwen3_vl.py:354-359 RMSNorm,
 * the residual adds of the layer, and the MLP's down_proj(act(gate) * up),
 * patches.py:541-548), each linear a BF16RotateLinearWrapper
 * (paroquant_marlin_w4a8.py:59-65).  No counterpart of the fusion itself in
 * the reference. */
int pq_w4a8_linear_group_fused(const void* x, const void* x2, const void* norm_weight, float eps, int mode,
                               void* h_out, void* sum_out, int x_dtype, const pq_linear_member* members, int count,
                               int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot, unsigned flags,
                               void* workspace, size_t workspace_bytes, void* stream);

/* pq_w4a8_linear_group (mode 0) or pq_w4a8_linear_group_fused (mode PQ_PRO_*)
 * in its two stages: stage 1 makes the rotation (+ quant) launches, whose
 * output stays in the workspace; stage 2 makes the GEMM launch from it.  The
 * two calls take the same arguments (stage 2 reads neither x nor the
 * prologue's, which may be NULL) and the same workspace, not touched in
 * between; in that order on one stream they make exactly the launches, and
 * give exactly the results, of the one-call form.  For callers that place
 * the stages apart (other work between them, separate graph nodes) and for
 * timing each kernel of the linear on its own.  No counterpart in the
 * reference, whose linear is one call (paroquant_marlin_w4a8.py:59-65). */
int pq_w4a8_linear_group_stage(int stage, const void* x, const void* x2, const void* norm_weight, float eps,
                               int mode, void* h_out, void* sum_out, int x_dtype, const pq_linear_member* members,
                               int count, int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot,
                               unsigned flags, void* workspace, size_t workspace_bytes, void* stream);

/* Parity form of pq_w4a8_linear_group (mode 0) and pq_w4a8_linear_group_fused
 * (mode PQ_PRO_*, prologue arguments as there): the same launches, chosen by
 * the same rules, up to the GEMM, whose kernel runs in its partials form
 * (same configuration, tiling and MFMA code; its epilogue replaced by stores
 * of the int32 accumulators).  Instead of y it returns, per member i:
 *   codes    int8  [count][m][k]   the int8 activation codes the GEMM multiplied
 *                                  (16-byte aligned);
 *   xscale   float [count][m]      the token scales its epilogue applies;
 *   partials int32 per-group partials sum_{k in g} (q[k, n] - z[g, n]) * codes[m, k],
 *            member i's [m][k/128][n_i] block at m*(k/128)*(n_0+...+n_{i-1}).
 * On the split pair path (one GEMM quantizing A in its prologue) codes and
 * xscale are the LDS image of A and the scales that kernel derived (written
 * by each member's first workgroup); on the other paths they are the codes
 * and scales the rotate+quant launches left in the workspace.  Members' bias
 * and y are not used.  A debugging / test entry point, not a fast path: it
 * exists so that the intermediates of every production path can be checked
 * against the reference semantics (per-token int8 quant and the Marlin
 * GEMM's int32 accumulators, paroquant_marlin_w4a8.py:319-333). */
int pq_w4a8_linear_group_intermediates(const void* x, const void* x2, const void* norm_weight, float eps, int mode,
                                       void* h_out, void* sum_out, int x_dtype, const pq_linear_member* members,
                                       int count, int64_t m, int64_t k, int krot, unsigned flags, void* workspace,
                                       size_t workspace_bytes, int8_t* codes, float* xscale, int32_t* partials,
                                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAROQUANT_HIP_H */
