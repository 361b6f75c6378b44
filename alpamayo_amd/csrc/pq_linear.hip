// The whole W4A8 linear (rotation + channel scale + per-token int8 quant +
// int4 x int8 GEMM) behind one entry point, pq_w4a8_linear.  Two kernels
// either way, chosen by the number of tokens m:
//
//   split (decode: m * k <= 12288, e.g. one token): the rotation runs with
//     one wave per 128-channel group (K/128 waves spread over the chip, each
//     rotation parameter read once) and writes the rotated rows plus each
//     row's absmax per group; the decode GEMM derives the token scales and
//     quantizes A into LDS in its prologue, while its first weight blocks
//     are already in flight.
//   rows (otherwise): pq_rotate_quant_i8 (rotation + absmax + int8 quant of
//     whole rows per workgroup) into the caller's workspace, then
//     pq_w4a8_gemm.
//
// A one-kernel variant (every workgroup rotating the token itself) was
// measured slower: the K/128 x 5 KB of rotation parameters, re-read by each
// of ~256 workgroups, saturate the per-CU load path ahead of the weights.
//
// Reference: BF16RotateLinearWrapper -> RotateLinearInt4 -> rotation::rotate
// -> MarlinW4A8Linear (src/alpamayo_r1/utils/quantization/
// paroquant_marlin_w4a8.py:59-65, 314-333; rotation_linear.py:120-124).
#include "pq_device.h"
#include "pq_internal.h"

namespace {

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Measured on the Qwen3-8B shapes: the split path wins while each GEMM
// workgroup can request all of A in its prologue at once (m * k <= 12288);
// beyond that the row kernel's whole-row quantization is faster.
bool use_split(int64_t m, int64_t k) { return m * k <= 12288 && pq::gemm_rotated_supported(m, k); }

size_t split_xr_bytes(int64_t m, int64_t k) { return align_up(static_cast<size_t>(m) * k * sizeof(float), 256); }

}  // namespace

extern "C" size_t pq_w4a8_linear_workspace_size(int64_t m, int64_t n, int64_t k, int krot) {
  (void)krot;
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 || n % 16) return 0;
  if (use_split(m, k)) return split_xr_bytes(m, k) + static_cast<size_t>(m) * (k / 128) * sizeof(float);
  return align_up(static_cast<size_t>(m) * k, 256) + static_cast<size_t>(m) * sizeof(float);
}

extern "C" int pq_w4a8_linear(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                              const float* scales, const uint8_t* wpack, const uint32_t* wmeta, const void* bias,
                              int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n, int64_t k, int krot,
                              unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  PQ_REQUIRE(m >= 0 && m <= 0x7fffffffLL, PQ_ERR_ARG, "pq_w4a8_linear: m=%lld", (long long)m);
  PQ_REQUIRE(n > 0 && n % 16 == 0 && n <= (1 << 20), PQ_ERR_ARG, "pq_w4a8_linear: n=%lld must be a positive multiple of 16",
             (long long)n);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= 16384, PQ_ERR_ARG,
             "pq_w4a8_linear: k=%lld must be a positive multiple of 128, at most 16384", (long long)k);
  PQ_REQUIRE(krot >= 1 && krot <= 16, PQ_ERR_UNSUPPORTED, "pq_w4a8_linear: krot=%d not in 1..16", krot);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_w4a8_linear: x dtype code %d", x_dtype);
  PQ_REQUIRE(y_dtype == PQ_F32 || y_dtype == PQ_F16 || y_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_w4a8_linear: y dtype code %d", y_dtype);
  PQ_REQUIRE(bias == nullptr || bias_dtype == PQ_F32 || bias_dtype == PQ_F16 || bias_dtype == PQ_BF16,
             PQ_ERR_UNSUPPORTED, "pq_w4a8_linear: bias dtype code %d", bias_dtype);
  PQ_REQUIRE((flags & ~(PQ_RQ_INPUT_FP16 | PQ_RQ_MATERIALIZE_FP16)) == 0, PQ_ERR_ARG,
             "pq_w4a8_linear: unknown flags 0x%x", flags);
  if (m == 0) return PQ_OK;
  PQ_REQUIRE(x && rot_idx && rot_cs && wpack && wmeta && y, PQ_ERR_ARG, "pq_w4a8_linear: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(rot_idx, 16) && pq::aligned_to(rot_cs, 16) && pq::aligned_to(wpack, 16) &&
                 pq::aligned_to(wmeta, 4) && pq::aligned_to(y, pq::dtype_size(y_dtype)),
             PQ_ERR_ARG, "pq_w4a8_linear: misaligned pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool split = use_split(m, k);
  const size_t need = pq_w4a8_linear_workspace_size(m, n, k, krot);
  PQ_REQUIRE(workspace != nullptr && workspace_bytes >= need && pq::aligned_to(workspace, 256), PQ_ERR_WORKSPACE,
             "pq_w4a8_linear: a 256-byte aligned workspace of %zu bytes is needed for m=%lld k=%lld, got %zu", need,
             (long long)m, (long long)k, workspace ? workspace_bytes : (size_t)0);
  if (split) {
    const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
    void* xr = workspace;
    float* gmax = reinterpret_cast<float*>(static_cast<char*>(workspace) + split_xr_bytes(m, k));
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
    pq::launch_rotate_split(x, x_dtype, rot_idx, rot_cs, scales, xr, gmax, M, K, krot, flags, s);
    int st = pq::launch_status("pq_w4a8_linear rotation launch");
    if (st != PQ_OK) return st;
    pq::launch_gemm_rotated(xr, mat16, gmax, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, s);
    return pq::launch_status("pq_w4a8_linear GEMM launch");
  }
  int8_t* xq = static_cast<int8_t*>(workspace);
  float* xs = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(static_cast<size_t>(m) * k, 256));
  int st = pq_rotate_quant_i8(x, x_dtype, rot_idx, rot_cs, scales, xq, xs, nullptr, m, k, krot, flags, stream);
  if (st != PQ_OK) return st;
  return pq_w4a8_gemm(xq, xs, wpack, wmeta, bias, bias_dtype, y, y_dtype, m, n, k, 128, nullptr, 0, stream);
}
