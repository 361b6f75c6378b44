// Load-time repack of AWQ int4 buffers into the GEMM kernels' layout.
//
// Replaces MarlinW4A8Linear.load_from_awq's vLLM repack
// (src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:274-312).
// Input: AWQ qweight int32 [K][N/8] and qzeros int32 [G][N/8] whose nibble i
// holds column 8c + (0,2,4,6,1,3,5,7)[i] (paroquant_marlin_w4a8.py:149-164),
// scales fp16 [G][N].  Output layout: see pq_gemm.hip.
#include "pq_common.h"

namespace {

// Nibble position of column offset o inside an AWQ word.
__device__ __forceinline__ int awq_nibble(int o) { return (o >> 1) + 4 * (o & 1); }

// W16 = false: metadata s | z << 16 (z from the AWQ qzeros, the W4A8 GEMM);
// W16 = true: s | sz << 16 (sz the fp16 scaled zero [G][N], the W4A16 GEMM).
template <bool W16>
__global__ __launch_bounds__(256) void prepack_kernel(const int32_t* __restrict__ qw, const uint16_t* __restrict__ sc,
                                                      const int32_t* __restrict__ qz, const uint16_t* __restrict__ sz,
                                                      uint32_t* __restrict__ wpack, uint32_t* __restrict__ wmeta,
                                                      int K, int N) {
  const int G = K >> 7;
  const int nw = N >> 3;
  const int64_t total = static_cast<int64_t>(N) * K / 8;   // output dwords
  const int64_t nmeta = static_cast<int64_t>(N) * G;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int d = static_cast<int>(idx & 3);
    const int slot = static_cast<int>((idx >> 2) & 63);
    const int64_t tg = idx >> 8;           // tile * G + g
    const int g = static_cast<int>(tg % G);
    const int tile = static_cast<int>(tg / G);
    const int j = slot >> 4;
    const int c = slot & 15;
    const int n = tile * 16 + c;
    const int kb = g * 128 + j * 32 + d * 8;
    const int shift = 4 * awq_nibble(n & 7);
    const int64_t col = n >> 3;
    uint32_t out = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (static_cast<uint32_t>(qw[static_cast<int64_t>(kb + i) * nw + col]) >> shift) & 0xfu;
      const uint32_t hi = (static_cast<uint32_t>(qw[static_cast<int64_t>(kb + 4 + i) * nw + col]) >> shift) & 0xfu;
      out |= (lo | (hi << 4)) << (8 * i);
    }
    wpack[idx] = out;
    if (idx < nmeta) {
      // meta index = (tile * G + g) * 16 + c
      const int mc = static_cast<int>(idx & 15);
      const int64_t mtg = idx >> 4;
      const int mg = static_cast<int>(mtg % G);
      const int mtile = static_cast<int>(mtg / G);
      const int mn = mtile * 16 + mc;
      const uint32_t s = sc[static_cast<int64_t>(mg) * N + mn];
      if constexpr (W16) {
        wmeta[idx] = s | (static_cast<uint32_t>(sz[static_cast<int64_t>(mg) * N + mn]) << 16);
      } else {
        const uint32_t z =
            (static_cast<uint32_t>(qz[static_cast<int64_t>(mg) * nw + (mn >> 3)]) >> (4 * awq_nibble(mn & 7))) & 0xfu;
        wmeta[idx] = s | (z << 16);
      }
    }
  }
}

}  // namespace

extern "C" int pq_w4a8_prepack(const int32_t* awq_qweight, const uint16_t* awq_scales, const int32_t* awq_qzeros,
                               uint8_t* wpack, uint32_t* wmeta, int64_t k, int64_t n, int group_size, void* stream) {
  PQ_REQUIRE(group_size == 128, PQ_ERR_UNSUPPORTED, "pq_w4a8_prepack: group_size=%d (only 128)", group_size);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= (1 << 20), PQ_ERR_ARG, "pq_w4a8_prepack: k=%lld", (long long)k);
  PQ_REQUIRE(n > 0 && n % 16 == 0 && n <= (1 << 20), PQ_ERR_ARG, "pq_w4a8_prepack: n=%lld", (long long)n);
  PQ_REQUIRE(awq_qweight && awq_scales && awq_qzeros && wpack && wmeta, PQ_ERR_ARG, "pq_w4a8_prepack: null pointer");
  PQ_REQUIRE(pq::aligned_to(wpack, 4) && pq::aligned_to(awq_qweight, 4) && pq::aligned_to(awq_qzeros, 4),
             PQ_ERR_ARG, "pq_w4a8_prepack: misaligned pointer");
  const int64_t total = n * k / 8;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  prepack_kernel<false><<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
      awq_qweight, awq_scales, awq_qzeros, nullptr, reinterpret_cast<uint32_t*>(wpack), wmeta, static_cast<int>(k),
      static_cast<int>(n));
  return pq::launch_status("pq_w4a8_prepack launch");
}

// The W4A16 GEMM's weights: the same packed codes, metadata s | sz << 16.
// Replaces the preparation WQLinear's buffers need before the reference's
// torch.ops.awq.gemv / gemm (src/alpamayo_r1/utils/quantization/
// qmodule.py:207-232): the codes arrive as AWQ int32 (unpack_wqlinear_qweight
// + pack_awq_int32), scales and scaled_zeros as fp16 [G][N].
extern "C" int pq_w4a16_prepack(const int32_t* awq_qweight, const uint16_t* scales, const uint16_t* scaled_zeros,
                                uint8_t* wpack, uint32_t* wmeta, int64_t k, int64_t n, int group_size, void* stream) {
  PQ_REQUIRE(group_size == 128, PQ_ERR_UNSUPPORTED, "pq_w4a16_prepack: group_size=%d (only 128)", group_size);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= (1 << 20), PQ_ERR_ARG, "pq_w4a16_prepack: k=%lld", (long long)k);
  PQ_REQUIRE(n > 0 && n % 16 == 0 && n <= (1 << 20), PQ_ERR_ARG, "pq_w4a16_prepack: n=%lld", (long long)n);
  PQ_REQUIRE(awq_qweight && scales && scaled_zeros && wpack && wmeta, PQ_ERR_ARG, "pq_w4a16_prepack: null pointer");
  PQ_REQUIRE(pq::aligned_to(wpack, 4) && pq::aligned_to(awq_qweight, 4) && pq::aligned_to(wmeta, 4) &&
                 pq::aligned_to(scales, 2) && pq::aligned_to(scaled_zeros, 2),
             PQ_ERR_ARG, "pq_w4a16_prepack: misaligned pointer");
  const int64_t total = n * k / 8;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  prepack_kernel<true><<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
      awq_qweight, scales, nullptr, scaled_zeros, reinterpret_cast<uint32_t*>(wpack), wmeta, static_cast<int>(k),
      static_cast<int>(n));
  return pq::launch_status("pq_w4a16_prepack launch");
}
