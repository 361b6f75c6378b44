// Weight prefetch: reads byte ranges of device memory once -- one 4-byte load
// per 128-byte line -- so that a kernel launched later finds those lines in
// the GPU's caches (L2, and the 256 MB Infinity Cache in front of HBM).
//
// Decode-size linears are latency-bound launch chains: the rotation kernel of
// a linear moves almost no bytes, and the GEMM streams its weights at about
// half of HBM's bandwidth.  This kernel reads a linear's weights ahead of its
// GEMM.  Measured at one token on the Qwen3-8B layer: the GEMM then runs
// 0.4-1.4 us faster, but the reads take about 6 us per linear, so the linear
// path does not use it; it stays as a measurement option.  No counterpart in
// the reference.
#include "pq_common.h"

namespace {

constexpr int kPrefetchMaxRanges = 16;
constexpr int kPrefetchThreads = 256;
constexpr int kLine = 128;

struct PrefetchRanges {
  const uint8_t* ptr[kPrefetchMaxRanges];
  uint64_t lines[kPrefetchMaxRanges];
  int count;
};

// grid.y = range.  Each thread touches lines tid, tid + stride, ... of its
// range, four loads in flight at a time; the loaded words are folded into a
// value stored only when `keep` is set (the host never sets it: the store
// exists so the loads cannot be dropped).
__global__ __launch_bounds__(kPrefetchThreads) void prefetch_kernel(const PrefetchRanges r, uint32_t* sink, int keep) {
  const int ri = blockIdx.y;
  const uint8_t* base = r.ptr[ri];
  const uint64_t n = r.lines[ri];
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kPrefetchThreads;
  uint32_t acc = 0;
  uint64_t l = static_cast<uint64_t>(blockIdx.x) * kPrefetchThreads + threadIdx.x;
  for (; l + 3 * stride < n; l += 4 * stride) {
    const uint32_t a = *reinterpret_cast<const uint32_t*>(base + l * kLine);
    const uint32_t b = *reinterpret_cast<const uint32_t*>(base + (l + stride) * kLine);
    const uint32_t c = *reinterpret_cast<const uint32_t*>(base + (l + 2 * stride) * kLine);
    const uint32_t d = *reinterpret_cast<const uint32_t*>(base + (l + 3 * stride) * kLine);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; l < n; l += stride) acc ^= *reinterpret_cast<const uint32_t*>(base + l * kLine);
  if (keep) sink[blockIdx.y * kPrefetchThreads + threadIdx.x] = acc;
}

}  // namespace

extern "C" int pq_prefetch(const void* const* ptrs, const size_t* bytes, int count, int blocks, void* stream) {
  const char* who = "pq_prefetch";
  PQ_REQUIRE(count >= 0 && count <= kPrefetchMaxRanges, PQ_ERR_ARG, "%s: count=%d not in 0..%d", who, count,
             kPrefetchMaxRanges);
  PQ_REQUIRE(blocks >= 0 && blocks <= 65535, PQ_ERR_ARG, "%s: blocks=%d not in 0..65535", who, blocks);
  PQ_REQUIRE(count == 0 || (ptrs != nullptr && bytes != nullptr), PQ_ERR_ARG, "%s: null range table", who);
  PrefetchRanges r{};
  int used = 0;
  for (int i = 0; i < count; ++i) {
    if (bytes[i] == 0) continue;
    PQ_REQUIRE(ptrs[i] != nullptr && pq::aligned_to(ptrs[i], 4) && bytes[i] % 4 == 0, PQ_ERR_ARG,
               "%s: range %d must be non-null, 4-byte aligned and a whole number of 4-byte words", who, i);
    r.ptr[used] = static_cast<const uint8_t*>(ptrs[i]);
    // lines whose first word lies inside the range: every load stays in bounds
    r.lines[used] = (bytes[i] - 4) / kLine + 1;
    ++used;
  }
  r.count = used;
  if (used == 0) return PQ_OK;
  const unsigned gx = blocks > 0 ? static_cast<unsigned>(blocks) : 64u;
  prefetch_kernel<<<dim3(gx, static_cast<unsigned>(used)), kPrefetchThreads, 0, static_cast<hipStream_t>(stream)>>>(
      r, nullptr, 0);
  return pq::launch_status("pq_prefetch launch");
}
