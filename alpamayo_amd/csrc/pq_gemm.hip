// Stage 3 of the W4A8 linear on gfx950: int4-weight x int8-activation GEMM
// with per-(128-group, column) fp16 scales and uint4 zero points, int32
// accumulation per group on the int8 MFMA units and an fp32 epilogue:
//
//   P[m, g, n] = sum_{k in g} (q[k, n] - z[g, n]) * xq[m, k]        (int32)
//   y[m, n]    = xscale[m] * sum_g s[g, n] * P[m, g, n] (+ bias[n])
//
// Reference: the Marlin W4A8 GEMM reached through apply_awq_marlin_linear
// (src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:314-333) with
// AWQ weight semantics (dequant_awq, 227-235).
//
// Weights use the layout written by pq_w4a8_prepack (pq_prepack.hip):
//   wpack [N/16][G][64 slots][16 B]: slot 16j + c = column 16*tile + c,
//     codes k = 128g + 32j + [0, 32); each dword holds 8 consecutive k,
//     low nibbles the first four, high nibbles the next four;
//   wmeta [N/16][G][16] uint32: fp16 scale bits | zero << 16.
//
// Unpacking: a dword of 8 codes becomes two dwords of 4 signed bytes
// (q - z) by  ((w & 0x0f0f0f0f) + (0x80808080 - z*0x01010101)) ^ 0x80808080
// -- every byte stays in [113, 143] before the xor, so no carry crosses a
// byte, and the xor maps 128 + d to the two's complement of d.
//
// Two kernels:
//   gemm_skinny  M <= 16: each wave streams 1 KB weight blocks (one 16-column
//                tile x one 128-group) with 16-byte loads, two
//                v_mfma_i32_16x16x64_i8 per block (activation rows padded to
//                16); the waves of a workgroup split K and add their partial
//                sums in LDS in a fixed order.
//   gemm_tiled   M > 16: 128x128 output tiles, A (int8) and B (int4) staged
//                through LDS one group at a time with the next group
//                prefetched into registers, 2x2 waves of 64x64, each
//                2x2 v_mfma_i32_32x32x32_i8 tiles per 32-deep K step.
#include "pq_device.h"
#include "pq_internal.h"

using namespace pqd;

namespace {

// ---------------------------------------------------------------------------
// Decode-size GEMM (M <= 16)
//
// Workgroup = W waves over NT 16-column tiles; wave w takes the groups
// w, w+W, w+2W, ... of K and issues the 16-byte loads of U groups at once.
// The W partial sums meet in LDS and are added in a fixed order, so no
// workgroup ever communicates with another (no split-K workspace, no
// device-scope fence).
// ---------------------------------------------------------------------------
//
// AQ selects where A comes from: 0 = int8 codes and token scales in global
// memory; 1 / 2 = rotated fp16 / fp32 rows plus per-group absmax (the split
// rotation's output): the workgroup derives each row's token scale, writes
// the int8 codes of all M rows into LDS (row stride K + 16 bytes, so the 16
// rows of an A fragment hit distinct banks) and reads A from there.  The
// first batch of weight loads is issued before that prologue.
constexpr int kSkinnyRows = 16;

template <int NT, int W, int U, bool PARTIALS, int AQ>
__global__ __launch_bounds__(W * 64, (W == 4 && NT == 1 && !PARTIALS) ? 3 : 1) void gemm_skinny(
    const int8_t* __restrict__ xq, const float* __restrict__ xs, const void* __restrict__ xr,
    const float* __restrict__ gmax, const uint8_t* __restrict__ wpack, const uint32_t* __restrict__ wmeta,
    const void* __restrict__ bias, int bias_dtype, void* __restrict__ y, int y_dtype, int32_t* __restrict__ partials,
    int M, int N, int K) {
  __shared__ float red[W][NT][4][64];
  __shared__ float s_amax[kSkinnyRows];
  extern __shared__ __attribute__((aligned(16))) int8_t aq[];
  const int G = K >> 7;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int j = lane >> 4;
  const bool arow = c < M;
  const int astride = K + 16;
  const int tile0 = blockIdx.x * NT;

  float acc[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[nt][v] = 0.0f;

  const int8_t* ap = xq + static_cast<int64_t>(arow ? c : 0) * K + j * 32;
  const int8_t* al = aq + (arow ? c : 0) * astride + j * 32;
  const int nthr = W * 64;
  const int k8 = K >> 3;

  // AQ prologue, part 1: request the per-group maxima and (when they fit in
  // kPre 8-element chunks per thread) the rotated rows before any weight
  // block, so that waiting for them does not mean waiting for the weights
  // (a wave's loads complete in issue order).
  constexpr int kPreMax = 2048 / (W * 64);    // gmax values per thread (covers M * G <= 2048)
  constexpr int kPre = W >= 8 ? 2 : 4;        // 8-element chunks of A per thread
  float gm[kPreMax];
  uint4 pre[kPre][AQ == 2 ? 2 : 1];
  bool preloaded = false;
  if constexpr (AQ != 0) {
#pragma unroll
    for (int q = 0; q < kPreMax; ++q) {
      const int i = threadIdx.x + q * nthr;
      gm[q] = i < M * G ? gmax[i] : 0.0f;
    }
    preloaded = M * k8 <= kPre * nthr;
    if (preloaded) {
#pragma unroll
      for (int q = 0; q < kPre; ++q) {
        const int e = threadIdx.x + q * nthr;
        if (e < M * k8) {
          const int r = e / k8;
          const int c8 = (e - r * k8) * 8;
          if constexpr (AQ == 1) {
            pre[q][0] =
                *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xr) + static_cast<int64_t>(r) * K + c8);
          } else {
            const uint4* src =
                reinterpret_cast<const uint4*>(static_cast<const float*>(xr) + static_cast<int64_t>(r) * K + c8);
            pre[q][0] = src[0];
            pre[q][AQ == 2 ? 1 : 0] = src[1];
          }
        }
      }
    }
  }

  // Every wave runs the same number of batches (a batch past G loads
  // nothing), so the prologue's barriers are reached by all waves.
  const int batches = (G + W * U - 1) / (W * U);
  // One batch of U groups per wave; batch 0 (which holds the prologue) is
  // peeled off the loop, so the common single-batch case has no back edge
  // (the compiler otherwise waits for earlier loads before reusing registers).
  auto run_batch = [&](const int it) {
    const int g0 = wave + it * W * U;
    v4i wb[U][NT];
    uint32_t wm[U][NT];
    v4i a0[U], a1[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g0 + W * u;
      if (g < G) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int64_t blk = static_cast<int64_t>(tile0 + nt) * G + g;
          wb[u][nt] = *reinterpret_cast<const v4i*>(wpack + blk * 1024 + lane * 16);
          wm[u][nt] = wmeta[blk * 16 + c];
        }
        if constexpr (AQ == 0) {
          // Unconditional (rows >= M read row 0 and are zeroed at use): a
          // branch around the loads would make the compiler wait early.
          a0[u] = *reinterpret_cast<const v4i*>(ap + static_cast<int64_t>(g) * 128);
          a1[u] = *reinterpret_cast<const v4i*>(ap + static_cast<int64_t>(g) * 128 + 16);
        }
      }
    }
    if constexpr (AQ != 0) {
      if (it == 0) {
        // Part 2: token scales, then the int8 image of A in LDS.
        if (threadIdx.x < kSkinnyRows) s_amax[threadIdx.x] = 0.0f;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPreMax; ++q) {   // absmax >= 0: unsigned order is float order
          const int i = threadIdx.x + q * nthr;
          if (i < M * G) atomicMax(reinterpret_cast<unsigned*>(&s_amax[i / G]), __float_as_uint(gm[q]));
        }
        for (int i = threadIdx.x + kPreMax * nthr; i < M * G; i += nthr)
          atomicMax(reinterpret_cast<unsigned*>(&s_amax[i / G]), __float_as_uint(gmax[i]));
        __syncthreads();
        auto quant8 = [&](int e, const uint4* v) {
          const int r = e / k8;
          const int c8 = (e - r * k8) * 8;
          float f[8];
          if constexpr (AQ == 1) {
            const uint32_t wds[4] = {v[0].x, v[0].y, v[0].z, v[0].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              f[2 * q] = pq_f16_to_f32(static_cast<uint16_t>(wds[q] & 0xffffu));
              f[2 * q + 1] = pq_f16_to_f32(static_cast<uint16_t>(wds[q] >> 16));
            }
          } else {
            f[0] = __uint_as_float(v[0].x); f[1] = __uint_as_float(v[0].y);
            f[2] = __uint_as_float(v[0].z); f[3] = __uint_as_float(v[0].w);
            f[4] = __uint_as_float(v[AQ == 2 ? 1 : 0].x); f[5] = __uint_as_float(v[AQ == 2 ? 1 : 0].y);
            f[6] = __uint_as_float(v[AQ == 2 ? 1 : 0].z); f[7] = __uint_as_float(v[AQ == 2 ? 1 : 0].w);
          }
          const float inv = inv_scale(s_amax[r]);
          uint2 o;
          o.x = quant4(f[0], f[1], f[2], f[3], inv);
          o.y = quant4(f[4], f[5], f[6], f[7], inv);
          *reinterpret_cast<uint2*>(aq + r * astride + c8) = o;
        };
        if (preloaded) {
#pragma unroll
          for (int q = 0; q < kPre; ++q) {
            const int e = threadIdx.x + q * nthr;
            if (e < M * k8) quant8(e, pre[q]);
          }
        } else {
          for (int e = threadIdx.x; e < M * k8; e += nthr) {
            const int r = e / k8;
            const int c8 = (e - r * k8) * 8;
            uint4 v[2];
            if constexpr (AQ == 1) {
              v[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xr) + static_cast<int64_t>(r) * K + c8);
            } else {
              const uint4* src =
                  reinterpret_cast<const uint4*>(static_cast<const float*>(xr) + static_cast<int64_t>(r) * K + c8);
              v[0] = src[0];
              v[1] = src[1];
            }
            quant8(e, v);
          }
        }
        __syncthreads();
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g0 + W * u;
      if (g < G) {
        if constexpr (AQ != 0) {   // A from the LDS image, next to its use
          a0[u] = *reinterpret_cast<const v4i*>(al + g * 128);
          a1[u] = *reinterpret_cast<const v4i*>(al + g * 128 + 16);
        }
        const v4i zero = {0, 0, 0, 0};
        const v4i av0 = arow ? a0[u] : zero, av1 = arow ? a1[u] : zero;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t meta = wm[u][nt];
          const uint32_t zb = meta_zero_bias(meta);
          const v4i w = wb[u][nt];
          const v4i b0 = unpack16(static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y), zb);
          const v4i b1 = unpack16(static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w), zb);
          v4i p = {0, 0, 0, 0};
          p = __builtin_amdgcn_mfma_i32_16x16x64_i8(av0, b0, p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_i32_16x16x64_i8(av1, b1, p, 0, 0, 0);
          if constexpr (PARTIALS) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int m = 4 * j + v;
              if (m < M) partials[(static_cast<int64_t>(m) * G + g) * N + (tile0 + nt) * 16 + c] = p[v];
            }
          } else {
            const float sc = meta_scale(meta);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[nt][v] = fmaf(static_cast<float>(p[v]), sc, acc[nt][v]);
          }
        }
      }
    }
  };
  run_batch(0);
  for (int it = 1; it < batches; ++it) run_batch(it);
  if constexpr (PARTIALS) return;

#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][nt][v][lane] = acc[nt][v];
  __syncthreads();
  for (int t = threadIdx.x; t < NT * 256; t += W * 64) {
    const int nt = t >> 8;
    const int rv = (t >> 6) & 3;
    const int rl = t & 63;
    const int m = 4 * (rl >> 4) + rv;
    if (m >= M) continue;
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) sum += red[w][nt][rv][rl];
    const int n = (tile0 + nt) * 16 + (rl & 15);
    const float xsm = AQ != 0 ? s_amax[m] / 127.0f : xs[m];
    pq_store_dyn(y, y_dtype, static_cast<int64_t>(m) * N + n, epilogue(sum, xsm, bias, bias_dtype, n));
  }
}

// ---------------------------------------------------------------------------
// Prefill-size GEMM (M > 16)
// ---------------------------------------------------------------------------
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kAPad = 144;  // LDS row stride of the A tile (bytes)

template <bool PARTIALS>
__global__ __launch_bounds__(256) void gemm_tiled(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                  const uint8_t* __restrict__ wpack,
                                                  const uint32_t* __restrict__ wmeta, const void* __restrict__ bias,
                                                  int bias_dtype, void* __restrict__ y, int y_dtype,
                                                  int32_t* __restrict__ partials, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) int8_t As[kBM * kAPad];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[8 * 1024];
  __shared__ uint32_t Ms[8 * 16];

  const int G = K >> 7;
  const int ntiles16 = N >> 4;
  const int nbn = (N + kBN - 1) / kBN;
  const int bm = blockIdx.x / nbn;
  const int bn = blockIdx.x % nbn;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int r32 = lane & 31;
  const int hj = lane >> 5;

  // Global -> register mapping of one group's tiles.
  const int a_row = t >> 1;
  const int a_half = t & 1;
  const int64_t a_grow = static_cast<int64_t>(bm) * kBM + a_row;
  const bool a_ok = a_grow < M;
  const int8_t* a_src = xq + (a_ok ? a_grow : 0) * K + a_half * 64;
  const int b_tile = t >> 5;
  const int b_off = (t & 31) * 32;
  const int b_gtile = bn * 8 + b_tile;
  const bool b_ok = b_gtile < ntiles16;
  const uint8_t* b_src = wpack + static_cast<int64_t>(b_ok ? b_gtile : 0) * G * 1024 + b_off;
  const int m_gtile = bn * 8 + (t >> 4);
  const bool m_ok = t < 128 && m_gtile < ntiles16;
  const uint32_t* m_src = wmeta + static_cast<int64_t>(m_ok ? m_gtile : 0) * G * 16 + (t & 15);

  v4i ra[4];
  v4i rb[2];
  uint32_t rm = 0;
  auto gload = [&](int g) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      ra[q] = a_ok ? *reinterpret_cast<const v4i*>(a_src + static_cast<int64_t>(g) * 128 + q * 16) : v4i{0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < 2; ++q)
      rb[q] = b_ok ? *reinterpret_cast<const v4i*>(b_src + static_cast<int64_t>(g) * 1024 + q * 16) : v4i{0, 0, 0, 0};
    rm = m_ok ? m_src[static_cast<int64_t>(g) * 16] : 0u;
  };

  float acc[2][2][16];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;

  int bt[2], bc[2];
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    const int nl = wn * 64 + ni * 32 + r32;
    bt[ni] = nl >> 4;
    bc[ni] = nl & 15;
  }

  gload(0);
  for (int g = 0; g < G; ++g) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<v4i*>(As + a_row * kAPad + a_half * 64 + q * 16) = ra[q];
#pragma unroll
    for (int q = 0; q < 2; ++q) *reinterpret_cast<v4i*>(Bs + b_tile * 1024 + b_off + q * 16) = rb[q];
    if (t < 128) Ms[t] = rm;
    __syncthreads();
    if (g + 1 < G) gload(g + 1);

    uint32_t zb[2];
    float sc[2];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const uint32_t meta = Ms[bt[ni] * 16 + bc[ni]];
      zb[ni] = zero_bias((meta >> 16) & 0xfu);
      sc[ni] = pq_f16_to_f32(static_cast<uint16_t>(meta & 0xffffu));
    }
    v16i T[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) T[mi][ni] = v16i{};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v4i a[2], b[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        a[mi] = *reinterpret_cast<const v4i*>(As + (wm * 64 + mi * 32 + r32) * kAPad + hj * 64 + i * 16);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const uint2 w =
            *reinterpret_cast<const uint2*>(Bs + bt[ni] * 1024 + ((2 * hj + (i >> 1)) * 16 + bc[ni]) * 16 + (i & 1) * 8);
        b[ni] = unpack16(w.x, w.y, zb[ni]);
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          T[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mi], b[ni], T[mi][ni], 0, 0, 0);
    }
    if constexpr (PARTIALS) {
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t m = static_cast<int64_t>(bm) * kBM + wm * 64 + mi * 32 + 8 * (v >> 2) + 4 * hj + (v & 3);
            const int n = bn * kBN + wn * 64 + ni * 32 + r32;
            if (m < M && n < N) partials[(m * G + g) * N + n] = T[mi][ni][v];
          }
    } else {
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            acc[mi][ni][v] = fmaf(static_cast<float>(T[mi][ni][v]), sc[ni], acc[mi][ni][v]);
    }
  }
  if constexpr (PARTIALS) return;

#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = static_cast<int64_t>(bm) * kBM + wm * 64 + mi * 32 + 8 * (v >> 2) + 4 * hj + (v & 3);
      if (m >= M) continue;
      const float xsm = xs[m];
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int n = bn * kBN + wn * 64 + ni * 32 + r32;
        if (n < N) pq_store_dyn(y, y_dtype, m * N + n, epilogue(acc[mi][ni][v], xsm, bias, bias_dtype, n));
      }
    }
}

// ---------------------------------------------------------------------------
// Host-side configuration
// ---------------------------------------------------------------------------
constexpr int kSkinnyMaxM = 16;

struct SkinnyCfg {
  int nt;  // 16-column tiles per workgroup
  int w;   // waves per workgroup (split K)
};

// Enough workgroups to cover the chip with every weight byte of a wave
// requested up front (<= 8 groups per wave), and more waves per workgroup
// when the column tiles are few.
SkinnyCfg choose_skinny(int64_t m, int64_t n, int64_t k) {
  const int G = static_cast<int>(k / 128);
  const int tiles = static_cast<int>(n / 16);
  const int nt = (m > 4 && tiles % 2 == 0 && tiles / 2 >= 128) ? 2 : 1;
  const int wgs = tiles / nt;
  int w = 4;
  if (wgs < 256 || G > 32) w = 8;
  if (wgs < 128 || G > 64) w = 16;
  return {nt, w};
}

template <int NT, int W, bool PARTIALS, int AQ>
void launch_skinny_nw(const int8_t* xq, const float* xs, const void* xr, const float* gmax, const uint8_t* wpack,
                      const uint32_t* wmeta, const void* bias, int bias_dtype, void* y, int y_dtype,
                      int32_t* partials, int M, int N, int K, hipStream_t stream) {
  constexpr int U = W >= 16 ? 4 : 8;
  const unsigned grid = static_cast<unsigned>((N / 16) / NT);
  const size_t lds = AQ != 0 ? static_cast<size_t>(M) * (K + 16) : 0;
  gemm_skinny<NT, W, U, PARTIALS, AQ><<<grid, W * 64, lds, stream>>>(xq, xs, xr, gmax, wpack, wmeta, bias, bias_dtype,
                                                                     y, y_dtype, partials, M, N, K);
}

template <bool PARTIALS, int AQ>
void launch_skinny(const SkinnyCfg& cfg, const int8_t* xq, const float* xs, const void* xr, const float* gmax,
                   const uint8_t* wpack, const uint32_t* wmeta, const void* bias, int bias_dtype, void* y, int y_dtype,
                   int32_t* partials, int M, int N, int K, hipStream_t stream) {
#define PQ_SKINNY(NT_, W_)                                                                                      \
  if (cfg.nt == NT_ && cfg.w == W_) {                                                                           \
    launch_skinny_nw<NT_, W_, PARTIALS, AQ>(xq, xs, xr, gmax, wpack, wmeta, bias, bias_dtype, y, y_dtype, partials, \
                                            M, N, K, stream);                                                   \
    return;                                                                                                     \
  }
  PQ_SKINNY(1, 4) PQ_SKINNY(1, 8) PQ_SKINNY(1, 16) PQ_SKINNY(2, 4) PQ_SKINNY(2, 8) PQ_SKINNY(2, 16)
#undef PQ_SKINNY
}

int check_gemm_args(const char* who, int64_t m, int64_t n, int64_t k, int group_size) {
  PQ_REQUIRE(group_size == 128, PQ_ERR_UNSUPPORTED, "%s: group_size=%d (only 128 is supported)", who, group_size);
  PQ_REQUIRE(m >= 0 && m <= 0x7fffffffLL, PQ_ERR_ARG, "%s: m=%lld", who, (long long)m);
  PQ_REQUIRE(n > 0 && n % 16 == 0 && n <= (1 << 20), PQ_ERR_ARG, "%s: n=%lld must be a positive multiple of 16", who,
             (long long)n);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= (1 << 20), PQ_ERR_ARG, "%s: k=%lld must be a positive multiple of 128",
             who, (long long)k);
  return PQ_OK;
}

}  // namespace

namespace pq {
bool gemm_rotated_supported(int64_t m, int64_t k) {
  return m >= 1 && m <= kSkinnyRows && k % 128 == 0 && k <= 16384 && m * (k + 16) <= 80 * 1024;
}

void launch_gemm_rotated(const void* xr, bool xr_fp16, const float* gmax, const uint8_t* wpack, const uint32_t* wmeta,
                         const void* bias, int bias_dtype, void* y, int y_dtype, int m, int n, int k,
                         hipStream_t stream) {
  SkinnyCfg cfg = choose_skinny(m, n, k);
  if (cfg.w == 16) cfg.nt = 1;   // two tiles x 16 waves would spill next to the prologue
  if (xr_fp16)
    launch_skinny<false, 1>(cfg, nullptr, nullptr, xr, gmax, wpack, wmeta, bias, bias_dtype, y, y_dtype, nullptr, m,
                            n, k, stream);
  else
    launch_skinny<false, 2>(cfg, nullptr, nullptr, xr, gmax, wpack, wmeta, bias, bias_dtype, y, y_dtype, nullptr, m,
                            n, k, stream);
}
}  // namespace pq

extern "C" size_t pq_w4a8_workspace_size(int64_t m, int64_t n, int64_t k, int group_size) {
  // No kernel of this version exchanges data between workgroups.
  (void)m, (void)n, (void)k, (void)group_size;
  return 0;
}

extern "C" int pq_w4a8_gemm(const int8_t* xq, const float* xscale, const uint8_t* wpack, const uint32_t* wmeta,
                            const void* bias, int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n,
                            int64_t k, int group_size, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_gemm_args("pq_w4a8_gemm", m, n, k, group_size);
  if (st != PQ_OK) return st;
  PQ_REQUIRE(y_dtype == PQ_F32 || y_dtype == PQ_F16 || y_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_w4a8_gemm: y dtype code %d", y_dtype);
  PQ_REQUIRE(bias == nullptr || bias_dtype == PQ_F32 || bias_dtype == PQ_F16 || bias_dtype == PQ_BF16,
             PQ_ERR_UNSUPPORTED, "pq_w4a8_gemm: bias dtype code %d", bias_dtype);
  if (m == 0) return PQ_OK;
  PQ_REQUIRE(xq && xscale && wpack && wmeta && y, PQ_ERR_ARG, "pq_w4a8_gemm: null pointer");
  PQ_REQUIRE(pq::aligned_to(xq, 16) && pq::aligned_to(wpack, 16) && pq::aligned_to(wmeta, 4) &&
                 pq::aligned_to(y, pq::dtype_size(y_dtype)),
             PQ_ERR_ARG, "pq_w4a8_gemm: xq and wpack must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
  if (m <= kSkinnyMaxM) {
    (void)workspace, (void)workspace_bytes;
    launch_skinny<false, 0>(choose_skinny(m, n, k), xq, xscale, nullptr, nullptr, wpack, wmeta, bias, bias_dtype, y, y_dtype, nullptr, M,
                         N, K, s);
  } else {
    const unsigned grid = static_cast<unsigned>(((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN));
    gemm_tiled<false><<<grid, 256, 0, s>>>(xq, xscale, wpack, wmeta, bias, bias_dtype, y, y_dtype, nullptr, M, N, K);
  }
  return pq::launch_status("pq_w4a8_gemm launch");
}

extern "C" int pq_w4a8_gemm_partials(const int8_t* xq, const uint8_t* wpack, const uint32_t* wmeta,
                                     int32_t* partials, int64_t m, int64_t n, int64_t k, int group_size,
                                     void* stream) {
  int st = check_gemm_args("pq_w4a8_gemm_partials", m, n, k, group_size);
  if (st != PQ_OK) return st;
  if (m == 0) return PQ_OK;
  PQ_REQUIRE(xq && wpack && wmeta && partials, PQ_ERR_ARG, "pq_w4a8_gemm_partials: null pointer");
  PQ_REQUIRE(pq::aligned_to(xq, 16) && pq::aligned_to(wpack, 16) && pq::aligned_to(wmeta, 4) &&
                 pq::aligned_to(partials, 4),
             PQ_ERR_ARG, "pq_w4a8_gemm_partials: misaligned pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
  if (m <= kSkinnyMaxM) {
    launch_skinny<true, 0>(choose_skinny(m, n, k), xq, nullptr, nullptr, nullptr, wpack, wmeta, nullptr, 0, nullptr, 0, partials, M, N,
                        K, s);
  } else {
    const unsigned grid = static_cast<unsigned>(((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN));
    gemm_tiled<true><<<grid, 256, 0, s>>>(xq, nullptr, wpack, wmeta, nullptr, 0, nullptr, 0, partials, M, N, K);
  }
  return pq::launch_status("pq_w4a8_gemm_partials launch");
}
