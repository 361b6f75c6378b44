// The whole W4A8 linear (rotation + channel scale + per-token int8 quant +
// int4 x int8 GEMM) behind one entry point, pq_w4a8_linear.
//
// Decode (M <= 4): one kernel, 16 waves in two roles.  Waves 0-7 rotate the
// M rows (each a share of the K groups, lane = pair, in LDS) and reduce the
// per-row absmax; waves 8-15 meanwhile have requested the weight blocks of
// their share of K for the workgroup's NT 16-column tiles.  Keeping the two
// kinds of loads in different waves matters: a wave's load counter retires
// in issue order, so a wave that issued weight loads first could not wait
// for its rotation parameters without also waiting for its weights.  After
// one barrier the GEMM waves quantize the rotated values straight into MFMA
// A fragments and run the GEMM.  Each workgroup repeats the (small)
// rotation of the M rows; in exchange no workgroup depends on another.
//
// Otherwise: pq_rotate_quant_i8 into the caller's workspace, then pq_w4a8_gemm.
//
// Reference: BF16RotateLinearWrapper -> RotateLinearInt4 -> rotation::rotate
// -> MarlinW4A8Linear (src/alpamayo_r1/utils/quantization/
// paroquant_marlin_w4a8.py:59-65, 314-333; rotation_linear.py:120-124).
#include "pq_device.h"

using namespace pqd;

namespace {

constexpr int kDW = 16;          // waves per decode workgroup
constexpr int kRW = 8;           // rotation waves (0..7); GEMM waves are 8..15
constexpr int kGW = kDW - kRW;
constexpr int kDMaxRows = 4;     // largest M of the fused decode kernel
constexpr int kDKrot = 8;        // rotation layers it keeps in registers
constexpr int kDMaxGpw = 12;     // K groups per GEMM wave with one tile (K <= 12288)
constexpr size_t kDMaxLds = 128 * 1024;

#define PQ_LDS_WAVE_FENCE() __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local")

template <int DT, int NT, int GMAX>
__global__ __launch_bounds__(kDW * 64) void linear_decode_kernel(
    const void* __restrict__ x, const uint8_t* __restrict__ pairs, const float2* __restrict__ cs,
    const float* __restrict__ scales, const uint8_t* __restrict__ wpack, const uint32_t* __restrict__ wmeta,
    const void* __restrict__ bias, int bias_dtype, void* __restrict__ y, int y_dtype, int M, int N, int K, int krot,
    unsigned flags) {
  extern __shared__ float rot[];                      // rotated rows: [G][M][128] fp32
  __shared__ float rowmax[kRW][kDMaxRows];
  __shared__ float red[kGW][NT][4][64];
  const int G = K >> 7;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int tile0 = blockIdx.x * NT;

  float acc[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[nt][v] = 0.0f;

  v4i wb[GMAX][NT];
  uint32_t wm[GMAX][NT];
  const int gw = wave - kRW;
  const int c = lane & 15;
  const int j = lane >> 4;

  if (wave < kRW) {
    // ---- rotation role: groups wave, wave+8, ... of the M rows ----------
    const bool in16 = (flags & PQ_RQ_INPUT_FP16) != 0;
    const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
    float rmax[kDMaxRows];
#pragma unroll
    for (int m = 0; m < kDMaxRows; ++m) rmax[m] = 0.0f;
    // Parameters and inputs of one group (indices clamped: unconditional loads).
    auto load_group = [&](int g, uint32_t (&pr)[kDKrot], float2 (&cc)[kDKrot], float (&xa)[kDMaxRows],
                          float (&xb)[kDMaxRows], float& s0, float& s1) {
#pragma unroll
      for (int r = 0; r < kDKrot; ++r) {
        const int rr = r < krot ? r : krot - 1;
        pr[r] = *reinterpret_cast<const uint16_t*>(pairs + static_cast<int64_t>(rr) * K + g * 128 + 2 * lane);
        cc[r] = cs[static_cast<int64_t>(rr) * (K >> 1) + g * 64 + lane];
      }
#pragma unroll
      for (int m = 0; m < kDMaxRows; ++m) {
        const int mm = m < M ? m : M - 1;
        xa[m] = pq_load_as_f32<DT>(x, static_cast<int64_t>(mm) * K + g * 128 + lane);
        xb[m] = pq_load_as_f32<DT>(x, static_cast<int64_t>(mm) * K + g * 128 + 64 + lane);
      }
      if (scales != nullptr) {
        s0 = scales[g * 128 + lane];
        s1 = scales[g * 128 + 64 + lane];
      }
    };
    uint32_t pr[kDKrot], prn[kDKrot];
    float2 cc[kDKrot], ccn[kDKrot];
    float xa[kDMaxRows], xb[kDMaxRows], xan[kDMaxRows], xbn[kDMaxRows];
    float s0 = 1.0f, s1 = 1.0f, s0n = 1.0f, s1n = 1.0f;
    if (wave < G) load_group(wave, pr, cc, xa, xb, s0, s1);
    for (int g = wave; g < G; g += kRW) {
      const int gn = g + kRW < G ? g + kRW : g;     // next group, requested before this one's layers
      load_group(gn, prn, ccn, xan, xbn, s0n, s1n);
      float* gb = rot + g * M * 128;
#pragma unroll
      for (int m = 0; m < kDMaxRows; ++m) {
        if (m < M) {
          gb[m * 128 + lane] = (in16 ? pq_round_f16(xa[m]) : xa[m]) * s0;
          gb[m * 128 + 64 + lane] = (in16 ? pq_round_f16(xb[m]) : xb[m]) * s1;
        }
      }
      PQ_LDS_WAVE_FENCE();
      float ni[kDMaxRows], nj[kDMaxRows];
      int i = 0, jj = 0;
#pragma unroll
      for (int r = 0; r < kDKrot; ++r) {
        if (r < krot) {
          i = pr[r] & 127;
          jj = (pr[r] >> 8) & 127;
#pragma unroll
          for (int m = 0; m < kDMaxRows; ++m) {
            if (m < M) {
              givens(gb[m * 128 + i], gb[m * 128 + jj], cc[r].x, cc[r].y, ni[m], nj[m]);
              gb[m * 128 + i] = ni[m];
              gb[m * 128 + jj] = nj[m];
            }
          }
          PQ_LDS_WAVE_FENCE();
        }
      }
#pragma unroll
      for (int m = 0; m < kDMaxRows; ++m) {
        if (m < M) {
          if (mat16) {
            ni[m] = pq_round_f16(ni[m]);
            nj[m] = pq_round_f16(nj[m]);
            gb[m * 128 + i] = ni[m];
            gb[m * 128 + jj] = nj[m];
          }
          rmax[m] = fmaxf(rmax[m], fmaxf(fabsf(ni[m]), fabsf(nj[m])));
        }
      }
      PQ_LDS_WAVE_FENCE();
#pragma unroll
      for (int r = 0; r < kDKrot; ++r) {
        pr[r] = prn[r];
        cc[r] = ccn[r];
      }
#pragma unroll
      for (int m = 0; m < kDMaxRows; ++m) {
        xa[m] = xan[m];
        xb[m] = xbn[m];
      }
      s0 = s0n;
      s1 = s1n;
    }
#pragma unroll
    for (int m = 0; m < kDMaxRows; ++m) {
      const float v = pq_wave_max(rmax[m]);
      if (lane == 0) rowmax[wave][m] = v;
    }
  } else {
    // ---- GEMM role: request this wave's weight blocks (groups gw, gw+8, ...)
#pragma unroll
    for (int u = 0; u < GMAX; ++u) {
      const int g = gw + kGW * u;
      const int gc = g < G ? g : G - 1;    // clamped: unconditional loads
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int64_t blk = static_cast<int64_t>(tile0 + nt) * G + gc;
        wb[u][nt] = *reinterpret_cast<const v4i*>(wpack + blk * 1024 + lane * 16);
        wm[u][nt] = wmeta[blk * 16 + c];
      }
    }
  }
  __syncthreads();

  if (wave >= kRW) {
    float am = 0.0f;
    if (c < M) {
#pragma unroll
      for (int w = 0; w < kRW; ++w) am = fmaxf(am, rowmax[w][c]);
    }
    const float inv = inv_scale(am);
#pragma unroll
    for (int u = 0; u < GMAX; ++u) {
      const int g = gw + kGW * u;
      if (g < G) {
        v4i a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
        if (c < M) {
          const float4* src = reinterpret_cast<const float4*>(rot + (g * M + c) * 128 + j * 32);
          const float4 f0 = src[0], f1 = src[1], f2 = src[2], f3 = src[3];
          const float4 f4 = src[4], f5 = src[5], f6 = src[6], f7 = src[7];
          a0.x = static_cast<int>(quant4(f0.x, f0.y, f0.z, f0.w, inv));
          a0.y = static_cast<int>(quant4(f1.x, f1.y, f1.z, f1.w, inv));
          a0.z = static_cast<int>(quant4(f2.x, f2.y, f2.z, f2.w, inv));
          a0.w = static_cast<int>(quant4(f3.x, f3.y, f3.z, f3.w, inv));
          a1.x = static_cast<int>(quant4(f4.x, f4.y, f4.z, f4.w, inv));
          a1.y = static_cast<int>(quant4(f5.x, f5.y, f5.z, f5.w, inv));
          a1.z = static_cast<int>(quant4(f6.x, f6.y, f6.z, f6.w, inv));
          a1.w = static_cast<int>(quant4(f7.x, f7.y, f7.z, f7.w, inv));
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t meta = wm[u][nt];
          const uint32_t zb = meta_zero_bias(meta);
          const v4i w = wb[u][nt];
          const v4i b0 = unpack16(static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y), zb);
          const v4i b1 = unpack16(static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w), zb);
          v4i p = {0, 0, 0, 0};
          p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, p, 0, 0, 0);
          const float sc = meta_scale(meta);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[nt][v] = fmaf(static_cast<float>(p[v]), sc, acc[nt][v]);
        }
      }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[gw][nt][v][lane] = acc[nt][v];
  }
  __syncthreads();

  // Add the 8 GEMM waves' K slices (fixed order) and write y.
  for (int t = threadIdx.x; t < NT * 256; t += kDW * 64) {
    const int nt = t >> 8;
    const int rv = (t >> 6) & 3;
    const int rl = t & 63;
    const int m = 4 * (rl >> 4) + rv;
    if (m >= M) continue;
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kGW; ++w) sum += red[w][nt][rv][rl];
    float amm = 0.0f;
#pragma unroll
    for (int w = 0; w < kRW; ++w) amm = fmaxf(amm, rowmax[w][m]);
    const int n = (tile0 + nt) * 16 + (rl & 15);
    pq_store_dyn(y, y_dtype, static_cast<int64_t>(m) * N + n, epilogue(sum, amm / 127.0f, bias, bias_dtype, n));
  }
}

struct DecodeCfg {
  bool fused;
  int nt;
  int gmax;  // 4 or 12 weight blocks per GEMM wave and tile
  size_t lds;
};

DecodeCfg choose_decode(int64_t m, int64_t n, int64_t k, int krot) {
  DecodeCfg cfg{false, 1, 4, 0};
  if (m < 1 || m > kDMaxRows || krot > kDKrot) return cfg;
  const int G = static_cast<int>(k / 128);
  const int gpw = (G + kGW - 1) / kGW;     // groups per GEMM wave
  if (gpw > kDMaxGpw) return cfg;
  const int tiles = static_cast<int>(n / 16);
  const int gmax = gpw <= 4 ? 4 : 12;
  const int nt = (tiles >= 512 && tiles % 2 == 0 && gmax == 4) ? 2 : 1;
  const size_t lds = static_cast<size_t>(G) * m * 128 * sizeof(float);
  if (lds > kDMaxLds) return cfg;
  return {true, nt, gmax, lds};
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

template <int DT>
void launch_decode(const DecodeCfg& cfg, const void* x, const uint8_t* pairs, const float* cs, const float* scales,
                   const uint8_t* wpack, const uint32_t* wmeta, const void* bias, int bias_dtype, void* y,
                   int y_dtype, int M, int N, int K, int krot, unsigned flags, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>((N / 16) / cfg.nt);
  const float2* cs2 = reinterpret_cast<const float2*>(cs);
#define PQ_DECODE(NT_, GM_)                                                                                   \
  if (cfg.nt == NT_ && cfg.gmax == GM_) {                                                                     \
    linear_decode_kernel<DT, NT_, GM_><<<grid, kDW * 64, cfg.lds, stream>>>(                                  \
        x, pairs, cs2, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags);             \
    return;                                                                                                   \
  }
  PQ_DECODE(1, 4) PQ_DECODE(1, 12) PQ_DECODE(2, 4)
#undef PQ_DECODE
}

}  // namespace

extern "C" size_t pq_w4a8_linear_workspace_size(int64_t m, int64_t n, int64_t k, int krot) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 || n % 16) return 0;
  if (choose_decode(m, n, k, krot).fused) return 0;
  return align_up(static_cast<size_t>(m) * k, 256) + static_cast<size_t>(m) * sizeof(float);
}

extern "C" int pq_w4a8_linear(const void* x, int x_dtype, const uint8_t* pairs, const float* cos_sin,
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
  PQ_REQUIRE(x && pairs && cos_sin && wpack && wmeta && y, PQ_ERR_ARG, "pq_w4a8_linear: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(cos_sin, 8) && pq::aligned_to(wpack, 16) &&
                 pq::aligned_to(wmeta, 4) && pq::aligned_to(y, pq::dtype_size(y_dtype)),
             PQ_ERR_ARG, "pq_w4a8_linear: misaligned pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const DecodeCfg cfg = choose_decode(m, n, k, krot);
  if (cfg.fused) {
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
    switch (x_dtype) {
      case PQ_F32: launch_decode<PQ_F32>(cfg, x, pairs, cos_sin, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags, s); break;
      case PQ_F16: launch_decode<PQ_F16>(cfg, x, pairs, cos_sin, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags, s); break;
      default: launch_decode<PQ_BF16>(cfg, x, pairs, cos_sin, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags, s); break;
    }
    return pq::launch_status("pq_w4a8_linear decode launch");
  }
  const size_t need = pq_w4a8_linear_workspace_size(m, n, k, krot);
  PQ_REQUIRE(workspace != nullptr && workspace_bytes >= need && pq::aligned_to(workspace, 256), PQ_ERR_WORKSPACE,
             "pq_w4a8_linear: a 256-byte aligned workspace of %zu bytes is needed for m=%lld k=%lld, got %zu", need,
             (long long)m, (long long)k, workspace ? workspace_bytes : (size_t)0);
  int8_t* xq = static_cast<int8_t*>(workspace);
  float* xs = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(static_cast<size_t>(m) * k, 256));
  int st = pq_rotate_quant_i8(x, x_dtype, pairs, cos_sin, scales, xq, xs, nullptr, m, k, krot, flags, stream);
  if (st != PQ_OK) return st;
  return pq_w4a8_gemm(xq, xs, wpack, wmeta, bias, bias_dtype, y, y_dtype, m, n, k, 128, nullptr, 0, stream);
}
