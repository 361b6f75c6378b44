// The whole W4A8 linear (rotation + channel scale + per-token int8 quant +
// int4 x int8 GEMM) behind one entry point, pq_w4a8_linear.
//
// Decode (M <= 4): one kernel, 16 waves in two roles.  Rotation waves rotate
// the M rows (each a share of the K groups, lane = pair, in LDS) and reduce
// the per-row absmax; GEMM waves meanwhile have requested the weight blocks
// of their share of K for the workgroup's 16-column tile.  Keeping the two
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
constexpr int kRW = 8;           // rotation waves 0..7; GEMM waves 8..15
constexpr int kGW = kDW - kRW;
constexpr int kDKP = 8;          // packed rotation layers (krot <= 8)

#define PQ_LDS_WAVE_FENCE() __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local")

struct DParams {            // one lane's packed parameters of one group (8 layers)
  uint32_t ij[4];
  float cs[16];
};

__device__ __forceinline__ void load_dparams(const uint16_t* __restrict__ rot_ij, const float* __restrict__ rot_cs,
                                             int g, int lane, DParams& p) {
  const int64_t o = (static_cast<int64_t>(g) * 64 + lane) * kDKP;
  const uint4 v = *reinterpret_cast<const uint4*>(rot_ij + o);
  p.ij[0] = v.x;
  p.ij[1] = v.y;
  p.ij[2] = v.z;
  p.ij[3] = v.w;
  const float4* c = reinterpret_cast<const float4*>(rot_cs + 2 * o);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 f = c[q];
    p.cs[4 * q] = f.x;
    p.cs[4 * q + 1] = f.y;
    p.cs[4 * q + 2] = f.z;
    p.cs[4 * q + 3] = f.w;
  }
}

// MR: rows held (M <= MR; rows past M repeat row M-1 and are never stored).
// NB: groups a rotation wave processes at once (its loads issued together,
// its LDS chains interleaved).  NT: 16-column tiles per workgroup.  The
// number of groups per wave, GPW = G/8, is a multiple of 4 (K a multiple of
// 4096), so no group index needs a bounds check.
template <int DT, int MR, int NB, int NT>
__global__ __launch_bounds__(kDW * 64) void linear_decode_kernel(
    const void* __restrict__ x, const uint16_t* __restrict__ rot_ij, const float* __restrict__ rot_cs,
    const float* __restrict__ scales, const uint8_t* __restrict__ wpack, const uint32_t* __restrict__ wmeta,
    const void* __restrict__ bias, int bias_dtype, void* __restrict__ y, int y_dtype, int M, int N, int K, int krot,
    unsigned flags) {
  extern __shared__ float rot[];                      // rotated rows: [G][MR][128] fp32
  __shared__ float rowmax[kRW][MR];
  __shared__ float red[kGW][NT][4][64];
  const int G = K >> 7;
  const int gpw = G / kRW;                            // groups per wave (multiple of 4)
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int tile0 = blockIdx.x * NT;
  const int c = lane & 15;
  const int j = lane >> 4;

  if (wave < kRW) {
    // ---- rotation role: groups wave + 8*u ---------------------------------
    const bool in16 = (flags & PQ_RQ_INPUT_FP16) != 0;
    const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
    float rmax[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) rmax[m] = 0.0f;
    for (int u0 = 0; u0 < gpw; u0 += NB) {
      DParams p[NB];
      float xa[NB][MR], xb[NB][MR];
      float s0[NB], s1[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int g = wave + kRW * (u0 + b);
        load_dparams(rot_ij, rot_cs, g, lane, p[b]);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const int mm = m < M ? m : M - 1;
          xa[b][m] = pq_load_as_f32<DT>(x, static_cast<int64_t>(mm) * K + g * 128 + lane);
          xb[b][m] = pq_load_as_f32<DT>(x, static_cast<int64_t>(mm) * K + g * 128 + 64 + lane);
        }
        s0[b] = scales != nullptr ? scales[g * 128 + lane] : 1.0f;
        s1[b] = scales != nullptr ? scales[g * 128 + 64 + lane] : 1.0f;
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float* gb = rot + (wave + kRW * (u0 + b)) * MR * 128;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          gb[m * 128 + lane] = (in16 ? pq_round_f16(xa[b][m]) : xa[b][m]) * s0[b];
          gb[m * 128 + 64 + lane] = (in16 ? pq_round_f16(xb[b][m]) : xb[b][m]) * s1[b];
        }
      }
      PQ_LDS_WAVE_FENCE();
      float ni[NB][MR], nj[NB][MR];
      int ia[NB], ja[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) ia[b] = ja[b] = 0;
#pragma unroll
      for (int r = 0; r < kDKP; ++r) {
        if (r < krot) {
          float xi[NB][MR], xj[NB][MR];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const float* gb = rot + (wave + kRW * (u0 + b)) * MR * 128;
            ia[b] = (p[b].ij[r >> 1] >> (16 * (r & 1))) & 127;
            ja[b] = (p[b].ij[r >> 1] >> (16 * (r & 1) + 8)) & 127;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
              xi[b][m] = gb[m * 128 + ia[b]];
              xj[b][m] = gb[m * 128 + ja[b]];
            }
          }
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            float* gb = rot + (wave + kRW * (u0 + b)) * MR * 128;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
              givens(xi[b][m], xj[b][m], p[b].cs[2 * r], p[b].cs[2 * r + 1], ni[b][m], nj[b][m]);
              gb[m * 128 + ia[b]] = ni[b][m];
              gb[m * 128 + ja[b]] = nj[b][m];
            }
          }
          PQ_LDS_WAVE_FENCE();
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float* gb = rot + (wave + kRW * (u0 + b)) * MR * 128;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if (mat16) {
            ni[b][m] = pq_round_f16(ni[b][m]);
            nj[b][m] = pq_round_f16(nj[b][m]);
            gb[m * 128 + ia[b]] = ni[b][m];
            gb[m * 128 + ja[b]] = nj[b][m];
          }
          rmax[m] = fmaxf(rmax[m], fmaxf(fabsf(ni[b][m]), fabsf(nj[b][m])));
        }
      }
      PQ_LDS_WAVE_FENCE();
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = pq_wave_max(rmax[m]);
      if (lane == 0) rowmax[wave][m] = v;
    }
    __syncthreads();
    __syncthreads();
  } else {
    // ---- GEMM role: groups gw + 8*u, in chunks of 4 groups x NT tiles ------
    const int gw = wave - kRW;
    float acc[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[nt][v] = 0.0f;
    float inv = 0.0f;
    constexpr int GC = NT == 1 ? 4 : 2;   // groups of weight loads in flight per chunk
    for (int u0 = 0; u0 < gpw; u0 += GC) {
      v4i wb[GC][NT];
      uint32_t wm[GC][NT];
#pragma unroll
      for (int b = 0; b < GC; ++b) {
        const int g = gw + kGW * (u0 + b);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int64_t blk = static_cast<int64_t>(tile0 + nt) * G + g;
          wb[b][nt] = *reinterpret_cast<const v4i*>(wpack + blk * 1024 + lane * 16);
          wm[b][nt] = wmeta[blk * 16 + c];
        }
      }
      if (u0 == 0) {
        __syncthreads();   // rotated rows and row maxima are ready
        float am = 0.0f;
        if (c < M) {
#pragma unroll
          for (int w = 0; w < kRW; ++w) am = fmaxf(am, rowmax[w][c < MR ? c : 0]);
        }
        inv = inv_scale(am);
      }
#pragma unroll
      for (int b = 0; b < GC; ++b) {
        const int g = gw + kGW * (u0 + b);
        v4i a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
        if (c < M) {
          const float4* src = reinterpret_cast<const float4*>(rot + (g * MR + c) * 128 + j * 32);
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
          const uint32_t meta = wm[b][nt];
          const uint32_t zb = meta_zero_bias(meta);
          const v4i w = wb[b][nt];
          const v4i b0 = unpack16(static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y), zb);
          const v4i b1 = unpack16(static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w), zb);
          v4i pp = {0, 0, 0, 0};
          pp = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, pp, 0, 0, 0);
          pp = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, pp, 0, 0, 0);
          const float sc = meta_scale(meta);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[nt][v] = fmaf(static_cast<float>(pp[v]), sc, acc[nt][v]);
        }
      }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[gw][nt][v][lane] = acc[nt][v];
    __syncthreads();
  }

  // Add the GEMM waves' K slices (fixed order) and write y.
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
  int mr;    // 1, 2 or 4
  int nt;    // 1 or 3
  size_t lds;
};

DecodeCfg choose_decode(int64_t m, int64_t n, int64_t k, int krot) {
  DecodeCfg cfg{false, 1, 1, 0};
  if (m < 1 || m > 4 || krot > kDKP || k % 4096 != 0 || k > 16384) return cfg;
  const int mr = m == 1 ? 1 : m == 2 ? 2 : 4;
  const int tiles = static_cast<int>(n / 16);
  const int nt = (tiles >= 768 && tiles % 3 == 0 && k == 4096) ? 3 : 1;
  const size_t lds = static_cast<size_t>(k / 128) * mr * 128 * sizeof(float);
  if (lds > 128 * 1024) return cfg;
  return {true, mr, nt, lds};
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

template <int DT>
void launch_decode(const DecodeCfg& cfg, const void* x, const uint16_t* rot_ij, const float* rot_cs,
                   const float* scales, const uint8_t* wpack, const uint32_t* wmeta, const void* bias, int bias_dtype,
                   void* y, int y_dtype, int M, int N, int K, int krot, unsigned flags, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>((N / 16) / cfg.nt);
#define PQ_DECODE(MR_, NB_, NT_)                                                                                 \
  if (cfg.mr == MR_ && cfg.nt == NT_) {                                                                          \
    linear_decode_kernel<DT, MR_, NB_, NT_><<<grid, kDW * 64, cfg.lds, stream>>>(                                \
        x, rot_ij, rot_cs, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags);            \
    return;                                                                                                      \
  }
  PQ_DECODE(1, 4, 1) PQ_DECODE(1, 4, 3) PQ_DECODE(2, 2, 1) PQ_DECODE(2, 2, 3) PQ_DECODE(4, 2, 1)
  PQ_DECODE(4, 2, 3)
#undef PQ_DECODE
}

}  // namespace

extern "C" size_t pq_w4a8_linear_workspace_size(int64_t m, int64_t n, int64_t k, int krot) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 || n % 16) return 0;
  if (choose_decode(m, n, k, krot).fused) return 0;
  return align_up(static_cast<size_t>(m) * k, 256) + static_cast<size_t>(m) * sizeof(float);
}

extern "C" int pq_w4a8_linear(const void* x, int x_dtype, const uint16_t* rot_ij, const float* rot_cs,
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
  PQ_REQUIRE(x && rot_ij && rot_cs && wpack && wmeta && y, PQ_ERR_ARG, "pq_w4a8_linear: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(rot_ij, 16) && pq::aligned_to(rot_cs, 16) && pq::aligned_to(wpack, 16) &&
                 pq::aligned_to(wmeta, 4) && pq::aligned_to(y, pq::dtype_size(y_dtype)),
             PQ_ERR_ARG, "pq_w4a8_linear: misaligned pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const DecodeCfg cfg = choose_decode(m, n, k, krot);
  if (cfg.fused) {
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
    switch (x_dtype) {
      case PQ_F32: launch_decode<PQ_F32>(cfg, x, rot_ij, rot_cs, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags, s); break;
      case PQ_F16: launch_decode<PQ_F16>(cfg, x, rot_ij, rot_cs, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags, s); break;
      default: launch_decode<PQ_BF16>(cfg, x, rot_ij, rot_cs, scales, wpack, wmeta, bias, bias_dtype, y, y_dtype, M, N, K, krot, flags, s); break;
    }
    return pq::launch_status("pq_w4a8_linear decode launch");
  }
  const size_t need = pq_w4a8_linear_workspace_size(m, n, k, krot);
  PQ_REQUIRE(workspace != nullptr && workspace_bytes >= need && pq::aligned_to(workspace, 256), PQ_ERR_WORKSPACE,
             "pq_w4a8_linear: a 256-byte aligned workspace of %zu bytes is needed for m=%lld k=%lld, got %zu", need,
             (long long)m, (long long)k, workspace ? workspace_bytes : (size_t)0);
  int8_t* xq = static_cast<int8_t*>(workspace);
  float* xs = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(static_cast<size_t>(m) * k, 256));
  int st = pq_rotate_quant_i8(x, x_dtype, rot_ij, rot_cs, scales, xq, xs, nullptr, m, k, krot, flags, stream);
  if (st != PQ_OK) return st;
  return pq_w4a8_gemm(xq, xs, wpack, wmeta, bias, bias_dtype, y, y_dtype, m, n, k, 128, nullptr, 0, stream);
}
