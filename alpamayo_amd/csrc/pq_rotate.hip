// Stage 1 and 2 of the W4A8 linear on gfx950:
//   pq_rotate           -- the rotation::rotate op (pairwise Givens + channel scale)
//   pq_rotate_quant_i8  -- rotation + per-token absmax + int8 quant, one pass
//   pq_quant_i8         -- per-token int8 quant of an existing tensor
//
// Reference semantics: kernels/paroquant_kernels/src/rotation.cuh:247-337
// (scale-multiply, KROT Givens layers xi' = c xi + s xj, xj' = -s xi + c xj
// on group-local pair indices, fp32 math, result rounded to the storage
// dtype) and vLLM's dynamic per-token int8 quant (scale = absmax/127,
// q = rne(x * 127/absmax)) as called at
// src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:319-333.
//
// All updates are written with explicit fmaf and the file is compiled with
// -ffp-contract=off, so the float32 sequence is fixed:
//   xi' = fma(xi, c, xj*s),  xj' = fma(xj, c, -(xi*s)).
#include <algorithm>
#include <type_traits>

#include "pq_device.h"
#include "pq_internal.h"

using pqd::quant4;

namespace {

constexpr int kRotRows = 16;   // rows per workgroup of the plain rotation kernel


// ---------------------------------------------------------------------------
// rotation::rotate.  A workgroup of 4 waves takes 16 rows x 128 channels (for
// group 64 the chunk holds two groups).  The 64 pairs' indices (masked to the
// group, so a bad index can never address outside the tile) and cos/sin of
// every layer are derived once per workgroup into LDS -- each sincos serves
// 16 rows.  Wave w owns rows 4w .. 4w+3 as a channel-major LDS tile (one
// float4 = the wave's 4 rows of a channel), so lane l applies a layer to its
// pair with two 16-byte reads and two 16-byte writes.
// ---------------------------------------------------------------------------
//
// MX: instead of the rotated values, their OCP MXFP4 quantization (fused
// rotate + quant): y receives the E2M1 codes [rows][h/2] (element 2i in the
// low nibble of byte i) and sc the E8M0 scales [rows][h/32] (0xFF when the
// block holds a NaN).  Lane l quantizes channels 2l, 2l+1 of its wave's rows;
// the 16 lanes of a 32-channel block exchange their absmax by shuffles.
constexpr int kRotWaves = 4;
constexpr int kRotRowsPerWave = 4;
constexpr int kRotMaxLayers = 16;

template <int DT, int G, bool SCALE, bool MX>
__global__ __launch_bounds__(kRotWaves * 64) void rotate_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                                uint8_t* __restrict__ sc,
                                                                const int16_t* __restrict__ idx,
                                                                const void* __restrict__ theta,
                                                                const void* __restrict__ scales, int64_t rows,
                                                                int h, int krot) {
  static_assert(kRotRows == kRotWaves * kRotRowsPerWave && kRotRowsPerWave == 4, "a float4 per channel and wave");
  __shared__ float4 tile[kRotWaves][128];
  __shared__ float2 s_cs[kRotMaxLayers][64];
  __shared__ uint32_t s_ij[kRotMaxLayers][64];
  constexpr int NT = kRotWaves * 64;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRotRows;
  const int ch0 = blockIdx.y * 128;

  // Layer parameters of the chunk's 64 pairs.  A pair past h (the second
  // half of a 64-channel tail) turns its own two channels, which hold zeros
  // and are never stored, by the identity.
  for (int e = t; e < krot * 64; e += NT) {
    const int r = e >> 6, p = e & 63;
    const int P = blockIdx.y * 64 + p;   // pair index within the row; theta column
    float c = 1.0f, sn = 0.0f;
    uint32_t ij = static_cast<uint32_t>(2 * p) | (static_cast<uint32_t>(2 * p + 1) << 8);
    if (P < (h >> 1)) {
      const int gi = P / (G / 2);
      const int pp = P % (G / 2);
      const int base = gi * G - ch0;   // group start inside the 128-channel tile
      const int64_t o = static_cast<int64_t>(r) * h + gi * G + 2 * pp;
      const int i = base + (idx[o] & (G - 1));
      const int j = base + (idx[o + 1] & (G - 1));
      const float th = pq_load_as_f32<DT>(theta, static_cast<int64_t>(r) * (h >> 1) + P);
      // cos and sin of the stored angle in float64, rounded once to float32:
      // the values the host derives for the fused kernels' operands, so this
      // kernel and those agree bit for bit
      double sd, cd;
      sincos(static_cast<double>(th), &sd, &cd);
      c = static_cast<float>(cd);
      sn = static_cast<float>(sd);
      ij = static_cast<uint32_t>(i) | (static_cast<uint32_t>(j) << 8);
    }
    s_cs[r][p] = make_float2(c, sn);
    s_ij[r][p] = ij;
  }
  // Wave w loads its own rows: lane l channels 2l, 2l+1 of each (coalesced).
  float4* wt = tile[w];
  {
    const int ch = ch0 + 2 * lane;
    float s0 = 1.0f, s1 = 1.0f;
    if (SCALE && ch < h) {
      s0 = pq_load_as_f32<DT>(scales, ch);
      s1 = pq_load_as_f32<DT>(scales, ch + 1);
    }
    float va[kRotRowsPerWave], vb[kRotRowsPerWave];
#pragma unroll
    for (int rr = 0; rr < kRotRowsPerWave; ++rr) {
      const int64_t row = row0 + w * kRotRowsPerWave + rr;
      va[rr] = 0.0f;
      vb[rr] = 0.0f;
      if (row < rows && ch < h) {
        va[rr] = pq_load_as_f32<DT>(x, row * h + ch);
        vb[rr] = pq_load_as_f32<DT>(x, row * h + ch + 1);
        if (SCALE) {
          va[rr] = va[rr] * s0;
          vb[rr] = vb[rr] * s1;
        }
      }
    }
    wt[2 * lane] = make_float4(va[0], va[1], va[2], va[3]);
    wt[2 * lane + 1] = make_float4(vb[0], vb[1], vb[2], vb[3]);
  }
  __syncthreads();

  for (int r = 0; r < krot; ++r) {
    const float2 cs = s_cs[r][lane];
    const uint32_t ij = s_ij[r][lane];
    const int i = static_cast<int>(ij & 0xffu), j = static_cast<int>(ij >> 8);
    const float4 xi = wt[i];
    const float4 xj = wt[j];
    float4 ni, nj;
    ni.x = fmaf(xi.x, cs.x, xj.x * cs.y);
    nj.x = fmaf(xj.x, cs.x, -(xi.x * cs.y));
    ni.y = fmaf(xi.y, cs.x, xj.y * cs.y);
    nj.y = fmaf(xj.y, cs.x, -(xi.y * cs.y));
    ni.z = fmaf(xi.z, cs.x, xj.z * cs.y);
    nj.z = fmaf(xj.z, cs.x, -(xi.z * cs.y));
    ni.w = fmaf(xi.w, cs.x, xj.w * cs.y);
    nj.w = fmaf(xj.w, cs.x, -(xi.w * cs.y));
    wt[i] = ni;
    wt[j] = nj;
    // The sub-tile is this wave's alone, and a wave's LDS operations complete
    // in issue order: the next layer's reads see these writes without a
    // workgroup barrier.  The fence keeps the compiler from moving them.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }

  // Lane l of wave w holds channels 2l, 2l+1 of the wave's 4 rows.
  const float4 fa = wt[2 * lane], fb = wt[2 * lane + 1];
  const float va[kRotRowsPerWave] = {fa.x, fa.y, fa.z, fa.w};
  const float vb[kRotRowsPerWave] = {fb.x, fb.y, fb.z, fb.w};
  const int ch = ch0 + 2 * lane;
  if constexpr (MX) {
    // a 32-channel block = 16 lanes: absmax and the NaN flag over them by shuffles
#pragma unroll
    for (int rr = 0; rr < kRotRowsPerWave; ++rr) {
      float am = fmaxf(fabsf(va[rr]), fabsf(vb[rr]));
      int nn = (va[rr] != va[rr]) || (vb[rr] != vb[rr]) ? 1 : 0;
#pragma unroll
      for (int d = 1; d < 16; d <<= 1) {
        am = fmaxf(am, __shfl_xor(am, d));
        nn |= __shfl_xor(nn, d);
      }
      const int ex = pqd::mx_shared_exp(am);
      const float inv = pqd::mx_inv_scale(ex);
      const uint32_t code = pqd::mx_e2m1(va[rr] * inv) | (pqd::mx_e2m1(vb[rr] * inv) << 4);
      const int64_t row = row0 + w * kRotRowsPerWave + rr;
      if (row < rows && ch < h) {
        static_cast<uint8_t*>(y)[row * (h >> 1) + (ch >> 1)] = static_cast<uint8_t>(code);
        if ((lane & 15) == 0) sc[row * (h >> 5) + (ch >> 5)] = nn ? 0xFFu : static_cast<uint8_t>(ex + 127);
      }
    }
  } else {
#pragma unroll
    for (int rr = 0; rr < kRotRowsPerWave; ++rr) {
      const int64_t row = row0 + w * kRotRowsPerWave + rr;
      if (row < rows && ch < h) {
        pq_store_from_f32<DT>(y, row * h + ch, va[rr]);
        pq_store_from_f32<DT>(y, row * h + ch + 1, vb[rr]);
      }
    }
  }
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  constexpr int NW = NT / 64;
  v = pq_wave_max_nonneg(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int k = 1; k < NW; ++k) m = fmaxf(m, red[k]);
  return m;
}

template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t elem, float f[8]) {
  if constexpr (DT == PQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    const float4 a = p[0], b = p[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = static_cast<uint16_t>(w[e] & 0xffffu), hi = static_cast<uint16_t>(w[e] >> 16);
      if constexpr (DT == PQ_F16) {
        f[2 * e] = pq_f16_to_f32(lo);
        f[2 * e + 1] = pq_f16_to_f32(hi);
      } else {
        f[2 * e] = pq_bf16_to_f32(lo);
        f[2 * e + 1] = pq_bf16_to_f32(hi);
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Fused rotate + quant over blocks of RB rows (RB a compile-time constant, so
// the RB rows are RB independent register chains with no per-row branches).
// 512 threads; wave w rotates groups w, w+8, ... for the block's rows: lane l
// loads channels l and l+64 of each row (coalesced) and runs the packed
// register chain (one cross-lane fetch per layer, no LDS traffic inside the
// layers), then stores the finished values into a row buffer [RB][h] (fp16
// when the result is materialized in fp16, fp32 otherwise).  The next group's
// parameters and inputs are requested before the current group's layers run.
// After a block-wide absmax per row the row buffer is quantized with
// coalesced stores.  Parameters are read once per group per RB rows.
// ---------------------------------------------------------------------------
constexpr int kRQWaves = 8;

//
// With NORM the rows first go through the prologue of nm.mode (PQ_PRO_*):
// RMSNORM computes the RMSNorm factor of each of the block's rows (wave r
// takes row r, with the same per-row routine as the split rotation) and
// rotates the normalized values; ADD rotates x + res; SWIGLU rotates
// silu(x) * up.  Member 0's blocks also write h / the residual sum s when
// asked.
//
// OUT selects what the block writes: kRqInt8 the int8 codes and token
// scales (and the fp16 rows when asked); kRqRows the rotated rows in x's
// dtype (the rotation::rotate result); kRqMxfp4 their OCP MXFP4 codes and
// E8M0 scales (mb.out / mb.xrot, the rotation::rotate_and_quant_mxfp4
// result).  The last two take no prologue, no fp16 rounding and no flags.
//
// IN fixes how the input reaches the rotation: kInAsIs as it is, kInF16
// rounded to fp16 (PQ_RQ_INPUT_FP16; the rounding and the channel scale
// then cost one v_cvt_f16_f32 and one v_fma_mix_f32), kInFlag as the flag
// says at run time.
//
// With MAT16 the row buffer is channel-major: channel c's RB fp16 values lie
// side by side at rowbuf[c * RB], so a lane stores a slot's RB rows with
// RB / 2 packed converts and one LDS write.
constexpr int kRqInt8 = 0, kRqRows = 1, kRqMxfp4 = 2;
constexpr int kInAsIs = 0, kInF16 = 1, kInFlag = 2;

template <int DT, int KP, bool MAT16, int RB, bool NORM, int OUT = kRqInt8, int IN = kInFlag>
__global__ __launch_bounds__(kRQWaves * 64) void rotate_quant_kernel(const void* __restrict__ x,
                                                                       const pq::RotGroup grp, int64_t row_begin,
                                                                       int h, int krot, unsigned flags,
                                                                       const pq::NormArgs nm) {
  static_assert(RB <= kRQWaves, "one wave per row for the norm factors");
  static_assert(OUT == kRqInt8 || (!MAT16 && !NORM), "plain and MXFP4 outputs come from the float32 rows");
  const pq::RotMember& mb = grp.mem[blockIdx.y];
  const uint32_t* __restrict__ rot_idx = mb.rot_idx;
  const float* __restrict__ rot_cs = mb.rot_cs;
  const float* __restrict__ scales = mb.scales;
  int8_t* __restrict__ xq = static_cast<int8_t*>(mb.out);
  float* __restrict__ xscale = mb.out_scale;
  uint16_t* __restrict__ xrot = static_cast<uint16_t*>(mb.xrot);
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  __shared__ float red[kRQWaves][RB];
  using RowT = typename std::conditional<MAT16, uint16_t, float>::type;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform: scalar branches
  const bool in16 = (flags & PQ_RQ_INPUT_FP16) != 0;
  const float nz = pqd::opaque_neg_zero();
  const int G = h >> 7;
  RowT* rowbuf = reinterpret_cast<RowT*>(lds_raw);
  const int64_t row0 = row_begin + static_cast<int64_t>(blockIdx.x) * RB;
  // Channel-scale loads stay unconditional: without scales they read
  // rot_cs[0] and the value is replaced by 1.
  const bool has_scales = scales != nullptr;
  const float* sp = has_scales ? scales : rot_cs;
  const int smask = has_scales ? 0x7fffffff : 0;

  float rmax[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) rmax[r] = 0.0f;

  // Two register sets, used alternately (the group loop is unrolled twice): the set of group g is
  // computed while the loads of group g + kRQWaves land in the other one, with no copies between them.
  pqd::RotLane<KP> rl[2];
  uint32_t xa[2][RB], xb[2][RB];
  float sa[2] = {1.0f, 1.0f}, sb[2] = {1.0f, 1.0f};
  // bfloat16 rows of the int8 path (16-byte aligned, h a multiple of 128)
  // are read as dwords: lanes 2i and 2i+1 load the same pair of channels and
  // each moves its own half into the high half of a float with one byte
  // permute (a 16-bit load costs a zero-extension here on top of the shift).
  constexpr bool kPairLoads = DT == PQ_BF16 && OUT == kRqInt8;
  const uint32_t psel = (lane & 1) ? 0x03020c0cu : 0x01000c0cu;
  static_assert(!kPairLoads || IN != kInFlag, "bfloat16 input fixes its treatment at compile time");
  auto raw_f32 = [&](uint32_t raw) -> float {
    if constexpr (kPairLoads) return __uint_as_float(__builtin_amdgcn_perm(0u, raw, psel));
    else return pq_raw_to_f32<DT>(raw);
  };
  const int lane_ch = kPairLoads ? (lane & ~1) : lane;
  // channel lane (+ c0) of the row that starts at element e0 (a multiple of 128)
  auto load_row = [&](const void* base, int64_t e0) -> uint32_t {
    if constexpr (kPairLoads) return *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(base) + e0 + lane_ch);
    else return pq_load_raw<DT>(base, e0 + lane_ch);
  };
  auto load_inputs = [&](int g, uint32_t (&va)[RB], uint32_t (&vb)[RB], float& s0, float& s1) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      va[r] = load_row(x, (row0 + r) * h + g * 128);
      vb[r] = load_row(x, (row0 + r) * h + g * 128 + 64);
    }
    s0 = sp[(g * 128 + lane) & smask];
    s1 = sp[(g * 128 + 64 + lane) & smask];
  };

  // Prologue: residual / up rows and norm weights ride along with the
  // inputs (unconditional loads; without a residual or weight they re-read x
  // and are unused).
  __shared__ float s_rinv[RB];
  const bool pro_norm = NORM && nm.mode == PQ_PRO_RMSNORM;
  const bool pro_glu = NORM && nm.mode == PQ_PRO_SWIGLU;
  const void* nres = NORM && nm.res != nullptr ? nm.res : x;
  const void* nwp = pro_norm ? nm.w : x;
  uint32_t ra[2][RB], rb[2][RB];
  uint32_t wa[2] = {0, 0}, wb[2] = {0, 0};
  auto load_norm = [&](int g, uint32_t (&va)[RB], uint32_t (&vb)[RB], uint32_t& w0, uint32_t& w1) {
    if constexpr (NORM) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        va[r] = load_row(nres, (row0 + r) * h + g * 128);
        vb[r] = load_row(nres, (row0 + r) * h + g * 128 + 64);
      }
      w0 = pq_load_raw<DT>(nwp, g * 128 + lane);
      w1 = pq_load_raw<DT>(nwp, g * 128 + 64 + lane);
    }
  };
  // the first group's loads go out before the RMSNorm factor is reduced, so
  // they are in flight while waves 0..RB-1 sum their rows
  if (w < G) {
    pqd::load_rot_lane<KP, false>(rot_idx, rot_cs, w, lane, rl[0]);
    load_inputs(w, xa[0], xb[0], sa[0], sb[0]);
    load_norm(w, ra[0], rb[0], wa[0], wb[0]);
  }
  if (pro_norm) {
    if (w < RB) {
      const float r = pqd::rms_inv(pqd::row_sumsq<DT>(x, nm.res, (row0 + w) * h, h, lane), h, nm.eps);
      if (lane == 0) s_rinv[w] = r;
    }
    pqd::lds_barrier();   // s_rinv is written (LDS only: the loads above stay in flight)
  }
  const bool write_norm = NORM && blockIdx.y == 0;   // the same for every member: member 0 writes

  for (int g0 = w; g0 < G; g0 += 2 * kRQWaves) {
#pragma unroll
    for (int ph = 0; ph < 2; ++ph) {
      const int g = g0 + ph * kRQWaves;
      if (g >= G) break;   // wave-uniform
      const int nx = ph ^ 1;
      const int gn = (g + kRQWaves < G) ? g + kRQWaves : g;   // clamped: the loads stay unconditional
      pqd::load_rot_lane<KP, false>(rot_idx, rot_cs, gn, lane, rl[nx]);
      load_inputs(gn, xa[nx], xb[nx], sa[nx], sb[nx]);
      load_norm(gn, ra[nx], rb[nx], wa[nx], wb[nx]);

      const pqd::RotLane<KP>& cur = rl[ph];
      const bool sw = pqd::rot_init_swapped(cur);
      const float s0 = has_scales ? sa[ph] : 1.0f, s1 = has_scales ? sb[ph] : 1.0f;
      float a[RB], b[RB];
      if constexpr (kPairLoads && !NORM) {
        // The initial slot swap rides in the byte permute that unpacks the
        // bfloat16 values: with the dword of channel lane + 64 as its upper
        // source, adding 4 to the selector's two data bytes takes that
        // channel instead (two selectors per group, no select per row).
        const uint32_t to_b = sw ? 0x04040000u : 0u;
        const uint32_t sel_a = psel + to_b, sel_b = psel + (0x04040000u - to_b);
        const float sc_a = sw ? s1 : s0, sc_b = sw ? s0 : s1;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const float va = __uint_as_float(__builtin_amdgcn_perm(xb[ph][r], xa[ph][r], sel_a));
          const float vb = __uint_as_float(__builtin_amdgcn_perm(xb[ph][r], xa[ph][r], sel_b));
          if constexpr (IN == kInF16) {
            a[r] = pqd::f16_scaled(va, sc_a, nz);
            b[r] = pqd::f16_scaled(vb, sc_b, nz);
          } else {
            a[r] = va * sc_a;
            b[r] = vb * sc_b;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          float lo = raw_f32(xa[ph][r]), hi = raw_f32(xb[ph][r]);
          if constexpr (NORM) {
            const int64_t ro = (row0 + r) * h + g * 128 + lane;
            if (pro_glu) {
              lo = pqd::swiglu<DT>(lo, raw_f32(ra[ph][r]));
              hi = pqd::swiglu<DT>(hi, raw_f32(rb[ph][r]));
            } else {
              if (nm.res != nullptr) {
                lo = pqd::round_to_dt<DT>(lo + raw_f32(ra[ph][r]));
                hi = pqd::round_to_dt<DT>(hi + raw_f32(rb[ph][r]));
              }
              if (write_norm && nm.s_out != nullptr) {
                pq_store_from_f32<DT>(nm.s_out, ro, lo);
                pq_store_from_f32<DT>(nm.s_out, ro + 64, hi);
              }
              if (pro_norm) {
                lo = pqd::rms_apply<DT>(lo, s_rinv[r], pq_raw_to_f32<DT>(wa[ph]));
                hi = pqd::rms_apply<DT>(hi, s_rinv[r], pq_raw_to_f32<DT>(wb[ph]));
              }
            }
            if ((pro_norm || pro_glu) && write_norm && nm.h_out != nullptr) {
              pq_store_from_f32<DT>(nm.h_out, ro, lo);
              pq_store_from_f32<DT>(nm.h_out, ro + 64, hi);
            }
          }
          if constexpr (IN == kInF16) {
            lo = pqd::f16_scaled(lo, s0, nz);
            hi = pqd::f16_scaled(hi, s1, nz);
          } else if constexpr (IN == kInFlag) {
            lo = (in16 ? pq_round_f16(lo) : lo) * s0;
            hi = (in16 ? pq_round_f16(hi) : hi) * s1;
          } else {
            lo = lo * s0;
            hi = hi * s1;
          }
          a[r] = sw ? hi : lo;
          b[r] = sw ? lo : hi;
        }
      }
      pqd::rot_layers<KP, RB>(cur, krot, a, b);
      const int fa = g * 128 + pqd::rot_final_a(cur), fb = g * 128 + pqd::rot_final_b(cur);
      if constexpr (MAT16) {   // (24-bit multiplies: full rate for 3 and 6 rows too)
        pqd::store_f16xn<RB>(rowbuf + __umul24(fa, RB), a);
        pqd::store_f16xn<RB>(rowbuf + __umul24(fb, RB), b);
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const float vi = a[r], vj = b[r];
        if constexpr (!MAT16) {
          rowbuf[r * h + fa] = vi;
          rowbuf[r * h + fb] = vj;
        }
        // the float32 values: rounding to fp16 is monotonic, so the row's
        // fp16 absmax is its float32 absmax rounded once (below)
        rmax[r] = fmaxf(rmax[r], fmaxf(fabsf(vi), fabsf(vj)));
      }
    }
  }

  if constexpr (OUT == kRqRows) {
    // the rotated rows in x's dtype, 8 elements (16 or 32 bytes) per thread per step
    __syncthreads();
    const int per_row = h >> 3;
    for (int e = t; e < RB * per_row; e += kRQWaves * 64) {
      const int r = e / per_row;
      const int c8 = (e - r * per_row) * 8;
      const float* src = reinterpret_cast<const float*>(rowbuf) + r * h + c8;
      const float4 a = *reinterpret_cast<const float4*>(src);
      const float4 b = *reinterpret_cast<const float4*>(src + 4);
      const int64_t o = (row0 + r) * h + c8;
      if constexpr (DT == PQ_F32) {
        float* dst = static_cast<float*>(mb.out) + o;
        *reinterpret_cast<float4*>(dst) = a;
        *reinterpret_cast<float4*>(dst + 4) = b;
      } else {
        const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t wd[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = DT == PQ_F16 ? pq_f32_to_f16(f[2 * q]) : pq_f32_to_bf16(f[2 * q]);
          const uint32_t hi = DT == PQ_F16 ? pq_f32_to_f16(f[2 * q + 1]) : pq_f32_to_bf16(f[2 * q + 1]);
          wd[q] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(mb.out) + o) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      }
    }
    return;
  } else if constexpr (OUT == kRqMxfp4) {
    // 32-channel blocks: 4 consecutive threads of 8 channels each exchange their absmax
    __syncthreads();
    const int per_row = h >> 3;
    uint8_t* __restrict__ codes = static_cast<uint8_t*>(mb.out);
    uint8_t* __restrict__ mxs = static_cast<uint8_t*>(mb.xrot);
    for (int e0 = 0; e0 < RB * per_row; e0 += kRQWaves * 64) {   // uniform trip count: the shuffles see every lane
      const int e = e0 + t;
      const bool live = e < RB * per_row;
      const int ee = live ? e : 0;
      const int r = ee / per_row;
      const int c8 = (ee - r * per_row) * 8;
      const float* src = reinterpret_cast<const float*>(rowbuf) + r * h + c8;
      const float4 a = *reinterpret_cast<const float4*>(src);
      const float4 b = *reinterpret_cast<const float4*>(src + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      float am = 0.0f;
      bool nan = false;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        am = fmaxf(am, fabsf(v[q]));
        nan = nan || (v[q] != v[q]);
      }
      am = fmaxf(am, __shfl_xor(am, 1));
      am = fmaxf(am, __shfl_xor(am, 2));
      int nn = nan ? 1 : 0;
      nn |= __shfl_xor(nn, 1);
      nn |= __shfl_xor(nn, 2);
      const int ex = pqd::mx_shared_exp(am);
      const float inv = pqd::mx_inv_scale(ex);
      uint32_t wd = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) wd |= pqd::mx_e2m1(v[q] * inv) << (4 * q);
      if (live) {
        const int64_t row = row0 + r;
        *reinterpret_cast<uint32_t*>(codes + row * (h >> 1) + (c8 >> 1)) = wd;
        if ((c8 & 31) == 0) mxs[row * (h >> 5) + (c8 >> 5)] = nn ? 0xFFu : static_cast<uint8_t>(ex + 127);
      }
    }
    return;
  }

  uint32_t ubits[RB];   // the rows' maxima are >= 0: their bits order like unsigned integers
#pragma unroll
  for (int r = 0; r < RB; ++r) ubits[r] = __float_as_uint(rmax[r]);
  pq_wave_umax_n<RB>(ubits);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RB; ++r) red[w][r] = __uint_as_float(ubits[r]);
  }
  __syncthreads();
  // Each row's 127 / absmax, and its token scale, once per row.
  __shared__ float s_inv[RB];
  if (t < RB) {
    float am = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kRQWaves; ++ww) am = fmaxf(am, red[ww][t]);
    if constexpr (MAT16) am = pq_round_f16(am);   // = the absmax of the fp16 rows
    s_inv[t] = pqd::inv_scale(am);
    if (xq != nullptr) xscale[row0 + t] = am / 127.0f;   // null: only the fp16 rows are wanted (W4A16)
  }
  __syncthreads();

  if constexpr (MAT16) {
    // Quantize the channel-major fp16 buffer: a thread takes 8 channels of all
    // RB rows (RB 16-byte reads), then writes each row's 8 codes (8 bytes,
    // coalesced across the threads) and, when asked, its 8 fp16 values.
    for (int e = t; e < (h >> 3); e += kRQWaves * 64) {
      const int c8 = e * 8;
      uint32_t d[4 * RB];   // (channel c8 + k, row r) is fp16 number k * RB + r of d
      const uint4* src = reinterpret_cast<const uint4*>(rowbuf + c8 * RB);
#pragma unroll
      for (int q = 0; q < RB; ++q) {
        const uint4 u = src[q];
        d[4 * q] = u.x;
        d[4 * q + 1] = u.y;
        d[4 * q + 2] = u.z;
        d[4 * q + 3] = u.w;
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int64_t ro = (row0 + r) * h + c8;
        if (xrot != nullptr) {
          uint32_t w[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) w[m] = pqd::f16_pair(d, 2 * m * RB + r, (2 * m + 1) * RB + r);
          *reinterpret_cast<uint4*>(xrot + ro) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if (xq != nullptr) {
          const float inv = s_inv[r];
          uint32_t c[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int i = k * RB + r;
            c[k] = pqd::quant_scaled(pqd::mul_f16(d[i >> 1], (i & 1) != 0, inv));
          }
          *reinterpret_cast<uint2*>(xq + ro) =
              make_uint2(pqd::pack4(c[0], c[1], c[2], c[3]), pqd::pack4(c[4], c[5], c[6], c[7]));
        }
      }
    }
  } else {
    // Quantize the row buffer: 8 elements per thread per step.
    const int per_row = h >> 3;
    for (int e = t; e < RB * per_row; e += kRQWaves * 64) {
      const int r = e / per_row;
      const int c8 = (e - r * per_row) * 8;
      const float inv = s_inv[r];
      float f[8];
      const float4 a = *reinterpret_cast<const float4*>(rowbuf + r * h + c8);
      const float4 b = *reinterpret_cast<const float4*>(rowbuf + r * h + c8 + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
      if (xrot != nullptr) {
        uint4 o;
        o.x = pqd::pk_f16(f[0], f[1]);
        o.y = pqd::pk_f16(f[2], f[3]);
        o.z = pqd::pk_f16(f[4], f[5]);
        o.w = pqd::pk_f16(f[6], f[7]);
        *reinterpret_cast<uint4*>(xrot + (row0 + r) * h + c8) = o;
      }
      if (xq != nullptr) {
        uint2 o;
        o.x = quant4(f[0], f[1], f[2], f[3], inv);
        o.y = quant4(f[4], f[5], f[6], f[7], inv);
        *reinterpret_cast<uint2*>(xq + (row0 + r) * h + c8) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split rotation for decode-size inputs: one wave per 128-channel group and
// MR rows (M <= MR <= 16; rows past M repeat row M-1 and are not stored), so
// the K/128 groups run on K/128 waves spread over the chip and every
// parameter byte is read once.  Writes the rotated rows (fp16 when
// materialized in fp16, else fp32) and each row's absmax per group; the
// GEMM that follows derives the token scale and quantizes.  One wave per
// workgroup: the waves share nothing, and single-wave workgroups spread over
// more CUs sooner (decode layer at M = 1: 43.5 -> 42.0 us against four waves
// per workgroup, 42.4 us with two).
// ---------------------------------------------------------------------------
constexpr int kSplitWaves = 1;

// With the RMSNorm prologue and one row per wave, WPB = kSplitNormWaves
// waves per workgroup take WPB consecutive groups of the row and share its
// sum of squares: wave w sums the chunk classes w, w + WPB, ... of the row,
// the eight partials meet in LDS and every wave adds them in the fixed order,
// which gives the bits a single wave gets summing the whole row, with 1/WPB
// of the loads per wave.  Four waves: against one wave per workgroup summing
// the whole row, the 36-layer verify block (M = 16) 2.160 -> 2.120 ms and the
// fused decode chain (M = 1) 1.550 -> 1.533 ms; eight waves 2.130 / 1.552 ms
// (fewer CUs at M = 1), two 2.128 / 1.533 ms.
constexpr int kSplitNormWaves = 4;

template <int DT, int KP, bool MAT16, int MR, bool NORM, int WPB = kSplitWaves>
__global__ __launch_bounds__(WPB * 64) void rotate_split_kernel(const void* __restrict__ x, const pq::RotGroup grp,
                                                                int M, int h, int krot, unsigned flags,
                                                                const pq::NormArgs nm) {
  constexpr bool kCoop = WPB > 1;
  static_assert(WPB == 1 || (pqd::kSumClasses % WPB == 0 && MR == 1 && NORM),
                "shared row sums: one row per wave, RMSNorm prologue");
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = blockIdx.x * WPB + wv;
  const pq::RotMember& mb = grp.mem[blockIdx.y];
  // the normalized rows and the residual sum are the same for every member: member 0 writes them
  const bool first = blockIdx.y == 0;
  // grid.z: chunks of MR rows; the row pointers move to the chunk's first row
  const int row0 = blockIdx.z * MR;
  const int64_t e0 = static_cast<int64_t>(row0) * h;
  constexpr int xsz = DT == PQ_F32 ? 4 : 2;
  auto at = [](const void* p, int64_t bytes) -> void* {
    return p == nullptr ? nullptr : const_cast<char*>(static_cast<const char*>(p)) + bytes;
  };
  float rinv = -1.0f;
  if constexpr (kCoop) {
    if (nm.mode == PQ_PRO_RMSNORM) {   // uniform over the launch
      constexpr int NC = pqd::kSumClasses / WPB;
      __shared__ float s_part[pqd::kSumClasses][64];
      float pw[NC];
      pqd::row_sumsq_part<DT, NC, NC >= 4 ? 1 : 4 / NC>(at(x, e0 * xsz), at(nm.res, e0 * xsz), 0, h, lane, wv, WPB,
                                                         pw);
#pragma unroll
      for (int j = 0; j < NC; ++j) s_part[wv + j * WPB][lane] = pw[j];
      pqd::lds_barrier();
      float p[pqd::kSumClasses];
#pragma unroll
      for (int c = 0; c < pqd::kSumClasses; ++c) p[c] = s_part[c][lane];
      rinv = pqd::rms_inv(pqd::row_sumsq_total(p), h, nm.eps);
    }
  }
  if (g >= (h >> 7)) return;   // whole waves, after the workgroup's only barrier
  pqd::rotate_group_rows<DT, KP, MAT16, MR, NORM>(
      at(x, e0 * xsz), mb.rot_idx, mb.rot_cs, mb.scales, at(mb.out, e0 * (MAT16 ? 2 : 4)),
      mb.out_scale + static_cast<int64_t>(row0) * (h >> 7), min(MR, M - row0), h, krot, flags, g, lane,
      at(nm.res, e0 * xsz), nm.w, first ? at(nm.h_out, e0 * xsz) : nullptr, first ? at(nm.s_out, e0 * xsz) : nullptr,
      nm.eps, nm.mode, rinv);
}

// Per-token int8 quantization of the split rotation's rows, for token counts
// where the GEMM should not re-derive it in every workgroup.  grid (chunks of
// 2048 channels, rows, members); each thread quantizes 8 channels.  The token
// absmax is the largest group maximum in the unsigned order of its bits (the
// maxima are >= 0), as the rotated decode GEMM takes it, so both give the
// same codes and scales.
template <bool MAT16>
__global__ __launch_bounds__(256) void quant_split_kernel(const pq::QuantGroup grp, int h) {
  const pq::QuantMember& mb = grp.mem[blockIdx.z];
  const int row = blockIdx.y;
  const int G = h >> 7;
  const int lane = threadIdx.x & 63;
  const int c8 = (blockIdx.x * 256 + threadIdx.x) * 8;
  // the thread's 8 values are requested together with the group maxima (one
  // memory round trip, not two); threads past h re-read the row's last 8
  const int64_t o = static_cast<int64_t>(row) * h + min(c8, h - 8);
  uint4 v16;
  float4 va, vb;
  if constexpr (MAT16) {
    v16 = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(mb.xr) + o);
  } else {
    va = *reinterpret_cast<const float4*>(static_cast<const float*>(mb.xr) + o);
    vb = *reinterpret_cast<const float4*>(static_cast<const float*>(mb.xr) + o + 4);
  }
  const float* gm = mb.gmax + static_cast<int64_t>(row) * G;
  uint32_t u = 0;
  // Up to 128 groups (k <= 16384 on every caller): two maxima per lane,
  // requested together, with clamped indices (a repeated maximum changes
  // nothing); a loop over them waited for each before requesting the next.
  if (G <= 128) {
    u = max(__float_as_uint(gm[min(lane, G - 1)]), __float_as_uint(gm[min(lane + 64, G - 1)]));
  } else {
    for (int i = lane; i < G; i += 64) u = max(u, __float_as_uint(gm[i]));
  }
  const float am = __uint_as_float(pq_wave_umax(u));
  if (c8 >= h) return;
  const float inv = pqd::inv_scale(am);
  uint2 q;
  if constexpr (MAT16) {
    q.x = pqd::quant4_f16(v16.x, v16.y, inv);
    q.y = pqd::quant4_f16(v16.z, v16.w, inv);
  } else {
    q.x = pqd::quant4(va.x, va.y, va.z, va.w, inv);
    q.y = pqd::quant4(vb.x, vb.y, vb.z, vb.w, inv);
  }
  *reinterpret_cast<uint2*>(mb.xq + o) = q;
  if (c8 == 0) mb.xscale[row] = am / 127.0f;
}

template <int DT, int KP, bool MAT16, bool NORM>
void launch_split_kp(const void* x, const pq::RotGroup& grp, int M, int h, int krot, unsigned flags,
                     const pq::NormArgs& nm, int rows_per_wave, hipStream_t stream) {
  const int rows = rows_per_wave > 0 && rows_per_wave < M ? rows_per_wave : M;
  if constexpr (NORM) {
    if (rows == 1 && nm.mode == PQ_PRO_RMSNORM) {
      constexpr int W = kSplitNormWaves;
      const dim3 grid(static_cast<unsigned>((h / 128 + W - 1) / W), static_cast<unsigned>(grp.count),
                      static_cast<unsigned>(M));
      rotate_split_kernel<DT, KP, MAT16, 1, true, W><<<grid, W * 64, 0, stream>>>(x, grp, M, h, krot, flags, nm);
      return;
    }
  }
  const dim3 grid(static_cast<unsigned>((h / 128 + kSplitWaves - 1) / kSplitWaves), static_cast<unsigned>(grp.count),
                  static_cast<unsigned>((M + rows - 1) / rows));
#define PQ_SPLIT(MR_)                                                                                      \
  if (rows <= MR_) {                                                                                       \
    rotate_split_kernel<DT, KP, MAT16, MR_, NORM><<<grid, kSplitWaves * 64, 0, stream>>>(x, grp, M, h, krot, \
                                                                                        flags, nm);          \
    return;                                                                                                \
  }
  PQ_SPLIT(1) PQ_SPLIT(2) PQ_SPLIT(4) PQ_SPLIT(8) PQ_SPLIT(16)
#undef PQ_SPLIT
}

template <int DT, bool NORM>
void launch_split_norm(const void* x, const pq::RotGroup& grp, int M, int h, int krot, unsigned flags,
                       const pq::NormArgs& nm, int rpw, hipStream_t stream) {
  const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
  if (krot <= 8) {
    if (mat16) launch_split_kp<DT, 8, true, NORM>(x, grp, M, h, krot, flags, nm, rpw, stream);
    else launch_split_kp<DT, 8, false, NORM>(x, grp, M, h, krot, flags, nm, rpw, stream);
  } else {
    if (mat16) launch_split_kp<DT, 16, true, NORM>(x, grp, M, h, krot, flags, nm, rpw, stream);
    else launch_split_kp<DT, 16, false, NORM>(x, grp, M, h, krot, flags, nm, rpw, stream);
  }
}

template <int DT>
void launch_split_dt(const void* x, const pq::RotGroup& grp, int M, int h, int krot, unsigned flags,
                     const pq::NormArgs* norm, int rpw, hipStream_t stream) {
  if (norm != nullptr) launch_split_norm<DT, true>(x, grp, M, h, krot, flags, *norm, rpw, stream);
  else launch_split_norm<DT, false>(x, grp, M, h, krot, flags, pq::NormArgs{}, rpw, stream);
}

// Per-token quant of an existing activation: absmax pass, then quant pass.
template <int DT, int NT>
__global__ __launch_bounds__(NT) void quant_kernel(const void* __restrict__ x, int8_t* __restrict__ xq,
                                                   float* __restrict__ xscale, int64_t rows, int h) {
  __shared__ float red[NT / 64];
  const int t = threadIdx.x;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t rbase = row * h;
    float amax = 0.0f;
    for (int v = t; v < (h >> 3); v += NT) {
      float f[8];
      load8<DT>(x, rbase + 8 * v, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
    }
    const float am = block_max<NT>(amax, red);
    const float inv = pqd::inv_scale(am);
    if (t == 0) xscale[row] = am / 127.0f;
    for (int v = t; v < (h >> 3); v += NT) {
      float f[8];
      load8<DT>(x, rbase + 8 * v, f);
      uint2 o;
      o.x = quant4(f[0], f[1], f[2], f[3], inv);
      o.y = quant4(f[4], f[5], f[6], f[7], inv);
      *reinterpret_cast<uint2*>(xq + rbase + 8 * v) = o;
    }
    __syncthreads();
  }
}

template <int DT, int G, bool SCALE>
void launch_rotate(const void* x, void* y, uint8_t* sc, const int16_t* idx, const void* theta, const void* scales,
                   int64_t rows, int h, int krot, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>((rows + kRotRows - 1) / kRotRows), static_cast<unsigned>((h + 127) / 128));
  if (sc != nullptr)
    rotate_kernel<DT, G, SCALE, true><<<grid, kRotWaves * 64, 0, stream>>>(x, y, sc, idx, theta, scales, rows, h, krot);
  else
    rotate_kernel<DT, G, SCALE, false><<<grid, kRotWaves * 64, 0, stream>>>(x, y, sc, idx, theta, scales, rows, h,
                                                                            krot);
}

// sc == nullptr: rotated values into y; else MXFP4 codes into y, scales into sc.
template <int DT>
void launch_rotate_dt(const void* x, void* y, uint8_t* sc, const int16_t* idx, const void* theta,
                      const void* scales, int64_t rows, int h, int krot, int group, hipStream_t stream) {
  if (group == 128) {
    if (scales) launch_rotate<DT, 128, true>(x, y, sc, idx, theta, scales, rows, h, krot, stream);
    else launch_rotate<DT, 128, false>(x, y, sc, idx, theta, scales, rows, h, krot, stream);
  } else {
    if (scales) launch_rotate<DT, 64, true>(x, y, sc, idx, theta, scales, rows, h, krot, stream);
    else launch_rotate<DT, 64, false>(x, y, sc, idx, theta, scales, rows, h, krot, stream);
  }
}

constexpr int64_t kMaxGrid = 1 << 20;

// Rows per block: more rows per block read the parameters fewer times, fewer
// keep enough blocks in flight; the row buffer stays within 96 KB.  Two rows
// up to 2048 rows (K = 4096, M = 1264: 15.4 -> 13.8 us against four), four
// from there (M = 3072: 21.8 us against 24.4 us with two, 28.7 us with eight),
// eight from 4096.  The fp16-row kernel from 2048 rows chooses by how its
// blocks fill the chip (rq_rows_fp16).
inline int rq_rows_per_block(int64_t rows, int h, bool mat16) {
  int rb = rows >= 4096 ? 8 : rows >= 2048 ? 4 : rows >= 256 ? 2 : 1;
  while (rb > 1 && static_cast<int64_t>(rb) * h * (mat16 ? 2 : 4) > 96 * 1024) rb >>= 1;
  return rb;
}

template <int DT, int KP, bool MAT16, int RB, bool NORM, int OUT, int IN>
void launch_rq_rb(const void* x, const pq::RotGroup& grp, int64_t row_begin, int64_t nblocks, int h, int krot,
                  unsigned flags, const pq::NormArgs& nm, hipStream_t stream) {
  if (nblocks <= 0) return;
  const size_t lds = static_cast<size_t>(RB) * h * (MAT16 ? 2 : 4);
  const dim3 grid(static_cast<unsigned>(nblocks), static_cast<unsigned>(grp.count));
  rotate_quant_kernel<DT, KP, MAT16, RB, NORM, OUT, IN><<<grid, kRQWaves * 64, lds, stream>>>(x, grp, row_begin,
                                                                                              h, krot, flags, nm);
}

// The device's CU count and LDS bytes per CU (queried once; 0 if unknown).
struct CuInfo {
  int cus = 0;
  int lds = 0;
};
inline CuInfo cu_info() {
  static const CuInfo info = [] {
    CuInfo c;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&c.lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess)
      c = CuInfo{};
    return c;
  }();
  return info;
}

// Blocks of one fp16-row instance that registers and waves allow per CU
// (the runtime's occupancy calculator without the row buffer), queried once.
template <int DT, int KP, int RB, bool NORM, int IN>
int rq_blocks_per_cu_regs() {
  static const int n = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, rotate_quant_kernel<DT, KP, true, RB, NORM, kRqInt8, IN>,
                                                     kRQWaves * 64, 0) != hipSuccess)
      b = 0;
    return b;
  }();
  return n;
}

// Rows per block of the fp16-row kernel from 2048 rows: every block of a
// launch is equal work, so the launch takes as many rounds as its blocks
// fill on the chip (CUs x blocks per CU), and a part-filled last round costs
// nearly a full one.  Among 8, 6, 4, 3 and 2 rows, with at least two blocks
// (16 waves) per CU and a row buffer within 96 KB, take the one whose blocks
// fill their rounds best; a smaller one only when it fills them better by
// more than 2 %, since more rows per block read the layer parameters fewer
// times.  At 3072 rows: 6 rows for K = 4096 (512 blocks, one round: 21.4 ->
// 21.2 us; the prefill layer 0.871 / 0.880 -> 0.857 / 0.860 ms), 3 for
// K = 12288 (2 rounds of 2 blocks per CU: 58.0 / 58.8 -> 51.5 / 51.6 us
// against 4 rows, whose 96 KB row buffer leaves one block per CU).
template <int DT, int KP, bool NORM, int IN>
int rq_rows_fp16(int64_t rows, int h, int members) {
  const CuInfo ci = cu_info();
  if (rows < 2048 || ci.cus <= 0 || ci.lds <= 0) return rq_rows_per_block(rows, h, true);
  const int cand[5] = {8, 6, 4, 3, 2};
  const int regs[5] = {rq_blocks_per_cu_regs<DT, KP, 8, NORM, IN>(), rq_blocks_per_cu_regs<DT, KP, 6, NORM, IN>(),
                       rq_blocks_per_cu_regs<DT, KP, 4, NORM, IN>(), rq_blocks_per_cu_regs<DT, KP, 3, NORM, IN>(),
                       rq_blocks_per_cu_regs<DT, KP, 2, NORM, IN>()};
  int best = 0;
  double best_fill = -1.0;
  for (int i = 0; i < 5; ++i) {
    const int64_t lds = static_cast<int64_t>(cand[i]) * h * 2;
    if (lds > 96 * 1024) continue;
    const int64_t per_cu = std::min<int64_t>(regs[i], ci.lds / (lds + 1024));   // + the static LDS
    if (per_cu < 2) continue;
    const int64_t blocks = rows / cand[i] * members;
    const int64_t cap = per_cu * ci.cus;
    const int64_t rounds = (blocks + cap - 1) / cap;
    const double fill = static_cast<double>(blocks) / static_cast<double>(rounds * cap);
    if (fill > best_fill + 0.02) {
      best = cand[i];
      best_fill = fill;
    }
  }
  return best > 0 ? best : rq_rows_per_block(rows, h, true);
}

template <int DT, int KP, bool MAT16, bool NORM, int OUT, int IN>
void launch_rq_in(const void* x, const pq::RotGroup& grp, int64_t rows, int h, int krot, unsigned flags,
                  const pq::NormArgs& nm, hipStream_t stream) {
  int rb = 0;
  if constexpr (MAT16) rb = rq_rows_fp16<DT, KP, NORM, IN>(rows, h, grp.count);
  else rb = rq_rows_per_block(rows, h, false);
  const int64_t full = rows / rb;
  switch (rb) {
    case 8: launch_rq_rb<DT, KP, MAT16, 8, NORM, OUT, IN>(x, grp, 0, full, h, krot, flags, nm, stream); break;
    case 4: launch_rq_rb<DT, KP, MAT16, 4, NORM, OUT, IN>(x, grp, 0, full, h, krot, flags, nm, stream); break;
    case 2: launch_rq_rb<DT, KP, MAT16, 2, NORM, OUT, IN>(x, grp, 0, full, h, krot, flags, nm, stream); break;
    case 6:
      if constexpr (MAT16) launch_rq_rb<DT, KP, MAT16, 6, NORM, OUT, IN>(x, grp, 0, full, h, krot, flags, nm, stream);
      break;
    case 3:
      if constexpr (MAT16) launch_rq_rb<DT, KP, MAT16, 3, NORM, OUT, IN>(x, grp, 0, full, h, krot, flags, nm, stream);
      break;
    default: break;
  }
  const int64_t done = rb > 1 ? full * rb : 0;   // the remaining rows, one block each
  launch_rq_rb<DT, KP, MAT16, 1, NORM, OUT, IN>(x, grp, done, rows - done, h, krot, flags, nm, stream);
}

// The input treatment as a compile-time choice: an fp16 input is already
// fp16 (its prologue rounds to x's dtype as well), a bfloat16 one gets an
// instance per flag value, float32 reads the flag at run time.  The plain and
// MXFP4 outputs take no flags.
template <int DT, int KP, bool MAT16, bool NORM, int OUT = kRqInt8>
void launch_rq(const void* x, const pq::RotGroup& grp, int64_t rows, int h, int krot, unsigned flags,
               const pq::NormArgs& nm, hipStream_t stream) {
  if constexpr (OUT != kRqInt8 || DT == PQ_F16) {
    launch_rq_in<DT, KP, MAT16, NORM, OUT, kInAsIs>(x, grp, rows, h, krot, flags, nm, stream);
  } else if constexpr (DT == PQ_BF16) {
    if (flags & PQ_RQ_INPUT_FP16) launch_rq_in<DT, KP, MAT16, NORM, OUT, kInF16>(x, grp, rows, h, krot, flags, nm, stream);
    else launch_rq_in<DT, KP, MAT16, NORM, OUT, kInAsIs>(x, grp, rows, h, krot, flags, nm, stream);
  } else {
    launch_rq_in<DT, KP, MAT16, NORM, OUT, kInFlag>(x, grp, rows, h, krot, flags, nm, stream);
  }
}

// The register-chain rotation of whole rows with a plain (OUT = kRqRows) or
// MXFP4 (kRqMxfp4) output, on packed operands.
template <int DT, int OUT>
void launch_rotate_rows_dt(const void* x, const pq::RotGroup& grp, int64_t rows, int h, int krot,
                           hipStream_t stream) {
  if (krot <= 8) launch_rq<DT, 8, false, false, OUT>(x, grp, rows, h, krot, 0u, pq::NormArgs{}, stream);
  else launch_rq<DT, 16, false, false, OUT>(x, grp, rows, h, krot, 0u, pq::NormArgs{}, stream);
}

template <int DT, bool NORM>
void launch_rotate_quant_norm(const void* x, const pq::RotGroup& grp, int64_t rows, int h, int krot,
                              unsigned flags, const pq::NormArgs& nm, hipStream_t stream) {
  const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
  if (krot <= 8) {
    if (mat16) launch_rq<DT, 8, true, NORM>(x, grp, rows, h, krot, flags, nm, stream);
    else launch_rq<DT, 8, false, NORM>(x, grp, rows, h, krot, flags, nm, stream);
  } else {
    if (mat16) launch_rq<DT, 16, true, NORM>(x, grp, rows, h, krot, flags, nm, stream);
    else launch_rq<DT, 16, false, NORM>(x, grp, rows, h, krot, flags, nm, stream);
  }
}

template <int DT>
void launch_rotate_quant(const void* x, const pq::RotGroup& grp, int64_t rows, int h, int krot, unsigned flags,
                         const pq::NormArgs* norm, hipStream_t stream) {
  if (norm != nullptr) launch_rotate_quant_norm<DT, true>(x, grp, rows, h, krot, flags, *norm, stream);
  else launch_rotate_quant_norm<DT, false>(x, grp, rows, h, krot, flags, pq::NormArgs{}, stream);
}

template <int DT>
void launch_quant(const void* x, int8_t* xq, float* xscale, int64_t rows, int h, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(rows < kMaxGrid ? rows : kMaxGrid);
  quant_kernel<DT, 256><<<grid, 256, 0, stream>>>(x, xq, xscale, rows, h);
}

}  // namespace

namespace pq {
void launch_rotate_split(const void* x, int x_dtype, const RotGroup& grp, int m, int h, int krot, unsigned flags,
                         hipStream_t stream, const NormArgs* norm, int rows_per_wave) {
  switch (x_dtype) {
    case PQ_F32: launch_split_dt<PQ_F32>(x, grp, m, h, krot, flags, norm, rows_per_wave, stream); break;
    case PQ_F16: launch_split_dt<PQ_F16>(x, grp, m, h, krot, flags, norm, rows_per_wave, stream); break;
    default: launch_split_dt<PQ_BF16>(x, grp, m, h, krot, flags, norm, rows_per_wave, stream); break;
  }
}

void launch_quant_split(const QuantGroup& grp, int m, int h, bool mat16, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((h / 8 + 255) / 256), static_cast<unsigned>(m), static_cast<unsigned>(grp.count));
  if (mat16) quant_split_kernel<true><<<grid, 256, 0, stream>>>(grp, h);
  else quant_split_kernel<false><<<grid, 256, 0, stream>>>(grp, h);
}

void launch_rotate_quant_group(const void* x, int x_dtype, const RotGroup& grp, int64_t rows, int h, int krot,
                               unsigned flags, hipStream_t stream, const NormArgs* norm) {
  switch (x_dtype) {
    case PQ_F32: launch_rotate_quant<PQ_F32>(x, grp, rows, h, krot, flags, norm, stream); break;
    case PQ_F16: launch_rotate_quant<PQ_F16>(x, grp, rows, h, krot, flags, norm, stream); break;
    default: launch_rotate_quant<PQ_BF16>(x, grp, rows, h, krot, flags, norm, stream); break;
  }
}
}  // namespace pq

extern "C" int pq_rotate(const void* x, void* y, const int16_t* idx_ij, const void* theta, const void* scales,
                         int64_t rows, int64_t h, int krot, int group_size, int dtype, void* stream) {
  PQ_REQUIRE(rows >= 0 && h > 0, PQ_ERR_ARG, "pq_rotate: rows=%lld h=%lld", (long long)rows, (long long)h);
  PQ_REQUIRE(group_size == 64 || group_size == 128, PQ_ERR_UNSUPPORTED,
             "pq_rotate: Unexpected group_size: %d (supported: 64, 128)", group_size);
  PQ_REQUIRE(krot == 1 || krot == 2 || krot == 4 || krot == 8 || krot == 16, PQ_ERR_UNSUPPORTED,
             "pq_rotate: Unsupported KROT = %d; compiled variants: 1/2/4/8/16", krot);
  PQ_REQUIRE(h % group_size == 0, PQ_ERR_ARG, "pq_rotate: h must be divisible by GROUP_SIZE (h=%lld, G=%d)",
             (long long)h, group_size);
  PQ_REQUIRE(h <= (1 << 24), PQ_ERR_ARG, "pq_rotate: h=%lld too large", (long long)h);
  PQ_REQUIRE(dtype == PQ_F32 || dtype == PQ_F16 || dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_rotate: rotate only supports Float, Half, and BFloat16 (dtype code %d)", dtype);
  if (rows == 0) return PQ_OK;
  PQ_REQUIRE(x && y && idx_ij && theta, PQ_ERR_ARG, "pq_rotate: null pointer");
  PQ_REQUIRE((rows + kRotRows - 1) / kRotRows <= 0x7fffffffLL, PQ_ERR_ARG, "pq_rotate: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(h);
  switch (dtype) {
    case PQ_F32: launch_rotate_dt<PQ_F32>(x, y, nullptr, idx_ij, theta, scales, rows, hh, krot, group_size, s); break;
    case PQ_F16: launch_rotate_dt<PQ_F16>(x, y, nullptr, idx_ij, theta, scales, rows, hh, krot, group_size, s); break;
    default: launch_rotate_dt<PQ_BF16>(x, y, nullptr, idx_ij, theta, scales, rows, hh, krot, group_size, s); break;
  }
  return pq::launch_status("pq_rotate launch");
}

// rotation::rotate followed by OCP MXFP4 quantization of the float32 result,
// in one pass.  The CDNA4 counterpart of the reference's NVFP4
// rotation::rotate_and_quant (kernels/paroquant_kernels/src/rotation.cu:62-111,
// 230-315): the same rotation, a different block format (32-element blocks,
// E8M0 scales, no second-level scale).
extern "C" int pq_rotate_mxfp4(const void* x, uint8_t* q_out, uint8_t* scale_out, const int16_t* idx_ij,
                               const void* theta, const void* scales, int64_t rows, int64_t h, int krot,
                               int group_size, int dtype, void* stream) {
  PQ_REQUIRE(rows >= 0 && h > 0, PQ_ERR_ARG, "pq_rotate_mxfp4: rows=%lld h=%lld", (long long)rows, (long long)h);
  PQ_REQUIRE(group_size == 64 || group_size == 128, PQ_ERR_UNSUPPORTED,
             "pq_rotate_mxfp4: Unexpected group_size: %d (supported: 64, 128)", group_size);
  PQ_REQUIRE(krot == 1 || krot == 2 || krot == 4 || krot == 8 || krot == 16, PQ_ERR_UNSUPPORTED,
             "pq_rotate_mxfp4: Unsupported KROT = %d; compiled variants: 1/2/4/8/16", krot);
  PQ_REQUIRE(h % group_size == 0, PQ_ERR_ARG, "pq_rotate_mxfp4: h must be divisible by GROUP_SIZE (h=%lld, G=%d)",
             (long long)h, group_size);
  PQ_REQUIRE(h <= (1 << 24), PQ_ERR_ARG, "pq_rotate_mxfp4: h=%lld too large", (long long)h);
  PQ_REQUIRE(dtype == PQ_F32 || dtype == PQ_F16 || dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_rotate_mxfp4: dtype code %d (Float, Half or BFloat16)", dtype);
  if (rows == 0) return PQ_OK;
  PQ_REQUIRE(x && q_out && scale_out && idx_ij && theta, PQ_ERR_ARG, "pq_rotate_mxfp4: null pointer");
  PQ_REQUIRE(pq::aligned_to(q_out, 4), PQ_ERR_ARG, "pq_rotate_mxfp4: q_out must be 4-byte aligned");
  PQ_REQUIRE((rows + kRotRows - 1) / kRotRows <= 0x7fffffffLL, PQ_ERR_ARG, "pq_rotate_mxfp4: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(h);
  switch (dtype) {
    case PQ_F32:
      launch_rotate_dt<PQ_F32>(x, q_out, scale_out, idx_ij, theta, scales, rows, hh, krot, group_size, s);
      break;
    case PQ_F16:
      launch_rotate_dt<PQ_F16>(x, q_out, scale_out, idx_ij, theta, scales, rows, hh, krot, group_size, s);
      break;
    default:
      launch_rotate_dt<PQ_BF16>(x, q_out, scale_out, idx_ij, theta, scales, rows, hh, krot, group_size, s);
      break;
  }
  return pq::launch_status("pq_rotate_mxfp4 launch");
}

// rotation::rotate / rotation::rotate_and_quant_mxfp4 on packed operands
// (pq_rotation_pack): the register-chain rotation of the fused kernels,
// whole rows per workgroup.  Its cos/sin are the packed float32 values the
// host derives in float64, as pq_rotate's kernel derives them on the device,
// and its layer arithmetic is the same, so the results equal pq_rotate's /
// pq_rotate_mxfp4's for the pairs and angles the operands were packed from.
extern "C" int pq_rotate_rows(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                              const float* scales, void* out, uint8_t* mx_scales, int64_t rows, int64_t h, int krot,
                              int out_mode, void* stream) {
  PQ_REQUIRE(rows >= 0 && rows <= 0x7fffffffLL && h > 0 && h % 128 == 0 && h <= 16384, PQ_ERR_ARG,
             "pq_rotate_rows: need h %% 128 == 0 and 0 < h <= 16384 (h=%lld, rows=%lld)", (long long)h,
             (long long)rows);
  PQ_REQUIRE(krot >= 1 && krot <= 16, PQ_ERR_UNSUPPORTED, "pq_rotate_rows: krot=%d not in 1..16", krot);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_rotate_rows: x dtype code %d", x_dtype);
  PQ_REQUIRE(out_mode == PQ_ROWS_SAME || out_mode == PQ_ROWS_MXFP4, PQ_ERR_ARG, "pq_rotate_rows: out_mode %d",
             out_mode);
  if (rows == 0) return PQ_OK;
  PQ_REQUIRE(x && rot_idx && rot_cs && out && (out_mode != PQ_ROWS_MXFP4 || mx_scales), PQ_ERR_ARG,
             "pq_rotate_rows: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(rot_idx, 16) && pq::aligned_to(rot_cs, 16) &&
                 pq::aligned_to(out, 16),
             PQ_ERR_ARG, "pq_rotate_rows: x, rot_idx, rot_cs and out must be 16-byte aligned");
  pq::RotGroup grp{};
  grp.count = 1;
  grp.mem[0] = {rot_idx, rot_cs, scales, out, nullptr, mx_scales};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(h);
  if (out_mode == PQ_ROWS_SAME) {
    switch (x_dtype) {
      case PQ_F32: launch_rotate_rows_dt<PQ_F32, kRqRows>(x, grp, rows, hh, krot, s); break;
      case PQ_F16: launch_rotate_rows_dt<PQ_F16, kRqRows>(x, grp, rows, hh, krot, s); break;
      default: launch_rotate_rows_dt<PQ_BF16, kRqRows>(x, grp, rows, hh, krot, s); break;
    }
  } else {
    switch (x_dtype) {
      case PQ_F32: launch_rotate_rows_dt<PQ_F32, kRqMxfp4>(x, grp, rows, hh, krot, s); break;
      case PQ_F16: launch_rotate_rows_dt<PQ_F16, kRqMxfp4>(x, grp, rows, hh, krot, s); break;
      default: launch_rotate_rows_dt<PQ_BF16, kRqMxfp4>(x, grp, rows, hh, krot, s); break;
    }
  }
  return pq::launch_status("pq_rotate_rows launch");
}

extern "C" int pq_rotate_quant_i8(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                                  const float* scales, int8_t* xq, float* xscale, void* xrot, int64_t rows,
                                  int64_t h, int krot, unsigned flags, void* stream) {
  PQ_REQUIRE(rows >= 0 && rows <= 0x7fffffffLL && h > 0 && h % 128 == 0 && h <= 16384, PQ_ERR_ARG,
             "pq_rotate_quant_i8: need h %% 128 == 0 and 0 < h <= 16384 (h=%lld, rows=%lld)", (long long)h,
             (long long)rows);
  PQ_REQUIRE(krot >= 1 && krot <= 16, PQ_ERR_UNSUPPORTED, "pq_rotate_quant_i8: krot=%d not in 1..16", krot);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_rotate_quant_i8: dtype code %d", x_dtype);
  PQ_REQUIRE((flags & ~(PQ_RQ_INPUT_FP16 | PQ_RQ_MATERIALIZE_FP16)) == 0, PQ_ERR_ARG,
             "pq_rotate_quant_i8: unknown flags 0x%x", flags);
  if (rows == 0) return PQ_OK;
  PQ_REQUIRE(x && rot_idx && rot_cs && xq && xscale, PQ_ERR_ARG, "pq_rotate_quant_i8: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(xq, 8) && pq::aligned_to(rot_idx, 16) &&
                 pq::aligned_to(rot_cs, 16) && (xrot == nullptr || pq::aligned_to(xrot, 16)),
             PQ_ERR_ARG,
             "pq_rotate_quant_i8: x, rot_idx, rot_cs and xrot must be 16-byte aligned, xq 8-byte aligned");
  pq::RotGroup grp{};
  grp.count = 1;
  grp.mem[0] = {rot_idx, rot_cs, scales, xq, xscale, xrot};
  pq::launch_rotate_quant_group(x, x_dtype, grp, rows, static_cast<int>(h), krot, flags,
                                static_cast<hipStream_t>(stream));
  return pq::launch_status("pq_rotate_quant_i8 launch");
}

extern "C" int pq_quant_i8(const void* x, int x_dtype, int8_t* xq, float* xscale, int64_t rows, int64_t h,
                           void* stream) {
  PQ_REQUIRE(rows >= 0 && h > 0 && h % 8 == 0 && h <= (1 << 24), PQ_ERR_ARG,
             "pq_quant_i8: need h %% 8 == 0 (h=%lld)", (long long)h);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "pq_quant_i8: dtype code %d", x_dtype);
  if (rows == 0) return PQ_OK;
  PQ_REQUIRE(x && xq && xscale, PQ_ERR_ARG, "pq_quant_i8: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(xq, 8), PQ_ERR_ARG,
             "pq_quant_i8: x must be 16-byte and xq 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(h);
  switch (x_dtype) {
    case PQ_F32: launch_quant<PQ_F32>(x, xq, xscale, rows, hh, s); break;
    case PQ_F16: launch_quant<PQ_F16>(x, xq, xscale, rows, hh, s); break;
    default: launch_quant<PQ_BF16>(x, xq, xscale, rows, hh, s); break;
  }
  return pq::launch_status("pq_quant_i8 launch");
}
