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
#include <type_traits>

#include "pq_device.h"

using pqd::quant4;

namespace {

constexpr int kRotRows = 4;   // rows per workgroup of the plain rotation kernel

#define PQ_LDS_WAVE_FENCE() __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local")

// ---------------------------------------------------------------------------
// rotation::rotate.  One wave per (4 rows x 128 channels); lane t owns pair t
// of the chunk (for group 64 the chunk holds two groups).  The 4 x 128 fp32
// tile lives in LDS; pairs are read per layer and masked to the group so a
// bad index can never address outside the tile.
// ---------------------------------------------------------------------------
template <int DT, int G, bool SCALE>
__global__ __launch_bounds__(64) void rotate_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                    const int16_t* __restrict__ idx,
                                                    const void* __restrict__ theta,
                                                    const void* __restrict__ scales, int64_t rows,
                                                    int h, int krot) {
  __shared__ float tile[kRotRows][128];
  const int t = threadIdx.x;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRotRows;
  const int ch0 = blockIdx.y * 128;

#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int local = t + 64 * half;
    const int ch = ch0 + local;
    float s = 1.0f;
    if (SCALE && ch < h) s = pq_load_as_f32<DT>(scales, ch);
#pragma unroll
    for (int r = 0; r < kRotRows; ++r) {
      const int64_t row = row0 + r;
      float v = 0.0f;
      if (row < rows && ch < h) v = pq_load_as_f32<DT>(x, row * h + ch) * s;
      tile[r][local] = v;
    }
  }

  const int P = blockIdx.y * 64 + t;  // pair index within the row; theta column
  const bool active = P < (h >> 1);
  const int gi = P / (G / 2);
  const int pp = P % (G / 2);
  const int base = gi * G - ch0;  // group start inside the 128-channel tile
  __syncthreads();

  for (int r = 0; r < krot; ++r) {
    if (active) {
      const int64_t o = static_cast<int64_t>(r) * h + gi * G + 2 * pp;
      const int i = base + (idx[o] & (G - 1));
      const int j = base + (idx[o + 1] & (G - 1));
      const float th = pq_load_as_f32<DT>(theta, static_cast<int64_t>(r) * (h >> 1) + P);
      float sn, cs;
      sincosf(th, &sn, &cs);
#pragma unroll
      for (int rr = 0; rr < kRotRows; ++rr) {
        const float xi = tile[rr][i];
        const float xj = tile[rr][j];
        tile[rr][i] = fmaf(xi, cs, xj * sn);
        tile[rr][j] = fmaf(xj, cs, -(xi * sn));
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int local = t + 64 * half;
    const int ch = ch0 + local;
#pragma unroll
    for (int r = 0; r < kRotRows; ++r) {
      const int64_t row = row0 + r;
      if (row < rows && ch < h) pq_store_from_f32<DT>(y, row * h + ch, tile[r][local]);
    }
  }
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  constexpr int NW = NT / 64;
  v = pq_wave_max(v);
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


// One lane's packed rotation parameters for one group: KP layers of
// (first | second << 8) in 16-byte words and of (cos, sin).  Layout (built by
// pq_rotation_pack): rot_ij [G][64][KP] uint16, rot_cs [G][64][KP][2] float.
template <int KP>
struct LaneParams {
  uint32_t ij[KP / 2];
  float cs[2 * KP];
};

template <int KP>
__device__ __forceinline__ void load_lane_params(const uint16_t* __restrict__ rot_ij, const float* __restrict__ rot_cs,
                                                 int g, int lane, LaneParams<KP>& p) {
  const int64_t o = (static_cast<int64_t>(g) * 64 + lane) * KP;
  const uint4* ij = reinterpret_cast<const uint4*>(rot_ij + o);
#pragma unroll
  for (int q = 0; q < KP / 8; ++q) {
    const uint4 v = ij[q];
    p.ij[4 * q] = v.x;
    p.ij[4 * q + 1] = v.y;
    p.ij[4 * q + 2] = v.z;
    p.ij[4 * q + 3] = v.w;
  }
  const float4* cs = reinterpret_cast<const float4*>(rot_cs + 2 * o);
#pragma unroll
  for (int q = 0; q < KP / 2; ++q) {
    const float4 v = cs[q];
    p.cs[4 * q] = v.x;
    p.cs[4 * q + 1] = v.y;
    p.cs[4 * q + 2] = v.z;
    p.cs[4 * q + 3] = v.w;
  }
}

template <int KP>
__device__ __forceinline__ int pair_first(const LaneParams<KP>& p, int r) {
  return (p.ij[r >> 1] >> (16 * (r & 1))) & 127;
}
template <int KP>
__device__ __forceinline__ int pair_second(const LaneParams<KP>& p, int r) {
  return (p.ij[r >> 1] >> (16 * (r & 1) + 8)) & 127;
}

// ---------------------------------------------------------------------------
// Fused rotate + quant over blocks of RB rows (RB a compile-time constant:
// the RB rows are RB independent LDS chains per layer, with no per-row
// branches).  512 threads; wave w rotates groups w, w+8, ... for the block's
// rows in a private fp32 scratch [RB][128] (lane t owns the pair the packed
// parameters give it; the packed order makes each layer's LDS accesses
// bank-conflict free) and stores the finished values in a row buffer
// [RB][h] (fp16 when the result is materialized in fp16, fp32 otherwise).
// The next group's parameters and inputs are requested before the current
// group's layers run.  After a block-wide absmax per row the row buffer is
// quantized with coalesced stores.  Parameters are read once per group per
// RB rows.
// ---------------------------------------------------------------------------
constexpr int kRQWaves = 8;

template <int DT, int KP, bool MAT16, int RB>
__global__ __launch_bounds__(kRQWaves * 64) void rotate_quant_kernel(
    const void* __restrict__ x, const uint16_t* __restrict__ rot_ij, const float* __restrict__ rot_cs,
    const float* __restrict__ scales, int8_t* __restrict__ xq, float* __restrict__ xscale,
    uint16_t* __restrict__ xrot, int64_t row_begin, int h, int krot, unsigned flags) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  __shared__ float red[kRQWaves][RB];
  using RowT = typename std::conditional<MAT16, uint16_t, float>::type;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  const bool in16 = (flags & PQ_RQ_INPUT_FP16) != 0;
  const int G = h >> 7;
  float* scratch = reinterpret_cast<float*>(lds_raw) + w * (RB * 128);
  RowT* rowbuf = reinterpret_cast<RowT*>(lds_raw + kRQWaves * RB * 128 * sizeof(float));
  const int64_t row0 = row_begin + static_cast<int64_t>(blockIdx.x) * RB;

  float rmax[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) rmax[r] = 0.0f;

  LaneParams<KP> cur, nxt;
  float xa[RB], xb[RB], xan[RB], xbn[RB];
  float sa = 1.0f, sb = 1.0f, san = 1.0f, sbn = 1.0f;
  auto load_inputs = [&](int g, float (&va)[RB], float (&vb)[RB], float& s0, float& s1) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      va[r] = pq_load_as_f32<DT>(x, (row0 + r) * h + g * 128 + lane);
      vb[r] = pq_load_as_f32<DT>(x, (row0 + r) * h + g * 128 + 64 + lane);
    }
    if (scales != nullptr) {
      s0 = scales[g * 128 + lane];
      s1 = scales[g * 128 + 64 + lane];
    }
  };

  if (w < G) {
    load_lane_params<KP>(rot_ij, rot_cs, w, lane, cur);
    load_inputs(w, xa, xb, sa, sb);
  }
  for (int g = w; g < G; g += kRQWaves) {
    const int gn = (g + kRQWaves < G) ? g + kRQWaves : g;   // clamped: the loads stay unconditional
    load_lane_params<KP>(rot_ij, rot_cs, gn, lane, nxt);
    load_inputs(gn, xan, xbn, san, sbn);

#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const float a = in16 ? pq_round_f16(xa[r]) : xa[r];
      const float b = in16 ? pq_round_f16(xb[r]) : xb[r];
      scratch[r * 128 + lane] = a * sa;
      scratch[r * 128 + 64 + lane] = b * sb;
    }
    PQ_LDS_WAVE_FENCE();
    float ni[RB], nj[RB];
    int i = 0, j = 0;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      if (k < krot) {
        i = pair_first(cur, k);
        j = pair_second(cur, k);
        const float c = cur.cs[2 * k], sn = cur.cs[2 * k + 1];
        float xi[RB], xj[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          xi[r] = scratch[r * 128 + i];
          xj[r] = scratch[r * 128 + j];
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          pqd::givens(xi[r], xj[r], c, sn, ni[r], nj[r]);
          scratch[r * 128 + i] = ni[r];
          scratch[r * 128 + j] = nj[r];
        }
        PQ_LDS_WAVE_FENCE();
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float vi = ni[r], vj = nj[r];
      if constexpr (MAT16) {
        const uint16_t hi = pq_f32_to_f16(vi), hj = pq_f32_to_f16(vj);
        rowbuf[r * h + g * 128 + i] = hi;
        rowbuf[r * h + g * 128 + j] = hj;
        vi = pq_f16_to_f32(hi);
        vj = pq_f16_to_f32(hj);
      } else {
        rowbuf[r * h + g * 128 + i] = vi;
        rowbuf[r * h + g * 128 + j] = vj;
      }
      rmax[r] = fmaxf(rmax[r], fmaxf(fabsf(vi), fabsf(vj)));
    }
    cur = nxt;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      xa[r] = xan[r];
      xb[r] = xbn[r];
    }
    sa = san;
    sb = sbn;
  }

#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const float v = pq_wave_max(rmax[r]);
    if (lane == 0) red[w][r] = v;
  }
  __syncthreads();

  // Quantize the row buffer: 8 elements per thread per step.
  const int per_row = h >> 3;
  for (int e = t; e < RB * per_row; e += kRQWaves * 64) {
    const int r = e / per_row;
    const int c8 = (e - r * per_row) * 8;
    float am = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kRQWaves; ++ww) am = fmaxf(am, red[ww][r]);
    const float inv = pqd::inv_scale(am);
    float f[8];
    if constexpr (MAT16) {
      const uint4 u = *reinterpret_cast<const uint4*>(rowbuf + r * h + c8);
      const uint32_t wds[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = pq_f16_to_f32(static_cast<uint16_t>(wds[q] & 0xffffu));
        f[2 * q + 1] = pq_f16_to_f32(static_cast<uint16_t>(wds[q] >> 16));
      }
      if (xrot != nullptr) *reinterpret_cast<uint4*>(xrot + (row0 + r) * h + c8) = u;
    } else {
      const float4 a = *reinterpret_cast<const float4*>(rowbuf + r * h + c8);
      const float4 b = *reinterpret_cast<const float4*>(rowbuf + r * h + c8 + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
      if (xrot != nullptr) {
        uint4 o;
        o.x = pq_f32_to_f16(f[0]) | (static_cast<uint32_t>(pq_f32_to_f16(f[1])) << 16);
        o.y = pq_f32_to_f16(f[2]) | (static_cast<uint32_t>(pq_f32_to_f16(f[3])) << 16);
        o.z = pq_f32_to_f16(f[4]) | (static_cast<uint32_t>(pq_f32_to_f16(f[5])) << 16);
        o.w = pq_f32_to_f16(f[6]) | (static_cast<uint32_t>(pq_f32_to_f16(f[7])) << 16);
        *reinterpret_cast<uint4*>(xrot + (row0 + r) * h + c8) = o;
      }
    }
    uint2 o;
    o.x = quant4(f[0], f[1], f[2], f[3], inv);
    o.y = quant4(f[4], f[5], f[6], f[7], inv);
    *reinterpret_cast<uint2*>(xq + (row0 + r) * h + c8) = o;
    if (c8 == 0) xscale[row0 + r] = am / 127.0f;
  }
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
void launch_rotate(const void* x, void* y, const int16_t* idx, const void* theta, const void* scales,
                   int64_t rows, int h, int krot, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>((rows + kRotRows - 1) / kRotRows), static_cast<unsigned>((h + 127) / 128));
  rotate_kernel<DT, G, SCALE><<<grid, 64, 0, stream>>>(x, y, idx, theta, scales, rows, h, krot);
}

template <int DT>
void launch_rotate_dt(const void* x, void* y, const int16_t* idx, const void* theta, const void* scales,
                      int64_t rows, int h, int krot, int group, hipStream_t stream) {
  if (group == 128) {
    if (scales) launch_rotate<DT, 128, true>(x, y, idx, theta, scales, rows, h, krot, stream);
    else launch_rotate<DT, 128, false>(x, y, idx, theta, scales, rows, h, krot, stream);
  } else {
    if (scales) launch_rotate<DT, 64, true>(x, y, idx, theta, scales, rows, h, krot, stream);
    else launch_rotate<DT, 64, false>(x, y, idx, theta, scales, rows, h, krot, stream);
  }
}

constexpr int64_t kMaxGrid = 1 << 20;

// Rows per block: more rows per block read the parameters fewer times, fewer
// keep enough blocks in flight; the row buffer stays within 96 KB.
inline int rq_rows_per_block(int64_t rows, int h, bool mat16) {
  int rb = rows >= 4096 ? 8 : rows >= 1024 ? 4 : rows >= 256 ? 2 : 1;
  while (rb > 1 && static_cast<int64_t>(rb) * h * (mat16 ? 2 : 4) > 96 * 1024) rb >>= 1;
  return rb;
}

template <int DT, int KP, bool MAT16, int RB>
void launch_rq_rb(const void* x, const uint16_t* rot_ij, const float* rot_cs, const float* scales, int8_t* xq,
                  float* xscale, void* xrot, int64_t row_begin, int64_t nblocks, int h, int krot, unsigned flags,
                  hipStream_t stream) {
  if (nblocks <= 0) return;
  const size_t lds = static_cast<size_t>(kRQWaves) * RB * 128 * sizeof(float) +
                     static_cast<size_t>(RB) * h * (MAT16 ? 2 : 4);
  rotate_quant_kernel<DT, KP, MAT16, RB><<<static_cast<unsigned>(nblocks), kRQWaves * 64, lds, stream>>>(
      x, rot_ij, rot_cs, scales, xq, xscale, static_cast<uint16_t*>(xrot), row_begin, h, krot, flags);
}

template <int DT, int KP, bool MAT16>
void launch_rq(const void* x, const uint16_t* rot_ij, const float* rot_cs, const float* scales, int8_t* xq,
               float* xscale, void* xrot, int64_t rows, int h, int krot, unsigned flags, hipStream_t stream) {
  const int rb = rq_rows_per_block(rows, h, MAT16);
  const int64_t full = rows / rb;
  switch (rb) {
    case 8: launch_rq_rb<DT, KP, MAT16, 8>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, 0, full, h, krot, flags, stream); break;
    case 4: launch_rq_rb<DT, KP, MAT16, 4>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, 0, full, h, krot, flags, stream); break;
    case 2: launch_rq_rb<DT, KP, MAT16, 2>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, 0, full, h, krot, flags, stream); break;
    default: break;
  }
  const int64_t done = rb > 1 ? full * rb : 0;   // the remaining rows, one block each
  launch_rq_rb<DT, KP, MAT16, 1>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, done, rows - done, h, krot, flags,
                                 stream);
}

template <int DT>
void launch_rotate_quant(const void* x, const uint16_t* rot_ij, const float* rot_cs, const float* scales, int8_t* xq,
                         float* xscale, void* xrot, int64_t rows, int h, int krot, unsigned flags,
                         hipStream_t stream) {
  const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
  if (krot <= 8) {
    if (mat16) launch_rq<DT, 8, true>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, h, krot, flags, stream);
    else launch_rq<DT, 8, false>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, h, krot, flags, stream);
  } else {
    if (mat16) launch_rq<DT, 16, true>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, h, krot, flags, stream);
    else launch_rq<DT, 16, false>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, h, krot, flags, stream);
  }
}

template <int DT>
void launch_quant(const void* x, int8_t* xq, float* xscale, int64_t rows, int h, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(rows < kMaxGrid ? rows : kMaxGrid);
  quant_kernel<DT, 256><<<grid, 256, 0, stream>>>(x, xq, xscale, rows, h);
}

}  // namespace

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
    case PQ_F32: launch_rotate_dt<PQ_F32>(x, y, idx_ij, theta, scales, rows, hh, krot, group_size, s); break;
    case PQ_F16: launch_rotate_dt<PQ_F16>(x, y, idx_ij, theta, scales, rows, hh, krot, group_size, s); break;
    default: launch_rotate_dt<PQ_BF16>(x, y, idx_ij, theta, scales, rows, hh, krot, group_size, s); break;
  }
  return pq::launch_status("pq_rotate launch");
}

extern "C" int pq_rotate_quant_i8(const void* x, int x_dtype, const uint16_t* rot_ij, const float* rot_cs,
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
  PQ_REQUIRE(x && rot_ij && rot_cs && xq && xscale, PQ_ERR_ARG, "pq_rotate_quant_i8: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(xq, 8) && pq::aligned_to(rot_ij, 16) &&
                 pq::aligned_to(rot_cs, 16) && (xrot == nullptr || pq::aligned_to(xrot, 16)),
             PQ_ERR_ARG,
             "pq_rotate_quant_i8: x, rot_ij, rot_cs and xrot must be 16-byte aligned, xq 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(h);
  switch (x_dtype) {
    case PQ_F32: launch_rotate_quant<PQ_F32>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, hh, krot, flags, s); break;
    case PQ_F16: launch_rotate_quant<PQ_F16>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, hh, krot, flags, s); break;
    default: launch_rotate_quant<PQ_BF16>(x, rot_ij, rot_cs, scales, xq, xscale, xrot, rows, hh, krot, flags, s); break;
  }
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
