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
// Unpacking, prefill kernel: a dword of 8 codes becomes two dwords of 4
// signed bytes (q - z) by ((w & 0x0f0f0f0f) + (0x80808080 - z*0x01010101))
// ^ 0x80808080 -- every byte stays in [113, 143] before the xor, so no carry
// crosses a byte, and the xor maps 128 + d to the two's complement of d.
// Decode kernel: the codes go in as plain nibbles q and the zero point as
// two more MFMAs against bytes of -z, which adds -z * sum_k a exactly.
//
// Two kernels:
//   gemm_skinny  M <= 64: each wave streams 1 KB weight blocks (one 16-column
//                tile x one 128-group) with 16-byte loads, four
//                v_mfma_i32_16x16x64_i8 per block (activation rows padded to
//                16; 17-64 rows on int8 A run as two to four row blocks of 16
//                in every workgroup, so the weights stream once); the
//                waves of a workgroup split K and add their partial sums in
//                LDS in a fixed order.
//   gemm_prefill M > 64: 192x256, 128x256, 128x128, 64x128 or 32x128 output
//                tiles (by the measured cost of rounds of 256 workgroups), 8 (or 4) waves
//                side by side along n, operands copied from global memory
//                straight into a 3-stage LDS ring, v_mfma_i32_32x32x32_i8
//                tiles, the output staged through LDS for 16-byte stores;
//                the 192x256 tiles run their 32-row tiles in pairs, scaling
//                the previous pair's partials under the current pair's MFMAs.
#include <type_traits>

#include "pq_device.h"
#include "pq_internal.h"

using namespace pqd;

namespace {

// ---------------------------------------------------------------------------
// Decode-size GEMM (M <= 16 per launch row block; int8 A up to 64 rows)
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
// first batch of weight loads is issued before that prologue.  3 / 4 = one /
// two fp16 rotated rows (K <= 16384) plus their group maxima, quantized in
// registers: every wave takes the token scales from the maxima (DPP maxima,
// no barrier), quantizes a dword of 4 codes per lane for two (group, row)
// slots at a time (lanes 0-31 one, 32-63 the other) and gathers its A
// fragments from them with ds_bpermute: no LDS image, no barrier before the
// first MFMA.
constexpr int kSkinnyRows = 16;

// The member of a group that owns workgroup tile `unit` (members own
// contiguous runs of tiles; the lookup is wave-uniform).
__device__ __forceinline__ int group_member(const pq::GemmGroup& grp, int unit) {
  int mi = 0;
#pragma unroll
  for (int i = 1; i < pq::kMaxGroup; ++i)
    if (i < grp.count && unit >= grp.first[i]) mi = i;
  return mi;
}

template <int NT, int W, int U, bool PARTIALS, int AQ, int RB = 1>
__global__ __launch_bounds__(W * 64, (W == 4 && NT == 1 && !PARTIALS) ? 3 : 1) void gemm_skinny(
    const pq::GemmGroup grp, int bias_dtype, int y_dtype, int M, int K) {
  __shared__ float red[W][NT][4][64];
  __shared__ float s_amax[kSkinnyRows];
  extern __shared__ __attribute__((aligned(16))) int8_t aq[];
  const int mi = group_member(grp, blockIdx.x);
  const pq::GemmMember& mb = grp.mem[mi];
  // RB > 1 (int8 A, 17-64 rows): the workgroup carries RB row blocks of 16
  // (block b: rows 16b .. 16b + 15, rows past M repeating row M - 1) as RB
  // MFMA chains on every weight fragment, so the weights stream once.
  // Separate instances, so that launches of up to 16 rows keep their code.
  static_assert(RB == 1 || AQ == 0, "row blocks on int8 A only");
  static_assert(RB >= 1 && RB <= 4, "up to 64 rows");
  const int8_t* __restrict__ xq = mb.xq;
  const float* __restrict__ xs = mb.xs;
  const void* __restrict__ xr = mb.xr;
  const float* __restrict__ gmax = mb.gmax;
  const uint8_t* __restrict__ wpack = mb.wpack;
  const uint32_t* __restrict__ wmeta = mb.wmeta;
  const void* __restrict__ bias = mb.bias;
  const int N = mb.n;
  void* __restrict__ y = mb.y;
  const int G = K >> 7;
  int32_t* __restrict__ partials = mb.partials;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int j = lane >> 4;
  const bool arow = c < M;
  const int astride = K + 16;
  const int tile0 = (blockIdx.x - grp.first[mi]) * NT;

  float acc[RB][NT][4];
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[b][nt][v] = 0.0f;

  const int8_t* ap = xq + static_cast<int64_t>(arow ? c : 0) * K + j * 32;
  // the further row blocks' rows
  const int8_t* apb[RB > 1 ? RB - 1 : 1];
#pragma unroll
  for (int b = 1; b < RB; ++b) apb[b - 1] = xq + static_cast<int64_t>(min(b * kSkinnyRows + c, M - 1)) * K + j * 32;
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
  // AQ 3 / 4: A quantized in registers, MQ = 1 / 2 rows
  constexpr bool kRegA = AQ == 3 || AQ == 4;
  constexpr int MQ = AQ == 4 ? 2 : 1;
  static_assert(!kRegA || RB == 1, "one row block");
  // the larger of the lane's group maxima (G <= 128): one row over the wave
  // (two per lane), or row lane / 32 over each half-wave (four per lane)
  uint32_t gm3 = 0;
  if constexpr (AQ == 3) {
    gm3 = max(__float_as_uint(gmax[min(lane, G - 1)]), __float_as_uint(gmax[min(lane + 64, G - 1)]));
  } else if constexpr (AQ == 4) {
    const float* gr = gmax + (lane >> 5) * G;
    const int l32 = lane & 31;
    gm3 = max(max(__float_as_uint(gr[min(l32, G - 1)]), __float_as_uint(gr[min(l32 + 32, G - 1)])),
              max(__float_as_uint(gr[min(l32 + 64, G - 1)]), __float_as_uint(gr[min(l32 + 96, G - 1)])));
  }
  // All of these loads are unconditional, with clamped indices (their values
  // are used only where the index is in range): behind a branch, the
  // compiler's wait before their first use also waited for the weight
  // blocks issued after them, which put the whole prologue behind the
  // weights' round trip.
  if constexpr (AQ == 1 || AQ == 2) {
#pragma unroll
    for (int q = 0; q < kPreMax; ++q) gm[q] = gmax[min(static_cast<int>(threadIdx.x) + q * nthr, M * G - 1)];
    preloaded = M * k8 <= kPre * nthr;
#pragma unroll
    for (int q = 0; q < kPre; ++q) {
      const int e = min(static_cast<int>(threadIdx.x) + q * nthr, M * k8 - 1);
      const int r = e / k8;
      const int c8 = (e - r * k8) * 8;
      if constexpr (AQ == 1) {
        pre[q][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xr) + static_cast<int64_t>(r) * K + c8);
      } else {
        const uint4* src =
            reinterpret_cast<const uint4*>(static_cast<const float*>(xr) + static_cast<int64_t>(r) * K + c8);
        pre[q][0] = src[0];
        pre[q][AQ == 2 ? 1 : 0] = src[1];
      }
    }
  }

  // Every wave runs the same number of batches (a batch past G loads
  // nothing), so the prologue's barriers are reached by all waves.
  const int batches = (G + W * U - 1) / (W * U);
  // One batch of U groups per wave; batch 0 (which holds the prologue) is
  // peeled off the loop, so the common single-batch case has no back edge
  // (the compiler otherwise waits for earlier loads before reusing registers).
  // Register A: a batch's (group u, row m) slots s = u * MQ + m go two to a
  // quantizer round, round r taking slots 2 r (lanes 0-31) and 2 r + 1 (lanes
  // 32-63); lane l quantizes codes 4 (l & 31) .. + 3 of its slot from 8 bytes
  // of the fp16 row (clamped, unconditional).  The first kPreB batches' bytes
  // are requested at once, ahead of the first weights; later batches request
  // theirs ahead of their own weights.
  constexpr int QR = (U * MQ + 1) / 2;
  float am3 = 0.0f, inv3 = 0.0f, am3b = 0.0f, inv3b = 0.0f;   // rows 0 and 1
  constexpr int kPreB = kRegA ? 4 : 1;
  auto load_ah = [&](const int it, uint2 (&ah)[QR]) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int sl = 2 * r + (lane >> 5);
      const int g = min(wave + it * W * U + W * min(sl / MQ, U - 1), G - 1);
      ah[r] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(xr) + (sl % MQ) * K + g * 128 +
                                              4 * (lane & 31));
    }
  };
  uint2 ahp[kPreB][QR];
  if constexpr (kRegA) {
#pragma unroll
    for (int b = 0; b < kPreB; ++b) load_ah(b, ahp[b]);
  }
  // PB: the batch's index into ahp when it is a constant below kPreB, else -1
  auto run_batch = [&](const int it, auto pb) {
    constexpr int PB = decltype(pb)::value;
    const int g0 = wave + it * W * U;
    v4i wb[U][NT];
    uint32_t wm[U][NT];
    v4i a0[U], a1[U];
    v4i a0b[RB > 1 ? RB - 1 : 1][U], a1b[RB > 1 ? RB - 1 : 1][U];   // the further row blocks' fragments
    uint2 ah[QR];
    if constexpr (kRegA) {
      if constexpr (PB >= 0) {
#pragma unroll
        for (int r = 0; r < QR; ++r) ah[r] = ahp[PB][r];
      } else {
        load_ah(it, ah);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // with the AQ prologue, a group past G loads group G-1 (unused) rather
      // than branching around the loads (see the prologue); without it the
      // branch measured faster
      const int g = AQ != 0 ? min(g0 + W * u, G - 1) : g0 + W * u;
      if (AQ != 0 || g < G) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int64_t blk = static_cast<int64_t>(tile0 + nt) * G + g;
          // Weights are read once per step: non-temporal loads keep them
          // from evicting what is re-read (rotation operands, activations)
          // from L2 and the Infinity Cache.
          wb[u][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wpack + blk * 1024 + lane * 16));
          wm[u][nt] = __builtin_nontemporal_load(wmeta + blk * 16 + c);
        }
        if constexpr (AQ == 0) {
          // Unconditional (rows >= M read row 0 and are zeroed at use): a
          // branch around the loads would make the compiler wait early.
          a0[u] = *reinterpret_cast<const v4i*>(ap + static_cast<int64_t>(g) * 128);
          a1[u] = *reinterpret_cast<const v4i*>(ap + static_cast<int64_t>(g) * 128 + 16);
#pragma unroll
          for (int b = 1; b < RB; ++b) {
            a0b[b - 1][u] = *reinterpret_cast<const v4i*>(apb[b - 1] + static_cast<int64_t>(g) * 128);
            a1b[b - 1][u] = *reinterpret_cast<const v4i*>(apb[b - 1] + static_cast<int64_t>(g) * 128 + 16);
          }
        }
      }
    }
    uint32_t qd[QR];
    if constexpr (kRegA) {
      if (it == 0) {   // the token scales, the same in every wave (maxima >= 0: unsigned order)
        if constexpr (MQ == 1) {
          am3 = __uint_as_float(pq_wave_umax(gm3));
        } else {
          // the first five steps of the wave maximum leave lanes 0-31's in lane 31, 32-63's in lane 63
          uint32_t u5 = pq_dpp_umax<0xb1, 0xf>(gm3);
          u5 = pq_dpp_umax<0x4e, 0xf>(u5);
          u5 = pq_dpp_umax<0x141, 0xf>(u5);
          u5 = pq_dpp_umax<0x140, 0xf>(u5);
          u5 = pq_dpp_umax<0x142, 0xa>(u5);
          am3 = __uint_as_float(__builtin_amdgcn_readlane(static_cast<int>(u5), 31));
          am3b = __uint_as_float(__builtin_amdgcn_readlane(static_cast<int>(u5), 63));
          inv3b = inv_scale(am3b);
        }
        inv3 = inv_scale(am3);
      }
      // a lane's slots all lie in row (lane / 32) % MQ
      const float inv_l = MQ == 2 && (lane >> 5) ? inv3b : inv3;
#pragma unroll
      for (int r = 0; r < QR; ++r) qd[r] = quant4_f16(ah[r].x, ah[r].y, inv_l);
      if constexpr (PARTIALS) {
        // Parity form: the member's first workgroup writes the codes and the token scales it multiplies.
        if (blockIdx.x == static_cast<unsigned>(grp.first[mi])) {
#pragma unroll
          for (int r = 0; r < QR; ++r) {
            const int sl = 2 * r + (lane >> 5), uu = sl / MQ, g = g0 + W * uu;
            if (uu < U && g < G)
              *reinterpret_cast<uint32_t*>(mb.a_out + (sl % MQ) * K + g * 128 + 4 * (lane & 31)) = qd[r];
          }
          if (it == 0 && threadIdx.x == 0) {
            mb.as_out[0] = am3 / 127.0f;
            if (MQ == 2) mb.as_out[1] = am3b / 127.0f;
          }
        }
      }
    }
    if constexpr (AQ == 1 || AQ == 2) {
      if (it == 0) {
        // Part 2: token scales, then the int8 image of A in LDS.
        if (threadIdx.x < kSkinnyRows) s_amax[threadIdx.x] = 0.0f;
        lds_barrier();
#pragma unroll
        for (int q = 0; q < kPreMax; ++q) {   // absmax >= 0: unsigned order is float order
          const int i = threadIdx.x + q * nthr;
          if (i < M * G) atomicMax(reinterpret_cast<unsigned*>(&s_amax[i / G]), __float_as_uint(gm[q]));
        }
        for (int i = threadIdx.x + kPreMax * nthr; i < M * G; i += nthr)
          atomicMax(reinterpret_cast<unsigned*>(&s_amax[i / G]), __float_as_uint(gmax[i]));
        lds_barrier();
        auto quant8 = [&](int e, const uint4* v) {
          const int r = e / k8;
          const int c8 = (e - r * k8) * 8;
          const float inv = inv_scale(s_amax[r]);
          uint2 o;
          if constexpr (AQ == 1) {
            o.x = quant4_f16(v[0].x, v[0].y, inv);
            o.y = quant4_f16(v[0].z, v[0].w, inv);
          } else {
            const uint4 b = v[AQ == 2 ? 1 : 0];
            o.x = quant4(__uint_as_float(v[0].x), __uint_as_float(v[0].y), __uint_as_float(v[0].z),
                         __uint_as_float(v[0].w), inv);
            o.y = quant4(__uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w), inv);
          }
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
        lds_barrier();
        if constexpr (PARTIALS) {
          // Parity form: the member's first workgroup also writes the A
          // operand it multiplies -- the int8 image just built in LDS -- and
          // the token scales its epilogue would apply.
          if (blockIdx.x == static_cast<unsigned>(grp.first[mi])) {
            const int c16s = K >> 4;
            for (int e = threadIdx.x; e < M * c16s; e += nthr) {
              const int r = e / c16s;
              const int c16 = (e - r * c16s) * 16;
              *reinterpret_cast<uint4*>(mb.a_out + static_cast<int64_t>(r) * K + c16) =
                  *reinterpret_cast<const uint4*>(aq + r * astride + c16);
            }
            if (static_cast<int>(threadIdx.x) < M) mb.as_out[threadIdx.x] = s_amax[threadIdx.x] / 127.0f;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g0 + W * u;
      // register A multiplies a group past G too (its clamped operands,
      // scaled by 0): behind this branch the compiler moved the batch's
      // weight loads down to their use, after the quantization
      if (kRegA || g < G) {
        if constexpr (AQ == 1 || AQ == 2) {   // A from the LDS image, next to its use
          a0[u] = *reinterpret_cast<const v4i*>(al + g * 128);
          a1[u] = *reinterpret_cast<const v4i*>(al + g * 128 + 16);
        } else if constexpr (kRegA) {
          // codes j*32 .. j*32+31 of group u, row c (rows past MQ repeat the last): dwords 8j .. 8j+7 of
          // the lanes that quantized slot u * MQ + row, all in round (u * MQ) / 2 (g is wave-uniform
          // here, so every lane takes part)
          const int sl = u * MQ + min(c, MQ - 1);
          const int src = ((sl & 1) * 32 + 8 * j) * 4;
          const int v = static_cast<int>(qd[(u * MQ) >> 1]);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            a0[u][q] = __builtin_amdgcn_ds_bpermute(src + 4 * q, v);
            a1[u][q] = __builtin_amdgcn_ds_bpermute(src + 16 + 4 * q, v);
          }
        }
        // Rows past M hold a copy of a real row: MFMA rows are independent
        // and those results are never stored, so they need no masking.
        const v4i av0 = a0[u], av1 = a1[u];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t meta = wm[u][nt];
          const v4i w = wb[u][nt];
          // sum a * (q - z) = sum a * q + sum a * (-z): the codes go in as
          // plain nibbles, the zero point as two more MFMAs on a constant
          // -z operand (cheaper in VALU than biasing every byte).
          const v4i b0 = nibbles16(static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y));
          const v4i b1 = nibbles16(static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w));
          const int nz = static_cast<int>(meta_neg_zero4(meta));
          const v4i bz = {nz, nz, nz, nz};
          v4i p[RB];
#pragma unroll
          for (int b = 0; b < RB; ++b) {   // the row blocks share the weight fragment
            const v4i x0 = b == 0 ? av0 : a0b[b > 0 ? b - 1 : 0][u], x1 = b == 0 ? av1 : a1b[b > 0 ? b - 1 : 0][u];
            p[b] = v4i{0, 0, 0, 0};
            p[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, b0, p[b], 0, 0, 0);
            p[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, b1, p[b], 0, 0, 0);
            p[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, bz, p[b], 0, 0, 0);
            p[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, bz, p[b], 0, 0, 0);
          }
          if constexpr (PARTIALS) {
#pragma unroll
            for (int b = 0; b < RB; ++b)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int m = b * kSkinnyRows + 4 * j + v;
                if (m < M && g < G)
                  partials[(static_cast<int64_t>(m) * G + g) * N + (tile0 + nt) * 16 + c] = p[b][v];
              }
          } else {
            const float sc = !kRegA || g < G ? meta_scale(meta) : 0.0f;
#pragma unroll
            for (int b = 0; b < RB; ++b)
#pragma unroll
              for (int v = 0; v < 4; ++v) acc[b][nt][v] = fmaf(static_cast<float>(p[b][v]), sc, acc[b][nt][v]);
          }
        }
      }
    }
  };
  using First = std::integral_constant<int, 0>;
  using Later = std::integral_constant<int, -1>;
  run_batch(0, First{});
  if constexpr (kRegA) {
    if (batches > 1) run_batch(1, std::integral_constant<int, 1>{});
    if (batches > 2) run_batch(2, std::integral_constant<int, 2>{});
    if (batches > 3) run_batch(3, std::integral_constant<int, 3>{});
    for (int it = kPreB; it < batches; ++it) run_batch(it, Later{});
  } else {
    for (int it = 1; it < batches; ++it) run_batch(it, Later{});
  }
  if constexpr (PARTIALS) return;

  // the row blocks one after the other through the same LDS
#pragma unroll
  for (int b = 0; b < RB; ++b) {
    if (b > 0) __syncthreads();   // the previous block's sums are read
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][nt][v][lane] = acc[b][nt][v];
    __syncthreads();
    for (int t = threadIdx.x; t < NT * 256; t += W * 64) {
      const int nt = t >> 8;
      const int rv = (t >> 6) & 3;
      const int rl = t & 63;
      const int m = b * kSkinnyRows + 4 * (rl >> 4) + rv;
      if (m >= M) continue;
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) sum += red[w][nt][rv][rl];
      const int n = (tile0 + nt) * 16 + (rl & 15);
      const float xsm = kRegA ? (m == 0 ? am3 : am3b) / 127.0f : AQ != 0 ? s_amax[m] / 127.0f : xs[m];
      pq_store_dyn(y, y_dtype, static_cast<int64_t>(m) * N + n, epilogue(sum, xsm, bias, bias_dtype, n));
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill-size GEMM (M > 64)
//
// Workgroup tile BM x BN; WM x WN waves, each a (BM/WM) x (BN/WN) block of
// TM x TN 32 x 32 tiles (v_mfma_i32_32x32x32_i8).  The operands of one K
// group -- A as BM rows of 128 int8, B as BN/16 packed 1 KB blocks, and BN
// metadata words -- go straight from global memory to LDS (global_load_lds,
// no register staging) into a 3-stage ring, so the loads of group g+2 are in
// flight while group g is computed.  Every wave issues the same number of
// loads per stage, so "stage g has landed" is one vmcnt wait plus a barrier.
// A rows keep their 16-byte chunks XOR-swizzled by row and B blocks sit at a
// 1152-byte stride, which keeps the fragment reads free of bank conflicts.
// B is unpacked to signed int8 (q - z) in registers at use.  After each
// group the int32 tiles are scaled by the group's fp16 scales into fp32
// accumulators.  The waves sit side by side along n (WM = 1): each B tile is
// then unpacked by one wave only -- the unpack and the per-group scaling
// are the kernel's VALU load, which bounds it (without packed fp32 the
// scaling alone costs as many VALU cycles as the int8 MFMAs of the group).
// ---------------------------------------------------------------------------
constexpr int kPfStages = 3;
constexpr int kPfGroupM = 4;   // tile rows walked together by one XCD's run of tiles
constexpr int kPfBStride = 1024 + 128;

// Wait until at most `ahead` groups of copies (L copies each) are in flight.
template <int L, int A>
__device__ __forceinline__ void wait_groups(int ahead) {
  if constexpr (A == 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= A) wait_vmcnt<L * A>();
    else wait_groups<L, A - 1>(ahead);
  }
}

template <int BM, int BN, int WM, int WN, bool PARTIALS, int ST = kPfStages, bool TP = false>
__global__ __launch_bounds__(WM * WN * 64) void gemm_prefill(
    const pq::GemmGroup grp, int bias_dtype, int y_dtype, int M, int K) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int A_BYTES = BM * 128;                 // BM/8 blocks of 1 KB (8 rows each)
  constexpr int B_BYTES = (BN / 16) * kPfBStride;   // BN/16 packed blocks
  constexpr int STAGE = A_BYTES + B_BYTES + BN * 4;
  constexpr int A_LD = BM / 8 / NW, B_LD = BN / 16 / NW, M_LD = 1;   // loads per wave per stage
  constexpr int LOADS = A_LD + B_LD + M_LD;
  static_assert(TM >= 1 && TN >= 1 && BM % (32 * WM) == 0 && BN % (32 * WN) == 0, "tile shape");
  static_assert((BM / 8) % NW == 0 && (BN / 16) % NW == 0 && BN / NW <= 64, "loads split evenly over the waves");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int G = K >> 7;
  const int nbn = grp.first[grp.count];   // BN-wide column tiles of all members
  // Tile order: workgroup b runs on XCD b % 8, so the grid is first cut
  // into 8 contiguous runs of tiles (one per XCD, when the count divides),
  // and each run walks kPfGroupM tile rows at a time, column by column:
  // the tiles one XCD holds at once share A rows and B columns in its L2.
  int t = blockIdx.x;
  if (gridDim.x % 8 == 0) t = (t % 8) * (gridDim.x / 8) + t / 8;
  const int nbm = (M + BM - 1) / BM;
  const int first_bm = t / (kPfGroupM * nbn) * kPfGroupM;
  const int gm = min(nbm - first_bm, kPfGroupM);
  const int bm = first_bm + (t % (kPfGroupM * nbn)) % gm;
  const int bn_all = (t % (kPfGroupM * nbn)) / gm;
  // The member owning this column tile (every member starts on a tile).
  const int mi = group_member(grp, bn_all);
  const pq::GemmMember& mb = grp.mem[mi];
  const int8_t* __restrict__ xq = mb.xq;
  const float* __restrict__ xs = mb.xs;
  const uint8_t* __restrict__ wpack = mb.wpack;
  const uint32_t* __restrict__ wmeta = mb.wmeta;
  const void* __restrict__ bias = mb.bias;
  void* __restrict__ y = mb.y;
  int32_t* __restrict__ partials = mb.partials;
  const int N = mb.n;
  const int ntiles16 = N >> 4;
  const int bn = bn_all - grp.first[mi];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int r32 = lane & 31;
  const int hj = lane >> 5;

  // Sources of this wave's loads (32-bit element offsets; rows past M and
  // blocks past N are clamped, their results are never stored; the host
  // keeps M*K and N*K/2 below 2^31).
  int a_off[A_LD], b_off[B_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int blk = wave * A_LD + i;          // rows 8*blk .. 8*blk+7
    const int row = blk * 8 + (lane >> 3);
    const int q = (lane & 7) ^ pf_swz(row);   // LDS chunk lane&7 of the row holds global chunk q
    a_off[i] = min(bm * BM + row, M - 1) * K + q * 16;
  }
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int blk = wave * B_LD + i;
    b_off[i] = min(bn * (BN / 16) + blk, ntiles16 - 1) * G * 1024 + lane * 16;
  }
  constexpr int MCOLS = BN / NW;   // metadata words per wave
  const int mcol = wave * MCOLS + (lane < MCOLS ? lane : 0);
  const int m_off = min(bn * (BN / 16) + (mcol >> 4), ntiles16 - 1) * G * 16 + (mcol & 15);

  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  auto issue = [&](int g, int stage) {
    const uint32_t base = lds0 + stage * STAGE;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) lds_copy16(xq + a_off[i] + g * 128, base + (wave * A_LD + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_LD; ++i)
      lds_copy16(wpack + b_off[i] + g * 1024, base + A_BYTES + (wave * B_LD + i) * kPfBStride);
    if (lane < MCOLS) lds_copy4(wmeta + m_off + g * 16, base + A_BYTES + B_BYTES + wave * MCOLS * 4);
  };

  float acc[TM][TN][16];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[tm][tn][v] = 0.0f;

  int arow[TM], bcol[TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) arow[tm] = wm * (BM / WM) + tm * 32 + r32;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) bcol[tn] = wn * (BN / WN) + tn * 32 + r32;

  // Matrix work of group g from its stage.  The loads of group ig (= g + 2)
  // are issued after the first two k-steps' MFMAs: issued at the top of the
  // group, right after the barrier, all waves' copies queue up at once in
  // the load path while no MFMA is in flight.
  auto compute = [&](int stage, int g, int ig) {
    const uint8_t* As = smem + stage * STAGE;
    const uint8_t* Bs = As + A_BYTES;
    const uint32_t* Ms = reinterpret_cast<const uint32_t*>(Bs + B_BYTES);
    uint32_t zb[TN];
    float sc[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const uint32_t meta = Ms[bcol[tn]];
      zb[tn] = meta_zero_bias(meta);
      sc[tn] = meta_scale(meta);
    }
    v16i T[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) T[tm][tn] = v16i{};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = hj * 4 + i;   // this lane's 16 k of the step: 16q .. 16q+15
      v4i a[TM], b[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        a[tm] = *reinterpret_cast<const v4i*>(As + arow[tm] * 128 + ((q ^ pf_swz(arow[tm])) << 4));
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        // packed slot (2*hj + i/2)*16 + col%16 of the column's block, bytes (i%2)*8 .. +8
        const uint2 w = *reinterpret_cast<const uint2*>(Bs + (bcol[tn] >> 4) * kPfBStride +
                                                        ((2 * hj + (i >> 1)) * 16 + (bcol[tn] & 15)) * 16 + (i & 1) * 8);
        b[tn] = unpack16(w.x, w.y, zb[tn]);
      }
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          T[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[tm], b[tn], T[tm][tn], 0, 0, 0);
      if (i == 1 && ig < G) issue(ig, ig % ST);
    }
    if constexpr (PARTIALS) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t m = static_cast<int64_t>(bm) * BM + arow[tm] - r32 + 8 * (v >> 2) + 4 * hj + (v & 3);
            const int n = bn * BN + bcol[tn];
            if (m < M && n < N) partials[(m * G + g) * N + n] = T[tm][tn][v];
          }
    } else {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            acc[tm][tn][v] = fmaf(static_cast<float>(T[tm][tn][v]), sc[tn], acc[tm][tn][v]);
    }
  };

  // Tile-pair form of compute (TP): the wave runs its tiles two at a time --
  // the four k-steps of tiles 2p and 2p+1, two independent MFMA chains --
  // and scales the previous pair's partials in between, one MFMA then eight
  // VALU (four converts, four fmas), enforced with sched_group_barrier.
  // Only two pairs of partials are live; the group's B fragments are
  // unpacked once up front.  The PARTIALS instance stores each pair's int32
  // tiles where the other scales them (same MFMA chains and fragments).
  auto store_partials = [&](int tile, int tn, int v, int g, int32_t val) {
    const int64_t m = static_cast<int64_t>(bm) * BM + arow[tile] - r32 + 8 * (v >> 2) + 4 * hj + (v & 3);
    const int n = bn * BN + bcol[tn];
    if (m < M && n < N) partials[(m * G + g) * N + n] = val;
  };
  auto compute_tp = [&](int stage, int g, int ig) {
    static_assert(!TP || TM % 2 == 0, "tiles in pairs");
    const uint8_t* As = smem + stage * STAGE;
    const uint8_t* Bs = As + A_BYTES;
    const uint32_t* Ms = reinterpret_cast<const uint32_t*>(Bs + B_BYTES);
    float sc[TN];
    v4i b[4][TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const uint32_t meta = Ms[bcol[tn]];
      const uint32_t zb = meta_zero_bias(meta);
      sc[tn] = meta_scale(meta);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 w = *reinterpret_cast<const uint2*>(Bs + (bcol[tn] >> 4) * kPfBStride +
                                                        ((2 * hj + (i >> 1)) * 16 + (bcol[tn] & 15)) * 16 + (i & 1) * 8);
        b[i][tn] = unpack16(w.x, w.y, zb);
      }
    }
    // A fragments of the current pair; each k-step's are reloaded for the
    // next pair right after their MFMAs issue (six MFMAs hide the latency)
    v4i a[2][4];
    auto load_frag = [&](int tile, int i) {
      const int r = arow[tile];
      return *reinterpret_cast<const v4i*>(As + r * 128 + (((hj * 4 + i) ^ pf_swz(r)) << 4));
    };
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int i = 0; i < 4; ++i) a[t2][i] = load_frag(t2, i);
    v16i T[2][2][TN];
#pragma unroll
    for (int p = 0; p < TM / 2; ++p) {
      const int cb = p & 1;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) T[cb][t2][tn] = v16i{};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn) {
            T[cb][t2][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[t2][i], b[i][tn], T[cb][t2][tn], 0, 0, 0);
            if (p > 0) {
#pragma unroll
              for (int v = 4 * i; v < 4 * i + 4; ++v) {
                if constexpr (PARTIALS) store_partials(2 * p - 2 + t2, tn, v, g, T[cb ^ 1][t2][tn][v]);
                else
                  acc[2 * p - 2 + t2][tn][v] =
                      fmaf(static_cast<float>(T[cb ^ 1][t2][tn][v]), sc[tn], acc[2 * p - 2 + t2][tn][v]);
              }
            }
          }
        if (p + 1 < TM / 2) {
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2) a[t2][i] = load_frag(2 * p + 2 + t2, i);
        }
      }
      if (!PARTIALS && p > 0) {
#pragma unroll
        for (int q = 0; q < 8 * TN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);   // eight VALU
        }
      }
      if (p == 0 && ig < G) issue(ig, ig % ST);
    }
    constexpr int LP = (TM / 2 - 1) & 1;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          if constexpr (PARTIALS) store_partials(TM - 2 + t2, tn, v, g, T[LP][t2][tn][v]);
          else acc[TM - 2 + t2][tn][v] = fmaf(static_cast<float>(T[LP][t2][tn][v]), sc[tn], acc[TM - 2 + t2][tn][v]);
        }
  };

  // Stage g % ST holds group g; the copies run ST-1 groups ahead.  Before
  // computing g, each wave waits for its own loads of g (those of the later
  // groups may stay in flight), then a barrier makes everybody's loads of g
  // visible and retires everybody's use of the stage that group g+ST-1 is
  // about to overwrite (group g-1's).
  // The tile's activation scales go to LDS past the ring ahead of every
  // other load, so the first wait covers them (the partials mode has none).
  if (!PARTIALS && wave * 64 < BM) {
    const int r = min(wave * 64 + lane, BM - 1);
    lds_copy4(xs + min(bm * BM + r, M - 1), lds0 + ST * STAGE + wave * 256);
  }
  static_assert(LOADS * (ST - 2) < 64, "vmcnt range");
#pragma unroll
  for (int q = 0; q < ST - 1; ++q)
    if (q < G) issue(q, q);
  for (int g = 0; g < G; ++g) {
    wait_groups<LOADS, ST - 2>(min(G - 1 - g, ST - 2));
    __builtin_amdgcn_s_barrier();
    if constexpr (TP) compute_tp(g % ST, g, g + ST - 1);
    else compute(g % ST, g, g + ST - 1);
  }
  if constexpr (PARTIALS) return;

  // Output, one 32-row slice per wave row at a time (WM*32 rows of the
  // tile): the waves write their values in the output type to LDS, then
  // every lane stores 16 contiguous bytes along n, non-temporal (streamed
  // out rather than left dirty in L2 for the end of the kernel to write
  // back).  The row pitch keeps the
  // two half-waves' writes (rows 4 apart) in different banks.  The bias
  // values are loaded once and the output type is a template parameter:
  // a global load or a dtype branch inside the element loop makes the
  // compiler wait for the stores in flight (vmcnt(0)) at every join.
  static_assert(ST * STAGE >= WM * 32 * (BN * 4 + 32), "output slice fits in the stage ring");
  const float* xs_tile = reinterpret_cast<const float*>(smem + ST * STAGE);
  const bool has_bias = bias != nullptr;
  float bv[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
    bv[tn] = has_bias ? pq_load_dyn(bias, bias_dtype, min(bn * BN + bcol[tn], N - 1)) : 0.0f;
  // This lane's activation scales, all read up front: rows 8j + 4hj .. +3 of
  // a 32-row tile are one 16-byte LDS read.  Read per value inside the slice
  // loop, each was an LDS round trip in front of its row's conversions.
  float xsv[TM][16];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 x4 = *reinterpret_cast<const float4*>(xs_tile + wm * (BM / WM) + tm * 32 + 8 * j + 4 * hj);
      xsv[tm][4 * j] = x4.x;
      xsv[tm][4 * j + 1] = x4.y;
      xsv[tm][4 * j + 2] = x4.z;
      xsv[tm][4 * j + 3] = x4.w;
    }
  auto emit = [&](auto out_dtype) {
    constexpr int DT = decltype(out_dtype)::value;
    constexpr int ESZ = DT == PQ_F32 ? 4 : 2;
    constexpr int PITCH = BN * ESZ + 32;
    constexpr int CPR = BN * ESZ / 16;   // 16-byte chunks per staged row
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      lds_barrier();   // the stages (or the previous slice) are no longer read
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = 8 * (v >> 2) + 4 * hj + (v & 3);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          float val = acc[tm][tn][v] * xsv[tm][v];
          if (has_bias) val = val + bv[tn];
          uint8_t* dst = smem + (wm * 32 + r) * PITCH + bcol[tn] * ESZ;
          if constexpr (DT == PQ_F32) *reinterpret_cast<float*>(dst) = val;
          else if constexpr (DT == PQ_F16) *reinterpret_cast<uint16_t*>(dst) = pq_f32_to_f16(val);
          else *reinterpret_cast<uint16_t*>(dst) = pq_f32_to_bf16(val);
        }
      }
      lds_barrier();
      for (int c = threadIdx.x; c < WM * 32 * CPR; c += NW * 64) {
        const int sr = c / CPR, cc = c % CPR;
        const int64_t m = static_cast<int64_t>(bm) * BM + (sr >> 5) * (BM / WM) + tm * 32 + (sr & 31);
        const int n0 = bn * BN + cc * (16 / ESZ);
        if (m < M && n0 < N)
          __builtin_nontemporal_store(*reinterpret_cast<const v4i*>(smem + sr * PITCH + cc * 16),
                                      reinterpret_cast<v4i*>(static_cast<uint8_t*>(y) + (m * N + n0) * ESZ));
      }
    }
  };
  if (y_dtype == PQ_F32) emit(std::integral_constant<int, PQ_F32>{});
  else if (y_dtype == PQ_F16) emit(std::integral_constant<int, PQ_F16>{});
  else emit(std::integral_constant<int, PQ_BF16>{});
}

template <int BM, int BN, int WM, int WN, bool PARTIALS, int ST = kPfStages, bool TP = false>
void launch_prefill_t(pq::GemmGroup grp, int bias_dtype, int y_dtype, int M, int K,
                      hipStream_t stream) {
  constexpr int STAGE = BM * 128 + (BN / 16) * kPfBStride + BN * 4;
  grp.first[0] = 0;
  for (int i = 0; i < grp.count; ++i) grp.first[i + 1] = grp.first[i] + (grp.mem[i].n + BN - 1) / BN;
  const unsigned grid = static_cast<unsigned>(((M + BM - 1) / BM) * grp.first[grp.count]);
  gemm_prefill<BM, BN, WM, WN, PARTIALS, ST, TP><<<grid, WM * WN * 64, ST * STAGE + BM * 4, stream>>>(
      grp, bias_dtype, y_dtype, M, K);
}

// Tile choice.  From half a round of 128 x 256 tiles up, the cheaper of
// 192 x 256 and 128 x 256 tiles (8 waves of 192 or 128 rows x 32 columns)
// by the measured cost of their rounds of 256 workgroups, in units of one
// full round of 192 x 256 tiles (K = 4096): a full round of 128 x 256 tiles
// takes 0.71, a last, partly filled round 0.77 of a full one on 192 x 256
// tiles and 0.9 on 128 x 256 tiles (M = 4096, N = 4096: 111 us on 192 x
// 256, 89 us expected on 128 x 256).  Below that, 128 x 128 (4 waves,
// several workgroups per CU) when those fill the chip, 32 x 128 when those
// fit in one round, else 64 x 128 (k/v at M = 3072: 43.4 -> 37.2 us).
template <bool PARTIALS>
void launch_prefill(const pq::GemmGroup& grp, int bias_dtype, int y_dtype, int M, int K,
                    hipStream_t stream) {
  int64_t bn_tiles = 0;
  for (int i = 0; i < grp.count; ++i) bn_tiles += (grp.mem[i].n + 255) / 256;
  int64_t bn128 = 0;
  for (int i = 0; i < grp.count; ++i) bn128 += (grp.mem[i].n + 127) / 128;
  // A group whose 192 x 256 tiles leave the last round of the 256 CUs part
  // empty, but whose leading members fill whole rounds: those members run on
  // their own, the rest in a second launch with its own tile choice (q/k/v at
  // M = 3072: q's 256 tiles, then k and v on 192 tiles of 128 x 256, instead
  // of 384 big tiles in 1.5 rounds).  Each member's outputs do not depend on
  // the tiling.
  const int64_t rows192 = (M + 191) / 192;
  if (grp.count > 1 && rows192 * bn_tiles > 256 && (rows192 * bn_tiles) % 256 != 0) {
    int64_t lead = 0;
    for (int i = 1; i < grp.count; ++i) {
      lead += rows192 * ((grp.mem[i - 1].n + 255) / 256);
      if (lead % 256 == 0) {
        pq::GemmGroup head{}, tail{};
        head.count = i;
        tail.count = grp.count - i;
        for (int j = 0; j < i; ++j) head.mem[j] = grp.mem[j];
        for (int j = i; j < grp.count; ++j) tail.mem[j - i] = grp.mem[j];
        launch_prefill<PARTIALS>(head, bias_dtype, y_dtype, M, K, stream);
        launch_prefill<PARTIALS>(tail, bias_dtype, y_dtype, M, K, stream);
        return;
      }
    }
  }
  const int64_t tiles192 = rows192 * bn_tiles;
  const int64_t tiles128x256 = static_cast<int64_t>((M + 127) / 128) * bn_tiles;
  auto rounds = [](int64_t tiles, double full, double partial) {
    return full * static_cast<double>(tiles / 256) + (tiles % 256 != 0 ? full * partial : 0.0);
  };
  if (tiles192 >= 256 || tiles128x256 >= 128) {
    if (rounds(tiles192, 1.0, 0.77) <= rounds(tiles128x256, 0.71, 0.9))
      launch_prefill_t<192, 256, 1, 8, PARTIALS, kPfStages, true>(grp, bias_dtype, y_dtype, M, K, stream);
    else
      launch_prefill_t<128, 256, 1, 8, PARTIALS, kPfStages, true>(grp, bias_dtype, y_dtype, M, K, stream);
  } else if (static_cast<int64_t>((M + 127) / 128) * bn128 >= 256)
    launch_prefill_t<128, 128, 1, 4, PARTIALS>(grp, bias_dtype, y_dtype, M, K, stream);
  else if (static_cast<int64_t>((M + 31) / 32) * bn128 <= 256)
    // at most one round of 32-row tiles (65-256 tokens at N = 4096; up to
    // 64 the decode kernel runs them): each workgroup walks all of K, so its
    // time follows its rows (25 -> 19 us at K = 4096, 65 -> 49.5 us at
    // K = 12288 against 64 x 128)
    launch_prefill_t<32, 128, 1, 4, PARTIALS>(grp, bias_dtype, y_dtype, M, K, stream);
  else   // narrow outputs (k/v): twice the workgroups of 128-row tiles
    launch_prefill_t<64, 128, 1, 4, PARTIALS>(grp, bias_dtype, y_dtype, M, K, stream);
}

// ---------------------------------------------------------------------------
// Host-side configuration
// ---------------------------------------------------------------------------
// The decode GEMM on int8 A takes up to 64 rows, all its row blocks of 16
// in every workgroup (the weights are read once): the grouped decode layer at
// M = 33-64 on it against the row rotate+quant kernel and the prefill GEMM's
// tiles is recorded in the design notes.
constexpr int kSkinnyMaxM = 64;

struct SkinnyCfg {
  int nt;  // 16-column tiles per workgroup
  int w;   // waves per workgroup (split K)
  int u;   // groups per wave per batch (loads in flight)
};

// Measured on the Qwen3-8B shapes at 1-16 tokens:
// - About 4-6 waves per SIMD over the whole grid: more waves with fewer
//   groups each shorten every wave's serial load -> MFMA -> scale chain.
//   Never more waves than K groups.
// - Two column tiles per workgroup for wide outputs (768+ tiles, e.g. a
//   gate/up pair), and where one tile per workgroup would put one workgroup
//   on some CUs and two on others (256 < tiles < 512: the q/k/v group's 384
//   tiles on int8 A, the M = 16 layer 60.6 -> 59.9 us, M = 3 50.1 -> 49.9 us,
//   the 36-layer verify block 2.342 -> 2.315 ms).  Other outputs keep one
//   tile per workgroup at every token count (two from 5 tokens up measured
//   slower there: the M = 8 layer 58.3 against 55.8 us, the verify block
//   2.45 against 2.41 ms).  Not when a member of a group has an odd tile
//   count, nor with 16 waves behind the LDS A-quantizing prologue (3-16
//   rows: that combination spills).  At one and two rows, whose A is
//   quantized in registers, two tiles on 16 waves stay (the q/k/v group: 192
//   workgroups, one batch; M = 1: GEMM launches 6.64 -> 6.60 us, the decode
//   chain 1.493 -> 1.484 ms; the M = 2 layer 42.8 / 42.9 -> 42.3 / 42.2 us).
// - Behind that prologue, where every workgroup first quantizes the whole
//   activation row into LDS, 16 waves per workgroup only up to 4 per SIMD
//   over the grid (the q/k/v group, 384 workgroups, on 8 waves: the M = 1
//   layer 42.4 -> 41.9 us in a sweep, 42.1 -> 42.0 us in an A/B run, the
//   36-layer decode chain 1.587 -> 1.575 ms, the M = 2 layer 45.6 -> 45.2
//   us; the other shapes measured no better).
// - The shallowest batch of at least two groups that divides the K groups
//   (an uneven last batch is masked by a scalar branch); one group per batch
//   on int8 A at 9-16 rows (the M = 12 layer 54.7 / 54.8 -> 53.8 / 53.7 us,
//   M = 16 57.2 / 57.4 -> 56.9 / 56.6 us, the verify block 2.109 -> 2.097 ms;
//   at M = 4 one group per batch measured slower, 47.6 -> 48.7 us).
SkinnyCfg choose_skinny(int64_t m, int64_t n, int64_t k, bool two_tiles_ok = true, bool aq = false) {
  const int G = static_cast<int>(k / 128);
  const int tiles = static_cast<int>(n / 16);
  auto waves_for = [](int64_t wgs) { return wgs * 16 <= 6144 ? 16 : wgs * 8 <= 6144 ? 8 : 4; };
  int nt = (two_tiles_ok && tiles % 2 == 0 && (tiles >= 768 || (tiles > 256 && tiles < 512))) ? 2 : 1;
  int w = waves_for(static_cast<int64_t>(tiles / nt));
  if (aq && m > 2 && nt == 2 && w == 16) {
    nt = 1;
    w = waves_for(tiles);
  }
  if (aq && w == 16 && static_cast<int64_t>(tiles / nt) * 16 > 4096) w = 8;
  while (w > 4 && w > G) w >>= 1;
  int u = 2;
  if (G <= w || (!aq && m > 8 && m <= kSkinnyRows) || m > 2 * kSkinnyRows) u = 1;
  else if (G % (w * 2) == 0) u = 2;
  else if (G % (w * 3) == 0) u = 3;
  else if (G % (w * 4) == 0) u = 4;
  return {nt, w, u};
}

template <int NT, int W, int U, bool PARTIALS, int AQ>
void launch_skinny_nwu(pq::GemmGroup grp, int bias_dtype, int y_dtype, int M, int K,
                       hipStream_t stream) {
  grp.first[0] = 0;
  for (int i = 0; i < grp.count; ++i) grp.first[i + 1] = grp.first[i] + grp.mem[i].n / 16 / NT;
  const unsigned tiles = static_cast<unsigned>(grp.first[grp.count]);
  const size_t lds = (AQ == 1 || AQ == 2) ? static_cast<size_t>(M) * (K + 16) : 0;
  if constexpr (AQ == 0) {
    // int8 A, 17-64 rows: every workgroup carries the ceil(M / 16) row blocks;
    // from 33 rows one group per batch (their A fragments fill the registers)
    if (M > 2 * kSkinnyRows) {
      if constexpr (U != 1) {
        launch_skinny_nwu<NT, W, 1, PARTIALS, AQ>(grp, bias_dtype, y_dtype, M, K, stream);
      } else if (M > 3 * kSkinnyRows) {
        gemm_skinny<NT, W, U, PARTIALS, AQ, 4><<<tiles, W * 64, 0, stream>>>(grp, bias_dtype, y_dtype, M, K);
      } else {
        gemm_skinny<NT, W, U, PARTIALS, AQ, 3><<<tiles, W * 64, 0, stream>>>(grp, bias_dtype, y_dtype, M, K);
      }
      return;
    }
    if (M > kSkinnyRows) {
      gemm_skinny<NT, W, U, PARTIALS, AQ, 2><<<tiles, W * 64, 0, stream>>>(grp, bias_dtype, y_dtype, M, K);
      return;
    }
  }
  gemm_skinny<NT, W, U, PARTIALS, AQ><<<tiles, W * 64, lds, stream>>>(grp, bias_dtype, y_dtype, M, K);
}

template <bool PARTIALS, int AQ>
void launch_skinny(const SkinnyCfg& cfg, const pq::GemmGroup& grp, int bias_dtype, int y_dtype, int M, int K,
                   hipStream_t stream) {
#define PQ_SKINNY(NT_, W_, U_)                                                                         \
  if (cfg.nt == NT_ && cfg.w == W_ && cfg.u == U_) {                                                   \
    launch_skinny_nwu<NT_, W_, U_, PARTIALS, AQ>(grp, bias_dtype, y_dtype, M, K, stream);              \
    return;                                                                                            \
  }
#define PQ_SKINNY_NT(NT_)                                                                              \
  PQ_SKINNY(NT_, 4, 1) PQ_SKINNY(NT_, 4, 2) PQ_SKINNY(NT_, 4, 3) PQ_SKINNY(NT_, 4, 4)                  \
  PQ_SKINNY(NT_, 8, 1) PQ_SKINNY(NT_, 8, 2) PQ_SKINNY(NT_, 8, 3) PQ_SKINNY(NT_, 8, 4)                  \
  PQ_SKINNY(NT_, 16, 1) PQ_SKINNY(NT_, 16, 2) PQ_SKINNY(NT_, 16, 3) PQ_SKINNY(NT_, 16, 4)
  PQ_SKINNY_NT(1)
  PQ_SKINNY_NT(2)
#undef PQ_SKINNY_NT
#undef PQ_SKINNY
  // every configuration choose_skinny makes is listed above; anything else
  // runs the generic one (any G, masked batches)
  if (cfg.nt == 2) launch_skinny_nwu<2, 4, 4, PARTIALS, AQ>(grp, bias_dtype, y_dtype, M, K, stream);
  else launch_skinny_nwu<1, 4, 4, PARTIALS, AQ>(grp, bias_dtype, y_dtype, M, K, stream);
}

// The decode GEMM's configuration for a group: the workgroup count is the
// sum over members; two tiles per workgroup only when every member's tile
// count is even.
SkinnyCfg choose_skinny_group(const pq::GemmGroup& grp, int64_t m, int64_t k, bool aq) {
  int64_t n = 0;
  bool even = true;
  for (int i = 0; i < grp.count; ++i) {
    n += grp.mem[i].n;
    even = even && (grp.mem[i].n / 16) % 2 == 0;
  }
  return choose_skinny(m, n, k, even, aq);
}

int check_gemm_args(const char* who, int64_t m, int64_t n, int64_t k, int group_size) {
  PQ_REQUIRE(group_size == 128, PQ_ERR_UNSUPPORTED, "%s: group_size=%d (only 128 is supported)", who, group_size);
  PQ_REQUIRE(m >= 0 && m <= 0x7fffffffLL, PQ_ERR_ARG, "%s: m=%lld", who, (long long)m);
  PQ_REQUIRE(n > 0 && n % 16 == 0 && n <= (1 << 20), PQ_ERR_ARG, "%s: n=%lld must be a positive multiple of 16", who,
             (long long)n);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= (1 << 20), PQ_ERR_ARG, "%s: k=%lld must be a positive multiple of 128",
             who, (long long)k);
  // the kernels address A and the packed weights with 32-bit element offsets
  PQ_REQUIRE(m * k < (int64_t(1) << 31) && n * k / 2 < (int64_t(1) << 31), PQ_ERR_ARG,
             "%s: m*k=%lld and n*k/2=%lld must stay below 2^31", who, (long long)(m * k), (long long)(n * k / 2));
  return PQ_OK;
}

}  // namespace

namespace pq {
bool gemm_rotated_supported(int64_t m, int64_t k) {
  return m >= 1 && m <= kSkinnyRows && k % 128 == 0 && k <= 16384 && m * (k + 16) <= 80 * 1024;
}

void launch_gemm_group(GemmGroup grp, int aq, int bias_dtype, int y_dtype, int m, int k, hipStream_t stream) {
  if (aq == 0 && m > kSkinnyMaxM) {
    launch_prefill<false>(grp, bias_dtype, y_dtype, m, k, stream);
    return;
  }
  const SkinnyCfg cfg = choose_skinny_group(grp, m, k, aq != 0);
  if (aq == 0) {
    launch_skinny<false, 0>(cfg, grp, bias_dtype, y_dtype, m, k, stream);
    return;
  }
  if (aq == 1 && m == 1) launch_skinny<false, 3>(cfg, grp, bias_dtype, y_dtype, m, k, stream);
  else if (aq == 1 && m == 2) launch_skinny<false, 4>(cfg, grp, bias_dtype, y_dtype, m, k, stream);
  else if (aq == 1) launch_skinny<false, 1>(cfg, grp, bias_dtype, y_dtype, m, k, stream);
  else launch_skinny<false, 2>(cfg, grp, bias_dtype, y_dtype, m, k, stream);
}

// The same choices as launch_gemm_group, with PARTIALS instances.
void launch_gemm_group_partials(GemmGroup grp, int aq, int m, int k, hipStream_t stream) {
  if (aq == 0 && m > kSkinnyMaxM) {
    launch_prefill<true>(grp, 0, 0, m, k, stream);
    return;
  }
  const SkinnyCfg cfg = choose_skinny_group(grp, m, k, aq != 0);
  if (aq == 0) launch_skinny<true, 0>(cfg, grp, 0, 0, m, k, stream);
  else if (aq == 1 && m == 1) launch_skinny<true, 3>(cfg, grp, 0, 0, m, k, stream);
  else if (aq == 1 && m == 2) launch_skinny<true, 4>(cfg, grp, 0, 0, m, k, stream);
  else if (aq == 1) launch_skinny<true, 1>(cfg, grp, 0, 0, m, k, stream);
  else launch_skinny<true, 2>(cfg, grp, 0, 0, m, k, stream);
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
  (void)workspace, (void)workspace_bytes;
  pq::GemmGroup grp{};
  grp.count = 1;
  grp.mem[0] = {xq, xscale, nullptr, nullptr, wpack, wmeta, bias, y, static_cast<int>(n)};
  pq::launch_gemm_group(grp, 0, bias_dtype, y_dtype, static_cast<int>(m), static_cast<int>(k),
                        static_cast<hipStream_t>(stream));
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
  const int M = static_cast<int>(m), K = static_cast<int>(k);
  pq::GemmGroup grp{};
  grp.count = 1;
  grp.mem[0] = {xq, nullptr, nullptr, nullptr, wpack, wmeta, nullptr, nullptr, static_cast<int>(n), partials};
  pq::launch_gemm_group_partials(grp, 0, M, K, s);
  return pq::launch_status("pq_w4a8_gemm_partials launch");
}
