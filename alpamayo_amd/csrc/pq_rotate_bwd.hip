// Backward of rotation::rotate: the gradients of y = R_{K-1} ... R_0 (s * x)
// with respect to x, the angles theta and the channel scales s.
//
// Reference: RotateTensorFunc.backward (kernels/paroquant_kernels/
// interface.py:30-93), which inverts y layer by layer with one rotation launch
// per layer and gathers the pairs in torch.  Here one kernel does all layers:
//
//   * each workgroup (4 waves, 4 rows per wave, a channel-major float4 per
//     channel in LDS: the forward tile kernel's layout) re-runs the forward
//     layers from x in float32 and keeps every layer's pair outputs (a', b')
//     in registers -- the values the forward computed, not a reconstruction
//     from the rounded y;
//   * then it walks the layers backwards on the incoming gradient: with
//     (g_a', g_b') the gradient at layer r's output, the angle gradient is
//     g_a' b' - g_b' a' (d(a', b')/d theta = (b', -a')), and the gradient at
//     the layer's input is the transposed rotation (c g_a' - s g_b',
//     s g_a' + c g_b');
//   * below layer 0: dx = s * g_t and ds = x * g_t (t = s * x).
//
// The angle and scale gradients are sums over all rows.  A workgroup walks
// its column of row tiles grid-stride and keeps running sums in registers,
// the 4 waves are summed through LDS in a fixed order, and each workgroup row
// writes one partial per angle / channel; a second kernel adds the partials
// in a fixed order.  The result is deterministic (no atomics).
#include "pq_device.h"
#include "pq_internal.h"

namespace {

constexpr int kBwdWaves = 4;
constexpr int kBwdRowsPerWave = 4;
constexpr int kBwdRows = kBwdWaves * kBwdRowsPerWave;
// Workgroup rows of the partial sums (each handles every kBwdMaxBlocks-th tile).
constexpr int64_t kBwdMaxBlocks = 64;

int64_t bwd_blocks(int64_t rows) {
  const int64_t tiles = (rows + kBwdRows - 1) / kBwdRows;
  return tiles < kBwdMaxBlocks ? tiles : kBwdMaxBlocks;
}

__device__ __forceinline__ float4 f4(float a, float b, float c, float d) { return make_float4(a, b, c, d); }

template <int DT, int G, bool SCALE, int KP>
__global__ __launch_bounds__(kBwdWaves * 64) void rotate_bwd_kernel(
    const void* __restrict__ x, const void* __restrict__ gy, void* __restrict__ gx, const int16_t* __restrict__ idx,
    const void* __restrict__ theta, const void* __restrict__ scales, float* __restrict__ part_th,
    float* __restrict__ part_s, int64_t rows, int h, int krot) {
  __shared__ float4 tile[kBwdWaves][128];
  __shared__ float2 s_cs[KP][64];
  __shared__ uint32_t s_ij[KP][64];
  __shared__ float red[kBwdWaves][KP + 2][64];
  constexpr int NT = kBwdWaves * 64;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  const int ch0 = blockIdx.y * 128;
  const int half = h >> 1;

  // The chunk's 64 pairs per layer, as the forward tile kernel derives them:
  // group-local indices masked to the group, cos / sin of the stored angle in
  // float64 rounded once.  A pair past h (the empty half of a 64-channel
  // tail) is the identity on two channels that hold zeros.
  for (int e = t; e < krot * 64; e += NT) {
    const int r = e >> 6, p = e & 63;
    const int P = blockIdx.y * 64 + p;
    float c = 1.0f, sn = 0.0f;
    uint32_t ij = static_cast<uint32_t>(2 * p) | (static_cast<uint32_t>(2 * p + 1) << 8);
    if (P < half) {
      const int gi = P / (G / 2);
      const int pp = P % (G / 2);
      const int base = gi * G - ch0;
      const int64_t o = static_cast<int64_t>(r) * h + gi * G + 2 * pp;
      const int i = base + (idx[o] & (G - 1));
      const int j = base + (idx[o + 1] & (G - 1));
      const float th = pq_load_as_f32<DT>(theta, static_cast<int64_t>(r) * half + P);
      double sd, cd;
      sincos(static_cast<double>(th), &sd, &cd);
      c = static_cast<float>(cd);
      sn = static_cast<float>(sd);
      ij = static_cast<uint32_t>(i) | (static_cast<uint32_t>(j) << 8);
    }
    s_cs[r][p] = make_float2(c, sn);
    s_ij[r][p] = ij;
  }
  __syncthreads();

  const int ch = ch0 + 2 * lane;
  const bool ch_ok = ch < h;
  float sc0 = 1.0f, sc1 = 1.0f;
  if (SCALE && ch_ok) {
    sc0 = pq_load_as_f32<DT>(scales, ch);
    sc1 = pq_load_as_f32<DT>(scales, ch + 1);
  }
  float acc_th[KP];
#pragma unroll
  for (int r = 0; r < KP; ++r) acc_th[r] = 0.0f;
  float acc_s0 = 0.0f, acc_s1 = 0.0f;
  float4* wt = tile[w];
  const int64_t tiles = (rows + kBwdRows - 1) / kBwdRows;

  for (int64_t tl = blockIdx.x; tl < tiles; tl += gridDim.x) {
    const int64_t row0 = tl * kBwdRows + w * kBwdRowsPerWave;
    // x rows (raw, for ds) and t = s * x into the wave's tile
    float xa[kBwdRowsPerWave], xb[kBwdRowsPerWave];
#pragma unroll
    for (int rr = 0; rr < kBwdRowsPerWave; ++rr) {
      const int64_t row = row0 + rr;
      xa[rr] = 0.0f;
      xb[rr] = 0.0f;
      if (row < rows && ch_ok) {
        xa[rr] = pq_load_as_f32<DT>(x, row * h + ch);
        xb[rr] = pq_load_as_f32<DT>(x, row * h + ch + 1);
      }
    }
    if (SCALE) {
      wt[2 * lane] = f4(xa[0] * sc0, xa[1] * sc0, xa[2] * sc0, xa[3] * sc0);
      wt[2 * lane + 1] = f4(xb[0] * sc1, xb[1] * sc1, xb[2] * sc1, xb[3] * sc1);
    } else {
      wt[2 * lane] = f4(xa[0], xa[1], xa[2], xa[3]);
      wt[2 * lane + 1] = f4(xb[0], xb[1], xb[2], xb[3]);
    }
    // The tile is this wave's alone and a wave's LDS operations complete in
    // issue order, so no barrier is needed between the layers; the fences
    // keep the compiler from reordering the LDS accesses.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);

    // Forward layers, keeping each layer's pair outputs.
    float4 oa[KP], ob[KP];
#pragma unroll
    for (int r = 0; r < KP; ++r) {
      if (r < krot) {
        const float2 cs = s_cs[r][lane];
        const uint32_t ij = s_ij[r][lane];
        const int i = static_cast<int>(ij & 0xffu), j = static_cast<int>(ij >> 8);
        const float4 a = wt[i], b = wt[j];
        float4 na, nb;
        na.x = fmaf(a.x, cs.x, b.x * cs.y);
        nb.x = fmaf(b.x, cs.x, -(a.x * cs.y));
        na.y = fmaf(a.y, cs.x, b.y * cs.y);
        nb.y = fmaf(b.y, cs.x, -(a.y * cs.y));
        na.z = fmaf(a.z, cs.x, b.z * cs.y);
        nb.z = fmaf(b.z, cs.x, -(a.z * cs.y));
        na.w = fmaf(a.w, cs.x, b.w * cs.y);
        nb.w = fmaf(b.w, cs.x, -(a.w * cs.y));
        wt[i] = na;
        wt[j] = nb;
        oa[r] = na;
        ob[r] = nb;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
      }
    }

    // The incoming gradient rows replace the tile.
    {
      float ga[kBwdRowsPerWave], gb[kBwdRowsPerWave];
#pragma unroll
      for (int rr = 0; rr < kBwdRowsPerWave; ++rr) {
        const int64_t row = row0 + rr;
        ga[rr] = 0.0f;
        gb[rr] = 0.0f;
        if (row < rows && ch_ok) {
          ga[rr] = pq_load_as_f32<DT>(gy, row * h + ch);
          gb[rr] = pq_load_as_f32<DT>(gy, row * h + ch + 1);
        }
      }
      wt[2 * lane] = f4(ga[0], ga[1], ga[2], ga[3]);
      wt[2 * lane + 1] = f4(gb[0], gb[1], gb[2], gb[3]);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }

    // Layers backwards: angle gradient from the layer's outputs, then the
    // transposed rotation of the gradient.
#pragma unroll
    for (int r = KP - 1; r >= 0; --r) {
      if (r < krot) {
        const float2 cs = s_cs[r][lane];
        const uint32_t ij = s_ij[r][lane];
        const int i = static_cast<int>(ij & 0xffu), j = static_cast<int>(ij >> 8);
        const float4 ga = wt[i], gb = wt[j];
        const float4 a = oa[r], b = ob[r];
        float d = fmaf(ga.x, b.x, -(gb.x * a.x));
        d += fmaf(ga.y, b.y, -(gb.y * a.y));
        d += fmaf(ga.z, b.z, -(gb.z * a.z));
        d += fmaf(ga.w, b.w, -(gb.w * a.w));
        acc_th[r] += d;
        float4 pa, pb;
        pa.x = fmaf(ga.x, cs.x, -(gb.x * cs.y));
        pb.x = fmaf(gb.x, cs.x, ga.x * cs.y);
        pa.y = fmaf(ga.y, cs.x, -(gb.y * cs.y));
        pb.y = fmaf(gb.y, cs.x, ga.y * cs.y);
        pa.z = fmaf(ga.z, cs.x, -(gb.z * cs.y));
        pb.z = fmaf(gb.z, cs.x, ga.z * cs.y);
        pa.w = fmaf(ga.w, cs.x, -(gb.w * cs.y));
        pb.w = fmaf(gb.w, cs.x, ga.w * cs.y);
        wt[i] = pa;
        wt[j] = pb;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
      }
    }

    // Gradient at t = s * x for channels ch, ch + 1 of the wave's rows.
    const float4 ta = wt[2 * lane], tb = wt[2 * lane + 1];
    const float gta[kBwdRowsPerWave] = {ta.x, ta.y, ta.z, ta.w};
    const float gtb[kBwdRowsPerWave] = {tb.x, tb.y, tb.z, tb.w};
#pragma unroll
    for (int rr = 0; rr < kBwdRowsPerWave; ++rr) {
      const int64_t row = row0 + rr;
      if (row < rows && ch_ok) {
        pq_store_from_f32<DT>(gx, row * h + ch, SCALE ? gta[rr] * sc0 : gta[rr]);
        pq_store_from_f32<DT>(gx, row * h + ch + 1, SCALE ? gtb[rr] * sc1 : gtb[rr]);
      }
      if (SCALE) {
        acc_s0 = fmaf(xa[rr], gta[rr], acc_s0);
        acc_s1 = fmaf(xb[rr], gtb[rr], acc_s1);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }

  // Sum the 4 waves (fixed order) and write this workgroup's partials.
#pragma unroll
  for (int r = 0; r < KP; ++r) red[w][r][lane] = acc_th[r];
  red[w][KP][lane] = acc_s0;
  red[w][KP + 1][lane] = acc_s1;
  __syncthreads();
  if (w == 0) {
    const int P = blockIdx.y * 64 + lane;
    for (int r = 0; r < krot; ++r) {
      const float v = ((red[0][r][lane] + red[1][r][lane]) + red[2][r][lane]) + red[3][r][lane];
      if (P < half) part_th[(static_cast<int64_t>(blockIdx.x) * krot + r) * half + P] = v;
    }
    if (SCALE && ch_ok) {
      float* ps = part_s + static_cast<int64_t>(blockIdx.x) * h;
      ps[ch] = ((red[0][KP][lane] + red[1][KP][lane]) + red[2][KP][lane]) + red[3][KP][lane];
      ps[ch + 1] = ((red[0][KP + 1][lane] + red[1][KP + 1][lane]) + red[2][KP + 1][lane]) + red[3][KP + 1][lane];
    }
  }
}

// grad_theta[r][P] = sum_b part_th[b][r][P]; grad_scales[c] = sum_b part_s[b][c]
// (b in order), rounded to the parameters' dtype.  nb == 0 writes zeros.
template <int DT>
__global__ __launch_bounds__(256) void rotate_bwd_reduce_kernel(const float* __restrict__ part_th,
                                                                const float* __restrict__ part_s,
                                                                void* __restrict__ g_theta,
                                                                void* __restrict__ g_scales, int nb, int n_th,
                                                                int h) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n_th) {
    float s = 0.0f;
    for (int b = 0; b < nb; ++b) s += part_th[static_cast<int64_t>(b) * n_th + i];
    pq_store_from_f32<DT>(g_theta, i, s);
  } else if (g_scales != nullptr && i < static_cast<int64_t>(n_th) + h) {
    const int64_t c = i - n_th;
    float s = 0.0f;
    for (int b = 0; b < nb; ++b) s += part_s[static_cast<int64_t>(b) * h + c];
    pq_store_from_f32<DT>(g_scales, c, s);
  }
}

template <int DT, int G, bool SCALE>
void launch_bwd_g(const void* x, const void* gy, void* gx, const int16_t* idx, const void* theta, const void* scales,
                  float* part_th, float* part_s, int64_t rows, int h, int krot, int nb, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(nb), static_cast<unsigned>((h + 127) / 128));
  if (krot <= 8)
    rotate_bwd_kernel<DT, G, SCALE, 8><<<grid, kBwdWaves * 64, 0, s>>>(x, gy, gx, idx, theta, scales, part_th,
                                                                        part_s, rows, h, krot);
  else
    rotate_bwd_kernel<DT, G, SCALE, 16><<<grid, kBwdWaves * 64, 0, s>>>(x, gy, gx, idx, theta, scales, part_th,
                                                                         part_s, rows, h, krot);
}

template <int DT>
void launch_bwd(const void* x, const void* gy, void* gx, void* g_theta, void* g_scales, const int16_t* idx,
                const void* theta, const void* scales, int64_t rows, int h, int krot, int group, float* ws,
                hipStream_t s) {
  const int nb = static_cast<int>(bwd_blocks(rows));
  const int n_th = krot * (h / 2);
  float* part_th = ws;
  float* part_s = ws + static_cast<int64_t>(nb) * n_th;
  if (nb > 0) {
    if (group == 128) {
      if (scales) launch_bwd_g<DT, 128, true>(x, gy, gx, idx, theta, scales, part_th, part_s, rows, h, krot, nb, s);
      else launch_bwd_g<DT, 128, false>(x, gy, gx, idx, theta, scales, part_th, part_s, rows, h, krot, nb, s);
    } else {
      if (scales) launch_bwd_g<DT, 64, true>(x, gy, gx, idx, theta, scales, part_th, part_s, rows, h, krot, nb, s);
      else launch_bwd_g<DT, 64, false>(x, gy, gx, idx, theta, scales, part_th, part_s, rows, h, krot, nb, s);
    }
  }
  const int64_t n_out = n_th + (scales ? h : 0);
  rotate_bwd_reduce_kernel<DT><<<static_cast<unsigned>((n_out + 255) / 256), 256, 0, s>>>(
      part_th, part_s, g_theta, scales ? g_scales : nullptr, nb, n_th, h);
}

}  // namespace

extern "C" size_t pq_rotate_backward_workspace_size(int64_t rows, int64_t h, int krot) {
  if (rows < 0 || h <= 0 || krot < 1 || krot > 16) return 0;
  return static_cast<size_t>(bwd_blocks(rows)) * (static_cast<size_t>(krot) * (h / 2) + h) * sizeof(float);
}

extern "C" int pq_rotate_backward(const void* x, const void* grad_y, void* grad_x, void* grad_theta,
                                  void* grad_scales, const int16_t* idx_ij, const void* theta, const void* scales,
                                  int64_t rows, int64_t h, int krot, int group_size, int dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  const char* who = "pq_rotate_backward";
  PQ_REQUIRE(rows >= 0 && h > 0, PQ_ERR_ARG, "%s: rows=%lld h=%lld", who, (long long)rows, (long long)h);
  PQ_REQUIRE(group_size == 64 || group_size == 128, PQ_ERR_UNSUPPORTED,
             "%s: Unexpected group_size: %d (supported: 64, 128)", who, group_size);
  PQ_REQUIRE(krot == 1 || krot == 2 || krot == 4 || krot == 8 || krot == 16, PQ_ERR_UNSUPPORTED,
             "%s: Unsupported KROT = %d; compiled variants: 1/2/4/8/16", who, krot);
  PQ_REQUIRE(h % group_size == 0, PQ_ERR_ARG, "%s: h must be divisible by GROUP_SIZE (h=%lld, G=%d)", who,
             (long long)h, group_size);
  // (h + 127) / 128 channel blocks go on grid.y, whose limit is 65535
  PQ_REQUIRE(h <= 65535LL * 128, PQ_ERR_ARG, "%s: h=%lld too large (at most %lld)", who, (long long)h,
             65535LL * 128);
  PQ_REQUIRE(dtype == PQ_F32 || dtype == PQ_F16 || dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "%s: dtype code %d (Float, Half or BFloat16)", who, dtype);
  PQ_REQUIRE((rows + kBwdRows - 1) / kBwdRows <= 0x7fffffffLL, PQ_ERR_ARG, "%s: too many rows", who);
  PQ_REQUIRE(grad_theta && idx_ij && theta, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE((scales == nullptr) == (grad_scales == nullptr), PQ_ERR_ARG,
             "%s: grad_scales must be given exactly when scales is", who);
  PQ_REQUIRE(rows == 0 || (x && grad_y && grad_x), PQ_ERR_ARG, "%s: null x / grad_y / grad_x", who);
  const size_t need = pq_rotate_backward_workspace_size(rows, h, krot);
  PQ_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need && pq::aligned_to(workspace, 16)),
             PQ_ERR_WORKSPACE, "%s: a 16-byte aligned workspace of %zu bytes is needed for rows=%lld h=%lld, got %zu",
             who, need, (long long)rows, (long long)h, workspace ? workspace_bytes : (size_t)0);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(h);
  float* ws = static_cast<float*>(workspace);
  switch (dtype) {
    case PQ_F32:
      launch_bwd<PQ_F32>(x, grad_y, grad_x, grad_theta, grad_scales, idx_ij, theta, scales, rows, hh, krot,
                         group_size, ws, s);
      break;
    case PQ_F16:
      launch_bwd<PQ_F16>(x, grad_y, grad_x, grad_theta, grad_scales, idx_ij, theta, scales, rows, hh, krot,
                         group_size, ws, s);
      break;
    default:
      launch_bwd<PQ_BF16>(x, grad_y, grad_x, grad_theta, grad_scales, idx_ij, theta, scales, rows, hh, krot,
                          group_size, ws, s);
      break;
  }
  return pq::launch_status("pq_rotate_backward launch");
}
