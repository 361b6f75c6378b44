// W4A16 linear on gfx950: int4 weights with per-(128-group, column) fp16
// scale s and scaled zero sz, fp16 activations, fp32 accumulation on the fp16
// MFMA units:
//
//   w[k, n] = fp16(q[k, n] * s[g, n] + sz[g, n])       (one rounding, a fused
//                                                        multiply-add in fp16)
//   y[m, n] = sum_k x[m, k] * w[k, n] (+ bias[n])       (fp32, rounded once)
//
// Reference: WQLinear.forward (src/alpamayo_r1/utils/quantization/
// qmodule.py:207-232), which calls the un-vendored torch.ops.awq.gemv (fewer
// than 8 rows) / torch.ops.awq.gemm on the WQLinear buffers; weight
// semantics of dequant_wqlinear (paroquant_marlin_w4a8.py:216-224).  Those
// kernels dequantize to fp16 before multiplying; the single fp16 rounding of
// q*s + sz above is that step.
//
// Weights: the same packed codes as the W4A8 GEMM (pq_w4a8_prepack's wpack:
// [N/16][G][64 slots][16 B], slot 16j + c = column 16*tile + c, codes
// k = 128g + 32j + [0, 32), a dword = 8 consecutive k, low nibbles first);
// the metadata word of a (group, column) is s | sz << 16 (pq_w4a16_prepack).
//
// Dequantization of a dword (8 codes) in 14 VALU operations: the codes are
// spread into bytes (and, shift), each pair of bytes becomes an fp16 pair
// 1024 + q by a byte permute against 0x64 (the exponent of 1024), 1024 is
// subtracted (exact), and one packed fp16 fma applies s and sz.  The weights
// are complete after that: no per-group epilogue, the MFMA accumulators run
// over all of K.
//
// Two kernels:
//   w16_skinny   M <= 16: as the W4A8 decode GEMM (waves split K by groups,
//                fixed-order LDS sum of their partials), four
//                v_mfma_f32_16x16x32_f16 per 1 KB weight block, A rows read
//                from memory (rows past M repeat row M-1, never stored).
//   w16_prefill  M > 16: 192x256 (or 128x128) tiles, 8 (or 4) waves side by
//                side along n, v_mfma_f32_32x32x16_f16.  A stage of the LDS
//                ring is half a K group (64 k): BM rows x 128 B of A
//                (16-byte chunks XOR-swizzled by row), the matching halves
//                of the BN/16 weight blocks and the group's BN metadata
//                words, copied global -> LDS directly; 4 stages, the copies
//                of step s+3 issued during step s.
#include <type_traits>

#include "pq_device.h"
#include "pq_internal.h"

using namespace pqd;

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

namespace {

struct W16Args {
  const uint16_t* x;       // fp16 [m][k]
  const uint8_t* wpack;    // packed codes
  const uint32_t* wmeta;   // s | sz << 16 per (tile, group, column)
  const void* bias;        // [n] or null
  void* y;                 // [m][n]
  int n;
};

__device__ __forceinline__ v2h as_h2(uint32_t u) { return __builtin_bit_cast(v2h, u); }
__device__ __forceinline__ uint32_t as_u32(v2h h) { return __builtin_bit_cast(uint32_t, h); }

// fp16 pairs {s, s} and {sz, sz} of a metadata word.
__device__ __forceinline__ v2h meta_s2(uint32_t meta) { return as_h2(__builtin_amdgcn_perm(meta, meta, 0x01000100u)); }
__device__ __forceinline__ v2h meta_z2(uint32_t meta) { return as_h2(__builtin_amdgcn_perm(meta, meta, 0x03020302u)); }

// One dword of codes (k order: the low nibbles of bytes 0..3, then the high
// nibbles) -> its 8 weights fp16(q * s + sz), in k order.
__device__ __forceinline__ v8h dequant8(uint32_t w, v2h s2, v2h z2) {
  const uint32_t lo = w & 0x0f0f0f0fu;
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
  // selector bytes 0..3 pick bytes of the second operand, 4 picks 0x64:
  // halves 0x6400 + q = 1024 + q
  constexpr uint32_t kE = 0x64646464u;
  const v2h off = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
  const v2h q01 = as_h2(__builtin_amdgcn_perm(kE, lo, 0x04010400u)) - off;
  const v2h q23 = as_h2(__builtin_amdgcn_perm(kE, lo, 0x04030402u)) - off;
  const v2h q45 = as_h2(__builtin_amdgcn_perm(kE, hi, 0x04010400u)) - off;
  const v2h q67 = as_h2(__builtin_amdgcn_perm(kE, hi, 0x04030402u)) - off;
  const uint4 r = {as_u32(__builtin_elementwise_fma(q01, s2, z2)), as_u32(__builtin_elementwise_fma(q23, s2, z2)),
                   as_u32(__builtin_elementwise_fma(q45, s2, z2)), as_u32(__builtin_elementwise_fma(q67, s2, z2))};
  return __builtin_bit_cast(v8h, r);
}

// ---------------------------------------------------------------------------
// Decode-size GEMM (M <= 16)
//
// Workgroup = W waves over NT 16-column tiles; wave w takes the groups
// w, w+W, ... of K, U groups of loads at a time.  Lane (j, c) holds the 32
// codes k = 32j + [0, 32) of column c of a block; its four MFMAs take 8 of
// them each, against the same 8 k of A row c (one 16-byte load each).
// ---------------------------------------------------------------------------
constexpr int kW16SkinnyRows = 16;

// Linears that share their input, as one decode GEMM launch: member i owns
// workgroups first[i] .. first[i+1]-1 (set by the launcher).
struct W16Group {
  W16Args mem[pq::kMaxGroup];
  int first[pq::kMaxGroup + 1];
  int count;
};

template <int NT, int W, int U>
__global__ __launch_bounds__(W * 64) void w16_skinny(const W16Group grp, int bias_dtype, int y_dtype, int M, int K) {
  __shared__ float red[W][NT][4][64];
  int mi = 0;   // the member that owns this workgroup (wave-uniform)
#pragma unroll
  for (int i = 1; i < pq::kMaxGroup; ++i)
    if (i < grp.count && static_cast<int>(blockIdx.x) >= grp.first[i]) mi = i;
  const W16Args& ar = grp.mem[mi];
  const int G = K >> 7;
  const int N = ar.n;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int j = lane >> 4;
  const int tile0 = (static_cast<int>(blockIdx.x) - grp.first[mi]) * NT;
  // Rows past M repeat row M-1: MFMA rows are independent and those results
  // are never stored.
  const uint16_t* ap = ar.x + static_cast<int64_t>(c < M ? c : M - 1) * K + j * 32;

  v4f acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  const int batches = (G + W * U - 1) / (W * U);
  auto run_batch = [&](const int it) {
    const int g0 = wave + it * W * U;
    v4i wb[U][NT];
    uint32_t wm[U][NT];
    v8h a[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g0 + W * u;
      if (g < G) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int64_t blk = static_cast<int64_t>(tile0 + nt) * G + g;
          // read once per call: non-temporal, so they do not evict the
          // activations and what the next launches re-read
          wb[u][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(ar.wpack + blk * 1024 + lane * 16));
          wm[u][nt] = __builtin_nontemporal_load(ar.wmeta + blk * 16 + c);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) a[u][t] = *reinterpret_cast<const v8h*>(ap + g * 128 + t * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g0 + W * u;
      if (g < G) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t meta = wm[u][nt];
          const v2h s2 = meta_s2(meta), z2 = meta_z2(meta);
          const v4i w = wb[u][nt];
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u][t], dequant8(static_cast<uint32_t>(w[t]), s2, z2),
                                                             acc[nt], 0, 0, 0);
        }
      }
    }
  };
  run_batch(0);
  for (int it = 1; it < batches; ++it) run_batch(it);

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
    if (ar.bias != nullptr) sum = sum + pq_load_dyn(ar.bias, bias_dtype, n);
    pq_store_dyn(ar.y, y_dtype, static_cast<int64_t>(m) * N + n, sum);
  }
}

// ---------------------------------------------------------------------------
// Prefill-size GEMM (M > 16)
// ---------------------------------------------------------------------------
constexpr int kW16Stages = 4;
constexpr int kW16GroupM = 4;   // tile rows walked together by one XCD's run of tiles

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void w16_prefill(const W16Args ar, int bias_dtype, int y_dtype, int M,
                                                            int K) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int A_BYTES = BM * 128;          // BM rows x 64 fp16
  constexpr int B_BYTES = (BN / 16) * 512;   // half of each 1 KB block
  constexpr int STAGE = A_BYTES + B_BYTES + BN * 4;
  constexpr int A_LD = BM / 8 / NW, B_LD = BN / 32 / NW, M_LD = 1;   // copies per wave per stage
  constexpr int LOADS = A_LD + B_LD + M_LD;
  constexpr int MCOLS = BN / NW;   // metadata words per wave
  static_assert(TM >= 1 && TN >= 1 && BM % (32 * WM) == 0 && BN % (32 * WN) == 0, "tile shape");
  static_assert((BM / 8) % NW == 0 && (BN / 32) % NW == 0 && MCOLS <= 64, "copies split evenly over the waves");
  static_assert(LOADS * (kW16Stages - 2) < 64, "vmcnt range");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int G = K >> 7;
  const int S = 2 * G;   // steps: half groups
  const int N = ar.n;
  const int ntiles16 = N >> 4;
  const int nbn = (N + BN - 1) / BN;
  // Tile order: workgroup b runs on XCD b % 8, so the grid is cut into 8
  // contiguous runs of tiles (one per XCD, when the count divides), each
  // walking kW16GroupM tile rows at a time, column by column.
  int t = blockIdx.x;
  if (gridDim.x % 8 == 0) t = (t % 8) * (gridDim.x / 8) + t / 8;
  const int nbm = (M + BM - 1) / BM;
  const int first_bm = t / (kW16GroupM * nbn) * kW16GroupM;
  const int gm = min(nbm - first_bm, kW16GroupM);
  const int bm = first_bm + (t % (kW16GroupM * nbn)) % gm;
  const int bn = (t % (kW16GroupM * nbn)) / gm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int r32 = lane & 31;
  const int hj = lane >> 5;

  // Copy sources (byte offsets; rows past M and tiles past N are clamped,
  // their results are never stored; the host keeps 2*M*K and N*K/2 below
  // 2^31).  Step s adds 128 s bytes to A, and to B the block of group s/2
  // and its half s%2.
  const uint8_t* xa = reinterpret_cast<const uint8_t*>(ar.x);
  int a_off[A_LD], b_off[B_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int blk = wave * A_LD + i;          // rows 8*blk .. 8*blk+7
    const int row = blk * 8 + (lane >> 3);
    const int q = (lane & 7) ^ pf_swz(row);   // LDS chunk lane&7 of the row holds global chunk q
    a_off[i] = min(bm * BM + row, M - 1) * (2 * K) + q * 16;
  }
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int pair = wave * B_LD + i;         // 16-column tiles 2*pair, 2*pair+1 of the workgroup tile
    const int t16 = min(bn * (BN / 16) + 2 * pair + (lane >> 5), ntiles16 - 1);
    b_off[i] = t16 * G * 1024 + (lane & 31) * 16;
  }
  const int mcol = wave * MCOLS + (lane < MCOLS ? lane : 0);
  const int m_off = min(bn * (BN / 16) + (mcol >> 4), ntiles16 - 1) * G * 16 + (mcol & 15);

  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  auto issue = [&](int s, int stage) {
    const uint32_t base = lds0 + stage * STAGE;
    const int g = s >> 1;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) lds_copy16(xa + a_off[i] + s * 128, base + (wave * A_LD + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_LD; ++i)
      lds_copy16(ar.wpack + b_off[i] + g * 1024 + (s & 1) * 512, base + A_BYTES + (wave * B_LD + i) * 1024);
    if (lane < MCOLS) lds_copy4(ar.wmeta + m_off + g * 16, base + A_BYTES + B_BYTES + wave * MCOLS * 4);
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = v16f{};

  int arow[TM], bcol[TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) arow[tm] = wm * (BM / WM) + tm * 32 + r32;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) bcol[tn] = wn * (BN / WN) + tn * 32 + r32;

  // One step (64 k) from its stage: k-step i of lane half hj covers the
  // step's k 32 hj + 8 i + [0, 8) -- A chunk 4 hj + i of the row, dword i of
  // the lane's 16 bytes in the column's half block (slot 16 hj + col % 16).
  auto compute = [&](int stage, int is) {
    const uint8_t* As = smem + stage * STAGE;
    const uint8_t* Bs = As + A_BYTES;
    const uint32_t* Ms = reinterpret_cast<const uint32_t*>(Bs + B_BYTES);
    v2h s2[TN], z2[TN];
    v4i bw[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const uint32_t meta = Ms[bcol[tn]];
      s2[tn] = meta_s2(meta);
      z2[tn] = meta_z2(meta);
      bw[tn] = *reinterpret_cast<const v4i*>(Bs + (bcol[tn] >> 4) * 512 + (hj * 16 + (bcol[tn] & 15)) * 16);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = hj * 4 + i;
      v8h a[TM], b[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        a[tm] = *reinterpret_cast<const v8h*>(As + arow[tm] * 128 + ((q ^ pf_swz(arow[tm])) << 4));
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) b[tn] = dequant8(static_cast<uint32_t>(bw[tn][i]), s2[tn], z2[tn]);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[tm], b[tn], acc[tm][tn], 0, 0, 0);
      if (i == 1 && is < S) issue(is, is % kW16Stages);
    }
  };

  // Stage s % 4 holds step s.  Before computing s, each wave waits for its
  // own copies of s (those of s+1 and s+2 may stay in flight), then a
  // barrier makes everybody's copies of s visible and retires everybody's
  // reads of the stage that step s+3 is about to overwrite (step s-1's).
  issue(0, 0);
  if (S > 1) issue(1, 1);
  if (S > 2) issue(2, 2);
  for (int s = 0; s < S; ++s) {
    const int ahead = min(S - 1 - s, kW16Stages - 2);
    if (ahead >= 2) wait_vmcnt<2 * LOADS>();
    else if (ahead == 1) wait_vmcnt<LOADS>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    compute(s % kW16Stages, s + kW16Stages - 1);
  }

  // Output, one 32-row slice per wave row at a time, staged through LDS in
  // the output type and stored 16 bytes per lane, non-temporal.
  static_assert(kW16Stages * STAGE >= WM * 32 * (BN * 4 + 32), "output slice fits in the stage ring");
  const bool has_bias = ar.bias != nullptr;
  float bv[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
    bv[tn] = has_bias ? pq_load_dyn(ar.bias, bias_dtype, min(bn * BN + bcol[tn], N - 1)) : 0.0f;
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
          float val = acc[tm][tn][v];
          if (has_bias) val = val + bv[tn];
          uint8_t* dst = smem + (wm * 32 + r) * PITCH + bcol[tn] * ESZ;
          if constexpr (DT == PQ_F32) *reinterpret_cast<float*>(dst) = val;
          else if constexpr (DT == PQ_F16) *reinterpret_cast<uint16_t*>(dst) = pq_f32_to_f16(val);
          else *reinterpret_cast<uint16_t*>(dst) = pq_f32_to_bf16(val);
        }
      }
      lds_barrier();
      for (int e = threadIdx.x; e < WM * 32 * CPR; e += NW * 64) {
        const int sr = e / CPR, cc = e % CPR;
        const int64_t m = static_cast<int64_t>(bm) * BM + (sr >> 5) * (BM / WM) + tm * 32 + (sr & 31);
        const int n0 = bn * BN + cc * (16 / ESZ);
        if (m < M && n0 < N)
          __builtin_nontemporal_store(*reinterpret_cast<const v4i*>(smem + sr * PITCH + cc * 16),
                                      reinterpret_cast<v4i*>(static_cast<uint8_t*>(ar.y) + (m * N + n0) * ESZ));
      }
    }
  };
  if (y_dtype == PQ_F32) emit(std::integral_constant<int, PQ_F32>{});
  else if (y_dtype == PQ_F16) emit(std::integral_constant<int, PQ_F16>{});
  else emit(std::integral_constant<int, PQ_BF16>{});
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN>
void launch_w16_prefill_t(const W16Args& ar, int bias_dtype, int y_dtype, int M, int K, hipStream_t stream) {
  constexpr int STAGE = BM * 128 + (BN / 16) * 512 + BN * 4;
  const unsigned grid = static_cast<unsigned>(((M + BM - 1) / BM) * ((ar.n + BN - 1) / BN));
  w16_prefill<BM, BN, WM, WN><<<grid, WM * WN * 64, kW16Stages * STAGE, stream>>>(ar, bias_dtype, y_dtype, M, K);
}

// 32 x 128 tiles when one round of them covers the output (below); else the
// cheapest of 192 x 256, 128 x 256 (8 waves of 192 or 128 rows x 32
// columns) and 128 x 128 tiles (4 waves) by the measured cost of their
// rounds of 256 workgroups (one per CU), in units of a full round of
// 192 x 256 tiles (K = 4096): a full round of 128 x 256 tiles takes 0.74 of
// it and one of 128 x 128 tiles 0.45; a last, partly filled round costs 0.77
// of a full one on 192 x 256 tiles and 0.9 on the smaller ones.  M = 4096,
// N = 4096: 171 -> 144 us (128 x 256); M = 1024, N = 4096: 46 us on 128 x 128
// against 57 us on 128 x 256.
void launch_w16_prefill(const W16Args& ar, int bias_dtype, int y_dtype, int M, int K, hipStream_t stream) {
  auto rounds = [](int64_t tiles, double full, double partial) {
    return full * static_cast<double>(tiles / 256) + (tiles % 256 != 0 ? full * partial : 0.0);
  };
  const double big = rounds(static_cast<int64_t>((M + 191) / 192) * ((ar.n + 255) / 256), 1.0, 0.77);
  const double mid = rounds(static_cast<int64_t>((M + 127) / 128) * ((ar.n + 255) / 256), 0.74, 0.9);
  const double small = rounds(static_cast<int64_t>((M + 127) / 128) * ((ar.n + 127) / 128), 0.45, 0.9);
  if (big <= mid && big <= small) launch_w16_prefill_t<192, 256, 1, 8>(ar, bias_dtype, y_dtype, M, K, stream);
  else if (mid <= small) launch_w16_prefill_t<128, 256, 1, 8>(ar, bias_dtype, y_dtype, M, K, stream);
  // at most one round of 32-row tiles (17-256 tokens at N = 4096): each
  // workgroup walks all of K, so its time follows its rows (M = 64-256: 42
  // -> 26 us at K = 4096, M = 128: 115 -> 71 us at K = 12288 against 128 x 128)
  else if (static_cast<int64_t>((M + 31) / 32) * ((ar.n + 127) / 128) <= 256)
    launch_w16_prefill_t<32, 128, 1, 4>(ar, bias_dtype, y_dtype, M, K, stream);
  else launch_w16_prefill_t<128, 128, 1, 4>(ar, bias_dtype, y_dtype, M, K, stream);
}

struct W16SkinnyCfg {
  int nt, w, u;
};

// About 4-6 waves per SIMD over the grid, two column tiles per workgroup
// for wide outputs (768+ tiles) and where one tile per workgroup would put
// one workgroup on some CUs and two on others (256 < tiles < 512: the
// q/k/v group's 384 tiles, grouped layer at M = 1 43.7 -> 43.3 us), never
// more waves than K groups, and the
// shallowest batch of at least two groups that divides the K groups.
// In a group, n is the members' total and two tiles per workgroup need an
// even tile count in every member.
W16SkinnyCfg choose_w16_skinny(int64_t n, int64_t k, bool even = true) {
  const int G = static_cast<int>(k / 128);
  const int tiles = static_cast<int>(n / 16);
  const int nt = (even && tiles % 2 == 0 && (tiles >= 768 || (tiles > 256 && tiles < 512))) ? 2 : 1;
  const int64_t wgs = tiles / nt;
  int w = wgs * 16 <= 6144 ? 16 : wgs * 8 <= 6144 ? 8 : 4;
  while (w > 4 && w > G) w >>= 1;
  int u = 2;
  if (G <= w) u = 1;
  else if (G % (w * 2) == 0) u = 2;
  else if (G % (w * 3) == 0) u = 3;
  else if (G % (w * 4) == 0) u = 4;
  return {nt, w, u};
}

template <int NT, int W, int U>
void launch_w16_skinny_nwu(W16Group grp, int bias_dtype, int y_dtype, int M, int K, hipStream_t stream) {
  grp.first[0] = 0;
  for (int i = 0; i < grp.count; ++i) grp.first[i + 1] = grp.first[i] + grp.mem[i].n / 16 / NT;
  const unsigned grid = static_cast<unsigned>(grp.first[grp.count]);
  w16_skinny<NT, W, U><<<grid, W * 64, 0, stream>>>(grp, bias_dtype, y_dtype, M, K);
}

void launch_w16_skinny(const W16Group& grp, int bias_dtype, int y_dtype, int M, int K, hipStream_t stream) {
  int64_t n = 0;
  bool even = true;
  for (int i = 0; i < grp.count; ++i) {
    n += grp.mem[i].n;
    even = even && (grp.mem[i].n / 16) % 2 == 0;
  }
  const W16SkinnyCfg cfg = choose_w16_skinny(n, K, even);
#define PQ_W16(NT_, W_, U_)                                                        \
  if (cfg.nt == NT_ && cfg.w == W_ && cfg.u == U_) {                               \
    launch_w16_skinny_nwu<NT_, W_, U_>(grp, bias_dtype, y_dtype, M, K, stream);     \
    return;                                                                        \
  }
#define PQ_W16_NT(NT_)                                                             \
  PQ_W16(NT_, 4, 1) PQ_W16(NT_, 4, 2) PQ_W16(NT_, 4, 3) PQ_W16(NT_, 4, 4)          \
  PQ_W16(NT_, 8, 1) PQ_W16(NT_, 8, 2) PQ_W16(NT_, 8, 3) PQ_W16(NT_, 8, 4)          \
  PQ_W16(NT_, 16, 1) PQ_W16(NT_, 16, 2) PQ_W16(NT_, 16, 3) PQ_W16(NT_, 16, 4)
  PQ_W16_NT(1)
  PQ_W16_NT(2)
#undef PQ_W16_NT
#undef PQ_W16
  // every configuration choose_w16_skinny makes is listed above
  if (cfg.nt == 2) launch_w16_skinny_nwu<2, 4, 4>(grp, bias_dtype, y_dtype, M, K, stream);
  else launch_w16_skinny_nwu<1, 4, 4>(grp, bias_dtype, y_dtype, M, K, stream);
}

// Decode sizes: one skinny launch over all members; larger m: one prefill
// launch per member.
void launch_w16_gemm_group(const W16Group& grp, int bias_dtype, int y_dtype, int M, int K, hipStream_t stream) {
  if (M <= kW16SkinnyRows) {
    launch_w16_skinny(grp, bias_dtype, y_dtype, M, K, stream);
  } else {
    for (int i = 0; i < grp.count; ++i) launch_w16_prefill(grp.mem[i], bias_dtype, y_dtype, M, K, stream);
  }
}

void launch_w16_gemm(const W16Args& ar, int bias_dtype, int y_dtype, int M, int K, hipStream_t stream) {
  W16Group grp{};
  grp.mem[0] = ar;
  grp.count = 1;
  launch_w16_gemm_group(grp, bias_dtype, y_dtype, M, K, stream);
}

int check_w16_args(const char* who, int64_t m, int64_t n, int64_t k, int bias_dtype, const void* bias, int y_dtype) {
  PQ_REQUIRE(m >= 0 && m <= 0x7fffffffLL, PQ_ERR_ARG, "%s: m=%lld", who, (long long)m);
  PQ_REQUIRE(n > 0 && n % 16 == 0 && n <= (1 << 20), PQ_ERR_ARG, "%s: n=%lld must be a positive multiple of 16", who,
             (long long)n);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= (1 << 20), PQ_ERR_ARG, "%s: k=%lld must be a positive multiple of 128",
             who, (long long)k);
  // the kernels address A (in bytes) and the packed weights with 32-bit offsets
  PQ_REQUIRE(2 * m * k < (int64_t(1) << 31) && n * k / 2 < (int64_t(1) << 31), PQ_ERR_ARG,
             "%s: 2*m*k=%lld and n*k/2=%lld must stay below 2^31", who, (long long)(2 * m * k),
             (long long)(n * k / 2));
  PQ_REQUIRE(y_dtype == PQ_F32 || y_dtype == PQ_F16 || y_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED, "%s: y dtype code %d",
             who, y_dtype);
  PQ_REQUIRE(bias == nullptr || bias_dtype == PQ_F32 || bias_dtype == PQ_F16 || bias_dtype == PQ_BF16,
             PQ_ERR_UNSUPPORTED, "%s: bias dtype code %d", who, bias_dtype);
  return PQ_OK;
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Workspace of the linear (one block per member of a group): the rotated
// fp16 rows [m][k] (256-byte aligned size), then -- decode sizes, where the
// split rotation runs -- its per-group maxima (unused by this GEMM); the
// block is rounded up to 256 bytes so that every member's rows start
// 256-byte aligned (the GEMM reads them with 16-byte vector loads).
size_t w16_linear_workspace(int64_t m, int64_t k) {
  if (m <= 0 || k <= 0 || k % 128) return 0;
  const size_t rows = align_up(static_cast<size_t>(m) * k * 2, 256);
  if (m <= pq::kSplitMaxRows) return align_up(rows + static_cast<size_t>(m) * (k / 128) * sizeof(float), 256);
  return rows;
}

}  // namespace

extern "C" int pq_w4a16_gemm(const void* x, const uint8_t* wpack, const uint32_t* wmeta, const void* bias,
                             int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n, int64_t k, int group_size,
                             void* stream) {
  PQ_REQUIRE(group_size == 128, PQ_ERR_UNSUPPORTED, "pq_w4a16_gemm: group_size=%d (only 128 is supported)",
             group_size);
  int st = check_w16_args("pq_w4a16_gemm", m, n, k, bias_dtype, bias, y_dtype);
  if (st != PQ_OK) return st;
  if (m == 0) return PQ_OK;
  PQ_REQUIRE(x && wpack && wmeta && y, PQ_ERR_ARG, "pq_w4a16_gemm: null pointer");
  PQ_REQUIRE(pq::aligned_to(x, 16) && pq::aligned_to(wpack, 16) && pq::aligned_to(wmeta, 4) &&
                 pq::aligned_to(y, pq::dtype_size(y_dtype)),
             PQ_ERR_ARG, "pq_w4a16_gemm: x and wpack must be 16-byte aligned");
  const W16Args ar = {static_cast<const uint16_t*>(x), wpack, wmeta, bias, y, static_cast<int>(n)};
  launch_w16_gemm(ar, bias_dtype, y_dtype, static_cast<int>(m), static_cast<int>(k),
                  static_cast<hipStream_t>(stream));
  return pq::launch_status("pq_w4a16_gemm launch");
}

extern "C" size_t pq_w4a16_linear_workspace_size(int64_t m, int64_t k) { return w16_linear_workspace(m, k); }

namespace {

// The rotations of all members in one launch (grid.y = member), each into
// its own workspace block, then one GEMM launch over all members at decode
// sizes.
int w16_linear_group(const char* who, const void* x, int x_dtype, const pq_linear_member* members, int count,
                     int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot, unsigned flags, void* workspace,
                     size_t workspace_bytes, hipStream_t s) {
  PQ_REQUIRE(count >= 1 && count <= pq::kMaxGroup, PQ_ERR_ARG, "%s: count=%d not in 1..%d", who, count,
             pq::kMaxGroup);
  PQ_REQUIRE(members != nullptr, PQ_ERR_ARG, "%s: null member table", who);
  for (int i = 0; i < count; ++i) {
    int st = check_w16_args(who, m, members[i].n, k, bias_dtype, members[i].bias, y_dtype);
    if (st != PQ_OK) return st;
  }
  PQ_REQUIRE(k <= 16384, PQ_ERR_ARG, "%s: k=%lld must be at most 16384", who, (long long)k);
  PQ_REQUIRE(krot >= 1 && krot <= 16, PQ_ERR_UNSUPPORTED, "%s: krot=%d not in 1..16", who, krot);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED, "%s: x dtype code %d",
             who, x_dtype);
  PQ_REQUIRE((flags & ~static_cast<unsigned>(PQ_RQ_INPUT_FP16)) == 0, PQ_ERR_ARG, "%s: unknown flags 0x%x", who,
             flags);
  if (m == 0) return PQ_OK;
  PQ_REQUIRE(x && pq::aligned_to(x, 16), PQ_ERR_ARG, "%s: x must be non-null and 16-byte aligned", who);
  for (int i = 0; i < count; ++i) {
    const pq_linear_member& mb = members[i];
    PQ_REQUIRE(mb.rot_idx && mb.rot_cs && mb.wpack && mb.wmeta && mb.y, PQ_ERR_ARG, "%s: member %d: null pointer",
               who, i);
    PQ_REQUIRE(pq::aligned_to(mb.rot_idx, 16) && pq::aligned_to(mb.rot_cs, 16) && pq::aligned_to(mb.wpack, 16) &&
                   pq::aligned_to(mb.wmeta, 4) && pq::aligned_to(mb.y, pq::dtype_size(y_dtype)),
               PQ_ERR_ARG, "%s: member %d: misaligned pointer", who, i);
  }
  const size_t per = w16_linear_workspace(m, k);
  const size_t need = count * per;
  PQ_REQUIRE(workspace != nullptr && workspace_bytes >= need && pq::aligned_to(workspace, 256), PQ_ERR_WORKSPACE,
             "%s: a 256-byte aligned workspace of %zu bytes is needed for m=%lld k=%lld count=%d, got %zu", who, need,
             (long long)m, (long long)k, count, workspace ? workspace_bytes : (size_t)0);

  // The rotation writes its result rounded to fp16 (the reference's
  // rotation output for fp16 activations), which is this GEMM's A operand.
  const int M = static_cast<int>(m), K = static_cast<int>(k);
  char* ws = static_cast<char*>(workspace);
  const bool split = m <= pq::kSplitMaxRows;
  pq::RotGroup rg{};
  W16Group gg{};
  rg.count = gg.count = count;
  for (int i = 0; i < count; ++i) {
    const pq_linear_member& mb = members[i];
    char* rows = ws + i * per;
    float* gmax = reinterpret_cast<float*>(rows + align_up(static_cast<size_t>(m) * k * 2, 256));
    if (split) rg.mem[i] = {mb.rot_idx, mb.rot_cs, mb.scales, rows, gmax, nullptr};
    else rg.mem[i] = {mb.rot_idx, mb.rot_cs, mb.scales, nullptr, nullptr, rows};
    gg.mem[i] = {reinterpret_cast<const uint16_t*>(rows), mb.wpack, mb.wmeta, mb.bias, mb.y, static_cast<int>(mb.n)};
  }
  const unsigned rflags = flags | PQ_RQ_MATERIALIZE_FP16;
  if (split) pq::launch_rotate_split(x, x_dtype, rg, M, K, krot, rflags, s);
  else pq::launch_rotate_quant_group(x, x_dtype, rg, m, K, krot, rflags, s);
  int st = pq::launch_status("W4A16 linear rotation launch");
  if (st != PQ_OK) return st;
  launch_w16_gemm_group(gg, bias_dtype, y_dtype, M, K, s);
  return pq::launch_status("W4A16 linear GEMM launch");
}

}  // namespace

extern "C" int pq_w4a16_linear(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                               const float* scales, const uint8_t* wpack, const uint32_t* wmeta, const void* bias,
                               int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n, int64_t k, int krot,
                               unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  const pq_linear_member one = {rot_idx, rot_cs, scales, wpack, wmeta, bias, y, n};
  return w16_linear_group("pq_w4a16_linear", x, x_dtype, &one, 1, bias_dtype, y_dtype, m, k, krot, flags, workspace,
                          workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" size_t pq_w4a16_linear_group_workspace_size(int64_t m, int64_t k, int count) {
  if (count < 1 || count > pq::kMaxGroup) return 0;
  return count * w16_linear_workspace(m, k);
}

extern "C" int pq_w4a16_linear_group(const void* x, int x_dtype, const pq_linear_member* members, int count,
                                     int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot, unsigned flags,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  return w16_linear_group("pq_w4a16_linear_group", x, x_dtype, members, count, bias_dtype, y_dtype, m, k, krot, flags,
                          workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
