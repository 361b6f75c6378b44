// The whole W4A8 linear (rotation + channel scale + per-token int8 quant +
// int4 x int8 GEMM) behind one entry point, pq_w4a8_linear.  Two or three
// launches, chosen by the number of tokens m and the row length k:
//
//   split (decode: m * k <= 8192, one or two tokens of 4096 channels, or
//     up to 2 tokens when k >= 8192): the rotation runs with
//     one wave per 128-channel group (K/128 waves spread over the chip, each
//     rotation parameter read once) and writes the rotated rows plus each
//     row's absmax per group; the decode GEMM derives the token scales and
//     quantizes A into LDS in its prologue, while its first weight blocks
//     are already in flight.
//   split3 (k >= 4096 beyond that, up to 64 tokens): the split rotation
//     with the rows spread over waves, a token-scale + int8 kernel, then
//     the decode GEMM on int8 A (three launches).
//   rows (otherwise): pq_rotate_quant_i8 (rotation + absmax + int8 quant of
//     whole rows per workgroup) into the caller's workspace, then
//     pq_w4a8_gemm.
//
// A one-kernel variant (every workgroup rotating the token itself) was
// measured slower: the K/128 x 5 KB of rotation parameters, re-read by each
// of ~256 workgroups, saturate the per-CU load path ahead of the weights.
//
// Reference: BF16RotateLinearWrapper -> RotateLinearInt4 -> rotation::rotate
// -> MarlinW4A8Linear (src/alpamayo_r1/utils/quantization/
// paroquant_marlin_w4a8.py:59-65, 314-333; rotation_linear.py:120-124).
#include <mutex>

#include "pq_device.h"
#include "pq_internal.h"

// Scratch of pq_w4a8_linear_noalloc: one array per GPU, resident until the
// process ends.  Host code never uses this name as an address (on the host it
// is only a handle); it reads each device's address once with
// hipGetSymbolAddress and passes that pointer to the kernels.
static __device__ __align__(256) unsigned char scratch[PQ_NOALLOC_SCRATCH_BYTES];

namespace {

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Measured on the Qwen3-8B shapes: the split path wins up to two tokens of
// 4096 channels (m * k <= 8192; the grouped decode layer at m = 3: 52.1 us
// on the row kernel against 55.1 us split, m = 4: 53.7 against 59.3 us; at
// m = 2 the row kernel loses, 49.2 against 47.0 us), and for long rows up
// to 2 tokens (from 3 the three-launch path below wins with one row per
// wave: the layer at m = 3 51.9 -> 50.3 us, m = 4 53.6 -> 50.9 us).
bool use_split(int64_t m, int64_t k) {
  return (m * k <= 8192 || (k >= 8192 && m <= 2)) && pq::gemm_rotated_supported(m, k);
}

// Rows of 4096 channels or more past the split pair, up to 64 tokens: the
// split rotation with its rows spread over waves (kSplitRowsPerWave rows
// each), a small kernel for the token scales and int8 codes, then the decode
// GEMM on int8 A.  The row kernel runs each row on one CU, whose VALU needs
// about 12 us for the 96 groups of a 12288-channel row (down, k = 12288, at
// m = 6: 17.8 us against 22.2 us; m = 16: 20.0 / 24.0).  At k = 4096 the
// three launches win too once the token-scale kernel requests its rows
// together with the group maxima (the grouped decode layer at m = 4:
// 50.0 -> 49.2 us, m = 16: 59.4 -> 59.1 us; the 36-layer verify block
// 2.298 -> 2.268 ms, where the RMSNorm in front of gate/up runs in the split
// rotation).  One row per wave: the verify block at 16 tokens 2.40 -> 2.34 ms
// against four rows per wave (2.36 ms with two, 2.50 ms with eight).
constexpr int kSplitRowsPerWave = 1;
// Up to 64 tokens: with one row per wave the split rotation takes any row
// count, and the decode GEMM on int8 A takes 64 rows (up to four row blocks
// per workgroup).  At 17-64 tokens the row kernel would run each
// 12288-channel row on one CU (the decode layer at M = 17: 80.1 us with down
// on the row kernel), and from 33 tokens the prefill GEMM's tiles re-read
// the weights per row tile.
constexpr int kSplit3MaxRows = 64;
bool use_split3(int64_t m, int64_t k) {
  return !use_split(m, k) && m >= 1 && m <= kSplit3MaxRows && k >= 4096 && k <= 16384 && k % 128 == 0;
}

enum class Path { kSplit, kSplit3, kRows };
Path choose_path(int64_t m, int64_t k) {
  return use_split(m, k) ? Path::kSplit : use_split3(m, k) ? Path::kSplit3 : Path::kRows;
}

size_t split_xr_bytes(int64_t m, int64_t k) { return align_up(static_cast<size_t>(m) * k * sizeof(float), 256); }
size_t xq_bytes(int64_t m, int64_t k) { return align_up(static_cast<size_t>(m) * k, 256); }

// Per member: the bytes of its row data (a) and of its per-row scalars (s).
// The workspace of a group of `count` linears holds count a-blocks, then
// count s-blocks.  split: a = rotated rows (fp32 bound), s = group maxima
// [m][k/128]; split3: a = rotated rows then int8 codes, s = group maxima then
// token scales [m]; rows: a = int8 codes, s = token scales.
void block_bytes(Path path, int64_t m, int64_t k, size_t* a, size_t* s) {
  const size_t gm = static_cast<size_t>(m) * (k / 128) * sizeof(float), ts = static_cast<size_t>(m) * sizeof(float);
  switch (path) {
    case Path::kSplit: *a = split_xr_bytes(m, k); *s = gm; break;
    case Path::kSplit3: *a = split_xr_bytes(m, k) + xq_bytes(m, k); *s = gm + ts; break;
    default: *a = xq_bytes(m, k); *s = ts; break;
  }
}

size_t group_workspace_size(int64_t m, int64_t k, int count) {
  if (m <= 0 || k <= 0 || k % 128 || count < 1 || count > pq::kMaxGroup) return 0;
  size_t a = 0, s = 0;
  block_bytes(choose_path(m, k), m, k, &a, &s);
  return count * (a + s);
}

// Outputs of the parity entry point (pq_w4a8_linear_group_intermediates):
// the int8 A operand and token scales each member's GEMM uses, and its int32
// per-group partials.
struct Probe {
  int8_t* codes;      // [count][m][k]
  float* xscale;      // [count][m]
  int32_t* partials;  // member i: [m][k/128][n_i] at m * (k/128) * (n_0 + ... + n_{i-1})
};

// probe: run the linear's launches with the GEMM in its partials form and
// return the intermediates instead of y (members' bias and y unused).
// stage: 0 = every launch; 1 = the rotation (+ quant) launches only, into
// the workspace; 2 = the GEMM launch only, from what stage 1 left there.
int linear_group(const char* who, const void* x, int x_dtype, const pq_linear_member* members, int count,
                 int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot, unsigned flags, void* workspace,
                 size_t workspace_bytes, hipStream_t s, const pq::NormArgs* norm = nullptr,
                 const Probe* probe = nullptr, int stage = 0) {
  PQ_REQUIRE(count >= 1 && count <= pq::kMaxGroup, PQ_ERR_ARG, "%s: count=%d not in 1..%d", who, count,
             pq::kMaxGroup);
  PQ_REQUIRE(members != nullptr, PQ_ERR_ARG, "%s: null member table", who);
  PQ_REQUIRE(m >= 0 && m <= 0x7fffffffLL, PQ_ERR_ARG, "%s: m=%lld", who, (long long)m);
  PQ_REQUIRE(k > 0 && k % 128 == 0 && k <= 16384, PQ_ERR_ARG,
             "%s: k=%lld must be a positive multiple of 128, at most 16384", who, (long long)k);
  PQ_REQUIRE(krot >= 1 && krot <= 16, PQ_ERR_UNSUPPORTED, "%s: krot=%d not in 1..16", who, krot);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "%s: x dtype code %d", who, x_dtype);
  PQ_REQUIRE(y_dtype == PQ_F32 || y_dtype == PQ_F16 || y_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "%s: y dtype code %d", who, y_dtype);
  PQ_REQUIRE((flags & ~(PQ_RQ_INPUT_FP16 | PQ_RQ_MATERIALIZE_FP16)) == 0, PQ_ERR_ARG, "%s: unknown flags 0x%x",
             who, flags);
  bool any_bias = false;
  for (int i = 0; i < count; ++i) {
    const pq_linear_member& mb = members[i];
    PQ_REQUIRE(mb.n > 0 && mb.n % 16 == 0 && mb.n <= (1 << 20), PQ_ERR_ARG,
               "%s: member %d: n=%lld must be a positive multiple of 16", who, i, (long long)mb.n);
    PQ_REQUIRE(mb.n * k / 2 < (int64_t(1) << 31), PQ_ERR_ARG, "%s: member %d: n*k/2 must stay below 2^31", who, i);
    any_bias = any_bias || (mb.bias != nullptr && probe == nullptr);
  }
  PQ_REQUIRE(!any_bias || bias_dtype == PQ_F32 || bias_dtype == PQ_F16 || bias_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED,
             "%s: bias dtype code %d", who, bias_dtype);
  if (m == 0) return PQ_OK;
  PQ_REQUIRE(m * k < (int64_t(1) << 31), PQ_ERR_ARG, "%s: m*k=%lld must stay below 2^31", who, (long long)(m * k));
  PQ_REQUIRE(stage == 2 || (x && pq::aligned_to(x, 16)), PQ_ERR_ARG, "%s: x must be non-null and 16-byte aligned",
             who);
  for (int i = 0; i < count; ++i) {
    const pq_linear_member& mb = members[i];
    PQ_REQUIRE(mb.rot_idx && mb.rot_cs && mb.wpack && mb.wmeta && (mb.y || probe), PQ_ERR_ARG,
               "%s: member %d: null pointer", who, i);
    PQ_REQUIRE(pq::aligned_to(mb.rot_idx, 16) && pq::aligned_to(mb.rot_cs, 16) && pq::aligned_to(mb.wpack, 16) &&
                   pq::aligned_to(mb.wmeta, 4) && (probe || pq::aligned_to(mb.y, pq::dtype_size(y_dtype))),
               PQ_ERR_ARG, "%s: member %d: misaligned pointer", who, i);
  }
  if (probe != nullptr)
    PQ_REQUIRE(probe->codes && probe->xscale && probe->partials && pq::aligned_to(probe->codes, 16) &&
                   pq::aligned_to(probe->xscale, 4) && pq::aligned_to(probe->partials, 4),
               PQ_ERR_ARG, "%s: codes (16-byte aligned), xscale and partials must be non-null", who);
  const size_t need = group_workspace_size(m, k, count);
  PQ_REQUIRE(workspace != nullptr && workspace_bytes >= need && pq::aligned_to(workspace, 256), PQ_ERR_WORKSPACE,
             "%s: a 256-byte aligned workspace of %zu bytes is needed for m=%lld k=%lld count=%d, got %zu", who,
             need, (long long)m, (long long)k, count, workspace ? workspace_bytes : (size_t)0);

  const int M = static_cast<int>(m), K = static_cast<int>(k);
  char* ws = static_cast<char*>(workspace);
  pq::RotGroup rg{};
  pq::GemmGroup gg{};
  rg.count = gg.count = count;
  const Path path = choose_path(m, k);
  size_t a_bytes = 0, s_bytes = 0;
  block_bytes(path, m, k, &a_bytes, &s_bytes);
  const bool mat16 = (flags & PQ_RQ_MATERIALIZE_FP16) != 0;
  pq::QuantGroup qg{};
  qg.count = count;
  for (int i = 0; i < count; ++i) {
    const pq_linear_member& mb = members[i];
    char* a = ws + i * a_bytes;
    float* sc = reinterpret_cast<float*>(ws + count * a_bytes + i * s_bytes);
    rg.mem[i] = {mb.rot_idx, mb.rot_cs, mb.scales, a, sc, nullptr};
    if (path == Path::kSplit) {
      gg.mem[i] = {nullptr, nullptr, a, sc, mb.wpack, mb.wmeta, mb.bias, mb.y, static_cast<int>(mb.n)};
    } else if (path == Path::kSplit3) {
      int8_t* xq = reinterpret_cast<int8_t*>(a + split_xr_bytes(m, k));
      float* xs = sc + m * (k / 128);
      qg.mem[i] = {a, sc, xq, xs};
      gg.mem[i] = {xq, xs, nullptr, nullptr, mb.wpack, mb.wmeta, mb.bias, mb.y, static_cast<int>(mb.n)};
    } else {
      gg.mem[i] = {reinterpret_cast<const int8_t*>(a), sc, nullptr, nullptr, mb.wpack, mb.wmeta, mb.bias, mb.y,
                   static_cast<int>(mb.n)};
    }
  }
  int st = PQ_OK;
  if (stage == 2) {
    // the GEMM alone, from the workspace stage 1 filled
  } else if (path == Path::kRows) {
    pq::launch_rotate_quant_group(x, x_dtype, rg, m, K, krot, flags, s, norm);
    st = pq::launch_status("linear rotate+quant launch");
  } else {
    pq::launch_rotate_split(x, x_dtype, rg, M, K, krot, flags, s, norm,
                            path == Path::kSplit3 ? kSplitRowsPerWave : 0);
    st = pq::launch_status("linear rotation launch");
    if (st == PQ_OK && path == Path::kSplit3) {
      pq::launch_quant_split(qg, M, K, mat16, s);
      st = pq::launch_status("linear quant launch");
    }
  }
  if (st != PQ_OK || stage == 1) return st;
  const int aq = path == Path::kSplit ? (mat16 ? 1 : 2) : 0;
  if (probe == nullptr) {
    pq::launch_gemm_group(gg, aq, bias_dtype, y_dtype, M, K, s);
    return pq::launch_status("linear GEMM launch");
  }
  // Parity form.  On the split pair path the GEMM writes the A image it
  // quantized in its prologue; otherwise A is the int8 codes and scales the
  // earlier launches left in the workspace, copied out as they are.
  int64_t col0 = 0;
  for (int i = 0; i < count; ++i) {
    gg.mem[i].partials = probe->partials + m * (k / 128) * col0;
    gg.mem[i].a_out = probe->codes + i * m * k;
    gg.mem[i].as_out = probe->xscale + i * m;
    gg.mem[i].y = nullptr;
    gg.mem[i].bias = nullptr;
    col0 += members[i].n;
    if (path != Path::kSplit) {
      hipError_t e = hipMemcpyAsync(gg.mem[i].a_out, gg.mem[i].xq, static_cast<size_t>(m * k), hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess)
        e = hipMemcpyAsync(gg.mem[i].as_out, gg.mem[i].xs, static_cast<size_t>(m) * sizeof(float),
                           hipMemcpyDeviceToDevice, s);
      PQ_REQUIRE(e == hipSuccess, PQ_ERR_HIP, "%s: copy of member %d's A operand: %s", who, i, hipGetErrorString(e));
    }
  }
  pq::launch_gemm_group_partials(gg, aq, M, K, s);
  return pq::launch_status("linear GEMM partials launch");
}

// The prologue arguments of the fused group entry points, checked.
int prologue_args(const char* who, const void* x2, const void* norm_weight, float eps, int mode, void* h_out,
                  void* sum_out, int x_dtype, int64_t m, pq::NormArgs* out) {
  PQ_REQUIRE(mode == PQ_PRO_RMSNORM || mode == PQ_PRO_ADD || mode == PQ_PRO_SWIGLU, PQ_ERR_ARG, "%s: mode %d", who,
             mode);
  PQ_REQUIRE(x_dtype == PQ_F32 || x_dtype == PQ_F16 || x_dtype == PQ_BF16, PQ_ERR_UNSUPPORTED, "%s: x dtype code %d",
             who, x_dtype);
  if (mode == PQ_PRO_RMSNORM)
    PQ_REQUIRE(eps >= 0.0f && eps < 1.0f, PQ_ERR_ARG, "%s: eps=%g must be in [0, 1)", who, static_cast<double>(eps));
  if (m > 0) {
    const size_t es = static_cast<size_t>(pq::dtype_size(x_dtype));
    if (mode == PQ_PRO_RMSNORM)
      PQ_REQUIRE(norm_weight != nullptr && pq::aligned_to(norm_weight, es), PQ_ERR_ARG,
                 "%s: norm_weight must be non-null and aligned to its dtype", who);
    else
      PQ_REQUIRE(x2 != nullptr, PQ_ERR_ARG, "%s: mode %d needs x2 (the residual / up rows)", who, mode);
    PQ_REQUIRE(x2 == nullptr || pq::aligned_to(x2, 16), PQ_ERR_ARG, "%s: x2 (the residual or up rows) must be 16-byte aligned", who);
    PQ_REQUIRE((h_out == nullptr || pq::aligned_to(h_out, es)) && (sum_out == nullptr || pq::aligned_to(sum_out, es)),
               PQ_ERR_ARG, "%s: h_out and sum_out must be aligned to x's dtype", who);
    PQ_REQUIRE(sum_out == nullptr || (mode != PQ_PRO_SWIGLU && x2 != nullptr), PQ_ERR_ARG,
               "%s: sum_out needs a residual (and no SwiGLU)", who);
    PQ_REQUIRE(h_out == nullptr || mode != PQ_PRO_ADD, PQ_ERR_ARG, "%s: h_out has no meaning for the add", who);
  }
  *out = {x2, mode == PQ_PRO_RMSNORM ? norm_weight : nullptr, h_out, sum_out, eps, mode};
  return PQ_OK;
}

}  // namespace

extern "C" size_t pq_w4a8_linear_workspace_size(int64_t m, int64_t n, int64_t k, int krot) {
  (void)krot;
  if (n <= 0 || n % 16) return 0;
  return group_workspace_size(m, k, 1);
}

extern "C" int pq_w4a8_linear_split_path(int64_t m, int64_t k) {
  return m > 0 && choose_path(m, k) != Path::kRows ? 1 : 0;
}

extern "C" size_t pq_w4a8_linear_group_workspace_size(int64_t m, int64_t k, int count) {
  return group_workspace_size(m, k, count);
}

extern "C" int pq_w4a8_linear(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                              const float* scales, const uint8_t* wpack, const uint32_t* wmeta, const void* bias,
                              int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n, int64_t k, int krot,
                              unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  const pq_linear_member one = {rot_idx, rot_cs, scales, wpack, wmeta, bias, y, n};
  return linear_group("pq_w4a8_linear", x, x_dtype, &one, 1, bias_dtype, y_dtype, m, k, krot, flags, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream));
}

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up on the
// first call made with that device current.
int noalloc_scratch(const char* who, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  PQ_REQUIRE(e == hipSuccess, PQ_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  PQ_REQUIRE(dev >= 0 && dev < kMaxDevices, PQ_ERR_UNSUPPORTED, "%s: device %d beyond the %d devices supported",
             who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    PQ_REQUIRE(e == hipSuccess && p != nullptr, PQ_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s",
               who, dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PQ_OK;
}

}  // namespace

extern "C" int pq_w4a8_linear_noalloc(const void* x, int x_dtype, const uint32_t* rot_idx, const float* rot_cs,
                                      const float* scales, const uint8_t* wpack, const uint32_t* wmeta,
                                      const void* bias, int bias_dtype, void* y, int y_dtype, int64_t m, int64_t n,
                                      int64_t k, int krot, unsigned flags, void* stream) {
  const char* who = "pq_w4a8_linear_noalloc";
  // Size check first, on the host: nothing touches the GPU for a rejected call.
  const size_t need = group_workspace_size(m, k, 1);
  PQ_REQUIRE(need <= PQ_NOALLOC_SCRATCH_BYTES, PQ_ERR_WORKSPACE,
             "%s: m=%lld k=%lld needs %zu bytes of scratch, above the library's fixed %zu bytes "
             "(use pq_w4a8_linear with a workspace)",
             who, (long long)m, (long long)k, need, (size_t)PQ_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (m > 0 && need > 0) {
    const int st = noalloc_scratch(who, &ws);
    if (st != PQ_OK) return st;
  }
  const pq_linear_member one = {rot_idx, rot_cs, scales, wpack, wmeta, bias, y, n};
  return linear_group(who, x, x_dtype, &one, 1, bias_dtype, y_dtype, m, k, krot, flags, ws,
                      ws != nullptr ? (size_t)PQ_NOALLOC_SCRATCH_BYTES : 0, static_cast<hipStream_t>(stream));
}

extern "C" int pq_w4a8_linear_group(const void* x, int x_dtype, const pq_linear_member* members, int count,
                                    int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot, unsigned flags,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  return linear_group("pq_w4a8_linear_group", x, x_dtype, members, count, bias_dtype, y_dtype, m, k, krot, flags,
                      workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int pq_w4a8_linear_group_fused(const void* x, const void* x2, const void* norm_weight, float eps, int mode,
                                          void* h_out, void* sum_out, int x_dtype, const pq_linear_member* members,
                                          int count, int bias_dtype, int y_dtype, int64_t m, int64_t k, int krot,
                                          unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "pq_w4a8_linear_group_fused";
  pq::NormArgs pro{};
  const int st = prologue_args(who, x2, norm_weight, eps, mode, h_out, sum_out, x_dtype, m, &pro);
  if (st != PQ_OK) return st;
  return linear_group(who, x, x_dtype, members, count, bias_dtype, y_dtype, m, k, krot, flags, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream), &pro);
}

extern "C" int pq_w4a8_linear_group_stage(int stage, const void* x, const void* x2, const void* norm_weight, float eps,
                                          int mode, void* h_out, void* sum_out, int x_dtype,
                                          const pq_linear_member* members, int count, int bias_dtype, int y_dtype,
                                          int64_t m, int64_t k, int krot, unsigned flags, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  const char* who = "pq_w4a8_linear_group_stage";
  PQ_REQUIRE(stage == 1 || stage == 2, PQ_ERR_ARG, "%s: stage %d (1 = rotation launches, 2 = GEMM)", who, stage);
  pq::NormArgs pro{};
  if (stage == 1 && mode != 0) {
    const int st = prologue_args(who, x2, norm_weight, eps, mode, h_out, sum_out, x_dtype, m, &pro);
    if (st != PQ_OK) return st;
  }
  return linear_group(who, x, x_dtype, members, count, bias_dtype, y_dtype, m, k, krot, flags, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream), stage == 1 && mode != 0 ? &pro : nullptr,
                      nullptr, stage);
}

extern "C" int pq_w4a8_linear_group_intermediates(const void* x, const void* x2, const void* norm_weight, float eps,
                                                  int mode, void* h_out, void* sum_out, int x_dtype,
                                                  const pq_linear_member* members, int count, int64_t m, int64_t k,
                                                  int krot, unsigned flags, void* workspace, size_t workspace_bytes,
                                                  int8_t* codes, float* xscale, int32_t* partials, void* stream) {
  const char* who = "pq_w4a8_linear_group_intermediates";
  pq::NormArgs pro{};
  if (mode != 0) {
    const int st = prologue_args(who, x2, norm_weight, eps, mode, h_out, sum_out, x_dtype, m, &pro);
    if (st != PQ_OK) return st;
  }
  const Probe probe = {codes, xscale, partials};
  return linear_group(who, x, x_dtype, members, count, PQ_BF16, PQ_BF16, m, k, krot, flags, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream), mode != 0 ? &pro : nullptr, &probe);
}

extern "C" int pq_w4a8_linear_group_rmsnorm(const void* x, const void* residual, const void* norm_weight, float eps,
                                            void* h_out, void* sum_out, int x_dtype,
                                            const pq_linear_member* members, int count, int bias_dtype,
                                            int y_dtype, int64_t m, int64_t k, int krot, unsigned flags,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  return pq_w4a8_linear_group_fused(x, residual, norm_weight, eps, PQ_PRO_RMSNORM, h_out, sum_out, x_dtype, members,
                                    count, bias_dtype, y_dtype, m, k, krot, flags, workspace, workspace_bytes,
                                    stream);
}
