// Host-side packing of rotation parameters into the kernels' operand layout.
//
// Reference parameters (src/alpamayo_r1/utils/quantization/rotation_linear.py:
// 39-43): pairs int16 [krot][h] with group-local indices (pair t of group g in
// layer r = pairs[r][g*128+2t], pairs[r][g*128+2t+1]) and angles [krot][h/2].
//
// The kernels rotate a 128-channel group with one wave and keep the data in
// registers: lane l loads channels l and l+64 (coalesced), and in every layer
// it holds the two channels of one pair in two slots A and B.  Before each
// layer a lane keeps one of its channels and fetches the other from the lane
// that holds it, with one ds_bpermute.  That works because the pairs of two
// consecutive layers form a union of even cycles (alternating between the
// two layers): walking each cycle, call the channel a pair shares with the
// next pair of the following layer "kept" and its other channel "given"; the
// lane of a pair then moves on to the pair of the next layer that contains
// its kept channel and receives the given channel of the next pair on the
// walk.  The load layout counts as a layer before the first one, with lane l
// holding the pair (l, l+64).  Slot A always holds the channel given away
// next, so every fetch reads slot A of its source lane; a per-layer flag says
// whether the received value enters slot A or slot B.
//
// Operands (KP = 8 for krot <= 8, else 16):
//   rot_idx [G][64][KP/2] uint32, per lane:
//     word 0      Af | Bf << 8 | init << 16: the channels in slots A and B
//                 after the last layer, and whether slot A starts with
//                 channel l+64 (else l)
//     byte 4 + r  (layer r = 0 .. krot-1) src | flag << 7: the lane the
//                 channel received before layer r comes from, and whether it
//                 enters slot A
//   rot_cs  [G][64][KP][2] float32 (cos, sin) of the lane's pair in layer r,
//                 sin negated when slot A holds the pair's second channel.
// A Givens update on (i, j) with angle theta equals the update on (j, i)
// with -theta bit for bit in the kernels' float32 form
//   a' = fma(a, c, b*s),  b' = fma(b, c, -(a*s))
// since b*(-s) == -(b*s) exactly, so the slot order is free.
#include <algorithm>
#include <cstring>
#include <vector>

#include "pq_common.h"

namespace {

struct Layer {
  int i[64], j[64];   // pair t = (first, second) as stored
  float c[64], s[64];
  int pos[128];       // channel -> pair index
};

}  // namespace

extern "C" int pq_rotation_pack(const int16_t* pairs, const float* cos_sin, int64_t h, int krot, uint32_t* rot_idx,
                                float* rot_cs) {
  PQ_REQUIRE(pairs && cos_sin && rot_idx && rot_cs, PQ_ERR_ARG, "pq_rotation_pack: null pointer");
  PQ_REQUIRE(h > 0 && h % 128 == 0 && h <= (1 << 20), PQ_ERR_ARG, "pq_rotation_pack: h=%lld", (long long)h);
  PQ_REQUIRE(krot >= 1 && krot <= 16, PQ_ERR_ARG, "pq_rotation_pack: krot=%d not in 1..16", krot);
  const int G = static_cast<int>(h / 128);
  const int KP = krot <= 8 ? 8 : 16;
  const int KW = KP / 2;
  const int NL = krot + 1;   // layer 0 = the load layout (l, l+64); layer k = reference layer k-1
  std::memset(rot_idx, 0, sizeof(uint32_t) * G * 64 * KW);
  std::memset(rot_cs, 0, sizeof(float) * G * 64 * KP * 2);
  std::vector<Layer> L(NL);
  for (int t = 0; t < 64; ++t) {
    L[0].i[t] = t;
    L[0].j[t] = t + 64;
    L[0].c[t] = 1.0f;
    L[0].s[t] = 0.0f;
    L[0].pos[t] = t;
    L[0].pos[t + 64] = t;
  }
  std::vector<int> give(NL * 64), nextpair(NL * 64), srcpair(NL * 64), lane_of(NL * 64);
  std::vector<int> slotA(NL * 64), slotB(NL * 64), src(NL * 64), flag(NL * 64);
  for (int g = 0; g < G; ++g) {
    for (int r = 0; r < krot; ++r) {
      Layer& l = L[r + 1];
      int seen[128] = {0};
      for (int t = 0; t < 64; ++t) {
        const int a = pairs[static_cast<int64_t>(r) * h + g * 128 + 2 * t];
        const int b = pairs[static_cast<int64_t>(r) * h + g * 128 + 2 * t + 1];
        PQ_REQUIRE(a >= 0 && a < 128 && b >= 0 && b < 128, PQ_ERR_ARG,
                   "pq_rotation_pack: pair index out of [0,128) in layer %d group %d", r, g);
        ++seen[a];
        ++seen[b];
        l.i[t] = a;
        l.j[t] = b;
        l.c[t] = cos_sin[(static_cast<int64_t>(r) * (h / 2) + g * 64 + t) * 2];
        l.s[t] = cos_sin[(static_cast<int64_t>(r) * (h / 2) + g * 64 + t) * 2 + 1];
        l.pos[a] = t;
        l.pos[b] = t;
      }
      for (int ch = 0; ch < 128; ++ch)
        PQ_REQUIRE(seen[ch] == 1, PQ_ERR_ARG,
                   "pq_rotation_pack: layer %d group %d does not pair every channel exactly once", r, g);
    }
    // Orientation of layer k's pairs from the cycles of layers k and k+1.
    std::fill(give.begin(), give.end(), -1);
    for (int k = 0; k + 1 < NL; ++k) {
      const Layer& a = L[k];
      const Layer& b = L[k + 1];
      for (int t0 = 0; t0 < 64; ++t0) {
        if (give[k * 64 + t0] >= 0) continue;
        int e = t0;
        int gv = a.i[e];   // the walk enters pair e through its given channel
        while (give[k * 64 + e] < 0) {
          const int keep = (a.i[e] == gv) ? a.j[e] : a.i[e];
          give[k * 64 + e] = gv;
          const int f = b.pos[keep];
          const int z = (b.i[f] == keep) ? b.j[f] : b.i[f];   // f's other channel
          const int e2 = a.pos[z];                              // the pair that gives z to f
          nextpair[k * 64 + e] = f;
          srcpair[(k + 1) * 64 + f] = e2;
          e = e2;
          gv = z;
        }
      }
    }
    // Lanes: layer 0 pair t is lane t; later layers inherit.
    for (int t = 0; t < 64; ++t) lane_of[t] = t;
    for (int k = 0; k + 1 < NL; ++k)
      for (int t = 0; t < 64; ++t) lane_of[(k + 1) * 64 + nextpair[k * 64 + t]] = lane_of[k * 64 + t];
    // Slots: A = the channel given away next (the last layer keeps its fetch order).
    for (int k = 0; k < NL; ++k) {
      const Layer& l = L[k];
      for (int t = 0; t < 64; ++t) {
        const int lane = lane_of[k * 64 + t];
        int A, B;
        if (k == 0) {
          A = give[t];
          B = (A == l.i[t]) ? l.j[t] : l.i[t];
        } else {
          const int e2 = srcpair[k * 64 + t];
          const int recv = give[(k - 1) * 64 + e2];
          const int keep = (l.i[t] == recv) ? l.j[t] : l.i[t];
          const int want = give[k * 64 + t] >= 0 ? give[k * 64 + t] : recv;
          const int fl = (want == recv) ? 1 : 0;
          A = fl ? recv : keep;
          B = fl ? keep : recv;
          src[k * 64 + lane] = lane_of[(k - 1) * 64 + e2];
          flag[k * 64 + lane] = fl;
          const int64_t o = (static_cast<int64_t>(g) * 64 + lane) * KP + (k - 1);
          rot_cs[2 * o] = l.c[t];
          rot_cs[2 * o + 1] = (A == l.i[t]) ? l.s[t] : -l.s[t];
        }
        slotA[k * 64 + lane] = A;
        slotB[k * 64 + lane] = B;
      }
    }
    for (int lane = 0; lane < 64; ++lane) {
      uint32_t* w = rot_idx + (static_cast<int64_t>(g) * 64 + lane) * KW;
      w[0] = static_cast<uint32_t>(slotA[krot * 64 + lane]) | static_cast<uint32_t>(slotB[krot * 64 + lane]) << 8 |
             static_cast<uint32_t>(slotA[lane] == lane + 64 ? 1 : 0) << 16;
      for (int r = 0; r < krot; ++r) {
        const int byte = 4 + r;
        const uint32_t v =
            static_cast<uint32_t>(src[(r + 1) * 64 + lane]) | static_cast<uint32_t>(flag[(r + 1) * 64 + lane]) << 7;
        w[byte / 4] |= v << (8 * (byte % 4));
      }
    }
  }
  return PQ_OK;
}
