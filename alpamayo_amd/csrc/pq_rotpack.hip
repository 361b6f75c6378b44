// Host-side packing of rotation parameters into the kernels' operand layout.
//
// Reference parameters (src/alpamayo_r1/utils/quantization/rotation_linear.py:
// 39-43): pairs int16 [krot][h] with group-local indices (pair t of group g in
// layer r = pairs[r][g*128+2t], pairs[r][g*128+2t+1]) and angles [krot][h/2].
// Kernel layout (one entry per (group, lane, layer); the lane owns one pair):
//   rot_ij [G][64][KP]     uint16  first | second << 8
//   rot_cs [G][64][KP][2]  float32 (cos, sin)
// with KP = krot rounded up to a multiple of 8, so one lane's indices for 8
// layers are 16 contiguous bytes and its angles 64 contiguous bytes.
//
// Which lane owns which pair, and which element of a pair comes first, is
// free: a Givens update on (i, j) with angle theta equals the update on
// (j, i) with -theta, bit for bit in the kernels' float32 form
// (fma(xi, c, xj*s) with s -> -s is fma(xi, c, -(xj*(-s)))...).  The packer
// uses that freedom to make every layer's LDS accesses bank-conflict free
// (32 banks of 4 bytes, a wave64 LDS access served as two halves of 32
// lanes): bank(ch) = ch mod 32, so the 64 pairs of a group and layer form a
// 4-regular multigraph on the 32 banks.  Orienting each component along an
// Euler circuit gives every bank in- and out-degree 2; the oriented edges
// then form a 2-regular bipartite graph (tail bank -> head bank), which
// splits into two perfect matchings.  Matching 0 goes to lanes 0..31 and
// matching 1 to lanes 32..63, lane = 32*m + tail bank, so in each half the
// first elements hit 32 distinct banks and so do the second elements.
#include <cstring>
#include <vector>

#include "pq_common.h"

namespace {

struct Edge {
  int a, b;      // channels of the pair (a first)
  float c, s;
  int u, v;      // banks of a, b
  int tail = -1, head = -1;
  int color = -1;
};

// Orients every edge of the bank multigraph along Euler circuits.
void orient(std::vector<Edge>& e) {
  const int nb = 32;
  std::vector<std::vector<int>> adj(nb);
  for (int k = 0; k < static_cast<int>(e.size()); ++k) {
    adj[e[k].u].push_back(k);
    if (e[k].v != e[k].u) adj[e[k].v].push_back(k);
    else adj[e[k].u].push_back(k);   // a loop appears twice in its bank's list
  }
  std::vector<size_t> next(nb, 0);
  std::vector<char> used(e.size(), 0);
  for (int start = 0; start < nb; ++start) {
    // Hierholzer walk: each traversed edge is oriented from where we stand.
    std::vector<int> stack{start};
    while (!stack.empty()) {
      const int x = stack.back();
      while (next[x] < adj[x].size() && used[adj[x][next[x]]]) ++next[x];
      if (next[x] == adj[x].size()) {
        stack.pop_back();
        continue;
      }
      const int k = adj[x][next[x]++];
      used[k] = 1;
      const int y = (e[k].u == x) ? e[k].v : e[k].u;
      e[k].tail = x;
      e[k].head = y;
      stack.push_back(y);
    }
  }
}

// Splits the oriented edges (every bank: out 2, in 2) into two matchings.
bool split(std::vector<Edge>& e) {
  const int nb = 32;
  std::vector<std::vector<int>> out(nb), in(nb);
  for (int k = 0; k < static_cast<int>(e.size()); ++k) {
    out[e[k].tail].push_back(k);
    in[e[k].head].push_back(k);
  }
  for (int b = 0; b < nb; ++b)
    if (out[b].size() != 2 || in[b].size() != 2) return false;
  for (int k0 = 0; k0 < static_cast<int>(e.size()); ++k0) {
    if (e[k0].color >= 0) continue;
    // Walk the alternating cycle: tail side shares color pairs 0/1, head side too.
    int k = k0, color = 0;
    while (e[k].color < 0) {
      e[k].color = color;
      // the other edge entering the same head gets the other color
      const int h = e[k].head;
      const int k2 = in[h][0] == k ? in[h][1] : in[h][0];
      if (e[k2].color >= 0) break;
      e[k2].color = 1 - color;
      // the other edge leaving k2's tail continues the cycle with `color`
      const int t = e[k2].tail;
      k = out[t][0] == k2 ? out[t][1] : out[t][0];
    }
  }
  int count0 = 0;
  for (auto& x : e) count0 += x.color == 0;
  return count0 == 32;
}

}  // namespace

extern "C" int pq_rotation_pack(const int16_t* pairs, const float* cos_sin, int64_t h, int krot, uint16_t* rot_ij,
                                float* rot_cs) {
  PQ_REQUIRE(pairs && cos_sin && rot_ij && rot_cs, PQ_ERR_ARG, "pq_rotation_pack: null pointer");
  PQ_REQUIRE(h > 0 && h % 128 == 0 && h <= (1 << 20), PQ_ERR_ARG, "pq_rotation_pack: h=%lld", (long long)h);
  PQ_REQUIRE(krot >= 1 && krot <= 64, PQ_ERR_ARG, "pq_rotation_pack: krot=%d", krot);
  const int G = static_cast<int>(h / 128);
  const int KP = (krot + 7) / 8 * 8;
  std::memset(rot_ij, 0, sizeof(uint16_t) * G * 64 * KP);
  std::memset(rot_cs, 0, sizeof(float) * G * 64 * KP * 2);
  std::vector<Edge> e(64);
  for (int g = 0; g < G; ++g) {
    for (int r = 0; r < krot; ++r) {
      int seen[128] = {0};
      for (int t = 0; t < 64; ++t) {
        const int a = pairs[static_cast<int64_t>(r) * h + g * 128 + 2 * t];
        const int b = pairs[static_cast<int64_t>(r) * h + g * 128 + 2 * t + 1];
        PQ_REQUIRE(a >= 0 && a < 128 && b >= 0 && b < 128, PQ_ERR_ARG,
                   "pq_rotation_pack: pair index out of [0,128) in layer %d group %d", r, g);
        ++seen[a];
        ++seen[b];
        Edge x;
        x.a = a;
        x.b = b;
        x.c = cos_sin[(static_cast<int64_t>(r) * (h / 2) + g * 64 + t) * 2];
        x.s = cos_sin[(static_cast<int64_t>(r) * (h / 2) + g * 64 + t) * 2 + 1];
        x.u = a & 31;
        x.v = b & 31;
        e[t] = x;
      }
      for (int ch = 0; ch < 128; ++ch)
        PQ_REQUIRE(seen[ch] == 1, PQ_ERR_ARG,
                   "pq_rotation_pack: layer %d group %d does not pair every channel exactly once", r, g);
      orient(e);
      PQ_REQUIRE(split(e), PQ_ERR_ARG, "pq_rotation_pack: internal error splitting layer %d group %d", r, g);
      for (const Edge& x : e) {
        const int lane = 32 * x.color + x.tail;
        int first = x.a, second = x.b;
        float s = x.s;
        if ((x.a & 31) != x.tail) {   // oriented against the stored order: swap, negate sin
          first = x.b;
          second = x.a;
          s = -x.s;
        }
        const int64_t o = (static_cast<int64_t>(g) * 64 + lane) * KP + r;
        rot_ij[o] = static_cast<uint16_t>(first | (second << 8));
        rot_cs[2 * o] = x.c;
        rot_cs[2 * o + 1] = s;
      }
    }
  }
  return PQ_OK;
}
