// Host check of the planner's list arithmetic shared with the attention kernels (compiled and run
// on the CPU by tests/test_list_slice.py): slice_from_masks, which builds a split's slice of the
// block list from the chunk masks in the planned pass's prologue (every thread of the workgroup a
// share of the blocks), against the list built directly, for every split of random masks and
// teams of several sizes; gap_range, which bounds the statistics writes between list
// entries, against the blocks strictly between two entries, and on entries of any value.
#include <climits>
#include <cstdio>
#include <vector>

#include "../kvskip_amd/csrc/attn_decode.hpp"

using namespace kvs;

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint32_t rnd() {
  rs ^= rs << 13;
  rs ^= rs >> 7;
  rs ^= rs << 17;
  return static_cast<uint32_t>(rs >> 11);
}

static int fails = 0;
#define CHECK(c, ...)                   \
  do {                                  \
    if (!(c) && fails++ < 10) {         \
      std::printf("FAIL " __VA_ARGS__); \
      std::printf("\n");                \
    }                                   \
  } while (0)

int main() {
  constexpr int SENT = INT_MIN + 7;
  int slices = 0;
  for (int it = 0; it < 3000; ++it) {
    const int nb = it < 8 ? (it + 1) * 512 : 1 + static_cast<int>(rnd() % MAX_NB);
    const int dens = it % 5 == 0 ? 1000 : it % 7 == 0 ? 0 : static_cast<int>(rnd() % 1001);
    std::vector<uint32_t> mask(WAVE * DCL, 0u);
    std::vector<int> list;
    for (int c = 0; c < WAVE * DCL; ++c)
      for (int bit = 0; bit < WCB; ++bit)
        if (c * WCB + bit < nb && static_cast<int>(rnd() % 1000) < dens) {
          mask[c] |= 1u << bit;
          list.push_back(c * WCB + bit);
        }
    std::vector<int> pre(WAVE * DCL);
    for (int c = 0, acc = 0; c < WAVE * DCL; ++c) {
      pre[c] = acc;
      acc += __builtin_popcount(mask[c]);
    }
    const int cnt = static_cast<int>(list.size());
    const int S = it < 8 ? 32 : 1 + static_cast<int>(rnd() % 96);
    for (int split = 0; split < S; ++split) {
      const int per = (cnt + S - 1) / S;
      const int a0 = std::min(cnt, split * per), a1 = std::min(cnt, a0 + per);
      std::vector<int> out(MAX_NB + 2, SENT);
      const int C = (nb + WCB - 1) / WCB, stride = it % 3 == 0 ? 256 : 1 + static_cast<int>(rnd() % 300);
      for (int t = 0; t < stride; ++t) slice_from_masks(mask.data(), pre.data(), C, a0, a1, out.data(), t, stride);
      if (a0 == 0) out[0] = -1;
      for (int pos = a0 - 1; pos < a1; ++pos)
        CHECK(out[pos - a0 + 1] == (pos < 0 ? -1 : list[pos]), "slice nb %d S %d split %d pos %d: %d", nb, S, split,
              pos, out[pos - a0 + 1]);
      for (int i = a1 - a0 + 1; i < MAX_NB + 2; ++i) CHECK(out[i] == SENT, "stray write nb %d split %d at %d", nb, split, i);
      ++slices;
    }
  }
  // gap_range: exact between valid ascending entries; inside [0, nb) for any entries
  const int ext[] = {INT_MIN, INT_MIN + 1, -1000000, -2, -1, 0, 1, 5, 63, 64, 4095, 4096, 4097, 1000000, INT_MAX - 1, INT_MAX};
  int gaps = 0;
  for (int nb : {1, 2, 7, 64, 512, 4096}) {
    for (int prev = -1; prev < std::min(nb, 70); ++prev)
      for (int cur = prev + 1; cur <= std::min(nb, 71); ++cur) {
        int a, len;
        gap_range(prev, cur, nb, a, len);
        CHECK(a == prev + 1 && len == cur - prev - 1, "gap nb %d prev %d cur %d: %d %d", nb, prev, cur, a, len);
        ++gaps;
      }
    for (int p : ext)
      for (int c : ext) {
        int a, len;
        gap_range(p, c, nb, a, len);
        CHECK(a >= 0 && a <= nb && (len <= 0 || a + len <= nb), "gap bounds nb %d prev %d cur %d: %d %d", nb, p, c, a, len);
        ++gaps;
      }
  }
  if (fails) {
    std::printf("%d failures\n", fails);
    return 1;
  }
  std::printf("ok: %d slices, %d gaps\n", slices, gaps);
  return 0;
}
