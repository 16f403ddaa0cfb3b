// Host check of ragged_piece_rank (tritonkv_amd/csrc/decode_common.h), the
// rank behind the longest-piece-first dispatch order: for random ragged
// batches (empty rows, rows of the full history, rows ending on a split
// boundary), every piece's rank must equal its position in a plain sort of
// all pieces by (length descending, s * B + b).  Built and run by
// tests/test_order_rank_host.py; prints "cases N bad M" and exits 1 on any
// mismatch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <random>
#include <tuple>
#include <vector>

#include "../tritonkv_amd/csrc/decode_common.h"

int main() {
  std::mt19937 g(7);
  long cases = 0, bad = 0;
  for (int it = 0; it < 3000; ++it) {
    const int B = 1 + g() % 40, ns = 1 + g() % 9, ss = 32 * (1 + g() % 8);
    int S = ns * ss - (int)(g() % ss);
    if (S <= (ns - 1) * ss) S = (ns - 1) * ss + 1;
    std::vector<int> L(B);
    for (auto& x : L) {
      const int m = g() % 5;
      x = m == 0 ? 0 : m == 1 ? S : m == 2 ? ss * (int)(g() % (ns + 1)) : (int)(g() % (S + 1));
      x = std::min(x, S);
    }
    std::vector<std::tuple<int, int>> keys;  // (-length, s * B + b)
    for (int s = 0; s < ns; ++s)
      for (int b = 0; b < B; ++b) keys.emplace_back(-std::max(0, std::min(L[b] - s * ss, ss)), s * B + b);
    std::sort(keys.begin(), keys.end());
    std::vector<int> want(B * ns);
    for (int r = 0; r < (int)keys.size(); ++r) want[std::get<1>(keys[r])] = r;
    auto lens = [&](int i) { return L[i]; };
    for (int s = 0; s < ns; ++s)
      for (int b = 0; b < B; ++b, ++cases)
        if (tkv::ragged_piece_rank(b, s, B, ss, lens) != want[s * B + b]) ++bad;
  }
  std::printf("cases %ld bad %ld\n", cases, bad);
  return bad != 0;
}
