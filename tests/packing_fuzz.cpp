// Malformed and well-formed packed request blocks through the host-side parser
// (laya-cuda_amd/csrc/packing.cpp), built with AddressSanitizer and UBSan by
// tests/test_packing_asan.py.  Every block lives in a heap buffer of exactly the layout's size, so
// a read or write past it is reported.  Well-formed blocks must be accepted with consistent derived
// lists; malformed ones must be refused with a message; nothing may touch memory out of bounds or
// overflow an int.
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "packing.hpp"

using namespace laya;

static int failures = 0;
#define CHECK(cond, ...)                   \
  do {                                     \
    if (!(cond)) {                         \
      std::fprintf(stderr, __VA_ARGS__);   \
      std::fprintf(stderr, "\n");          \
      ++failures;                          \
    }                                      \
  } while (0)

struct Shape {
  int m, b, k, block, tiles;
};

// A well-formed block: sequences packed back to back at 16-row starts, questions on them.
static void fill_valid(std::mt19937& rng, const Shape& s, const Layout& L, int32_t* P, const PackLimits& lim) {
  std::fill(P, P + L.total, 0);
  int row = 0, n_seq = 0;
  while (n_seq < s.b && row < s.m) {
    const int room = s.m - row;
    const int len = 1 + static_cast<int>(rng() % static_cast<unsigned>(room));
    P[L.starts + n_seq] = row;
    P[L.lengths + n_seq] = len;
    row += (len + 15) / 16 * 16;
    ++n_seq;
    if (rng() % 3 == 0) break;
  }
  P[L.meta] = n_seq;
  for (int i = 0; i < s.m; ++i) {
    P[L.ids + i] = static_cast<int32_t>(rng() % static_cast<unsigned>(lim.vocab));
    P[L.positions + i] = static_cast<int32_t>(rng() % static_cast<unsigned>(lim.positions));
    P[L.kinds + i] = static_cast<int32_t>(rng() % 3);
    P[L.rows + i] = -1;
  }
  const int n_q = n_seq ? 1 + static_cast<int>(rng() % static_cast<unsigned>(s.b)) : 0;
  P[L.meta + 1] = n_q;
  for (int q = 0; q < n_q; ++q) {
    const int sq = static_cast<int>(rng() % static_cast<unsigned>(n_seq));
    const int cnt = static_cast<int>(rng() % static_cast<unsigned>(s.k + 1));
    P[L.counts + q] = cnt;
    P[L.qkind + q] = static_cast<int32_t>(rng() % 3);
    for (int j = 0; j <= cnt; ++j)
      P[L.indices + static_cast<size_t>(q) * (s.k + 1) + j] =
          P[L.starts + sq] + static_cast<int32_t>(rng() % static_cast<unsigned>(P[L.lengths + sq]));
  }
}

static void check_derived(const Shape& s, const Layout& L, const int32_t* P, int nt_cap) {
  // Tiles cover every row once; n_sel counts the CLS and option rows of every question.
  std::vector<int> cover(s.m, 0);
  for (int t = 0; t < nt_cap; ++t) {
    const int32_t* q = P + L.tiles + 4 * t;
    for (int r = q[0]; r < q[1]; ++r) {
      CHECK(r >= 0 && r < s.m, "tile row %d outside [0, %d)", r, s.m);
      if (r >= 0 && r < s.m) ++cover[r];
    }
    CHECK(q[1] - q[0] <= s.block, "tile of %d rows > block %d", q[1] - q[0], s.block);
  }
  for (int r = 0; r < s.m; ++r) CHECK(cover[r] == 1, "row %d covered %d times", r, cover[r]);
  // The used entries are the front of the list, and n_tiles counts them.
  int used = 0;
  while (used < nt_cap && P[L.tiles + 4 * used] < P[L.tiles + 4 * used + 1]) ++used;
  CHECK(P[L.n_tiles] == used, "n_tiles %d != %d used entries", P[L.n_tiles], used);
  for (int t = used; t < nt_cap; ++t)
    CHECK(P[L.tiles + 4 * t] == P[L.tiles + 4 * t + 1], "used entry %d after an unused one", t);
  int want = 0;
  for (int q = 0; q < P[L.meta + 1]; ++q) want += P[L.counts + q] + 1;
  CHECK(P[L.n_sel] == want, "n_sel %d != %d", P[L.n_sel], want);
}

static const int32_t kWild[] = {INT_MIN, INT_MIN + 1, -65536, -17, -1, 0, 1, 15, 16, 17, 1 << 20, INT_MAX - 15,
                                INT_MAX};

int main() {
  std::mt19937 rng(12345);
  const PackLimits lim{1000, 512, true};
  const Shape shapes[] = {{96, 1, 8, 32, 6}, {512, 2, 8, 32, 21}, {1024, 4, 8, 256, 13}, {2048, 16, 32, 128, 49},
                          {64, 3, 4, 64, 4}};
  int accepted = 0, refused = 0;
  for (const Shape& s : shapes) {
    const Layout L = make_layout(s.m, s.b, s.k);
    CHECK(L.total >= L.user_end && L.tiles % 4 == 0, "layout");
    const int nt_cap = s.tiles < L.T ? s.tiles : L.T;
    for (int it = 0; it < 400; ++it) {
      std::vector<int32_t> block;  // exactly the layout's size: ASan reports any access past it
      int32_t* P = new int32_t[L.total];
      fill_valid(rng, s, L, P, lim);
      // The generator keeps blocks within the tile bound of an actual slot: at most
      // m / block + 2 b + 1 tiles; with a smaller cap a dense request may overflow, which is refused.
      const char* err = derive_packed(lim, s.m, s.b, s.k, L, P, s.block, nt_cap);
      if (!err) {
        ++accepted;
        check_derived(s, L, P, nt_cap);
      } else {
        CHECK(std::strstr(err, "tile list") != nullptr, "valid block refused: %s", err);
      }
      // Corrupt one field of the caller's part with a wild value, then parse again.
      fill_valid(rng, s, L, P, lim);
      const size_t at = rng() % L.user_end;
      P[at] = kWild[rng() % (sizeof(kWild) / sizeof(kWild[0]))];
      err = derive_packed(lim, s.m, s.b, s.k, L, P, s.block, nt_cap);
      if (err) {
        ++refused;
      } else {
        check_derived(s, L, P, nt_cap);
      }
      // Fully random caller part.
      for (size_t i = 0; i < L.user_end; ++i)
        P[i] = (rng() & 1) ? kWild[rng() % (sizeof(kWild) / sizeof(kWild[0]))] : static_cast<int32_t>(rng() % 64);
      err = derive_packed(lim, s.m, s.b, s.k, L, P, s.block, nt_cap);
      if (err) ++refused;
      delete[] P;
    }
  }
  // build_attention_tiles on its own: wild starts and lengths, small lists.
  for (int it = 0; it < 2000; ++it) {
    const int n = 1 + static_cast<int>(rng() % 6), m = 16 * static_cast<int>(rng() % 40), block = 16 << (rng() % 4);
    int32_t* starts = new int32_t[n];
    int32_t* lengths = new int32_t[n];
    for (int i = 0; i < n; ++i) {
      starts[i] = (rng() & 3) ? static_cast<int32_t>(16 * (rng() % 40)) : kWild[rng() % 13];
      lengths[i] = (rng() & 3) ? static_cast<int32_t>(rng() % 300) : kWild[rng() % 13];
    }
    const int cap = static_cast<int>(rng() % 50);
    int32_t* tiles = new int32_t[4 * static_cast<size_t>(cap) + 1];
    const int nt = build_attention_tiles(starts, lengths, n, m, block, tiles, cap);
    CHECK(nt >= -1 && nt <= cap, "tile count %d outside [-1, %d]", nt, cap);
    delete[] tiles;
    delete[] starts;
    delete[] lengths;
  }
  std::printf("accepted %d well-formed blocks, refused %d malformed ones, %d failures\n", accepted, refused, failures);
  return failures ? 1 : 0;
}
