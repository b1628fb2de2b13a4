// Packed request block: layout, validation and derived work lists (see packing.hpp).
#include "packing.hpp"

#include <algorithm>

namespace laya {

Layout make_layout(int m, int b, int k) {
  Layout L{};
  size_t o = 0;
  auto take = [&](size_t n) { size_t at = o; o += n; return at; };
  auto take16 = [&](size_t n) { o = (o + 3) / 4 * 4; return take(n); };  // 16-byte aligned
  L.meta = take(4);
  L.ids = take(m);
  L.positions = take(m);
  L.rows = take(m);
  L.kinds = take(m);
  L.starts = take(b);
  L.lengths = take(b);
  L.counts = take(b);
  L.qkind = take(b);
  L.indices = take(static_cast<size_t>(b) * (k + 1));
  L.user_end = o;
  L.T = m / 16;
  L.R = b * (k + 1);
  L.qoff = take(b);
  L.tiles = take16(static_cast<size_t>(4) * L.T);
  L.sel_src = take(L.R);
  L.sel_q = take(L.R);
  L.n_sel = take(1);
  L.n_tiles = take(1);
  L.total = o;
  return L;
}

namespace {
// Rows a sequence of `len` tokens spans (16-row alignment), in 64-bit so no length overflows.
long long span16(long long len) { return (len + 15) / 16 * 16; }
}  // namespace

const char* derive_packed(const PackLimits& lim, int m, int b, int k, const Layout& L, int32_t* P, int attn_block,
                          int attn_tiles) {
  const int n_seq = P[L.meta], n_q = P[L.meta + 1];
  if (n_seq < 0 || n_seq > b || n_q < 0 || n_q > b) return "sequence/question count exceeds the shape class";
  for (int i = 0; i < m; ++i) {
    if (P[L.ids + i] < 0 || P[L.ids + i] >= lim.vocab) return "token id out of range";
    if (P[L.positions + i] < 0 || P[L.positions + i] >= lim.positions) return "position out of range";
    if (lim.token_kinds && (P[L.kinds + i] < 0 || P[L.kinds + i] >= 3)) return "question kind out of range";
  }
  // Sequences in increasing start order, 16-aligned, non-overlapping, inside the slot.
  long long end = 0;
  for (int sq = 0; sq < n_seq; ++sq) {
    const long long st = P[L.starts + sq], len = P[L.lengths + sq];
    if (st % 16 || st < end || len < 0 || st + span16(len) > m)
      return "sequences must start at increasing multiples of 16 rows and fit the shape class";
    end = st + span16(len);
  }
  const int nt = build_attention_tiles(P + L.starts, P + L.lengths, n_seq, m, attn_block, P + L.tiles, attn_tiles);
  if (nt < 0) return "attention tile list overflow";
  P[L.n_tiles] = nt;
  // Compact head rows: per question its CLS row then its option rows.
  int ns = 0;
  for (int q = 0; q < n_q; ++q) {
    const int cnt = P[L.counts + q];
    if (cnt < 0 || cnt > k) return "option count exceeds the shape class";
    if (P[L.qkind + q] < 0 || P[L.qkind + q] >= 3) return "question kind out of range";
    P[L.qoff + q] = ns;
    for (int j = 0; j <= cnt; ++j) {
      const int src = P[L.indices + static_cast<size_t>(q) * (k + 1) + j];
      if (src < 0 || src >= m) return "readout index out of range";
      P[L.sel_src + ns] = src;
      P[L.sel_q + ns] = q;
      ++ns;
    }
  }
  for (int q = n_q; q < b; ++q) P[L.qoff + q] = ns;
  P[L.n_sel] = ns;
  return nullptr;
}

int build_attention_tiles(const int32_t* starts, const int32_t* lengths, int n_seq, int m, int block,
                          int32_t* tiles, int max_tiles) {
  if (block <= 0 || block % 16 || max_tiles < 0 || n_seq < 0 || m < 0) return -1;
  int nt = 0;
  long long row = 0;
  auto put = [&](long long r0, long long r1, long long kstart, long long klen) {
    if (nt >= max_tiles) return false;
    tiles[4 * nt] = static_cast<int32_t>(r0);
    tiles[4 * nt + 1] = static_cast<int32_t>(r1);
    tiles[4 * nt + 2] = static_cast<int32_t>(kstart);
    tiles[4 * nt + 3] = static_cast<int32_t>(klen);
    ++nt;
    return true;
  };
  auto run = [&](long long upto, long long kstart, long long klen) {
    while (row < upto) {
      const long long r1 = (upto - row > block) ? row + block : upto;
      if (!put(row, r1, kstart, klen)) return false;
      row = r1;
    }
    return true;
  };
  for (int s = 0; s < n_seq; ++s) {
    const long long st = starts[s], len = lengths[s], e = st + span16(len);
    if (st % 16 || st < row || len < 0 || e > m) return -1;
    if (!run(st, 0, -1) || !run(e, st, len)) return -1;
  }
  if (!run(m, 0, -1)) return -1;
  // Longest key ranges first: workgroups start in list order, so the long tiles of a ragged batch
  // do not end up in the last round (their cost grows with the key count).  Ties by first row: a
  // total order, so the list is the same on every call (std::sort allocates nothing).
  struct Quad {
    int32_t v[4];
  };
  Quad* quads = reinterpret_cast<Quad*>(tiles);
  std::sort(quads, quads + nt, [](const Quad& x, const Quad& y) {
    return x.v[3] != y.v[3] ? x.v[3] > y.v[3] : x.v[0] < y.v[0];
  });
  for (int t = nt; t < max_tiles; ++t) {
    tiles[4 * t] = tiles[4 * t + 1] = tiles[4 * t + 2] = 0;
    tiles[4 * t + 3] = -1;
  }
  return nt;
}

}  // namespace laya
