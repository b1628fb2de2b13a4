// Host-side handling of the packed int32 request block: its layout, validation of what a caller
// supplies, and the work lists derived from it before the single upload.  Plain C++ (no HIP), so
// it also builds on its own under AddressSanitizer for the malformed-block tests.
#pragma once

#include <cstddef>
#include <cstdint>

namespace laya {

// Packed input layout for shape (m, b, k): the caller's block (laya_packed_ints) followed by the
// derived work lists the host builds before the single upload.
struct Layout {
  size_t meta, ids, positions, rows, kinds, starts, lengths, counts, qkind, indices, user_end;
  size_t qoff, tiles, sel_src, sel_q, n_sel, n_tiles, total;
  int T, R;
};
Layout make_layout(int m, int b, int k);

// What the block is checked against: token ids < vocab, positions < positions, and (head
// transformer layers) per-token question kinds in [0, 3).
struct PackLimits {
  int vocab, positions;
  bool token_kinds;
};

// Validates the caller's part of the block `P` (L.user_end ints) for shape (m, b, k) and writes the
// derived lists (question offsets, attention tiles of at most `attn_block` rows, at most
// `attn_tiles` of them, and the compact head rows) into the rest of `P` (L.total ints).  Returns
// null on success, else a static message naming what was wrong (nothing derived is then valid).
const char* derive_packed(const PackLimits& lim, int m, int b, int k, const Layout& L, int32_t* P, int attn_block,
                          int attn_tiles);

// Attention work list of packed sequences (starts multiples of 16, increasing, spans of 16 rows):
// tiles of at most `block` query rows of one sequence plus zero-tiles for rows of no sequence, as
// (row0, row1, kstart, klen) quads, longest key range first; fills all max_tiles entries (unused
// ones as empty ranges) and returns the used count, or -1 for a bad layout or too small a list.
int build_attention_tiles(const int32_t* starts, const int32_t* lengths, int n_seq, int m, int block,
                          int32_t* tiles, int max_tiles);

}  // namespace laya
