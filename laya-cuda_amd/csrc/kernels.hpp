// Kernel argument blocks and launchers for the encoder forward path (gfx950).
#pragma once

#include "common.hpp"

namespace laya {

enum class DType : int { F32 = 0, F16 = 1, BF16 = 2 };

// ---- embedding gather (+ learned position + type row) (+ LayerNorm) ----
struct EmbedArgs {
  const int32_t* ids;
  const int32_t* positions;
  const float* table;      // [vocab][d]
  const float* pos_table;  // [n_positions][d] or null
  const float* type_row;   // [d] or null
  const float* gamma;      // null: no LayerNorm (pure gather + adds)
  const float* beta;
  float eps;
  float* out32;  // [rows][d] or null
  void* out16;   // [rows][d] 16-bit or null
  int rows, vocab, n_positions;
};

// ---- residual add (+ split-K partial sum + bias) (+ LayerNorm) ----
struct AddNormArgs {
  float* residual;         // [rows][d]
  const float* parts;      // [splits][rows][d] branch partials, or null
  int splits;
  long long part_stride;   // elements between partials
  const float* bias;       // [d] added to the branch, or null
  const float* gamma;      // null: no LayerNorm
  const float* beta;
  float eps;
  float* sum_out;  // pre-norm sum residual+branch, or null
  float* out32;    // normalised (or sum, if gamma is null) fp32, may alias residual
  void* out16;     // same as 16-bit, or null
  int rows;
  const float* row_table;    // [n][d] rows added per token (question types), or null
  const int32_t* row_index;  // [rows] row of row_table for each token
  const void* branch16;      // [rows][d] 16-bit branch (bias already added), instead of parts, or null
};

bool norm_width_supported(int width);
hipError_t launch_embed(const EmbedArgs& a, int width, DType t, hipStream_t stream);
hipError_t launch_add_norm(const AddNormArgs& a, int width, DType t, hipStream_t stream);

// ---- MFMA GEMM: out[M][N] = A[M][K] * B[N][K]^T (+ bias), fp32 accumulate ----
// QKV_ROPE is the QKV epilogue with RoPE compiled in: launch_gemm picks it for Epi::QKV when rope
// tables are given, so the QKV kernels without RoPE carry none of its code.
enum class Epi : int { F32 = 0, HALF = 1, GELU = 2, QKV = 3, RELU = 4, GEGLU = 5, QKV_ROPE = 6 };

struct GemmArgs {
  const void* a;  // [M][lda] 16-bit
  const void* b;  // [N][ldb] 16-bit
  int M, N, K, lda, ldb;
  const float* bias;        // [N] or null (F32 epilogue: only with splits == 1)
  void* out;                // F32: float [splits][M][ldo]; HALF/GELU: 16-bit [M][ldo]
  long long ldo;
  long long split_stride;   // F32: elements between split partials
  int splits;
  // QKV epilogue: columns [0,w) -> q, [w,2w) -> k, [2w,3w) -> vt.
  // q, k: [heads][M][64]; vt: [heads][64][M] (keys contiguous).
  void* q;
  void* k;
  void* vt;
  int width;
  // QKV with RoPE (null: none): cos/sin [positions][32] of this layer's theta, positions [M].
  const float* rope_cos;
  const float* rope_sin;
  const int32_t* positions;
  int rows_major;  // XCD share of the tile grid split by tile rows (A larger than B) or columns
};

struct GemmTile {
  int bm, bn;
};
int gemm_tile_count();
GemmTile gemm_tile(int id);
// Packed rows from which a problem counts as batched: the planner costs tiles by their operand
// bytes per CU, and shape slots keep the out/down projections as 16-bit rows (no split-K).
constexpr int kBatchedRows = 4096;
// Chooses a tile and split count for a problem on `cus` compute units: the measured plan table
// (gemm_plans.inc) when it has the problem and `measured`, else the heuristic.
// rope: the QKV epilogue applies RoPE, which needs wave tiles of 64-column multiples.
void gemm_plan(int M, int N, int K, Epi epi, DType t, int cus, int* tile, int* splits, bool rope = false,
               bool measured = true);
hipError_t gemm_prepare();  // sets LDS attributes of the large-tile kernels (call once per device)
// Pipelined tiles read their operands through buffer resources with 32-bit byte offsets: true when
// both operands ([M][lda] and [N][ldb] 16-bit) span fewer than 2^32 bytes.
bool gemm_operands_addressable(long long M, long long lda, long long N, long long ldb);
hipError_t launch_gemm(const GemmArgs& a, Epi epi, DType t, int tile, hipStream_t stream);

// ---- fused bidirectional attention over packed rows ----
// tiles: [max_tiles][3] = (row0, row1, seq); seq < 0 marks rows to zero.
// Attention work list entry (16-byte aligned int4): query rows [row0, row1) of one sequence whose
// keys are rows [kstart, kstart + klen); klen < 0 marks rows of no sequence (written as zeros), and
// row0 == row1 an unused entry.
struct AttnArgs {
  const void* q;   // [heads][m][64]
  const void* k;   // [heads][m][64]
  const void* vt;  // [heads][64][m]
  void* out;       // [m][heads*64]
  const int32_t* tiles;  // [max_tiles][4] = (row0, row1, kstart, klen)
  int m, heads, max_tiles;
  int window;  // local attention half-window (|query - key| <= window), or -1 for global
  // Device count of the used entries at the front of `tiles`, or null: then the whole list is
  // walked (unused entries exit).  With the count, the shared-K/V kernel spreads only the used
  // entries evenly over the XCDs.
  const int32_t* n_tiles = nullptr;
};
// Attention kernels: kAttnSharedKV - a workgroup of `waves` waves owns 32*waves queries and stages
// each K/V block once in LDS for all of them (large batches); kAttnSplitKeys - a workgroup owns 32
// queries and its `waves` waves split the keys, merging at the end (few query tiles: batch 1).
// kAttnPairKeys - a workgroup owns 64 queries as two 32-query groups whose waves share each key
// group's LDS-staged blocks, the waves/2 key groups splitting the keys (long batch-1 sequences).
enum AttnMode : int { kAttnSharedKV = 0, kAttnSplitKeys = 1, kAttnPairKeys = 2 };
int attention_block_rows(int mode, int waves);
bool attention_mode_valid(int mode, int waves);
hipError_t launch_attention(const AttnArgs& a, DType t, int mode, int waves, hipStream_t stream);

// ---- decision head (no head transformer layers) ----
struct HeadGatherArgs {
  const float* residual;  // [m][d]
  const int32_t* sel_src; // [cap] packed source row of each compact head row
  const int32_t* sel_q;   // [cap] question of each compact head row
  const int32_t* qkind;   // [b]
  const int32_t* n_sel;   // device scalar
  const float* type_emb;  // [3][d] or null
  const float* gamma;     // scorer.0
  const float* beta;
  float eps;
  float* selected;  // [cap][d] gathered rows (+ type row)
  float* normed;    // [cap][d] LayerNorm of selected
  int cap;
  // The encoder's last residual + LayerNorm, applied here to the gathered source rows only (no
  // other row of that layer's output is read), or n_gamma null: residual already final.  The
  // branch is the sum of `splits` fp32 partials plus `bias`, or 16-bit rows with the bias in them,
  // added exactly as the residual+LayerNorm kernel adds them.
  const float* parts = nullptr;
  int splits = 0;
  long long part_stride = 0;
  const void* branch16 = nullptr;
  const float* bias = nullptr;
  const float* n_gamma = nullptr;
  const float* n_beta = nullptr;
  float n_eps = 0.f;
};
hipError_t launch_head_gather(const HeadGatherArgs& a, int width, DType t, hipStream_t stream);

// Compact readout rows for the last head transformer layer: dst32[r] = src32[idx[r]] and
// dst16[r] = src16[idx[r]] (bit-exact copies) for r < *n; rows n..cap-1 are zeroed.  Either pair
// may be null (that copy is skipped).
struct GatherRowsArgs {
  const float* src32;
  float* dst32;
  const void* src16;
  void* dst16;
  const int32_t* idx;
  const int32_t* n;
  int cap;
};
hipError_t launch_gather_rows(const GatherRowsArgs& a, int width, DType t, hipStream_t stream);

struct HeadGemmArgs {
  const float* x;  // [cap][ldx] (row r of the product is x row x_rows[r] when x_rows is set)
  const float* w;  // [N][ldw]
  float* parts;    // [splits][cap][N]
  const int32_t* n_rows;  // device scalar (rows actually present)
  int cap, N, K, splits;
  long long split_stride;
  const int32_t* x_rows = nullptr;  // optional row map into x, clamped to [0, x_cap)
  int x_cap = 0;
  int ldx = 0, ldw = 0;  // row strides; 0: K
};
int head_gemm_splits(int rows, int N, int K, int cus);
// Two independent products in one launch (the scorer's hidden layer and the act head's CLS-row
// columns); b.cap == 0 launches the first alone.
hipError_t launch_head_gemm(const HeadGemmArgs& a, const HeadGemmArgs& b, hipStream_t stream);

// Head tail, one workgroup per question slot (laya.py:238-245, kernels.cu:167-183):
//   logit  = w3 . gelu(sum of scorer.1 partials + b1) + b3 for its CLS and option rows;
//   features: p1, p1-p2, entropy/log(max(n,2)), max(n,2)/255 of the option logits;
//   hidden = gelu(act_head.0's CLS-row partials + its feature columns . features + a0);
//   acts   = A2 hidden + a2.
// Unused question slots of the shape class get zero logits and acts.
struct HeadTailArgs {
  const float* parts;  // scorer.1 partial products [splits][cap][d]
  int splits;
  long long split_stride;
  const float* b1;  // scorer.1 bias [d]
  const float* w3;  // scorer.3 weight [d]
  const float* b3;  // scorer.3 bias [1]
  const float* aparts;  // act_head.0 partial products over the CLS row's d columns [asplits][b][hidden]
  int asplits;
  long long asplit_stride;
  const float* a0w;  // act_head.0 weight [hidden][a0_ld]: columns d..d+3 take the features
  int a0_ld;
  const float* a0b;  // [hidden]
  const float* a2w;  // [n_act][hidden]
  const float* a2b;  // [n_act]
  const int32_t* counts;  // [b]
  const int32_t* qoff;    // [b] first compact head row of each question
  const int32_t* n_q;     // device scalar
  float* logits;  // [b][k+1]
  float* acts;    // [b][n_act]
  int b, k, hidden, n_act;
};
hipError_t launch_head_tail(const HeadTailArgs& a, int width, hipStream_t stream);
// Once per device before the first tail launch: the tail kernels' dynamic LDS limit.
hipError_t head_prepare();

}  // namespace laya
