// Native runtime behind the C ABI: resident weights, shape slots with one hipGraph each, LRU.
//
// Mirrors the ownership of the reference's Runtime/Slot (laya_cuda/runtime.py:28-197) in C++:
//   * one engine per device, one non-blocking stream (default priority), weights resident in HBM
//     for the engine's lifetime (matrices in the MFMA operand type, the rest fp32);
//   * a slot per shape class (rows, questions, options) holding ONE device allocation (its arena)
//     plus pinned staging, built on a cache miss and evicted least-recently-used;
//   * the slot's forward is captured into a hipGraph on first use and replayed afterwards; the
//     packed inputs are uploaded with one H2D copy before the launch (runtime.py:52-68, 115-133).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "kernels.hpp"
#include "laya_hip.h"
#include "packing.hpp"
#include "scope.hpp"

// Device scratch of laya_predict_static: the whole shape-slot arena of one forward (packed block,
// activations, split-K partials, head buffers) for callers that cannot allocate.  The loader gives
// every device that runs this library its own copy, held until the process ends; host code takes
// its address per device with hipGetSymbolAddress (prepare_device) and never uses this name.
constexpr size_t kScratchBytes = static_cast<size_t>(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace laya {
namespace {

thread_local std::string g_error;

struct Failure {
  int code;
  std::string message;
};

#define LAYA_HIP(expr)                                                                     \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      throw Failure{e_ == hipErrorOutOfMemory ? LAYA_ENOMEM : LAYA_EDEVICE,                \
                    std::string(#expr) + ": " + hipGetErrorString(e_)};                     \
  } while (0)

#define LAYA_REQUIRE(cond, msg)                     \
  do {                                              \
    if (!(cond)) throw Failure{LAYA_EINVAL, (msg)}; \
  } while (0)

int span16(int n) { return (n + 15) / 16 * 16; }

// ---- host dtype conversion (round to nearest even) ----
uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}
float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  std::memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

float host_value(const void* data, int dtype, size_t i) {
  switch (dtype) {
    case LAYA_F32: return static_cast<const float*>(data)[i];
    case LAYA_F16: return f16_bits_to_f32(static_cast<const uint16_t*>(data)[i]);
    default: return bf16_bits_to_f32(static_cast<const uint16_t*>(data)[i]);
  }
}

struct DevTensor {
  void* ptr = nullptr;
  DType dtype = DType::F32;
  std::vector<int64_t> shape;
  size_t count = 0;
  size_t bytes = 0;
  bool geglu = false;  // rows resident in the GeGLU interleave (see geglu_row)
};

struct Expected {
  std::vector<int64_t> shape;
  bool mfma = false;   // resident in the 16-bit MFMA operand type
  bool geglu = false;  // a [2f][d] gate|value matrix, resident with interleaved rows
};

// GeGLU up-projection rows [gate 0..f-1 | value 0..f-1] are stored in 32-row groups (16 gate rows,
// then their 16 value rows) so the GEMM epilogue finds each gate column and its value column in
// one lane.  Resident row r holds checkpoint row geglu_row(r, f).
int64_t geglu_row(int64_t r, int64_t f) {
  const int64_t group = r / 32, in = r % 32;
  return in < 16 ? group * 16 + in : f + group * 16 + (in - 16);
}

struct Slot {
  int m = 0, b = 0, k = 0;
  Layout L{};
  void* arena = nullptr;
  size_t bytes = 0;
  int32_t* d_packed = nullptr;
  int32_t* h_packed = nullptr;
  // Pinned host copy of the device logits and acts, which the arena keeps next to each other: one
  // D2H copy brings both (h_acts points into the same allocation, at the device layout's offset).
  float* h_logits = nullptr;
  float* h_acts = nullptr;
  size_t h_out_bytes = 0;
  float* residual = nullptr;
  void *x = nullptr, *q = nullptr, *kk = nullptr, *vt = nullptr, *attn = nullptr, *ff = nullptr;
  float* part = nullptr;
  float *selected = nullptr, *normed = nullptr, *hpart = nullptr, *logits = nullptr, *acts = nullptr;
  float* apart = nullptr;
  // Last head transformer layer, on the compact readout rows: attention rows, normalised rows,
  // FFN rows and split-K partials.
  void *attn_sel = nullptr, *x_sel = nullptr, *ff_sel = nullptr;
  float* part_sel = nullptr;
  int tile[4] = {0, 0, 0, 0}, splits[4] = {1, 1, 1, 1};  // qkv, o, up, down
  // Batched slots store the out and down projections as 16-bit rows with the bias added before
  // the rounding (the reference's branch buffer, runtime.py:70-75 with kernels.cu:20-35 and
  // 50-55); batch-1 slots keep fp32 split-K partials, summed with the bias in the norm kernel.
  bool branch16 = false;
  // Head transformer layers: in_proj, out_proj, linear1, linear2 over all rows, then out_proj,
  // linear1, linear2 over the readout rows.
  int htile[7] = {0, 0, 0, 0, 0, 0, 0}, hsplits[7] = {1, 1, 1, 1, 1, 1, 1};
  int attn_mode = 0, attn_waves = 2, attn_tiles = 0, head_splits = 1, act_splits = 1;
  hipGraphExec_t graph = nullptr;
  hipEvent_t start = nullptr, end = nullptr;
};

// Encoder layer.  BERT-style: n1 = post-attention norm, n2 = post-FFN norm, biases everywhere.
// ModernBERT: n1 = attn_norm (null in layer 0), n2 = mlp_norm, no biases (null), wi interleaved.
struct Layer {
  const void *wqkv, *wo, *wi, *wo2;
  const float *bqkv, *bo, *bi, *bo2, *n1g, *n1b, *n2g, *n2b;
  bool local;  // ModernBERT local layer: +-window attention, local RoPE theta
};

// Decision-head transformer layer (torch TransformerEncoderLayer, norm_first, ReLU, 4d).
struct HeadLayer {
  const void *in_w, *out_w, *l1_w, *l2_w;
  const float *in_b, *out_b, *l1_b, *l2_b, *n1g, *n1b, *n2g, *n2b;
};

struct Engine {
  LayaConfig cfg{};
  int device = 0, cus = 256, max_slots = 16;
  hipStream_t stream = nullptr;
  std::unordered_map<std::string, Expected> expected;
  std::unordered_map<std::string, DevTensor> weights;
  size_t weight_bytes = 0, slot_bytes = 0;
  bool finalized = false;
  std::vector<Layer> layers;
  std::vector<HeadLayer> head_layers;
  bool modern = false;  // ModernBERT executor variant (pre-LN, RoPE, GeGLU, windows, head layers)
  const float* final_norm = nullptr;
  float* rope = nullptr;  // cos and sin tables [2 thetas][2][rope_rows][32]
  int rope_rows = 0;
  const float *tok = nullptr, *pos = nullptr, *type0 = nullptr, *emb_g = nullptr, *emb_b = nullptr;
  const float *type_emb = nullptr, *s0w = nullptr, *s0b = nullptr, *s1w = nullptr, *s1b = nullptr;
  const float *s3w = nullptr, *s3b = nullptr, *a0w = nullptr, *a0b = nullptr, *a2w = nullptr, *a2b = nullptr;
  std::list<Slot*> lru;  // front = least recently used
  hipEvent_t static_start = nullptr, static_end = nullptr;  // timing of laya_predict_static
  std::string error;

  DType mfma() const { return cfg.mfma_dtype == LAYA_F16 ? DType::F16 : DType::BF16; }
};

void check_config(const LayaConfig& c) {
  LAYA_REQUIRE(c.heads > 0 && c.width == c.heads * 64, "width must equal heads * 64 (64-wide attention heads)");
  LAYA_REQUIRE(norm_width_supported(c.width), "unsupported width " + std::to_string(c.width));
  LAYA_REQUIRE(c.width % 64 == 0 && c.width >= 64, "width must be a multiple of 64");
  LAYA_REQUIRE(c.layers >= 1 && c.intermediate > 0 && c.intermediate % 64 == 0,
               "intermediate size must be a positive multiple of 64");
  LAYA_REQUIRE(c.vocab > 0 && c.max_positions > 0 && c.type_vocab > 0, "vocab/positions/type rows must be positive");
  LAYA_REQUIRE(c.max_len > 0 && span16(c.max_len) <= (c.pos_kind == LAYA_POS_LEARNED ? span16(c.max_positions) : 1 << 20),
               "max_len exceeds the position table");
  LAYA_REQUIRE(c.n_act >= 1 && c.act_hidden >= 64 && c.act_hidden % 64 == 0 && c.act_hidden <= 16384,
               "act head hidden width must be a positive multiple of 64");
  LAYA_REQUIRE(c.mfma_dtype == LAYA_BF16 || c.mfma_dtype == LAYA_F16, "mfma_dtype must be LAYA_BF16 or LAYA_F16");
  LAYA_REQUIRE(c.eps > 0.f, "eps must be positive");
  // Two encoder variants are built: BERT-style (post-LN, learned positions, GELU FFN with biases,
  // global attention, no head layers) and the reference's ModernBERT executor (pre-LN, RoPE,
  // GeGLU, no biases, local windows every layer but each global_every-th, head layers).
  const bool bert = c.norm_order == LAYA_NORM_POST && c.pos_kind == LAYA_POS_LEARNED && c.ffn_kind == LAYA_FFN_GELU &&
                    c.bias == 1 && c.window < 0 && c.head_layers == 0;
  const bool modern = c.norm_order == LAYA_NORM_PRE && c.pos_kind == LAYA_POS_ROPE && c.ffn_kind == LAYA_FFN_GEGLU &&
                      c.bias == 0 && c.global_every >= 1 && c.head_layers >= 1 && c.head_layers <= 64 &&
                      c.theta_global > 0.f && c.theta_local > 0.f;
  LAYA_REQUIRE(bert || modern,
               "encoder variant not built: BERT-style (post-LN, learned positions, GELU FFN with biases, global "
               "attention, no head layers) or ModernBERT (pre-LN, RoPE, GeGLU without biases, head layers)");
  LAYA_REQUIRE(!modern || c.width * 4 <= 4 * 2048, "head layers need 4*width FFN rows");
}

// Checkpoint tensor table of the ModernBERT variant (the reference's, laya.py:167-190).
void build_expected_modern(Engine& E) {
  const LayaConfig& c = E.cfg;
  const int64_t d = c.width, f = c.intermediate;
  auto put = [&](const std::string& n, std::vector<int64_t> s, bool mf = false, bool gg = false) {
    E.expected[n] = Expected{s, mf, gg};
  };
  put("encoder.embeddings.tok_embeddings.weight", {c.vocab, d});
  put("encoder.embeddings.norm.weight", {d});
  put("encoder.final_norm.weight", {d});
  for (int i = 0; i < c.layers; ++i) {
    const std::string p = "encoder.layers." + std::to_string(i) + ".";
    put(p + "attn.Wqkv.weight", {3 * d, d}, true);
    put(p + "attn.Wo.weight", {d, d}, true);
    put(p + "mlp.Wi.weight", {2 * f, d}, true, true);
    put(p + "mlp.Wo.weight", {d, f}, true);
    put(p + "mlp_norm.weight", {d});
    if (i) put(p + "attn_norm.weight", {d});
  }
  for (int i = 0; i < c.head_layers; ++i) {
    const std::string p = "head.layers." + std::to_string(i) + ".";
    put(p + "self_attn.in_proj_weight", {3 * d, d}, true);
    put(p + "self_attn.in_proj_bias", {3 * d});
    put(p + "self_attn.out_proj.weight", {d, d}, true);
    put(p + "self_attn.out_proj.bias", {d});
    put(p + "linear1.weight", {4 * d, d}, true);
    put(p + "linear1.bias", {4 * d});
    put(p + "linear2.weight", {d, 4 * d}, true);
    put(p + "linear2.bias", {d});
    put(p + "norm1.weight", {d});
    put(p + "norm1.bias", {d});
    put(p + "norm2.weight", {d});
    put(p + "norm2.bias", {d});
  }
}

void build_expected(Engine& E) {
  const LayaConfig& c = E.cfg;
  const int64_t d = c.width, f = c.intermediate;
  auto put = [&](const std::string& n, std::vector<int64_t> s, bool mf = false) { E.expected[n] = Expected{s, mf}; };
  if (E.modern) {
    build_expected_modern(E);
  } else {
  put("encoder.embeddings.tok_embeddings.weight", {c.vocab, d});
  put("encoder.embeddings.position_embeddings.weight", {c.max_positions, d});
  put("encoder.embeddings.token_type_embeddings.weight", {c.type_vocab, d});
  put("encoder.embeddings.norm.weight", {d});
  put("encoder.embeddings.norm.bias", {d});
  for (int i = 0; i < c.layers; ++i) {
    const std::string p = "encoder.layers." + std::to_string(i) + ".";
    put(p + "attn.Wqkv.weight", {3 * d, d}, true);
    put(p + "attn.Wqkv.bias", {3 * d});
    put(p + "attn.Wo.weight", {d, d}, true);
    put(p + "attn.Wo.bias", {d});
    put(p + "post_attn_norm.weight", {d});
    put(p + "post_attn_norm.bias", {d});
    put(p + "mlp.Wi.weight", {f, d}, true);
    put(p + "mlp.Wi.bias", {f});
    put(p + "mlp.Wo.weight", {d, f}, true);
    put(p + "mlp.Wo.bias", {d});
    put(p + "post_mlp_norm.weight", {d});
    put(p + "post_mlp_norm.bias", {d});
  }
  }
  put("type_emb.weight", {3, d});
  put("scorer.0.weight", {d});
  put("scorer.0.bias", {d});
  put("scorer.1.weight", {d, d});
  put("scorer.1.bias", {d});
  put("scorer.3.weight", {1, d});
  put("scorer.3.bias", {1});
  put("act_head.0.weight", {c.act_hidden, d + 4});
  put("act_head.0.bias", {c.act_hidden});
  put("act_head.2.weight", {c.n_act, c.act_hidden});
  put("act_head.2.bias", {c.n_act});
}

const DevTensor& need(Engine& E, const std::string& name) {
  auto it = E.weights.find(name);
  LAYA_REQUIRE(it != E.weights.end(), "missing tensor: " + name);
  return it->second;
}
const float* f32(Engine& E, const std::string& name) { return static_cast<const float*>(need(E, name).ptr); }

void destroy_slot(Engine& E, Slot* s) {
  if (s->graph) (void)hipGraphExecDestroy(s->graph);
  if (s->start) (void)hipEventDestroy(s->start);
  if (s->end) (void)hipEventDestroy(s->end);
  if (s->arena) (void)hipFree(s->arena);
  if (s->h_packed) (void)hipHostFree(s->h_packed);
  if (s->h_logits) (void)hipHostFree(s->h_logits);
  E.slot_bytes -= s->bytes;
  delete s;
}

// Packed rows from which a slot keeps the projection outputs that feed a residual add in 16 bits:
// there the GEMMs need no split-K and the fp32 partials would be the largest HBM stream of the
// add+LayerNorm kernels.  Below it the out and down projections need split-K to fill the chip
// (at 512 rows the 16-bit form saves 8 us of add+LayerNorm per forward but costs 80 us of GEMM).
constexpr int kBranch16Rows = kBatchedRows;

// Launch plans of a slot of shape (m, b, k): GEMM tiles and split-K, attention kernel, head
// splits.  Host arithmetic only (no allocation).
void plan_slot(const Engine& E, Slot* s, int m, int b, int k) {
  const LayaConfig& c = E.cfg;
  s->m = m;
  s->b = b;
  s->k = k;
  s->L = make_layout(m, b, k);
  const int d = c.width, f = c.intermediate;
  LAYA_REQUIRE(gemm_operands_addressable(m, std::max(f, 4 * d), std::max(3 * d, 4 * d), std::max(f, 4 * d)),
               "a shape class of " + std::to_string(m) + " packed rows exceeds the 4 GiB GEMM operand limit");
  gemm_plan(m, 3 * d, d, Epi::QKV, E.mfma(), E.cus, &s->tile[0], &s->splits[0], E.modern);
  gemm_plan(m, d, d, Epi::F32, E.mfma(), E.cus, &s->tile[1], &s->splits[1]);
  if (E.modern) {
    gemm_plan(m, 2 * f, d, Epi::GEGLU, E.mfma(), E.cus, &s->tile[2], &s->splits[2]);
  } else {
    gemm_plan(m, f, d, Epi::GELU, E.mfma(), E.cus, &s->tile[2], &s->splits[2]);
  }
  gemm_plan(m, d, f, Epi::F32, E.mfma(), E.cus, &s->tile[3], &s->splits[3]);
  s->splits[0] = s->splits[2] = 1;
  if (m >= kBranch16Rows) {
    s->branch16 = true;
    gemm_plan(m, d, d, Epi::HALF, E.mfma(), E.cus, &s->tile[1], &s->splits[1]);
    gemm_plan(m, d, f, Epi::HALF, E.mfma(), E.cus, &s->tile[3], &s->splits[3]);
    s->splits[1] = s->splits[3] = 1;
  }
  const int R = s->L.R;
  if (E.modern) {  // head transformer layers: all rows, then the readout rows of the last one
    gemm_plan(m, 3 * d, d, Epi::QKV, E.mfma(), E.cus, &s->htile[0], &s->hsplits[0]);
    gemm_plan(m, d, d, Epi::F32, E.mfma(), E.cus, &s->htile[1], &s->hsplits[1]);
    gemm_plan(m, 4 * d, d, Epi::RELU, E.mfma(), E.cus, &s->htile[2], &s->hsplits[2]);
    gemm_plan(m, d, 4 * d, Epi::F32, E.mfma(), E.cus, &s->htile[3], &s->hsplits[3]);
    gemm_plan(R, d, d, Epi::F32, E.mfma(), E.cus, &s->htile[4], &s->hsplits[4]);
    gemm_plan(R, 4 * d, d, Epi::RELU, E.mfma(), E.cus, &s->htile[5], &s->hsplits[5]);
    gemm_plan(R, d, 4 * d, Epi::F32, E.mfma(), E.cus, &s->htile[6], &s->hsplits[6]);
    s->hsplits[0] = s->hsplits[2] = s->hsplits[5] = 1;
  }
  // Few 128-query tiles (batch-1 requests): split each tile's keys across waves instead of
  // sharing LDS-staged keys between query tiles, so the serial key loop is short.
  if (static_cast<long long>(m / 128) * c.heads >= 2LL * E.cus) {
    s->attn_mode = kAttnSharedKV;
    s->attn_waves = 8;
  } else {
    // Each 32-query tile's keys split across waves.  More waves shorten the serial key blocks
    // per wave while the workgroups fit one round on the CUs (one workgroup per CU: four waves
    // hold one per SIMD, eight two); at 512 tokens four waves measured 6.6 against 8.7 us for two
    // (192 workgroups) and eight waves, one 64-key block each, 6.1 us, while at 1,024 tokens
    // (384 workgroups) two waves, two workgroups per CU and one round win, 15.9 against 17.8 us.
    s->attn_mode = kAttnSplitKeys;
    const bool one_round = static_cast<long long>((m + 31) / 32) * c.heads <= E.cus;
    s->attn_waves = !one_round ? 2 : m >= 8 * 64 ? 8 : 4;
    // Past 512 keys a split-key wave needs more than one block: pair the 32-query groups instead,
    // so each K/V block serves 64 queries (measured per launch, 12 heads: 640 tokens 9.0 against
    // 12.0 us, 1,024 tokens 11.4 against 15.8, 2,048 tokens with four waves 36.0 against 37.5; at
    // 512 tokens the split-key kernel's 6.3 us beats 7.5).
    if (m > 8 * 64) {
      s->attn_mode = kAttnPairKeys;
      s->attn_waves = m > 1536 ? 4 : 8;
    }
  }
  // Tiles of at most `block` rows: every sequence, and every run of rows between or after
  // sequences, adds at most one partial tile, so this bounds the work list of any request.
  const int block = attention_block_rows(s->attn_mode, s->attn_waves);
  s->attn_tiles = std::min(s->L.T, m / block + 2 * b + 1);
  s->head_splits = head_gemm_splits(s->L.R, d, d, E.cus);
  // act_head.0's CLS-row columns: at least enough splits that each covers at most 128 columns (one
  // staged chunk, one memory round trip), so this product ends no later than the scorer's.
  s->act_splits = head_gemm_splits(b, c.act_hidden, d, E.cus);
  while (d / s->act_splits > 128 && d % (s->act_splits * 2 * 32) == 0) s->act_splits *= 2;
}

// The device buffers of a planned slot, in arena order, each starting at a 256-byte boundary.
// Writes the buffer pointers relative to `base` (null: offsets only) and returns the arena size.
size_t carve_slot(const Engine& E, Slot* s, char* base) {
  const LayaConfig& c = E.cfg;
  const int m = s->m, b = s->b, k = s->k, d = c.width, f = c.intermediate;
  const int max_split = std::max(std::max(s->splits[1], s->splits[3]), std::max(s->hsplits[1], s->hsplits[3]));
  const int sel_split = std::max(s->hsplits[4], s->hsplits[6]);
  const size_t ff_cols = E.modern ? std::max(f, 4 * d) : f;  // GeGLU output f; head linear1 4d
  const size_t h2 = 2;  // 16-bit element
  const size_t md = static_cast<size_t>(m) * d, Rz = s->L.R;
  const size_t rows_sel = E.modern ? Rz : 0;  // compact head-layer buffers (ModernBERT only)
  struct Part {
    void** dst;
    size_t bytes;
  };
  const Part parts[] = {
      {reinterpret_cast<void**>(&s->d_packed), s->L.total * 4},
      {reinterpret_cast<void**>(&s->residual), md * 4},
      {&s->x, md * h2},
      {&s->q, md * h2},
      {&s->kk, md * h2},
      {&s->vt, md * h2},
      {&s->attn, md * h2},
      {&s->ff, static_cast<size_t>(m) * ff_cols * h2},
      {reinterpret_cast<void**>(&s->part), md * 4 * max_split},
      {reinterpret_cast<void**>(&s->selected), Rz * d * 4},
      {reinterpret_cast<void**>(&s->normed), Rz * d * 4},
      {reinterpret_cast<void**>(&s->hpart), Rz * d * 4 * s->head_splits},
      {&s->attn_sel, rows_sel * d * h2},
      {&s->x_sel, rows_sel * d * h2},
      {&s->ff_sel, rows_sel * 4 * d * h2},
      {reinterpret_cast<void**>(&s->part_sel), rows_sel * d * 4 * sel_split},
      {reinterpret_cast<void**>(&s->apart), static_cast<size_t>(b) * c.act_hidden * 4 * s->act_splits},
      {reinterpret_cast<void**>(&s->logits), static_cast<size_t>(b) * (k + 1) * 4},
      {reinterpret_cast<void**>(&s->acts), static_cast<size_t>(b) * c.n_act * 4},
  };
  size_t at = 0;
  for (const Part& p : parts) {
    *p.dst = base ? base + at : nullptr;
    at += (p.bytes + 255) / 256 * 256;
  }
  return at;
}

// Host side of Slot.fill's contract: validate the caller's block, then derive the attention tile
// list and the compact head-row list into the same staging buffer (packing.cpp).
void derive_inputs(const Engine& E, Slot& s) {
  const PackLimits lim{E.cfg.vocab, E.modern ? E.rope_rows : E.cfg.max_positions, E.modern};
  const char* err = derive_packed(lim, s.m, s.b, s.k, s.L, s.h_packed,
                                  attention_block_rows(s.attn_mode, s.attn_waves), s.attn_tiles);
  if (err) throw Failure{LAYA_EINVAL, err};
}

void check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Failure{LAYA_EDEVICE, std::string(what) + ": " + hipGetErrorString(e)};
}

// The forward as a list of launches ("stages"); forward() runs them in order, and the timing
// entry point replays one of them in isolation.  Encoder stages repeat per encoder layer, head
// stages (ModernBERT variant) per head transformer layer.
enum Stage : int {
  kEmbed = 0, kQkv, kAttention, kAttnOut, kAttnNorm, kFfnUp, kFfnDown, kFfnNorm,
  kTypeNorm, kHlQkv, kHlAttention, kHlGather, kHlOut, kHlNorm2, kHlUp, kHlDown, kHlNorm,
  kHeadGather, kHeadScorer, kHeadTail, kStageCount
};
const char* const kStageNames[kStageCount] = {
    "embed_norm", "qkv", "attention", "attn_out", "attn_norm", "ffn_up", "ffn_down", "ffn_norm",
    "type_norm", "head_qkv", "head_attention", "head_gather_rows", "head_out", "head_norm2", "head_up",
    "head_down", "head_norm", "head_gather", "head_scorer", "head_tail"};
bool per_layer(int stage) { return stage >= kQkv && stage <= kFfnNorm; }
bool per_head_layer(int stage) { return stage >= kHlQkv && stage <= kHlNorm; }
// Whether a stage belongs to this engine's forward (for layer `layer` of its kind).
bool stage_used(const Engine& E, int stage, int layer) {
  // BERT-style: the last layer's residual + LayerNorm runs inside the head gather, on the gathered
  // rows only.
  if (stage == kFfnNorm && !E.modern && layer == E.cfg.layers - 1) return false;
  if (per_layer(stage)) return layer >= 0 && layer < E.cfg.layers;
  if (per_head_layer(stage)) {
    const int last = E.cfg.head_layers - 1;
    return E.modern && layer >= 0 && layer <= last && (stage != kHlGather || layer == last);
  }
  if (stage == kTypeNorm) return E.modern;
  if (stage == kHeadGather) return !E.modern;
  return stage >= 0 && stage < kStageCount;
}

// Batched slots: the norm after the out/down projection adds their 16-bit output (bias included)
// instead of summing fp32 partials and the bias.
void use_branch16(const Slot& s, AddNormArgs& na) {
  if (!s.branch16) return;
  na.branch16 = na.parts;
  na.parts = nullptr;
  na.splits = 1;
  na.bias = nullptr;
}

void launch_stage(Engine& E, Slot& s, int stage, int layer) {
  const LayaConfig& c = E.cfg;
  const int m = s.m, d = c.width, f = c.intermediate, R = s.L.R;
  const DType t = E.mfma();
  const int32_t* P = s.d_packed;
  const Layout& L = s.L;
  hipStream_t st = E.stream;
  const long long md = static_cast<long long>(m) * d, rd = static_cast<long long>(R) * d;
  const Layer* ly = per_layer(stage) ? &E.layers[layer] : nullptr;
  const HeadLayer* hl = per_head_layer(stage) ? &E.head_layers[layer] : nullptr;
  const bool last_head = hl && layer == c.head_layers - 1;
  GemmArgs g{};
  switch (stage) {
    case kEmbed: {
      // BERT-style: + position row + type row 0, LN with bias.  ModernBERT: token row, LN without
      // bias; layer 0 has no attention norm, so x is the normalised embedding itself.
      EmbedArgs ea{P + L.ids, P + L.positions, E.tok, E.pos, E.type0, E.emb_g, E.emb_b, c.eps,
                   s.residual, s.x, m, c.vocab, c.max_positions};
      check_launch(launch_embed(ea, d, t, st), "embed");
      break;
    }
    case kQkv:
      g.a = s.x; g.b = ly->wqkv; g.M = m; g.N = 3 * d; g.K = d; g.lda = d; g.ldb = d;
      g.bias = ly->bqkv; g.splits = 1; g.q = s.q; g.k = s.kk; g.vt = s.vt; g.width = d;
      if (E.modern) {
        const size_t table = static_cast<size_t>(E.rope_rows) * 32;
        g.rope_cos = E.rope + (ly->local ? 2 : 0) * table;
        g.rope_sin = g.rope_cos + table;
        g.positions = P + L.positions;
      }
      check_launch(launch_gemm(g, Epi::QKV, t, s.tile[0], st), "qkv");
      break;
    case kAttention: {
      AttnArgs aa{s.q, s.kk, s.vt, s.attn, P + L.tiles, m, c.heads, s.attn_tiles, ly->local ? c.window : -1,
                  P + L.n_tiles};
      check_launch(launch_attention(aa, t, s.attn_mode, s.attn_waves, st), "attention");
      break;
    }
    case kAttnOut:
      g.a = s.attn; g.b = ly->wo; g.M = m; g.N = d; g.K = d; g.lda = d; g.ldb = d;
      g.out = s.part; g.ldo = d; g.split_stride = md; g.splits = s.splits[1];
      if (s.branch16) g.bias = ly->bo;  // null for ModernBERT
      check_launch(launch_gemm(g, s.branch16 ? Epi::HALF : Epi::F32, t, s.tile[1], st), "attn out");
      break;
    case kAttnNorm: {
      // BERT-style: residual = LN(residual + branch + bias).  ModernBERT (pre-LN):
      // residual += branch, x = mlp_norm(residual).
      AddNormArgs na = E.modern
          ? AddNormArgs{s.residual, s.part, s.splits[1], md, nullptr, ly->n2g, nullptr, c.eps, s.residual, nullptr, s.x, m}
          : AddNormArgs{s.residual, s.part, s.splits[1], md, ly->bo, ly->n1g, ly->n1b, c.eps, nullptr, s.residual, s.x, m};
      use_branch16(s, na);
      check_launch(launch_add_norm(na, d, t, st), "attention norm");
      break;
    }
    case kFfnUp:
      g.a = s.x; g.b = ly->wi; g.M = m; g.K = d; g.lda = d; g.ldb = d; g.bias = ly->bi; g.out = s.ff;
      g.ldo = f; g.splits = 1;
      g.N = E.modern ? 2 * f : f;
      check_launch(launch_gemm(g, E.modern ? Epi::GEGLU : Epi::GELU, t, s.tile[2], st), "ffn up");
      break;
    case kFfnDown:
      g.a = s.ff; g.b = ly->wo2; g.M = m; g.N = d; g.K = f; g.lda = f; g.ldb = f;
      g.out = s.part; g.ldo = d; g.split_stride = md; g.splits = s.splits[3];
      if (s.branch16) g.bias = ly->bo2;  // null for ModernBERT
      check_launch(launch_gemm(g, s.branch16 ? Epi::HALF : Epi::F32, t, s.tile[3], st), "ffn down");
      break;
    case kFfnNorm: {
      AddNormArgs na{};
      if (!E.modern) {
        na = AddNormArgs{s.residual, s.part, s.splits[3], md, ly->bo2, ly->n2g, ly->n2b, c.eps, nullptr, s.residual, s.x, m};
      } else if (layer + 1 < c.layers) {  // residual += branch, x = next layer's attn_norm(residual)
        na = AddNormArgs{s.residual, s.part, s.splits[3], md, nullptr, E.layers[layer + 1].n1g, nullptr, c.eps,
                         s.residual, nullptr, s.x, m};
      } else {  // last layer: residual = final_norm(residual + branch), in place (runtime.py:107-109)
        na = AddNormArgs{s.residual, s.part, s.splits[3], md, nullptr, E.final_norm, nullptr, c.eps, nullptr,
                         s.residual, nullptr, m};
      }
      use_branch16(s, na);
      check_launch(launch_add_norm(na, d, t, st), "ffn norm");
      break;
    }
    case kTypeNorm: {  // residual += type_emb[kind of each row] (laya.py:218), x = norm1 of head layer 0
      const HeadLayer& h0 = E.head_layers[0];
      AddNormArgs na{s.residual, nullptr, 1, 0, nullptr, h0.n1g, h0.n1b, 1e-5f, s.residual, nullptr, s.x, m,
                     E.type_emb, P + L.kinds};
      check_launch(launch_add_norm(na, d, t, st), "type norm");
      break;
    }
    case kHlQkv:
      g.a = s.x; g.b = hl->in_w; g.M = m; g.N = 3 * d; g.K = d; g.lda = d; g.ldb = d;
      g.bias = hl->in_b; g.splits = 1; g.q = s.q; g.k = s.kk; g.vt = s.vt; g.width = d;
      check_launch(launch_gemm(g, Epi::QKV, t, s.htile[0], st), "head in_proj");
      break;
    case kHlAttention: {
      AttnArgs aa{s.q, s.kk, s.vt, s.attn, P + L.tiles, m, c.heads, s.attn_tiles, -1, P + L.n_tiles};
      check_launch(launch_attention(aa, t, s.attn_mode, s.attn_waves, st), "head attention");
      break;
    }
    case kHlGather: {  // last head layer: only the readout rows go on (laya.py:225-228)
      GatherRowsArgs ga{s.residual, s.selected, s.attn, s.attn_sel, P + L.sel_src, P + L.n_sel, R};
      check_launch(launch_gather_rows(ga, d, t, st), "head gather rows");
      break;
    }
    case kHlOut:
      g.b = hl->out_w; g.N = d; g.K = d; g.lda = d; g.ldb = d; g.ldo = d;
      if (last_head) {
        g.a = s.attn_sel; g.M = R; g.out = s.part_sel; g.split_stride = rd; g.splits = s.hsplits[4];
        check_launch(launch_gemm(g, Epi::F32, t, s.htile[4], st), "head out_proj");
      } else {
        g.a = s.attn; g.M = m; g.out = s.part; g.split_stride = md; g.splits = s.hsplits[1];
        check_launch(launch_gemm(g, Epi::F32, t, s.htile[1], st), "head out_proj");
      }
      break;
    case kHlNorm2: {  // residual += out_proj(attention) + bias, x = norm2(residual)
      AddNormArgs na = last_head
          ? AddNormArgs{s.selected, s.part_sel, s.hsplits[4], rd, hl->out_b, hl->n2g, hl->n2b, 1e-5f, s.selected,
                        nullptr, s.x_sel, R}
          : AddNormArgs{s.residual, s.part, s.hsplits[1], md, hl->out_b, hl->n2g, hl->n2b, 1e-5f, s.residual,
                        nullptr, s.x, m};
      check_launch(launch_add_norm(na, d, t, st), "head norm2");
      break;
    }
    case kHlUp:
      g.b = hl->l1_w; g.N = 4 * d; g.K = d; g.lda = d; g.ldb = d; g.bias = hl->l1_b; g.ldo = 4 * d; g.splits = 1;
      if (last_head) {
        g.a = s.x_sel; g.M = R; g.out = s.ff_sel;
        check_launch(launch_gemm(g, Epi::RELU, t, s.htile[5], st), "head linear1");
      } else {
        g.a = s.x; g.M = m; g.out = s.ff;
        check_launch(launch_gemm(g, Epi::RELU, t, s.htile[2], st), "head linear1");
      }
      break;
    case kHlDown:
      g.b = hl->l2_w; g.N = d; g.K = 4 * d; g.lda = 4 * d; g.ldb = 4 * d; g.ldo = d;
      if (last_head) {
        g.a = s.ff_sel; g.M = R; g.out = s.part_sel; g.split_stride = rd; g.splits = s.hsplits[6];
        check_launch(launch_gemm(g, Epi::F32, t, s.htile[6], st), "head linear2");
      } else {
        g.a = s.ff; g.M = m; g.out = s.part; g.split_stride = md; g.splits = s.hsplits[3];
        check_launch(launch_gemm(g, Epi::F32, t, s.htile[3], st), "head linear2");
      }
      break;
    case kHlNorm: {
      // residual += linear2(...) + bias; then the next head layer's norm1, or - after the last
      // layer, on the readout rows - the scorer's LayerNorm (scorer.0, fp32 rows for its GEMM).
      AddNormArgs na{};
      if (last_head) {
        na = AddNormArgs{s.selected, s.part_sel, s.hsplits[6], rd, hl->l2_b, E.s0w, E.s0b, 1e-5f, s.selected,
                         s.normed, nullptr, R};
      } else {
        const HeadLayer& nx = E.head_layers[layer + 1];
        na = AddNormArgs{s.residual, s.part, s.hsplits[3], md, hl->l2_b, nx.n1g, nx.n1b, 1e-5f, s.residual,
                         nullptr, s.x, m};
      }
      check_launch(launch_add_norm(na, d, t, st), "head norm");
      break;
    }
    case kHeadGather: {
      // The last layer's residual + LayerNorm runs here on the gathered rows only.
      const Layer& last = E.layers[c.layers - 1];
      HeadGatherArgs hg{s.residual, P + L.sel_src, P + L.sel_q, P + L.qkind, P + L.n_sel, E.type_emb,
                        E.s0w, E.s0b, 1e-5f, s.selected, s.normed, L.R};
      hg.n_gamma = last.n2g;
      hg.n_beta = last.n2b;
      hg.n_eps = c.eps;
      if (s.branch16) {
        hg.branch16 = s.part;
      } else {
        hg.parts = s.part;
        hg.splits = s.splits[3];
        hg.part_stride = static_cast<long long>(md);
        hg.bias = last.bo2;
      }
      check_launch(launch_head_gather(hg, d, t, st), "head gather");
      break;
    }
    case kHeadScorer: {
      // scorer.1 over the head rows and, in the same launch, act_head.0's CLS-row columns (its
      // input is the question's CLS row of `selected` and four features the tail adds).
      HeadGemmArgs hm{s.normed, E.s1w, s.hpart, P + L.n_sel, L.R, d, d, s.head_splits, static_cast<long long>(L.R) * d};
      HeadGemmArgs ha{s.selected, E.a0w, s.apart, P + L.meta + 1, s.b, c.act_hidden, d, s.act_splits,
                      static_cast<long long>(s.b) * c.act_hidden};
      ha.x_rows = P + L.qoff;
      ha.x_cap = L.R;
      ha.ldx = d;
      ha.ldw = d + 4;  // act_head.0.weight rows: the d CLS columns, then the four feature columns
      check_launch(launch_head_gemm(hm, ha, st), "scorer");
      break;
    }
    case kHeadTail: {
      HeadTailArgs ht{s.hpart, s.head_splits, static_cast<long long>(L.R) * d, E.s1b, E.s3w, E.s3b,
                      s.apart, s.act_splits, static_cast<long long>(s.b) * c.act_hidden, E.a0w, d + 4,
                      E.a0b, E.a2w, E.a2b, P + L.counts, P + L.qoff, P + L.meta + 1, s.logits, s.acts,
                      s.b, s.k, c.act_hidden, c.n_act};
      check_launch(launch_head_tail(ht, d, st), "head tail");
      break;
    }
    default:
      throw Failure{LAYA_EINVAL, "unknown stage"};
  }
}

// The whole forward on the engine's stream.  With `marks`, the kernel of every launch of stage
// `marked` records marks[2i] and marks[2i+1] at its start and end (its i-th launch), for timing
// the stage where it runs in the forward.
void forward(Engine& E, Slot& s, int marked = -1, hipEvent_t* marks = nullptr) {
  int mark = 0;
  auto run = [&](int stage, int layer) {
    const bool timed = marks && stage == marked;
    if (timed) {
      launch_timing = LaunchTiming{marks[2 * mark], marks[2 * mark + 1]};
      ++mark;
    }
    // However the stage ends (a launch that fails before its kernel takes the events throws), no
    // event pair stays armed for a later launch on this thread: the caller destroys the events.
    const ScopeExit disarm([&] { if (timed) launch_timing = LaunchTiming{}; });
    launch_stage(E, s, stage, layer);
    if (timed && launch_timing.start)  // the stage launched nothing (no rows): nothing to time
      throw Failure{LAYA_EINVAL, "timed stage launched no kernel"};
  };
  run(kEmbed, 0);
  for (int i = 0; i < E.cfg.layers; ++i)
    for (int stage = kQkv; stage <= kFfnNorm; ++stage)
      if (stage_used(E, stage, i)) run(stage, i);
  if (E.modern) {
    run(kTypeNorm, 0);
    for (int j = 0; j < E.cfg.head_layers; ++j)
      for (int stage = kHlQkv; stage <= kHlNorm; ++stage)
        if (stage_used(E, stage, j)) run(stage, j);
  } else {
    run(kHeadGather, 0);
  }
  for (int stage = kHeadScorer; stage < kStageCount; ++stage) run(stage, 0);
}

Slot* create_slot(Engine& E, int m, int b, int k) {
  Slot* s = new Slot();
  try {
    plan_slot(E, s, m, b, k);
    const size_t total = carve_slot(E, s, nullptr);
    LAYA_HIP(hipMalloc(&s->arena, total));
    s->bytes = total;
    E.slot_bytes += total;
    carve_slot(E, s, static_cast<char*>(s->arena));
    LAYA_HIP(hipHostMalloc(reinterpret_cast<void**>(&s->h_packed), s->L.total * 4, hipHostMallocDefault));
    const size_t acts_at = reinterpret_cast<char*>(s->acts) - reinterpret_cast<char*>(s->logits);
    s->h_out_bytes = acts_at + static_cast<size_t>(b) * E.cfg.n_act * 4;
    LAYA_HIP(hipHostMalloc(reinterpret_cast<void**>(&s->h_logits), s->h_out_bytes, hipHostMallocDefault));
    s->h_acts = reinterpret_cast<float*>(reinterpret_cast<char*>(s->h_logits) + acts_at);
    LAYA_HIP(hipEventCreate(&s->start));
    LAYA_HIP(hipEventCreate(&s->end));
  } catch (...) {
    destroy_slot(E, s);
    throw;
  }
  return s;
}

// ModernBERT variant: layer tables and the RoPE cos/sin tables of both thetas (runtime.py:159-165:
// freq_i = 1 / theta^(2i/64), angle = position * freq_i), over every position a packed row can hold.
void finalize_modern(Engine& E) {
  const LayaConfig& c = E.cfg;
  E.final_norm = f32(E, "encoder.final_norm.weight");
  E.pos = nullptr;
  E.type0 = nullptr;
  E.emb_b = nullptr;
  for (int i = 0; i < c.layers; ++i) {
    const std::string p = "encoder.layers." + std::to_string(i) + ".";
    Layer ly{};
    ly.wqkv = need(E, p + "attn.Wqkv.weight").ptr;
    ly.wo = need(E, p + "attn.Wo.weight").ptr;
    ly.wi = need(E, p + "mlp.Wi.weight").ptr;
    ly.wo2 = need(E, p + "mlp.Wo.weight").ptr;
    ly.n1g = i ? f32(E, p + "attn_norm.weight") : nullptr;
    ly.n2g = f32(E, p + "mlp_norm.weight");
    ly.local = i % c.global_every != 0;
    E.layers.push_back(ly);
  }
  for (int i = 0; i < c.head_layers; ++i) {
    const std::string p = "head.layers." + std::to_string(i) + ".";
    HeadLayer h{};
    h.in_w = need(E, p + "self_attn.in_proj_weight").ptr;
    h.in_b = f32(E, p + "self_attn.in_proj_bias");
    h.out_w = need(E, p + "self_attn.out_proj.weight").ptr;
    h.out_b = f32(E, p + "self_attn.out_proj.bias");
    h.l1_w = need(E, p + "linear1.weight").ptr;
    h.l1_b = f32(E, p + "linear1.bias");
    h.l2_w = need(E, p + "linear2.weight").ptr;
    h.l2_b = f32(E, p + "linear2.bias");
    h.n1g = f32(E, p + "norm1.weight");
    h.n1b = f32(E, p + "norm1.bias");
    h.n2g = f32(E, p + "norm2.weight");
    h.n2b = f32(E, p + "norm2.bias");
    E.head_layers.push_back(h);
  }
  const int rows = span16(c.max_len);
  std::vector<float> tables(static_cast<size_t>(4) * rows * 32);
  const float theta[2] = {c.theta_global, c.theta_local};
  for (int t = 0; t < 2; ++t)
    for (int i = 0; i < 32; ++i) {
      const float freq = 1.0f / std::pow(theta[t], static_cast<float>(2 * i) / 64.0f);
      for (int p = 0; p < rows; ++p) {
        const float angle = static_cast<float>(p) * freq;
        tables[(static_cast<size_t>(2 * t) * rows + p) * 32 + i] = std::cos(angle);
        tables[(static_cast<size_t>(2 * t + 1) * rows + p) * 32 + i] = std::sin(angle);
      }
    }
  if (E.rope) {
    (void)hipFree(E.rope);
    E.weight_bytes -= static_cast<size_t>(4) * E.rope_rows * 32 * 4;
    E.rope = nullptr;
  }
  LAYA_HIP(hipMalloc(reinterpret_cast<void**>(&E.rope), tables.size() * 4));
  E.rope_rows = rows;
  E.weight_bytes += tables.size() * 4;
  LAYA_HIP(hipMemcpy(E.rope, tables.data(), tables.size() * 4, hipMemcpyHostToDevice));
}

Slot* find_slot(Engine& E, int m, int b, int k, bool* miss) {
  for (auto it = E.lru.begin(); it != E.lru.end(); ++it) {
    Slot* s = *it;
    if (s->m == m && s->b == b && s->k == k) {
      E.lru.erase(it);
      E.lru.push_back(s);
      *miss = false;
      return s;
    }
  }
  *miss = true;
  if (static_cast<int>(E.lru.size()) >= E.max_slots) {
    LAYA_HIP(hipStreamSynchronize(E.stream));
    Slot* old = E.lru.front();
    E.lru.pop_front();
    destroy_slot(E, old);
  }
  Slot* s = create_slot(E, m, b, k);
  E.lru.push_back(s);
  return s;
}

int fail(Engine* E, const Failure& f) {
  g_error = f.message;
  if (E) E->error = f.message;
  return f.code;
}

template <typename F>
int guarded(Engine* E, F&& body) {
  try {
    body();
    return LAYA_OK;
  } catch (const Failure& f) {
    return fail(E, f);
  } catch (const std::exception& x) {
    return fail(E, Failure{LAYA_EINVAL, x.what()});
  }
}

std::mutex g_prepare_mutex;
std::vector<int> g_prepared;
// Per device: the device address of `scratch` (each device holds its own copy of the array).
constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};
// One-time set-up of the current device: GEMM and head-tail kernel attributes and the scratch
// address.
void prepare_device() {
  int dev = 0;
  LAYA_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_prepare_mutex);
  for (int d : g_prepared)
    if (d == dev) return;
  LAYA_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index beyond the library's device table");
  LAYA_HIP(gemm_prepare());
  LAYA_HIP(head_prepare());
  void* ptr = nullptr;
  LAYA_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  LAYA_REQUIRE(ptr != nullptr, "no device address for the scratch array");
  g_scratch[dev] = ptr;
  g_prepared.push_back(dev);
}

// laya_predict_static: host staging of the packed block (pageable, process-wide) and the lock
// that serialises the calls, which share each device's scratch.
constexpr size_t kStaticStageInts = static_cast<size_t>(1) << 18;
int32_t g_static_stage[kStaticStageInts];
std::mutex g_static_mutex;

}  // namespace
}  // namespace laya

using namespace laya;

extern "C" {

int laya_abi_version(void) { return LAYA_ABI_VERSION; }

int64_t laya_packed_ints(const LayaShape* shape) {
  if (!shape || shape->rows <= 0 || shape->batch <= 0 || shape->options <= 0) return -1;
  return static_cast<int64_t>(make_layout(shape->rows, shape->batch, shape->options).user_end);
}

int laya_device_count(int* count) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(count != nullptr, "null argument");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || e == hipErrorInsufficientDriver) {
      (void)hipGetLastError();
      n = 0;
    } else {
      LAYA_HIP(e);
    }
    *count = n;
  });
}

int laya_device_info(int device, LayaDevice* out) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(out != nullptr, "null argument");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    LAYA_REQUIRE(device >= 0 && device < n, "no HIP device " + std::to_string(device));
    hipDeviceProp_t p;
    LAYA_HIP(hipGetDeviceProperties(&p, device));
    std::memset(out, 0, sizeof(*out));
    std::strncpy(out->name, p.name, sizeof(out->name) - 1);
    std::strncpy(out->arch, p.gcnArchName, sizeof(out->arch) - 1);
    out->hbm_bytes = static_cast<int64_t>(p.totalGlobalMem);
    out->compute_units = p.multiProcessorCount;
    out->lds_bytes_per_cu = static_cast<int32_t>(p.maxSharedMemoryPerMultiProcessor);
    out->clock_khz = p.clockRate;
    out->supported = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
    int current = 0;
    LAYA_HIP(hipGetDevice(&current));
    LAYA_HIP(hipSetDevice(device));
    size_t free_bytes = 0, total = 0;
    const hipError_t e = hipMemGetInfo(&free_bytes, &total);
    (void)hipSetDevice(current);
    LAYA_HIP(e);
    out->free_bytes = static_cast<int64_t>(free_bytes);
  });
}

int laya_create(const LayaConfig* cfg, int device, int max_slots, void** handle) {
  if (!handle || !cfg) return fail(nullptr, Failure{LAYA_EINVAL, "null argument"});
  *handle = nullptr;
  Engine* E = new Engine();
  const int rc = guarded(nullptr, [&] {
    LAYA_REQUIRE(max_slots >= 1 && max_slots <= 64, "max_cached_shapes must be an integer between 1 and 64");
    check_config(*cfg);
    E->cfg = *cfg;
    E->device = device;
    E->max_slots = max_slots;
    int count = 0;
    LAYA_HIP(hipGetDeviceCount(&count));
    LAYA_REQUIRE(device >= 0 && device < count, "no HIP device " + std::to_string(device));
    LAYA_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    LAYA_HIP(hipGetDeviceProperties(&prop, device));
    LAYA_REQUIRE(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0,
                 std::string(prop.name) + " is " + prop.gcnArchName + "; liblaya_hip is built for gfx950 (MI355X)");
    E->cus = prop.multiProcessorCount;
    E->modern = cfg->norm_order == LAYA_NORM_PRE;
    prepare_device();
    LAYA_HIP(hipStreamCreateWithFlags(&E->stream, hipStreamNonBlocking));
    LAYA_HIP(hipEventCreate(&E->static_start));
    LAYA_HIP(hipEventCreate(&E->static_end));
    build_expected(*E);
  });
  if (rc != LAYA_OK) {
    if (E->static_start) (void)hipEventDestroy(E->static_start);
    if (E->static_end) (void)hipEventDestroy(E->static_end);
    if (E->stream) (void)hipStreamDestroy(E->stream);
    delete E;
    return rc;
  }
  *handle = E;
  return LAYA_OK;
}

int laya_load_weight(void* handle, const char* name, const void* host_data, int host_dtype, const int64_t* shape,
                     int ndim) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    LAYA_REQUIRE(name && host_data && (ndim == 0 || shape), "null argument");
    LAYA_REQUIRE(host_dtype == LAYA_F32 || host_dtype == LAYA_F16 || host_dtype == LAYA_BF16, "bad host dtype");
    const std::string n(name);
    auto it = E->expected.find(n);
    LAYA_REQUIRE(it != E->expected.end(), "Checkpoint tensor names do not match the Laya adapter: " + n);
    LAYA_REQUIRE(static_cast<size_t>(ndim) == it->second.shape.size() &&
                     std::equal(shape, shape + ndim, it->second.shape.begin()),
                 "Incompatible tensor shape: " + n);
    LAYA_HIP(hipSetDevice(E->device));
    size_t count = 1;
    for (int i = 0; i < ndim; ++i) count *= static_cast<size_t>(shape[i]);
    DevTensor t;
    t.shape.assign(shape, shape + ndim);
    t.count = count;
    std::vector<uint8_t> staged;
    const void* src = host_data;
    if (it->second.mfma) {
      t.dtype = E->mfma();
      t.bytes = count * 2;
      staged.resize(t.bytes);
      uint16_t* o = reinterpret_cast<uint16_t*>(staged.data());
      const bool bf = t.dtype == DType::BF16;
      if ((bf && host_dtype == LAYA_BF16) || (!bf && host_dtype == LAYA_F16)) {
        std::memcpy(o, host_data, t.bytes);
      } else {
        for (size_t i = 0; i < count; ++i) {
          const float v = host_value(host_data, host_dtype, i);
          o[i] = bf ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        }
      }
      if (it->second.geglu) {  // interleave gate and value rows (geglu_row)
        const int64_t rows = shape[0], cols = shape[1], f = rows / 2;
        LAYA_REQUIRE(f % 16 == 0, "GeGLU intermediate size must be a multiple of 16: " + n);
        std::vector<uint16_t> inter(count);
        for (int64_t r = 0; r < rows; ++r)
          std::memcpy(&inter[static_cast<size_t>(r) * cols], &o[static_cast<size_t>(geglu_row(r, f)) * cols], cols * 2);
        std::memcpy(o, inter.data(), t.bytes);
        t.geglu = true;
      }
      src = staged.data();
    } else {
      t.dtype = DType::F32;
      t.bytes = count * 4;
      if (host_dtype != LAYA_F32) {
        staged.resize(t.bytes);
        float* o = reinterpret_cast<float*>(staged.data());
        for (size_t i = 0; i < count; ++i) o[i] = host_value(host_data, host_dtype, i);
        src = staged.data();
      }
    }
    auto old = E->weights.find(n);
    if (old != E->weights.end()) {
      (void)hipFree(old->second.ptr);
      E->weight_bytes -= old->second.bytes;
      E->weights.erase(old);
    }
    LAYA_HIP(hipMalloc(&t.ptr, t.bytes));
    E->weight_bytes += t.bytes;
    E->weights[n] = t;
    LAYA_HIP(hipMemcpy(t.ptr, src, t.bytes, hipMemcpyHostToDevice));
    E->finalized = false;
  });
}

int laya_finalize(void* handle) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    for (auto& kv : E->expected) LAYA_REQUIRE(E->weights.count(kv.first), "missing tensor: " + kv.first);
    E->tok = f32(*E, "encoder.embeddings.tok_embeddings.weight");
    E->emb_g = f32(*E, "encoder.embeddings.norm.weight");
    E->layers.clear();
    E->head_layers.clear();
    if (E->modern) {
      finalize_modern(*E);
    } else {
    E->pos = f32(*E, "encoder.embeddings.position_embeddings.weight");
    E->type0 = f32(*E, "encoder.embeddings.token_type_embeddings.weight");
    E->emb_b = f32(*E, "encoder.embeddings.norm.bias");
    for (int i = 0; i < E->cfg.layers; ++i) {
      const std::string p = "encoder.layers." + std::to_string(i) + ".";
      Layer ly;
      ly.wqkv = need(*E, p + "attn.Wqkv.weight").ptr;
      ly.bqkv = f32(*E, p + "attn.Wqkv.bias");
      ly.wo = need(*E, p + "attn.Wo.weight").ptr;
      ly.bo = f32(*E, p + "attn.Wo.bias");
      ly.n1g = f32(*E, p + "post_attn_norm.weight");
      ly.n1b = f32(*E, p + "post_attn_norm.bias");
      ly.wi = need(*E, p + "mlp.Wi.weight").ptr;
      ly.bi = f32(*E, p + "mlp.Wi.bias");
      ly.wo2 = need(*E, p + "mlp.Wo.weight").ptr;
      ly.bo2 = f32(*E, p + "mlp.Wo.bias");
      ly.n2g = f32(*E, p + "post_mlp_norm.weight");
      ly.n2b = f32(*E, p + "post_mlp_norm.bias");
      ly.local = false;
      E->layers.push_back(ly);
    }
    }
    E->type_emb = f32(*E, "type_emb.weight");
    E->s0w = f32(*E, "scorer.0.weight");
    E->s0b = f32(*E, "scorer.0.bias");
    E->s1w = f32(*E, "scorer.1.weight");
    E->s1b = f32(*E, "scorer.1.bias");
    E->s3w = f32(*E, "scorer.3.weight");
    E->s3b = f32(*E, "scorer.3.bias");
    E->a0w = f32(*E, "act_head.0.weight");
    E->a0b = f32(*E, "act_head.0.bias");
    E->a2w = f32(*E, "act_head.2.weight");
    E->a2b = f32(*E, "act_head.2.bias");
    // Graphs captured earlier hold old weight pointers: drop every slot.
    for (Slot* s : E->lru) destroy_slot(*E, s);
    E->lru.clear();
    E->finalized = true;
  });
}

// Slot lookup, validation and the single H2D upload shared by predict and the timing entry point.
static Slot* stage_inputs(Engine* E, const int32_t* host_packed, const LayaShape* shape, bool* miss) {
  if (!E->finalized) throw Failure{LAYA_ESTATE, "predict before laya_finalize"};
  LAYA_REQUIRE(host_packed && shape, "null argument");
  const int m = shape->rows, b = shape->batch, k = shape->options;
  LAYA_REQUIRE(m > 0 && m % 16 == 0 && m <= (1 << 22) && b > 0 && b <= (1 << 16) && k > 0 && k <= (1 << 12),
               "invalid shape class");
  LAYA_HIP(hipSetDevice(E->device));
  Slot* s = find_slot(*E, m, b, k, miss);
  std::memcpy(s->h_packed, host_packed, s->L.user_end * 4);
  derive_inputs(*E, *s);
  LAYA_HIP(hipMemcpyAsync(s->d_packed, s->h_packed, s->L.total * 4, hipMemcpyHostToDevice, E->stream));
  return s;
}

int laya_predict(void* handle, const int32_t* host_packed, const LayaShape* shape, int capture, float* host_logits,
                 float* host_acts, LayaMetrics* metrics) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    LAYA_REQUIRE(host_logits && host_acts, "null argument");
    bool miss = false;
    Slot* s = stage_inputs(E, host_packed, shape, &miss);
    const int b = s->b, k = s->k;
    const bool captured_now = capture && !s->graph;
    if (captured_now) {
      LAYA_HIP(hipStreamBeginCapture(E->stream, hipStreamCaptureModeThreadLocal));
      hipGraph_t graph = nullptr;
      try {
        forward(*E, *s);
      } catch (...) {
        (void)hipStreamEndCapture(E->stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
      }
      LAYA_HIP(hipStreamEndCapture(E->stream, &graph));
      const hipError_t ie = hipGraphInstantiate(&s->graph, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      LAYA_HIP(ie);
    }
    LAYA_HIP(hipEventRecord(s->start, E->stream));
    if (capture && s->graph) {
      LAYA_HIP(hipGraphLaunch(s->graph, E->stream));
    } else {
      forward(*E, *s);
    }
    LAYA_HIP(hipEventRecord(s->end, E->stream));
    LAYA_HIP(hipMemcpyAsync(s->h_logits, s->logits, s->h_out_bytes, hipMemcpyDeviceToHost, E->stream));
    LAYA_HIP(hipStreamSynchronize(E->stream));
    float ms = 0.f;
    LAYA_HIP(hipEventElapsedTime(&ms, s->start, s->end));
    for (int q = 0; q < b; ++q)
      std::memcpy(host_logits + static_cast<size_t>(q) * k, s->h_logits + static_cast<size_t>(q) * (k + 1) + 1, k * 4);
    std::memcpy(host_acts, s->h_acts, static_cast<size_t>(b) * E->cfg.n_act * 4);
    if (metrics) {
      metrics->gpu_ms = ms;
      metrics->cache_miss = miss;
      metrics->graph_capture = captured_now;
      metrics->graph_replay = capture && s->graph != nullptr;
      metrics->owned_gpu_bytes = static_cast<int64_t>(E->weight_bytes + E->slot_bytes);
    }
  });
}

int laya_predict_static(void* handle, const int32_t* host_packed, const LayaShape* shape, float* host_logits,
                        float* host_acts, LayaMetrics* metrics) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    if (!E->finalized) throw Failure{LAYA_ESTATE, "predict before laya_finalize"};
    LAYA_REQUIRE(host_packed && shape && host_logits && host_acts, "null argument");
    const int m = shape->rows, b = shape->batch, k = shape->options;
    LAYA_REQUIRE(m > 0 && m % 16 == 0 && m <= (1 << 22) && b > 0 && b <= (1 << 16) && k > 0 && k <= (1 << 12),
                 "invalid shape class");
    Slot s;  // plans and views into the scratch; owns nothing
    plan_slot(*E, &s, m, b, k);
    const size_t need = carve_slot(*E, &s, nullptr);
    LAYA_REQUIRE(need <= kScratchBytes,
                 "shape class (" + std::to_string(m) + ", " + std::to_string(b) + ", " + std::to_string(k) +
                     ") needs " + std::to_string(need) + " bytes of device scratch; laya_predict_static holds " +
                     std::to_string(kScratchBytes) + " (use laya_predict)");
    LAYA_REQUIRE(s.L.total <= kStaticStageInts, "packed block exceeds the static staging buffer (use laya_predict)");
    LAYA_HIP(hipSetDevice(E->device));
    char* base = static_cast<char*>(g_scratch[E->device]);
    LAYA_REQUIRE(base != nullptr, "device scratch not set up");
    std::lock_guard<std::mutex> lock(g_static_mutex);
    // On any error below, the copies and kernels already queued may still write the shared scratch:
    // drain the stream before the lock is released, so the next caller's work cannot overlap them.
    ScopeExit drain([&] { (void)hipStreamSynchronize(E->stream); });
    carve_slot(*E, &s, base);
    s.h_packed = g_static_stage;
    std::memcpy(s.h_packed, host_packed, s.L.user_end * 4);
    derive_inputs(*E, s);
    LAYA_HIP(hipMemcpyAsync(s.d_packed, s.h_packed, s.L.total * 4, hipMemcpyHostToDevice, E->stream));
    LAYA_HIP(hipEventRecord(E->static_start, E->stream));
    forward(*E, s);
    LAYA_HIP(hipEventRecord(E->static_end, E->stream));
    // logits: option slots 1..k of each question's row (laya.py:208), straight into the caller's rows
    LAYA_HIP(hipMemcpy2DAsync(host_logits, static_cast<size_t>(k) * 4, s.logits + 1, static_cast<size_t>(k + 1) * 4,
                              static_cast<size_t>(k) * 4, b, hipMemcpyDeviceToHost, E->stream));
    LAYA_HIP(hipMemcpyAsync(host_acts, s.acts, static_cast<size_t>(b) * E->cfg.n_act * 4, hipMemcpyDeviceToHost,
                            E->stream));
    drain.release();
    LAYA_HIP(hipStreamSynchronize(E->stream));
    float ms = 0.f;
    LAYA_HIP(hipEventElapsedTime(&ms, E->static_start, E->static_end));
    if (metrics) {
      metrics->gpu_ms = ms;
      metrics->cache_miss = 0;
      metrics->graph_capture = 0;
      metrics->graph_replay = 0;
      metrics->owned_gpu_bytes = static_cast<int64_t>(E->weight_bytes + E->slot_bytes);
    }
  });
}

int laya_stage_count(void) { return kStageCount; }

const char* laya_stage_name(int stage) { return stage >= 0 && stage < kStageCount ? kStageNames[stage] : nullptr; }

int laya_stage_launches(void* handle, int stage, int* launches, int* first_layer) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    LAYA_REQUIRE(launches && first_layer, "null output");
    LAYA_REQUIRE(stage >= 0 && stage < kStageCount, "unknown stage");
    const int span = per_layer(stage) ? E->cfg.layers : per_head_layer(stage) ? E->cfg.head_layers : 1;
    *launches = 0;
    *first_layer = -1;
    for (int j = 0; j < span; ++j)
      if (stage_used(*E, stage, j)) {
        if (*launches == 0) *first_layer = j;
        ++*launches;
      }
  });
}

int laya_time_stage(void* handle, const int32_t* host_packed, const LayaShape* shape, int stage, int layer, int reps,
                    float* avg_ms) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    LAYA_REQUIRE(avg_ms && reps >= 1 && reps <= 100000, "reps must be in [1, 100000]");
    LAYA_REQUIRE(stage >= 0 && stage < kStageCount, "unknown stage");
    if (layer == -1) {  // in-forward timing: every kernel of the stage inside `reps` eager forwards
      LAYA_REQUIRE(reps <= 1000, "in-forward timing takes at most 1000 forwards");
      int launches = 0;
      const int span = per_layer(stage) ? E->cfg.layers : per_head_layer(stage) ? E->cfg.head_layers : 1;
      for (int j = 0; j < span; ++j) launches += stage_used(*E, stage, j);
      LAYA_REQUIRE(launches > 0, "stage not in this model's forward");
      bool miss = false;
      Slot* s = stage_inputs(E, host_packed, shape, &miss);
      // One event pair per timed launch of every repetition, the forwards queued back to back
      // behind the warm one and read after a single synchronisation.  The events skip the
      // system-scope fence (timing only): with it, each recording wrote back and invalidated the
      // caches around the timed kernel, which in a kernel trace then started after a 12 us gap and
      // ran 15.3 against 13.5 us (the 1,024-token attention) - no longer the forward's kernel.
      const size_t pairs = static_cast<size_t>(launches) * reps;
      std::vector<hipEvent_t> marks(2 * pairs, nullptr);
      double total = 0.0;
      try {
        for (hipEvent_t& e : marks) LAYA_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
        forward(*E, *s);  // warm: the first forward of a fresh slot pays first-touch costs
        for (int r = 0; r < reps; ++r) forward(*E, *s, stage, marks.data() + 2 * static_cast<size_t>(launches) * r);
        LAYA_HIP(hipStreamSynchronize(E->stream));
        for (size_t i = 0; i < pairs; ++i) {
          float ms = 0.f;
          LAYA_HIP(hipEventElapsedTime(&ms, marks[2 * i], marks[2 * i + 1]));
          total += ms;
        }
      } catch (...) {
        for (hipEvent_t e : marks)
          if (e) (void)hipEventDestroy(e);
        throw;
      }
      for (hipEvent_t e : marks) (void)hipEventDestroy(e);
      *avg_ms = static_cast<float>(total / (static_cast<double>(reps) * launches));
      return;
    }
    LAYA_REQUIRE(stage_used(*E, stage, layer), "stage or layer not in this model's forward");
    bool miss = false;
    Slot* s = stage_inputs(E, host_packed, shape, &miss);
    forward(*E, *s);  // every buffer the stage reads now holds this request's values
    LAYA_HIP(hipEventRecord(s->start, E->stream));
    for (int r = 0; r < reps; ++r) launch_stage(*E, *s, stage, layer);
    LAYA_HIP(hipEventRecord(s->end, E->stream));
    LAYA_HIP(hipStreamSynchronize(E->stream));
    float ms = 0.f;
    LAYA_HIP(hipEventElapsedTime(&ms, s->start, s->end));
    *avg_ms = ms / static_cast<float>(reps);
  });
}

int laya_read_weight(void* handle, const char* name, float* host_out, int64_t count) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return fail(nullptr, Failure{LAYA_EINVAL, "null handle"});
  return guarded(E, [&] {
    LAYA_REQUIRE(name && host_out, "null argument");
    auto it = E->weights.find(name);
    LAYA_REQUIRE(it != E->weights.end(), std::string("no resident tensor: ") + name);
    const DevTensor& t = it->second;
    LAYA_REQUIRE(static_cast<size_t>(count) == t.count, "element count mismatch");
    LAYA_HIP(hipSetDevice(E->device));
    if (t.dtype == DType::F32) {
      LAYA_HIP(hipMemcpy(host_out, t.ptr, t.bytes, hipMemcpyDeviceToHost));
    } else {
      std::vector<uint16_t> raw(t.count);
      LAYA_HIP(hipMemcpy(raw.data(), t.ptr, t.bytes, hipMemcpyDeviceToHost));
      const int64_t cols = t.shape.size() == 2 ? t.shape[1] : 1, f = t.shape.empty() ? 0 : t.shape[0] / 2;
      for (size_t i = 0; i < t.count; ++i) {
        // resident element i sits at checkpoint row geglu_row(row) for interleaved matrices
        const size_t dst = t.geglu ? static_cast<size_t>(geglu_row(static_cast<int64_t>(i) / cols, f)) * cols + i % cols : i;
        host_out[dst] = t.dtype == DType::BF16 ? bf16_bits_to_f32(raw[i]) : f16_bits_to_f32(raw[i]);
      }
    }
  });
}

int64_t laya_used_bytes(void* handle) {
  Engine* E = static_cast<Engine*>(handle);
  return E ? static_cast<int64_t>(E->weight_bytes + E->slot_bytes) : 0;
}

int laya_slot_count(void* handle) {
  Engine* E = static_cast<Engine*>(handle);
  return E ? static_cast<int>(E->lru.size()) : 0;
}

int laya_destroy(void* handle) {
  Engine* E = static_cast<Engine*>(handle);
  if (!E) return LAYA_OK;
  (void)hipSetDevice(E->device);
  if (E->stream) (void)hipStreamSynchronize(E->stream);
  for (Slot* s : E->lru) destroy_slot(*E, s);
  E->lru.clear();
  for (auto& kv : E->weights) (void)hipFree(kv.second.ptr);
  E->weights.clear();
  if (E->rope) (void)hipFree(E->rope);
  if (E->static_start) (void)hipEventDestroy(E->static_start);
  if (E->static_end) (void)hipEventDestroy(E->static_end);
  if (E->stream) (void)hipStreamDestroy(E->stream);
  delete E;
  return LAYA_OK;
}

const char* laya_last_error(void* handle) {
  Engine* E = static_cast<Engine*>(handle);
  return E ? E->error.c_str() : g_error.c_str();
}

// ---------------- kernel-level entry points ----------------

int laya_attention_block(int mode, int waves) {
  return attention_mode_valid(mode, waves) ? attention_block_rows(mode, waves) : -1;
}

int laya_attention_tiles(const int32_t* starts, const int32_t* lengths, int n_seq, int m, int block, int32_t* tiles,
                         int max_tiles) {
  if (!starts || !lengths || !tiles || n_seq < 0) return -1;
  return build_attention_tiles(starts, lengths, n_seq, m, block, tiles, max_tiles);
}

static DType half_type(int dtype16) { return dtype16 == LAYA_F16 ? DType::F16 : DType::BF16; }

int laya_op_embed(const int32_t* ids, const int32_t* positions, const float* table, const float* pos_table,
                  const float* type_row, const float* gamma, const float* beta, float eps, float* out32, void* out16,
                  int dtype16, int rows, int width, int vocab, int n_positions, void* stream) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(norm_width_supported(width), "unsupported width");
    EmbedArgs a{ids, positions, table, pos_table, type_row, gamma, beta, eps, out32, out16, rows, vocab, n_positions};
    check_launch(launch_embed(a, width, half_type(dtype16), static_cast<hipStream_t>(stream)), "embed");
  });
}

int laya_op_norm(float* residual, const float* branch, int splits, int64_t part_stride, const float* bias,
                 const float* gamma, const float* beta, float eps, float* sum_out, float* out32, void* out16,
                 int dtype16, int rows, int width, void* stream) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(norm_width_supported(width), "unsupported width");
    AddNormArgs a{residual, branch, splits < 1 ? 1 : splits, part_stride, bias, gamma, beta, eps, sum_out, out32, out16, rows};
    check_launch(launch_add_norm(a, width, half_type(dtype16), static_cast<hipStream_t>(stream)), "norm");
  });
}

int laya_op_linear(const void* x, const void* w, const float* bias, void* out, int kind, int dtype16, int M, int N,
                   int K, int splits, int tile, void* stream) {
  return guarded(nullptr, [&] {
    prepare_device();
    LAYA_REQUIRE(kind >= 0 && kind <= 4,
                 "kind must be 0 (fp32), 1 (16-bit), 2 (16-bit GELU), 3 (16-bit ReLU) or 4 (16-bit GeGLU)");
    const Epi epi = kind == 0 ? Epi::F32 : kind == 1 ? Epi::HALF : kind == 2 ? Epi::GELU : kind == 3 ? Epi::RELU
                                                                                                    : Epi::GEGLU;
    int cus = 256;
    if (tile < 0) {
      gemm_plan(M, N, K, epi, half_type(dtype16), cus, &tile, &splits, false, tile == -1);
      if (bias) splits = 1;
    }
    LAYA_REQUIRE(tile < gemm_tile_count(), "bad tile id");
    LAYA_REQUIRE(K % 64 == 0 && N % gemm_tile(tile).bn == 0, "K must be a multiple of 64 and N of the tile width");
    GemmArgs g{};
    g.a = x; g.b = w; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldb = K; g.bias = bias; g.out = out;
    g.ldo = epi == Epi::GEGLU ? N / 2 : N;
    g.split_stride = static_cast<long long>(M) * N; g.splits = splits < 1 ? 1 : splits;
    check_launch(launch_gemm(g, epi, half_type(dtype16), tile, static_cast<hipStream_t>(stream)), "linear");
  });
}

int laya_op_qkv(const void* x, const void* w, const float* bias, void* q, void* k, void* vt, const float* rope_cos,
                const float* rope_sin, const int32_t* positions, int dtype16, int M, int width, int tile,
                void* stream) {
  return guarded(nullptr, [&] {
    prepare_device();
    int splits = 1;
    const bool rope = rope_cos != nullptr;
    LAYA_REQUIRE(!rope || (rope_sin && positions), "RoPE needs cos, sin and positions");
    if (tile < 0) gemm_plan(M, 3 * width, width, Epi::QKV, half_type(dtype16), 256, &tile, &splits, rope, tile == -1);
    LAYA_REQUIRE(tile < gemm_tile_count(), "bad tile id");
    LAYA_REQUIRE(width % 64 == 0 && (3 * width) % gemm_tile(tile).bn == 0, "width does not fit the tile");
    LAYA_REQUIRE(M % 8 == 0, "rows must be a multiple of 8 (V^T is stored in runs of 8 tokens)");
    GemmArgs g{};
    g.a = x; g.b = w; g.M = M; g.N = 3 * width; g.K = width; g.lda = width; g.ldb = width; g.bias = bias;
    g.splits = 1; g.q = q; g.k = k; g.vt = vt; g.width = width;
    g.rope_cos = rope_cos; g.rope_sin = rope_sin; g.positions = positions;
    check_launch(launch_gemm(g, Epi::QKV, half_type(dtype16), tile, static_cast<hipStream_t>(stream)), "qkv");
  });
}

int laya_op_attention(const void* q, const void* k, const void* vt, void* out, const int32_t* tiles, int m,
                      int heads, int max_tiles, int mode, int waves, int window, int dtype16, void* stream) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(attention_mode_valid(mode, waves),
                 "mode 0 (shared K/V) takes 1, 2, 4 or 8 waves; mode 1 (split keys) 2, 4 or 8; mode 2 (paired "
                 "query groups) 4 or 8");
    LAYA_REQUIRE(m % 16 == 0, "rows must be a multiple of 16");
    LAYA_REQUIRE((reinterpret_cast<uintptr_t>(tiles) & 15) == 0, "tile list must be 16-byte aligned");
    AttnArgs a{q, k, vt, out, tiles, m, heads, max_tiles, window < 0 ? -1 : window};
    check_launch(launch_attention(a, half_type(dtype16), mode, waves, static_cast<hipStream_t>(stream)),
                 "attention");
  });
}

int laya_op_gather_rows(const float* src32, float* dst32, const void* src16, void* dst16, int dtype16,
                        const int32_t* indices, const int32_t* n_live, int rows, int width, void* stream) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(norm_width_supported(width), "unsupported width");
    LAYA_REQUIRE(rows >= 0 && indices && n_live, "indices and the live row count are required");
    LAYA_REQUIRE(!src32 == !dst32 && !src16 == !dst16, "each copy needs both its source and destination");
    LAYA_REQUIRE(!src16 || dtype16 == LAYA_F16 || dtype16 == LAYA_BF16, "dtype16 must be LAYA_F16 or LAYA_BF16");
    GatherRowsArgs a{src32, dst32, src16, dst16, indices, n_live, rows};
    check_launch(launch_gather_rows(a, width, half_type(dtype16), static_cast<hipStream_t>(stream)), "gather rows");
  });
}

int laya_op_head_gather(const float* src, const int32_t* src_rows, const int32_t* row_question,
                        const int32_t* question_kind, const int32_t* n_live, const float* type_rows,
                        const float* gamma, const float* beta, float eps, float* selected, float* normed,
                        int rows, int width, void* stream) {
  return guarded(nullptr, [&] {
    LAYA_REQUIRE(norm_width_supported(width), "unsupported width");
    LAYA_REQUIRE(rows >= 0 && src && src_rows && n_live && selected && normed && gamma && beta,
                 "null argument");
    LAYA_REQUIRE(!type_rows || (row_question && question_kind), "type rows need the question map and kinds");
    HeadGatherArgs a{src, src_rows, row_question, question_kind, n_live, type_rows, gamma, beta, eps, selected,
                     normed, rows};
    check_launch(launch_head_gather(a, width, DType::F16, static_cast<hipStream_t>(stream)), "head gather");
  });
}

}  // extern "C"
