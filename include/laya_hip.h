/*
 * liblaya_hip: C ABI of the MI355X (gfx950) encoder forward path.
 *
 * This is the drop-in boundary under laya-cuda's Python runtime.  The reference's Runtime
 * (laya_cuda/runtime.py:136-197) owns a CuPy memory pool, one stream, the resident weights and an
 * LRU of shape slots, each with a CUDA graph; Ops (laya_cuda/ops.py:19-71) owns NVRTC kernels and
 * cuBLAS.  Here one opaque engine handle owns all of that natively: an HBM arena per slot, one
 * non-blocking HIP stream, resident weights, and one hipGraph per shape slot.
 *
 * Conventions: every entry point returns 0 (LAYA_OK) or a LAYA_E* status; the message of the
 * last failure is laya_last_error(handle) (handle may be NULL for failures that have none).
 * Pointers named host_* are host memory; every other buffer pointer of the laya_op_* entry
 * points is device memory.  `stream` is a hipStream_t (NULL = the null stream).  A handle is
 * single-threaded: callers serialise access (as the reference's Engine and BatchEngine do).
 */
#ifndef LAYA_HIP_H
#define LAYA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LAYA_ABI_VERSION 2

enum {
  LAYA_OK = 0,
  LAYA_EINVAL = 1,   /* bad argument, name, shape or configuration */
  LAYA_EDEVICE = 2,  /* HIP runtime failure */
  LAYA_ENOMEM = 3,   /* device or pinned allocation failed */
  LAYA_ESTATE = 4    /* call out of order (e.g. predict before finalize) */
};

/* Element types of host weights and of the 16-bit MFMA operand type. */
enum { LAYA_F32 = 0, LAYA_F16 = 1, LAYA_BF16 = 2 };

/* Encoder variants (the reference's executor is pre-LN/RoPE/GeGLU, laya_cuda/laya.py:59-79). */
enum { LAYA_NORM_POST = 0, LAYA_NORM_PRE = 1 };
enum { LAYA_POS_LEARNED = 0, LAYA_POS_ROPE = 1 };
enum { LAYA_FFN_GELU = 0, LAYA_FFN_GEGLU = 1 };

/* Model configuration: the fields the reference's adapter exposes to Runtime
 * (width, heads, layers, intermediate, eps, max_len, n_act, ...; laya_cuda/laya.py:61-81). */
typedef struct LayaConfig {
  int32_t width;          /* d_model; heads * 64 */
  int32_t heads;
  int32_t layers;
  int32_t intermediate;   /* FFN width f */
  int32_t vocab;
  int32_t max_positions;  /* learned position rows */
  int32_t type_vocab;     /* token-type rows (row 0 is added) */
  int32_t norm_order;     /* LAYA_NORM_* */
  int32_t pos_kind;       /* LAYA_POS_* */
  int32_t ffn_kind;       /* LAYA_FFN_* */
  int32_t bias;           /* encoder linear layers carry biases */
  float eps;              /* encoder LayerNorm epsilon */
  int32_t window;         /* local attention half-window, -1 = global */
  int32_t global_every;
  int32_t head_layers;    /* decision-head transformer layers */
  int32_t n_act;          /* act-head outputs */
  int32_t act_hidden;     /* act-head hidden width (256 in Laya) */
  int32_t max_len;        /* longest sequence, tokens */
  int32_t mfma_dtype;     /* LAYA_BF16 or LAYA_F16: resident matrices and MFMA operands */
  float theta_global;     /* RoPE theta of global layers (LAYA_POS_ROPE; laya.py:72-78) */
  float theta_local;      /* RoPE theta of local (windowed) layers */
} LayaConfig;

/* Shape class of one predict: the reference's slot key (laya_cuda/runtime.py:20-25). */
typedef struct LayaShape {
  int32_t rows;     /* packed token rows m (multiple of 16) */
  int32_t batch;    /* question capacity b (also the sequence capacity) */
  int32_t options;  /* option capacity k per question */
} LayaShape;

typedef struct LayaMetrics {
  float gpu_ms;            /* stream time of the forward (graph replay or eager), events */
  int32_t cache_miss;      /* the slot was created by this call */
  int32_t graph_capture;   /* the slot's graph was captured by this call */
  int32_t graph_replay;    /* the forward ran as a graph replay */
  int64_t owned_gpu_bytes; /* weights + slot arenas */
} LayaMetrics;

/*
 * Packed int32 input block of a predict, laid out for shape (m, b, k):
 *   meta[4]          n_seq, n_questions, 0, 0
 *   ids[m] positions[m] rows[m] kinds[m]            per packed token (runtime.py:35-36)
 *   starts[b] lengths[b]                            per sequence
 *   counts[b] qkind[b]                              per question
 *   indices[b*(k+1)]                                per question: CLS row, then option rows,
 *                                                   absolute packed rows (runtime.py:63-66)
 * laya_packed_ints(shape) gives its length.  Sequences start at multiples of 16 rows; rows of
 * no sequence carry rows[i] = -1.
 */
int64_t laya_packed_ints(const LayaShape* shape);

/* One HIP device as the doctor reports it (laya_cuda/cli.py:118-176 reports CUDA devices through
 * CuPy; here the library itself answers, from hipGetDeviceProperties and hipMemGetInfo). */
typedef struct LayaDevice {
  char name[256];
  char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int64_t hbm_bytes;        /* total device memory */
  int64_t free_bytes;       /* free device memory now */
  int32_t compute_units;
  int32_t lds_bytes_per_cu;
  int32_t clock_khz;
  int32_t supported;        /* 1: gfx950, the architecture this library is built for */
} LayaDevice;

/* Number of HIP devices (0 without a driver or device: not an error); the doctor's
 * getDeviceCount (cli.py:140-141). */
int laya_device_count(int* count);
/* Properties of HIP device `device`; the doctor's getDeviceProperties (cli.py:142-147). */
int laya_device_info(int device, LayaDevice* out);

/* Runtime(adapter, device, max_cached_shapes) construction (runtime.py:137-146). */
int laya_create(const LayaConfig* cfg, int device, int max_slots, void** handle);

/* Upload one named checkpoint tensor (runtime.py:147-158): the name set and shapes are those of
 * the adapter's weight_shapes(); matrices feeding MFMA become resident in cfg->mfma_dtype, all
 * other tensors in fp32.  host_dtype is LAYA_F32/F16/BF16, shape has ndim entries. */
int laya_load_weight(void* handle, const char* name, const void* host_data, int host_dtype,
                     const int64_t* shape, int ndim);

/* Checks that every tensor is present (the name-set check of runtime.py:149-151) and resolves the
 * layer tables.  Required before predict. */
int laya_finalize(void* handle);

/* Runtime.predict / Slot.run (runtime.py:115-133, 171-186): find or create the shape slot (LRU
 * eviction at max_slots), upload the packed block, capture the slot's graph on first use when
 * capture != 0, replay (or run eagerly), and copy back host_logits [b][k] (option slots 1..k,
 * laya.py:208) and host_acts [b][n_act]. */
int laya_predict(void* handle, const int32_t* host_packed, const LayaShape* shape, int capture,
                 float* host_logits, float* host_acts, LayaMetrics* metrics);

/* No counterpart in the reference.  For callers that cannot allocate device or pinned memory
 * (tight serving loops, harnesses that forbid hipMalloc): the forward of laya_predict without a
 * shape slot.  Its arena (packed block, activations, split-K partials, head buffers) lives in a
 * fixed 64 MiB device array that every device running the library holds for the life of the
 * process; the packed block is staged through a fixed host array of 2^18 int32.  A shape class
 * whose arena or block does not fit is refused with LAYA_EINVAL (12L/768 requests of up to 1,024
 * packed rows fit).  The forward runs eagerly on the engine's stream (no graph), outputs and
 * metrics as laya_predict (cache_miss, graph_capture and graph_replay are 0).  The call makes no
 * allocation.  Calls share each device's array and the host staging: the library serialises them
 * with a process-wide lock, held until the outputs are on the host; calls that overlapped would
 * race on the array, and each call overwrites what the previous one left there. */
int laya_predict_static(void* handle, const int32_t* host_packed, const LayaShape* shape, float* host_logits,
                        float* host_acts, LayaMetrics* metrics);

/* Per-launch timing, the native counterpart of the reference's profiling hook that records events
 * around every Ops.call/linear (tools/profile_long.py:21-67).  The forward is a fixed list of
 * stages (embed_norm; per layer qkv, attention, attn_out, attn_norm, ffn_up, ffn_down, ffn_norm;
 * head_gather, head_scorer, head_tail).  laya_time_stage uploads the request like
 * laya_predict, runs one eager forward so every buffer holds this request's values, then launches
 * stage `stage` of layer `layer` `reps` times back to back between two events on the engine's
 * stream and stores the average per launch in *avg_ms.  Stages that normalise in place
 * (attn_norm, ffn_norm) change the residual on every repetition: time them, do not read results
 * afterwards.  layer = -1 times the stage where it runs: `reps` (at most 1000) eager forwards,
 * queued back to back, in which every kernel of the stage (all its layers) records the start and
 * end of its own execution (hipExtLaunchKernel events, the interval a kernel trace reports);
 * *avg_ms is their average. */
int laya_stage_count(void);
const char* laya_stage_name(int stage);
/* How many times this engine's forward launches `stage` (0: not part of this model) and the first
 * layer index it runs for, the `layer` argument of laya_time_stage.  Per-launch times times these
 * counts give the per-forward breakdown of tools/profile_long.py:21-67. */
int laya_stage_launches(void* handle, int stage, int* launches, int* first_layer);
int laya_time_stage(void* handle, const int32_t* host_packed, const LayaShape* shape, int stage, int layer,
                    int reps, float* avg_ms);

/* Read a resident tensor back as fp32 (runtime.weights[name], tests/test_custom_models.py:46). */
int laya_read_weight(void* handle, const char* name, float* host_out, int64_t count);
int64_t laya_used_bytes(void* handle);   /* weights + slots: CuPy pool used_bytes() */
int laya_slot_count(void* handle);       /* len(runtime.slots) */
int laya_destroy(void* handle);          /* Runtime.close (runtime.py:188-197) */
const char* laya_last_error(void* handle);  /* the exception text of ops.py:45-48, runtime.py:149-153 */
/* No counterpart in the reference: the version of the struct layouts above, which a binding
 * compares with the one it mirrors before it binds anything else. */
int laya_abi_version(void);

/* ------------------------------------------------------------------------------------------
 * Kernel-level entry points: the Ops surface the reference's kernel tests drive
 * (laya_cuda/ops.py:50-66; tests/test_gpu.py, tests/test_attention.py).
 * ------------------------------------------------------------------------------------------ */

/* Attention work list for packed sequences (Slot.attend's ragged rows, runtime.py:82-88): tiles of
 * up to `block` query rows of one sequence plus zero-tiles for rows of no sequence, as int32 quads
 * (row0, row1, kstart, klen) with klen = -1 for zero-tiles; all max_tiles quads are written (unused
 * ones as empty ranges).  Returns the used count, or -1 for a bad layout or too small a list.
 * Host-only. */
int laya_attention_tiles(const int32_t* starts, const int32_t* lengths, int n_seq, int m, int block,
                         int32_t* tiles, int max_tiles);
/* Query rows per tile of an attention kernel: mode 0 (K/V blocks staged once in LDS and shared by
 * `waves` = 1, 2, 4 or 8 waves of 32 queries each; large batches) -> 32*waves; mode 1 (one tile of
 * 32 queries whose keys are split across `waves` = 2, 4 or 8 waves; batch-1 latency) -> 32; mode 2
 * (64 queries as two 32-query groups sharing each of waves/2 key groups' blocks, waves = 4 or 8;
 * long batch-1 sequences) -> 64.  -1 for an invalid pair. */
int laya_attention_block(int mode, int waves);

/* embed (kernels.cu:16-19) fused with the embeddings norm (runtime.py:93-95):
 * v = table[ids] (+ pos_table[positions]) (+ type_row); LayerNorm if gamma; writes out32 and/or
 * out16 (dtype16 = LAYA_BF16/F16). */
int laya_op_embed(const int32_t* ids, const int32_t* positions, const float* table,
                  const float* pos_table, const float* type_row, const float* gamma,
                  const float* beta, float eps, float* out32, void* out16, int dtype16, int rows,
                  int width, int vocab, int n_positions, void* stream);

/* layer_norm (kernels.cu:20-49): v = residual + (sum of `splits` branch partials + bias);
 * sum_out = v; LayerNorm if gamma; out32/out16 = result.  out32 may alias residual. */
int laya_op_norm(float* residual, const float* branch, int splits, int64_t part_stride,
                 const float* bias, const float* gamma, const float* beta, float eps,
                 float* sum_out, float* out32, void* out16, int dtype16, int rows, int width,
                 void* stream);

/* Ops.linear (ops.py:58-66) with the activate modes (kernels.cu:59-67) as epilogues:
 * out[M][N] = x[M][K] w[N][K]^T (+ bias).  kind 0: fp32 out (split-K partials at out + z*M*N when
 * splits > 1, bias then must be NULL), 1: 16-bit out, 2: 16-bit exact-GELU out, 3: 16-bit ReLU out,
 * 4: GeGLU, out[M][N/2] = gelu(gate) * value with w's rows in the resident GeGLU interleave
 * (32-row groups: 16 gate rows, then their 16 value rows).  tile -1 lets the planner choose tile
 * and splits (splits ignored): the measured plan table when it holds the problem, else the
 * heuristic; tile -2 takes the heuristic alone (the baseline the plan table is measured against). */
int laya_op_linear(const void* x, const void* w, const float* bias, void* out, int kind,
                   int dtype16, int M, int N, int K, int splits, int tile, void* stream);

/* QKV projection with the head-major epilogue that replaces `layout` (kernels.cu:68-82):
 * q, k [heads][M][64], vt [heads][64][M].  With rope_cos non-NULL, Q and K are rotated (rotate-half
 * RoPE, kernels.cu:73-77) in fp32 before rounding, by the [positions][32] cos/sin tables at each
 * row's positions[row].  M must be a multiple of 8.  tile -1 / -2 as for laya_op_linear. */
int laya_op_qkv(const void* x, const void* w, const float* bias, void* q, void* k, void* vt,
                const float* rope_cos, const float* rope_sin, const int32_t* positions, int dtype16,
                int M, int width, int tile, void* stream);

/* attention (kernels.cu:90-154) over a device copy (16-byte aligned) of a tile list from
 * laya_attention_tiles built with laya_attention_block(mode, waves) rows per tile; q, k [heads][m][64],
 * vt [heads][64][m], out [m][heads*64]; window >= 0 keeps only keys with |query - key| <= window (the
 * local layers, kernels.cu:106-107), window < 0 is global attention. */
int laya_op_attention(const void* q, const void* k, const void* vt, void* out, const int32_t* tiles,
                      int m, int heads, int max_tiles, int mode, int waves, int window, int dtype16,
                      void* stream);

/* gather / gather_half (kernels.cu:159-166), the option-position row gather of the decision head
 * (laya.py:226-227, 237): for r < *n_live, dst32[r] = src32[indices[r]] and dst16[r] =
 * src16[indices[r]] (16-bit rows of dtype16), bit-exact copies in the order of `indices`
 * (duplicates allowed); rows n_live..rows-1 are written as zeros.  n_live is a device int32 (the
 * forward reads the live row count on the device); either src/dst pair may be NULL to skip it. */
int laya_op_gather_rows(const float* src32, float* dst32, const void* src16, void* dst16, int dtype16,
                        const int32_t* indices, const int32_t* n_live, int rows, int width, void* stream);

/* The scorer input rows (type_add + gather, kernels.cu:155-162; laya.py:236-238): for r < *n_live,
 * selected[r] = src[src_rows[r]] + type_rows[question_kind[row_question[r]]] (the type row only
 * when type_rows is non-NULL; one fp32 add, bit-exact), and normed[r] = LayerNorm(selected[r];
 * gamma, beta, eps) (scorer.0).  All pointers are device memory; n_live a device int32. */
int laya_op_head_gather(const float* src, const int32_t* src_rows, const int32_t* row_question,
                        const int32_t* question_kind, const int32_t* n_live, const float* type_rows,
                        const float* gamma, const float* beta, float eps, float* selected, float* normed,
                        int rows, int width, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LAYA_HIP_H */
