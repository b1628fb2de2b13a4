// Bandwidth kernels: embedding gather + LayerNorm, and residual add + LayerNorm.
//
// One wave (64 lanes) owns one token row; a 256-thread workgroup covers 4 rows.  Each lane keeps
// its d/64 values in registers, so the two-pass mean/variance of the reference's layer_norm
// (laya_cuda/kernels.cu:32-48) costs one HBM read per element instead of three, and the
// reductions are wave-wide butterflies with no LDS and no barriers.
#include "kernels.hpp"
#include "rowops.hpp"

namespace laya {

namespace {

template <int D, typename T>
__global__ __launch_bounds__(256) void embed_norm_kernel(EmbedArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  NormParams<D> np;
  if (a.gamma) np.load(a.gamma, a.beta, lane);
  int id = a.ids[row];
  id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);  // host validates; never read out of bounds
  float v[D / 64];
  load_row<D>(a.table + static_cast<size_t>(id) * D, lane, v);
  if (a.pos_table) {
    int p = a.positions[row];
    p = p < 0 ? 0 : (p >= a.n_positions ? a.n_positions - 1 : p);
    float t[D / 64];
    load_row<D>(a.pos_table + static_cast<size_t>(p) * D, lane, t);
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + t[i];
  }
  if (a.type_row) {
    float t[D / 64];
    load_row<D>(a.type_row, lane, t);
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + t[i];
  }
  if (a.gamma) normalize<D>(v, np, a.eps);
  if (a.out32) store_row<D>(a.out32 + static_cast<size_t>(row) * D, lane, v);
  if (a.out16) store_row16<D, T>(static_cast<T*>(a.out16) + static_cast<size_t>(row) * D, lane, v);
}

// NS: the number of split-K partials when it is known at launch (1..kMaxFixedSplits), so that
// every partial's row, the bias and the residual are loaded before the first add (one memory round
// trip; a loop over a run-time split count waited for each partial in turn); 0: no partials (the
// 16-bit branch, or none); -1: any other split count, loaded in a loop.
constexpr int kMaxFixedSplits = 8;
constexpr int kOneWaveRows = 4096;

template <int D, typename T, int NS>
__global__ __launch_bounds__(256) void add_norm_kernel(AddNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const size_t off = static_cast<size_t>(row) * D;
  NormParams<D> np;
  if (a.gamma) np.load(a.gamma, a.beta, lane);
  float v[D / 64];
  load_row<D>(a.residual + off, lane, v);
  if constexpr (NS > 0) {
    // branch = sum of the split-K partial products, then + bias, then added to the residual:
    // one fp32 rounding per add, in a fixed order, so graph replays are bit-identical.
    float br[NS][D / 64], bias[D / 64];
#pragma unroll
    for (int s = 0; s < NS; ++s) load_row<D>(a.parts + static_cast<size_t>(s) * a.part_stride + off, lane, br[s]);
    if (a.bias) load_row<D>(a.bias, lane, bias);
#pragma unroll
    for (int s = 1; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < D / 64; ++i) br[0][i] = br[0][i] + br[s][i];
    if (a.bias) {
#pragma unroll
      for (int i = 0; i < D / 64; ++i) br[0][i] = br[0][i] + bias[i];
    }
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + br[0][i];
  } else if constexpr (NS < 0) {
    float br[D / 64];
    load_row<D>(a.parts + off, lane, br);
    for (int s = 1; s < a.splits; ++s) {
      float t[D / 64];
      load_row<D>(a.parts + static_cast<size_t>(s) * a.part_stride + off, lane, t);
#pragma unroll
      for (int i = 0; i < D / 64; ++i) br[i] = br[i] + t[i];
    }
    if (a.bias) {
      float t[D / 64];
      load_row<D>(a.bias, lane, t);
#pragma unroll
      for (int i = 0; i < D / 64; ++i) br[i] = br[i] + t[i];
    }
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + br[i];
  } else if (a.branch16) {
    // 16-bit projection output with its bias already added before rounding (the reference's
    // layer_norm adds a half branch to the fp32 residual, kernels.cu:20-35).
    float br[D / 64];
    load_row16<D, T>(static_cast<const T*>(a.branch16) + off, lane, br);
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + br[i];
  }
  if (a.row_table) {  // question-type row of this token (type_add, kernels.cu:155-158)
    float t[D / 64];
    load_row<D>(a.row_table + static_cast<size_t>(a.row_index[row]) * D, lane, t);
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + t[i];
  }
  if (a.sum_out) store_row<D>(a.sum_out + off, lane, v);
  if (a.gamma) normalize<D>(v, np, a.eps);
  if (a.out32) store_row<D>(a.out32 + off, lane, v);
  if (a.out16) store_row16<D, T>(static_cast<T*>(a.out16) + off, lane, v);
}

template <typename T>
hipError_t launch_embed_t(const EmbedArgs& a, int width, hipStream_t stream) {
  const dim3 grid((a.rows + 3) / 4), block(256);
  switch (width) {
#define LAYA_CASE(D) case D: LAYA_LAUNCH((embed_norm_kernel<D, T>), grid, block, 0, stream, a); break;
    LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
    LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int D>
void launch_add_norm_d(const AddNormArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  const int ns = !a.parts ? 0 : a.splits <= kMaxFixedSplits ? a.splits : -1;
  switch (ns) {
#define LAYA_NS(N) case N: LAYA_LAUNCH((add_norm_kernel<D, T, N>), grid, block, 0, stream, a); break;
    LAYA_NS(0) LAYA_NS(1) LAYA_NS(2) LAYA_NS(3) LAYA_NS(4) LAYA_NS(5) LAYA_NS(6) LAYA_NS(7) LAYA_NS(8)
#undef LAYA_NS
    default: LAYA_LAUNCH((add_norm_kernel<D, T, -1>), grid, block, 0, stream, a); break;
  }
}

template <typename T>
hipError_t launch_add_norm_t(const AddNormArgs& a, int width, hipStream_t stream) {
  // A wave per row.  Few rows (batch-1 requests): one-wave workgroups, so the rows spread over
  // every CU and each CU fetches fewer of them (the fill of one CU, not HBM, bounds these
  // launches); many rows: four-wave workgroups.
  const int wpb = a.rows <= kOneWaveRows ? 1 : 4;
  const dim3 grid((a.rows + wpb - 1) / wpb), block(64 * wpb);
  switch (width) {
#define LAYA_CASE(D) case D: launch_add_norm_d<T, D>(a, grid, block, stream); break;
    LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
    LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool norm_width_supported(int width) {
  switch (width) {
    case 64: case 128: case 256: case 384: case 512: case 768: case 1024: case 1088: case 1280:
    case 1536: case 2048: return true;
    default: return false;
  }
}

hipError_t launch_embed(const EmbedArgs& a, int width, DType t, hipStream_t stream) {
  if (a.rows <= 0) return hipSuccess;
  return t == DType::F16 ? launch_embed_t<f16>(a, width, stream) : launch_embed_t<bf16>(a, width, stream);
}

hipError_t launch_add_norm(const AddNormArgs& a, int width, DType t, hipStream_t stream) {
  if (a.rows <= 0) return hipSuccess;
  return t == DType::F16 ? launch_add_norm_t<f16>(a, width, stream) : launch_add_norm_t<bf16>(a, width, stream);
}

}  // namespace laya
