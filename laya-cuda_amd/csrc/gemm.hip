// MFMA-tiled GEMM for the encoder projections: out = A * B^T (+ bias) with fused epilogues.
//
// Both operands are K-contiguous ("NT": activations [M][K], weights [N][K], the reference's
// cublasGemmEx orientation at laya_cuda/ops.py:63-64), which is exactly what the gfx950
// v_mfma_f32_32x32x16_{bf16,f16} operands want: each lane feeds 8 consecutive k of one row.
//
// Workgroup: 4 or 8 waves on a WM x WN grid; each wave owns (BM/WM) x (BN/WN) made of 32x32 MFMA
// tiles (8 waves put two waves on each SIMD of the CU, so one issues MFMAs while the other waits on
// LDS or a barrier).  Two main loops share one epilogue:
//   gemm_kernel       register-staged tiles: 64-deep K slabs staged through registers into two LDS
//                     buffers, PF slabs of global loads in flight;
//   gemm_pipe_kernel  an S-stage pipeline of K slabs loaded straight from global memory into LDS,
//                     LDS fragment reads of the next k-step overlapped with the MFMAs of the current
//                     one: deep pipelines of small tiles for batch-1 problems, and for batched
//                     problems large tiles, the 256x256 ones with a ring of half-slab buffers.
// LDS rows hold one slab row with the 16-byte chunk index XOR-swizzled (swz, swz_k below), so the
// lanes reading one k-chunk of consecutive rows hit distinct banks.
//
// Epilogues (all fp32 until the single final rounding, bias added before it as in
// laya_cuda/kernels.cu:50-55):
//   F32  - fp32 partial of split z to out + z*split_stride (split-K reduction happens in the
//          residual+LayerNorm kernel that consumes it);
//   HALF - + bias, rounded to 16-bit;
//   GELU - + bias, exact-erf GELU, rounded to 16-bit (FFN up);
//   RELU - + bias, ReLU, rounded to 16-bit (FFN up of the head layers);
//   GEGLU - gelu(gate) * value of the gate/value rows interleaved in 32-row groups, rounded to
//          16-bit, N/2 wide (ModernBERT FFN up);
//   QKV  - + bias, rounded, written head-major: Q,K [h][M][64] and V transposed [h][64][M]
//          (replaces the reference's separate `layout` pass, kernels.cu:68-82);
//   QKV_ROPE - QKV with rotate-half RoPE applied to Q and K in fp32 before the rounding.
#include "kernels.hpp"

#include <atomic>
#include <type_traits>

namespace laya {

namespace {

constexpr int BK = 64;

// LDS tiles: rows of BK 16-bit elements (128 B) as eight 16-byte chunks, the chunk index
// XOR-swizzled by (row / 2) % 8.  A 16-byte LDS read is served 16 lanes per pass from 64 banks
// (256 B); the 16 lanes of a pass fetch the same k-chunk of 16 consecutive rows, i.e. eight
// 256-byte row pairs, and (row / 2) % 8 puts those eight pairs on eight different chunk
// positions (measured on gfx950: swizzling by row % 8 instead leaves the two rows 8 apart on the
// same banks, and rocprof's SQ_LDS_BANK_CONFLICT counts stalls for half of all LDS cycles).
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// Workgroup tile coordinates.  Workgroups are dealt to the 8 XCDs round-robin by linear dispatch
// id, so consecutive ids run on different L2s.  When the workgroup count allows, the logical index
// is laid out instead so that each XCD gets one contiguous share, decoded split-major: with split-K
// an XCD works on whole K-slices (or an equal part of one) and fetches only those slices of both
// operands.  Inside a slice, tiles are walked so the operand that is larger in HBM is fetched into
// one L2 once: with many rows (A larger), groups of 4 tile rows with the column index outer; with
// fewer rows than columns (B, the weights, larger), whole tile columns one after another.
// Coordinates of logical tile `id` (0 .. nx ny nz - 1): the workgroup with linear dispatch id `id`
// in the order above.
__device__ __forceinline__ void tile_of(int id, int nx, int ny, int nz, bool rows_major, int* x, int* y, int* z) {
  const int per_z = nx * ny, total = per_z * nz;
  if (total % 8) {
    *x = id % nx;
    *y = (id / nx) % ny;
    *z = id / per_z;
    return;
  }
  const int l = (id % 8) * (total / 8) + id / 8;
  *z = l / per_z;
  const int t = l - *z * per_z;
  if (rows_major) {
    constexpr int G = 4;
    const int group = t / (G * nx), first = group * G, size = min(G, ny - first), in = t - group * G * nx;
    *y = first + in % size;
    *x = in / size;
  } else {
    *x = t / ny;
    *y = t - *x * ny;
  }
}
__device__ __forceinline__ void tile_coords(int nx, int ny, int nz, bool rows_major, int* x, int* y, int* z) {
  tile_of(blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z), nx, ny, nz, rows_major, x, y, z);
}

// Bytes of LDS the epilogue stages through: one 32 x 36 fp32 (or 32 x 40 16-bit) region per wave.
constexpr int kEpilogueStageBytes = 32 * 36 * 4;

// QKV with RoPE: the position of each of this lane's output rows (one per 32-row tile), loaded at
// kernel start.  Read in the epilogue, the position and then the cos/sin row it selects were two
// dependent memory round trips at the end of every launch; loaded here, the position is in a
// register long before the epilogue and only the table read remains there.  The load is older
// than every operand load of the main loop, so its waits cover it.
template <int TM, Epi E>
__device__ __forceinline__ void load_early_pos(const GemmArgs& a, int row, int (&pos)[TM]) {
#pragma unroll
  for (int i = 0; i < TM; ++i) pos[i] = E == Epi::QKV_ROPE ? a.positions[min(row + i * 32, a.M - 1)] : 0;
}

// Epilogue shared by both GEMM kernels: acc holds this wave's (BM/WM) x (BN/WN) block of C^T as
// 32x32 MFMA tiles; smem_raw must have kEpilogueStageBytes per wave free (the caller's main loop is
// done with LDS: its last barrier has passed).
// acc[i][j][4 r4 + e] holds element e of the lane's column quad r4 of 32x32 output region (i, j):
// with 32x32x16 MFMAs (L16 false) row lane % 32, columns 8 r4 + 4 (lane / 32) .. +3; with 16x16x32
// MFMAs (L16 true; quad r4 is the 16x16 block (r4 / 2, r4 % 2) of the region) row 16 (r4 / 2) +
// lane % 16, columns 16 (r4 % 2) + 4 (lane % 64 / 16) .. +3.
template <bool L16>
__device__ __forceinline__ int quad_row(int lane, int r4) { return L16 ? ((r4 >> 1) << 4) + (lane & 15) : lane & 31; }
template <bool L16>
__device__ __forceinline__ int quad_col(int lane, int r4) {
  return L16 ? ((r4 & 1) << 4) + ((lane >> 4) << 2) : 8 * r4 + 4 * (lane >> 5);
}

// Column quad r4 of a 32x32 accumulator region (one 16-register tile).
__device__ __forceinline__ f32x4 acc_quad(const f32x16& v, int r4) {
  return f32x4{v[4 * r4], v[4 * r4 + 1], v[4 * r4 + 2], v[4 * r4 + 3]};
}

template <typename T, int BM, int BN, int WM, int WN, Epi E, bool kEarlyBias, bool L16 = false, typename Acc>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, Acc (&acc)[BM / WM / 32][BN / WN / 32],
                                              const float4 (&early_bias)[kEarlyBias ? BN / WN / 32 : 1][4],
                                              const int (&early_pos)[BM / WM / 32], int m0, int n0, int z,
                                              unsigned char* smem_raw, int lane, int wave) {
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  static_assert(!L16 || (E != Epi::GEGLU && E != Epi::QKV_ROPE && !kEarlyBias),
                "the 16x16 accumulator order serves the row-major and head-major epilogues without RoPE");
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
  const int lrow = lane & 31, kg = lane >> 5;
  const bool with_bias = (E != Epi::F32 || a.splits == 1) && a.bias;
  // Epilogue.  Element r of lane l in a 32x32 tile of C^T is output column 8*(r/4) + 4*(l/32) +
  // r%4 of output row l%32: a lane holds columns c..c+3 of one row for each r/4.  The bias joins in
  // fp32 before the single rounding.
  auto take = [&](int i, int j, int r4, float (&v)[4]) {
    const f32x4 q = acc_quad(acc[i][j], r4);
    v[0] = q[0];
    v[1] = q[1];
    v[2] = q[2];
    v[3] = q[3];
    if (with_bias) {
      const float4 b = kEarlyBias ? early_bias[kEarlyBias ? j : 0][r4]
                                  : *reinterpret_cast<const float4*>(a.bias + n0 + wn0 + j * 32 + quad_col<L16>(lane, r4));
      v[0] = v[0] + b.x; v[1] = v[1] + b.y; v[2] = v[2] + b.z; v[3] = v[3] + b.w;
    }
  };
  typedef typename Vec4<T>::type T4;
  if constexpr (E == Epi::GEGLU) {
    // Weight rows interleaved in 32-row groups (16 gate rows, then their 16 value rows), so a lane
    // holds gate column c (r4 < 2) and its value column c + 16 (r4 + 2): out[f] = gelu(gate) *
    // value, 16 features per 32 columns (the reference's activate mode 2).
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm0 + i * 32 + lrow;
      if (row >= a.M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int fbase = ((n0 + wn0 + j * 32) >> 1) + 4 * kg;
#pragma unroll
        for (int r4 = 0; r4 < 2; ++r4) {
          float gate[4], value[4];
          take(i, j, r4, gate);
          take(i, j, r4 + 2, value);
          T4 h;
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = to_half<T>(gelu16(gate[e]) * value[e]);
          *reinterpret_cast<T4*>(static_cast<T*>(a.out) + static_cast<long long>(row) * a.ldo + fbase + 8 * r4) = h;
        }
      }
    }
    return;
  }

  // Every other epilogue leaves through LDS, one 32x32 tile at a time in this wave's own region
  // (the main loop's buffers are free: its last barrier has passed): the lanes write their column
  // quads, then read back 16-byte chunks of whole row segments, so each store instruction covers
  // 16 rows x 64 B (16-bit) or 8 rows x 128 B (fp32) instead of 32 rows x 8-16 B.  V^T goes through
  // a transposed stage, so its stores are runs of 8 consecutive tokens.  A wave's LDS accesses
  // execute in issue order, so the region needs no barrier between writes and reads.
  constexpr int SP = E == Epi::F32 ? 36 : 40;  // stage pitch in elements: 144 B / 80 B, 16-byte aligned
  typedef typename std::conditional<E == Epi::F32, float, T>::type S;
  S* stg = reinterpret_cast<S*>(smem_raw) + wave * 32 * SP;
  const int rbase = m0 + wm0;  // first output row of this wave
  // Row-major 32x32 tile: lane values h[r4] = the column quad r4 (quad_row, quad_col); chunk
  // (r, c) (tile row r, first column c) is stored at dst(row, c) when row = rbase + 32 i + r < M.
  auto emit_rows = [&](int i, const auto (&h)[4], auto dst) {
    typedef typename std::remove_cv<typename std::remove_reference<decltype(h[0])>::type>::type Q;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      *reinterpret_cast<Q*>(stg + quad_row<L16>(lane, r4) * SP + quad_col<L16>(lane, r4)) = h[r4];
    constexpr int EPC = 16 / sizeof(S), CPR = 32 / EPC;  // elements per chunk, chunks per row
#pragma unroll
    for (int t = 0; t < 32 * CPR / 64; ++t) {
      const int c = lane + 64 * t, r = c / CPR, col = (c % CPR) * EPC;
      const i32x4 v = *reinterpret_cast<const i32x4*>(stg + r * SP + col);
      const int row = rbase + i * 32 + r;
      if (row < a.M) *reinterpret_cast<i32x4*>(dst(row, col)) = v;
    }
  };

  if constexpr (E == Epi::F32) {
    float* out = static_cast<float*>(a.out) + z * a.split_stride;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float4 h[4];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          float v[4];
          take(i, j, r4, v);
          h[r4] = make_float4(v[0], v[1], v[2], v[3]);
        }
        const int col0 = n0 + wn0 + j * 32;
        emit_rows(i, h, [&](int row, int col) { return out + static_cast<long long>(row) * a.ldo + col0 + col; });
      }
  } else if constexpr (E == Epi::QKV || E == Epi::QKV_ROPE) {
    T* const vt = static_cast<T*>(a.vt);
    // RoPE on Q and K (rotate-half, the reference's `layout`, kernels.cu:73-77) on the fp32
    // accumulator before the single rounding: tiles j and j+1 hold dims d and d+32 of one head.  The
    // cos/sin values of this lane's rows (dims 8 r4 + 4 kg .. +3 of each row's position) are all
    // read before the first tile is emitted: one memory round trip instead of one per row tile.
    constexpr bool rope = E == Epi::QKV_ROPE;
    float4 rcos[rope ? TM : 1][4], rsin[rope ? TM : 1][4];
    if constexpr (rope) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const size_t at = static_cast<size_t>(early_pos[i]) * 32 + 8 * r4 + 4 * kg;
          rcos[i][r4] = *reinterpret_cast<const float4*>(a.rope_cos + at);
          rsin[i][r4] = *reinterpret_cast<const float4*>(a.rope_sin + at);
        }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col0 = n0 + wn0 + j * 32;
        const int part = col0 / a.width, hn = col0 - part * a.width, head = hn >> 6, dim0 = hn & 63;
        if (part < 2) {
          T* const qk = static_cast<T*>(part == 0 ? a.q : a.k) + static_cast<size_t>(head) * a.M * 64;
          auto qdst = [&](int d0) {
            return [=](int row, int col) { return qk + static_cast<size_t>(row) * 64 + d0 + col; };
          };
          if constexpr (rope) {
            if (j & 1) continue;  // emitted with its pair
            if constexpr (TN >= 2) {
              T4 lo[4], hi[4];
#pragma unroll
              for (int r4 = 0; r4 < 4; ++r4) {
                float v0[4], v1[4];
                take(i, j, r4, v0);
                take(i, j + 1, r4, v1);
                const float c4[4] = {rcos[i][r4].x, rcos[i][r4].y, rcos[i][r4].z, rcos[i][r4].w};
                const float s4[4] = {rsin[i][r4].x, rsin[i][r4].y, rsin[i][r4].z, rsin[i][r4].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  lo[r4][e] = to_half<T>(v0[e] * c4[e] - v1[e] * s4[e]);
                  hi[r4][e] = to_half<T>(v1[e] * c4[e] + v0[e] * s4[e]);
                }
              }
              emit_rows(i, lo, qdst(0));
              emit_rows(i, hi, qdst(32));
            }
            continue;
          }
          T4 h[4];
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            float v[4];
            take(i, j, r4, v);
#pragma unroll
            for (int e = 0; e < 4; ++e) h[r4][e] = to_half<T>(v[e]);
          }
          emit_rows(i, h, qdst(dim0));
        } else {
          // V^T [head][64][M]: stage transposed (tile column = head dim as the LDS row, 32 tokens
          // per row), then store runs of 8 tokens; M is a multiple of 8, so a run is all in or out.
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            float v[4];
            take(i, j, r4, v);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              stg[(quad_col<L16>(lane, r4) + e) * SP + quad_row<L16>(lane, r4)] = to_half<T>(v[e]);
          }
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int c = lane + 64 * t, d = c >> 2, tok = (c & 3) * 8;
            const i32x4 v = *reinterpret_cast<const i32x4*>(stg + d * SP + tok);
            const int row = rbase + i * 32 + tok;
            if (row < a.M)
              *reinterpret_cast<i32x4*>(vt + (static_cast<size_t>(head) * 64 + dim0 + d) * a.M + row) = v;
          }
        }
      }
    }
  } else {
    T* out = static_cast<T*>(a.out);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        T4 h[4];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          float v[4];
          take(i, j, r4, v);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            h[r4][e] = to_half<T>(E == Epi::GELU ? gelu16(v[e]) : E == Epi::RELU ? fmaxf(v[e], 0.f) : v[e]);
        }
        const int col0 = n0 + wn0 + j * 32;
        emit_rows(i, h, [&](int row, int col) { return out + static_cast<long long>(row) * a.ldo + col0 + col; });
      }
  }
}

template <typename T, int BM, int BN, int WM, int WN, int PF, Epi E>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmArgs a) {
  constexpr int NT = 64 * WM * WN;
  static_assert(WM * WN == 4 || WM * WN == 8, "four or eight waves per workgroup");
  static_assert(PF >= 2, "register-staged slabs in flight (large tiles use gemm_pipe_kernel)");
  static_assert(WM * WN * kEpilogueStageBytes <= 2 * (BM + BN) * BK * 2, "the epilogue's staging fits the LDS");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "32x32 MFMA tiles");
  constexpr int ACH = BM * 8 / NT;  // 16-byte chunks per thread per slab
  constexpr int BCH = BN * 8 / NT;
  static_assert(ACH >= 1 && BCH >= 1 && ACH * NT == BM * 8 && BCH * NT == BN * 8, "whole chunks per thread");
  typedef typename Vec8<T>::type T8;

  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* sA = reinterpret_cast<T*>(smem_raw);
  T* sB = sA + 2 * BM * BK;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
  int tx, ty, z;
  tile_coords(gridDim.x, gridDim.y, gridDim.z, a.rows_major, &tx, &ty, &z);
  const int n0 = tx * BN, m0 = ty * BM;

  const T* A = static_cast<const T*>(a.a);
  const T* B = static_cast<const T*>(a.b);
  const int nk = a.K / BK;
  const int per = (nk + a.splits - 1) / a.splits;
  const int kb = z * per, ke = min(nk, kb + per);

  auto gload = [&](int kt, i32x4 (&xa)[ACH], i32x4 (&xb)[BCH]) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + NT * i, row = c >> 3, ch = c & 7;
      const int g = min(m0 + row, a.M - 1);
      xa[i] = *reinterpret_cast<const i32x4*>(A + static_cast<size_t>(g) * a.lda + k0 + ch * 8);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + NT * i, row = c >> 3, ch = c & 7;
      xb[i] = *reinterpret_cast<const i32x4*>(B + static_cast<size_t>(n0 + row) * a.ldb + k0 + ch * 8);
    }
  };
  auto lstore = [&](int buf, const i32x4 (&xa)[ACH], const i32x4 (&xb)[BCH]) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + NT * i, row = c >> 3, ch = c & 7;
      *reinterpret_cast<i32x4*>(sA + buf * BM * BK + row * BK + ((ch ^ swz(row)) << 3)) = xa[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + NT * i, row = c >> 3, ch = c & 7;
      *reinterpret_cast<i32x4*>(sB + buf * BN * BK + row * BK + ((ch ^ swz(row)) << 3)) = xb[i];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, kg = lane >> 5;
  // Small wave tiles fetch their bias at kernel start (16 floats per 32 columns per lane), so its
  // latency hides under the main loop instead of opening the epilogue.
  constexpr bool kEarlyBias = TN == 1;
  const bool with_bias = (E != Epi::F32 || a.splits == 1) && a.bias;
  float4 early_bias[1][4];
  if constexpr (kEarlyBias) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      early_bias[0][r4] = with_bias ? *reinterpret_cast<const float4*>(a.bias + n0 + wn0 + 8 * r4 + 4 * kg)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  int early_pos[TM];
  load_early_pos<TM, E>(a, m0 + wm0 + lrow, early_pos);
  // One 64-deep slab from LDS buffer `buf`: four 16-deep MFMA steps.  With at most 8 MFMA tiles per
  // wave the fragments are double-buffered in registers, so the LDS reads of step kk+1 are in
  // flight while the MFMAs of step kk run; larger wave tiles have no registers to spare for that.
  constexpr bool kFrag2 = TM * TN <= 8;
  auto compute = [&](int buf) {
    const T* cA = sA + buf * BM * BK;
    const T* cB = sB + buf * BN * BK;
    T8 af[kFrag2 ? 2 : 1][TM], bfr[kFrag2 ? 2 : 1][TN];
    auto fetch = [&](int kk, int s) {
      const int ch = kk * 2 + kg;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm0 + i * 32 + lrow;
        af[s][i] = *reinterpret_cast<const T8*>(cA + r * BK + ((ch ^ swz(r)) << 3));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn0 + j * 32 + lrow;
        bfr[s][j] = *reinterpret_cast<const T8*>(cB + r * BK + ((ch ^ swz(r)) << 3));
      }
    };
    if constexpr (kFrag2) fetch(0, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int s = kFrag2 ? (kk & 1) : 0;
      if constexpr (kFrag2) {
        if (kk + 1 < BK / 16) fetch(kk + 1, (kk + 1) & 1);
      } else {
        fetch(kk, 0);
      }
      // Weights as the MFMA A operand: the accumulator holds C^T, so each lane ends with four
      // consecutive output columns of one row.
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(bfr[s][j], af[s][i], acc[i][j]);
    }
  };

  const int n = ke - kb;
  {
    // Small tiles (batch-1 problems): slab s >= 1 travels in register set (s-1) % PF, issued PF
    // slabs ahead of its use, so PF slabs of global loads are in flight while the MFMAs consume the
    // slab in LDS.  Two LDS buffers; one barrier per slab.  Every step issues its loads
    // unconditionally (slab indices past the end are clamped to the last slab and never used), so
    // the number of loads in flight is the same on every path and the compiler's wait counts keep
    // the PF-1 younger sets in flight.
    if (n > 0) {
      i32x4 ra[PF][ACH], rb[PF][BCH];
      auto step = [&](int it, int u) {
        compute(it & 1);
        lstore((it + 1) & 1, ra[u], rb[u]);  // at it = n-1 this fills the idle buffer; never read
        gload(kb + min(it + 1 + PF, n - 1), ra[u], rb[u]);
        __syncthreads();
      };
      gload(kb, ra[0], rb[0]);
      lstore(0, ra[0], rb[0]);
#pragma unroll
      for (int p = 0; p < PF; ++p) gload(kb + min(1 + p, n - 1), ra[p], rb[p]);
      __syncthreads();
      int it = 0;
      for (; it + PF <= n; it += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) step(it + u, u);
      }
#pragma unroll
      for (int u = 0; u < PF; ++u)
        if (it + u < n) step(it + u, u);
    }
    __syncthreads();  // the epilogue reuses LDS
  }

  gemm_epilogue<T, BM, BN, WM, WN, E, kEarlyBias>(a, acc, early_bias, early_pos, m0, n0, z, smem_raw, lane, wave);
}

// LDS layout of the pipelined kernel: rows of BKS 16-bit elements, CPR = BKS / 8 chunks of 16 B per
// row, the chunk index XOR-swizzled by (row / (16 / CPR)) % CPR.  The 16 lanes of one LDS read
// pass fetch the same k-chunk of 16 consecutive rows; 16 / CPR rows fill one 256-byte line of the
// 64 banks, and the swizzle gives the rows that share a position in that line distinct chunks, so
// the pass touches 16 distinct 16-byte bank groups (BKS = 64: the swz above).
template <int BKS>
__device__ __forceinline__ int swz_k(int row) {
  constexpr int CPR = BKS / 8;
  return (row / (16 / CPR)) % CPR;
}

// Large tiles (batched problems): a multi-stage pipeline of K slabs moved from global memory
// straight into LDS (buffer_load_dwordx4 ... lds: no register staging, no LDS store instructions).
// A load instruction fills 1 KB of LDS = 64 / CPR rows, lane l at row l / CPR of its group and
// physical chunk l % CPR, fetching the logical chunk (l % CPR) ^ swz_k(row).
//
// S LDS stages hold slabs it .. it+S-2 while slab it is consumed; per slab (KS = BKS / 16 k-steps):
//   k-steps 0..KS-2: LDS fragments of step kk+1 are read while the MFMAs of step kk run (two
//                    register sets); the direct loads of slab it+S-1 (into the stage slab it-1
//                    used) are spread over these steps;
//   then each wave waits until its own loads of slab it+1 have landed (those of the S-2 younger
//   slabs stay in flight) and its own LDS reads are done, and one barrier makes slab it+1 visible
//   and frees stage it for the loads issued in the next slab;
//   k-step KS-1: its fragments are already in registers, so its MFMAs start right after the
//                barrier while step 0 of slab it+1 is read.
// 256x256 tiles (kFront) instead issue all loads of slab it+S in k-step KS-1, into the stage the
// barrier has just released (slab it's): S slabs are then in flight between barriers, and each
// load has S-1 whole slabs of MFMAs to land (4-5% faster on 64K-row projections).
// Loads are issued unconditionally (slab indices past the end are clamped to the last slab and
// land in a stage that is never read again), so the loop body is one straight-line block that the
// scheduling-group hints interleave: one MFMA, then one LDS read or one global load, so neither
// queue starves the matrix pipe.  Two waves per SIMD (register budget 256), except for 128x128
// wave tiles whose accumulators alone take 256 registers: 8-wave workgroups own a CU, 4-wave ones
// with smaller wave tiles share it with a second workgroup (whose main loop then covers this one's
// epilogue).
template <typename T, int BM, int BN, int WM, int WN, int BKS, int S, Epi E, bool RING, bool M16 = false>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(BM * BN / (WM * WN) >= 128 * 128 ? 1 : 2)))
void gemm_pipe_kernel(GemmArgs a) {
  constexpr int NW = WM * WN;
  static_assert(NW == 4 || NW == 8, "four or eight waves per workgroup");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "32x32 MFMA tiles");
  constexpr int CPR = BKS / 8, RPI = 64 / CPR, KS = BKS / 16;
  static_assert(BKS == 32 || BKS == 64, "32- or 64-deep slabs");
  constexpr int AG = BM / RPI / NW, BG = BN / RPI / NW, NLD = AG + BG;  // load instructions per wave per slab
  static_assert(AG * RPI * NW == BM && BG * RPI * NW == BN, "whole load groups per wave");
  static_assert(S >= 2, "at least two stages");
  constexpr int SLAB = (BM + BN) * BKS;  // 16-bit elements per stage: A rows, then B rows
  static_assert(NW * kEpilogueStageBytes <= S * SLAB * 2, "the epilogue's staging fits the LDS");
  // Load schedule: 256x256 tiles issue all loads of slab it+S right after the barrier that ends the
  // reads of slab it's stage (kFront: a whole slab before the barrier that first waits on them);
  // smaller tiles spread the loads of slab it+S-1 over the k-steps before the barrier.
  constexpr bool kFront = !RING && BM * BN >= 256 * 256;
  // RING: the LDS holds five half-slab buffers (one operand's rows of one slab each), see below.
  static_assert(!RING || (BM == BN && S == 5), "ring: five equal half-slab buffers");
  constexpr int HALFE = BM * BKS;  // 16-bit elements of a ring buffer
  // Loads of younger slabs (ring: of the youngest A half) that stay in flight at a slab's end.
  constexpr int kKeep = RING ? AG : NLD * (S - 2);
  constexpr int kKeepFirst = RING ? 2 * AG + BG : kFront ? NLD * (S - 1) : kKeep;  // after the prologue
  static_assert(kKeepFirst < 64, "vmcnt range");
  constexpr int kWaitSlab = waitcnt_vm(kKeep);
  constexpr int kWaitFirst = waitcnt_vm(kKeepFirst);
  constexpr int kWaitAll = waitcnt_vm(0);
  typedef typename Vec8<T>::type T8;

  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* const lds = reinterpret_cast<T*>(smem_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
  int tx, ty, z;
  tile_coords(gridDim.x, gridDim.y, gridDim.z, a.rows_major, &tx, &ty, &z);
  const int n0 = tx * BN, m0 = ty * BM;

  const int nk = a.K / BKS;
  const int per = (nk + a.splits - 1) / a.splits;
  const int kb = z * per, ke = min(nk, kb + per);
  const int n = ke - kb;

  // Operands are read through buffer resources (buffer_load_dwordx4 ... lds): a per-lane 32-bit byte
  // offset of each of this wave's load instructions (slab 0), the slab's K offset in the scalar
  // offset; 9% more L2-to-LDS throughput per CU than global_load_lds_dwordx4 in a streaming probe,
  // 3-4% faster 64K-row projections.  dst: the load's LDS offset.
  const i32x4 rsA = buffer_resource(a.a, static_cast<unsigned>(static_cast<size_t>(a.M) * a.lda * 2));
  const i32x4 rsB = buffer_resource(a.b, static_cast<unsigned>(static_cast<size_t>(a.N) * a.ldb * 2));
  unsigned src[NLD];
  int dst[NLD];
  {
    const int lr = lane / CPR, pch = lane % CPR;
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      const bool isA = q < AG;
      const int grp = wave + NW * (isA ? q : q - AG);
      const int row = grp * RPI + lr;
      const int ch = pch ^ swz_k<BKS>(row);
      if (isA) {
        const int g = min(m0 + row, a.M - 1);  // rows past M read row M-1, never stored
        src[q] = static_cast<unsigned>((static_cast<size_t>(g) * a.lda + ch * 8) * 2);
        dst[q] = grp * RPI * BKS;
      } else {
        src[q] = static_cast<unsigned>((static_cast<size_t>(n0 + row) * a.ldb + ch * 8) * 2);
        dst[q] = BM * BKS + grp * RPI * BKS;
      }
    }
  }
  // Small tiles (batch-1 problems) fetch their bias (16 floats per 32 columns per lane) before the
  // main loop: loaded in the epilogue it cost one more memory round trip at the end of every launch.
  // The load is older than every operand load, and loads complete in order, so the main loop's
  // vmcnt waits cover it.
  constexpr bool kEarlyBias = BM * BN <= 128 * 128 && TN <= 2;
  float4 early_bias[kEarlyBias ? TN : 1][4];
  if constexpr (kEarlyBias) {
    const bool with_bias = (E != Epi::F32 || a.splits == 1) && a.bias;
    const int kg = lane >> 5;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        early_bias[j][r4] = with_bias ? *reinterpret_cast<const float4*>(a.bias + n0 + wn0 + j * 32 + 8 * r4 + 4 * kg)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) early_bias[0][r4] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  int early_pos[TM];
  load_early_pos<TM, E>(a, m0 + wm0 + (lane & 31), early_pos);
  const unsigned lds_base = lds_address(smem_raw);
  auto issue_at = [&](int q, int kt, int base) {  // base: element offset of the load's LDS destination
    lds_load16_buffer(q < AG ? rsA : rsB, src[q], static_cast<unsigned>(kt) * BKS * 2,
                      lds_base + static_cast<unsigned>(base + dst[q]) * 2);
  };
  auto issue = [&](int q, int kt, int st) { issue_at(q, kt, st * SLAB); };
  // Ring buffers take one operand's rows: B loads drop the A rows' offset that dst[] carries.
  auto issue_ring = [&](int q, int kt, int buf) { issue_at(q, kt, buf * HALFE - (q < AG ? 0 : BM * BKS)); };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, kg = lane >> 5;
  T8 af[2][TM], bfr[2][TN];
  auto fetch_at = [&](const T* cA, const T* cB, int kk, int s) {
    const int ch = kk * 2 + kg;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm0 + i * 32 + lrow;
      af[s][i] = *reinterpret_cast<const T8*>(cA + r * BKS + ((ch ^ swz_k<BKS>(r)) << 3));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn0 + j * 32 + lrow;
      bfr[s][j] = *reinterpret_cast<const T8*>(cB + r * BKS + ((ch ^ swz_k<BKS>(r)) << 3));
    }
  };
  auto fetch = [&](int st, int kk, int s) { fetch_at(lds + st * SLAB, lds + st * SLAB + BM * BKS, kk, s); };
  // Weights as the MFMA A operand: the accumulator holds C^T, so each lane ends with four
  // consecutive output columns of one row.
  auto mma = [&](int s) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(bfr[s][j], af[s][i], acc[i][j]);
  };
  constexpr int NMF = TM * TN, NDS = TM + TN;
  // Interleave hint for one k-step: NMF MFMAs, NDS LDS reads and `nvm` global loads.  The LDS reads
  // go first, two per MFMA, so the fragments of the next step have most of this step's MFMAs to
  // land; the global loads fill the slots after the later MFMAs.
  // Small wave tiles have fewer MFMAs than reads per k-step: the reads then go several per slot.
  constexpr int DPM = NDS > 2 * NMF ? (NDS + NMF - 1) / NMF : 2;  // LDS reads issued per MFMA slot
  auto interleave = [&](auto nvm_c) {
    constexpr int nvm = decltype(nvm_c)::value;
#pragma unroll
    for (int t = 0; t < NMF; ++t) {
#pragma unroll
      for (int d = 0; d < DPM; ++d)
        if (t * DPM + d < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                        // one MFMA
      const int v = t - (NMF - nvm);
      if (v >= 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
    }
  };
  // The NLD loads of a slab are spread over the KS-1 k-steps before the barrier.
  constexpr int KPRE = KS - 1;
  constexpr int LPS = (NLD + KPRE - 1) / KPRE;  // loads per pre-barrier k-step

  if constexpr (M16) {
    // The ring below with 16x16x32 MFMAs: each wave's (BM/WM) x (BN/WN) block is (2 TM) x (2 TN)
    // blocks of 16x16, a k-step is 32 deep (lane l feeds k 8 (l / 16) .. +7 of row l % 16), so a
    // 64-deep slab is two k-steps of 4 TN TM MFMAs and 2 (TM + TN) LDS reads: the same LDS bytes
    // as the 32x32x16 form, but the MFMA stream measured 5-7% faster on the 64K-row projections
    // (register-only streams: 2.06 against 1.80 PFLOP/s on random operands, two waves per SIMD).
    static_assert(RING && BKS == 64, "16x16x32 MFMAs: the ring with 64-deep slabs");
    constexpr int KS16 = BKS / 32, MB = TM * 2, NB = TN * 2;
    T8 a16[2][MB], b16[2][NB];
    f32x4 acc16[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc16[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int l16 = lane & 15, kq = lane >> 4;
    auto fetch16 = [&](const T* cA, const T* cB, int kk, int s) {
      const int ch = kk * 4 + kq;
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int r = wm0 + i * 16 + l16;
        a16[s][i] = *reinterpret_cast<const T8*>(cA + r * BKS + ((ch ^ swz_k<BKS>(r)) << 3));
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int r = wn0 + j * 16 + l16;
        b16[s][j] = *reinterpret_cast<const T8*>(cB + r * BKS + ((ch ^ swz_k<BKS>(r)) << 3));
      }
    };
    auto mma16 = [&](int s) {  // weights as the A operand: the accumulator holds C^T
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc16[i][j] = ::laya::mfma16(b16[s][j], a16[s][i], acc16[i][j]);
    };
    auto interleave16 = [&]() {  // two LDS reads per MFMA slot, first
#pragma unroll
      for (int t = 0; t < MB * NB; ++t) {
        if (2 * t < MB + NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (2 * t + 1 < MB + NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    };
    if (n > 0) {
#pragma unroll
      for (int h = 0; h < 5; ++h) {
        const int kt = kb + min(h / 2, n - 1);
#pragma unroll
        for (int q = (h & 1) ? AG : 0; q < ((h & 1) ? NLD : AG); ++q) issue_ring(q, kt, h);
      }
      publish_stage<kWaitFirst>();
      fetch16(lds, lds + HALFE, 0, 0);
      int abuf = 0;
      for (int it = 0; it < n; ++it) {
        const int bbuf = abuf == 4 ? 0 : abuf + 1;
        const int nabuf = abuf >= 3 ? abuf - 3 : abuf + 2, nbbuf = nabuf == 4 ? 0 : nabuf + 1;
#pragma unroll
        for (int kk = 0; kk < KS16 - 1; ++kk) {
          fetch16(lds + abuf * HALFE, lds + bbuf * HALFE, kk + 1, (kk + 1) & 1);
          mma16(kk & 1);
          interleave16();
          __builtin_amdgcn_sched_barrier(0);
        }
        publish_stage<kWaitSlab>();
        __builtin_amdgcn_sched_barrier(0);
        fetch16(lds + nabuf * HALFE, lds + nbbuf * HALFE, 0, 0);
        const int kt2 = kb + min(it + 2, n - 1), kt3 = kb + min(it + 3, n - 1);
#pragma unroll
        for (int q = AG; q < NLD; ++q) issue_ring(q, kt2, abuf);
#pragma unroll
        for (int q = 0; q < AG; ++q) issue_ring(q, kt3, bbuf);
        mma16((KS16 - 1) & 1);
        interleave16();
        __builtin_amdgcn_sched_barrier(0);
        abuf = nabuf;
      }
    }
    // Quad r4 of 32x32 region (i, j) is 16x16 block (2 i + r4 / 2, 2 j + r4 % 2) (quad_row/quad_col).
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = acc16[2 * i + (q >> 1)][2 * j + (q & 1)][e];
  }
  if (RING && !M16 && n > 0) {
    // Ring of five half-slab buffers (160 KB for 256x256 tiles): half h (slab h / 2, A rows for
    // even h, B rows for odd) lives in buffer h % 5.  While slab it is consumed from halves 2it and
    // 2it+1, halves 2it+2 .. 2it+4 are landed or in flight; the barrier after its last LDS reads
    // waits for slab it+1 only, so the A half of slab it+2 stays in flight across it and the
    // operand stream never drains; right after it, the two freed buffers take halves 2it+5 and
    // 2it+6 (B of slab it+2, A of slab it+3).
#pragma unroll
    for (int h = 0; h < 5; ++h) {
      const int kt = kb + min(h / 2, n - 1);
#pragma unroll
      for (int q = (h & 1) ? AG : 0; q < ((h & 1) ? NLD : AG); ++q) issue_ring(q, kt, h);
    }
    publish_stage<kWaitFirst>();
    fetch_at(lds, lds + HALFE, 0, 0);
    int abuf = 0;  // buffer of slab it's A half; its B half is in the next one
    for (int it = 0; it < n; ++it) {
      const int bbuf = abuf == 4 ? 0 : abuf + 1;
      const int nabuf = abuf >= 3 ? abuf - 3 : abuf + 2, nbbuf = nabuf == 4 ? 0 : nabuf + 1;
#pragma unroll
      for (int kk = 0; kk < KPRE; ++kk) {
        fetch_at(lds + abuf * HALFE, lds + bbuf * HALFE, kk + 1, (kk + 1) & 1);
        mma(kk & 1);
        interleave(std::integral_constant<int, 0>());
        __builtin_amdgcn_sched_barrier(0);
      }
      publish_stage<kWaitSlab>();
      __builtin_amdgcn_sched_barrier(0);
      fetch_at(lds + nabuf * HALFE, lds + nbbuf * HALFE, 0, 0);
      const int kt2 = kb + min(it + 2, n - 1), kt3 = kb + min(it + 3, n - 1);
#pragma unroll
      for (int q = AG; q < NLD; ++q) issue_ring(q, kt2, abuf);
#pragma unroll
      for (int q = 0; q < AG; ++q) issue_ring(q, kt3, bbuf);
      mma((KS - 1) & 1);
      interleave(std::integral_constant<int, 0>());
      __builtin_amdgcn_sched_barrier(0);
      abuf = nabuf;
    }
  }
  if (!RING && n > 0) {
#pragma unroll
    for (int p = 0; p < (kFront ? S : S - 1); ++p)
#pragma unroll
      for (int q = 0; q < NLD; ++q) issue(q, kb + min(p, n - 1), p);
    publish_stage<kWaitFirst>();
    fetch(0, 0, 0);
    int cur = 0, ldst = S - 1;  // stage of slab it, stage receiving slab it+S-1 (spread schedule)
    for (int it = 0; it < n; ++it) {
      const int lslab = kb + min(it + (kFront ? S : S - 1), n - 1);
      const int nxt = cur + 1 == S ? 0 : cur + 1;
#pragma unroll
      for (int kk = 0; kk < KPRE; ++kk) {
        if constexpr (!kFront) {
#pragma unroll
          for (int q = kk * LPS; q < (kk + 1) * LPS && q < NLD; ++q) issue(q, lslab, ldst);
        }
        fetch(cur, kk + 1, (kk + 1) & 1);
        mma(kk & 1);
        constexpr int nvm_max = kFront ? 0 : LPS < NMF ? LPS : NMF;  // loads beyond the MFMA slots go unhinted
        interleave(std::integral_constant<int, nvm_max>());
        __builtin_amdgcn_sched_barrier(0);
      }
      publish_stage<kWaitSlab>();
      __builtin_amdgcn_sched_barrier(0);
      fetch(nxt, 0, 0);
      if constexpr (kFront) {
        // Every wave is past its reads of stage cur (this k-step runs from registers).
#pragma unroll
        for (int q = 0; q < NLD; ++q) issue(q, lslab, cur);
      }
      mma((KS - 1) & 1);
      interleave(std::integral_constant<int, 0>());
      __builtin_amdgcn_sched_barrier(0);
      cur = nxt;
      ldst = ldst + 1 == S ? 0 : ldst + 1;
    }
  }
  // The clamped loads of the last slabs may still be landing: drain them before the epilogue
  // reuses LDS.
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  __syncthreads();
  gemm_epilogue<T, BM, BN, WM, WN, E, kEarlyBias, M16>(a, acc, early_bias, early_pos, m0, n0, z, smem_raw, lane,
                                                       wave);
}

// Persistent form of the eight-wave 256x256 ring (tile 26: tile 19 looping over tiles).  A launch
// of tile 19 runs in rounds of one 160 KB workgroup per CU, and every workgroup of a round fills its
// pipeline, and later writes its 128 KB of output, at the same moment, with no other workgroup's
// MFMAs to cover either.  Here a grid of at most one workgroup per CU walks the tiles id, id + G,
// id + 2G, ... (G workgroups; the same XCD-aware order as a launch of all tiles, since workgroup id
// and id + G run on the same XCD when G is a multiple of 8), and the ring's operand stream runs on
// across tile boundaries: the loads issued during a tile's last two slabs fetch the next tile's
// first slabs, so the next tile's MFMAs start as soon as the epilogue is done.  The epilogue stages
// its rows in the ring buffer of the last slab's A half - free once the barrier after that slab's
// LDS reads has passed, and no load is in flight into it - and the two loads the ring would issue
// into that slab's buffers are issued after the epilogue instead.  Each tile's bias is loaded at the
// tile's start, before any load of the next tile's slabs: vector memory operations complete in
// issue order, so a bias load issued in the epilogue would wait for the whole prefetch (measured:
// 5.5% of the up projection's time).  16-bit outputs without RoPE only (the fp32 epilogue's staging,
// 37 KB, needs more than one 32 KB buffer); every tile's K range must hold at least three slabs
// (the ring prefetches two slabs and an A half).
template <typename T, Epi E>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_ring_persist_kernel(GemmArgs a) {
  constexpr int BM = 256, BN = 256, WM = 2, WN = 4, NW = WM * WN, BKS = 64;
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  constexpr int CPR = BKS / 8, RPI = 64 / CPR, KS = BKS / 16;
  constexpr int AG = BM / RPI / NW, BG = BN / RPI / NW, NLD = AG + BG;
  constexpr int HALFE = BM * BKS;  // 16-bit elements of a ring buffer
  static_assert(E != Epi::F32, "16-bit epilogues: their staging fits one ring buffer");
  static_assert(NW * 32 * 40 * 2 <= HALFE * 2, "16-bit epilogue staging within one ring buffer");
  static_assert(E != Epi::QKV_ROPE, "no RoPE (its cos/sin registers do not fit beside the tile loop's)");
  constexpr int kWaitSlab = waitcnt_vm(AG);
  constexpr int kWaitFirst = waitcnt_vm(2 * AG + BG);
  constexpr int kWaitAll = waitcnt_vm(0);
  typedef typename Vec8<T>::type T8;

  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* const lds = reinterpret_cast<T*>(smem_raw);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
  const int lrow = lane & 31, kg = lane >> 5;

  const int nx = a.N / BN, ny = (a.M + BM - 1) / BM, nz = a.splits, total = nx * ny * nz;
  const int G = gridDim.x;
  const int n = a.K / BKS / a.splits;  // slabs per tile (the launcher checks K / 64 % splits == 0, n >= 3)
  int id = blockIdx.x;
  if (id >= total) return;

  // Operands through per-tile buffer resources based at the tile's first A row and first B row:
  // a lane's byte offset in a tile's rows is the same for every tile (one register per load
  // instruction), and A rows past M fall outside the A resource's range (M - m0 rows), which
  // suppresses those loads; they feed only output rows past M, which are never stored.
  const int lr = lane / CPR, pch = lane % CPR;
  auto src_of = [&](int q) {  // unsigned: 32-bit offsets (the launcher bounds each operand below 4 GiB)
    const int row = (wave + NW * (q < AG ? q : q - AG)) * RPI + lr;
    const unsigned ld = static_cast<unsigned>(q < AG ? a.lda : a.ldb);
    return (static_cast<unsigned>(row) * ld + (static_cast<unsigned>(pch ^ swz_k<BKS>(row)) << 3)) * 2u;
  };
  auto dst_of = [&](int q) { return (wave + NW * (q < AG ? q : q - AG)) * RPI * BKS; };
  auto res_a = [&](int m0) {
    return buffer_resource(static_cast<const T*>(a.a) + static_cast<size_t>(m0) * a.lda,
                           static_cast<unsigned>(static_cast<size_t>(a.M - m0) * a.lda * 2));
  };
  auto res_b = [&](int n0) {
    return buffer_resource(static_cast<const T*>(a.b) + static_cast<size_t>(n0) * a.ldb,
                           static_cast<unsigned>(static_cast<size_t>(a.N - n0) * a.ldb * 2));
  };
  auto decode = [&](int t, int& m0, int& n0, int& z) {
    int tx, ty;
    tile_of(t, nx, ny, nz, a.rows_major, &tx, &ty, &z);
    n0 = tx * BN;
    m0 = ty * BM;
  };
  const unsigned lds_base = lds_address(smem_raw);

  int m0, n0, z;
  decode(id, m0, n0, z);
  int kb = z * n;
  i32x4 rsA = res_a(m0), rsB = res_b(n0);
  int nid = id + G, nm0 = m0, nn0 = n0, nzz = z;
  bool has_next = nid < total;
  if (has_next) decode(nid, nm0, nn0, nzz);
  i32x4 nrsA = res_a(nm0), nrsB = res_b(nn0);
  int nkb = nzz * n;

  // One half (A rows: q < AG, or B rows) of stream slab `s` counted from this tile's first slab:
  // this tile's slab s, the next tile's slab s - n, or (last tile) this tile's last slab again,
  // landing in a buffer that is never read.
  auto issue_half = [&](bool isB, int s, int buf) {
    const bool next = s >= n && has_next;
    const int kt = next ? nkb + (s - n) : kb + min(s, n - 1);
    const i32x4 r = isB ? (next ? nrsB : rsB) : (next ? nrsA : rsA);
#pragma unroll
    for (int q = isB ? AG : 0; q < (isB ? NLD : AG); ++q)
      lds_load16_buffer(r, src_of(q), static_cast<unsigned>(kt) * BKS * 2,
                        lds_base + static_cast<unsigned>(buf * HALFE + dst_of(q)) * 2);
  };

  // The tile's bias for this lane's column quads (as the small tiles' early bias), and the RoPE-free
  // positions placeholder the epilogue takes.
  float4 bias[TN][4];
  auto load_bias = [&]() {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        bias[j][r4] = a.bias ? *reinterpret_cast<const float4*>(a.bias + n0 + wn0 + j * 32 + quad_col<false>(lane, r4))
                             : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  int early_pos[TM] = {};
  load_bias();

  f32x16 acc[TM][TN];
  T8 af[2][TM], bfr[2][TN];
  auto fetch = [&](int abuf, int bbuf, int kk, int s) {
    const T* cA = lds + abuf * HALFE;
    const T* cB = lds + bbuf * HALFE;
    const int ch = kk * 2 + kg;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm0 + i * 32 + lrow;
      af[s][i] = *reinterpret_cast<const T8*>(cA + r * BKS + ((ch ^ swz_k<BKS>(r)) << 3));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn0 + j * 32 + lrow;
      bfr[s][j] = *reinterpret_cast<const T8*>(cB + r * BKS + ((ch ^ swz_k<BKS>(r)) << 3));
    }
  };
  auto mma = [&](int s) {  // weights as the MFMA A operand: the accumulator holds C^T
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(bfr[s][j], af[s][i], acc[i][j]);
  };
  auto hint = [&]() {  // LDS reads first, two per MFMA slot (as gemm_pipe_kernel's ring)
    constexpr int NMF = TM * TN, NDS = TM + TN;
#pragma unroll
    for (int t = 0; t < NMF; ++t) {
      if (2 * t < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (2 * t + 1 < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  };
  // The k-steps of a slab before its barrier: fragments of step kk+1 read during the MFMAs of kk.
  auto slab_front = [&](int abuf, int bbuf) {
#pragma unroll
    for (int kk = 0; kk < KS - 1; ++kk) {
      fetch(abuf, bbuf, kk + 1, (kk + 1) & 1);
      mma(kk & 1);
      hint();
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue: halves 0 .. 4 of the stream (slabs 0 and 1, A of slab 2) into buffers 0 .. 4.
#pragma unroll
  for (int h = 0; h < 5; ++h) issue_half(h & 1, h / 2, h);
  publish_stage<kWaitFirst>();
  fetch(0, 1, 0, 0);
  int abuf = 0;  // buffer of the current slab's A half; its B half is in the next one
  for (;;) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    for (int it = 0; it < n - 1; ++it) {
      const int bbuf = abuf == 4 ? 0 : abuf + 1;
      const int nabuf = abuf >= 3 ? abuf - 3 : abuf + 2, nbbuf = nabuf == 4 ? 0 : nabuf + 1;
      slab_front(abuf, bbuf);
      publish_stage<kWaitSlab>();
      __builtin_amdgcn_sched_barrier(0);
      fetch(nabuf, nbbuf, 0, 0);
      issue_half(true, it + 2, abuf);   // B half of slab it+2 into the freed A buffer
      issue_half(false, it + 3, bbuf);  // A half of slab it+3 into the freed B buffer
      mma((KS - 1) & 1);
      hint();
      __builtin_amdgcn_sched_barrier(0);
      abuf = nabuf;
    }
    // The tile's last slab.
    const int bbuf = abuf == 4 ? 0 : abuf + 1;
    const int nabuf = abuf >= 3 ? abuf - 3 : abuf + 2, nbbuf = nabuf == 4 ? 0 : nabuf + 1;
    slab_front(abuf, bbuf);
    publish_stage<kWaitSlab>();
    __builtin_amdgcn_sched_barrier(0);
    mma((KS - 1) & 1);
    if (!has_next) {
      // The clamped loads of the last slabs may still be landing: drain them before the epilogue
      // reuses LDS (and before the workgroup ends).
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __syncthreads();
      gemm_epilogue<T, BM, BN, WM, WN, E, true>(a, acc, bias, early_pos, m0, n0, z, smem_raw, lane, wave);
      return;
    }
    gemm_epilogue<T, BM, BN, WM, WN, E, true>(a, acc, bias, early_pos, m0, n0, z,
                                              smem_raw + static_cast<size_t>(abuf) * HALFE * 2, lane, wave);
    // Every wave's staging reads are done before the ring loads below overwrite the buffer (the
    // epilogue's global stores stay in flight).
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0_keep_vm());
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // Next tile: it becomes the current one, and the one after it the next.
    id = nid;
    m0 = nm0;
    n0 = nn0;
    z = nzz;
    kb = nkb;
    rsA = nrsA;
    rsB = nrsB;
    nid = id + G;
    has_next = nid < total;
    if (has_next) {
      decode(nid, nm0, nn0, nzz);
      nrsA = res_a(nm0);
      nrsB = res_b(nn0);
      nkb = nzz * n;
    }
    load_bias();
    // The two loads the last slab's iteration deferred: B of the tile's slab 1, A of its slab 2.
    issue_half(true, 1, abuf);
    issue_half(false, 2, bbuf);
    fetch(nabuf, nbbuf, 0, 0);
    abuf = nabuf;
  }
}

struct TileDef {
  int bm, bn, wm, wn;
  int pf;      // >= 2: register-staged kernel with pf slabs in flight; 0: pipelined direct-to-LDS kernel
  int bk, st;  // pipelined kernel: slab depth and LDS stages (ring: five half-slab buffers)
  bool ring;
  bool m16 = false;  // ring with 16x16x32 MFMAs (row-major and head-major epilogues without RoPE)
  bool persist = false;  // ring looping over tiles, one workgroup per CU (16-bit epilogues)
  int threads() const { return 64 * wm * wn; }
};
// Tile menu; the planner picks per problem.  Ids are part of the op-level ABI (tests sweep them).
// Register-staged tiles keep pf K slabs of global loads in flight (deep for the small tiles of
// batch-1 problems, whose few MFMAs per slab cannot cover HBM latency); pipelined tiles keep st-1.
constexpr TileDef kTiles[] = {
    {256, 256, 2, 2, 0, 64, 2},  // 0: 4 waves of 128x128, large M (batched)
    {256, 128, 2, 2, 0, 64, 2},  // 1: 4 waves of 128x64
    {128, 128, 2, 2, 2, 64, 0},  // 2: wave 64x64
    {128, 64, 2, 2, 3, 64, 0},   // 3: wave 64x32
    {64, 128, 2, 2, 3, 64, 0},   // 4: wave 32x64
    {64, 64, 2, 2, 4, 64, 0},    // 5: wave 32x32, small M (batch-1 latency)
    {32, 128, 1, 4, 4, 64, 0},   // 6: wave 32x32, very small M
    {256, 256, 2, 4, 0, 64, 2},  // 7: 8 waves of 128x64, large M
    {256, 128, 4, 2, 0, 64, 2},  // 8: 8 waves of 64x64
    {128, 256, 2, 4, 0, 64, 2},  // 9: 8 waves of 64x64
    {128, 64, 4, 1, 3, 64, 0},   // 10: wave 32x64, whole heads per wave for RoPE when N is not a multiple of 128
    {256, 256, 2, 4, 0, 32, 4},  // 11: 8 waves of 128x64, 32-deep slabs, three in flight
    {256, 128, 2, 2, 0, 32, 3},  // 12: 4 waves of 128x64, two workgroups per CU
    {128, 256, 2, 2, 0, 32, 3},  // 13: 4 waves of 64x128, two workgroups per CU
    // Pipelined small tiles for batch-1 problems: up to ten 64-deep slabs in flight, so a tile's
    // K loop costs about one memory round trip instead of K / (64 PF).
    {64, 64, 2, 2, 0, 64, 8},    // 14: wave 32x32
    {128, 64, 2, 2, 0, 64, 6},   // 15: wave 64x32
    {64, 128, 2, 2, 0, 64, 6},   // 16: wave 32x64
    {32, 128, 1, 4, 0, 64, 8},   // 17: wave 32x32, very small M
    {128, 128, 2, 2, 0, 64, 4},  // 18: wave 64x64
    // 256x256 tiles whose operand stream stays in flight across the slab barriers (ring of five
    // half-slab LDS buffers, 160 KB).
    {256, 256, 2, 4, 0, 64, 5, true},  // 19: 8 waves of 128x64
    {256, 256, 2, 2, 0, 64, 5, true},  // 20: 4 waves of 128x128
    // 192-column tiles for batched problems whose 256-column tiles leave CUs idle (a 15,360-row
    // batch: 240 tiles of 256x192 for N = 768 instead of 180 of 256x256): 12.5% fewer operand bytes
    // per tile, in a two-stage pipeline (the ring needs square tiles).
    {256, 192, 4, 2, 0, 64, 2},  // 21: 8 waves of 64x96
    // Tile 19 with 16x16x32 MFMAs (faster MFMA stream, same LDS traffic); not for RoPE or GeGLU.
    {256, 256, 2, 4, 0, 64, 5, true, true},  // 22
    // Eight-wave forms of the pipelined batch-1 tiles: a CU's direct loads from L2 run about twice
    // as fast from eight waves as from four (45-49 against 22-25 bytes per clock in a streaming
    // probe), and at batch 1 each CU's operand stream is what bounds a tile.
    {128, 64, 4, 2, 0, 64, 6},   // 23: 8 waves of 32x32
    {64, 128, 2, 4, 0, 64, 6},   // 24: 8 waves of 32x32
    {128, 128, 4, 2, 0, 64, 4},  // 25: 8 waves of 32x64
    // Persistent form of tile 19 (gemm_ring_persist_kernel): a workgroup per CU walks the tiles, its
    // operand stream running on from one tile into the next.
    {256, 256, 2, 4, 0, 64, 5, true, false, true},  // 26
};
constexpr int kTileCount = sizeof(kTiles) / sizeof(kTiles[0]);

constexpr size_t lds_bytes(const TileDef& d) {
  return d.pf     ? static_cast<size_t>(2) * (d.bm + d.bn) * BK * 2
         : d.ring ? static_cast<size_t>(5) * d.bm * d.bk * 2
                  : static_cast<size_t>(d.st) * (d.bm + d.bn) * d.bk * 2;
}

// Compute units of the current device (the persistent tiles' grid), queried once per device.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v <= 0 && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
    cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

template <typename T, Epi E>
hipError_t launch_t(const GemmArgs& a, int tile, hipStream_t stream) {
  const TileDef& d = kTiles[tile];
  const dim3 grid(a.N / d.bn, (a.M + d.bm - 1) / d.bm, a.splits), block(d.threads());
  const size_t lds = lds_bytes(d);
  switch (tile) {
#define LAYA_TILE(ID, BM_, BN_, WM_, WN_, PF_) \
  case ID: LAYA_LAUNCH((gemm_kernel<T, BM_, BN_, WM_, WN_, PF_, E>), grid, block, lds, stream, a); break;
#define LAYA_PIPE(ID, BM_, BN_, WM_, WN_, BK_, ST_) \
  case ID: LAYA_LAUNCH((gemm_pipe_kernel<T, BM_, BN_, WM_, WN_, BK_, ST_, E, false>), grid, block, lds, stream, a); break;
#define LAYA_RING(ID, BM_, BN_, WM_, WN_) \
  case ID: LAYA_LAUNCH((gemm_pipe_kernel<T, BM_, BN_, WM_, WN_, 64, 5, E, true>), grid, block, lds, stream, a); break;
    LAYA_PIPE(0, 256, 256, 2, 2, 64, 2)
    LAYA_PIPE(1, 256, 128, 2, 2, 64, 2)
    LAYA_TILE(2, 128, 128, 2, 2, 2)
    LAYA_TILE(3, 128, 64, 2, 2, 3)
    LAYA_TILE(4, 64, 128, 2, 2, 3)
    LAYA_TILE(5, 64, 64, 2, 2, 4)
    LAYA_TILE(6, 32, 128, 1, 4, 4)
    LAYA_PIPE(7, 256, 256, 2, 4, 64, 2)
    LAYA_PIPE(8, 256, 128, 4, 2, 64, 2)
    LAYA_PIPE(9, 128, 256, 2, 4, 64, 2)
    LAYA_TILE(10, 128, 64, 4, 1, 3)
    LAYA_PIPE(11, 256, 256, 2, 4, 32, 4)
    LAYA_PIPE(12, 256, 128, 2, 2, 32, 3)
    LAYA_PIPE(13, 128, 256, 2, 2, 32, 3)
    LAYA_PIPE(14, 64, 64, 2, 2, 64, 8)
    LAYA_PIPE(15, 128, 64, 2, 2, 64, 6)
    LAYA_PIPE(16, 64, 128, 2, 2, 64, 6)
    LAYA_PIPE(17, 32, 128, 1, 4, 64, 8)
    LAYA_PIPE(18, 128, 128, 2, 2, 64, 4)
    LAYA_RING(19, 256, 256, 2, 4)
    LAYA_RING(20, 256, 256, 2, 2)
    LAYA_PIPE(21, 256, 192, 4, 2, 64, 2)
    case 22:
      if constexpr (E == Epi::GEGLU || E == Epi::QKV_ROPE) return hipErrorInvalidValue;
      else LAYA_LAUNCH((gemm_pipe_kernel<T, 256, 256, 2, 4, 64, 5, E, true, true>), grid, block, lds, stream, a);
      break;
    LAYA_PIPE(23, 128, 64, 4, 2, 64, 6)
    LAYA_PIPE(24, 64, 128, 2, 4, 64, 6)
    LAYA_PIPE(25, 128, 128, 4, 2, 64, 4)
    case 26: {
      if constexpr (E == Epi::F32 || E == Epi::QKV_ROPE) {
        return hipErrorInvalidValue;
      } else {
        const int cus = device_cus();
        if (cus <= 0) return hipErrorInvalidDevice;
        const dim3 pgrid(min(static_cast<long long>(grid.x) * grid.y * grid.z, static_cast<long long>(cus)));
        LAYA_LAUNCH((gemm_ring_persist_kernel<T, E>), pgrid, block, lds, stream, a);
      }
      break;
    }
#undef LAYA_RING
#undef LAYA_TILE
#undef LAYA_PIPE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, Epi E>
hipError_t set_lds_attr() {
  hipError_t e = hipSuccess;
#define LAYA_ATTR(ID, ...)                                                                              \
  if (e == hipSuccess)                                                                                \
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&__VA_ARGS__),                                \
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes(kTiles[ID])));
  LAYA_ATTR(0, gemm_pipe_kernel<T, 256, 256, 2, 2, 64, 2, E, false>)
  LAYA_ATTR(1, gemm_pipe_kernel<T, 256, 128, 2, 2, 64, 2, E, false>)
  LAYA_ATTR(2, gemm_kernel<T, 128, 128, 2, 2, 2, E>)
  LAYA_ATTR(7, gemm_pipe_kernel<T, 256, 256, 2, 4, 64, 2, E, false>)
  LAYA_ATTR(8, gemm_pipe_kernel<T, 256, 128, 4, 2, 64, 2, E, false>)
  LAYA_ATTR(9, gemm_pipe_kernel<T, 128, 256, 2, 4, 64, 2, E, false>)
  LAYA_ATTR(11, gemm_pipe_kernel<T, 256, 256, 2, 4, 32, 4, E, false>)
  LAYA_ATTR(12, gemm_pipe_kernel<T, 256, 128, 2, 2, 32, 3, E, false>)
  LAYA_ATTR(13, gemm_pipe_kernel<T, 128, 256, 2, 2, 32, 3, E, false>)
  LAYA_ATTR(14, gemm_pipe_kernel<T, 64, 64, 2, 2, 64, 8, E, false>)
  LAYA_ATTR(15, gemm_pipe_kernel<T, 128, 64, 2, 2, 64, 6, E, false>)
  LAYA_ATTR(16, gemm_pipe_kernel<T, 64, 128, 2, 2, 64, 6, E, false>)
  LAYA_ATTR(17, gemm_pipe_kernel<T, 32, 128, 1, 4, 64, 8, E, false>)
  LAYA_ATTR(18, gemm_pipe_kernel<T, 128, 128, 2, 2, 64, 4, E, false>)
  LAYA_ATTR(19, gemm_pipe_kernel<T, 256, 256, 2, 4, 64, 5, E, true>)
  LAYA_ATTR(20, gemm_pipe_kernel<T, 256, 256, 2, 2, 64, 5, E, true>)
  LAYA_ATTR(21, gemm_pipe_kernel<T, 256, 192, 4, 2, 64, 2, E, false>)
  if constexpr (E != Epi::GEGLU && E != Epi::QKV_ROPE) {
    LAYA_ATTR(22, gemm_pipe_kernel<T, 256, 256, 2, 4, 64, 5, E, true, true>)
  }
  LAYA_ATTR(23, gemm_pipe_kernel<T, 128, 64, 4, 2, 64, 6, E, false>)
  LAYA_ATTR(24, gemm_pipe_kernel<T, 64, 128, 2, 4, 64, 6, E, false>)
  LAYA_ATTR(25, gemm_pipe_kernel<T, 128, 128, 4, 2, 64, 4, E, false>)
  if constexpr (E != Epi::F32 && E != Epi::QKV_ROPE) {
    LAYA_ATTR(26, gemm_ring_persist_kernel<T, E>)
  }
#undef LAYA_ATTR
  return e;
}

template <typename T>
hipError_t set_lds_all() {
  hipError_t e = set_lds_attr<T, Epi::F32>();
  if (e == hipSuccess) e = set_lds_attr<T, Epi::HALF>();
  if (e == hipSuccess) e = set_lds_attr<T, Epi::GELU>();
  if (e == hipSuccess) e = set_lds_attr<T, Epi::QKV>();
  if (e == hipSuccess) e = set_lds_attr<T, Epi::QKV_ROPE>();
  if (e == hipSuccess) e = set_lds_attr<T, Epi::RELU>();
  if (e == hipSuccess) e = set_lds_attr<T, Epi::GEGLU>();
  return e;
}

}  // namespace

int gemm_tile_count() { return kTileCount; }
GemmTile gemm_tile(int id) { return GemmTile{kTiles[id].bm, kTiles[id].bn}; }

hipError_t gemm_prepare() {
  hipError_t e = set_lds_all<bf16>();
  if (e == hipSuccess) e = set_lds_all<f16>();
  // The persistent tile's grid reads the CU count at launch: query it here, before any capture.
  if (e == hipSuccess && device_cus() <= 0) e = hipErrorInvalidDevice;
  return e;
}

// Measured plans: for the batch-1 GEMM problems of the encoder shapes in gemm_plans.inc (each timed
// on an MI355X through the op-level entry points with every tile and split count), the (tile,
// split-K) launch that timed fastest where it beat the heuristic below by more than 3%.  Keyed by
// CU count, so another part keeps the heuristic.
struct PlanEntry {
  int cus, M, N, K, epi, dtype, rope, tile, splits;
};
constexpr PlanEntry kPlans[] = {
#include "gemm_plans.inc"
    {0, 0, 0, 0, 0, 0, 0, 0, 0},  // end marker
};

bool gemm_operands_addressable(long long M, long long lda, long long N, long long ldb) {
  return M * lda * 2 < (1LL << 32) && N * ldb * 2 < (1LL << 32);
}

void gemm_plan(int M, int N, int K, Epi epi, DType t, int cus, int* tile, int* splits, bool rope, bool measured) {
  for (const PlanEntry& e : kPlans) {
    if (!measured) break;
    if (e.cus == cus && e.M == M && e.N == N && e.K == K && e.epi == static_cast<int>(epi) &&
        e.dtype == static_cast<int>(t) && e.rope == static_cast<int>(rope) && e.tile < kTileCount) {
      *tile = e.tile;
      *splits = e.splits;
      return;
    }
  }
  // Largest tile that still gives every CU a workgroup; small problems fall back to small tiles
  // and, for the fp32 (split-K capable) epilogue, to K splits until the grid covers the chip.
  // Eight-wave tiles first: with two waves per SIMD they sustain the most MFMA throughput when
  // the grid is large enough (the 256x256 one as the ring, whose operand stream stays in flight
  // across slab barriers: up to 7% faster than tile 7 on 64K-row projections); then the pipelined
  // four-wave tiles from large to small (measured 13-21% faster than the register-staged tiles of
  // the same shapes on 512-row problems).
  // Tile 10 is only the RoPE fallback for N not a multiple of 128 (odd head counts): every other
  // RoPE-capable tile is 128 or more columns wide.
  const int order[] = {19, 9, 8, 20, 1, 18, 15, 16, 14, 17};
  int best = rope ? (N % 128 ? 10 : 16) : 14, best_split = 1;
  if (M >= kBatchedRows) {
    // Batched problems: the main loops are bound by each CU's operand stream from L2, so a launch
    // takes about (tiles per CU, rounded up) x (BM + BN) x K operand bytes per CU.  That favours
    // the 256x256 ring even when it leaves CUs idle: on a 15,360 x 768 x 3,072 problem its 180
    // tiles (one round) beat the 360 tiles of 128x256 (two rounds of 1.5x the bytes per FLOP).
    // Non-ring tiles are charged 7% for their shallower pipelines (measured on 64K-row problems).
    long long best_cost = -1;
    for (int id : {19, 21, 9, 8, 1, 18}) {
      const TileDef& d = kTiles[id];
      if (N % d.bn || (rope && (d.bn / d.wn) % 64)) continue;
      const long long rows = (M + d.bm - 1) / d.bm;
      if ((rows * d.bm - M) * 4 > M) continue;  // more than 25% padding rows
      const long long cost = (rows * (N / d.bn) + cus - 1) / cus * (d.bm + d.bn) * (d.ring ? 100 : 107);
      if (best_cost < 0 || cost < best_cost) {
        best = id;
        best_cost = cost;
      }
    }
    if (best_cost >= 0) {
      // The ring with 16x16x32 MFMAs for the row-major epilogues: out/down 2-6%, up 5% faster on
      // 64K rows; the head-major QKV epilogue measured 4% slower with it, so QKV keeps tile 19.
      // Both give way to the persistent ring (tile 26) when some CUs get more than one tile and a
      // tile's K loop is at most 32 slabs: measured against the better of 19 and 22, 2-7% faster on
      // the 64K-row QKV, up and out projections and 5-8% on the 15,360-row QKV and up projections,
      // but 3-5% slower on the 64-slab down projection (four tiles per CU).
      const long long tiles = static_cast<long long>((M + 255) / 256) * (N / 256);
      const bool persist_ok = epi != Epi::F32 && !rope && tiles > cus && K / BK >= 3 && K / BK <= 32;
      if (best == 19 && persist_ok) best = 26;
      if (best == 19 && (epi == Epi::F32 || epi == Epi::HALF || epi == Epi::GELU || epi == Epi::RELU)) best = 22;
      *tile = best;
      *splits = 1;
      return;
    }
  }
  for (int id : order) {
    const TileDef& d = kTiles[id];
    if (N % d.bn) continue;
    if (rope && (d.bn / d.wn) % 64) continue;
    const long long wgs = static_cast<long long>((M + d.bm - 1) / d.bm) * (N / d.bn);
    const long long waste_rows = static_cast<long long>((M + d.bm - 1) / d.bm) * d.bm - M;
    if (waste_rows * 4 > M) continue;  // more than 25% padding rows
    if (wgs >= cus) {
      best = id;
      best_split = 1;
      break;
    }
    best = id;
  }
  const TileDef& d = kTiles[best];
  const long long wgs = static_cast<long long>((M + d.bm - 1) / d.bm) * (N / d.bn);
  if (epi == Epi::F32) {
    const int nk = K / BK;
    while (wgs * best_split < cus && best_split * 2 <= nk / 4 && best_split < 8) best_split *= 2;
  }
  *tile = best;
  *splits = best_split;
}

hipError_t launch_gemm(const GemmArgs& args, Epi epi, DType t, int tile, hipStream_t stream) {
  if (tile < 0 || tile >= kTileCount) return hipErrorInvalidValue;
  GemmArgs a = args;
  a.rows_major = a.M > a.N;
  if (a.M <= 0) return hipSuccess;
  if (a.K % BK || a.N % kTiles[tile].bn || a.splits < 1) return hipErrorInvalidValue;
  if (epi != Epi::F32 && a.splits != 1) return hipErrorInvalidValue;
  // Pipelined tiles address their operands by 32-bit byte offsets into buffer resources.
  if (!kTiles[tile].pf && !gemm_operands_addressable(a.M, a.lda, a.N, a.ldb)) return hipErrorInvalidValue;
  if (epi == Epi::QKV_ROPE && !a.rope_cos) return hipErrorInvalidValue;
  if (epi == Epi::QKV && a.rope_cos) epi = Epi::QKV_ROPE;
  // RoPE needs both halves of a head in one lane: wave tiles of 64-column multiples.
  const TileDef& td = kTiles[tile];
  if (td.m16 && (epi == Epi::QKV_ROPE || epi == Epi::GEGLU)) return hipErrorInvalidValue;
  // Persistent tiles: 16-bit outputs without RoPE, at least three 64-deep slabs per tile.
  if (td.persist && (epi == Epi::F32 || epi == Epi::QKV_ROPE || (a.K / BK) % a.splits || a.K / BK / a.splits < 3))
    return hipErrorInvalidValue;
  if (epi == Epi::QKV_ROPE && (td.bn / td.wn) % 64) return hipErrorInvalidValue;
  if ((epi == Epi::QKV || epi == Epi::QKV_ROPE) && a.M % 8) return hipErrorInvalidValue;  // V^T: runs of 8 tokens
  if (epi == Epi::GEGLU && (a.N % 32 || a.ldo * 2 < a.N)) return hipErrorInvalidValue;
  if (epi == Epi::F32 && a.splits != 1 && a.bias) return hipErrorInvalidValue;  // bias joins the sum later
  const bool h = t == DType::F16;
  switch (epi) {
    case Epi::F32: return h ? launch_t<f16, Epi::F32>(a, tile, stream) : launch_t<bf16, Epi::F32>(a, tile, stream);
    case Epi::HALF: return h ? launch_t<f16, Epi::HALF>(a, tile, stream) : launch_t<bf16, Epi::HALF>(a, tile, stream);
    case Epi::GELU: return h ? launch_t<f16, Epi::GELU>(a, tile, stream) : launch_t<bf16, Epi::GELU>(a, tile, stream);
    case Epi::QKV: return h ? launch_t<f16, Epi::QKV>(a, tile, stream) : launch_t<bf16, Epi::QKV>(a, tile, stream);
    case Epi::QKV_ROPE:
      return h ? launch_t<f16, Epi::QKV_ROPE>(a, tile, stream) : launch_t<bf16, Epi::QKV_ROPE>(a, tile, stream);
    case Epi::RELU: return h ? launch_t<f16, Epi::RELU>(a, tile, stream) : launch_t<bf16, Epi::RELU>(a, tile, stream);
    case Epi::GEGLU: return h ? launch_t<f16, Epi::GEGLU>(a, tile, stream) : launch_t<bf16, Epi::GEGLU>(a, tile, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace laya
