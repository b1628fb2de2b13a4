// Decision head: option-row gather, scorer, per-question softmax features and act head.
//
// Follows laya_cuda/laya.py:214-245 with no head transformer layers (laya.py:236-237), kept in
// fp32 end to end (the returned probabilities are computed from these logits):
//   gather  : selected = residual[indices] + type_emb[kind]   (kernels.cu:155-162; bit-exact), the
//             encoder's last residual + LayerNorm applied first to just those source rows
//   scorer  : logit = w3 . gelu(W1 LN(selected; eps 1e-5) + b1) + b3   (laya.py:238-241)
//   features: CLS row | p1, p1-p2, entropy/log(max(n,2)), max(n,2)/255  (kernels.cu:167-183)
//   act head: acts = A2 gelu(A0 features + a0) + a2                      (laya.py:243-245)
//
// Only the head rows that exist are computed: the host lists them compactly (question by
// question: CLS, then each option), so a slot whose option capacity is padded to a power of two
// does no work for the padding.  Launches: gather+LN; one launch of the fp32 MFMA GEMM for both
// scorer.1 (split-K) and the CLS-row columns of act_head.0 (every input of the act head but the
// four features, which depend on the logits); the tail, a workgroup per question (its logits,
// features, the act head's four feature columns, GELU and output layer).  Three dependent launches
// where each stage of laya.py:238-245 was one: the work is a few microseconds of memory round
// trips, so the launch count sets the head's latency.
#include "kernels.hpp"
#include "rowops.hpp"

namespace laya {

namespace {

template <int D, typename T>
__global__ __launch_bounds__(256) void head_gather_kernel(HeadGatherArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.cap || r >= *a.n_sel) return;
  NormParams<D> np;
  np.load(a.gamma, a.beta, lane);
  const int src = a.sel_src[r];
  const size_t off = static_cast<size_t>(src) * D;
  float v[D / 64];
  load_row<D>(a.residual + off, lane, v);
  if (a.n_gamma) {  // the encoder's last residual + LayerNorm of this source row
    NormParams<D> pn;
    pn.load(a.n_gamma, a.n_beta, lane);
    float br[D / 64];
    if (a.parts) {
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
    } else {
      load_row16<D, T>(static_cast<const T*>(a.branch16) + off, lane, br);
    }
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + br[i];
    normalize<D>(v, pn, a.n_eps);
  }
  if (a.type_emb) {
    float t[D / 64];
    load_row<D>(a.type_emb + static_cast<size_t>(a.qkind[a.sel_q[r]]) * D, lane, t);
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = v[i] + t[i];
  }
  store_row<D>(a.selected + static_cast<size_t>(r) * D, lane, v);
  normalize<D>(v, np, a.eps);
  store_row<D>(a.normed + static_cast<size_t>(r) * D, lane, v);
}

template <int D, typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(GatherRowsArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.cap) return;
  const bool live = r < *a.n;
  const int src = live ? a.idx[r] : 0;
  if (a.src32) {
    float v[D / 64];
    if (live) {
      load_row<D>(a.src32 + static_cast<size_t>(src) * D, lane, v);
    } else {
#pragma unroll
      for (int i = 0; i < D / 64; ++i) v[i] = 0.f;
    }
    store_row<D>(a.dst32 + static_cast<size_t>(r) * D, lane, v);
  }
  if (a.src16) {  // 16-bit rows: 8 elements (one 16-byte chunk) per lane per step
    const i32x4* s16 = reinterpret_cast<const i32x4*>(static_cast<const T*>(a.src16) + static_cast<size_t>(src) * D);
    i32x4* d16 = reinterpret_cast<i32x4*>(static_cast<T*>(a.dst16) + static_cast<size_t>(r) * D);
    for (int c = lane; c < D / 8; c += 64) d16[c] = live ? s16[c] : i32x4{0, 0, 0, 0};
  }
}

// fp32 GEMM on the fp32 matrix cores (v_mfma_f32_16x16x4_f32): parts[z] = X W^T over split z.
// Workgroup tile 32 rows x 64 cols, 4 waves of 16x32.  The split's K range is staged in LDS up to
// 128 columns at a time, every 16-byte load of a chunk issued before the first LDS store, so a
// split of up to 128 columns costs one memory round trip (these tiny products are all latency).
__device__ __forceinline__ void head_gemm_tile(const HeadGemmArgs& a, int bx, int by, int z) {
  constexpr int BM = 32, BN = 64, KC = 128, KP = KC + 4;  // pitch KP: 16-byte rows, conflict-free reads
  constexpr int AV = BM * KC / 4 / 256, BV = BN * KC / 4 / 256;  // float4 loads per thread per chunk
  // The live row count is a device scalar of this request; it is only consulted for the stores,
  // so its load does not delay the operand loads (rows up to the capacity are in the buffers).
  const int n_rows = *a.n_rows;
  const int m0 = by * BM, n0 = bx * BN;
  const int ldx = a.ldx ? a.ldx : a.K, ldw = a.ldw ? a.ldw : a.K;
  if (m0 >= a.cap) return;
  // Row blocks past the live rows exit at once (ragged batches fill a small part of their
  // capacity); the first row block never waits for the count, so batch-1 launches keep their
  // operand loads ahead of it.
  if (m0 > 0 && m0 >= n_rows) return;
  __shared__ __align__(16) float sA[BM][KP];
  __shared__ __align__(16) float sB[BN][KP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 16, wn = (wave & 1) * 32;
  const int per = a.K / a.splits;  // a multiple of 32
  const int kb = z * per, ke = kb + per;
  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  // Source row of each of this thread's A loads (the same in every chunk); a mapped row costs one
  // index load before the first chunk.
  int xr[AV];
#pragma unroll
  for (int i = 0; i < AV; ++i) {
    const int rr = min(m0 + (tid + 256 * i) / (KC / 4), a.cap - 1);
    xr[i] = a.x_rows ? min(max(a.x_rows[rr], 0), a.x_cap - 1) : rr;
  }
  for (int k0 = kb; k0 < ke; k0 += KC) {
    const int kn = min(KC, ke - k0);
    // Chunk loads, all in flight together: rows past the capacity and columns past the split read
    // a clamped in-range address; such rows are never stored, such columns never multiplied.
    f32x4 ra[AV], rb[BV];
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int e = tid + 256 * i, c = 4 * (e % (KC / 4));
      ra[i] = *reinterpret_cast<const f32x4*>(a.x + static_cast<size_t>(xr[i]) * ldx + k0 + min(c, kn - 4));
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int e = tid + 256 * i, r = e / (KC / 4), c = 4 * (e % (KC / 4));
      rb[i] = *reinterpret_cast<const f32x4*>(a.w + static_cast<size_t>(n0 + r) * ldw + k0 + min(c, kn - 4));
    }
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int e = tid + 256 * i, r = e / (KC / 4), c = 4 * (e % (KC / 4));
      *reinterpret_cast<f32x4*>(&sA[r][c]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int e = tid + 256 * i, r = e / (KC / 4), c = 4 * (e % (KC / 4));
      *reinterpret_cast<f32x4*>(&sB[r][c]) = rb[i];
    }
    __syncthreads();
    for (int kk = 0; kk < kn; kk += 4) {
      const float av = sA[wm + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float bv = sB[wn + t * 16 + (lane & 15)][kk + (lane >> 4)];
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[t], 0, 0, 0);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + wm + 4 * (lane >> 4) + e, col = n0 + wn + t * 16 + (lane & 15);
      if (row < a.cap && row < n_rows) a.parts[z * a.split_stride + static_cast<size_t>(row) * a.N + col] = acc[t][e];
    }
}

// Workgroups of two independent products in one flat grid: the first `blocks0` ids walk product 0
// (column block fastest, then row block, then split), the rest product 1.
struct HeadGemmPair {
  HeadGemmArgs g0, g1;
  int blocks0;
};
int head_gemm_blocks(const HeadGemmArgs& a) { return (a.N / 64) * ((a.cap + 31) / 32) * a.splits; }
__global__ __launch_bounds__(256) void head_gemm_kernel(HeadGemmPair p) {
  auto run = [](const HeadGemmArgs& a, int id) {
    const int nx = a.N / 64, ny = (a.cap + 31) / 32;
    head_gemm_tile(a, id % nx, (id / nx) % ny, id / (nx * ny));
  };
  const int id = blockIdx.x;
  if (id < p.blocks0) run(p.g0, id);
  else run(p.g1, id - p.blocks0);
}

// Head tail, one workgroup (8 waves) per question slot.  Everything that does not depend on the
// logits is loaded first: each thread's act_head.0 output (its CLS-row partials summed in split
// order, its four feature weights, its bias) and each wave's act_head.2 row.  Then the question's
// CLS and option rows' logits (a wave per row: scorer.1 partials summed in split order, + b1, GELU,
// dot w3, + b3) go to LDS and the logits output; wave 0 takes the softmax statistics of the option
// logits (the four features); every thread finishes its act_head.0 outputs (+ the feature columns,
// GELU) into LDS, and each wave takes act outputs (dot with act_head.2's row, + a2).
constexpr int kTailThreads = 512, kTailWaves = kTailThreads / 64;
constexpr int kTailHidden = 256;  // act_head.0 outputs whose inputs are prefetched (one per thread)
template <int D>
__global__ __launch_bounds__(kTailThreads) void head_tail_kernel(HeadTailArgs a) {
  extern __shared__ float tl[];  // row logits [k+1] | features [4] | act hidden [hidden]
  float* const zl = tl;
  float* const fv = tl + a.k + 1;
  float* const hid = fv + 4;
  const int q = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* const logits = a.logits + static_cast<size_t>(q) * (a.k + 1);
  float* const acts = a.acts + static_cast<size_t>(q) * a.n_act;
  const int n_q = *a.n_q;
  // act_head.0 output `tid` (the first kTailHidden outputs) and act_head.2 row `wave`, prefetched.
  auto act_partial = [&](int o) {
    const size_t off = static_cast<size_t>(q) * a.hidden + o;
    float v = 0.f;  // CLS-row partials in split order, eight loads in flight per group
    for (int s0 = 0; s0 < a.asplits; s0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = a.aparts[min(s0 + u, a.asplits - 1) * a.asplit_stride + off];
#pragma unroll
      for (int u = 0; u < 8; ++u) v = s0 + u < a.asplits ? v + t[u] : v;
    }
    return v;
  };
  const int po = min(tid, a.hidden - 1);
  const float pv = act_partial(po), pb = a.a0b[po];
  const float4 pw = *reinterpret_cast<const float4*>(a.a0w + static_cast<size_t>(po) * a.a0_ld + D);
  constexpr int HR = kTailHidden / 64;  // act_head.2 values per lane of the prefetched row
  float w2[HR];
  {
    const float* w = a.a2w + static_cast<size_t>(min(wave, a.n_act - 1)) * a.hidden;
#pragma unroll
    for (int j = 0; j < HR; ++j) w2[j] = w[min(lane + 64 * j, a.hidden - 1)];
  }
  if (q >= n_q) {  // unused question slots of the shape class (the prefetches above stay in bounds)
    for (int j = tid; j <= a.k; j += kTailThreads) logits[j] = 0.f;
    for (int j = tid; j < a.n_act; j += kTailThreads) acts[j] = 0.f;
    return;
  }

  const int count = a.counts[q], base = a.qoff[q];
  float b1[D / 64], w3[D / 64];
  load_row<D>(a.b1, lane, b1);
  load_row<D>(a.w3, lane, w3);
  constexpr int G = D <= 1024 ? 8 : 4;  // scorer.1 partials in flight per group
  for (int r = wave; r <= count; r += kTailWaves) {
    const size_t off = static_cast<size_t>(base + r) * D;
    // Partials loaded G at a time (clamped to the last split, whose copies are not added): one
    // memory round trip per group instead of one per split.
    float v[D / 64];
#pragma unroll
    for (int i = 0; i < D / 64; ++i) v[i] = 0.f;
    for (int s0 = 0; s0 < a.splits; s0 += G) {
      float t[G][D / 64];
#pragma unroll
      for (int u = 0; u < G; ++u) load_row<D>(a.parts + min(s0 + u, a.splits - 1) * a.split_stride + off, lane, t[u]);
#pragma unroll
      for (int u = 0; u < G; ++u)
#pragma unroll
        for (int i = 0; i < D / 64; ++i) v[i] = s0 + u < a.splits ? v[i] + t[u][i] : v[i];
    }
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < D / 64; ++i) dot += gelu(v[i] + b1[i]) * w3[i];
    const float logit = wave_sum(dot) + a.b3[0];
    if (lane == 0) {
      zl[r] = logit;
      logits[r] = logit;
    }
  }
  for (int j = count + 1 + tid; j <= a.k; j += kTailThreads) logits[j] = 0.f;
  __syncthreads();
  if (wave == 0) {
    const float* z = zl + 1;
    float mx = -INFINITY;
    for (int j = lane; j < count; j += 64) mx = fmaxf(mx, z[j]);
    mx = wave_max(mx);
    float se = 0.f;
    for (int j = lane; j < count; j += 64) se += expf(z[j] - mx);
    se = wave_sum(se);
    float ent = 0.f, t1 = 0.f, t2 = 0.f;  // entropy and the two largest probabilities
    for (int j = lane; j < count; j += 64) {
      const float p = expf(z[j] - mx) / se;
      ent -= p * logf(fmaxf(p, 1e-9f));
      if (p > t1) {
        t2 = t1;
        t1 = p;
      } else {
        t2 = fmaxf(t2, p);
      }
    }
    ent = wave_sum(ent);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const float o1 = __shfl_xor(t1, d, 64), o2 = __shfl_xor(t2, d, 64);
      t2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
      t1 = fmaxf(t1, o1);
    }
    if (lane == 0) {
      const int n = max(count, 2);
      fv[0] = t1;
      fv[1] = t1 - t2;
      fv[2] = ent / logf(static_cast<float>(n));
      fv[3] = static_cast<float>(n) / 255.f;
    }
  }
  __syncthreads();
  const float f0 = fv[0], f1 = fv[1], f2 = fv[2], f3 = fv[3];
  auto finish = [&](float v, float4 w, float bias) {  // + the four feature columns, + a0, GELU
    v = v + w.x * f0;
    v = v + w.y * f1;
    v = v + w.z * f2;
    v = v + w.w * f3;
    return gelu(v + bias);
  };
  if (tid < a.hidden) hid[tid] = finish(pv, pw, pb);
  for (int o = tid + kTailThreads; o < a.hidden; o += kTailThreads)
    hid[o] = finish(act_partial(o), *reinterpret_cast<const float4*>(a.a0w + static_cast<size_t>(o) * a.a0_ld + D),
                    a.a0b[o]);
  __syncthreads();
  for (int o = wave; o < a.n_act; o += kTailWaves) {
    float s = 0.f;
    if (o == wave && a.hidden <= kTailHidden) {
#pragma unroll
      for (int j = 0; j < HR; ++j)
        if (lane + 64 * j < a.hidden) s += hid[lane + 64 * j] * w2[j];
    } else {
      const float* w = a.a2w + static_cast<size_t>(o) * a.hidden;
      for (int e = lane; e < a.hidden; e += 64) s += hid[e] * w[e];
    }
    s = wave_sum(s);
    if (lane == 0) acts[o] = s + a.a2b[o];
  }
}

}  // namespace

hipError_t launch_head_gather(const HeadGatherArgs& a, int width, DType t, hipStream_t stream) {
  if (a.cap <= 0) return hipSuccess;
  if (a.n_gamma && !a.parts && !a.branch16) return hipErrorInvalidValue;
  const dim3 grid((a.cap + 3) / 4), block(256);
  const bool h = t == DType::F16;
  switch (width) {
#define LAYA_CASE(D)                                                                                \
  case D:                                                                                         \
    if (h) LAYA_LAUNCH((head_gather_kernel<D, f16>), grid, block, 0, stream, a);               \
    else LAYA_LAUNCH((head_gather_kernel<D, bf16>), grid, block, 0, stream, a);                \
    break;
    LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
    LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gather_rows(const GatherRowsArgs& a, int width, DType t, hipStream_t stream) {
  if (a.cap <= 0) return hipSuccess;
  const dim3 grid((a.cap + 3) / 4), block(256);
  const bool h = t == DType::F16;
  switch (width) {
#define LAYA_CASE(D)                                                                                      \
  case D:                                                                                               \
    if (h) LAYA_LAUNCH((gather_rows_kernel<D, f16>), grid, block, 0, stream, a);                  \
    else LAYA_LAUNCH((gather_rows_kernel<D, bf16>), grid, block, 0, stream, a);                   \
    break;
    LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
    LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int head_gemm_splits(int rows, int N, int K, int cus) {
  const long long wgs = static_cast<long long>((rows + 31) / 32) * (N / 64);
  int s = 1;
  while (wgs * s < cus && K % (s * 2 * 32) == 0 && K / (s * 2) >= 64) s *= 2;
  return s;
}

hipError_t launch_head_gemm(const HeadGemmArgs& a, const HeadGemmArgs& b, hipStream_t stream) {
  if (a.cap <= 0) return hipSuccess;
  if (a.N % 64 || a.K % (a.splits * 32)) return hipErrorInvalidValue;
  if (b.cap > 0 && (b.N % 64 || b.K % (b.splits * 32))) return hipErrorInvalidValue;
  const HeadGemmPair p{a, b, head_gemm_blocks(a)};
  const int blocks = p.blocks0 + (b.cap > 0 ? head_gemm_blocks(b) : 0);
  LAYA_LAUNCH(head_gemm_kernel, dim3(blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

// The tail's LDS (logits, features, act hidden) can pass the default 64 KB for wide act heads or
// large option capacities: allow the whole 160 KB of a gfx950 CU, once per device.
constexpr size_t kTailMaxLds = 160 * 1024;
hipError_t head_prepare() {
  hipError_t e = hipSuccess;
#define LAYA_CASE(D)                                                                                     \
  if (e == hipSuccess)                                                                                   \
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&head_tail_kernel<D>),                         \
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kTailMaxLds));
  LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
  LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
  return e;
}

hipError_t launch_head_tail(const HeadTailArgs& a, int width, hipStream_t stream) {
  if (a.b <= 0) return hipSuccess;
  const size_t lds = static_cast<size_t>(a.k + 1 + 4 + a.hidden) * sizeof(float);
  if (lds > kTailMaxLds || a.a0_ld < width + 4) return hipErrorInvalidValue;
  const dim3 grid(a.b), block(kTailThreads);
  switch (width) {
#define LAYA_CASE(D) case D: LAYA_LAUNCH((head_tail_kernel<D>), grid, block, lds, stream, a); break;
    LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
    LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace laya
