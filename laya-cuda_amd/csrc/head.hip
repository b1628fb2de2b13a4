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
// does no work for the padding.  Launches: gather+LN, scorer.1 (fp32 MFMA, split-K), scorer tail
// (a wave per row), features (a workgroup per question), act_head.0 (the same fp32 MFMA GEMM over
// all questions, K padded with zeros to a multiple of 256 so it splits 8-16 ways), act output.
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
__global__ __launch_bounds__(256) void head_gemm_kernel(HeadGemmArgs a) {
  constexpr int BM = 32, BN = 64, KC = 128, KP = KC + 4;  // pitch KP: 16-byte rows, conflict-free reads
  constexpr int AV = BM * KC / 4 / 256, BV = BN * KC / 4 / 256;  // float4 loads per thread per chunk
  // The live row count is a device scalar of this request; it is only consulted for the stores,
  // so its load does not delay the operand loads (rows up to the capacity are in the buffers).
  const int n_rows = *a.n_rows;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN, z = blockIdx.z;
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
  for (int k0 = kb; k0 < ke; k0 += KC) {
    const int kn = min(KC, ke - k0);
    // Chunk loads, all in flight together: rows past the capacity and columns past the split read
    // a clamped in-range address; such rows are never stored, such columns never multiplied.
    f32x4 ra[AV], rb[BV];
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int e = tid + 256 * i, r = e / (KC / 4), c = 4 * (e % (KC / 4));
      const int rr = min(m0 + r, a.cap - 1), cc = min(c, kn - 4);
      ra[i] = *reinterpret_cast<const f32x4*>(a.x + static_cast<size_t>(rr) * a.K + k0 + cc);
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int e = tid + 256 * i, r = e / (KC / 4), c = 4 * (e % (KC / 4));
      rb[i] = *reinterpret_cast<const f32x4*>(a.w + static_cast<size_t>(n0 + r) * a.K + k0 + min(c, kn - 4));
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

// Scorer tail, one wave per compact head row (CLS or option): logit = w3 . gelu(v + b1) + b3.
template <int D>
__global__ __launch_bounds__(256) void head_logit_kernel(HeadLogitArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.cap) return;
  const int n_sel = *a.n_sel;  // consulted only before the stores (rows up to the capacity exist)
  const size_t off = static_cast<size_t>(r) * D;
  float b1[D / 64], w3[D / 64];
  load_row<D>(a.b1, lane, b1);
  load_row<D>(a.w3, lane, w3);
  // Partials summed in split order; loaded four at a time (clamped to the last split, whose copies
  // are not added) so each group costs one memory round trip instead of one per split.
  float v[D / 64];
#pragma unroll
  for (int i = 0; i < D / 64; ++i) v[i] = 0.f;
  for (int s0 = 0; s0 < a.splits; s0 += 4) {
    float t[4][D / 64];
#pragma unroll
    for (int u = 0; u < 4; ++u) load_row<D>(a.parts + min(s0 + u, a.splits - 1) * a.split_stride + off, lane, t[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < D / 64; ++i) v[i] = s0 + u < a.splits ? v[i] + t[u][i] : v[i];
  }
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) dot += gelu(v[i] + b1[i]) * w3[i];
  const float logit = wave_sum(dot) + a.b3[0];
  if (r >= n_sel) return;
  if (lane == 0) {
    const int q = a.sel_q[r];
    a.row_logit[r] = logit;
    a.logits[static_cast<size_t>(q) * (a.k + 1) + (r - a.qoff[q])] = logit;
  }
}

// One workgroup per question slot: softmax statistics over its option logits (slots 1..count),
// written with its CLS row as the act head's input row (zero-padded to kp columns).
__global__ __launch_bounds__(256) void head_features_kernel(HeadFeatureArgs a) {
  const int q = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* logits = a.logits + static_cast<size_t>(q) * (a.k + 1);
  float* feat = a.feat + static_cast<size_t>(q) * a.kp;
  if (q >= *a.n_q) {  // unused question slots of the shape class
    for (int j = tid; j <= a.k; j += 256) logits[j] = 0.f;
    for (int j = tid; j < a.kp; j += 256) feat[j] = 0.f;
    for (int j = tid; j < a.n_act; j += 256) a.acts[static_cast<size_t>(q) * a.n_act + j] = 0.f;
    return;
  }
  const int count = a.counts[q], base = a.qoff[q];
  for (int j = count + 1 + tid; j <= a.k; j += 256) logits[j] = 0.f;
  for (int e = tid; e < a.width; e += 256) feat[e] = a.selected[static_cast<size_t>(base) * a.width + e];
  for (int e = a.width + 4 + tid; e < a.kp; e += 256) feat[e] = 0.f;
  if (wave != 0) return;
  const float* z = a.row_logit + base + 1;
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
    feat[a.width] = t1;
    feat[a.width + 1] = t1 - t2;
    feat[a.width + 2] = ent / logf(static_cast<float>(n));
    feat[a.width + 3] = static_cast<float>(n) / 255.f;
  }
}

// act head output, one workgroup per question: hidden = gelu(sum of partials + a0b) in LDS, then
// one wave per act output.
__global__ __launch_bounds__(256) void act_out_kernel(ActOutArgs a) {
  const int q = blockIdx.x;
  const int n_q = *a.n_q;  // consulted only before the stores (all b question slots exist)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  extern __shared__ float hid[];  // [hidden]
  for (int o = tid; o < a.hidden; o += 256) {
    const size_t off = static_cast<size_t>(q) * a.hidden + o;
    // Partials summed in split order, loaded eight at a time (one round trip per group).
    const float bias = a.a0b[o];
    float v = 0.f;
    for (int s0 = 0; s0 < a.splits; s0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = a.parts[min(s0 + u, a.splits - 1) * a.split_stride + off];
#pragma unroll
      for (int u = 0; u < 8; ++u) v = s0 + u < a.splits ? v + t[u] : v;
    }
    hid[o] = gelu(v + bias);
  }
  __syncthreads();
  for (int o = wave; o < a.n_act; o += 4) {
    const float* w = a.a2w + static_cast<size_t>(o) * a.hidden;
    float s = 0.f;
    for (int e = lane; e < a.hidden; e += 64) s += hid[e] * w[e];
    s = wave_sum(s);
    if (lane == 0 && q < n_q) a.acts[static_cast<size_t>(q) * a.n_act + o] = s + a.a2b[o];
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

hipError_t launch_head_gemm(const HeadGemmArgs& a, hipStream_t stream) {
  if (a.cap <= 0) return hipSuccess;
  if (a.N % 64 || a.K % (a.splits * 32)) return hipErrorInvalidValue;
  const dim3 grid(a.N / 64, (a.cap + 31) / 32, a.splits);
  LAYA_LAUNCH(head_gemm_kernel, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_head_logit(const HeadLogitArgs& a, int width, hipStream_t stream) {
  if (a.cap <= 0) return hipSuccess;
  const dim3 grid((a.cap + 3) / 4), block(256);
  switch (width) {
#define LAYA_CASE(D) case D: LAYA_LAUNCH((head_logit_kernel<D>), grid, block, 0, stream, a); break;
    LAYA_CASE(64) LAYA_CASE(128) LAYA_CASE(256) LAYA_CASE(384) LAYA_CASE(512) LAYA_CASE(768)
    LAYA_CASE(1024) LAYA_CASE(1088) LAYA_CASE(1280) LAYA_CASE(1536) LAYA_CASE(2048)
#undef LAYA_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_head_features(const HeadFeatureArgs& a, hipStream_t stream) {
  if (a.b <= 0) return hipSuccess;
  if (a.kp < a.width + 4) return hipErrorInvalidValue;
  LAYA_LAUNCH(head_features_kernel, dim3(a.b), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_act_out(const ActOutArgs& a, hipStream_t stream) {
  if (a.b <= 0) return hipSuccess;
  const size_t lds = static_cast<size_t>(a.hidden) * sizeof(float);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  LAYA_LAUNCH(act_out_kernel, dim3(a.b), dim3(256), lds, stream, a);
  return hipGetLastError();
}

}  // namespace laya
