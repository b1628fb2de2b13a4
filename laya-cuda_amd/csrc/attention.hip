// Fused bidirectional attention over packed rows on gfx950 MFMA (QK^T, masked online softmax, PV).
//
// Semantics follow the reference's `attention` kernel (laya_cuda/kernels.cu:90-154) with
// window = -1: each query of a sequence attends to every key of that sequence, scores are
// scaled by 1/sqrt(64), the softmax is fp32 and single-pass (running max, rescaled sums), and
// query rows that are not tokens of a sequence (span padding, rows past the last sequence)
// are written as exact zeros.
//
// Work decomposition (MI355X-first, not the reference's one-warp-per-16-queries):
//   * one workgroup per (tile, head); a tile is a run of up to 32*NW query rows of ONE sequence,
//     listed by the host so no tile straddles sequences (ragged batches waste no key blocks);
//   * NW waves, each owning 32 queries; K and V^T blocks of 64 keys are staged through LDS,
//     double-buffered, and shared by the waves;
//   * the wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (keys as rows, queries as
//     columns).  In that accumulator layout a lane holds one query's scores for 16 keys, so
//     the row softmax needs only one cross-lane exchange (lanes l and l^32), and the
//     probabilities are *already* the B operand of O^T = V^T P^T: P never leaves registers.
//     V^T's LDS rows store keys permuted within each 16-key group to match that lane order.
#include "kernels.hpp"

namespace laya {

namespace {

constexpr int KB = 64;  // keys per block

template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void attention_kernel(AttnArgs a) {
  typedef typename Vec8<T>::type T8;
  typedef typename Vec4<T>::type T4;
  constexpr int NT = 64 * NW;
  constexpr int CH = KB * 8 / NT;  // 16-byte chunks per thread per K (and per V) block

  const int tile = blockIdx.x, head = blockIdx.y;
  if (tile >= a.max_tiles || tile >= *a.n_tiles) return;
  const int row0 = a.tiles[3 * tile], row1 = a.tiles[3 * tile + 1], seq = a.tiles[3 * tile + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ld = a.heads * 64;
  T* out = static_cast<T*>(a.out);

  if (seq < 0) {  // rows that belong to no sequence: zeros (kernels.cu:102)
    const int n = (row1 - row0) * 64;
    for (int e = tid; e < n; e += NT) {
      const int r = row0 + (e >> 6), c = e & 63;
      out[static_cast<size_t>(r) * ld + head * 64 + c] = to_half<T>(0.f);
    }
    return;
  }

  const int start = a.starts[seq], len = a.lengths[seq], kend = start + len;
  const int ql = lane & 31, g = lane >> 5;
  const int q = row0 + wave * 32 + ql;
  const bool qin = q < row1;
  const bool qvalid = qin && q < kend;

  const size_t plane = static_cast<size_t>(head) * a.m * 64;
  const T* Q = static_cast<const T*>(a.q) + plane;
  const T* K = static_cast<const T*>(a.k) + plane;
  const T* Vt = static_cast<const T*>(a.vt) + plane;

  // Q^T fragments for the four 16-wide head-dim steps: lane (g, q) holds Q[q][16ks + 8g + 0..7].
  T8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (qin) {
      qf[ks] = *reinterpret_cast<const T8*>(Q + static_cast<size_t>(q) * 64 + 16 * ks + 8 * g);
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) qf[ks][s] = to_half<T>(0.f);
    }
  }

  __shared__ __align__(16) T sK[2][KB * 64];
  __shared__ __align__(16) T sV[2][64 * KB];

  i32x4 rk[CH], rv[CH];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + NT * i, r = c >> 3, u = c & 7;
      const int key = kb + r;
      rk[i] = key < a.m ? *reinterpret_cast<const i32x4*>(K + static_cast<size_t>(key) * 64 + u * 8) : i32x4{0, 0, 0, 0};
      const int k8 = kb + u * 8;  // V^T row r = head dim, keys k8..k8+7
      rv[i] = k8 < a.m ? *reinterpret_cast<const i32x4*>(Vt + static_cast<size_t>(r) * a.m + k8) : i32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + NT * i, r = c >> 3, u = c & 7;
      *reinterpret_cast<i32x4*>(&sK[buf][r * 64 + ((u ^ (r & 7)) << 3)]) = rk[i];
      // Keys 8u..8u+7 of V^T row r: group cg = u/2, half = u%2.  Logical keys 4g..4g+3 and
      // 8+4g..8+4g+3 of a 16-key group must sit at physical 8g..8g+7 (one 16-byte read per lane).
      const int cg = u >> 1, half = u & 1;
      T* vrow = &sV[buf][r * KB];
      const int p0 = ((2 * cg) ^ (r & 7)) << 3, p1 = ((2 * cg + 1) ^ (r & 7)) << 3;
      *reinterpret_cast<int2*>(vrow + p0 + 4 * half) = make_int2(rv[i][0], rv[i][1]);
      *reinterpret_cast<int2*>(vrow + p1 + 4 * half) = make_int2(rv[i][2], rv[i][3]);
    }
  };

  f32x16 o[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.f;
  float mrow = -INFINITY, lsum = 0.f;
  const float scale = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) in the exp2 domain

  const int nkb = (len + KB - 1) / KB;
  gload(start);
  lstore(0);
  __syncthreads();
  for (int j = 0; j < nkb; ++j) {
    const int cur = j & 1, kb = start + j * KB;
    if (j + 1 < nkb) gload(kb + KB);

    // S^T for keys kb..kb+63 (two 32-key tiles) against this wave's 32 queries.
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
      const int kr = kt * 32 + ql;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int ch = 2 * ks + g;
        const T8 kf = *reinterpret_cast<const T8*>(&sK[cur][kr * 64 + ((ch ^ (kr & 7)) << 3)]);
        s[kt] = mfma32(kf, qf[ks], s[kt]);
      }
    }
    // Mask keys past the sequence, scale, and take this block's max per query.
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float x = key < kend ? s[kt][r] * scale : -INFINITY;
        s[kt][r] = x;
        bmax = fmaxf(bmax, x);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(mrow, bmax);
    const float alpha = mrow == -INFINITY ? 0.f : exp2f(mrow - mnew);
    mrow = mnew;
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = s[kt][r] == -INFINITY ? 0.f : exp2f(s[kt][r] - mnew);
        s[kt][r] = p;
        psum += p;
      }
    lsum = lsum * alpha + psum;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] *= alpha;

    // O^T += V^T P^T over four 16-key chunks.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      T8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = to_half<T>(s[c >> 1][8 * (c & 1) + e]);
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int vr = d * 32 + ql;
        const T8 vf = *reinterpret_cast<const T8*>(&sV[cur][vr * KB + (((2 * c + g) ^ (vr & 7)) << 3)]);
        o[d] = mfma32(vf, pb, o[d]);
      }
    }
    if (j + 1 < nkb) lstore(cur ^ 1);
    __syncthreads();
  }

  if (!qin) return;
  const float total = lsum + __shfl_xor(lsum, 32, 64);
  const float inv = qvalid ? 1.0f / total : 0.f;
  T* orow = out + static_cast<size_t>(q) * ld + head * 64;
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      T4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = to_half<T>(qvalid ? o[d][4 * r4 + e] * inv : 0.f);
      *reinterpret_cast<T4*>(orow + d * 32 + 8 * r4 + 4 * g) = v;
    }
}

// Split-key variant for small batches (few query tiles): a workgroup owns 32 queries of one
// sequence and one head, and its NW waves split that sequence's 64-key blocks (wave w takes
// blocks w, w+NW, ...).  Each wave reads its K and V^T fragments straight from global memory into
// MFMA operand registers (no reuse between waves, so no LDS staging) and prefetches its next block
// while computing the current one; the serial chain per wave is ceil(blocks / NW) instead of
// blocks.  The NW partial (max, sum, O) triples are merged through LDS at the end.
template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void attention_split_kernel(AttnArgs a) {
  typedef typename Vec8<T>::type T8;
  typedef typename Vec4<T>::type T4;
  constexpr int NT = 64 * NW;
  constexpr int OP = 65;  // LDS pitch of a merged query row (floats): conflict-free column writes

  const int tile = blockIdx.x, head = blockIdx.y;
  if (tile >= a.max_tiles || tile >= *a.n_tiles) return;
  const int row0 = a.tiles[3 * tile], row1 = a.tiles[3 * tile + 1], seq = a.tiles[3 * tile + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ld = a.heads * 64;
  T* out = static_cast<T*>(a.out);

  if (seq < 0) {  // rows that belong to no sequence: zeros (kernels.cu:102)
    const int n = (row1 - row0) * 64;
    for (int e = tid; e < n; e += NT) {
      const int r = row0 + (e >> 6), c = e & 63;
      out[static_cast<size_t>(r) * ld + head * 64 + c] = to_half<T>(0.f);
    }
    return;
  }

  const int start = a.starts[seq], len = a.lengths[seq], kend = start + len;
  const int ql = lane & 31, g = lane >> 5;
  const int q = row0 + ql;
  const bool qin = q < row1;
  const size_t plane = static_cast<size_t>(head) * a.m * 64;
  const T* Q = static_cast<const T*>(a.q) + plane;
  const T* K = static_cast<const T*>(a.k) + plane;
  const T* Vt = static_cast<const T*>(a.vt) + plane;

  T8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (qin) {
      qf[ks] = *reinterpret_cast<const T8*>(Q + static_cast<size_t>(q) * 64 + 16 * ks + 8 * g);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = to_half<T>(0.f);
    }
  }

  // Fragments of one 64-key block.  K (A operand of S^T = K Q^T): lane (ql, g) holds key
  // kb + 32kt + ql, dims 16ks + 8g..+7.  V^T (A operand of O^T = V^T P^T): lane holds head dim
  // 32d + ql and, of the 16-key chunk c, keys 4g..4g+3 and 8+4g..8+4g+3 - the keys whose
  // probabilities the S^T accumulator leaves in this lane.
  T8 kf[2][4], vf[4][2];
  auto load_block = [&](int kb, T8 (&kfr)[2][4], T8 (&vfr)[4][2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = kb + 32 * kt + ql;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (key < a.m) {
          kfr[kt][ks] = *reinterpret_cast<const T8*>(K + static_cast<size_t>(key) * 64 + 16 * ks + 8 * g);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) kfr[kt][ks][e] = to_half<T>(0.f);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k0 = kb + 16 * c + 4 * g, k1 = k0 + 8;
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const T* row = Vt + static_cast<size_t>(32 * d + ql) * a.m;
        T4 lo, hi;
        if (k0 < a.m) {
          lo = *reinterpret_cast<const T4*>(row + k0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) lo[e] = to_half<T>(0.f);
        }
        if (k1 < a.m) {
          hi = *reinterpret_cast<const T4*>(row + k1);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) hi[e] = to_half<T>(0.f);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vfr[c][d][e] = lo[e];
          vfr[c][d][4 + e] = hi[e];
        }
      }
    }
  };

  f32x16 o[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.f;
  float mrow = -INFINITY, lsum = 0.f;
  const float scale = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) in the exp2 domain

  const int nkb = (len + 63) / 64;
  T8 kn[2][4], vn[4][2];
  if (wave < nkb) load_block(start + 64 * wave, kn, vn);
  for (int j = wave; j < nkb; j += NW) {
    const int kb = start + 64 * j;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kf[kt][ks] = kn[kt][ks];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int d = 0; d < 2; ++d) vf[c][d] = vn[c][d];
    if (j + NW < nkb) load_block(kb + 64 * NW, kn, vn);

    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) s[kt] = mfma32(kf[kt][ks], qf[ks], s[kt]);
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float x = key < kend ? s[kt][r] * scale : -INFINITY;
        s[kt][r] = x;
        bmax = fmaxf(bmax, x);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(mrow, bmax);
    const float alpha = mrow == -INFINITY ? 0.f : exp2f(mrow - mnew);
    mrow = mnew;
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = s[kt][r] == -INFINITY ? 0.f : exp2f(s[kt][r] - mnew);
        s[kt][r] = p;
        psum += p;
      }
    lsum = lsum * alpha + psum;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      T8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = to_half<T>(s[c >> 1][8 * (c & 1) + e]);
#pragma unroll
      for (int d = 0; d < 2; ++d) o[d] = mfma32(vf[c][d], pb, o[d]);
    }
  }

  // Merge the waves' partial results: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w.
  __shared__ float sO[NW][32 * OP];
  __shared__ float sM[NW][32], sL[NW][32];
  const float ltot = lsum + __shfl_xor(lsum, 32, 64);
  if (g == 0) {
    sM[wave][ql] = mrow;
    sL[wave][ql] = ltot;
  }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) sO[wave][ql * OP + 32 * d + 8 * (r >> 2) + 4 * g + (r & 3)] = o[d][r];
  __syncthreads();

  constexpr int DPT = 64 * 32 / NT;  // head dims per thread in the merge
  const int mq = tid & 31, d0 = (tid >> 5) * DPT;
  const int qo = row0 + mq;
  if (qo >= row1) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) mx = fmaxf(mx, sM[w][mq]);
  float wt[NW], total = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    wt[w] = sM[w][mq] == -INFINITY ? 0.f : exp2f(sM[w][mq] - mx);
    total += wt[w] * sL[w][mq];
  }
  const bool valid = qo < kend && total > 0.f;
  const float inv = valid ? 1.0f / total : 0.f;
  T* orow = out + static_cast<size_t>(qo) * ld + head * 64 + d0;
#pragma unroll
  for (int e = 0; e < DPT; e += 4) {
    T4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) acc += wt[w] * sO[w][mq * OP + d0 + e + i];
      v[i] = to_half<T>(valid ? acc * inv : 0.f);
    }
    *reinterpret_cast<T4*>(orow + e) = v;
  }
}

template <typename T>
hipError_t launch_t(const AttnArgs& a, int mode, int waves, hipStream_t stream) {
  const dim3 grid(a.max_tiles, a.heads);
  if (mode == kAttnSplitKeys) {
    switch (waves) {
      case 2: hipLaunchKernelGGL((attention_split_kernel<T, 2>), grid, dim3(128), 0, stream, a); break;
      case 4: hipLaunchKernelGGL((attention_split_kernel<T, 4>), grid, dim3(256), 0, stream, a); break;
      case 8: hipLaunchKernelGGL((attention_split_kernel<T, 8>), grid, dim3(512), 0, stream, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (waves) {
    case 1: hipLaunchKernelGGL((attention_kernel<T, 1>), grid, dim3(64), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((attention_kernel<T, 2>), grid, dim3(128), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((attention_kernel<T, 4>), grid, dim3(256), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

int attention_block_rows(int mode, int waves) { return mode == kAttnSplitKeys ? 32 : 32 * waves; }

bool attention_mode_valid(int mode, int waves) {
  if (mode == kAttnSharedKV) return waves == 1 || waves == 2 || waves == 4;
  if (mode == kAttnSplitKeys) return waves == 2 || waves == 4 || waves == 8;
  return false;
}

hipError_t launch_attention(const AttnArgs& a, DType t, int mode, int waves, hipStream_t stream) {
  if (a.max_tiles <= 0) return hipSuccess;
  if (!attention_mode_valid(mode, waves)) return hipErrorInvalidValue;
  return t == DType::F16 ? launch_t<f16>(a, mode, waves, stream) : launch_t<bf16>(a, mode, waves, stream);
}

}  // namespace laya
