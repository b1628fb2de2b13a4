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
//     double-buffered, and shared by the waves (large batches), or - for batch-1 requests with few
//     query tiles - the NW waves of a 32-query tile split the keys and merge their partial results
//     (past 512 keys two 32-query groups share each staged block, halving the K/V reads per query);
//   * the wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (keys as rows, queries as
//     columns).  In that accumulator layout a lane holds one query's scores for 16 keys, so
//     the row softmax needs only one cross-lane exchange (lanes l and l^32), and the
//     probabilities are *already* the B operand of O^T = V^T P^T: P never leaves registers.
//     K's LDS rows hold the keys of each 16-key group in the order 0-3, 8-11, 4-7, 12-15, which
//     leaves each lane the scores of 8 consecutive keys, so V^T's LDS rows keep keys in order.
#include "kernels.hpp"
#include <type_traits>

namespace laya {

namespace {

constexpr int KB = 64;  // keys per block

// LDS rows of K and V^T blocks are 128 B (64 16-bit values) as eight 16-byte chunks, the chunk index
// XOR-swizzled by (row / 2) % 8: a 16-byte LDS read is served 16 lanes per pass from 64 banks, the
// lanes of a pass read one chunk position of 16 consecutive rows (eight 256-byte row pairs), and
// the swizzle spreads those pairs over the eight chunk positions (row % 8 would put rows 8 apart on
// the same banks).
__device__ __forceinline__ int kvswz(int row) { return (row >> 1) & 7; }

// max(a, b, c) in one v_max3_f32.  Written out because fmaxf chains over MFMA results compile to
// a v_max_f32 x, x (NaN quieting) per input before the combining instructions: 31 instructions for
// a 32-score block maximum instead of 16.  The scores are never NaN (masked keys are -inf).
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// The same for the first instruction that reads an MFMA's result registers: a VALU read of an
// MFMA destination needs wait states after the MFMA (the pass count plus a few for the 8-pass
// 32x32x16 MFMAs here) that the compiler inserts for its own instructions but not in front of inline
// assembly, so this one carries 16 of them itself; every later read of those registers depends on
// its result.  (Without them, a half-block variant whose first read came right after its MFMA
// gave results that differed from run to run.)
__device__ __forceinline__ float max3_after_mfma(float a, float b, float c) {
  float r;
  asm("s_nop 7\n\ts_nop 7\n\tv_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Combine a value with the one held by lane l ^ 32 (the other half of the S^T accumulator's k-slots
// for the same query) with v_permlane32_swap: a VALU lane exchange, no LDS round trip.
__device__ __forceinline__ float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max3(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// acc + p.x + p.y for two 16-bit probabilities, in fp32 (v_dot2_f32_{f16,bf16} against (1, 1)).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float sum2(f16x2 p, float acc) {
  return __builtin_amdgcn_fdot2(p, f16x2{1.0f16, 1.0f16}, acc, false);
}
__device__ __forceinline__ float sum2(bf16x2 p, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(p, bf16x2{static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)}, acc, false);
}

// Key order of K's LDS rows: row p of a block holds key kperm(p), bits 2 and 3 of p swapped (an
// involution).  The S^T accumulator's element r of lane (q, g) is row 8(r/4) + 4g + r%4 of its
// 32-key tile, i.e. key 16(r/8) + 8g + r%8: lane group g holds keys 8g..8g+7 of each 16-key group,
// in order, exactly the k-slots it feeds the O^T = V^T P^T MFMA.
__device__ __forceinline__ int kperm(int p) { return (p & ~12) | ((p >> 1) & 4) | ((p << 1) & 8); }

// One 64-key block of the single-pass softmax for this lane's query q.  s holds the raw QK^T
// scores of keys kb + 32kt + 16(r/8) + 8g + r%8 (the S^T accumulator layout over kperm-ordered
// K rows); the reference max
// `mrow` is kept in the scaled log2 domain (x * log2(e) / 8), so each probability costs one FMA
// and one exp2.  Keys outside this lane's visible range [qlo, qhi) are masked: the sequence's end,
// and on local layers the keys farther than the window from the query (kernels.cu:106-107).  Only
// blocks flagged `edge` by the caller can hold such keys.  The mask is a select per score, not a
// branch.
//
// The reference max only moves when a block's max exceeds it by more than 8 (so probabilities
// stay <= 2^8: exact enough as 16-bit MFMA operands), and the O/lsum rescale runs only when some
// lane of the wave moved it: after the first blocks most blocks skip it.  The normaliser uses the
// same reference as the numerators, so the result is the softmax either way.  A block whose keys
// are all masked for this query leaves its state untouched.  On return s holds the block's
// unnormalised probabilities and lsum and o are rescaled; the caller adds the block's probabilities
// to lsum as it rounds them to the 16-bit MFMA operands (so the weights that multiply V are the
// ones the normaliser sums).
__device__ __forceinline__ void softmax_block(f32x16 (&s)[2], f32x16 (&o)[2], float& mrow, float& lsum, int kb,
                                              bool edge, int qlo, int qhi, int g) {
  constexpr float c = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) in the exp2 domain
  constexpr float kSlack = 8.f;                       // log2 of the largest unnormalised probability
  if (edge) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + kt * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
        const bool out = (key < qlo) | (key >= qhi);
        s[kt][r] = out ? -INFINITY : s[kt][r];
      }
  }
  // Block maximum of the lane's 32 scores: two chains of v_max3 (16 instructions), each opened by
  // the instruction that waits for its MFMA results; s[1][15] is read only after its chain's opener.
  float mx[2] = {max3_after_mfma(s[0][0], s[0][1], s[0][2]), max3_after_mfma(s[1][0], s[1][1], s[1][2])};
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 3; r < 15; r += 2) mx[kt] = max3(mx[kt], s[kt][r], s[kt][r + 1]);
  float bmax = max3(mx[0], mx[1], s[0][15]);
  bmax = max3(bmax, s[1][15], s[1][15]);
  bmax = half_max(bmax) * c;
  const bool grow = bmax > mrow + kSlack;  // false while everything seen so far is masked
  if (__builtin_amdgcn_ballot_w64(grow)) {
    // Lanes that keep their reference (including ones that have seen only masked keys) scale by 1;
    // a lane's first visible block scales its empty state by exp2(-inf) = 0.
    const float alpha = grow ? __builtin_amdgcn_exp2f(mrow - bmax) : 1.f;
    mrow = grow ? bmax : mrow;
    lsum *= alpha;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
  }
  const float base = mrow == -INFINITY ? 0.f : mrow;  // nothing seen yet: probabilities are 0
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      s[kt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], c, -base));  // masked: exp2(-inf) = 0
}

// Workgroup -> (tile, head).  Workgroups are dealt to the 8 XCDs round-robin by linear id; when the
// count allows, each XCD instead gets a contiguous, head-major share, so all query tiles of a
// (sequence, head) pair run on one XCD and its K and V are fetched into that L2 once.
__device__ __forceinline__ void work_item(int nx, int ny, int* tile, int* head) {
  const int total = nx * ny;
  if (total % 8) {
    *tile = blockIdx.x;
    *head = blockIdx.y;
    return;
  }
  const int id = blockIdx.x + nx * blockIdx.y;
  const int l = (id % 8) * (total / 8) + id / 8;
  *head = l / nx;
  *tile = l - *head * nx;
}

// Workgroup -> (tile, head) over the `used` entries of the work list only (the grid covers its
// capacity, which a ragged batch fills partly), tile-major: the list is sorted longest key range
// first, so workgroups start in decreasing order of work across all heads, and the hardware's
// round-robin of consecutive workgroups over the eight XCDs gives every XCD the same mix of long
// and short items (longest-processing-time-first on each).  Returns false past the work.  With
// equal tiles (dense batches) and 8 | heads, head h lands on XCD h % 8 for every tile, so a
// sequence's K and V of one head are fetched into one L2.
__device__ __forceinline__ bool work_item_used(int nx, int ny, int used, int* tile, int* head) {
  const int id = blockIdx.x + nx * blockIdx.y;
  if (id >= used * ny) return false;
  *tile = id / ny;
  *head = id - *tile * ny;
  return true;
}

// One 64-key block of K and V^T in LDS: 64 rows of 128 bytes each (K: one key's 64 head dims, in
// kperm order; V^T: one head dim's 64 keys, in order), the 16-byte chunk index XOR-swizzled by
// kvswz(row).  Thread chunk c of a block is row c / 8, physical chunk c % 8, which holds logical
// chunk (c % 8) ^ kvswz(row).  Rows past the end of the slot are read from its last row (K) or its
// last 8 keys (V^T) instead (branch-free loads): such keys lie past the end of every sequence, so
// the softmax gives them probability exactly 0, and the values they read are finite values of
// this slot.
template <typename T>
__device__ __forceinline__ const T* k_source(const T* K, int m, int kb, int c) {
  const int r = c >> 3, lu = (c & 7) ^ kvswz(r);
  return K + static_cast<size_t>(min(kb + kperm(r), m - 1)) * 64 + lu * 8;
}
template <typename T>
__device__ __forceinline__ const T* v_source(const T* Vt, int m, int kb, int c) {
  const int r = c >> 3, lu = (c & 7) ^ kvswz(r);
  return Vt + static_cast<size_t>(r) * m + min(kb + lu * 8, m - 8);  // V^T row r = head dim
}

// Register-staged copy of a block by NTH cooperating threads (the split-key kernel's per-wave
// stages): coalesced 16-byte global loads into registers, then 16-byte LDS stores.
template <typename T, int NTH>
struct KVStage {
  static constexpr int CH = KB * 8 / NTH;  // 16-byte chunks per thread per K (and per V) block
  static_assert(CH >= 1 && CH * NTH == KB * 8, "whole chunks per thread");
  i32x4 rk[CH], rv[CH];

  __device__ __forceinline__ void load(const T* K, const T* Vt, int m, int kb, int tid) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      rk[i] = *reinterpret_cast<const i32x4*>(k_source(K, m, kb, tid + NTH * i));
      rv[i] = *reinterpret_cast<const i32x4*>(v_source(Vt, m, kb, tid + NTH * i));
    }
  }
  __device__ __forceinline__ void store(T* sK, T* sV, int tid) const {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + NTH * i;
      *reinterpret_cast<i32x4*>(sK + c * 8) = rk[i];
      *reinterpret_cast<i32x4*>(sV + c * 8) = rv[i];
    }
  }
};

// Direct copy of a block by NT threads (the shared-K/V kernel): global_load_lds_dwordx4, each
// wave filling whole 1 KB runs (8 rows) of the block, so no registers or LDS store instructions
// take part.  The caller publishes the block with publish_stage before reading it.
template <typename T, int NT>
__device__ __forceinline__ void kv_load_direct(const T* K, const T* Vt, int m, int kb, unsigned sk, unsigned sv,
                                               int tid, int wave) {
  constexpr int CH = KB * 8 / NT;
  static_assert(CH >= 1 && CH * NT == KB * 8, "whole chunks per thread");
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = tid + NT * i;
    const unsigned run = static_cast<unsigned>(wave + NT / 64 * i) * 1024u;  // this wave's 1 KB run
    lds_load16(k_source(K, m, kb, c), sk + run);
    lds_load16(v_source(Vt, m, kb, c), sv + run);
  }
}

// This lane's fragment reads in a staged block, as element offsets from the block's first row:
// row ql, logical chunk 2i + g (k-step i) at its swizzled position.  The lane's other rows are 32
// rows (2,048 elements) further on and the same chunk positions (kvswz(ql + 32) = kvswz(ql)), and a
// block's V^T rows follow its K rows (KB * 64 elements), so every fragment read of a block is one
// of these four addresses plus a constant: the reads carry it as their immediate offset.
__device__ __forceinline__ void fragment_offsets(int lane, int (&off)[4]) {
  const int ql = lane & 31, g = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) off[i] = ql * 64 + (((2 * i + g) ^ kvswz(ql)) << 3);
}

// One wave's work on one LDS-resident 64-key block for its 32 queries: S^T = K Q^T
// (v_mfma_f32_32x32x16: keys as rows, queries as columns, so a lane holds one query's scores for
// 16 keys), the online-softmax step, and O^T += V^T P^T with P straight from registers.  frag[i]
// is the block's first K row plus fragment_offsets' offset i (V^T rows follow the K rows).
template <typename T>
__device__ __forceinline__ void attend_block(const T* const (&frag)[4], const typename Vec8<T>::type (&qf)[4],
                                             f32x16 (&o)[2], float& mrow, float& lsum, int kb, bool edge, int qlo,
                                             int qhi, int lane) {
  typedef typename Vec8<T>::type T8;
  const int g = lane >> 5;
  f32x16 s[2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const T8 kf = *reinterpret_cast<const T8*>(frag[ks] + kt * 32 * 64);
      s[kt] = mfma32(kf, qf[ks], s[kt]);
    }
  }
  softmax_block(s, o, mrow, lsum, kb, edge, qlo, qhi, g);
  float rs[2] = {0.f, 0.f};  // two short dependency chains of row-sum dot products
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    T8 pb;
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[e] = to_half<T>(s[c >> 1][8 * (c & 1) + e]);
    rs[0] = sum2(__builtin_shufflevector(pb, pb, 0, 1), rs[0]);
    rs[1] = sum2(__builtin_shufflevector(pb, pb, 2, 3), rs[1]);
    rs[0] = sum2(__builtin_shufflevector(pb, pb, 4, 5), rs[0]);
    rs[1] = sum2(__builtin_shufflevector(pb, pb, 6, 7), rs[1]);
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const T8 vf = *reinterpret_cast<const T8*>(frag[c] + KB * 64 + d * 32 * KB);
      o[d] = mfma32(vf, pb, o[d]);
    }
  }
  lsum += rs[0] + rs[1];
}

// Rows of no sequence (span padding, rows past the last sequence) are exact zeros (kernels.cu:102).
template <typename T>
__device__ __forceinline__ void zero_rows(T* out, int ld, int head, int row0, int row1, int tid, int nt) {
  const int n = (row1 - row0) * 64;
  for (int e = tid; e < n; e += nt) {
    const int r = row0 + (e >> 6), c = e & 63;
    out[static_cast<size_t>(r) * ld + head * 64 + c] = to_half<T>(0.f);
  }
}

// Q^T fragments for the four 16-wide head-dim steps: lane (g, q) holds Q[q][16ks + 8g + 0..7].
template <typename T>
__device__ __forceinline__ void load_q(const T* Q, int q, bool qin, int g, typename Vec8<T>::type (&qf)[4]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (qin) {
      qf[ks] = *reinterpret_cast<const typename Vec8<T>::type*>(Q + static_cast<size_t>(q) * 64 + 16 * ks + 8 * g);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = to_half<T>(0.f);
    }
  }
}

// Large batches: a workgroup of NW waves owns 32*NW queries of one sequence and one head; every
// K/V block is staged once in LDS (double-buffered, the next block's global loads in flight during
// the current block's MFMAs) and shared by all NW waves.
template <typename T, int NW>
__device__ __forceinline__ void attention_shared(const AttnArgs& a) {
  typedef typename Vec8<T>::type T8;
  typedef typename Vec4<T>::type T4;
  constexpr int NT = 64 * NW;

  int tile, head;
  if (a.n_tiles) {
    const int used = min(*a.n_tiles, a.max_tiles);
    if (!work_item_used(a.max_tiles, a.heads, used, &tile, &head)) return;
  } else {
    work_item(a.max_tiles, a.heads, &tile, &head);
  }
  const int4 td = reinterpret_cast<const int4*>(a.tiles)[tile];
  const int row0 = td.x, row1 = td.y, start = td.z, len = td.w;
  if (row0 >= row1) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ld = a.heads * 64;
  T* out = static_cast<T*>(a.out);
  if (len < 0) {
    zero_rows(out, ld, head, row0, row1, tid, NT);
    return;
  }

  const int kend = start + len;
  const int ql = lane & 31, g = lane >> 5;
  const int q = row0 + wave * 32 + ql;
  const bool qin = q < row1;
  const bool qvalid = qin && q < kend;
  const size_t plane = static_cast<size_t>(head) * a.m * 64;
  const T* K = static_cast<const T*>(a.k) + plane;
  const T* Vt = static_cast<const T*>(a.vt) + plane;
  T8 qf[4];
  load_q(static_cast<const T*>(a.q) + plane, q, qin, g, qf);

  // Two block buffers, each K's rows then V^T's rows.
  __shared__ __align__(16) T skv[2][2 * KB * 64];
  const int uwave = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform, for M0
  const unsigned ldsK[2] = {lds_address(skv[0]), lds_address(skv[1])};
  const unsigned ldsV[2] = {lds_address(skv[0] + KB * 64), lds_address(skv[1] + KB * 64)};
  int off[4];
  fragment_offsets(lane, off);
  const T* frag0[4];
  const T* frag1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    frag0[i] = skv[0] + off[i];
    frag1[i] = skv[1] + off[i];
  }

  f32x16 o[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.f;
  float mrow = -INFINITY, lsum = 0.f;

  // Keys this tile can see: the whole sequence, or on local layers the window around its rows
  // (first block 16-aligned, so the 16-byte V^T loads stay aligned); this lane's query sees [qlo, qhi).
  const bool local = a.window >= 0;
  const int klo = local ? max(start, (row0 - a.window) & ~15) : start;
  const int khi = local ? min(kend, row1 + a.window) : kend;
  const int nkb = (khi - klo + KB - 1) / KB;
  const int qlo = local ? max(start, q - a.window) : start;
  const int qhi = local ? max(qlo, min(kend, q + a.window + 1)) : kend;
  // Double-buffered blocks: block j+1 streams into the other buffer (whose reads all ended at the
  // previous barrier) while block j is consumed; each wave then waits for its own loads and one
  // barrier publishes the block to all waves.
  kv_load_direct<T, NT>(K, Vt, a.m, klo, ldsK[0], ldsV[0], tid, uwave);
  publish_stage<waitcnt_vm(0)>();
  // Waves past the tile's last row (the short last tile of a sequence) stage keys with the others
  // but skip the block math: in ragged batches that is a fifth of the query slots.
  const bool active = row0 + wave * 32 < row1;
  // Block j from buffer cur (a constant in each copy of the step, so the fragment reads keep fixed
  // addresses) while block j+1 streams into the other buffer.
  auto step = [&](int j, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    const int kb = klo + j * KB;
    if (j + 1 < nkb) kv_load_direct<T, NT>(K, Vt, a.m, kb + KB, ldsK[cur ^ 1], ldsV[cur ^ 1], tid, uwave);
    if (active)
      attend_block<T>(cur ? frag1 : frag0, qf, o, mrow, lsum, kb, local || kb + KB > kend, qlo, qhi, lane);
    publish_stage<waitcnt_vm(0)>();
  };
  for (int j = 0; j < nkb; j += 2) {
    step(j, std::integral_constant<int, 0>());
    if (j + 1 < nkb) step(j + 1, std::integral_constant<int, 1>());
  }

  if (!qin) return;
  const float total = half_sum(lsum);
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

template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void attention_kernel(AttnArgs a) {
  attention_shared<T, NW>(a);
}
// Eight waves: capped at 128 VGPRs so that two 512-thread workgroups share a CU.
template <typename T>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void attention_kernel8(AttnArgs a) {
  attention_shared<T, 8>(a);
}

// Small batches (few query tiles): a workgroup owns 32 queries of one sequence and one head, and
// its NW waves split that sequence's 64-key blocks (wave w takes blocks w, w+NW, ...), so the
// serial chain per wave is ceil(blocks / NW) instead of blocks.  Each wave stages its own blocks
// through its own LDS region with coalesced loads (the next block in flight in registers while it
// computes the current one; one region suffices, since a wave's LDS accesses execute in issue
// order, and 16 KB per wave lets two four-wave workgroups share a CU); the NW partial (max, sum, O)
// triples are merged through LDS.
template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void attention_split_kernel(AttnArgs a) {
  typedef typename Vec8<T>::type T8;
  typedef typename Vec4<T>::type T4;
  constexpr int NT = 64 * NW;
  constexpr int OP = 65;  // LDS pitch of a merged query row (floats): conflict-free column writes
  constexpr int STAGE = 2 * KB * 64;  // per wave: one K block and one V^T block (16-bit elements)

  int tile, head;
  work_item(a.max_tiles, a.heads, &tile, &head);
  const int4 td = reinterpret_cast<const int4*>(a.tiles)[tile];
  const int row0 = td.x, row1 = td.y, start = td.z, len = td.w;
  if (row0 >= row1) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ld = a.heads * 64;
  T* out = static_cast<T*>(a.out);
  if (len < 0) {
    zero_rows(out, ld, head, row0, row1, tid, NT);
    return;
  }

  const int kend = start + len;
  const int ql = lane & 31, g = lane >> 5;
  const int q = row0 + ql;
  const bool qin = q < row1;
  const size_t plane = static_cast<size_t>(head) * a.m * 64;
  const T* K = static_cast<const T*>(a.k) + plane;
  const T* Vt = static_cast<const T*>(a.vt) + plane;
  T8 qf[4];
  load_q(static_cast<const T*>(a.q) + plane, q, qin, g, qf);

  // Staging area during the key loop, merge area after it.
  static_assert(NW * STAGE * sizeof(T) >= NW * 32 * OP * sizeof(float), "merge area fits the staging area");
  __shared__ __align__(16) T lds[NW * STAGE];
  __shared__ float sM[NW][32], sL[NW][32];
  T* mine = lds + wave * STAGE;
  KVStage<T, 64> st;

  f32x16 o[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.f;
  float mrow = -INFINITY, lsum = 0.f;

  // LDS accesses of one wave execute in issue order, so a wave's own staging needs no barrier.
  // Key range of the tile and of this lane's query as in attention_shared.
  const bool local = a.window >= 0;
  const int klo = local ? max(start, (row0 - a.window) & ~15) : start;
  const int khi = local ? min(kend, row1 + a.window) : kend;
  const int nkb = (khi - klo + KB - 1) / KB;
  const int qlo = local ? max(start, q - a.window) : start;
  const int qhi = local ? max(qlo, min(kend, q + a.window + 1)) : kend;
  if (wave < nkb) st.load(K, Vt, a.m, klo + KB * wave, lane);
  T* const sK = mine;
  T* const sV = mine + KB * 64;
  int off[4];
  fragment_offsets(lane, off);
  const T* frag[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) frag[i] = sK + off[i];
  for (int j = wave; j < nkb; j += NW) {
    st.store(sK, sV, lane);
    if (j + NW < nkb) st.load(K, Vt, a.m, klo + KB * (j + NW), lane);
    attend_block<T>(frag, qf, o, mrow, lsum, klo + KB * j, local || klo + KB * (j + 1) > kend, qlo, qhi, lane);
  }

  // Merge the waves' partial results: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w.
  __syncthreads();  // every wave is done with the staging area
  float* sO = reinterpret_cast<float*>(lds) + wave * 32 * OP;
  const float ltot = half_sum(lsum);
  if (g == 0) {
    sM[wave][ql] = mrow;
    sL[wave][ql] = ltot;
  }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) sO[ql * OP + 32 * d + 8 * (r >> 2) + 4 * g + (r & 3)] = o[d][r];
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
    wt[w] = __builtin_amdgcn_exp2f(sM[w][mq] - mx);  // a wave with no block: exp2(-inf) = 0
    total += wt[w] * sL[w][mq];
  }
  const bool valid = qo < kend && total > 0.f;
  const float inv = valid ? 1.0f / total : 0.f;
  const float* merged = reinterpret_cast<const float*>(lds);
  T* orow = out + static_cast<size_t>(qo) * ld + head * 64 + d0;
#pragma unroll
  for (int e = 0; e < DPT; e += 4) {
    T4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) acc += wt[w] * merged[w * 32 * OP + mq * OP + d0 + e + i];
      v[i] = to_half<T>(valid ? acc * inv : 0.f);
    }
    *reinterpret_cast<T4*>(orow + e) = v;
  }
}

// Batch-1 sequences of 1,000+ keys: a workgroup owns 64 queries of one sequence and one head as two
// 32-query groups, and its NW/2 key groups split the sequence's 64-key blocks (group g takes
// blocks g, g + NW/2, ...).  The two waves of a key group (one per query group) copy its blocks
// into one LDS region together and both read them, so each K/V byte serves 64 queries instead of
// the split-key kernel's 32: half the K/V traffic per query, which bounds that kernel at 1,024
// tokens.  All key groups step together (two workgroup barriers per step); the NW/2 partial (max,
// sum, O) triples of each query group are merged through LDS.
template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void attention_pair_kernel(AttnArgs a) {
  typedef typename Vec8<T>::type T8;
  typedef typename Vec4<T>::type T4;
  constexpr int QG = 2, KG = NW / QG, NT = 64 * NW;
  constexpr int OP = 65;  // LDS pitch of a merged query row (floats): conflict-free column writes
  constexpr int STAGE = 2 * KB * 64;  // per key group: one K block and one V^T block (16-bit elements)
  constexpr size_t kStageBytes = KG * STAGE * sizeof(T), kMergeBytes = NW * 32 * OP * sizeof(float);

  int tile, head;
  work_item(a.max_tiles, a.heads, &tile, &head);
  const int4 td = reinterpret_cast<const int4*>(a.tiles)[tile];
  const int row0 = td.x, row1 = td.y, start = td.z, len = td.w;
  if (row0 >= row1) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ld = a.heads * 64;
  T* out = static_cast<T*>(a.out);
  if (len < 0) {
    zero_rows(out, ld, head, row0, row1, tid, NT);
    return;
  }

  const int qg = wave % QG, kg = wave / QG;
  const int kend = start + len;
  const int ql = lane & 31, g = lane >> 5;
  const int q = row0 + qg * 32 + ql;
  const bool qin = q < row1;
  const size_t plane = static_cast<size_t>(head) * a.m * 64;
  const T* K = static_cast<const T*>(a.k) + plane;
  const T* Vt = static_cast<const T*>(a.vt) + plane;
  T8 qf[4];
  load_q(static_cast<const T*>(a.q) + plane, q, qin, g, qf);

  // Key-group staging areas during the key loop, merge area after it.
  __shared__ __align__(16) unsigned char lds[kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes];
  __shared__ float sM[NW][32], sL[NW][32];
  T* const sK = reinterpret_cast<T*>(lds) + kg * STAGE;
  T* const sV = sK + KB * 64;
  const int gt = qg * 64 + lane;  // thread index within the key group
  KVStage<T, 64 * QG> st;

  f32x16 o[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.f;
  float mrow = -INFINITY, lsum = 0.f;

  // Key range of the tile and of this lane's query as in attention_shared.
  const bool local = a.window >= 0;
  const int klo = local ? max(start, (row0 - a.window) & ~15) : start;
  const int khi = local ? min(kend, row1 + a.window) : kend;
  const int nkb = (khi - klo + KB - 1) / KB;
  const int qlo = local ? max(start, q - a.window) : start;
  const int qhi = local ? max(qlo, min(kend, q + a.window + 1)) : kend;
  const bool active = row0 + qg * 32 < row1;  // a query group past the tile's rows only stages keys
  const int steps = (nkb + KG - 1) / KG;
  int off[4];
  fragment_offsets(lane, off);
  const T* frag[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) frag[i] = sK + off[i];
  if (kg < nkb) st.load(K, Vt, a.m, klo + KB * kg, gt);
  for (int b = 0; b < steps; ++b) {
    const int j = kg + KG * b;
    if (j < nkb) st.store(sK, sV, gt);
    __syncthreads();  // the key group's block is in LDS
    if (j + KG < nkb) st.load(K, Vt, a.m, klo + KB * (j + KG), gt);
    if (j < nkb && active)
      attend_block<T>(frag, qf, o, mrow, lsum, klo + KB * j, local || klo + KB * (j + 1) > kend, qlo, qhi, lane);
    __syncthreads();  // both waves are done reading it
  }

  // Merge the key groups' partial results of each query group: O = sum_k 2^(m_k - M) O_k /
  // sum_k 2^(m_k - M) l_k.
  float* sO = reinterpret_cast<float*>(lds) + wave * 32 * OP;
  const float ltot = half_sum(lsum);
  if (g == 0) {
    sM[wave][ql] = mrow;
    sL[wave][ql] = ltot;
  }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) sO[ql * OP + 32 * d + 8 * (r >> 2) + 4 * g + (r & 3)] = o[d][r];
  __syncthreads();

  constexpr int DPT = 64 * 32 * QG / NT;  // head dims per thread in the merge
  const int mq = tid % (32 * QG), d0 = (tid / (32 * QG)) * DPT;
  const int mg = mq / 32, mr = mq % 32, qo = row0 + mq;
  if (qo >= row1) return;
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < KG; ++k) mx = fmaxf(mx, sM[mg + QG * k][mr]);
  float wt[KG], total = 0.f;
#pragma unroll
  for (int k = 0; k < KG; ++k) {
    wt[k] = __builtin_amdgcn_exp2f(sM[mg + QG * k][mr] - mx);  // a group with no block: exp2(-inf) = 0
    total += wt[k] * sL[mg + QG * k][mr];
  }
  const bool valid = qo < kend && total > 0.f;
  const float inv = valid ? 1.0f / total : 0.f;
  const float* merged = reinterpret_cast<const float*>(lds);
  T* orow = out + static_cast<size_t>(qo) * ld + head * 64 + d0;
#pragma unroll
  for (int e = 0; e < DPT; e += 4) {
    T4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KG; ++k) acc += wt[k] * merged[(mg + QG * k) * 32 * OP + mr * OP + d0 + e + i];
      v[i] = to_half<T>(valid ? acc * inv : 0.f);
    }
    *reinterpret_cast<T4*>(orow + e) = v;
  }
}

template <typename T>
hipError_t launch_t(const AttnArgs& a, int mode, int waves, hipStream_t stream) {
  const dim3 grid(a.max_tiles, a.heads);
  if (mode == kAttnPairKeys) {
    switch (waves) {
      case 4: LAYA_LAUNCH((attention_pair_kernel<T, 4>), grid, dim3(256), 0, stream, a); break;
      case 8: LAYA_LAUNCH((attention_pair_kernel<T, 8>), grid, dim3(512), 0, stream, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (mode == kAttnSplitKeys) {
    switch (waves) {
      case 2: LAYA_LAUNCH((attention_split_kernel<T, 2>), grid, dim3(128), 0, stream, a); break;
      case 4: LAYA_LAUNCH((attention_split_kernel<T, 4>), grid, dim3(256), 0, stream, a); break;
      case 8: LAYA_LAUNCH((attention_split_kernel<T, 8>), grid, dim3(512), 0, stream, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (waves) {
    case 1: LAYA_LAUNCH((attention_kernel<T, 1>), grid, dim3(64), 0, stream, a); break;
    case 2: LAYA_LAUNCH((attention_kernel<T, 2>), grid, dim3(128), 0, stream, a); break;
    case 4: LAYA_LAUNCH((attention_kernel<T, 4>), grid, dim3(256), 0, stream, a); break;
    case 8: LAYA_LAUNCH((attention_kernel8<T>), grid, dim3(512), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

int attention_block_rows(int mode, int waves) {
  return mode == kAttnSplitKeys ? 32 : mode == kAttnPairKeys ? 64 : 32 * waves;
}

bool attention_mode_valid(int mode, int waves) {
  if (mode == kAttnSharedKV) return waves == 1 || waves == 2 || waves == 4 || waves == 8;
  if (mode == kAttnSplitKeys) return waves == 2 || waves == 4 || waves == 8;
  if (mode == kAttnPairKeys) return waves == 4 || waves == 8;
  return false;
}

hipError_t launch_attention(const AttnArgs& a, DType t, int mode, int waves, hipStream_t stream) {
  if (a.max_tiles <= 0) return hipSuccess;
  if (!attention_mode_valid(mode, waves)) return hipErrorInvalidValue;
  return t == DType::F16 ? launch_t<f16>(a, mode, waves, stream) : launch_t<bf16>(a, mode, waves, stream);
}

}  // namespace laya
