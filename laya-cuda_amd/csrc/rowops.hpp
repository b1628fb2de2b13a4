// Wave-per-row helpers: a 64-lane wave holds one d-wide fp32 row in registers.
#pragma once

#include "common.hpp"

namespace laya {

// Lane-to-element map: chunk c of a lane holds elements c*64*V + lane*V .. +V-1 (V-wide vectors),
// so a wave's loads of one chunk are one contiguous, coalesced span of the row.
template <int D> struct RowMap {
  static constexpr int V = (D % 256 == 0) ? 4 : (D % 128 == 0) ? 2 : 1;
  static constexpr int C = D / (64 * V);
  static_assert(D % 64 == 0, "row width must be a multiple of 64");
  __device__ static int index(int c, int lane, int i) { return c * 64 * V + lane * V + i; }
};

template <int D> __device__ __forceinline__ void load_row(const float* src, int lane, float (&v)[D / 64]) {
  using R = RowMap<D>;
#pragma unroll
  for (int c = 0; c < R::C; ++c) {
    if constexpr (R::V == 4) {
      float4 t = *reinterpret_cast<const float4*>(src + R::index(c, lane, 0));
      v[c * 4 + 0] = t.x; v[c * 4 + 1] = t.y; v[c * 4 + 2] = t.z; v[c * 4 + 3] = t.w;
    } else if constexpr (R::V == 2) {
      float2 t = *reinterpret_cast<const float2*>(src + R::index(c, lane, 0));
      v[c * 2 + 0] = t.x; v[c * 2 + 1] = t.y;
    } else {
      v[c] = src[R::index(c, lane, 0)];
    }
  }
}

template <int D> __device__ __forceinline__ void store_row(float* dst, int lane, const float (&v)[D / 64]) {
  using R = RowMap<D>;
#pragma unroll
  for (int c = 0; c < R::C; ++c) {
    if constexpr (R::V == 4) {
      *reinterpret_cast<float4*>(dst + R::index(c, lane, 0)) =
          make_float4(v[c * 4 + 0], v[c * 4 + 1], v[c * 4 + 2], v[c * 4 + 3]);
    } else if constexpr (R::V == 2) {
      *reinterpret_cast<float2*>(dst + R::index(c, lane, 0)) = make_float2(v[c * 2 + 0], v[c * 2 + 1]);
    } else {
      dst[R::index(c, lane, 0)] = v[c];
    }
  }
}

template <int D, typename T>
__device__ __forceinline__ void store_row16(T* dst, int lane, const float (&v)[D / 64]) {
  using R = RowMap<D>;
#pragma unroll
  for (int c = 0; c < R::C; ++c) {
    if constexpr (R::V == 4) {
      typename Vec4<T>::type t;
      t[0] = to_half<T>(v[c * 4 + 0]); t[1] = to_half<T>(v[c * 4 + 1]);
      t[2] = to_half<T>(v[c * 4 + 2]); t[3] = to_half<T>(v[c * 4 + 3]);
      *reinterpret_cast<typename Vec4<T>::type*>(dst + R::index(c, lane, 0)) = t;
    } else {
#pragma unroll
      for (int i = 0; i < R::V; ++i) dst[R::index(c, lane, i)] = to_half<T>(v[c * R::V + i]);
    }
  }
}

template <int D, typename T>
__device__ __forceinline__ void load_row16(const T* src, int lane, float (&v)[D / 64]) {
  using R = RowMap<D>;
#pragma unroll
  for (int c = 0; c < R::C; ++c) {
    if constexpr (R::V == 4) {
      const typename Vec4<T>::type t = *reinterpret_cast<const typename Vec4<T>::type*>(src + R::index(c, lane, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[c * 4 + i] = to_float<T>(t[i]);
    } else {
#pragma unroll
      for (int i = 0; i < R::V; ++i) v[c * R::V + i] = to_float<T>(src[R::index(c, lane, i)]);
    }
  }
}

// LayerNorm parameters of a row, loaded into registers at kernel start so that their latency
// overlaps the row's own loads instead of following the reductions.
template <int D> struct NormParams {
  float g[D / 64], b[D / 64];
  __device__ __forceinline__ void load(const float* gamma, const float* beta, int lane) {
    if (gamma) load_row<D>(gamma, lane, g);
    if (beta) {
      load_row<D>(beta, lane, b);
    } else {
#pragma unroll
      for (int i = 0; i < D / 64; ++i) b[i] = 0.f;
    }
  }
};

// In-register LayerNorm of one row: two passes (mean, then centred variance) as in
// laya_cuda/kernels.cu:38-46, with wave butterflies for the sums.
template <int D>
__device__ __forceinline__ void normalize(float (&v)[D / 64], const NormParams<D>& p, float eps) {
  constexpr int N = D / 64;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) s += v[i];
  const float mean = wave_sum(s) / static_cast<float>(D);
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float c = v[i] - mean;
    sq += c * c;
  }
  const float inv = 1.0f / sqrtf(wave_sum(sq) / static_cast<float>(D) + eps);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = (v[i] - mean) * inv * p.g[i] + p.b[i];
}

}  // namespace laya
