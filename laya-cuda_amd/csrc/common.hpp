// Shared device helpers for the gfx950 (CDNA4) encoder kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>

namespace laya {

// Kernel-level timing on request: when the host has set `launch_timing` on this thread, the next
// LAYA_LAUNCH records that event pair from the kernel's own dispatch (hipExtLaunchKernel: start
// and end of the kernel, the interval a kernel trace reports, without the extra stream packets of
// hipEventRecord around the launch) and clears it.  Never set while a stream is being captured.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
inline thread_local LaunchTiming launch_timing;

#define LAYA_LAUNCH(kernel, grid, block, lds, stream, ...)                                          \
  do {                                                                                              \
    if (::laya::launch_timing.start) {                                                              \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, ::laya::launch_timing.start,          \
                            ::laya::launch_timing.stop, 0, __VA_ARGS__);                            \
      ::laya::launch_timing = ::laya::LaunchTiming{};                                              \
    } else {                                                                                        \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                            \
    }                                                                                               \
  } while (0)

// 16-bit MFMA operand types.  Storage in HBM is raw 16-bit; arithmetic is always fp32.
typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

template <typename T> struct Vec8;
template <> struct Vec8<bf16> { typedef bf16x8 type; };
template <> struct Vec8<f16> { typedef f16x8 type; };
template <typename T> struct Vec4;
template <> struct Vec4<bf16> { typedef bf16x4 type; };
template <> struct Vec4<f16> { typedef f16x4 type; };

// D = A(32x16) * B(16x32) + C, fp32 accumulate.  Lane l supplies row/col l%32 and the 8
// consecutive k-slots of group l/32; the accumulator's element r of lane l is
// C[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// D = A(16x32) * B(32x16) + C; element r of lane l is C[4*(l/16) + r][l%16].
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Direct global -> LDS load (global_load_lds_dwordx4): the wave's 64 lanes each fetch 16 bytes from
// their own address `g` and the hardware writes them, lane by lane, to the 1 KB of LDS starting at
// byte address `lds` (wave-uniform; M0 holds it).  Issued from inline assembly: the compiler's own
// form makes its wait-counter model assume that each such load may overwrite any LDS a pending
// read targets, so it drains every LDS read before each load.  Here a load's destination is read
// only after publish_stage below, which waits for the loads explicitly.  The {m0} operand lets the
// compiler write M0 and know it is live; one s_nop separates that write from the LDS DMA.
__device__ __forceinline__ void lds_load16(const void* g, unsigned lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds));
}
// The same direct load through a buffer resource (buffer_load_dwordx4 ... offen lds): lane l fetches
// 16 bytes at resource base + voffset(l) + soffset and the hardware writes them to LDS byte address
// lds + 16 l (lds wave-uniform, in M0).  Loads past the resource's byte range return zeros.
// soffset must be wave-uniform; readfirstlane puts it in an SGPR where the compiler computed it with
// vector instructions (integer division of uniform values), and folds away where it already is one.
__device__ __forceinline__ void lds_load16_buffer(i32x4 rsrc, unsigned voffset, unsigned soffset, unsigned lds) {
  soffset = __builtin_amdgcn_readfirstlane(soffset);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voffset), "s"(rsrc), "s"(soffset),
               "{m0}"(lds));
}
// 128-bit buffer resource of `bytes` bytes at `base` (raw buffer: stride 0, byte offsets), wave-uniform.
__device__ __forceinline__ i32x4 buffer_resource(const void* base, unsigned bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(p & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((p >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  r[3] = 0x00020000;  // dword 3 of a raw gfx9 buffer resource: 32-bit data format
  return r;
}
// Byte address of an LDS object, as M0 wants it.
__device__ __forceinline__ unsigned lds_address(const void* p) {
  typedef __attribute__((address_space(3))) const void* LdsPtr;
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>((LdsPtr)p));
}
// Publishes LDS written by direct loads: wait for this wave's memory operations up to the
// s_waitcnt immediate `kWait`, then one workgroup barrier.  s_waitcnt and s_barrier are intrinsics
// without memory semantics in LLVM IR, so the empty asm with a memory clobber keeps the compiler
// from moving the following LDS reads above them; it emits no instruction.
template <int kWait>
__device__ __forceinline__ void publish_stage() {
  __builtin_amdgcn_s_waitcnt(kWait);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// s_waitcnt immediate (gfx9 layout: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8) that waits
// until at most `vm` vector memory operations are outstanding and every LDS access has completed.
constexpr int waitcnt_vm(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }
// s_waitcnt immediate that waits until at most `vm` vector memory operations are outstanding and
// leaves LDS accesses in flight.
constexpr int waitcnt_vm_only(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (15 << 8); }
// s_waitcnt immediate that waits for every LDS access (lgkmcnt 0) and no vector memory operation.
constexpr int waitcnt_lgkm0_keep_vm() { return 15 | (3 << 14) | (7 << 4); }

template <typename T> __device__ __forceinline__ T to_half(float v) { return static_cast<T>(v); }
template <typename T> __device__ __forceinline__ float to_float(T v) { return static_cast<float>(v); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, kWave));
  return v;
}

// Exact-erf GELU, computed in fp32 with the device libm's erff (the fp32 decision head).
__device__ __forceinline__ float gelu(float v) { return 0.5f * v * (1.0f + erff(v * 0.7071067811865475f)); }

// Exact-erf GELU for values rounded to 16 bits right after (the FFN-up GEMM epilogue), with erfc
// from Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26:
//   erfc(z) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2),  t = 1 / (1 + p z),  z >= 0,
// absolute error <= 1.5e-7 (far below the 2^-11 relative rounding of fp16 that follows).
// With q = Phi(-|x|) = erfc(|x|/sqrt(2))/2, GELU(x) = x Phi(x) is x (1 - q) for x >= 0 and x q for
// x < 0, i.e. max(x, 0) - |x| q: one max and one FMA instead of a compare, a select and two
// products, and large negative inputs never subtract nearly equal numbers.  The 1/sqrt(2) is folded
// into p and the 1/2 into the a_i, so a value costs one reciprocal, one exp2 and nine VALU
// operations instead of the libm erff's range reduction: the epilogue of a 65536 x 4096 GEMM runs
// this 268M times.
__device__ __forceinline__ float gelu16(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f * 0.7071067811865475f, ax, 1.0f));
  float poly = __builtin_fmaf(t, 0.5f * 1.061405429f, 0.5f * -1.453152027f);
  poly = __builtin_fmaf(t, poly, 0.5f * 1.421413741f);
  poly = __builtin_fmaf(t, poly, 0.5f * -0.284496736f);
  poly = __builtin_fmaf(t, poly, 0.5f * 0.254829592f);
  // exp(-z^2) = exp2(-x^2 log2(e) / 2)
  const float q = t * poly * __builtin_amdgcn_exp2f(x * x * (-0.5f * 1.4426950408889634f));
  return __builtin_fmaf(-ax, q, fmaxf(x, 0.f));
}

}  // namespace laya
