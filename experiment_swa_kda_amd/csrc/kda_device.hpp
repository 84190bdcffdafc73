// Device-side primitives shared by the gfx950 kernels of libkda_mi355x.
//
// wave64 CDNA4: 64 lanes per wavefront, MFMA v_mfma_f32_16x16x32_bf16 with the operand
// layout (verified on MI355X):
//   lane l, e = 0..7 :  A[l % 16][8 * (l / 16) + e]     (16 x 32, row-major view)
//                       B[8 * (l / 16) + e][l % 16]     (32 x 16)
//   lane l, r = 0..3 :  C[4 * (l / 16) + r][l % 16]     (16 x 16, f32)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kda {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kChunk = 64;   // tokens per chunk
constexpr int kSub = 16;     // tokens per MFMA row block

__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() {
  f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return z;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Full-precision sigmoid used where the value feeds a gradient chain.
__device__ __forceinline__ float sigmoid_acc(float x) {
  if (x >= 0.f) return 1.0f / (1.0f + expf(-x));
  float e = expf(x);
  return e / (1.0f + e);
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
  // sum over aligned groups of W lanes (W power of two, W <= 64)
#pragma unroll
  for (int m = W / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// 8 consecutive bf16 -> float
__device__ __forceinline__ void load8(const bf16* p, float* out) {
  bf16x8 x = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)x[e];
}

__device__ __forceinline__ void store8(bf16* p, const float* in) {
  bf16x8 x;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (bf16)in[e];
  *reinterpret_cast<bf16x8*>(p) = x;
}

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X (linear id mod 8),
// each XCD with its own L2.  For a 1-D grid of kXcds * NS * ceil(NR / kXcds) workgroups,
// this maps linear id -> (recurrence r, strip) so the NS strips of one recurrence, which
// read identical per-chunk operands, land on the same XCD.  Returns false past NR.
constexpr int kXcds = 8;
__device__ __forceinline__ bool xcd_strip_coords(int NR, int NS, int& r, int& strip) {
  const int L = blockIdx.x;
  const int x = L % kXcds, rest = L / kXcds;
  strip = rest % NS;
  r = (rest / NS) * kXcds + x;
  return r < NR;
}

// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): two MFMAs with (hi, lo) recover
// ~16 mantissa bits of an f32 operand.
__device__ __forceinline__ void split8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    hi[e] = (bf16)x[e];
    lo[e] = (bf16)(x[e] - (float)hi[e]);
  }
}

__device__ __forceinline__ void load8f(const float* p, float* out) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

}  // namespace kda
