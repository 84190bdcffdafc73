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

// Sigmoid from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; each about 1 ulp):
// five VALU instructions, no branch.  For elementwise kernels whose results are rounded to
// bf16, where the accurate form below would make them VALU-bound.  Saturates correctly:
// exp(-x) -> inf gives 0, exp(-x) -> 0 gives 1.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// Full-precision sigmoid used where the value feeds a gradient chain.
__device__ __forceinline__ float sigmoid_acc(float x) {
  if (x >= 0.f) return 1.0f / (1.0f + expf(-x));
  float e = expf(x);
  return e / (1.0f + e);
}

// Cross-lane sums without LDS round trips.  Within a 16-lane row, DPP modifiers fold the
// partner's value into a VALU add (quad_perm, row mirrors, row rotates); across rows,
// gfx950's v_permlane16_swap / v_permlane32_swap exchange whole rows.  Every step adds two
// values commutatively, so all lanes of a group end with bit-identical sums.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
// v(lane) + v(lane ^ 16)
__device__ __forceinline__ float swap16_sum(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
// v(lane) + v(lane ^ 32)
__device__ __forceinline__ float swap32_sum(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
  // sum over aligned groups of W lanes (W power of two, W <= 64), result in every lane
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width");
  if constexpr (W >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (W >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (W >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror: quad 0 <-> quad 1
  if constexpr (W >= 16) v += dpp_mov<0x140>(v); // row_mirror: half-row 0 <-> half-row 1
  if constexpr (W >= 32) v = swap16_sum(v);
  if constexpr (W >= 64) v = swap32_sum(v);
  return v;
}

// Sum over the lanes congruent to this lane modulo S (S in {8, 16, 32, 64}): lanes that
// hold the same column of a [64/S][S] lane grid.  Result in every such lane.
template <int S>
__device__ __forceinline__ float lane_stride_sum(float v) {
  static_assert(S == 8 || S == 16 || S == 32 || S == 64, "stride");
  if constexpr (S <= 8) v += dpp_mov<0x128>(v);  // row_ror:8 within 16 lanes: lane ^ 8
  if constexpr (S <= 16) v = swap16_sum(v);
  if constexpr (S <= 32) v = swap32_sum(v);
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

// MFMA operand fragment holding 8 consecutive rows of one column of a row-major bf16 LDS
// matrix: lane (l % 16, l / 16) gets m[r0 + 8 (l / 16) + e][c0 + l % 16], e = 0..7 (the
// contraction runs down the rows).  Two gfx950 transposing reads ds_read_b64_tr_b16: within
// each 16-lane group, lane j supplies the address of 4 consecutive bf16 and lane i receives
// element i % 4 of lanes i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12; pointing lane j at row
// 8 (l / 16) + j / 4, columns 4 (j % 4).. of the block gives the column fragment.  The pitch
// and c0 must be multiples of 4 elements (8-byte aligned reads).
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef short short8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ bf16x8 lds_col_frag(const bf16* m, int pitch, int r0, int c0, int lane) {
  const int lr = lane % 16, kg = lane / 16;
  const bf16* p = m + (r0 + 8 * kg + lr / 4) * pitch + c0 + 4 * (lr % 4);
  const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)p);
  const short4_t hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(p + 4 * pitch));
  // one whole-vector reinterpretation (element-wise casts of the halves miscompile here)
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Column fragment whose two halves are 4-row groups from different row bases: lane
// (l % 16, l / 16) gets m[ra + 4 (l / 16) + e][c0 + l % 16] for e < 4 and
// m[rb + 4 (l / 16) + e - 4][c0 + l % 16] for e >= 4.
__device__ __forceinline__ bf16x8 lds_col_frag_split(const bf16* m, int pitch, int ra, int rb, int c0, int lane) {
  const int lr = lane % 16, kg = lane / 16;
  const int off = (4 * kg + lr / 4) * pitch + c0 + 4 * (lr % 4);
  const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(m + ra * pitch + off));
  const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(m + rb * pitch + off));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Four-row column fragment (the B operand of a 16-deep MFMA, or an A operand read down a
// column): lane (l % 16, l / 16) gets m[r0 + 4 (l / 16) + e][c0 + l % 16], e = 0..3, from one
// transposing read (same lane mapping as lds_col_frag, four rows per lane group).
__device__ __forceinline__ bf16x4 lds_col_frag4(const bf16* m, int pitch, int r0, int c0, int lane) {
  const int lr = lane % 16, kg = lane / 16;
  const bf16* p = m + (r0 + 4 * kg + lr / 4) * pitch + c0 + 4 * (lr % 4);
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)p));
}

// v_mfma_f32_16x16x16_bf16: A[l % 16][4 (l / 16) + e], B[4 (l / 16) + e][l % 16], C as above.
__device__ __forceinline__ f32x4 mfma16k16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a), __builtin_bit_cast(short4_t, b), c, 0, 0, 0);
}

// 16 bytes per lane from global memory straight into LDS at lds_base + 16 * lane.
__device__ __forceinline__ void dma16(const void* src, char* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt, lgkmcnt left open)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier that orders the surrounding memory accesses for the compiler only; the
// hardware waits the ring protocol needs (vmcnt / lgkmcnt) are issued explicitly.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off inside one launch.  Each XCD has its own L2, so data one
// workgroup stores and a workgroup on another XCD loads must either go through memory with
// system-coherent cache policy (sc0 sc1: stores write through the L2, loads miss in the
// non-coherent caches) or be written back with an agent-scope release (which costs a write-back
// of the XCD's whole L2).  Buffer accesses take a wave-uniform base.
// ---------------------------------------------------------------------------
constexpr int kCoherentPolicy = 1 | 16;  // sc0 | sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// A byte offset beyond raw_rsrc's range: a buffer load from it reads zeros.
constexpr int kDropOffset = (int)0x80000000u;
__device__ __forceinline__ bf16x4 f4_to_bf16x4(float4 x) {
  bf16x4 r;
  r[0] = to_bf16(x.x); r[1] = to_bf16(x.y); r[2] = to_bf16(x.z); r[3] = to_bf16(x.w);
  return r;
}
__device__ __forceinline__ void store8_coherent(void* base, int byte_off, bf16x4 x) {
  typedef int i2 __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i2, x), raw_rsrc(base), byte_off, 0, kCoherentPolicy);
}
__device__ __forceinline__ void store16_coherent(void* base, int byte_off, bf16x8 x) {
  typedef int i4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4, x), raw_rsrc(base), byte_off, 0, kCoherentPolicy);
}
__device__ __forceinline__ bf16x8 load16_coherent_bf16(const void* base, int byte_off) {
  typedef int i4 __attribute__((ext_vector_type(4)));
  const i4 v = __builtin_amdgcn_raw_buffer_load_b128(raw_rsrc(base), byte_off, 0, kCoherentPolicy);
  return __builtin_bit_cast(bf16x8, v);
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

// Weight-gradient finish: out[i] = sum over `parts` partials (row-major [parts][n]),
// launched with kDwRedLanes threads per output.  Lane l of an output loads partials l,
// l + kDwRedLanes, ... (a batch of loads issued before any is added), sums them in order,
// and the lanes combine through group_sum's fixed tree (deterministic, no atomics).
constexpr int kDwRedLanes = 32;
template <typename OutT>
__global__ __launch_bounds__(256) void dw_reduce_kernel(int parts, int n,
                                                        const float* __restrict__ part,
                                                        OutT* __restrict__ out) {
  constexpr int kRedLanes = kDwRedLanes, kBatch = 8;
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int i = gid / kRedLanes, l = gid % kRedLanes;
  const int ic = i < n ? i : n - 1;
  float acc = 0.f;
  for (int p0 = l; p0 < parts; p0 += kBatch * kRedLanes) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int p = p0 + u * kRedLanes;
      v[u] = p < parts ? part[(size_t)p * n + ic] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) acc += v[u];
  }
  acc = group_sum<kRedLanes>(acc);
  if (l == 0 && i < n) out[i] = (OutT)acc;
}

}  // namespace kda
