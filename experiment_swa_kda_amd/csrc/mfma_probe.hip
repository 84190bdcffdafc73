// Measurement kernel: the bf16 MFMA throughput this device actually sustains, against which
// the chunk kernels' algorithmic TFLOP/s are also reported (the published dense peak,
// 2.5 PFLOP/s, assumes 2.4 GHz).  Every wave issues kChains independent chains of one MFMA
// shape -- v_mfma_f32_16x16x32_bf16 (16,384 FLOP, the shape the chunk kernels use) or
// v_mfma_f32_32x32x16_bf16 (32,768 FLOP) -- with no memory traffic in the loop; 8
// workgroups of four waves per CU keep every SIMD's matrix unit busy.  Workgroup 0 also
// records the shader-clock cycles and the 100 MHz wall-clock ticks of its loop, from which
// the sustained clock and the cycles per MFMA follow.  No counterpart in the reference.
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kProbeThreads = 256;  // 4 waves
constexpr int kChains = 8;

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int SHAPE>
__global__ __launch_bounds__(kProbeThreads) void mfma_probe_kernel(int iters, float* __restrict__ sink) {
  const int lane = threadIdx.x % kWave;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = to_bf16(0.001f * (lane + e));
    b[e] = to_bf16(0.002f * (lane - e));
  }
  float s = 0.f;
  const long long c0 = clock64(), w0 = wall_clock64();
  if (SHAPE == 0) {
    f32x4 c[kChains];
#pragma unroll
    for (int i = 0; i < kChains; ++i) c[i] = zero4();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < kChains; ++i) c[i] = mfma16(a, b, c[i]);
    }
#pragma unroll
    for (int i = 0; i < kChains; ++i) s += c[i][0] + c[i][1] + c[i][2] + c[i][3];
  } else {
    f32x16 c[kChains / 2];
#pragma unroll
    for (int i = 0; i < kChains / 2; ++i) c[i] = (f32x16)0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < kChains / 2; ++i) c[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[i], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kChains / 2; ++i) s += c[i][0] + c[i][5] + c[i][10] + c[i][15];
  }
  const long long c1 = clock64(), w1 = wall_clock64();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    sink[0] = (float)(c1 - c0);
    sink[1] = (float)(w1 - w0);
  }
  if (s == 1234.5f) sink[2 + blockIdx.x] = s;  // keeps the chains; never true for these inputs
}

}  // namespace kda

extern "C" int kda_mfma_probe(int32_t shape, int32_t workgroups, int32_t iters, float* sink, double* flop,
                              hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE((shape == 0 || shape == 1) && workgroups > 0 && iters > 0 && sink && flop,
              "mfma_probe: invalid arguments");
  if (shape == 0)
    hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(workgroups), dim3(kProbeThreads), 0, stream, iters, sink);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(workgroups), dim3(kProbeThreads), 0, stream, iters, sink);
  KDA_LAUNCH_CHECK("mfma_probe");
  // both shapes: 8 x 16,384 FLOP per wave and iteration (16x16x32: 8 chains; 32x32x16: 4)
  *flop = (double)workgroups * (kProbeThreads / kWave) * kChains * (double)iters * 16384.0;
  return KDA_OK;
}
