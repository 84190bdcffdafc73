// Fused output RMSNorm * weight * sigmoid(gate) over rows of D channels (D = 64 or 128).
// Reference: nanochat/mixers/cuda_kda/rmsnorm_gate.cu:31-184; semantics
// nanochat/mixers/kda.py:46-59 (F.rms_norm(x, weight) * sigmoid(gate)).
//
// HBM-bound.  D/8 lanes own one row (one 16-byte bf16x8 vector each), so a wave covers
// 64/(D/8) rows per pass with coalesced loads and an in-wave shuffle reduction.  The
// grid is a fixed number of workgroups striding over rows, so the per-workgroup weight
// gradient partials are summed in a fixed order (deterministic).  Arithmetic is f32 with
// one rounding to bf16 at the store.
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kNormBlocksMax = 512;

template <int D>
__global__ __launch_bounds__(256) void norm_gate_fwd_kernel(long rows, const bf16* __restrict__ x,
                                                            const bf16* __restrict__ gate,
                                                            const float* __restrict__ weight,
                                                            float eps, bf16* __restrict__ y,
                                                            float* __restrict__ inv_rms) {
  constexpr int LPR = D / 8;
  constexpr int RPB = 256 / LPR;
  const int lane = threadIdx.x % LPR;
  const int c0 = lane * 8;
  float w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = weight[c0 + e];
  for (long r = (long)blockIdx.x * RPB + threadIdx.x / LPR; r < rows; r += (long)gridDim.x * RPB) {
    float xv[8], gv[8], o[8];
    load8(x + r * D + c0, xv);
    load8(gate + r * D + c0, gv);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
    ss = group_sum<LPR>(ss);
    const float inv = rsqrtf(ss / D + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = xv[e] * inv * w[e] * sigmoid_acc(gv[e]);
    store8(y + r * D + c0, o);
    if (lane == 0) inv_rms[r] = inv;
  }
}

template <int D>
__global__ __launch_bounds__(256) void norm_gate_bwd_kernel(
    long rows, const bf16* __restrict__ x, const bf16* __restrict__ gate,
    const float* __restrict__ weight, const float* __restrict__ inv_rms,
    const bf16* __restrict__ dy, bf16* __restrict__ dx, bf16* __restrict__ dgate,
    float* __restrict__ dw_part) {
  constexpr int LPR = D / 8;
  constexpr int RPB = 256 / LPR;
  __shared__ float s_dw[RPB][D + 1];
  const int lane = threadIdx.x % LPR;
  const int slot = threadIdx.x / LPR;
  const int c0 = lane * 8;
  float w[8], dwacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] = weight[c0 + e];
    dwacc[e] = 0.f;
  }
  for (long r = (long)blockIdx.x * RPB + slot; r < rows; r += (long)gridDim.x * RPB) {
    float xv[8], gv[8], g[8], dn[8], n[8], o[8], og[8];
    load8(x + r * D + c0, xv);
    load8(gate + r * D + c0, gv);
    load8(dy + r * D + c0, g);
    const float inv = inv_rms[r];
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s = sigmoid_acc(gv[e]);
      n[e] = xv[e] * inv;
      dn[e] = g[e] * s * w[e];
      dot += dn[e] * n[e];
      og[e] = g[e] * n[e] * w[e] * s * (1.f - s);
      dwacc[e] += g[e] * s * n[e];
    }
    dot = group_sum<LPR>(dot) / D;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = inv * (dn[e] - n[e] * dot);
    store8(dx + r * D + c0, o);
    store8(dgate + r * D + c0, og);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_dw[slot][c0 + e] = dwacc[e];
  __syncthreads();
  if (threadIdx.x < D) {
    float acc = 0.f;
    for (int s = 0; s < RPB; ++s) acc += s_dw[s][threadIdx.x];
    dw_part[(size_t)blockIdx.x * D + threadIdx.x] = acc;
  }
}

// dweight[c] = sum over workgroup partials.  Workgroup j owns 8 channels; thread
// (part, c) sums partials part, part + 32, ... in order and the 32 part-sums are combined
// in order through LDS (deterministic, no atomics).
constexpr int kRedParts = 32;
__global__ __launch_bounds__(256) void norm_dw_reduce_kernel(int blocks, int D,
                                                             const float* __restrict__ part,
                                                             float* __restrict__ dw) {
  __shared__ float s_red[kRedParts][8];
  const int c = blockIdx.x * 8 + threadIdx.x % 8, q = threadIdx.x / 8;
  float acc = 0.f;
  if (c < D)
    for (int b = q; b < blocks; b += kRedParts) acc += part[(size_t)b * D + c];
  s_red[q][threadIdx.x % 8] = acc;
  __syncthreads();
  if (threadIdx.x < 8 && c < D) {
    float t = 0.f;
    for (int k = 0; k < kRedParts; ++k) t += s_red[k][threadIdx.x];
    dw[c] = t;
  }
}

static int norm_blocks(long rows, int dim) {
  const long rpb = 256 / (dim / 8);
  long nb = (rows + rpb - 1) / rpb;
  if (nb > kNormBlocksMax) nb = kNormBlocksMax;
  if (nb < 1) nb = 1;
  return (int)nb;
}

}  // namespace kda

extern "C" int kda_rmsnorm_gate_forward(int64_t rows, int32_t dim, const void* x,
                                        const void* gate, const float* weight, float eps,
                                        void* output, float* inv_rms, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0, "rmsnorm_gate_forward: invalid rows");
  KDA_REQUIRE(dim == 64 || dim == 128, "rmsnorm_gate_forward: dim must be 64 or 128");
  KDA_REQUIRE(eps > 0.f, "rmsnorm_gate_forward: eps must be positive");
  KDA_REQUIRE(weight && (rows == 0 || (x && gate && output && inv_rms)),
              "rmsnorm_gate_forward: null pointer");
  if (rows == 0) return KDA_OK;
  const int nb = norm_blocks(rows, dim);
  if (dim == 128)
    hipLaunchKernelGGL(norm_gate_fwd_kernel<128>, dim3(nb), dim3(256), 0, stream, (long)rows,
                       (const bf16*)x, (const bf16*)gate, weight, eps, (bf16*)output, inv_rms);
  else
    hipLaunchKernelGGL(norm_gate_fwd_kernel<64>, dim3(nb), dim3(256), 0, stream, (long)rows,
                       (const bf16*)x, (const bf16*)gate, weight, eps, (bf16*)output, inv_rms);
  KDA_LAUNCH_CHECK("rmsnorm_gate_forward");
  return KDA_OK;
}

extern "C" size_t kda_rmsnorm_gate_backward_scratch_bytes(int64_t rows, int32_t dim) {
  return kda::align256((size_t)kda::norm_blocks(rows, dim) * dim * sizeof(float)) + 256;
}

extern "C" int kda_rmsnorm_gate_backward(int64_t rows, int32_t dim, const void* x,
                                         const void* gate, const float* weight,
                                         const float* inv_rms, const void* grad_output,
                                         float eps, void* dx, void* dgate, float* dweight,
                                         void* scratch, hipStream_t stream) {
  using namespace kda;
  (void)eps;
  KDA_REQUIRE(rows >= 0, "rmsnorm_gate_backward: invalid rows");
  KDA_REQUIRE(dim == 64 || dim == 128, "rmsnorm_gate_backward: dim must be 64 or 128");
  KDA_REQUIRE(weight && dweight && scratch, "rmsnorm_gate_backward: null pointer");
  KDA_REQUIRE(rows == 0 || (x && gate && inv_rms && grad_output && dx && dgate),
              "rmsnorm_gate_backward: null pointer");
  const int nb = norm_blocks(rows, dim);
  float* part = (float*)scratch;
  if (rows > 0) {
    if (dim == 128)
      hipLaunchKernelGGL(norm_gate_bwd_kernel<128>, dim3(nb), dim3(256), 0, stream, (long)rows,
                         (const bf16*)x, (const bf16*)gate, weight, inv_rms,
                         (const bf16*)grad_output, (bf16*)dx, (bf16*)dgate, part);
    else
      hipLaunchKernelGGL(norm_gate_bwd_kernel<64>, dim3(nb), dim3(256), 0, stream, (long)rows,
                         (const bf16*)x, (const bf16*)gate, weight, inv_rms,
                         (const bf16*)grad_output, (bf16*)dx, (bf16*)dgate, part);
    KDA_LAUNCH_CHECK("rmsnorm_gate_backward");
  }
  hipLaunchKernelGGL(norm_dw_reduce_kernel, dim3((dim + 7) / 8), dim3(256), 0, stream, rows > 0 ? nb : 0, dim,
                     (const float*)part, dweight);
  KDA_LAUNCH_CHECK("rmsnorm_gate_dweight_reduce");
  return KDA_OK;
}
