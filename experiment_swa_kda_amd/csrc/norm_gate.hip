// Fused output RMSNorm * weight * sigmoid(gate) over rows of D channels (D = 64 or 128).
// Reference: nanochat/mixers/cuda_kda/rmsnorm_gate.cu:31-184; semantics
// nanochat/mixers/kda.py:46-59 (F.rms_norm(x, weight) * sigmoid(gate)).
//
// HBM-bound.  D/8 lanes own one row (one 16-byte bf16x8 vector each); a thread handles
// kRows rows spaced one row-pass apart, so every load instruction of a wave is coalesced
// and all of a thread's loads are issued before any is consumed.  A workgroup owns a
// contiguous block of 256 / (D/8) * kRows rows; reductions over a row are in-wave
// shuffles.  The per-workgroup weight-gradient partials are summed in a fixed order
// (deterministic).  Arithmetic is f32 with one rounding to bf16 at the store.
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kRows = 4;  // rows per thread

template <int D>
__global__ __launch_bounds__(256) void norm_gate_fwd_kernel(long rows, const bf16* __restrict__ x,
                                                            const bf16* __restrict__ gate,
                                                            const float* __restrict__ weight,
                                                            float eps, bf16* __restrict__ y,
                                                            float* __restrict__ inv_rms) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;  // rows per pass of the workgroup
  const int lane = threadIdx.x % LPR;
  const int c0 = lane * 8;
  const long r0 = (long)blockIdx.x * RPP * kRows + threadIdx.x / LPR;
  bf16x8 xr[kRows], gr[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    long r = r0 + (long)i * RPP;
    r = r < rows ? r : rows - 1;
    xr[i] = *reinterpret_cast<const bf16x8*>(x + r * D + c0);
    gr[i] = *reinterpret_cast<const bf16x8*>(gate + r * D + c0);
  }
  float w[8];
  load8f(weight + c0, w);
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const long r = r0 + (long)i * RPP;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf((float)xr[i][e], (float)xr[i][e], ss);
    ss = group_sum<LPR>(ss);
    const float inv = rsqrtf(ss / D + eps);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (float)xr[i][e] * inv * w[e] * sigmoid_fast((float)gr[i][e]);
    if (r < rows) {
      store8(y + r * D + c0, o);
      if (lane == 0) inv_rms[r] = inv;
    }
  }
}

template <int D>
__global__ __launch_bounds__(256) void norm_gate_bwd_kernel(
    long rows, int heads, const bf16* __restrict__ x, const bf16* __restrict__ gate, long gld,
    const float* __restrict__ weight, const float* __restrict__ inv_rms,
    const bf16* __restrict__ dy, bf16* __restrict__ dx, bf16* __restrict__ dgate, long dgld,
    float* __restrict__ dw_part) {
  // row r = (token r / heads, head r % heads); gate and dgate rows of a token are gld / dgld
  // elements apart (heads = 1, gld = dgld = D for dense [rows, D])
  auto goff = [&](long r, long ld) { return (r / heads) * ld + (r % heads) * D; };
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  __shared__ float s_dw[256 / kWave][D];
  const int lane = threadIdx.x % LPR;
  const int c0 = lane * 8;
  const long r0 = (long)blockIdx.x * RPP * kRows + threadIdx.x / LPR;
  bf16x8 xr[kRows], gr[kRows], dr[kRows];
  float ir[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    long r = r0 + (long)i * RPP;
    r = r < rows ? r : rows - 1;
    xr[i] = *reinterpret_cast<const bf16x8*>(x + r * D + c0);
    gr[i] = *reinterpret_cast<const bf16x8*>(gate + goff(r, gld) + c0);
    dr[i] = *reinterpret_cast<const bf16x8*>(dy + r * D + c0);
    ir[i] = inv_rms[r];
  }
  float w[8], dwacc[8];
  load8f(weight + c0, w);
#pragma unroll
  for (int e = 0; e < 8; ++e) dwacc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const long r = r0 + (long)i * RPP;
    const bool live = r < rows;
    const float inv = ir[i];
    float dn[8], n[8], o[8], og[8];
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = live ? (float)dr[i][e] : 0.f;
      const float s = sigmoid_fast((float)gr[i][e]);
      n[e] = (float)xr[i][e] * inv;
      dn[e] = g * s * w[e];
      dot = fmaf(dn[e], n[e], dot);
      og[e] = g * n[e] * w[e] * s * (1.f - s);
      dwacc[e] = fmaf(g * s, n[e], dwacc[e]);
    }
    dot = group_sum<LPR>(dot) / D;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = inv * (dn[e] - n[e] * dot);
    if (live) {
      store8(dx + r * D + c0, o);
      store8(dgate + goff(r, dgld) + c0, og);
    }
  }
  // rows of one channel slot: reduce the wave's kWave/LPR row slots across lanes, then
  // the waves through LDS, in a fixed order
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = dwacc[e];
    v = lane_stride_sum<LPR>(v);
    if (threadIdx.x % kWave < LPR) s_dw[wave][c0 + e] = v;
  }
  __syncthreads();
  if (threadIdx.x < D) {
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < 256 / kWave; ++s) acc += s_dw[s][threadIdx.x];
    dw_part[(size_t)blockIdx.x * D + threadIdx.x] = acc;
  }
}

static int norm_blocks(long rows, int dim) {
  const long rpb = 256 / (dim / 8) * kRows;
  long nb = (rows + rpb - 1) / rpb;
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
  KDA_REQUIRE(aligned16(x, gate, weight, output),
              "rmsnorm_gate_forward: x, gate, weight and output must be 16-byte aligned");
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

extern "C" int kda_rmsnorm_gate_backward_strided(int64_t rows, int32_t dim, int32_t heads, const void* x,
                                                 const void* gate, int64_t gate_row_stride,
                                                 const float* weight, const float* inv_rms,
                                                 const void* grad_output, float eps, void* dx, void* dgate,
                                                 int64_t dgate_row_stride, float* dweight, void* scratch,
                                                 hipStream_t stream) {
  using namespace kda;
  (void)eps;
  KDA_REQUIRE(rows >= 0, "rmsnorm_gate_backward: invalid rows");
  KDA_REQUIRE(dim == 64 || dim == 128, "rmsnorm_gate_backward: dim must be 64 or 128");
  KDA_REQUIRE(heads >= 1 && rows % heads == 0, "rmsnorm_gate_backward: rows must be a multiple of heads >= 1");
  KDA_REQUIRE(gate_row_stride >= (int64_t)heads * dim && gate_row_stride % 8 == 0 &&
                  dgate_row_stride >= (int64_t)heads * dim && dgate_row_stride % 8 == 0,
              "rmsnorm_gate_backward: gate / dgate row strides must be multiples of 8 of at least heads * dim");
  KDA_REQUIRE(weight && dweight && scratch, "rmsnorm_gate_backward: null pointer");
  KDA_REQUIRE(rows == 0 || (x && gate && inv_rms && grad_output && dx && dgate),
              "rmsnorm_gate_backward: null pointer");
  KDA_REQUIRE(aligned16(x, gate, weight, grad_output, dx, dgate, scratch),
              "rmsnorm_gate_backward: x, gate, weight, grad_output, dx, dgate and scratch must be 16-byte aligned");
  const int nb = norm_blocks(rows, dim);
  float* part = (float*)scratch;
  if (rows > 0) {
    if (dim == 128)
      hipLaunchKernelGGL(norm_gate_bwd_kernel<128>, dim3(nb), dim3(256), 0, stream, (long)rows, (int)heads,
                         (const bf16*)x, (const bf16*)gate, (long)gate_row_stride, weight, inv_rms,
                         (const bf16*)grad_output, (bf16*)dx, (bf16*)dgate, (long)dgate_row_stride, part);
    else
      hipLaunchKernelGGL(norm_gate_bwd_kernel<64>, dim3(nb), dim3(256), 0, stream, (long)rows, (int)heads,
                         (const bf16*)x, (const bf16*)gate, (long)gate_row_stride, weight, inv_rms,
                         (const bf16*)grad_output, (bf16*)dx, (bf16*)dgate, (long)dgate_row_stride, part);
    KDA_LAUNCH_CHECK("rmsnorm_gate_backward");
  }
  hipLaunchKernelGGL(dw_reduce_kernel<float>, dim3((dim * kDwRedLanes + 255) / 256), dim3(256), 0, stream,
                     rows > 0 ? nb : 0, dim, (const float*)part, dweight);
  KDA_LAUNCH_CHECK("rmsnorm_gate_dweight_reduce");
  return KDA_OK;
}

extern "C" int kda_rmsnorm_gate_backward(int64_t rows, int32_t dim, const void* x,
                                         const void* gate, const float* weight,
                                         const float* inv_rms, const void* grad_output,
                                         float eps, void* dx, void* dgate, float* dweight,
                                         void* scratch, hipStream_t stream) {
  return kda_rmsnorm_gate_backward_strided(rows, dim, 1, x, gate, dim, weight, inv_rms, grad_output, eps, dx,
                                           dgate, dim, dweight, scratch, stream);
}
