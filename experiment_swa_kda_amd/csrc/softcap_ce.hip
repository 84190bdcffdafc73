// Soft-capped cross entropy over the logits of the trainer's lm_head, fused into one read
// of the bf16 logits forward and one read + one write backward.
//
// Reference: nanochat/gpt.py:600-608 computes, under torch.compile,
//   z = softcap * tanh(float(logits[..., :vocab]) / softcap)
//   loss = cross_entropy(z, targets, ignore_index=-1)    (mean over non-ignored rows)
// which eager PyTorch runs as a chain of full-size f32 passes over an N x vocab tensor.
//
// Because |z| <= softcap, sum_j exp(z_j) <= vocab * e^softcap is finite in f32 for any
// softcap <= 60 and vocab <= 2^24, so the log-sum-exp needs no running maximum: one pass
// sums exp(z) and the backward recomputes z from the logits and the saved lse:
//   d logits_j = g * (exp(z_j - lse) - [j == t]) * (1 - (z_j / softcap)^2)
// with g = dL/dloss / (number of non-ignored rows), read from device memory so that no
// host synchronisation is needed.  Columns vocab..stride-1 (vocabulary padding) get zero
// gradient.  HBM-bound: one workgroup per row, 16-byte vector loads issued kCeBatch at a
// time, row sums reduced in a fixed order (deterministic).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kCeThreads = 256;
constexpr int kCeBatch = 8;  // 16-byte vectors in flight per thread
constexpr float kLog2e = 1.4426950408889634f;

// tanh(x) = 1 - 2 / (e^{2x} + 1) from v_exp_f32 / v_rcp_f32 (each about 1 ulp; absolute
// error ~1e-7).  Saturates to +-1 through exp -> inf / 0.
__device__ __forceinline__ float tanh_fast(float x) {
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(2.0f * kLog2e * x) + 1.0f);
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kCeThreads / kWave; ++w) s += red[w];
  return s;
}

__global__ __launch_bounds__(kCeThreads) void softcap_ce_fwd_kernel(
    int vocab, long stride, float cap, const bf16* __restrict__ logits,
    const int64_t* __restrict__ targets, int64_t ignore_index, float* __restrict__ loss_row,
    float* __restrict__ lse_row) {
  __shared__ float red[kCeThreads / kWave];
  const long row = blockIdx.x;
  const bf16* p = logits + row * stride;
  const float inv_cap = 1.0f / cap;
  const int last = ((vocab - 1) / 8) * 8;  // last vector start that holds a vocabulary column
  float sum = 0.f;
  for (int base = 0; base < vocab; base += kCeThreads * 8 * kCeBatch) {
    bf16x8 x[kCeBatch];
#pragma unroll
    for (int b = 0; b < kCeBatch; ++b) {
      const int c = base + (b * kCeThreads + threadIdx.x) * 8;
      x[b] = *reinterpret_cast<const bf16x8*>(p + (c < last ? c : last));
    }
#pragma unroll
    for (int b = 0; b < kCeBatch; ++b) {
      const int c = base + (b * kCeThreads + threadIdx.x) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float z = cap * tanh_fast((float)x[b][e] * inv_cap);
        const float ez = __builtin_amdgcn_exp2f(kLog2e * z);
        sum += (c + e < vocab) ? ez : 0.f;
      }
    }
  }
  sum = block_sum(sum, red);
  if (threadIdx.x == 0) {
    const float lse = __logf(sum);
    const int64_t t = targets[row];
    float loss;
    if (t == ignore_index) {
      loss = 0.f;
    } else if (t < 0 || t >= vocab) {
      loss = __builtin_nanf("");  // out-of-range target: poison the mean
    } else {
      loss = lse - cap * tanh_fast((float)p[t] * inv_cap);
    }
    loss_row[row] = loss;
    lse_row[row] = lse;
  }
}

__global__ __launch_bounds__(kCeThreads) void softcap_ce_bwd_kernel(
    int vocab, long stride, float cap, const bf16* __restrict__ logits,
    const int64_t* __restrict__ targets, int64_t ignore_index, const float* __restrict__ lse_row,
    const float* __restrict__ grad_scale, bf16* __restrict__ grad) {
  const long row = blockIdx.x;
  const bf16* p = logits + row * stride;
  bf16* q = grad + row * stride;
  const float inv_cap = 1.0f / cap;
  const int64_t t = targets[row];
  const float g = (t == ignore_index) ? 0.f : *grad_scale;
  const float lse = lse_row[row];
  const int tc = (t >= 0 && t < vocab) ? (int)t : -1;
  for (long base = 0; base < stride; base += kCeThreads * 8 * kCeBatch) {
    bf16x8 x[kCeBatch];
#pragma unroll
    for (int b = 0; b < kCeBatch; ++b) {
      const long c = base + (b * kCeThreads + threadIdx.x) * 8;
      x[b] = *reinterpret_cast<const bf16x8*>(p + (c < stride ? c : stride - 8));
    }
#pragma unroll
    for (int b = 0; b < kCeBatch; ++b) {
      const long c = base + (b * kCeThreads + threadIdx.x) * 8;
      bf16x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float th = tanh_fast((float)x[b][e] * inv_cap);
        const float pr = __builtin_amdgcn_exp2f(kLog2e * (cap * th - lse));
        const float d = g * (pr - (c + e == tc ? 1.0f : 0.0f)) * (1.0f - th * th);
        y[e] = to_bf16(c + e < vocab ? d : 0.f);
      }
      if (c < stride) *reinterpret_cast<bf16x8*>(q + c) = y;
    }
  }
}

}  // namespace kda

static int check_ce_args(int64_t rows, int32_t vocab, int64_t stride, float softcap,
                         const void* logits, const void* targets) {
  KDA_REQUIRE(rows >= 0 && rows <= 0x7fffffff, "softcap_cross_entropy: invalid row count");
  KDA_REQUIRE(vocab > 0 && vocab <= (1 << 24), "softcap_cross_entropy: vocab must be in [1, 2^24]");
  KDA_REQUIRE(stride >= vocab && stride % 8 == 0,
              "softcap_cross_entropy: row stride must be >= vocab and a multiple of 8");
  KDA_REQUIRE(softcap > 0.f && softcap <= 60.f, "softcap_cross_entropy: softcap must be in (0, 60]");
  KDA_REQUIRE(logits && targets, "softcap_cross_entropy: null pointer");
  KDA_REQUIRE(kda::aligned16(logits), "softcap_cross_entropy: logits must be 16-byte aligned");
  return KDA_OK;
}

extern "C" int kda_softcap_cross_entropy_forward(int64_t rows, int32_t vocab, int64_t stride,
                                                 float softcap, const void* logits,
                                                 const int64_t* targets, int64_t ignore_index,
                                                 float* loss_rows, float* lse_rows,
                                                 hipStream_t stream) {
  using namespace kda;
  int rc = check_ce_args(rows, vocab, stride, softcap, logits, targets);
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(loss_rows && lse_rows, "softcap_cross_entropy_forward: null output");
  if (rows == 0) return KDA_OK;
  hipLaunchKernelGGL(softcap_ce_fwd_kernel, dim3((unsigned)rows), dim3(kCeThreads), 0, stream, vocab,
                     (long)stride, softcap, (const bf16*)logits, targets, ignore_index, loss_rows,
                     lse_rows);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_forward");
  return KDA_OK;
}

extern "C" int kda_softcap_cross_entropy_backward(int64_t rows, int32_t vocab, int64_t stride,
                                                  float softcap, const void* logits,
                                                  const int64_t* targets, int64_t ignore_index,
                                                  const float* lse_rows, const float* grad_scale,
                                                  void* grad_logits, hipStream_t stream) {
  using namespace kda;
  int rc = check_ce_args(rows, vocab, stride, softcap, logits, targets);
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(lse_rows && grad_scale && grad_logits, "softcap_cross_entropy_backward: null pointer");
  KDA_REQUIRE(aligned16(grad_logits), "softcap_cross_entropy_backward: grad must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  hipLaunchKernelGGL(softcap_ce_bwd_kernel, dim3((unsigned)rows), dim3(kCeThreads), 0, stream, vocab,
                     (long)stride, softcap, (const bf16*)logits, targets, ignore_index, lse_rows,
                     grad_scale, (bf16*)grad_logits);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_backward");
  return KDA_OK;
}

namespace kda {

// Mean of the row losses over the rows whose target is not ignore_index, and that count,
// in one workgroup with a fixed summation order (thread t sums rows t, t + 1024, ...; then
// a fixed tree).  Keeps the loss reduction inside the library: a multi-block library
// reduction would record memory-set nodes when captured in a HIP graph.
constexpr int kMeanThreads = 1024;

__global__ __launch_bounds__(kMeanThreads) void softcap_ce_mean_kernel(
    long rows, const float* __restrict__ loss_row, const int64_t* __restrict__ targets,
    int64_t ignore_index, float* __restrict__ loss, float* __restrict__ count) {
  __shared__ float red_s[kMeanThreads / kWave], red_c[kMeanThreads / kWave];
  float s = 0.f, c = 0.f;
  for (long r = threadIdx.x; r < rows; r += kMeanThreads) {
    const bool valid = targets[r] != ignore_index;
    s += valid ? loss_row[r] : 0.f;
    c += valid ? 1.f : 0.f;
  }
  s = wave_sum(s);
  c = wave_sum(c);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    red_s[wave] = s;
    red_c[wave] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float ts = 0.f, tc = 0.f;
    for (int w = 0; w < kMeanThreads / kWave; ++w) {
      ts += red_s[w];
      tc += red_c[w];
    }
    *loss = ts / tc;  // NaN when every row is ignored, as the library cross entropy
    *count = tc;
  }
}

}  // namespace kda

extern "C" int kda_softcap_cross_entropy_mean(int64_t rows, const float* loss_rows, const int64_t* targets,
                                              int64_t ignore_index, float* loss, float* count,
                                              hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0, "softcap_cross_entropy_mean: negative row count");
  KDA_REQUIRE(loss && count && (rows == 0 || (loss_rows && targets)),
              "softcap_cross_entropy_mean: null pointer");
  hipLaunchKernelGGL(softcap_ce_mean_kernel, dim3(1), dim3(kMeanThreads), 0, stream, (long)rows, loss_rows,
                     targets, ignore_index, loss, count);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_mean");
  return KDA_OK;
}
