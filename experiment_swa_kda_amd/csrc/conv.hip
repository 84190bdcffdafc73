// Depthwise causal short convolution + SiLU (forward and backward) on gfx950.
// Reference: nanochat/mixers/cuda_kda/causal_convolution_forward.cu:42-238 and
// causal_convolution_backward.cu:74-453; semantics nanochat/mixers/kda.py:136-212.
//
// With xp = concat(state[:, :, 1:], x) along time (state holds the W most recent inputs
// including the current token):  pre[t] = sum_j xp[t + j] * w[j],  y = silu(pre),
// final_state = xp[T-1 .. T+W-2].
//
// HBM-bound.  One thread owns 8 consecutive channels (one 16-byte bf16x8 vector) and a
// tile of kTile tokens; adjacent threads own adjacent channel groups so each token row
// [C] bf16 is read with fully coalesced 16-byte loads.  The W-1 token halo is re-read
// from L2.  Arithmetic is f32; products are not rounded to bf16 before accumulation.
// The weight gradient is written as per-tile partials and summed over tiles in a fixed
// order (deterministic, no atomics).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kConvTile = 16;  // tokens per thread

template <int W>
__device__ __forceinline__ void load_xp8(const bf16* __restrict__ x, const bf16* __restrict__ st,
                                         int b, int T, int C, int c0, int p, float* out) {
  // xp[p] for 8 channels: p >= W-1 -> x[p-(W-1)], else state[.., p+1]
  const int t = p - (W - 1);
  if (t >= 0) {
    load8(x + ((size_t)b * T + t) * C + c0, out);
  } else if (st) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = to_f32(st[((size_t)b * C + c0 + e) * W + p + 1]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = 0.f;
  }
}

template <int W>
__global__ __launch_bounds__(256) void conv_fwd_kernel(int B, int T, int C,
                                                       const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ st,
                                                       bf16* __restrict__ y) {
  const int CG = C / 8;
  const int NTB = (T + kConvTile - 1) / kConvTile;
  const long item = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (long)B * NTB * CG) return;
  const int cg = item % CG;
  const int tb = (item / CG) % NTB;
  const int b = item / ((long)CG * NTB);
  const int c0 = cg * 8, t0 = tb * kConvTile;
  float wt[8][W];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) wt[e][j] = to_f32(w[(c0 + e) * W + j]);
  float win[W][8];  // win[j] = xp[t + j] for the current t
#pragma unroll
  for (int j = 0; j < W - 1; ++j) load_xp8<W>(x, st, b, T, C, c0, t0 + j, win[j]);
  const int t1 = min(T, t0 + kConvTile);
  for (int t = t0; t < t1; ++t) {
    load8(x + ((size_t)b * T + t) * C + c0, win[W - 1]);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float pre = 0.f;
#pragma unroll
      for (int j = 0; j < W; ++j) pre = fmaf(win[j][e], wt[e][j], pre);
      o[e] = pre * sigmoid_acc(pre);
    }
    store8(y + ((size_t)b * T + t) * C + c0, o);
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[j][e] = win[j + 1][e];
  }
}

template <int W>
__global__ void conv_final_state_kernel(int B, int T, int C, const bf16* __restrict__ x,
                                        const bf16* __restrict__ st, bf16* __restrict__ fin) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * C * W) return;
  const int j = i % W;
  const int c = (i / W) % C;
  const int b = i / ((long)W * C);
  const int p = T - 1 + j;  // xp position
  const int t = p - (W - 1);
  float val;
  if (t >= 0)
    val = to_f32(x[((size_t)b * T + t) * C + c]);
  else
    val = st ? to_f32(st[((size_t)b * C + c) * W + p + 1]) : 0.f;
  fin[i] = to_bf16(val);
}

__device__ __forceinline__ float silu_grad(float pre) {
  float s = sigmoid_acc(pre);
  return s * (1.f + pre * (1.f - s));
}

template <int W>
__global__ __launch_bounds__(256) void conv_bwd_kernel(int B, int T, int C,
                                                       const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ st,
                                                       const bf16* __restrict__ dy,
                                                       const bf16* __restrict__ dfin,
                                                       bf16* __restrict__ dx,
                                                       float* __restrict__ dw_part) {
  const int CG = C / 8;
  const int NTB = (T + kConvTile - 1) / kConvTile;
  const long item = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (long)B * NTB * CG) return;
  const int cg = item % CG;
  const int tb = (item / CG) % NTB;
  const int b = item / ((long)CG * NTB);
  const int c0 = cg * 8, t0 = tb * kConvTile;
  float wt[8][W];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) wt[e][j] = to_f32(w[(c0 + e) * W + j]);
  float dwacc[8][W];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) dwacc[e][j] = 0.f;

  // dp[j] = dpre[t + j] for the current t (j = 0..W-1); win[j] = xp[s + j] for s = t+W-1
  float dp[W][8];
  float win[W][8];
#pragma unroll
  for (int j = 0; j < W; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) dp[j][e] = 0.f;
  // prime: dpre for tokens t0 .. t0+W-2
#pragma unroll
  for (int j = 0; j < W - 1; ++j) load_xp8<W>(x, st, b, T, C, c0, t0 + j, win[j]);
  const int t1 = min(T, t0 + kConvTile);
  // helper computing dpre at token s given win holding xp[s .. s+W-1]
  auto dpre_at = [&](int s, float* out) {
    if (s >= T) {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = 0.f;
      return;
    }
    float g[8];
    load8(dy + ((size_t)b * T + s) * C + c0, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float pre = 0.f;
#pragma unroll
      for (int j = 0; j < W; ++j) pre = fmaf(win[j][e], wt[e][j], pre);
      out[e] = g[e] * silu_grad(pre);
    }
  };
  // Walk s from t0 to t1+W-2 computing dpre[s]; win slides over xp.
  // dx[t] = sum_j dpre[t+W-1-j] w[j]  (+ grad of final state)
  for (int s = t0; s < t1 + W - 1; ++s) {
    // load xp[s + W - 1]
    if (s < T)
      load8(x + ((size_t)b * T + s) * C + c0, win[W - 1]);
    // dpre at s (zero beyond T)
    float cur[8];
    dpre_at(s, cur);
    if (s < t1) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int j = 0; j < W; ++j) dwacc[e][j] = fmaf(cur[e], win[j][e], dwacc[e][j]);
    }
    // shift dp: dp[j] holds dpre[s - (W-1) + j]
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) dp[j][e] = dp[j + 1][e];
#pragma unroll
    for (int e = 0; e < 8; ++e) dp[W - 1][e] = cur[e];
    const int t = s - (W - 1);
    if (t >= t0) {
      float o[8];
      const int jf = t + W - T;  // final-state slot fed by xp[t+W-1]
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(dp[W - 1 - j][e], wt[e][j], acc);
        if (dfin && jf >= 0 && jf < W) acc += to_f32(dfin[((size_t)b * C + c0 + e) * W + jf]);
        o[e] = acc;
      }
      store8(dx + ((size_t)b * T + t) * C + c0, o);
    }
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[j][e] = win[j + 1][e];
  }
  float* part = dw_part + ((size_t)b * NTB + tb) * C * W;
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) part[(c0 + e) * W + j] = dwacc[e][j];
}

// dweight[c][j] = sum over (b, tile) of partials, fixed order.
__global__ void conv_dw_reduce_kernel(int tiles, int CW, const float* __restrict__ part,
                                      bf16* __restrict__ dw) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= CW) return;
  float acc = 0.f;
  for (int t = 0; t < tiles; ++t) acc += part[(size_t)t * CW + i];
  dw[i] = to_bf16(acc);
}

// dstate[b][c][i] = dxp[i-1] for i >= 1 (0 for i = 0); dxp[p] = sum_j dpre[p-j] w[j]
// plus the final-state gradient when xp[p] is part of the final state (short T).
template <int W>
__global__ void conv_dstate_kernel(int B, int T, int C, const bf16* __restrict__ x,
                                   const bf16* __restrict__ w, const bf16* __restrict__ st,
                                   const bf16* __restrict__ dy, const bf16* __restrict__ dfin,
                                   bf16* __restrict__ dst) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * C) return;
  const int c = i % C;
  const int b = i / C;
  auto xp = [&](int p) -> float {
    int t = p - (W - 1);
    if (t >= 0) return t < T ? to_f32(x[((size_t)b * T + t) * C + c]) : 0.f;
    return to_f32(st[((size_t)b * C + c) * W + p + 1]);
  };
  float wt[W];
#pragma unroll
  for (int j = 0; j < W; ++j) wt[j] = to_f32(w[c * W + j]);
  float dpre[W];
  for (int s = 0; s < W - 1; ++s) {
    if (s < T) {
      float pre = 0.f;
      for (int j = 0; j < W; ++j) pre = fmaf(xp(s + j), wt[j], pre);
      dpre[s] = to_f32(dy[((size_t)b * T + s) * C + c]) * silu_grad(pre);
    } else {
      dpre[s] = 0.f;
    }
  }
  bf16* out = dst + ((size_t)b * C + c) * W;
  out[0] = to_bf16(0.f);
  for (int s = 1; s < W; ++s) {
    const int p = s - 1;
    float acc = 0.f;
    for (int j = 0; j < W; ++j) {
      const int q = p - j;
      if (q >= 0 && q < T) acc = fmaf(dpre[q], wt[j], acc);
    }
    const int jf = p - (T - 1);
    if (dfin && jf >= 0 && jf < W) acc += to_f32(dfin[((size_t)b * C + c) * W + jf]);
    out[s] = to_bf16(acc);
  }
}

template <int W>
static int conv_forward_w(int B, int T, int C, const void* x, const void* w, const void* st,
                          void* y, void* fin, hipStream_t stream) {
  const int NTB = (T + kConvTile - 1) / kConvTile;
  const long items = (long)B * NTB * (C / 8);
  if (items > 0) {
    hipLaunchKernelGGL(conv_fwd_kernel<W>, dim3((items + 255) / 256), dim3(256), 0, stream, B,
                       T, C, (const bf16*)x, (const bf16*)w, (const bf16*)st, (bf16*)y);
    KDA_LAUNCH_CHECK("causal_conv_forward");
  }
  if (fin) {
    const long n = (long)B * C * W;
    hipLaunchKernelGGL(conv_final_state_kernel<W>, dim3((n + 255) / 256), dim3(256), 0, stream,
                       B, T, C, (const bf16*)x, (const bf16*)st, (bf16*)fin);
    KDA_LAUNCH_CHECK("causal_conv_final_state");
  }
  return KDA_OK;
}

template <int W>
static int conv_backward_w(int B, int T, int C, const void* x, const void* w, const void* st,
                           const void* dy, const void* dfin, void* dx, void* dw, void* dst,
                           void* scratch, hipStream_t stream) {
  const int NTB = (T + kConvTile - 1) / kConvTile;
  const long items = (long)B * NTB * (C / 8);
  float* part = (float*)scratch;
  if (items > 0) {
    hipLaunchKernelGGL(conv_bwd_kernel<W>, dim3((items + 255) / 256), dim3(256), 0, stream, B, T,
                       C, (const bf16*)x, (const bf16*)w, (const bf16*)st, (const bf16*)dy,
                       (const bf16*)dfin, (bf16*)dx, part);
    KDA_LAUNCH_CHECK("causal_conv_backward");
  }
  const int CW = C * W;
  hipLaunchKernelGGL(conv_dw_reduce_kernel, dim3((CW + 255) / 256), dim3(256), 0, stream,
                     B * NTB, CW, (const float*)part, (bf16*)dw);
  KDA_LAUNCH_CHECK("causal_conv_dweight_reduce");
  if (dst) {
    const long n = (long)B * C;
    hipLaunchKernelGGL(conv_dstate_kernel<W>, dim3((n + 255) / 256), dim3(256), 0, stream, B, T,
                       C, (const bf16*)x, (const bf16*)w, (const bf16*)st, (const bf16*)dy,
                       (const bf16*)dfin, (bf16*)dst);
    KDA_LAUNCH_CHECK("causal_conv_dstate");
  }
  return KDA_OK;
}

}  // namespace kda

#define KDA_CONV_DISPATCH(W_, CALL) \
  switch (W_) {                     \
    case 1: return CALL(1);         \
    case 2: return CALL(2);         \
    case 3: return CALL(3);         \
    case 4: return CALL(4);         \
    case 5: return CALL(5);         \
    case 6: return CALL(6);         \
    case 7: return CALL(7);         \
    case 8: return CALL(8);         \
    default: break;                 \
  }

extern "C" int kda_causal_conv_forward(int32_t batch, int32_t seq_len, int32_t channels,
                                       int32_t width, const void* x, const void* weight,
                                       const void* initial_state, void* output,
                                       void* final_state, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(batch >= 0 && seq_len >= 0 && channels > 0, "causal_conv_forward: invalid shape");
  KDA_REQUIRE(channels % 8 == 0, "causal_conv_forward: channels must be a multiple of 8");
  KDA_REQUIRE(width >= 1 && width <= 8, "causal_conv_forward: width must be in [1, 8]");
  KDA_REQUIRE(weight && (seq_len == 0 || (x && output)), "causal_conv_forward: null pointer");
#define CALL(W) conv_forward_w<W>(batch, seq_len, channels, x, weight, initial_state, output, final_state, stream)
  KDA_CONV_DISPATCH(width, CALL)
#undef CALL
  return set_error(KDA_ERR_INVALID, "causal_conv_forward: unsupported width");
}

extern "C" size_t kda_causal_conv_backward_scratch_bytes(int32_t batch, int32_t seq_len,
                                                         int32_t channels, int32_t width) {
  const size_t ntb = (size_t)(seq_len + kda::kConvTile - 1) / kda::kConvTile;
  return kda::align256((size_t)batch * ntb * channels * width * sizeof(float)) + 256;
}

extern "C" int kda_causal_conv_backward(int32_t batch, int32_t seq_len, int32_t channels,
                                        int32_t width, const void* x, const void* weight,
                                        const void* initial_state, const void* grad_output,
                                        const void* grad_final_state, void* dx, void* dweight,
                                        void* dinitial_state, void* scratch,
                                        hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(batch >= 0 && seq_len >= 0 && channels > 0, "causal_conv_backward: invalid shape");
  KDA_REQUIRE(channels % 8 == 0, "causal_conv_backward: channels must be a multiple of 8");
  KDA_REQUIRE(width >= 1 && width <= 8, "causal_conv_backward: width must be in [1, 8]");
  KDA_REQUIRE(weight && dweight && scratch, "causal_conv_backward: null pointer");
  KDA_REQUIRE(seq_len == 0 || (x && grad_output && dx), "causal_conv_backward: null pointer");
  KDA_REQUIRE(!dinitial_state || initial_state,
              "causal_conv_backward: dinitial_state requires initial_state");
#define CALL(W) conv_backward_w<W>(batch, seq_len, channels, x, weight, initial_state, grad_output, grad_final_state, dx, dweight, dinitial_state, scratch, stream)
  KDA_CONV_DISPATCH(width, CALL)
#undef CALL
  return set_error(KDA_ERR_INVALID, "causal_conv_backward: unsupported width");
}
