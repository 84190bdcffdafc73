// Depthwise causal short convolution + SiLU (forward and backward) on gfx950.
// Reference: nanochat/mixers/cuda_kda/causal_convolution_forward.cu:42-238 and
// causal_convolution_backward.cu:74-453; semantics nanochat/mixers/kda.py:136-212.
//
// With xp = concat(state[:, :, 1:], x) along time (state holds the W most recent inputs
// including the current token):  pre[t] = sum_j xp[t + j] * w[j],  y = silu(pre),
// final_state = xp[T-1 .. T+W-2].
//
// HBM-bound.  A thread owns 8 consecutive channels (one 16-byte bf16x8 vector) and
// kTok consecutive tokens; a 256-thread workgroup covers kGroups channel groups x
// kSlices token slices, so adjacent lanes read adjacent 16-byte vectors of a token row.
// The W-1 token halo is re-read through L1/L2.  Arithmetic is f32 (products are not
// rounded to bf16 before accumulation).  The weight gradient is reduced inside the
// workgroup through LDS, written as one partial per workgroup and summed over
// workgroups in a fixed order (deterministic, no atomics).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kTok = 4;       // tokens per thread
constexpr int kGroups = 8;    // channel groups (of 8 channels) per workgroup
constexpr int kSlices = 32;   // token slices per workgroup (256 threads)
constexpr int kBlockTok = kTok * kSlices;

struct ConvGeom {
  int B, T, C, CG, ncb, ntb;  // channel groups, channel blocks, token blocks
  __host__ __device__ ConvGeom(int B_, int T_, int C_)
      : B(B_), T(T_), C(C_), CG(C_ / 8), ncb((C_ / 8 + kGroups - 1) / kGroups),
        ntb((T_ + kBlockTok - 1) / kBlockTok) {}
  __host__ __device__ int blocks() const { return B * ntb * ncb; }
};

template <int W>
__device__ __forceinline__ void load_xp8(const bf16* __restrict__ x, const bf16* __restrict__ st,
                                         int b, int T, int C, int c0, int p, float* out) {
  // xp[p] for 8 channels: p >= W-1 -> x[p-(W-1)], else state[.., p+1]
  const int t = p - (W - 1);
  if (t >= 0 && t < T) {
    load8(x + ((size_t)b * T + t) * C + c0, out);
  } else if (t < 0 && st) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = to_f32(st[((size_t)b * C + c0 + e) * W + p + 1]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = 0.f;
  }
}

__device__ __forceinline__ float silu_grad(float pre) {
  float s = sigmoid_acc(pre);
  return s * (1.f + pre * (1.f - s));
}

template <int W>
__global__ __launch_bounds__(256) void conv_fwd_kernel(ConvGeom g, const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ st,
                                                       bf16* __restrict__ y) {
  const int cb = blockIdx.x % g.ncb, tb = (blockIdx.x / g.ncb) % g.ntb, b = blockIdx.x / (g.ncb * g.ntb);
  const int cg = cb * kGroups + threadIdx.x % kGroups;
  const int t0 = tb * kBlockTok + (threadIdx.x / kGroups) * kTok;
  if (cg >= g.CG || t0 >= g.T) return;
  const int c0 = cg * 8;
  float wt[8][W];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) wt[e][j] = to_f32(w[(c0 + e) * W + j]);
  float xp[kTok + W - 1][8];  // xp[t0 .. t0+kTok+W-2]
#pragma unroll
  for (int i = 0; i < kTok + W - 1; ++i) load_xp8<W>(x, st, b, g.T, g.C, c0, t0 + i, xp[i]);
#pragma unroll
  for (int u = 0; u < kTok; ++u) {
    if (t0 + u >= g.T) break;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float pre = 0.f;
#pragma unroll
      for (int j = 0; j < W; ++j) pre = fmaf(xp[u + j][e], wt[e][j], pre);
      o[e] = pre * sigmoid_acc(pre);
    }
    store8(y + ((size_t)b * g.T + t0 + u) * g.C + c0, o);
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

// dx[t] = sum_j dpre[t + W-1-j] w[j] (+ grad of the final state); dpre = dy * silu'(pre).
// dweight[c][j] = sum_t dpre[t] xp[t + j]: per-thread sums over its kTok tokens, reduced
// over the workgroup's token slices in LDS, one partial per workgroup.
template <int W>
__global__ __launch_bounds__(256) void conv_bwd_kernel(ConvGeom g, const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ st,
                                                       const bf16* __restrict__ dy,
                                                       const bf16* __restrict__ dfin,
                                                       bf16* __restrict__ dx,
                                                       float* __restrict__ dw_part) {
  __shared__ float s_dw[256 / kWave][kGroups * 8 * W];
  const int cb = blockIdx.x % g.ncb, tb = (blockIdx.x / g.ncb) % g.ntb, b = blockIdx.x / (g.ncb * g.ntb);
  const int lg = threadIdx.x % kGroups, slice = threadIdx.x / kGroups;
  const int cg = cb * kGroups + lg;
  const int t0 = tb * kBlockTok + slice * kTok;
  float dwacc[8][W];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) dwacc[e][j] = 0.f;
  if (cg < g.CG && t0 < g.T) {
    const int c0 = cg * 8;
    float wt[8][W];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int j = 0; j < W; ++j) wt[e][j] = to_f32(w[(c0 + e) * W + j]);
    // dpre for tokens t0 .. t0+kTok+W-2 needs xp[t0 .. t0+kTok+2W-3]
    constexpr int NP = kTok + W - 1;
    float xp[NP + W - 1][8];
#pragma unroll
    for (int i = 0; i < NP + W - 1; ++i) load_xp8<W>(x, st, b, g.T, g.C, c0, t0 + i, xp[i]);
    float dp[NP][8];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int s = t0 + i;
      if (s < g.T) {
        float gy[8];
        load8(dy + ((size_t)b * g.T + s) * g.C + c0, gy);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float pre = 0.f;
#pragma unroll
          for (int j = 0; j < W; ++j) pre = fmaf(xp[i + j][e], wt[e][j], pre);
          dp[i][e] = gy[e] * silu_grad(pre);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) dp[i][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kTok; ++u) {
      const int t = t0 + u;
      if (t >= g.T) break;
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int j = 0; j < W; ++j) dwacc[e][j] = fmaf(dp[u][e], xp[u + j][e], dwacc[e][j]);
      float o[8];
      const int jf = t + W - g.T;  // final-state slot fed by xp[t+W-1]
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(dp[u + W - 1 - j][e], wt[e][j], acc);
        if (dfin && jf >= 0 && jf < W) acc += to_f32(dfin[((size_t)b * g.C + c0 + e) * W + jf]);
        o[e] = acc;
      }
      store8(dx + ((size_t)b * g.T + t) * g.C + c0, o);
    }
  }
  // reduce the 8 token slices of each wave with shuffles, then the 4 waves through LDS
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) {
      float v = dwacc[e][j];
      v += __shfl_xor(v, 8, kWave);
      v += __shfl_xor(v, 16, kWave);
      v += __shfl_xor(v, 32, kWave);
      if (lane < kGroups) s_dw[wave][(lg * 8 + e) * W + j] = v;
    }
  __syncthreads();
  for (int i = threadIdx.x; i < kGroups * 8 * W; i += 256) {
    float acc = 0.f;
    for (int s = 0; s < 256 / kWave; ++s) acc += s_dw[s][i];
    const int c = cb * kGroups * 8 + i / W;
    if (c < g.C) dw_part[(size_t)(b * g.ntb + tb) * g.C * W + (size_t)c * W + i % W] = acc;
  }
}

// dweight[c][j] = sum over (b, token block) partials.  Workgroup j owns 8 outputs; thread
// (part, i) sums partials part, part + 32, ... in order, then the 32 part-sums are
// combined in order through LDS (deterministic, no atomics).
__global__ __launch_bounds__(256) void conv_dw_reduce_kernel(int tiles, int CW,
                                                             const float* __restrict__ part,
                                                             bf16* __restrict__ dw) {
  __shared__ float s_red[32][8];
  const int i = blockIdx.x * 8 + threadIdx.x % 8, q = threadIdx.x / 8;
  float acc = 0.f;
  if (i < CW)
    for (int t = q; t < tiles; t += 32) acc += part[(size_t)t * CW + i];
  s_red[q][threadIdx.x % 8] = acc;
  __syncthreads();
  if (threadIdx.x < 8 && i < CW) {
    float t = 0.f;
    for (int k = 0; k < 32; ++k) t += s_red[k][threadIdx.x];
    dw[i] = to_bf16(t);
  }
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
  const ConvGeom g(B, T, C);
  if (T > 0 && B > 0) {
    hipLaunchKernelGGL(conv_fwd_kernel<W>, dim3(g.blocks()), dim3(256), 0, stream, g,
                       (const bf16*)x, (const bf16*)w, (const bf16*)st, (bf16*)y);
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
  const ConvGeom g(B, T, C);
  float* part = (float*)scratch;
  const int tiles = B * g.ntb;
  if (T > 0 && B > 0) {
    hipLaunchKernelGGL(conv_bwd_kernel<W>, dim3(g.blocks()), dim3(256), 0, stream, g,
                       (const bf16*)x, (const bf16*)w, (const bf16*)st, (const bf16*)dy,
                       (const bf16*)dfin, (bf16*)dx, part);
    KDA_LAUNCH_CHECK("causal_conv_backward");
  }
  const int CW = C * W;
  hipLaunchKernelGGL(conv_dw_reduce_kernel, dim3((CW + 7) / 8), dim3(256), 0, stream,
                     (T > 0 && B > 0) ? tiles : 0, CW, (const float*)part, (bf16*)dw);
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
  const kda::ConvGeom g(batch, seq_len, channels);
  return kda::align256((size_t)batch * g.ntb * channels * width * sizeof(float)) + 256;
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
