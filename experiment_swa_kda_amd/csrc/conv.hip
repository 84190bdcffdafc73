// Depthwise causal short convolution + SiLU (forward and backward) on gfx950.
// Reference: nanochat/mixers/cuda_kda/causal_convolution_forward.cu:42-238 and
// causal_convolution_backward.cu:74-453; semantics nanochat/mixers/kda.py:136-212.
//
// With xp = concat(state[:, :, 1:], x) along time (state holds the W most recent inputs
// including the current token):  pre[t] = sum_j xp[t + j] * w[j],  y = silu(pre),
// final_state = xp[T-1 .. T+W-2].
//
// HBM-bound.  A thread owns 8 consecutive channels (one 16-byte bf16x8 vector) and kTok
// consecutive tokens.  A 256-thread workgroup is kCgs channel groups x kSlices token
// slices with the channel group fastest, so each load instruction of a wave covers
// 256 / kCgs contiguous 256-byte row segments.  Every thread issues all of its row loads
// (clamped to valid rows, no branches) before it consumes any of them, so the loads of a
// thread are in flight together; rows outside [0, T) are replaced afterwards by the
// initial state or zero.  The W-1 token halo is re-read through L1/L2.  Arithmetic is
// f32 (products are not rounded to bf16 before accumulation).  The weight gradient is
// reduced inside the workgroup (shuffles, then LDS), written as one partial per
// workgroup and summed over workgroups in a fixed order (deterministic, no atomics).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

// Tile shapes (tokens per thread, channel groups per workgroup); the token slices per
// workgroup are 256 / channel groups.  Overridable at build time for tuning sweeps.
#ifndef KDA_CONV_FWD_TOK
#define KDA_CONV_FWD_TOK 2
#endif
#ifndef KDA_CONV_FWD_CGS
#define KDA_CONV_FWD_CGS 16
#endif
#ifndef KDA_CONV_BWD_TOK
#define KDA_CONV_BWD_TOK 4
#endif
#ifndef KDA_CONV_BWD_CGS
#define KDA_CONV_BWD_CGS 8
#endif

// `halo` is the overlap of consecutive token blocks (the backward's W-1; 0 forward).
template <int TOK, int CGS>
struct ConvGeom {
  static constexpr int kTok = TOK, kCgs = CGS, kSlices = 256 / CGS, kBlockTok = TOK * kSlices;
  int B, T, C, CG, ncb, ntb;  // channel groups, channel blocks, token blocks
  long ldx, ldd;              // row strides (elements per token) of x and of dx (default C)
  __host__ __device__ ConvGeom(int B_, int T_, int C_, int halo = 0)
      : B(B_), T(T_), C(C_), CG(C_ / 8), ncb((C_ / 8 + kCgs - 1) / kCgs),
        ntb((T_ + kBlockTok - halo - 1) / (kBlockTok - halo)), ldx(C_), ldd(C_) {}
  __host__ __device__ int blocks() const { return B * ntb * ncb; }
};
using FwdGeom = ConvGeom<KDA_CONV_FWD_TOK, KDA_CONV_FWD_CGS>;
using BwdGeom = ConvGeom<KDA_CONV_BWD_TOK, KDA_CONV_BWD_CGS>;

// Workgroup -> (batch, token block, channel block); thread -> (channel group, slice).
struct ConvPos {
  int b, tb, cb, cg, slice, t0, c0;
  template <typename G>
  __device__ ConvPos(const G& g) {
    cb = blockIdx.x % g.ncb;
    tb = (blockIdx.x / g.ncb) % g.ntb;
    b = blockIdx.x / (g.ncb * g.ntb);
    cg = cb * G::kCgs + threadIdx.x % G::kCgs;
    slice = threadIdx.x / G::kCgs;
    t0 = tb * G::kBlockTok + slice * G::kTok;
    c0 = cg * 8;
  }
};

// W taps of 8 channels: w[c0 + e][j] = 8*W contiguous bf16 (16-byte aligned, c0 % 8 == 0).
template <int W>
__device__ __forceinline__ void load_taps(const bf16* __restrict__ w, int c0, float (&wt)[8][W]) {
  bf16x8 v[W];
#pragma unroll
  for (int i = 0; i < W; ++i) v[i] = *reinterpret_cast<const bf16x8*>(w + (size_t)c0 * W + 8 * i);
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) wt[e][j] = (float)v[(e * W + j) / 8][(e * W + j) % 8];
}

// N rows of 8 channels of x at tokens t = p0 - (W-1) + i (i < N), i.e. xp[p0 + i].
// issue_xp_row issues one row's load (row index clamped into [0, T-1]); fix_xp_rows then
// replaces rows with t < 0 by the initial state (or zero) and rows with t >= T by zero.
// The fix-up is a per-lane branch that waits for every row it may overwrite, so all other
// loads a thread needs are issued before it (one memory round trip, not two).
template <int W>
__device__ __forceinline__ bf16x8 issue_xp_row(const bf16* __restrict__ x, int b, int T, long ldx, int c0,
                                               int p0, int i) {
  int t = p0 - (W - 1) + i;
  t = t < 0 ? 0 : (t >= T ? T - 1 : t);
  return *reinterpret_cast<const bf16x8*>(x + (size_t)b * T * ldx + c0 + (size_t)t * ldx);
}

template <int W, int N>
__device__ __forceinline__ void fix_xp_rows(const bf16* __restrict__ st, int b, int T, int C, int c0, int p0,
                                            bf16x8 (&raw)[N]) {
  const bf16 zero = (bf16)0.f;
  if (p0 < W - 1 || p0 - (W - 1) + N > T) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int t = p0 - (W - 1) + i;
      if (t < 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          raw[i][e] = st ? st[((size_t)b * C + c0 + e) * W + (p0 + i) + 1] : zero;
      } else if (t >= T) {
#pragma unroll
        for (int e = 0; e < 8; ++e) raw[i][e] = zero;
      }
    }
  }
}

__device__ __forceinline__ float silu_grad(float pre) {
  float s = sigmoid_fast(pre);
  return s * (1.f + pre * (1.f - s));
}

template <int W>
__global__ __launch_bounds__(256) void conv_fwd_kernel(FwdGeom g, const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ st,
                                                       bf16* __restrict__ y) {
  const ConvPos P(g);
  if (P.cg >= g.CG || P.t0 >= g.T) return;
  constexpr int kTok = FwdGeom::kTok;
  constexpr int NX = kTok + W - 1;  // xp[t0 .. t0 + kTok + W - 2]
  // the taps first: every token's arithmetic needs them, and loads complete in order
  float wt[8][W];
  load_taps<W>(w, P.c0, wt);
  bf16x8 xr[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) xr[i] = issue_xp_row<W>(x, P.b, g.T, g.ldx, P.c0, P.t0, i);
  fix_xp_rows<W, NX>(st, P.b, g.T, g.C, P.c0, P.t0, xr);
  bf16* yb = y + ((size_t)P.b * g.T + P.t0) * g.C + P.c0;
#pragma unroll
  for (int u = 0; u < kTok; ++u) {
    if (P.t0 + u >= g.T) break;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float pre = 0.f;
#pragma unroll
      for (int j = 0; j < W; ++j) pre = fmaf((float)xr[u + j][e], wt[e][j], pre);
      o[e] = pre * sigmoid_fast(pre);
    }
    store8(yb + (size_t)u * g.C, o);
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

// Backward.  dpre[s] = dy[s] * silu'(pre[s]);  dx[t] = sum_j dpre[t + W-1-j] w[j] (+ the
// final-state gradient);  dweight[c][j] = sum_s dpre[s] xp[s + j].
// A workgroup computes dpre for a block of kBlockTok tokens (each thread for its own kTok
// tokens: no recomputation inside the block) and shares it through LDS; it writes dx
// and accumulates dweight for the first kOut = kBlockTok - (W-1) tokens, so consecutive
// blocks overlap by the W-1 tokens whose dpre the last outputs need.  dweight is reduced
// over the workgroup (shuffles within a wave, LDS across waves) into one partial per
// workgroup.
template <int W>
__global__ __launch_bounds__(256) void conv_bwd_kernel(BwdGeom g, const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ st,
                                                       const bf16* __restrict__ dy,
                                                       const bf16* __restrict__ dfin,
                                                       bf16* __restrict__ dx,
                                                       float* __restrict__ dw_part) {
  constexpr int kTok = BwdGeom::kTok, kCgs = BwdGeom::kCgs, kBlk = BwdGeom::kBlockTok;
  constexpr int kOut = kBlk - (W - 1);
  static_assert(kWave % kCgs == 0, "a wave must hold whole token slices");
  static_assert(kOut > 0, "token block shorter than the filter");
  // dpre in LDS as [u][half][thread] float4 (u < kTok, half = channels 0-3 / 4-7): a
  // wave's store of one (u, half) is 64 consecutive 16-byte words (no bank conflicts).
  __shared__ __attribute__((aligned(16))) float4 s_dp[kTok * 2 * 256];
  __shared__ float s_dw[256 / kWave][kCgs * 8 * W];
  const int cb = blockIdx.x % g.ncb, tb = (blockIdx.x / g.ncb) % g.ntb;
  const int b = blockIdx.x / (g.ncb * g.ntb);
  const int lg = threadIdx.x % kCgs, slice = threadIdx.x / kCgs;
  const int cg = cb * kCgs + lg, c0 = cg * 8;
  const int l0 = slice * kTok;          // first local token of this thread
  const int s0 = tb * kOut + l0;        // its global token
  const bool active = cg < g.CG;
  float dwacc[8][W];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < W; ++j) dwacc[e][j] = 0.f;
  float wt[8][W];
  if (active) {
    // the taps first (loads complete in order and every token needs them); then
    // dpre[s] for s = s0 .. s0+kTok-1 needs xp[s .. s+W-1], i.e. xp[s0 .. s0+kTok+W-2]
    load_taps<W>(w, c0, wt);
    constexpr int NX = kTok + W - 1;
    bf16x8 xr[NX], gr[kTok];
    // in the order the tokens consume them (loads complete in order): token u needs
    // rows u .. u+W-1 of xp and dy row u
    const bf16* dyb = dy + (size_t)b * g.T * g.C + c0;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) xr[i] = issue_xp_row<W>(x, b, g.T, g.ldx, c0, s0, i);
#pragma unroll
    for (int u = 0; u < kTok; ++u) {
      xr[u + W - 1] = issue_xp_row<W>(x, b, g.T, g.ldx, c0, s0, u + W - 1);
      const int sc = s0 + u < g.T ? s0 + u : g.T - 1;
      gr[u] = *reinterpret_cast<const bf16x8*>(dyb + (size_t)sc * g.C);
    }
    fix_xp_rows<W, NX>(st, b, g.T, g.C, c0, s0, xr);
#pragma unroll
    for (int u = 0; u < kTok; ++u) {
      const bool live = s0 + u < g.T;
      const bool owned = live && l0 + u < kOut;
      float dp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float xv[W];
#pragma unroll
        for (int j = 0; j < W; ++j) xv[j] = (float)xr[u + j][e];
        float pre = 0.f;
#pragma unroll
        for (int j = 0; j < W; ++j) pre = fmaf(xv[j], wt[e][j], pre);
        // computed for every lane, then selected (a conditional expression around the
        // exp/rcp chain compiles to a branch per element, which serialises the chains)
        const float d = (float)gr[u][e] * silu_grad(pre);
        dp[e] = live ? d : 0.f;
        const float dpo = owned ? dp[e] : 0.f;
#pragma unroll
        for (int j = 0; j < W; ++j) dwacc[e][j] = fmaf(dpo, xv[j], dwacc[e][j]);
      }
      s_dp[(u * 2) * 256 + threadIdx.x] = make_float4(dp[0], dp[1], dp[2], dp[3]);
      s_dp[(u * 2 + 1) * 256 + threadIdx.x] = make_float4(dp[4], dp[5], dp[6], dp[7]);
    }
  }
  __syncthreads();
  if (active) {
    // dx for this thread's owned tokens: dpre rows l0 .. l0+kTok+W-2 (all inside the block
    // for owned tokens, since l0 + u < kOut)
    constexpr int ND = kTok + W - 1;
    float dpw[ND][8];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      // local token l0 + i was computed by slice (l0 + i) / kTok as its token (i % kTok)
      int src = threadIdx.x + (i / kTok) * kCgs;
      src = src < 256 ? src : 255;  // only read for tokens a thread does not output
      const float4 a = s_dp[((i % kTok) * 2) * 256 + src];
      const float4 c = s_dp[((i % kTok) * 2 + 1) * 256 + src];
      dpw[i][0] = a.x; dpw[i][1] = a.y; dpw[i][2] = a.z; dpw[i][3] = a.w;
      dpw[i][4] = c.x; dpw[i][5] = c.y; dpw[i][6] = c.z; dpw[i][7] = c.w;
    }
    bf16* dxb = dx + ((size_t)b * g.T + s0) * g.ldd + c0;
#pragma unroll
    for (int u = 0; u < kTok; ++u) {
      const int t = s0 + u;
      if (l0 + u >= kOut || t >= g.T) break;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(dpw[u + W - 1 - j][e], wt[e][j], acc);
        o[e] = acc;
      }
      const int jf = t + W - g.T;  // final-state slot fed by xp[t+W-1]
      if (dfin && jf >= 0 && jf < W) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += to_f32(dfin[((size_t)b * g.C + c0 + e) * W + jf]);
      }
      store8(dxb + (size_t)u * g.ldd, o);
    }
  }
  // the 8 token slices of a wave (lane bits 3-5) summed by halving exchanges: at each
  // step a lane keeps half of its values and adds its partner's copy of that half, so
  // after the lane ^ 8, ^ 16 and ^ 32 steps each lane holds W of the 8W sums (no masked
  // per-value chains); then the waves through LDS, in a fixed order
  static_assert(kCgs == 8, "slice bits are lane bits 3-5");
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  float h1[4 * W], h2[2 * W], h3[W];
  const bool b3 = lane & 8, b4 = lane & 16, b5 = lane & 32;
#pragma unroll
  for (int i = 0; i < 4 * W; ++i) {
    const float lo = dwacc[i / W][i % W], hi = dwacc[(i + 4 * W) / W][(i + 4 * W) % W];
    const float keep = b3 ? hi : lo, give = b3 ? lo : hi;
    h1[i] = keep + dpp_mov<0x128>(give);  // row_ror:8: the value of lane ^ 8
  }
#pragma unroll
  for (int i = 0; i < 2 * W; ++i) {
    // even rows keep h1[i], odd rows h1[i + 2W]; the swap hands each row its partner's half
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, h1[i]),
                                                    __builtin_bit_cast(unsigned, h1[i + 2 * W]), false, false);
    h2[i] = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  }
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, h2[i]),
                                                    __builtin_bit_cast(unsigned, h2[i + W]), false, false);
    h3[i] = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  }
  {
    const int base = (b3 ? 4 * W : 0) + (b4 ? 2 * W : 0) + (b5 ? W : 0);
#pragma unroll
    for (int i = 0; i < W; ++i) s_dw[wave][lg * 8 * W + base + i] = h3[i];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kCgs * 8 * W; i += 256) {
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < 256 / kWave; ++s) acc += s_dw[s][i];
    const int c = cb * kCgs * 8 + i / W;
    if (c < g.C) dw_part[(size_t)(b * g.ntb + tb) * g.C * W + (size_t)c * W + i % W] = acc;
  }
}

// dstate[b][c][i] = dxp[i-1] for i >= 1 (0 for i = 0); dxp[p] = sum_j dpre[p-j] w[j]
// plus the final-state gradient when xp[p] is part of the final state (short T).
template <int W>
__global__ void conv_dstate_kernel(int B, int T, int C, long ldx, const bf16* __restrict__ x,
                                   const bf16* __restrict__ w, const bf16* __restrict__ st,
                                   const bf16* __restrict__ dy, const bf16* __restrict__ dfin,
                                   bf16* __restrict__ dst) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * C) return;
  const int c = i % C;
  const int b = i / C;
  auto xp = [&](int p) -> float {
    int t = p - (W - 1);
    if (t >= 0) return t < T ? to_f32(x[((size_t)b * T + t) * ldx + c]) : 0.f;
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
  const FwdGeom g(B, T, C);
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
static int conv_backward_w(int B, int T, int C, const void* x, long ldx, const void* w, const void* st,
                           const void* dy, const void* dfin, void* dx, long ldd, void* dw, void* dst,
                           void* scratch, hipStream_t stream) {
  BwdGeom g(B, T, C, W - 1);
  g.ldx = ldx;
  g.ldd = ldd;
  float* part = (float*)scratch;
  const int tiles = B * g.ntb;
  if (T > 0 && B > 0) {
    hipLaunchKernelGGL(conv_bwd_kernel<W>, dim3(g.blocks()), dim3(256), 0, stream, g,
                       (const bf16*)x, (const bf16*)w, (const bf16*)st, (const bf16*)dy,
                       (const bf16*)dfin, (bf16*)dx, part);
    KDA_LAUNCH_CHECK("causal_conv_backward");
  }
  const int CW = C * W;
  hipLaunchKernelGGL(dw_reduce_kernel<bf16>, dim3((CW * kDwRedLanes + 255) / 256), dim3(256), 0, stream,
                     (T > 0 && B > 0) ? tiles : 0, CW, (const float*)part, (bf16*)dw);
  KDA_LAUNCH_CHECK("causal_conv_dweight_reduce");
  if (dst) {
    const long n = (long)B * C;
    hipLaunchKernelGGL(conv_dstate_kernel<W>, dim3((n + 255) / 256), dim3(256), 0, stream, B, T,
                       C, ldx, (const bf16*)x, (const bf16*)w, (const bf16*)st, (const bf16*)dy,
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
  KDA_REQUIRE(aligned16(x, weight, output), "causal_conv_forward: x, weight and output must be 16-byte aligned");
#define CALL(W) conv_forward_w<W>(batch, seq_len, channels, x, weight, initial_state, output, final_state, stream)
  KDA_CONV_DISPATCH(width, CALL)
#undef CALL
  return set_error(KDA_ERR_INVALID, "causal_conv_forward: unsupported width");
}

extern "C" size_t kda_causal_conv_backward_scratch_bytes(int32_t batch, int32_t seq_len,
                                                         int32_t channels, int32_t width) {
  if (width < 1 || width > 8) return 256;
  const kda::BwdGeom g(batch, seq_len, channels, width - 1);
  return kda::align256((size_t)batch * g.ntb * channels * width * sizeof(float)) + 256;
}

extern "C" int kda_causal_conv_backward_strided(int32_t batch, int32_t seq_len, int32_t channels,
                                                int32_t width, const void* x, int64_t x_row_stride,
                                                const void* weight, const void* initial_state,
                                                const void* grad_output, const void* grad_final_state,
                                                void* dx, int64_t dx_row_stride, void* dweight,
                                                void* dinitial_state, void* scratch, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(batch >= 0 && seq_len >= 0 && channels > 0, "causal_conv_backward: invalid shape");
  KDA_REQUIRE(channels % 8 == 0, "causal_conv_backward: channels must be a multiple of 8");
  KDA_REQUIRE(width >= 1 && width <= 8, "causal_conv_backward: width must be in [1, 8]");
  KDA_REQUIRE(x_row_stride >= channels && x_row_stride % 8 == 0 && dx_row_stride >= channels &&
                  dx_row_stride % 8 == 0,
              "causal_conv_backward: row strides must be multiples of 8 of at least the channel count");
  KDA_REQUIRE(weight && dweight && scratch, "causal_conv_backward: null pointer");
  KDA_REQUIRE(seq_len == 0 || (x && grad_output && dx), "causal_conv_backward: null pointer");
  KDA_REQUIRE(aligned16(x, weight, grad_output, dx, scratch),
              "causal_conv_backward: x, weight, grad_output, dx and scratch must be 16-byte aligned");
  KDA_REQUIRE(!dinitial_state || initial_state,
              "causal_conv_backward: dinitial_state requires initial_state");
#define CALL(W) conv_backward_w<W>(batch, seq_len, channels, x, x_row_stride, weight, initial_state, grad_output, grad_final_state, dx, dx_row_stride, dweight, dinitial_state, scratch, stream)
  KDA_CONV_DISPATCH(width, CALL)
#undef CALL
  return set_error(KDA_ERR_INVALID, "causal_conv_backward: unsupported width");
}

extern "C" int kda_causal_conv_backward(int32_t batch, int32_t seq_len, int32_t channels,
                                        int32_t width, const void* x, const void* weight,
                                        const void* initial_state, const void* grad_output,
                                        const void* grad_final_state, void* dx, void* dweight,
                                        void* dinitial_state, void* scratch,
                                        hipStream_t stream) {
  return kda_causal_conv_backward_strided(batch, seq_len, channels, width, x, channels, weight, initial_state,
                                          grad_output, grad_final_state, dx, channels, dweight, dinitial_state,
                                          scratch, stream);
}
