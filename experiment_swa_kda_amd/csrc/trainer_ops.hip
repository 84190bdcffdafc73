// Elementwise and row-normalisation trainer glue of the all-KDA decoder, fused so each op
// is one pass over HBM.
// Reference: nanochat/gpt.py (the per-layer residual mix x = resid_lambdas[i] x +
// x0_lambdas[i] x0 at :585-587, and the MLP activation relu(x)^2 at :151-156), which the
// reference fuses with torch.compile (scripts/base_train.py:267).
//
// HBM-bound.  Each thread moves 16-byte bf16x8 vectors, kVecs of them in flight, f32 math,
// one rounding to bf16 per output.  The scalar-weight gradients of the residual mix are
// per-workgroup partials summed afterwards in a fixed order (deterministic, no atomics).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kGlueThreads = 256;
constexpr int kGlueVecs = 4;  // bf16x8 vectors per thread
constexpr long kGlueBlock = (long)kGlueThreads * kGlueVecs * 8;  // elements per workgroup

__device__ __forceinline__ void unpack8(const bf16x8& v, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (float)v[e];
}

__device__ __forceinline__ bf16x8 pack8(const float (&f)[8]) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = to_bf16(f[e]);
  return v;
}

// y = a x + b x0 with a = wa[0], b = wb[0] (device scalars)
__global__ __launch_bounds__(kGlueThreads) void resid_mix_fwd_kernel(long n, const float* __restrict__ wa,
                                                                     const float* __restrict__ wb,
                                                                     const bf16* __restrict__ x,
                                                                     const bf16* __restrict__ x0,
                                                                     bf16* __restrict__ y) {
  const float a = wa[0], b = wb[0];
  const long base = (long)blockIdx.x * kGlueBlock + threadIdx.x * 8;
  bf16x8 xv[kGlueVecs], zv[kGlueVecs];
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    const long ic = i < n ? i : 0;
    xv[u] = *reinterpret_cast<const bf16x8*>(x + ic);
    zv[u] = *reinterpret_cast<const bf16x8*>(x0 + ic);
  }
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    float fx[8], fz[8], o[8];
    unpack8(xv[u], fx);
    unpack8(zv[u], fz);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fmaf(a, fx[e], b * fz[e]);
    if (i < n) *reinterpret_cast<bf16x8*>(y + i) = pack8(o);
  }
}

// dx = a g, dx0 = b g; part[block] = {sum g x, sum g x0} over the workgroup's elements
__global__ __launch_bounds__(kGlueThreads) void resid_mix_bwd_kernel(
    long n, const float* __restrict__ wa, const float* __restrict__ wb, const bf16* __restrict__ x,
    const bf16* __restrict__ x0, const bf16* __restrict__ g, bf16* __restrict__ dx,
    bf16* __restrict__ dx0, float* __restrict__ part) {
  __shared__ float red[2][kGlueThreads / kWave];
  const float a = wa[0], b = wb[0];
  const long base = (long)blockIdx.x * kGlueBlock + threadIdx.x * 8;
  bf16x8 xv[kGlueVecs], zv[kGlueVecs], gv[kGlueVecs];
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    const long ic = i < n ? i : 0;
    xv[u] = *reinterpret_cast<const bf16x8*>(x + ic);
    zv[u] = *reinterpret_cast<const bf16x8*>(x0 + ic);
    gv[u] = *reinterpret_cast<const bf16x8*>(g + ic);
  }
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    float fx[8], fz[8], fg[8], ox[8], oz[8];
    unpack8(xv[u], fx);
    unpack8(zv[u], fz);
    unpack8(gv[u], fg);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ox[e] = a * fg[e];
      oz[e] = b * fg[e];
    }
    if (i < n) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sa = fmaf(fg[e], fx[e], sa);
        sb = fmaf(fg[e], fz[e], sb);
      }
      *reinterpret_cast<bf16x8*>(dx + i) = pack8(ox);
      *reinterpret_cast<bf16x8*>(dx0 + i) = pack8(oz);
    }
  }
  sa = wave_sum(sa);
  sb = wave_sum(sb);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    red[0][wave] = sa;
    red[1][wave] = sb;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kGlueThreads / kWave; ++w) t += red[threadIdx.x][w];
    part[(size_t)threadIdx.x * gridDim.x + blockIdx.x] = t;
  }
}

// Both scalar gradients of the residual mix from the per-workgroup partials (rows 0 and 1 of
// `part`), each by one wave in a fixed order, written into vectors of nslots entries: the
// sum at `slot`, zero elsewhere (the gradient of lambda[slot] for a whole lambda vector).
__global__ __launch_bounds__(2 * kWave) void resid_mix_reduce_kernel(int parts, const float* __restrict__ part,
                                                                     int slot, int nslots, float* __restrict__ da,
                                                                     float* __restrict__ db) {
  const int row = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const float* p = part + (size_t)row * parts;
  float acc = 0.f;
  for (int i = lane; i < parts; i += kWave) acc += p[i];
  acc = wave_sum(acc);
  float* out = row == 0 ? da : db;
  for (int j = lane; j < nslots; j += kWave) out[j] = j == slot ? acc : 0.f;
}

// y = relu(x)^2
__global__ __launch_bounds__(kGlueThreads) void relu2_fwd_kernel(long n, const bf16* __restrict__ x,
                                                                 bf16* __restrict__ y) {
  const long base = (long)blockIdx.x * kGlueBlock + threadIdx.x * 8;
  bf16x8 xv[kGlueVecs];
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    xv[u] = *reinterpret_cast<const bf16x8*>(x + (i < n ? i : 0));
  }
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    float f[8];
    unpack8(xv[u], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float r = fmaxf(f[e], 0.f);
      f[e] = r * r;
    }
    if (i < n) *reinterpret_cast<bf16x8*>(y + i) = pack8(f);
  }
}

// dx = 2 relu(x) g
__global__ __launch_bounds__(kGlueThreads) void relu2_bwd_kernel(long n, const bf16* __restrict__ x,
                                                                 const bf16* __restrict__ g,
                                                                 bf16* __restrict__ dx) {
  const long base = (long)blockIdx.x * kGlueBlock + threadIdx.x * 8;
  bf16x8 xv[kGlueVecs], gv[kGlueVecs];
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    const long ic = i < n ? i : 0;
    xv[u] = *reinterpret_cast<const bf16x8*>(x + ic);
    gv[u] = *reinterpret_cast<const bf16x8*>(g + ic);
  }
#pragma unroll
  for (int u = 0; u < kGlueVecs; ++u) {
    const long i = base + (long)u * kGlueThreads * 8;
    float f[8], fg[8];
    unpack8(xv[u], f);
    unpack8(gv[u], fg);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = 2.f * fmaxf(f[e], 0.f) * fg[e];
    if (i < n) *reinterpret_cast<bf16x8*>(dx + i) = pack8(f);
  }
}

inline unsigned glue_blocks(long n) { return (unsigned)((n + kGlueBlock - 1) / kGlueBlock); }

// RMS normalisation without weight over rows of D = 128 J channels (the decoder's norm(),
// F.rms_norm(x, (D,)), nanochat/gpt.py:46-48).  16 lanes own a row, each lane J 16-byte
// vectors (channels 8 l + 128 j), so a wave covers 4 rows with fully coalesced accesses;
// row sums are 16-lane DPP reductions.  Forward writes y and 1/rms per row; backward
//   dx = r (g - y mean(g y)),  r = 1/rms.
constexpr int kNormLanes = 16;
constexpr int kNormRowsPerBlock = 256 / kNormLanes;

// MIX: the normalised row is first formed as s = a x + b x2 (a = wa[0], b = wb[0], 1 where
// the pointer is null), rounded to bf16 and stored -- a residual add or mix fused into the
// norm that follows it.
template <int J, bool MIX = false>
__global__ __launch_bounds__(256) void rms_norm_fwd_kernel(long rows, float eps, const bf16* __restrict__ x,
                                                           bf16* __restrict__ y, float* __restrict__ rinv,
                                                           const bf16* __restrict__ x2 = nullptr,
                                                           const float* __restrict__ wa = nullptr,
                                                           const float* __restrict__ wb = nullptr,
                                                           bf16* __restrict__ s = nullptr) {
  constexpr int D = 128 * J;
  const long row = (long)blockIdx.x * kNormRowsPerBlock + threadIdx.x / kNormLanes;
  const int l = threadIdx.x % kNormLanes;
  const long rc = row < rows ? row : rows - 1;
  bf16x8 xv[J], x2v[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    xv[j] = *reinterpret_cast<const bf16x8*>(x + rc * D + 128 * j + 8 * l);
    if constexpr (MIX) x2v[j] = *reinterpret_cast<const bf16x8*>(x2 + rc * D + 128 * j + 8 * l);
  }
  if constexpr (MIX) {
    const float a = wa ? wa[0] : 1.f, b = wb ? wb[0] : 1.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float fx[8], fz[8], o[8];
      unpack8(xv[j], fx);
      unpack8(x2v[j], fz);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = fmaf(a, fx[e], b * fz[e]);  // as resid_mix_fwd_kernel
      xv[j] = pack8(o);
      if (row < rows) *reinterpret_cast<bf16x8*>(s + row * D + 128 * j + 8 * l) = xv[j];
    }
  }
  float f[J][8], ss = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    unpack8(xv[j], f[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(f[j][e], f[j][e], ss);
  }
  ss = group_sum<kNormLanes>(ss);
  const float r = rsqrtf(ss / D + eps);
  if (row < rows) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f[j][e] * r;
      *reinterpret_cast<bf16x8*>(y + row * D + 128 * j + 8 * l) = pack8(o);
    }
    if (l == 0) rinv[row] = r;
  }
}

// ADD: dx also takes the gradient gadd that reaches x by another path (a residual branch),
// added in f32 before the one rounding.
template <int J, bool ADD = false>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(long rows, const bf16* __restrict__ x,
                                                           const float* __restrict__ rinv,
                                                           const bf16* __restrict__ g, bf16* __restrict__ dx,
                                                           const bf16* __restrict__ gadd = nullptr) {
  constexpr int D = 128 * J;
  const long row = (long)blockIdx.x * kNormRowsPerBlock + threadIdx.x / kNormLanes;
  const int l = threadIdx.x % kNormLanes;
  const long rc = row < rows ? row : rows - 1;
  bf16x8 xv[J], gv[J], av[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    xv[j] = *reinterpret_cast<const bf16x8*>(x + rc * D + 128 * j + 8 * l);
    gv[j] = *reinterpret_cast<const bf16x8*>(g + rc * D + 128 * j + 8 * l);
    if constexpr (ADD) av[j] = *reinterpret_cast<const bf16x8*>(gadd + rc * D + 128 * j + 8 * l);
  }
  const float r = rinv[rc];
  float yf[J][8], gf[J][8], dot = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    unpack8(xv[j], yf[j]);
    unpack8(gv[j], gf[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      yf[j][e] *= r;
      dot = fmaf(gf[j][e], yf[j][e], dot);
    }
  }
  dot = group_sum<kNormLanes>(dot) / D;
  if (row < rows) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = r * (gf[j][e] - yf[j][e] * dot);
      if constexpr (ADD) {
        float fa[8];
        unpack8(av[j], fa);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += fa[e];
      }
      *reinterpret_cast<bf16x8*>(dx + row * D + 128 * j + 8 * l) = pack8(o);
    }
  }
}

}  // namespace kda

#define KDA_GLUE_CHECK(n, ...)                                                              \
  do {                                                                                      \
    KDA_REQUIRE((n) >= 0 && (n) % 8 == 0 && (n) / kda::kGlueBlock < 0x7fffffff,           \
                "elementwise op: length must be a non-negative multiple of 8");             \
    KDA_REQUIRE(kda::aligned16(__VA_ARGS__), "elementwise op: tensors must be 16-byte aligned"); \
  } while (0)

extern "C" size_t kda_resid_mix_backward_scratch_bytes(int64_t n) {
  return n > 0 ? 2 * (size_t)kda::glue_blocks(n) * sizeof(float) : 0;
}

extern "C" int kda_resid_mix_forward(int64_t n, const float* a, const float* b, const void* x,
                                     const void* x0, void* y, hipStream_t stream) {
  using namespace kda;
  KDA_GLUE_CHECK(n, x, x0, y);
  KDA_REQUIRE(a && b && (n == 0 || (x && x0 && y)), "resid_mix_forward: null pointer");
  if (n == 0) return KDA_OK;
  hipLaunchKernelGGL(resid_mix_fwd_kernel, dim3(glue_blocks(n)), dim3(kGlueThreads), 0, stream, (long)n, a,
                     b, (const bf16*)x, (const bf16*)x0, (bf16*)y);
  KDA_LAUNCH_CHECK("resid_mix_forward");
  return KDA_OK;
}

extern "C" int kda_resid_mix_backward(int64_t n, const float* a, const float* b, const void* x,
                                      const void* x0, const void* grad, void* dx, void* dx0,
                                      float* da, float* db, int32_t slot, int32_t nslots, void* scratch,
                                      hipStream_t stream) {
  using namespace kda;
  KDA_GLUE_CHECK(n, x, x0, grad, dx, dx0);
  KDA_REQUIRE(a && b && da && db && (n == 0 || (x && x0 && grad && dx && dx0 && scratch)),
              "resid_mix_backward: null pointer");
  KDA_REQUIRE(nslots >= 1 && slot >= 0 && slot < nslots, "resid_mix_backward: slot out of range");
  const unsigned blocks = n > 0 ? glue_blocks(n) : 0;
  float* part = (float*)scratch;
  if (n > 0) {
    hipLaunchKernelGGL(resid_mix_bwd_kernel, dim3(blocks), dim3(kGlueThreads), 0, stream, (long)n, a, b,
                       (const bf16*)x, (const bf16*)x0, (const bf16*)grad, (bf16*)dx, (bf16*)dx0, part);
    KDA_LAUNCH_CHECK("resid_mix_backward");
  }
  // da = sum of the first row of partials, db of the second (fixed order), one launch
  hipLaunchKernelGGL(resid_mix_reduce_kernel, dim3(1), dim3(2 * kWave), 0, stream, (int)blocks,
                     (const float*)part, (int)slot, (int)nslots, da, db);
  KDA_LAUNCH_CHECK("resid_mix_backward reduce");
  return KDA_OK;
}

#define KDA_NORM_DISPATCH(J_, CALL) \
  switch (J_) {                      \
    case 1: CALL(1); break;          \
    case 2: CALL(2); break;          \
    case 3: CALL(3); break;          \
    case 4: CALL(4); break;          \
    case 6: CALL(6); break;          \
    case 8: CALL(8); break;          \
    default: break;                  \
  }

static bool norm_dim_ok(int32_t dim) {
  const int J = dim / 128;
  return dim > 0 && dim % 128 == 0 && (J <= 4 || J == 6 || J == 8);
}

extern "C" int kda_rms_norm_forward(int64_t rows, int32_t dim, float eps, const void* x, void* y,
                                    float* rinv, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0 && norm_dim_ok(dim), "rms_norm_forward: dim must be 128 x {1,2,3,4,6,8}");
  KDA_REQUIRE(aligned16(x, y), "rms_norm_forward: tensors must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  KDA_REQUIRE(x && y && rinv, "rms_norm_forward: null pointer");
  const unsigned blocks = (unsigned)((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
#define CALL(J) hipLaunchKernelGGL(rms_norm_fwd_kernel<J>, dim3(blocks), dim3(256), 0, stream, (long)rows, eps, \
                                   (const bf16*)x, (bf16*)y, rinv)
  KDA_NORM_DISPATCH(dim / 128, CALL)
#undef CALL
  KDA_LAUNCH_CHECK("rms_norm_forward");
  return KDA_OK;
}

extern "C" int kda_rms_norm_backward(int64_t rows, int32_t dim, const void* x, const float* rinv,
                                     const void* grad, void* dx, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0 && norm_dim_ok(dim), "rms_norm_backward: dim must be 128 x {1,2,3,4,6,8}");
  KDA_REQUIRE(aligned16(x, grad, dx), "rms_norm_backward: tensors must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  KDA_REQUIRE(x && rinv && grad && dx, "rms_norm_backward: null pointer");
  const unsigned blocks = (unsigned)((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
#define CALL(J) hipLaunchKernelGGL(rms_norm_bwd_kernel<J>, dim3(blocks), dim3(256), 0, stream, (long)rows, \
                                   (const bf16*)x, rinv, (const bf16*)grad, (bf16*)dx)
  KDA_NORM_DISPATCH(dim / 128, CALL)
#undef CALL
  KDA_LAUNCH_CHECK("rms_norm_backward");
  return KDA_OK;
}

extern "C" int kda_mix_rms_norm_forward(int64_t rows, int32_t dim, float eps, const float* a, const float* b,
                                        const void* x, const void* x2, void* sum, void* y, float* rinv,
                                        hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0 && norm_dim_ok(dim), "mix_rms_norm_forward: dim must be 128 x {1,2,3,4,6,8}");
  KDA_REQUIRE(aligned16(x, x2, sum, y), "mix_rms_norm_forward: tensors must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  KDA_REQUIRE(x && x2 && sum && y && rinv, "mix_rms_norm_forward: null pointer");
  const unsigned blocks = (unsigned)((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
#define CALL(J) hipLaunchKernelGGL((rms_norm_fwd_kernel<J, true>), dim3(blocks), dim3(256), 0, stream, (long)rows, \
                                   eps, (const bf16*)x, (bf16*)y, rinv, (const bf16*)x2, a, b, (bf16*)sum)
  KDA_NORM_DISPATCH(dim / 128, CALL)
#undef CALL
  KDA_LAUNCH_CHECK("mix_rms_norm_forward");
  return KDA_OK;
}

extern "C" int kda_rms_norm_backward_add(int64_t rows, int32_t dim, const void* x, const float* rinv,
                                         const void* grad, const void* grad_add, void* dx, hipStream_t stream) {
  using namespace kda;
  if (grad_add == nullptr) return kda_rms_norm_backward(rows, dim, x, rinv, grad, dx, stream);
  KDA_REQUIRE(rows >= 0 && norm_dim_ok(dim), "rms_norm_backward: dim must be 128 x {1,2,3,4,6,8}");
  KDA_REQUIRE(aligned16(x, grad, grad_add, dx), "rms_norm_backward: tensors must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  KDA_REQUIRE(x && rinv && grad && dx, "rms_norm_backward: null pointer");
  const unsigned blocks = (unsigned)((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
#define CALL(J) hipLaunchKernelGGL((rms_norm_bwd_kernel<J, true>), dim3(blocks), dim3(256), 0, stream, (long)rows, \
                                   (const bf16*)x, rinv, (const bf16*)grad, (bf16*)dx, (const bf16*)grad_add)
  KDA_NORM_DISPATCH(dim / 128, CALL)
#undef CALL
  KDA_LAUNCH_CHECK("rms_norm_backward");
  return KDA_OK;
}

extern "C" int kda_relu2_forward(int64_t n, const void* x, void* y, hipStream_t stream) {
  using namespace kda;
  KDA_GLUE_CHECK(n, x, y);
  if (n == 0) return KDA_OK;
  KDA_REQUIRE(x && y, "relu2_forward: null pointer");
  hipLaunchKernelGGL(relu2_fwd_kernel, dim3(glue_blocks(n)), dim3(kGlueThreads), 0, stream, (long)n,
                     (const bf16*)x, (bf16*)y);
  KDA_LAUNCH_CHECK("relu2_forward");
  return KDA_OK;
}

extern "C" int kda_relu2_backward(int64_t n, const void* x, const void* grad, void* dx,
                                  hipStream_t stream) {
  using namespace kda;
  KDA_GLUE_CHECK(n, x, grad, dx);
  if (n == 0) return KDA_OK;
  KDA_REQUIRE(x && grad && dx, "relu2_backward: null pointer");
  hipLaunchKernelGGL(relu2_bwd_kernel, dim3(glue_blocks(n)), dim3(kGlueThreads), 0, stream, (long)n,
                     (const bf16*)x, (const bf16*)grad, (bf16*)dx);
  KDA_LAUNCH_CHECK("relu2_backward");
  return KDA_OK;
}

namespace kda {

// ---------------------------------------------------------------------------------------
// Token-embedding gradient (the backward of the decoder's wte lookup, nanochat/gpt.py:559)
// without sorting: dW[v] = sum over tokens t with idx[t] == v of dy[t], summed in token
// order (deterministic, no atomics, no memset).  A workgroup owns kEmbRows vocabulary rows
// and every row of dW it owns is written exactly once (zeros for unseen rows).  It walks
// the token ids in windows of kEmbWindow, compacts the tokens that hit its rows into an
// LDS list in token order (per-thread counts + a fixed-order workgroup scan), then each
// wave accumulates the dy rows of its own rows (wave w owns rows w, w+4, ...) in f32.
// Every workgroup reads the whole id vector (8 B per token, from L2 after the first).
// ---------------------------------------------------------------------------------------
constexpr int kEmbRows = 32;                          // vocabulary rows per workgroup
constexpr int kEmbThreads = 256;                      // 4 waves x 8 rows
constexpr int kEmbPerThread = 8;                      // ids per thread per window
constexpr int kEmbWindow = kEmbThreads * kEmbPerThread;
constexpr int kEmbRowsPerWave = kEmbRows / (kEmbThreads / kWave);
constexpr int kEmbMaxDim = kWave * 8;                 // one 16-byte vector per lane and row

__global__ __launch_bounds__(kEmbThreads) void embedding_bwd_kernel(long n_tok, int vocab, int dim,
                                                                    const int64_t* __restrict__ idx,
                                                                    const bf16* __restrict__ dy,
                                                                    bf16* __restrict__ dw) {
  __shared__ int list[kEmbWindow];   // (token - window start) << 5 | local row
  __shared__ int wave_total[kEmbThreads / kWave];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const long r0 = (long)blockIdx.x * kEmbRows;
  const int nvec = dim / 8;
  const bool active = lane < nvec;
  float acc[kEmbRowsPerWave][8];
#pragma unroll
  for (int r = 0; r < kEmbRowsPerWave; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;

  for (long w0 = 0; w0 < n_tok; w0 += kEmbWindow) {
    // ids of this thread's contiguous run of the window
    int hits[kEmbPerThread];
    int count = 0;
#pragma unroll
    for (int u = 0; u < kEmbPerThread; ++u) {
      const long t = w0 + tid * kEmbPerThread + u;
      const long v = t < n_tok ? (long)idx[t] : -1;
      const long d = v - r0;
      hits[u] = (d >= 0 && d < kEmbRows) ? (int)d : -1;
      count += hits[u] >= 0;
    }
    // exclusive scan of the counts in thread order: wave prefix by shuffles, then the
    // wave totals in order
    int incl = count;
#pragma unroll
    for (int s = 1; s < kWave; s <<= 1) {
      const int o = __shfl_up(incl, s, kWave);
      if (lane >= s) incl += o;
    }
    if (lane == kWave - 1) wave_total[wave] = incl;
    __syncthreads();
    int pos = incl - count, n_list = 0;
#pragma unroll
    for (int w = 0; w < kEmbThreads / kWave; ++w) {
      pos += w < wave ? wave_total[w] : 0;
      n_list += wave_total[w];
    }
#pragma unroll
    for (int u = 0; u < kEmbPerThread; ++u)
      if (hits[u] >= 0) list[pos++] = ((tid * kEmbPerThread + u) << 5) | hits[u];
    __syncthreads();
    // accumulate this wave's rows, four list entries' loads in flight at a time
    for (int e0 = 0; e0 < n_list; e0 += 4) {
      bf16x8 v[4];
      int ent[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        ent[u] = __builtin_amdgcn_readfirstlane(e0 + u < n_list ? list[e0 + u] : -1);
        const bool mine = ent[u] >= 0 && (ent[u] & 31) % (kEmbThreads / kWave) == wave;
        if (mine && active) {
          v[u] = *reinterpret_cast<const bf16x8*>(dy + (w0 + (ent[u] >> 5)) * dim + lane * 8);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[u][e] = to_bf16(0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (ent[u] < 0 || (ent[u] & 31) % (kEmbThreads / kWave) != wave) continue;
        const int rl = (ent[u] & 31) / (kEmbThreads / kWave);
#pragma unroll
        for (int r = 0; r < kEmbRowsPerWave; ++r)
          if (rl == r)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[r][e] += (float)v[u][e];
      }
    }
    __syncthreads();  // the list is rebuilt for the next window
  }
#pragma unroll
  for (int r = 0; r < kEmbRowsPerWave; ++r) {
    const long row = r0 + wave + r * (kEmbThreads / kWave);
    if (row < vocab && active) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_bf16(acc[r][e]);
      *reinterpret_cast<bf16x8*>(dw + row * dim + lane * 8) = o;
    }
  }
}

}  // namespace kda

extern "C" int kda_embedding_backward(int64_t n_tokens, int32_t vocab, int32_t dim, const int64_t* idx,
                                      const void* grad_output, void* grad_weight, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(n_tokens >= 0 && vocab >= 0, "embedding_backward: negative size");
  KDA_REQUIRE(dim > 0 && dim % 8 == 0 && dim <= kEmbMaxDim,
              "embedding_backward: dim must be a positive multiple of 8, at most %d", kEmbMaxDim);
  KDA_REQUIRE(vocab == 0 || grad_weight, "embedding_backward: null grad_weight");
  KDA_REQUIRE(n_tokens == 0 || (idx && grad_output), "embedding_backward: null input");
  KDA_REQUIRE(aligned16(grad_output, grad_weight), "embedding_backward: buffers must be 16-byte aligned");
  if (vocab == 0) return KDA_OK;
  hipLaunchKernelGGL(embedding_bwd_kernel, dim3((unsigned)((vocab + kEmbRows - 1) / kEmbRows)),
                     dim3(kEmbThreads), 0, stream, (long)n_tokens, vocab, dim, idx,
                     (const bf16*)grad_output, (bf16*)grad_weight);
  KDA_LAUNCH_CHECK("embedding_backward");
  return KDA_OK;
}

