// Fused output RMSNorm * weight * sigmoid(gate) over rows of D channels (D = 64 or 128 on
// the vector kernels below; any D <= 1024 on the one-wave-per-row kernels).
// Reference: nanochat/mixers/cuda_kda/rmsnorm_gate.cu:31-184; semantics
// nanochat/mixers/kda.py:46-59 (F.rms_norm(x, weight) * sigmoid(gate)).
//
// HBM-bound.  D/8 lanes own one row (one 16-byte bf16x8 vector each); a thread handles
// a few rows (kRowsFwd, kRowsBwd) spaced one row-pass apart, so every load instruction of a wave is coalesced
// and all of a thread's loads are issued before any is consumed.  A workgroup owns a
// contiguous block of 256 / (D/8) rows per row pass; reductions over a row are in-wave
// shuffles.  The per-workgroup weight-gradient partials are summed in a fixed order
// (deterministic).  Arithmetic is f32 with one rounding to bf16 at the store.
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

// Rows per thread.  Forward: 1, 16 rows per workgroup at D = 128 (1,536 workgroups for the
// 24,576 rows of B2 T4096 H3; measured 3.5 us against 3.7 with 2, 4.0 with 3, 4.5 with 4).
// Backward: 768 threads x 2 rows, 96 rows per workgroup (one workgroup per CU, 12 waves),
// and half the weight-gradient partials for the reduction launch (measured at config 2:
// 8.98 us against 9.06 with 512 x 3, 9.3 with 256 x 6 or 1024 x 2, 10.2 with 256 x 3).
// Summing the partials in the launch itself (the last workgroup to finish, counted by one
// atomic word) was slower than the separate launch: 11.7 us.
#ifndef KDA_NORM_ROWS_FWD
#define KDA_NORM_ROWS_FWD 1
#endif
#ifndef KDA_NORM_ROWS_BWD
#define KDA_NORM_ROWS_BWD 2
#endif
#ifndef KDA_NORM_BWD_THREADS
#define KDA_NORM_BWD_THREADS 768
#endif
constexpr int kRowsFwd = KDA_NORM_ROWS_FWD, kRowsBwd = KDA_NORM_ROWS_BWD, kBwdThreads = KDA_NORM_BWD_THREADS;

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
  const long r0 = (long)blockIdx.x * RPP * kRowsFwd + threadIdx.x / LPR;
  // the weight first: loads complete in order, and every row's arithmetic needs it
  float w[8];
  load8f(weight + c0, w);
  bf16x8 xr[kRowsFwd], gr[kRowsFwd];
#pragma unroll
  for (int i = 0; i < kRowsFwd; ++i) {
    long r = r0 + (long)i * RPP;
    r = r < rows ? r : rows - 1;
    xr[i] = *reinterpret_cast<const bf16x8*>(x + r * D + c0);
    gr[i] = *reinterpret_cast<const bf16x8*>(gate + r * D + c0);
  }
  // every row load issued before any use: left alone, the compiler sinks a gate row's load
  // into the row's store branch (its only use), behind the wait for the earlier rows -- a
  // second memory round trip.  The empty asm "uses" the gate rows here.
#pragma unroll
  for (int i = 0; i < kRowsFwd; ++i) asm volatile("" : "+v"(gr[i]));
#pragma unroll
  for (int i = 0; i < kRowsFwd; ++i) {
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
__global__ __launch_bounds__(kBwdThreads) void norm_gate_bwd_kernel(
    long rows, int heads, const bf16* __restrict__ x, const bf16* __restrict__ gate, long gld,
    const float* __restrict__ weight, const float* __restrict__ inv_rms,
    const bf16* __restrict__ dy, bf16* __restrict__ dx, bf16* __restrict__ dgate, long dgld,
    float* __restrict__ dw_part) {
  // row r = (token r / heads, head r % heads); gate and dgate rows of a token are gld / dgld
  // elements apart (heads = 1, gld = dgld = D for dense [rows, D]).  32-bit division by the
  // uniform head count (rows < 2^31): a 64-bit division expands to a long branchy sequence
  // per row that sat between the row loads.
  auto goff = [&](long r, long ld) {
    const unsigned tok = (unsigned)r / (unsigned)heads;
    return (long)tok * ld + (long)((unsigned)r - tok * (unsigned)heads) * D;
  };
  constexpr int LPR = D / 8;
  constexpr int RPP = kBwdThreads / LPR;
  __shared__ float s_dw[kBwdThreads / kWave][D];
  const int lane = threadIdx.x % LPR;
  const int c0 = lane * 8;
  const long r0 = (long)blockIdx.x * RPP * kRowsBwd + threadIdx.x / LPR;
  // the weight and the rows' 1/rms first (loads complete in order; row i's arithmetic
  // then waits only for its own three vectors)
  float w[8], dwacc[8];
  load8f(weight + c0, w);
  float ir[kRowsBwd];
#pragma unroll
  for (int i = 0; i < kRowsBwd; ++i) {
    const long r = r0 + (long)i * RPP;
    ir[i] = inv_rms[r < rows ? r : rows - 1];
  }
  bf16x8 xr[kRowsBwd], gr[kRowsBwd], dr[kRowsBwd];
#pragma unroll
  for (int i = 0; i < kRowsBwd; ++i) {
    long r = r0 + (long)i * RPP;
    r = r < rows ? r : rows - 1;
    xr[i] = *reinterpret_cast<const bf16x8*>(x + r * D + c0);
    gr[i] = *reinterpret_cast<const bf16x8*>(gate + goff(r, gld) + c0);
    dr[i] = *reinterpret_cast<const bf16x8*>(dy + r * D + c0);
  }
  __builtin_amdgcn_sched_barrier(0);  // every row load issued before any use (as above)
#pragma unroll
  for (int e = 0; e < 8; ++e) dwacc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < kRowsBwd; ++i) {
    const long r = r0 + (long)i * RPP;
    const bool live = r < rows;
    const float inv = ir[i];
    // with gs = dy s, dn = gs w, t = dn n:  dgate = t (1 - s),  dw += gs n,
    // dx = inv (dn - n mean(t))
    float dn[8], n[8], o[8], og[8];
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = live ? (float)dr[i][e] : 0.f;
      const float s = sigmoid_fast((float)gr[i][e]);
      const float gs = g * s;
      n[e] = (float)xr[i][e] * inv;
      dn[e] = gs * w[e];
      const float t = dn[e] * n[e];
      dot += t;
      og[e] = fmaf(-t, s, t);
      dwacc[e] = fmaf(gs, n[e], dwacc[e]);
    }
    dot = group_sum<LPR>(dot) * (1.0f / D);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = inv * fmaf(-n[e], dot, dn[e]);
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
    for (int s = 0; s < kBwdThreads / kWave; ++s) acc += s_dw[s][threadIdx.x];
    dw_part[(size_t)blockIdx.x * D + threadIdx.x] = acc;
  }
}

// Any other row width D <= 1024 (the reference takes any): one wave per row, lane l owning
// channels l + 64 i (scalar bf16 accesses), wave-wide sums.  The backward's workgroups
// stride over the rows and leave one weight-gradient partial each (kGenNormBlocks at most).
constexpr int kGenNormMaxD = 1024;
constexpr int kGenNormBlocks = 512;

template <int NI>
__global__ __launch_bounds__(256) void norm_gate_fwd_generic_kernel(long rows, int D, const bf16* __restrict__ x,
                                                                    const bf16* __restrict__ gate,
                                                                    const float* __restrict__ weight, float eps,
                                                                    bf16* __restrict__ y, float* __restrict__ inv_rms) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const long r = (long)blockIdx.x * 4 + wave;
  if (r >= rows) return;  // whole wave
  float xv[NI], gv[NI], ss = 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int c = lane + 64 * i;
    xv[i] = c < D ? (float)x[r * D + c] : 0.f;
    gv[i] = c < D ? (float)gate[r * D + c] : 0.f;
    ss = fmaf(xv[i], xv[i], ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / D + eps);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int c = lane + 64 * i;
    if (c < D) y[r * D + c] = to_bf16(xv[i] * inv * weight[c] * sigmoid_fast(gv[i]));
  }
  if (lane == 0) inv_rms[r] = inv;
}

template <int NI>
__global__ __launch_bounds__(256) void norm_gate_bwd_generic_kernel(
    long rows, int D, int heads, const bf16* __restrict__ x, const bf16* __restrict__ gate, long gld,
    const float* __restrict__ weight, const float* __restrict__ inv_rms, const bf16* __restrict__ dy,
    bf16* __restrict__ dx, bf16* __restrict__ dgate, long dgld, float* __restrict__ dw_part) {
  __shared__ float s_dw[4][kGenNormMaxD];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  float dwacc[NI], w[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int c = lane + 64 * i;
    dwacc[i] = 0.f;
    w[i] = c < D ? weight[c] : 0.f;
  }
  for (long r = (long)blockIdx.x * 4 + wave; r < rows; r += (long)gridDim.x * 4) {
    const long tok = r / heads, hh = r - tok * heads;
    const long go = tok * gld + hh * D, dgo = tok * dgld + hh * D;
    const float inv = inv_rms[r];
    float n[NI], dn[NI], s[NI], gs[NI], dot = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int c = lane + 64 * i;
      const bool ok = c < D;
      const float g = ok ? (float)dy[r * D + c] : 0.f;
      s[i] = ok ? sigmoid_fast((float)gate[go + c]) : 0.f;
      n[i] = ok ? (float)x[r * D + c] * inv : 0.f;
      gs[i] = g * s[i];
      dn[i] = gs[i] * w[i];
      dot = fmaf(dn[i], n[i], dot);
      dwacc[i] = fmaf(gs[i], n[i], dwacc[i]);
    }
    dot = wave_sum(dot) / D;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int c = lane + 64 * i;
      if (c < D) {
        const float t = dn[i] * n[i];
        dx[r * D + c] = to_bf16(inv * fmaf(-n[i], dot, dn[i]));
        dgate[dgo + c] = to_bf16(fmaf(-t, s[i], t));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NI; ++i)
    if (lane + 64 * i < D) s_dw[wave][lane + 64 * i] = dwacc[i];
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += 256)
    dw_part[(size_t)blockIdx.x * D + c] = ((s_dw[0][c] + s_dw[1][c]) + s_dw[2][c]) + s_dw[3][c];
}

static int gen_norm_ni(int D) { return D <= 64 ? 1 : D <= 128 ? 2 : D <= 256 ? 4 : D <= 512 ? 8 : 16; }

static int gen_norm_blocks(long rows) {
  const long nb = (rows + 3) / 4;
  return (int)(nb < 1 ? 1 : (nb > kGenNormBlocks ? kGenNormBlocks : nb));
}

#define KDA_GEN_NORM_DISPATCH(D_, CALL) \
  switch (gen_norm_ni(D_)) {            \
    case 1: CALL(1); break;             \
    case 2: CALL(2); break;             \
    case 4: CALL(4); break;             \
    case 8: CALL(8); break;             \
    default: CALL(16); break;           \
  }

static bool fast_dim(int dim) { return dim == 64 || dim == 128; }

static int norm_blocks(long rows, int dim, int rows_per_thread, int threads = 256) {
  const long rpb = threads / (dim / 8) * rows_per_thread;
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
  KDA_REQUIRE(dim >= 1 && dim <= kGenNormMaxD, "rmsnorm_gate_forward: dim must be in [1, %d]", kGenNormMaxD);
  KDA_REQUIRE(eps > 0.f, "rmsnorm_gate_forward: eps must be positive");
  KDA_REQUIRE(weight && (rows == 0 || (x && gate && output && inv_rms)),
              "rmsnorm_gate_forward: null pointer");
  KDA_REQUIRE(!fast_dim(dim) || aligned16(x, gate, weight, output),
              "rmsnorm_gate_forward: x, gate, weight and output must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  if (!fast_dim(dim)) {
#define KDA_GEN_NORM_FWD(NI)                                                                                  \
  hipLaunchKernelGGL(norm_gate_fwd_generic_kernel<NI>, dim3((rows + 3) / 4), dim3(256), 0, stream, (long)rows, \
                     (int)dim, (const bf16*)x, (const bf16*)gate, weight, eps, (bf16*)output, inv_rms)
    KDA_GEN_NORM_DISPATCH(dim, KDA_GEN_NORM_FWD)
#undef KDA_GEN_NORM_FWD
    KDA_LAUNCH_CHECK("rmsnorm_gate_forward");
    return KDA_OK;
  }
  const int nb = norm_blocks(rows, dim, kRowsFwd);
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
  if (dim < 1 || dim > kda::kGenNormMaxD) return 0;
  const size_t nb = kda::fast_dim(dim) ? kda::norm_blocks(rows, dim, kda::kRowsBwd, kda::kBwdThreads) : kda::gen_norm_blocks(rows);
  return kda::align256(nb * dim * sizeof(float)) + 256;
}

extern "C" int kda_rmsnorm_gate_backward_strided(int64_t rows, int32_t dim, int32_t heads, const void* x,
                                                 const void* gate, int64_t gate_row_stride,
                                                 const float* weight, const float* inv_rms,
                                                 const void* grad_output, float eps, void* dx, void* dgate,
                                                 int64_t dgate_row_stride, float* dweight, void* scratch,
                                                 hipStream_t stream) {
  using namespace kda;
  (void)eps;
  KDA_REQUIRE(rows >= 0 && rows < (1LL << 31), "rmsnorm_gate_backward: rows must be in [0, 2^31)");
  KDA_REQUIRE(dim >= 1 && dim <= kGenNormMaxD, "rmsnorm_gate_backward: dim must be in [1, %d]", kGenNormMaxD);
  KDA_REQUIRE(heads >= 1 && rows % heads == 0, "rmsnorm_gate_backward: rows must be a multiple of heads >= 1");
  KDA_REQUIRE(gate_row_stride >= (int64_t)heads * dim && dgate_row_stride >= (int64_t)heads * dim &&
                  (!fast_dim(dim) || (gate_row_stride % 8 == 0 && dgate_row_stride % 8 == 0)),
              "rmsnorm_gate_backward: gate / dgate row strides must be at least heads * dim (multiples of 8 "
              "for dim 64 / 128)");
  KDA_REQUIRE(weight && dweight && scratch, "rmsnorm_gate_backward: null pointer");
  KDA_REQUIRE(rows == 0 || (x && gate && inv_rms && grad_output && dx && dgate),
              "rmsnorm_gate_backward: null pointer");
  KDA_REQUIRE(aligned16(scratch) && (!fast_dim(dim) || aligned16(x, gate, weight, grad_output, dx, dgate)),
              "rmsnorm_gate_backward: x, gate, weight, grad_output, dx, dgate and scratch must be 16-byte aligned");
  float* part = (float*)scratch;
  if (!fast_dim(dim)) {
    const int gnb = gen_norm_blocks(rows);
    if (rows > 0) {
#define KDA_GEN_NORM_BWD(NI)                                                                                  \
  hipLaunchKernelGGL(norm_gate_bwd_generic_kernel<NI>, dim3(gnb), dim3(256), 0, stream, (long)rows, (int)dim, \
                     (int)heads, (const bf16*)x, (const bf16*)gate, (long)gate_row_stride, weight, inv_rms,   \
                     (const bf16*)grad_output, (bf16*)dx, (bf16*)dgate, (long)dgate_row_stride, part)
      KDA_GEN_NORM_DISPATCH(dim, KDA_GEN_NORM_BWD)
#undef KDA_GEN_NORM_BWD
      KDA_LAUNCH_CHECK("rmsnorm_gate_backward");
    }
    hipLaunchKernelGGL(dw_reduce_kernel<float>, dim3((dim * kDwRedLanes + 255) / 256), dim3(256), 0, stream,
                       rows > 0 ? gnb : 0, dim, (const float*)part, dweight);
    KDA_LAUNCH_CHECK("rmsnorm_gate_dweight_reduce");
    return KDA_OK;
  }
  const int nb = norm_blocks(rows, dim, kRowsBwd, kBwdThreads);
  if (rows > 0) {
    if (dim == 128)
      hipLaunchKernelGGL(norm_gate_bwd_kernel<128>, dim3(nb), dim3(kBwdThreads), 0, stream, (long)rows, (int)heads,
                         (const bf16*)x, (const bf16*)gate, (long)gate_row_stride, weight, inv_rms,
                         (const bf16*)grad_output, (bf16*)dx, (bf16*)dgate, (long)dgate_row_stride, part);
    else
      hipLaunchKernelGGL(norm_gate_bwd_kernel<64>, dim3(nb), dim3(kBwdThreads), 0, stream, (long)rows, (int)heads,
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
