// Single-token recurrent KDA step on gfx950 (HBM-bound: one read and one write of the
// f32 state).  Reference: nanochat/mixers/cuda_kda/recurrent_decode.cu:24-181.
//
//   S1 = diag(exp(g)) S ;  r = v - k^T S1 ;  S' = S1 + beta k r^T ;  o = q^T S'
//
// State layout is V-first [B,H,V,K] f32, so one V row is K contiguous floats.  A
// workgroup owns 32 V rows of one (b,h); a row is covered by K/4 lanes holding a float4
// each, so every state access is a coalesced 16-byte load/store and the row reductions
// are in-wave shuffles.  Every lane loads what it needs (its 4 keys of q, k, gate, the
// state rows and their v) before it consumes anything, and derives its own keys'
// normalised q, k and decay itself: the L2 norms are reductions over the K/4 lanes of a
// row group, so there is no LDS and no barrier.  Grid: (B*H) x (V/32) workgroups of 256.
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kDecodeRowsPerBlock = 32;

__device__ __forceinline__ void load4bf(const bf16* p, float* out) {
  const bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (float)x[e];
}

template <int K>
__global__ __launch_bounds__(256) void decode_kernel(
    int heads, int V, int gate_mode, float lb, float scale, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, const void* __restrict__ gate,
    const bf16* __restrict__ beta_logits, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* initial_state, bf16* __restrict__ out,
    float* final_state) {
  constexpr int LPR = K / 4;          // lanes per V row
  constexpr int RPP = kWave / LPR;    // rows per wave pass
  constexpr int NPASS = kDecodeRowsPerBlock / (4 * RPP);  // rows per thread
  const int bh = blockIdx.x;
  const int h = bh % heads;
  const int tid = threadIdx.x;
  const size_t tok = (size_t)bh;  // [B,1,H,*] flattened: (b*H + h)
  const int wave = tid / kWave, lane = tid % kWave;
  const int sub = lane / LPR, kl = lane % LPR;
  const int k0 = kl * 4;
  const int row_base = blockIdx.y * kDecodeRowsPerBlock;

  // every load first: state rows, their v, and this lane's 4 keys
  float4 sv4[NPASS];
  float vr[NPASS];
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int row = row_base + ps * 4 * RPP + wave * RPP + sub;
    const int rc = row < V ? row : V - 1;
    const size_t off = ((size_t)bh * V + rc) * K + k0;
    sv4[ps] = initial_state ? *reinterpret_cast<const float4*>(initial_state + off)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    vr[ps] = (float)v[tok * V + rc];
  }
  float qv[4], kv[4], gv[4];
  load4bf(q + tok * K + k0, qv);
  load4bf(k + tok * K + k0, kv);
  const float bl = (float)beta_logits[tok];
  if (gate_mode == KDA_GATE_K3) {
    float raw[4];
    load4bf(reinterpret_cast<const bf16*>(gate) + tok * K + k0, raw);
    const float4 db = *reinterpret_cast<const float4*>(dt_bias + (size_t)h * K + k0);
    const float ea = expf(A_log[h]);
    const float dbv[4] = {db.x, db.y, db.z, db.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) gv[e] = lb * sigmoid_acc(ea * (raw[e] + dbv[e]));
  } else {
    const float4 g4 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(gate) + tok * K + k0);
    gv[0] = g4.x; gv[1] = g4.y; gv[2] = g4.z; gv[3] = g4.w;
  }
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    sq = fmaf(qv[e], qv[e], sq);
    sk = fmaf(kv[e], kv[e], sk);
  }
  sq = group_sum<LPR>(sq);
  sk = group_sum<LPR>(sk);
  const float rq = scale / fmaxf(sqrtf(sq), 1e-12f);
  const float rk = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
  const float beta = sigmoid_acc(bl);
  float qk[4], kk[4], kd[4], eg[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    eg[e] = expf(gv[e]);
    qk[e] = qv[e] * rq;
    kk[e] = kv[e] * rk;
    kd[e] = kk[e] * eg[e];
  }
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int row = row_base + ps * 4 * RPP + wave * RPP + sub;
    const size_t off = ((size_t)bh * V + row) * K + k0;
    float sv[4] = {sv4[ps].x, sv4[ps].y, sv4[ps].z, sv4[ps].w};
    float pred = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) pred = fmaf(kd[e], sv[e], pred);
    pred = group_sum<LPR>(pred);
    const float r = vr[ps] - pred;
    float o = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sv[e] = eg[e] * sv[e] + beta * kk[e] * r;
      o = fmaf(qk[e], sv[e], o);
    }
    o = group_sum<LPR>(o);
    if (row < V) {
      if (final_state)
        *reinterpret_cast<float4*>(final_state + off) = make_float4(sv[0], sv[1], sv[2], sv[3]);
      if (kl == 0) out[tok * V + row] = to_bf16(o);
    }
  }
}

}  // namespace kda

extern "C" int kda_recurrent_decode(int32_t batch, int32_t heads, int32_t key_dim,
                                    int32_t value_dim, int32_t gate_mode, float lower_bound,
                                    float scale, const void* q, const void* k, const void* v,
                                    const void* gate, const void* beta_logits,
                                    const float* A_log, const float* dt_bias,
                                    const float* initial_state, void* output,
                                    float* final_state, hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(batch >= 0 && heads > 0, "recurrent_decode: invalid batch/heads");
  KDA_REQUIRE(key_dim == 64 || key_dim == 128, "recurrent_decode: key_dim must be 64 or 128");
  KDA_REQUIRE(value_dim > 0 && value_dim <= 4096, "recurrent_decode: invalid value_dim");
  KDA_REQUIRE(gate_mode == KDA_GATE_K3 || gate_mode == KDA_GATE_LOGDECAY,
              "recurrent_decode: invalid gate_mode");
  KDA_REQUIRE(q && k && v && gate && beta_logits && output, "recurrent_decode: null pointer");
  KDA_REQUIRE(gate_mode != KDA_GATE_K3 || (A_log && dt_bias),
              "recurrent_decode: K3 gate needs A_log and dt_bias");
  KDA_REQUIRE(aligned16(q, k, gate, dt_bias, initial_state, final_state),
              "recurrent_decode: q, k, gate, dt_bias and the states must be 16-byte aligned");
  if (batch == 0) return KDA_OK;
  dim3 grid(batch * heads, (value_dim + kDecodeRowsPerBlock - 1) / kDecodeRowsPerBlock);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, heads, value_dim, gate_mode,
                       lower_bound, scale, (const bf16*)q, (const bf16*)k, (const bf16*)v, gate,
                       (const bf16*)beta_logits, A_log, dt_bias, initial_state, (bf16*)output,
                       final_state);
  };
  if (key_dim == 128)
    args(decode_kernel<128>);
  else
    args(decode_kernel<64>);
  KDA_LAUNCH_CHECK("recurrent_decode");
  return KDA_OK;
}
