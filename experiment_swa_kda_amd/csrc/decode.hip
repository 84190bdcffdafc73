// Single-token recurrent KDA step on gfx950 (HBM-bound: one read and one write of the
// f32 state).  Reference: nanochat/mixers/cuda_kda/recurrent_decode.cu:24-181.
//
//   S1 = diag(exp(g)) S ;  r = v - k^T S1 ;  S' = S1 + beta k r^T ;  o = q^T S'
//
// State layout is V-first [B,H,V,K] f32, so one V row is K contiguous floats.  A
// workgroup owns kDecodeRowsPerBlock V rows of one (b,h); a row is covered by K/4 lanes
// holding a float4 each, so every state access is a coalesced 16-byte load/store and the
// row reductions are in-wave DPP / permlane sums.  The per-key work (L2 norms of q and k,
// the K3 gate, exp(g), beta) is done once per workgroup by the first K/4 lanes of wave 0,
// four keys each, and handed to every wave through LDS: done per lane, it was most of the
// kernel's VALU time.  Its inputs are loaded before the state rows (loads complete in
// order), so it runs while the state rows are in flight.
#include "chunk_host.hpp"
#include "kda_device.hpp"
#include "kda_host.hpp"

#include <type_traits>

namespace kda {

#ifndef KDA_DECODE_ROWS
#define KDA_DECODE_ROWS 32  // V rows per workgroup
#endif
#ifndef KDA_DECODE_THREADS
#define KDA_DECODE_THREADS 256
#endif
constexpr int kDecodeRowsPerBlock = KDA_DECODE_ROWS;
constexpr int kDecodeThreads = KDA_DECODE_THREADS;

__device__ __forceinline__ void load4bf(const bf16* p, float* out) {
  const bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (float)x[e];
}

// GATE (the gate mode) and HAS_STATE (initial_state != NULL) are template parameters, so no
// branch separates the loads: a branch join makes the compiler wait for every load in
// flight, which serialised the state-row loads.
template <int K, int GATE, bool HAS_STATE>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(
    int heads, int V, float lb, float scale, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, const void* __restrict__ gate,
    const bf16* __restrict__ beta_logits, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* initial_state, bf16* __restrict__ out,
    float* final_state) {
  constexpr int LPR = K / 4;          // lanes per V row
  constexpr int RPP = kWave / LPR;    // rows per wave pass
  constexpr int NW = kDecodeThreads / kWave;
  constexpr int NPASS = kDecodeRowsPerBlock / (NW * RPP);  // rows per thread
  static_assert(NPASS * NW * RPP == kDecodeRowsPerBlock, "rows per workgroup");
  const int bh = blockIdx.x;
  const int h = bh % heads;
  const int tid = threadIdx.x;
  const size_t tok = (size_t)bh;  // [B,1,H,*] flattened: (b*H + h)
  const int wave = tid / kWave, lane = tid % kWave;
  const int sub = lane / LPR, kl = lane % LPR;
  const int k0 = kl * 4;
  const int row_base = blockIdx.y * kDecodeRowsPerBlock;

  __shared__ float4 s_q[K / 4], s_k[K / 4], s_kd[K / 4], s_eg[K / 4];
  __shared__ float s_beta;
  const bool prep = wave == 0 && lane < LPR;  // the lanes that derive the per-key values
  // raw loads only here (converted after the state loads are issued: a conversion inside
  // this branch would make the wave wait for these loads before issuing the state rows)
  bf16x4 qb = {}, kb = {}, rb = {};
  bf16 blb = {};
  float4 db = make_float4(0.f, 0.f, 0.f, 0.f), g4 = db;
  float alog = 0.f;
  if (prep) {
    qb = *reinterpret_cast<const bf16x4*>(q + tok * K + k0);
    kb = *reinterpret_cast<const bf16x4*>(k + tok * K + k0);
    blb = beta_logits[tok];
    if constexpr (GATE == KDA_GATE_K3) {
      rb = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16*>(gate) + tok * K + k0);
      db = *reinterpret_cast<const float4*>(dt_bias + (size_t)h * K + k0);
      alog = A_log[h];
    } else {
      g4 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(gate) + tok * K + k0);
    }
  }
  float4 sv4[NPASS];
  float vr[NPASS];
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int row = row_base + ps * NW * RPP + wave * RPP + sub;
    const int rc = row < V ? row : V - 1;
    const size_t off = ((size_t)bh * V + rc) * K + k0;
    if constexpr (HAS_STATE)
      sv4[ps] = *reinterpret_cast<const float4*>(initial_state + off);
    else
      sv4[ps] = make_float4(0.f, 0.f, 0.f, 0.f);
    vr[ps] = (float)v[tok * V + rc];
  }
  if (prep) {
    float qv[4], kv[4], raw[4], gv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qv[e] = (float)qb[e];
      kv[e] = (float)kb[e];
      raw[e] = (float)rb[e];
    }
    const float bl = (float)blb;
    if constexpr (GATE == KDA_GATE_K3) {
      const float ea = expf(alog);
      const float dbv[4] = {db.x, db.y, db.z, db.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) gv[e] = lb * sigmoid_acc(ea * (raw[e] + dbv[e]));
    } else {
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
    float eg[4], kk[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      eg[e] = expf(gv[e]);
      kk[e] = kv[e] * rk;
    }
    s_q[kl] = make_float4(qv[0] * rq, qv[1] * rq, qv[2] * rq, qv[3] * rq);
    s_k[kl] = make_float4(kk[0], kk[1], kk[2], kk[3]);
    s_kd[kl] = make_float4(kk[0] * eg[0], kk[1] * eg[1], kk[2] * eg[2], kk[3] * eg[3]);
    s_eg[kl] = make_float4(eg[0], eg[1], eg[2], eg[3]);
    if (kl == 0) s_beta = sigmoid_acc(bl);
  }
  // LDS writes complete, then a barrier that does not wait for the state loads in flight
  wait_lgkm0();
  ring_barrier();
  const float4 q4 = s_q[kl], k4 = s_k[kl], kd4 = s_kd[kl], e4 = s_eg[kl];
  const float qk[4] = {q4.x, q4.y, q4.z, q4.w}, kk[4] = {k4.x, k4.y, k4.z, k4.w};
  const float kd[4] = {kd4.x, kd4.y, kd4.z, kd4.w}, eg[4] = {e4.x, e4.y, e4.z, e4.w};
  const float beta = s_beta;
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int row = row_base + ps * NW * RPP + wave * RPP + sub;
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
  KDA_REQUIRE(key_dim >= 1 && key_dim <= 256, "recurrent_decode: key_dim must be in [1, 256]");
  KDA_REQUIRE(value_dim > 0 && value_dim <= 4096, "recurrent_decode: invalid value_dim");
  KDA_REQUIRE(gate_mode == KDA_GATE_K3 || gate_mode == KDA_GATE_LOGDECAY,
              "recurrent_decode: invalid gate_mode");
  KDA_REQUIRE(q && k && v && gate && beta_logits && output, "recurrent_decode: null pointer");
  KDA_REQUIRE(gate_mode != KDA_GATE_K3 || (A_log && dt_bias),
              "recurrent_decode: K3 gate needs A_log and dt_bias");
  KDA_REQUIRE(aligned16(q, k, gate, dt_bias, initial_state, final_state),
              "recurrent_decode: q, k, gate, dt_bias and the states must be 16-byte aligned");
  if (batch == 0) return KDA_OK;
  if (key_dim != 64 && key_dim != 128) {
    // other key dims: one step of the token-serial kernel (generic.hip); it reads each
    // state element before writing it from the same lane, so final_state may alias the
    // initial state
    kda_chunk_problem one = {};
    one.batch = batch;
    one.seq_len = 1;
    one.heads = heads;
    one.key_dim = key_dim;
    one.value_dim = value_dim;
    one.num_seqs = batch;
    one.gate_mode = gate_mode;
    one.lower_bound = lower_bound;
    one.scale = scale;
    return generic_forward(&one, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state, output,
                           final_state, nullptr, stream);
  }
  dim3 grid(batch * heads, (value_dim + kDecodeRowsPerBlock - 1) / kDecodeRowsPerBlock);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kDecodeThreads), 0, stream, heads, value_dim, lower_bound, scale,
                       (const bf16*)q, (const bf16*)k, (const bf16*)v, gate, (const bf16*)beta_logits, A_log,
                       dt_bias, initial_state, (bf16*)output, final_state);
  };
  auto by_dim = [&](auto gate_c, auto state_c) {
    constexpr int G = decltype(gate_c)::value;
    constexpr bool S = decltype(state_c)::value;
    if (key_dim == 128)
      args(decode_kernel<128, G, S>);
    else
      args(decode_kernel<64, G, S>);
  };
  using K3 = std::integral_constant<int, KDA_GATE_K3>;
  using LD = std::integral_constant<int, KDA_GATE_LOGDECAY>;
  if (gate_mode == KDA_GATE_K3)
    initial_state ? by_dim(K3{}, std::true_type{}) : by_dim(K3{}, std::false_type{});
  else
    initial_state ? by_dim(LD{}, std::true_type{}) : by_dim(LD{}, std::false_type{});
  KDA_LAUNCH_CHECK("recurrent_decode");
  return KDA_OK;
}
