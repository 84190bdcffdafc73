// Token-serial KDA for the head dimensions the chunked kernels do not take (K, V other
// than 64 / 128): forward, backward and single-token decode.
//
// Reference: the generic lane of the CUDA backend, nanochat/mixers/cuda_kda/chunk.cu:135-213
// (forward, one thread per (b, h, value column) walking the tokens) and :578-870 (analytic
// token-serial backward over a stored state history), dispatched at chunk.cu:1716-1750 for
// every shape outside the production one.  Per token, with S the K x V state:
//   S1 = diag(e^g) S ;  r = v - S1^T k ;  S' = S1 + beta k r^T ;  o = S'^T q
// and in reverse, with X = dL/dS' (plus q do^T from the output):
//   dr = beta X^T k,  dv = dr,  dbeta = r . (X^T k),  dk = beta X r - S1 dr,  dq = S' do,
//   dS1 = X - k dr^T,  dg = rowsum(S1 o dS1),  dL/dS = diag(e^g) dS1.
//
// MI355X mapping.  The columns of S evolve independently, so a value column is owned by
// 16 lanes of a wave (lane kl holds keys kl + 16 m, m < KPL, in registers: K <= 256) and a
// wave owns 4 columns; a workgroup (4 waves) owns 16 columns of one (sequence, head).  The
// per-token reductions over K are 16-lane DPP sums, so the token loop has no barrier.  The
// per-token key vectors (normalised q and k, e^g) and beta, v, dO are staged per block of
// 16 tokens in LDS, derived once per workgroup; the next block's loads are issued before the
// current block is processed (double-buffered), one barrier per block.
// The forward stores the state at every block start (f32 checkpoints, the workspace); the
// backward walks the blocks in reverse, recomputes each block's states from its checkpoint
// into registers (sub-blocks of up to 16 tokens; a sub-block is recomputed from the block
// start) and runs the reverse step.  Per-key gradients (dq, dk, dg) and dbeta are summed
// over a wave's 4 columns in registers and written per wave; a second kernel sums the
// waves in a fixed order and applies the L2-norm, sigmoid and K3 gate chains; the gate
// parameters are reduced over tokens in a fixed order.  No atomics: results are
// deterministic.
#include "chunk_host.hpp"
#include "kda_device.hpp"

#include <type_traits>

namespace kda {

constexpr int kGenTB = 16;        // tokens per staged block = checkpoint interval
constexpr int kGenThreads = 256;  // 4 waves x 4 columns x 16 lanes
constexpr int kGenCols = 16;      // value columns per workgroup
constexpr int kGenRanges = 64;    // token ranges of the gate-parameter reduction
constexpr int kGenMaxK = 256;
constexpr int kGenMaxV = 4096;

struct GenArgs {
  int T, H, K, V, num_seqs, rows;  // rows: total token rows (B * T)
  const int* cu;                   // cu_seqlens (device) or null
  int gate_mode;
  float lb, scale;
  const bf16 *q, *k, *v;
  const void* gate;
  const bf16* beta;
  long beta_ld;
  const float *A_log, *dt_bias, *s0;
  bf16* out;
  float* sfin;
  float* ckpt;  // [slot][H][V][K] state at each block start, or null (decode)
  // backward
  const bf16* dout;
  const float* dsfin;
  bf16 *dq, *dk, *dv;
  long gld_qk, gld_v;
  void* dgate;
  bf16* dbeta;
  long dbeta_ld;
  int dbeta_pad;
  float *dA_log, *ddt_bias, *ds0;
  float* part;    // [V/4 waves][rows * H][3K + 1] per-wave partial dq^, dk^, dg, dbeta
  float* dz;      // [rows * H][K] f32 raw-gate gradient (K3)
  float* dapart;  // [rows * H] dA_log per token row (K3)
  float* ppart;   // [H][kGenRanges][K + 1] range partials of ddt_bias / dA_log (K3)
};

constexpr int gen_kpl(int K) { return K <= 16 ? 1 : K <= 32 ? 2 : K <= 64 ? 4 : K <= 128 ? 8 : 16; }

// Rows of the sequence s: [row0, row0 + len), checkpoint slots from slot0.  Slots of
// packed sequences start at floor(row0 / TB) + s, which never overlap and stay below
// floor(T / TB) + num_seqs + 1 even for a malformed (clamped) table.
__device__ __forceinline__ void gen_seq(const GenArgs& a, int s, int& row0, int& len, int& slot0) {
  if (a.cu) {
    int b = a.cu[s], e = a.cu[s + 1];
    b = b < 0 ? 0 : (b > a.T ? a.T : b);
    e = e < b ? b : (e > a.T ? a.T : e);
    row0 = b;
    len = e - b;
    slot0 = b / kGenTB + s;
  } else {
    row0 = s * a.T;
    len = a.T;
    slot0 = s * ((a.T + kGenTB - 1) / kGenTB);
  }
}

template <int KPL, bool BWD>
struct GenLds {
  static constexpr int KP = 16 * KPL;
  static constexpr int Q = 0, Kk = Q + 2 * kGenTB * KP, E = Kk + 2 * kGenTB * KP,
                       B = E + 2 * kGenTB * KP, Vv = B + 2 * kGenTB, DO = Vv + 2 * kGenTB * kGenCols,
                       floats = DO + (BWD ? 2 * kGenTB * kGenCols : 0);
  static constexpr size_t bytes = (size_t)floats * 4;
};

// A block's raw inputs in registers, between their loads and their staging.  Raw bf16 (or
// f32 log decay) values: converting them at the load would make the wave wait for them.
template <int NJ, int GATE>
struct GenStage {
  using GT = typename std::conditional<GATE == KDA_GATE_K3, bf16, float>::type;
  bf16 q[4][NJ], k[4][NJ];
  GT g[4][NJ];
  bf16 v, dov, bl;
};

template <int KPL, int GATE, bool BWD>
__device__ __forceinline__ void gen_stage_load(const GenArgs& a, GenStage<(16 * KPL + 63) / 64, GATE>& r,
                                               int row0, int t0, int len, int h, int vg) {
  constexpr int NJ = (16 * KPL + 63) / 64;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int t = t0 + wave + 4 * jj;
    const size_t base = ((size_t)(row0 + (t < len ? t : len - 1)) * a.H + h) * a.K;
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int key = lane + 64 * i;
      const size_t o = base + (key < a.K ? key : 0);
      r.q[jj][i] = a.q[o];
      r.k[jj][i] = a.k[o];
      r.g[jj][i] = reinterpret_cast<const typename GenStage<NJ, GATE>::GT*>(a.gate)[o];
    }
  }
  const int tt = tid / kGenCols, c = vg * kGenCols + tid % kGenCols;
  const int t = t0 + tt;
  const size_t vo = ((size_t)(row0 + (t < len ? t : len - 1)) * a.H + h) * a.V + (c < a.V ? c : a.V - 1);
  r.v = a.v[vo];
  if constexpr (BWD) r.dov = a.dout[vo];
  if (tid < kGenTB) {
    const int tb = t0 + tid;
    r.bl = a.beta[(size_t)(row0 + (tb < len ? tb : len - 1)) * a.beta_ld + h];
  }
}

// Normalise and write the block's key vectors, beta, v (and dO) into LDS buffer buf.
template <int KPL, int GATE, bool BWD>
__device__ __forceinline__ void gen_stage_store(const GenArgs& a, const GenStage<(16 * KPL + 63) / 64, GATE>& r,
                                                float* lds, int buf, int t0, int len, int vg, float ea,
                                                const float* bias) {
  constexpr int KP = 16 * KPL, NJ = (KP + 63) / 64;
  using L = GenLds<KPL, BWD>;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int tt = wave + 4 * jj;
    const bool valid = t0 + tt < len;
    float qv[NJ], kv[NJ], sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const bool ok = valid && lane + 64 * i < a.K;
      qv[i] = ok ? (float)r.q[jj][i] : 0.f;
      kv[i] = ok ? (float)r.k[jj][i] : 0.f;
      sq = fmaf(qv[i], qv[i], sq);
      sk = fmaf(kv[i], kv[i], sk);
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    const float rq = a.scale / fmaxf(sqrtf(sq), 1e-12f);
    const float rk = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
    const int row = buf * kGenTB + tt;
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int key = lane + 64 * i;
      if (key < KP) {
        const bool ok = valid && key < a.K;
        float g;
        if constexpr (GATE == KDA_GATE_K3)
          g = a.lb * sigmoid_acc(ea * ((float)r.g[jj][i] + bias[i]));
        else
          g = (float)r.g[jj][i];
        lds[L::Q + row * KP + key] = qv[i] * rq;
        lds[L::Kk + row * KP + key] = kv[i] * rk;
        lds[L::E + row * KP + key] = ok ? expf(g) : 0.f;
      }
    }
  }
  const int tt = tid / kGenCols, c = vg * kGenCols + tid % kGenCols;
  const bool ok = t0 + tt < len && c < a.V;
  lds[L::Vv + (buf * kGenTB + tt) * kGenCols + tid % kGenCols] = ok ? (float)r.v : 0.f;
  if constexpr (BWD) lds[L::DO + (buf * kGenTB + tt) * kGenCols + tid % kGenCols] = ok ? (float)r.dov : 0.f;
  if (tid < kGenTB) lds[L::B + buf * kGenTB + tid] = t0 + tid < len ? sigmoid_acc((float)r.bl) : 0.f;
}

// One forward token on a column's registers (keys kl + 16 m): S <- S1 + beta k r, returns r.
template <int KPL>
__device__ __forceinline__ float gen_step(float* S, const float* kk, const float* e, float beta, float v) {
  float pred = 0.f;
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    S[m] *= e[m];
    pred = fmaf(kk[m], S[m], pred);
  }
  pred = group_sum<16>(pred);
  const float r = v - pred;
  const float br = beta * r;
#pragma unroll
  for (int m = 0; m < KPL; ++m) S[m] = fmaf(kk[m], br, S[m]);
  return r;
}

template <int KPL, bool BWD>
__device__ __forceinline__ void gen_token(const float* lds, int buf, int i, int kl, int c, float* q, float* kk,
                                          float* e, float& beta, float& v, float& dov) {
  constexpr int KP = 16 * KPL;
  using L = GenLds<KPL, BWD>;
  const int row = buf * kGenTB + i;
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    q[m] = lds[L::Q + row * KP + kl + 16 * m];
    kk[m] = lds[L::Kk + row * KP + kl + 16 * m];
    e[m] = lds[L::E + row * KP + kl + 16 * m];
  }
  beta = lds[L::B + row];
  v = lds[L::Vv + row * kGenCols + c];
  if constexpr (BWD) dov = lds[L::DO + row * kGenCols + c];
}

template <int KPL, int GATE>
__global__ __launch_bounds__(kGenThreads) void gen_fwd_kernel(GenArgs a) {
  constexpr int NJ = (16 * KPL + 63) / 64;
  using L = GenLds<KPL, false>;
  extern __shared__ float lds[];
  const int vgroups = (a.V + kGenCols - 1) / kGenCols;
  const int rec = blockIdx.x / vgroups, vg = blockIdx.x % vgroups;
  const int s = rec / a.H, h = rec % a.H;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, kl = lane % 16;
  const int cl = wave * 4 + lane / 16;  // column within the workgroup
  const int col = vg * kGenCols + cl;
  const bool colok = col < a.V;
  int row0, len, slot0;
  gen_seq(a, s, row0, len, slot0);
  float ea = 0.f, bias[NJ];
#pragma unroll
  for (int i = 0; i < NJ; ++i) bias[i] = 0.f;
  if constexpr (GATE == KDA_GATE_K3) {
    ea = expf(a.A_log[h]);
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int key = lane + 64 * i;
      bias[i] = a.dt_bias[h * a.K + (key < a.K ? key : 0)];
    }
  }
  float S[KPL];
  const size_t srow = ((size_t)rec * a.V + (colok ? col : 0)) * a.K;
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    const int key = kl + 16 * m;
    S[m] = (a.s0 && colok && key < a.K) ? a.s0[srow + key] : 0.f;
  }
  const int nb = (len + kGenTB - 1) / kGenTB;
  GenStage<NJ, GATE> st;
  if (nb > 0) {
    gen_stage_load<KPL, GATE, false>(a, st, row0, 0, len, h, vg);
    gen_stage_store<KPL, GATE, false>(a, st, lds, 0, 0, len, vg, ea, bias);
  }
  __syncthreads();
  for (int j = 0; j < nb; ++j) {
    const int buf = j & 1, t0 = j * kGenTB;
    if (j + 1 < nb) gen_stage_load<KPL, GATE, false>(a, st, row0, t0 + kGenTB, len, h, vg);
    if (a.ckpt && colok) {
      float* ck = a.ckpt + (((size_t)(slot0 + j) * a.H + h) * a.V + col) * a.K;
#pragma unroll
      for (int m = 0; m < KPL; ++m)
        if (kl + 16 * m < a.K) ck[kl + 16 * m] = S[m];
    }
    const int n = len - t0 < kGenTB ? len - t0 : kGenTB;
    for (int i = 0; i < n; ++i) {
      float q[KPL], kk[KPL], e[KPL], beta, v, dov;
      gen_token<KPL, false>(lds, buf, i, kl, cl, q, kk, e, beta, v, dov);
      gen_step<KPL>(S, kk, e, beta, v);
      float o = 0.f;
#pragma unroll
      for (int m = 0; m < KPL; ++m) o = fmaf(q[m], S[m], o);
      o = group_sum<16>(o);
      if (kl == 0 && colok) a.out[((size_t)(row0 + t0 + i) * a.H + h) * a.V + col] = to_bf16(o);
    }
    if (j + 1 < nb) gen_stage_store<KPL, GATE, false>(a, st, lds, buf ^ 1, t0 + kGenTB, len, vg, ea, bias);
    __syncthreads();
  }
  if (a.sfin && colok) {
#pragma unroll
    for (int m = 0; m < KPL; ++m)
      if (kl + 16 * m < a.K) a.sfin[srow + kl + 16 * m] = S[m];
  }
  (void)L::bytes;
}

template <int KPL, int GATE>
__global__ __launch_bounds__(kGenThreads) void gen_bwd_kernel(GenArgs a) {
  constexpr int NJ = (16 * KPL + 63) / 64;
  constexpr int RB = 64 / KPL < kGenTB ? 64 / KPL : kGenTB;  // tokens whose states stay in registers
  extern __shared__ float lds[];
  const int vgroups = (a.V + kGenCols - 1) / kGenCols;
  const int rec = blockIdx.x / vgroups, vg = blockIdx.x % vgroups;
  const int s = rec / a.H, h = rec % a.H;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, kl = lane % 16;
  const int cl = wave * 4 + lane / 16;
  const int col = vg * kGenCols + cl;
  const bool colok = col < a.V;
  const int vw = vg * 4 + wave;                // this wave's partial set
  const bool wave_live = vw * 4 < a.V;         // some column of the wave is a real one
  const size_t rowsH = (size_t)a.rows * a.H;
  const int PK = 3 * a.K + 1;
  int row0, len, slot0;
  gen_seq(a, s, row0, len, slot0);
  float ea = 0.f, bias[NJ];
#pragma unroll
  for (int i = 0; i < NJ; ++i) bias[i] = 0.f;
  if constexpr (GATE == KDA_GATE_K3) {
    ea = expf(a.A_log[h]);
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int key = lane + 64 * i;
      bias[i] = a.dt_bias[h * a.K + (key < a.K ? key : 0)];
    }
  }
  const size_t srow = ((size_t)rec * a.V + (colok ? col : 0)) * a.K;
  float X[KPL], Cn[KPL];
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    const int key = kl + 16 * m;
    X[m] = (a.dsfin && colok && key < a.K) ? a.dsfin[srow + key] : 0.f;
    Cn[m] = 0.f;
  }
  auto ck_load = [&](int j, float* C) {
    const float* ck = a.ckpt + (((size_t)(slot0 + j) * a.H + h) * a.V + (colok ? col : 0)) * a.K;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
      const int key = kl + 16 * m;
      C[m] = ck[key < a.K ? key : 0];
    }
  };
  const int nb = (len + kGenTB - 1) / kGenTB;
  GenStage<NJ, GATE> st;
  if (nb > 0) {
    gen_stage_load<KPL, GATE, true>(a, st, row0, (nb - 1) * kGenTB, len, h, vg);
    gen_stage_store<KPL, GATE, true>(a, st, lds, (nb - 1) & 1, (nb - 1) * kGenTB, len, vg, ea, bias);
    ck_load(nb - 1, Cn);
  }
  __syncthreads();
  for (int j = nb - 1; j >= 0; --j) {
    const int buf = j & 1, t0 = j * kGenTB;
    float C[KPL];
#pragma unroll
    for (int m = 0; m < KPL; ++m) C[m] = Cn[m];
    if (j > 0) {
      gen_stage_load<KPL, GATE, true>(a, st, row0, t0 - kGenTB, len, h, vg);
      ck_load(j - 1, Cn);
    }
    const int n = len - t0 < kGenTB ? len - t0 : kGenTB;
    for (int sb = (n - 1) / RB; sb >= 0; --sb) {
      float S[KPL];
#pragma unroll
      for (int m = 0; m < KPL; ++m) S[m] = C[m] * (colok ? 1.f : 0.f);
      for (int i = 0; i < sb * RB; ++i) {
        float q[KPL], kk[KPL], e[KPL], beta, v, dov;
        gen_token<KPL, true>(lds, buf, i, kl, cl, q, kk, e, beta, v, dov);
        gen_step<KPL>(S, kk, e, beta, v);
      }
      float P[RB][KPL];  // the state entering each token of the sub-block
#pragma unroll
      for (int ii = 0; ii < RB; ++ii) {
        const int i = sb * RB + ii;
#pragma unroll
        for (int m = 0; m < KPL; ++m) P[ii][m] = S[m];
        if (i < n) {
          float q[KPL], kk[KPL], e[KPL], beta, v, dov;
          gen_token<KPL, true>(lds, buf, i, kl, cl, q, kk, e, beta, v, dov);
          gen_step<KPL>(S, kk, e, beta, v);
        }
      }
#pragma unroll
      for (int ii = RB - 1; ii >= 0; --ii) {
        const int i = sb * RB + ii;
        if (i >= n) continue;
        float q[KPL], kk[KPL], e[KPL], beta, v, dov;
        gen_token<KPL, true>(lds, buf, i, kl, cl, q, kk, e, beta, v, dov);
        float S1[KPL], pred = 0.f;
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
          S1[m] = e[m] * P[ii][m];
          pred = fmaf(kk[m], S1[m], pred);
        }
        pred = group_sum<16>(pred);
        const float r = v - pred;
        const float br = beta * r;
        float dqp[KPL], Xt[KPL], u = 0.f;
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
          dqp[m] = fmaf(kk[m], br, S1[m]) * dov;  // S' do
          Xt[m] = fmaf(q[m], dov, X[m]);
          u = fmaf(kk[m], Xt[m], u);
        }
        u = group_sum<16>(u);
        const float dr = beta * u;
        float dbp = r * u, dkp[KPL], dgp[KPL];
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
          dkp[m] = fmaf(beta * r, Xt[m], -dr * S1[m]);
          const float d1 = fmaf(-kk[m], dr, Xt[m]);
          dgp[m] = S1[m] * d1;
          X[m] = e[m] * d1;
        }
        const int row = row0 + t0 + i;
        if (kl == 0 && colok) a.dv[(size_t)row * a.gld_v + (size_t)h * a.V + col] = to_bf16(dr);
        // sum over the wave's 4 columns (lanes kl, kl + 16, kl + 32, kl + 48)
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
          dqp[m] = lane_stride_sum<16>(dqp[m]);
          dkp[m] = lane_stride_sum<16>(dkp[m]);
          dgp[m] = lane_stride_sum<16>(dgp[m]);
        }
        dbp = lane_stride_sum<16>(dbp);
        if (wave_live && lane < 16) {
          float* pp = a.part + ((size_t)vw * rowsH + (size_t)row * a.H + h) * PK;
#pragma unroll
          for (int m = 0; m < KPL; ++m) {
            const int key = kl + 16 * m;
            if (key < a.K) {
              pp[key] = dqp[m];
              pp[a.K + key] = dkp[m];
              pp[2 * a.K + key] = dgp[m];
            }
          }
          if (kl == 0) pp[3 * a.K] = dbp;
        }
      }
    }
    if (j > 0) gen_stage_store<KPL, GATE, true>(a, st, lds, buf ^ 1, t0 - kGenTB, len, vg, ea, bias);
    __syncthreads();
  }
  if (a.ds0 && colok) {
#pragma unroll
    for (int m = 0; m < KPL; ++m)
      if (kl + 16 * m < a.K) a.ds0[srow + kl + 16 * m] = X[m];
  }
}

// One wave per (token row, head): sums the per-wave partials in a fixed order and applies
// the L2-norm, beta-sigmoid and gate chains (kda_oracle.kda_backward's tail).
template <int GATE>
__global__ __launch_bounds__(256) void gen_finalize_kernel(GenArgs a, int nvw) {
  constexpr int NJ = kGenMaxK / 64;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const size_t rowsH = (size_t)a.rows * a.H;
  const size_t rh = (size_t)blockIdx.x * 4 + wave;
  if (rh >= rowsH) return;  // whole wave
  const int row = (int)(rh / a.H), h = (int)(rh % a.H);
  const int K = a.K, PK = 3 * K + 1;
  float dqh[NJ], dkh[NJ], dg[NJ], q[NJ], k[NJ];
  float db = 0.f;
  const size_t xo = ((size_t)row * a.H + h) * K;
#pragma unroll
  for (int i = 0; i < NJ; ++i) {
    dqh[i] = dkh[i] = dg[i] = 0.f;
    const int key = lane + 64 * i;
    q[i] = key < K ? (float)a.q[xo + key] : 0.f;
    k[i] = key < K ? (float)a.k[xo + key] : 0.f;
  }
  for (int w = 0; w < nvw; ++w) {
    const float* pp = a.part + ((size_t)w * rowsH + rh) * PK;
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int key = lane + 64 * i;
      if (key < K) {
        dqh[i] += pp[key];
        dkh[i] += pp[K + key];
        dg[i] += pp[2 * K + key];
      }
    }
    db += pp[3 * K];
  }
  // dx = (dy - y (y . dy)) / n for n > 1e-12, else dy / 1e-12  (y = x / max(n, 1e-12))
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int i = 0; i < NJ; ++i) {
    sq = fmaf(q[i], q[i], sq);
    sk = fmaf(k[i], k[i], sk);
  }
  const float nq = sqrtf(wave_sum(sq)), nk = sqrtf(wave_sum(sk));
  const float iq = 1.0f / fmaxf(nq, 1e-12f), ik = 1.0f / fmaxf(nk, 1e-12f);
  float dq_dot = 0.f, dk_dot = 0.f;
#pragma unroll
  for (int i = 0; i < NJ; ++i) {
    dqh[i] *= a.scale;
    dq_dot = fmaf(q[i] * iq, dqh[i], dq_dot);
    dk_dot = fmaf(k[i] * ik, dkh[i], dk_dot);
  }
  dq_dot = wave_sum(dq_dot);
  dk_dot = wave_sum(dk_dot);
  const float ea = GATE == KDA_GATE_K3 ? expf(a.A_log[h]) : 0.f;
  float dap = 0.f;
#pragma unroll
  for (int i = 0; i < NJ; ++i) {
    const int key = lane + 64 * i;
    if (key < K) {
      const float dqv = nq > 1e-12f ? (dqh[i] - q[i] * iq * dq_dot) * iq : dqh[i] * 1e12f;
      const float dkv = nk > 1e-12f ? (dkh[i] - k[i] * ik * dk_dot) * ik : dkh[i] * 1e12f;
      a.dq[(size_t)row * a.gld_qk + (size_t)h * K + key] = to_bf16(dqv);
      a.dk[(size_t)row * a.gld_qk + (size_t)h * K + key] = to_bf16(dkv);
      if constexpr (GATE == KDA_GATE_K3) {
        const float pre = (float)reinterpret_cast<const bf16*>(a.gate)[xo + key] + a.dt_bias[h * K + key];
        const float sg = sigmoid_acc(ea * pre);
        const float dz = dg[i] * a.lb * sg * (1.f - sg) * ea;
        reinterpret_cast<bf16*>(a.dgate)[xo + key] = to_bf16(dz);
        a.dz[rh * K + key] = dz;
        dap = fmaf(dz, pre, dap);
      } else {
        reinterpret_cast<float*>(a.dgate)[xo + key] = dg[i];
      }
    }
  }
  if constexpr (GATE == KDA_GATE_K3) {
    dap = wave_sum(dap);
    if (lane == 0) a.dapart[rh] = dap;
  }
  bf16* drow = a.dbeta + (size_t)row * a.dbeta_ld;
  if (lane == 0) {
    const float bt = sigmoid_acc((float)a.beta[(size_t)row * a.beta_ld + h]);
    drow[h] = to_bf16(db * bt * (1.f - bt));
  }
  if (h == 0)
    for (int e = lane; e < a.dbeta_pad; e += kWave) drow[a.H + e] = to_bf16(0.f);
}

// K3 gate parameters, pass 1: per (head, token range) sums of dz over the range's rows
// (ddt_bias) and of the rows' dA_log terms, in a fixed order.
__global__ __launch_bounds__(256) void gen_param_part_kernel(GenArgs a) {
  const int h = blockIdx.x, rg = blockIdx.y;
  const int r0 = (int)((long)a.rows * rg / kGenRanges), r1 = (int)((long)a.rows * (rg + 1) / kGenRanges);
  float* out = a.ppart + ((size_t)h * kGenRanges + rg) * (a.K + 1);
  for (int key = threadIdx.x; key < a.K; key += blockDim.x) {
    float acc = 0.f;
    for (int r = r0; r < r1; ++r) acc += a.dz[((size_t)r * a.H + h) * a.K + key];
    out[key] = acc;
  }
  __shared__ float red[256];
  float acc = 0.f;
  for (int r = r0 + (int)threadIdx.x; r < r1; r += blockDim.x) acc += a.dapart[(size_t)r * a.H + h];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < 256; ++i) t += red[i];
    out[a.K] = t;
  }
}

// Pass 2: the ranges in order.
__global__ __launch_bounds__(256) void gen_param_final_kernel(GenArgs a) {
  const int h = blockIdx.x;
  for (int key = threadIdx.x; key <= a.K; key += blockDim.x) {
    float acc = 0.f;
    for (int rg = 0; rg < kGenRanges; ++rg) acc += a.ppart[((size_t)h * kGenRanges + rg) * (a.K + 1) + key];
    if (key < a.K)
      a.ddt_bias[h * a.K + key] = acc;
    else
      a.dA_log[h] = acc;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool generic_dims(const kda_chunk_problem* p) {
  return !((p->key_dim == 64 || p->key_dim == 128) && (p->value_dim == 64 || p->value_dim == 128));
}

static size_t gen_slots(const kda_chunk_problem* p) {
  if (p->cu_seqlens) return (size_t)p->seq_len / kGenTB + p->num_seqs + 1;
  return (size_t)p->batch * ((p->seq_len + kGenTB - 1) / kGenTB);
}

static int gen_nvw(const kda_chunk_problem* p) { return (p->value_dim + 3) / 4; }

size_t generic_ws_bytes(const kda_chunk_problem* p) {
  return align256(gen_slots(p) * p->heads * p->value_dim * p->key_dim * sizeof(float)) + 256;
}

// Scratch regions of the generic backward, in order: part, dz, dapart, ppart.
static void gen_sc_layout(const kda_chunk_problem* p, size_t off[5]) {
  const size_t rowsH = (size_t)p->batch * p->seq_len * p->heads;
  off[0] = 0;
  off[1] = off[0] + align256((size_t)gen_nvw(p) * rowsH * (3 * p->key_dim + 1) * sizeof(float));
  off[2] = off[1] + align256(rowsH * p->key_dim * sizeof(float));
  off[3] = off[2] + align256(rowsH * sizeof(float));
  off[4] = off[3] + align256((size_t)p->heads * kGenRanges * (p->key_dim + 1) * sizeof(float));
}

size_t generic_sc_bytes(const kda_chunk_problem* p) {
  size_t off[5];
  gen_sc_layout(p, off);
  return off[4] + 256;
}

static int gen_check(const kda_chunk_problem* p, const char* who) {
  KDA_REQUIRE(p->key_dim >= 1 && p->key_dim <= kGenMaxK, "%s: key_dim must be in [1, %d]", who, kGenMaxK);
  KDA_REQUIRE(p->value_dim >= 1 && p->value_dim <= kGenMaxV, "%s: value_dim must be in [1, %d]", who, kGenMaxV);
  return KDA_OK;
}

template <typename F>
static int gen_dispatch(int K, F&& f) {
  switch (gen_kpl(K)) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return f(std::integral_constant<int, 16>{});
  }
}

static GenArgs gen_args(const kda_chunk_problem* p) {
  GenArgs a{};
  a.T = p->seq_len;
  a.H = p->heads;
  a.K = p->key_dim;
  a.V = p->value_dim;
  a.num_seqs = p->num_seqs;
  a.rows = p->batch * p->seq_len;
  a.cu = p->cu_seqlens;
  a.gate_mode = p->gate_mode;
  a.lb = p->lower_bound;
  a.scale = p->scale;
  a.beta_ld = p->beta_row_stride > 0 ? p->beta_row_stride : p->heads;
  return a;
}

int generic_forward(const kda_chunk_problem* p, const void* q, const void* k, const void* v, const void* gate,
                    const void* beta_logits, const float* A_log, const float* dt_bias, const float* initial_state,
                    void* output, float* final_state, void* workspace, hipStream_t stream) {
  int rc = gen_check(p, "chunk_forward");
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(p->norm_gate_row_stride == 0, "chunk_forward: norm_gate_row_stride needs head dims 64 or 128");
  GenArgs a = gen_args(p);
  a.q = (const bf16*)q;
  a.k = (const bf16*)k;
  a.v = (const bf16*)v;
  a.gate = gate;
  a.beta = (const bf16*)beta_logits;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.s0 = initial_state;
  a.out = (bf16*)output;
  a.sfin = final_state;
  a.ckpt = (float*)workspace;
  const int nrec = p->num_seqs * p->heads;
  if (nrec == 0) return KDA_OK;
  const int grid = nrec * ((p->value_dim + kGenCols - 1) / kGenCols);
  auto launch = [&](auto kpl_c) -> int {
    constexpr int KPL = decltype(kpl_c)::value;
    const size_t smem = GenLds<KPL, false>::bytes;
    const void* f = p->gate_mode == KDA_GATE_K3 ? (const void*)gen_fwd_kernel<KPL, KDA_GATE_K3>
                                                : (const void*)gen_fwd_kernel<KPL, KDA_GATE_LOGDECAY>;
    hipError_t e = ensure_lds_limit(f, (int)smem);
    if (e != hipSuccess) return set_error(KDA_ERR_LAUNCH, "chunk_forward (generic): LDS attribute: %s", hipGetErrorString(e));
    if (p->gate_mode == KDA_GATE_K3)
      hipLaunchKernelGGL((gen_fwd_kernel<KPL, KDA_GATE_K3>), dim3(grid), dim3(kGenThreads), smem, stream, a);
    else
      hipLaunchKernelGGL((gen_fwd_kernel<KPL, KDA_GATE_LOGDECAY>), dim3(grid), dim3(kGenThreads), smem, stream, a);
    KDA_LAUNCH_CHECK("chunk_forward (generic)");
    return KDA_OK;
  };
  return gen_dispatch(p->key_dim, launch);
}

int generic_backward(const kda_chunk_problem* p, const void* q, const void* k, const void* v, const void* gate,
                     const void* beta_logits, const float* A_log, const float* dt_bias, const void* workspace,
                     const void* grad_output, const float* grad_final_state, void* dq, void* dk, void* dv,
                     void* dgate, void* dbeta_logits, float* dA_log, float* ddt_bias, float* dinitial_state,
                     void* scratch, hipStream_t stream) {
  int rc = gen_check(p, "chunk_backward");
  if (rc != KDA_OK) return rc;
  GenArgs a = gen_args(p);
  a.q = (const bf16*)q;
  a.k = (const bf16*)k;
  a.v = (const bf16*)v;
  a.gate = gate;
  a.beta = (const bf16*)beta_logits;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.ckpt = (float*)const_cast<void*>(workspace);
  a.dout = (const bf16*)grad_output;
  a.dsfin = grad_final_state;
  a.dq = (bf16*)dq;
  a.dk = (bf16*)dk;
  a.dv = (bf16*)dv;
  a.gld_qk = p->grad_row_stride > 0 ? p->grad_row_stride : (long)p->heads * p->key_dim;
  a.gld_v = p->grad_row_stride > 0 ? p->grad_row_stride : (long)p->heads * p->value_dim;
  a.dgate = dgate;
  a.dbeta = (bf16*)dbeta_logits;
  a.dbeta_ld = p->beta_row_stride > 0 ? p->beta_row_stride : p->heads;
  a.dbeta_pad = p->beta_grad_pad;
  a.dA_log = dA_log;
  a.ddt_bias = ddt_bias;
  a.ds0 = dinitial_state;
  size_t off[5];
  gen_sc_layout(p, off);
  char* sc = (char*)scratch;
  a.part = (float*)(sc + off[0]);
  a.dz = (float*)(sc + off[1]);
  a.dapart = (float*)(sc + off[2]);
  a.ppart = (float*)(sc + off[3]);
  const bool k3 = p->gate_mode == KDA_GATE_K3;
  const int nrec = p->num_seqs * p->heads;
  if (nrec > 0) {
    const int grid = nrec * ((p->value_dim + kGenCols - 1) / kGenCols);
    auto launch = [&](auto kpl_c) -> int {
      constexpr int KPL = decltype(kpl_c)::value;
      const size_t smem = GenLds<KPL, true>::bytes;
      const void* f = k3 ? (const void*)gen_bwd_kernel<KPL, KDA_GATE_K3>
                         : (const void*)gen_bwd_kernel<KPL, KDA_GATE_LOGDECAY>;
      hipError_t e = ensure_lds_limit(f, (int)smem);
      if (e != hipSuccess)
        return set_error(KDA_ERR_LAUNCH, "chunk_backward (generic): LDS attribute: %s", hipGetErrorString(e));
      if (k3)
        hipLaunchKernelGGL((gen_bwd_kernel<KPL, KDA_GATE_K3>), dim3(grid), dim3(kGenThreads), smem, stream, a);
      else
        hipLaunchKernelGGL((gen_bwd_kernel<KPL, KDA_GATE_LOGDECAY>), dim3(grid), dim3(kGenThreads), smem, stream, a);
      KDA_LAUNCH_CHECK("chunk_backward (generic)");
      return KDA_OK;
    };
    rc = gen_dispatch(p->key_dim, launch);
    if (rc != KDA_OK) return rc;
  }
  const size_t rowsH = (size_t)a.rows * a.H;
  if (rowsH > 0) {
    const int blocks = (int)((rowsH + 3) / 4);
    if (k3)
      hipLaunchKernelGGL(gen_finalize_kernel<KDA_GATE_K3>, dim3(blocks), dim3(256), 0, stream, a, gen_nvw(p));
    else
      hipLaunchKernelGGL(gen_finalize_kernel<KDA_GATE_LOGDECAY>, dim3(blocks), dim3(256), 0, stream, a, gen_nvw(p));
    KDA_LAUNCH_CHECK("chunk_backward finalize (generic)");
  }
  if (k3) {
    hipLaunchKernelGGL(gen_param_part_kernel, dim3(p->heads, kGenRanges), dim3(256), 0, stream, a);
    KDA_LAUNCH_CHECK("chunk_backward params (generic)");
    hipLaunchKernelGGL(gen_param_final_kernel, dim3(p->heads), dim3(256), 0, stream, a);
    KDA_LAUNCH_CHECK("chunk_backward params (generic)");
  }
  return KDA_OK;
}


// ---------------------------------------------------------------------------
// zero-padded route: K <= 128 and V <= 128 run the chunked kernels at K, V rounded up to 64
// or 128.  Zero keys and zero value columns are exact: a zero key row of q and k leaves the
// L2 norms, every k^T S and q^T S and the state rows of the real keys unchanged, and its own
// state row never leaves zero; a zero value column (v = 0, no state, dO = 0) keeps its state
// column and every gradient contribution at zero.  The padded copies of q, k, v and the gate
// live behind the chunked workspace, so the backward reads the same padded inputs.
// ---------------------------------------------------------------------------

// dst[t][h][c] = c < w_src ? src[t][h][c] : 0 for c < w_dst, rows of H heads; token strides
// ld_src / ld_dst (elements), head strides w_src / w_dst.  One wave per (token, head) row.
template <typename T>
__global__ __launch_bounds__(256) void pad_rows_kernel(int nrows, int H, int w_src, long ld_src, int w_dst,
                                                       long ld_dst, const T* __restrict__ src, T* __restrict__ dst) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int r = blockIdx.x * 4 + wave; r < nrows; r += gridDim.x * 4) {
    const int t = r / H, h = r - t * H;
    const T* s = src + (size_t)t * ld_src + (size_t)h * w_src;
    T* d = dst + (size_t)t * ld_dst + (size_t)h * w_dst;
    for (int c = lane; c < w_dst; c += kWave) d[c] = c < w_src ? s[c] : T(0.f);
  }
}

template <typename T>
static int pad_rows(long nrows, int H, int w_src, long ld_src, int w_dst, long ld_dst, const void* src, void* dst,
                    hipStream_t stream) {
  if (nrows <= 0) return KDA_OK;
  KDA_REQUIRE(nrows < (1L << 31), "padded KDA: too many rows");
  const long blocks = (nrows + 3) / 4;
  hipLaunchKernelGGL(pad_rows_kernel<T>, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, stream,
                     (int)nrows, H, w_src, ld_src, w_dst, ld_dst, (const T*)src, (T*)dst);
  KDA_LAUNCH_CHECK("padded KDA copy");
  return KDA_OK;
}

bool padded_route(const kda_chunk_problem* p) {
  return generic_dims(p) && p->key_dim <= 128 && p->value_dim <= 128;
}

static kda_chunk_problem padded_problem(const kda_chunk_problem* p) {
  kda_chunk_problem pp = *p;
  pp.key_dim = p->key_dim <= 64 ? 64 : 128;
  pp.value_dim = p->value_dim <= 64 ? 64 : 128;
  pp.grad_row_stride = 0;
  pp.norm_gate_row_stride = 0;
  return pp;
}

// Regions behind the chunked workspace: qp, kp, vp, gp, dtp, s0p, outp, sfinp.
enum { PW_FAST, PW_Q, PW_K, PW_V, PW_G, PW_DT, PW_S0, PW_OUT, PW_SFIN, PW_END };
// Regions of the backward scratch: the chunked scratch, then dop, dsfp, dqp, dkp, dvp, dgp, ddtp, ds0p.
enum { PS_FAST, PS_DO, PS_DSF, PS_DQ, PS_DK, PS_DV, PS_DG, PS_DDT, PS_DS0, PS_END };

static void padded_ws_layout(const kda_chunk_problem* p, size_t off[PW_END + 1]) {
  const kda_chunk_problem pp = padded_problem(p);
  const size_t rowsH = (size_t)p->batch * p->seq_len * p->heads;
  const size_t gsz = p->gate_mode == KDA_GATE_K3 ? 2 : 4;
  const size_t st = (size_t)p->num_seqs * p->heads * pp.value_dim * pp.key_dim * 4;
  const size_t sz[PW_END] = {kda_chunk_workspace_bytes(&pp), rowsH * pp.key_dim * 2, rowsH * pp.key_dim * 2,
                             rowsH * pp.value_dim * 2,        rowsH * pp.key_dim * gsz,
                             (size_t)p->heads * pp.key_dim * 4, st, rowsH * pp.value_dim * 2, st};
  off[0] = 0;
  for (int i = 0; i < PW_END; ++i) off[i + 1] = off[i] + align256(sz[i]);
}

static void padded_sc_layout(const kda_chunk_problem* p, size_t off[PS_END + 1]) {
  const kda_chunk_problem pp = padded_problem(p);
  const size_t rowsH = (size_t)p->batch * p->seq_len * p->heads;
  const size_t gsz = p->gate_mode == KDA_GATE_K3 ? 2 : 4;
  const size_t st = (size_t)p->num_seqs * p->heads * pp.value_dim * pp.key_dim * 4;
  const size_t sz[PS_END] = {kda_chunk_backward_scratch_bytes(&pp), rowsH * pp.value_dim * 2, st,
                             rowsH * pp.key_dim * 2, rowsH * pp.key_dim * 2, rowsH * pp.value_dim * 2,
                             rowsH * pp.key_dim * gsz, (size_t)p->heads * pp.key_dim * 4, st};
  off[0] = 0;
  for (int i = 0; i < PS_END; ++i) off[i + 1] = off[i] + align256(sz[i]);
}

size_t padded_ws_bytes(const kda_chunk_problem* p) {
  size_t off[PW_END + 1];
  padded_ws_layout(p, off);
  return off[PW_END] + 256;
}

size_t padded_sc_bytes(const kda_chunk_problem* p) {
  size_t off[PS_END + 1];
  padded_sc_layout(p, off);
  return off[PS_END] + 256;
}

#define KDA_TRY(call)              \
  do {                             \
    const int _rc = (call);        \
    if (_rc != KDA_OK) return _rc; \
  } while (0)

int padded_forward(const kda_chunk_problem* p, const void* q, const void* k, const void* v, const void* gate,
                   const void* beta_logits, const float* A_log, const float* dt_bias, const float* initial_state,
                   void* output, float* final_state, void* workspace, hipStream_t stream) {
  const kda_chunk_problem pp = padded_problem(p);
  size_t off[PW_END + 1];
  padded_ws_layout(p, off);
  char* w = (char*)workspace;
  const int K = p->key_dim, V = p->value_dim, Kp = pp.key_dim, Vp = pp.value_dim, H = p->heads;
  const long toks = (long)p->batch * p->seq_len, nst = (long)p->num_seqs * H * V;
  const bool k3 = p->gate_mode == KDA_GATE_K3;
  KDA_TRY(pad_rows<bf16>(toks * H, H, K, (long)H * K, Kp, (long)H * Kp, q, w + off[PW_Q], stream));
  KDA_TRY(pad_rows<bf16>(toks * H, H, K, (long)H * K, Kp, (long)H * Kp, k, w + off[PW_K], stream));
  KDA_TRY(pad_rows<bf16>(toks * H, H, V, (long)H * V, Vp, (long)H * Vp, v, w + off[PW_V], stream));
  if (k3) {
    KDA_TRY(pad_rows<bf16>(toks * H, H, K, (long)H * K, Kp, (long)H * Kp, gate, w + off[PW_G], stream));
    KDA_TRY(pad_rows<float>(H, H, K, (long)H * K, Kp, (long)H * Kp, dt_bias, w + off[PW_DT], stream));
  } else {
    KDA_TRY(pad_rows<float>(toks * H, H, K, (long)H * K, Kp, (long)H * Kp, gate, w + off[PW_G], stream));
  }
  float* s0p = nullptr;
  if (initial_state) {
    // [N][H][V][K] -> [N][H][Vp][Kp]: rows (n, h, v) padded to Kp, then the Vp - V zero rows
    s0p = (float*)(w + off[PW_S0]);
    KDA_TRY(pad_rows<float>((long)p->num_seqs * H, 1, V * K, (long)V * K, Vp * Kp, (long)Vp * Kp, initial_state,
                            s0p, stream));  // zero tail of each (n, h) block
    KDA_TRY(pad_rows<float>(nst, V, K, (long)V * K, Kp, (long)Vp * Kp, initial_state, s0p, stream));
  }
  float* sfp = final_state ? (float*)(w + off[PW_SFIN]) : nullptr;
  bf16* outp = (bf16*)(w + off[PW_OUT]);
  KDA_TRY(kda_chunk_forward(&pp, w + off[PW_Q], w + off[PW_K], w + off[PW_V], w + off[PW_G], beta_logits, A_log,
                            k3 ? (const float*)(w + off[PW_DT]) : dt_bias, s0p, outp, sfp, w + off[PW_FAST],
                            stream));
  KDA_TRY(pad_rows<bf16>(toks * H, H, Vp, (long)H * Vp, V, (long)H * V, outp, output, stream));
  if (final_state) KDA_TRY(pad_rows<float>(nst, V, Kp, (long)Vp * Kp, K, (long)V * K, sfp, final_state, stream));
  return KDA_OK;
}

int padded_backward(const kda_chunk_problem* p, const void* beta_logits, const float* A_log, const void* workspace,
                    const void* grad_output, const float* grad_final_state, void* dq, void* dk, void* dv,
                    void* dgate, void* dbeta_logits, float* dA_log, float* ddt_bias, float* dinitial_state,
                    void* scratch, hipStream_t stream) {
  const kda_chunk_problem pp = padded_problem(p);
  size_t wo[PW_END + 1], so[PS_END + 1];
  padded_ws_layout(p, wo);
  padded_sc_layout(p, so);
  const char* w = (const char*)workspace;
  char* sc = (char*)scratch;
  const int K = p->key_dim, V = p->value_dim, Kp = pp.key_dim, Vp = pp.value_dim, H = p->heads;
  const long toks = (long)p->batch * p->seq_len, nst = (long)p->num_seqs * H * V;
  const bool k3 = p->gate_mode == KDA_GATE_K3;
  const long gld_qk = p->grad_row_stride > 0 ? p->grad_row_stride : (long)H * K;
  const long gld_v = p->grad_row_stride > 0 ? p->grad_row_stride : (long)H * V;
  KDA_TRY(pad_rows<bf16>(toks * H, H, V, (long)H * V, Vp, (long)H * Vp, grad_output, sc + so[PS_DO], stream));
  float* dsfp = nullptr;
  if (grad_final_state) {
    dsfp = (float*)(sc + so[PS_DSF]);
    KDA_TRY(pad_rows<float>((long)p->num_seqs * H, 1, V * K, (long)V * K, Vp * Kp, (long)Vp * Kp,
                            grad_final_state, dsfp, stream));
    KDA_TRY(pad_rows<float>(nst, V, K, (long)V * K, Kp, (long)Vp * Kp, grad_final_state, dsfp, stream));
  }
  float* ds0p = dinitial_state ? (float*)(sc + so[PS_DS0]) : nullptr;
  KDA_TRY(kda_chunk_backward(&pp, w + wo[PW_Q], w + wo[PW_K], w + wo[PW_V], w + wo[PW_G], beta_logits, A_log,
                             k3 ? (const float*)(w + wo[PW_DT]) : nullptr, nullptr, w + wo[PW_FAST],
                             sc + so[PS_DO], dsfp, sc + so[PS_DQ], sc + so[PS_DK], sc + so[PS_DV],
                             sc + so[PS_DG], dbeta_logits, dA_log, k3 ? (float*)(sc + so[PS_DDT]) : nullptr,
                             ds0p, sc + so[PS_FAST], stream));
  KDA_TRY(pad_rows<bf16>(toks * H, H, Kp, (long)H * Kp, K, gld_qk, sc + so[PS_DQ], dq, stream));
  KDA_TRY(pad_rows<bf16>(toks * H, H, Kp, (long)H * Kp, K, gld_qk, sc + so[PS_DK], dk, stream));
  KDA_TRY(pad_rows<bf16>(toks * H, H, Vp, (long)H * Vp, V, gld_v, sc + so[PS_DV], dv, stream));
  if (k3) {
    KDA_TRY(pad_rows<bf16>(toks * H, H, Kp, (long)H * Kp, K, (long)H * K, sc + so[PS_DG], dgate, stream));
    KDA_TRY(pad_rows<float>(H, H, Kp, (long)H * Kp, K, (long)H * K, sc + so[PS_DDT], ddt_bias, stream));
  } else {
    KDA_TRY(pad_rows<float>(toks * H, H, Kp, (long)H * Kp, K, (long)H * K, sc + so[PS_DG], dgate, stream));
  }
  if (dinitial_state) KDA_TRY(pad_rows<float>(nst, V, Kp, (long)Vp * Kp, K, (long)V * K, ds0p, dinitial_state, stream));
  return KDA_OK;
}

int padded_status(const kda_chunk_problem* p, const void* scratch, hipStream_t stream) {
  const kda_chunk_problem pp = padded_problem(p);
  return kda_chunk_backward_status(&pp, scratch, stream);
}

}  // namespace kda
