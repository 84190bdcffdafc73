// Chunked (C = 64) WY forward of Kimi Delta Attention on gfx950.
//
// Reference algebra: nanochat/mixers/cuda_kda/chunk_wy_forward.cu (A/M build and solve
// :125-405, U/W :761-863, inter-chunk state scan :940-1276, output :1498-1588).  For a
// chunk with inclusive in-chunk cumulative log decay G (per key channel):
//   A[i,j]  = sum_c qh[i,c] kh[j,c] exp(G[i,c]-G[j,c])            j <= i
//   M'[i,j] = sum_c kh[i,c] kh[j,c] exp(G[i,c]-G[j,c])            j <  i
//   T = (I + diag(beta) M')^-1,  U = T (beta v),  W = T (beta kh exp(G))
//   delta = U - W S ;  O = (qh exp(G)) S + A delta ;  S <- diag(exp(G_last)) S + Kd^T delta
// with qh = scale * q/||q||, kh = k/||k||, Kd = kh exp(G_last - G).
//
// MI355X design:
//  * kda_chunk_prep: builds the chunk / sequence tables (B x T or packed cu_seqlens).
//  * intra kernel: one 256-thread workgroup per (chunk, head) tile, everything staged in
//    LDS (f32 qh/kh/G).  The 64x64 A and M' are built as 16x16 MFMA tiles
//    (v_mfma_f32_16x16x32_bf16).  Pairwise decays exp(G_i - G_j) are factorised around
//    the first row r of the row block: exp(G_i - G_r) <= 1 and, for j < r,
//    exp(G_r - G_j) <= 1, so no factor can overflow; only the diagonal block can, and a
//    diagonal block whose decay span exceeds 80 nats falls back to an exact per-pair
//    f32 loop.  T is formed in f32 by blocked forward substitution (16x16 blocks), then
//    U and W by MFMA.  Factors are written once to the workspace in both row- and
//    column-major form so every later MFMA operand is a contiguous 16-byte load.
//  * scan kernel: one workgroup per (sequence, head, 16-wide V strip) walks the chunks
//    in order holding its 128x16 f32 state slice in VGPRs as MFMA accumulators; the V
//    columns of the state evolve independently, so strips never communicate.  Each step
//    computes delta = U - W S, the output tile, and S <- lam S + Kd^T delta, and records
//    the bf16 state and delta for the backward pass.
// Every reduction has a fixed order, so the forward is bitwise deterministic.
#include "chunk_host.hpp"
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

struct FwdArgs {
  int H;
  int num_seqs;
  int gate_mode;
  float lb;
  float scale;
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const void* gate;
  const bf16* beta;
  const float* A_log;
  const float* dt_bias;
  const float* s0;
  bf16* out;
  float* sfin;
  Regions ws;
};

// ---------------------------------------------------------------------------
// chunk / sequence tables
// ---------------------------------------------------------------------------
__global__ void chunk_prep_kernel(int B, int T, int num_seqs, const int* __restrict__ cu,
                                  int max_chunks, int4* __restrict__ chunks,
                                  int2* __restrict__ seqs) {
  __shared__ int s_total;
  const int tid = threadIdx.x;
  if (cu == nullptr) {
    const int nc = (T + kChunk - 1) / kChunk;
    for (int c = tid; c < max_chunks; c += blockDim.x) {
      const int s = c / nc, j = c % nc;
      chunks[c] = make_int4(s * T + j * kChunk, min(kChunk, T - j * kChunk), s, j);
    }
    for (int s = tid; s < num_seqs; s += blockDim.x) seqs[s] = make_int2(s * nc, nc);
    return;
  }
  if (tid == 0) {
    int acc = 0;
    for (int s = 0; s < num_seqs; ++s) {
      // clamp to [0, T] so a malformed cu_seqlens can never address outside the inputs
      int a = min(max(cu[s], 0), T), b = min(max(cu[s + 1], 0), T);
      int n = b > a ? (b - a + kChunk - 1) / kChunk : 0;
      if (acc + n > max_chunks) n = 0;
      seqs[s] = make_int2(acc, n);
      acc += n;
    }
    s_total = acc;
  }
  __syncthreads();
  for (int c = s_total + tid; c < max_chunks; c += blockDim.x) chunks[c] = make_int4(0, 0, -1, 0);
  for (int s = tid; s < num_seqs; s += blockDim.x) {
    const int2 sq = seqs[s];
    const int a = min(max(cu[s], 0), T), b = min(max(cu[s + 1], 0), T);
    for (int j = 0; j < sq.y; ++j)
      chunks[sq.x + j] = make_int4(a + j * kChunk, min(kChunk, b - a - j * kChunk), s, j);
  }
}

// ---------------------------------------------------------------------------
// intra-chunk kernel
// ---------------------------------------------------------------------------
template <int K, int V>
struct IntraSmem {
  static constexpr int KP = K + 1;  // f32 row stride (odd: conflict-free column access)
  static constexpr int VP = V + 8;  // bf16 row stride
  static constexpr int MP = 65;
  static constexpr size_t off_q = 0;
  static constexpr size_t off_k = off_q + 64 * KP * 4;
  static constexpr size_t off_g = off_k + 64 * KP * 4;
  static constexpr size_t off_m = off_g + 64 * KP * 4;
  static constexpr size_t off_t = off_m + 64 * MP * 4;
  static constexpr size_t off_x = off_t + 64 * MP * 4;
  static constexpr size_t off_v = off_x + 3 * 16 * 17 * 4;
  static constexpr size_t off_b = off_v + 64 * VP * 2;
  static constexpr size_t off_f = off_b + 64 * 4;
  static constexpr size_t off_as = off_f + 16;                 // bf16 [64][AP] A staging
  static constexpr int AP = 64 + 8;
  static constexpr size_t bytes = off_as + 64 * AP * 2;
  // W staging (bf16 [64][K + 8]) reuses the q_hat region once Qg has been emitted
  static_assert(64 * (K + 8) * 2 <= 64 * KP * 4, "W staging must fit the q_hat region");
};

// Writes the MFMA A-operand fragments of an R x C matrix whose element (r, c) is val(r, c)
// (see frag_off); one 16-byte piece per thread iteration, contiguous across threads.
template <int R, int C, int NT, typename F>
__device__ __forceinline__ void emit_frags(bf16* dst, int tid, F val) {
  for (int idx = tid; idx < R * C / 8; idx += NT) {
    const int lane = idx % 64, s = (idx / 64) % (C / 32), rt = idx / (64 * (C / 32));
    const int r = 16 * rt + lane % 16, c0 = 32 * s + 8 * (lane / 16);
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = val(r, c0 + e);
    *(bf16x8*)(dst + (size_t)idx * 8) = x;
  }
}

constexpr int kIntraThreads = 1024;
constexpr int kIntraWaves = kIntraThreads / kWave;

__device__ __constant__ int kPairA[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
__device__ __constant__ int kPairB[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};

template <int K, int V>
__global__ __launch_bounds__(kIntraThreads) void chunk_fwd_intra_kernel(FwdArgs a) {
  using L = IntraSmem<K, V>;
  constexpr int KP = L::KP, VP = L::VP, MP = L::MP;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  float* sQ = (float*)(smem + L::off_q);
  float* sK = (float*)(smem + L::off_k);
  float* sG = (float*)(smem + L::off_g);
  float* sM = (float*)(smem + L::off_m);
  float* sT = (float*)(smem + L::off_t);
  float* sX = (float*)(smem + L::off_x);
  bf16* sV = (bf16*)(smem + L::off_v);
  float* sB = (float*)(smem + L::off_b);
  int* sF = (int*)(smem + L::off_f);
  bf16* sAs = (bf16*)(smem + L::off_as);
  bf16* sWs = (bf16*)(smem + L::off_q);  // after Qg/Kd fragments are written
  constexpr int AP = L::AP, WP = K + 8;

  const int4 ch = ((const int4*)a.ws.p[R_CHUNKS])[blockIdx.x];
  const int len = ch.y;
  if (len <= 0) return;
  const int H = a.H, h = blockIdx.y;
  const size_t tile = (size_t)blockIdx.x * H + h;
  const int row0 = ch.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;

  if (tid < 4) sF[tid] = 0;
  for (int i = tid; i < 64 * MP; i += kIntraThreads) sT[i] = 0.f;

  // ---- phase 1: load, normalise, activate ----
  {
    constexpr int LPR = K / 8;
    constexpr int RPP = kIntraThreads / LPR;
    const int c0 = (tid % LPR) * 8;
    const float* A_log = a.A_log;
    for (int t = tid / LPR; t < 64; t += RPP) {
      float qv[8], kv[8], gv[8];
      if (t < len) {
        const size_t base = ((size_t)(row0 + t) * H + h) * K + c0;
        load8(a.q + base, qv);
        load8(a.k + base, kv);
        if (a.gate_mode == KDA_GATE_K3) {
          float raw[8];
          load8((const bf16*)a.gate + base, raw);
          const float ea = expf(A_log[h]);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            gv[e] = a.lb * sigmoid_acc(ea * (raw[e] + a.dt_bias[h * K + c0 + e]));
        } else {
          const float4* gp = (const float4*)((const float*)a.gate + base);
          float4 g0 = gp[0], g1 = gp[1];
          gv[0] = g0.x; gv[1] = g0.y; gv[2] = g0.z; gv[3] = g0.w;
          gv[4] = g1.x; gv[5] = g1.y; gv[6] = g1.z; gv[7] = g1.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = kv[e] = gv[e] = 0.f;
      }
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sq += qv[e] * qv[e];
        sk += kv[e] * kv[e];
      }
      sq = group_sum<LPR>(sq);
      sk = group_sum<LPR>(sk);
      const float rq = a.scale / fmaxf(sqrtf(sq), 1e-12f);
      const float rk = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sQ[t * KP + c0 + e] = qv[e] * rq;
        sK[t * KP + c0 + e] = kv[e] * rk;
        sG[t * KP + c0 + e] = gv[e];
      }
      if (tid % LPR == 0) {
        const float bt = t < len ? sigmoid_acc(to_f32(a.beta[(size_t)(row0 + t) * H + h])) : 0.f;
        sB[t] = bt;
        ((float*)a.ws.p[R_RQ])[tile * 64 + t] = rq;
        ((float*)a.ws.p[R_RK])[tile * 64 + t] = rk;
        ((float*)a.ws.p[R_BETA])[tile * 64 + t] = bt;
      }
    }
  }
  __syncthreads();
  // beta * v (bf16) and the in-chunk cumulative decay
  for (int idx = tid; idx < 64 * (V / 8); idx += kIntraThreads) {
    const int t = idx / (V / 8), c0 = (idx % (V / 8)) * 8;
    float vv[8];
    if (t < len) {
      load8(a.v + ((size_t)(row0 + t) * H + h) * V + c0, vv);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) vv[e] = 0.f;
    }
    const float bt = sB[t];
#pragma unroll
    for (int e = 0; e < 8; ++e) sV[t * VP + c0 + e] = to_bf16(bt * vv[e]);
  }
  if (tid < K) {
    const int c = tid;
    float* Gout = (float*)a.ws.p[R_G] + tile * 64 * K;
    float acc = 0.f;
    for (int t = 0; t < 64; ++t) {
      acc += sG[t * KP + c];
      sG[t * KP + c] = acc;
      Gout[t * K + c] = acc;
    }
    ((float*)a.ws.p[R_LAM])[tile * K + c] = expf(acc);
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (sG[(16 * b) * KP + c] - sG[(16 * b + 15) * KP + c] > 80.f) atomicOr(&sF[b], 1);
  }
  __syncthreads();

  // ---- phase 2: A and M' (16x16 tiles of the lower triangle) ----
  float* MPout = (float*)a.ws.p[R_MP] + tile * 64 * 64;
  for (int p = wave; p < 10; p += kIntraWaves) {
    const int ba = kPairA[p], bb = kPairB[p];
    const int r = 16 * ba;
    f32x4 accA = zero4(), accM = zero4();
    if (!(ba == bb && sF[ba])) {
      const int i = 16 * ba + lr, j = 16 * bb + lr;
#pragma unroll
      for (int s = 0; s < K / 32; ++s) {
        const int c = 32 * s + 8 * kg;
        bf16x8 fq, fk, fb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float gr = sG[r * KP + c + e];
          const float ei = __expf(sG[i * KP + c + e] - gr);
          const float ej = __expf(gr - sG[j * KP + c + e]);
          fq[e] = to_bf16(sQ[i * KP + c + e] * ei);
          fk[e] = to_bf16(sK[i * KP + c + e] * ei);
          fb[e] = to_bf16(sK[j * KP + c + e] * ej);
        }
        accA = mfma16(fq, fb, accA);
        accM = mfma16(fk, fb, accM);
      }
    } else {
      // exact pairwise path for a diagonal block with a large decay span
      const int jj = 16 * bb + lr;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ii = 16 * ba + 4 * kg + rr;
        float sa = 0.f, sm = 0.f;
        if (jj <= ii) {
          for (int c = 0; c < K; ++c) {
            const float e = expf(sG[ii * KP + c] - sG[jj * KP + c]);
            const float kj = sK[jj * KP + c] * e;
            sa = fmaf(sQ[ii * KP + c], kj, sa);
            sm = fmaf(sK[ii * KP + c], kj, sm);
          }
        }
        accA[rr] = sa;
        accM[rr] = sm;
      }
    }
    const int jj = 16 * bb + lr;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ii = 16 * ba + 4 * kg + rr;
      const float av = jj <= ii ? accA[rr] : 0.f;
      const float mv = jj < ii ? accM[rr] : 0.f;
      sAs[ii * AP + jj] = to_bf16(av);
      sM[ii * MP + jj] = mv;
      MPout[ii * 64 + jj] = mv;
    }
  }
  // strictly-upper 16x16 blocks are zero
  for (int idx = tid; idx < 64 * 64; idx += kIntraThreads) {
    const int ii = idx / 64, jj = idx % 64;
    if (jj / 16 > ii / 16) {
      sAs[ii * AP + jj] = to_bf16(0.f);
      sM[ii * MP + jj] = 0.f;
      MPout[ii * 64 + jj] = 0.f;
    }
  }
  __syncthreads();

  // ---- A, Qg = qh exp(G), Kd = kh exp(G_last - G) as MFMA fragments (+ transposes) ----
  {
    constexpr int NT = kIntraThreads;
    emit_frags<64, 64, NT>((bf16*)a.ws.p[R_AF] + tile * 64 * 64, tid,
                           [&](int r, int c) { return sAs[r * AP + c]; });
    emit_frags<64, 64, NT>((bf16*)a.ws.p[R_ATF] + tile * 64 * 64, tid,
                           [&](int r, int c) { return sAs[c * AP + r]; });
    const float* gl = sG + 63 * KP;
    emit_frags<64, K, NT>((bf16*)a.ws.p[R_QGF] + tile * 64 * K, tid, [&](int r, int c) {
      return to_bf16(sQ[r * KP + c] * expf(sG[r * KP + c]));
    });
    emit_frags<K, 64, NT>((bf16*)a.ws.p[R_QGTF] + tile * K * 64, tid, [&](int r, int c) {
      return to_bf16(sQ[c * KP + r] * expf(sG[c * KP + r]));
    });
    emit_frags<64, K, NT>((bf16*)a.ws.p[R_KDF] + tile * 64 * K, tid, [&](int r, int c) {
      return to_bf16(sK[r * KP + c] * expf(gl[c] - sG[r * KP + c]));
    });
    emit_frags<K, 64, NT>((bf16*)a.ws.p[R_KDTF] + tile * K * 64, tid, [&](int r, int c) {
      return to_bf16(sK[c * KP + r] * expf(gl[r] - sG[c * KP + r]));
    });
  }

  // ---- phase 3: T = (I + diag(beta) M')^-1, blocked forward substitution ----
  if (tid < 64) {
    const int blk = tid / 16, j = tid % 16;
    const int o = 16 * blk;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = (i == j) ? 1.f : 0.f;
      const float bi = sB[o + i];
#pragma unroll
      for (int m = 0; m < i; ++m)
        if (m >= j) s -= bi * sM[(o + i) * MP + o + m] * x[m];
      x[i] = (i < j) ? 0.f : s;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sT[(o + i) * MP + o + j] = x[i];
  }
  __syncthreads();
  for (int ba = 1; ba < 4; ++ba) {
    for (int idx = tid; idx < ba * 256; idx += kIntraThreads) {
      const int bb = idx / 256, i = (idx % 256) / 16, j = idx % 16;
      const float bi = sB[16 * ba + i];
      float s = 0.f;
      for (int m = 16 * bb; m < 16 * ba; ++m)
        s = fmaf(sM[(16 * ba + i) * MP + m], sT[m * MP + 16 * bb + j], s);
      sX[(bb * 16 + i) * 17 + j] = bi * s;
    }
    __syncthreads();
    for (int idx = tid; idx < ba * 256; idx += kIntraThreads) {
      const int bb = idx / 256, i = (idx % 256) / 16, j = idx % 16;
      float s = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m)
        s = fmaf(sT[(16 * ba + i) * MP + 16 * ba + m], sX[(bb * 16 + m) * 17 + j], s);
      sT[(16 * ba + i) * MP + 16 * bb + j] = -s;
    }
    __syncthreads();
  }
  {
    float* Tout = (float*)a.ws.p[R_T] + tile * 64 * 64;
    for (int idx = tid; idx < 64 * 64; idx += kIntraThreads) Tout[idx] = sT[(idx / 64) * MP + idx % 64];
  }

  // ---- phase 4: U = T (beta v), W = T (beta kh exp(G)) ----
  {
    bf16* Uout = (bf16*)a.ws.p[R_UF] + tile * 64 * V;
    constexpr int NU = 4 * (V / 16), NW = 4 * (K / 16);
    for (int p = wave; p < NU + NW; p += kIntraWaves) {
      const bool isU = p < NU;
      const int q = isU ? p : p - NU;
      const int rt = q % 4, ct = q / 4;
      const int i = 16 * rt + lr, col = 16 * ct + lr;
      f32x4 acc = zero4();
      const int nsteps = (16 * rt + 15) / 32 + 1;
      for (int s = 0; s < nsteps; ++s) {
        const int j0 = 32 * s + 8 * kg;
        bf16x8 fa, fb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          fa[e] = to_bf16(sT[i * MP + j0 + e]);
          const int j = j0 + e;
          fb[e] = isU ? sV[j * VP + col]
                      : to_bf16(sB[j] * sK[j * KP + col] * __expf(sG[j * KP + col]));
        }
        acc = mfma16(fa, fb, acc);
      }
      if (isU) {
        // C layout kept as is: [strip = ct][row tile][lane][4]
        bf16x4 x;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) x[rr] = to_bf16(acc[rr]);
        *(bf16x4*)(Uout + ((size_t)(ct * 4 + rt) * 64 + lane) * 4) = x;
      } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sWs[(16 * rt + 4 * kg + rr) * WP + col] = to_bf16(acc[rr]);
      }
    }
  }
  __syncthreads();
  emit_frags<64, K, kIntraThreads>((bf16*)a.ws.p[R_WF] + tile * 64 * K, tid,
                                   [&](int r, int c) { return sWs[r * WP + c]; });
  emit_frags<K, 64, kIntraThreads>((bf16*)a.ws.p[R_WTF] + tile * K * 64, tid,
                                   [&](int r, int c) { return sWs[c * WP + r]; });

}

// ---------------------------------------------------------------------------
// inter-chunk state scan
// ---------------------------------------------------------------------------
// One 256-thread workgroup per (sequence, head, 16-wide V strip).  The critical path
// per chunk is: publish S (LDS) -> delta = U - W S -> publish delta (LDS) ->
// S <- lam S + Kd^T delta, two barriers.  All global operands of a chunk are loaded
// into a register ring kFwdRing chunks ahead, so the HBM latency (~1-2 us) overlaps
// several chunk steps.  Every per-step global access is one vector instruction (CDNA
// counts loads and stores on the same vmcnt, which must stay below 64 in flight).
constexpr int kFwdRing = 4;

template <int K>
struct FwdScanFrag {
  bf16x8 w[K / 32];      // W rows of this wave's delta tile
  bf16x4 ut;             // U: the 4 entries of this lane's delta outputs (C layout)
  bf16x8 kdt[K / 64][2]; // Kd^T rows of this wave's state tiles
  float4 lam[K / 64];    // exp(G_last) of this lane's state rows
};

template <int K, int V>
__global__ __launch_bounds__(256) void chunk_fwd_scan_kernel(FwdArgs a) {
  constexpr int KT = K / 16 / 4;  // 16-row key tiles of the state per wave
  constexpr int SP = K + 8;
  constexpr int DP = 64 + 8;
  constexpr int FP = 16 + 4;
  __shared__ __attribute__((aligned(16))) bf16 sS[2][16 * SP];  // bf16 S as [v][k]
  __shared__ __attribute__((aligned(16))) float sSf[K * FP];    // f32 S as [k][v]
  __shared__ __attribute__((aligned(16))) bf16 sD[16 * DP];     // delta as [v][t]
  const int H = a.H;
  int rec, strip;
  if (!xcd_strip_coords(a.num_seqs * H, V / 16, rec, strip)) return;
  const int seq = rec / H, h = rec % H, v0 = strip * 16;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;
  const int2 sq = ((const int2*)a.ws.p[R_SEQS])[seq];
  const int i = 16 * wave + lr;

  auto load = [&](int chunk, FwdScanFrag<K>& f) {
    const size_t tile = (size_t)chunk * H + h;
    const bf16* WF = (const bf16*)a.ws.p[R_WF] + tile * 64 * K;
    const bf16* UF = (const bf16*)a.ws.p[R_UF] + tile * 64 * V;
    const bf16* KDTF = (const bf16*)a.ws.p[R_KDTF] + tile * K * 64;
    const float* lam = (const float*)a.ws.p[R_LAM] + tile * K;
#pragma unroll
    for (int s = 0; s < K / 32; ++s) f.w[s] = *(const bf16x8*)(WF + frag_off(K, wave, s, lane));
    f.ut = *(const bf16x4*)(UF + ((size_t)(strip * 4 + wave) * 64 + lane) * 4);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int kb = 16 * (wave * KT + kt);
#pragma unroll
      for (int s = 0; s < 2; ++s) f.kdt[kt][s] = *(const bf16x8*)(KDTF + frag_off(64, wave * KT + kt, s, lane));
      f.lam[kt] = *(const float4*)(lam + kb + 4 * kg);
    }
  };

  f32x4 S[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int k0 = 16 * (wave * KT + kt) + 4 * kg;
    if (a.s0) {
      const float4 s = *(const float4*)(a.s0 + (((size_t)seq * H + h) * V + v0 + lr) * K + k0);
      S[kt][0] = s.x; S[kt][1] = s.y; S[kt][2] = s.z; S[kt][3] = s.w;
    } else {
      S[kt] = zero4();
    }
  }
  const int n = sq.y;
  FwdScanFrag<K> ring[kFwdRing];
  if (n > 0) {
#pragma unroll
    for (int d = 0; d < kFwdRing; ++d) load(sq.x + min(d, n - 1), ring[d]);
  }

  auto step = [&](int ci, FwdScanFrag<K>& f) {
    const int chunk = sq.x + ci;
    const size_t tile = (size_t)chunk * H + h;
    bf16* sSp = sS[ci & 1];
    // (1) publish S: bf16 [v][k] (MFMA operand) and f32 [k][v] (history staging)
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int k0 = 16 * (wave * KT + kt) + 4 * kg;
      bf16x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = to_bf16(S[kt][r]);
        sSf[(k0 + r) * FP + lr] = S[kt][r];
      }
      *(bf16x4*)(sSp + lr * SP + k0) = x;
    }
    __syncthreads();
    // (2) state histories: f32 [K][V] and bf16 [V][K] (fixed-count vector stores)
    {
      float* SH = (float*)a.ws.p[R_SH] + tile * K * V;
#pragma unroll
      for (int it = 0; it < K / 64; ++it) {
        const int idx = tid + 256 * it;
        const int kk = idx / 4, q4 = (idx % 4) * 4;
        *(float4*)(SH + (size_t)kk * V + v0 + q4) = *(const float4*)(sSf + kk * FP + q4);
      }
      // bf16 state as B-operand fragments of this strip (read by the output kernel)
      bf16* SHBF = (bf16*)a.ws.p[R_SHBF] + tile * V * K + (size_t)strip * 16 * K;
      if (tid < 16 * K / 8) {
        const int sl = tid / 64, ln = tid % 64;
        *(bf16x8*)(SHBF + ((size_t)sl * 64 + ln) * 8) =
            *(const bf16x8*)(sSp + (ln % 16) * SP + 32 * sl + 8 * (ln / 16));
      }
    }
    // (3) delta rows 16*wave.. = U - W S  (two accumulators halve the MFMA chain)
    {
      f32x4 acc0 = zero4(), acc1 = zero4();
#pragma unroll
      for (int s = 0; s < K / 32; s += 2) {
        acc0 = mfma16(f.w[s], *(const bf16x8*)(sSp + lr * SP + 32 * s + 8 * kg), acc0);
        acc1 = mfma16(f.w[s + 1], *(const bf16x8*)(sSp + lr * SP + 32 * (s + 1) + 8 * kg), acc1);
      }
      bf16x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = to_bf16(to_f32(f.ut[r]) - (acc0[r] + acc1[r]));
      *(bf16x4*)(sD + lr * DP + 16 * wave + 4 * kg) = x;
    }
    __syncthreads();
    // (3b) delta as B-operand fragments of this strip [2][64 lanes][8]
    if (tid < 128) {
      bf16* DLF = (bf16*)a.ws.p[R_DLF] + tile * 64 * V + (size_t)strip * 16 * 64;
      const int sl = tid / 64, ln = tid % 64;
      *(bf16x8*)(DLF + ((size_t)sl * 64 + ln) * 8) =
          *(const bf16x8*)(sD + (ln % 16) * DP + 32 * sl + 8 * (ln / 16));
    }
    // (4) S <- lam S + Kd^T delta
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x4 acc = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s)
        acc = mfma16(f.kdt[kt][s], *(const bf16x8*)(sD + lr * DP + 32 * s + 8 * kg), acc);
      S[kt][0] = fmaf(f.lam[kt].x, S[kt][0], acc[0]);
      S[kt][1] = fmaf(f.lam[kt].y, S[kt][1], acc[1]);
      S[kt][2] = fmaf(f.lam[kt].z, S[kt][2], acc[2]);
      S[kt][3] = fmaf(f.lam[kt].w, S[kt][3], acc[3]);
    }
  };

  // Ring loads are unconditional (the index is clamped to the last chunk) so no register
  // of the ring is redefined under control flow; otherwise the compiler must wait for
  // every load in flight at each join.
  for (int c0 = 0; c0 < n; c0 += kFwdRing) {
#pragma unroll
    for (int d = 0; d < kFwdRing; ++d) {
      const int ci = c0 + d;
      if (ci < n) step(ci, ring[d]);
      load(sq.x + min(ci + kFwdRing, n - 1), ring[d]);
    }
  }
  if (a.sfin) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int k0 = 16 * (wave * KT + kt) + 4 * kg;
      *(float4*)(a.sfin + (((size_t)seq * H + h) * V + v0 + lr) * K + k0) =
          make_float4(S[kt][0], S[kt][1], S[kt][2], S[kt][3]);
    }
  }
}

// ---------------------------------------------------------------------------
// output:  O = Qg S + A delta  (chunk-parallel, after the scan)
// ---------------------------------------------------------------------------
// One 256-thread workgroup per (chunk, head); wave w owns the 16-token row tile w and
// walks the V/16 column tiles, so its Qg and A operands are loaded once.
template <int K, int V>
__global__ __launch_bounds__(256) void chunk_fwd_output_kernel(FwdArgs a) {
  const int4 ch = ((const int4*)a.ws.p[R_CHUNKS])[blockIdx.x];
  const int len = ch.y;
  if (len <= 0) return;
  const int H = a.H, h = blockIdx.y;
  const size_t tile = (size_t)blockIdx.x * H + h;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;
  const int i = 16 * wave + lr;
  const bf16* QGF = (const bf16*)a.ws.p[R_QGF] + tile * 64 * K;
  const bf16* AF = (const bf16*)a.ws.p[R_AF] + tile * 64 * 64;
  const bf16* SHBF = (const bf16*)a.ws.p[R_SHBF] + tile * V * K;
  const bf16* DLF = (const bf16*)a.ws.p[R_DLF] + tile * 64 * V;
  bf16x8 fq[K / 32], fa[2];
#pragma unroll
  for (int s = 0; s < K / 32; ++s) fq[s] = *(const bf16x8*)(QGF + frag_off(K, wave, s, lane));
#pragma unroll
  for (int s = 0; s < 2; ++s) fa[s] = *(const bf16x8*)(AF + frag_off(64, wave, s, lane));
#pragma unroll 2
  for (int ct = 0; ct < V / 16; ++ct) {
    const int vcol = 16 * ct + lr;
    const bf16* sb = SHBF + (size_t)ct * 16 * K;
    const bf16* db = DLF + (size_t)ct * 16 * 64;
    f32x4 o0 = zero4(), o1 = zero4();
#pragma unroll
    for (int s = 0; s < K / 32; s += 2) {
      o0 = mfma16(fq[s], *(const bf16x8*)(sb + ((size_t)s * 64 + lane) * 8), o0);
      o1 = mfma16(fq[s + 1], *(const bf16x8*)(sb + ((size_t)(s + 1) * 64 + lane) * 8), o1);
    }
    o0 = mfma16(fa[0], *(const bf16x8*)(db + (size_t)lane * 8), o0);
    o1 = mfma16(fa[1], *(const bf16x8*)(db + (size_t)(64 + lane) * 8), o1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * wave + 4 * kg + r;
      if (t < len) a.out[((size_t)(ch.x + t) * H + h) * V + vcol] = to_bf16(o0[r] + o1[r]);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int validate_problem(const kda_chunk_problem* p, const char* who) {
  KDA_REQUIRE(p, "%s: null problem", who);
  KDA_REQUIRE(p->batch >= 0 && p->seq_len >= 0 && p->heads > 0, "%s: invalid B/T/H", who);
  KDA_REQUIRE(p->key_dim == 64 || p->key_dim == 128, "%s: key_dim must be 64 or 128", who);
  KDA_REQUIRE(p->value_dim == 64 || p->value_dim == 128, "%s: value_dim must be 64 or 128", who);
  KDA_REQUIRE(p->gate_mode == KDA_GATE_K3 || p->gate_mode == KDA_GATE_LOGDECAY,
              "%s: invalid gate_mode", who);
  if (p->cu_seqlens) {
    KDA_REQUIRE(p->batch == 1, "%s: cu_seqlens requires batch == 1", who);
    KDA_REQUIRE(p->num_seqs >= 1, "%s: cu_seqlens requires num_seqs >= 1", who);
  } else {
    KDA_REQUIRE(p->num_seqs == p->batch, "%s: num_seqs must equal batch without cu_seqlens", who);
  }
  KDA_REQUIRE(p->gate_mode != KDA_GATE_K3 || p->lower_bound < 0.f,
              "%s: lower_bound must be negative", who);
  return KDA_OK;
}

ChunkGeom make_geom(const kda_chunk_problem* p) {
  ChunkGeom g;
  const int nc = (p->seq_len + kChunk - 1) / kChunk;
  g.max_chunks = p->cu_seqlens ? nc + p->num_seqs : p->batch * nc;
  g.heads = p->heads;
  g.K = p->key_dim;
  g.V = p->value_dim;
  g.num_seqs = p->num_seqs;
  return g;
}

template <int K, int V>
static int launch_forward(const kda_chunk_problem* p, const ChunkGeom& g, FwdArgs& a,
                          hipStream_t stream, int stages) {
  if (g.max_chunks > 0 && (stages & (1 << KDA_STAGE_FWD_INTRA))) {
    constexpr size_t smem = IntraSmem<K, V>::bytes;
    static bool attr = false;
    if (!attr) {
      hipError_t e = hipFuncSetAttribute((const void*)chunk_fwd_intra_kernel<K, V>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      if (e != hipSuccess)
        return set_error(KDA_ERR_LAUNCH, "chunk_forward: LDS attribute: %s", hipGetErrorString(e));
      attr = true;
    }
    auto intra = chunk_fwd_intra_kernel<K, V>;
    hipLaunchKernelGGL(intra, dim3(g.max_chunks, p->heads), dim3(kIntraThreads),
                       smem, stream, a);
    KDA_LAUNCH_CHECK("chunk_forward intra");
  }
  if (p->num_seqs > 0 && (stages & (1 << KDA_STAGE_FWD_SCAN))) {
    auto scan = chunk_fwd_scan_kernel<K, V>;
    const int nrec = p->num_seqs * p->heads;
    const int grid = kXcds * (V / 16) * ((nrec + kXcds - 1) / kXcds);
    hipLaunchKernelGGL(scan, dim3(grid), dim3(256), 0, stream, a);
    KDA_LAUNCH_CHECK("chunk_forward scan");
  }
  if (g.max_chunks > 0 && (stages & (1 << KDA_STAGE_FWD_OUTPUT))) {
    auto outk = chunk_fwd_output_kernel<K, V>;
    hipLaunchKernelGGL(outk, dim3(g.max_chunks, p->heads), dim3(256), 0, stream, a);
    KDA_LAUNCH_CHECK("chunk_forward output");
  }
  return KDA_OK;
}

int launch_chunk_prep(const kda_chunk_problem* p, const ChunkGeom& g, const Regions& ws,
                      hipStream_t stream) {
  if (g.max_chunks == 0 && p->num_seqs == 0) return KDA_OK;
  hipLaunchKernelGGL(chunk_prep_kernel, dim3(1), dim3(256), 0, stream, p->batch, p->seq_len,
                     p->num_seqs, p->cu_seqlens, g.max_chunks, (int4*)ws.p[R_CHUNKS],
                     (int2*)ws.p[R_SEQS]);
  KDA_LAUNCH_CHECK("chunk_prep");
  return KDA_OK;
}

}  // namespace kda

extern "C" size_t kda_chunk_workspace_bytes(const kda_chunk_problem* p) {
  if (kda::validate_problem(p, "chunk_workspace_bytes") != KDA_OK) return 0;
  return kda::ws_total_bytes(kda::make_geom(p));
}

extern "C" size_t kda_chunk_backward_scratch_bytes(const kda_chunk_problem* p) {
  if (kda::validate_problem(p, "chunk_backward_scratch_bytes") != KDA_OK) return 0;
  return kda::sc_total_bytes(kda::make_geom(p));
}

static int chunk_forward_impl(int stages, const kda_chunk_problem* p, const void* q, const void* k,
                                 const void* v, const void* gate, const void* beta_logits,
                                 const float* A_log, const float* dt_bias,
                                 const float* initial_state, void* output, float* final_state,
                                 void* workspace, hipStream_t stream) {
  using namespace kda;
  int rc = validate_problem(p, "chunk_forward");
  if (rc != KDA_OK) return rc;
  const bool empty = (size_t)p->batch * p->seq_len == 0;
  KDA_REQUIRE(empty || (q && k && v && gate && beta_logits && output),
              "chunk_forward: null input/output pointer");
  KDA_REQUIRE(aligned16(q, k, v, gate, output, initial_state, final_state),
              "chunk_forward: q, k, v, gate, output and the states must be 16-byte aligned");
  KDA_REQUIRE(p->gate_mode != KDA_GATE_K3 || (A_log && dt_bias),
              "chunk_forward: K3 gate needs A_log and dt_bias");
  KDA_REQUIRE(workspace && ((uintptr_t)workspace % 256) == 0,
              "chunk_forward: workspace must be non-null and 256-byte aligned");
  const ChunkGeom g = make_geom(p);
  FwdArgs a;
  a.H = p->heads;
  a.num_seqs = p->num_seqs;
  a.gate_mode = p->gate_mode;
  a.lb = p->lower_bound;
  a.scale = p->scale;
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
  a.ws = ws_regions(g, workspace);
  if (stages & (1 << KDA_STAGE_PREP)) {
    rc = launch_chunk_prep(p, g, a.ws, stream);
    if (rc != KDA_OK) return rc;
  }
  if (p->key_dim == 128 && p->value_dim == 128) return launch_forward<128, 128>(p, g, a, stream, stages);
  if (p->key_dim == 64 && p->value_dim == 64) return launch_forward<64, 64>(p, g, a, stream, stages);
  if (p->key_dim == 128 && p->value_dim == 64) return launch_forward<128, 64>(p, g, a, stream, stages);
  return launch_forward<64, 128>(p, g, a, stream, stages);
}

extern "C" int kda_chunk_forward(const kda_chunk_problem* p, const void* q, const void* k,
                                 const void* v, const void* gate, const void* beta_logits,
                                 const float* A_log, const float* dt_bias,
                                 const float* initial_state, void* output, float* final_state,
                                 void* workspace, hipStream_t stream) {
  return chunk_forward_impl(~0, p, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state,
                            output, final_state, workspace, stream);
}

extern "C" int kda_chunk_forward_stage(int32_t stage, const kda_chunk_problem* p, const void* q,
                                       const void* k, const void* v, const void* gate,
                                       const void* beta_logits, const float* A_log,
                                       const float* dt_bias, const float* initial_state,
                                       void* output, float* final_state, void* workspace,
                                       hipStream_t stream) {
  if (stage != KDA_STAGE_PREP && stage != KDA_STAGE_FWD_INTRA && stage != KDA_STAGE_FWD_SCAN &&
      stage != KDA_STAGE_FWD_OUTPUT)
    return kda::set_error(KDA_ERR_INVALID, "chunk_forward_stage: unknown stage %d", stage);
  return chunk_forward_impl(1 << stage, p, q, k, v, gate, beta_logits, A_log, dt_bias,
                            initial_state, output, final_state, workspace, stream);
}
