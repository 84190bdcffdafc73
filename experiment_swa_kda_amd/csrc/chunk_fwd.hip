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
//  * intra kernel: one workgroup per (chunk, head) tile, everything staged in LDS (f32
//    qh/kh/G).  The 64x64 A and M' are built as 16x16 MFMA tiles
//    (v_mfma_f32_16x16x32_bf16).  Pairwise decays exp(G_i - G_j) are factorised around
//    the first row r of the row block: exp(G_i - G_r) <= 1 and, for j < r,
//    exp(G_r - G_j) <= 1, so no factor can overflow; only the diagonal block can, and a
//    diagonal block whose decay span exceeds 80 nats falls back to an exact per-pair
//    f32 loop.  T is formed in f32 by blocked forward substitution (16x16 blocks), then
//    U and W by MFMA.  Factors are written once to the workspace in both row- and
//    column-major form so every later MFMA operand is a contiguous 16-byte load.
//  * scan kernel: one workgroup per (sequence, head, 16-wide V strip) walks the chunks
//    in order; four compute waves hold the K x 16 f32 state slice in MFMA accumulators and
//    run delta = U - W S and S <- lam S + Kd^T delta, exchanging the packed state and the
//    delta tiles through LDS; two loader waves feed them through a direct global->LDS ring
//    and a store wave drains the bf16 state / delta histories.
//  * output kernel: O = Qg S + A delta, chunk-parallel after the scan; optionally the
//    mixer's output RMSNorm * sigmoid(gate) in its epilogue.
// Every reduction has a fixed order, so the forward is bitwise deterministic.
#include "chunk_host.hpp"
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

struct FwdArgs {
  int H;
  int num_seqs;
  int fixed_T;  // > 0: every sequence has this length and the intra kernel fills the tables
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
  // optional output RMSNorm * weight * sigmoid(gate) epilogue (all null / unused if ng_out is null)
  const bf16* ng_gate;
  long ng_gate_ld;  // elements between tokens' rows of ng_gate
  long beta_ld;     // elements between tokens' rows of beta
  const float* ng_weight;
  float ng_eps;
  bf16* ng_out;
  float* ng_inv_rms;
  // optional short convolution + SiLU prologue of the intra kernel (conv_x null: q, k, v
  // are the kernel's inputs).  conv_x rows are tokens (ld elements apart) holding the
  // pre-convolution q, k, v projections side by side (columns [0, HK), [HK, 2HK),
  // [2HK, 3HK)); conv_w is [3HK][conv_W] bf16 in the same channel order.  The intra kernel
  // writes the post-SiLU q, k, v to q, k, v (as bf16, the values it computes with).
  const bf16* conv_x;
  long conv_ld;
  const bf16* conv_w;
  int conv_W;
};

// Chunk table entry {row0, len, sequence, index}: arithmetic for sequences of one length.
template <class Args>
__device__ __forceinline__ int4 chunk_entry(const Args& a, int c) {
  if (a.fixed_T > 0) {
    const int nc = (a.fixed_T + kChunk - 1) / kChunk, sq = c / nc, j = c % nc;
    return make_int4(sq * a.fixed_T + j * kChunk, min(kChunk, a.fixed_T - j * kChunk), sq, j);
  }
  return ((const int4*)a.ws.p[R_CHUNKS])[c];
}

// Sequence table entry {first chunk, chunk count}: arithmetic for sequences of one length
// (no dependent load at a kernel's start), else the table chunk_prep_kernel built.
template <class Args>
__device__ __forceinline__ int2 seq_entry(const Args& a, int seq) {
  if (a.fixed_T > 0) {
    const int nc = (a.fixed_T + kChunk - 1) / kChunk;
    return make_int2(seq * nc, nc);
  }
  return ((const int2*)a.ws.p[R_SEQS])[seq];
}

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
// Column of element e held by lane group kg in 32-wide step s of a fragment: natural
// (32s + 8kg + e) or permuted to match two MFMA accumulator tiles (32s + 16(e/4) + 4kg +
// e%4: a lane's accumulator rows of tiles 2s and 2s+1), see the scan kernel.
template <bool PERM>
__device__ __forceinline__ int frag_col(int s, int kg, int e) {
  return PERM ? 32 * s + 16 * (e / 4) + 4 * kg + (e % 4) : 32 * s + 8 * kg + e;
}

// Writes the MFMA A-operand fragments of an R x C matrix whose element (r, c) is val(r, c)
// (see frag_off; PERM selects the permuted column order of frag_col); one 16-byte piece
// per thread iteration, contiguous across threads.
template <int R, int C, int NT, bool PERM = false, typename F>
__device__ __forceinline__ void emit_frags(bf16* dst, int tid, F val) {
  for (int idx = tid; idx < R * C / 8; idx += NT) {
    const int lane = idx % 64, s = (idx / 64) % (C / 32), rt = idx / (64 * (C / 32));
    const int r = 16 * rt + lane % 16, kg = lane / 16;
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = val(r, frag_col<PERM>(s, kg, e));
    *(bf16x8*)(dst + (size_t)idx * 8) = x;
  }
}

// emit_frags of the transpose of a row-major bf16 LDS matrix m (element (r, c) of the emitted
// R x C matrix is m[c][r]): each 16-byte piece is a column fragment of m, read with two
// transposing LDS reads instead of eight 2-byte ones.  NT must be a multiple of the wave
// size (the reads depend on the hardware lane), the pitch a multiple of 4 elements.
template <int R, int C, int NT, bool PERM = false>
__device__ __forceinline__ void emit_frags_tr(bf16* dst, int tid, const bf16* m, int pitch) {
  static_assert(NT % kWave == 0, "lanes of a piece are the hardware lanes");
  for (int idx = tid; idx < R * C / 8; idx += NT) {
    const int lane = idx % 64, s = (idx / 64) % (C / 32), rt = idx / (64 * (C / 32));
    bf16x8 x;
    if constexpr (PERM) {
      // elements 0..3: rows 32 s + 4 kg + e; 4..7: rows 32 s + 16 + 4 kg + e (frag_col<true>)
      x = lds_col_frag_split(m, pitch, 32 * s, 32 * s + 16, 16 * rt, lane);
    } else {
      x = lds_col_frag(m, pitch, 32 * s, 16 * rt, lane);  // rows 32 s + 8 kg + e
    }
    *(bf16x8*)(dst + (size_t)idx * 8) = x;
  }
}

// ---------------------------------------------------------------------------
// intra-chunk kernel
// ---------------------------------------------------------------------------
// One workgroup per (chunk, head) tile of 4 x kIntraNH waves; wave w owns the 16-row block
// rb = w % 4 and the channel part hh = w / 4 (K / kIntraNH channels; V likewise).  Lane
// (lr, kg) holds row 16rb + lr on the channels 32s + 8kg + e of its part (e < 8): exactly
// the A-operand fragments of its row block, so the bf16 MFMA operands of A and M' are
// formed in registers.  The in-chunk cumulative decay is a DPP scan across the 16 rows of
// a wave plus a 3-term prefix of the block totals; row norms are two permlane swaps and a
// sum over the parts through LDS.  A tile is a chain of short dependent phases (one tile
// alone on a CU is latency-bound), so the elementwise work, the A / M' products (partial
// sums over the channel parts, added in a fixed order) and the U / W products are split
// over the parts; the 16 x 16 triangular solves stay with part 0.  LDS stays under 80 KB
// so two tiles share a CU.
#ifndef KDA_INTRA_NH
#define KDA_INTRA_NH 2
#endif
constexpr int kIntraNH = KDA_INTRA_NH;
constexpr int kIntraThreads = 256 * kIntraNH;

template <int K, int V>
struct IntraLds {
  static constexpr int NS = K / 32;
  static constexpr int RS = K + 8;   // bf16 row stride of [64][K] staging
  static constexpr int cmax(int a, int b) { return a > b ? a : b; }
  static constexpr int VS = V + 8;   // bf16 row stride of [64][V] staging
  static_assert(RS % 8 == 0 && VS % 8 == 0, "vector rows and transposing reads need 16-byte rows");
  // X1: Fq / Fk fragments (A, M') -> beta v, beta kh e^G (U, W) -> Qg, Kd staging
  static constexpr int x1 = 0;
  static constexpr int x1_bytes = cmax(cmax(2 * 64 * K * 2, 64 * (VS + RS) * 2), 2 * 64 * RS * 2);
  // X3: M' f32 [64][65] -> W bf16 [64][RS]
  static constexpr int x3 = x1 + x1_bytes;
  static constexpr int x3_bytes = cmax(64 * 65 * 4, 64 * RS * 2);
  // X4: A f32 [64][65] -> T f32 [64][65]
  static constexpr int x4 = x3 + x3_bytes;
  static constexpr int x4_bytes = 64 * 65 * 4;
  // per-wave 16 x 17 f32 product scratch (T solve)
  static constexpr int scr = x4 + x4_bytes;
  static constexpr int scr_bytes = 4 * 16 * 17 * 4;
  static constexpr int gref = scr + scr_bytes;   // f32 [5][K]: G of rows 0, 16, 32, 48 and 63
  static constexpr int tot = gref + 5 * K * 4;   // f32 [4][K]: block totals of g
  static constexpr int beta = tot + 4 * K * 4;   // f32 [64]
  static constexpr int nrm = beta + 64 * 4;      // f32 [parts][64][2]: per-part sums of q^2, k^2
  static constexpr int wide = nrm + kIntraNH * 64 * 2 * 4;  // int [8]: per-wave wide-diagonal flags
  static constexpr int bytes = wide + 8 * 4;
};

template <int CTRL>
__device__ __forceinline__ float dpp_shr(float v) {
  // row_shr with bound_ctrl: lanes shifted in from outside the 16-lane row read 0
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Inclusive prefix sum across the 16 lanes of each DPP row (lane order = row order).
__device__ __forceinline__ float row_prefix16(float x) {
  x += dpp_shr<0x111>(x);
  x += dpp_shr<0x112>(x);
  x += dpp_shr<0x114>(x);
  x += dpp_shr<0x118>(x);
  return x;
}

// Exact A / M' entries of a diagonal block whose decay span is too large for the
// factorised MFMA form: lane (lr, kg) computes (i = 16w + 4kg + r, j = 16w + lr), r < 4,
// from the global inputs and the G rows this workgroup already wrote.
template <int K>
__device__ void intra_exact_block(const FwdArgs& a, int w, int lane, int row0, int len, int h,
                                  const float* G, const float* RQ, const float* RK, f32x4& accA,
                                  f32x4& accM) {
  const int lr = lane % 16, kg = lane / 16, H = a.H;
  const int j = 16 * w + lr;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 16 * w + 4 * kg + r;
    float sa = 0.f, sm = 0.f;
    if (j <= i && i < len) {
      const size_t bi = ((size_t)(row0 + i) * H + h) * K, bj = ((size_t)(row0 + j) * H + h) * K;
      const float rqi = RQ[i], rki = RK[i], rkj = RK[j];
#pragma unroll 1
      for (int c0 = 0; c0 < K; c0 += 8) {
        const bf16x8 qi = *(const bf16x8*)(a.q + bi + c0), ki = *(const bf16x8*)(a.k + bi + c0),
                     kj = *(const bf16x8*)(a.k + bj + c0);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = expf(G[i * K + c0 + e] - G[j * K + c0 + e]) * (float)kj[e] * rkj;
          sa = fmaf((float)qi[e] * rqi, d, sa);
          sm = fmaf((float)ki[e] * rki, d, sm);
        }
      }
    }
    accA[r] = sa;
    accM[r] = sm;
  }
}

// ---------------------------------------------------------------------------
// short convolution + SiLU prologue (fused conv path)
// ---------------------------------------------------------------------------
// Lane (lr, kg) of wave w holds token row i = 16 w + lr of the chunk.  The convolution of
// row i needs rows i-1 .. i-(W-1): within the wave they are the rows of lanes lr-1 ..
// (DPP row shift); rows before the wave's block come from a halo row that lanes 13..15
// load (row i - 16) and a DPP row rotate hands to lanes 0..2.  Rows before the sequence
// start are zero (no convolution state on this path).  Arithmetic and rounding follow the
// separate convolution kernel exactly (f32 fma chain over the taps in order, sigmoid_fast,
// one bf16 rounding), so the fused path reproduces the unfused one bit for bit.
template <int SHIFT>
__device__ __forceinline__ unsigned row_take(unsigned own, unsigned halo, int lr) {
  const unsigned a = (unsigned)__builtin_amdgcn_update_dpp(0, (int)own, 0x110 + SHIFT, 0xf, 0xf, true);   // row_shr
  const unsigned b = (unsigned)__builtin_amdgcn_update_dpp(0, (int)halo, 0x120 + SHIFT, 0xf, 0xf, false); // row_ror
  return lr >= SHIFT ? a : b;
}

template <int W>
__device__ __forceinline__ bf16x8 conv_silu8(bf16x8 own, bf16x8 halo, const float* wt, int lr) {
  // xs[j] = row i - (W-1) + j, j = W-1 the own row
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 o = __builtin_bit_cast(u4, own), hl = __builtin_bit_cast(u4, halo);
  bf16x8 xs[W];
  xs[W - 1] = own;
#pragma unroll
  for (int d = 1; d < W; ++d) {
    u4 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (d == 1) r[q] = row_take<1>(o[q], hl[q], lr);
      if (d == 2) r[q] = row_take<2>(o[q], hl[q], lr);
      if (d == 3) r[q] = row_take<3>(o[q], hl[q], lr);
    }
    xs[W - 1 - d] = __builtin_bit_cast(bf16x8, r);
  }
  bf16x8 y;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float pre = 0.f;
#pragma unroll
    for (int j = 0; j < W; ++j) pre = fmaf((float)xs[j][e], wt[e * 4 + j], pre);
    y[e] = to_bf16(pre * sigmoid_fast(pre));
  }
  return y;
}

template <int K, int V, bool CONV = false>
__global__ __launch_bounds__(kIntraThreads, 2 * kIntraNH) void chunk_fwd_intra_kernel(FwdArgs a) {
  using L = IntraLds<K, V>;
  constexpr int NH = kIntraNH;
  constexpr int NS = K / 32, NV = V / 32, RS = L::RS;
  constexpr int NSH = NS / NH, NVH = NV / NH;  // 32-channel steps of this wave's part (K, V)
  static_assert(NH == 1 || NH == 2, "one or two channel parts");
  static_assert(NS % NH == 0 && NV % NH == 0 && (V / 16) % NH == 0 && (K / 16) % NH == 0, "even channel parts");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* sF = (bf16*)(smem + L::x1);        // Fq / Fk fragments
  constexpr int VS = L::VS;
  bf16* sBV = (bf16*)(smem + L::x1);       // beta v [64][VS]
  bf16* sBK = sBV + 64 * VS;               // beta kh e^G [64][RS]
  bf16* sQg = (bf16*)(smem + L::x1);       // Qg [64][RS]
  bf16* sKd = sQg + 64 * RS;               // Kd [64][RS]
  float* sM = (float*)(smem + L::x3);      // M' [64][65]
  bf16* sW = (bf16*)(smem + L::x3);        // W [64][RS]
  float* sA = (float*)(smem + L::x4);      // A [64][65]
  float* sT = (float*)(smem + L::x4);      // T [64][65]
  float* sScr = (float*)(smem + L::scr);
  float* sGref = (float*)(smem + L::gref);
  float* sTot = (float*)(smem + L::tot);
  float* sBeta = (float*)(smem + L::beta);
  float* sNrm = (float*)(smem + L::nrm);
  int* sWide = (int*)(smem + L::wide);

  // Fixed-length problems derive their chunk from the index and publish the chunk and
  // sequence tables for the later kernels (which run after this one on the stream);
  // variable-length problems read the tables chunk_prep_kernel built.
  int4 ch;
  if (a.fixed_T > 0) {
    const int nc = (a.fixed_T + kChunk - 1) / kChunk;
    const int sq = blockIdx.x / nc, j = blockIdx.x % nc;
    ch = make_int4(sq * a.fixed_T + j * kChunk, min(kChunk, a.fixed_T - j * kChunk), sq, j);
    if (blockIdx.y == 0 && threadIdx.x == 0) {
      ((int4*)a.ws.p[R_CHUNKS])[blockIdx.x] = ch;
      if (j == 0) ((int2*)a.ws.p[R_SEQS])[sq] = make_int2(blockIdx.x, nc);
    }
  } else {
    ch = ((const int4*)a.ws.p[R_CHUNKS])[blockIdx.x];
  }
  const int len = ch.y;
  if (len <= 0) return;
  const int H = a.H, h = blockIdx.y;
  const size_t tile = (size_t)blockIdx.x * H + h;
  const int row0 = ch.x;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  const int rb = w % 4, hh = w / 4;  // row block, channel part
  const int lr = lane % 16, kg = lane / 16;
  const int i = 16 * rb + lr;
  const bool live = i < len;
  const size_t rbase = (size_t)(row0 + (live ? i : len - 1)) * H + h;
  // channel step s' of this wave's part is the global step S(s') = NSH hh + s' (V: NVH hh + s')
  auto S = [&](int s) { return NSH * hh + s; };
  auto SV = [&](int s) { return NVH * hh + s; };

  // ---- phase 1: loads (all issued first), norms, gate, beta, cumulative decay ----
  bf16x8 qr[NSH], kr[NSH];
  float g[NSH][8];
  if constexpr (CONV) {
    static_assert(K == V, "the fused convolution serves q, k, v of one head width");
    // taps of this head's q, k, v channels as f32 [3][K][4] in the (still unused) X1 region
    float* sWt = (float*)(smem + L::x1);
    const int HK = H * K, W = a.conv_W;
    for (int idx = tid; idx < 3 * K; idx += kIntraThreads) {
      const int t = idx / K, c = idx % K;
      const bf16* src = a.conv_w + (size_t)(t * HK + h * K + c) * W;
      float4 wv = make_float4(0.f, 0.f, 0.f, 0.f);
      wv.x = (float)src[0];
      if (W > 1) wv.y = (float)src[1];
      if (W > 2) wv.z = (float)src[2];
      if (W > 3) wv.w = (float)src[3];
      *(float4*)(sWt + idx * 4) = wv;
    }
    // own rows (clamped like rbase) and, for lanes 13..15, the halo row i - 16 (zero before
    // the sequence start); every load issued before the first use
    const int pos = ch.w * kChunk + i;  // token index in the sequence
    const bf16* xo = a.conv_x + (size_t)(row0 + (live ? i : len - 1)) * a.conv_ld + h * K + 8 * kg;
    // halo row i - 16 of lanes 13..15: a token of this sequence and of this chunk's rows
    // (lanes 13..15 themselves may lie past a partial chunk's end)
    const bool has_halo = lr >= 13 && pos >= 16 && i - 16 < len;
    const bf16* xh = has_halo ? a.conv_x + (size_t)(row0 + i - 16) * a.conv_ld + h * K + 8 * kg
                              : xo;  // the own row (unused)
    bf16x8 ho[3][NSH], vr[NSH];
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      qr[s] = *(const bf16x8*)(xo + 32 * S(s));
      kr[s] = *(const bf16x8*)(xo + HK + 32 * S(s));
      vr[s] = *(const bf16x8*)(xo + 2 * HK + 32 * S(s));
    }
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      ho[0][s] = *(const bf16x8*)(xh + 32 * S(s));
      ho[1][s] = *(const bf16x8*)(xh + HK + 32 * S(s));
      ho[2][s] = *(const bf16x8*)(xh + 2 * HK + 32 * S(s));
      if (!has_halo)
#pragma unroll
        for (int e = 0; e < 8; ++e) ho[0][s][e] = ho[1][s][e] = ho[2][s][e] = to_bf16(0.f);
    }
    __syncthreads();  // taps staged
    bf16* qo = (bf16*)a.q + rbase * K + 8 * kg;
    bf16* ko = (bf16*)a.k + rbase * K + 8 * kg;
    bf16* vo = (bf16*)a.v + rbase * V + 8 * kg;
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      const int c0 = 32 * S(s) + 8 * kg;
      if (W == 4) {
        qr[s] = conv_silu8<4>(qr[s], ho[0][s], sWt + (0 * K + c0) * 4, lr);
        kr[s] = conv_silu8<4>(kr[s], ho[1][s], sWt + (1 * K + c0) * 4, lr);
        vr[s] = conv_silu8<4>(vr[s], ho[2][s], sWt + (2 * K + c0) * 4, lr);
      } else if (W == 3) {
        qr[s] = conv_silu8<3>(qr[s], ho[0][s], sWt + (0 * K + c0) * 4, lr);
        kr[s] = conv_silu8<3>(kr[s], ho[1][s], sWt + (1 * K + c0) * 4, lr);
        vr[s] = conv_silu8<3>(vr[s], ho[2][s], sWt + (2 * K + c0) * 4, lr);
      } else if (W == 2) {
        qr[s] = conv_silu8<2>(qr[s], ho[0][s], sWt + (0 * K + c0) * 4, lr);
        kr[s] = conv_silu8<2>(kr[s], ho[1][s], sWt + (1 * K + c0) * 4, lr);
        vr[s] = conv_silu8<2>(vr[s], ho[2][s], sWt + (2 * K + c0) * 4, lr);
      } else {
        qr[s] = conv_silu8<1>(qr[s], ho[0][s], sWt + (0 * K + c0) * 4, lr);
        kr[s] = conv_silu8<1>(kr[s], ho[1][s], sWt + (1 * K + c0) * 4, lr);
        vr[s] = conv_silu8<1>(vr[s], ho[2][s], sWt + (2 * K + c0) * 4, lr);
      }
      if (live) {
        *(bf16x8*)(qo + 32 * S(s)) = qr[s];
        *(bf16x8*)(ko + 32 * S(s)) = kr[s];
        *(bf16x8*)(vo + 32 * S(s)) = vr[s];
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      qr[s] = *(const bf16x8*)(a.q + rbase * K + 32 * S(s) + 8 * kg);
      kr[s] = *(const bf16x8*)(a.k + rbase * K + 32 * S(s) + 8 * kg);
    }
  }
  const float bl = (float)a.beta[(size_t)(row0 + (live ? i : len - 1)) * a.beta_ld + h];
  if (a.gate_mode == KDA_GATE_K3) {
    const float ea = expf(a.A_log[h]);
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      const int c0 = 32 * S(s) + 8 * kg;
      const bf16x8 raw = *(const bf16x8*)((const bf16*)a.gate + rbase * K + c0);
      float db[8];
      load8f(a.dt_bias + h * K + c0, db);
#pragma unroll
      for (int e = 0; e < 8; ++e) g[s][e] = a.lb * sigmoid_fast(ea * ((float)raw[e] + db[e]));
    }
  } else {
#pragma unroll
    for (int s = 0; s < NSH; ++s) load8f((const float*)a.gate + rbase * K + 32 * S(s) + 8 * kg, g[s]);
  }
  // q and k stay bf16 in registers (rows past the chunk end zeroed); the normalised values
  // qh = q rq, kh = k rk are formed in f32 where they are used
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int s = 0; s < NSH; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (!live) {
        qr[s][e] = to_bf16(0.f);
        kr[s][e] = to_bf16(0.f);
        g[s][e] = 0.f;
      }
      sq = fmaf((float)qr[s][e], (float)qr[s][e], sq);
      sk = fmaf((float)kr[s][e], (float)kr[s][e], sk);
      g[s][e] = row_prefix16(g[s][e]);  // inclusive in-block prefix over the 16 rows
    }
  sq = swap32_sum(swap16_sum(sq));
  sk = swap32_sum(swap16_sum(sk));
  if (NH > 1 && kg == 0) {  // this part's sums of squares; the parts add up after the barrier
    sNrm[(hh * 64 + i) * 2] = sq;
    sNrm[(hh * 64 + i) * 2 + 1] = sk;
  }
  if (lr == 15) {
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      float* t = sTot + rb * K + 32 * S(s) + 8 * kg;
      *(float4*)t = make_float4(g[s][0], g[s][1], g[s][2], g[s][3]);
      *(float4*)(t + 4) = make_float4(g[s][4], g[s][5], g[s][6], g[s][7]);
    }
  }
  __syncthreads();
  if (NH > 1) {  // fixed order: part 0 + part 1 in every wave
    sq = sNrm[i * 2] + sNrm[(64 + i) * 2];
    sk = sNrm[i * 2 + 1] + sNrm[(64 + i) * 2 + 1];
  }
  const float rq = a.scale / fmaxf(sqrtf(sq), 1e-12f);
  const float rk = 1.0f / fmaxf(sqrtf(sk), 1e-12f);
  const float beta = live ? sigmoid_acc(bl) : 0.f;
  auto qh = [&](int s, int e) { return (float)qr[s][e] * rq; };
  auto kh = [&](int s, int e) { return (float)kr[s][e] * rk; };
  if (hh == 0 && kg == 0) {
    sBeta[i] = beta;
    ((float*)a.ws.p[R_RQ])[tile * 64 + i] = rq;
    ((float*)a.ws.p[R_RK])[tile * 64 + i] = rk;
    ((float*)a.ws.p[R_BETA])[tile * 64 + i] = beta;
  }
  // G = in-block prefix + totals of the preceding blocks (fixed order)
  for (int b = 0; b < rb; ++b) {
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      float t[8];
      load8f(sTot + b * K + 32 * S(s) + 8 * kg, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) g[s][e] += t[e];
    }
  }
  float* Gout = (float*)a.ws.p[R_G] + tile * 64 * K;
#pragma unroll
  for (int s = 0; s < NSH; ++s) {
    float* o = Gout + i * K + 32 * S(s) + 8 * kg;
    *(float4*)o = make_float4(g[s][0], g[s][1], g[s][2], g[s][3]);
    *(float4*)(o + 4) = make_float4(g[s][4], g[s][5], g[s][6], g[s][7]);
    if (lr == 0 || i == 63) {
      float* r = sGref + (lr == 0 ? rb : 4) * K + 32 * S(s) + 8 * kg;
      *(float4*)r = make_float4(g[s][0], g[s][1], g[s][2], g[s][3]);
      *(float4*)(r + 4) = make_float4(g[s][4], g[s][5], g[s][6], g[s][7]);
    }
  }
  __syncthreads();

  // ---- phase 2: A and M' = (factorised) 16 x 16 blocks; row factors e^{G_i - G_r} ----
  bool wide = false;  // this row block's diagonal block spans more than 80 nats on some channel
  {
    float gr[NSH][8];
#pragma unroll
    for (int s = 0; s < NSH; ++s) load8f(sGref + rb * K + 32 * S(s) + 8 * kg, gr[s]);
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      bf16x8 fq, fk;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = __expf(g[s][e] - gr[s][e]);
        fq[e] = (bf16)(qh(s, e) * f);
        fk[e] = (bf16)(kh(s, e) * f);
        wide |= (lr == 15) && (gr[s][e] - g[s][e] > 80.f);
      }
      *(bf16x8*)(sF + ((size_t)(rb * NS + S(s)) * 64 + lane) * 8) = fq;
      *(bf16x8*)(sF + ((size_t)((4 + rb) * NS + S(s)) * 64 + lane) * 8) = fk;
    }
  }
  wide = __builtin_amdgcn_ballot_w64(wide) != 0;
  if (NH > 1 && lane == 0) sWide[w] = wide;
  // A and M' start as zero: entries outside the masks (and the blocks above the diagonal)
  // are never written
  for (int idx = tid; idx < 64 * 65 / 4; idx += kIntraThreads) {
    ((float4*)sA)[idx] = make_float4(0.f, 0.f, 0.f, 0.f);
    ((float4*)sM)[idx] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __syncthreads();  // also drains the G, RQ, RK stores: the exact diagonal path reads them back
  if (NH > 1) wide = (sWide[rb] | sWide[4 + rb]) != 0;
  // wave (rb, hh) computes the pairs (ba, rb) for ba >= rb over its channel part, one pair
  // per round: part 0 stores its partial products, part 1 adds its own after the round's
  // barrier (fixed order; one pair's accumulators held at a time)
  const int jj = 16 * rb + lr;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int ba = rb + q;
    const bool pair = ba < 4 && !(ba == rb && wide);  // a wide diagonal block: exact path below
    f32x4 accA = zero4(), accM = zero4();
    if (pair) {
      float gr[NSH][8];
#pragma unroll
      for (int s = 0; s < NSH; ++s) load8f(sGref + ba * K + 32 * S(s) + 8 * kg, gr[s]);
#pragma unroll
      for (int s = 0; s < NSH; ++s) {
        bf16x8 cf;
#pragma unroll
        for (int e = 0; e < 8; ++e) cf[e] = (bf16)(kh(s, e) * __expf(gr[s][e] - g[s][e]));
        accA = mfma16(*(const bf16x8*)(sF + ((size_t)(ba * NS + S(s)) * 64 + lane) * 8), cf, accA);
        accM = mfma16(*(const bf16x8*)(sF + ((size_t)((4 + ba) * NS + S(s)) * 64 + lane) * 8), cf, accM);
      }
      if (hh == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ii = 16 * ba + 4 * kg + r;
          if (jj <= ii) sA[ii * 65 + jj] = accA[r];
          if (jj < ii) sM[ii * 65 + jj] = accM[r];
        }
      }
    }
    if (NH > 1) {
      __syncthreads();
      if (hh == 1 && pair) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ii = 16 * ba + 4 * kg + r;
          if (jj <= ii) sA[ii * 65 + jj] += accA[r];
          if (jj < ii) sM[ii * 65 + jj] += accM[r];
        }
      }
    }
  }
  if (wide && hh == 0) {  // part 0 computes the whole exact diagonal block (rare)
    f32x4 accA, accM;
    __threadfence_block();
    intra_exact_block<K>(a, rb, lane, row0, len, h, Gout, (const float*)a.ws.p[R_RQ] + tile * 64,
                         (const float*)a.ws.p[R_RK] + tile * 64, accA, accM);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ii = 16 * rb + 4 * kg + r;
      if (jj <= ii) sA[ii * 65 + jj] = accA[r];
      if (jj < ii) sM[ii * 65 + jj] = accM[r];
    }
  }
  __syncthreads();

  // ---- phase 2b: A fragments, M' to HBM, beta v and beta kh e^G (natural rows) to LDS ----
  // v again (from L2; the fused convolution wrote it above): not held across phases 1-2
  bf16x8 vr2[NVH];
#pragma unroll
  for (int s = 0; s < NVH; ++s) vr2[s] = *(const bf16x8*)(a.v + rbase * V + 32 * SV(s) + 8 * kg);
  emit_frags<64, 64, kIntraThreads, true>((bf16*)a.ws.p[R_AF] + tile * 64 * 64, tid,
                                          [&](int r, int c) { return (bf16)sA[r * 65 + c]; });
  {
    float* MPout = (float*)a.ws.p[R_MP] + tile * 64 * 64;
    for (int idx = tid; idx < 64 * 64; idx += kIntraThreads) MPout[idx] = sM[(idx / 64) * 65 + idx % 64];
  }
  // beta v and beta kh e^G overwrite the Fq / Fk fragments (read by every wave above)
#pragma unroll
  for (int s = 0; s < NVH; ++s) {
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (bf16)(beta * (live ? (float)vr2[s][e] : 0.f));
    *(bf16x8*)(sBV + i * VS + 32 * SV(s) + 8 * kg) = x;
  }
#pragma unroll
  for (int s = 0; s < NSH; ++s) {
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (bf16)(beta * kh(s, e) * __expf(g[s][e]));
    *(bf16x8*)(sBK + i * RS + 32 * S(s) + 8 * kg) = x;
  }
  // Qg = qh e^G and Kd = kh e^{G_last - G} (bf16) are all that phase 5 needs of this row;
  // Kd's natural fragments are exactly what this lane holds
  bf16x8 xq[NSH], xk[NSH];
  {
    bf16* KDF = (bf16*)a.ws.p[R_KDF] + tile * 64 * K;
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      float gl[8];
      load8f(sGref + 4 * K + 32 * S(s) + 8 * kg, gl);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xq[s][e] = (bf16)(qh(s, e) * __expf(g[s][e]));
        xk[s][e] = (bf16)(kh(s, e) * __expf(gl[e] - g[s][e]));
      }
      *(bf16x8*)(KDF + frag_off(K, rb, S(s), lane)) = xk[s];
    }
  }
  __syncthreads();

  // ---- phase 3: T = (I + diag(beta) M')^-1 (waves of part 0) ----
  // Diagonal blocks: N = diag(beta) M' on a 16 x 16 diagonal block is strictly lower, so
  // N^16 = 0 and (I + N)^-1 = (I + P)(I + P^2)(I + P^4)(I + P^8) with P = -N: three
  // squarings and three updates X <- X + X P^(2^k), every product four
  // v_mfma_f32_16x16x4_f32 steps on registers.  A matrix M is held in the accumulator layout
  // (lane (c, q) holds M[4q + r][c], r < 4); with the contraction index of step s and lane
  // group q taken as k = 4q + s, that layout is the B operand as it stands and the A operand
  // of M^T, so each matrix is carried together with its transpose (P with Q = P^T, X with
  // Y = X^T).  All 64 lanes work, and the chain is 6 products deep instead of a 16-step
  // substitution per column.
  {
    const int o = 16 * rb;
    if (hh == 0) {
      auto mm = [&](const f32x4& at, const f32x4& b, f32x4 acc) {  // acc + A B, at = A^T's registers
#pragma unroll
        for (int st = 0; st < 4; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(at[st], b[st], acc, 0, 0, 0);
        return acc;
      };
      f32x4 P, Q, X, Y;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ii = 4 * kg + r;  // row of this register, lr the column
        P[r] = ii > lr ? -sBeta[o + ii] * sM[(o + ii) * 65 + o + lr] : 0.f;  // -N[ii][lr]
        Q[r] = lr > ii ? -sBeta[o + lr] * sM[(o + lr) * 65 + o + ii] : 0.f;  // -N[lr][ii]
        X[r] = P[r] + (ii == lr ? 1.f : 0.f);
        Y[r] = Q[r] + (ii == lr ? 1.f : 0.f);
      }
#pragma unroll
      for (int it = 0; it < 3; ++it) {
        const f32x4 P2 = mm(Q, P, zero4());  // P^2 (A = P through Q = P^T)
        const f32x4 Xn = mm(Y, P2, X);       // X + X P^2
        if (it < 2) {
          const f32x4 Q2 = mm(P, Q, zero4());  // (P^2)^T = Q Q
          Y = mm(P2, Y, Y);                    // Y + (P^2)^T Y = (X + X P^2)^T
          Q = Q2;
        }
        P = P2;
        X = Xn;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) sT[(o + 4 * kg + r) * 65 + o + lr] = X[r];
      for (int idx = lane; idx < 16 * 16 * (3 - rb); idx += kWave) {  // zero blocks right of the diagonal
        const int cb = rb + 1 + idx / 256, rr = (idx % 256) / 16, cc = idx % 16;
        sT[(o + rr) * 65 + 16 * cb + cc] = 0.f;
      }
    }
  }
  __syncthreads();
  // off-diagonal blocks by levels: T_ab = -D_a sum_{m=b}^{a-1} N_am T_mb, N = diag(beta) M'.
  // 16 x 16 x 16 f32 products on v_mfma_f32_16x16x4_f32 (A[lr][kg], B[kg][lr] per 4-step).
  auto prod_NT = [&](int ra, int cm, int cb, f32x4 acc) {  // acc += N[ra-block][cm-block] T[cm][cb]
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kk = 4 * st + kg;
      const float av = sBeta[16 * ra + lr] * sM[(16 * ra + lr) * 65 + 16 * cm + kk];
      const float bv = sT[(16 * cm + kk) * 65 + 16 * cb + lr];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
    }
    return acc;
  };
  float* scr = sScr + rb * 16 * 17;
  for (int lvl = 1; lvl < 4; ++lvl) {
    const int b = rb, ra = rb + lvl;
    if (hh == 0 && ra < 4) {
      f32x4 z = zero4();
      for (int m = b; m < ra; ++m) z = prod_NT(ra, m, b, z);
#pragma unroll
      for (int r = 0; r < 4; ++r) scr[(4 * kg + r) * 17 + lr] = z[r];
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave reads its own scratch next
      f32x4 t = zero4();
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int kk = 4 * st + kg;
        t = __builtin_amdgcn_mfma_f32_16x16x4f32(sT[(16 * ra + lr) * 65 + 16 * ra + kk], scr[kk * 17 + lr], t, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) sT[(16 * ra + 4 * kg + r) * 65 + 16 * b + lr] = -t[r];
    }
    __syncthreads();
  }
  {
    bf16* Tout = (bf16*)a.ws.p[R_T] + tile * 64 * 64;
    for (int idx = 4 * tid; idx < 64 * 64; idx += 4 * kIntraThreads) {
      const float* t = sT + (idx / 64) * 65 + idx % 64;
      bf16x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = to_bf16(t[e]);
      *(bf16x4*)(Tout + idx) = x;
    }
  }

  // ---- phase 4: U = T (beta v), W = T (beta kh e^G); wave (rb, hh) = row tile rb, column
  // tiles of part hh ----
  {
    const int rt = rb, nst = (16 * rt + 15) / 32 + 1;
    bf16x8 fa[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      bf16x8 x;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (bf16)sT[(16 * rt + lr) * 65 + 32 * st + 8 * kg + e];
      fa[st] = x;
    }
    bf16* Uout = (bf16*)a.ws.p[R_UF] + tile * 64 * V;
    constexpr int UCT = V / 16 / NH, WCT = K / 16 / NH;
#pragma unroll
    for (int c = 0; c < UCT; ++c) {
      const int ct = UCT * hh + c;
      f32x4 acc = zero4();
#pragma unroll
      for (int st = 0; st < 2; ++st)  // T is lower triangular: row tile rt needs nst steps
        if (st < nst) acc = mfma16(fa[st], lds_col_frag(sBV, VS, 32 * st, 16 * ct, lane), acc);
      bf16x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = (bf16)acc[r];
      *(bf16x4*)(Uout + ((size_t)(ct * 4 + rt) * 64 + lane) * 4) = x;
    }
    __syncthreads();  // M' (aliasing W) is no longer read
#pragma unroll
    for (int c = 0; c < WCT; ++c) {
      const int ct = WCT * hh + c;
      f32x4 acc = zero4();
#pragma unroll
      for (int st = 0; st < 2; ++st)
        if (st < nst) acc = mfma16(fa[st], lds_col_frag(sBK, RS, 32 * st, 16 * ct, lane), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) sW[(16 * rt + 4 * kg + r) * RS + 16 * ct + lr] = (bf16)acc[r];
    }
  }
  __syncthreads();
  // -W fragments; Qg and Kd staged for their permuted / transposed fragments (the
  // backward forms W^T, Qg^T and A^T operands with transposing LDS reads, so only Kd^T, which
  // the forward scan streams, is stored in both orientations)
  emit_frags<64, K, kIntraThreads, true>((bf16*)a.ws.p[R_WF] + tile * 64 * K, tid,
                                         [&](int r, int c) { return (bf16)(-(float)sW[r * RS + c]); });
#pragma unroll
  for (int s = 0; s < NSH; ++s) {
    *(bf16x8*)(sQg + i * RS + 32 * S(s) + 8 * kg) = xq[s];
    *(bf16x8*)(sKd + i * RS + 32 * S(s) + 8 * kg) = xk[s];
  }
  __syncthreads();
  emit_frags<64, K, kIntraThreads, true>((bf16*)a.ws.p[R_QGF] + tile * 64 * K, tid,
                                         [&](int r, int c) { return sQg[r * RS + c]; });
  emit_frags_tr<K, 64, kIntraThreads, true>((bf16*)a.ws.p[R_KDTF] + tile * K * 64, tid, sKd, RS);
  // lam = e^{G_last}, one channel per thread from the staged last row (off the critical
  // path: computed by the lanes holding row 63 it delayed every wave at the cumulative-decay
  // barrier)
  if (tid < K) ((float*)a.ws.p[R_LAM])[tile * K + tid] = expf(sGref[4 * K + tid]);
}

// ---------------------------------------------------------------------------
// inter-chunk state scan
// ---------------------------------------------------------------------------
// One workgroup per (sequence, head, 16-wide V strip): four compute waves, two loader waves
// and a store wave.  The V columns of the state evolve independently, so strips never
// communicate.
//
// The K x 16 f32 state slice is held as K/16 MFMA accumulator tiles (lane l: rows
// 16kt + 4(l/16) + r, column l%16), split evenly over the compute waves; each chunk step is
//   delta = U + (-W) S     (S as the B operand; U is the accumulator input),
//   S     = lam S + Kd^T delta  (delta as B; lam S is the accumulator input).
// Compute wave c owns the 16-token delta row tile c and state tiles c K/64 .. (c+1) K/64 - 1.
// The B operand of a 32-deep MFMA step wants 8 values per lane; the two accumulator tiles
// 2s and 2s+1 give a lane exactly 8 values of its column, so the intra kernel stores W and
// Qg with their key columns (and Kd^T and A with their token columns) in the matching
// permuted order (frag_col<true>): an accumulator becomes the next product's operand with
// one conversion.  The waves exchange the packed state and the delta tiles through LDS and
// meet at two barriers per chunk:
//   B1(ci): slot ci loaded, state entering chunk ci staged -> each wave's delta tile
//           (one K/32-deep MFMA chain)
//   B2(ci): every delta tile staged -> each wave's state tiles (two MFMAs each).
// Split over four SIMDs the step's dependent chain is K/32 + 2 MFMAs deep instead of the
// single-wave 16 + 16.
//
// The loader waves stream each chunk's -W and Kd^T fragments, U strip and lam into a
// kScanRing-deep LDS ring with direct global->LDS loads, kScanRing - 1 chunks ahead (the
// step is bound by memory latency: a deeper ring measured faster).  The compute waves write
// the f32 state history straight to HBM (nothing in their stream waits on those stores);
// the store wave copies the bf16 state and delta histories out of the double-buffered
// exchange one step later.
constexpr int kScanRing = 4;
constexpr int kScanCompute = 4;                 // compute waves (one 16-token delta tile each)
constexpr int kScanThreads = (kScanCompute + 3) * kWave;  // + two loader waves and a store wave

template <int K, int V>
struct ScanLds {
  static constexpr int off_w = 0;                       // -W fragments, 64 x K bf16
  static constexpr int off_kdt = off_w + 64 * K * 2;    // Kd^T fragments, K x 64 bf16
  static constexpr int off_u = off_kdt + K * 64 * 2;    // U strip, C layout, 64 x 16 bf16
  static constexpr int off_lam = off_u + 64 * 16 * 2;   // lam, K f32
  static constexpr int slot = off_lam + K * 4;
  static constexpr int n_load0 = (64 * K * 2) / 1024 + 2;  // loader 0: W blocks + U strip
  static constexpr int n_load1 = (K * 64 * 2) / 1024 + 1;  // loader 1: Kd^T blocks + lam
  // staging (x2): f32 state in accumulator order, bf16 state and delta fragments
  static constexpr int st_sb = 0;
  static constexpr int st_dl = st_sb + 16 * K * 2;
  static constexpr int stage = st_dl + 16 * 64 * 2;
  static constexpr int off_stage = kScanRing * slot;
  static constexpr int bytes = off_stage + 2 * stage;
};

__device__ __forceinline__ bf16x8 pack_tiles(const f32x4& lo, const f32x4& hi) {
  bf16x8 x;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[r] = to_bf16(lo[r]);
    x[4 + r] = to_bf16(hi[r]);
  }
  return x;
}

template <int K, int V>
__global__ __launch_bounds__(kScanThreads) void chunk_fwd_scan_kernel(FwdArgs a) {
  using L = ScanLds<K, V>;
  constexpr int KT = K / 16, NB = K / 32, KPW = KT / kScanCompute;
  static_assert(KT % kScanCompute == 0, "state tiles split evenly over the compute waves");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int H = a.H;
  int rec, strip;
  if (!xcd_strip_coords(a.num_seqs * H, V / 16, rec, strip)) return;
  const int seq = rec / H, h = rec % H, v0 = strip * 16;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lr = lane % 16, kg = lane / 16;
  const int2 sq = seq_entry(a, seq);  // {first chunk, chunk count}
  const int n = sq.y;
  if (n <= 0) {
    if (wave == 0 && a.sfin) {
      for (int kt = 0; kt < KT; ++kt) {
        const size_t o = (((size_t)seq * H + h) * V + v0 + lr) * K + 16 * kt + 4 * kg;
        *(float4*)(a.sfin + o) = a.s0 ? *(const float4*)(a.s0 + o) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    return;
  }

  if (wave == kScanCompute || wave == kScanCompute + 1) {
    // ---- loader waves ----
    const int lw = wave - kScanCompute;
    auto issue = [&](int ci) {
      const int c = ci < n ? ci : n - 1;  // fixed load count per chunk (clamped index)
      const size_t tile = (size_t)(sq.x + c) * H + h;
      char* slot = smem + (ci % kScanRing) * L::slot;
      if (lw == 0) {
        const char* w = (const char*)((const bf16*)a.ws.p[R_WF] + tile * 64 * K) + lane * 16;
#pragma unroll
        for (int b = 0; b < (64 * K * 2) / 1024; ++b) dma16(w + b * 1024, slot + L::off_w + b * 1024);
        const char* u = (const char*)((const bf16*)a.ws.p[R_UF] + tile * 64 * V + (size_t)strip * 64 * 16) +
                        lane * 16;
        dma16(u, slot + L::off_u);
        dma16(u + 1024, slot + L::off_u + 1024);
      } else {
        const char* kd = (const char*)((const bf16*)a.ws.p[R_KDTF] + tile * K * 64) + lane * 16;
#pragma unroll
        for (int b = 0; b < (K * 64 * 2) / 1024; ++b) dma16(kd + b * 1024, slot + L::off_kdt + b * 1024);
        if (lane < K / 4) dma16((const float*)a.ws.p[R_LAM] + tile * K + lane * 4, slot + L::off_lam);
      }
    };
#pragma unroll
    for (int d = 0; d < kScanRing - 1; ++d) issue(d);
    for (int ci = 0; ci < n; ++ci) {
      // the slot of chunk ci is complete once at most (ring - 2) chunks' loads are newer
      if (lw == 0)
        wait_vmcnt<(kScanRing - 2) * L::n_load0>();
      else
        wait_vmcnt<(kScanRing - 2) * L::n_load1>();
      ring_barrier();  // B1(ci): every read of slot ci - 1 finished before B2(ci - 1)
      issue(ci + kScanRing - 1);
      ring_barrier();  // B2(ci)
    }
    ring_barrier();   // B1(n)
    wait_vmcnt<0>();  // no LDS write may land after the workgroup ends
    return;
  }

  if (wave == kScanCompute + 2) {
    // ---- store wave: histories of chunk ci - 1, read between B1(ci) and B2(ci) (the
    // compute waves refill that staging buffer after B2(ci)), written to HBM after ----
    for (int ci = 0; ci <= n; ++ci) {
      ring_barrier();  // B1(ci)
      bf16x8 sb[NB], dl[2];
      if (ci > 0) {
        const char* st = smem + L::off_stage + ((ci - 1) & 1) * L::stage;
#pragma unroll
        for (int s = 0; s < NB; ++s) sb[s] = *(const bf16x8*)(st + L::st_sb + (s * 64 + lane) * 16);
#pragma unroll
        for (int s = 0; s < 2; ++s) dl[s] = *(const bf16x8*)(st + L::st_dl + (s * 64 + lane) * 16);
        wait_lgkm0();
      }
      if (ci < n) ring_barrier();  // B2(ci)
      if (ci == 0) continue;
      const size_t tile = (size_t)(sq.x + ci - 1) * H + h;
      bf16* SHBF = (bf16*)a.ws.p[R_SHBF] + tile * V * K + (size_t)strip * 16 * K;
#pragma unroll
      for (int s = 0; s < NB; ++s) *(bf16x8*)(SHBF + ((size_t)s * 64 + lane) * 8) = sb[s];
      bf16* DLF = (bf16*)a.ws.p[R_DLF] + tile * 64 * V + (size_t)strip * 16 * 64;
#pragma unroll
      for (int s = 0; s < 2; ++s) *(bf16x8*)(DLF + ((size_t)s * 64 + lane) * 8) = dl[s];
    }
    return;
  }

  // ---- compute wave c: delta row tile c, state tiles c*KPW .. c*KPW + KPW - 1 ----
  const int cw = wave;
  f32x4 S[KPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const int k0 = 16 * (cw * KPW + j) + 4 * kg;
    if (a.s0) {
      const float4 s = *(const float4*)(a.s0 + (((size_t)seq * H + h) * V + v0 + lr) * K + k0);
      S[j][0] = s.x; S[j][1] = s.y; S[j][2] = s.z; S[j][3] = s.w;
    } else {
      S[j] = zero4();
    }
  }
  // the bf16 state (B operand of the delta product) lives in the staging buffer of the
  // chunk it enters: fragment s packs state tiles 2s (low half) and 2s + 1 (high half)
  auto put_state = [&](char* st) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int kt = cw * KPW + j;
      bf16x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = to_bf16(S[j][r]);
      *(bf16x4*)(st + L::st_sb + ((kt / 2) * 64 + lane) * 16 + (kt % 2) * 8) = x;
    }
  };
  put_state(smem + L::off_stage);
  wait_lgkm0();
  for (int ci = 0; ci < n; ++ci) {
    ring_barrier();  // B1(ci): slot ci loaded, the state entering chunk ci staged
    const char* slot = smem + (ci % kScanRing) * L::slot;
    char* st = smem + L::off_stage + (ci & 1) * L::stage;
    bf16x8 wf[NB], Bs[NB], kf[KPW][2];
    float4 lamf[KPW];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      wf[s] = *(const bf16x8*)(slot + L::off_w + ((cw * NB + s) * 64 + lane) * 16);
      Bs[s] = *(const bf16x8*)(st + L::st_sb + (s * 64 + lane) * 16);
    }
    const bf16x4 uf = *(const bf16x4*)(slot + L::off_u + (cw * 64 + lane) * 8);
    __builtin_amdgcn_sched_barrier(0);
    // delta tile c = U + (-W) S: one K/32-deep chain
    f32x4 dl;
#pragma unroll
    for (int r = 0; r < 4; ++r) dl[r] = to_f32(uf[r]);
#pragma unroll
    for (int s = 0; s < NB; ++s) dl = mfma16(wf[s], Bs[s], dl);
    // meanwhile: the f32 history of the entering state (straight to HBM: nothing in this
    // wave waits on its stores), and this wave's Kd^T rows and lam
    float* SH = (float*)a.ws.p[R_SH] + ((size_t)(sq.x + ci) * H + h) * K * V + v0 + lr;
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int kt = cw * KPW + j;
#pragma unroll
      for (int r = 0; r < 4; ++r) SH[(size_t)(16 * kt + 4 * kg + r) * V] = S[j][r];
      kf[j][0] = *(const bf16x8*)(slot + L::off_kdt + ((kt * 2) * 64 + lane) * 16);
      kf[j][1] = *(const bf16x8*)(slot + L::off_kdt + ((kt * 2 + 1) * 64 + lane) * 16);
      lamf[j] = *(const float4*)(slot + L::off_lam + (16 * kt + 4 * kg) * 4);
    }
    {
      bf16x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = to_bf16(dl[r]);
      // delta B fragment t packs row tiles 2t (low half) and 2t + 1 (high half)
      *(bf16x4*)(st + L::st_dl + ((cw / 2) * 64 + lane) * 16 + (cw % 2) * 8) = x;
    }
    f32x4 acc[KPW];
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      acc[j][0] = lamf[j].x * S[j][0];
      acc[j][1] = lamf[j].y * S[j][1];
      acc[j][2] = lamf[j].z * S[j][2];
      acc[j][3] = lamf[j].w * S[j][3];
    }
    wait_lgkm0();
    ring_barrier();  // B2(ci): every delta tile staged
    const bf16x8 D0 = *(const bf16x8*)(st + L::st_dl + lane * 16);
    const bf16x8 D1 = *(const bf16x8*)(st + L::st_dl + (64 + lane) * 16);
    // S = lam S + Kd^T delta
#pragma unroll
    for (int j = 0; j < KPW; ++j) S[j] = mfma16(kf[j][0], D0, acc[j]);
#pragma unroll
    for (int j = 0; j < KPW; ++j) S[j] = mfma16(kf[j][1], D1, S[j]);
    put_state(smem + L::off_stage + ((ci + 1) & 1) * L::stage);
    wait_lgkm0();
  }
  ring_barrier();  // B1(n)
  if (a.sfin) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int k0 = 16 * (cw * KPW + j) + 4 * kg;
      *(float4*)(a.sfin + (((size_t)seq * H + h) * V + v0 + lr) * K + k0) =
          make_float4(S[j][0], S[j][1], S[j][2], S[j][3]);
    }
  }
}

// ---------------------------------------------------------------------------
// segmented scan: the 64-step chain of a long sequence cut into parallel segments
// ---------------------------------------------------------------------------
// One chunk maps the state affinely, S' = M S + Kd^T U with M = diag(lam) - Kd^T W, and the
// columns of S evolve independently.  A segment of L chunks therefore maps its entering
// state as S_out = P S_in + Sigma with P = M_L ... M_1 (K x K) and Sigma its end state from
// a zero start.  Three launches replace the one sequential pass:
//  1. local (chunk_fwd_seg_kernel<.., false>): every segment but the last of every
//     recurrence runs its chunks from the augmented start [0 | I] (V + K columns; the
//     identity columns see U = 0), giving [Sigma | P] -- segments run in parallel;
//  2. combine (chunk_fwd_combine_kernel): S_in(j+1) = P_j S_in(j) + Sigma_j, sequential over
//     the segments of one recurrence, one wave per V strip (S as hi + lo bf16 operands);
//  3. replay (chunk_fwd_seg_kernel<.., true>): every segment reruns its chunks from its true
//     entering state and writes the state / delta histories exactly as the one-pass scan.
// Sequential depth: L + (segments - 1) + L steps instead of the chunk count.  In the
// segment kernels one workgroup owns several strips and every compute wave owns whole
// strips (its delta tiles and state tiles), so a step needs no exchange between waves:
// a loader wave fills an LDS ring with the chunk's -W, Kd^T, U strips and lam, and the one
// barrier per chunk only recycles ring slots.
constexpr int kSegRing = 3;
constexpr int kSegCompute = 4;   // compute waves, one strip each (every wave reads the
                                 // chunk's whole -W and Kd^T from LDS)
constexpr int kSegSPW = 1;
constexpr int kSegThreads = (kSegCompute + 1) * kWave;

template <int K, int V, bool REPLAY>
struct SegCfg {
  static constexpr int NSTRIPS = REPLAY ? V / 16 : (V + K) / 16;  // strips per (rec, segment)
  static constexpr int SPW = kSegSPW;                               // strips per compute wave
  static constexpr int SPG = kSegCompute * SPW;                     // strips per workgroup
  static constexpr int GROUPS = NSTRIPS / SPG;                      // workgroups per (rec, segment)
  static_assert(NSTRIPS % SPG == 0, "strips split evenly over the workgroups");
  static constexpr int off_w = 0;                      // -W fragments, 64 x K bf16
  static constexpr int off_kdt = off_w + 64 * K * 2;   // Kd^T fragments, K x 64 bf16
  static constexpr int off_u = off_kdt + K * 64 * 2;   // U, C layout, SPG strips x 2 KB
  static constexpr int off_lam = off_u + SPG * 2048;   // lam, K f32
  static constexpr int slot = off_lam + K * 4;
  static constexpr int n_load = (64 * K * 2) / 1024 + (K * 64 * 2) / 1024 + 2 * SPG + 1;
  static constexpr int bytes = kSegRing * slot;
};

template <int K, int V, bool REPLAY>
__global__ __launch_bounds__(kSegThreads) void chunk_fwd_seg_kernel(FwdArgs a, int seg_len, int max_segs) {
  using C = SegCfg<K, V, REPLAY>;
  constexpr int KT = K / 16, NB = K / 32, VS = V / 16, SPW = C::SPW;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int H = a.H;
  int rs, group;
  if (!xcd_strip_coords(a.num_seqs * H * max_segs, C::GROUPS, rs, group)) return;
  const int rec = rs / max_segs, seg = rs % max_segs;
  const int seq = rec / H, h = rec % H;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lr = lane % 16, kg = lane / 16;
  const int2 sq = seq_entry(a, seq);  // {first chunk, chunk count}
  const int n = sq.y;
  const int nseg = (n + seg_len - 1) / seg_len;
  const int u_first = group * C::SPG;  // the workgroup's strips, V strips first
  int strip[SPW];
#pragma unroll
  for (int j = 0; j < SPW; ++j) strip[j] = u_first + (wave < kSegCompute ? wave : 0) * SPW + j;
  if (REPLAY) {
    if (n <= 0) {  // empty sequence: the final state is the initial one
      if (seg == 0 && wave < kSegCompute && a.sfin) {
        for (int j = 0; j < SPW; ++j)
          for (int kt = 0; kt < KT; ++kt) {
            const size_t o = (((size_t)seq * H + h) * V + 16 * strip[j] + lr) * K + 16 * kt + 4 * kg;
            *(float4*)(a.sfin + o) = a.s0 ? *(const float4*)(a.s0 + o) : make_float4(0.f, 0.f, 0.f, 0.f);
          }
      }
      return;
    }
    if (seg >= nseg) return;
  } else if (seg >= nseg - 1) {
    return;  // the last segment's map is never needed
  }
  const int c_begin = seg * seg_len;
  const int steps = min(n, c_begin + seg_len) - c_begin;

  if (wave == kSegCompute) {
    // ---- loader wave: direct global->LDS ring, a fixed number of loads per chunk ----
    auto issue = [&](int ci) {
      const int c = c_begin + (ci < steps ? ci : steps - 1);
      const size_t tile = (size_t)(sq.x + c) * H + h;
      char* slot = smem + (ci % kSegRing) * C::slot;
      const char* w = (const char*)((const bf16*)a.ws.p[R_WF] + tile * 64 * K) + lane * 16;
#pragma unroll
      for (int b = 0; b < (64 * K * 2) / 1024; ++b) dma16(w + b * 1024, slot + C::off_w + b * 1024);
      const char* kd = (const char*)((const bf16*)a.ws.p[R_KDTF] + tile * K * 64) + lane * 16;
#pragma unroll
      for (int b = 0; b < (K * 64 * 2) / 1024; ++b) dma16(kd + b * 1024, slot + C::off_kdt + b * 1024);
      const char* u0 = (const char*)((const bf16*)a.ws.p[R_UF] + tile * 64 * V) + lane * 16;
#pragma unroll
      for (int j = 0; j < C::SPG; ++j) {
        const int us = min(u_first + j, VS - 1);  // strips past V load a valid strip, unused
        dma16(u0 + (size_t)us * 2048, slot + C::off_u + j * 2048);
        dma16(u0 + (size_t)us * 2048 + 1024, slot + C::off_u + j * 2048 + 1024);
      }
      if (lane < K / 4) dma16((const float*)a.ws.p[R_LAM] + tile * K + lane * 4, slot + C::off_lam);
    };
#pragma unroll
    for (int d = 0; d < kSegRing - 1; ++d) issue(d);
    for (int ci = 0; ci < steps; ++ci) {
      wait_vmcnt<(kSegRing - 2) * C::n_load>();  // chunk ci's loads have landed
      ring_barrier();                             // B(ci); the slot of ci - 1 fully read
      issue(ci + kSegRing - 1);
    }
    ring_barrier();   // B(steps)
    wait_vmcnt<0>();  // no LDS write may land after the workgroup ends
    return;
  }

  // ---- compute wave: SPW strips, all of their delta and state tiles ----
  f32x4 S[SPW][KT];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const float* sin = nullptr;
    size_t sin_off = 0;
    if (REPLAY) {
      sin = seg == 0 ? a.s0 : (const float*)a.ws.p[R_SIN] + ((size_t)rec * max_segs + seg) * V * K;
      sin_off = (seg == 0 ? ((size_t)seq * H + h) * V * K : 0) + (size_t)(16 * strip[j] + lr) * K;
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int k0 = 16 * kt + 4 * kg;
      if (REPLAY) {
        if (sin) {
          const float4 x = *(const float4*)(sin + sin_off + k0);
          S[j][kt][0] = x.x; S[j][kt][1] = x.y; S[j][kt][2] = x.z; S[j][kt][3] = x.w;
        } else {
          S[j][kt] = zero4();
        }
      } else {
        // Sigma strips start at zero; P strip p starts as columns 16p.. of the identity
        const int col = 16 * (strip[j] - VS) + lr;
#pragma unroll
        for (int r = 0; r < 4; ++r) S[j][kt][r] = (strip[j] >= VS && k0 + r == col) ? 1.f : 0.f;
      }
    }
  }
  for (int ci = 0; ci < steps; ++ci) {
    ring_barrier();  // B(ci): slot ci loaded
    const char* slot = smem + (ci % kSegRing) * C::slot;
    // every operand of the step requested before the first product
    bf16x8 wf[4][NB], kf[KT][2];
    float4 lam[KT];
    bf16x4 uf[SPW][4];
    // (issued in the order of first use: LDS reads return in order, so the first products
    // wait only for their own operands)
#pragma unroll
    for (int j = 0; j < SPW; ++j)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
        uf[j][rt] = *(const bf16x4*)(slot + C::off_u + (strip[j] - u_first) * 2048 + (rt * 64 + lane) * 8);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < NB; ++s)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) wf[rt][s] = *(const bf16x8*)(slot + C::off_w + ((rt * NB + s) * 64 + lane) * 16);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) lam[kt] = *(const float4*)(slot + C::off_lam + (16 * kt + 4 * kg) * 4);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) kf[kt][t] = *(const bf16x8*)(slot + C::off_kdt + ((kt * 2 + t) * 64 + lane) * 16);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of every product
    // the state as B operands: fragment s packs tiles 2s (low half) and 2s + 1 (high half)
    bf16x8 Bs[SPW][NB];
#pragma unroll
    for (int j = 0; j < SPW; ++j)
#pragma unroll
      for (int s = 0; s < NB; ++s) Bs[j][s] = pack_tiles(S[j][2 * s], S[j][2 * s + 1]);
    const size_t tile = (size_t)(sq.x + c_begin + ci) * H + h;
    if (REPLAY) {
      // histories of the entering state: f32 [K][V] and the bf16 B-operand fragments
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        float* SH = (float*)a.ws.p[R_SH] + tile * K * V + 16 * strip[j] + lr;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) SH[(size_t)(16 * kt + 4 * kg + r) * V] = S[j][kt][r];
        bf16* SHBF = (bf16*)a.ws.p[R_SHBF] + tile * V * K + (size_t)strip[j] * 16 * K;
#pragma unroll
        for (int s = 0; s < NB; ++s) *(bf16x8*)(SHBF + ((size_t)s * 64 + lane) * 8) = Bs[j][s];
      }
    }
    // delta = U + (-W) S: 4 x SPW independent row-tile chains sharing each -W fragment
    f32x4 dl[SPW][4];
#pragma unroll
    for (int j = 0; j < SPW; ++j)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) dl[j][rt][r] = strip[j] < VS ? to_f32(uf[j][rt][r]) : 0.f;
#pragma unroll
    for (int s = 0; s < NB; ++s)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int j = 0; j < SPW; ++j) dl[j][rt] = mfma16(wf[rt][s], Bs[j][s], dl[j][rt]);
    // delta as B operands (fragment t packs row tiles 2t and 2t + 1)
    bf16x8 D[SPW][2];
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      D[j][0] = pack_tiles(dl[j][0], dl[j][1]);
      D[j][1] = pack_tiles(dl[j][2], dl[j][3]);
      if (REPLAY) {
        bf16* DLF = (bf16*)a.ws.p[R_DLF] + tile * 64 * V + (size_t)strip[j] * 16 * 64;
        *(bf16x8*)(DLF + (size_t)lane * 8) = D[j][0];
        *(bf16x8*)(DLF + (size_t)(64 + lane) * 8) = D[j][1];
      }
    }
    // S = lam S + Kd^T delta: KT x SPW independent chains
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        f32x4 acc;
        acc[0] = lam[kt].x * S[j][kt][0];
        acc[1] = lam[kt].y * S[j][kt][1];
        acc[2] = lam[kt].z * S[j][kt][2];
        acc[3] = lam[kt].w * S[j][kt][3];
        S[j][kt] = mfma16(kf[kt][0], D[j][0], acc);
      }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int j = 0; j < SPW; ++j) S[j][kt] = mfma16(kf[kt][1], D[j][1], S[j][kt]);
  }
  ring_barrier();  // B(steps)
  // segment end
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    if (REPLAY) {
      if (seg == nseg - 1 && a.sfin) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
          *(float4*)(a.sfin + (((size_t)seq * H + h) * V + 16 * strip[j] + lr) * K + 16 * kt + 4 * kg) =
              make_float4(S[j][kt][0], S[j][kt][1], S[j][kt][2], S[j][kt][3]);
      }
    } else if (strip[j] < VS) {
      float* sg = (float*)a.ws.p[R_SEGS] + ((size_t)rec * max_segs + seg) * V * K + (size_t)(16 * strip[j] + lr) * K;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
        *(float4*)(sg + 16 * kt + 4 * kg) = make_float4(S[j][kt][0], S[j][kt][1], S[j][kt][2], S[j][kt][3]);
    } else {
      // P as bf16 A-operand fragments with the permuted contraction order of the combine
      // kernel's state operands; this lane holds column
      // 16p + lr of rows 16kt + 4kg .. + 3
      bf16* pg = (bf16*)a.ws.p[R_SEGP] + ((size_t)rec * max_segs + seg) * K * K;
      const int col = 16 * (strip[j] - VS) + lr;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) pg[perm_frag_elem(K, 16 * kt + 4 * kg + r, col)] = to_bf16(S[j][kt][r]);
    }
  }
}

// S_in(j+1) = P_j S_in(j) + Sigma_j over the segments of one recurrence.  One workgroup per
// (recurrence, V strip); wave w owns state tiles w * TPW .. (w + 1) * TPW - 1.  Each step the
// waves publish their tiles as hi + lo bf16 B-operand halves in LDS (about 16 mantissa
// bits of the state), one barrier, and every wave multiplies its rows of P_j (bf16
// fragments written by the local kernel, prefetched a step ahead) by the whole state.
constexpr int kCombThreads = 4 * kWave;
constexpr int kCombBatch = 8;

template <int K, int V>
__global__ __launch_bounds__(kCombThreads) void chunk_fwd_combine_kernel(FwdArgs a, int seg_len, int max_segs) {
  constexpr int KT = K / 16, NB = K / 32, VS = V / 16, TPW = KT / 4;
  __shared__ __attribute__((aligned(16))) char sB[2][2][NB][kWave * 16];  // [parity][hi/lo][frag]
  const int H = a.H;
  int rec, strip;
  if (!xcd_strip_coords(a.num_seqs * H, VS, rec, strip)) return;
  const int seq = rec / H, h = rec % H;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, lr = lane % 16, kg = lane / 16;
  const int n = seq_entry(a, seq).y;
  const int nseg = (n + seg_len - 1) / seg_len;
  if (nseg <= 1) return;
  const int v = 16 * strip + lr;
  f32x4 S[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int kt = wave * TPW + t;
    if (a.s0) {
      const float4 x = *(const float4*)(a.s0 + (((size_t)seq * H + h) * V + v) * K + 16 * kt + 4 * kg);
      S[t][0] = x.x; S[t][1] = x.y; S[t][2] = x.z; S[t][3] = x.w;
    } else {
      S[t] = zero4();
    }
  }
  const bf16* P0 = (const bf16*)a.ws.p[R_SEGP] + (size_t)rec * max_segs * K * K;
  const float* G0 = (const float*)a.ws.p[R_SEGS] + (size_t)rec * max_segs * V * K + (size_t)v * K;
  // every step's P rows and Sigma for this wave, requested up front in batches of
  // kCombBatch steps (one memory round trip per batch instead of one per step)
  bf16x8 pa[kCombBatch][TPW][NB];
  float4 sg[kCombBatch][TPW];
  for (int j = 0; j + 1 < nseg; ++j) {
    const int jb = j % kCombBatch;
    if (jb == 0) {
#pragma unroll
      for (int b = 0; b < kCombBatch; ++b) {
        const int jj = min(j + b, nseg - 2);
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          const int kt = wave * TPW + t;
#pragma unroll
          for (int s = 0; s < NB; ++s)
            pa[b][t][s] = *(const bf16x8*)(P0 + (size_t)jj * K * K + (((size_t)kt * NB + s) * 64 + lane) * 8);
          sg[b][t] = *(const float4*)(G0 + (size_t)jj * V * K + 16 * kt + 4 * kg);
        }
      }
    }
    char(*buf)[NB][kWave * 16] = sB[j & 1];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int kt = wave * TPW + t;
      bf16x4 hi, lo;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        hi[r] = to_bf16(S[t][r]);
        lo[r] = to_bf16(S[t][r] - to_f32(hi[r]));
      }
      *(bf16x4*)(buf[0][kt / 2] + lane * 16 + (kt % 2) * 8) = hi;
      *(bf16x4*)(buf[1][kt / 2] + lane * 16 + (kt % 2) * 8) = lo;
    }
    // LDS only: a fence-free barrier (the prefetched loads and earlier stores stay in flight)
    wait_lgkm0();
    ring_barrier();
    bf16x8 Bh[NB], Bl[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      Bh[s] = *(const bf16x8*)(buf[0][s] + lane * 16);
      Bl[s] = *(const bf16x8*)(buf[1][s] + lane * 16);
    }
    // pick this step's operands (jb is uniform; unrolled select keeps them in registers)
    bf16x8 pc[TPW][NB];
    float4 gc[TPW];
#pragma unroll
    for (int b = 0; b < kCombBatch; ++b)
      if (b == jb) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          gc[t] = sg[b][t];
#pragma unroll
          for (int s = 0; s < NB; ++s) pc[t][s] = pa[b][t][s];
        }
      }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      f32x4 acc;
      acc[0] = gc[t].x; acc[1] = gc[t].y; acc[2] = gc[t].z; acc[3] = gc[t].w;
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        acc = mfma16(pc[t][s], Bh[s], acc);
        acc = mfma16(pc[t][s], Bl[s], acc);
      }
      S[t] = acc;
    }
    float* out = (float*)a.ws.p[R_SIN] + ((size_t)rec * max_segs + j + 1) * V * K + (size_t)v * K;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
      *(float4*)(out + 16 * (wave * TPW + t) + 4 * kg) = make_float4(S[t][0], S[t][1], S[t][2], S[t][3]);
  }
}

// ---------------------------------------------------------------------------
// output:  O = Qg S + A delta  (chunk-parallel, after the scan)
// ---------------------------------------------------------------------------
// One 256-thread workgroup per (chunk, head); wave w owns the 16-token row tile w and
// walks the V/16 column tiles, so its Qg and A operands are loaded once.
#ifndef KDA_OUT_AHEAD
#define KDA_OUT_AHEAD 2  // column tiles whose fragments are in flight ahead of the products
#endif
template <int K, int V>
__global__ __launch_bounds__(256) void chunk_fwd_output_kernel(FwdArgs a) {
  constexpr int OP = V + 8;  // bf16 row stride of a wave's 16-row staging tile
  __shared__ __attribute__((aligned(16))) bf16 sOut[4][16 * OP];
  const int4 ch = chunk_entry(a, blockIdx.x);
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
  // the optional norm epilogue's gate values and weights, requested with the operands (after
  // the products they were a round trip of their own)
  const bool ng = a.ng_out != nullptr;
  bf16 gvr[V / 16][4];
  float w[V / 16];
  if (ng) {
#pragma unroll
    for (int ct = 0; ct < V / 16; ++ct) {
      w[ct] = a.ng_weight[16 * ct + lr];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = min(16 * wave + 4 * kg + r, len - 1);
        gvr[ct][r] = a.ng_gate[(size_t)(ch.x + t) * a.ng_gate_ld + (size_t)h * V + 16 * ct + lr];
      }
    }
  }
  // o of this lane's 4 rows x V/16 columns, kept for the optional norm epilogue.  The state
  // and delta fragments of KDA_OUT_AHEAD column tiles are requested before the first
  // product (left to the scheduler, only 2-4 were in flight: a chain of round trips).
  constexpr int kAhead = KDA_OUT_AHEAD < V / 16 ? KDA_OUT_AHEAD : V / 16;
  bf16x8 sf[V / 16][K / 32], df[V / 16][2];
  auto fetch = [&](int ct) {
    const bf16* sb = SHBF + (size_t)ct * 16 * K;
    const bf16* db = DLF + (size_t)ct * 16 * 64;
#pragma unroll
    for (int s = 0; s < K / 32; ++s) sf[ct][s] = *(const bf16x8*)(sb + ((size_t)s * 64 + lane) * 8);
    df[ct][0] = *(const bf16x8*)(db + (size_t)lane * 8);
    df[ct][1] = *(const bf16x8*)(db + (size_t)(64 + lane) * 8);
  };
#pragma unroll
  for (int ct = 0; ct < kAhead; ++ct) fetch(ct);
  __builtin_amdgcn_sched_barrier(0);
  float ov[V / 16][4];
#pragma unroll
  for (int ct = 0; ct < V / 16; ++ct) {
    if (ct + kAhead < V / 16) fetch(ct + kAhead);
    const int vcol = 16 * ct + lr;
    f32x4 o0 = zero4(), o1 = zero4();
#pragma unroll
    for (int s = 0; s < K / 32; s += 2) {
      o0 = mfma16(fq[s], sf[ct][s], o0);
      o1 = mfma16(fq[s + 1], sf[ct][s + 1], o1);
    }
    o0 = mfma16(fa[0], df[ct][0], o0);
    o1 = mfma16(fa[1], df[ct][1], o1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bf16 ob = to_bf16(o0[r] + o1[r]);
      ov[ct][r] = to_f32(ob);
      sOut[wave][(4 * kg + r) * OP + vcol] = ob;
    }
  }
  // the wave's 16 x V tile leaves through LDS as 16-byte row pieces
  bf16* so = sOut[wave];
  auto store_tile = [&](bf16* dst) {
#pragma unroll
    for (int it = 0; it < 16 * V / 8 / kWave; ++it) {
      const int idx = it * kWave + lane, rr = idx / (V / 8), c8 = (idx % (V / 8)) * 8;
      const int t = 16 * wave + rr;
      if (t < len) *(bf16x8*)(dst + ((size_t)(ch.x + t) * H + h) * V + c8) = *(const bf16x8*)(so + rr * OP + c8);
    }
  };
  __builtin_amdgcn_wave_barrier();
  store_tile(a.out);
  if (!ng) return;
  // fused RMSNorm * weight * sigmoid(gate) over each token's V values of this head, from the
  // bf16-rounded o exactly as the standalone norm kernel reads it: a row's V values live in
  // the 16 lanes of one lane group (V/16 columns each)
  float gv[V / 16][4];
#pragma unroll
  for (int ct = 0; ct < V / 16; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) gv[ct][r] = to_f32(gvr[ct][r]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float ss = 0.f;
#pragma unroll
    for (int ct = 0; ct < V / 16; ++ct) ss = fmaf(ov[ct][r], ov[ct][r], ss);
    ss = group_sum<16>(ss);
    const float inv = rsqrtf(ss / V + a.ng_eps);
    const int t = 16 * wave + 4 * kg + r;
#pragma unroll
    for (int ct = 0; ct < V / 16; ++ct)
      so[(4 * kg + r) * OP + 16 * ct + lr] = to_bf16(ov[ct][r] * inv * w[ct] * sigmoid_fast(gv[ct][r]));
    if (lr == 0 && t < len) a.ng_inv_rms[(size_t)(ch.x + t) * H + h] = inv;
  }
  __builtin_amdgcn_wave_barrier();
  store_tile(a.ng_out);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int validate_problem(const kda_chunk_problem* p, const char* who) {
  KDA_REQUIRE(p, "%s: null problem", who);
  KDA_REQUIRE(p->batch >= 0 && p->seq_len >= 0 && p->heads > 0, "%s: invalid B/T/H", who);
  // 64 / 128 run the chunked kernels; other sizes the token-serial kernels (generic.hip)
  KDA_REQUIRE(p->key_dim >= 1 && p->key_dim <= 256, "%s: key_dim must be in [1, 256]", who);
  KDA_REQUIRE(p->value_dim >= 1 && p->value_dim <= 4096, "%s: value_dim must be in [1, 4096]", who);
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
  KDA_REQUIRE(p->beta_grad_pad >= 0, "%s: beta_grad_pad must be non-negative", who);
  KDA_REQUIRE(p->beta_row_stride == 0 || (long)p->beta_row_stride >= (long)p->heads + p->beta_grad_pad,
              "%s: beta_row_stride must be 0 or at least heads + beta_grad_pad", who);
  KDA_REQUIRE(p->beta_row_stride > 0 || p->beta_grad_pad == 0,
              "%s: beta_grad_pad needs a beta_row_stride", who);
  KDA_REQUIRE(p->norm_gate_row_stride == 0 || (long)p->norm_gate_row_stride >= (long)p->heads * p->value_dim,
              "%s: norm_gate_row_stride must be 0 or at least heads * value_dim", who);
  return KDA_OK;
}

// Segmented scans: when the (sequence, head) recurrences times the V/16 column strips are
// too few to fill the chip and sequences are long, each sequence's chunks are cut into
// segments of ~sqrt(chunks) chunks that are scanned in parallel (see the segmented scan
// kernels).  A pure function of the problem, so workspace sizing and launches agree.
constexpr int kSegMinChunks = 96;     // shorter sequences run in one pass (measured: no gain at 64)
constexpr int kSegStripLimit = 512;   // recurrences x V/16 strips at which one pass fills the chip

ChunkGeom make_geom(const kda_chunk_problem* p) {
  ChunkGeom g;
  const int nc = (p->seq_len + kChunk - 1) / kChunk;
  g.max_chunks = p->cu_seqlens ? nc + p->num_seqs : p->batch * nc;
  g.heads = p->heads;
  g.K = p->key_dim;
  g.V = p->value_dim;
  g.num_seqs = p->num_seqs;
  g.seg_len = 0;
  g.max_segs = 1;
  // nc bounds the chunk count of any one sequence (a packed sequence has at most T tokens)
  if (nc >= kSegMinChunks && (long)p->num_seqs * p->heads * (p->value_dim / 16) < kSegStripLimit) {
    int L = 4;
    while (L * L < nc) ++L;
    g.seg_len = L;
    g.max_segs = (nc + L - 1) / L;
  }
  return g;
}

template <int K, int V>
static int launch_forward(const kda_chunk_problem* p, const ChunkGeom& g, FwdArgs& a,
                          hipStream_t stream, int stages) {
  if (g.max_chunks > 0 && (stages & (1 << KDA_STAGE_FWD_INTRA))) {
    constexpr size_t smem = IntraLds<K, V>::bytes;
    for (const void* f : {(const void*)chunk_fwd_intra_kernel<K, V, false>, (const void*)chunk_fwd_intra_kernel<K, V, K == V>}) {
      hipError_t e = ensure_lds_limit(f, (int)smem);
      if (e != hipSuccess)
        return set_error(KDA_ERR_LAUNCH, "chunk_forward: LDS attribute: %s", hipGetErrorString(e));
    }
    auto intra = a.conv_x ? chunk_fwd_intra_kernel<K, V, K == V> : chunk_fwd_intra_kernel<K, V, false>;
    hipLaunchKernelGGL(intra, dim3(g.max_chunks, p->heads), dim3(kIntraThreads), smem, stream, a);
    KDA_LAUNCH_CHECK("chunk_forward intra");
  }
  if (p->num_seqs > 0 && (stages & (1 << KDA_STAGE_FWD_SCAN))) {
    auto scan = chunk_fwd_scan_kernel<K, V>;
    constexpr size_t smem = ScanLds<K, V>::bytes;
    {
      hipError_t e = ensure_lds_limit((const void*)scan, (int)smem);
      if (e != hipSuccess)
        return set_error(KDA_ERR_LAUNCH, "chunk_forward: scan LDS attribute: %s", hipGetErrorString(e));
    }
    const int nrec = p->num_seqs * p->heads;
    if (g.seg_len == 0) {
      const int grid = kXcds * (V / 16) * ((nrec + kXcds - 1) / kXcds);
      hipLaunchKernelGGL(scan, dim3(grid), dim3(kScanThreads), smem, stream, a);
      KDA_LAUNCH_CHECK("chunk_forward scan");
    } else {
      auto local = chunk_fwd_seg_kernel<K, V, false>;
      auto replay = chunk_fwd_seg_kernel<K, V, true>;
      using CL = SegCfg<K, V, false>;
      using CR = SegCfg<K, V, true>;
      if (ensure_lds_limit((const void*)local, (int)CL::bytes) != hipSuccess ||
          ensure_lds_limit((const void*)replay, (int)CR::bytes) != hipSuccess)
        return set_error(KDA_ERR_LAUNCH, "chunk_forward: segmented scan LDS attribute failed");
      const int nrs = nrec * g.max_segs;
      hipLaunchKernelGGL(local, dim3(kXcds * CL::GROUPS * ((nrs + kXcds - 1) / kXcds)), dim3(kSegThreads),
                         CL::bytes, stream, a, g.seg_len, g.max_segs);
      KDA_LAUNCH_CHECK("chunk_forward segment maps");
      auto comb = chunk_fwd_combine_kernel<K, V>;
      hipLaunchKernelGGL(comb, dim3(kXcds * (V / 16) * ((nrec + kXcds - 1) / kXcds)), dim3(kCombThreads), 0, stream,
                         a, g.seg_len, g.max_segs);
      KDA_LAUNCH_CHECK("chunk_forward segment combine");
      hipLaunchKernelGGL(replay, dim3(kXcds * CR::GROUPS * ((nrs + kXcds - 1) / kXcds)), dim3(kSegThreads),
                         CR::bytes, stream, a, g.seg_len, g.max_segs);
      KDA_LAUNCH_CHECK("chunk_forward segment replay");
    }
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
  if (kda::generic_dims(p)) return kda::padded_route(p) ? kda::padded_ws_bytes(p) : kda::generic_ws_bytes(p);
  return kda::ws_total_bytes(kda::make_geom(p));
}

extern "C" size_t kda_chunk_backward_scratch_bytes(const kda_chunk_problem* p) {
  if (kda::validate_problem(p, "chunk_backward_scratch_bytes") != KDA_OK) return 0;
  if (kda::generic_dims(p)) return kda::padded_route(p) ? kda::padded_sc_bytes(p) : kda::generic_sc_bytes(p);
  return kda::sc_total_bytes(kda::make_geom(p));
}

static int chunk_forward_impl(int stages, const kda_chunk_problem* p, const void* q, const void* k,
                                 const void* v, const void* gate, const void* beta_logits,
                                 const float* A_log, const float* dt_bias,
                                 const float* initial_state, void* output, float* final_state,
                                 void* workspace, hipStream_t stream,
                                 const void* norm_gate = nullptr, const float* norm_weight = nullptr,
                                 float norm_eps = 0.f, void* norm_output = nullptr,
                                 float* norm_inv_rms = nullptr, const void* conv_x = nullptr,
                                 long conv_ld = 0, const void* conv_w = nullptr, int conv_W = 0) {
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
  if (generic_dims(p)) {
    KDA_REQUIRE(stages == ~0 && !norm_gate && !conv_x,
                "chunk_forward: stage entry points and fused epilogues need head dims 64 or 128");
    if (padded_route(p))
      return padded_forward(p, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state, output, final_state,
                            workspace, stream);
    return generic_forward(p, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state, output, final_state,
                           workspace, stream);
  }
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
  a.ng_gate = (const bf16*)norm_gate;
  a.ng_gate_ld = p->norm_gate_row_stride > 0 ? p->norm_gate_row_stride : (long)p->heads * p->value_dim;
  a.beta_ld = p->beta_row_stride > 0 ? p->beta_row_stride : p->heads;
  a.ng_weight = norm_weight;
  a.ng_eps = norm_eps;
  a.ng_out = (bf16*)norm_output;
  a.ng_inv_rms = norm_inv_rms;
  a.conv_x = (const bf16*)conv_x;
  a.conv_ld = conv_ld;
  a.conv_w = (const bf16*)conv_w;
  a.conv_W = conv_W;
  // fixed-length problems with at least one chunk get their tables from the intra kernel
  a.fixed_T = (p->cu_seqlens == nullptr && g.max_chunks > 0) ? p->seq_len : 0;
  if ((stages & (1 << KDA_STAGE_PREP)) && a.fixed_T == 0) {
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

extern "C" int kda_chunk_forward_norm_gate(const kda_chunk_problem* p, const void* q, const void* k,
                                           const void* v, const void* gate, const void* beta_logits,
                                           const float* A_log, const float* dt_bias,
                                           const float* initial_state, void* output,
                                           float* final_state, void* workspace,
                                           const void* norm_gate, const float* norm_weight,
                                           float epsilon, void* norm_output, float* inverse_rms,
                                           hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(p != nullptr, "chunk_forward_norm_gate: null problem");
  const bool empty = (size_t)p->batch * p->seq_len == 0;
  KDA_REQUIRE(p->value_dim == 64 || p->value_dim == 128,
              "chunk_forward_norm_gate: value_dim must be 64 or 128");
  KDA_REQUIRE(empty || (norm_gate && norm_weight && norm_output && inverse_rms),
              "chunk_forward_norm_gate: null norm pointer");
  KDA_REQUIRE(epsilon >= 0.f, "chunk_forward_norm_gate: epsilon must be non-negative");
  return chunk_forward_impl(~0, p, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state,
                            output, final_state, workspace, stream, norm_gate, norm_weight, epsilon,
                            norm_output, inverse_rms);
}

extern "C" int kda_chunk_forward_conv_norm_gate(const kda_chunk_problem* p, const void* conv_x,
                                                int64_t conv_ld, const void* conv_weight,
                                                int32_t conv_width, void* q, void* k, void* v,
                                                const void* gate, const void* beta_logits,
                                                const float* A_log, const float* dt_bias,
                                                void* output, void* workspace,
                                                const void* norm_gate, const float* norm_weight,
                                                float epsilon, void* norm_output, float* inverse_rms,
                                                hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(p != nullptr, "chunk_forward_conv_norm_gate: null problem");
  const bool empty = (size_t)p->batch * p->seq_len == 0;
  KDA_REQUIRE(p->cu_seqlens == nullptr, "chunk_forward_conv_norm_gate: cu_seqlens is not supported");
  KDA_REQUIRE(p->key_dim == p->value_dim && (p->value_dim == 64 || p->value_dim == 128),
              "chunk_forward_conv_norm_gate: key_dim and value_dim must be equal, 64 or 128");
  KDA_REQUIRE(conv_width >= 1 && conv_width <= 4, "chunk_forward_conv_norm_gate: conv_width must be in [1, 4]");
  KDA_REQUIRE(empty || (conv_x && conv_weight && q && k && v),
              "chunk_forward_conv_norm_gate: null convolution pointer");
  KDA_REQUIRE(conv_ld >= 3 * (int64_t)p->heads * p->key_dim && conv_ld % 8 == 0,
              "chunk_forward_conv_norm_gate: conv_ld must be a multiple of 8 and >= 3 * heads * key_dim");
  KDA_REQUIRE(aligned16(conv_x), "chunk_forward_conv_norm_gate: conv_x must be 16-byte aligned");
  KDA_REQUIRE(empty || (norm_gate && norm_weight && norm_output && inverse_rms),
              "chunk_forward_conv_norm_gate: null norm pointer");
  KDA_REQUIRE(epsilon >= 0.f, "chunk_forward_conv_norm_gate: epsilon must be non-negative");
  return chunk_forward_impl(~0, p, q, k, v, gate, beta_logits, A_log, dt_bias, nullptr, output,
                            nullptr, workspace, stream, norm_gate, norm_weight, epsilon, norm_output,
                            inverse_rms, empty ? nullptr : conv_x, conv_ld, conv_weight, conv_width);
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
