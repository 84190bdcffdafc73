// Exact chunked backward of Kimi Delta Attention on gfx950.
//
// Reference: the production WY backward nanochat/mixers/cuda_kda/chunk_wy_backward.cu
// (reverse dH scan :2026-2584, chunk VJP :2818-3331, pair VJPs :3337-3552, prefix
// reverse :3787-3800, finalize :3802-3894, parameter reductions :3896-3990) and the
// analytic token-serial statement chunk.cu:578-870.
//
// Per chunk (forward: delta = U - W S, O = Qg S + A delta, S' = lam S + Kd^T delta):
//   scan (reverse, sequential):  dDelta = A^T dO + Kd dS' ;  dS = Qg^T dO + lam dS' - W^T dDelta
//   dense VJP (chunk-parallel):  dA = tril(dO delta^T), dQg = dO S^T, dKd = delta dS'^T,
//       dlam = rowsum(S * dS'), dW = -dDelta S^T, dU = dDelta,
//       dT = dU (beta v)^T + dW (beta kh e^G)^T, d(beta v) = T^T dU, d(beta kh e^G) = T^T dW,
//       dM = -T^T dT T^T (strictly lower)
//   decay-structured VJP:  A[i,j] = sum_c qh kh exp(G_i - G_j) and M' likewise give
//       row-side (dqh, dkh) and column-side (dkh) terms and dG = qh*Rq + kh*Rk - kh*C.
//   finalize: dg = reverse in-chunk cumsum of dG, K3 gate chain, L2-norm and sigmoid
//       chains; gate parameter gradients are reduced in a fixed order (no atomics).
//
// MI355X mapping:
//  * scan kernel: one workgroup per (sequence, head, 16-wide V strip); dS columns are
//    independent, so the 128x16 f32 slice of dS lives in VGPRs as MFMA accumulators of four
//    compute waves, fed by two loader waves through an LDS ring of direct global->LDS loads.
//    The launch also carries cache-warming workgroups for the CUs the scan leaves idle.
//  * dense and decay VJPs: one workgroup per (chunk, head) tile, both bodies in one kernel
//    (role by workgroup index) launched as full rounds over "all dense tiles, then all
//    decay tiles".  Dense: 16x16x32 bf16 MFMA tiles with f32 accumulation, every global
//    operand requested in one batch.  Decay: the decay-scaled operands are built once per
//    tile around the first (row side) or last (column side) row of each 16-row block, so
//    every factor is <= 1 or bounded by the block's span; a tile with a block whose decay
//    span exceeds 80 nats runs an exact per-pair f32 loop instead.
//  * fused launch (the whole backward in one call): the scan members, the prep workgroups
//    and the tile workgroups share one grid; a tile runs its dense and decay parts as soon as the scan
//    has finalised its chunk, so the VJP work overlaps the latency-bound scan (see
//    chunk_bwd_fused_kernel).  The staged entry points keep the separate launches.
#include "chunk_host.hpp"
#include "kda_device.hpp"

#include <atomic>
#include <cstdlib>

namespace kda {

struct BwdArgs {
  int H;
  int num_seqs;
  int gate_mode;
  float lb;
  float scale;
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const void* gate;
  const bf16* beta_logits;
  const float* A_log;
  const float* dt_bias;
  const bf16* dout;
  const float* dsfin;
  bf16* dq;
  bf16* dk;
  bf16* dv;
  void* dgate;
  bf16* dbeta;
  float* dA_log;
  float* ddt_bias;
  float* ds0;
  Regions ws;
  Regions sc;
  long gld_qk, gld_v;  // row strides (elements per token) of dq / dk and of dv
  long dbeta_ld;       // row stride of dbeta; the dbeta_pad elements after a row's H are zeroed
  int dbeta_pad;
  int fixed_T;  // > 0: every sequence has this length (chunk c = sequence * n + index)
};

// Chunk table entry {row0, len, sequence, index}: arithmetic for sequences of one length.
__device__ __forceinline__ int4 chunk_entry(const BwdArgs& a, int c) {
  if (a.fixed_T > 0) {
    const int nc = (a.fixed_T + kChunk - 1) / kChunk, sq = c / nc, j = c % nc;
    return make_int4(sq * a.fixed_T + j * kChunk, min(kChunk, a.fixed_T - j * kChunk), sq, j);
  }
  return ((const int4*)a.ws.p[R_CHUNKS])[c];
}

// Sequence table entry {first chunk, chunk count}: arithmetic for sequences of one length.
__device__ __forceinline__ int2 seq_entry(const BwdArgs& a, int seq) {
  if (a.fixed_T > 0) {
    const int nc = (a.fixed_T + kChunk - 1) / kChunk;
    return make_int2(seq * nc, nc);
  }
  return ((const int2*)a.ws.p[R_SEQS])[seq];
}

// ---------------------------------------------------------------------------
// reverse state-gradient scan (transition form)
// ---------------------------------------------------------------------------
// With X_c = dL/dS at the end of chunk c (X_{n-1} = the final-state gradient),
//   dDelta_c = A^T dO + Kd X_c,   X_{c-1} = lam o X_c + Qg^T dO - W^T dDelta_c
//            = lam o X_c - G_c X_c + E_c,   G_c = W_c^T Kd_c,  E_c = Qg_c^T dO - W_c^T (A_c^T dO),
// and X_{-1} is the initial-state gradient.  G and E need nothing from the recurrence, so a
// chunk-parallel kernel forms them first (chunk_bwd_prep_kernel); the sequential scan then
// streams per chunk only -G (K x K bf16), its strip of E (K x 16 f32) and lam, and its chain
// is one K/32-deep MFMA product with one barrier per chunk.  dDelta_c is formed by the VJP
// tile of chunk c from X_c (dense_tile).
//
// Prep: one workgroup (four waves) per tile.  -G is emitted as permuted A fragments straight
// from the accumulators of -G^T = Kd^T (-W) (the accumulator tiles 2s and 2s + 1 of column
// block b give a lane exactly the 8 contraction values of fragment (b, s)); E in the scan's
// accumulator order [strip][key tile][lane][4].
constexpr int kPrepThreads = 256;

template <int K, int V>
struct PrepLds {
  static constexpr int OP = V + 8, KP = K + 8, AP = 64 + 8;  // row pitches (bf16), 16-byte aligned rows
  static constexpr int off_do = 0;                       // dO [64][OP], rows >= len zero
  static constexpr int off_ado = off_do + 64 * OP * 2;   // bf16(A^T dO) [64][OP]
  static constexpr int off_kd = off_ado + 64 * OP * 2;   // Kd [64][KP], then Qg [64][KP]
  static constexpr int off_w = off_kd + 64 * KP * 2;     // -W [64][KP]
  static constexpr int off_a = off_w + 64 * KP * 2;      // A [64][AP]
  static constexpr int bytes = off_a + 64 * AP * 2;
};

// Row-major staging of a permuted fragment array (64 rows; fragment (rt, s) element e of lane
// l is row 16 rt + l % 16, column 32 s + 16 (e / 4) + 4 (l / 16) + e % 4): one 16-byte piece
// (fragment-major index idx) written as two 8-byte row pieces.
__device__ __forceinline__ void stage_permuted_piece(bf16* m, int pitch, int ncols, int idx, const bf16x8& x) {
  const int l = idx % 64, fs = (idx / 64) % (ncols / 32), rt = idx / (64 * (ncols / 32));
  const int r = 16 * rt + l % 16, g = l / 16;
  bf16x4 lo, hi;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    lo[e] = x[e];
    hi[e] = x[4 + e];
  }
  *(bf16x4*)(m + r * pitch + 32 * fs + 4 * g) = lo;
  *(bf16x4*)(m + r * pitch + 32 * fs + 16 + 4 * g) = hi;
}

// The fused launch's scheduling (sync words, tile order; defined with chunk_bwd_sched_kernel).
__device__ __forceinline__ void bwd_sched_body(const BwdArgs& a, int max_chunks, int sync_words);

// The prep of tile (cidx, h), run by kPrepThreads threads.  COHERENT: its outputs (-G, E)
// are read by scan members of the same launch on other XCDs, so they are written through
// to memory (the caller waits for the stores before it publishes the tile).
template <int K, int V, bool COHERENT>
__device__ __forceinline__ void bwd_prep_body(const BwdArgs& a, int cidx, int h) {
  using L = PrepLds<K, V>;
  constexpr int OP = L::OP, KP = L::KP, AP = L::AP, KB = K / 16, VB = V / 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* sDO = (bf16*)(smem + L::off_do);
  bf16* sADO = (bf16*)(smem + L::off_ado);
  bf16* sKd = (bf16*)(smem + L::off_kd);
  bf16* sQg = sKd;  // Qg replaces Kd once -G is formed
  bf16* sW = (bf16*)(smem + L::off_w);
  bf16* sA = (bf16*)(smem + L::off_a);
  const int H = a.H;
  const int4 ch = chunk_entry(a, cidx);
  const int len = ch.y, row0 = ch.x;
  if (len <= 0) return;
  const size_t tile = (size_t)cidx * H + h;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;
  const bf16* KDF = (const bf16*)a.ws.p[R_KDF] + tile * 64 * K;
  const bf16* WF = (const bf16*)a.ws.p[R_WF] + tile * 64 * K;
  const bf16* QGF = (const bf16*)a.ws.p[R_QGF] + tile * 64 * K;
  const bf16* AF = (const bf16*)a.ws.p[R_AF] + tile * 64 * 64;
  // ---- every global load first: dO rows, Kd, -W, Qg and A fragments (4 x 16 bytes per
  // thread each of Kd, -W and Qg, 2 x 16 of A at K = V = 128).  A^T, W^T and Qg^T are
  // formed from the row-major stagings with transposing LDS reads ----
  constexpr int NDO = 64 * V / 8 / kPrepThreads, NKF = 64 * K / 8 / kPrepThreads, NAF = 64 * 64 / 8 / kPrepThreads;
  bf16x8 xo[NDO], xk[NKF], xw[NKF], xq[NKF], xa[NAF];
#pragma unroll
  for (int q = 0; q < NDO; ++q) {
    const int idx = q * kPrepThreads + tid, t = idx / (V / 8), c0 = (idx % (V / 8)) * 8;
    xo[q] = *(const bf16x8*)(a.dout + ((size_t)(row0 + (t < len ? t : len - 1)) * H + h) * V + c0);
  }
#pragma unroll
  for (int q = 0; q < NKF; ++q) {
    xk[q] = *(const bf16x8*)(KDF + (size_t)(q * kPrepThreads + tid) * 8);
    xw[q] = *(const bf16x8*)(WF + (size_t)(q * kPrepThreads + tid) * 8);
  }
#pragma unroll
  for (int q = 0; q < NAF; ++q) xa[q] = *(const bf16x8*)(AF + (size_t)(q * kPrepThreads + tid) * 8);
#pragma unroll
  for (int q = 0; q < NKF; ++q) xq[q] = *(const bf16x8*)(QGF + (size_t)(q * kPrepThreads + tid) * 8);
  // ---- stage dO (rows past the chunk zero), Kd and -W as row-major [t][k] ----
#pragma unroll
  for (int q = 0; q < NDO; ++q) {
    const int idx = q * kPrepThreads + tid, t = idx / (V / 8), c0 = (idx % (V / 8)) * 8;
    bf16x8 x = xo[q];
    if (t >= len) x = bf16x8{};
    *(bf16x8*)(sDO + t * OP + c0) = x;
  }
#pragma unroll
  for (int q = 0; q < NKF; ++q) {
    // natural fragment piece idx: row 16 rt + l % 16, columns 32 s + 8 (l / 16) ..
    const int idx = q * kPrepThreads + tid, l = idx % 64, fs = (idx / 64) % (K / 32), rt = idx / (64 * (K / 32));
    const int r = 16 * rt + l % 16, g = l / 16;
    *(bf16x8*)(sKd + r * KP + 32 * fs + 8 * g) = xk[q];
    stage_permuted_piece(sW, KP, K, idx, xw[q]);  // -W and A are stored permuted
  }
#pragma unroll
  for (int q = 0; q < NAF; ++q) stage_permuted_piece(sA, AP, 64, q * kPrepThreads + tid, xa[q]);
  __syncthreads();
  // ---- A^T dO: wave w owns row tile w (tokens 16 w ..), every column tile; the A^T
  // fragments are column reads of A ----
  bf16x8 atf[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) atf[s] = lds_col_frag(sA, AP, 32 * s, 16 * wave, lane);
#pragma unroll
  for (int ct = 0; ct < VB; ++ct) {
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) acc = mfma16(atf[s], lds_col_frag(sDO, OP, 32 * s, 16 * ct, lane), acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) sADO[(16 * wave + 4 * kg + r) * OP + 16 * ct + lr] = to_bf16(acc[r]);
  }
  // ---- -G fragments: fragment (b, s) packs the accumulator tiles (2s, b), (2s+1, b) of
  // -G^T = Kd^T (-W); wave w owns fragment rows b = w, w + 4, ... ----
  bf16* NG = (bf16*)a.sc.p[S_NG] + tile * K * K;
  for (int b = wave; b < KB; b += 4) {
    bf16x8 wb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) wb[s] = lds_col_frag(sW, KP, 32 * s, 16 * b, lane);
#pragma unroll
    for (int fs = 0; fs < K / 32; ++fs) {
      f32x4 lo = zero4(), hi = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        lo = mfma16(lds_col_frag(sKd, KP, 32 * s, 16 * (2 * fs), lane), wb[s], lo);
        hi = mfma16(lds_col_frag(sKd, KP, 32 * s, 16 * (2 * fs + 1), lane), wb[s], hi);
      }
      bf16x8 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = to_bf16(lo[r]);
        x[4 + r] = to_bf16(hi[r]);
      }
      if constexpr (COHERENT)
        store16_coherent(NG, (int)frag_off(K, b, fs, lane) * 2, x);
      else
        *(bf16x8*)(NG + frag_off(K, b, fs, lane)) = x;
    }
  }
  __syncthreads();  // A^T dO staged, every read of Kd done
#pragma unroll
  for (int q = 0; q < NKF; ++q) stage_permuted_piece(sQg, KP, K, q * kPrepThreads + tid, xq[q]);
  __syncthreads();
  // ---- E = Qg^T dO - W^T bf16(A^T dO) = Qg^T dO + (-W)^T bf16(A^T dO): wave w owns key
  // tiles w, w + 4, ...; Qg^T and (-W)^T fragments are column reads of the stagings ----
  char* E = (char*)a.sc.p[S_E] + tile * K * V * kEBytes;
  for (int kt = wave; kt < KB; kt += 4) {
    bf16x8 qf[2], wf[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      qf[s] = lds_col_frag(sQg, KP, 32 * s, 16 * kt, lane);
      wf[s] = lds_col_frag(sW, KP, 32 * s, 16 * kt, lane);
    }
#pragma unroll
    for (int ct = 0; ct < VB; ++ct) {
      f32x4 pq = zero4(), pw = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        pq = mfma16(qf[s], lds_col_frag(sDO, OP, 32 * s, 16 * ct, lane), pq);
        pw = mfma16(wf[s], lds_col_frag(sADO, OP, 32 * s, 16 * ct, lane), pw);
      }
      const f32x4 ev = pq + pw;
      const size_t eo = (((size_t)ct * KB + kt) * 64 + lane) * 4;
      if constexpr (kEBytes == 2) {
        bf16x4 eb;
#pragma unroll
        for (int q = 0; q < 4; ++q) eb[q] = to_bf16(ev[q]);
        if constexpr (COHERENT)
          store8_coherent(E, (int)eo * 2, eb);
        else
          *(bf16x4*)(E + eo * 2) = eb;
      } else {
        *(f32x4*)(E + eo * 4) = ev;
      }
    }
  }
}

template <int K, int V>
__global__ __launch_bounds__(kPrepThreads) void chunk_bwd_prep_kernel(BwdArgs a, int sched_words) {
  const int cidx = blockIdx.x, h = blockIdx.y;
  if (sched_words > 0 && cidx == (int)gridDim.x - 1) {
    // one extra column of workgroups: (x = last, y = 0) does the fused launch's scheduling
    // (sync words, tile order), saving a launch of its own
    if (h == 0) bwd_sched_body(a, cidx, sched_words);
    return;
  }
  bwd_prep_body<K, V, false>(a, cidx, h);
}

// One workgroup per (sequence, head, 16-wide V strip) walks the chunks backwards: four
// compute waves (wave w owns the X tiles w K/64 .., as MFMA accumulators, and loads its own
// rows of each chunk's -G into registers one step ahead), a loader wave that streams each
// chunk's E strip and lam into a kBwdRing-deep LDS ring with direct global->LDS loads (two
// chunks ahead), and a history wave that copies X_c out of LDS to the strip-major history
// and, in the fused launch, publishes the step.  Per chunk the waves meet at one barrier
// S(r): X_c staged as bf16 (the B operand, in the permuted contraction order -G was emitted
// in), slot r loaded.
#ifndef KDA_BWD_PREFETCH
#define KDA_BWD_PREFETCH 4
#endif
constexpr int kBwdPrefetch = KDA_BWD_PREFETCH;  // fused launch: steps of L2 look-ahead
#ifndef KDA_PUB_LAG
#define KDA_PUB_LAG 3
#endif
// fused launch: the history wave publishes step r - kPubLag at step r, so the write-through
// stores of kPubLag - 1 steps stay in flight (their completion takes longer than a step when
// the VJP tiles load the memory system)
constexpr int kPubLag = KDA_PUB_LAG;
constexpr int kScanCW = 4;                        // compute waves per V strip
constexpr int kBwdThreads = (kScanCW + 2) * kWave;  // one strip + the loader and the history wave
#ifndef KDA_FUSED_PREP
#define KDA_FUSED_PREP 1  // the prep inside the fused launch (0: a launch of its own before it)
#endif
#ifndef KDA_FUSED_SPW
#define KDA_FUSED_SPW 1
#endif
constexpr int kFusedSPW = KDA_FUSED_SPW;           // V strips per scan member of the fused launch

constexpr int kBwdRing = 3;
template <int K, int V>
struct BwdScanLds {
  static constexpr int off_e = 0;                         // E strip [K/16][64][4] (f32 or bf16)
  static constexpr int off_lam = off_e + K * 16 * kEBytes;  // lam, K f32
  static constexpr int slot = off_lam + K * 4;
  static constexpr int n_load = (K * 16 * kEBytes) / 1024 + 1;
  static constexpr int SP = K + 8;
  static constexpr int off_ds = kBwdRing * slot;          // X_c bf16 [v][k] (x2, by step parity)
  static constexpr int bytes = off_ds + 2 * 16 * SP * 2;
  static_assert(n_load < 64, "vmcnt range");
};

// The scan's per-chunk operands.  Workgroups of the scan launch past the scan's own touch
// one word of every 128-byte line of them while the scan runs on its few CUs, so the scan's
// latency-bound loads find their lines in the caches.  Loads only: the results are folded
// into a value that is never stored.
constexpr int kMaxPrefetch = 20;
struct PrefetchList {
  const char* p[kMaxPrefetch];
  unsigned long long lines[kMaxPrefetch];
  int n;
};

__device__ __forceinline__ void prefetch_lines(const PrefetchList& pf, int w, int nw, char* sink) {
  const unsigned long long stride = (unsigned long long)nw * kBwdThreads;
  unsigned acc = 0;
  for (int r = 0; r < pf.n; ++r) {
    const char* base = pf.p[r];
    const unsigned long long n = pf.lines[r];
    unsigned long long l = (unsigned long long)w * kBwdThreads + threadIdx.x;
    for (; l + 7 * stride < n; l += 8 * stride) {
      unsigned x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *(const unsigned*)(base + (l + u * stride) * 128);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= x[u];
    }
    for (; l < n; l += stride) acc ^= *(const unsigned*)(base + l * 128);
  }
  if (acc == 0x9e3779b9u) *(unsigned*)sink = acc;  // keeps the loads; the value is irrelevant
}

// Scan -> dense hand-off inside the fused backward: the histories go through memory with
// the system-coherent helpers of kda_device.hpp (write-through stores, coherent loads), so no
// L2 write-back or invalidate is needed around the counts -- the write-back of a whole L2 per
// scan step costs microseconds on the scan's serial chain.

// Layout of the fused backward's sync words (ints): [0] unused, [1] abort, then per record
// rec one 128-byte line at kSyncRec + 32 rec holding each V strip's count of finished steps,
// then one word per tile: the prep workgroups' ready flags.
constexpr int kSyncRec = 32;
__host__ __device__ inline int sync_words(int nrec, int tiles) { return kSyncRec + 32 * nrec + tiles; }

// One more step of this strip is in memory: every store of the step was written through and
// waited for (vmcnt) before the call.  Each strip raises its own word (a store, nothing to
// wait for on the scan's chain); a waiting tile takes the minimum over the record's strips.
__device__ __forceinline__ void publish_strip(int* sync, int rec, int strip, int step) {
  __hip_atomic_store(sync + kSyncRec + 32 * rec + strip, step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The scan of SPW V strips of one (sequence, head) per workgroup: per strip four compute
// waves (X tiles in MFMA accumulators), then one loader wave and one history wave for all
// strips.  PUB: the workgroup is a scan member of the fused backward launch, where it takes
// a whole CU like every tile workgroup (two strips per workgroup would leave half the scan's
// CUs to the VJP tiles, but measured slower: 123 against 98 us for the backward call, the
// scan's step lengthening with two compute waves per SIMD).  Its next waves pull the
// operands into L2 ahead of the steps, the rest exit, and after each step's history (X_c)
// is stored the strip's progress word is raised: r + 1 means the strip has finished the
// r + 1 last chunks of the sequence.
template <int K, int V, bool PUB, int SPW>
__device__ __forceinline__ void bwd_scan_body(const BwdArgs& a, int* progress, const int* prep_flags = nullptr,
                                              long long spin_limit = 0) {
  using L = BwdScanLds<K, V>;
  constexpr int CW = kScanCW, KT = K / 16 / CW, NB = K / 32, SP = L::SP;
  static_assert(KT >= 1 && KT * CW == K / 16, "X tiles split evenly over the compute waves");
  constexpr int NSG = V / 16 / SPW;  // strip groups (workgroups) per record
  constexpr int kLoader = CW * SPW, kHistory = kLoader + 1, kPrefetch0 = kLoader + 2;
  constexpr int kPrefetchWaves = 2 * SPW;  // look-ahead lanes: this group's shared lines + its E lines
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int H = a.H;
  int rec, sg;
  if (!xcd_strip_coords(a.num_seqs * H, NSG, rec, sg)) return;
  const int seq = rec / H, h = rec % H;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;
  const int2 sq = seq_entry(a, seq);  // {first chunk, chunk count}
  const int n = sq.y;
  auto tile_of = [&](int r) { return (size_t)(sq.x + max(n - 1 - r, 0)) * H + h; };  // step r's chunk
  auto group = [&](int g) { return smem + g * L::bytes; };  // a strip's LDS (E ring, X staging)
  // Fused launch with the prep inside it: a chunk's -G and E exist once its prep workgroup
  // raised the chunk's flag (after its write-through stores completed).  The loader waits for
  // the flag of step r + 2 before the barrier S(r) after which it, and (one step later) the
  // compute waves, load that step's operands; a first barrier S(-1) covers steps 0 and 1.
  const bool prep_wait = PUB && prep_flags != nullptr;
  auto prep_ready = [&](int q) {
    return __hip_atomic_load(prep_flags + tile_of(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  };
  auto wait_prep = [&](int q) {
    if (!prep_wait || q >= n || lane != 0) return;
    const long long t0 = wall_clock64();
    int* abort_word = progress + 1;
    while (!prep_ready(q)) {
      if (__hip_atomic_load(abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
          wall_clock64() - t0 > spin_limit) {
        __hip_atomic_store(abort_word, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
  };

  if (PUB && wave >= kPrefetch0) {
    // Look-ahead waves pull the operands of the step kBwdPrefetch ahead into the XCD's L2:
    // the shared -G and lam lines split over the record's strip groups (every strip of a
    // record runs on one XCD), plus this group's own E lines.  The lines land in a scratch
    // LDS row.
    if (n <= 0 || wave >= kPrefetch0 + kPrefetchWaves) return;
    const int pl = (wave - kPrefetch0) * kWave + lane;
    char* sink = smem + SPW * L::bytes + (wave & 1) * 1024;
    constexpr int kG = K * K * 2 / 128, kLam = K * 4 / 128, kE = K * 16 * kEBytes / 128;
    constexpr int kShared = (kG + kLam + NSG - 1) / NSG;  // lanes for this group's share
    // (a hint: when the lanes are fewer than the lines, the last lines are not pulled ahead)
    auto prefetch = [&](int q) {
      if (q >= n) return;
      if (prep_wait && !prep_ready(q)) return;  // not written yet: no stale line pulled into L2
      const size_t tile = tile_of(q);
      const char* src = nullptr;
      if (pl < kShared) {
        const int l = sg + NSG * pl;
        if (l < kG) src = (const char*)((const bf16*)a.sc.p[S_NG] + tile * K * K) + l * 128;
        else if (l < kG + kLam) src = (const char*)((const float*)a.ws.p[R_LAM] + tile * K) + (l - kG) * 128;
      } else if (pl - kShared < SPW * kE) {
        const int g = (pl - kShared) / kE, l = (pl - kShared) % kE;
        src = (const char*)a.sc.p[S_E] + (tile * K * V + (size_t)(sg * SPW + g) * K * 16) * kEBytes + l * 128;
      }
      if (src) dma16(src, sink);
    };
    if (prep_wait) ring_barrier();  // S(-1)
    for (int q = 0; q < kBwdPrefetch; ++q) prefetch(q);
    for (int b = 0; b < n; ++b) {
      ring_barrier();  // S(b)
      prefetch(b + kBwdPrefetch);
    }
    ring_barrier();  // final
    wait_vmcnt<0>();  // no LDS write may land after the workgroup ends
    return;
  }
  if (n <= 0) {
    // an empty sequence: the initial-state gradient is the final-state gradient
    if (wave < kLoader && wave % CW == 0 && a.ds0) {
      const int v0 = (sg * SPW + wave / CW) * 16;
      for (int kt = 0; kt < K / 16; ++kt) {
        const size_t o = (((size_t)seq * H + h) * V + v0 + lr) * K + 16 * kt + 4 * kg;
        *(float4*)(a.ds0 + o) = a.dsfin ? *(const float4*)(a.dsfin + o) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    return;
  }
  if (wave == kLoader) {
    // ---- loader wave: step r's slot (r % kBwdRing) of each strip holds its E strip and lam ----
    auto issue = [&](int r) {
      const size_t tile = tile_of(r);  // clamped past the last step: a fixed load count
#pragma unroll
      for (int g = 0; g < SPW; ++g) {
        char* slot = group(g) + (r % kBwdRing) * L::slot;
        const char* e = (const char*)a.sc.p[S_E] + (tile * K * V + (size_t)(sg * SPW + g) * K * 16) * kEBytes + lane * 16;
#pragma unroll
        for (int b = 0; b < (K * 16 * kEBytes) / 1024; ++b) dma16(e + b * 1024, slot + L::off_e + b * 1024);
        if (lane < K / 4) dma16((const float*)a.ws.p[R_LAM] + tile * K + lane * 4, slot + L::off_lam);
      }
    };
    if (prep_wait) {
      wait_prep(0);
      wait_prep(1);
      ring_barrier();  // S(-1)
    }
    issue(0);
    issue(1);
    for (int r = 0; r < n; ++r) {
      wait_vmcnt<SPW * L::n_load>();  // slot r complete (step r + 1's loads may be in flight)
      wait_prep(r + 2);
      ring_barrier();                 // S(r): slot r - 1 is consumed
      issue(r + 2);
    }
    if (PUB) ring_barrier();  // final
    wait_vmcnt<0>();  // no LDS write may land after the workgroup ends
    return;
  }
  if (wave == kHistory) {
    // ---- history wave: X_c of step r (bf16 [v][k] in LDS) is read after S(r) and stored
    // into each strip's [K][16] block of the strip-major history, 512 contiguous bytes per
    // store instruction.  In the fused launch step r - kPubLag is published once its stores
    // have completed (write-through stores may take microseconds) ----
    if (prep_wait) ring_barrier();  // S(-1)
    for (int r = 0; r < n; ++r) {
      // step r - kPubLag's stores (each later step added SPW (K / 16 stores + one publish))
      if (PUB && r >= kPubLag) wait_vmcnt<(kPubLag - 1) * SPW * (K / 16 + 1)>();
      ring_barrier();  // S(r)
      if (PUB && r >= kPubLag && lane == 0)
#pragma unroll
        for (int g = 0; g < SPW; ++g) publish_strip(progress, rec, sg * SPW + g, r - kPubLag);
#pragma unroll
      for (int g = 0; g < SPW; ++g) {
        // X_c as bf16 [v][k] (the compute waves' B-operand staging): one transposing read
        // per 16 keys gives lane l keys 16 it + l % 16, values 4 (l / 16) .. + 3
        const bf16* sx = (const bf16*)(group(g) + L::off_ds + (r & 1) * 16 * SP * 2);
        bf16x4 hv[K / 16];
#pragma unroll
        for (int it = 0; it < K / 16; ++it) hv[it] = lds_col_frag4(sx, SP, 0, 16 * it, lane);
        bf16* DSH = (bf16*)a.sc.p[S_DSH] + tile_of(r) * K * V + (size_t)(sg * SPW + g) * K * 16;
#pragma unroll
        for (int it = 0; it < K / 16; ++it) {
          const int kk = 16 * it + lr, c4 = 4 * kg;
          if (PUB)
            store8_coherent(DSH, (kk * 16 + c4) * 2, hv[it]);
          else
            *(bf16x4*)(DSH + (size_t)kk * 16 + c4) = hv[it];
        }
      }
    }
    if (PUB) {
      wait_vmcnt<0>();
      if (lane == 0)
#pragma unroll
        for (int g = 0; g < SPW; ++g) publish_strip(progress, rec, sg * SPW + g, n - 1);
      ring_barrier();  // final
    }
    return;
  }
  if (wave > kHistory) return;  // (only in a launch with more waves than the roles need)

  // ---- compute waves of strip g: X tiles cw * KT .. (rows 16 kt + 4 (l / 16) + r, column
  // l % 16) ----
  const int g = wave / CW, cw = wave % CW;
  const int v0 = (sg * SPW + g) * 16;
  char* gl = group(g);
  f32x4 X[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int k0 = 16 * (cw * KT + kt) + 4 * kg;
    if (a.dsfin) {
      const float4 s = *(const float4*)(a.dsfin + (((size_t)seq * H + h) * V + v0 + lr) * K + k0);
      X[kt][0] = s.x; X[kt][1] = s.y; X[kt][2] = s.z; X[kt][3] = s.w;
    } else {
      X[kt] = zero4();
    }
  }
  // Step r's -G rows of this wave's X tiles (permuted A fragments, 8 KB per wave) go straight
  // from memory into registers, one step ahead of their use: staged in LDS (a DMA write and a
  // read of 32 KB per step) they made the CU's LDS bandwidth the bound of the step.  The prep
  // launch wrote them; the fused launch's look-ahead waves pull them into L2 a few steps
  // earlier.
  struct Ops {
    bf16x8 g[KT][NB];
  };
  auto load_ops = [&](Ops& o, int r) {
    const bf16* G = (const bf16*)a.sc.p[S_NG] + tile_of(r) * K * K;  // clamped past the last step
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int s = 0; s < NB; ++s) o.g[kt][s] = *(const bf16x8*)(G + frag_off(K, cw * KT + kt, s, lane));
  };
  auto step = [&](int r, const Ops& o) {
    bf16* sDS = (bf16*)(gl + L::off_ds + (r & 1) * 16 * SP * 2);
    // stage X_c as bf16 [v][k]: the B operand of the strip's compute waves, and the history's
    // source
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int k0 = 16 * (cw * KT + kt) + 4 * kg;
      bf16x4 x;
#pragma unroll
      for (int q = 0; q < 4; ++q) x[q] = to_bf16(X[kt][q]);
      *(bf16x4*)(sDS + lr * SP + k0) = x;
    }
    wait_lgkm0();
    ring_barrier();  // S(r)
    // B fragments of X_c in the permuted contraction order of -G's fragments: element e of
    // lane l is key 32 s + 16 (e / 4) + 4 (l / 16) + e % 4
    bf16x8 xb[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const bf16x4 lo = *(const bf16x4*)(sDS + lr * SP + 32 * s + 4 * kg);
      const bf16x4 hi = *(const bf16x4*)(sDS + lr * SP + 32 * s + 16 + 4 * kg);
      xb[s] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    const char* slot = gl + (r % kBwdRing) * L::slot;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int ktg = cw * KT + kt;
      const float4 lam = *(const float4*)(slot + L::off_lam + (16 * ktg + 4 * kg) * 4);
      f32x4 e;
      if constexpr (kEBytes == 2) {
        const bf16x4 eb = *(const bf16x4*)(slot + L::off_e + (ktg * 64 + lane) * 8);
#pragma unroll
        for (int q = 0; q < 4; ++q) e[q] = (float)eb[q];
      } else {
        e = *(const f32x4*)(slot + L::off_e + (ktg * 64 + lane) * 16);
      }
      f32x4 acc;
      acc[0] = fmaf(lam.x, X[kt][0], e[0]);
      acc[1] = fmaf(lam.y, X[kt][1], e[1]);
      acc[2] = fmaf(lam.z, X[kt][2], e[2]);
      acc[3] = fmaf(lam.w, X[kt][3], e[3]);
#pragma unroll
      for (int s = 0; s < NB; ++s) acc = mfma16(o.g[kt][s], xb[s], acc);
      X[kt] = acc;
    }
  };
  Ops o0, o1;
  if (prep_wait) ring_barrier();  // S(-1)
  load_ops(o0, 0);
  for (int r = 0; r < n; r += 2) {
    load_ops(o1, r + 1);
    step(r, o0);
    if (r + 1 < n) {
      load_ops(o0, r + 2);
      step(r + 1, o1);
    }
  }
  if (PUB) ring_barrier();  // final
  if (a.ds0) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int k0 = 16 * (cw * KT + kt) + 4 * kg;
      *(float4*)(a.ds0 + (((size_t)seq * H + h) * V + v0 + lr) * K + k0) =
          make_float4(X[kt][0], X[kt][1], X[kt][2], X[kt][3]);
    }
  }
}

template <int K, int V>
__global__ __launch_bounds__(kBwdThreads) void chunk_bwd_scan_kernel(BwdArgs a, PrefetchList pf, int scan_blocks) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  if ((int)blockIdx.x >= scan_blocks) {
    prefetch_lines(pf, blockIdx.x - scan_blocks, gridDim.x - scan_blocks, smem);
    return;
  }
  bwd_scan_body<K, V, false, 1>(a, nullptr);
}

// ---------------------------------------------------------------------------
// dense chunk VJP
// ---------------------------------------------------------------------------
constexpr int kVjpThreads = 1024;  // 16 waves per (chunk, head): hides global-load latency
constexpr int kVjpWaves = kVjpThreads / kWave;

// 1024 threads per tile.  Every global operand of the tile is requested in one batch at the
// start (dO, v and beta kh e^G rows staged in LDS, the state rows in registers), so a tile
// waits on one global round trip instead of one per row tile and item.  T, dT, T^T dT and dW
// only ever feed bf16 MFMA operands and are stored as bf16; T, dT and T^T dT reuse the
// (spare, delta) region once the dQg / dKd / dW / dA phase is done.
constexpr int kDenseThreads = 1024;
constexpr int kDenseWaves = kDenseThreads / kWave;

template <int K, int V>
struct DenseSmem {
  static constexpr int TP = 64 + 8;   // bf16 row stride of the 64 x 64 matrices
  static_assert(TP % 8 == 0 && (K + 8) % 4 == 0 && (V + 8) % 4 == 0,
                "column-fragment reads need 8-byte rows, the PD row reads 16-byte rows");
  static constexpr int KP = K + 8;    // bf16 row stride of dW
  static constexpr int VP = V + 8;
  static constexpr size_t off_du = 0;                           // bf16 [64][VP] dU
  static constexpr size_t off_dul = off_du + 64 * VP * 2;       // bf16 [64][VP] spare (T, dT, T^T dT after PA)
  static constexpr size_t off_dl = off_dul + 64 * VP * 2;       // bf16 [64][VP] delta
  static constexpr size_t off_dw = off_dl + 64 * VP * 2;        // bf16 [64][KP] dW
  static constexpr size_t off_b = off_dw + 64 * KP * 2;         // f32 [64] beta
  static constexpr size_t off_pv = off_b + 64 * 4;              // f32 [V/16][64] dbeta partials
  static constexpr size_t off_pm = off_pv + (V / 16) * 64 * 4;  // f32 [4][64]
  static constexpr size_t off_do = off_pm + 4 * 64 * 4;        // bf16 [64][VP] dO (rows >= len zero)
  static constexpr size_t off_v = off_do + 64 * VP * 2;          // bf16 [64][VP] v (rows >= len zero)
  static constexpr size_t off_kb = off_v + 64 * VP * 2;          // bf16 [64][KP] beta kh e^G
  static constexpr size_t off_a = off_kb + 64 * KP * 2;          // bf16 [64][TP] A (its A^T fragments)
  static constexpr size_t end = off_a + 64 * TP * 2;
  // T, dT, T^T dT (bf16 [64][TP] each, after dA): in the dU-lo / delta region when it is
  // large enough (V = 128), else behind everything
  static constexpr bool kAlias = 3 * 64 * TP * 2 <= 2 * 64 * VP * 2;
  static constexpr size_t off_t = kAlias ? off_dul : end;
  static constexpr size_t off_dt = off_t + 64 * TP * 2;
  static constexpr size_t off_y = off_dt + 64 * TP * 2;
  static constexpr size_t bytes = kAlias ? end : off_y + 64 * TP * 2;
};

// Gate: called by every thread of the tile once its scan-independent loads are in flight
// and before its first read of the scan's histories (dS', dDelta); a no-op when the scan
// completed in an earlier launch.
struct NoGate {
  static constexpr bool kCoherent = false;  // histories from an earlier launch: plain loads
  __device__ void operator()() const {}
};

template <int K, int V, class Gate = NoGate>
__device__ __forceinline__ void dense_tile(const BwdArgs& a, int cidx, int hidx, int4 ch, const Gate& gate = Gate()) {
  using L = DenseSmem<K, V>;
  constexpr int MP = L::TP, KP = L::KP, VP = L::VP;
  constexpr int kVjpThreads = kDenseThreads, kVjpWaves = kDenseWaves;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* sT = (bf16*)(smem + L::off_t);
  bf16* sDT = (bf16*)(smem + L::off_dt);
  bf16* sY = (bf16*)(smem + L::off_y);
  bf16* sDW = (bf16*)(smem + L::off_dw);
  bf16* sDU = (bf16*)(smem + L::off_du);
  bf16* sDL = (bf16*)(smem + L::off_dl);
  float* sB = (float*)(smem + L::off_b);
  float* sPV = (float*)(smem + L::off_pv);
  float* sPM = (float*)(smem + L::off_pm);
  bf16* sDO = (bf16*)(smem + L::off_do);
  bf16* sV = (bf16*)(smem + L::off_v);
  bf16* sKB = (bf16*)(smem + L::off_kb);

  // ch: the chunk's table entry {row0, len, ...}
  const int len = ch.y;
  if (len <= 0) return;
  const int H = a.H, h = hidx;
  const size_t tile = (size_t)cidx * H + h;
  const int row0 = ch.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;

  const bf16* Tg = (const bf16*)a.ws.p[R_T] + tile * 64 * 64;
  const float* MPg = (const float*)a.ws.p[R_MP] + tile * 64 * 64;
  const float* Gg = (const float*)a.ws.p[R_G] + tile * 64 * K;
  const float* RK = (const float*)a.ws.p[R_RK] + tile * 64;
  const float* SH = (const float*)a.ws.p[R_SH] + tile * K * V;
  const bf16* DLF = (const bf16*)a.ws.p[R_DLF] + tile * 64 * V;
  const bf16* DSH = (const bf16*)a.sc.p[S_DSH] + tile * K * V;
  // X_c (dS' at the chunk end, K x V) staged for dU = dDelta = A^T dO + Kd X_c after the gate:
  // keys 0..63 in the spare region, keys 64.. in the dW region (both free until PA), pitch VP
  static_assert(K <= 64 || V <= K, "X_c's second key half fits the dW region");
  bf16* sX0 = (bf16*)(smem + L::off_dul);
  bf16* sX1 = (bf16*)(smem + L::off_dw);
  float* DQG = (float*)a.sc.p[S_DQG] + tile * 64 * K;
  float* DKD = (float*)a.sc.p[S_DKD] + tile * 64 * K;
  float* DKB = (float*)a.sc.p[S_DKB] + tile * 64 * K;
  bf16* DA = (bf16*)a.sc.p[S_DA] + tile * 64 * 64;
  bf16* DMP = (bf16*)a.sc.p[S_DMP] + tile * 64 * 64;

  // PA's state rows: wave w owns key tile w / (4 / RPW) and RPW row tiles; its f32 S and
  // dS' rows are requested first, with everything P0 loads
  constexpr int NKT = 4 * (K / 16);
  constexpr int RPW = NKT / kVjpWaves;  // row tiles per wave (2 for K = 128, 1 for K = 64)
  constexpr int NVS = V / 32;
  static_assert(RPW >= 1 && 4 % RPW == 0, "row tiles per wave");
  const int pa_ct = wave / (4 / RPW), pa_rt0 = (wave % (4 / RPW)) * RPW;
  float xs[NVS][8];
  bf16x8 xd[NVS];
  const int pa_c = 16 * pa_ct + lr;
#pragma unroll
  for (int sv = 0; sv < NVS; ++sv) load8f(SH + (size_t)pa_c * V + 32 * sv + 8 * kg, xs[sv]);

  // ---- P0: stage dU, delta, beta, dO, v, beta kh e^G; clear partials; T waits in
  // registers until after dA ----
  // Every load of P0 is issued before the first LDS write (fixed per-thread counts), so the
  // stage costs one global round trip.
  static_assert(64 * 64 % (4 * kDenseThreads) == 0, "T staging");
  static_assert(64 * V / 8 <= kDenseThreads && 64 * K / 8 <= kDenseThreads, "one row chunk per thread");
  constexpr int NDL = (64 * V / 8 + kDenseThreads - 1) / kDenseThreads;
  // rows of dO, v (8 values per thread and matrix) and k, G: clamped rows, zeroed after
  const int t = tid / (V / 8), c0 = (tid % (V / 8)) * 8;
  const int tk = tid / (K / 8), ck = (tid % (K / 8)) * 8, tkc = tk < 64 ? tk : 63;
  const size_t rv = (size_t)(row0 + (t < len ? t : len - 1)) * H + h;
  const size_t rk = (size_t)(row0 + (tk < len ? tk : len - 1)) * H + h;
  bf16x8 xo = *(const bf16x8*)(a.dout + rv * V + c0);
  bf16x8 xv = *(const bf16x8*)(a.v + rv * V + c0);
  const bf16x8 xk = *(const bf16x8*)(a.k + rk * K + ck);
  float gk[8];
  load8f(Gg + tkc * K + ck, gk);
  const float bt = ((const float*)a.ws.p[R_BETA])[tile * 64 + tkc], rkt = RK[tkc];
  bf16x4 treg[64 * 64 / (4 * kDenseThreads)];
#pragma unroll
  for (int q = 0; q < 64 * 64 / (4 * kDenseThreads); ++q) treg[q] = *(const bf16x4*)(Tg + (q * kDenseThreads + tid) * 4);
  bf16x8 dlf[NDL];
#pragma unroll
  for (int q = 0; q < NDL; ++q) dlf[q] = *(const bf16x8*)(DLF + (size_t)min(q * kDenseThreads + tid, 64 * V / 8 - 1) * 8);
  // dU tiles of this wave: tile id = wave + 16 j -> row tile id % 4, column tile id / 4; the
  // A^T and Kd fragments of its row tile
  constexpr int NDU = (4 * V / 16) / kDenseWaves;  // 2 at V = 128, 1 at V = 64
  static_assert(NDU >= 1 && NDU * kDenseWaves == 4 * V / 16, "dU tiles per wave");
  const int du_rt = wave % 4;
  bf16x8 du_at[2], du_kd[K / 32];
  // A (permuted fragments, one 16-byte piece per thread of the first 512), staged row-major
  // in P0: the A^T fragments of dU = A^T dO are column reads of it
  const bf16x8 xa = tid < 512 ? *(const bf16x8*)((const bf16*)a.ws.p[R_AF] + tile * 64 * 64 + (size_t)tid * 8)
                              : bf16x8{};
#pragma unroll
  for (int s2 = 0; s2 < K / 32; ++s2)
    du_kd[s2] = *(const bf16x8*)((const bf16*)a.ws.p[R_KDF] + tile * 64 * K + frag_off(K, du_rt, s2, lane));
  // operands of later phases, requested with the rest (each would otherwise cost a global
  // round trip of its own after the gate): beta rows and lam of PA's key column
  const float beta_row = ((const float*)a.ws.p[R_BETA])[tile * 64 + (tid & 63)];
  const float lam_pa = ((const float*)a.ws.p[R_LAM])[tile * K + pa_c];
  // ---- P0 (scan-independent, before the gate): stage dO, v, beta kh e^G, delta, beta;
  // dQg = dO S^T and dA = tril(dO delta^T) need nothing from the scan ----
  {
    const float bk = tk < len ? bt * rkt : 0.f;
    bf16x8 xb;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xo[e] = t < len ? xo[e] : to_bf16(0.f);
      xv[e] = t < len ? xv[e] : to_bf16(0.f);
      xb[e] = to_bf16(bk * to_f32(xk[e]) * __expf(gk[e]));
    }
    if (t < 64) {
      *(bf16x8*)(sDO + t * VP + c0) = xo;
      *(bf16x8*)(sV + t * VP + c0) = xv;
    }
    if (tk < 64) *(bf16x8*)(sKB + tk * KP + ck) = xb;
  }
  // delta from its B-operand fragments [strip][2][64 lanes][8] in the scan's permuted
  // token order: element e of lane l is t = 32 s + 16 (e/4) + 4 (l/16) + e%4
#pragma unroll
  for (int q = 0; q < NDL; ++q) {
    const int idx = q * kDenseThreads + tid;
    if (idx >= 64 * V / 8) break;
    const int lane_ = idx % 64, sl = (idx / 64) % 2, strip = idx / 128;
    const int vv = 16 * strip + lane_ % 16, t0 = 32 * sl + 4 * (lane_ / 16);
#pragma unroll
    for (int e = 0; e < 8; ++e) sDL[(t0 + 16 * (e / 4) + e % 4) * VP + vv] = dlf[q][e];
  }
  if (tid < 64) sB[tid] = beta_row;
  if (tid < 512) stage_permuted_piece((bf16*)(smem + L::off_a), L::TP, 64, tid, xa);
  for (int idx = tid; idx < 4 * 64; idx += kVjpThreads) sPM[idx] = 0.f;
  __syncthreads();
  // dQg for PA's items: wave w owns key tile pa_ct and RPW row tiles; the f32 state rows
  // S[c][.] of its 16 keys are split into hi + lo bf16 where they are used (a few VALU
  // operations instead of registers held across the phases)
  {
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int rt = pa_rt0 + q, i = 16 * rt + lr;
      const int p = rt + 4 * pa_ct;
      f32x4 accQ = zero4();
#pragma unroll
      for (int sv = 0; sv < NVS; ++sv) {
        bf16x8 sHi, sLo;
        split8(xs[sv], sHi, sLo);
        const bf16x8 aO = *(const bf16x8*)(sDO + i * VP + 32 * sv + 8 * kg);
        accQ = mfma16(aO, sHi, accQ);
        accQ = mfma16(aO, sLo, accQ);
      }
      // raw dQg in C-layout item order (consumed with the same lane ownership)
      *(f32x4*)(DQG + ((size_t)p * 64 + lane) * 4) = accQ;
    }
  }
  // dA = tril(dO delta^T), 16x16 blocks of the lower triangle; upper blocks zero
  for (int p = wave; p < 16; p += kVjpWaves) {
    const int ba = p / 4, bb = p % 4;
    if (bb > ba) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) DA[(16 * ba + 4 * kg + rr) * 64 + 16 * bb + lr] = to_bf16(0.f);
      continue;
    }
    const int i = 16 * ba + lr, j = 16 * bb + lr;
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < V / 32; ++s) {
      const int vv = 32 * s + 8 * kg;
      acc = mfma16(*(const bf16x8*)(sDO + i * VP + vv), *(const bf16x8*)(sDL + j * VP + vv), acc);
    }
    const int jj = 16 * bb + lr;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ii = 16 * ba + 4 * kg + rr;
      DA[ii * 64 + jj] = to_bf16(jj <= ii ? acc[rr] : 0.f);
    }
  }

  // the scan-independent half of dU: A^T dO (dO staged above, tokens down the contraction)
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) du_at[s2] = lds_col_frag((const bf16*)(smem + L::off_a), L::TP, 32 * s2, 16 * du_rt, lane);
  f32x4 du_acc[NDU];
#pragma unroll
  for (int j = 0; j < NDU; ++j) {
    const int ct = (wave + kDenseWaves * j) / 4;
    du_acc[j] = zero4();
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) du_acc[j] = mfma16(du_at[s2], lds_col_frag(sDO, VP, 32 * s2, 16 * ct, lane), du_acc[j]);
  }

  // xs made opaque: PA splits it again instead of keeping this split's 32 registers alive
#pragma unroll
  for (int sv = 0; sv < NVS; ++sv)
#pragma unroll
    for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(xs[sv][e]));

  gate();
  // ---- the scan's histories (bf16, strip-major as the scan's strips wrote them): dS'
  // rows of PA's key tile from [V/16][K][16], dU = dDelta from [V/16][4][16 v][16 t] ----
#pragma unroll
  for (int sv = 0; sv < NVS; ++sv) {
    const int col = 32 * sv + 8 * kg;  // 8 columns inside strip col / 16
    const size_t off = (size_t)(col / 16) * K * 16 + (size_t)pa_c * 16 + col % 16;
    if (Gate::kCoherent) {
      xd[sv] = load16_coherent_bf16(DSH, (int)off * 2);
    } else {
      xd[sv] = *(const bf16x8*)(DSH + off);
    }
  }
  // X_c from the strip-major history [V/16][K][16]: 16-byte piece p = (strip, key, half)
  // -> row key, columns 16 strip + 8 half of the staged [key][VP] matrix
  {
    constexpr int NP = K * V / 8, NPT = (NP + kDenseThreads - 1) / kDenseThreads;
    bf16x8 xp[NPT];
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int p = min(q * kDenseThreads + tid, NP - 1);
      xp[q] = Gate::kCoherent ? load16_coherent_bf16(DSH, p * 16) : *(const bf16x8*)(DSH + (size_t)p * 8);
    }
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
      const int p = q * kDenseThreads + tid;
      if (p >= NP) break;
      const int st = p / (K * 2), key = (p / 2) % K, half = p % 2;
      bf16* row = key < 64 ? sX0 + key * VP : sX1 + (key - 64) * VP;
      *(bf16x8*)(row + 16 * st + 8 * half) = xp[q];
    }
  }
  __syncthreads();
  // dU = A^T dO + Kd X_c (bf16, the operand of PA and PB)
#pragma unroll
  for (int j = 0; j < NDU; ++j) {
    const int ct = (wave + kDenseWaves * j) / 4;
#pragma unroll
    for (int s2 = 0; s2 < K / 32; ++s2) {
      const bf16* xm = s2 < 2 ? sX0 : sX1;
      du_acc[j] = mfma16(du_kd[s2], lds_col_frag(xm, VP, 32 * (s2 % 2), 16 * ct, lane), du_acc[j]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sDU[(16 * du_rt + 4 * kg + r) * VP + 16 * ct + lr] = to_bf16(du_acc[j][r]);
  }
  __syncthreads();

  // ---- PA: dKd, dW over the 64 x K grid (same items as dQg) ----
  // The f32 rows S[c][.] of the wave's 16 keys (split into hi + lo bf16 where they are used)
  // and their bf16 dS'[c][.]; the same rows give dlam = lam * sum_v S dS'.
  {
    const int ct = pa_ct, rt0 = pa_rt0;
    const int c = 16 * ct + lr;
    const float lamc = lam_pa;  // c == pa_c
    float dl = 0.f;
#pragma unroll
    for (int sv = 0; sv < NVS; ++sv)
#pragma unroll
      for (int e = 0; e < 8; ++e) dl = fmaf(xs[sv][e], to_f32(xd[sv][e]), dl);
    dl = swap32_sum(swap16_sum(dl));
    if (rt0 == 0 && kg == 0) ((float*)a.sc.p[S_DGL])[tile * K + c] = dl * lamc;
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int rt = rt0 + q, i = 16 * rt + lr;
      const int p = rt + 4 * ct;
      f32x4 accK = zero4(), accW = zero4();
#pragma unroll
      for (int sv = 0; sv < NVS; ++sv) {
        const int vv = 32 * sv + 8 * kg;
        bf16x8 sHi, sLo;
        split8(xs[sv], sHi, sLo);
        const bf16x8 uHi = *(const bf16x8*)(sDU + i * VP + vv);
        const bf16x8 aL = *(const bf16x8*)(sDL + i * VP + vv);
        accK = mfma16(aL, xd[sv], accK);
        accW = mfma16(uHi, sHi, accW);
        accW = mfma16(uHi, sLo, accW);
      }
      *(f32x4*)(DKD + ((size_t)p * 64 + lane) * 4) = accK;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) sDW[(16 * rt + 4 * kg + rr) * KP + c] = to_bf16(-accW[rr]);
    }
  }
  __syncthreads();
  // delta is consumed: the spare and delta regions now hold T (bf16) and a zeroed dT
#pragma unroll
  for (int q = 0; q < 64 * 64 / (4 * kDenseThreads); ++q) {
    const int idx = (q * kDenseThreads + tid) * 4, i = idx / 64, j = idx % 64;
    bf16* t = sT + i * MP + j;
    *(bf16x4*)t = treg[q];
    bf16* z = sDT + i * MP + j;
    z[0] = z[1] = z[2] = z[3] = to_bf16(0.f);
  }
  __syncthreads();

  // PD's M' entries (wave p < 10 owns PD item p), requested before PB and PC
  static_assert(kVjpWaves >= 10, "one PD item per wave");
  float mp_pd[4] = {0.f, 0.f, 0.f, 0.f};
  if (wave < 10) {
    const int ba = wave < 1 ? 0 : wave < 3 ? 1 : wave < 6 ? 2 : 3;
    const int bb = wave - (ba * (ba + 1)) / 2;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) mp_pd[rr] = MPg[(16 * ba + 4 * kg + rr) * 64 + 16 * bb + lr];
  }
  // The decay part's first loads (q and k rows, G of the tile) touched once per 128-byte
  // line, so they come from L2 when the decay part starts; the value is only kept alive.
  float warm = 0.f;
  {
    constexpr int LQ = K * 2 / 128, LG = K * 4 / 128;  // lines per row of q / k and of G
    constexpr int NQK = 64 * LQ;
    static_assert(2 * NQK + 64 * LG <= kDenseThreads, "one line per thread");
    if (tid < 2 * NQK) {
      const int r = min((tid % NQK) / LQ, len - 1), l = tid % LQ;
      const bf16* base = tid < NQK ? a.q : a.k;
      warm = *(const float*)(base + ((size_t)(row0 + r) * H + h) * K + 64 * l);
    } else if (tid < 2 * NQK + 64 * LG) {
      warm = Gg[(size_t)(tid - 2 * NQK) * 32];
    }
  }

  // ---- PB: dT (lower blocks), d(beta v), d(beta kh e^G) ----
  for (int p = wave; p < 10; p += kVjpWaves) {
    const int ba = p < 1 ? 0 : p < 3 ? 1 : p < 6 ? 2 : 3;
    const int bb = p - (ba * (ba + 1)) / 2;
    const int i = 16 * ba + lr, j = 16 * bb + lr;
    const float bj = j < len ? sB[j] : 0.f;
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < V / 32; ++s) {
      const bf16x8 vr = *(const bf16x8*)(sV + j * VP + 32 * s + 8 * kg);
      bf16x8 fb;
#pragma unroll
      for (int e = 0; e < 8; ++e) fb[e] = to_bf16(bj * to_f32(vr[e]));
      acc = mfma16(*(const bf16x8*)(sDU + i * VP + 32 * s + 8 * kg), fb, acc);
    }
#pragma unroll
    for (int s = 0; s < K / 32; ++s)
      acc = mfma16(*(const bf16x8*)(sDW + i * KP + 32 * s + 8 * kg), *(const bf16x8*)(sKB + j * KP + 32 * s + 8 * kg), acc);
    const int jj = 16 * bb + lr;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sDT[(16 * ba + 4 * kg + rr) * MP + jj] = to_bf16(acc[rr]);
  }
  // d(beta v) = T^T dU  -> dv and beta partials
  for (int p = wave; p < 4 * (V / 16); p += kVjpWaves) {
    const int rt = p % 4, ct = p / 4;
    const int j = 16 * rt + lr, col = 16 * ct + lr;
    f32x4 acc = zero4();
    for (int s = (16 * rt) / 32; s < 2; ++s)
      acc = mfma16(lds_col_frag(sT, MP, 32 * s, 16 * rt, lane), lds_col_frag(sDU, VP, 32 * s, 16 * ct, lane), acc);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int jj = 16 * rt + 4 * kg + rr;
      float part = 0.f;
      if (jj < len) {
        const size_t off = (size_t)(row0 + jj) * a.gld_v + (size_t)h * V + col;
        a.dv[off] = to_bf16(sB[jj] * acc[rr]);
        part = acc[rr] * to_f32(sV[jj * VP + col]);
      }
      part = group_sum<16>(part);
      if (lr == 0) sPV[ct * 64 + jj] = part;
    }
  }
  // d(beta kh e^G) = T^T dW, raw in C-layout item order (the decay kernel applies it)
  for (int p = wave; p < NKT; p += kVjpWaves) {
    const int rt = p % 4, ct = p / 4;
    const int j = 16 * rt + lr, c = 16 * ct + lr;
    f32x4 acc = zero4();
    for (int s = (16 * rt) / 32; s < 2; ++s)
      acc = mfma16(lds_col_frag(sT, MP, 32 * s, 16 * rt, lane), lds_col_frag(sDW, KP, 32 * s, 16 * ct, lane), acc);
    *(f32x4*)(DKB + ((size_t)p * 64 + lane) * 4) = acc;
  }
  __syncthreads();

  // ---- PC: Y = T^T dT ----
  for (int p = wave; p < 16; p += kVjpWaves) {
    const int rt = p / 4, ct = p % 4;
    const int i = 16 * rt + lr, jcol = 16 * ct + lr;
    f32x4 acc = zero4();
    for (int s = (16 * rt) / 32; s < 2; ++s)
      acc = mfma16(lds_col_frag(sT, MP, 32 * s, 16 * rt, lane), lds_col_frag(sDT, MP, 32 * s, 16 * ct, lane), acc);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sY[(16 * rt + 4 * kg + rr) * MP + jcol] = to_bf16(acc[rr]);
  }
  __syncthreads();

  // ---- PD: dM = -(Y T^T), strictly lower; dM' = beta_i dM ----
  for (int p = wave; p < 10; p += kVjpWaves) {
    const int ba = p < 1 ? 0 : p < 3 ? 1 : p < 6 ? 2 : 3;
    const int bb = p - (ba * (ba + 1)) / 2;
    const int i = 16 * ba + lr, j = 16 * bb + lr;
    const float* mp = mp_pd;  // M' entries of this lane's outputs (p == wave)
    f32x4 acc = zero4();
    const int nsteps = (16 * bb + 15) / 32 + 1;
    for (int s = 0; s < nsteps; ++s) {
      const int b0 = 32 * s + 8 * kg;  // rows are 16-byte aligned (MP * 2 = 144 bytes)
      acc = mfma16(*(const bf16x8*)(sY + i * MP + b0), *(const bf16x8*)(sT + j * MP + b0), acc);
    }
    const int jj = 16 * bb + lr;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ii = 16 * ba + 4 * kg + rr;
      const float dm = jj < ii ? -acc[rr] : 0.f;
      DMP[ii * 64 + jj] = to_bf16(sB[ii] * dm);
      float part = dm * mp[rr];
      part = group_sum<16>(part);
      if (lr == 0) sPM[bb * 64 + ii] = part;
    }
  }
  for (int idx = tid; idx < 64 * 64; idx += kVjpThreads) {
    const int ii = idx / 64, jj = idx % 64;
    if (jj / 16 > ii / 16) DMP[idx] = to_bf16(0.f);
  }
  __syncthreads();

  // ---- PE: dbeta partial (U and M' terms); lam * dL/dlam was written in PA ----
  if (tid < 64) {
    float db = 0.f;
    for (int c = 0; c < V / 16; ++c) db += sPV[c * 64 + tid];
    for (int b = 0; b < 4; ++b) db += sPM[b * 64 + tid];
    ((float*)a.sc.p[S_DBETA])[tile * 64 + tid] = db;
  }
  asm volatile("" ::"v"(warm));
}

// ---------------------------------------------------------------------------
// decay-structured VJP and finalisation
// ---------------------------------------------------------------------------
template <int K>
struct DecaySmem {
  static constexpr int QP = K + 8;                               // bf16 row stride of q, k
  static constexpr int GP = K + 4;                               // f32 row stride of G
  static constexpr int AP = 64 + 8;                              // bf16 row stride of dA, dM'
  static constexpr int HALF = K / 2;                             // key columns per pass
  static constexpr int OP = HALF + 8;                            // bf16 row stride of the operands
  static constexpr int NSEG = kVjpThreads / K;                   // cumsum segments per column
  static constexpr size_t off_q = 0;                             // bf16 [64][QP] q, later dq
  static constexpr size_t off_k = off_q + 64 * QP * 2;           // bf16 [64][QP] k, later dk
  static constexpr size_t off_g = off_k + 64 * QP * 2;           // f32 [64][GP] G, later dG
  static constexpr size_t off_da = off_g + 64 * GP * 4;          // bf16 [64][AP] dA
  static constexpr size_t off_dm = off_da + 64 * AP * 2;         // bf16 [64][AP] dM'
  static constexpr size_t off_op = off_dm + 64 * AP * 2;         // bf16 6 x [64][OP] operands
  static constexpr size_t off_pb = off_op + 6 * 64 * OP * 2;     // f32 [K/16][64] dbeta partials
  static constexpr size_t off_pq = off_pb + (K / 16) * 64 * 4;   // f32 [K/16][64] qh . dqh
  static constexpr size_t off_pk = off_pq + (K / 16) * 64 * 4;   // f32 [K/16][64] kh . dkh
  static constexpr size_t off_gl = off_pk + (K / 16) * 64 * 4;   // f32 [4][K] dG_last partials
  static constexpr size_t off_row = off_gl + 4 * K * 4;          // f32 [5][64] beta, rq, rk, fq, fk
  static constexpr size_t off_f = off_row + 5 * 64 * 4;          // int [4] unsafe-block flags
  static constexpr size_t bytes = off_f + 16;
  // after the item phase the operand region holds the cumsum segments and parameter partials
  static constexpr size_t off_seg = off_op;                      // f32 [NSEG][K]
  static constexpr size_t off_p0 = off_seg + NSEG * K * 4;       // f32 [NSEG][K]
  static constexpr size_t off_p1 = off_p0 + NSEG * K * 4;        // f32 [NSEG][K]
  static_assert(off_p1 + NSEG * K * 4 <= off_pb, "cumsum scratch must fit in the operand region");
  static_assert(QP % 8 == 0 && AP % 4 == 0 && OP % 4 == 0, "vector rows and transposing reads");
};

// Decay-structured VJP: gathers every dependence of the loss on qh, kh and G for one
// (chunk, head), applies the L2-norm, beta and gate chains and writes dq, dk, dbeta, dgate.
//   dqh = dQg e^G + Rq
//   dkh = dKd e^{GL-G} + beta e^G dKb + Rk + Cq + Ck
//   dG  = dQg Qg - dKd Kd + dKb Kb + qh Rq + kh Rk - kh (Cq + Ck),   dGL += sum_i dKd Kd
// with Rq = sum_j dA_ij kh_j e^{G_i-G_j}, Rk = sum_j dM'_ij kh_j e^{G_i-G_j} (row side) and
// Cq = sum_i dA_ij qh_i e^{G_i-G_j}, Ck = sum_i dM'_ij kh_i e^{G_i-G_j} (column side).
// The sums run over 16-token blocks b, each factor split around a reference row of b:
//   row side:    e^{G_i-G_j} = e^{G_i-G_f(b)} e^{G_f(b)-G_j},  f(b) = 16b, the first row
//   column side: e^{G_i-G_j} = e^{G_i-G_l(b)} e^{G_l(b)-G_j},  l(b) = 16b + 15, the last row
// so the decay-scaled operands KR = kh e^{G_f-G}, QC = qh e^{G-G_l}, KC = kh e^{G-G_l} are
// built once per tile (every factor within a block is at most e^span <= e^80) and each
// (row tile, key tile) item is a sum over blocks of 16-deep MFMAs scaled by one factor per
// row (at most 1).  The operands are split hi + lo bf16: their rounding is systematic across
// the row and column terms of dG, which nearly cancel.  A tile with a block whose decay spans
// more than 80 nats runs an exact per-pair f32 loop instead.  Items are owned in MFMA C
// layout, the layout in which the dense kernel stored dQg, dKd and dKb, so every
// per-element term stays in registers.  The key columns go in two passes of K/2 (the
// operands of one pass fit in LDS beside q, k and G).
template <int K, class Gate = NoGate>
__device__ __forceinline__ void decay_tile(const BwdArgs& a, int cidx, int hidx, int4 ch, const Gate& gate = Gate()) {
  using L = DecaySmem<K>;
  constexpr int QP = L::QP, GP = L::GP, AP = L::AP, HALF = L::HALF, OP = L::OP, NSEG = L::NSEG;
  constexpr int NKT = 4 * (K / 16);
  constexpr int IPW = (NKT + kVjpWaves - 1) / kVjpWaves;  // items per wave
  constexpr int NIH = 4 * (HALF / 16);                    // items per pass
  static_assert(NIH <= kVjpWaves && 64 * HALF / 4 <= kVjpThreads, "one item and one operand group per thread and pass");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* sQ = (bf16*)(smem + L::off_q);
  bf16* sK = (bf16*)(smem + L::off_k);
  float* sG = (float*)(smem + L::off_g);
  bf16* sDA = (bf16*)(smem + L::off_da);
  bf16* sDM = (bf16*)(smem + L::off_dm);
  bf16* sKRh = (bf16*)(smem + L::off_op);
  bf16* sKRl = sKRh + 64 * OP;
  bf16* sQCh = sKRl + 64 * OP;
  bf16* sQCl = sQCh + 64 * OP;
  bf16* sKCh = sQCl + 64 * OP;
  bf16* sKCl = sKCh + 64 * OP;
  float* sPB = (float*)(smem + L::off_pb);
  float* sPQ = (float*)(smem + L::off_pq);
  float* sPK = (float*)(smem + L::off_pk);
  float* sGL = (float*)(smem + L::off_gl);
  float* sBeta = (float*)(smem + L::off_row);
  float* sRq = sBeta + 64;
  float* sRk = sBeta + 128;
  float* sFq = sBeta + 192;
  float* sFk = sBeta + 256;
  int* sF = (int*)(smem + L::off_f);

  // ch: the chunk's table entry {row0, len, ...}
  const int len = ch.y;
  if (len <= 0) return;
  const int H = a.H, h = hidx;
  const size_t tile = (size_t)cidx * H + h;
  const int row0 = ch.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lr = lane % 16, kg = lane / 16;

  const float* Gg = (const float*)a.ws.p[R_G] + tile * 64 * K;
  const bf16* DA = (const bf16*)a.sc.p[S_DA] + tile * 64 * 64;
  const bf16* DMP = (const bf16*)a.sc.p[S_DMP] + tile * 64 * 64;
  // dQg/dKd/dKb of this tile (from the dense role)
  const float* DQG = (const float*)a.sc.p[S_DQG] + tile * 64 * K;
  const float* DKD = (const float*)a.sc.p[S_DKD] + tile * 64 * K;
  const float* DKB = (const float*)a.sc.p[S_DKB] + tile * 64 * K;
  // each wave's dqh, dkh and dG of its item in pass 0 and pass 1, held in registers across
  // the barrier that completes the per-row dot products
  f32x4 keep_q[2], keep_k[2], keep_g[2];

  // ---- P0: stage q, k (bf16), G, dA, dM' (bf16), beta and the per-row norm factors ----
  if (tid < 4) sF[tid] = 0;
  {
    // every load first (clamped rows, zeroed after), so they are in flight together
    constexpr int LPR = K / 8;
    static_assert(64 * LPR <= kVjpThreads, "one row chunk per thread");
    const int t = tid / LPR, c0 = (tid % LPR) * 8;
    const bool act = tid < 64 * LPR;
    const int tc = act ? t : 0;
    const size_t base = ((size_t)(row0 + (tc < len ? tc : len - 1)) * H + h) * K + c0;
    bf16x8 qr = *(const bf16x8*)(a.q + base), kr = *(const bf16x8*)(a.k + base);
    const float rq = ((const float*)a.ws.p[R_RQ])[tile * 64 + tc];
    const float rk = ((const float*)a.ws.p[R_RK])[tile * 64 + tc];
    const float bt = ((const float*)a.ws.p[R_BETA])[tile * 64 + tc];
    float gv[8];
    load8f(Gg + tc * K + c0, gv);
    gate();  // everything below reads the dense role's results
    // dA, dM': 64 x 64 f32 each, 4 consecutive per thread
    const int ai = tid * 4;
    bf16x4 ya = {}, ym = {};
    if (ai < 64 * 64) {
      ya = *(const bf16x4*)(DA + ai);
      ym = *(const bf16x4*)(DMP + ai);
    }
    if (act) {
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (!(tc < len)) {
          qr[e] = to_bf16(0.f);
          kr[e] = to_bf16(0.f);
        }
        const float qv = to_f32(qr[e]), kv = to_f32(kr[e]);
        sq += qv * qv;
        sk += kv * kv;
      }
      *(bf16x8*)(sQ + t * QP + c0) = qr;
      *(bf16x8*)(sK + t * QP + c0) = kr;
      *(float4*)(sG + t * GP + c0) = make_float4(gv[0], gv[1], gv[2], gv[3]);
      *(float4*)(sG + t * GP + c0 + 4) = make_float4(gv[4], gv[5], gv[6], gv[7]);
      sq = group_sum<LPR>(sq);
      sk = group_sum<LPR>(sk);
      if (c0 == 0) {
        // dx = r (g - xhat (xhat . g)) with xhat = x/||x||; expressed through qh = r x:
        // dx = r g - qh (qh . g) / (||x||^2 r); clamped norms pass r g through
        sRq[t] = rq;
        sRk[t] = rk;
        sFq[t] = sqrtf(sq) > 1e-12f ? 1.f / (sq * rq) : 0.f;
        sFk[t] = sqrtf(sk) > 1e-12f ? 1.f / (sk * rk) : 0.f;
        sBeta[t] = bt;
      }
    }
    if (ai < 64 * 64) {
      *(bf16x4*)(sDA + (ai / 64) * AP + ai % 64) = ya;
      *(bf16x4*)(sDM + (ai / 64) * AP + ai % 64) = ym;
    }
  }
  __syncthreads();
  if (tid < K) {
    const int c = tid;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (sG[(16 * b) * GP + c] - sG[(16 * b + 15) * GP + c] > 80.f) atomicOr(&sF[b], 1);
  }
  __syncthreads();
  const bool unsafe = (sF[0] | sF[1] | sF[2] | sF[3]) != 0;

  // the dense part's dbeta partial of row tid (needed after P1; requested now)
  const float dbeta_dense = tid < 64 ? ((const float*)a.sc.p[S_DBETA])[tile * 64 + tid] : 0.f;
  // ---- P1: per pass (K/2 key columns) build the decay-scaled operands, then one item per
  // wave: row side + column side + all per-element terms ----
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    const int cb = pass * HALF;  // first key column of the pass
    // lane coordinates made opaque per pass: keeps the compiler from hoisting dozens of
    // lane-dependent LDS addresses out of the pass loop (they would be spilled)
    int ptid = tid, plane = lane, lr = lane % 16, kg = lane / 16;
    asm volatile("" : "+v"(ptid), "+v"(plane), "+v"(lr), "+v"(kg));
    // this wave's item of the pass; its raw dQg/dKd/dKb are not needed before the
    // per-element terms, so their loads are issued first and overlap the operand build
    const int rt = wave % 4, ctl = wave / 4, ct = cb / 16 + ctl;
    const int p = rt + 4 * ct;
    const int c = 16 * ct + lr;
    const int pi = wave < NIH ? p : 0;
    const f32x4 rdQ = *(const f32x4*)(DQG + ((size_t)pi * 64 + plane) * 4);
    const f32x4 rdK = *(const f32x4*)(DKD + ((size_t)pi * 64 + plane) * 4);
    const f32x4 rdB = *(const f32x4*)(DKB + ((size_t)pi * 64 + plane) * 4);
    if (!unsafe) {
      // operand group: row t, 4 consecutive columns
      const int t = ptid / (HALF / 4), c4 = (ptid % (HALF / 4)) * 4;
      if (t < 64) {
        const int cc = cb + c4, bf = t & ~15, bl = bf + 15;
        const float4 g = *(const float4*)(sG + t * GP + cc);
        const float4 gf = *(const float4*)(sG + bf * GP + cc);
        const float4 gl = *(const float4*)(sG + bl * GP + cc);
        const bf16x4 qq = *(const bf16x4*)(sQ + t * QP + cc), kk = *(const bf16x4*)(sK + t * QP + cc);
        const float rq = sRq[t], rk = sRk[t];
        const float gt[4] = {g.x, g.y, g.z, g.w}, gft[4] = {gf.x, gf.y, gf.z, gf.w}, glt[4] = {gl.x, gl.y, gl.z, gl.w};
        bf16x4 krh, krl, qch, qcl, kch, kcl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float qh = to_f32(qq[e]) * rq, kh = to_f32(kk[e]) * rk;
          const float e1 = __expf(gft[e] - gt[e]), e2 = __expf(gt[e] - glt[e]);
          const float kr = kh * e1, qc = qh * e2, kc = kh * e2;
          krh[e] = to_bf16(kr);
          krl[e] = to_bf16(kr - to_f32(krh[e]));
          qch[e] = to_bf16(qc);
          qcl[e] = to_bf16(qc - to_f32(qch[e]));
          kch[e] = to_bf16(kc);
          kcl[e] = to_bf16(kc - to_f32(kch[e]));
        }
        const int o = t * OP + c4;
        *(bf16x4*)(sKRh + o) = krh;
        *(bf16x4*)(sKRl + o) = krl;
        *(bf16x4*)(sQCh + o) = qch;
        *(bf16x4*)(sQCl + o) = qcl;
        *(bf16x4*)(sKCh + o) = kch;
        *(bf16x4*)(sKCl + o) = kcl;
      }
    }
    __syncthreads();
    if (wave < NIH) {
      f32x4 rq = zero4(), rk = zero4(), cq = zero4(), ck = zero4();
      if (!unsafe) {
        const float gf_rt = sG[(16 * rt) * GP + c], gl_rt = sG[(16 * rt + 15) * GP + c];
        // row side: blocks b <= rt, A = dA / dM' rows of tile rt, B = KR rows of block b
        for (int b = 0; b <= rt; ++b) {
          const bf16x4 fa = *(const bf16x4*)(sDA + (16 * rt + lr) * AP + 16 * b + 4 * kg);
          const bf16x4 fm = *(const bf16x4*)(sDM + (16 * rt + lr) * AP + 16 * b + 4 * kg);
          const bf16x4 bh = lds_col_frag4(sKRh, OP, 16 * b, 16 * ctl, plane);
          const bf16x4 bl = lds_col_frag4(sKRl, OP, 16 * b, 16 * ctl, plane);
          const f32x4 pq = mfma16k16(fa, bl, mfma16k16(fa, bh, zero4()));
          const f32x4 pk = mfma16k16(fm, bl, mfma16k16(fm, bh, zero4()));
          // e^{G_i - G_f(b)} = e^{G_i - G_f(rt)} e^{G_f(rt) - G_f(b)}: the block factor is
          // one per lane (<= 1), the row factor is applied once after the block sum
          const float f = __expf(gf_rt - sG[(16 * b) * GP + c]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            rq[r] = fmaf(pq[r], f, rq[r]);
            rk[r] = fmaf(pk[r], f, rk[r]);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float f = __expf(sG[(16 * rt + 4 * kg + r) * GP + c] - gf_rt);
          rq[r] *= f;
          rk[r] *= f;
        }
        // column side: blocks b >= rt, A = dA^T / dM'^T (columns of tile rt), B = QC / KC
        for (int b = rt; b < 4; ++b) {
          const bf16x4 fa = lds_col_frag4(sDA, AP, 16 * b, 16 * rt, plane);
          const bf16x4 fm = lds_col_frag4(sDM, AP, 16 * b, 16 * rt, plane);
          const bf16x4 qh = lds_col_frag4(sQCh, OP, 16 * b, 16 * ctl, plane);
          const bf16x4 ql = lds_col_frag4(sQCl, OP, 16 * b, 16 * ctl, plane);
          const bf16x4 kh = lds_col_frag4(sKCh, OP, 16 * b, 16 * ctl, plane);
          const bf16x4 kl = lds_col_frag4(sKCl, OP, 16 * b, 16 * ctl, plane);
          const f32x4 pq = mfma16k16(fa, ql, mfma16k16(fa, qh, zero4()));
          const f32x4 pk = mfma16k16(fm, kl, mfma16k16(fm, kh, zero4()));
          // e^{G_l(b) - G_j} = e^{G_l(b) - G_l(rt)} e^{G_l(rt) - G_j}, both <= 1
          const float f = __expf(sG[(16 * b + 15) * GP + c] - gl_rt);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            cq[r] = fmaf(pq[r], f, cq[r]);
            ck[r] = fmaf(pk[r], f, ck[r]);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float f = __expf(gl_rt - sG[(16 * rt + 4 * kg + r) * GP + c]);
          cq[r] *= f;
          ck[r] *= f;
        }
      } else {
        // a block whose decay spans more than 80 nats: exact per-pair f32 factors (dA, dM'
        // as the dense part stored them, bf16)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int ii = 16 * rt + 4 * kg + rr;
          const float gi = sG[ii * GP + c];
          float sq = 0.f, sk = 0.f;
          for (int j = 0; j <= ii; ++j) {
            const float kj = to_f32(sK[j * QP + c]) * sRk[j] * expf(gi - sG[j * GP + c]);
            sq = fmaf(to_f32(DA[ii * 64 + j]), kj, sq);
            sk = fmaf(to_f32(DMP[ii * 64 + j]), kj, sk);
          }
          float tq = 0.f, tk = 0.f;
          for (int i = ii; i < 64; ++i) {
            const float e = expf(sG[i * GP + c] - gi);
            tq = fmaf(to_f32(DA[i * 64 + ii]), to_f32(sQ[i * QP + c]) * sRq[i] * e, tq);
            tk = fmaf(to_f32(DMP[i * 64 + ii]), to_f32(sK[i * QP + c]) * sRk[i] * e, tk);
          }
          rq[rr] = sq;
          rk[rr] = sk;
          cq[rr] = tq;
          ck[rr] = tk;
        }
      }
      const float GL = sG[63 * GP + c];
      float glp = 0.f;
      f32x4 dqs, dks, dgs;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ii = 16 * rt + 4 * kg + rr;
        const float qh = to_f32(sQ[ii * QP + c]) * sRq[ii], kh = to_f32(sK[ii * QP + c]) * sRk[ii];
        const float G = sG[ii * GP + c];
        const float bt = sBeta[ii];
        const float eG = __expf(G), eKd = __expf(GL - G);
        const float dQg = rdQ[rr], dKd = rdK[rr], dKb = rdB[rr];
        const float cc = cq[rr] + ck[rr];
        const float dqh = fmaf(dQg, eG, rq[rr]);
        const float dkh = dKd * eKd + bt * eG * dKb + rk[rr] + cc;
        const float kdd = dKd * kh * eKd;
        const float kbb = dKb * kh * eG;  // dbeta partial (the beta factor of Kb removed)
        dgs[rr] = dQg * qh * eG - kdd + bt * kbb + qh * rq[rr] + kh * rk[rr] - kh * cc;
        dqs[rr] = dqh;
        dks[rr] = dkh;
        glp += kdd;
        const float pb = group_sum<16>(kbb);
        const float pq = group_sum<16>(qh * dqh);
        const float pk = group_sum<16>(kh * dkh);
        if (lr == 0) {
          sPB[ct * 64 + ii] = pb;
          sPQ[ct * 64 + ii] = pq;
          sPK[ct * 64 + ii] = pk;
        }
      }
      if (pass == 0) {
        keep_q[0] = dqs; keep_k[0] = dks; keep_g[0] = dgs;
      } else {
        keep_q[1] = dqs; keep_k[1] = dks; keep_g[1] = dgs;
      }
      glp = lane_stride_sum<16>(glp);
      if (kg == 0) sGL[rt * K + c] = glp;
    }
    __syncthreads();  // the next pass rebuilds the operands
  }

  // per-row dot products (fixed order) and dbeta
  if (tid < 64) {
    const int t = tid;
    float dotq = 0.f, dotk = 0.f, db = dbeta_dense;
#pragma unroll
    for (int q = 0; q < K / 16; ++q) {
      dotq += sPQ[q * 64 + t];
      dotk += sPK[q * 64 + t];
      db += sPB[q * 64 + t];
    }
    sPQ[t] = dotq * sFq[t];
    sPK[t] = dotk * sFk[t];
    if (t < len) {
      const float bt = sBeta[t];
      bf16* drow = a.dbeta + (size_t)(row0 + t) * a.dbeta_ld;
      drow[h] = to_bf16(db * bt * (1.f - bt));
      if (h == 0)
        for (int e = 0; e < a.dbeta_pad; ++e) drow[H + e] = to_bf16(0.f);
    }
  }
  __syncthreads();

  // ---- P2: L2-norm chains; dq, dk (bf16) and dG into LDS (q, k, G are consumed) ----
  // (the items of P1: wave w < NIH owns item (w % 4, w / 4 + pass * HALF / 16) of each pass)
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    if (wave >= NIH) break;
    const int rt = wave % 4, ct = n * (HALF / 16) + wave / 4;
    const int c = 16 * ct + lr;
    const f32x4 dqs = keep_q[n], dks = keep_k[n], dgs = keep_g[n];
    float dqv[4], dkv[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ii = 16 * rt + 4 * kg + rr;
      dqv[rr] = sRq[ii] * dqs[rr] - to_f32(sQ[ii * QP + c]) * sRq[ii] * sPQ[ii];
      dkv[rr] = sRk[ii] * dks[rr] - to_f32(sK[ii * QP + c]) * sRk[ii] * sPK[ii];
    }
    // every read of this element's q / k happened in this lane; write back in place
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ii = 16 * rt + 4 * kg + rr;
      sQ[ii * QP + c] = to_bf16(dqv[rr]);
      sK[ii * QP + c] = to_bf16(dkv[rr]);
      sG[ii * GP + c] = ii < len ? dgs[rr] : 0.f;
    }
  }
  __syncthreads();

  // ---- P3: coalesced dq, dk writes ----
  {
    constexpr int LPR = K / 8;
    // the thread index made opaque: P0's row / column of the same thread is otherwise kept
    // alive through P1 and P2 (a spilled register at K = 64)
    int ptid = tid;
    asm volatile("" : "+v"(ptid));
    for (int idx = ptid; idx < 64 * LPR; idx += kVjpThreads) {
      const int t = idx / LPR, c0 = (idx % LPR) * 8;
      if (t >= len) continue;
      const size_t base = (size_t)(row0 + t) * a.gld_qk + (size_t)h * K + c0;
      *(bf16x8*)(a.dq + base) = *(const bf16x8*)(sQ + t * QP + c0);
      *(bf16x8*)(a.dk + base) = *(const bf16x8*)(sK + t * QP + c0);
    }
  }

  // ---- P4: dg = reverse cumsum of dG (+ dG_last) in NSEG segments per key, gate chain ----
  constexpr int RPS = 64 / NSEG;
  float* sSeg = (float*)(smem + L::off_seg);
  float* sP0 = (float*)(smem + L::off_p0);
  float* sP1 = (float*)(smem + L::off_p1);
  const int c = tid % K, seg = tid / K;
  const bool k3 = a.gate_mode == KDA_GATE_K3;
  // K3: this thread's raw gate values, requested together before the segment sums (rows
  // past the chunk end read the last row and are not used), with the column's dG_last part
  // and gate parameters (loaded after the barrier they were a round trip of their own)
  const float dgl = ((const float*)a.sc.p[S_DGL])[tile * K + c];
  const float alog = k3 ? a.A_log[h] : 0.f;
  const float bias = k3 ? a.dt_bias[h * K + c] : 0.f;
  float graw[RPS];
  if (k3) {
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      const int t = min(seg * RPS + r, len - 1);
      graw[r] = to_f32(((const bf16*)a.gate)[((size_t)(row0 + t) * H + h) * K + c]);
    }
  }
  {
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < RPS; ++r) sum += sG[(seg * RPS + r) * GP + c];
    sSeg[seg * K + c] = sum;
  }
  __syncthreads();
  {
    float acc = dgl;
#pragma unroll
    for (int q = 0; q < 4; ++q) acc += sGL[q * K + c];
    for (int s = NSEG - 1; s > seg; --s) acc += sSeg[s * K + c];
    float p0 = 0.f, p1 = 0.f;
    const float ea = k3 ? expf(alog) : 0.f;
#pragma unroll
    for (int r = RPS - 1; r >= 0; --r) {
      const int t = seg * RPS + r;
      acc += sG[t * GP + c];
      if (t < len) {
        const size_t off = ((size_t)(row0 + t) * H + h) * K + c;
        if (k3) {
          const float pre = graw[r] + bias;
          const float s = sigmoid_fast(ea * pre);  // the forward gate uses the same form
          const float dz = acc * a.lb * s * (1.f - s) * ea;
          ((bf16*)a.dgate)[off] = to_bf16(dz);
          p0 += dz;
          p1 = fmaf(dz, pre, p1);
        } else {
          ((float*)a.dgate)[off] = acc;
        }
      }
    }
    if (k3) {
      sP0[seg * K + c] = p0;
      sP1[seg * K + c] = p1;
    }
  }
  if (a.gate_mode == KDA_GATE_K3) {
    __syncthreads();
    if (tid < K) {
      float p0 = 0.f, p1 = 0.f;
      for (int s = 0; s < NSEG; ++s) {
        p0 += sP0[s * K + tid];
        p1 += sP1[s * K + tid];
      }
      float* PP = (float*)a.sc.p[S_PP] + tile * 2 * K;
      PP[tid] = p0;
      PP[K + tid] = p1;
    }
  }
}

// ---------------------------------------------------------------------------
// dense and decay tiles in one launch
// ---------------------------------------------------------------------------
// Workgroup i < dense_count runs the dense VJP of tile dense_begin + i; the others run the
// decay VJP of tile decay_begin + (i - dense_count).  The backward cuts the sequence "all
// dense tiles, then all decay tiles" into launches of one workgroup per CU, so a launch that
// finishes the dense tiles also starts the decay tiles whose dense tiles an earlier launch
// completed: no round runs half empty, and no workgroup waits on another.
static_assert(kDenseThreads == kVjpThreads, "dense and decay tiles share the block size");
template <int K, int V>
__global__ __launch_bounds__(kVjpThreads) void chunk_bwd_vjp_kernel(BwdArgs a, int dense_begin, int dense_count,
                                                                    int decay_begin) {
  const int item = blockIdx.x;
  if (item < dense_count) {
    const int t = dense_begin + item;
    dense_tile<K, V>(a, t / a.H, t % a.H, chunk_entry(a, t / a.H));
  } else {
    const int t = decay_begin + item - dense_count;
    decay_tile<K>(a, t / a.H, t % a.H, chunk_entry(a, t / a.H));
  }
}

// ---------------------------------------------------------------------------
// fused backward: scan, dense and decay tiles in one launch
// ---------------------------------------------------------------------------
// The scan members (the first scan_blocks workgroups) run the reverse scan and publish each
// step; the next prep_blocks workgroups form the scan's per-chunk inputs.  Every other
// workgroup runs the dense and then the decay VJP of one tile, workgroup index order = the
// order the scan finalises the tiles (last chunks of every sequence first), each reading
// its position's record {chunk, row0, len, sequence, steps to wait for} written by the
// scheduling launch: one load before the tile's own loads (a ticket counter and the chunk
// table lookups were three dependent round trips, ≈3 µs under the launch's load).  The
// dense part waits until every strip of the tile's record has passed its chunk; the decay
// part reads what the same workgroup's dense part stored.
//
// Dispatch-order assumption: every wait is on scan members, which wait on nothing.  The
// launch drains only if the scan members are resident while tiles wait.  They are the lowest
// workgroup indices of the grid, so the dispatcher places them first, before any tile
// workgroup can occupy a CU slot; this is how the hardware dispatches a 1-D grid, but it is not
// a documented guarantee.  Each wait is therefore bounded (the launch argument spin_limit,
// in ticks of the 100 MHz wall clock; 2 s by default).  A tile whose wait gives up sets the
// abort word (every later wait then gives up at once) and the failure is made visible:
// the tile writes NaN over all of its gradient rows (dq, dk, dv, dgate, dbeta and its
// K3-parameter partials, so dA_log and ddt_bias are NaN too), and the abort word stays set
// in the scratch until the next call's scheduling kernel clears it, where
// kda_chunk_backward_status() reads it.
constexpr long long kSpinLimitDefault = 200000000LL;  // 2 s

struct SyncView {
  int* abort;
  int* base;
};

__device__ __forceinline__ SyncView sync_view(const BwdArgs& a) {
  int* base = (int*)a.sc.p[S_SYNC];
  return {base + 1, base};
}

// Thread 0 waits for *p >= need, sleeping about 0.4 us per missing step between polls (the
// scan finishes a step about every microsecond; dense polling by a couple of hundred
// waiting workgroups slows the scan's own memory traffic), then a workgroup barrier.  The
// data behind the count is read with coherent loads, so no cache invalidation is needed.
// A wait that gives up (or finds the abort word set) records it in *failed (LDS).
struct ScanGate {
  static constexpr bool kCoherent = true;
  const int* p;  // the record's strip counts
  int nstrips;
  int need;
  int* abort;
  long long spin_limit;
  int* failed;
  __device__ void operator()() const {
    if (threadIdx.x == 0) {
      const long long t0 = wall_clock64();
      for (;;) {
        // up to 8 strips (V <= 128): the loads are issued together, then reduced
        int w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          w[i] = i < nstrips ? __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : INT_MAX;
        int v = w[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) v = min(v, w[i]);
        if (v >= need) break;
        if (__hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
          *failed = 1;
          break;
        }
        if (wall_clock64() - t0 > spin_limit) {
          __hip_atomic_store(abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          *failed = 1;
          break;
        }
        for (int k = min(need - v, 8); k > 0; --k) __builtin_amdgcn_s_sleep(15);  // ~0.4 us each
      }
    }
    ring_barrier();
  }
};

// Overwrites every gradient of tile (cidx, h) with NaN: its rows of dq, dk, dv, dgate and
// dbeta and its K3-parameter partials (the parameter reduction then yields NaN).
template <int K, int V>
__device__ void poison_tile(const BwdArgs& a, int cidx, int h) {
  const int4 ch = chunk_entry(a, cidx);
  const int row0 = ch.x, len = ch.y, H = a.H;
  const float nan = __builtin_nanf("");
  const bf16 nanb = to_bf16(nan);
  const size_t tile = (size_t)cidx * H + h;
  for (int i = threadIdx.x; i < len * K; i += blockDim.x) {
    const int t = i / K, c = i % K;
    a.dq[(size_t)(row0 + t) * a.gld_qk + (size_t)h * K + c] = nanb;
    a.dk[(size_t)(row0 + t) * a.gld_qk + (size_t)h * K + c] = nanb;
    const size_t g = ((size_t)(row0 + t) * H + h) * K + c;
    if (a.gate_mode == KDA_GATE_K3)
      ((bf16*)a.dgate)[g] = nanb;
    else
      ((float*)a.dgate)[g] = nan;
  }
  for (int i = threadIdx.x; i < len * V; i += blockDim.x)
    a.dv[(size_t)(row0 + i / V) * a.gld_v + (size_t)h * V + i % V] = nanb;
  for (int t = threadIdx.x; t < len; t += blockDim.x) a.dbeta[(size_t)(row0 + t) * a.dbeta_ld + h] = nanb;
  if (a.gate_mode == KDA_GATE_K3)
    for (int i = threadIdx.x; i < 2 * K; i += blockDim.x) ((float*)a.sc.p[S_PP])[tile * 2 * K + i] = nan;
}

// Clears the sync words and writes the chunk order: chunk c of sequence s with n chunks
// has reverse rank r = n - 1 - (index in s); chunks go by r, then by sequence.  Position
// of c = sum over sequences s' of min(n_s', r) + #{s' < s : n_s' > r}; chunks past the
// last sequence keep their index.  Each position holds the chunk's table entry and the
// step count its tiles wait for, so a tile reads one record before its loads.
__device__ __forceinline__ void bwd_sched_body(const BwdArgs& a, int max_chunks, int sync_words) {
  int* sync = (int*)a.sc.p[S_SYNC];
  int4* order = (int4*)a.sc.p[S_ORDER];
  const int4* chunks = (const int4*)a.ws.p[R_CHUNKS];
  const int2* seqs = (const int2*)a.ws.p[R_SEQS];
  for (int i = threadIdx.x; i < sync_words; i += blockDim.x) sync[i] = 0;
  for (int c = threadIdx.x; c < max_chunks; c += blockDim.x) {
    const int4 ch = chunks[c];
    if (ch.z < 0 || ch.y <= 0) {
      order[2 * c] = make_int4(c, ch.x, ch.y, -1);
      order[2 * c + 1] = make_int4(0, 0, 0, 0);
      continue;
    }
    const int r = seqs[ch.z].y - 1 - ch.w;
    int pos = 0;
    for (int s = 0; s < a.num_seqs; ++s) {
      const int n = seqs[s].y;
      pos += min(n, r) + (s < ch.z && n > r ? 1 : 0);
    }
    order[2 * pos] = make_int4(c, ch.x, ch.y, ch.z);
    order[2 * pos + 1] = make_int4(r + 1, 0, 0, 0);
  }
}

__global__ __launch_bounds__(1024) void chunk_bwd_sched_kernel(BwdArgs a, int max_chunks, int sync_words) {
  bwd_sched_body(a, max_chunks, sync_words);
}

// Position p of the fused backward's order -> chunk, its table entry {row0, len, seq, -} and
// the steps its record must publish.  Sequences of one length: arithmetic (position
// p = rank * sequences + sequence); otherwise the scheduling launch's record.
struct TilePos {
  int cidx, need;
  int4 ch;
};
__device__ __forceinline__ TilePos tile_position(const BwdArgs& a, int p) {
  if (a.fixed_T > 0) {
    const int n = (a.fixed_T + kChunk - 1) / kChunk;
    const int r = p / a.num_seqs, seq = p % a.num_seqs, j = n - 1 - r;
    return {seq * n + j, r + 1, make_int4(seq * a.fixed_T + j * kChunk, min(kChunk, a.fixed_T - j * kChunk), seq, 0)};
  }
  const int4* rec4 = (const int4*)a.sc.p[S_ORDER] + 2 * p;
  const int4 r0 = rec4[0], r1 = rec4[1];
  return {r0.x, r1.x, make_int4(r0.y, r0.z, r0.w, 0)};
}

template <int K, int V>
__global__ __launch_bounds__(kVjpThreads) void chunk_bwd_fused_kernel(BwdArgs a, int scan_blocks, int prep_blocks,
                                                                      long long spin_limit) {
  const SyncView sv = sync_view(a);
  int* prep_flags = sv.base + kSyncRec + 32 * a.num_seqs * a.H;  // one word per tile
  if ((int)blockIdx.x < scan_blocks) {
    bwd_scan_body<K, V, true, kFusedSPW>(a, sv.base, prep_blocks > 0 ? prep_flags : nullptr, spin_limit);
    return;
  }
  if ((int)blockIdx.x < scan_blocks + prep_blocks) {
    // a prep workgroup: tile number blockIdx - scan_blocks in the scan's order, so the scan's
    // first steps find their operands first
    if (threadIdx.x >= kPrepThreads) return;
    const int i = blockIdx.x - scan_blocks;
    const int cidx = tile_position(a, i / a.H).cidx, h = i % a.H;
    bwd_prep_body<K, V, true>(a, cidx, h);
    wait_vmcnt<0>();  // every write-through store of the tile is complete
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(prep_flags + (size_t)cidx * a.H + h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  __shared__ int s_failed;
  if (threadIdx.x == 0) s_failed = 0;  // ordered before the gate by the dense part's barriers
  // tile t in the scan's order: workgroups are dispatched in index order, so the tiles start
  // in the order the scan finalises them (a tile waits only on scan members)
  const int t = blockIdx.x - scan_blocks - prep_blocks, H = a.H, h = t % H;
  const TilePos tp = tile_position(a, t / H);
  const int cidx = tp.cidx;
  const int4 ch = tp.ch;  // {row0, len, seq, -}
  int need = 0, rec = 0;
  if (ch.y > 0) {
    rec = ch.z * H + h;
    need = tp.need;
  }
  ScanGate gate{sv.base + kSyncRec + 32 * rec, V / 16, need, sv.abort, spin_limit, &s_failed};
  dense_tile<K, V>(a, cidx, h, ch, gate);
  __syncthreads();  // the dense part's stores are complete and visible to this workgroup
  decay_tile<K>(a, cidx, h, ch);
  __syncthreads();
  if (s_failed && ch.y > 0) poison_tile<K, V>(a, cidx, h);  // computed from unwritten histories
}

// ---------------------------------------------------------------------------
// gate parameter reduction (fixed order)
// ---------------------------------------------------------------------------
constexpr int kParamThreads = 1024;

// Thread (part, c) sums the chunks part, part + P, ... (P = kParamThreads / K) in order;
// the P partials and then the K channels are combined in a fixed order.
template <int K>
__global__ __launch_bounds__(kParamThreads) void chunk_bwd_params_kernel(BwdArgs a, int max_chunks) {
  constexpr int P = kParamThreads / K;
  __shared__ float s0[P][K], s1[P][K];
  const int h = blockIdx.x, c = threadIdx.x % K, part = threadIdx.x / K;
  const int4* chunks = (const int4*)a.ws.p[R_CHUNKS];
  const float* PP = (const float*)a.sc.p[S_PP];
  float p0 = 0.f, p1 = 0.f;
  // batches of 16 chunks (one batch per part at 128 chunks): every load of a batch is issued
  // before any is used (empty chunks' partials were never written and are selected away,
  // not multiplied)
  constexpr int U = 16;
  for (int chn0 = part; chn0 < max_chunks; chn0 += U * P) {
    float x0[U], x1[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int chn = min(chn0 + u * P, max_chunks - 1);
      const size_t tile = (size_t)chn * a.H + h;
      live[u] = chn0 + u * P < max_chunks && chunks[chn].y > 0;
      x0[u] = PP[tile * 2 * K + c];
      x1[u] = PP[tile * 2 * K + K + c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      p0 += live[u] ? x0[u] : 0.f;
      p1 += live[u] ? x1[u] : 0.f;
    }
  }
  s0[part][c] = p0;
  s1[part][c] = p1;
  __syncthreads();
  __shared__ float s_wave[K / 64];
  if (part == 0) {
    float t0 = 0.f, t1 = 0.f;
    for (int q = 0; q < P; ++q) {
      t0 += s0[q][c];
      t1 += s1[q][c];
    }
    a.ddt_bias[h * K + c] = t0;
    t1 = wave_sum(t1);  // fixed butterfly order within the wave
    if (c % 64 == 0) s_wave[c / 64] = t1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int q = 0; q < K / 64; ++q) t += s_wave[q];
    a.dA_log[h] = t;
  }
}

// Bound of each wait in the fused backward (ticks of the 100 MHz wall clock), set by
// kda_debug_set_wait_limit; negative: the default.
static std::atomic<long long> g_wait_limit{-1};
static long long wait_limit_ticks() {
  const long long v = g_wait_limit.load(std::memory_order_relaxed);
  return v < 0 ? kSpinLimitDefault : v;
}

// KDA_BWD_FUSED=0 selects the three-launch backward (scan, then rounds of dense / decay
// tiles).
static bool fused_backward_enabled() {
  static const bool on = [] {
    const char* e = getenv("KDA_BWD_FUSED");
    return !(e && e[0] == '0');
  }();
  return on;
}


template <int K, int V>
static int launch_backward(const kda_chunk_problem* p, const ChunkGeom& g, BwdArgs& a,
                           hipStream_t stream, int stages) {
  const int all = (1 << (KDA_STAGE_BWD_SCAN - 10)) | (1 << (KDA_STAGE_BWD_DENSE - 10)) |
                  (1 << (KDA_STAGE_BWD_DECAY - 10));
  // the reverse scan's per-chunk transition -G and inhomogeneous term E (chunk-parallel)
  // sched_words > 0: the prep launch also clears the fused launch's sync words and writes
  // its tile order (one extra column of workgroups)
  auto launch_prep = [&](int sched_words) -> int {
    auto prep = chunk_bwd_prep_kernel<K, V>;
    constexpr int smem_p = PrepLds<K, V>::bytes;
    if (ensure_lds_limit((const void*)prep, smem_p) != hipSuccess)
      return set_error(KDA_ERR_LAUNCH, "chunk_backward: prep LDS attribute failed");
    hipLaunchKernelGGL(prep, dim3(g.max_chunks + (sched_words > 0 ? 1 : 0), p->heads), dim3(kPrepThreads), smem_p,
                       stream, a, sched_words);
    KDA_LAUNCH_CHECK("chunk_backward prep");
    return KDA_OK;
  };
  if ((stages & all) == all && p->num_seqs > 0 && g.max_chunks > 0 && fused_backward_enabled()) {
    // one launch: scan members + prep workgroups + dense / decay tiles (see chunk_bwd_fused_kernel)
    constexpr size_t smem =
        cmax_sz(kFusedSPW * BwdScanLds<K, V>::bytes + 2048, cmax_sz(DenseSmem<K, V>::bytes, DecaySmem<K>::bytes));
    static_assert(smem + 16 <= 160 * 1024, "fused backward LDS");
    static_assert(PrepLds<K, V>::bytes <= smem, "fused backward LDS (prep workgroups)");
    auto fused = chunk_bwd_fused_kernel<K, V>;
    if (ensure_lds_limit((const void*)fused, (int)smem) != hipSuccess)
      return set_error(KDA_ERR_LAUNCH, "chunk_backward: fused LDS attribute failed");
    const int nrec = p->num_seqs * p->heads;
    const int scan_blocks = kXcds * (V / 16 / kFusedSPW) * ((nrec + kXcds - 1) / kXcds);
    const int N = g.max_chunks * p->heads;
#if KDA_FUSED_PREP
    // the prep runs inside the fused launch (workgroups between the scan members and the
    // VJP tiles); a one-workgroup launch clears the sync words and writes the tile order
    hipLaunchKernelGGL(chunk_bwd_sched_kernel, dim3(1), dim3(1024), 0, stream, a, g.max_chunks, sync_words(nrec, N));
    KDA_LAUNCH_CHECK("chunk_backward sched");
    hipLaunchKernelGGL(fused, dim3(scan_blocks + 2 * N), dim3(kVjpThreads), smem, stream, a, scan_blocks, N,
                       wait_limit_ticks());
#else
    int rc = launch_prep(sync_words(nrec, N));
    if (rc != KDA_OK) return rc;
    hipLaunchKernelGGL(fused, dim3(scan_blocks + N), dim3(kVjpThreads), smem, stream, a, scan_blocks, 0,
                       wait_limit_ticks());
#endif
    KDA_LAUNCH_CHECK("chunk_backward fused");
    stages &= ~all;
  } else if ((stages & all) == all && g.max_chunks > 0) {
    // the staged backward never waits; clearing the sync words keeps
    // kda_chunk_backward_status meaningful after it
    const int nrec = p->num_seqs * p->heads;
    hipLaunchKernelGGL(chunk_bwd_sched_kernel, dim3(1), dim3(1024), 0, stream, a, g.max_chunks,
                       sync_words(nrec, g.max_chunks * p->heads));
    KDA_LAUNCH_CHECK("chunk_backward sched");
  }
  if (p->num_seqs > 0 && (stages & (1 << (KDA_STAGE_BWD_SCAN - 10)))) {
    if (g.max_chunks > 0) {
      int rc = launch_prep(0);
      if (rc != KDA_OK) return rc;
    }
    auto scan = chunk_bwd_scan_kernel<K, V>;
    constexpr size_t smem_s = BwdScanLds<K, V>::bytes;
    if (ensure_lds_limit((const void*)scan, (int)smem_s) != hipSuccess)
      return set_error(KDA_ERR_LAUNCH, "chunk_backward: scan LDS attribute failed");
    const int nrec = p->num_seqs * p->heads;
    const int grid = kXcds * (V / 16) * ((nrec + kXcds - 1) / kXcds);
    PrefetchList pf = {};
    const size_t rows = (size_t)p->batch * p->seq_len * p->heads;
    auto add = [&](const void* ptr, size_t bytes) {
      if (ptr && bytes >= 128 && pf.n < kMaxPrefetch) {
        pf.p[pf.n] = (const char*)ptr;
        pf.lines[pf.n++] = bytes / 128;
      }
    };
    (void)rows;
    add(a.sc.p[S_NG], sc_region_bytes(g, S_NG));
    add(a.sc.p[S_E], sc_region_bytes(g, S_E));
    add(a.ws.p[R_LAM], ws_region_bytes(g, R_LAM));
    const int cus = device_cu_count();
    const int extra = cus > grid ? cus - grid : 0;
    hipLaunchKernelGGL(scan, dim3(grid + extra), dim3(kBwdThreads), smem_s, stream, a, pf, grid);
    KDA_LAUNCH_CHECK("chunk_backward scan");
  }
  if (g.max_chunks > 0) {
    constexpr size_t smem = DenseSmem<K, V>::bytes > DecaySmem<K>::bytes ? DenseSmem<K, V>::bytes
                                                                          : DecaySmem<K>::bytes;
    auto vjp = chunk_bwd_vjp_kernel<K, V>;
    if (ensure_lds_limit((const void*)vjp, (int)smem) != hipSuccess)
      return set_error(KDA_ERR_LAUNCH, "chunk_backward: LDS attribute failed");
    const bool dense = stages & (1 << (KDA_STAGE_BWD_DENSE - 10));
    const bool decay = stages & (1 << (KDA_STAGE_BWD_DECAY - 10));
    const int N = g.max_chunks * p->heads;
    const int R = device_cu_count();
    auto launch = [&](int dense_begin, int dense_count, int decay_begin, int items) {
      hipLaunchKernelGGL(vjp, dim3(items), dim3(kVjpThreads), smem, stream, a, dense_begin, dense_count, decay_begin);
    };
    if (dense && decay && R > 0 && N >= R) {
      // items 0..N-1 dense, N..2N-1 decay, in launches of R: decay tile j (item N + j) is
      // always in a later launch than dense tile j (item j) because N >= R
      for (int start = 0; start < 2 * N; start += R) {
        const int end = start + R < 2 * N ? start + R : 2 * N;
        const int dcount = start < N ? (end < N ? end : N) - start : 0;
        launch(start < N ? start : 0, dcount, (start > N ? start : N) - N, end - start);
        KDA_LAUNCH_CHECK("chunk_backward dense/decay");
      }
    } else {
      if (dense) {
        launch(0, N, 0, N);
        KDA_LAUNCH_CHECK("chunk_backward dense");
      }
      if (decay) {
        launch(0, 0, 0, N);
        KDA_LAUNCH_CHECK("chunk_backward decay");
      }
    }
  }
  if (p->gate_mode == KDA_GATE_K3 && (stages & (1 << (KDA_STAGE_BWD_PARAMS - 10)))) {
    auto params = chunk_bwd_params_kernel<K>;
    hipLaunchKernelGGL(params, dim3(p->heads), dim3(kParamThreads), 0, stream, a, g.max_chunks);
    KDA_LAUNCH_CHECK("chunk_backward params");
  }
  return KDA_OK;
}

}  // namespace kda

static int chunk_backward_impl(int stages, const kda_chunk_problem* p, const void* q, const void* k,
                                  const void* v, const void* gate, const void* beta_logits,
                                  const float* A_log, const float* dt_bias,
                                  const float* initial_state, const void* workspace,
                                  const void* grad_output, const float* grad_final_state,
                                  void* dq, void* dk, void* dv, void* dgate, void* dbeta_logits,
                                  float* dA_log, float* ddt_bias, float* dinitial_state,
                                  void* scratch, hipStream_t stream) {
  using namespace kda;
  int rc = validate_problem(p, "chunk_backward");
  if (rc != KDA_OK) return rc;
  (void)initial_state;
  const bool empty = (size_t)p->batch * p->seq_len == 0;
  KDA_REQUIRE(empty || (q && k && v && gate && beta_logits && grad_output && dq && dk && dv &&
                        dgate && dbeta_logits),
              "chunk_backward: null input/output pointer");
  KDA_REQUIRE(aligned16(q, k, v, gate, grad_output, dq, dk, dv, dgate),
              "chunk_backward: q, k, v, gate, grad_output and the gradients must be 16-byte aligned");
  KDA_REQUIRE(p->gate_mode != KDA_GATE_K3 || (A_log && dt_bias && dA_log && ddt_bias),
              "chunk_backward: K3 gate needs A_log, dt_bias, dA_log and ddt_bias");
  KDA_REQUIRE(p->grad_row_stride == 0 ||
                  (p->grad_row_stride % 8 == 0 &&
                   (long)p->grad_row_stride >= (long)p->heads * (p->key_dim > p->value_dim ? p->key_dim : p->value_dim)),
              "chunk_backward: grad_row_stride must be 0 or a multiple of 8 of at least H * max(K, V)");
  KDA_REQUIRE(workspace && ((uintptr_t)workspace % 256) == 0,
              "chunk_backward: workspace must be non-null and 256-byte aligned");
  KDA_REQUIRE(scratch && ((uintptr_t)scratch % 256) == 0,
              "chunk_backward: scratch must be non-null and 256-byte aligned");
  if (generic_dims(p)) {
    KDA_REQUIRE(stages == ~0, "chunk_backward_stage: stage entry points need head dims 64 or 128");
    if (padded_route(p))
      return padded_backward(p, beta_logits, A_log, workspace, grad_output, grad_final_state, dq, dk, dv, dgate,
                             dbeta_logits, dA_log, ddt_bias, dinitial_state, scratch, stream);
    return generic_backward(p, q, k, v, gate, beta_logits, A_log, dt_bias, workspace, grad_output,
                            grad_final_state, dq, dk, dv, dgate, dbeta_logits, dA_log, ddt_bias,
                            dinitial_state, scratch, stream);
  }
  const ChunkGeom g = make_geom(p);
  BwdArgs a;
  a.H = p->heads;
  a.num_seqs = p->num_seqs;
  a.fixed_T = (p->cu_seqlens == nullptr && g.max_chunks > 0) ? p->seq_len : 0;
  a.gate_mode = p->gate_mode;
  a.lb = p->lower_bound;
  a.scale = p->scale;
  a.q = (const bf16*)q;
  a.k = (const bf16*)k;
  a.v = (const bf16*)v;
  a.gate = gate;
  a.beta_logits = (const bf16*)beta_logits;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
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
  a.ws = ws_regions(g, const_cast<void*>(workspace));
  a.sc = sc_regions(g, scratch);
  if (p->key_dim == 128 && p->value_dim == 128) return launch_backward<128, 128>(p, g, a, stream, stages);
  if (p->key_dim == 64 && p->value_dim == 64) return launch_backward<64, 64>(p, g, a, stream, stages);
  if (p->key_dim == 128 && p->value_dim == 64) return launch_backward<128, 64>(p, g, a, stream, stages);
  return launch_backward<64, 128>(p, g, a, stream, stages);
}

extern "C" int kda_chunk_backward(const kda_chunk_problem* p, const void* q, const void* k,
                                  const void* v, const void* gate, const void* beta_logits,
                                  const float* A_log, const float* dt_bias,
                                  const float* initial_state, const void* workspace,
                                  const void* grad_output, const float* grad_final_state,
                                  void* dq, void* dk, void* dv, void* dgate, void* dbeta_logits,
                                  float* dA_log, float* ddt_bias, float* dinitial_state,
                                  void* scratch, hipStream_t stream) {
  return chunk_backward_impl(~0, p, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state,
                             workspace, grad_output, grad_final_state, dq, dk, dv, dgate,
                             dbeta_logits, dA_log, ddt_bias, dinitial_state, scratch, stream);
}

extern "C" int kda_chunk_backward_stage(int32_t stage, const kda_chunk_problem* p, const void* q,
                                        const void* k, const void* v, const void* gate,
                                        const void* beta_logits, const float* A_log,
                                        const float* dt_bias, const float* initial_state,
                                        const void* workspace, const void* grad_output,
                                        const float* grad_final_state, void* dq, void* dk,
                                        void* dv, void* dgate, void* dbeta_logits,
                                        float* dA_log, float* ddt_bias, float* dinitial_state,
                                        void* scratch, hipStream_t stream) {
  if ((stage < KDA_STAGE_BWD_SCAN || stage > KDA_STAGE_BWD_PARAMS) && stage != KDA_STAGE_BWD_VJP)
    return kda::set_error(KDA_ERR_INVALID, "chunk_backward_stage: unknown stage %d", stage);
  const int mask = stage == KDA_STAGE_BWD_VJP ? (1 << (KDA_STAGE_BWD_DENSE - 10)) | (1 << (KDA_STAGE_BWD_DECAY - 10))
                                              : 1 << (stage - 10);
  return chunk_backward_impl(mask, p, q, k, v, gate, beta_logits, A_log, dt_bias,
                             initial_state, workspace, grad_output, grad_final_state, dq, dk, dv,
                             dgate, dbeta_logits, dA_log, ddt_bias, dinitial_state, scratch,
                             stream);
}

extern "C" int kda_debug_set_wait_limit(int64_t ticks) {
  kda::g_wait_limit.store(ticks < 0 ? -1 : ticks, std::memory_order_relaxed);
  return KDA_OK;
}

extern "C" int kda_chunk_backward_status(const kda_chunk_problem* p, const void* scratch,
                                         hipStream_t stream) {
  using namespace kda;
  int rc = validate_problem(p, "chunk_backward_status");
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(scratch && ((uintptr_t)scratch % 256) == 0,
              "chunk_backward_status: scratch must be non-null and 256-byte aligned");
  if (padded_route(p)) return padded_status(p, scratch, stream);
  if (generic_dims(p)) return KDA_OK;  // the token-serial backward has no waits
  const Regions sc = sc_regions(make_geom(p), const_cast<void*>(scratch));
  int word = 0;
  hipError_t e = hipMemcpyAsync(&word, sc.p[S_SYNC] + sizeof(int), sizeof(int), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return set_error(KDA_ERR_LAUNCH, "chunk_backward_status: %s", hipGetErrorString(e));
  if (word != 0)
    return set_error(KDA_ERR_TIMEOUT,
                     "chunk_backward: a VJP tile's wait for the reverse scan timed out; the "
                     "affected gradients were overwritten with NaN");
  return KDA_OK;
}

// ---------------------------------------------------------------------------------------
// Allocation-free backward: the scratch lives in a file-scope device array instead of a
// caller buffer.  Each device that loads the library holds its own copy of the array for
// the life of the process; host code reaches it only through the address
// hipGetSymbolAddress returns on that device (the array's name is not a device address
// in host code).  The kernels write every scratch element they read, so nothing needs
// clearing between calls; calls that overlap on one device share the array and race.
// ---------------------------------------------------------------------------------------
#include <mutex>

namespace kda {

constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices] = {};
static std::mutex g_scratch_mu;

// Device address of this device's scratch array, looked up once per device.
static int noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(KDA_ERR_LAUNCH, "chunk_backward_noalloc: no current device (or device index >= %d)",
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(KDA_ERR_LAUNCH, "chunk_backward_noalloc: hipGetSymbolAddress failed on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return KDA_OK;
}

}  // namespace kda

extern "C" size_t kda_chunk_backward_noalloc_max_scratch_bytes(void) { return kda::kNoAllocScratchBytes; }

extern "C" int kda_chunk_backward_noalloc(const kda_chunk_problem* p, const void* q, const void* k,
                                          const void* v, const void* gate, const void* beta_logits,
                                          const float* A_log, const float* dt_bias,
                                          const float* initial_state, const void* workspace,
                                          const void* grad_output, const float* grad_final_state,
                                          void* dq, void* dk, void* dv, void* dgate, void* dbeta_logits,
                                          float* dA_log, float* ddt_bias, float* dinitial_state,
                                          hipStream_t stream) {
  using namespace kda;
  int rc = validate_problem(p, "chunk_backward_noalloc");
  if (rc != KDA_OK) return rc;
  const size_t need = !generic_dims(p) ? sc_total_bytes(make_geom(p))
                                        : padded_route(p) ? padded_sc_bytes(p) : generic_sc_bytes(p);
  KDA_REQUIRE(need <= kNoAllocScratchBytes,
              "chunk_backward_noalloc: problem needs %zu bytes of scratch, more than the %zu-byte "
              "static array (use kda_chunk_backward with a caller buffer)",
              need, kNoAllocScratchBytes);
  void* sc = nullptr;
  rc = noalloc_scratch(&sc);
  if (rc != KDA_OK) return rc;
  return chunk_backward_impl(~0, p, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state,
                             workspace, grad_output, grad_final_state, dq, dk, dv, dgate,
                             dbeta_logits, dA_log, ddt_bias, dinitial_state, sc, stream);
}
