// Workspace layout shared by the chunked forward and backward kernels.
//
// Work is cut into "tiles" = (chunk of <= 64 tokens of one sequence, head).  The chunk
// table maps a chunk index to {first flat token row, length, sequence, index in
// sequence}; the sequence table maps a sequence to {first chunk, chunk count}.  Every
// per-tile region below is an array [n_tiles][...] with tile = chunk * H + head.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace kda {

// Element size of the reverse scan's per-chunk input E (f32, or bf16 with KDA_E_BF16).
#ifndef KDA_E_BF16
#define KDA_E_BF16 1
#endif
constexpr int kEBytes = KDA_E_BF16 ? 2 : 4;

// "Fragment-major" arrays hold a matrix in the exact order the MFMA A/B operand registers
// of v_mfma_f32_16x16x32_bf16 consume it: for a row-major R x C matrix X, fragment
// (rt, s) is the 16 x 32 block rows 16rt.., columns 32s..; lane l holds
// X[16rt + l%16][32s + 8(l/16) + e], e = 0..7, and the 64 lanes' 16-byte pieces are
// contiguous.  A wave loads one operand with one fully coalesced 1 KB access.
__host__ __device__ inline size_t frag_off(int C, int rt, int s, int lane) {
  return ((((size_t)rt * (C / 32) + s) * 64) + lane) * 8;
}

// Offsets (bf16 elements) of element X[row][col] of a C-column matrix in fragment-major
// order, natural (contraction index 32s + 8(l/16) + e) and permuted (see below).
__host__ __device__ inline size_t nat_frag_elem(int C, int row, int col) {
  const int lane = row % 16 + 16 * ((col % 32) / 8);
  return (((size_t)(row / 16) * (C / 32) + col / 32) * 64 + lane) * 8 + col % 8;
}
__host__ __device__ inline size_t perm_frag_elem(int C, int row, int col) {
  const int lane = row % 16 + 16 * ((col % 16) / 4);
  const int e = 4 * ((col % 32) / 16) + col % 4;
  return (((size_t)(row / 16) * (C / 32) + col / 32) * 64 + lane) * 8 + e;
}

// Arrays marked "permuted" keep their fragment shape but order each 32-wide step of the
// contraction index as 32s + 16(e/4) + 4(l/16) + e%4 for element e of lane l (instead of
// 32s + 8(l/16) + e): the order in which a lane holds two stacked MFMA accumulator tiles,
// so the scan feeds accumulators straight back in as operands.
enum WsRegion {
  R_CHUNKS = 0,  // int4 [max_chunks]   {row0, len, seq, index_in_seq}
  R_SEQS,        // int2 [num_seqs]     {first_chunk, n_chunks}
  R_QGF,         // bf16 fragments of Qg = q_hat exp(G) (64 x K; q_hat includes the scale), permuted
  R_KDF,         // bf16 fragments of Kd = k_hat exp(G_last - G) (64 x K)
  R_KDTF,        // bf16 fragments of Kd^T (K x 64), permuted
  R_WF,          // bf16 fragments of -W, W = T (beta k_hat exp(G)) (64 x K), permuted
  R_UF,          // bf16 U = T (beta v) in MFMA C layout: [V/16 strip][4 row tile][64 lane][4]
  R_AF,          // bf16 fragments of A (64 x 64, lower incl. diagonal), permuted
  R_T,           // bf16 [tile][64][64] T = (I + diag(beta) M')^-1 (only ever a bf16 MFMA operand)
  R_MP,          // f32  [tile][64][64] M' (strictly lower, without beta)
  R_G,           // f32  [tile][64][K]  G = inclusive cumsum of g in the chunk
  R_LAM,         // f32  [tile][K]      exp(G_last)
  R_RQ,          // f32  [tile][64]     scale / max(||q||, 1e-12)
  R_RK,          // f32  [tile][64]     1 / max(||k||, 1e-12)
  R_BETA,        // f32  [tile][64]     sigmoid(beta_logits)
  R_SH,          // f32  [tile][K][V]   state entering the chunk (written by the scan)
  R_SHBF,        // bf16 the same state as B-operand fragments [V/16 strip][K/32][64][8], permuted
  R_DLF,         // bf16 delta = U - W S as B-operand fragments [V/16 strip][2][64][8] (scan), permuted
  // segmented scan (only when ChunkGeom::seg_len > 0; [rec = seq * H + head][segment] ...)
  R_SEGP,        // bf16 [rec][seg] K x K  P = product of the segment's chunk maps, as MFMA A fragments
  R_SEGS,        // f32  [rec][seg][V][K]  Sigma = the segment's end state from a zero start (V-first)
  R_SIN,         // f32  [rec][seg][V][K]  true state entering the segment (V-first; seg >= 1)
  R_COUNT
};

enum ScRegion {
  S_DSH = 0,  // bf16 [tile][V/16][K][16]  dL/dS at the chunk end, strip-major (a bf16 MFMA operand of dKd)
  S_NG,       // bf16 [tile] K x K  -G = -(W^T Kd) as MFMA A fragments, permuted (the reverse scan's transition)
  S_E,        // f32 (bf16: KDA_E_BF16) [tile][V/16][K/16][64 lane][4]  E = Qg^T dO - W^T (A^T dO) in the scan's accumulator order
  S_DA,       // bf16 [tile][64][64] dL/dA (masked lower; the decay VJP's MFMA operand)
  S_DMP,      // bf16 [tile][64][64] dL/dM' (strictly lower, beta folded in; same)
  S_DQG,      // f32  [tile][item][64 lane][4]  dL/dQg  in MFMA C layout (item = row tile + 4 col tile)
  S_DKD,      // f32  [tile][item][64 lane][4]  dL/dKd  (same layout)
  S_DKB,      // f32  [tile][item][64 lane][4]  dL/d(beta kh exp(G))  (same layout)
  S_PP,       // f32  [tile][2][K]   gate parameter partials {sum draw, sum draw*(z+b)}
  S_DGL,      // f32  [tile][K]      lam * dL/dlam (the state-decay part of dL/dG_last)
  S_DBETA,    // f32  [tile][64]     dL/dbeta from the dense VJP (U, M' terms)
  S_SYNC,     // int  fused backward: ticket, abort, per-record step counts, per-tile strip arrivals
  S_ORDER,    // int4 [max_chunks][2] the fused backward's order (reverse rank, then sequence): position p ->
              //   {chunk, row0, len, seq} {steps the tile's record must publish, 0, 0, 0}
  S_COUNT
};

struct ChunkGeom {
  int max_chunks;
  int heads;
  int K;
  int V;
  int num_seqs;
  int seg_len;   // chunks per scan segment; 0: the scans run each sequence in one pass
  int max_segs;  // segments of the longest possible sequence (1 when seg_len == 0)
};

__host__ __device__ inline size_t ws_region_bytes(const ChunkGeom& g, int r) {
  const size_t nt = (size_t)g.max_chunks * g.heads;
  const size_t K = g.K, V = g.V;
  switch (r) {
    case R_CHUNKS: return (size_t)g.max_chunks * 16;
    case R_SEQS: return (size_t)g.num_seqs * 8;
    case R_QGF: case R_KDF: case R_KDTF: case R_WF: return nt * 64 * K * 2;
    case R_UF: return nt * 64 * V * 2;
    case R_AF: return nt * 64 * 64 * 2;
    case R_T: return nt * 64 * 64 * 2;
    case R_MP: return nt * 64 * 64 * 4;
    case R_G: return nt * 64 * K * 4;
    case R_LAM: return nt * K * 4;
    case R_RQ: case R_RK: case R_BETA: return nt * 64 * 4;
    case R_SH: return nt * K * V * 4;
    case R_SHBF: return nt * K * V * 2;
    case R_DLF: return nt * 64 * V * 2;
    case R_SEGP: return g.seg_len ? (size_t)g.num_seqs * g.heads * g.max_segs * K * K * 2 : 0;
    case R_SEGS: case R_SIN: return g.seg_len ? (size_t)g.num_seqs * g.heads * g.max_segs * V * K * 4 : 0;
    default: return 0;
  }
}

__host__ __device__ inline size_t sc_region_bytes(const ChunkGeom& g, int r) {
  const size_t nt = (size_t)g.max_chunks * g.heads;
  const size_t K = g.K, V = g.V;
  switch (r) {
    case S_DSH: return nt * K * V * 2;
    case S_NG: return nt * K * K * 2;
    case S_E: return nt * K * V * kEBytes;
    case S_DA: case S_DMP: return nt * 64 * 64 * 2;
    case S_DQG: case S_DKD: case S_DKB: return nt * 64 * K * 4;
    case S_PP: return nt * 2 * K * 4;
    case S_DGL: return nt * K * 4;
    case S_DBETA: return nt * 64 * 4;
    case S_SYNC: return (32 + 32 * (size_t)g.num_seqs * g.heads + nt) * 4;
    case S_ORDER: return (size_t)g.max_chunks * 32;
    default: return 0;
  }
}

struct Regions {
  char* p[(int)R_COUNT > (int)S_COUNT ? (int)R_COUNT : (int)S_COUNT];
};

__host__ __device__ inline size_t round256(size_t x) { return (x + 255) & ~size_t(255); }

inline size_t ws_total_bytes(const ChunkGeom& g) {
  size_t t = 0;
  for (int r = 0; r < R_COUNT; ++r) t += round256(ws_region_bytes(g, r));
  return t;
}

inline size_t sc_total_bytes(const ChunkGeom& g) {
  size_t t = 0;
  for (int r = 0; r < S_COUNT; ++r) t += round256(sc_region_bytes(g, r));
  return t;
}

inline Regions ws_regions(const ChunkGeom& g, void* base) {
  Regions out;
  char* p = (char*)base;
  for (int r = 0; r < R_COUNT; ++r) {
    out.p[r] = p;
    p += round256(ws_region_bytes(g, r));
  }
  return out;
}

inline Regions sc_regions(const ChunkGeom& g, void* base) {
  Regions out;
  char* p = (char*)base;
  for (int r = 0; r < S_COUNT; ++r) {
    out.p[r] = p;
    p += round256(sc_region_bytes(g, r));
  }
  return out;
}

}  // namespace kda
