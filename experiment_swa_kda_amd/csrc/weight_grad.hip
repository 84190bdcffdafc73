// Weight gradient of a linear layer, dW[N, K] (f32) = dy[M, N]^T x[M, K] (bf16), for the
// trainer's projections (M = batch * tokens, N and K a few hundred).
//
// Reference: the weight-gradient GEMM that autograd runs for nanochat's Linear
// (nanochat/gpt.py:52-57: F.linear on the bf16 cast of an f32 master weight).  Library
// GEMMs tile this shape (a long contraction, a small output) into a few dozen workgroups;
// here the contraction is split into ranges of 512-row blocks, one workgroup per (output tile,
// range), as many ranges as it takes to fill the chip,
// and the f32 partials are summed in a fixed order by a second kernel (deterministic, no
// atomics).
//
// Both operands are row-major in M, while an MFMA operand fragment holds 8 consecutive
// contraction rows of one column.  Two kernels:
//  - outputs of at least kWgDmaMinTiles 128 x 128 tiles with aligned operands: LDS stages
//    filled by dedicated loader waves with global -> LDS buffer loads, fragments read down the
//    columns with transposing LDS reads (weight_grad_dma_kernel, below);
//  - otherwise 64 x 64 tiles (four times the tiles, so fewer ranges and partials): each
//    thread loads an 8 x 8 block (8 rows of one 16-byte
// column group), transposes it in registers and writes 8 16-byte rows of the transposed
// slab [column][row] to LDS, so every global access and every LDS access is 16 bytes wide.
// A workgroup covers kWgDepth 128-row steps of the contraction and issues all of their
// global loads up front; one barrier per step (double-buffered LDS).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kWgThreads = 256;
constexpr int kWgTile = 64;          // output tile: 64 (n) x 64 (k)
constexpr int kWgRows = 128;         // contraction rows per step
constexpr int kWgDepth = 4;         // contraction steps whose loads are in flight
constexpr int kWgPitch = kWgRows + 8;  // bf16 per transposed LDS row (+16 B against bank conflicts)

struct WgLds {
  bf16 dyT[2][kWgTile * kWgPitch];
  bf16 xT[2][kWgTile * kWgPitch];
};

// Loads this thread's 8 x 8 block: rows m0 + r (r < 8), columns c .. c + 7 of a row-major
// [M, ncols] operand with leading dimension ld.  Rows >= m_end and columns >= ncols read
// as zero.  Every load is issued unconditionally from a clamped address and masked with
// bit operations afterwards, so no branch separates a load from its use (a branch would
// make the compiler wait for all outstanding loads at the join).  VEC: ld and the base are
// 16-byte aligned and ncols % 8 == 0.
template <bool VEC>
__device__ __forceinline__ void load_block(const bf16* __restrict__ p, long ld, int ncols, int m0,
                                           int m_end, int c, bf16x8 (&v)[8]) {
  if constexpr (VEC) {
    const bool cok = c < ncols;
    const int cc = cok ? c : 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int m = m0 + r;
      const int mc = m < m_end ? m : m_end - 1;
      v[r] = *reinterpret_cast<const bf16x8*>(p + (long)mc * ld + cc);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const unsigned keep = (cok && m0 + r < m_end) ? 0xffffffffu : 0u;
      uint4 u = __builtin_bit_cast(uint4, v[r]);
      u.x &= keep; u.y &= keep; u.z &= keep; u.w &= keep;
      v[r] = __builtin_bit_cast(bf16x8, u);
    }
  } else {
    unsigned short e16[8][8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int m = m0 + r;
      const int mc = m < m_end ? m : m_end - 1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int ce = c + e < ncols ? c + e : ncols - 1;
        e16[r][e] = reinterpret_cast<const unsigned short*>(p)[(long)mc * ld + ce];
      }
    }
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned short keep = (m0 + r < m_end && c + e < ncols) ? 0xffff : 0;
        v[r][e] = __builtin_bit_cast(bf16, (unsigned short)(e16[r][e] & keep));
      }
  }
}

// 16-byte chunk c of transposed row `row` lives at chunk c ^ ((row / 8) % 8): the eight
// threads that write one chunk index into rows 8 cb + j (cb = 0..7) then hit eight
// different bank groups instead of one.
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 3) & 7); }

// Writes the transpose of an 8 x 8 block: LDS row (column c0 + j) gets rows 8 mb .. 8 mb + 7.
__device__ __forceinline__ void store_transposed(bf16* slab, int col0, int mb, const bf16x8 (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bf16x8 w;
#pragma unroll
    for (int r = 0; r < 8; ++r) w[r] = v[r][j];
    const int row = col0 + j;
    *reinterpret_cast<bf16x8*>(slab + row * kWgPitch + 8 * swz(row, mb)) = w;
  }
}

template <bool VEC>
__global__ __launch_bounds__(kWgThreads) void weight_grad_kernel(
    int M, int N, int K, const bf16* __restrict__ dy, long ldd, const bf16* __restrict__ x, long ldx,
    int rows_per_split, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) WgLds s;
  // 1-D grid of kXcds * per_xcd: workgroups are dispatched round-robin over the XCDs
  // (linear id mod 8), and XCD x takes the items x * per_xcd .. of the (split, tile) order,
  // so the tiles of one split (the same dy / x rows) share an XCD and its L2, and every row
  // range is fetched from HBM about once.
  const int tiles_k = (K + kWgTile - 1) / kWgTile;
  const int tiles = tiles_k * ((N + kWgTile - 1) / kWgTile);
  const int splits = (max(M, 1) + rows_per_split - 1) / rows_per_split;
  const int per_xcd = (tiles * splits + kXcds - 1) / kXcds;
  const int item = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (item >= tiles * splits) return;  // grid rounding
  const int tile = item % tiles, split = item / tiles;
  const int n0 = (tile / tiles_k) * kWgTile, k0 = (tile % tiles_k) * kWgTile;
  const int m_begin = split * rows_per_split;
  const int m_end = min(M, m_begin + rows_per_split);
  const int tid = threadIdx.x;
  // loader role: threads 0..127 stage dy, 128..255 stage x; block (mb, cb) of the step
  const bool is_x = tid >= 128;
  const int b = tid % 128, mb = b / 8, cb = b % 8;
  const bf16* src = is_x ? x : dy;
  const long ld = is_x ? ldx : ldd;
  const int ncols = is_x ? K : N;
  const int col = (is_x ? k0 : n0) + 8 * cb;
  // compute role: wave (wn, wk) owns the 32 x 32 sub-tile (32 wn.., 32 wk..)
  const int wave = tid / kWave, lane = tid % kWave;
  const int wn = wave / 2, wk = wave % 2;
  const int lr = lane % 16, kg = lane / 16;

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero4();

  if (m_end <= m_begin) {  // M == 0: the gradient is zero, and there is no row to load
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int k = k0 + 32 * wk + 16 * j + lr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = n0 + 32 * wn + 16 * i + 4 * kg + r;
          if (n < N && k < K) out[(size_t)n * K + k] = 0.f;
        }
      }
    return;
  }
  // The range is a whole number of blocks of kWgDepth 128-row steps (rows past m_end are
  // zero); all global loads of a block are issued before its first step.  The LDS buffer
  // parity continues across blocks (kWgDepth is even), so one barrier per step still
  // separates a buffer's reuse from its last reads.
  static_assert(kWgDepth % 2 == 0, "buffer parity across blocks");
  for (int blk = m_begin; blk < m_end; blk += kWgDepth * kWgRows) {
  bf16x8 v[kWgDepth][8];
#pragma unroll
  for (int d = 0; d < kWgDepth; ++d)
    load_block<VEC>(src, ld, ncols, blk + d * kWgRows + 8 * mb, m_end, col, v[d]);
#pragma unroll
  for (int st = 0; st < kWgDepth; ++st) {
    const int buf = st & 1;
    store_transposed(is_x ? s.xT[buf] : s.dyT[buf], 8 * cb, mb, v[st]);
    __syncthreads();
    const bf16* A = s.dyT[buf];
    const bf16* B = s.xT[buf];
#pragma unroll
    for (int ks = 0; ks < kWgRows / 32; ++ks) {
      bf16x8 a[2], bb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = 32 * wn + 16 * i + lr;
        a[i] = *reinterpret_cast<const bf16x8*>(A + row * kWgPitch + 8 * swz(row, 4 * ks + kg));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = 32 * wk + 16 * j + lr;
        bb[j] = *reinterpret_cast<const bf16x8*>(B + row * kWgPitch + 8 * swz(row, 4 * ks + kg));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma16(a[i], bb[j], acc[i][j]);
    }
  }
  }
  float* o = out + (size_t)split * N * K;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int k = k0 + 32 * wk + 16 * j + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = n0 + 32 * wn + 16 * i + 4 * kg + r;
        if (n < N && k < K) o[(size_t)n * K + k] = acc[i][j][r];
      }
    }
}

// ---------------------------------------------------------------------------------------
// Aligned operands: 128 x 128 output tiles.  Two loader waves stream 32-row contraction steps
// of dy (128 columns) and x (128 columns) into LDS with buffer loads (global -> LDS, no
// registers), kWgStages - 1 steps ahead; four compute waves own 64 x 64 each (4 x 4 MFMA
// accumulators) and read their operand fragments, 8 consecutive contraction rows of one
// column, with transposing LDS reads, one step ahead of the products.  A stage row is the
// 256 bytes of one contraction row; its 16-byte chunk q sits in slot q ^ 2 (row % 4), so the
// four rows one transposing read touches fall on different banks.
// ---------------------------------------------------------------------------------------
constexpr int kWgBT = 128;                          // output tile (n and k)
constexpr int kWgBR = 32;                           // contraction rows per step
constexpr int kWgStages = 6;
constexpr int kWgCompute = 4;
constexpr int kWgDmaThreads = (kWgCompute + 2) * kWave;
constexpr int kWgRowBytes = kWgBT * 2;              // 256
constexpr int kWgPart = kWgBR * kWgRowBytes;        // 8 KB: one operand's step
constexpr int kWgStage = 2 * kWgPart;
constexpr int kWgNI = kWgPart / 1024;               // loads per step and loader (8)
constexpr int kWgDmaLds = kWgStages * kWgStage;     // 96 KB
static_assert((kWgStages - 2) * kWgNI < 64, "vmcnt range");

__device__ __forceinline__ int wg_slot_off(int r, int col) {
  // byte offset of column col (a multiple of 4) of stage row r
  return r * kWgRowBytes + (((col >> 3) ^ (2 * (r & 3))) << 4) + ((col >> 2) & 1) * 8;
}

// lane (l % 16, l / 16) gets rows 8 (l / 16) + e (e < 8) of column c0 + l % 16 of one operand's
// stage (two transposing reads; the second four rows are 4 rows = 1 KB further)
__device__ __forceinline__ bf16x8 wg_col_frag(const char* part, int c0, int lane) {
  const int lr = lane % 16, kg = lane / 16;
  const char* p = part + wg_slot_off(8 * kg + lr / 4, c0 + 4 * (lr % 4));
  const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)p);
  const short4_t hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(p + 4 * kWgRowBytes));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

__global__ __launch_bounds__(kWgDmaThreads) void weight_grad_dma_kernel(
    int M, int N, int K, const bf16* __restrict__ dy, long ldd, const bf16* __restrict__ x, long ldx,
    int rows_per_split, float* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tiles_k = (K + kWgBT - 1) / kWgBT;
  const int tiles = tiles_k * ((N + kWgBT - 1) / kWgBT);
  const int splits = (max(M, 1) + rows_per_split - 1) / rows_per_split;
  const int per_xcd = (tiles * splits + kXcds - 1) / kXcds;
  const int item = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (item >= tiles * splits) return;  // grid rounding (the whole workgroup)
  const int tile = item % tiles, split = item / tiles;
  const int n0 = (tile / tiles_k) * kWgBT, k0 = (tile % tiles_k) * kWgBT;
  const int m_begin = split * rows_per_split, m_end = min(M, m_begin + rows_per_split);
  const int nsteps = (max(m_end - m_begin, 0) + kWgBR - 1) / kWgBR;
  // uniform wave index: the loaders' descriptors and LDS bases must be scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;

  if (wave >= kWgCompute) {
    // ---- loader waves: wave 4 moves dy rows (columns n0..), wave 5 x rows (k0..) ----
    if (nsteps == 0) return;
    const bool isd = wave == kWgCompute;
    const __amdgpu_buffer_rsrc_t rs = raw_rsrc(isd ? (const void*)dy : (const void*)x);
    const long ld = isd ? ldd : ldx;
    const int c0 = isd ? n0 : k0, ncols = isd ? N : K;
    auto issue = [&](int q) {
      char* st = smem + (q % kWgStages) * kWgStage + (isd ? 0 : kWgPart);
      const int m0 = m_begin + q * kWgBR;
#pragma unroll
      for (int i = 0; i < kWgNI; ++i) {
        const int r = 4 * i + lane / 16, qc = (lane % 16) ^ (2 * (r & 3));
        const int m = m0 + r, c = c0 + 8 * qc;
        const bool ok = m < m_end && c < ncols;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(st + 4 * i * kWgRowBytes),
                                                 16, ok ? (int)(((long)m * ld + c) * 2) : kDropOffset, 0, 0, 0);
      }
    };
    constexpr int P = kWgStages - 1;
    auto wait_landed = [&](int later) {  // step t landed: at most `later` steps issued after it
      switch (later) {
        case 4: wait_vmcnt<4 * kWgNI>(); break;
        case 3: wait_vmcnt<3 * kWgNI>(); break;
        case 2: wait_vmcnt<2 * kWgNI>(); break;
        case 1: wait_vmcnt<kWgNI>(); break;
        default: wait_vmcnt<0>(); break;
      }
    };
    for (int q = 0; q < P && q < nsteps; ++q) issue(q);
    wait_landed(min(P - 1, nsteps - 1));
    ring_barrier();  // B0: step 0 visible
    for (int q = 0; q < nsteps; ++q) {
      wait_landed(max(0, min(P - 2, nsteps - 2 - q)));
      ring_barrier();  // A(q): step q + 1 visible; step q - 1's slot is free
      if (q + P < nsteps) issue(q + P);
    }
    return;
  }

  // ---- compute wave (wn, wk): output rows n0 + 64 wn.., columns k0 + 64 wk.. ----
  const int wn = wave / 2, wk = wave % 2;
  const int lr = lane % 16, kg = lane / 16;
  f32x4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = zero4();
  if (nsteps > 0) {
    auto read_frags = [&](int q, bf16x8 (&a)[4], bf16x8 (&b)[4]) {
      const char* st = smem + (q % kWgStages) * kWgStage;
#pragma unroll
      for (int t = 0; t < 4; ++t) a[t] = wg_col_frag(st, 64 * wn + 16 * t, lane);
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = wg_col_frag(st + kWgPart, 64 * wk + 16 * u, lane);
    };
    auto step = [&](int q, const bf16x8 (&a)[4], const bf16x8 (&b)[4], bf16x8 (&an)[4], bf16x8 (&bn)[4]) {
      ring_barrier();  // A(q)
      if (q + 1 < nsteps) read_frags(q + 1, an, bn);  // overlaps the products below
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[t][u] = mfma16(a[t], b[u], acc[t][u]);
    };
    bf16x8 a0[4], b0[4], a1[4], b1[4];
    ring_barrier();  // B0
    read_frags(0, a0, b0);
    int q = 0;
    for (; q + 1 < nsteps; q += 2) {
      step(q, a0, b0, a1, b1);
      step(q + 1, a1, b1, a0, b0);
    }
    if (q < nsteps) step(q, a0, b0, a1, b1);
  }
  // lane (lr, kg) holds rows 16 t + 4 kg + r (n), column 16 u + lr (k) of the wave's block
  float* o = out + (size_t)split * N * K;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + 64 * wn + 16 * t + 4 * kg + r;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0 + 64 * wk + 16 * u + lr;
        if (n < N && k < K) o[(size_t)n * K + k] = acc[t][u][r];
      }
    }
}

// out[i] = sum_p part[p][i] in order p = 0, 1, ...; four outputs per thread, the loads of
// kSumBatch partials issued before any is added.
constexpr int kSumBatch = 8;
__global__ __launch_bounds__(256) void partial_sum_kernel(int parts, long n, const float* __restrict__ part,
                                                          float* __restrict__ out) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (n % 4 == 0) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int p0 = 0; p0 < parts; p0 += kSumBatch) {
      float4 v[kSumBatch];
#pragma unroll
      for (int u = 0; u < kSumBatch; ++u) {
        const int p = p0 + u < parts ? p0 + u : parts - 1;
        v[u] = *reinterpret_cast<const float4*>(part + (size_t)p * n + i);
      }
#pragma unroll
      for (int u = 0; u < kSumBatch; ++u) {
        if (p0 + u < parts) {
          acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
        }
      }
    }
    *reinterpret_cast<float4*>(out + i) = acc;
  } else {
    for (long e = i; e < i + 4 && e < n; ++e) {
      float acc = 0.f;
      for (int p = 0; p < parts; ++p) acc += part[(size_t)p * n + e];
      out[e] = acc;
    }
  }
}

struct WgPlan {
  int tiles, splits, rows_per_split;
};

// Enough (tile, range) workgroups to fill the chip about twice over (kWgTarget), with as few
// ranges as that allows: every extra range adds an f32 partial of the whole output that the
// reduction writes and reads back.  A range is a whole number of 512-row blocks.
constexpr int kWgTarget = 1024;
constexpr int kWgDmaTarget = 384;  // the 128 x 128 kernel: about one and a half workgroups per CU (measured best of 256, 384, 512)
constexpr int kWgDmaMinTiles = 24;  // fewer 128 x 128 tiles: the 64 x 64 kernel (fewer partials)

// The aligned kernel's plan: 128 x 128 tiles, ranges of whole 32-row steps.
static bool use_weight_grad_dma(int N, int K) {
  return ((N + kWgBT - 1) / kWgBT) * ((K + kWgBT - 1) / kWgBT) >= kWgDmaMinTiles;
}

static WgPlan plan_weight_grad_dma(int M, int N, int K) {
  WgPlan p;
  p.tiles = ((N + kWgBT - 1) / kWgBT) * ((K + kWgBT - 1) / kWgBT);
  const int steps = max(1, (M + kWgBR - 1) / kWgBR);
  const int want = max(1, min(steps, (kWgDmaTarget + p.tiles - 1) / p.tiles));
  const int per_split = (steps + want - 1) / want;
  p.rows_per_split = per_split * kWgBR;
  p.splits = (steps + per_split - 1) / per_split;
  return p;
}

static WgPlan plan_weight_grad(int M, int N, int K) {
  WgPlan p;
  p.tiles = ((N + kWgTile - 1) / kWgTile) * ((K + kWgTile - 1) / kWgTile);
  const int block = kWgDepth * kWgRows;
  const int blocks = max(1, (M + block - 1) / block);
  const int want = max(1, min(blocks, (kWgTarget + p.tiles - 1) / p.tiles));
  const int per_split = (blocks + want - 1) / want;
  p.rows_per_split = per_split * block;
  p.splits = (blocks + per_split - 1) / per_split;
  return p;
}

}  // namespace kda

extern "C" size_t kda_weight_grad_scratch_bytes(int64_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || M > 0x7fffffff) return 0;
  // enough for either kernel (which one runs depends on the operands' alignment)
  const kda::WgPlan p = kda::plan_weight_grad((int)M, N, K), q = kda::plan_weight_grad_dma((int)M, N, K);
  const int splits = std::max(p.splits > 1 ? p.splits : 0, q.splits > 1 ? q.splits : 0);
  return (size_t)splits * N * K * sizeof(float);
}

extern "C" int kda_weight_grad(int64_t M, int32_t N, int32_t K, const void* dy, int64_t ldd,
                               const void* x, int64_t ldx, float* dweight, void* scratch,
                               hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(M >= 0 && M <= 0x7fffffff && N > 0 && K > 0, "weight_grad: invalid shape");
  KDA_REQUIRE(ldd >= N && ldx >= K, "weight_grad: leading dimensions must cover the rows");
  KDA_REQUIRE(dweight && (M == 0 || (dy && x)), "weight_grad: null pointer");
  // M == 0: one split with no steps writes the zero gradient (no memset node, so the call
  // stays capturable)
  const bool vec = aligned16(dy, x) && ldd % 8 == 0 && ldx % 8 == 0 && N % 8 == 0 && K % 8 == 0;
  const bool dma = vec && use_weight_grad_dma(N, K);
  // M == 0 with the aligned kernel: one split with no steps writes zeros too
  const WgPlan p = dma ? plan_weight_grad_dma((int)std::max<int64_t>(M, 1), N, K)
                 : M > 0 ? plan_weight_grad((int)M, N, K)
                         : WgPlan{((N + kWgTile - 1) / kWgTile) * ((K + kWgTile - 1) / kWgTile), 1, 1};
  KDA_REQUIRE(p.splits == 1 || scratch, "weight_grad: scratch required (kda_weight_grad_scratch_bytes)");
  KDA_REQUIRE(aligned16(scratch, dweight), "weight_grad: dweight and scratch must be 16-byte aligned");
  KDA_REQUIRE(!dma || M == 0 || (((M - 1) * std::max(ldd, ldx) + std::max(N, K)) * 2 < 0x7fffff00LL),
              "weight_grad: operands exceed 2 GiB");
  float* part = p.splits > 1 ? (float*)scratch : dweight;
  dim3 grid(kXcds * ((p.tiles * p.splits + kXcds - 1) / kXcds));
  if (dma) {
    hipError_t e = ensure_lds_limit((const void*)weight_grad_dma_kernel, kWgDmaLds);
    if (e != hipSuccess) return set_error(KDA_ERR_LAUNCH, "weight_grad: LDS attribute: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(weight_grad_dma_kernel, grid, dim3(kWgDmaThreads), kWgDmaLds, stream, (int)M, N, K,
                       (const bf16*)dy, (long)ldd, (const bf16*)x, (long)ldx, p.rows_per_split, part);
  } else if (vec) {
    hipLaunchKernelGGL(weight_grad_kernel<true>, grid, dim3(kWgThreads), 0, stream, (int)M, N, K,
                       (const bf16*)dy, (long)ldd, (const bf16*)x, (long)ldx, p.rows_per_split, part);
  } else
    hipLaunchKernelGGL(weight_grad_kernel<false>, grid, dim3(kWgThreads), 0, stream, (int)M, N, K,
                       (const bf16*)dy, (long)ldd, (const bf16*)x, (long)ldx, p.rows_per_split, part);
  KDA_LAUNCH_CHECK("weight_grad");
  if (p.splits > 1) {
    const long n = (long)N * K;
    const unsigned blocks = (unsigned)((n + 4 * 256 - 1) / (4 * 256));
    hipLaunchKernelGGL(partial_sum_kernel, dim3(blocks), dim3(256), 0, stream, p.splits, n,
                       (const float*)part, dweight);
    KDA_LAUNCH_CHECK("weight_grad reduce");
  }
  return KDA_OK;
}
