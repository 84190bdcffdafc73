// Soft-capped cross entropy over the logits of the trainer's lm_head, fused into one read
// of the bf16 logits forward and one read + one write backward.
//
// Reference: nanochat/gpt.py:600-608 computes, under torch.compile,
//   z = softcap * tanh(float(logits[..., :vocab]) / softcap)
//   loss = cross_entropy(z, targets, ignore_index=-1)    (mean over non-ignored rows)
// which eager PyTorch runs as a chain of full-size f32 passes over an N x vocab tensor.
//
// Because |z| <= softcap, sum_j exp(z_j) <= vocab * e^softcap is finite in f32 for any
// softcap <= 60 and vocab <= 2^24, so the log-sum-exp needs no running maximum: one pass
// sums exp(z) and the backward recomputes z from the logits and the saved lse:
//   d logits_j = g * (exp(z_j - lse) - [j == t]) * (1 - (z_j / softcap)^2)
// with g = dL/dloss / (number of non-ignored rows), read from device memory so that no
// host synchronisation is needed.  Columns vocab..stride-1 (vocabulary padding) get zero
// gradient.  HBM-bound: a persistent grid of one wave per row at a time, 16-byte vector
// loads double-buffered in chunks of kCeBatch per lane, z and its factors looked up per bf16 bit
// pattern in an LDS table, row sums reduced in a fixed order (deterministic).
#include "kda_device.hpp"
#include "kda_host.hpp"

namespace kda {

constexpr int kCeThreads = 256;
constexpr int kCeBatch = 8;  // 16-byte vectors in flight per thread

// Per-element transcendentals (tanh's exp and reciprocal, then exp(z)) at a quarter of the
// VALU rate would cost more than the row's HBM read.  A bf16 logit has only 2^16 bit
// patterns, so the per-pattern values are tabulated in LDS (accurate tanhf / expf), once
// per workgroup of a persistent grid.  The table covers the binary
// exponents kTabELo .. kTabEHi, i.e. |x| in [2^-24, 2^9); a pattern outside is clamped to
// the nearest end of the range.  Below it exp(z) = 1 to within 2^-23; above it
// 1 - tanh(x / cap) <= 2 e^(-2 * 512 / 60) < 1e-7 for every cap <= 60, i.e. tanh has
// saturated to within one f32 ulp.  Inf clamps to +-(2^9 - 2).  NaN patterns (magnitude bits
// above 0x7f80) would clamp too, so the forward keeps a running packed maximum of the
// magnitude bits per lane and makes the row's sum NaN when it exceeds 0x7f80: a NaN logit
// gives a NaN row loss and lse (as tanh + library cross entropy would) and so a NaN gradient
// row in the backward.  Index: sign * kTabHalf + clamp(bits & 0x7fff) - (kTabELo << 7).
constexpr int kTabELo = 127 - 24, kTabEHi = 127 + 8;
constexpr int kTabHalf = (kTabEHi - kTabELo + 1) * 128;  // 4224 patterns per sign
constexpr int kTabSize = 2 * kTabHalf;
// workgroups per CU that the LDS tables allow: 33 KB forward, 66 KB backward
constexpr int kCeFwdPerCu = 4, kCeBwdPerCu = 2;

__device__ __forceinline__ float tab_pattern_value(int i) {
  const unsigned sign = i >= kTabHalf ? 0x8000u : 0u;
  const unsigned key = (unsigned)(i % kTabHalf) + (kTabELo << 7);
  return __uint_as_float((sign | key) << 16);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Table indices of the two bf16 patterns packed in one 32-bit word, in packed 16-bit integer
// arithmetic: clamp(bits & 0x7fff) - (kTabELo << 7) + sign * kTabHalf, both < 2^14.  The fast
// paths drop the constant - (kTabELo << 7) (tab_index2_biased) and index a table pointer
// moved back by it instead.
__device__ __forceinline__ void tab_index2_biased(unsigned w, int& lo, int& hi) {
  u16x2 k = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
  k = __builtin_elementwise_max(k, (u16x2)(kTabELo << 7));
  k = __builtin_elementwise_min(k, (u16x2)((kTabEHi << 7) | 127));
  const u16x2 sg = __builtin_bit_cast(u16x2, (w >> 15) & 0x00010001u);
  const u16x2 idx = k + sg * (u16x2)kTabHalf;  // < 17408 + 4224
  const unsigned r = __builtin_bit_cast(unsigned, idx);
  lo = (int)(r & 0xffffu);
  hi = (int)(r >> 16);
}

__device__ __forceinline__ void tab_index2(unsigned w, int& lo, int& hi) {
  tab_index2_biased(w, lo, hi);
  lo -= kTabELo << 7;
  hi -= kTabELo << 7;
}

__device__ __forceinline__ unsigned bf16_bits(bf16 v) { return (unsigned)__builtin_bit_cast(unsigned short, v); }

__device__ __forceinline__ int tab_index(unsigned bits16) {
  int lo, hi;
  tab_index2(bits16, lo, hi);
  return lo;
}

// One wave per row (rows gw, gw + waves, ...), so a row's reduction is a wave reduction and
// no barrier stalls the loads.  A row is read in chunks of kCeBatch 16-byte vectors per lane
// (kCeChunk columns); chunks are double-buffered across the wave's whole sequence of
// (row, chunk) items, so the next chunk's loads, also the next row's, are in flight while
// the current one is reduced.
//
// The forward walks the rows last to first.  It runs right after the lm_head GEMM has
// written the logits, and the last-written rows are still dirty in the memory-side cache:
// reading them first hits there, instead of evicting them (a write-back to HBM) to make room
// for the first rows (in the trainer, 159 -> 137 us per 8192 x 32768 call).  The backward
// walks first to last, so it starts on the rows the forward read last.
constexpr int kCeChunk = kWave * 8 * kCeBatch;

struct CeRows {
  long gw, nw, nch, items, last_row;
  bool reverse;
  __device__ CeRows(long rows, long cols, bool rev) : last_row(rows - 1), reverse(rev) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    gw = (long)blockIdx.x * (kCeThreads / kWave) + wave;
    nw = (long)gridDim.x * (kCeThreads / kWave);
    nch = (cols + kCeChunk - 1) / kCeChunk;
    items = gw < rows ? ((rows - 1 - gw) / nw + 1) * nch : 0;
  }
  __device__ long row(long j) const {
    const long r = gw + (j / nch) * nw;
    return reverse ? last_row - r : r;
  }
  __device__ long col0(long j) const { return (j % nch) * kCeChunk; }
};

// loads item j's chunk; columns past `last` re-read the vector at `last` (masked later)
__device__ __forceinline__ void ce_load(const CeRows& it, long j, const bf16* __restrict__ base,
                                        long stride, long last, bf16x8* x) {
  const bf16* p = base + it.row(j) * stride;
  const long c0 = it.col0(j) + (threadIdx.x % kWave) * 8;
#pragma unroll
  for (int b = 0; b < kCeBatch; ++b) {
    const long c = c0 + b * kWave * 8;
    x[b] = *reinterpret_cast<const bf16x8*>(p + (c < last ? c : last));
  }
}

__global__ __launch_bounds__(kCeThreads) void softcap_ce_fwd_kernel(
    long rows, int vocab, long stride, float cap, const bf16* __restrict__ logits,
    const int64_t* __restrict__ targets, int64_t ignore_index, float* __restrict__ loss_row,
    float* __restrict__ lse_row) {
  __shared__ float tab[kTabSize];
  for (int i = threadIdx.x; i < kTabSize; i += kCeThreads)
    tab[i] = expf(cap * tanhf(tab_pattern_value(i) / cap));
  __syncthreads();
  const CeRows it(rows, vocab, true);
  const float* tabz = tab - (kTabELo << 7);
  const long last = ((vocab - 1) / 8) * 8;  // last vector start that holds a vocabulary column
  const int lane = threadIdx.x % kWave;
  float sum = 0.f;
  u16x2 mag = (u16x2)0;  // running maximum of the magnitude bits (NaN detection)
  auto consume = [&](long j, const bf16x8* x) {
    const int c0 = (int)it.col0(j) + lane * 8;
    if ((int)it.col0(j) + kCeChunk <= vocab) {  // whole chunk inside the vocabulary (uniform)
#pragma unroll
      for (int b = 0; b < kCeBatch; ++b) {
        const uint4 w = __builtin_bit_cast(uint4, x[b]);
        const unsigned ws[4] = {w.x, w.y, w.z, w.w};
        float sb = 0.f;  // per-vector partial: short dependent-add chains
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          int i0, i1;
          tab_index2_biased(ws[e], i0, i1);
          mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2, ws[e] & 0x7fff7fffu));
          sb += tabz[i0] + tabz[i1];
        }
        sum += sb;
      }
    } else {
#pragma unroll
      for (int b = 0; b < kCeBatch; ++b) {
        const int c = c0 + b * kWave * 8;
        float sb = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const unsigned bits = bf16_bits(x[b][e]);
          const float ez = tab[tab_index(bits)];
          sb += (c + e < vocab) ? ez : 0.f;
          if (c + e < vocab && (bits & 0x7fffu) > 0x7f80u) mag = (u16x2)0xffff;
        }
        sum += sb;
      }
    }
    if (j % it.nch == it.nch - 1) {
      const bool nan_here = mag.x > 0x7f80 || mag.y > 0x7f80;
      const float tot = wave_sum(nan_here ? __builtin_nanf("") : sum);
      sum = 0.f;
      mag = (u16x2)0;
      if (lane == 0) {
        const long row = it.row(j);
        const int64_t t = targets[row];
        const float lse = __logf(tot);
        float loss;
        if (t == ignore_index) {
          loss = 0.f;
        } else if (t < 0 || t >= vocab) {
          loss = __builtin_nanf("");  // out-of-range target: poison the mean
        } else {
          loss = lse - cap * tanhf((float)logits[row * stride + t] / cap);
        }
        loss_row[row] = loss;
        lse_row[row] = lse;
      }
    }
  };
  bf16x8 xa[kCeBatch], xb[kCeBatch];
  if (it.items > 0) ce_load(it, 0, logits, stride, last, xa);
  for (long j = 0; j < it.items; j += 2) {
    if (j + 1 < it.items) ce_load(it, j + 1, logits, stride, last, xb);
    consume(j, xa);
    if (j + 1 >= it.items) break;
    if (j + 2 < it.items) ce_load(it, j + 2, logits, stride, last, xa);
    consume(j + 1, xb);
  }
}

// backward table: (exp(z), 1 - tanh^2) per pattern
__global__ __launch_bounds__(kCeThreads) void softcap_ce_bwd_kernel(
    long rows, int vocab, long stride, float cap, const bf16* __restrict__ logits,
    const int64_t* __restrict__ targets, int64_t ignore_index, const float* __restrict__ lse_row,
    const float* __restrict__ grad_scale, bf16* __restrict__ grad) {
  __shared__ float2 tab[kTabSize];
  for (int i = threadIdx.x; i < kTabSize; i += kCeThreads) {
    const float th = tanhf(tab_pattern_value(i) / cap);
    tab[i] = make_float2(expf(cap * th), 1.0f - th * th);
  }
  __syncthreads();
  const CeRows it(rows, stride, false);
  const float2* tabz = tab - (kTabELo << 7);
  const float gs = *grad_scale;
  const int lane = threadIdx.x % kWave;
  float g = 0.f, einv = 0.f, ge = 0.f;
  int tc = -1;
  auto consume = [&](long j, const bf16x8* x) {
    const long row = it.row(j);
    if (j % it.nch == 0) {
      const int64_t t = targets[row];
      g = (t == ignore_index) ? 0.f : gs;
      einv = __expf(-lse_row[row]);
      tc = (t >= 0 && t < vocab) ? (int)t : -1;
      ge = g * einv;
    }
    bf16* q = grad + row * stride;
    const int c0 = (int)it.col0(j) + lane * 8;
    const bool full = (int)it.col0(j) + kCeChunk <= vocab;  // uniform over the wave
#pragma unroll
    for (int b = 0; b < kCeBatch; ++b) {
      const int c = c0 + b * kWave * 8;
      bf16x8 y;
      if (full && (unsigned)(tc - c) >= 8u) {  // no padding column, no target column
        const uint4 w = __builtin_bit_cast(uint4, x[b]);
        const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          int i0, i1;
          tab_index2_biased(ws[e], i0, i1);
          const float2 v0 = tabz[i0], v1 = tabz[i1];
          y[2 * e] = to_bf16(v0.x * ge * v0.y);
          y[2 * e + 1] = to_bf16(v1.x * ge * v1.y);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float2 v = tab[tab_index(bf16_bits(x[b][e]))];
          const float d = g * (v.x * einv - (c + e == tc ? 1.0f : 0.0f)) * v.y;
          y[e] = to_bf16(c + e < vocab ? d : 0.f);
        }
      }
      if (c < stride) *reinterpret_cast<bf16x8*>(q + c) = y;
    }
  };
  bf16x8 xa[kCeBatch], xb[kCeBatch];
  if (it.items > 0) ce_load(it, 0, logits, stride, stride - 8, xa);
  for (long j = 0; j < it.items; j += 2) {
    if (j + 1 < it.items) ce_load(it, j + 1, logits, stride, stride - 8, xb);
    consume(j, xa);
    if (j + 1 >= it.items) break;
    if (j + 2 < it.items) ce_load(it, j + 2, logits, stride, stride - 8, xa);
    consume(j + 1, xb);
  }
}

// Forward and backward in one pass for rows of 4096 NV columns, all of them vocabulary
// (NV <= 8: up to 32768; other shapes take the two-kernel path): one 512-thread workgroup
// per row at a time holds the whole row in registers (NV 16-byte vectors per thread, the
// next row's already in flight), sums exp(z) over the row (waves, then eight partials
// through LDS in a fixed order), and from the same registers writes the gradient for the
// expected upstream gradient (*grad_scale = expected dL/dmean / count).  The logits are read
// once instead of twice; the backward only has to confirm the scale.  Row loss, lse and
// gradient use the forward's and the backward's formulas (the row sum is taken in another
// order, so they agree with the two-kernel path to rounding, not bit for bit).  The body is
// free of per-lane branches (their exec masks spilled the scalar registers): the one thread
// holding the target column reads its logit and afterwards re-stores its vector with the
// target's term.
constexpr int kCeFusedThreads = 512;               // 8 waves per row
constexpr int kCeFusedCols = kCeFusedThreads * 8;  // columns per 16-byte vector pass of a workgroup
constexpr int kCeFusedMaxVec = 8;                  // rows up to 32768 columns (two rows in registers)
constexpr int kCeFusedPerCu = 1;                   // 66 KB table, 8 waves per workgroup

template <int NV>
__global__ __launch_bounds__(kCeFusedThreads) void softcap_ce_fused_kernel(
    long rows, int vocab, float cap, const bf16* __restrict__ logits, const int64_t* __restrict__ targets,
    int64_t ignore_index, const float* __restrict__ grad_scale, float* __restrict__ loss_row,
    float* __restrict__ lse_row, bf16* __restrict__ grad) {
  __shared__ float2 tab[kTabSize];
  __shared__ float s_part[2][kCeFusedThreads / kWave];
  __shared__ float s_zt[2];
  for (int i = threadIdx.x; i < kTabSize; i += kCeFusedThreads) {
    const float th = tanhf(tab_pattern_value(i) / cap);
    tab[i] = make_float2(expf(cap * th), 1.0f - th * th);
  }
  __syncthreads();
  const float2* tabz = tab - (kTabELo << 7);
  const float gs = *grad_scale;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const long G = gridDim.x;
  constexpr long kRow = (long)NV * kCeFusedCols;  // = vocab = row stride
  auto load = [&](long r, bf16x8* x) {
    const bf16* p = logits + r * kRow + tid * 8;
#pragma unroll
    for (int v = 0; v < NV; ++v) x[v] = *reinterpret_cast<const bf16x8*>(p + v * kCeFusedCols);
  };
  auto process = [&](long r, const bf16x8* x, int64_t t, int slot) {
    const bool ign = t == ignore_index, in_range = t >= 0 && t < vocab;
    const int tc = in_range ? (int)t : -1;
    const bool owner = in_range && (tc % kCeFusedCols) / 8 == tid;  // holds the target column
    const int vt = tc / kCeFusedCols, et = tc % 8;
    // the row sum of exp(z) (NaN if a logit is NaN)
    float sum = 0.f;
    u16x2 mag = (u16x2)0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const uint4 w = __builtin_bit_cast(uint4, x[v]);
      const unsigned ws[4] = {w.x, w.y, w.z, w.w};
      float sb = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int i0, i1;
        tab_index2_biased(ws[e], i0, i1);
        mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2, ws[e] & 0x7fff7fffu));
        sb += tabz[i0].x + tabz[i1].x;
      }
      sum += sb;
    }
    if (owner) {
      float raw = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e) raw = (v == vt && e == et) ? (float)x[v][e] : raw;
      s_zt[slot] = cap * tanhf(raw / cap);
    }
    const bool nan_here = mag.x > 0x7f80 || mag.y > 0x7f80;
    const float wsum = wave_sum(nan_here ? __builtin_nanf("") : sum);
    if (lane == 0) s_part[slot][wave] = wsum;
    wait_lgkm0();
    ring_barrier();  // the partials (and the target's z) are in LDS; loads stay in flight
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kCeFusedThreads / kWave; ++w) tot += s_part[slot][w];
    const float lse = __logf(tot);
    if (tid == 0) {
      loss_row[r] = ign ? 0.f : (in_range ? lse - s_zt[slot] : __builtin_nanf(""));
      lse_row[r] = lse;
    }
    // the gradient, as the backward kernel forms it
    const float g = ign ? 0.f : gs;
    const float einv = __expf(-lse);
    const float ge = g * einv;
    bf16* q = grad + r * kRow + tid * 8;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const uint4 w = __builtin_bit_cast(uint4, x[v]);
      const unsigned ws[4] = {w.x, w.y, w.z, w.w};
      bf16x8 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int i0, i1;
        tab_index2_biased(ws[e], i0, i1);
        const float2 v0 = tabz[i0], v1 = tabz[i1];
        y[2 * e] = to_bf16(v0.x * ge * v0.y);
        y[2 * e + 1] = to_bf16(v1.x * ge * v1.y);
      }
      *reinterpret_cast<bf16x8*>(q + v * kCeFusedCols) = y;
    }
    if (owner) {  // the target's vector again, every element in the backward's general form
#pragma unroll
      for (int v = 0; v < NV; ++v)
        if (v == vt) {
          bf16x8 y;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float2 vv = tab[tab_index(bf16_bits(x[v][e]))];
            y[e] = to_bf16(g * (vv.x * einv - (e == et ? 1.0f : 0.0f)) * vv.y);
          }
          *reinterpret_cast<bf16x8*>(q + v * kCeFusedCols) = y;
        }
    }
  };
  // rows blockIdx.x, + G, ...; two register buffers, the next row's loads issued before the
  // current row is processed; the LDS slots alternate so one barrier per row suffices
  bf16x8 xa[NV], xb[NV];
  long r = blockIdx.x;
  int64_t ta = 0, tb = 0;
  if (r < rows) {
    load(r, xa);
    ta = targets[r];
  }
  for (; r < rows; r += 2 * G) {
    const long r1 = r + G;
    if (r1 < rows) {
      load(r1, xb);
      tb = targets[r1];
    }
    process(r, xa, ta, 0);
    if (r1 >= rows) break;
    const long r2 = r1 + G;
    if (r2 < rows) {
      load(r2, xa);
      ta = targets[r2];
    }
    process(r1, xb, tb, 1);
  }
}

// Non-ignored target count and the gradient scale the fused kernel assumes:
// count = #(t != ignore_index), grad_scale = expected / count (one workgroup, fixed order).
__global__ __launch_bounds__(1024) void softcap_ce_count_kernel(long rows, const int64_t* __restrict__ targets,
                                                                int64_t ignore_index, float expected,
                                                                float* __restrict__ count,
                                                                float* __restrict__ grad_scale) {
  __shared__ long long red[1024 / kWave];
  long long c = 0;
  for (long r = threadIdx.x; r < rows; r += 1024) c += targets[r] != ignore_index ? 1 : 0;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) c += __shfl_xor(c, o);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    long long tc = 0;
    for (int w = 0; w < 1024 / kWave; ++w) tc += red[w];
    *count = (float)tc;
    *grad_scale = expected / (float)tc;
  }
}

// data *= actual / expected, unless *actual == expected (then nothing is touched): the
// backward of the fused cross entropy when the upstream gradient is not the one assumed.
__global__ __launch_bounds__(256) void bf16_rescale_kernel(long n8, bf16* __restrict__ data,
                                                           const float* __restrict__ actual, float expected) {
  const float a = *actual;
  if (a == expected) return;
  const float f = a / expected;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n8; i += (long)gridDim.x * 256) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(data + i * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = to_bf16((float)v[e] * f);
    *reinterpret_cast<bf16x8*>(data + i * 8) = v;
  }
}

static unsigned ce_grid(int64_t rows, int per_cu) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const long g = (long)cus * per_cu;
  const long need = (rows + kCeThreads / kWave - 1) / (kCeThreads / kWave);
  return (unsigned)(need < g ? need : g);
}

}  // namespace kda

static int check_ce_args(int64_t rows, int32_t vocab, int64_t stride, float softcap,
                         const void* logits, const void* targets) {
  KDA_REQUIRE(rows >= 0 && rows <= 0x7fffffff, "softcap_cross_entropy: invalid row count");
  KDA_REQUIRE(vocab > 0 && vocab <= (1 << 24), "softcap_cross_entropy: vocab must be in [1, 2^24]");
  KDA_REQUIRE(stride >= vocab && stride % 8 == 0 && stride <= (1 << 30),
              "softcap_cross_entropy: row stride must be >= vocab, a multiple of 8 and <= 2^30");
  KDA_REQUIRE(softcap > 0.f && softcap <= 60.f, "softcap_cross_entropy: softcap must be in (0, 60]");
  KDA_REQUIRE(logits && targets, "softcap_cross_entropy: null pointer");
  KDA_REQUIRE(kda::aligned16(logits), "softcap_cross_entropy: logits must be 16-byte aligned");
  return KDA_OK;
}

extern "C" int kda_softcap_cross_entropy_forward(int64_t rows, int32_t vocab, int64_t stride,
                                                 float softcap, const void* logits,
                                                 const int64_t* targets, int64_t ignore_index,
                                                 float* loss_rows, float* lse_rows,
                                                 hipStream_t stream) {
  using namespace kda;
  int rc = check_ce_args(rows, vocab, stride, softcap, logits, targets);
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(loss_rows && lse_rows, "softcap_cross_entropy_forward: null output");
  if (rows == 0) return KDA_OK;
  hipLaunchKernelGGL(softcap_ce_fwd_kernel, dim3(ce_grid(rows, kCeFwdPerCu)), dim3(kCeThreads), 0, stream, (long)rows, vocab,
                     (long)stride, softcap, (const bf16*)logits, targets, ignore_index, loss_rows,
                     lse_rows);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_forward");
  return KDA_OK;
}

extern "C" int kda_softcap_cross_entropy_backward(int64_t rows, int32_t vocab, int64_t stride,
                                                  float softcap, const void* logits,
                                                  const int64_t* targets, int64_t ignore_index,
                                                  const float* lse_rows, const float* grad_scale,
                                                  void* grad_logits, hipStream_t stream) {
  using namespace kda;
  int rc = check_ce_args(rows, vocab, stride, softcap, logits, targets);
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(lse_rows && grad_scale && grad_logits, "softcap_cross_entropy_backward: null pointer");
  KDA_REQUIRE(aligned16(grad_logits), "softcap_cross_entropy_backward: grad must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  hipLaunchKernelGGL(softcap_ce_bwd_kernel, dim3(ce_grid(rows, kCeBwdPerCu)), dim3(kCeThreads), 0, stream, (long)rows, vocab,
                     (long)stride, softcap, (const bf16*)logits, targets, ignore_index, lse_rows,
                     grad_scale, (bf16*)grad_logits);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_backward");
  return KDA_OK;
}

extern "C" int kda_softcap_cross_entropy_fused_supported(int32_t vocab, int64_t stride) {
  return vocab > 0 && (int64_t)vocab == stride && stride % kda::kCeFusedCols == 0 &&
         stride <= (int64_t)kda::kCeFusedCols * kda::kCeFusedMaxVec;
}

extern "C" int kda_softcap_cross_entropy_fused(int64_t rows, int32_t vocab, int64_t stride, float softcap,
                                               const void* logits, const int64_t* targets,
                                               int64_t ignore_index, const float* grad_scale,
                                               float* loss_rows, float* lse_rows, void* grad_logits,
                                               hipStream_t stream) {
  using namespace kda;
  int rc = check_ce_args(rows, vocab, stride, softcap, logits, targets);
  if (rc != KDA_OK) return rc;
  KDA_REQUIRE(kda_softcap_cross_entropy_fused_supported(vocab, stride),
              "softcap_cross_entropy_fused: needs vocab == stride, a multiple of %d and at most %d",
              kCeFusedCols, kCeFusedCols * kCeFusedMaxVec);
  KDA_REQUIRE(grad_scale && loss_rows && lse_rows && grad_logits, "softcap_cross_entropy_fused: null pointer");
  KDA_REQUIRE(aligned16(grad_logits), "softcap_cross_entropy_fused: grad must be 16-byte aligned");
  if (rows == 0) return KDA_OK;
  // one workgroup per CU (at most one per row)
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const unsigned grid = (unsigned)(rows < (long)cus * kCeFusedPerCu ? rows : (long)cus * kCeFusedPerCu);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kCeFusedThreads), 0, stream, (long)rows, vocab, softcap,
                       (const bf16*)logits, targets, ignore_index, grad_scale, loss_rows, lse_rows,
                       (bf16*)grad_logits);
  };
  switch (stride / kCeFusedCols) {
    case 1: launch(softcap_ce_fused_kernel<1>); break;
    case 2: launch(softcap_ce_fused_kernel<2>); break;
    case 3: launch(softcap_ce_fused_kernel<3>); break;
    case 4: launch(softcap_ce_fused_kernel<4>); break;
    case 5: launch(softcap_ce_fused_kernel<5>); break;
    case 6: launch(softcap_ce_fused_kernel<6>); break;
    case 7: launch(softcap_ce_fused_kernel<7>); break;
    default: launch(softcap_ce_fused_kernel<8>); break;
  }
  KDA_LAUNCH_CHECK("softcap_cross_entropy_fused");
  return KDA_OK;
}

extern "C" int kda_softcap_cross_entropy_count(int64_t rows, const int64_t* targets, int64_t ignore_index,
                                               float expected_grad, float* count, float* grad_scale,
                                               hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0, "softcap_cross_entropy_count: negative row count");
  KDA_REQUIRE(count && grad_scale && (rows == 0 || targets), "softcap_cross_entropy_count: null pointer");
  hipLaunchKernelGGL(softcap_ce_count_kernel, dim3(1), dim3(1024), 0, stream, (long)rows, targets, ignore_index,
                     expected_grad, count, grad_scale);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_count");
  return KDA_OK;
}

extern "C" int kda_bf16_rescale_if_changed(int64_t n, void* data, const float* actual, float expected,
                                           hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(n >= 0 && n % 8 == 0, "bf16_rescale_if_changed: n must be a non-negative multiple of 8");
  KDA_REQUIRE(actual && (n == 0 || data), "bf16_rescale_if_changed: null pointer");
  KDA_REQUIRE(expected != 0.f, "bf16_rescale_if_changed: expected must be nonzero");
  KDA_REQUIRE(aligned16(data), "bf16_rescale_if_changed: data must be 16-byte aligned");
  if (n == 0) return KDA_OK;
  const long n8 = n / 8;
  const long blocks = (n8 + 255) / 256;
  hipLaunchKernelGGL(bf16_rescale_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, stream,
                     n8, (bf16*)data, actual, expected);
  KDA_LAUNCH_CHECK("bf16_rescale_if_changed");
  return KDA_OK;
}

namespace kda {

// Mean of the row losses over the rows whose target is not ignore_index, and that count,
// in one workgroup with a fixed summation order (thread t sums rows t, t + 1024, ...; then
// a fixed tree).  The count is kept in integers (exact for every row count the forward
// accepts) and converted once for the division.  Keeps the loss reduction inside the library: a multi-block library
// reduction would record memory-set nodes when captured in a HIP graph.
constexpr int kMeanThreads = 1024;

__global__ __launch_bounds__(kMeanThreads) void softcap_ce_mean_kernel(
    long rows, const float* __restrict__ loss_row, const int64_t* __restrict__ targets,
    int64_t ignore_index, float* __restrict__ loss, float* __restrict__ count) {
  __shared__ float red_s[kMeanThreads / kWave];
  __shared__ long long red_c[kMeanThreads];
  float s = 0.f;
  long long c = 0;
  for (long r = threadIdx.x; r < rows; r += kMeanThreads) {
    const bool valid = targets[r] != ignore_index;
    s += valid ? loss_row[r] : 0.f;
    c += valid ? 1 : 0;
  }
  s = wave_sum(s);
  red_c[threadIdx.x] = c;
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) red_s[wave] = s;
  __syncthreads();
  if (threadIdx.x < 32) {  // 32 partial counts of 32 threads each, then one sum of those
    long long p = 0;
    for (int t = 0; t < 32; ++t) p += red_c[threadIdx.x * 32 + t];
    red_c[threadIdx.x * 32] = p;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float ts = 0.f;
    long long tc = 0;
    for (int w = 0; w < kMeanThreads / kWave; ++w) ts += red_s[w];
    for (int t = 0; t < 32; ++t) tc += red_c[t * 32];
    *loss = ts / (float)tc;  // NaN when every row is ignored, as the library cross entropy
    *count = (float)tc;
  }
}

}  // namespace kda

extern "C" int kda_softcap_cross_entropy_mean(int64_t rows, const float* loss_rows, const int64_t* targets,
                                              int64_t ignore_index, float* loss, float* count,
                                              hipStream_t stream) {
  using namespace kda;
  KDA_REQUIRE(rows >= 0, "softcap_cross_entropy_mean: negative row count");
  KDA_REQUIRE(loss && count && (rows == 0 || (loss_rows && targets)),
              "softcap_cross_entropy_mean: null pointer");
  hipLaunchKernelGGL(softcap_ce_mean_kernel, dim3(1), dim3(kMeanThreads), 0, stream, (long)rows, loss_rows,
                     targets, ignore_index, loss, count);
  KDA_LAUNCH_CHECK("softcap_cross_entropy_mean");
  return KDA_OK;
}
