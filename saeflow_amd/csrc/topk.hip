// Row-wise top-k on gfx950 for the TopK SAE: values sorted descending, int32 indices.
// Reference semantics: ops._topk (saeflow/ops.py:12-16), i.e. f.topk(k, dim=-1) of the
// dense ReLU output.
//
// One 256-thread block per row, radix select on order-preserving keys:
//  1. 8-bit digit histograms in LDS, most significant digit first (2 passes for 16-bit
//     values, 4 for fp32), narrow the k-th largest key to one exact value T and the
//     number `need` of elements equal to T that belong to the top k;
//  2. elements with key > T are gathered into LDS;
//  3. elements equal to T: if exactly `need` exist they are all taken, otherwise the
//     `need` lowest column indices are taken by an in-order block scan (deterministic);
//  4. a bitonic sort of the k (key, column) pairs orders them by value descending and
//     column ascending.
// Keys order values as f.topk compares them: -0.0 and +0.0 are equal, every NaN (either
// sign) ranks above +inf and all NaNs are equal; equal values go by increasing column. The
// values written are re-read from f at the selected columns, so their bits are the input's.
// Rows of 16-B aligned chunks (topk_vec_kernel) are read with 16-B loads, and a row of up
// to 48 KB is read from global memory once and from an LDS copy in every later pass.
// Histogram increments are aggregated per wave when the lanes agree on a bin: a ReLU row is
// mostly zeros, whose keys all fall in one bin and would otherwise serialise on one LDS
// counter. Ties at the cut are then taken in column order by rounds of whole chunks with a
// block prefix (one barrier per round). Rows of other strides take topk_kernel.
#include "common.h"

namespace {

constexpr int NT = 256;
constexpr int KMAX = 1024;

// Output row of input row `row`. Plain calls (n_live NULL) write row `row`. The gathered form
// (sf_topk_gather) takes the input rows i < clamp(*n_live - off, 0, M) and writes row i to output
// row rows[off + i]; other rows, and targets outside [0, m_out), do nothing (returns -1). Every
// thread of a block gets the same answer, so a block returns as a whole before any barrier.
struct RowMap {
  const int32_t* n_live;
  int64_t off;
  const int32_t* rows;
  int64_t m_out;
};
__device__ __forceinline__ int64_t out_row(const RowMap& r, int64_t row, int64_t M) {
  if (r.n_live == nullptr) return row;
  int64_t live = (int64_t)*r.n_live - r.off;
  live = live < 0 ? 0 : (live > M ? M : live);
  if (row >= live) return -1;
  const int64_t o = r.rows[r.off + row];
  return o >= 0 && o < r.m_out ? o : -1;
}

// Selection keys: unsigned order of keys = f.topk's order of values. nanmag is the smallest
// 16-bit NaN magnitude minus one (0x7f80 for bf16, 0x7c00 for fp16): magnitudes above it are NaN.
__device__ __forceinline__ uint32_t topk_key16(uint32_t b, uint32_t nanmag) {
  const uint32_t mag = b & 0x7fffu;
  if (mag == 0) return 0x8000u;       // -0.0 ranks with +0.0
  if (mag > nanmag) return 0xffffu;   // any NaN above +inf
  return float_key16(b);
}
__device__ __forceinline__ uint32_t topk_key32(uint32_t b) {
  const uint32_t mag = b & 0x7fffffffu;
  if (mag == 0) return 0x80000000u;
  if (mag > 0x7f800000u) return 0xffffffffu;
  return float_key32(b);
}

__device__ __forceinline__ uint32_t load_key(const char* rp, int64_t i, int64_t sfn, int es, uint32_t nanmag) {
  if (es == 2) return topk_key16(*(const u16*)(rp + i * sfn * 2), nanmag);
  return topk_key32(*(const uint32_t*)(rp + i * sfn * 4));
}

// value bits of element i of a row (written out for a selected column)
__device__ __forceinline__ void copy_value(const char* rp, int64_t col, int64_t sfn, int es, char* values, int64_t o) {
  if (es == 2) ((u16*)values)[o] = *(const u16*)(rp + col * sfn * 2);
  else ((uint32_t*)values)[o] = *(const uint32_t*)(rp + col * sfn * 4);
}

__global__ __launch_bounds__(NT) void topk_kernel(const char* f, int64_t sfm, int64_t sfn, int es, uint32_t nanmag,
                                                  int64_t M, int64_t N, int k, char* values, int32_t* indices,
                                                  RowMap map) {
  __shared__ uint32_t hist[256];
  __shared__ uint64_t s_sel[KMAX];  // (key << 32) | ~column, sorted descending
  __shared__ uint32_t s_prefix, s_need, s_eqcount, s_gt, s_eq;
  __shared__ int s_wtot[NT / 64];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = blockIdx.x;
  const int64_t orow = out_row(map, row, M);
  if (orow < 0) return;
  const char* rp = f + row * sfm * es;
  const int nbits = es * 8;

  // ---- 1. radix select of the k-th largest key
  uint32_t prefix = 0, mask = 0, need = (uint32_t)k;
  for (int shift = nbits - 8; shift >= 0; shift -= 8) {
    hist[t] = 0;
    __syncthreads();
    for (int64_t i = t; i < N; i += NT) {
      const uint32_t key = load_key(rp, i, sfn, es, nanmag);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (t == 0) {
      uint32_t cum = 0;
      int sel = 0;
      for (int d = 255; d >= 0; --d) {
        if (cum + hist[d] >= need) {
          sel = d;
          break;
        }
        cum += hist[d];
      }
      s_prefix = prefix | ((uint32_t)sel << shift);
      s_need = need - cum;
      s_eqcount = hist[sel];
    }
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    mask |= 255u << shift;
  }
  const uint32_t T = prefix;
  const uint32_t ngt = (uint32_t)k - need;  // elements strictly above T
  const uint32_t neq_total = s_eqcount;      // elements equal to T

  // ---- 2./3. gather
  if (t == 0) {
    s_gt = 0;
    s_eq = 0;
  }
  __syncthreads();
  const bool all_eq = neq_total == need;
  for (int64_t i = t; i < N; i += NT) {
    const uint32_t key = load_key(rp, i, sfn, es, nanmag);
    if (key > T) {
      uint32_t slot = atomicAdd(&s_gt, 1u);
      if (slot < ngt) s_sel[slot] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
    } else if (all_eq && key == T) {
      uint32_t slot = atomicAdd(&s_eq, 1u);
      if (slot < need) s_sel[ngt + slot] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
    }
  }
  if (!all_eq) {
    // in-order: the `need` equal elements with the lowest columns
    uint32_t base = 0;
    for (int64_t i0 = 0; i0 < N && base < need; i0 += NT) {
      int64_t i = i0 + t;
      bool eq = false;
      if (i < N) {
        eq = load_key(rp, i, sfn, es, nanmag) == T;
      }
      uint64_t bal = __ballot(eq);
      if (lane == 0) s_wtot[w] = __popcll(bal);
      __syncthreads();
      uint32_t before = 0, tot = 0;
      for (int q = 0; q < NT / 64; ++q) {
        if (q < w) before += s_wtot[q];
        tot += s_wtot[q];
      }
      if (eq) {
        uint32_t slot = base + before + __popcll(bal & ((1ull << lane) - 1ull));
        if (slot < need) s_sel[ngt + slot] = ((uint64_t)T << 32) | (uint32_t)~(uint32_t)i;
      }
      base += tot;
      __syncthreads();
    }
  }
  __syncthreads();

  // ---- 4. bitonic sort (descending) of the k selected pairs, padded to a power of two
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = k + t; i < P; i += NT) s_sel[i] = 0;
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < P / 2; i += NT) {
        int lo = 2 * i - (i & (stride - 1));
        int hi = lo + stride;
        bool desc = (lo & size) == 0;
        uint64_t a = s_sel[lo], b = s_sel[hi];
        if (desc ? (a < b) : (a > b)) {
          s_sel[lo] = b;
          s_sel[hi] = a;
        }
      }
      __syncthreads();
    }
  }

  // ---- write: the selected columns and their values
  for (int i = t; i < k; i += NT) {
    const uint32_t col = ~(uint32_t)s_sel[i];
    const int64_t o = orow * (int64_t)k + i;
    indices[o] = (int32_t)col;
    copy_value(rp, col, sfn, es, values, o);
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int64_t LDS_ROW_MAX = 48 * 1024;  // rows up to this many bytes are cached in LDS

template <int ES>
__device__ __forceinline__ uint32_t chunk_key(const u32x4& c, int e, uint32_t nanmag) {
  if constexpr (ES == 2) return topk_key16((c[e >> 1] >> ((e & 1) * 16)) & 0xffffu, nanmag);
  else return topk_key32(c[e]);
}

// hist[bin] += 1 for every lane with `valid`. The lanes whose bin equals the first valid
// lane's bin are added with one atomic by that lane. Called by all lanes of the wave.
__device__ __forceinline__ void hist_add(uint32_t* hist, bool valid, uint32_t bin, int lane) {
  const uint64_t vm = __ballot(valid);
  if (vm == 0) return;  // wave-uniform
  const int l0 = __builtin_ctzll(vm);
  const uint32_t ref = __builtin_amdgcn_readlane(bin, l0);
  const bool same = valid && bin == ref;
  const uint64_t sm = __ballot(same);
  if (lane == l0) atomicAdd(&hist[ref], (uint32_t)__popcll(sm));
  if (valid && !same) atomicAdd(&hist[bin], 1u);
}

// One wave picks the digit of the k-th largest key from a 256-bin histogram: the highest bin
// d whose count from the top, sum of hist[d..255], reaches `need`. Lane l holds bins
// 255-4l .. 252-4l; an inclusive wave scan of the lane totals gives each lane the count
// above its bins, and the lane where the running count crosses `need` writes the result.
__device__ __forceinline__ void select_bin(const uint32_t* hist, uint32_t need, int lane, uint32_t prefix, int shift,
                                           uint32_t& s_prefix, uint32_t& s_need, uint32_t& s_eqcount,
                                           uint32_t& s_gt, uint32_t& s_eq) {
  uint32_t h[4], own = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = hist[255 - 4 * lane - i];
    own += h[i];
  }
  uint32_t incl = own;  // inclusive prefix over lanes 0..lane
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  uint32_t cum = incl - own;  // keys in bins above this lane's
  const uint64_t crossing = __ballot(cum < need && incl >= need);
  if (lane == __builtin_ctzll(crossing)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (cum + h[i] >= need) {
        const int d = 255 - 4 * lane - i;
        s_prefix = prefix | ((uint32_t)d << shift);
        s_need = need - cum;
        s_eqcount = h[i];
        s_gt = 0;
        s_eq = 0;
        break;
      }
      cum += h[i];
    }
  }
}

template <int ES, bool CACHED>
__global__ __launch_bounds__(NT) void topk_vec_kernel(const char* f, int64_t sfm, uint32_t nanmag, int64_t M,
                                                      int64_t N, int k, char* values, int32_t* indices, RowMap map) {
  extern __shared__ __attribute__((aligned(16))) char s_row[];  // CACHED: the row's whole chunks
  __shared__ uint32_t hist[256];
  __shared__ uint64_t s_sel[KMAX];  // (key << 32) | ~column
  __shared__ uint32_t s_prefix, s_need, s_eqcount, s_gt, s_eq;
  __shared__ int s_wtot[2][NT / 64];
  constexpr int EPC = 16 / ES, NBITS = ES * 8;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = blockIdx.x;
  const int64_t orow = out_row(map, row, M);
  if (orow < 0) return;
  const char* rp = f + row * sfm * ES;
  const int64_t nch = N / EPC;          // whole 16-B chunks
  const int ntail = (int)(N - nch * EPC);  // trailing elements, fewer than EPC
  auto tail_key = [&](int i) -> uint32_t {
    const char* p = rp + (nch * EPC + i) * ES;
    return ES == 2 ? topk_key16(*(const u16*)p, nanmag) : topk_key32(*(const uint32_t*)p);
  };
  // chunk c of the row; the first pass reads global memory (and fills the LDS copy)
  auto chunk = [&](int64_t c, bool first) -> u32x4 {
    if (CACHED && !first) return *(const u32x4*)(s_row + c * 16);
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)(rp + c * 16));
    if (CACHED) *(u32x4*)(s_row + c * 16) = v;
    return v;
  };

  // ---- 1. radix select of the k-th largest key, 8 bits per pass
  uint32_t prefix = 0, mask = 0, need = (uint32_t)k;
  for (int shift = NBITS - 8; shift >= 0; shift -= 8) {
    const bool first = shift == NBITS - 8;
    hist[t] = 0;
    __syncthreads();
    for (int64_t c0 = 0; c0 < nch; c0 += NT) {
      const int64_t c = c0 + t;
      const bool in = c < nch;
      const u32x4 v = in ? chunk(c, first) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const uint32_t key = chunk_key<ES>(v, e, nanmag);
        hist_add(hist, in && (key & mask) == prefix, (key >> shift) & 255u, lane);
      }
    }
    if (t < ntail) {
      const uint32_t key = tail_key(t);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (w == 0) select_bin(hist, need, lane, prefix, shift, s_prefix, s_need, s_eqcount, s_gt, s_eq);
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    mask |= 255u << shift;
  }
  const uint32_t T = prefix;
  const uint32_t ngt = (uint32_t)k - need;  // elements strictly above T, all taken
  const bool all_eq = s_eqcount == need;    // every element equal to T is taken

  // ---- 2. elements above T (and all equal ones when all_eq): at most k, in any order
  for (int64_t c0 = 0; c0 < nch; c0 += NT) {
    const int64_t c = c0 + t;
    if (c >= nch) break;
    const u32x4 v = chunk(c, false);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const uint32_t key = chunk_key<ES>(v, e, nanmag);
      const uint32_t col = (uint32_t)(c * EPC + e);
      if (key > T) {
        const uint32_t slot = atomicAdd(&s_gt, 1u);
        if (slot < ngt) s_sel[slot] = ((uint64_t)key << 32) | (uint32_t)~col;
      } else if (all_eq && key == T) {
        const uint32_t slot = atomicAdd(&s_eq, 1u);
        if (slot < need) s_sel[ngt + slot] = ((uint64_t)key << 32) | (uint32_t)~col;
      }
    }
  }
  if (t < ntail) {
    const uint32_t key = tail_key(t), col = (uint32_t)(nch * EPC + t);
    if (key > T) {
      const uint32_t slot = atomicAdd(&s_gt, 1u);
      if (slot < ngt) s_sel[slot] = ((uint64_t)key << 32) | (uint32_t)~col;
    } else if (all_eq && key == T) {
      const uint32_t slot = atomicAdd(&s_eq, 1u);
      if (slot < need) s_sel[ngt + slot] = ((uint64_t)key << 32) | (uint32_t)~col;
    }
  }

  // ---- 3. otherwise the `need` elements equal to T with the lowest columns, in rounds of
  // NT chunks: thread t's chunk precedes thread t+1's, and its elements are in column order
  if (!all_eq) {
    uint32_t base = 0;
    int par = 0;
    for (int64_t c0 = 0; c0 < nch && base < need; c0 += NT, par ^= 1) {
      const int64_t c = c0 + t;
      uint32_t em = 0;
      if (c < nch) {
        const u32x4 v = chunk(c, false);
#pragma unroll
        for (int e = 0; e < EPC; ++e) em |= (chunk_key<ES>(v, e, nanmag) == T ? 1u : 0u) << e;
      }
      int pre, tot;
      wave_scan16(__popc(em), lane, pre, tot);
      if (lane == 0) s_wtot[par][w] = tot;
      __syncthreads();  // s_wtot[par] was last read before the previous round's barrier
      uint32_t before = 0, all = 0;
#pragma unroll
      for (int q = 0; q < NT / 64; ++q) {
        const uint32_t x = (uint32_t)s_wtot[par][q];
        all += x;
        before += q < w ? x : 0;
      }
      uint32_t slot = base + before + (uint32_t)pre;
      while (em) {
        const int e = __builtin_ctz(em);
        em &= em - 1;
        if (slot < need) s_sel[ngt + slot] = ((uint64_t)T << 32) | (uint32_t)~(uint32_t)(c * EPC + e);
        ++slot;
      }
      base += all;
    }
    if (t == 0) {  // the tail columns come last
      for (int i = 0; i < ntail && base < need; ++i)
        if (tail_key(i) == T) {
          s_sel[ngt + base] = ((uint64_t)T << 32) | (uint32_t)~(uint32_t)(nch * EPC + i);
          ++base;
        }
    }
  }
  __syncthreads();

  // ---- 4. sort the k pairs descending (value, then lower column first), write
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = k + t; i < P; i += NT) s_sel[i] = 0;
  __syncthreads();
  block_bitonic_sort(s_sel, P, t, NT, true);
  for (int i = t; i < k; i += NT) {
    const uint32_t col = ~(uint32_t)s_sel[i];
    const int64_t o = orow * (int64_t)k + i;
    indices[o] = (int32_t)col;
    copy_value(rp, col, 1, ES, values, o);
  }
}

// ===================================================================================
// Top-k for k above KMAX. The selected pairs no longer fit in LDS, so they are staged in the
// row's own output: the column in indices[], the order-preserving key in values[] (a key has
// exactly the value's width, 16 or 32 bits), and the k pairs are sorted in place there. The
// sort is a bitonic network in the direction-free form (the first compare of every merge pairs
// i with its mirror in the block, the later ones i with i + stride, larger pair first), run
// over the next power of two P >= k: positions k..P-1 are virtual minima, and since every
// compare keeps the larger pair at the lower index, a real pair is never moved into them,
// so they need no storage. Compares between pairs less than LCH/2 apart run on LCH-pair
// chunks copied to LDS; wider ones run on global memory, one barrier per step (the block's
// waves share one CU, so its global writes are visible to the block after the barrier).
// Results are identical to topk_kernel's: the same selection (ties at the cut by lowest
// column) and the same order (value descending, equal values by increasing column).
// ===================================================================================
constexpr int LCH = 2048;  // pairs per LDS chunk (16 KiB)

// The output rows are written and re-read by every wave of the block between barriers. A
// workgroup barrier does not wait for this wave's global stores to land (the compiler emits
// s_barrier with no vmcnt wait for them), and a later load may hit a line the CU's L1 cached
// before another wave's store. So every barrier after stores waits for them (vmcnt(0)), and
// every load of the rows is a device-scope (sc1) buffer load, served by the L2.
struct RowBufs {
  __amdgpu_buffer_rsrc_t v, i;
  char* vrow;
  int32_t* irow;
};
__device__ __forceinline__ void sync_global() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores have completed
  __syncthreads();
}
constexpr int AUX_SC1 = 16;  // buffer-load cache policy: device scope, no L1 hit

template <int ES>
__device__ __forceinline__ uint64_t pair_at(const RowBufs& b, int64_t i) {
  const uint32_t key = ES == 2 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(b.v, (int)(i * 2), 0, AUX_SC1)
                               : __builtin_amdgcn_raw_buffer_load_b32(b.v, (int)(i * 4), 0, AUX_SC1);
  const uint32_t col = __builtin_amdgcn_raw_buffer_load_b32(b.i, (int)(i * 4), 0, AUX_SC1);
  return ((uint64_t)key << 32) | (uint32_t)~col;
}
template <int ES>
__device__ __forceinline__ void pair_put(const RowBufs& b, int64_t i, uint64_t p) {
  if constexpr (ES == 2) ((u16*)b.vrow)[i] = (u16)(p >> 32);
  else ((uint32_t*)b.vrow)[i] = (uint32_t)(p >> 32);
  b.irow[i] = (int32_t)~(uint32_t)p;
}

// Compare-exchange of global pairs lo < hi (larger pair to lo); hi >= n is a virtual minimum.
template <int ES>
__device__ __forceinline__ void cmpx_global(const RowBufs& b, int64_t lo, int64_t hi, int64_t n) {
  if (hi >= n) return;
  const uint64_t x = pair_at<ES>(b, lo), y = pair_at<ES>(b, hi);
  if (x < y) {
    pair_put<ES>(b, lo, y);
    pair_put<ES>(b, hi, x);
  }
}

// Runs, on every LCH-pair chunk of [0, n), the compares of the current merge whose stride is
// below `from` (from <= LCH), or with `full` a whole sort of the chunk (merges of size 2 to
// LCH). Virtual pairs load as 0, below every real pair. Ends with every store landed.
template <int ES>
__device__ void chunk_pass(const RowBufs& b, int64_t n, uint64_t* s, bool full, int from, int t) {
  for (int64_t c0 = 0; c0 < n; c0 += LCH) {
    for (int i = t; i < LCH; i += NT) s[i] = c0 + i < n ? pair_at<ES>(b, c0 + i) : 0ull;
    __syncthreads();
    for (int size = full ? 2 : LCH * 2; size <= (full ? LCH : LCH * 2); size <<= 1) {
      int stride = full ? size >> 1 : from >> 1;
      if (full) {  // the mirror compare that opens each merge
        for (int i = t; i < LCH / 2; i += NT) {
          const int half = size >> 1, blk = i / half, off = i % half;
          const int lo = blk * size + off, hi = blk * size + size - 1 - off;
          const uint64_t x = s[lo], y = s[hi];
          if (x < y) {
            s[lo] = y;
            s[hi] = x;
          }
        }
        __syncthreads();
        stride >>= 1;
      }
      for (; stride > 0; stride >>= 1) {
        for (int i = t; i < LCH / 2; i += NT) {
          const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
          const uint64_t x = s[lo], y = s[hi];
          if (x < y) {
            s[lo] = y;
            s[hi] = x;
          }
        }
        __syncthreads();
      }
    }
    for (int i = t; i < LCH && c0 + i < n; i += NT) pair_put<ES>(b, c0 + i, s[i]);
    sync_global();
  }
}

template <int ES>
__global__ __launch_bounds__(NT) void topk_large_kernel(const char* f, int64_t sfm, int64_t sfn, uint32_t nanmag,
                                                        int64_t M, int64_t N, int64_t k, char* values,
                                                        int32_t* indices, RowMap map) {
  __shared__ uint32_t hist[256];
  __shared__ uint64_t s_chunk[LCH];
  __shared__ uint32_t s_prefix, s_need, s_eqcount, s_gt, s_eq;
  __shared__ int s_wtot[2][NT / 64];
  constexpr int NBITS = ES * 8;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = blockIdx.x;
  const int64_t orow = out_row(map, row, M);
  if (orow < 0) return;
  const char* rp = f + row * sfm * ES;
  RowBufs rb;
  rb.vrow = values + orow * k * ES;
  rb.irow = indices + orow * k;
  rb.v = __builtin_amdgcn_make_buffer_rsrc(rb.vrow, (short)0, (int)(k * ES), 0x00020000);
  rb.i = __builtin_amdgcn_make_buffer_rsrc(rb.irow, (short)0, (int)(k * 4), 0x00020000);
  auto key_at = [&](int64_t i) -> uint32_t {
    return ES == 2 ? topk_key16(*(const u16*)(rp + i * sfn * 2), nanmag) : topk_key32(*(const uint32_t*)(rp + i * sfn * 4));
  };

  // ---- 1. radix select of the k-th largest key (as topk_kernel)
  uint32_t prefix = 0, mask = 0, need = (uint32_t)k;
  for (int shift = NBITS - 8; shift >= 0; shift -= 8) {
    hist[t] = 0;
    __syncthreads();
    for (int64_t i0 = 0; i0 < N; i0 += NT) {
      const int64_t i = i0 + t;
      const uint32_t key = i < N ? key_at(i) : 0u;
      hist_add(hist, i < N && (key & mask) == prefix, (key >> shift) & 255u, lane);
    }
    __syncthreads();
    if (w == 0) select_bin(hist, need, lane, prefix, shift, s_prefix, s_need, s_eqcount, s_gt, s_eq);
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    mask |= 255u << shift;
  }
  const uint32_t T = prefix;
  const uint32_t ngt = (uint32_t)k - need;
  const bool all_eq = s_eqcount == need;

  // ---- 2. keys above T (and every key equal to T when all are taken) into the output row
  for (int64_t i = t; i < N; i += NT) {
    const uint32_t key = key_at(i);
    uint32_t slot = ~0u;
    if (key > T) {
      const uint32_t sl = atomicAdd(&s_gt, 1u);
      if (sl < ngt) slot = sl;
    } else if (all_eq && key == T) {
      const uint32_t sl = atomicAdd(&s_eq, 1u);
      if (sl < need) slot = ngt + sl;
    }
    if (slot != ~0u) pair_put<ES>(rb, slot, ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i);
  }
  // ---- 3. otherwise the `need` keys equal to T with the lowest columns, in column order
  if (!all_eq) {
    uint32_t base = 0;
    int par = 0;
    for (int64_t i0 = 0; i0 < N && base < need; i0 += NT, par ^= 1) {
      const int64_t i = i0 + t;
      const bool eq = i < N && key_at(i) == T;
      const uint64_t bal = __ballot(eq);
      if (lane == 0) s_wtot[par][w] = __popcll(bal);
      __syncthreads();
      uint32_t before = 0, all = 0;
#pragma unroll
      for (int q = 0; q < NT / 64; ++q) {
        const uint32_t x = (uint32_t)s_wtot[par][q];
        all += x;
        before += q < w ? x : 0;
      }
      const uint32_t slot = base + before + __popcll(bal & lanemask_lt(lane));
      if (eq && slot < need) pair_put<ES>(rb, ngt + slot, ((uint64_t)T << 32) | (uint32_t)~(uint32_t)i);
      base += all;
    }
  }
  sync_global();

  // ---- 4. sort the k pairs in place, larger pair first
  const int64_t n = k;
  int64_t P = 1;
  while (P < n) P <<= 1;
  chunk_pass<ES>(rb, n, s_chunk, true, 0, t);
  for (int64_t size = 2 * LCH; size <= P; size <<= 1) {
    const int64_t half = size >> 1;
    for (int64_t i = t; i < P / 2; i += NT) {
      const int64_t blk = i / half, off = i % half;
      cmpx_global<ES>(rb, blk * size + off, blk * size + size - 1 - off, n);
    }
    sync_global();
    for (int64_t stride = half >> 1; stride >= LCH; stride >>= 1) {
      for (int64_t i = t; i < P / 2; i += NT) {
        const int64_t lo = 2 * i - (i & (stride - 1));
        cmpx_global<ES>(rb, lo, lo + stride, n);
      }
      sync_global();
    }
    chunk_pass<ES>(rb, n, s_chunk, false, LCH, t);
  }

  // ---- 5. the keys are replaced by the selected columns' values
  for (int64_t i = t; i < n; i += NT) {
    const uint32_t col = __builtin_amdgcn_raw_buffer_load_b32(rb.i, (int)(i * 4), 0, AUX_SC1);
    copy_value(rp, col, sfn, ES, rb.vrow, i);
  }
}

// Top-k of a row's candidate list (see rows_to_csr_kernel): sort the (value, column) keys
// descending (values descending, equal values by increasing column) and keep the first k.
// A row with fewer than k candidates is completed with zero values at the lowest columns not
// among them, which is the dense top-k when every nonzero of the row is a candidate.
__global__ __launch_bounds__(NT) void rows_topk_kernel(const int32_t* cnt, const int32_t* cidx, const char* cval,
                                                       int es, uint32_t nanmag, int64_t cap, int64_t M, int k,
                                                       char* values, int32_t* indices) {
  __shared__ uint64_t s[SF_ROWS_CAP_MAX];
  __shared__ uint32_t s_used[2 * SF_ROWS_CAP_MAX / 32];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  int64_t n64 = cnt[row];
  n64 = n64 < 0 ? 0 : (n64 > cap ? cap : n64);
  const int n = (int)n64;
  int P = 1;
  while (P < n) P <<= 1;
  const int32_t* ri = cidx + row * cap;
  const char* rv = cval + row * cap * es;
  for (int i = t; i < P; i += NT) {
    uint64_t e = 0;
    if (i < n) {
      const uint32_t vb = es == 2 ? *(const u16*)(rv + i * 2) : *(const uint32_t*)(rv + i * 4);
      const uint32_t key = es == 2 ? topk_key16(vb, nanmag) : topk_key32(vb);
      e = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)ri[i];
    }
    s[i] = e;
  }
  for (int i = t; i < 2 * SF_ROWS_CAP_MAX / 32; i += NT) s_used[i] = 0;
  __syncthreads();
  if (n > 1) block_bitonic_sort(s, P, t, NT, true);
  const int take = n < k ? n : k;
  for (int i = t; i < take; i += NT) {
    const uint64_t e = s[i];
    const uint32_t key = (uint32_t)(e >> 32), col = ~(uint32_t)e;
    const int64_t o = row * (int64_t)k + i;
    indices[o] = (int32_t)col;
    // a key gives back its value's bits except for a NaN (all NaNs share one key): then the
    // candidate of that column is looked up (NaN rows only; candidates are never zeros)
    if (key == (es == 2 ? 0xffffu : 0xffffffffu)) {
      int j = 0;
      while (j < n - 1 && (uint32_t)ri[j] != col) ++j;
      if (es == 2) ((u16*)values)[o] = *(const u16*)(rv + j * 2);
      else ((uint32_t*)values)[o] = *(const uint32_t*)(rv + j * 4);
    } else if (es == 2) {
      ((u16*)values)[o] = (u16)((key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu));
    } else {
      ((uint32_t*)values)[o] = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
    }
  }
  if (n < k) {  // block-uniform
    for (int i = t; i < n; i += NT) {
      const uint32_t c = (uint32_t)ri[i];
      if (c < (uint32_t)(2 * k)) atomicOr(&s_used[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
    if (t == 0) {
      uint32_t c = 0;
      for (int i = n; i < k; ++i) {
        while (s_used[c >> 5] & (1u << (c & 31))) ++c;
        const int64_t o = row * (int64_t)k + i;
        indices[o] = (int32_t)c;
        if (es == 2) ((u16*)values)[o] = 0;
        else ((uint32_t*)values)[o] = 0;
        ++c;
      }
    }
  }
}

}  // namespace

extern "C" int sf_rows_topk(const int32_t* cand_cnt, const int32_t* cand_idx, const void* cand_val, int val_dt,
                            int64_t cap, int64_t M, int64_t N, int64_t k, void* values, int32_t* indices,
                            void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0, "sf_rows_topk: negative size");
  SF_REQUIRE(sf_valid_dtype(val_dt), "sf_rows_topk: bad dtype code %d", val_dt);
  SF_REQUIRE(k >= 0 && k <= N, "sf_rows_topk: selected index k=%lld out of range for N=%lld", (long long)k,
             (long long)N);
  SF_REQUIRE(k <= SF_ROWS_CAP_MAX, "sf_rows_topk: k=%lld above the supported maximum %d", (long long)k,
             SF_ROWS_CAP_MAX);
  SF_REQUIRE(cap >= 0 && cap <= SF_ROWS_CAP_MAX, "sf_rows_topk: capacity %lld above %d", (long long)cap,
             SF_ROWS_CAP_MAX);
  SF_REQUIRE(M < (1LL << 31), "sf_rows_topk: too many rows");
  if (M == 0 || k == 0) return SF_OK;
  SF_REQUIRE(cand_cnt && values && indices && (cap == 0 || (cand_idx && cand_val)), "sf_rows_topk: NULL buffer");
  const uint32_t nanmag = val_dt == SF_F16 ? 0x7c00u : 0x7f80u;
  hipLaunchKernelGGL(rows_topk_kernel, dim3((unsigned)M), dim3(NT), 0, (hipStream_t)stream, cand_cnt, cand_idx,
                     (const char*)cand_val, sf_dtype_size(val_dt), nanmag, cap, M, (int)k, (char*)values, indices);
  SF_LAUNCH_CHECK("rows_topk_kernel");
  return SF_OK;
}

namespace {
int topk_impl(const char* fn, const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N, int64_t k,
              void* values, int32_t* indices, const RowMap& map, void* stream) {
  SF_REQUIRE(M >= 0 && N >= 0, "%s: negative size", fn);
  SF_REQUIRE(sf_valid_dtype(f_dt), "%s: bad dtype code %d", fn, f_dt);
  SF_REQUIRE(k >= 0 && k <= N, "%s: selected index k=%lld out of range for N=%lld", fn, (long long)k, (long long)N);
  SF_REQUIRE(N < (1LL << 31) && M < (1LL << 31), "%s: size too large", fn);
  if (M == 0 || k == 0) return SF_OK;
  SF_REQUIRE(f && values && indices, "%s: NULL buffer", fn);
  const int es = sf_dtype_size(f_dt);
  const uint32_t nanmag = f_dt == SF_F16 ? 0x7c00u : 0x7f80u;  // 16-bit NaN magnitudes lie above it
  hipStream_t s = (hipStream_t)stream;
  const char* fp = (const char*)f;
  char* vp = (char*)values;
  if (k > KMAX) {
    SF_REQUIRE(k < (1LL << 29), "%s: k=%lld too large for 32-bit row offsets", fn, (long long)k);
    if (es == 2)
      hipLaunchKernelGGL(topk_large_kernel<2>, dim3((unsigned)M), dim3(NT), 0, s, fp, sfm, sfn, nanmag, M, N, k, vp,
                         indices, map);
    else
      hipLaunchKernelGGL(topk_large_kernel<4>, dim3((unsigned)M), dim3(NT), 0, s, fp, sfm, sfn, nanmag, M, N, k, vp,
                         indices, map);
  } else if (sfn == 1 && (uintptr_t)f % 16 == 0 && (sfm * es) % 16 == 0) {
    const int64_t row_bytes = N / (16 / es) * 16;  // whole chunks
    const dim3 grid((unsigned)M), block(NT);
    if (row_bytes <= LDS_ROW_MAX) {
      const size_t lds = (size_t)row_bytes;
      if (es == 2)
        hipLaunchKernelGGL((topk_vec_kernel<2, true>), grid, block, lds, s, fp, sfm, nanmag, M, N, (int)k, vp, indices,
                           map);
      else
        hipLaunchKernelGGL((topk_vec_kernel<4, true>), grid, block, lds, s, fp, sfm, nanmag, M, N, (int)k, vp, indices,
                           map);
    } else {
      if (es == 2)
        hipLaunchKernelGGL((topk_vec_kernel<2, false>), grid, block, 0, s, fp, sfm, nanmag, M, N, (int)k, vp, indices,
                           map);
      else
        hipLaunchKernelGGL((topk_vec_kernel<4, false>), grid, block, 0, s, fp, sfm, nanmag, M, N, (int)k, vp, indices,
                           map);
    }
  } else {
    hipLaunchKernelGGL(topk_kernel, dim3((unsigned)M), dim3(NT), 0, s, fp, sfm, sfn, es, nanmag, M, N, (int)k, vp,
                       indices, map);
  }
  SF_LAUNCH_CHECK("topk_kernel");
  return SF_OK;
}
}  // namespace

extern "C" int sf_topk(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N, int64_t k,
                       void* values, int32_t* indices, void* stream) {
  sf_clear_error();
  return topk_impl("sf_topk", f, sfm, sfn, f_dt, M, N, k, values, indices, RowMap{nullptr, 0, nullptr, 0}, stream);
}

extern "C" int sf_topk_gather(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N, int64_t k,
                              const int32_t* n_rows, int64_t row_off, const int32_t* out_rows, int64_t M_out,
                              void* values, int32_t* indices, void* stream) {
  sf_clear_error();
  SF_REQUIRE(row_off >= 0 && M_out >= 0, "sf_topk_gather: negative size");
  SF_REQUIRE(M == 0 || k == 0 || (n_rows && out_rows), "sf_topk_gather: NULL row list or row count");
  return topk_impl("sf_topk_gather", f, sfm, sfn, f_dt, M, N, k, values, indices,
                   RowMap{n_rows, row_off, out_rows, M_out}, stream);
}

namespace {
// One workgroup of OV_NT threads: rows[0 .. n) = the rows m with cnt[m] > cap in increasing
// order, *n_rows = n, in rounds of OV_NT rows with a block prefix of the flags.
constexpr int OV_NT = 1024;
__global__ __launch_bounds__(OV_NT) void overflow_rows_kernel(const int32_t* cnt, int64_t M, int64_t cap,
                                                              int32_t* rows, int32_t* n_rows) {
  __shared__ int s_wtot[2][OV_NT / 64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int64_t base = 0;
  int par = 0;
  for (int64_t r0 = 0; r0 < M; r0 += OV_NT, par ^= 1) {
    const int64_t m = r0 + t;
    const bool over = m < M && (int64_t)cnt[m] > cap;
    const uint64_t bal = __ballot(over);
    if (lane == 0) s_wtot[par][w] = __popcll(bal);
    __syncthreads();  // s_wtot[par] was last read before the previous round's barrier
    int64_t before = 0, all = 0;
#pragma unroll
    for (int q = 0; q < OV_NT / 64; ++q) {
      const int x = s_wtot[par][q];
      all += x;
      before += q < w ? x : 0;
    }
    if (over) rows[base + before + __popcll(bal & lanemask_lt(lane))] = (int32_t)m;
    base += all;
  }
  if (t == 0) *n_rows = (int32_t)base;
}
}  // namespace

extern "C" int sf_overflow_rows(const int32_t* cand_cnt, int64_t M, int64_t cap, int32_t* rows, int32_t* n_rows,
                                void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && M < (1LL << 31), "sf_overflow_rows: bad row count %lld", (long long)M);
  SF_REQUIRE(cap >= 0, "sf_overflow_rows: negative capacity");
  SF_REQUIRE(n_rows && (M == 0 || (cand_cnt && rows)), "sf_overflow_rows: NULL buffer");
  hipLaunchKernelGGL(overflow_rows_kernel, dim3(1), dim3(OV_NT), 0, (hipStream_t)stream, cand_cnt, M, cap, rows,
                     n_rows);
  SF_LAUNCH_CHECK("overflow_rows_kernel");
  return SF_OK;
}
