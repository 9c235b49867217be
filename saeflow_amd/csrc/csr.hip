// Dense -> CSR on gfx950: per-row nonzero counts, exclusive scan to int64 indptr, and
// order-preserving compaction; plus the CSR -> dense scatter.
//
// Reference semantics: dense_to_csr (saeflow/kernels/decode.py:77-94), _compact_kernel
// (decode.py:61-74), csr_to_dense (decode.py:123-126) and the TopK dense scatter
// (ops.py:21-25).
//
// Compaction: one workgroup owns one row of f (one wave per row for strided f). The row is
// streamed once, in 16-B non-temporal chunks, 2048 contiguous chunks per group with the next
// group in flight while the current one is compacted; each lane turns its chunk into a
// nonzero bit mask, and wave ballot prefixes plus the wave totals exchanged through LDS give
// every nonzero its slot, so the output is in increasing column order without any atomics.
// The entries of a row longer than one group are staged in LDS and stored once at its end.
// A row stops being read as soon as all indptr-announced nonzeros of the row have been found.
#include <type_traits>

#include "common.h"

namespace {

constexpr int WPB = 4;  // waves (rows) per 256-thread block

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// nonzero mask of the elements of a 16-B chunk (8 x 16-bit or 4 x 32-bit)
template <int ES>
__device__ __forceinline__ uint32_t chunk_mask(const u32x4& v) {
  uint32_t m = 0;
  if constexpr (ES == 2) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      m |= ((v[d] & 0x7fffu) != 0) << (2 * d);
      m |= ((v[d] & 0x7fff0000u) != 0) << (2 * d + 1);
    }
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) m |= ((v[d] & 0x7fffffffu) != 0) << d;
  }
  return m;
}

// The same nonzero test with fewer instructions, as flags for counting: x + 0x7fff (or
// 0x7fffffff) carries into a 16-bit (32-bit) element's top bit exactly when its magnitude
// bits x are nonzero, and cannot carry past it. Element 2d / 2d+1 of a 16-bit chunk lands
// on bit 15-d / 31-d, element d of an fp32 chunk on bit 31-d; popc gives the count.
template <int ES>
__device__ __forceinline__ uint32_t chunk_flags(const u32x4& v) {
  uint32_t f = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (ES == 2) f |= (((v[d] & 0x7fff7fffu) + 0x7fff7fffu) & 0x80008000u) >> d;
    else f |= (((v[d] & 0x7fffffffu) + 0x7fffffffu) & 0x80000000u) >> d;
  }
  return f;
}

template <int ES>
__device__ __forceinline__ uint32_t chunk_elem_bits(const u32x4& v, int e) {
  if constexpr (ES == 2) return (v[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
  else return v[e];
}

__device__ __forceinline__ uint32_t load_bits(const char* p, int es) {
  return es == 2 ? *(const u16*)p : *(const uint32_t*)p;
}
__device__ __forceinline__ void store_bits(char* p, uint32_t b, int es) {
  if (es == 2) *(u16*)p = (u16)b;
  else *(uint32_t*)p = b;
}

// ----------------------------------------------------------------------------- counts
// Rows of 16-B aligned chunks: one 256-thread workgroup per row, U contiguous 1024-chunk
// runs in flight per thread, block sum through LDS.
template <int ES>
__global__ __launch_bounds__(256) void count_row_kernel(const char* f, int64_t sfm, int64_t N, int32_t* counts) {
  constexpr int EPC = 16 / ES, U = 8;
  __shared__ int s_sum[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = blockIdx.x;
  const char* rp = f + row * sfm * ES;
  const int64_t nch = N / EPC;
  int c = 0;
  for (int64_t c0 = 0; c0 < nch; c0 += 256 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t ch = c0 + u * 256 + t;
      v[u] = __builtin_nontemporal_load((const u32x4*)(rp + (ch < nch ? ch : nch - 1) * 16));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) c += c0 + u * 256 + t < nch ? __popc(chunk_flags<ES>(v[u])) : 0;
  }
  for (int64_t i = nch * EPC + t; i < N; i += 256) c += bits_nonzero(load_bits(rp + i * ES, ES), ES);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
  if (lane == 0) s_sum[w] = c;
  __syncthreads();
  if (t == 0) counts[row] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
}

// Rows of any strides: one wave per row, element by element.
template <int ES>
__global__ __launch_bounds__(256) void count_kernel(const char* f, int64_t sfm, int64_t sfn, int64_t M,
                                                    int64_t N, int32_t* counts) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= M) return;
  const char* rp = f + row * sfm * ES;
  int c = 0;
  for (int64_t i = lane; i < N; i += 64) c += bits_nonzero(load_bits(rp + i * sfn * ES, ES), ES);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
  if (lane == 0) counts[row] = c;
}

// ----------------------------------------------------------------------------- scan
// indptr[0] = 0, indptr[i+1] = counts[0] + ... + counts[i], in tiles of SCAN_TILE counts (256
// threads x 16 consecutive counts each, read as 16-B vectors where aligned):
//  1. scan_tiles_kernel: each tile's total, parked in indptr[tile*SCAN_TILE + 1] (a slot
//     that only this tile's final pass writes);
//  2. scan_totals_kernel: one block turns the parked totals into exclusive tile offsets, in
//     place;
//  3. scan_final_kernel: each tile reads its offset, then writes its inclusive prefixes.
// One tile needs only the last pass (offset 0).
constexpr int SCAN_PER = 16, SCAN_TILE = 256 * SCAN_PER;

__device__ __forceinline__ void load_counts16(const int32_t* counts, int64_t M, int64_t i0, int32_t (&c)[SCAN_PER]) {
  if (i0 + SCAN_PER <= M && ((uintptr_t)(counts + i0) % 16) == 0) {
#pragma unroll
    for (int q = 0; q < SCAN_PER / 4; ++q) {
      const int4 v = *(const int4*)(counts + i0 + 4 * q);
      c[4 * q] = v.x;
      c[4 * q + 1] = v.y;
      c[4 * q + 2] = v.z;
      c[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < SCAN_PER; ++q) c[q] = i0 + q < M ? counts[i0 + q] : 0;
  }
}

__global__ __launch_bounds__(256) void scan_tiles_kernel(const int32_t* counts, int64_t M, int64_t* indptr) {
  __shared__ int64_t s_w[4];
  const int64_t i0 = (int64_t)blockIdx.x * SCAN_TILE + threadIdx.x * SCAN_PER;
  int32_t c[SCAN_PER];
  load_counts16(counts, M, i0, c);
  int64_t s = 0;
#pragma unroll
  for (int q = 0; q < SCAN_PER; ++q) s += c[q];
  int64_t total;
  block_exclusive_i64(s, s_w, total);
  if (threadIdx.x == 0) indptr[(int64_t)blockIdx.x * SCAN_TILE + 1] = total;
}

__global__ __launch_bounds__(256) void scan_totals_kernel(int64_t ntiles, int64_t* indptr) {
  __shared__ int64_t s_w[4];
  int64_t carry = 0;
  for (int64_t b0 = 0; b0 < ntiles; b0 += 256) {
    const int64_t b = b0 + threadIdx.x;
    const int64_t v = b < ntiles ? indptr[b * SCAN_TILE + 1] : 0;
    int64_t total;
    const int64_t ex = block_exclusive_i64(v, s_w, total);
    if (b < ntiles) indptr[b * SCAN_TILE + 1] = carry + ex;
    carry += total;
    __syncthreads();  // s_w is rewritten by the next round
  }
}

__global__ __launch_bounds__(256) void scan_final_kernel(const int32_t* counts, int64_t M, int64_t* indptr,
                                                         int has_offsets) {
  __shared__ int64_t s_w[4];
  __shared__ int64_t s_off;
  const int64_t i0 = (int64_t)blockIdx.x * SCAN_TILE + threadIdx.x * SCAN_PER;
  if (threadIdx.x == 0) s_off = has_offsets ? indptr[(int64_t)blockIdx.x * SCAN_TILE + 1] : 0;
  int32_t c[SCAN_PER];
  load_counts16(counts, M, i0, c);
  int64_t s = 0;
#pragma unroll
  for (int q = 0; q < SCAN_PER; ++q) s += c[q];
  int64_t total;
  int64_t run = block_exclusive_i64(s, s_w, total) + s_off;  // the barrier inside orders s_off
#pragma unroll
  for (int q = 0; q < SCAN_PER; ++q) {
    run += c[q];
    if (i0 + q < M) indptr[i0 + q + 1] = run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) indptr[0] = 0;
}

// ----------------------------------------------------------------------------- compact
// Rows of any strides: one wave per row, 64 elements per step, ballot prefix for the slots.
template <int ES>
__global__ __launch_bounds__(256) void compact_kernel(const char* f, int64_t sfm, int64_t sfn, int64_t M,
                                                      int64_t N, const int64_t* indptr, int64_t nnz,
                                                      int32_t* indices, char* values) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= M) return;
  int64_t pos = indptr[row], end = indptr[row + 1];
  pos = pos < 0 ? 0 : (pos > nnz ? nnz : pos);
  end = end < pos ? pos : (end > nnz ? nnz : end);
  const char* rp = f + row * sfm * ES;
  for (int64_t i0 = 0; i0 < N && pos < end; i0 += 64) {
    int64_t i = i0 + lane;
    uint32_t b = i < N ? load_bits(rp + i * sfn * ES, ES) : 0;
    bool nz = i < N && bits_nonzero(b, ES);
    uint64_t bal = __ballot(nz);
    if (nz) {
      int64_t slot = pos + __popcll(bal & lanemask_lt(lane));
      if (slot < end) {
        indices[slot] = (int32_t)i;
        store_bits(values + slot * ES, b, ES);
      }
    }
    pos += __popcll(bal);
  }
}

// Compaction of rows made of 16-B aligned chunks: one workgroup of NW waves per row. The
// row is streamed in groups of NT * U contiguous chunks (thread t takes chunks u*NT + t of
// the group), the next group in flight while this one is compacted, so the workgroups in
// flight read a few long contiguous runs of the matrix. The first group's loads go out before
// the row's bounds are read. A nonzero's slot = row start + nonzeros of earlier groups + of
// earlier passes u of this group + of lower threads in pass u: the last from per-wave ballot
// prefixes (skipped by a wave whose 64 chunks of the pass hold no nonzero, most of them at a
// sparse f) plus the wave totals exchanged through LDS, one barrier per group. Loop bounds and
// `pos` are the same in every wave, so all waves take every barrier. Slots outside
// [indptr[row], indptr[row+1]) are never written.
//
// A row of at most CR_STAGE nonzeros is staged in LDS and stored once, after its last group,
// with non-temporal stores as one contiguous run: scattered stores of 4 and 2 bytes in every
// group, interleaved with the streamed reads, cost C3 0.345-0.36 ms against 0.303 ms for the
// same loop without stores; staged with plain stores 0.345, staged with non-temporal stores
// 0.328. Longer rows store directly.
// (waves, 16-B chunks per thread per load group, staging): 8 x 4 with staging for rows longer
// than one 32 KB group; 4 x 8 with direct stores for rows of one group, whose stores follow
// their only group anyway (C2's 32 KB rows: staging cost 0.130 against 0.119 ms), and no next
// group to load in flight (C2 0.107 against 0.118 ms with the prefetch of a group past the row).
constexpr int CR_STAGE = 2048;  // nonzeros of a row staged in LDS
constexpr int64_t CR_ONE_GROUP = 32768;  // row bytes up to which the 4 x 8 shape is used
// Row bytes from which the 16 x 2 shape is used: at 2 GiB of f, 16 waves of 2 chunks against 8
// of 4 per 32 KB group measured 0.483 / 0.328 ms for 256 KB rows, 0.385 / 0.334 for 512 KB,
// 0.323 / 0.331 for 1 MB and 0.317 / 0.336 for 2 MB rows (C5's)
constexpr int64_t CR_LONG_ROW = 1 << 20;
static_assert(CR_ONE_GROUP == 4 * 64 * 8 * 16, "the 4 x 8 shape reads a one-group row in one group");

// s_waitcnt lgkmcnt(0), then a workgroup barrier without __syncthreads()'s release fence,
// which would also wait for the next group's loads in flight. Only the LDS wave totals
// must be visible past the barrier; the signal fences keep the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int ES>
using elem_t = typename std::conditional<ES == 2, u16, uint32_t>::type;

template <int ES, int NW, int U, bool STAGE, bool ONE>
__global__ __launch_bounds__(NW * 64) void compact_row_kernel(const char* f, int64_t sfm, int64_t N,
                                                              const int64_t* indptr, int64_t nnz, int32_t* indices,
                                                              char* values) {
  constexpr int EPC = 16 / ES, NT = NW * 64, G = NT * U;
  __shared__ int s_tot[2][U][NW];  // [group parity][pass][wave]: nonzeros of each wave's chunks
  constexpr int SN = STAGE ? CR_STAGE : 1;
  __shared__ int32_t s_idx[SN];
  __shared__ elem_t<ES> s_val[SN];
  __shared__ int64_t s_filled;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = blockIdx.x;
  const char* rp = f + row * sfm * ES;
  const int64_t nch = N / EPC;
  // Chunks past the row end load the row's last chunk and are masked out where they are
  // consumed: branch-free loads with no use right after them keep the compiler's wait
  // counts exact, so the next group stays in flight while this one is compacted.
  auto load_group = [&](u32x4 (&v)[U], int64_t c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t ch = c0 + u * NT + t;
      v[u] = __builtin_nontemporal_load((const u32x4*)(rp + (ch < nch ? ch : nch - 1) * 16));
    }
  };
  u32x4 v[U], nx[U];
  if (nch > 0) load_group(v, 0);  // before the row's bounds are known
  int64_t pos = indptr[row], end = indptr[row + 1];
  pos = pos < 0 ? 0 : (pos > nnz ? nnz : pos);
  end = end < pos ? pos : (end > nnz ? nnz : end);
  if (pos == end) return;
  const int64_t start = pos;
  const bool staged = STAGE && end - start <= CR_STAGE;  // the same in every thread
  auto put = [&](int64_t slot, int64_t col, uint32_t bits) {
    if (staged) {
      s_idx[slot - start] = (int32_t)col;
      s_val[slot - start] = (elem_t<ES>)bits;
    } else {
      indices[slot] = (int32_t)col;
      store_bits(values + slot * ES, bits, ES);
    }
  };
  int par = 0;
  for (int64_t c0 = 0; c0 < nch && pos < end; c0 += G, par ^= 1) {
    if constexpr (!ONE) load_group(nx, c0 + G);  // ONE: the row is this group (N * ES <= G * 16)
    uint32_t fl[U];
    int pre[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      fl[u] = c0 + u * NT + t < nch ? chunk_flags<ES>(v[u]) : 0u;
      int tot;
      if (__ballot(fl[u] != 0) != 0) {
        wave_scan16(__popc(fl[u]), lane, pre[u], tot);
      } else {  // no nonzero in the wavefront's 64 chunks (most of them at L0 64 of 65536)
        pre[u] = 0;
        tot = 0;
      }
      if (lane == 0) s_tot[par][u][w] = tot;
    }
    // s_tot[par] was last read two groups ago, before the previous group's barrier
    lds_barrier();
    int64_t base = pos;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int before = 0, all = 0;
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        const int x = s_tot[par][u][q];
        all += x;
        before += q < w ? x : 0;
      }
      if (fl[u]) {  // few lanes: the element-order mask only here
        uint32_t mm = chunk_mask<ES>(v[u]);
        int64_t slot = base + before + pre[u];
        const int64_t col0 = (c0 + u * NT + t) * EPC;
        while (mm) {
          const int e = __builtin_ctz(mm);
          mm &= mm - 1;
          if (slot < end) put(slot, col0 + e, chunk_elem_bits<ES>(v[u], e));
          ++slot;
        }
      }
      base += all;
    }
    pos = base;
    if constexpr (ONE) break;
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = nx[u];
  }
  // the last N % EPC columns, element by element in wave 0
  if (w == 0) {
    for (int64_t i0 = nch * EPC; i0 < N && pos < end; i0 += 64) {
      const int64_t i = i0 + lane;
      const uint32_t b = i < N ? load_bits(rp + i * ES, ES) : 0;
      const bool nz = i < N && bits_nonzero(b, ES);
      const uint64_t bal = __ballot(nz);
      if (nz) {
        const int64_t slot = pos + __popcll(bal & lanemask_lt(lane));
        if (slot < end) put(slot, i, b);
      }
      pos += __popcll(bal);
    }
  }
  if (!staged) return;
  // Every slot of [start, end) was staged unless the row held fewer nonzeros than indptr
  // announces; only the slots the row filled are written out. Wave 0 holds the final
  // position (the tail is its own).
  if (t == 0) s_filled = min(end, pos) - start;
  __syncthreads();
  const int64_t filled = s_filled;
  for (int64_t i = t; i < filled; i += NT) {
    __builtin_nontemporal_store(s_idx[i], indices + start + i);
    __builtin_nontemporal_store(s_val[i], (elem_t<ES>*)values + start + i);
  }
}

// ----------------------------------------------------------------------------- csr -> dense
// One 256-thread block per row: zero the row, then place the row's entries. A CSR row whose
// columns are all distinct is placed in parallel; a row with repeated columns is summed
// serially in entry order, as successive additions in the value type (to_dense of a CSR
// tensor sums them). Distinctness costs one O(n) pass for rows whose columns strictly increase
// (canonical CSR); other rows are compared pairwise when short, and taken as possibly
// repeating, i.e. placed serially in O(n), when longer than DUP_PAIRWISE_MAX entries.
// Fixed-width rows (indptr NULL: the TopK scatter, zeros.scatter_(-1, indices, values)) are
// always placed in parallel, each value's bits stored as they are, as scatter_ stores them;
// top-k columns are distinct, and a repeated column keeps one of its values, as with scatter_.
constexpr int64_t DUP_PAIRWISE_MAX = 1024;
__global__ __launch_bounds__(256) void csr_to_dense_kernel(const int64_t* indptr, int64_t width,
                                                           const int32_t* indices, const void* values,
                                                           int val_dt, int64_t nnz, int64_t M, int64_t d_sae,
                                                           char* out, int64_t som, int out_dt) {
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int oes = sf_dtype_size(out_dt);
  char* orow = out + row * som * oes;
  const int64_t nb = d_sae * oes;
  // zero-fill (16-B vector stores when the row start is aligned)
  if (((uintptr_t)orow & 15) == 0) {
    for (int64_t i = (int64_t)t * 16; i + 16 <= nb; i += 256 * 16) *(u32x4*)(orow + i) = u32x4{0, 0, 0, 0};
    for (int64_t i = (nb & ~(int64_t)15) + t; i < nb; i += 256) orow[i] = 0;
  } else {
    for (int64_t i = t; i < nb; i += 256) orow[i] = 0;
  }
  int64_t lo, hi;
  if (indptr) {
    lo = indptr[row];
    hi = indptr[row + 1];
  } else {
    lo = row * width;
    hi = lo + width;
  }
  lo = lo < 0 ? 0 : (lo > nnz ? nnz : lo);
  hi = hi < lo ? lo : (hi > nnz ? nnz : hi);
  // The entries are stored over the zeros (and, with repeats, added to them) by other waves:
  // the barriers below do not wait for global stores, so this thread's zeros must land first.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  int local = 0;
  if (indptr)
    for (int64_t j = lo + 1 + t; j < hi; j += 256) local |= indices[j] <= indices[j - 1];
  int dup = 0;
  if (__syncthreads_or(local)) {  // block-uniform
    if (hi - lo <= DUP_PAIRWISE_MAX) {
      int found = 0;
      for (int64_t j = lo + t; j < hi && !found; j += 256) {
        const int32_t c = indices[j];
        for (int64_t i = lo; i < j; ++i)
          if (indices[i] == c) {
            found = 1;
            break;
          }
      }
      dup = __syncthreads_or(found);
    } else {
      dup = 1;
    }
  }
  if (!dup) {
    for (int64_t j = lo + t; j < hi; j += 256) {
      int64_t c = indices[j];
      if (c < 0 || c >= d_sae) continue;
      store_bits(orow + c * oes, f32_to_bits(load_as_f32(values, val_dt, j), out_dt), oes);
    }
  } else if (t == 0) {
    for (int64_t j = lo; j < hi; ++j) {
      int64_t c = indices[j];
      if (c < 0 || c >= d_sae) continue;
      float cur = load_as_f32(orow, out_dt, c);
      store_bits(orow + c * oes, f32_to_bits(cur + load_as_f32(values, val_dt, j), out_dt), oes);
    }
  }
}

bool vec_rows(const void* f, int64_t sfm, int64_t sfn, int es) {
  return sfn == 1 && ((uintptr_t)f % 16) == 0 && ((sfm * es) % 16) == 0;
}

// ----------------------------------------------------------------------------- rows -> csr
// A row's candidates (column, value), appended in arbitrary order by the row-candidate encode,
// are sorted by column and written to the row's CSR segment. Rows of at most WS_MAX
// candidates (all of them at L0 64-128) are sorted by one wavefront in registers, 1, 2 or 4
// keys per lane as the row needs (rows_to_csr_wave_kernel, 4 rows per block, no LDS and no
// barriers); longer rows by a 256-thread block in LDS (rows_to_csr_kernel: a block checks 16
// rows at once and sorts only their long ones, so the many short rows cost it little). Rows whose list overflowed (count > cap) are
// skipped: their segments are the caller's to fill. The segment length indptr[row+1] -
// indptr[row] bounds what is written. Keys (column << 32 | value bits) are distinct within a
// row, so both kernels write the same segment.
constexpr int WS_R = 4, WS_MAX = 64 * WS_R;  // keys per lane, rows the wavefront sort takes
constexpr int LS_ROWS = 16;                  // rows per block of the LDS sort

// The row's valid candidate count (0 for an overflowed row) and its CSR segment start.
__device__ __forceinline__ int row_candidates(const int32_t* cnt, int64_t cap, const int64_t* indptr, int64_t nnz,
                                              int64_t row, int64_t& lo) {
  lo = indptr[row];
  int64_t hi = indptr[row + 1];
  lo = lo < 0 ? 0 : (lo > nnz ? nnz : lo);
  hi = hi < lo ? lo : (hi > nnz ? nnz : hi);
  int64_t n = cnt[row];
  if (n > cap) return 0;  // overflowed: not in the list
  n = n < 0 ? 0 : n;
  return (int)(n > hi - lo ? hi - lo : n);
}

// Ascending bitonic sort of the wavefront's 64 * R keys, key r*64 + lane in v[r]: exchanges
// across lanes with xor shuffles, across registers within a lane.
template <int R>
__device__ __forceinline__ void wave_bitonic_sort(uint64_t (&v)[R], int lane) {
#pragma unroll
  for (int k = 2; k <= 64 * R; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int jr = j / 64;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r & jr) continue;
          const bool asc = ((r * 64 + lane) & k) == 0;
          const uint64_t a = v[r], b = v[r | jr];
          const bool sw = asc ? a > b : a < b;
          v[r] = sw ? b : a;
          v[r | jr] = sw ? a : b;
        }
      } else {
        const bool low = (lane & j) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint64_t a = v[r];
          const uint64_t b = (uint64_t)__shfl_xor((unsigned long long)a, j);
          const bool asc = ((r * 64 + lane) & k) == 0;
          v[r] = (low == asc) ? (a < b ? a : b) : (a < b ? b : a);
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void rows_to_csr_wave_kernel(const int32_t* cnt, const int32_t* cidx,
                                                               const char* cval, int es, int64_t cap, int64_t M,
                                                               const int64_t* indptr, int64_t nnz, int32_t* indices,
                                                               char* values) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // whole wavefront
  int64_t lo;
  const int n = row_candidates(cnt, cap, indptr, nnz, row, lo);
  if (n == 0 || n > WS_MAX) return;  // wavefront-uniform; longer rows: rows_to_csr_kernel
  const int32_t* ri = cidx + row * cap;
  const char* rv = cval + row * cap * es;
  // as few keys per lane as the row needs (wavefront-uniform): the sort's cost grows with them
  auto sort_row = [&](auto r_tag) {
    constexpr int R = decltype(r_tag)::value;
    uint64_t v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * 64 + lane;
      v[r] = ~0ull;
      if (i < n) {
        const uint32_t vb = es == 2 ? *(const u16*)(rv + i * 2) : *(const uint32_t*)(rv + i * 4);
        v[r] = ((uint64_t)(uint32_t)ri[i] << 32) | vb;
      }
    }
    wave_bitonic_sort<R>(v, lane);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * 64 + lane;
      if (i < n) {
        indices[lo + i] = (int32_t)(v[r] >> 32);
        store_bits(values + (lo + i) * es, (uint32_t)v[r], es);
      }
    }
  };
  if (n <= 64) sort_row(std::integral_constant<int, 1>{});
  else if (n <= 128) sort_row(std::integral_constant<int, 2>{});
  else sort_row(std::integral_constant<int, WS_R>{});
}

__global__ __launch_bounds__(256) void rows_to_csr_kernel(const int32_t* cnt, const int32_t* cidx, const char* cval,
                                                          int es, int64_t cap, int64_t M, const int64_t* indptr,
                                                          int64_t nnz, int32_t* indices, char* values) {
  __shared__ uint64_t s[SF_ROWS_CAP_MAX];
  __shared__ int s_long[LS_ROWS];
  __shared__ int s_nlong;
  const int t = threadIdx.x;
  // the block's LS_ROWS rows are checked at once; only the long ones are sorted here
  if (t == 0) s_nlong = 0;
  __syncthreads();
  if (t < LS_ROWS) {
    const int64_t row = (int64_t)blockIdx.x * LS_ROWS + t;
    int64_t lo;
    if (row < M && row_candidates(cnt, cap, indptr, nnz, row, lo) > WS_MAX) s_long[atomicAdd(&s_nlong, 1)] = t;
  }
  __syncthreads();
  const int nlong = s_nlong;
  for (int q = 0; q < nlong; ++q) {  // any order: each row has its own segment
    const int64_t row = (int64_t)blockIdx.x * LS_ROWS + s_long[q];
    int64_t lo;
    const int n = row_candidates(cnt, cap, indptr, nnz, row, lo);
    int P = 1;
    while (P < n) P <<= 1;
    const int32_t* ri = cidx + row * cap;
    const char* rv = cval + row * cap * es;
    for (int i = t; i < P; i += 256) {
      uint64_t e = ~0ull;
      if (i < n) {
        const uint32_t vb = es == 2 ? *(const u16*)(rv + i * 2) : *(const uint32_t*)(rv + i * 4);
        e = ((uint64_t)(uint32_t)ri[i] << 32) | vb;
      }
      s[i] = e;
    }
    __syncthreads();
    block_bitonic_sort(s, P, t, 256, false);
    for (int i = t; i < n; i += 256) {
      const uint64_t e = s[i];
      indices[lo + i] = (int32_t)(e >> 32);
      store_bits(values + (lo + i) * es, (uint32_t)e, es);
    }
    __syncthreads();  // s is refilled for the block's next long row
  }
}

}  // namespace

extern "C" int sf_rows_to_csr(const int32_t* cand_cnt, const int32_t* cand_idx, const void* cand_val, int val_dt,
                              int64_t cap, int64_t M, const int64_t* indptr, int64_t nnz, int32_t* indices,
                              void* values, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && nnz >= 0, "sf_rows_to_csr: negative size");
  SF_REQUIRE(sf_valid_dtype(val_dt), "sf_rows_to_csr: bad dtype code %d", val_dt);
  SF_REQUIRE(cap >= 0 && cap <= SF_ROWS_CAP_MAX, "sf_rows_to_csr: capacity %lld above %d", (long long)cap,
             SF_ROWS_CAP_MAX);
  SF_REQUIRE(M < (1LL << 31), "sf_rows_to_csr: too many rows");
  if (M == 0 || nnz == 0 || cap == 0) return SF_OK;
  SF_REQUIRE(cand_cnt && cand_idx && cand_val && indptr && indices && values, "sf_rows_to_csr: NULL buffer");
  hipLaunchKernelGGL(rows_to_csr_wave_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     cand_cnt, cand_idx, (const char*)cand_val, sf_dtype_size(val_dt), cap, M, indptr, nnz, indices,
                     (char*)values);
  SF_LAUNCH_CHECK("rows_to_csr_wave_kernel");
  if (cap > WS_MAX) {  // rows longer than the wavefront sort takes
    hipLaunchKernelGGL(rows_to_csr_kernel, dim3((unsigned)((M + LS_ROWS - 1) / LS_ROWS)), dim3(256), 0,
                       (hipStream_t)stream, cand_cnt, cand_idx, (const char*)cand_val, sf_dtype_size(val_dt), cap, M,
                       indptr, nnz, indices, (char*)values);
    SF_LAUNCH_CHECK("rows_to_csr_kernel");
  }
  return SF_OK;
}

extern "C" int sf_count_nonzero(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N,
                                int32_t* counts, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0, "sf_count_nonzero: negative size");
  SF_REQUIRE(sf_valid_dtype(f_dt), "sf_count_nonzero: bad dtype code %d", f_dt);
  SF_REQUIRE(N < (1LL << 31), "sf_count_nonzero: N too large");
  if (M == 0) return SF_OK;
  SF_REQUIRE(counts && (f || N == 0), "sf_count_nonzero: NULL buffer");
  const int es = sf_dtype_size(f_dt);
  const bool vec = vec_rows(f, sfm, sfn, es);
  hipStream_t s = (hipStream_t)stream;
  const char* fp = (const char*)f;
  if (vec) {  // one workgroup per row
    SF_REQUIRE(M <= INT32_MAX, "sf_count_nonzero: M too large for one workgroup per row");
    if (es == 2) hipLaunchKernelGGL((count_row_kernel<2>), dim3((unsigned)M), dim3(256), 0, s, fp, sfm, N, counts);
    else hipLaunchKernelGGL((count_row_kernel<4>), dim3((unsigned)M), dim3(256), 0, s, fp, sfm, N, counts);
  } else {
    dim3 grid((unsigned)((M + WPB - 1) / WPB)), block(256);
    if (es == 2) hipLaunchKernelGGL((count_kernel<2>), grid, block, 0, s, fp, sfm, sfn, M, N, counts);
    else hipLaunchKernelGGL((count_kernel<4>), grid, block, 0, s, fp, sfm, sfn, M, N, counts);
  }
  SF_LAUNCH_CHECK("count_kernel");
  return SF_OK;
}

extern "C" int sf_scan_counts(const int32_t* counts, int64_t M, int64_t* indptr, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0, "sf_scan_counts: negative size");
  SF_REQUIRE(indptr && (counts || M == 0), "sf_scan_counts: NULL buffer");
  hipStream_t s = (hipStream_t)stream;
  const int64_t ntiles = (M + SCAN_TILE - 1) / SCAN_TILE;
  SF_REQUIRE(ntiles < (1LL << 31), "sf_scan_counts: too many counts");
  if (ntiles <= 1) {
    hipLaunchKernelGGL(scan_final_kernel, dim3(1), dim3(256), 0, s, counts, M, indptr, 0);
    SF_LAUNCH_CHECK("scan_final_kernel");
    return SF_OK;
  }
  hipLaunchKernelGGL(scan_tiles_kernel, dim3((unsigned)ntiles), dim3(256), 0, s, counts, M, indptr);
  SF_LAUNCH_CHECK("scan_tiles_kernel");
  hipLaunchKernelGGL(scan_totals_kernel, dim3(1), dim3(256), 0, s, ntiles, indptr);
  SF_LAUNCH_CHECK("scan_totals_kernel");
  hipLaunchKernelGGL(scan_final_kernel, dim3((unsigned)ntiles), dim3(256), 0, s, counts, M, indptr, 1);
  SF_LAUNCH_CHECK("scan_final_kernel");
  return SF_OK;
}

extern "C" int sf_compact(const void* f, int64_t sfm, int64_t sfn, int f_dt, int64_t M, int64_t N,
                          const int64_t* indptr, int64_t nnz, int32_t* indices, void* values, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && N >= 0 && nnz >= 0, "sf_compact: negative size");
  SF_REQUIRE(sf_valid_dtype(f_dt), "sf_compact: bad dtype code %d", f_dt);
  SF_REQUIRE(N < (1LL << 31), "sf_compact: N too large for int32 indices");
  if (M == 0 || nnz == 0) return SF_OK;
  SF_REQUIRE(f && indptr && indices && values, "sf_compact: NULL buffer");
  const int es = sf_dtype_size(f_dt);
  const bool vec = vec_rows(f, sfm, sfn, es);
  hipStream_t s = (hipStream_t)stream;
  const char* fp = (const char*)f;
  char* vp = (char*)values;
  if (vec) {  // one workgroup per row
    SF_REQUIRE(M <= INT32_MAX, "sf_compact: M too large for one workgroup per row");
    const dim3 grid((unsigned)M);
    if (N * es <= CR_ONE_GROUP) {
      if (es == 2) hipLaunchKernelGGL((compact_row_kernel<2, 4, 8, false, true>), grid, dim3(256), 0, s, fp, sfm, N, indptr, nnz, indices, vp);
      else hipLaunchKernelGGL((compact_row_kernel<4, 4, 8, false, true>), grid, dim3(256), 0, s, fp, sfm, N, indptr, nnz, indices, vp);
    } else if (N * es >= CR_LONG_ROW) {
      if (es == 2) hipLaunchKernelGGL((compact_row_kernel<2, 16, 2, true, false>), grid, dim3(1024), 0, s, fp, sfm, N, indptr, nnz, indices, vp);
      else hipLaunchKernelGGL((compact_row_kernel<4, 16, 2, true, false>), grid, dim3(1024), 0, s, fp, sfm, N, indptr, nnz, indices, vp);
    } else {
      if (es == 2) hipLaunchKernelGGL((compact_row_kernel<2, 8, 4, true, false>), grid, dim3(512), 0, s, fp, sfm, N, indptr, nnz, indices, vp);
      else hipLaunchKernelGGL((compact_row_kernel<4, 8, 4, true, false>), grid, dim3(512), 0, s, fp, sfm, N, indptr, nnz, indices, vp);
    }
  } else {  // strided rows: one wave per row, element by element
    dim3 grid((unsigned)((M + WPB - 1) / WPB)), block(256);
    if (es == 2) hipLaunchKernelGGL((compact_kernel<2>), grid, block, 0, s, fp, sfm, sfn, M, N, indptr, nnz, indices, vp);
    else hipLaunchKernelGGL((compact_kernel<4>), grid, block, 0, s, fp, sfm, sfn, M, N, indptr, nnz, indices, vp);
  }
  SF_LAUNCH_CHECK("compact_kernel");
  return SF_OK;
}

extern "C" int sf_csr_to_dense(const int64_t* indptr, int64_t width, const int32_t* indices, const void* values,
                               int val_dt, int64_t nnz, int64_t M, int64_t d_sae, void* out, int64_t som,
                               int out_dt, void* stream) {
  sf_clear_error();
  SF_REQUIRE(M >= 0 && d_sae >= 0 && nnz >= 0, "sf_csr_to_dense: negative size");
  SF_REQUIRE(sf_valid_dtype(val_dt) && sf_valid_dtype(out_dt), "sf_csr_to_dense: bad dtype code");
  SF_REQUIRE(indptr != nullptr || width >= 0, "sf_csr_to_dense: fixed-width rows need width >= 0");
  SF_REQUIRE(som >= d_sae, "sf_csr_to_dense: row stride %lld < d_sae %lld", (long long)som, (long long)d_sae);
  if (M == 0 || d_sae == 0) return SF_OK;
  SF_REQUIRE(out && (nnz == 0 || (indices && values)), "sf_csr_to_dense: NULL buffer");
  SF_REQUIRE(M < (1LL << 31), "sf_csr_to_dense: M too large");
  hipLaunchKernelGGL(csr_to_dense_kernel, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream, indptr, width,
                     indices, values, val_dt, nnz, M, d_sae, (char*)out, som, out_dt);
  SF_LAUNCH_CHECK("csr_to_dense_kernel");
  return SF_OK;
}
