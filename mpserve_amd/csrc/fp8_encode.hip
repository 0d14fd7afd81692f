// GPU sidecar builder for the FP8 + Huffman weight path (MI355X, gfx950).
//
// Produces byte for byte what the reference's host builder
// huffman_build_fp8_decode_tables_entry (kernel/build_huffman.cu:292-969) produces:
//   1. histogram of (scale, fp8) keys x BF16 symbols    (:392-401)   -> LDS-atomic pre-aggregation
//                                                                        into a global open-addressing table
//   2. keys in ascending order -> table id (gid)         (:403-412)   -> ballot/prefix-scan compaction,
//                                                                        counting sort by key, scans
//   3. per key: ESC selection, package-merge lengths,    (:445-578)   -> one work-item per key
//      canonical codes in (count asc, sym asc) order,
//      decode LUT and packed 4-bit lengths
//   4. row buckets, bucket_table, U/uniq/uidx            (:582-783)   -> host (O(rows)) + one work-item
//                                                                        per bucket
//   5. per-lane bit counts, u32 lane starts, 64-bit      (:786-925)   -> two passes over the lanes with a
//      aligned bucket bases, MSB-first packing                           scan between them; words shared by
//                                                                        two lanes are merged with atomicOr
// The reference is single-threaded; here every O(N) pass runs on the GPU.
#include <hip/hip_runtime.h>

#include <rocprim/device/device_segmented_radix_sort.hpp>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "mps_common.h"

namespace mps {
namespace {

constexpr uint64_t kEmpty = ~0ull;
constexpr uint32_t kRaw = 1u << 31;  // code word flag: 16 raw symbol bits follow the code

// Code word of one element: bits 0..15 code, 16..20 length, bit 31 raw16 follows.
__device__ __forceinline__ uint32_t cw_len(uint32_t cw) { return (cw >> 16) & 0x1Fu; }

__device__ __forceinline__ uint64_t hash64(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

// ---------------------------------------------------------------------------
// Element addressing shared by the passes.
// ---------------------------------------------------------------------------
struct ScaleMap {
  // mode 0: scalar/per-row (row_sidx[row]); mode 1: block-2D (block_sidx[br*nb1+bc])
  int32_t mode;
  const uint16_t *row_sidx;
  const uint16_t *block_sidx;
  int64_t sb0, sb1, nb1;
};

__device__ __forceinline__ uint32_t sidx_of(const ScaleMap &S, int64_t row, int64_t col) {
  if (S.mode == 0) return S.row_sidx[row];
  return S.block_sidx[(row / S.sb0) * S.nb1 + col / S.sb1];
}

// key40 = sidx << 24 | fp8 << 16 | sym
__device__ __forceinline__ uint64_t key40(uint32_t sidx, uint32_t q, uint32_t sym) {
  return ((uint64_t)sidx << 24) | ((uint64_t)q << 16) | (uint64_t)sym;
}

// ---------------------------------------------------------------------------
// 1. Histogram
// ---------------------------------------------------------------------------
constexpr int kHistBlock = 256;
constexpr int kLdsSlots = 2048;

__device__ bool global_insert(uint64_t *keys, uint32_t *counts, uint64_t cap_mask, uint64_t k, uint32_t add) {
  uint64_t h = hash64(k) & cap_mask;
  for (uint64_t probe = 0; probe <= cap_mask; ++probe) {
    unsigned long long *slot = reinterpret_cast<unsigned long long *>(keys + h);
    unsigned long long cur = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (cur == kEmpty) {
      cur = atomicCAS(slot, (unsigned long long)kEmpty, (unsigned long long)k);
      if (cur == kEmpty) cur = k;
    }
    if (cur == k) {
      atomicAdd(counts + h, add);
      return true;
    }
    h = (h + 1) & cap_mask;
  }
  return false;
}

__global__ __launch_bounds__(kHistBlock) void hist_kernel(const uint16_t *__restrict__ bf16, const uint8_t *__restrict__ fp8,
                                                          int64_t n, int64_t m, ScaleMap S, uint32_t qmask,
                                                          int64_t elems_per_block, uint64_t *keys, uint32_t *counts,
                                                          uint64_t cap_mask, uint32_t *overflow) {
  __shared__ unsigned long long s_keys[kLdsSlots];
  __shared__ uint32_t s_cnt[kLdsSlots];
  for (int i = threadIdx.x; i < kLdsSlots; i += kHistBlock) {
    s_keys[i] = kEmpty;
    s_cnt[i] = 0;
  }
  __syncthreads();
  const int64_t numel = n * m;
  const int64_t e0 = (int64_t)blockIdx.x * elems_per_block;
  const int64_t e1 = e0 + elems_per_block < numel ? e0 + elems_per_block : numel;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += kHistBlock) {
    const int64_t row = e / m, col = e - row * m;
    const uint64_t k = key40(sidx_of(S, row, col), fp8[e] & qmask, bf16[e]);
    // LDS first: a short probe, then the global table.
    uint32_t h = (uint32_t)(hash64(k) & (kLdsSlots - 1));
    bool done = false;
    for (int probe = 0; probe < 16 && !done; ++probe) {
      unsigned long long cur = s_keys[h];
      if (cur == kEmpty) {
        cur = atomicCAS(&s_keys[h], (unsigned long long)kEmpty, (unsigned long long)k);
        if (cur == kEmpty) cur = k;
      }
      if (cur == k) {
        atomicAdd(&s_cnt[h], 1u);
        done = true;
      }
      h = (h + 1) & (kLdsSlots - 1);
    }
    if (!done && !global_insert(keys, counts, cap_mask, k, 1)) atomicOr(overflow, 1u);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kLdsSlots; i += kHistBlock) {
    if (s_keys[i] != kEmpty && !global_insert(keys, counts, cap_mask, s_keys[i], s_cnt[i])) atomicOr(overflow, 1u);
  }
}

// ---------------------------------------------------------------------------
// 2. Compaction (ballot + prefix within the wave, one atomic per wave)
// ---------------------------------------------------------------------------
__global__ void compact_kernel(const uint64_t *__restrict__ keys, const uint32_t *__restrict__ counts, uint64_t cap,
                               uint64_t *ckey, uint32_t *ccount, uint32_t *cslot, uint32_t *num) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = i < cap && keys[i] != kEmpty;
  const uint64_t mask = __ballot(live);
  const int lane = threadIdx.x & 63;
  const uint32_t below = (uint32_t)__popcll(mask & ((1ull << lane) - 1ull));
  uint32_t base = 0;
  if (lane == 0 && mask) base = atomicAdd(num, (uint32_t)__popcll(mask));
  base = __shfl(base, 0);
  if (live) {
    ckey[base + below] = keys[i];
    ccount[base + below] = counts[i];
    cslot[base + below] = (uint32_t)i;
  }
}

// ---------------------------------------------------------------------------
// Generic exclusive scan of u32 (two levels, up to 2^24 elements per level pair)
// ---------------------------------------------------------------------------
constexpr int kScanBlock = 1024;
constexpr int kScanItems = 4;  // per thread
constexpr int kScanTile = kScanBlock * kScanItems;

__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *s_tmp, uint32_t *total) {
  // wave-level inclusive scan, then across waves
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == 63) s_tmp[wave] = x;
  __syncthreads();
  if (wave == 0) {
    const int nw = blockDim.x >> 6;
    uint32_t w = lane < nw ? s_tmp[lane] : 0u;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t y = __shfl_up(w, d);
      if (lane >= d) w += y;
    }
    if (lane < nw) s_tmp[lane] = w;
  }
  __syncthreads();
  const uint32_t before = wave > 0 ? s_tmp[wave - 1] : 0u;
  if (total) *total = s_tmp[(blockDim.x >> 6) - 1];
  __syncthreads();
  return before + x - v;
}

__global__ __launch_bounds__(kScanBlock) void scan_tiles(const uint32_t *in, uint32_t *out, uint64_t n,
                                                         uint32_t *tile_sums) {
  __shared__ uint32_t s_tmp[16];
  const uint64_t base = (uint64_t)blockIdx.x * kScanTile + (uint64_t)threadIdx.x * kScanItems;
  uint32_t v[kScanItems], s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    v[j] = base + j < n ? in[base + j] : 0u;
    s += v[j];
  }
  uint32_t total = 0;
  uint32_t ex = block_exclusive_scan(s, s_tmp, &total);
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    if (base + j < n) out[base + j] = ex;
    ex += v[j];
  }
  if (threadIdx.x == 0 && tile_sums) tile_sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(kScanBlock) void scan_add(uint32_t *out, uint64_t n, const uint32_t *tile_offsets) {
  const uint64_t base = (uint64_t)blockIdx.x * kScanTile + (uint64_t)threadIdx.x * kScanItems;
  const uint32_t add = tile_offsets[blockIdx.x];
#pragma unroll
  for (int j = 0; j < kScanItems; ++j)
    if (base + j < n) out[base + j] += add;
}

// ---------------------------------------------------------------------------
// Table grouping
// ---------------------------------------------------------------------------
__global__ void table_count_kernel(const uint64_t *ckey, uint32_t num, uint32_t *tcount) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < num) atomicAdd(tcount + (ckey[i] >> 16), 1u);
}

__global__ void nonzero_kernel(const uint32_t *tcount, uint64_t T, uint32_t *nz) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < T) nz[i] = tcount[i] ? 1u : 0u;
}

__global__ void scatter_kernel(const uint64_t *ckey, const uint32_t *ccount, const uint32_t *cslot, uint32_t num,
                               const uint32_t *toff, uint32_t *tfill, uint16_t *seg_sym, uint32_t *seg_cnt,
                               uint32_t *seg_slot) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num) return;
  const uint64_t tk = ckey[i] >> 16;
  const uint32_t pos = toff[tk] + atomicAdd(tfill + tk, 1u);
  seg_sym[pos] = (uint16_t)(ckey[i] & 0xFFFF);
  seg_cnt[pos] = ccount[i];
  seg_slot[pos] = cslot[i];
}

// gid -> table key, for the non-empty table keys in ascending order
__global__ void table_list_kernel(const uint32_t *tcount, const uint32_t *tgid, uint64_t T, uint32_t *gid_tkey) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < T && tcount[i]) gid_tkey[tgid[i]] = (uint32_t)i;
}

// ---------------------------------------------------------------------------
// 3. Code book of one key (one work-item per key)
// ---------------------------------------------------------------------------
// Items (count, sym) compare as the reference's std::pair<int, uint16_t>.
// Items are ordered by (count, symbol) with counts compared as int, as the
// reference's item lists are: the sort key flips the count's sign bit so that
// an unsigned 64-bit compare orders it as a signed one.
__device__ __forceinline__ uint64_t item_key(uint32_t count, uint32_t sym) {
  return ((uint64_t)(count ^ 0x80000000u) << 16) | (sym & 0xFFFFu);
}
__device__ __forceinline__ uint32_t key_count(uint64_t k) { return (uint32_t)(k >> 16) ^ 0x80000000u; }

// Sorts n (key, value) pairs by key (distinct keys) with a bottom-up merge
// sort over runs of 16 made by insertion; tk/tv are scratch of n each. The
// result is in k/v.
__device__ void sort_pairs(uint64_t *k, uint32_t *v, uint64_t *tk, uint32_t *tv, uint32_t n) {
  constexpr uint32_t kRun = 16;
  for (uint32_t lo = 0; lo < n; lo += kRun) {
    const uint32_t hi = lo + kRun < n ? lo + kRun : n;
    for (uint32_t i = lo + 1; i < hi; ++i) {
      const uint64_t x = k[i];
      const uint32_t y = v[i];
      uint32_t j = i;
      for (; j > lo && k[j - 1] > x; --j) {
        k[j] = k[j - 1];
        v[j] = v[j - 1];
      }
      k[j] = x;
      v[j] = y;
    }
  }
  uint64_t *sk = k, *dk = tk;
  uint32_t *sv = v, *dv = tv;
  for (uint32_t width = kRun; width < n; width *= 2) {
    for (uint32_t lo = 0; lo < n; lo += 2 * width) {
      const uint32_t mid = lo + width < n ? lo + width : n;
      const uint32_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      uint32_t i = lo, j = mid, o = lo;
      while (i < mid && j < hi) {
        const bool right = sk[j] < sk[i];
        dk[o] = right ? sk[j] : sk[i];
        dv[o] = right ? sv[j] : sv[i];
        i += right ? 0u : 1u;
        j += right ? 1u : 0u;
        ++o;
      }
      for (; i < mid; ++i, ++o) {
        dk[o] = sk[i];
        dv[o] = sv[i];
      }
      for (; j < hi; ++j, ++o) {
        dk[o] = sk[j];
        dv[o] = sv[j];
      }
    }
    uint64_t *t64 = sk;
    sk = dk;
    dk = t64;
    uint32_t *t32 = sv;
    sv = dv;
    dv = t32;
  }
  if (sk != k) {
    for (uint32_t i = 0; i < n; ++i) {
      k[i] = sk[i];
      v[i] = sv[i];
    }
  }
}

// Code lengths of n ascending weights by the package-merge (build_huffman.cu:46-118),
// in the level-count form: with cur_0 = the leaves and cur_j = merge(leaves,
// pairs of cur_{j-1}) (leaf first on equal weight, at most 4(n-1) items), the
// reference selects the first 2(n-1) items of cur_{L-1} and, recursively, the
// first 2p items of cur_{j-1} for the p packages selected in cur_j. Leaves keep
// their sorted order in every cur_j, so a level's selected prefix holds leaves
// 0..x_j-1, and a leaf's length is the number of levels with x_j above its
// index. The levels are built once, bottom-up (O(L n)); each keeps only a bit
// per item saying whether it is a leaf (masks: L words per 32 items of 4(n-1)),
// and the selection then walks them top-down. A and B hold 4(n-1) ints each.
__device__ void package_merge_lengths(const int32_t *w, int n, int L, int32_t *A, int32_t *B, uint32_t *masks,
                                      int32_t *lens) {
  for (int i = 0; i < n; ++i) lens[i] = 0;
  if (n == 1) {
    lens[0] = 1;
    return;
  }
  const int keep = 4 * (n - 1);
  const int words = (keep + 31) / 32;
  int na[16];
  int cur = n < keep ? n : keep;
  for (int i = 0; i < cur; ++i) A[i] = w[i];
  for (int i = 0; i < words; ++i) {
    const int b = cur - 32 * i;
    masks[i] = b >= 32 ? 0xFFFFFFFFu : (b > 0 ? (1u << b) - 1u : 0u);
  }
  na[0] = cur;
  for (int j = 1; j < L; ++j) {
    uint32_t *mk = masks + j * words;
    for (int i = 0; i < words; ++i) mk[i] = 0u;
    const int np = cur / 2;  // packages: pairs (0,1), (2,3), ... of the previous level
    int a = 0, b = 0, o = 0;
    while (o < keep && (a < n || b < np)) {
      const int32_t pw = b < np ? (int32_t)((uint32_t)A[2 * b] + (uint32_t)A[2 * b + 1]) : 0;
      if (a < n && (b >= np || w[a] <= pw)) {
        B[o] = w[a++];
        mk[o >> 5] |= 1u << (o & 31);
      } else {
        B[o] = pw;
        ++b;
      }
      ++o;
    }
    int32_t *t = A;
    A = B;
    B = t;
    cur = o;
    na[j] = o;
  }
  int c = 2 * (n - 1);  // selected prefix at the top level
  for (int level = L - 1; level >= 0 && c > 0; --level) {
    const int cc = c < na[level] ? c : na[level];
    const uint32_t *mk = masks + level * words;
    int x = 0;
    for (int i = 0; i < cc / 32; ++i) x += __popc(mk[i]);
    if (cc & 31) x += __popc(mk[cc / 32] & ((1u << (cc & 31)) - 1u));
    for (int i = 0; i < x; ++i) lens[i] += 1;
    c = 2 * (cc - x);
  }
}

// ESC rules of the three builders:
//  kEscFp8        build_huffman.cu:485-535 and :205-228: esc_sym = smallest u16 not kept, list re-sorted
//                 (count asc, sym asc), the ESC entries' nibble is len | 8.
//  kEscAwqBucket  build_huffman.cu:1775-1836: as kEscFp8 (ESC weight at least 1), but the ESC code
//                 has length L and its one LUT entry has nibble 15.
//  kEscAwqByScale build_huffman.cu:1251-1316: esc_sym = smallest u16 absent from all of the key's
//                 symbols (0xFFFF if none is); the list stays (count desc, sym asc) with ESC last, and
//                 the lengths package-merge returns for the sorted weights apply to it by position;
//                 ESC length L, nibble 15.
enum : int { kEscFp8 = 0, kEscAwqBucket = 1, kEscAwqByScale = 2 };

struct CodebookArgs {
  const uint32_t *gid_tkey;
  const uint32_t *toff;
  const uint32_t *tcount;
  uint16_t *seg_sym;  // sorted in place
  uint32_t *seg_cnt;
  uint32_t *seg_slot;  // hash slot of each entry; sorted along with seg_sym/seg_cnt
  int32_t *ws;        // per key: kWsSort ints per histogram entry + kWsPerItem per list item (ws_size_kernel)
  const uint32_t *ws_off;
  const uint16_t *scale_values;  // sidx -> scale u16
  uint32_t *cw_slot;             // hash slot -> code word
  uint16_t *decode_syms;         // [G, 2^L]
  uint8_t *decode_lens;          // [G, 2^(L-1)] (or [G,1] when L == 1)
  uint16_t *table_scale;
  uint16_t *table_fp8;
  uint32_t G;
  int L;
  int esc_mode;  // kEscFp8, kEscAwqBucket or kEscAwqByScale
  uint32_t *err;
  uint32_t *esc_stats;  // [0] keys with ESC, [1] collisions (elements)
};

// Workspace per key, in ints: sort scratch over the ni histogram entries
// (two 64-bit keys and two 32-bit values each, later the entry -> list
// position map), then per list item (nmax = min(ni, 2^L)): weights, symbols,
// lengths, histogram index, code, two package-merge lists of 4 items, the
// level masks (2, plus kWsFixed for the per-level rounding) and the sorted
// weights.
constexpr uint32_t kWsSort = 6;
constexpr uint32_t kWsPerItem = 16;
constexpr uint32_t kWsFixed = 20;

// One work-item per key: ESC selection, package-merge lengths, canonical codes
// in list order, the decode table and the code word of each histogram entry.
__global__ void codebook_kernel(CodebookArgs a) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= a.G) return;
  const int L = a.L;
  const uint32_t T = 1u << L;
  const uint32_t tk = a.gid_tkey[g];
  const uint32_t off = a.toff[tk];
  const uint32_t ni = a.tcount[tk];
  uint16_t *sym = a.seg_sym + off;
  uint32_t *cnt = a.seg_cnt + off;
  uint32_t *slot = a.seg_slot + off;
  a.table_scale[g] = a.scale_values[tk >> 8];
  a.table_fp8[g] = (uint16_t)(tk & 0xFF);
  uint16_t *dsyms = a.decode_syms + (uint64_t)g * T;
  uint8_t *dlens = a.decode_lens + (uint64_t)g * (T / 2 > 0 ? T / 2 : 1);

  if (ni == 1) {
    for (uint32_t j = 0; j < T; ++j) dsyms[j] = sym[0];
    for (uint32_t j = 0; j < T / 2; ++j) dlens[j] = 0x11;  // len 1 in both nibbles
    a.cw_slot[slot[0]] = (1u << 16) | 0u;
    return;
  }
  int32_t *ws = a.ws + a.ws_off[g];
  uint64_t *sk = reinterpret_cast<uint64_t *>(ws);  // 8-byte aligned: every key's size is even
  uint64_t *tk64 = sk + ni;
  uint32_t *sv = reinterpret_cast<uint32_t *>(tk64 + ni);
  uint32_t *tv = sv + ni;
  const uint32_t nmax = ni < T ? ni : T;
  int32_t *lw = ws + kWsSort * ni;  // weights of the coded list
  int32_t *ls = lw + nmax;          // its symbols
  int32_t *lens = ls + nmax;
  int32_t *hidx = lens + nmax;      // histogram entry of each list item (-1: the ESC item)
  uint32_t *code = reinterpret_cast<uint32_t *>(hidx + nmax);
  int32_t *A = reinterpret_cast<int32_t *>(code + nmax);
  int32_t *Bv = A + 4 * nmax;
  uint32_t *masks = reinterpret_cast<uint32_t *>(Bv + 4 * nmax);  // L * ceil(4(nmax-1)/32) <= 2 nmax + 16
  int32_t *sw = reinterpret_cast<int32_t *>(masks + 2 * nmax + 16);  // sorted weights (kEscAwqByScale)

  // (count asc, sym asc)
  for (uint32_t i = 0; i < ni; ++i) {
    sk[i] = item_key(cnt[i], sym[i]);
    sv[i] = slot[i];
  }
  sort_pairs(sk, sv, tk64, tv, ni);
  for (uint32_t i = 0; i < ni; ++i) {
    sym[i] = (uint16_t)(sk[i] & 0xFFFFu);
    cnt[i] = key_count(sk[i]);
    slot[i] = sv[i];
  }

  uint32_t nl = 0;
  bool use_esc = false;
  uint32_t esc_sym = 0;
  if (ni > T) {
    // ESC (build_huffman.cu:485-535): keep the 2^L-1 most frequent by (count
    // desc, sym asc); ESC weight = sum of the rest. In (count asc, sym asc)
    // order, count groups are taken from the top, each from its smallest symbol.
    use_esc = true;
    const uint32_t keep = T - 1;
    uint32_t taken = 0;
    int64_t i = (int64_t)ni - 1;
    while (taken < keep && i >= 0) {
      int64_t j = i;
      while (j > 0 && cnt[j - 1] == cnt[i]) --j;
      const uint32_t gsize = (uint32_t)(i - j + 1);
      const uint32_t take = gsize < keep - taken ? gsize : keep - taken;
      for (uint32_t t = 0; t < take; ++t) {
        lw[nl] = (int32_t)cnt[j + t];
        ls[nl] = sym[j + t];
        hidx[nl] = (int32_t)(j + t);
        ++nl;
      }
      taken += take;
      i = j - 1;
    }
    // ESC weight: total minus kept (int sums as in the reference)
    uint32_t total = 0;
    for (uint32_t t = 0; t < ni; ++t) total += cnt[t];
    uint32_t kept_sum = 0;
    for (uint32_t t = 0; t < nl; ++t) kept_sum += (uint32_t)lw[t];
    const uint32_t esc_w = total - kept_sum;
    if (a.esc_mode == kEscAwqByScale) {
      // Smallest u16 absent from all ni (distinct) symbols: the largest c with
      // #{sym < c} == c, found by bisection over c in [0, 65536].
      uint32_t lo = 0, hi = 65536;
      while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        uint32_t below = 0;
        for (uint32_t t = 0; t < ni; ++t) below += sym[t] < mid;
        if (below == mid) lo = mid;
        else hi = mid - 1;
      }
      esc_sym = lo > 0xFFFFu ? 0xFFFFu : lo;
      // The list keeps its (count desc, sym asc) order with ESC last; the
      // package-merge gets the same weights ascending: the kept ones reversed,
      // the ESC weight merged in.
      const int32_t ew = (int32_t)esc_w;
      uint32_t o = 0;
      bool placed = false;
      for (int64_t t = (int64_t)nl - 1; t >= 0; --t) {
        if (!placed && ew <= lw[t]) {
          sw[o++] = ew;
          placed = true;
        }
        sw[o++] = lw[t];
      }
      if (!placed) sw[o++] = ew;
      lw[nl] = ew;
      ls[nl] = (int32_t)esc_sym;
      hidx[nl] = -1;
      ++nl;
      atomicAdd(&a.esc_stats[0], 1u);
    } else {
      // smallest u16 not among the kept: their symbols sorted
      for (uint32_t t = 0; t < nl; ++t) {
        sk[t] = (uint64_t)(uint32_t)ls[t];
        sv[t] = 0u;
      }
      sort_pairs(sk, sv, tk64, tv, nl);
      uint32_t cand = 0;
      for (uint32_t p = 0; p < nl; ++p) {
        if ((uint32_t)sk[p] == cand) ++cand;
        else if ((uint32_t)sk[p] > cand) break;
      }
      esc_sym = cand & 0xFFFF;
      lw[nl] = (a.esc_mode == kEscAwqBucket && (int32_t)esc_w <= 0) ? 1 : (int32_t)esc_w;
      ls[nl] = (int32_t)esc_sym;
      hidx[nl] = -1;
      ++nl;
      // the list in (count asc, sym asc) order, with each item's histogram entry
      for (uint32_t t = 0; t < nl; ++t) {
        sk[t] = item_key((uint32_t)lw[t], (uint32_t)ls[t]);
        sv[t] = (uint32_t)hidx[t];
      }
      sort_pairs(sk, sv, tk64, tv, nl);
      for (uint32_t t = 0; t < nl; ++t) {
        lw[t] = (int32_t)key_count(sk[t]);
        ls[t] = (int32_t)(sk[t] & 0xFFFFu);
        hidx[t] = (int32_t)sv[t];
      }
      atomicAdd(&a.esc_stats[0], 1u);
    }
  } else {
    for (uint32_t t = 0; t < ni; ++t) {
      lw[t] = (int32_t)cnt[t];
      ls[t] = sym[t];
      hidx[t] = (int32_t)t;
    }
    nl = ni;
  }
  if (a.esc_mode == kEscAwqByScale && use_esc) {
    // package-merge sorts the weights and returns lengths by sorted position;
    // the reference applies them to its (unsorted) list position by position
    package_merge_lengths(sw, (int)nl, L, A, Bv, masks, lens);
  } else {
    // weights are ascending (as int); package-merge expects that order
    package_merge_lengths(lw, (int)nl, L, A, Bv, masks, lens);
  }
  // canonical codes (build_huffman.cu:171-203), handed out in list order
  uint32_t bl_count[16], next_code[16];
  for (int b = 0; b < 16; ++b) bl_count[b] = 0;
  for (uint32_t t = 0; t < nl; ++t) {
    if (lens[t] <= 0 || lens[t] > L) {
      atomicOr(a.err, 2u);
      return;
    }
    if (use_esc && a.esc_mode != kEscFp8 && (uint32_t)ls[t] == esc_sym) lens[t] = L;  // AWQ: ESC code has length L
    bl_count[lens[t]]++;
  }
  uint32_t cd = 0;
  next_code[0] = 0;
  for (int b = 1; b < 16; ++b) {
    cd = (cd + bl_count[b - 1]) << 1;
    next_code[b] = cd;
  }
  for (uint32_t j = 0; j < T; ++j) dsyms[j] = 0;
  for (uint32_t j = 0; j < T / 2; ++j) dlens[j] = 0;
  uint32_t esc_cw = 0;
  for (uint32_t t = 0; t < nl; ++t) {
    const int len = lens[t];
    const uint32_t c = next_code[len]++;
    code[t] = c;
    const uint32_t fill = 1u << (L - len);
    const uint32_t base = c << (L - len);
    const bool is_esc = use_esc && (uint32_t)ls[t] == esc_sym;
    const uint32_t nib = is_esc ? (a.esc_mode == kEscFp8 ? ((uint32_t)len | 0x8u) : 15u) : (uint32_t)len;
    for (uint32_t f = 0; f < fill; ++f) {
      const uint32_t e = base + f;
      dsyms[e] = (uint16_t)ls[t];
      if (T >= 2) dlens[e >> 1] |= (uint8_t)((nib & 0xF) << ((e & 1) * 4));
    }
    if (is_esc) esc_cw = ((uint32_t)len << 16) | (c & 0xFFFF);
  }
  // code word of every histogram entry: its list item's code; an entry outside
  // the list is coded as ESC + 16 raw bits, except one whose symbol is esc_sym
  // (the ESC code alone: a collision, as in the reference)
  int32_t *pos_of = ws;  // the sort scratch is free again
  for (uint32_t t = 0; t < ni; ++t) pos_of[t] = -1;
  for (uint32_t p = 0; p < nl; ++p)
    if (hidx[p] >= 0) pos_of[hidx[p]] = (int32_t)p;
  for (uint32_t t = 0; t < ni; ++t) {
    const int32_t p = pos_of[t];
    uint32_t cw;
    if (p >= 0) {
      cw = ((uint32_t)lens[p] << 16) | (code[p] & 0xFFFF);
    } else if (use_esc && sym[t] == esc_sym) {
      cw = esc_cw;
      atomicAdd(&a.esc_stats[1], cnt[t]);
    } else {
      cw = esc_cw | kRaw;  // outside the map: ESC code + raw16
    }
    a.cw_slot[slot[t]] = cw;
  }
}

// ---------------------------------------------------------------------------
// Codebooks with a wave per key (L <= 11). The keys' histogram entries are
// sorted for all keys at once beforehand (a segmented radix sort of the
// (count, symbol) keys), so a key's entries arrive in (count asc, sym asc)
// order; one 64-lane workgroup then builds its codebook in LDS, with the same
// results as codebook_kernel:
//  - the ESC keep set from the sorted counts: the entry at ni - (2^L - 1) fixes
//    the boundary count c; every entry above c's run is kept, and the run's
//    first ones (smallest symbols) fill the rest;
//  - esc_sym from a 65536-bit set of the symbols in LDS;
//  - the package-merge levels built once, bottom-up, each level's outputs split
//    over the lanes by merge path (a lane finds how many leaves precede its
//    first output by binary search, then merges its run), keeping a leaf bit
//    per item; the selection then counts leaf bits top-down;
//  - canonical codes in list order, ranked within each length by ballots;
//  - the decode table, and each histogram entry's code word from its list
//    position, which follows from its sorted index.
// NMAX bounds the coded list (min(ni, 2^L)); keys outside (lo, hi] of it are
// left to another launch.
// ---------------------------------------------------------------------------
constexpr int kCbLanes = 64;

__device__ __forceinline__ uint32_t cb_count(uint64_t k) { return key_count(k); }
__device__ __forceinline__ uint32_t cb_sym(uint64_t k) { return (uint32_t)(k & 0xFFFFu); }

template <int NMAX>
struct CbShared {
  int32_t lw[NMAX];   // list weights
  int32_t sw[NMAX];   // ascending weights for the package-merge (kEscAwqByScale ESC lists)
  int32_t hidx[NMAX];
  uint16_t ls[NMAX];  // list symbols
  uint16_t code[NMAX];
  uint8_t lens[NMAX];
  union {
    struct {
      int32_t A[4 * NMAX];
      int32_t B[4 * NMAX];
      uint32_t masks[11 * (NMAX / 8) + 16];
    } pm;
    uint32_t symset[65536 / 32];
    uint8_t nibs[2048];
  } u;
  int32_t na[16];
  int32_t xs[16];
  uint32_t blc[16], ncode[16], run[16];
  uint32_t acc, acc2, flag;
};

// Sum over the workgroup's 64 lanes (one wave), returned to every lane.
__device__ __forceinline__ uint32_t cb_sum(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o);
  return v;
}
__device__ __forceinline__ uint32_t cb_min(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = (uint32_t)__shfl_xor((int)v, o);
    v = w < v ? w : v;
  }
  return v;
}

// First index in [lo, hi) of the sorted keys whose count is >= c (lower) or > c (upper).
__device__ __forceinline__ uint32_t cb_bound(const uint64_t *k, uint32_t lo, uint32_t hi, uint32_t c, bool upper) {
  const int32_t ci = (int32_t)c;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    const int32_t x = (int32_t)cb_count(k[mid]);
    if (upper ? x <= ci : x < ci) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

template <int NMAX>
__global__ __launch_bounds__(kCbLanes) void codebook_wave_kernel(CodebookArgs a, const uint64_t *__restrict__ skeys,
                                                                 const uint32_t *__restrict__ sslots, uint32_t lo_n,
                                                                 uint32_t hi_n) {
  __shared__ CbShared<NMAX> S;
  const uint32_t g = blockIdx.x;
  const int lane = threadIdx.x;
  const int L = a.L;
  const uint32_t T = 1u << L;
  const uint32_t tk = a.gid_tkey[g];
  const uint32_t off = a.toff[tk];
  const uint32_t ni = a.tcount[tk];
  const uint32_t nmax = ni < T ? ni : T;
  if (nmax <= lo_n || nmax > hi_n) return;
  const uint64_t *keys = skeys + off;
  const uint32_t *slots = sslots + off;
  uint16_t *dsyms = a.decode_syms + (uint64_t)g * T;
  uint8_t *dlens = a.decode_lens + (uint64_t)g * (T / 2 > 0 ? T / 2 : 1);
  if (lane == 0) {
    a.table_scale[g] = a.scale_values[tk >> 8];
    a.table_fp8[g] = (uint16_t)(tk & 0xFF);
  }
  if (ni == 1) {
    for (uint32_t j = lane; j < T; j += kCbLanes) dsyms[j] = (uint16_t)cb_sym(keys[0]);
    for (uint32_t j = lane; j < T / 2; j += kCbLanes) dlens[j] = 0x11;  // len 1 in both nibbles
    if (lane == 0) a.cw_slot[slots[0]] = (1u << 16) | 0u;
    return;
  }

  // --- the coded list ---
  const bool use_esc = ni > T;
  const uint32_t keep = T - 1;
  uint32_t nl, s0 = 0, s1 = 0, r = 0, esc_sym = 0, esc_pos = 0;
  int32_t esc_w = 0;
  if (!use_esc) {
    for (uint32_t p = lane; p < ni; p += kCbLanes) {
      const uint64_t k = keys[p];
      S.lw[p] = (int32_t)cb_count(k);
      S.ls[p] = (uint16_t)cb_sym(k);
      S.hidx[p] = (int32_t)p;
    }
    nl = ni;
  } else {
    // kept: [s0, s0 + r) and [s1, ni), the top 2^L - 1 by (count desc, sym asc)
    const uint32_t c = cb_count(keys[ni - keep]);
    s0 = cb_bound(keys, 0, ni, c, false);
    s1 = cb_bound(keys, s0, ni, c, true);
    r = keep - (ni - s1);
    uint32_t tot = 0, kept = 0;
    for (uint32_t t = lane; t < ni; t += kCbLanes) {
      const uint32_t cnt = cb_count(keys[t]);
      tot += cnt;
      kept += (t >= s1 || (t >= s0 && t < s0 + r)) ? cnt : 0u;
    }
    tot = cb_sum(tot);
    kept = cb_sum(kept);
    const uint32_t ew = tot - kept;  // int sums as in the reference
    // esc_sym: the smallest u16 absent from the key's symbols (kEscAwqByScale) or
    // from the kept ones (the other builders)
    for (uint32_t i = lane; i < 65536 / 32; i += kCbLanes) S.u.symset[i] = 0u;
    __syncthreads();
    for (uint32_t t = lane; t < ni; t += kCbLanes) {
      const bool in = a.esc_mode == kEscAwqByScale || t >= s1 || (t >= s0 && t < s0 + r);
      if (in) {
        const uint32_t sy = cb_sym(keys[t]);
        atomicOr(&S.u.symset[sy >> 5], 1u << (sy & 31));
      }
    }
    __syncthreads();
    uint32_t cand = 0xFFFFFFFFu;
    for (uint32_t i = lane; i < 65536 / 32; i += kCbLanes) {
      const uint32_t wv = ~S.u.symset[i];
      if (wv != 0u && cand == 0xFFFFFFFFu) cand = 32u * i + (uint32_t)__builtin_ctz(wv);
    }
    cand = cb_min(cand);
    __syncthreads();
    if (a.esc_mode == kEscAwqByScale) {
      esc_sym = cand == 0xFFFFFFFFu ? 0xFFFFu : cand;
      esc_w = (int32_t)ew;
      // (count desc, sym asc), ESC last: an entry of a run [g0, g1) above c sits
      // at (ni - g1) + (t - g0); the boundary run's first r follow them
      for (uint32_t t = lane; t < ni; t += kCbLanes) {
        uint32_t pos;
        if (t >= s1) {
          const uint32_t cc = cb_count(keys[t]);
          const uint32_t g0 = cb_bound(keys, s1, t + 1, cc, false);
          const uint32_t g1 = cb_bound(keys, t, ni, cc, true);
          pos = (ni - g1) + (t - g0);
        } else if (t >= s0 && t < s0 + r) {
          pos = (ni - s1) + (t - s0);
        } else {
          continue;
        }
        const uint64_t k = keys[t];
        S.lw[pos] = (int32_t)cb_count(k);
        S.ls[pos] = (uint16_t)cb_sym(k);
        S.hidx[pos] = (int32_t)t;
      }
      // the package-merge's weights, ascending: the kept counts in sorted order
      // with the ESC weight merged in (ties: any order gives the same list)
      uint32_t e_pos = 0;
      {
        uint32_t below = 0;  // kept counts < the ESC weight (as int)
        for (uint32_t j = lane; j < keep; j += kCbLanes) {
          const uint32_t t = j < r ? s0 + j : s1 + (j - r);
          below += (int32_t)cb_count(keys[t]) < esc_w ? 1u : 0u;
        }
        e_pos = cb_sum(below);
      }
      for (uint32_t j = lane; j < keep; j += kCbLanes) {
        const uint32_t t = j < r ? s0 + j : s1 + (j - r);
        S.sw[j + (j >= e_pos ? 1u : 0u)] = (int32_t)cb_count(keys[t]);
      }
      if (lane == 0) {
        S.sw[e_pos] = esc_w;
        S.lw[keep] = esc_w;
        S.ls[keep] = (uint16_t)esc_sym;
        S.hidx[keep] = -1;
      }
      esc_pos = keep;
    } else {
      esc_sym = cand & 0xFFFFu;
      esc_w = (a.esc_mode == kEscAwqBucket && (int32_t)ew <= 0) ? 1 : (int32_t)ew;
      // (count asc, sym asc): the kept entries in sorted order with the ESC item
      // inserted at its key's place
      const uint64_t ek = item_key((uint32_t)esc_w, esc_sym);
      uint32_t below = 0;
      for (uint32_t j = lane; j < keep; j += kCbLanes) {
        const uint32_t t = j < r ? s0 + j : s1 + (j - r);
        below += item_key(cb_count(keys[t]), cb_sym(keys[t])) < ek ? 1u : 0u;
      }
      esc_pos = cb_sum(below);
      for (uint32_t j = lane; j < keep; j += kCbLanes) {
        const uint32_t t = j < r ? s0 + j : s1 + (j - r);
        const uint32_t p = j + (j >= esc_pos ? 1u : 0u);
        const uint64_t k = keys[t];
        S.lw[p] = (int32_t)cb_count(k);
        S.ls[p] = (uint16_t)cb_sym(k);
        S.hidx[p] = (int32_t)t;
      }
      if (lane == 0) {
        S.lw[esc_pos] = esc_w;
        S.ls[esc_pos] = (uint16_t)esc_sym;
        S.hidx[esc_pos] = -1;
      }
    }
    nl = T;
    if (lane == 0) atomicAdd(&a.esc_stats[0], 1u);
  }
  __syncthreads();

  // --- package-merge lengths (see package_merge_lengths) ---
  {
    const int32_t *W = (use_esc && a.esc_mode == kEscAwqByScale) ? S.sw : S.lw;
    const int n = (int)nl;
    const int keep_pm = 4 * (n - 1);
    const int words = (keep_pm + 31) / 32;
    int32_t *A = S.u.pm.A, *B = S.u.pm.B;
    int cur = n < keep_pm ? n : keep_pm;
    for (int i = lane; i < cur; i += kCbLanes) A[i] = W[i];
    for (int i = lane; i < words; i += kCbLanes) {
      const int b = cur - 32 * i;
      S.u.pm.masks[i] = b >= 32 ? 0xFFFFFFFFu : (b > 0 ? (1u << b) - 1u : 0u);
    }
    if (lane == 0) S.na[0] = cur;
    __syncthreads();
    for (int j = 1; j < L; ++j) {
      const int np = cur / 2;
      const int o = keep_pm < n + np ? keep_pm : n + np;
      const int chunk = (((o + kCbLanes - 1) / kCbLanes) + 31) & ~31;  // whole mask words per lane
      const int k0 = lane * chunk;
      const int k1 = k0 + chunk < o ? k0 + chunk : o;
      uint32_t *mk = S.u.pm.masks + j * words;
      if (k0 < k1) {
        // leaves among the first k0 outputs: the largest a with leaf a-1 before package k0-a
        int lo = k0 - np > 0 ? k0 - np : 0, hi = k0 < n ? k0 : n;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          const int b = k0 - mid;
          const bool ok = b >= np || W[mid - 1] <= (int32_t)((uint32_t)A[2 * b] + (uint32_t)A[2 * b + 1]);
          if (ok) lo = mid;
          else hi = mid - 1;
        }
        int ai = lo, bi = k0 - lo;
        uint32_t bits = 0;
        for (int k = k0; k < k1; ++k) {
          const int32_t pw = bi < np ? (int32_t)((uint32_t)A[2 * bi] + (uint32_t)A[2 * bi + 1]) : 0;
          const bool leaf = ai < n && (bi >= np || W[ai] <= pw);
          B[k] = leaf ? W[ai] : pw;
          ai += leaf ? 1 : 0;
          bi += leaf ? 0 : 1;
          bits |= (leaf ? 1u : 0u) << (k & 31);
          if ((k & 31) == 31 || k + 1 == k1) {
            mk[k >> 5] = bits;
            bits = 0;
          }
        }
      }
      __syncthreads();
      int32_t *t = A;
      A = B;
      B = t;
      cur = o;
      if (lane == 0) S.na[j] = o;
    }
    __syncthreads();
    // top-down: leaves among each level's selected prefix
    int c = 2 * (n - 1);
    int nx = 0;
    for (int level = L - 1; level >= 0 && c > 0; --level) {
      const int cc = c < S.na[level] ? c : S.na[level];
      const uint32_t *mk = S.u.pm.masks + level * words;
      uint32_t x = 0;
      for (int i = lane; i < (cc + 31) / 32; i += kCbLanes) {
        const uint32_t wv = mk[i];
        const int rem = cc - 32 * i;
        x += __popc(rem >= 32 ? wv : (wv & ((1u << rem) - 1u)));
      }
      x = cb_sum(x);
      if (lane == 0) S.xs[nx] = (int32_t)x;
      ++nx;
      c = 2 * (cc - (int)x);
    }
    __syncthreads();
    for (int i = lane; i < n; i += kCbLanes) {
      int len = 0;
      for (int q = 0; q < nx; ++q) len += i < S.xs[q] ? 1 : 0;
      S.lens[i] = (uint8_t)len;
    }
    if (lane < 16) {
      S.blc[lane] = 0;
      S.run[lane] = 0;
    }
    if (lane == 0) S.flag = 0;
    __syncthreads();
  }

  // --- canonical codes (build_huffman.cu:171-203), handed out in list order ---
  for (uint32_t p = lane; p < nl; p += kCbLanes) {
    int len = S.lens[p];
    if (len <= 0 || len > L) {
      S.flag = 1;
      continue;
    }
    if (use_esc && a.esc_mode != kEscFp8 && (uint32_t)S.ls[p] == esc_sym) {  // AWQ: ESC code has length L
      len = L;
      S.lens[p] = (uint8_t)L;
    }
    atomicAdd(&S.blc[len], 1u);
  }
  __syncthreads();
  if (S.flag) {
    if (lane == 0) atomicOr(a.err, 2u);
    return;
  }
  if (lane == 0) {
    uint32_t cd = 0;
    S.ncode[0] = 0;
    for (int b = 1; b < 16; ++b) {
      cd = (cd + S.blc[b - 1]) << 1;
      S.ncode[b] = cd;
    }
  }
  __syncthreads();
  for (uint32_t base = 0; base < nl; base += kCbLanes) {
    const uint32_t p = base + lane;
    const int len = p < nl ? S.lens[p] : 0;
    uint32_t rank = 0, mine = 0;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int v = 1; v <= L; ++v) {
      const uint64_t m = __ballot(len == v);
      if (len == v) rank = (uint32_t)__popcll(m & below);
      if (lane == v) mine = (uint32_t)__popcll(m);  // lane v keeps length v's count of this chunk
    }
    if (p < nl) S.code[p] = (uint16_t)(S.ncode[len] + S.run[len] + rank);
    __syncthreads();
    if (lane >= 1 && lane <= L) S.run[lane] += mine;
    __syncthreads();
  }

  // --- decode table ---
  for (uint32_t j = lane; j < T; j += kCbLanes) {
    dsyms[j] = 0;
    S.u.nibs[j] = 0;
  }
  __syncthreads();
  uint32_t esc_cw = 0;
  for (uint32_t p = lane; p < nl; p += kCbLanes) {
    const uint32_t len = S.lens[p];
    const uint32_t c = S.code[p];
    const bool is_esc = use_esc && (uint32_t)S.ls[p] == esc_sym;
    const uint32_t nib = is_esc ? (a.esc_mode == kEscFp8 ? (len | 0x8u) : 15u) : len;
    const uint32_t fill = 1u << (L - len);
    const uint32_t base = c << (L - len);
    for (uint32_t f = 0; f < fill; ++f) {
      dsyms[base + f] = S.ls[p];
      S.u.nibs[base + f] = (uint8_t)nib;
    }
  }
  if (use_esc) esc_cw = ((uint32_t)S.lens[esc_pos] << 16) | (S.code[esc_pos] & 0xFFFFu);
  __syncthreads();
  for (uint32_t j = lane; j < (T / 2 > 0 ? T / 2 : 1); j += kCbLanes)
    dlens[j] = T >= 2 ? (uint8_t)((S.u.nibs[2 * j] & 0xF) | ((S.u.nibs[2 * j + 1] & 0xF) << 4)) : 0;

  // --- code word of every histogram entry, from its list position ---
  for (uint32_t t = lane; t < ni; t += kCbLanes) {
    int32_t p = -1;
    if (!use_esc) {
      p = (int32_t)t;
    } else if (a.esc_mode == kEscAwqByScale) {
      if (t >= s1) {
        const uint32_t cc = cb_count(keys[t]);
        const uint32_t g0 = cb_bound(keys, s1, t + 1, cc, false);
        const uint32_t g1 = cb_bound(keys, t, ni, cc, true);
        p = (int32_t)((ni - g1) + (t - g0));
      } else if (t >= s0 && t < s0 + r) {
        p = (int32_t)((ni - s1) + (t - s0));
      }
    } else {
      int32_t j = -1;
      if (t >= s0 && t < s0 + r) j = (int32_t)(t - s0);
      else if (t >= s1) j = (int32_t)(r + (t - s1));
      if (j >= 0) p = j + (j >= (int32_t)esc_pos ? 1 : 0);
    }
    uint32_t cw;
    if (p >= 0) {
      cw = ((uint32_t)S.lens[p] << 16) | (S.code[p] & 0xFFFFu);
    } else if (cb_sym(keys[t]) == esc_sym) {
      cw = esc_cw;  // a data symbol equal to esc_sym: the ESC code alone
      atomicAdd(&a.esc_stats[1], cb_count(keys[t]));
    } else {
      cw = esc_cw | kRaw;  // outside the map: ESC code + raw16
    }
    a.cw_slot[slots[t]] = cw;
  }
}

__global__ void item_keys_kernel(const uint16_t *__restrict__ sym, const uint32_t *__restrict__ cnt, uint64_t n,
                                 uint64_t *__restrict__ keys) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) keys[i] = item_key(cnt[i], sym[i]);
}

__global__ void segment_bounds_kernel(const uint32_t *gid_tkey, const uint32_t *toff, const uint32_t *tcount,
                                      uint32_t G, uint32_t *beg, uint32_t *end) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  const uint32_t tk = gid_tkey[g];
  beg[g] = toff[tk];
  end[g] = toff[tk] + tcount[tk];
}

__global__ void ws_size_kernel(const uint32_t *gid_tkey, const uint32_t *tcount, uint32_t G, uint32_t T,
                               uint32_t *sz) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  const uint32_t ni = tcount[gid_tkey[g]];
  const uint32_t n = kWsSort * ni + kWsPerItem * (ni < T ? ni : T) + kWsFixed;
  sz[g] = (n + 1u) & ~1u;  // even, so that every key's 64-bit sort keys are 8-byte aligned
}

// ---------------------------------------------------------------------------
// 4. bucket_table, U / unique gids / fp8 -> uidx (one work-item per bucket)
// ---------------------------------------------------------------------------
// qvals = 256 (FP8 bytes; also U/uniq/uidx) or 16 (AWQ int4 values, build_huffman.cu:1973-1982).
__global__ void bucket_table_kernel(const uint16_t *bucket_sidx, uint32_t B, int qvals, const uint32_t *tcount,
                                    const uint32_t *tgid, int32_t *btab, int32_t *bU, int32_t *uniq, int16_t *uidx) {
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const uint64_t t0 = (uint64_t)bucket_sidx[b] * 256;
  if (qvals != 256) {
    for (int c = 0; c < qvals; ++c) btab[b * qvals + c] = tcount[t0 + c] ? (int32_t)tgid[t0 + c] : -1;
    return;
  }
  int32_t U = 0;
  for (int c = 0; c < 256; ++c) {
    const int32_t gid = tcount[t0 + c] ? (int32_t)tgid[t0 + c] : -1;
    btab[b * 256 + c] = gid;
    uniq[b * 256 + c] = -1;
    uidx[b * 256 + c] = -1;
  }
  // gids of one bucket are distinct (one scale, distinct fp8 bytes): first-appearance order is fp8 order
  for (int c = 0; c < 256; ++c) {
    const int32_t gid = btab[b * 256 + c];
    if (gid < 0) continue;
    uniq[b * 256 + U] = gid;
    uidx[b * 256 + c] = (int16_t)U;
    ++U;
  }
  bU[b] = U;
}

// ---------------------------------------------------------------------------
// 5. Bitstream
// ---------------------------------------------------------------------------
struct LaneArgs {
  const uint16_t *bf16;
  const uint8_t *fp8;
  ScaleMap S;
  int64_t m;
  const int32_t *row_offsets;
  const int32_t *row_indices;
  const int32_t *col_start;
  const int32_t *col_len;
  const int32_t *row_col;     // per-row column start (groups of the by-scale layout) or null
  uint32_t qmask;
  const uint32_t *lane_base;  // [B+1] cumulative k_eff
  uint32_t B;
  int64_t k;
  const uint64_t *keys;
  const uint32_t *cw_slot;
  uint64_t cap_mask;
  uint32_t *cw_elem;    // [numel]
  uint32_t *lane_bits;  // [B, k+1] (count of lane t at [b][t+1])
  uint32_t *err;
};

__device__ __forceinline__ uint32_t find_bucket(const uint32_t *lane_base, uint32_t B, uint32_t g) {
  uint32_t lo = 0, hi = B;  // largest b with lane_base[b] <= g
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (lane_base[mid] <= g) lo = mid;
    else hi = mid;
  }
  return lo;
}

__global__ void lane_bits_kernel(LaneArgs a) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= a.lane_base[a.B]) return;
  const uint32_t b = find_bucket(a.lane_base, a.B, g);
  const uint32_t t = g - a.lane_base[b];
  const int32_t ra = a.row_offsets[b], rows = a.row_offsets[b + 1] - ra;
  const int32_t c0 = a.row_col ? 0 : a.col_start[b], cl = a.col_len[b];
  const int64_t total = (int64_t)rows * cl;
  const int64_t k_eff = a.lane_base[b + 1] - a.lane_base[b];
  uint64_t bits = 0;
  for (int64_t e = t; e < total; e += k_eff) {
    const int64_t rr = e / cl, cc = e - rr * cl;
    const int64_t row = a.row_indices[ra + rr];
    const int64_t col = (a.row_col ? a.row_col[ra + rr] : c0) + cc;
    const int64_t idx = row * a.m + col;
    const uint64_t k = key40(sidx_of(a.S, row, col), a.fp8[idx] & a.qmask, a.bf16[idx]);
    uint64_t h = hash64(k) & a.cap_mask;
    while (a.keys[h] != k) {
      if (a.keys[h] == kEmpty) {
        atomicOr(a.err, 4u);
        return;
      }
      h = (h + 1) & a.cap_mask;
    }
    const uint32_t cw = a.cw_slot[h];
    a.cw_elem[idx] = cw;
    bits += cw_len(cw) + ((cw & kRaw) ? 16u : 0u);
  }
  a.lane_bits[(uint64_t)b * (a.k + 1) + t + 1] = (uint32_t)bits;
}

// per bucket: inclusive scan of lane bits -> u32 starts; inactive lanes -> starts[k_eff]
__global__ __launch_bounds__(1024) void lane_starts_kernel(uint32_t *startbit, const uint32_t *lane_base, int64_t k,
                                                           uint32_t *bucket_bits) {
  __shared__ uint32_t s_tmp[16];
  const uint32_t b = blockIdx.x;
  const int64_t k_eff = lane_base[b + 1] - lane_base[b];
  uint32_t *sb = startbit + (uint64_t)b * (k + 1);
  const int t = threadIdx.x;
  const uint32_t v = t < k_eff ? sb[t + 1] : 0u;
  uint32_t total = 0;
  const uint32_t ex = block_exclusive_scan(v, s_tmp, &total);
  __syncthreads();
  if (t == 0) sb[0] = 0;
  if (t < k) sb[t + 1] = t < k_eff ? ex + v : total;
  if (t == 0) bucket_bits[b] = total;
}

struct PackArgs {
  const uint16_t *bf16;
  int64_t m;
  const int32_t *row_offsets;
  const int32_t *row_indices;
  const int32_t *col_start;
  const int32_t *col_len;
  const int32_t *row_col;  // as LaneArgs::row_col
  const uint32_t *lane_base;
  uint32_t B;
  int64_t k;
  const uint32_t *cw_elem;
  const uint32_t *startbit;
  const int64_t *bit_base;
  unsigned long long *bits;  // zeroed
};

__device__ __forceinline__ void flush_word(unsigned long long *bits, uint64_t w, uint64_t v, uint64_t first_w,
                                           uint64_t last_w) {
  if (v == 0) return;
  if (w == first_w || w == last_w) atomicOr(bits + w, (unsigned long long)v);
  else bits[w] = v;
}

__global__ void pack_kernel(PackArgs a) {
  const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= a.lane_base[a.B]) return;
  const uint32_t b = find_bucket(a.lane_base, a.B, g);
  const uint32_t t = g - a.lane_base[b];
  const int32_t ra = a.row_offsets[b], rows = a.row_offsets[b + 1] - ra;
  const int32_t c0 = a.row_col ? 0 : a.col_start[b], cl = a.col_len[b];
  const int64_t total = (int64_t)rows * cl;
  const int64_t k_eff = a.lane_base[b + 1] - a.lane_base[b];
  const uint32_t *sb = a.startbit + (uint64_t)b * (a.k + 1);
  const uint64_t p0 = (uint64_t)a.bit_base[b] + sb[t];
  const uint64_t p1 = (uint64_t)a.bit_base[b] + sb[t + 1];
  if (p1 == p0) return;
  const uint64_t first_w = p0 >> 6, last_w = (p1 - 1) >> 6;
  uint64_t w = first_w;
  uint64_t acc = 0;          // current word, MSB-first
  uint32_t used = (uint32_t)(p0 & 63);  // bits of the current word already taken by earlier lanes
  auto put = [&](uint32_t v, uint32_t n) {  // append the low n bits of v
    while (n > 0) {
      const uint32_t room = 64 - used;
      const uint32_t take = n < room ? n : room;
      const uint64_t part = (uint64_t)((v >> (n - take)) & ((take == 32) ? 0xFFFFFFFFu : ((1u << take) - 1u)));
      acc |= part << (room - take);
      used += take;
      n -= take;
      if (used == 64) {
        flush_word(a.bits, w, acc, first_w, last_w);
        ++w;
        acc = 0;
        used = 0;
      }
    }
  };
  for (int64_t e = t; e < total; e += k_eff) {
    const int64_t rr = e / cl, cc = e - rr * cl;
    const int64_t idx = (int64_t)a.row_indices[ra + rr] * a.m + (a.row_col ? a.row_col[ra + rr] : c0) + cc;
    const uint32_t cw = a.cw_elem[idx];
    put(cw & 0xFFFF, cw_len(cw));
    if (cw & kRaw) put(a.bf16[idx], 16);
  }
  if (used > 0) flush_word(a.bits, w, acc, first_w, last_w);
}

// ---------------------------------------------------------------------------
// Host orchestration
// ---------------------------------------------------------------------------
template <typename T>
struct DevBuf {
  T *p = nullptr;
  size_t n = 0;
  ~DevBuf() { reset(); }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  hipError_t alloc(size_t count) {
    reset();
    n = count;
    return hipMalloc(&p, sizeof(T) * (count > 0 ? count : 1));
  }
};

hipError_t device_scan(const uint32_t *in, uint32_t *out, uint64_t n, hipStream_t s, uint32_t *total_out) {
  // exclusive scan; total (sum of all) written to host *total_out when non-null (synchronises)
  if (n == 0) {
    if (total_out) *total_out = 0;
    return hipSuccess;
  }
  const uint64_t tiles = (n + kScanTile - 1) / kScanTile;
  DevBuf<uint32_t> sums, sums_ex;
  hipError_t e = sums.alloc(tiles + 1);
  if (e != hipSuccess) return e;
  if ((e = sums_ex.alloc(tiles + 1)) != hipSuccess) return e;
  hipLaunchKernelGGL(scan_tiles, dim3((unsigned)tiles), dim3(kScanBlock), 0, s, in, out, n, sums.p);
  if (tiles > 1) {
    if ((e = device_scan(sums.p, sums_ex.p, tiles, s, nullptr)) != hipSuccess) return e;
    hipLaunchKernelGGL(scan_add, dim3((unsigned)tiles), dim3(kScanBlock), 0, s, out, n, sums_ex.p);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (total_out) {
    uint32_t last_in = 0, last_out = 0;
    if ((e = hipMemcpyAsync(&last_in, in + n - 1, 4, hipMemcpyDeviceToHost, s)) != hipSuccess) return e;
    if ((e = hipMemcpyAsync(&last_out, out + n - 1, 4, hipMemcpyDeviceToHost, s)) != hipSuccess) return e;
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
    *total_out = last_in + last_out;
  }
  return hipSuccess;
}

}  // namespace
}  // namespace mps

using namespace mps;

// Result object: device arrays in the reference's 17-output order.
struct mps_fp8_sidecar {
  DevBuf<uint16_t> decode_syms, table_scale, table_fp8, bucket_scale;
  DevBuf<uint8_t> decode_lens;
  DevBuf<int32_t> bucket_row_offsets, row_indices, bucket_table, bucket_col_start, bucket_col_len, bucket_U,
      bucket_unique_gid;
  DevBuf<uint32_t> bucket_thread_startbit;
  DevBuf<int64_t> bucket_bit_base, shape_nmk;
  DevBuf<uint64_t> bitstream;
  DevBuf<int16_t> bucket_fp8_uidx;
  int64_t sizes[17] = {};
  int64_t stats[4] = {};  // esc keys, esc collision elements, distinct (key, symbol) pairs, hash capacity
};

namespace mps {
namespace {

enum : int { kFmtFp8 = kEscFp8, kFmtAwqBucket = kEscAwqBucket, kFmtAwqByScale = kEscAwqByScale };

// One builder run, after the entry point's own argument checks.
struct EncodeSpec {
  const uint16_t *bf16;
  const uint8_t *q;  // FP8 bytes, or AWQ int4 values (low nibble)
  const uint16_t *scales;
  int64_t n, m, scale_numel;
  bool scalar, per_row, block2d;
  int64_t nb0, nb1, sb0, sb1;
  int64_t L, k, group_cap;
  int format;
};

int encode_impl(const EncodeSpec &sp, hipStream_t s, mps_fp8_sidecar **out) {
  const int64_t n = sp.n, m = sp.m, numel = n * m, L = sp.L, kth = sp.k, scale_numel = sp.scale_numel;
  const bool scale_scalar = sp.scalar, scale_block2d = sp.block2d;
  const int64_t nb0 = sp.nb0, nb1 = sp.nb1, sb0 = sp.sb0, sb1 = sp.sb1;
  const uint32_t qmask = sp.format == kFmtFp8 ? 0xFFu : 0x0Fu;
  const int qvals = sp.format == kFmtFp8 ? 256 : 16;
  hipError_t e;
#define HC(x)                                                   \
  do {                                                          \
    if ((e = (x)) != hipSuccess) return hip_fail(e, #x);        \
  } while (0)

  // --- scales to host, dense scale index (sorted unique values) ---
  std::vector<uint16_t> hsc((size_t)scale_numel);
  HC(hipMemcpyAsync(hsc.data(), sp.scales, sizeof(uint16_t) * scale_numel, hipMemcpyDeviceToHost, s));
  HC(hipStreamSynchronize(s));
  std::vector<uint16_t> uniq_sc(hsc);
  std::sort(uniq_sc.begin(), uniq_sc.end());
  uniq_sc.erase(std::unique(uniq_sc.begin(), uniq_sc.end()), uniq_sc.end());
  const uint32_t S = (uint32_t)uniq_sc.size();
  auto sidx_of_value = [&](uint16_t v) -> uint16_t {
    return (uint16_t)(std::lower_bound(uniq_sc.begin(), uniq_sc.end(), v) - uniq_sc.begin());
  };

  // --- buckets (build_huffman.cu:611-696), host ---
  std::vector<int32_t> row_indices, row_offsets{0}, col_start, col_len;
  std::vector<uint16_t> bucket_scale;
  std::vector<uint16_t> row_sidx, block_sidx;
  std::vector<int32_t> group_col;  // by scale: column start of each group
  const bool by_scale = sp.format == kFmtAwqByScale;
  if (by_scale) {
    // quantisation groups (row, column start) bucketed by exact scale, scales
    // ascending, groups in (row, column) order, <= group_cap a bucket
    // (build_huffman.cu:1350-1385)
    const int64_t gsz = scale_block2d ? sb1 : m;
    const int64_t gpr = scale_block2d ? nb1 : 1;
    if (!scale_block2d) {
      row_sidx.resize((size_t)n);
      for (int64_t r = 0; r < n; ++r) row_sidx[(size_t)r] = sidx_of_value(scale_scalar ? hsc[0] : hsc[(size_t)r]);
    } else {
      block_sidx.resize((size_t)(nb0 * nb1));
      for (int64_t i = 0; i < nb0 * nb1; ++i) block_sidx[(size_t)i] = sidx_of_value(hsc[(size_t)i]);
    }
    std::vector<uint64_t> gk((size_t)(n * gpr));
    for (int64_t r = 0; r < n; ++r)
      for (int64_t bc = 0; bc < gpr; ++bc) {
        const uint16_t v = scale_scalar ? hsc[0] : !scale_block2d ? hsc[(size_t)r] : hsc[(size_t)((r / sb0) * nb1 + bc)];
        gk[(size_t)(r * gpr + bc)] = ((uint64_t)v << 40) | (uint64_t)(r * gpr + bc);
      }
    std::sort(gk.begin(), gk.end());
    size_t i = 0;
    while (i < gk.size()) {
      size_t j = i;
      while (j < gk.size() && (gk[j] >> 40) == (gk[i] >> 40)) ++j;
      for (size_t off = i; off < j; off += (size_t)sp.group_cap) {
        const size_t take = std::min<size_t>((size_t)sp.group_cap, j - off);
        for (size_t q = 0; q < take; ++q) {
          const int64_t gi = (int64_t)(gk[off + q] & 0xFFFFFFFFFFull);
          row_indices.push_back((int32_t)(gi / gpr));
          group_col.push_back((int32_t)((gi % gpr) * gsz));
        }
        bucket_scale.push_back((uint16_t)(gk[i] >> 40));
        col_start.push_back(0);
        col_len.push_back((int32_t)gsz);
        row_offsets.push_back((int32_t)row_indices.size());
      }
      i = j;
    }
  } else if (!scale_block2d) {
    row_sidx.resize((size_t)n);
    std::vector<std::pair<uint16_t, int32_t>> order((size_t)n);
    for (int64_t r = 0; r < n; ++r) {
      const uint16_t v = scale_scalar ? hsc[0] : hsc[(size_t)r];
      order[(size_t)r] = {v, (int32_t)r};
      row_sidx[(size_t)r] = sidx_of_value(v);
    }
    std::stable_sort(order.begin(), order.end(),
                     [](const std::pair<uint16_t, int32_t> &x, const std::pair<uint16_t, int32_t> &y) {
                       return x.first < y.first;
                     });
    size_t i = 0;
    while (i < order.size()) {
      size_t j = i;
      while (j < order.size() && order[j].first == order[i].first) ++j;
      for (size_t off = i; off < j; off += 128) {
        const size_t take = std::min<size_t>(128, j - off);
        for (size_t q = 0; q < take; ++q) row_indices.push_back(order[off + q].second);
        bucket_scale.push_back(order[i].first);
        col_start.push_back(0);
        col_len.push_back((int32_t)m);
        row_offsets.push_back((int32_t)row_indices.size());
      }
      i = j;
    }
  } else {
    block_sidx.resize((size_t)(nb0 * nb1));
    for (int64_t i = 0; i < nb0 * nb1; ++i) block_sidx[(size_t)i] = sidx_of_value(hsc[(size_t)i]);
    for (int64_t br = 0; br < nb0; ++br) {
      for (int64_t bc = 0; bc < nb1; ++bc) {
        const uint16_t sc = hsc[(size_t)(br * nb1 + bc)];
        for (int64_t off = 0; off < sb0; off += 128) {
          const int64_t take = std::min<int64_t>(128, sb0 - off);
          for (int64_t q = 0; q < take; ++q) row_indices.push_back((int32_t)(br * sb0 + off + q));
          bucket_scale.push_back(sc);
          col_start.push_back((int32_t)(bc * sb1));
          col_len.push_back((int32_t)sb1);
          row_offsets.push_back((int32_t)row_indices.size());
        }
      }
    }
  }
  const uint32_t B = (uint32_t)bucket_scale.size();
  std::vector<uint32_t> lane_base(B + 1, 0);
  std::vector<uint16_t> bucket_sidx(B);
  for (uint32_t b = 0; b < B; ++b) {
    const int64_t total = (int64_t)(row_offsets[b + 1] - row_offsets[b]) * col_len[b];
    const int64_t k_eff = std::min<int64_t>(kth, std::max<int64_t>(1, total));
    lane_base[b + 1] = lane_base[b] + (uint32_t)k_eff;
    bucket_sidx[b] = sidx_of_value(bucket_scale[b]);
  }

  auto sc = std::make_unique<mps_fp8_sidecar>();
  DevBuf<uint16_t> d_row_sidx, d_block_sidx, d_bucket_sidx, d_scale_values;
  DevBuf<uint32_t> d_lane_base;
  HC(d_row_sidx.alloc(row_sidx.size()));
  HC(d_block_sidx.alloc(block_sidx.size()));
  HC(d_bucket_sidx.alloc(B));
  HC(d_scale_values.alloc(S));
  HC(d_lane_base.alloc(B + 1));
  if (!row_sidx.empty())
    HC(hipMemcpyAsync(d_row_sidx.p, row_sidx.data(), 2 * row_sidx.size(), hipMemcpyHostToDevice, s));
  if (!block_sidx.empty())
    HC(hipMemcpyAsync(d_block_sidx.p, block_sidx.data(), 2 * block_sidx.size(), hipMemcpyHostToDevice, s));
  HC(hipMemcpyAsync(d_bucket_sidx.p, bucket_sidx.data(), 2 * (size_t)B, hipMemcpyHostToDevice, s));
  HC(hipMemcpyAsync(d_scale_values.p, uniq_sc.data(), 2 * (size_t)S, hipMemcpyHostToDevice, s));
  HC(hipMemcpyAsync(d_lane_base.p, lane_base.data(), 4 * (size_t)(B + 1), hipMemcpyHostToDevice, s));

  HC(sc->bucket_scale.alloc(B));
  HC(sc->bucket_row_offsets.alloc(B + 1));
  HC(sc->row_indices.alloc(row_indices.size()));
  HC(sc->bucket_col_start.alloc(by_scale ? group_col.size() : (size_t)B));
  HC(sc->bucket_col_len.alloc(B));
  HC(hipMemcpyAsync(sc->bucket_scale.p, bucket_scale.data(), 2 * (size_t)B, hipMemcpyHostToDevice, s));
  HC(hipMemcpyAsync(sc->bucket_row_offsets.p, row_offsets.data(), 4 * (size_t)(B + 1), hipMemcpyHostToDevice, s));
  if (!row_indices.empty())
    HC(hipMemcpyAsync(sc->row_indices.p, row_indices.data(), 4 * row_indices.size(), hipMemcpyHostToDevice, s));
  if (by_scale) {
    if (!group_col.empty())
      HC(hipMemcpyAsync(sc->bucket_col_start.p, group_col.data(), 4 * group_col.size(), hipMemcpyHostToDevice, s));
  } else {
    HC(hipMemcpyAsync(sc->bucket_col_start.p, col_start.data(), 4 * (size_t)B, hipMemcpyHostToDevice, s));
  }
  HC(hipMemcpyAsync(sc->bucket_col_len.p, col_len.data(), 4 * (size_t)B, hipMemcpyHostToDevice, s));

  ScaleMap smap;
  smap.mode = scale_block2d ? 1 : 0;
  smap.row_sidx = d_row_sidx.p;
  smap.block_sidx = d_block_sidx.p;
  smap.sb0 = sb0;
  smap.sb1 = sb1;
  smap.nb1 = nb1;

  // --- 1. histogram (retry with a larger table on overflow) ---
  DevBuf<uint64_t> keys;
  DevBuf<uint32_t> counts, flags;  // flags: [0] overflow, [1] error bits, [2..3] esc stats, [4] compact count
  HC(flags.alloc(8));
  uint64_t cap = 1u << 16;
  while (cap < (uint64_t)std::min<int64_t>(numel, (int64_t)1 << 22) * 2) cap <<= 1;
  const int64_t per_block = 1 << 14;
  const unsigned hist_blocks = (unsigned)((numel + per_block - 1) / per_block);
  uint32_t hflags[8] = {};
  for (;;) {
    HC(keys.alloc(cap));
    HC(counts.alloc(cap));
    HC(hipMemsetAsync(keys.p, 0xFF, sizeof(uint64_t) * cap, s));
    HC(hipMemsetAsync(counts.p, 0, sizeof(uint32_t) * cap, s));
    HC(hipMemsetAsync(flags.p, 0, sizeof(uint32_t) * 8, s));
    hipLaunchKernelGGL(hist_kernel, dim3(hist_blocks), dim3(kHistBlock), 0, s, sp.bf16, sp.q, n, m, smap,
                       qmask, per_block, keys.p, counts.p, cap - 1, flags.p);
    HC(hipGetLastError());
    HC(hipMemcpyAsync(hflags, flags.p, sizeof(hflags), hipMemcpyDeviceToHost, s));
    HC(hipStreamSynchronize(s));
    if (!hflags[0]) break;
    if (cap >= ((uint64_t)1 << 34)) return fail(MPS_ERR_RUNTIME, "histogram table overflow");
    cap <<= 1;
  }

  // --- 2. compaction and grouping by (scale, fp8) key ---
  DevBuf<uint64_t> ckey;
  DevBuf<uint32_t> ccount, cslot;
  // bound for the compact arrays: count first
  uint32_t D = 0;
  {
    HC(ckey.alloc(cap));
    HC(ccount.alloc(cap));
    HC(cslot.alloc(cap));
    hipLaunchKernelGGL(compact_kernel, dim3((unsigned)((cap + 255) / 256)), dim3(256), 0, s, keys.p, counts.p, cap,
                       ckey.p, ccount.p, cslot.p, flags.p + 4);
    HC(hipGetLastError());
    HC(hipMemcpyAsync(&D, flags.p + 4, 4, hipMemcpyDeviceToHost, s));
    HC(hipStreamSynchronize(s));
  }
  const uint64_t T = (uint64_t)S * 256;
  DevBuf<uint32_t> tcount, toff, tfill, tnz, tgid;
  HC(tcount.alloc(T));
  HC(toff.alloc(T));
  HC(tfill.alloc(T));
  HC(tnz.alloc(T));
  HC(tgid.alloc(T));
  HC(hipMemsetAsync(tcount.p, 0, 4 * T, s));
  HC(hipMemsetAsync(tfill.p, 0, 4 * T, s));
  hipLaunchKernelGGL(table_count_kernel, dim3((D + 255) / 256), dim3(256), 0, s, ckey.p, D, tcount.p);
  HC(hipGetLastError());
  uint32_t D_check = 0, G = 0;
  HC(device_scan(tcount.p, toff.p, T, s, &D_check));
  hipLaunchKernelGGL(nonzero_kernel, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, s, tcount.p, T, tnz.p);
  HC(hipGetLastError());
  HC(device_scan(tnz.p, tgid.p, T, s, &G));
  if (D_check != D) return fail(MPS_ERR_RUNTIME, "internal error: histogram grouping mismatch");
  DevBuf<uint16_t> seg_sym;
  DevBuf<uint32_t> seg_cnt, seg_slot, gid_tkey, ws_off, cw_slot;
  HC(seg_sym.alloc(D));
  HC(seg_cnt.alloc(D));
  HC(seg_slot.alloc(D));
  HC(gid_tkey.alloc(G));
  hipLaunchKernelGGL(scatter_kernel, dim3((D + 255) / 256), dim3(256), 0, s, ckey.p, ccount.p, cslot.p, D, toff.p,
                     tfill.p, seg_sym.p, seg_cnt.p, seg_slot.p);
  hipLaunchKernelGGL(table_list_kernel, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, s, tcount.p, tgid.p, T,
                     gid_tkey.p);
  HC(hipGetLastError());

  // --- 3. code books ---
  const uint32_t Tsz = 1u << L;
  const uint32_t packed = Tsz / 2 > 0 ? Tsz / 2 : 1;
  HC(sc->decode_syms.alloc((size_t)G * Tsz));
  HC(sc->decode_lens.alloc((size_t)G * packed));
  HC(sc->table_scale.alloc(G));
  HC(sc->table_fp8.alloc(G));
  HC(cw_slot.alloc(cap));
  // Codebooks. L <= 11 (the FP8 and AWQ formats): the keys' histogram entries
  // are sorted for all keys at once, then a wave per key builds each codebook in
  // LDS (codebook_wave_kernel; one launch for lists of up to 512 items, one for
  // the larger). Longer codes (L up to 15, reachable through the op's max_len)
  // keep the work-item-per-key kernel and its global workspace.
  const bool wave_cb = L <= 11;
  DevBuf<uint64_t> keys_in, keys_sorted;
  DevBuf<uint32_t> slots_sorted, seg_beg, seg_end;
  DevBuf<char> sort_tmp;
  if (wave_cb && G) {
    HC(keys_in.alloc(D));
    HC(keys_sorted.alloc(D));
    HC(slots_sorted.alloc(D));
    HC(seg_beg.alloc(G));
    HC(seg_end.alloc(G));
    if (D)
      hipLaunchKernelGGL(item_keys_kernel, dim3((D + 255) / 256), dim3(256), 0, s, seg_sym.p, seg_cnt.p, (uint64_t)D,
                         keys_in.p);
    hipLaunchKernelGGL(segment_bounds_kernel, dim3((G + 255) / 256), dim3(256), 0, s, gid_tkey.p, toff.p, tcount.p, G,
                       seg_beg.p, seg_end.p);
    HC(hipGetLastError());
    size_t tmp_bytes = 0;
    HC(rocprim::segmented_radix_sort_pairs(nullptr, tmp_bytes, keys_in.p, keys_sorted.p, seg_slot.p, slots_sorted.p,
                                           D, G, seg_beg.p, seg_end.p, 0, 48, s));
    HC(sort_tmp.alloc(tmp_bytes));
    HC(rocprim::segmented_radix_sort_pairs(sort_tmp.p, tmp_bytes, keys_in.p, keys_sorted.p, seg_slot.p,
                                           slots_sorted.p, D, G, seg_beg.p, seg_end.p, 0, 48, s));
  }
  // per-key workspace of the work-item-per-key kernel, sized by each key's list length
  DevBuf<uint32_t> ws_sz;
  HC(ws_sz.alloc(G));
  HC(ws_off.alloc(G));
  uint32_t ws_total = 0;
  if (G && !wave_cb) {
    hipLaunchKernelGGL(ws_size_kernel, dim3((G + 255) / 256), dim3(256), 0, s, gid_tkey.p, tcount.p, G, Tsz,
                       ws_sz.p);
    HC(hipGetLastError());
    HC(device_scan(ws_sz.p, ws_off.p, G, s, &ws_total));
  }
  DevBuf<int32_t> ws;
  HC(ws.alloc(ws_total));
  CodebookArgs cba;
  cba.gid_tkey = gid_tkey.p;
  cba.toff = toff.p;
  cba.tcount = tcount.p;
  cba.seg_sym = seg_sym.p;
  cba.seg_cnt = seg_cnt.p;
  cba.seg_slot = seg_slot.p;
  cba.ws = ws.p;
  cba.ws_off = ws_off.p;
  cba.scale_values = d_scale_values.p;
  cba.cw_slot = cw_slot.p;
  cba.decode_syms = sc->decode_syms.p;
  cba.decode_lens = sc->decode_lens.p;
  cba.table_scale = sc->table_scale.p;
  cba.table_fp8 = sc->table_fp8.p;
  cba.G = G;
  cba.L = (int)L;
  cba.esc_mode = sp.format;
  cba.err = flags.p + 1;
  cba.esc_stats = flags.p + 2;
  if (G && wave_cb) {
    hipLaunchKernelGGL(codebook_wave_kernel<512>, dim3(G), dim3(kCbLanes), 0, s, cba, keys_sorted.p, slots_sorted.p,
                       0u, 512u);
    hipLaunchKernelGGL(codebook_wave_kernel<2048>, dim3(G), dim3(kCbLanes), 0, s, cba, keys_sorted.p,
                       slots_sorted.p, 512u, 2048u);
  } else if (G) {
    hipLaunchKernelGGL(codebook_kernel, dim3((G + 63) / 64), dim3(64), 0, s, cba);
  }
  HC(hipGetLastError());

  // --- 4. bucket tables ---
  const bool fp8 = sp.format == kFmtFp8;
  HC(sc->bucket_table.alloc((size_t)B * qvals));
  HC(sc->bucket_U.alloc(fp8 ? B : 0));
  HC(sc->bucket_unique_gid.alloc(fp8 ? (size_t)B * 256 : 0));
  HC(sc->bucket_fp8_uidx.alloc(fp8 ? (size_t)B * 256 : 0));
  if (B)
    hipLaunchKernelGGL(bucket_table_kernel, dim3((B + 63) / 64), dim3(64), 0, s, d_bucket_sidx.p, B, qvals, tcount.p,
                       tgid.p, sc->bucket_table.p, sc->bucket_U.p, sc->bucket_unique_gid.p, sc->bucket_fp8_uidx.p);
  HC(hipGetLastError());

  // --- 5. bitstream ---
  HC(sc->bucket_thread_startbit.alloc((size_t)B * (kth + 1)));
  HC(hipMemsetAsync(sc->bucket_thread_startbit.p, 0, 4 * (size_t)B * (kth + 1), s));
  DevBuf<uint32_t> cw_elem, bucket_bits;
  HC(cw_elem.alloc((size_t)numel));
  HC(bucket_bits.alloc(B));
  const uint32_t lanes = lane_base[B];
  LaneArgs la;
  la.bf16 = sp.bf16;
  la.fp8 = sp.q;
  la.qmask = qmask;
  la.row_col = by_scale ? sc->bucket_col_start.p : nullptr;
  la.S = smap;
  la.m = m;
  la.row_offsets = sc->bucket_row_offsets.p;
  la.row_indices = sc->row_indices.p;
  la.col_start = sc->bucket_col_start.p;
  la.col_len = sc->bucket_col_len.p;
  la.lane_base = d_lane_base.p;
  la.B = B;
  la.k = kth;
  la.keys = keys.p;
  la.cw_slot = cw_slot.p;
  la.cap_mask = cap - 1;
  la.cw_elem = cw_elem.p;
  la.lane_bits = sc->bucket_thread_startbit.p;
  la.err = flags.p + 1;
  if (lanes) hipLaunchKernelGGL(lane_bits_kernel, dim3((lanes + 255) / 256), dim3(256), 0, s, la);
  HC(hipGetLastError());
  if (B) hipLaunchKernelGGL(lane_starts_kernel, dim3(B), dim3(1024), 0, s, sc->bucket_thread_startbit.p,
                            d_lane_base.p, kth, bucket_bits.p);
  HC(hipGetLastError());
  std::vector<uint32_t> h_bucket_bits(B);
  if (B) HC(hipMemcpyAsync(h_bucket_bits.data(), bucket_bits.p, 4 * (size_t)B, hipMemcpyDeviceToHost, s));
  HC(hipMemcpyAsync(hflags, flags.p, sizeof(hflags), hipMemcpyDeviceToHost, s));
  HC(hipStreamSynchronize(s));
  if (hflags[1] & 2u) return fail(MPS_ERR_RUNTIME, "invalid code length");
  if (hflags[1] & 4u)
    return fail(MPS_ERR_RUNTIME, fp8 ? "missing enc table for (scale,fp8) key" : "missing enc table for (scale,qv) key");
  // 64-bit aligned bucket bases (build_huffman.cu:813-818), final cursor unaligned
  std::vector<int64_t> bit_base(B + 1, 0);
  int64_t pos = 0;
  for (uint32_t b = 0; b < B; ++b) {
    if (pos & 63) pos = (pos + 63) & ~(int64_t)63;
    bit_base[b] = pos;
    pos += h_bucket_bits[b];
  }
  bit_base[B] = pos;
  const int64_t W = (pos + 63) >> 6;
  HC(sc->bucket_bit_base.alloc(B + 1));
  HC(hipMemcpyAsync(sc->bucket_bit_base.p, bit_base.data(), 8 * (size_t)(B + 1), hipMemcpyHostToDevice, s));
  HC(sc->bitstream.alloc((size_t)W));
  if (W) HC(hipMemsetAsync(sc->bitstream.p, 0, 8 * (size_t)W, s));
  PackArgs pa;
  pa.bf16 = sp.bf16;
  pa.row_col = by_scale ? sc->bucket_col_start.p : nullptr;
  pa.m = m;
  pa.row_offsets = sc->bucket_row_offsets.p;
  pa.row_indices = sc->row_indices.p;
  pa.col_start = sc->bucket_col_start.p;
  pa.col_len = sc->bucket_col_len.p;
  pa.lane_base = d_lane_base.p;
  pa.B = B;
  pa.k = kth;
  pa.cw_elem = cw_elem.p;
  pa.startbit = sc->bucket_thread_startbit.p;
  pa.bit_base = sc->bucket_bit_base.p;
  pa.bits = reinterpret_cast<unsigned long long *>(sc->bitstream.p);
  if (lanes && W) hipLaunchKernelGGL(pack_kernel, dim3((lanes + 255) / 256), dim3(256), 0, s, pa);
  HC(hipGetLastError());
  const int64_t shape[4] = {n, m, kth, by_scale ? (int64_t)col_len.front() : 0};
  const int nshape = by_scale ? 4 : 3;
  HC(sc->shape_nmk.alloc(nshape));
  HC(hipMemcpyAsync(sc->shape_nmk.p, shape, 8 * nshape, hipMemcpyHostToDevice, s));
  HC(hipMemcpyAsync(hflags, flags.p, sizeof(hflags), hipMemcpyDeviceToHost, s));
  HC(hipStreamSynchronize(s));

  // by scale, slots 5, 6 and 8 hold the group offsets, group rows and group column starts
  const int64_t sizes[17] = {(int64_t)G * Tsz, (int64_t)G * packed, G, G, B, B + 1, (int64_t)row_indices.size(),
                             (int64_t)B * qvals, by_scale ? (int64_t)group_col.size() : B, by_scale ? 0 : B,
                             (int64_t)B * (kth + 1), B + 1, W, nshape, fp8 ? B : 0, fp8 ? (int64_t)B * 256 : 0,
                             fp8 ? (int64_t)B * 256 : 0};
  std::memcpy(sc->sizes, sizes, sizeof(sizes));
  sc->stats[0] = hflags[2];
  sc->stats[1] = hflags[3];
  sc->stats[2] = D;
  sc->stats[3] = (int64_t)cap;
  *out = sc.release();
  return MPS_OK;
#undef HC
}

}  // namespace
}  // namespace mps

extern "C" {

int mps_fp8_encode(const mps_fp8_encode_in *in, void *stream, mps_fp8_sidecar **out) {
  last_error().clear();
  if (!in || !out) return fail(MPS_ERR_INVALID_ARGUMENT, "inputs must be defined");
  *out = nullptr;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t L = in->max_len, kth = in->threads_per_block;
  if (L <= 0 || L > 15) return fail(MPS_ERR_INVALID_ARGUMENT, "max_len must be in [1, 15]");
  if (kth <= 0 || kth > 1024) return fail(MPS_ERR_INVALID_ARGUMENT, "threads_per_block must be in [1, 1024]");
  const int64_t numel = in->numel;
  if (in->ndim < 0 || in->ndim > 8 || in->scale_ndim < 0 || in->scale_ndim > 8)
    return fail(MPS_ERR_INVALID_ARGUMENT, "too many dimensions");
  // scale modes (build_huffman.cu:325-366)
  const int64_t scale_numel = in->scale_numel;
  const bool scale_scalar = scale_numel == 1;
  const bool scale_per_elem = scale_numel == numel;
  bool scale_per_row = false, scale_block2d = false;
  int64_t n_rows = -1, n_cols = -1, sb0 = -1, sb1 = -1, nb0 = -1, nb1 = -1;
  if (!scale_scalar && !scale_per_elem && in->ndim == 2) {
    n_rows = in->dims[0];
    n_cols = in->dims[1];
    scale_per_row = scale_numel == n_rows;
    if (!scale_per_row && in->scale_ndim == 2) {
      nb0 = in->scale_dims[0];
      nb1 = in->scale_dims[1];
      if (nb0 > 0 && nb1 > 0 && n_rows % nb0 == 0 && n_cols % nb1 == 0) {
        sb0 = n_rows / nb0;
        sb1 = n_cols / nb1;
        if (sb0 > 0 && sb1 > 0) scale_block2d = true;
      }
    }
  }
  if (!scale_scalar && !scale_per_elem && !scale_per_row && !scale_block2d)
    return fail(MPS_ERR_INVALID_ARGUMENT,
                "unsupported scales shape: use scalar, per-row (n,), per-element (numel), or 2D block-wise "
                "[n/bs0,m/bs1]");
  // The reference builds the tables before it checks the bucket layout; the
  // checks below raise the same errors without the wasted work.
  if (in->ndim != 2) return fail(MPS_ERR_INVALID_ARGUMENT, "bucket packing requires bf16_params to be 2D [n,m]");
  const int64_t n = in->dims[0], m = in->dims[1];
  if (n <= 0 || m <= 0) return fail(MPS_ERR_INVALID_ARGUMENT, "bf16_params shape must be non-empty");
  if (!scale_block2d && !(scale_scalar || (!scale_per_elem && scale_per_row)))
    return fail(MPS_ERR_INVALID_ARGUMENT,
                "bucket packing requires scales to be scalar, per-row (n,), or 2D block-wise");
  if (numel != n * m) return fail(MPS_ERR_INVALID_ARGUMENT, "bf16_params and fp8_params must have same numel");
  if (numel >= (int64_t)1 << 32) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor too large for the GPU builder");
  EncodeSpec sp{in->bf16, in->fp8, in->scales, n, m, scale_numel, scale_scalar, scale_per_row, scale_block2d,
                nb0, nb1, sb0, sb1, L, kth, 0, kFmtFp8};
  return encode_impl(sp, s, out);
}


int mps_awq_encode(const mps_awq_encode_in *in, void *stream, mps_fp8_sidecar **out) {
  last_error().clear();
  if (!in || !out) return fail(MPS_ERR_INVALID_ARGUMENT, "inputs must be defined");
  *out = nullptr;
  // checks of build_huffman.cu:1097-1153 (by scale) and :1605-1650, in order
  const int64_t L = in->max_len, kth = in->threads_per_block, n = in->n, m = in->m;
  if (L <= 0 || L > 15) return fail(MPS_ERR_INVALID_ARGUMENT, "max_len must be in (0,15]");
  if (kth <= 0 || kth > 1024) return fail(MPS_ERR_INVALID_ARGUMENT, "threads_per_block must be in [1,1024]");
  if (in->by_scale && in->group_cap <= 0) return fail(MPS_ERR_INVALID_ARGUMENT, "group_cap must be > 0");
  if (n <= 0 || m <= 0) return fail(MPS_ERR_INVALID_ARGUMENT, "bf16_params shape must be non-empty");
  if (in->scale_ndim < 0 || in->scale_ndim > 2) return fail(MPS_ERR_INVALID_ARGUMENT,
      "unsupported scales_u16 shape: use scalar, per-row (n,), or 2D block-wise [n/bs0,m/bs1]");
  const int64_t scale_numel = in->scale_numel;
  const bool scalar = scale_numel == 1;
  const bool per_row = !scalar && in->scale_ndim == 1 && scale_numel == n;
  bool block2d = false;
  int64_t nb0 = -1, nb1 = -1, sb0 = -1, sb1 = -1;
  if (!scalar && !per_row && in->scale_ndim == 2) {
    nb0 = in->scale_dims[0];
    nb1 = in->scale_dims[1];
    if (nb0 > 0 && nb1 > 0 && n % nb0 == 0 && m % nb1 == 0) {
      sb0 = n / nb0;
      sb1 = m / nb1;
      block2d = sb0 > 0 && sb1 > 0;
    }
  }
  if (!scalar && !per_row && !block2d)
    return fail(MPS_ERR_INVALID_ARGUMENT,
                "unsupported scales_u16 shape: use scalar, per-row (n,), or 2D block-wise [n/bs0,m/bs1]");
  if (n * m >= (int64_t)1 << 32) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor too large for the GPU builder");
  if (in->by_scale && n * (block2d ? nb1 : 1) >= (int64_t)1 << 31)
    return fail(MPS_ERR_INVALID_ARGUMENT, "too many quantisation groups for the GPU builder");
  EncodeSpec sp{in->bf16, in->int4, in->scales, n, m, scale_numel, scalar, per_row, block2d, nb0, nb1, sb0, sb1,
                L, kth, in->group_cap, in->by_scale ? kFmtAwqByScale : kFmtAwqBucket};
  return encode_impl(sp, reinterpret_cast<hipStream_t>(stream), out);
}

int mps_fp8_sidecar_sizes(const mps_fp8_sidecar *sc, int64_t *sizes17) {
  if (!sc || !sizes17) return fail(MPS_ERR_INVALID_ARGUMENT, "NULL argument");
  std::memcpy(sizes17, sc->sizes, sizeof(sc->sizes));
  return MPS_OK;
}

int mps_fp8_sidecar_stats(const mps_fp8_sidecar *sc, int64_t *stats4) {
  if (!sc || !stats4) return fail(MPS_ERR_INVALID_ARGUMENT, "NULL argument");
  std::memcpy(stats4, sc->stats, sizeof(sc->stats));
  return MPS_OK;
}

int mps_fp8_sidecar_copy(const mps_fp8_sidecar *sc, void *const *dst17, void *stream) {
  last_error().clear();
  if (!sc || !dst17) return fail(MPS_ERR_INVALID_ARGUMENT, "NULL argument");
  const void *src[17] = {sc->decode_syms.p, sc->decode_lens.p, sc->table_scale.p, sc->table_fp8.p,
                         sc->bucket_scale.p, sc->bucket_row_offsets.p, sc->row_indices.p, sc->bucket_table.p,
                         sc->bucket_col_start.p, sc->bucket_col_len.p, sc->bucket_thread_startbit.p,
                         sc->bucket_bit_base.p, sc->bitstream.p, sc->shape_nmk.p, sc->bucket_U.p,
                         sc->bucket_unique_gid.p, sc->bucket_fp8_uidx.p};
  const int esize[17] = {2, 1, 2, 2, 2, 4, 4, 4, 4, 4, 4, 8, 8, 8, 4, 4, 2};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int i = 0; i < 17; ++i) {
    const size_t bytes = (size_t)sc->sizes[i] * esize[i];
    if (bytes == 0) continue;
    if (!dst17[i]) return fail(MPS_ERR_INVALID_ARGUMENT, "NULL destination %d", i);
    MPS_HIP_CHECK(hipMemcpyAsync(dst17[i], src[i], bytes, hipMemcpyDefault, s));
  }
  MPS_HIP_CHECK(hipStreamSynchronize(s));
  return MPS_OK;
}

int mps_fp8_sidecar_free(mps_fp8_sidecar *sc) {
  delete sc;
  return MPS_OK;
}

}  // extern "C"
