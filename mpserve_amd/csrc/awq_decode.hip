// AWQ int4 + Huffman-sidecar -> BF16 decode for MI355X (gfx950).
//
// Format (reference kernel/build_huffman.cu:1075-1580 and :1583-2126): bucket b
// owns a list of rows (row layout: row_indices[row_offsets[b] ..] x columns
// [col_start, col_start + col_len)) or of quantisation groups (by-scale
// layout: group g = row group_rows[g], columns [group_col_start[g],
// + group_size)). Its elements, flattened row (group) major, are dealt
// round-robin to k_eff = min(k, total) lanes; lane t codes e = t, t+k_eff, ...
// as one MSB-first substream from bit bucket_bit_base[b] + startbit[b][t].
// A code is looked up with the next 11 bits in the table of
// (bucket scale, int4 value); a length nibble of 15 marks ESC: the code is
// 11 bits and 16 raw BF16 bits follow (decode_huffman.cu:454-460). A table id
// of -1 decodes as ESC too, as the reference kernel does.
//
// Mapping to CDNA4: one workgroup of 1024 work-items per bucket, one lane per
// work-item. The bucket's 16 tables are expanded once into LDS as 32-bit
// entries {sym:16 | nibble:4} indexed (qv << 11) | peek (128 KiB), and the
// bucket's row (group) start offsets are staged next to them (32 KiB), so an
// element costs one ds_read_b32 for its code and one for its row offset. The
// table fill issues all of a work-item's global loads before its first LDS
// store (one memory round trip per bucket). The bit supply is a 64-bit
// MSB-aligned buffer topped up to >= 32 bits after every element from a
// register queue of 8 32-bit chunks; an aligned quad of 4 chunks (more than a
// block of kDepth = 8 codes can take without ESC) and the block's int4 bytes
// are loaded one block ahead, one 16-byte request per quad. ESC payloads can drain the queue, which then reads a
// chunk straight from memory. A tensor with fewer buckets than CUs runs two
// 512-work-item workgroups per bucket, each with its own copy of the tables.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <new>
#include <type_traits>
#include <utility>
#include <vector>

#include "mps_common.h"

namespace mps {
namespace {

constexpr int kAwqL = 11;
constexpr int kAwqTable = 1 << kAwqL;     // 2048 entries per code table
constexpr int kAwqPacked = kAwqTable / 2; // 1024 bytes of packed 4-bit lengths
constexpr int kAwqBlock = 1024;           // work-items per bucket workgroup (>= k)
constexpr int kLutEntries = 16 * kAwqTable;
constexpr int kRowSlots = 8192;           // row (group) start offsets staged in LDS
constexpr uint32_t kBadBase = 0xFFFFFFFFu;
// Elements per block, and the chunk queue: a block of kDepth codes without
// ESC takes at most 3 32-bit chunks from the queue; a quad of kStage chunks is
// staged (loaded) one block ahead, and the queue holds kQueue.
#ifndef MPS_AWQ_DEPTH
#define MPS_AWQ_DEPTH 8
#endif
constexpr int kDepth = MPS_AWQ_DEPTH;
constexpr int kStage = 4;   // chunks staged a block: one 16-byte aligned quad
constexpr int kQueue = 8;
static_assert((kDepth * kAwqL + 31) / 32 <= kQueue - kStage, "a block's codes must fit the queue after an append");

// A global-address-space atomic, not a generic one: an outstanding generic
// (flat) access makes the compiler turn every later memory wait into a full one.
__device__ __forceinline__ void flag(uint32_t *status, unsigned int f) {
  __hip_atomic_fetch_or((__attribute__((address_space(1))) uint32_t *)(status), f, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
}
// A load through a global pointer, for the same reason.
template <typename V>
__device__ __forceinline__ V gload(const V *p) {
  return *(const __attribute__((address_space(1))) V *)(p);
}

// Stream chunk c (32 bits, stream order) of u64 words stored little-endian:
// word w's first 32 stream bits are u32 2w+1. Past the end the last chunk is
// re-read: a well-formed lane never consumes those bits, and an 11-bit peek
// that runs past its last code selects an entry whose low bits do not matter.
__device__ __forceinline__ uint32_t chunk_at(const uint32_t *__restrict__ bs32, uint64_t nchunks, uint64_t c) {
  const uint64_t cc = c < nchunks ? c : nchunks - 1;
  return bs32[cc ^ 1u];
}

__device__ uint32_t g_awq_zero_chunks[2];

// Element offset (row * m + column start) of row (group) rr of the bucket;
// kStaged: every row of the bucket is staged in LDS.
template <bool kStaged>
__device__ __forceinline__ uint32_t row_base(const mps_awq_tensor &T, const uint32_t *__restrict__ s_base,
                                             int32_t ra, int32_t rr, int32_t c0, int32_t cl) {
  if (kStaged || rr < kRowSlots) return s_base[rr];
  const int64_t row = T.row_indices[ra + rr];
  const int64_t col = T.group_col_start ? (int64_t)T.group_col_start[ra + rr] : (int64_t)c0;
  if (row < 0 || row >= T.n || col < 0 || col + cl > T.m) return kBadBase;
  return (uint32_t)(row * T.m + col);
}

// One lane's substream (the element walk, the bit supply and the stores).
template <bool kStaged>
__device__ __forceinline__ void awq_lane(const mps_awq_tensor &T, const uint32_t *__restrict__ lut,
                                         const uint32_t *__restrict__ s_base, int64_t b, int32_t ra, int32_t c0,
                                         int32_t cl, int64_t total, int32_t k, int32_t k_eff, int lane,
                                         uint32_t *status) {
  const uint32_t *__restrict__ sb = T.bucket_thread_startbit + b * ((int64_t)k + 1);
  const uint64_t pos0 = (uint64_t)T.bucket_bit_base[b] + sb[lane];
  const uint64_t pos_end = (uint64_t)T.bucket_bit_base[b] + sb[lane + 1];
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_awq_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;

  // Initial fill: buffer from chunks cb, cb+1; queue = the next kQueue chunks.
  const uint64_t cb = pos0 >> 5;
  const int skip = (int)(pos0 & 31u);
  uint64_t buf = (((uint64_t)chunk_at(bs32, nchunks, cb) << 32) | chunk_at(bs32, nchunks, cb + 1)) << skip;
  int cnt = 64 - skip;
  // The queue starts with the chunks up to the next multiple of 4, so that
  // every later stage is one aligned quad.
  uint32_t qq[kQueue];
#pragma unroll
  for (int j = 0; j < kQueue; ++j) qq[j] = j < 3 ? chunk_at(bs32, nchunks, cb + 2 + j) : 0u;
  int qn = (int)((4u - ((cb + 2) & 3u)) & 3u);
  uint64_t tail = cb + 2 + qn;  // index of the first chunk not yet in buf/queue

  // Element walk e = tid + i*k_eff -> (rr, cc) = (e / cl, e % cl), incrementally.
  int32_t rr = lane / cl;
  int32_t cc = lane - rr * cl;
  const int32_t dr = k_eff / cl, dc = k_eff - dr * cl;
  const int32_t count = (int32_t)((total - lane + k_eff - 1) / k_eff);
  const uint8_t *__restrict__ qv = T.int4;
  char *__restrict__ outb = reinterpret_cast<char *>(T.out);
  const uint32_t first = row_base<kStaged>(T, s_base, ra, rr, c0, cl);
  const uint32_t safe = first == kBadBase ? 0u : first + (uint32_t)cc;  // an address every lane may read
  int32_t walked = 0;
  auto next_block = [&](uint32_t (&idx)[kDepth]) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      uint32_t v = kBadBase;
      if (walked + j < count) {
        const uint32_t base = row_base<kStaged>(T, s_base, ra, rr, c0, cl);
        if (base != kBadBase) v = base + (uint32_t)cc;
      }
      idx[j] = v;
      cc += dc;
      rr += dr;
      if (cc >= cl) {
        cc -= cl;
        rr += 1;
      }
    }
    walked += kDepth;
  };
  uint32_t ia[kDepth], ib[kDepth], qa[kDepth], qb[kDepth];
  next_block(ia);
#pragma unroll
  for (int j = 0; j < kDepth; ++j) qa[j] = qv[ia[j] == kBadBase ? safe : ia[j]];
  // Chunks tail .. tail+3: one 16-byte load when the quad is aligned and whole
  // (u32 words 4j .. 4j+3 hold chunks 4j+1, 4j, 4j+3, 4j+2), else four loads.
  const bool aligned16 = (reinterpret_cast<uintptr_t>(bs32) & 15u) == 0;
  auto stage = [&](uint32_t (&st)[kStage]) {
    if (aligned16 && (tail & 3u) == 0 && tail + 4 <= nchunks) {
      const uint4 v = *reinterpret_cast<const uint4 *>(bs32 + tail);
      st[0] = v.y;
      st[1] = v.x;
      st[2] = v.w;
      st[3] = v.z;
    } else {
#pragma unroll
      for (int j = 0; j < kStage; ++j) st[j] = chunk_at(bs32, nchunks, tail + j);
    }
  };
  uint32_t st[kStage];
  stage(st);
  bool stale = false;

  auto refill = [&]() {
    if (cnt < 32) {
      if (qn > 0) {
        buf |= (uint64_t)qq[0] << (32 - cnt);
#pragma unroll
        for (int j = 0; j + 1 < kQueue; ++j) qq[j] = qq[j + 1];
        --qn;
      } else {
        // Queue drained by ESC payloads: read the chunk straight from memory.
        const uint32_t ch = chunk_at(bs32, nchunks, tail);
        buf |= (uint64_t)ch << (32 - cnt);
        ++tail;
        stale = true;
      }
      cnt += 32;
    }
  };
  auto decode_one = [&](uint32_t q, uint32_t idx) {
    const uint32_t peek = (uint32_t)(buf >> (64 - kAwqL));
    const uint32_t ent = lut[((q & 15u) << kAwqL) | peek];
    const uint32_t nib = ent & 15u;
    uint32_t sym = ent >> 16;
    if (nib == 15u) {
      // ESC: the code is L bits, then 16 raw bits (decode_huffman.cu:454-460)
      buf <<= kAwqL;
      sym = (uint32_t)(buf >> 48);
      buf <<= 16;
      cnt -= kAwqL + 16;
    } else {
      buf <<= nib;
      cnt -= (int)nib;
    }
    // saddr store: the byte offset fits 32 bits (n*m < 2^31)
    if (idx != kBadBase) *reinterpret_cast<uint16_t *>(outb + (idx << 1)) = (uint16_t)sym;
    refill();
  };
  auto block = [&](int32_t i0, uint32_t (&qc)[kDepth], uint32_t (&ic)[kDepth], uint32_t (&qnx)[kDepth],
                   uint32_t (&inx)[kDepth]) {
    // Append the chunks staged one block ago if they are current and fit.
    if (!stale && qn <= kQueue - kStage) {
#pragma unroll
      for (int j = 0; j < kQueue; ++j)
#pragma unroll
        for (int t = 0; t < kStage; ++t)
          if (j == qn + t) qq[j] = st[t];
      qn += kStage;
      tail += kStage;
    }
    stale = false;
    next_block(inx);
#pragma unroll
    for (int j = 0; j < kDepth; ++j) qnx[j] = qv[inx[j] == kBadBase ? safe : inx[j]];
    stage(st);
    if (i0 + kDepth <= count) {
#pragma unroll
      for (int j = 0; j < kDepth; ++j) decode_one(qc[j], ic[j]);
    } else {
#pragma unroll
      for (int j = 0; j < kDepth; ++j)
        if (i0 + j < count) decode_one(qc[j], ic[j]);
    }
  };
  for (int32_t i0 = 0; i0 < count; i0 += 2 * kDepth) {
    block(i0, qa, ia, qb, ib);
    if (i0 + kDepth >= count) break;
    block(i0 + kDepth, qb, ib, qa, ia);
  }
  // The next unread bit must be where the next lane's substream begins.
  if (tail * 32u - (uint64_t)(cnt + 32 * qn) != pos_end) flag(status, MPS_STATUS_DESYNC);
}

// kSplit workgroups of kAwqBlock / kSplit work-items share a bucket: each
// stages the bucket's tables and decodes its slice of the lanes (launches with
// fewer buckets than CUs use several CUs per bucket).
template <int kSplit>
__device__ __forceinline__ void awq_bucket(const mps_awq_tensor &T, int64_t b, int part, uint32_t *__restrict__ lut,
                                           uint32_t *__restrict__ s_base, uint32_t *status) {
  constexpr int kThreads = kAwqBlock / kSplit;
  const int tid = threadIdx.x;
  const int lane = part * kThreads + tid;
  // Bucket geometry (decode_huffman.cu:417-444, :528-545).
  const int32_t ra = T.bucket_row_offsets[b], rb = T.bucket_row_offsets[b + 1];
  const int32_t rows = rb - ra;
  if (rows <= 0) return;
  const bool by_scale = T.group_col_start != nullptr;
  const int32_t c0 = by_scale ? 0 : T.bucket_col_start[b];
  const int32_t cl = by_scale ? (int32_t)T.group_size : T.bucket_col_len[b];
  if (cl <= 0 || ra < 0 || (int64_t)rb > T.num_row_indices ||
      (!by_scale && (c0 < 0 || (int64_t)c0 + cl > T.m))) {
    if (tid == 0) flag(status, MPS_STATUS_BAD_BUCKET);
    return;
  }
  const int64_t total = (int64_t)rows * cl;
  const int32_t k = (int32_t)T.k;
  const int32_t k_eff = total < k ? (int32_t)total : k;

  // Tables: entry (q << 11) | p = sym << 16 | nibble; a missing table (id -1)
  // is all ESC entries, as the reference decodes it. The 16 table ids are
  // bucket-uniform (scalar loads); every work-item then fills 32 entries, two
  // per table, with all 64 global loads issued before the first LDS store
  // (addresses of missing tables are clamped to table 0 and the entry selected
  // afterwards), so the fill costs one memory round trip, not 32.
  int32_t gid[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) gid[q] = T.bucket_table[b * 16 + q];
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if (gid[q] < -1 || gid[q] >= T.num_tables) flag(status, MPS_STATUS_BAD_TABLE);
  }
  const int64_t G = T.num_tables;
  if (G <= 0) {
    for (int i = tid; i < kLutEntries; i += kThreads) lut[i] = 15u;
  } else for (int part = 0; part < kSplit; ++part) {  // kSplit rounds of 32 entries a work-item
    uint32_t sy[32], ln[32];
#pragma unroll
    for (int it = 0; it < 32; ++it) {
      const int i = (part * 32 + it) * kThreads + tid;
      const int q = i >> kAwqL, p = i & (kAwqTable - 1);
      const uint32_t g = (gid[q] >= 0 && gid[q] < G) ? (uint32_t)gid[q] : 0u;  // table 0 exists: G > 0
      sy[it] = T.decode_syms[(size_t)g * kAwqTable + p];
      ln[it] = T.decode_lens[(size_t)g * kAwqPacked + (p >> 1)];
    }
#pragma unroll
    for (int it = 0; it < 32; ++it) {
      const int i = (part * 32 + it) * kThreads + tid;
      const int q = i >> kAwqL, p = i & (kAwqTable - 1);
      const bool ok = gid[q] >= 0 && gid[q] < G;
      lut[i] = ok ? (sy[it] << 16) | ((p & 1) ? (ln[it] >> 4) : (ln[it] & 15u)) : 15u;
    }
  }
  const int32_t staged = rows < kRowSlots ? rows : kRowSlots;
  for (int r = tid; r < staged; r += kThreads) {
    const int64_t row = T.row_indices[ra + r];
    const int64_t col = by_scale ? (int64_t)T.group_col_start[ra + r] : (int64_t)c0;
    uint32_t base = kBadBase;
    if (row >= 0 && row < T.n && col >= 0 && col + cl <= T.m) base = (uint32_t)(row * T.m + col);
    else flag(status, MPS_STATUS_BAD_ROW);
    s_base[r] = base;
  }
  __syncthreads();
  if (lane >= k_eff) return;

  if (rows <= kRowSlots) awq_lane<true>(T, lut, s_base, b, ra, c0, cl, total, k, k_eff, lane, status);
  else awq_lane<false>(T, lut, s_base, b, ra, c0, cl, total, k, k_eff, lane, status);
}

template <int kSplit>
__global__ __launch_bounds__(kAwqBlock) void awq_decode_kernel(mps_awq_tensor T, uint32_t *status) {
  // Row offsets (the slab path's queue) first: the tables' base then rides in
  // the LDS instructions' offset field, and the queue's address needs no add.
  __shared__ __attribute__((aligned(16))) uint32_t lds[kRowSlots + kLutEntries];
  uint32_t *s_base = lds, *lut = lds + kRowSlots;
  awq_bucket<kSplit>(T, blockIdx.x / kSplit, (int)(blockIdx.x % kSplit), lut, s_base, status);
}

// ---------------------------------------------------------------------------
// Slab path: by-scale buckets with k = 1024 substreams and groups of 128
// columns (8 to 1024 groups). Element e of such a bucket is column e % 128 of
// its group e / 128, and substream t codes e = t, t + 1024, ...: the i-th
// element of every substream lies in *slab* i, the bucket's groups 8i .. 8i+7.
// Lane l = 16R + v of wave w decodes substream t = 64w + 4v + R, four elements
// (slabs 4g .. 4g+3) per step, in the register layout of the FP8 slab decode:
//  - lane (R, v) loads one dword of int4 bytes, columns 64(w & 1) + 4v .. +3 of
//    slab 4g+R's group 8(4g+R) + w/2, so each 16-lane row reads 64 contiguous
//    bytes; a 4x4 byte transpose across lanes (0,v) .. (3,v) gives every lane
//    its own four bytes;
//  - the inverse transpose of the BF16 symbols gives lane (R, v) those columns'
//    values for one 8-byte store (a 128-byte segment per 16-lane row);
//  - the wave's group bases (row * m + column start + 64(w & 1)) for slabs
//    l and l + 64 sit in lane l of two VGPRs and are fetched with ds_bpermute;
//  - the bit supply is the FP8 slab path's: an 8-chunk LDS queue per lane fed
//    from a register reserve that requests aligned 64-byte blocks.
// Codes are up to 11 bits, so a step cuts two 32-bit windows, two codes each.
// An ESC entry's low bits are 27 (its 11-bit code and the 16 raw bits), so bit
// 4 flags it and the running shift steps over the raw bits; a step holding an
// ESC code is decoded again code by code, reading the raw symbol.
// ---------------------------------------------------------------------------
// A plan's work record (a workgroup decodes one at a time, taking them from
// the plan's queue: awq_decode_plan).
//  kind 0: buckets bucket .. bucket + nsub - 1 on the per-lane path (one scale, shared tables;
//          with `tiny`, buckets of one code a lane that look their codes up in the global tables);
//  kind 1: slab-path buckets bucket .. bucket + nsub - 1 with identical table ids (a by-scale run);
//  kind 2: rows [range * range_rows, +range_rows) of a slab-path row bucket split into
//          `ranges` ranges, starting from the lane checkpoints at ckpt + (range - 1) * 1024
//          and ending at ckpt + range * 1024 (the bucket's own start and end bits at its ends);
//  kind 3: ranges range .. range + 1024 / k - 1 of a row bucket with k 256 or 512 split into
//          `ranges` ranges, side by side on the slab path: range r starts at checkpoint row
//          r and ends at row r + 1 of ckpt ([ranges + 1][k]).
struct AwqWork {
  int32_t tensor, bucket, nsub, kind;
  int32_t range, range_rows, ranges;
  int32_t tiny;  // kind 0: 1 when every bucket codes at most one element a lane (awq_tiny_lane)
  int64_t ckpt;
  int64_t elems;  // (the plan's ordering key)
};
static_assert(sizeof(AwqWork) == 48, "work record layout");

constexpr uint32_t kAwqEscBit = 1u << 4;
constexpr uint32_t kAwqEscLow = 27u;          // 11 + 16: an ESC entry's low bits
constexpr int kSlabQSlots = 8;                // LDS queue chunks per lane
constexpr uint32_t kSlabBsPast = 0x80000000u; // bitstream offset beyond every bucket's range
constexpr uint32_t kSlabOutPast = 0xFFFFFFF0u;  // BF16 byte offset beyond every output (2*n*m < 2^32)
constexpr uint32_t kSlabInPast = 0x80000000u;   // int4 byte offset beyond every input (n*m < 2^31)
constexpr int kSlabCacheNT = 2;               // buffer cache-policy bits: non-temporal
constexpr int kSlabMinGroups = 8, kSlabMaxGroups = 1024;
constexpr uint32_t kRunTables = 1u << 8;        // run_flags: a run's tables are in the LDS
static_assert(kSlabQSlots * kAwqBlock <= kRowSlots, "the slab queue lives in the row-offset region");

// Buffer resource over [base, base + bytes): raw buffer loads past the end
// return 0 and stores past the end are dropped (gfx9 V# with stride 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t awq_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t awq_uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// Slab layouts: by-scale groups, or row buckets whose column range is P blocks
// of 1024 (P >= 4) with P % 4 == 0 (a step's four slabs in one row) or not (a
// step can straddle two rows; each lane picks its row's offset).
enum : int { kLayGroups = 0, kLayRows = 1, kLayRowsWrap = 2 };

// base_lo / base_hi: lane l holds slab l's and l + 64's base (groups), or row
// l's and l + 64's offset (rows, column start included); rows and P describe a
// row bucket (rows x P elements per lane).
// kShift: log2 of the substream count k (the row layouts' block stride), 10,
// or 0 for the run-time `kshift` (kLayRows with k 256 or 512, several row
// ranges side by side: `lane` is the work-item's substream within its range's
// group of k, `qlane` the work-item, whose LDS queue column it owns).
template <bool kEsc, int kLay, int kShift = 10>
__device__ __forceinline__ void awq_slab_decode(const mps_awq_tensor &T, const uint32_t *__restrict__ lut,
                                                uint32_t *__restrict__ queue, uint32_t qlane, uint32_t lane,
                                                uint32_t kshift, uint32_t count,
                                                uint32_t base_lo, uint32_t base_hi, uint32_t rows, uint32_t P,
                                                uint64_t bucket_bit, const uint2 (&first)[4], uint32_t pos,
                                                uint32_t pos_end, uint32_t *status) {
#ifndef MPS_AWQ_SLAB_PREFETCH
#define MPS_AWQ_SLAB_PREFETCH 8
#endif
#ifndef MPS_AWQ_FEED_EVERY
#define MPS_AWQ_FEED_EVERY 2
#endif
  constexpr int DF = MPS_AWQ_SLAB_PREFETCH;  // int4 prefetch distance (steps)
  constexpr int FE = MPS_AWQ_FEED_EVERY;     // steps per bitstream feed (16 bytes: 2 x 44 bits fit)
  static_assert(DF % FE == 0 && (FE == 1 || FE == 2), "a feed every one or two steps");
#ifndef MPS_AWQ_RB
#define MPS_AWQ_RB 4
#endif
  constexpr int RB = MPS_AWQ_RB;  // 16-byte blocks per bitstream request
  static_assert(kShift == 10 || (kShift == 0 && kLay != kLayRowsWrap), "k < 1024: no steps across rows");
  count = awq_uni(count);
  kshift = kShift ? (uint32_t)kShift : awq_uni(kshift);
  bucket_bit = ((uint64_t)awq_uni((uint32_t)(bucket_bit >> 32)) << 32) | awq_uni((uint32_t)bucket_bit);
  const uint32_t nfull = count >> 2;
  const uint32_t tail = count & 3u;  // elements of the last, partial step
  const uint32_t gall = nfull + (tail ? 1u : 0u);
  const uint32_t nm = (uint32_t)(T.n * T.m);
  const __amdgpu_buffer_rsrc_t r_q = awq_rsrc(T.int4, nm);
  const __amdgpu_buffer_rsrc_t r_out = awq_rsrc(T.out, 2u * nm);
  const uint64_t bs_bytes = T.bitstream_words > 0 ? (uint64_t)T.bitstream_words * 8u : 0u;
  const uint64_t base_byte = bucket_bit >> 3;
  const uint32_t win_bytes = base_byte < bs_bytes ? (uint32_t)(bs_bytes - base_byte) : 0u;
  const __amdgpu_buffer_rsrc_t r_bs =
      awq_rsrc(reinterpret_cast<const uint8_t *>(T.bitstream) + (base_byte < bs_bytes ? base_byte : 0), win_bytes);

  const uint32_t lane4 = qlane << 2;
  const uint32_t R = (lane >> 4) & 3u;
  const uint32_t R4 = R << 2;
  const uint32_t v4 = (lane & 15u) << 2;
  const char *qbytes = reinterpret_cast<const char *>(queue);
  const char *lbytes = reinterpret_cast<const char *>(lut);
  // byte selectors of the int4-byte transpose (v_perm: 0-3 pick the second operand's bytes, 4-7 the first's)
  const uint32_t selA = (R & 2u) ? 0x07060302u : 0x05040100u;
  const uint32_t selB = (R & 1u) ? 0x07030501u : 0x06020400u;

  // --- bitstream queue: chunk h (32 stream bits) of this lane in slot (~h) & 7 ---
  auto chunk_mem = [&](uint32_t h) -> uint32_t {  // biased chunk h from memory (h < 2: zeros)
    return __builtin_amdgcn_raw_buffer_load_b32(r_bs, ((h - 2u) ^ 1u) << 2, 0, 0);
  };
  auto put_pair = [&](uint32_t h, uint32_t hi, uint32_t lo) {  // chunks h (even) and h + 1
    uint32_t *slot = queue + (((~h << 10) & 0x1800u) | qlane);
    slot[0] = lo;
    slot[1024] = hi;
  };
  const uint32_t phase =
      ((uint32_t)reinterpret_cast<uintptr_t>(T.bitstream) + (uint32_t)(bucket_bit >> 3)) & (16u * RB - 1u);
  const uint32_t rq0 = ((pos >> 5) & ~1u) + 2u;
  const uint32_t nfirst = ((phase + 4u * (rq0 - 2u)) & 15u) ? 6u : 8u;
#pragma unroll
  for (int i = 0; i < 3; ++i) put_pair(rq0 + 2 * i, first[i].y, first[i].x);
  if (nfirst == 8u) put_pair(rq0 + 6u, first[3].y, first[3].x);
  uint32_t wqb = (rq0 + nfirst) << 5;  // 32 x (first chunk not yet written)
  uint32_t rqb = wqb;                  // 32 x (first chunk not yet requested)
  uint32_t np = 0u - (pos + 64u);      // negated biased position

  auto window = [&](uint32_t npv) -> uint32_t {  // 32 stream bits at -npv
    const uint32_t t7 = npv << 7;
    const uint32_t c0 = *reinterpret_cast<const uint32_t *>(qbytes + ((t7 & 0x7000u) | lane4));
    const uint32_t c1 = *reinterpret_cast<const uint32_t *>(qbytes + (((t7 - 4096u) & 0x7000u) | lane4));
    uint32_t w = __builtin_amdgcn_alignbit(c0, c1, npv);
    const bool dry = (int32_t)(wqb + npv) <= 31;
    if (__builtin_amdgcn_ballot_w64(dry)) {
      if (dry) {
        const uint32_t h = (~npv) >> 5;
        w = __builtin_amdgcn_alignbit(chunk_mem(h), chunk_mem(h + 1u), npv);
        __asm__ volatile("" ::"v"(w));  // wait for the loads here, not at a later join
      }
    }
    return w;
  };
#ifndef MPS_AWQ_WIN64
#define MPS_AWQ_WIN64 1
#endif
  // 64 stream bits at -npv as {hi, lo}: three queue chunks, or memory for
  // lanes whose queue lacks the third.
  auto window64 = [&](uint32_t npv, uint32_t &hi, uint32_t &lo) {
    const uint32_t t7 = npv << 7;
    uint32_t c0 = *reinterpret_cast<const uint32_t *>(qbytes + ((t7 & 0x7000u) | lane4));
    uint32_t c1 = *reinterpret_cast<const uint32_t *>(qbytes + (((t7 - 4096u) & 0x7000u) | lane4));
    uint32_t c2 = *reinterpret_cast<const uint32_t *>(qbytes + (((t7 - 8192u) & 0x7000u) | lane4));
    const bool dry = (int32_t)(wqb + npv) <= 63;
    if (__builtin_amdgcn_ballot_w64(dry)) {
      if (dry) {
        const uint32_t h = (~npv) >> 5;
        c0 = chunk_mem(h);
        c1 = chunk_mem(h + 1u);
        c2 = chunk_mem(h + 2u);
        __asm__ volatile("" ::"v"(c0), "v"(c1), "v"(c2));  // wait for the loads here, not at a later join
      }
    }
    hi = __builtin_amdgcn_alignbit(c0, c1, npv);
    lo = __builtin_amdgcn_alignbit(c1, c2, npv);
  };
  // Register reserve of up to RB 16-byte blocks after the queue's last chunk,
  // refilled by aligned 64-byte requests that land in inb.
  uint4 rv[RB], inb[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) rv[i] = inb[i] = make_uint4(0u, 0u, 0u, 0u);
  uint32_t rcnt = 0, ninb = 0;
  bool ifl = false;
  // A feed writes chunks h .. h + 3 (h = wqb / 32, even) as two slot pairs,
  // ((~h) >> 1) & 3 and the one below; the next feed's h is 4 more, so both
  // pair indices flip bit 1: their byte addresses are kept and XORed with 0x4000.
  char *const qw = reinterpret_cast<char *>(queue);
  uint32_t fa = ((((~(wqb >> 5)) << 10) & 0x1800u) | qlane) << 2;
  uint32_t fb = ((((~((wqb >> 5) + 2u)) << 10) & 0x1800u) | qlane) << 2;
  auto feed = [&]() {
    const bool f = rcnt != 0u && (int32_t)(wqb + np) < 128;
    if (f) {
      *reinterpret_cast<uint32_t *>(qw + fa) = rv[0].x;          // chunk h + 1
      *reinterpret_cast<uint32_t *>(qw + fa + 4096u) = rv[0].y;  // chunk h
      *reinterpret_cast<uint32_t *>(qw + fb) = rv[0].z;          // chunk h + 3
      *reinterpret_cast<uint32_t *>(qw + fb + 4096u) = rv[0].w;  // chunk h + 2
#pragma unroll
      for (int i = 0; i + 1 < RB; ++i) rv[i] = rv[i + 1];
    }
    const uint32_t flip = f ? 0x4000u : 0u;
    fa ^= flip;
    fb ^= flip;
    wqb += f ? 128u : 0u;
    rcnt -= f ? 1u : 0u;
  };
  // The first request (is_first) runs up to the next 16 RB-byte boundary of the
  // bitstream; every later one is RB whole blocks from that boundary on.
  auto land = [&]() {
    const bool l = ifl && rcnt == 0u;
    if (l) {
#pragma unroll
      for (int i = 0; i < RB; ++i) rv[i] = inb[i];
    }
    rcnt = l ? ninb : rcnt;
    ifl = ifl && !l;
  };
  auto reserve = [&](auto is_first) {
    constexpr bool kFirst = decltype(is_first)::value;
    const bool req = !ifl && rcnt <= 1u && (int32_t)(rqb - (pos_end + 192u)) < 0;
    const uint32_t off = (rqb >> 3) - 8u;
    const uint32_t nreq = kFirst ? (16u * RB - ((phase + off) & (16u * RB - 1u))) >> 4 : (uint32_t)RB;
    if (req) {
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(
            r_bs, (!kFirst || (uint32_t)i < nreq) ? off + 16u * (uint32_t)i : kSlabBsPast, 0, 0);
        inb[i] = make_uint4(v[0], v[1], v[2], v[3]);
      }
      ninb = nreq;
    }
    ifl = ifl || req;
    rqb += req ? nreq << 7 : 0u;
  };
  // after every second step: a 16-byte feed covers the 2 x 44 bits two steps can take.
  // Requests are considered at every MPS_AWQ_REQ_EVERY-th of these: lanes reach
  // the request point on different steps, so a request's loads carry few
  // active lanes, and asking less often gathers more of them into each load.
#ifndef MPS_AWQ_REQ_EVERY
#define MPS_AWQ_REQ_EVERY 2
#endif
  static_assert(MPS_AWQ_REQ_EVERY >= 1 && (MPS_AWQ_REQ_EVERY & (MPS_AWQ_REQ_EVERY - 1)) == 0, "a power of two");
  uint32_t bstep = 0;  // bitstream steps taken (uniform)
  auto bitstream_step = [&]() {
    land();
    if ((bstep & (MPS_AWQ_REQ_EVERY - 1)) == 0u) reserve(std::false_type{});
    bstep = awq_uni(bstep + 1u);
    feed();
  };

  // --- walker: the int4 load of step g; returns its BF16 store byte offset
  // (kLayRows: the step's uniform element offset; the lane adds its own) ---
  rows = awq_uni(rows);
  P = awq_uni(P);
  uint32_t w_g = 0, w_row = 0, w_blk = 0;
  auto row_offset = [&](uint32_t r) -> uint32_t {
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)base_lo, (int)(r & 63u));
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)base_hi, (int)(r & 63u));
    return r < 64u ? a : b;
  };
  uint32_t w_off = 0, w_next = 0;
  if constexpr (kLay != kLayGroups) {
    w_off = row_offset(0);
    w_next = row_offset(rows > 1u ? 1u : 0u);  // offset of row w_row + 1 (kLayRowsWrap)
  }
  const uint32_t colw = (lane & ~63u) | v4;    // 64w + 4v: the lane's columns within a k-block
  const uint32_t vf_al = (R << kshift) + colw;  // ... and its block within an aligned step
  auto load_step = [&](uint32_t &F) -> uint32_t {
    uint32_t ret;
    if constexpr (kLay == kLayGroups) {
      // this lane's slab is 4 w_g + R: its base sits in lane (4 w_g + R) & 63 of
      // base_lo (slabs below 64) or base_hi (the four slabs are all below or all above)
      const bool hi = w_g >= 16u;
      const uint32_t src = hi ? base_hi : base_lo;
      const uint32_t base = (uint32_t)__builtin_amdgcn_ds_bpermute((int)(((w_g << 4) + R4) & 0xFCu), (int)src);
      const bool ok = (int32_t)R < (int32_t)awq_uni(count - 4u * w_g);
      const uint32_t off = base + v4;
      F = __builtin_amdgcn_raw_buffer_load_b32(r_q, ok ? off : kSlabInPast, 0, 0);
      ret = ok ? off << 1 : kSlabOutPast;
    } else if constexpr (kLay == kLayRows) {
      const uint32_t so = awq_uni(w_off + (w_blk << kshift));
      F = __builtin_amdgcn_raw_buffer_load_b32(r_q, vf_al, so, 0);
      ret = so;
    } else {
      const uint32_t b = w_blk + R;
      const bool wrap = b >= P;
      const bool ok = !wrap || w_row + 1u < rows;
      const uint32_t off = (wrap ? w_next : w_off) + ((wrap ? b - P : b) << kshift) + colw;
      F = __builtin_amdgcn_raw_buffer_load_b32(r_q, ok ? off : kSlabInPast, 0, 0);
      ret = ok ? off << 1 : kSlabOutPast;
    }
    const bool more = w_g + 1u < gall;
    if constexpr (kLay != kLayGroups) {
      // advance the row walk (past the last step it stays there)
      const uint32_t nb = w_blk + 4u;
      const bool wr = nb >= P;
      const uint32_t nrow = w_row + ((more && wr) ? 1u : 0u);
      const uint32_t noff = row_offset(nrow);
      const uint32_t nnext = row_offset(nrow + 1u < rows ? nrow + 1u : nrow);
      w_blk = awq_uni(more ? (wr ? nb - P : nb) : w_blk);
      w_off = awq_uni(nrow != w_row ? noff : w_off);
      w_next = awq_uni(nrow != w_row ? nnext : w_next);
      w_row = awq_uni(nrow);
    }
    w_g = awq_uni(w_g + (more ? 1u : 0u));
    return ret;
  };

  auto lookup = [&](uint32_t qb, uint32_t x) -> uint32_t {  // entry of int4 value qb at peek bits x[12:2]
    return *reinterpret_cast<const uint32_t *>(lbytes + ((qb & 15u) << 13 | (x & 0x1FFCu)));
  };
  auto step = [&](auto is_tail, uint32_t F, uint32_t so) {
    constexpr bool kTail = decltype(is_tail)::value;
    const auto p1 = __builtin_amdgcn_permlane32_swap(F, F, false, false);
    const uint32_t gq = __builtin_amdgcn_perm(p1[1], p1[0], selA);
    const auto p2 = __builtin_amdgcn_permlane16_swap(gq, gq, false, false);
    const uint32_t fq = __builtin_amdgcn_perm(p2[1], p2[0], selB);  // byte j = element j's int4 byte
    const uint32_t np0 = np;
    uint32_t e[4];
#if MPS_AWQ_WIN64
    {
      // 64 stream bits at -np: the first two codes come from the high word; the
      // second window starts where they end, cut from the same two words.
      uint32_t hi, lo;
      window64(np, hi, lo);
      uint32_t s = 19u;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (!kTail || (uint32_t)j < tail) {
          e[j] = lookup(fq >> (8 * j), __builtin_amdgcn_alignbit(hi, hi, s));
          s -= e[j];
        } else {
          e[j] = 0u;
        }
      }
      // the window 19 - s bits on: ({hi, lo} >> (32 - (19 - s)))[31:0] (the
      // shift is taken mod 32, so the entries' high bits in s do not matter)
      const uint32_t win = __builtin_amdgcn_alignbit(hi, lo, s + 13u);
      uint32_t s2 = 19u;
#pragma unroll
      for (int j = 2; j < 4; ++j) {
        if (!kTail || (uint32_t)j < tail) {
          e[j] = lookup(fq >> (8 * j), __builtin_amdgcn_alignbit(win, win, s2));
          s2 -= e[j];
        } else {
          e[j] = 0u;
        }
      }
      np += (uint32_t)((int32_t)(s << 16) >> 16) + (uint32_t)((int32_t)(s2 << 16) >> 16) - 38u;
    }
#else
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t win = window(np);
      uint32_t s = 19u;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * h + jj;
        if (!kTail || (uint32_t)j < tail) {
          e[j] = lookup(fq >> (8 * j), __builtin_amdgcn_alignbit(win, win, s));
          s -= e[j];
        } else {
          e[j] = 0u;
        }
      }
      np += (uint32_t)((int32_t)(s << 16) >> 16) - 19u;  // minus the bits consumed
    }
#endif
    if constexpr (kEsc) {
      // A wave with an ESC code in the step decodes the step again one code at
      // a time, every lane: the slow decode gives the fast one's result where
      // there is no ESC, so no lane needs to be masked off.
      if (__builtin_amdgcn_ballot_w64(((e[0] | e[1] | e[2] | e[3]) & kAwqEscBit) != 0u)) {
        uint32_t p = np0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!kTail || (uint32_t)j < tail) {
            const uint32_t w = window(p);
            uint32_t ent = lookup(fq >> (8 * j), w >> 19);
            p -= ent & 15u;
            if (ent & kAwqEscBit) {
              ent = window(p) & 0xFFFF0000u;  // the symbol: the 16 raw bits after the code
              p -= 16u;
            }
            e[j] = ent;
          }
        }
        np = p;
      }
    }
    const auto t0 = __builtin_amdgcn_permlane32_swap(e[0], e[2], false, false);
    const auto t1 = __builtin_amdgcn_permlane32_swap(e[1], e[3], false, false);
    const uint32_t a = __builtin_amdgcn_perm(t0[1], t0[0], 0x07060302u);
    const uint32_t b = __builtin_amdgcn_perm(t1[1], t1[0], 0x07060302u);
    const auto t2 = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    const v2u o = {__builtin_amdgcn_perm(t2[1], t2[0], 0x05040100u), __builtin_amdgcn_perm(t2[1], t2[0], 0x07060302u)};
    if constexpr (kLay == kLayRows) __builtin_amdgcn_raw_buffer_store_b64(o, r_out, vf_al << 1, awq_uni(so) << 1, kSlabCacheNT);
    else __builtin_amdgcn_raw_buffer_store_b64(o, r_out, so, 0, kSlabCacheNT);
  };

  uint32_t Fr[DF], SOr[DF];
#pragma unroll
  for (int u = 0; u < DF; ++u) SOr[u] = load_step(Fr[u]);
  reserve(std::true_type{});  // the first request (nothing to feed yet)
  // Wave priorities, as in the FP8 slab decode: the issue arbiter favours the
  // oldest ready wave, so a wave lowers its priority by one level per quarter
  // of its steps, counted from a head start that grows with its age.
#ifndef MPS_AWQ_PRIO
#define MPS_AWQ_PRIO 1
#endif
#ifndef MPS_AWQ_PRIO_LEAD
#define MPS_AWQ_PRIO_LEAD 16
#endif
  const uint32_t quarter = awq_uni(nfull / 4u > 0u ? nfull / 4u : 1u);
  const uint32_t lead = (3u - (awq_uni(qlane) >> 8)) * (quarter * MPS_AWQ_PRIO_LEAD / 16u);  // head start (steps)
  uint32_t prio = 3u - (lead / quarter < 3u ? lead / quarter : 3u);
  uint32_t prio_at = (lead / quarter + 1u) * quarter - lead;  // steps done when the priority next drops
  if (MPS_AWQ_PRIO) {
    if (prio == 3u) __builtin_amdgcn_s_setprio(3);
    else if (prio == 2u) __builtin_amdgcn_s_setprio(2);
    else if (prio == 1u) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
  }
  uint32_t g = 0;
  for (; g + (uint32_t)DF <= nfull; g += (uint32_t)DF) {
    if (MPS_AWQ_PRIO && g >= prio_at) {
      prio_at += quarter;
      --prio;
      if (prio == 2u) __builtin_amdgcn_s_setprio(2);
      else if (prio == 1u) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
#pragma unroll
    for (int u = 0; u < DF; ++u) {
      const uint32_t F = Fr[u], so = SOr[u];
      SOr[u] = load_step(Fr[u]);  // the step DF ahead
      step(std::false_type{}, F, so);
      if (u % FE == FE - 1) bitstream_step();
    }
  }
  if (MPS_AWQ_PRIO) __builtin_amdgcn_s_setprio(0);
  // the last (fewer than DF) full steps and the partial one; their bytes are already loaded
#pragma unroll
  for (int u = 0; u < DF; ++u) {
    if (g + (uint32_t)u < gall) {
      if (g + (uint32_t)u < nfull) step(std::false_type{}, Fr[u], SOr[u]);
      else step(std::true_type{}, Fr[u], SOr[u]);
      if (u % FE == FE - 1) bitstream_step();
    }
  }
  if (0u - np - 64u != pos_end) flag(status, MPS_STATUS_DESYNC);
}

// One slab-path bucket, checked by the plan: k = 1024 and either by-scale
// with 128-column groups and 8 .. 1024 groups, or a row bucket of 1 .. 128 rows
// whose column range is P >= 4 blocks of 1024. Set-up in two levels of loads,
// each issued in full before any result is used: (1) the table ids, the
// wave's group rows and column starts (or the bucket's rows), the lane's start
// and end bits; (2) the tables' slices and the lane's first bitstream words.
// Thread tid expands entries 32c .. 32c+31 of the table of int4 value tid / 64
// (c = tid % 64).
// kRanged: 0 a whole bucket, 1 a row range (kind 2), 2 row ranges side by side
// (kind 3: k 256 or 512, the work-items [s k, (s + 1) k) decode range
// wk.range + s, from checkpoint rows range + s and range + s + 1 of a full
// [ranges + 1][k] set); whole buckets compile without the range logic.
// A by-scale record may hold a run of buckets b with identical table ids: the
// first that gets past its checks (`tables`) loads and expands the tables and
// records in run_flags that it did (kRunTables) and whether they have an ESC
// entry (bit 1); the others reuse both.
template <int kRanged>
__device__ __forceinline__ void awq_slab_bucket(const mps_awq_tensor &T, const AwqWork &wk, int64_t b, bool tables,
                                                uint32_t &run_flags, const uint32_t *__restrict__ ckpt,
                                                uint32_t *__restrict__ lut, uint32_t *__restrict__ region,
                                                uint32_t *status) {
  int tid;
  __asm__ volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
  const bool by_scale = T.group_col_start != nullptr;
  const int32_t ra = T.bucket_row_offsets[b], rb = T.bucket_row_offsets[b + 1];
  const int32_t groups = rb - ra;  // groups (by-scale) or rows
  const int32_t c0 = by_scale ? 0 : T.bucket_col_start[b];
  const int32_t cl = by_scale ? 128 : T.bucket_col_len[b];
  constexpr bool kMulti = kRanged == 2;
  const int32_t K = kMulti ? (int32_t)T.k : kAwqBlock;  // substreams (the block stride)
  const uint32_t ks = K == 256 ? 8u : K == 512 ? 9u : 10u;
  const bool shape_ok =
      by_scale ? (groups >= (kMulti ? 1 : kSlabMinGroups) && groups <= kSlabMaxGroups && T.group_size == 128)
               : (groups >= 1 && groups <= 128 && cl >= 4 * K && cl % (kMulti ? 4 * K : K) == 0 && c0 >= 0 &&
                  (int64_t)c0 + cl <= T.m);
  const bool k_ok = kMulti ? (K == 256 || K == 512) : T.k == kAwqBlock;
  if (!shape_ok || !k_ok || ra < 0 || (int64_t)rb > T.num_row_indices) {
    if (tid == 0) flag(status, MPS_STATUS_BAD_BUCKET);
    return;
  }
  const uint32_t P = by_scale ? 0u : (uint32_t)cl >> ks;
  // a row range (kinds 2, 3): its first row and row count; its lanes start and
  // end at checkpoints. Kind 3: this work-item's group of K (uniform per wave)
  // and its range; a last record's spare groups have no rows and only take
  // part in the barriers. A by-scale kind 3 range is a range of slabs (K / 128
  // groups each): [s0, s0 + ns) of the bucket's slabs.
  const bool ranged = kRanged != 0 && !by_scale;
  const bool from_ckpt = ranged || kMulti;  // lanes start (and end) at checkpoints
  const int32_t sub = kMulti ? (int32_t)awq_uni((uint32_t)tid >> ks) : 0;
  const int32_t range = wk.range + sub;
  const int32_t first_row = ranged ? range * wk.range_rows : 0;
  const int32_t nr_all = ranged ? (groups - first_row < wk.range_rows ? groups - first_row : wk.range_rows) : groups;
  const int32_t gps = K >> 7;  // by-scale: groups per slab
  const int32_t s0 = kMulti && by_scale ? range * wk.range_rows : 0;
  const int32_t ns_all = (groups + gps - 1) / gps - s0;
  const int32_t ns = kMulti && by_scale ? (ns_all < wk.range_rows ? ns_all : wk.range_rows) : 0;
  // rows of the range (rows), or the bucket's groups (by-scale); 0 for a spare group
  const int32_t nr = kMulti ? (range < wk.ranges && (by_scale ? ns > 0 : nr_all > 0) ? nr_all : 0) : nr_all;
  if (!kMulti && nr <= 0) {
    if (tid == 0) flag(status, MPS_STATUS_BAD_BUCKET);
    return;
  }
  const uint32_t lane = kMulti ? (uint32_t)tid & (uint32_t)(K - 1) : (uint32_t)tid;  // within the group of K
  const uint32_t w = lane >> 6, wl = (uint32_t)tid & 63u;  // wave within the group of K, lane within the wave
  const uint32_t t = (w << 6) | (((uint32_t)tid & 15u) << 2) | (((uint32_t)tid >> 4) & 3u);  // substream
  const int q = tid >> 6, c = tid & 63;
  // level 1
  const __amdgpu_buffer_rsrc_t r_tab = awq_rsrc(T.bucket_table + b * 16, 64u);
  const int32_t gq = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_tab, (uint32_t)q * 4u, 0, 0);
  const __amdgpu_buffer_rsrc_t r_grow = awq_rsrc(T.row_indices + ra + first_row, (uint32_t)(nr > 0 ? nr : 0) * 4u);
  const __amdgpu_buffer_rsrc_t r_gcol = awq_rsrc(by_scale ? T.group_col_start + ra : nullptr, by_scale ? (uint32_t)groups * 4u : 0u);
  // by-scale: groups gps (s0 + wl) + w/2 and gps (s0 + wl + 64) + w/2 (slabs s0 + wl and s0 + wl + 64);
  // rows: rows wl and wl + 64
  const uint32_t gi0 = by_scale ? (uint32_t)gps * ((uint32_t)s0 + wl) + (w >> 1) : wl;
  const uint32_t gi1 = by_scale ? (uint32_t)gps * ((uint32_t)s0 + wl + 64u) + (w >> 1) : wl + 64u;
  const int32_t row0 = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_grow, gi0 * 4u, 0, 0);
  const int32_t col0 = by_scale ? (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_gcol, gi0 * 4u, 0, 0) : c0;
  const int32_t row1 = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_grow, gi1 * 4u, 0, 0);
  const int32_t col1 = by_scale ? (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_gcol, gi1 * 4u, 0, 0) : c0;
  const __amdgpu_buffer_rsrc_t r_sb = awq_rsrc(T.bucket_thread_startbit + b * (kAwqBlock + 1), (kAwqBlock + 1) * 4u);
  // kind 2: ranges - 1 checkpoint rows (between ranges); kind 3: ranges + 1 (the ends too)
  const uint32_t ck_rows = !from_ckpt ? 0u : kMulti ? (uint32_t)wk.ranges + 1u : (uint32_t)wk.ranges - 1u;
  const __amdgpu_buffer_rsrc_t r_ck = awq_rsrc(from_ckpt ? ckpt + wk.ckpt : nullptr, ck_rows * (uint32_t)K * 4u);
  // one unconditional load each from the chosen array (a load under a branch is
  // waited for where the branch joins, which would serialise the set-up's loads)
  const bool from_ck = from_ckpt && (kMulti || wk.range > 0), to_ck = from_ckpt && (kMulti || wk.range + 1 < wk.ranges);
  const __amdgpu_buffer_rsrc_t r_pos = from_ck ? r_ck : r_sb;
  const __amdgpu_buffer_rsrc_t r_end = to_ck ? r_ck : r_sb;
  const uint32_t ck0 = kMulti ? (uint32_t)range : (uint32_t)(wk.range - 1);  // checkpoint row of the range's start
  const uint32_t live = kMulti && nr <= 0 ? kSlabBsPast : 0u;               // spare groups load nothing
  const uint32_t pos = __builtin_amdgcn_raw_buffer_load_b32(
      r_pos, live | (from_ck ? ((ck0 << ks) + t) * 4u : t * 4u), 0, 0);
  const uint32_t pos_end = __builtin_amdgcn_raw_buffer_load_b32(
      r_end, live | (to_ck ? (((ck0 + 1u) << ks) + t) * 4u : (t + 1u) * 4u), 0, 0);
  const uint64_t bucket_bit = (uint64_t)T.bucket_bit_base[b];
  // Offset of the lane's first bitstream words and the descriptor's bitstream
  // fields, computed here, before the table loads (the words themselves are
  // loaded after the table expansion).
  uint32_t off0 = ((pos >> 5) & ~1u) * 4u;
  __asm__ volatile("" : "+v"(off0));
  const uint8_t *bs_ptr = reinterpret_cast<const uint8_t *>(T.bitstream);
  int64_t bs_words = T.bitstream_words;
  __asm__ volatile("" : "+s"(bs_ptr), "+s"(bs_words));
  // level 2
  const bool tab_ok = gq >= 0 && gq < T.num_tables;
  const bool tab_load = tables && tab_ok;
  const uint32_t G = (uint32_t)(T.num_tables > 0 ? T.num_tables : 0);
  const __amdgpu_buffer_rsrc_t r_syms = awq_rsrc(T.decode_syms, G * (uint32_t)(kAwqTable * 2));
  const __amdgpu_buffer_rsrc_t r_lens = awq_rsrc(T.decode_lens, G * (uint32_t)kAwqPacked);
  uint4 sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(
        r_syms, tab_load ? (uint32_t)gq * (uint32_t)(kAwqTable * 2) + (uint32_t)c * 64u + 16u * (uint32_t)i : kSlabBsPast,
        0, 0);
    sv[i] = make_uint4(x[0], x[1], x[2], x[3]);
  }
  const auto ln = __builtin_amdgcn_raw_buffer_load_b128(
      r_lens, tab_load ? (uint32_t)gq * (uint32_t)kAwqPacked + (uint32_t)c * 16u : kSlabBsPast, 0, 0);
  if (tables && tid == 0) {
    bool bad = false;
#pragma unroll
    for (int qq = 0; qq < 16; ++qq) {
      const int32_t id = gload(T.bucket_table + b * 16 + qq);
      bad |= id < -1 || id >= T.num_tables;
    }
    if (bad) flag(status, MPS_STATUS_BAD_TABLE);
  }
  // expansion: entry p of value q = sym << 16 | (nibble 15 ? 27 : nibble); a
  // missing table is all ESC entries, as the reference decodes it. The
  // nibbles go to bytes (even entries in `fl`, odd ones in `fh`); a byte b
  // becomes b + 12 when it is 15 (the carry of b + 1 into bit 4, times 3/4
  // of 16), and one byte permute per entry joins it with its symbol.
  uint32_t esc_seen = tab_ok ? 0u : 1u;
  if (tables) {
    const uint32_t nib32[4] = {ln[0], ln[1], ln[2], ln[3]};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = nib32[i] & 0x0F0F0F0Fu, hi = (nib32[i] >> 4) & 0x0F0F0F0Fu;
      const uint32_t el = ((lo + 0x01010101u) & 0x10101010u) >> 2, eh = ((hi + 0x01010101u) & 0x10101010u) >> 2;
      esc_seen |= el | eh;
      const uint32_t fl = tab_ok ? lo + el + (el << 1) : 0x1B1B1B1Bu;
      const uint32_t fh = tab_ok ? hi + eh + (eh << 1) : 0x1B1B1B1Bu;
      const uint32_t w4[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};  // zero for a missing table
      uint32_t e[8];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        e[2 * cc] = __builtin_amdgcn_perm(w4[cc], fl, 0x05040C00u | (uint32_t)cc);
        e[2 * cc + 1] = __builtin_amdgcn_perm(w4[cc], fh, 0x07060C00u | (uint32_t)cc);
      }
      uint4 *dst = reinterpret_cast<uint4 *>(lut + (q << kAwqL) + 32 * c + 8 * i);
      dst[0] = make_uint4(e[0], e[1], e[2], e[3]);
      dst[1] = make_uint4(e[4], e[5], e[6], e[7]);
    }
  }
  // The lane's first four bitstream words (two 16-byte loads), issued once the
  // wave's own tables are in LDS: issued before, these scattered loads (64
  // lines a wave) queued ahead of the other waves' table loads; here they
  // overlap the other waves' expansion and the barriers, and the decode waits
  // for them after issuing its first int4 loads.
  __builtin_amdgcn_sched_barrier(0);
  uint2 first[4];
  {
    const uint64_t bs_bytes = bs_words > 0 ? (uint64_t)bs_words * 8u : 0u;
    const uint64_t base_byte = bucket_bit >> 3;
    const uint32_t win_bytes = base_byte < bs_bytes ? (uint32_t)(bs_bytes - base_byte) : 0u;
    const __amdgpu_buffer_rsrc_t r_bs = awq_rsrc(bs_ptr + (base_byte < bs_bytes ? base_byte : 0), win_bytes);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(r_bs, off0 + 16u * (uint32_t)i, 0, 0);
      first[2 * i] = make_uint2(x[0], x[1]);
      first[2 * i + 1] = make_uint2(x[2], x[3]);
    }
  }
  // group bases of this wave for slabs wl and wl + 64 (by-scale), or the
  // offsets of rows wl and wl + 64 with the column start (rows)
  const uint32_t m = (uint32_t)T.m;
  auto gbase = [&](uint32_t gi, int32_t row, int32_t col, bool &bad) -> uint32_t {
    if (gi >= (uint32_t)nr) return 0u;
    bad |= row < 0 || (int64_t)row >= T.n || col < 0 || (int64_t)col + cl > T.m;
    return (uint32_t)row * m + (uint32_t)col + (by_scale ? ((w & 1u) << 6) : 0u);
  };
  bool bad_row = false;
  const uint32_t base_lo = gbase(gi0, row0, col0, bad_row);
  const uint32_t base_hi = gbase(gi1, row1, col1, bad_row);
  uint32_t *s_wflag = region + 5 * kAwqBlock;  // queue slot 5 until the decode starts
  {
    const uint32_t wf = (__builtin_amdgcn_ballot_w64(bad_row) ? 1u : 0u) |
                        (__builtin_amdgcn_ballot_w64(esc_seen != 0u) ? 2u : 0u);
    if (wl == 0) s_wflag[tid >> 6] = wf;  // one word per wave of the workgroup
  }
  __syncthreads();
  uint32_t bflags = 0;
#pragma unroll
  for (int i = 0; i < kAwqBlock / 64; ++i) bflags |= s_wflag[i];
  __syncthreads();  // the flag words belong to the queue from here on
  bflags = awq_uni(bflags);
  if (tables) run_flags = (bflags & 2u) | kRunTables;
  else bflags = (bflags & ~2u) | (run_flags & 2u);
  if (bflags & 1u) {
    if (tid == 0) flag(status, MPS_STATUS_BAD_ROW);
    return;
  }
  // this wave's elements per lane: by-scale, every full slab and the partial
  // last one when its group w/2 exists; rows, rows x P
  const uint32_t count = by_scale ? (uint32_t)groups / 8u + ((w >> 1) < ((uint32_t)groups & 7u) ? 1u : 0u)
                                  : (uint32_t)nr * P;
  const bool esc = (bflags & 2u) != 0u;
  if constexpr (kMulti) {
    if (nr <= 0) return;  // a spare group
    if (by_scale) {
      // this wave's slabs in the range: those whose group gps i + w/2 exists
      const int32_t cw = groups > (int32_t)(w >> 1) ? (groups - (int32_t)(w >> 1) + gps - 1) / gps : 0;
      const int32_t cnt = cw - s0 < 0 ? 0 : cw - s0 < ns ? cw - s0 : ns;
      if (esc)
        awq_slab_decode<true, kLayGroups, 0>(T, lut, region, (uint32_t)tid, lane, ks, (uint32_t)cnt, base_lo,
                                             base_hi, (uint32_t)groups, 0u, bucket_bit, first, pos, pos_end, status);
      else
        awq_slab_decode<false, kLayGroups, 0>(T, lut, region, (uint32_t)tid, lane, ks, (uint32_t)cnt, base_lo,
                                              base_hi, (uint32_t)groups, 0u, bucket_bit, first, pos, pos_end, status);
      return;
    }
    if (esc)
      awq_slab_decode<true, kLayRows, 0>(T, lut, region, (uint32_t)tid, lane, ks, count, base_lo, base_hi,
                                         (uint32_t)nr, P, bucket_bit, first, pos, pos_end, status);
    else
      awq_slab_decode<false, kLayRows, 0>(T, lut, region, (uint32_t)tid, lane, ks, count, base_lo, base_hi,
                                          (uint32_t)nr, P, bucket_bit, first, pos, pos_end, status);
    return;
  }
#define MPS_AWQ_SLAB(ESC, LAY)                                                                               \
  awq_slab_decode<ESC, LAY>(T, lut, region, (uint32_t)tid, (uint32_t)tid, 10u, count, base_lo, base_hi,       \
                            (uint32_t)nr, P, bucket_bit, first, pos, pos_end, status)
  if (by_scale) {
    if (esc) MPS_AWQ_SLAB(true, kLayGroups);
    else MPS_AWQ_SLAB(false, kLayGroups);
  } else if (P % 4u == 0u) {
    if (esc) MPS_AWQ_SLAB(true, kLayRows);
    else MPS_AWQ_SLAB(false, kLayRows);
  } else {
    if (esc) MPS_AWQ_SLAB(true, kLayRowsWrap);
    else MPS_AWQ_SLAB(false, kLayRowsWrap);
  }
#undef MPS_AWQ_SLAB
}

// A later bucket of a by-scale run, once the run's tables are in the LDS:
// each wave sets up and decodes its own part without meeting the others. A
// lane's queue slots and a wave's group bases are its own, so nothing here
// needs the workgroup: a wave that ends one bucket starts the next one's
// loads while the others still decode, and their latency hides behind them.
// A row or column out of range in a wave's groups flags and skips that
// wave's part (its groups only).
__device__ __forceinline__ void awq_slab_bucket_wave(const mps_awq_tensor &T, int64_t b, uint32_t run_flags,
                                                     const uint32_t *__restrict__ lut,
                                                     uint32_t *__restrict__ region, uint32_t *status) {
  int tid;
  __asm__ volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
  const int32_t ra = T.bucket_row_offsets[b], rb = T.bucket_row_offsets[b + 1];
  const int32_t groups = rb - ra;
  if (!(groups >= kSlabMinGroups && groups <= kSlabMaxGroups && T.group_size == 128) || ra < 0 ||
      (int64_t)rb > T.num_row_indices || T.k != kAwqBlock) {
    if (tid == 0) flag(status, MPS_STATUS_BAD_BUCKET);
    return;
  }
  const uint32_t w = (uint32_t)tid >> 6, wl = (uint32_t)tid & 63u;
  const uint32_t t = (w << 6) | (((uint32_t)tid & 15u) << 2) | (((uint32_t)tid >> 4) & 3u);  // substream
  // level 1: this wave's groups 8 wl + w/2 and 8 (wl + 64) + w/2, the lane's start and end bits
  const __amdgpu_buffer_rsrc_t r_grow = awq_rsrc(T.row_indices + ra, (uint32_t)groups * 4u);
  const __amdgpu_buffer_rsrc_t r_gcol = awq_rsrc(T.group_col_start + ra, (uint32_t)groups * 4u);
  const uint32_t gi0 = 8u * wl + (w >> 1), gi1 = 8u * (wl + 64u) + (w >> 1);
  const int32_t row0 = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_grow, gi0 * 4u, 0, 0);
  const int32_t col0 = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_gcol, gi0 * 4u, 0, 0);
  const int32_t row1 = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_grow, gi1 * 4u, 0, 0);
  const int32_t col1 = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_gcol, gi1 * 4u, 0, 0);
  const __amdgpu_buffer_rsrc_t r_sb = awq_rsrc(T.bucket_thread_startbit + b * (kAwqBlock + 1), (kAwqBlock + 1) * 4u);
  const uint32_t pos = __builtin_amdgcn_raw_buffer_load_b32(r_sb, t * 4u, 0, 0);
  const uint32_t pos_end = __builtin_amdgcn_raw_buffer_load_b32(r_sb, (t + 1u) * 4u, 0, 0);
  const uint64_t bucket_bit = (uint64_t)T.bucket_bit_base[b];
  // level 2: the lane's first bitstream words
  uint2 first[4];
  {
    const uint64_t bs_bytes = T.bitstream_words > 0 ? (uint64_t)T.bitstream_words * 8u : 0u;
    const uint64_t base_byte = bucket_bit >> 3;
    const uint32_t win_bytes = base_byte < bs_bytes ? (uint32_t)(bs_bytes - base_byte) : 0u;
    const __amdgpu_buffer_rsrc_t r_bs = awq_rsrc(
        reinterpret_cast<const uint8_t *>(T.bitstream) + (base_byte < bs_bytes ? base_byte : 0), win_bytes);
    const uint32_t off0 = ((pos >> 5) & ~1u) * 4u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(r_bs, off0 + 16u * (uint32_t)i, 0, 0);
      first[2 * i] = make_uint2(x[0], x[1]);
      first[2 * i + 1] = make_uint2(x[2], x[3]);
    }
  }
  const uint32_t m = (uint32_t)T.m;
  auto gbase = [&](uint32_t gi, int32_t row, int32_t col, bool &bad) -> uint32_t {
    if (gi >= (uint32_t)groups) return 0u;
    bad |= row < 0 || (int64_t)row >= T.n || col < 0 || (int64_t)col + 128 > T.m;
    return (uint32_t)row * m + (uint32_t)col + ((w & 1u) << 6);
  };
  bool bad_row = false;
  const uint32_t base_lo = gbase(gi0, row0, col0, bad_row);
  const uint32_t base_hi = gbase(gi1, row1, col1, bad_row);
  if (__builtin_amdgcn_ballot_w64(bad_row)) {
    if (wl == 0) flag(status, MPS_STATUS_BAD_ROW);
    return;
  }
  const uint32_t count = (uint32_t)groups / 8u + ((w >> 1) < ((uint32_t)groups & 7u) ? 1u : 0u);
  if (run_flags & 2u)
    awq_slab_decode<true, kLayGroups>(T, lut, region, (uint32_t)tid, (uint32_t)tid, 10u, count, base_lo, base_hi,
                                      (uint32_t)groups, 0u, bucket_bit, first, pos, pos_end, status);
  else
    awq_slab_decode<false, kLayGroups>(T, lut, region, (uint32_t)tid, (uint32_t)tid, 10u, count, base_lo, base_hi,
                                       (uint32_t)groups, 0u, bucket_bit, first, pos, pos_end, status);
}

// Lane checkpoints of a slab-path row bucket split into row ranges: where each
// substream stands at the first row of every range after the first, found by
// walking it through the code lengths once (the int4 value picks the table, the
// next 11 bits the length nibble; a nibble of 15 is an 11-bit ESC code and 16
// raw bits). One workgroup per bucket to split; lane t < k walks substream t,
// whose element (row r, block p) is column c0 + t + k p of the bucket's row r. A
// row index or table id out of range stops the walk and marks the job failed
// (the plan then keeps the bucket whole, and its decode reports them). A `full`
// job (ranges side by side, k 256 or 512) also writes rows 0 (the substreams'
// start bits) and `ranges` (their end bits). A by-scale job's ranges are ranges
// of slabs (`range_rows` slabs of k / 128 groups each; `rows`: the groups).
struct AwqSplitJob {
  int32_t tensor, bucket, P, rows;
  int32_t c0, range_rows, ranges, full;
  int64_t out;  // first u32 of the job's checkpoints: [ranges - 1][k], or [ranges + 1][k] when full
};

__global__ __launch_bounds__(kAwqBlock) void awq_checkpoints(const mps_awq_tensor *__restrict__ tensors,
                                                             const AwqSplitJob *__restrict__ jobs,
                                                             uint32_t *__restrict__ ckpt,
                                                             uint32_t *__restrict__ failed) {
  __shared__ int32_t s_gid[16];
  __shared__ uint8_t s_lens[16 * kAwqPacked];  // packed length nibbles of each int4 value's table
  const AwqSplitJob J = jobs[blockIdx.x];
  const mps_awq_tensor &T = tensors[J.tensor];
  const int tid = threadIdx.x;
  if (tid < 16) {
    int32_t g = T.bucket_table[(int64_t)J.bucket * 16 + tid];
    if (g < -1 || g >= T.num_tables) {
      failed[blockIdx.x] = 1u;
      g = -1;
    }
    s_gid[tid] = g;
  }
  __syncthreads();
  for (int i = tid; i < 16 * kAwqPacked; i += kAwqBlock) {
    const int32_t g = s_gid[i / kAwqPacked];
    s_lens[i] = g >= 0 ? T.decode_lens[(int64_t)g * kAwqPacked + i % kAwqPacked] : 0xFFu;  // missing: all ESC
  }
  __syncthreads();
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_awq_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;
  const int32_t K = (int32_t)T.k;
  if (tid >= K) return;
  const uint64_t bit_base = (uint64_t)T.bucket_bit_base[J.bucket];
  const int32_t ra = T.bucket_row_offsets[J.bucket];
  const uint32_t *sb = T.bucket_thread_startbit + (int64_t)J.bucket * (K + 1);
  const int64_t row0 = J.out - (J.full ? 0 : K);  // where checkpoint row 0 would go
  if (J.full) {
    ckpt[row0 + tid] = sb[tid];
    ckpt[row0 + (int64_t)J.ranges * K + tid] = sb[tid + 1];
  }
  uint64_t pos = bit_base + sb[tid];
  uint64_t cidx = ~0ull;
  uint32_t ca = 0, cb = 0;
  auto step = [&](uint32_t q) {  // past the code of one element with int4 value q
    const uint64_t c = pos >> 5;
    if (c != cidx) {
      cidx = c;
      ca = chunk_at(bs32, nchunks, c);
      cb = chunk_at(bs32, nchunks, c + 1);
    }
    const uint32_t peek = (uint32_t)(((((uint64_t)ca << 32) | cb) << (pos & 31u)) >> (64 - kAwqL));
    const uint32_t nib = (s_lens[q * kAwqPacked + (peek >> 1)] >> ((peek & 1u) * 4u)) & 0xFu;
    pos += nib == 15u ? (uint64_t)kAwqEscLow : (uint64_t)nib;
  };
  if (T.group_col_start) {
    // by-scale (J.rows groups of 128 columns): ranges of J.range_rows slabs of K / 128
    // groups; substream t's element in slab i is column t % 128 of group (K / 128) i + t / 128
    const int32_t gps = K >> 7, gsub = tid >> 7, col = tid & 127;
    for (int j = 1; j < J.ranges; ++j) {
      for (int32_t i = (j - 1) * J.range_rows; i < j * J.range_rows; ++i) {
        const int32_t g = gps * i + gsub;
        if (g >= J.rows) break;
        const int32_t row = T.row_indices[ra + g], c0 = T.group_col_start[ra + g];
        if (row < 0 || row >= T.n || c0 < 0 || (int64_t)c0 + 128 > T.m) {
          failed[blockIdx.x] = 1u;
          return;
        }
        step(T.int4[(int64_t)row * T.m + c0 + col] & 15u);
      }
      ckpt[row0 + (int64_t)j * K + tid] = (uint32_t)(pos - bit_base);
    }
    return;
  }
  for (int j = 1; j < J.ranges; ++j) {
    for (int32_t r = (j - 1) * J.range_rows; r < j * J.range_rows; ++r) {
      const int32_t row = T.row_indices[ra + r];
      if (row < 0 || row >= T.n) {
        failed[blockIdx.x] = 1u;
        return;
      }
      const uint8_t *qrow = T.int4 + (int64_t)row * T.m + J.c0 + tid;
      for (int32_t p = 0; p < J.P; ++p) step(qrow[(int64_t)p * K] & 15u);
    }
    ckpt[row0 + (int64_t)j * K + tid] = (uint32_t)(pos - bit_base);
  }
}

// Plan launch: workgroup i decodes buckets work[i].y .. work[i].y + work[i].z - 1
// of tensor work[i].x; work[i].w = 1 marks one slab-path bucket (above). A
// record's buckets have identical table ids (one scale),
// so they share the tables in LDS; each gets kAwqBlock / nsub work-items (its k
// lanes) and a kRowSlots / nsub slice of the row offsets. With k = 256 four
// buckets run in one workgroup instead of one (the tables allow one
// workgroup per CU).
// out_delta: elements every tensor's output moves by (a plan decoding into a
// buffer laid out like, but other than, the one it was created with).
// kRanges: bit 0, the plan has row ranges (kind 2 records); bit 1, row ranges
// side by side (kind 3); bit 2, tiny buckets (awq_tiny_lane). Plans without
// them launch the instantiation that leaves that path out: the range path's
// code in the same kernel measured 4.6% slower on a by-scale layer, the tiny
// path's 4.4% slower on a row-bucket layer.
// A bucket with no more elements than substreams codes one element a lane
// (k_eff = its element count), so staging its 16 tables in LDS (128 KiB) costs
// far more than its decode: each lane looks its one code up in the global
// tables instead (decode_huffman.cu:417-468 for one element: the peek, the
// length nibble, ESC with its 16 raw bits), and checks that the code ends
// where the next lane's begins.
__device__ __forceinline__ void awq_tiny_lane(const mps_awq_tensor &T, int64_t b, int32_t ra, int32_t c0, int32_t cl,
                                              int32_t k, int lane, uint32_t *status) {
  const uint32_t *__restrict__ sb = T.bucket_thread_startbit + b * ((int64_t)k + 1);
  const uint64_t pos0 = (uint64_t)T.bucket_bit_base[b] + gload(sb + lane);
  const uint64_t pos_end = (uint64_t)T.bucket_bit_base[b] + gload(sb + lane + 1);
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_awq_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;
  const uint64_t cb = pos0 >> 5;
  // 64 bits from the code's first chunk: the code and an ESC payload (27 bits) fit after any skip < 32
  const uint64_t buf = (((uint64_t)chunk_at(bs32, nchunks, cb) << 32) | chunk_at(bs32, nchunks, cb + 1))
                       << (pos0 & 31u);
  const int32_t rr = lane / cl, cc = lane - rr * cl;
  const int64_t row = gload(T.row_indices + ra + rr);
  const int64_t col = T.group_col_start ? (int64_t)gload(T.group_col_start + ra + rr) : (int64_t)c0;
  const bool ok = row >= 0 && row < T.n && col >= 0 && col + cl <= T.m;
  if (!ok) flag(status, MPS_STATUS_BAD_ROW);
  const uint32_t idx = ok ? (uint32_t)(row * T.m + col) + (uint32_t)cc : 0u;
  const uint32_t q = ok ? (uint32_t)gload(T.int4 + idx) & 15u : 0u;
  const int32_t gid = gload(T.bucket_table + b * 16 + q);
  const uint32_t peek = (uint32_t)(buf >> (64 - kAwqL));
  uint32_t nib = 15u, sym = 0u;
  if (gid >= 0 && gid < T.num_tables) {  // a missing table decodes as ESC, as the reference's kernel does
    const uint32_t ln = gload(T.decode_lens + (size_t)gid * kAwqPacked + (peek >> 1));
    nib = (peek & 1u) ? (ln >> 4) & 15u : ln & 15u;
    sym = gload(T.decode_syms + (size_t)gid * kAwqTable + peek);
  }
  uint32_t len = nib;
  if (nib == 15u) {  // ESC: the code is L bits, then 16 raw bits (decode_huffman.cu:454-460)
    sym = (uint32_t)((buf << kAwqL) >> 48);
    len = kAwqL + 16u;
  }
  if (ok) *(__attribute__((address_space(1))) uint16_t *)(T.out + idx) = (uint16_t)sym;
  if (pos0 + len != pos_end) flag(status, MPS_STATUS_DESYNC);
}

template <int kRanges>
__device__ __forceinline__ void awq_plan_record(const mps_awq_tensor *__restrict__ tensors, const AwqWork &wk,
                                                const uint32_t *__restrict__ ckpt, uint32_t *status,
                                                int64_t out_delta, uint32_t *__restrict__ lut,
                                                uint32_t *__restrict__ s_base) {
  const int4 w = make_int4(wk.tensor, wk.bucket, wk.nsub, wk.kind);
  mps_awq_tensor T = tensors[w.x];
  T.out += out_delta;
  uint32_t run_flags = 0;
  if (wk.kind == 1) {
    // a run of nsub buckets with identical table ids: the first bucket that
    // passes its checks loads the tables (the whole workgroup); the buckets
    // after it run wave by wave. Until the tables are in, every bucket takes
    // the workgroup path, whose checks are uniform, so all waves meet at its
    // barriers.
    for (int r = 0; r < wk.nsub; ++r) {
      const int64_t b = (int64_t)wk.bucket + r;
      if ((run_flags & kRunTables) == 0u) {
        awq_slab_bucket<0>(T, wk, b, true, run_flags, ckpt, lut, s_base, status);
      } else {
        awq_slab_bucket_wave(T, b, run_flags, lut, s_base, status);
      }
    }
    return;
  }
  if constexpr ((kRanges & 1) != 0) {
    if (wk.kind == 2) {
      awq_slab_bucket<1>(T, wk, wk.bucket, true, run_flags, ckpt, lut, s_base, status);
      return;
    }
  }
  if constexpr ((kRanges & 2) != 0) {
    if (wk.kind == 3) {
      awq_slab_bucket<2>(T, wk, wk.bucket, true, run_flags, ckpt, lut, s_base, status);
      return;
    }
  }
  const int nsub = w.z;
  const int per = kAwqBlock / nsub;
  const int slots = kRowSlots / nsub;
  const int tid = threadIdx.x;
  const int sub = tid / per, lane = tid - sub * per;
  const int64_t b = (int64_t)w.y + (sub < nsub ? sub : 0);
  if ((kRanges & 4) != 0 && wk.tiny) {
    // Tiny buckets (the plan checked that each has no more elements than k):
    // no tables in LDS, no barrier. Compiled only into the plans that have
    // such records: the path costs the others registers.
    if (tid == 0) {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int32_t g = gload(T.bucket_table + (int64_t)w.y * 16 + q);
        if (g < -1 || g >= T.num_tables) flag(status, MPS_STATUS_BAD_TABLE);
      }
    }
    if (sub >= nsub) return;
    const int32_t ra = T.bucket_row_offsets[b], rb = T.bucket_row_offsets[b + 1];
    const bool by_scale = T.group_col_start != nullptr;
    const int32_t c0 = by_scale ? 0 : T.bucket_col_start[b];
    const int32_t cl = by_scale ? (int32_t)T.group_size : T.bucket_col_len[b];
    if (rb <= ra) return;
    if (cl <= 0 || ra < 0 || (int64_t)rb > T.num_row_indices || (!by_scale && (c0 < 0 || (int64_t)c0 + cl > T.m))) {
      if (lane == 0) flag(status, MPS_STATUS_BAD_BUCKET);
      return;
    }
    const int64_t total = (int64_t)(rb - ra) * cl;
    if (lane < total && lane < (int)T.k) awq_tiny_lane(T, b, ra, c0, cl, (int32_t)T.k, lane, status);
    return;
  }

  // Tables of the record's first bucket, filled by all work-items (as awq_bucket<1>).
  {
    const int64_t b0 = w.y;
    int32_t gid[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) gid[q] = T.bucket_table[b0 * 16 + q];
    if (tid == 0) {
#pragma unroll
      for (int q = 0; q < 16; ++q)
        if (gid[q] < -1 || gid[q] >= T.num_tables) flag(status, MPS_STATUS_BAD_TABLE);
    }
    const int64_t G = T.num_tables;
    if (G <= 0) {
      for (int i = tid; i < kLutEntries; i += kAwqBlock) lut[i] = 15u;
    } else {
      uint32_t sy[32], ln[32];
#pragma unroll
      for (int it = 0; it < 32; ++it) {
        const int i = it * kAwqBlock + tid;
        const int q = i >> kAwqL, p = i & (kAwqTable - 1);
        const uint32_t g = (gid[q] >= 0 && gid[q] < G) ? (uint32_t)gid[q] : 0u;
        sy[it] = T.decode_syms[(size_t)g * kAwqTable + p];
        ln[it] = T.decode_lens[(size_t)g * kAwqPacked + (p >> 1)];
      }
#pragma unroll
      for (int it = 0; it < 32; ++it) {
        const int i = it * kAwqBlock + tid;
        const int q = i >> kAwqL, p = i & (kAwqTable - 1);
        const bool ok = gid[q] >= 0 && gid[q] < G;
        lut[i] = ok ? (sy[it] << 16) | ((p & 1) ? (ln[it] >> 4) : (ln[it] & 15u)) : 15u;
      }
    }
  }
  // This work-item's bucket (decode_huffman.cu:417-444, :528-545).
  const int32_t ra = T.bucket_row_offsets[b], rb = T.bucket_row_offsets[b + 1];
  const int32_t rows = rb - ra;
  const bool by_scale = T.group_col_start != nullptr;
  const int32_t c0 = by_scale ? 0 : T.bucket_col_start[b];
  const int32_t cl = by_scale ? (int32_t)T.group_size : T.bucket_col_len[b];
  bool ok = sub < nsub && rows > 0;
  if (ok && (cl <= 0 || ra < 0 || (int64_t)rb > T.num_row_indices ||
             (!by_scale && (c0 < 0 || (int64_t)c0 + cl > T.m)))) {
    if (lane == 0) flag(status, MPS_STATUS_BAD_BUCKET);
    ok = false;
  }
  uint32_t *__restrict__ my_base = s_base + sub * slots;
  if (ok) {
    const int32_t staged = rows < slots ? rows : slots;
    for (int r = lane; r < staged; r += per) {
      const int64_t row = T.row_indices[ra + r];
      const int64_t col = by_scale ? (int64_t)T.group_col_start[ra + r] : (int64_t)c0;
      uint32_t base = kBadBase;
      if (row >= 0 && row < T.n && col >= 0 && col + cl <= T.m) base = (uint32_t)(row * T.m + col);
      else flag(status, MPS_STATUS_BAD_ROW);
      my_base[r] = base;
    }
  }
  __syncthreads();
  if (!ok) return;
  const int64_t total = (int64_t)rows * cl;
  const int32_t k = (int32_t)T.k;
  const int32_t k_eff = total < k ? (int32_t)total : k;
  if (lane >= k_eff) return;
  // nsub > 1 only for buckets whose rows all fit their slice (the plan checks)
  if (rows <= slots) awq_lane<true>(T, lut, my_base, b, ra, c0, cl, total, k, k_eff, lane, status);
  else awq_lane<false>(T, lut, my_base, b, ra, c0, cl, total, k, k_eff, lane, status);
}

// Record trace, in instrumented builds only (python -m mpserve_amd.build
// --define MPS_TRACE_ITEMS=1 --out LIB; mpserve_amd.item_trace reads it):
// record r < kAwqTraceRecs stores the real-time clock (100 MHz) at its start
// and after a closing barrier, kind << 32 | nsub, and its ordering key.
#ifndef MPS_TRACE_ITEMS
#define MPS_TRACE_ITEMS 0
#endif
#if MPS_TRACE_ITEMS
constexpr int kAwqTraceRecs = 8192;
__device__ uint64_t g_awq_trace[kAwqTraceRecs * 4];
#endif

// The plan kernel is persistent (one workgroup per CU) and takes its records
// from a queue, as the FP8 plan kernel does: workgroup g starts with record g;
// thread 0 takes a ticket t from queue[0] as its wave finishes a record, and
// the workgroup's next record is gridDim.x + t. The records are sorted largest
// first, so the CUs that drew small records take more of them, and no record
// pays a workgroup launch. The last workgroup to leave (queue[1] counts them)
// puts both words back to zero: launches of one queue must not overlap.
__device__ __forceinline__ uint32_t queue_add(uint32_t *q, uint32_t v) {
  return __hip_atomic_fetch_add((__attribute__((address_space(1))) uint32_t *)(q), v, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}

template <int kRanges>
__global__ __launch_bounds__(kAwqBlock) void awq_decode_plan(const mps_awq_tensor *__restrict__ tensors,
                                                             const AwqWork *__restrict__ work, int64_t nwork,
                                                             const uint32_t *__restrict__ ckpt, uint32_t *status,
                                                             int64_t out_delta, uint32_t *queue) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[kRowSlots + kLutEntries];  // as in awq_decode_kernel
  uint32_t *s_base = lds, *lut = lds + kRowSlots;
  if ((int64_t)blockIdx.x < nwork) {
    int64_t r = blockIdx.x;
    for (;;) {
#if MPS_TRACE_ITEMS
      const uint64_t tr0 = __builtin_amdgcn_s_memrealtime();
#endif
      const AwqWork wk = work[r];
      awq_plan_record<kRanges>(tensors, wk, ckpt, status, out_delta, lut, s_base);
      // The ticket is taken once wave 0 is through with the record, so the
      // next record goes to a workgroup that is about to be free (taken at the
      // record's start, a long record's successor would wait behind it); its
      // round trip overlaps the other waves' last steps. Every wave is then
      // done with the LDS (the record's queue, where the ticket goes), thread 0
      // hands out the ticket, and every wave has read it before the next
      // record's set-up writes the LDS.
      uint32_t t = 0;
      if (threadIdx.x == 0) t = queue_add(queue, 1u);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (threadIdx.x == 0) lds[0] = t;
      __syncthreads();
      const int64_t next = (int64_t)gridDim.x + (int64_t)lds[0];
      __syncthreads();
#if MPS_TRACE_ITEMS
      if (threadIdx.x == 0 && r < kAwqTraceRecs) {
        uint64_t *tp = g_awq_trace + (size_t)r * 4;
        tp[0] = tr0;
        tp[1] = __builtin_amdgcn_s_memrealtime();
        tp[2] = ((uint64_t)(uint32_t)wk.kind << 32) | (uint32_t)wk.nsub;
        tp[3] = (uint64_t)wk.elems;
      }
#endif
      if (next >= nwork) break;
      r = next;
    }
  }
  if (threadIdx.x == 0) {
    if (queue_add(queue + 1, 1u) == gridDim.x - 1) {
      __hip_atomic_exchange((__attribute__((address_space(1))) uint32_t *)(queue), 0u, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_exchange((__attribute__((address_space(1))) uint32_t *)(queue + 1), 0u, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

int check_awq(const mps_awq_tensor *t) {
  if (!t) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor is NULL");
  if (t->n <= 0 || t->m <= 0) return fail(MPS_ERR_INVALID_ARGUMENT, "n,m must be > 0");
  if (t->n * t->m >= ((int64_t)1 << 31)) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor too large (n*m >= 2^31)");
  if (t->k <= 0 || t->k > kAwqBlock)
    return fail(MPS_ERR_INVALID_ARGUMENT, "bucket_thread_startbit_u32 has invalid k (must be 1..1024)");
  if (t->num_buckets < 0 || t->num_buckets >= ((int64_t)1 << 31))
    return fail(MPS_ERR_INVALID_ARGUMENT, "invalid bucket count");
  if (t->num_buckets > 0 && (!t->int4 || !t->bucket_table || !t->bucket_row_offsets || !t->row_indices ||
                             !t->bucket_thread_startbit || !t->bucket_bit_base || !t->out))
    return fail(MPS_ERR_INVALID_ARGUMENT, "NULL sidecar array");
  if (t->group_col_start) {
    if (t->group_size <= 0 || t->group_size > t->m) return fail(MPS_ERR_INVALID_ARGUMENT, "group_size must be in (0,m]");
  } else if (t->num_buckets > 0 && (!t->bucket_col_start || !t->bucket_col_len)) {
    return fail(MPS_ERR_INVALID_ARGUMENT, "NULL sidecar array");
  }
  if (t->num_tables > 0 && (!t->decode_syms || !t->decode_lens))
    return fail(MPS_ERR_INVALID_ARGUMENT, "NULL sidecar array");
  return MPS_OK;
}

}  // namespace
}  // namespace mps

using namespace mps;

// A plan owns one device allocation: its status word, the tensor descriptors,
// the work records, and the split jobs and lane checkpoints of its row ranges.
// Work queues of a plan: one per stream that launches it (two u32 words each,
// 64 bytes apart), so that launches on different streams never share one.
constexpr int kAwqPlanQueues = 32;
constexpr size_t kAwqQueueStride = 64;

struct mps_awq_plan {
  int device = 0;
  int64_t count = 0, nwork = 0;
  // kAwqPlanQueues work queues (zero between launches); queue i serves
  // streams[i], assigned at the stream's first launch
  uint32_t *d_queue = nullptr;
  std::mutex mu;
  std::vector<void *> streams;
  uint16_t *first_out = nullptr;  // the first tensor's output at creation (decode_into moves from it)
  void *d_block = nullptr;
  uint32_t *d_status = nullptr;
  mps_awq_tensor *d_tensors = nullptr;
  AwqWork *d_work = nullptr;
  uint32_t *d_ckpt = nullptr;  // lane checkpoints of the row buckets split into ranges
  int64_t splits = 0;          // row buckets split into ranges
  // bit 0: some work record is a row range (kind 2); bit 1: ranges side by side
  // (kind 3); bit 2: tiny buckets (kind 0 with `tiny`)
  int ranges_mode = 0;
};

extern "C" {

#if MPS_TRACE_ITEMS
// The record trace's host side (instrumented builds only; not part of the product ABI).
int mps_awq_trace_clear(void) {
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_awq_trace)) != hipSuccess) return MPS_ERR_HIP;
  return hipMemset(p, 0, sizeof(g_awq_trace)) == hipSuccess ? MPS_OK : MPS_ERR_HIP;
}
int mps_awq_trace_read(uint64_t *dst, int64_t words) {
  if (!dst || words < (int64_t)(sizeof(g_awq_trace) / 8)) return MPS_ERR_INVALID_ARGUMENT;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_awq_trace), sizeof(g_awq_trace)) == hipSuccess ? MPS_OK : MPS_ERR_HIP;
}
#endif


int mps_awq_decode(const mps_awq_tensor *tensor, int64_t max_len, void *stream) {
  last_error().clear();
  if (max_len != kAwqL) return fail(MPS_ERR_INVALID_ARGUMENT, "AWQ bucket decode kernel is specialized: max_len must be 11");
  int rc = check_awq(tensor);
  if (rc != MPS_OK) return rc;
  if (tensor->num_buckets == 0) return MPS_OK;
  int dev = 0;
  MPS_HIP_CHECK(hipGetDevice(&dev));
  uint32_t *status = nullptr;
  rc = status_word(dev, &status);
  if (rc != MPS_OK) return rc;
  // Fewer buckets than CUs: split each bucket's lanes over 2 workgroups.
  int cus = 0;
  MPS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int64_t B = tensor->num_buckets;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (B >= cus)
    hipLaunchKernelGGL(awq_decode_kernel<1>, dim3((unsigned)B), dim3(kAwqBlock), 0, s, *tensor, status);
  else
    hipLaunchKernelGGL(awq_decode_kernel<2>, dim3((unsigned)(2 * B)), dim3(kAwqBlock / 2), 0, s, *tensor, status);
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

int mps_awq_plan_create(const mps_awq_tensor *tensors, int64_t count, void *stream, mps_awq_plan **plan_out) {
  last_error().clear();
  if (!plan_out) return fail(MPS_ERR_INVALID_ARGUMENT, "plan_out is NULL");
  *plan_out = nullptr;
  if (count < 0 || count >= ((int64_t)1 << 31) || (count > 0 && !tensors))
    return fail(MPS_ERR_INVALID_ARGUMENT, "invalid tensor list");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // The sidecars may still be being written by work on the caller's stream.
  MPS_HIP_CHECK(hipStreamSynchronize(st));
  int dev = 0, cus = 0;
  MPS_HIP_CHECK(hipGetDevice(&dev));
  MPS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  // Work records (AwqWork). Slab-eligible buckets get one record each (kind 1),
  // except that by-scale ones take in the following buckets with identical
  // table ids (nsub in all); the others run in runs of up to 1024 / k
  // consecutive buckets of one tensor with identical table ids (one scale) and
  // at most kRowSlots / 4 rows each, so they can share a workgroup's tables
  // (kind 0).
  std::vector<AwqWork> base;
  std::vector<int32_t> roff, clen, cst, btab, gcol;
  // Elements a by-scale slab record's run of buckets may hold: a CU's share
  // of the plan (records go out largest first, so the large ones run early
  // and small ones fill the end; half a share measured 0.9% slower on an 8B
  // layer, a quarter 4.8%).
  int64_t all_elems = 0;
  for (int64_t i = 0; i < count; ++i)
    if (tensors[i].n > 0 && tensors[i].m > 0 && tensors[i].n < ((int64_t)1 << 31) && tensors[i].m < ((int64_t)1 << 31))
      all_elems += tensors[i].n * tensors[i].m;
#ifndef MPS_AWQ_RUN_DIV
#define MPS_AWQ_RUN_DIV 1
#endif
  const int64_t run_cap = std::max<int64_t>(1, all_elems / (MPS_AWQ_RUN_DIV * (int64_t)std::max(cus, 1)));
  // row-layout slab records: rows, P, column start; k for the records of
  // buckets whose ranges may run side by side (0: others)
  std::vector<int32_t> rows_of_rec, p_of_rec, c0_of_rec, k_of_rec;
  const char *slab_env = std::getenv("MPSERVE_AWQ_SLAB");
  const bool slab_on = !(slab_env && slab_env[0] == '0');
  int64_t total = 0;
  for (int64_t i = 0; i < count; ++i) {
    const mps_awq_tensor &T = tensors[i];
    int rc = check_awq(&T);
    if (rc != MPS_OK) return rc;
    const int64_t B = T.num_buckets;
    if (B == 0) continue;
    roff.resize((size_t)B + 1);
    btab.resize((size_t)B * 16);
    MPS_HIP_CHECK(hipMemcpy(roff.data(), T.bucket_row_offsets, sizeof(int32_t) * (B + 1), hipMemcpyDefault));
    MPS_HIP_CHECK(hipMemcpy(btab.data(), T.bucket_table, sizeof(int32_t) * B * 16, hipMemcpyDefault));
    if (!T.group_col_start) {
      clen.resize((size_t)B);
      MPS_HIP_CHECK(hipMemcpy(clen.data(), T.bucket_col_len, sizeof(int32_t) * B, hipMemcpyDefault));
    }
    // The slab path (k = 1024: by-scale with 128-column groups, or row buckets of
    // 1..128 rows over P >= 4 blocks of 1024 columns) loads int4 bytes as dwords
    // and stores 8 bytes a lane: every group or column range must start on a
    // 4-element boundary and the buffers must be aligned to match.
    bool slab_tensor = slab_on && T.k == kAwqBlock && (!T.group_col_start || T.group_size == 128) && T.m % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(T.int4) & 3u) == 0 && (reinterpret_cast<uintptr_t>(T.out) & 7u) == 0;
    // By-scale sidecars with k 256 or 512 and 128-column groups: buckets cut into
    // ranges of slabs (k / 128 groups each), 1024 / k ranges side by side a record.
    bool bmulti_tensor = slab_on && (T.k == 256 || T.k == 512) && T.group_col_start && T.group_size == 128 &&
                         T.m % 4 == 0 && (reinterpret_cast<uintptr_t>(T.int4) & 3u) == 0 &&
                         (reinterpret_cast<uintptr_t>(T.out) & 7u) == 0;
    if ((slab_tensor || bmulti_tensor) && T.group_col_start && T.num_row_indices > 0) {
      gcol.resize((size_t)T.num_row_indices);
      MPS_HIP_CHECK(hipMemcpy(gcol.data(), T.group_col_start, sizeof(int32_t) * T.num_row_indices, hipMemcpyDefault));
      const bool aligned = std::all_of(gcol.begin(), gcol.end(), [](int32_t c) { return (c & 3) == 0; });
      slab_tensor = slab_tensor && aligned;
      bmulti_tensor = bmulti_tensor && aligned;
    }
    // Row buckets with k 256 or 512 and P = col_len / k a multiple of 4: the
    // slab path at stride k, with 1024 / k row ranges side by side a record
    // (kind 3), else a bucket fills only k of the 1024 work-items.
    const bool multi_tensor = slab_on && (T.k == 256 || T.k == 512) && !T.group_col_start && T.m % 4 == 0 &&
                              (reinterpret_cast<uintptr_t>(T.int4) & 3u) == 0 &&
                              (reinterpret_cast<uintptr_t>(T.out) & 7u) == 0;
    if ((slab_tensor || multi_tensor) && !T.group_col_start) {
      cst.resize((size_t)B);
      MPS_HIP_CHECK(hipMemcpy(cst.data(), T.bucket_col_start, sizeof(int32_t) * B, hipMemcpyDefault));
    }
    auto rows_of = [&](int64_t b) { return std::max<int64_t>(0, (int64_t)roff[(size_t)b + 1] - roff[(size_t)b]); };
    auto elems_of = [&](int64_t b) {
      const int64_t cols = T.group_col_start ? T.group_size : (int64_t)clen[(size_t)b];
      return rows_of(b) * std::max<int64_t>(0, cols);
    };
    const int64_t maxsub = T.k <= kAwqBlock / 4 ? 4 : T.k <= kAwqBlock / 2 ? 2 : 1;
    const int64_t row_cap = kRowSlots / 4;
    // (cst holds the column starts only for a slab-eligible row-layout tensor)
    auto slab_ok = [&](int64_t bb) {
      const bool shape =
          slab_tensor &&
          (T.group_col_start
               ? rows_of(bb) >= kSlabMinGroups && rows_of(bb) <= kSlabMaxGroups
               : rows_of(bb) >= 1 && rows_of(bb) <= 128 && clen[(size_t)bb] >= 4 * kAwqBlock &&
                     clen[(size_t)bb] % kAwqBlock == 0 && cst[(size_t)bb] >= 0 && (cst[(size_t)bb] & 3) == 0 &&
                     (int64_t)cst[(size_t)bb] + clen[(size_t)bb] <= T.m);
      return shape && roff[(size_t)bb] >= 0 && roff[(size_t)bb + 1] <= T.num_row_indices;
    };
    auto multi_ok = [&](int64_t bb) {
      const int64_t kk = T.k;
      if (roff[(size_t)bb] < 0 || roff[(size_t)bb + 1] > T.num_row_indices) return false;
      // by-scale: at least 32 slabs (below that the set-up outweighs the decode, and
      // runs of same-scale buckets on the per-lane path share one set-up)
      if (T.group_col_start) return bmulti_tensor && rows_of(bb) >= 32 * (kk / 128) && rows_of(bb) <= kSlabMaxGroups;
      return multi_tensor && rows_of(bb) >= 1 && rows_of(bb) <= 128 && clen[(size_t)bb] >= 4 * kk &&
             clen[(size_t)bb] % (4 * kk) == 0 && cst[(size_t)bb] >= 0 && (cst[(size_t)bb] & 3) == 0 &&
             (int64_t)cst[(size_t)bb] + clen[(size_t)bb] <= T.m;
    };
    auto same_tables = [&](int64_t x, int64_t y) {
      return std::equal(btab.begin() + x * 16, btab.begin() + x * 16 + 16, btab.begin() + y * 16);
    };
    int64_t b = 0;
    while (b < B) {
      total += elems_of(b);
      if (slab_ok(b)) {
        // by-scale: a run of following buckets with identical table ids (one
        // scale's group-cap chunks) joins the record, up to run_cap elements
        int64_t run = 1, elems = elems_of(b);
        if (T.group_col_start) {
          while (b + run < B && elems + elems_of(b + run) <= run_cap && slab_ok(b + run) && same_tables(b, b + run)) {
            elems += elems_of(b + run);
            total += elems_of(b + run);
            ++run;
          }
        }
        base.push_back(AwqWork{(int32_t)i, (int32_t)b, (int32_t)run, 1, 0, 0, 1, 0, 0, elems});
        rows_of_rec.push_back(T.group_col_start ? 0 : (int32_t)rows_of(b));
        p_of_rec.push_back(T.group_col_start ? 0 : clen[(size_t)b] / kAwqBlock);
        c0_of_rec.push_back(T.group_col_start ? 0 : cst[(size_t)b]);
        k_of_rec.push_back(0);
        b += run;
        continue;
      }
      if (multi_ok(b)) {
        // a per-lane record (kind 0), replaced by side-by-side ranges once its
        // checkpoint walk succeeds
        base.push_back(AwqWork{(int32_t)i, (int32_t)b, 1, 0, 0, 0, 1, 0, 0, elems_of(b)});
        rows_of_rec.push_back((int32_t)rows_of(b));  // rows, or groups (by-scale: P = 0)
        p_of_rec.push_back(T.group_col_start ? 0 : (int32_t)(clen[(size_t)b] / T.k));
        c0_of_rec.push_back(T.group_col_start ? 0 : cst[(size_t)b]);
        k_of_rec.push_back((int32_t)T.k);
        ++b;
        continue;
      }
      int64_t nsub = 1, elems = elems_of(b);
      // Tiny: every bucket of the record codes at most one element a lane (k =
      // 1024 only: with k 256 / 512 such buckets run in same-scale runs that
      // share one table set-up, and the tiny path measured 2.9% slower there)
      bool tiny = T.k == kAwqBlock && elems_of(b) <= T.k;
      if (rows_of(b) <= row_cap) {
        while (nsub < maxsub && b + nsub < B && rows_of(b + nsub) <= row_cap && !multi_ok(b + nsub) &&
               same_tables(b, b + nsub)) {
          elems += elems_of(b + nsub);
          total += elems_of(b + nsub);
          tiny = tiny && elems_of(b + nsub) <= T.k;
          ++nsub;
        }
      }
      base.push_back(AwqWork{(int32_t)i, (int32_t)b, (int32_t)nsub, 0, 0, 0, 1, tiny ? 1 : 0, 0, elems});
      rows_of_rec.push_back(0);
      p_of_rec.push_back(0);
      c0_of_rec.push_back(0);
      k_of_rec.push_back(0);
      b += nsub;
    }
  }
  // Row ranges: a slab-path row bucket with more than total / (2 * CUs) elements
  // is split into row ranges of at least 64 elements a lane, each started from
  // lane checkpoints that one walk over the bucket's substreams finds.
  // A bucket with k 256 or 512 (k_of_rec) is always cut, into up to 1024 / k
  // ranges a record (one record per total / (2 * CUs) elements), which share
  // the record's set-up.
  const int64_t target = std::max<int64_t>(1, total / (2 * (int64_t)std::max(cus, 1)));
  std::vector<AwqSplitJob> jobs;
  std::vector<size_t> job_rec;  // the base record each job splits
  int64_t ck_words = 0;
  for (size_t r = 0; r < base.size(); ++r) {
    const AwqWork &w = base[r];
    const int32_t rows = rows_of_rec[r], P = p_of_rec[r];
    if (k_of_rec[r] > 0) {
      // units: rows, or slabs of k / 128 groups (by-scale, at most 128 a range: the
      // slab path keeps a wave's 128 group bases in two registers)
      // More than one record only while each range keeps >= 64 elements a lane.
      const int64_t S = kAwqBlock / k_of_rec[r];
      const int64_t gps = k_of_rec[r] / 128;
      const int64_t units = P > 0 ? rows : (rows + gps - 1) / gps;
      const int64_t min_units = P > 0 ? (64 + P - 1) / P : 64;
      const int64_t recs = std::min(std::max<int64_t>(1, (w.elems + target - 1) / target),
                                    std::max<int64_t>(1, units / (S * min_units)));
      int64_t ranges = std::min<int64_t>(units, S * recs);
      if (P == 0) ranges = std::max<int64_t>(ranges, (units + 127) / 128);
      const int32_t rr = (int32_t)((units + ranges - 1) / ranges);
      ranges = (units + rr - 1) / rr;
      jobs.push_back(AwqSplitJob{w.tensor, w.bucket, P, rows, c0_of_rec[r], rr, (int32_t)ranges, 1, ck_words});
      job_rec.push_back(r);
      ck_words += (ranges + 1) * k_of_rec[r];
      continue;
    }
    if (w.kind != 1 || rows < 2 || w.elems <= target) continue;
    const int64_t want = (w.elems + target - 1) / target;
    int32_t rr = (int32_t)((rows + want - 1) / want);
    rr = std::max<int32_t>(rr, (64 + P - 1) / P);
    const int32_t ranges = (rows + rr - 1) / rr;
    if (ranges < 2) continue;
    jobs.push_back(AwqSplitJob{w.tensor, w.bucket, P, rows, c0_of_rec[r], rr, ranges, 0, ck_words});
    job_rec.push_back(r);
    ck_words += (int64_t)(ranges - 1) * kAwqBlock;
  }
  auto make_records = [&](const std::vector<uint32_t> &failed) {
    std::vector<AwqWork> out;
    std::vector<int> split_of(base.size(), -1);
    for (size_t j = 0; j < jobs.size(); ++j)
      if (failed.empty() || failed[j] == 0u) split_of[job_rec[j]] = (int)j;
    for (size_t r = 0; r < base.size(); ++r) {
      if (split_of[r] < 0) {
        out.push_back(base[r]);
        continue;
      }
      const AwqSplitJob &J = jobs[(size_t)split_of[r]];
      if (J.full) {
        // 1024 / k ranges a record; the cost: one range's elements a work-item, x 1024
        const int32_t S = kAwqBlock / k_of_rec[r];
        const int32_t gps = k_of_rec[r] / 128;
        const int32_t units = J.P > 0 ? J.rows : (J.rows + gps - 1) / gps;
        for (int32_t g = 0; g < J.ranges; g += S) {
          const int32_t n = std::min(J.range_rows, units - g * J.range_rows);
          out.push_back(AwqWork{J.tensor, J.bucket, 1, 3, g, J.range_rows, J.ranges, 0, J.out,
                                (int64_t)n * std::max(J.P, 1) * kAwqBlock});
        }
        continue;
      }
      for (int32_t g = 0; g < J.ranges; ++g) {
        const int32_t nrows = std::min(J.range_rows, J.rows - g * J.range_rows);
        out.push_back(AwqWork{J.tensor, J.bucket, 1, 2, g, J.range_rows, J.ranges, 0, J.out,
                              (int64_t)nrows * J.P * kAwqBlock});
      }
    }
    // largest first, so the launch's last workgroups are its smallest
    std::stable_sort(out.begin(), out.end(), [](const AwqWork &x, const AwqWork &y) { return x.elems > y.elems; });
    return out;
  };
  std::vector<AwqWork> items = make_records({});
  auto plan = new (std::nothrow) mps_awq_plan();
  if (!plan) return fail(MPS_ERR_NO_MEMORY, "out of memory");
  plan->device = dev;
  plan->count = count;
  plan->nwork = (int64_t)items.size();
  plan->first_out = count > 0 ? tensors[0].out : nullptr;
  // status word (zero) | work queues (zero) | descriptors | work records | split jobs | checkpoints | job failure flags
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t o_queues = 256;
  const size_t o_tensors = o_queues + up(kAwqQueueStride * kAwqPlanQueues);
  const size_t o_work = o_tensors + up(sizeof(mps_awq_tensor) * (size_t)count);
  const size_t o_jobs = o_work + up(sizeof(AwqWork) * items.size());
  const size_t o_ckpt = o_jobs + up(sizeof(AwqSplitJob) * jobs.size());
  const size_t o_failed = o_ckpt + up(sizeof(uint32_t) * (size_t)ck_words);
  std::vector<char> host(o_failed + up(sizeof(uint32_t) * jobs.size()), 0);
  if (count > 0) std::memcpy(host.data() + o_tensors, tensors, sizeof(mps_awq_tensor) * (size_t)count);
  if (!items.empty()) std::memcpy(host.data() + o_work, items.data(), sizeof(AwqWork) * items.size());
  if (!jobs.empty()) std::memcpy(host.data() + o_jobs, jobs.data(), sizeof(AwqSplitJob) * jobs.size());
  hipError_t e = hipMalloc(&plan->d_block, host.size());
  if (e == hipSuccess) {
    char *blk = static_cast<char *>(plan->d_block);
    plan->d_status = reinterpret_cast<uint32_t *>(blk);
    plan->d_queue = reinterpret_cast<uint32_t *>(blk + o_queues);
    plan->d_tensors = reinterpret_cast<mps_awq_tensor *>(blk + o_tensors);
    plan->d_work = reinterpret_cast<AwqWork *>(blk + o_work);
    plan->d_ckpt = reinterpret_cast<uint32_t *>(blk + o_ckpt);
    e = hipMemcpyAsync(blk, host.data(), host.size(), hipMemcpyHostToDevice, st);
    if (e == hipSuccess && !jobs.empty()) {
      hipLaunchKernelGGL(awq_checkpoints, dim3((unsigned)jobs.size()), dim3(kAwqBlock), 0, st, plan->d_tensors,
                         reinterpret_cast<const AwqSplitJob *>(blk + o_jobs), plan->d_ckpt,
                         reinterpret_cast<uint32_t *>(blk + o_failed));
      e = hipGetLastError();
      std::vector<uint32_t> failed(jobs.size(), 0u);
      if (e == hipSuccess)
        e = hipMemcpyAsync(failed.data(), blk + o_failed, sizeof(uint32_t) * jobs.size(), hipMemcpyDeviceToHost, st);
      if (e == hipSuccess) e = hipStreamSynchronize(st);
      if (e == hipSuccess && std::any_of(failed.begin(), failed.end(), [](uint32_t f) { return f != 0u; })) {
        // keep the buckets whose walk failed whole (fewer records than before)
        items = make_records(failed);
        plan->nwork = (int64_t)items.size();
        e = hipMemcpyAsync(blk + o_work, items.data(), sizeof(AwqWork) * items.size(), hipMemcpyHostToDevice, st);
      }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
  }
  if (e != hipSuccess) {
    mps_awq_plan_destroy(plan);
    return hip_fail(e, "mps_awq_plan_create");
  }
  plan->splits = (int64_t)jobs.size();
  plan->ranges_mode = (std::any_of(items.begin(), items.end(), [](const AwqWork &w) { return w.tiny != 0; }) ? 4 : 0) |
                      (std::any_of(items.begin(), items.end(), [](const AwqWork &w) { return w.kind == 2; }) ? 1 : 0) |
                      (std::any_of(items.begin(), items.end(), [](const AwqWork &w) { return w.kind == 3; }) ? 2 : 0);
  *plan_out = plan;
  return MPS_OK;
}

static int awq_plan_launch(mps_awq_plan *plan, int64_t out_delta, uint32_t *status, void *stream) {
  if (plan->nwork == 0) return MPS_OK;
  // The stream's work queue: the one it was given at its first launch, or the
  // next free one. A launch leaves its queue as it found it, so launches on
  // one stream share one; a graph captured on a stream replays with its queue.
  uint32_t *queue = nullptr;
  {
    std::lock_guard<std::mutex> lock(plan->mu);
    size_t i = 0;
    while (i < plan->streams.size() && plan->streams[i] != stream) ++i;
    if (i == plan->streams.size()) {
      if (i >= (size_t)kAwqPlanQueues)
        return fail(MPS_ERR_RUNTIME, "an AWQ decode plan serves at most %d streams", kAwqPlanQueues);
      plan->streams.push_back(stream);
    }
    queue = plan->d_queue + i * (kAwqQueueStride / sizeof(uint32_t));
  }
  int cus = 0;
  MPS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, plan->device));
  const unsigned grid = (unsigned)std::min<int64_t>(plan->nwork, std::max(cus, 1));
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kAwqBlock), 0, reinterpret_cast<hipStream_t>(stream), plan->d_tensors,
                       plan->d_work, plan->nwork, plan->d_ckpt, status, out_delta, queue);
  };
  switch (plan->ranges_mode) {
    case 0: launch(awq_decode_plan<0>); break;
    case 1: launch(awq_decode_plan<1>); break;
    case 2: launch(awq_decode_plan<2>); break;
    case 3: launch(awq_decode_plan<3>); break;
    case 4: launch(awq_decode_plan<4>); break;
    case 5: launch(awq_decode_plan<5>); break;
    case 6: launch(awq_decode_plan<6>); break;
    default: launch(awq_decode_plan<7>); break;
  }
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

int mps_awq_plan_decode(mps_awq_plan *plan, void *stream) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  return awq_plan_launch(plan, 0, plan->d_status, stream);
}

int mps_awq_plan_decode_into(mps_awq_plan *plan, uint16_t *out, void *stream) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (!out) return fail(MPS_ERR_INVALID_ARGUMENT, "out is NULL");
  if (plan->count == 0) return MPS_OK;
  uint32_t *status = nullptr;
  const int rc = status_word(plan->device, &status);
  if (rc != MPS_OK) return rc;
  const intptr_t delta = reinterpret_cast<intptr_t>(out) - reinterpret_cast<intptr_t>(plan->first_out);
  // the slab path stores 8 bytes a lane: the moved outputs keep its alignment
  if (delta % 8 != 0) return fail(MPS_ERR_INVALID_ARGUMENT, "out must be aligned like the plan's outputs (8 bytes)");
  return awq_plan_launch(plan, (int64_t)(delta / (intptr_t)sizeof(uint16_t)), status, stream);
}

int mps_awq_plan_info(const mps_awq_plan *plan, int64_t *work_items) {
  if (!plan || !work_items) return fail(MPS_ERR_INVALID_ARGUMENT, "NULL argument");
  *work_items = plan->nwork;
  return MPS_OK;
}

int mps_awq_plan_read_status(mps_awq_plan *plan, void *stream, uint32_t *status_out) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (!status_out) return fail(MPS_ERR_INVALID_ARGUMENT, "status_out is NULL");
  return read_and_clear(plan->device, plan->d_status, stream, "mps_awq_plan_read_status", status_out);
}

int mps_awq_plan_destroy(mps_awq_plan *plan) {
  if (!plan) return MPS_OK;
  if (plan->d_block) (void)hipFree(plan->d_block);
  delete plan;
  return MPS_OK;
}

}  // extern "C"
