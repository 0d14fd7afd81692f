// FP8 + Huffman-sidecar -> BF16 decode for MI355X (gfx950).
//
// Format (reference kernel/build_huffman.cu:786-925): bucket b owns rows
// row_indices[row_offsets[b] .. row_offsets[b+1]) x columns [col_start, col_start+col_len).
// Its elements, flattened row-major, are dealt round-robin to k_eff = min(k, total)
// lanes: lane t codes e = t, t+k_eff, ...; each lane's codes form one MSB-first
// substream starting at bit bucket_bit_base[b] + bucket_thread_startbit[b][t].
// A code is looked up with the next 7 bits in the table of the key
// (bucket scale, fp8 byte of the element); a length nibble with bit 3 set marks
// ESC: 16 raw BF16 bits follow the code.
//
// Mapping to CDNA4: one workgroup of 1024 work-items per bucket (one lane per
// work-item, 16 wave64s). The bucket's 256 code tables are expanded once into
// LDS as 32-bit entries {sym:16 | len:3 | esc:1} (128 KiB), so one ds_read_b32
// per element resolves symbol, length and ESC. The bitstream is read as 32-bit
// chunks into a 64-bit MSB-aligned register buffer that is topped up whenever
// fewer than 32 bits remain, which keeps 7 + 16 bits available for any code
// plus its ESC payload.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <queue>
#include <type_traits>
#include <vector>

#include "mps_common.h"

namespace mps {

namespace {

constexpr int kL = 7;
constexpr int kTable = 1 << kL;           // 128 entries per code table
constexpr int kPacked = kTable / 2;       // 64 bytes of packed 4-bit lengths
constexpr int kBlock = 1024;              // work-items per bucket workgroup (>= k)
constexpr int kRowsLds = 256;             // row indices staged in LDS
// LDS code table entry: sym << 16 | esc << 4 | len. A shift by the whole entry
// shifts by len (its low 5 bits), and a 16-bit store of the high half stores sym.
constexpr uint32_t kEscBit = 1u << 4;
constexpr int kMaxDevices = 64;

// A load through a global (not generic) pointer: generic (flat) loads count in
// two counters, and an outstanding one makes the compiler turn every later
// memory wait into a full one.
template <typename V>
__device__ __forceinline__ V gload(const V *p) {
  return *(const __attribute__((address_space(1))) V *)(p);
}
// The same, not merged with its neighbours (which would make an unaligned wide
// load, and a generic one).
template <typename V>
__device__ __forceinline__ V gload_single(const V *p) {
  return *(const volatile __attribute__((address_space(1))) V *)(p);
}

// A store through a global pointer, for the same reason.
template <typename V>
__device__ __forceinline__ void gstore(V *p, V v) {
  *(__attribute__((address_space(1))) V *)(p) = v;
}

// Integrity flags go to a per-device status word passed to every launch. The
// atomic addresses global memory, not a generic pointer: an outstanding
// generic (flat) access makes the compiler turn every later memory wait into a
// full one.
__device__ __forceinline__ void flag(uint32_t *status, unsigned int f) {
  __hip_atomic_fetch_or((__attribute__((address_space(1))) uint32_t *)(status), f, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
}

// Stream chunk c (32 bits, stream order) of a bitstream of u64 words stored
// little-endian: word w's high half (its first 32 stream bits) is u32 2w+1.
// Past the end the last chunk is re-read instead of zeros, so the load needs no
// branch: a well-formed stream never consumes those bits, and a 7-bit peek that
// runs past its last code selects a table entry whose low bits do not matter.
__device__ __forceinline__ uint32_t chunk_at(const uint32_t *__restrict__ bs32, uint64_t nchunks, uint64_t c) {
  const uint64_t cc = c < nchunks ? c : nchunks - 1;
  return gload(bs32 + (cc ^ 1u));
}

__device__ uint32_t g_zero_chunks[2];

// Decode path of a bucket.
enum : int32_t { kPathBad = 0, kPathGeneric = 1, kPathFast = 2, kPathK1024 = 3 };
// A plan's fast-path item whose 1024 / k_eff row ranges of one bucket run side
// by side, one per k_eff work-items (WorkItem::path bit 4; bits 8..15: rows a range).
constexpr int32_t kMultiRange = 0x10;

struct BucketShape {
  int32_t rows;   // 0 for a bad bucket
  int32_t k_eff;  // lanes with elements
  int32_t path;
};

// Shape and decode path of the bucket with row range [ra, rb) and column
// range [c0, c0 + cl) of tensor T. A range outside the tensor (or more rows
// than the LDS stages) makes the bucket bad. Shared by the plan builder (host)
// and the single-tensor kernel (device).
__host__ __device__ inline BucketShape bucket_shape(int32_t ra, int32_t rb, int32_t c0, int32_t cl,
                                                    const mps_fp8_tensor &T) {
  const bool ok = ra >= 0 && rb >= ra && (int64_t)rb <= T.num_row_indices && rb - ra <= kRowsLds && cl > 0 &&
                  c0 >= 0 && (int64_t)c0 + cl <= T.m;
  BucketShape s;
  s.rows = ok ? rb - ra : 0;
  const int64_t total = (int64_t)s.rows * cl;
  s.k_eff = (int32_t)(T.k < total ? T.k : (total > 0 ? total : 1));
  const uint64_t nm = (uint64_t)T.n * (uint64_t)T.m;
  const bool small_stream = (uint64_t)T.bitstream_words < 0x10000000ull;
  // k = 1024 path (any tensor below 2^31 elements) and the general fast path.
  const bool k1024 = ok && s.rows <= 128 && s.k_eff == 1024 && cl % 1024 == 0 && nm <= (1ull << 31) - 16u &&
                     small_stream;
  const bool fast = !k1024 && ok && s.rows <= 128 && cl % s.k_eff == 0 && nm <= (1ull << 29) && small_stream;
  s.path = !ok ? kPathBad : k1024 ? kPathK1024 : fast ? kPathFast : kPathGeneric;
  return s;
}

// One unit of decode work: a bucket, or a range of its rows. Its tensor,
// column range, shape and the addresses of its per-bucket arrays. Substream
// (lane) t starts at bit bit_base + startbits[t] and ends at bit_base +
// endbits[t]: for a whole bucket, its start bits and the next lane's
// (endbits = startbits + 1); for a row range, the lane checkpoints the plan
// computed at the range's first and next range's first row. A plan builds
// these once (64 bytes: one scalar load per item, which leaves the table ids,
// row indices and start bits one dependent load away); the single-tensor
// kernel builds them on the fly.
struct WorkItem {
  int32_t tensor;       // index into the plan's descriptors
  int32_t c0, cl;       // col_start[b], col_len[b]
  int32_t rows, k_eff;
  int32_t path;                // decode path (bits 0..3); kMultiRange (bit 4): ranges side by side, bits 8..15 their rows
  int64_t bit_base;            // bucket_bit_base[b]
  const int32_t *table_ids;    // bucket_table + 256 b
  const uint32_t *startbits;   // per substream: start bit, relative to bit_base
  const uint32_t *endbits;     // per substream: end bit, relative to bit_base
  const int32_t *row_idx;      // row_indices + row_offsets[b] (+ the range's first row)
};
static_assert(sizeof(WorkItem) == 64, "one scalar load per work item");

// One lane: decode its substream.
//
// Memory discipline (gfx9 counts loads and stores in one in-order vmcnt): all
// global loads of a block of kDepth elements - the block's FP8 bytes and the
// next two bitstream chunks - are issued together one block ahead, and no load
// is issued inside the element loop. The wait at the top of a block is then a
// static vmcnt(kDepth) (the previous block's stores may stay in flight) on
// loads issued a whole block earlier.
//
// Bit supply: a 64-bit MSB-aligned buffer `buf` holding `cnt` bits, topped up
// by 32 bits from a 4-chunk register queue whenever cnt < 32. Without ESC a
// block consumes <= 7*kDepth = 56 bits, i.e. at most two chunks; the two
// chunks staged per block keep the queue at >= 2 chunks at every block start.
// ESC payloads can drain the queue; then a chunk is read directly (slow path).
constexpr int kDepth = 8;

template <typename Idx>
__device__ __forceinline__ void decode_lane(const mps_fp8_tensor &T, uint16_t *__restrict__ out,
                                            const uint32_t *__restrict__ lut,
                                            const int32_t *__restrict__ s_rows, int32_t lane, int32_t k_eff,
                                            int64_t total, int32_t c0, int32_t cl, uint64_t pos0, uint64_t pos_end,
                                            uint32_t *status) {
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;

  // Initial fill: buffer from chunks c0, c0+1; queue = c0+2 .. c0+5; tail = c0+6.
  const uint64_t cb = pos0 >> 5;
  const int skip = (int)(pos0 & 31u);
  uint64_t buf = (((uint64_t)chunk_at(bs32, nchunks, cb) << 32) | chunk_at(bs32, nchunks, cb + 1)) << skip;
  int cnt = 64 - skip;
  uint32_t q0 = chunk_at(bs32, nchunks, cb + 2), q1 = chunk_at(bs32, nchunks, cb + 3);
  uint32_t q2 = chunk_at(bs32, nchunks, cb + 4), q3 = chunk_at(bs32, nchunks, cb + 5);
  int qn = 4;
  uint64_t tail = cb + 6;  // index of the first chunk not yet in buf/queue

  // Element walk e = lane + i*k_eff -> (rr, cc) = (e / cl, e % cl), incrementally.
  int32_t rr = lane / cl;
  int32_t cc = lane - rr * cl;
  const int32_t dr = k_eff / cl;
  const int32_t dc = k_eff - dr * cl;
  const int32_t count = (int32_t)((total - lane + k_eff - 1) / k_eff);
  const int32_t last_row = (int32_t)((total - 1) / cl);
  const Idx m = (Idx)T.m;
  const uint8_t *__restrict__ fp8 = T.fp8;

  // Addresses of the next kDepth elements (elements past `count` repeat the
  // lane's first element, whose address is always valid).
  const Idx first = (Idx)s_rows[rr] * m + (Idx)c0 + (Idx)cc;
  int32_t walked = 0;
  auto next_block = [&](Idx (&idx)[kDepth]) {
    int32_t rrs[kDepth], ccs[kDepth];
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      rrs[j] = rr < last_row ? rr : last_row;
      ccs[j] = cc;
      cc += dc;
      rr += dr;
      if (cc >= cl) {
        cc -= cl;
        rr += 1;
      }
    }
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      const Idx v = (Idx)s_rows[rrs[j]] * m + (Idx)c0 + (Idx)ccs[j];
      idx[j] = (walked + j < count) ? v : first;
    }
    walked += kDepth;
  };

  Idx ia[kDepth], ib[kDepth];
  uint32_t qa[kDepth], qb[kDepth];
  next_block(ia);
#pragma unroll
  for (int j = 0; j < kDepth; ++j) qa[j] = gload(fp8 + ia[j]);
  uint32_t s0 = chunk_at(bs32, nchunks, tail), s1 = chunk_at(bs32, nchunks, tail + 1);
  bool stale = false;  // the staged pair no longer starts at `tail`

  // Each branch merges its own chunk into buf: a loaded value that both
  // branches shared would force a full vmcnt wait on every element.
  auto refill = [&]() {
    if (cnt < 32) {
      if (qn > 0) {
        buf |= (uint64_t)q0 << (32 - cnt);
        q0 = q1;
        q1 = q2;
        q2 = q3;
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
  auto decode_one = [&](uint32_t q, Idx idx) {
    const uint32_t peek = (uint32_t)(buf >> (64 - kL));
    const uint32_t ent = lut[(q << kL) | peek];
    const int len = (int)(ent & 7u);
    buf <<= len;
    cnt -= len;
    uint32_t sym = ent >> 16;
    if (ent & kEscBit) {
      sym = (uint32_t)(buf >> 48);
      buf <<= 16;
      cnt -= 16;
    }
    gstore(out + idx, (uint16_t)sym);
    refill();
  };
  // One block: decode (qc, ic) while (qn_, in_) receive the next block's loads.
  auto block = [&](int32_t i0, uint32_t (&qc)[kDepth], Idx (&ic)[kDepth], uint32_t (&qnx)[kDepth],
                   Idx (&inx)[kDepth]) {
    // Append the pair staged one block ago if it is current and fits.
    if (!stale && qn <= 2) {
      q0 = (qn == 0) ? s0 : q0;
      q1 = (qn == 0) ? s1 : (qn == 1) ? s0 : q1;
      q2 = (qn == 1) ? s1 : (qn == 2) ? s0 : q2;
      q3 = (qn == 2) ? s1 : q3;
      qn += 2;
      tail += 2;
    }
    stale = false;
    next_block(inx);
#pragma unroll
    for (int j = 0; j < kDepth; ++j) qnx[j] = gload(fp8 + inx[j]);
    s0 = chunk_at(bs32, nchunks, tail);
    s1 = chunk_at(bs32, nchunks, tail + 1);
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
  // The next unread bit must be where the next lane's substream begins:
  // buf holds cnt bits and the queue qn chunks, all before chunk `tail`.
  if (tail * 32u - (uint64_t)(cnt + 32 * qn) != pos_end) flag(status, MPS_STATUS_DESYNC);
}

// Buffer resource over [base, base + bytes): raw buffer loads past the end
// return 0 and stores past the end are dropped (gfx9 V# with stride 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// ---------------------------------------------------------------------------
// Fast path: buckets whose column range is a multiple of k_eff and that hold
// at most 128 rows (every bucket of a Llama-shaped tensor with k = 1024).
// Then every lane owns exactly rows * P elements (P = col_len / k_eff), and
// lane t's i-th element sits at row i / P, column c0 + t + (i % P) * k_eff:
// the walk is the same for every lane. It runs in scalar registers and feeds
// the FP8 loads and BF16 stores as the buffer soffset; the per-lane voffset
// is the lane (x2 for BF16).
//
// Bit supply. Each lane keeps the next chunks (32 stream bits) of its
// substream in an 8-deep LDS queue (slot-major: chunk c of lane t at
// [(c % 8) * 1024 + t], so a wave's accesses hit 64 distinct banks). Chunks
// arrive in aligned pairs (one u64 bitstream word): every block of kDepth
// elements each lane requests the next pair if it holds fewer than kAhead
// chunks ahead of its read position, and writes the pair requested kRing
// blocks earlier into the queue. The request is one unconditional
// buffer_load_dwordx2 per block (lanes that do not need a pair read out of
// range and ignore the zeros), so every block issues the same memory
// instructions - 1 bitstream load, kDepth FP8 loads, kDepth stores - and the
// compiler's in-order vmcnt waits stay kRing - 1 blocks deep. A group of kG = 4
// elements decodes from a 32-bit window cut out of two queued chunks (4 codes
// of <= 7 bits). An ESC code (16 raw bits follow) re-reads the window; a
// lane whose queue has run dry reads its two chunks from memory directly.
// ---------------------------------------------------------------------------
constexpr int kG = 4;
#ifndef MPS_DECODE_RING
#define MPS_DECODE_RING 4
#endif
constexpr int kRing = MPS_DECODE_RING;     // blocks in flight: FP8 ring slots and bitstream request slots
constexpr uint32_t kAhead = 7;             // request while fewer chunks than this are queued ahead
constexpr int kQSlots = 8;                 // LDS queue depth (chunks per lane)
constexpr uint32_t kPast = 0x40000000u;    // offset beyond every fast-path buffer (2*n*m <= 2^30)
constexpr uint32_t kBsPast = 0x80000000u;  // bitstream offset beyond every bucket's range
constexpr uint32_t kSlabPast = 0xFFFFFFF0u;  // BF16 byte offset beyond every k = 1024 output (2*n*m < 2^32 - 16)
constexpr int kCacheNT = 2;                  // buffer cache-policy bits: non-temporal (gfx950 NT)
// Cache-policy bits of the slab path's streams (tuning builds only; gfx950
// encodes sc0 = 1, nt = 2, sc1 = 16): the BF16 stores, the FP8 loads and the
// bitstream reserve loads.
#ifndef MPS_SLAB_OUT_CPOL
#define MPS_SLAB_OUT_CPOL kCacheNT
#endif
#ifndef MPS_SLAB_FP8_CPOL
#define MPS_SLAB_FP8_CPOL 0
#endif
#ifndef MPS_SLAB_BS_CPOL
#define MPS_SLAB_BS_CPOL 0
#endif

// LDS: the queue (kQSlots x kBlock u32) at offset 0, then 256 tables x 128 u32
// entries. During set-up the queue region also holds the fp8 -> table map; the
// generic path keeps the bucket's row indices there.
constexpr int kQWords = kQSlots * kBlock;
constexpr int kLutWords = 256 * kTable;
constexpr int kLdsWords = kQWords + kLutWords;

__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

__device__ __forceinline__ void decode_rows_fast(const mps_fp8_tensor &T, uint16_t *out,
                                                 const uint32_t *__restrict__ lut,
                                                 uint32_t *__restrict__ queue, uint32_t qlane, uint32_t lane,
                                                 uint32_t k_eff, uint32_t rows, uint32_t P, uint32_t rowoff_lo,
                                                 uint32_t rowoff_hi, uint64_t bucket_bit,
                                                 uint2 first[3], uint32_t pos, uint32_t pos_end,
                                                 uint32_t *status) {
  // Uniform values computed on the VALU (the division above, selects) would
  // otherwise stay in VGPRs and drag the whole walk, and the buffer offsets it
  // feeds, into vector registers.
  k_eff = uni(k_eff);
  rows = uni(rows);
  P = uni(P);
  bucket_bit = ((uint64_t)uni((uint32_t)(bucket_bit >> 32)) << 32) | uni((uint32_t)bucket_bit);
  const uint32_t nm = (uint32_t)(T.n * T.m);
  const __amdgpu_buffer_rsrc_t r_fp8 = make_rsrc(T.fp8, nm);
  const __amdgpu_buffer_rsrc_t r_out = make_rsrc(out, 2u * nm);
  // Bitstream window of this bucket: from its 64-bit aligned base to the end.
  const uint64_t bs_bytes = T.bitstream_words > 0 ? (uint64_t)T.bitstream_words * 8u : 0u;
  const uint64_t base_byte = bucket_bit >> 3;
  const uint32_t win_bytes = base_byte < bs_bytes ? (uint32_t)(bs_bytes - base_byte) : 0u;
  const __amdgpu_buffer_rsrc_t r_bs =
      make_rsrc(reinterpret_cast<const uint8_t *>(T.bitstream) + (base_byte < bs_bytes ? base_byte : 0), win_bytes);
  // Stream chunk c (relative to the bucket base): u32 at byte (c ^ 1) * 4.
  auto chunk_mem = [&](uint32_t c) -> uint32_t {
    return __builtin_amdgcn_raw_buffer_load_b32(r_bs, (c ^ 1u) << 2, 0, 0);
  };
  auto qidx = [&](uint32_t c) -> uint32_t { return ((c & (kQSlots - 1)) * kBlock) + qlane; };

  // Initial queue: the three pairs loaded during set-up.
  const uint32_t rq0 = (pos >> 5) & ~1u;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    queue[qidx(rq0 + 2 * i)] = first[i].y;      // high half = first chunk of the pair
    queue[qidx(rq0 + 2 * i + 1)] = first[i].x;
  }
  uint32_t rq = rq0 + 6;  // next pair to request
  uint32_t wq = rq0 + 6;  // chunks below wq are (or were) in the queue

  // Uniform element walker: offset (elements) of the next element, then advance.
  const uint32_t count = rows * P;
  auto row_offset = [&](uint32_t r) -> uint32_t {
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)rowoff_lo, (int)(r & 63u));
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)rowoff_hi, (int)(r & 63u));
    return r < 64u ? a : b;
  };
  struct Walker {
    uint32_t r, p, off;
  };
  auto walk = [&](Walker &w) -> uint32_t {
    const uint32_t so = w.r < rows ? w.off : kPast;
    w.off += k_eff;
    if (++w.p == P) {
      w.p = 0;
      ++w.r;
      w.off = row_offset(w.r < rows ? w.r : rows - 1u);
    }
    return so;
  };
  Walker wl{0u, 0u, row_offset(0)}, ws{0u, 0u, row_offset(0)};

  uint32_t qr[kRing][kDepth];  // FP8 bytes, one ring slot per block
  uint2 inflight[kRing];       // requested pairs, one slot per block of the ring
  bool valid[kRing];
#pragma unroll
  for (int s = 0; s < kRing; ++s) valid[s] = false;
#pragma unroll
  for (int b = 0; b < kRing - 1; ++b)
#pragma unroll
    for (int j = 0; j < kDepth; ++j) qr[b][j] = __builtin_amdgcn_raw_buffer_load_b8(r_fp8, lane, walk(wl), 0);
#pragma unroll
  for (int s = 0; s < kRing; ++s) inflight[s] = make_uint2(0u, 0u);

  // Window of the next 32 stream bits at `pos`, from the queue or (if the
  // queue has not got them yet) from memory.
  auto window_at = [&](uint32_t p) -> uint32_t {
    const uint32_t c = p >> 5;
    uint32_t c0 = queue[qidx(c)];
    uint32_t c1 = queue[qidx(c + 1)];
    const bool dry = c + 1u >= wq;
    if (__builtin_amdgcn_ballot_w64(dry)) {
      if (dry) {
        c0 = chunk_mem(c);
        c1 = chunk_mem(c + 1);
        __asm__ volatile("" ::"v"(c0), "v"(c1));  // wait for the loads here, not at a later join
      }
    }
    const uint64_t w = ((uint64_t)c0 << 32) | c1;
    return (uint32_t)(w >> (32u - (p & 31u)));
  };

  auto decode_block = [&](uint32_t (&q)[kDepth], uint32_t nvalid) {
#pragma unroll
    for (int g = 0; g < kDepth; g += kG) {
      uint32_t win = window_at(pos);
#pragma unroll
      for (int j = g; j < g + kG; ++j) {
        if ((uint32_t)j < nvalid) {
          const uint32_t so = walk(ws);
          const uint32_t idx = (q[j] << kL) | (win >> (32 - kL));
          uint32_t ent = lut[idx];
          const uint32_t len = ent & 7u;
          win <<= len;
          pos += len;
          uint32_t sym = ent >> 16;
          if (ent & kEscBit) {
            // ESC: the symbol is the next 16 raw bits.
            sym = window_at(pos) >> 16;
            pos += 16;
            win = window_at(pos);
          }
          __builtin_amdgcn_raw_buffer_store_b16((uint16_t)sym, r_out, 2u * lane, 2u * so, 0);
        }
      }
    }
  };

  auto block = [&](int slot, uint32_t nvalid) {
    const int ps = slot;
    // 1. the pair requested kRing blocks ago joins the queue
    if (valid[ps]) {
      queue[qidx(wq)] = inflight[ps].y;
      queue[qidx(wq + 1)] = inflight[ps].x;
      wq += 2;
    }
    // 2. request the next pair if fewer than kAhead chunks are queued ahead
    const bool need = (int32_t)(rq - (pos >> 5)) < (int32_t)kAhead;
    {
      const uint32_t off = need ? rq * 4u : kBsPast;
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(r_bs, off, 0, 0);
      inflight[ps] = make_uint2(v[0], v[1]);
    }
    valid[ps] = need;
    rq += need ? 2u : 0u;
    // 3. FP8 bytes kRing - 1 blocks ahead
#pragma unroll
    for (int j = 0; j < kDepth; ++j)
      qr[(slot + kRing - 1) % kRing][j] = __builtin_amdgcn_raw_buffer_load_b8(r_fp8, lane, walk(wl), 0);
    // 4. decode this block
    decode_block(qr[slot], nvalid);
  };

  const uint32_t nfull = count / kDepth;
  const uint32_t rem = count % kDepth;
  uint32_t b0 = 0;
  for (; b0 + kRing <= nfull; b0 += kRing) {
#pragma unroll
    for (int slot = 0; slot < kRing; ++slot) block(slot, kDepth);
  }
  // last round: remaining full blocks, then the partial block
#pragma unroll
  for (int slot = 0; slot < kRing; ++slot) {
    const uint32_t bi = b0 + (uint32_t)slot;
    if (bi < nfull) block(slot, kDepth);
    else if (bi == nfull && rem) block(slot, rem);
  }
  if (pos != pos_end) flag(status, MPS_STATUS_DESYNC);
}

// ---------------------------------------------------------------------------
// k = 1024, col_len = P * 1024 (every bucket of a checkpoint written with the
// compress CLI's default of 1024 substreams whose column range is a multiple
// of 1024: every Llama linear has P >= 4).
//
// Element i of a substream lives in slab i: the 1024 columns
// [c0 + 1024 (i % P), +1024) of the bucket's row i / P. Lane l of wave w,
// in 16-lane row R = l / 16 at position v = l % 16, decodes substream
// (column) t = 64w + 4v + R, four elements (one "group", slabs 4g..4g+3) at a
// time. Per group and wave:
//  - FP8: lane (R, v) loads the dword of slab 4g+R at columns 64w+4v..+3, so
//    each 16-lane row reads one contiguous 64-byte segment. A 4x4 byte
//    transpose between the lanes (0, v), (1, v), (2, v), (3, v) (one
//    permlane32 swap, one permlane16 swap and two byte permutes) leaves each
//    lane the four bytes of its own column.
//  - decode: one 32-bit window cut from the lane's LDS bitstream queue covers
//    the group's four codes (<= 7 bits each). The window is never shifted: the
//    7-bit peek of the code that starts o bits in is rotr(window, 23 - o)
//    bits 8..2, which with the FP8 byte << 9 is the code table entry's byte
//    address. The running shift s = 23 - o is decremented by whole entries
//    (their low bits are the length) and only its low 16 bits are kept.
//  - BF16: the inverse transpose (two permlane32 swaps, one permlane16 swap,
//    four byte permutes) gives lane (R, v) slab 4g+R's symbols for columns
//    64w+4v..+3, written with one 8-byte store; each 16-lane row again writes
//    one contiguous 128-byte segment.
// Bitstream: a lane requests up to 64 bytes at a time into a register reserve
// (aligned so that each request touches one half of a 128-byte line) and,
// once per four groups, moves 16 bytes from the reserve into its LDS queue;
// a window whose chunks are not queued is read from memory. FP8 dwords are
// loaded DF groups ahead. Every group issues the same vector-memory
// instructions, so the in-order vmcnt waits stay static.
//
// The queue here stores chunk h in slot (~h) & 7 (slot-major, 4 KiB per
// slot), and positions are kept negated (np = -p, with p biased by two
// chunks: queue chunk h holds stream chunk h - 2 and bit position p is kept
// as p + 64), so the window's slot addresses and its funnel shift come
// straight from np.
//
// ESC (kEsc: the bucket's tables hold ESC entries). An ESC entry's low half is
// 16 + len, so the running shift already steps over the 16 raw bits that
// follow the code; but four codes with ESC payloads can need more than one
// 32-bit window. A lane whose group holds an ESC code (one ballot per group)
// decodes that group again one code at a time, a window per code, taking the
// symbol from the 16 raw bits. ESC codes are rare (the symbols a key's
// 127 most frequent leave out), so the wave almost never takes that branch.
// ---------------------------------------------------------------------------
// kWrap: 0 when P % 4 == 0 (a group's four slabs lie in one row); 1 when P > 4
// and P % 4 != 0 (they may straddle two rows); 2 when P < 4 (they span two to
// four rows: slab i is row i / P, block i % P, taken per lane).
template <int kWrap, bool kEsc, int kShift>
__device__ __forceinline__ void decode_slab4(const mps_fp8_tensor &T, uint16_t *out, const uint32_t *__restrict__ lut,
                                             uint32_t *__restrict__ queue, uint32_t qlane, uint32_t lane,
                                             uint32_t kshift, uint32_t rows, uint32_t P,
                                             uint32_t rowoff_lo, uint32_t rowoff_hi, uint64_t bucket_bit,
                                             const uint2 (&first)[4], uint32_t pos, uint32_t pos_end,
                                             uint32_t *status) {
#ifndef MPS_SLAB_PREFETCH
#define MPS_SLAB_PREFETCH 8
#endif
  constexpr int DF = MPS_SLAB_PREFETCH;  // FP8 prefetch distance (groups)
  static_assert(DF >= 4 && DF % 4 == 0, "the bitstream is served once per four groups");
  rows = uni(rows);
  P = uni(P);
  kshift = kShift ? (uint32_t)kShift : uni(kshift);
  bucket_bit = ((uint64_t)uni((uint32_t)(bucket_bit >> 32)) << 32) | uni((uint32_t)bucket_bit);
  const uint32_t count = rows * P;  // elements per lane
  const uint32_t nfull = count >> 2;
  const uint32_t tail = count & 3u;  // elements of the last, partial group (only when P % 4 != 0)
  const uint32_t gall = nfull + (tail ? 1u : 0u);
  const uint32_t nm = (uint32_t)(T.n * T.m);
  const __amdgpu_buffer_rsrc_t r_fp8 = make_rsrc(T.fp8, nm);
  const __amdgpu_buffer_rsrc_t r_out = make_rsrc(out, 2u * nm);
  const uint64_t bs_bytes = T.bitstream_words > 0 ? (uint64_t)T.bitstream_words * 8u : 0u;
  const uint64_t base_byte = bucket_bit >> 3;
  const uint32_t win_bytes = base_byte < bs_bytes ? (uint32_t)(bs_bytes - base_byte) : 0u;
  const __amdgpu_buffer_rsrc_t r_bs =
      make_rsrc(reinterpret_cast<const uint8_t *>(T.bitstream) + (base_byte < bs_bytes ? base_byte : 0), win_bytes);

  const uint32_t lane4 = qlane << 2;  // the work-item's queue column
  const uint32_t R = (lane >> 4) & 3u;
  const uint32_t colw = (lane & ~63u) | ((lane & 15u) << 2);  // 64w + 4v
  const char *qbytes = reinterpret_cast<const char *>(queue);
  const char *lbytes = reinterpret_cast<const char *>(lut);
  // byte selectors of the FP8 transpose (v_perm: 0-3 pick the second operand's bytes, 4-7 the first's)
  const uint32_t selA = (R & 2u) ? 0x07060302u : 0x05040100u;
  const uint32_t selB = (R & 1u) ? 0x07030501u : 0x06020400u;

  // --- bitstream queue -----------------------------------------------------
  auto chunk_mem = [&](uint32_t h) -> uint32_t {  // biased chunk h from memory (h < 2: out of range, zeros)
    return __builtin_amdgcn_raw_buffer_load_b32(r_bs, ((h - 2u) ^ 1u) << 2, 0, 0);
  };
  // Chunks h (even) and h + 1: slots (~h) & 7 and the one below it.
  auto put_pair = [&](uint32_t h, uint32_t hi, uint32_t lo) {
    uint32_t *slot = queue + (((~h << 10) & 0x1800u) | qlane);
    slot[0] = lo;     // chunk h + 1
    slot[1024] = hi;  // chunk h: the high half of a bitstream word is its first chunk
  };
#ifndef MPS_SLAB_ALIGN
#define MPS_SLAB_ALIGN 1
#endif
#ifndef MPS_SLAB_RESERVE_BLOCKS
#define MPS_SLAB_RESERVE_BLOCKS 4
#endif
  constexpr int RB = MPS_SLAB_RESERVE_BLOCKS;  // 16-byte blocks per bitstream request
  // Byte address of the bucket's bitstream modulo one request (16 * RB bytes):
  // requests after the first start on that boundary, so each one touches a
  // single cache-line half (RB = 4) or line (RB = 8).
  const uint32_t line_phase = (uint32_t)reinterpret_cast<uintptr_t>(T.bitstream) + (uint32_t)(bucket_bit >> 3);
  const uint32_t phase = line_phase & (16u * RB - 1u);
  // The initial queue (written below): the four words read during set-up, or
  // three when the fourth would leave the next request off a 16-byte boundary.
  const uint32_t rq0 = ((pos >> 5) & ~1u) + 2u;
  const uint32_t nfirst = (MPS_SLAB_ALIGN && ((phase + 4u * (rq0 - 2u)) & 15u)) ? 6u : 8u;
  uint32_t wqb = (rq0 + nfirst) << 5;  // 32 x (first chunk not yet written)
  uint32_t rqb = wqb;                  // 32 x (first chunk not yet requested)
  uint32_t np = 0u - (pos + 64u);      // negated biased position

  // 32 stream bits at -npv; from memory for lanes whose queue lacks the two
  // chunks. (Checking once per four groups instead, with an unchecked copy of
  // the groups, measured slower: the extra branch splits the scheduling region.)
  auto window = [&](uint32_t npv) -> uint32_t {
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

  // Register reserve: up to RB 16-byte blocks that follow the queue's last
  // chunk. Every eighth group (MPS_SLAB_REQ_EVERY below), a lane whose reserve
  // is down to one block requests the next RB * 16 bytes (loads from the same
  // lines, so a 128-byte line is fetched about twice instead of once per 16
  // bytes); they land in the reserve four or more groups later, once it is
  // empty. Every fourth group the reserve's front block moves into the queue
  // if four slots are free.
  uint4 rv[RB], inb[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) rv[i] = inb[i] = make_uint4(0u, 0u, 0u, 0u);
  uint32_t rcnt = 0;  // blocks in rv
  bool ifl = false;   // a request is in flight (into inb)
  auto feed = [&]() {
    const bool f = rcnt != 0u && (int32_t)(wqb + np) < 128;
    if (f) {
      const uint32_t h = wqb >> 5;
      put_pair(h, rv[0].y, rv[0].x);
      put_pair(h + 2u, rv[0].w, rv[0].z);
#pragma unroll
      for (int i = 0; i + 1 < RB; ++i) rv[i] = rv[i + 1];
    }
    wqb += f ? 128u : 0u;
    rcnt -= f ? 1u : 0u;
  };
  uint32_t ninb = 0;  // blocks of the request in flight
#ifndef MPS_SLAB_REQ_EVERY
#define MPS_SLAB_REQ_EVERY 2
#endif
#ifndef MPS_SLAB_REQ_AT
#define MPS_SLAB_REQ_AT 1
#endif
  // Requests are considered every MPS_SLAB_REQ_EVERY-th bitstream step, by
  // lanes whose reserve is down to MPS_SLAB_REQ_AT blocks; landing and feeding
  // run every step. Lanes reach the request point on different steps, so a
  // request's four loads carry few active lanes; asking every other step
  // gathers about twice as many into each load and halves their number.
  static_assert(MPS_SLAB_REQ_EVERY >= 1 && (MPS_SLAB_REQ_EVERY & (MPS_SLAB_REQ_EVERY - 1)) == 0,
                "a power of two");
  uint32_t bstep = 0;  // bitstream steps taken (uniform)
  auto land = [&]() {
    const bool l = ifl && rcnt == 0u;
    if (l) {
#pragma unroll
      for (int i = 0; i < RB; ++i) rv[i] = inb[i];
    }
    rcnt = l ? ninb : rcnt;
    ifl = ifl && !l;
  };
  auto reserve = [&]() {
    const uint32_t off = (rqb >> 3) - 8u;
    // no requests past the substream's end (biased end + the window's reach)
    const bool req = !ifl && rcnt <= (uint32_t)MPS_SLAB_REQ_AT && (int32_t)(rqb - (pos_end + 192u)) < 0;
    // blocks up to the next request boundary (the first request may be short)
    const uint32_t nreq = MPS_SLAB_ALIGN ? (16u * RB - ((phase + off) & (16u * RB - 1u))) >> 4 : (uint32_t)RB;
    if (req) {
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r_bs, (uint32_t)i < nreq ? off + 16u * (uint32_t)i : kBsPast,
                                                             0, MPS_SLAB_BS_CPOL);
        inb[i] = make_uint4(v[0], v[1], v[2], v[3]);
      }
      ninb = nreq;
    }
    ifl = ifl || req;
    rqb += req ? nreq << 7 : 0u;
  };
  // Once per four groups: one 16-byte feed covers the 4 x 28 bits they can consume.
  auto bitstream_step = [&]() {
    land();
    if ((bstep & (MPS_SLAB_REQ_EVERY - 1)) == 0u) reserve();
    bstep = uni(bstep + 1u);
    feed();
  };

  // --- group walker ----------------------------------------------------------
  auto row_offset = [&](uint32_t r) -> uint32_t {
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)rowoff_lo, (int)(r & 63u));
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)rowoff_hi, (int)(r & 63u));
    return r < 64u ? a : b;
  };
  uint32_t w_g = 0, w_row = 0, w_blk = 0;
  uint32_t w_off = row_offset(0);
  uint32_t w_next = row_offset(rows > 1u ? 1u : 0u);  // offset of row w_row + 1 (kWrap)
  const uint32_t vf_al = (R << kshift) + colw;       // lane's FP8 byte offset within an aligned group
  // FP8 load of the walker's group; returns the group's BF16 store offset
  // (aligned: the uniform element offset of slab 4g; kWrap: the lane's byte offset).
  auto load_group = [&](uint32_t &F) -> uint32_t {
    uint32_t ret;
    if constexpr (!kWrap) {
      const uint32_t so = uni(w_off + (w_blk << kshift));
      F = __builtin_amdgcn_raw_buffer_load_b32(r_fp8, vf_al, so, MPS_SLAB_FP8_CPOL);
      ret = so;
    } else if constexpr (kWrap == 1) {
      const uint32_t b = w_blk + R;
      const bool wrap = b >= P;
      const bool ok = !wrap || w_row + 1u < rows;
      const uint32_t off = (wrap ? w_next : w_off) + ((wrap ? b - P : b) << kshift) + colw;
      F = __builtin_amdgcn_raw_buffer_load_b32(r_fp8, ok ? off : 0u, 0, MPS_SLAB_FP8_CPOL);
      ret = ok ? off << 1 : kSlabPast;
    } else {
      // P < 4: lane R's slab 4g + R is row w_row + d, block b - d P, where
      // b = w_blk + R < 6 and d = b / P < 4. Slabs past the bucket's last row
      // (a partial last group) load in bounds and store out of range.
      const uint32_t b = w_blk + R;
      const uint32_t d = P == 1u ? b : P == 2u ? (b >> 1) : (b >= 3u ? 1u : 0u);
      const uint32_t o0 = row_offset(w_row), o1 = row_offset(w_row + 1u);
      const uint32_t o2 = row_offset(w_row + 2u), o3 = row_offset(w_row + 3u);
      const bool ok = w_row + d < rows;
      const uint32_t off = (d == 0u ? o0 : d == 1u ? o1 : d == 2u ? o2 : o3) + ((b - d * P) << kshift) + colw;
      F = __builtin_amdgcn_raw_buffer_load_b32(r_fp8, ok ? off : 0u, 0, MPS_SLAB_FP8_CPOL);
      ret = ok ? off << 1 : kSlabPast;
    }
    // advance (branch-free; past the last group the walk stays on it)
    const bool more = w_g + 1u < gall;
    const uint32_t nb = w_blk + 4u;
    if constexpr (kWrap == 2) {
      // four slabs on: P = 1 and 2 move whole rows, P = 3 one or two rows
      const uint32_t dr = P == 1u ? 4u : P == 2u ? 2u : (nb >= 6u ? 2u : 1u);
      w_blk = uni(more ? nb - dr * P : w_blk);
      w_row = uni(w_row + (more ? dr : 0u));
      w_g = uni(w_g + (more ? 1u : 0u));
      return ret;
    }
    const bool wr = nb >= P;
    const uint32_t nrow = w_row + ((more && wr) ? 1u : 0u);
    const uint32_t noff = row_offset(nrow);
    const uint32_t nnext = row_offset(nrow + 1u < rows ? nrow + 1u : nrow);
    // uni(): selects of uniform values may be computed on the VALU, which would
    // pull the walk (and the loads' soffset) into vector registers.
    w_blk = uni(more ? (wr ? nb - P : nb) : w_blk);
    w_off = uni(nrow != w_row ? noff : w_off);
    w_next = uni(nrow != w_row ? nnext : w_next);
    w_row = uni(nrow);
    w_g = uni(w_g + (more ? 1u : 0u));
    return ret;
  };

  // --- one group ---------------------------------------------------------------
  auto group = [&](auto is_tail, uint32_t F, uint32_t so) {
    constexpr bool kTail = decltype(is_tail)::value;
    const auto p1 = __builtin_amdgcn_permlane32_swap(F, F, false, false);
    const uint32_t gq = __builtin_amdgcn_perm(p1[1], p1[0], selA);
    const auto p2 = __builtin_amdgcn_permlane16_swap(gq, gq, false, false);
    const uint32_t fq = __builtin_amdgcn_perm(p2[1], p2[0], selB);  // byte j = element j's FP8 byte
    const uint32_t np0 = np;
    const uint32_t win = window(np);
    uint32_t e[4];
    uint32_t s = 23u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!kTail || (uint32_t)j < tail) {
        const uint32_t qb = (fq >> (8 * j)) & 0xFFu;
        const uint32_t q9 = qb << 9;
        const uint32_t x = __builtin_amdgcn_alignbit(win, win, s);
        e[j] = *reinterpret_cast<const uint32_t *>(lbytes + ((x & 0x1FCu) ^ q9));
        s -= e[j];
      } else {
        e[j] = 0u;
      }
    }
    np += (uint32_t)((int32_t)(s << 16) >> 16) - 23u;  // minus the bits consumed
    if constexpr (kEsc) {
      // The first ESC code of the group is read from the right place, so its
      // flag is seen even when the window does not reach the codes after it.
      const bool esc = ((e[0] | e[1] | e[2] | e[3]) & kEscBit) != 0u;
      if (__builtin_amdgcn_ballot_w64(esc)) {
        if (esc) {
          uint32_t p = np0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (!kTail || (uint32_t)j < tail) {
              const uint32_t qb = (fq >> (8 * j)) & 0xFFu;
              const uint32_t q9 = qb << 9;
              const uint32_t w = window(p);
              uint32_t ent = *reinterpret_cast<const uint32_t *>(lbytes + (((w >> 23) & 0x1FCu) ^ q9));
              p -= ent & 7u;
              if (ent & kEscBit) {
                ent = window(p) & 0xFFFF0000u;  // the symbol: the 16 raw bits after the code
                p -= 16u;
              }
              e[j] = ent;
            }
          }
          np = p;
        }
      }
    }
    const auto t0 = __builtin_amdgcn_permlane32_swap(e[0], e[2], false, false);
    const auto t1 = __builtin_amdgcn_permlane32_swap(e[1], e[3], false, false);
    const uint32_t a = __builtin_amdgcn_perm(t0[1], t0[0], 0x07060302u);
    const uint32_t b = __builtin_amdgcn_perm(t1[1], t1[0], 0x07060302u);
    const auto t2 = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    const v2u o = {__builtin_amdgcn_perm(t2[1], t2[0], 0x05040100u), __builtin_amdgcn_perm(t2[1], t2[0], 0x07060302u)};
    // Non-temporal: the output is written once, and L2 is better spent on the
    // lanes' bitstream lines and the FP8 lines that wave pairs share.
    if constexpr (!kWrap) __builtin_amdgcn_raw_buffer_store_b64(o, r_out, vf_al << 1, uni(so) << 1, MPS_SLAB_OUT_CPOL);
    else __builtin_amdgcn_raw_buffer_store_b64(o, r_out, so, 0, MPS_SLAB_OUT_CPOL);
  };

  uint32_t Fr[DF], SOr[DF];
#pragma unroll
  for (int u = 0; u < DF; ++u) SOr[u] = load_group(Fr[u]);
  // The initial queue, written once the first FP8 loads are in flight: the
  // wait for the set-up's bitstream words overlaps them.
#pragma unroll
  for (int i = 0; i < 3; ++i) put_pair(rq0 + 2 * i, first[i].y, first[i].x);
  if (nfirst == 8u) put_pair(rq0 + 6u, first[3].y, first[3].x);
  // Every wave of the workgroup decodes the same number of groups, but the
  // issue arbiter favours the oldest ready wave (waves 4r..4r+3 are the r-th
  // oldest on their SIMDs): left alone, the oldest waves finish first and the
  // bucket ends with a few young waves and little latency hiding. So a wave
  // lowers its priority by one level per quarter of its groups, counted from
  // a head start that grows with its age: older waves yield issue slots to
  // younger ones, and a wave that is ahead to the ones behind.
#ifndef MPS_PRIO_LEAD
#define MPS_PRIO_LEAD 8
#endif
  const uint32_t quarter = uni(nfull / 4u > 0u ? nfull / 4u : 1u);
  const uint32_t lead = (3u - (uni(qlane) >> 8)) * (quarter * MPS_PRIO_LEAD / 16u);  // head start (groups)
  uint32_t prio = 3u - (lead / quarter < 3u ? lead / quarter : 3u);
  uint32_t prio_at = (lead / quarter + 1u) * quarter - lead;  // groups done when the priority next drops
  if (prio == 3u) __builtin_amdgcn_s_setprio(3);
  else if (prio == 2u) __builtin_amdgcn_s_setprio(2);
  else if (prio == 1u) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
  uint32_t g = 0;
  for (; g + (uint32_t)DF <= nfull; g += (uint32_t)DF) {
    if (g >= prio_at) {
      prio_at += quarter;
      --prio;
      if (prio == 2u) __builtin_amdgcn_s_setprio(2);
      else if (prio == 1u) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
#pragma unroll
    for (int u = 0; u < DF; ++u) {
      if (u % 4 == 0) bitstream_step();
      const uint32_t F = Fr[u], so = SOr[u];
      SOr[u] = load_group(Fr[u]);  // the group DF ahead
      group(std::false_type{}, F, so);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // the last (fewer than DF) full groups and the partial one; their FP8 is already loaded
#pragma unroll
  for (int u = 0; u < DF; ++u) {
    if (g + (uint32_t)u < gall) {
      if (u % 4 == 0) bitstream_step();
      if (g + (uint32_t)u < nfull) group(std::false_type{}, Fr[u], SOr[u]);
      else group(std::true_type{}, Fr[u], SOr[u]);
    }
  }
  if (0u - np - 64u != pos_end) flag(status, MPS_STATUS_DESYNC);
}

// The work item of bucket b of tensor T (the single-tensor kernel).
__device__ __forceinline__ WorkItem bucket_item(const mps_fp8_tensor &T, int64_t b) {
  WorkItem w;
  w.tensor = 0;
  const int32_t ra = T.bucket_row_offsets[b];
  const int32_t rb = T.bucket_row_offsets[b + 1];
  w.c0 = T.bucket_col_start[b];
  w.cl = T.bucket_col_len[b];
  const BucketShape s = bucket_shape(ra, rb, w.c0, w.cl, T);
  w.rows = s.rows;
  w.k_eff = s.k_eff;
  w.path = s.path;
  w.bit_base = T.bucket_bit_base[b];
  w.table_ids = T.bucket_table + b * 256;
  w.startbits = T.bucket_thread_startbit + b * (T.k + 1);
  w.endbits = w.startbits + 1;
  w.row_idx = T.row_indices + (s.path != kPathBad ? ra : 0);
  return w;
}

// Item trace, in instrumented builds only (python -m mpserve_amd.build --define
// MPS_TRACE_ITEMS=1 --out LIB; mpserve_amd.item_trace reads it). decode_bucket
// then also notes the real-time clock after its set-up's last barrier.
#ifndef MPS_TRACE_ITEMS
#define MPS_TRACE_ITEMS 0
#endif
#if MPS_TRACE_ITEMS
#define MPS_TR_PARAM , uint64_t (&tr)[4]
#define MPS_TR_ARG , tr
#else
#define MPS_TR_PARAM
#define MPS_TR_ARG
#endif

// kQueue: the work item also takes the ticket of the workgroup's next one
// from the launch's work counter (queue[0]), at the start of its set-up, so
// that the atomic's round trip overlaps the set-up's loads; every thread
// gets it in `ticket` (zero without kQueue).
// kSlabK: fast-path buckets with k_eff 256 or 512 take the slab path (else the
// scalar element walk). Only launches whose tensors have such
// k compile it in: the extra slab instances cost the k = 1024 launches 1.5%
// (registers), though their own code is unchanged.
template <bool kQueue, bool kSlabK>
__device__ __forceinline__ void decode_bucket(const mps_fp8_tensor &T, uint16_t *out, const WorkItem &w,
                                              uint32_t *lds, uint32_t *status, uint32_t *queue,
                                              uint32_t &ticket, int32_t wg_part, int32_t wg_parts MPS_TR_PARAM) {
  uint32_t *qregion = lds;
  uint32_t *lut = lds + kQWords;
  int32_t *s_rows = reinterpret_cast<int32_t *>(qregion) + 6 * kBlock;    // queue slot 6 (generic path)
  uint32_t *s_wflag = qregion + 5 * kBlock;                             // queue slot 5: the waves' flag words
  // The work-item id through an opaque move: the per-lane constants of every
  // decode path derive from it, and hoisted out of the bucket loop they would
  // all stay live across the set-up, which then runs out of VGPRs.
  int tid;
  __asm__ volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));

  const int32_t path = w.path & 0xF;
  const int32_t c0 = w.c0, cl = w.cl, k_eff = w.k_eff;
  const bool bucket_ok = path != kPathBad;
  const bool k1024 = path == kPathK1024;
  const bool fast = path == kPathFast;
  // A multi-range item (fast path, k_eff 256 or 512): work-items
  // [sub * k_eff, (sub + 1) * k_eff) decode its sub-th range, whose rows,
  // start bits and end bits follow the previous range's (uniform per wave).
  const bool multi = (w.path & kMultiRange) != 0;
  const int32_t mrr = (w.path >> 8) & 0xFF;
  const int32_t sub = multi ? (int32_t)uni((uint32_t)(tid >> (k_eff == 256 ? 8 : 9))) : 0;
  const int32_t rows = multi ? max(0, min(mrr, w.rows - sub * mrr)) : w.rows;
  const int64_t total = (int64_t)rows * cl;
  const uint64_t nm = (uint64_t)T.n * (uint64_t)T.m;
  const int lane = multi ? (tid & (k_eff - 1)) : tid;  // the lane's substream (work-item within its range)
  // Substream of this work-item: the k = 1024 paths give wave w's 16-lane row
  // R, position v the column 64w + 4v + R (see decode_slab4); the others, the lane.
  // A fast-path bucket with k_eff 256 or 512 takes the slab path too (kSlabK).
  const bool slab = kSlabK && fast && (k_eff == 256 || k_eff == 512);
  const int col = k1024 ? ((tid & ~63) | ((tid & 15) << 2) | ((tid >> 4) & 3))
                  : slab ? ((lane & ~63) | ((lane & 15) << 2) | ((lane >> 4) & 3)) : lane;
  const bool active = bucket_ok && rows > 0 && lane < k_eff;
  const uint32_t *sb = w.startbits + (int64_t)sub * k_eff;
  const uint32_t *eb = w.endbits + (int64_t)sub * k_eff;
  const int32_t *row_idx = w.row_idx + (int64_t)sub * mrr;
  const uint64_t base = (uint64_t)w.bit_base;

  // Set-up: two levels of loads, each issued in full before any of its
  // results is used. (1) From the work record alone: the table ids, the row
  // indices (fast paths) and the lane's start bits. (2) From those: the
  // tables' contents and the lane's first bitstream words. They are buffer
  // loads, whose lanes out of range read zeros, so that none sits behind a
  // branch: a load under a branch is waited for where the branch joins.
  //
  // Thread tid expands the 16-byte slice tid % 16 of the tables of FP8 bytes
  // tid / 16 + 64 i (i < 4); 16 threads read each id.
  constexpr int kSlices = 256 * (kTable / 8) / kBlock;  // 4
  const bool rows_fast = k1024 || fast;
  const int wl = lane & 63;
  // The ticket: a buffer atomic that only thread 0 addresses in range (the
  // others' are dropped), so no branch holds the set-up's loads behind it.
  uint32_t tk = 0;
  if (kQueue) {
    const __amdgpu_buffer_rsrc_t r_q = make_rsrc(queue, 4u);
    tk = (uint32_t)__builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(1, r_q, tid == 0 ? 0u : kBsPast, 0, 0);
    tk = tid == 0 ? tk : 0u;
  }
  const __amdgpu_buffer_rsrc_t r_ids = make_rsrc(w.table_ids, 256u * 4u);
  const __amdgpu_buffer_rsrc_t r_rows = make_rsrc(row_idx, rows_fast ? (uint32_t)rows * 4u : 0u);
  const __amdgpu_buffer_rsrc_t r_sb = make_rsrc(sb, rows_fast ? (uint32_t)k_eff * 4u : 0u);
  const __amdgpu_buffer_rsrc_t r_eb = make_rsrc(eb, rows_fast ? (uint32_t)k_eff * 4u : 0u);
  int32_t gids[kSlices];
#pragma unroll
  for (int i = 0; i < kSlices; ++i)
    gids[i] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_ids, (uint32_t)((tid >> 4) + 64 * i) * 4u, 0, 0);
  const int32_t r_lo = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_rows, (uint32_t)wl * 4u, 0, 0);
  const int32_t r_hi = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r_rows, (uint32_t)(wl + 64) * 4u, 0, 0);
  const uint32_t sb_off = active ? (uint32_t)col * 4u : kBsPast;
  uint32_t pos = __builtin_amdgcn_raw_buffer_load_b32(r_sb, sb_off, 0, 0);
  uint32_t pos_end = __builtin_amdgcn_raw_buffer_load_b32(r_eb, sb_off, 0, 0);

#if MPS_TRACE_ITEMS
  const uint64_t tr_start = __builtin_amdgcn_s_memrealtime();
  __asm__ volatile("" ::"v"(gids[0]), "v"(gids[3]), "v"(r_lo), "v"(r_hi), "v"(pos), "v"(pos_end));
  const uint64_t tr_l1 = __builtin_amdgcn_s_memrealtime();
#endif
  bool bad_table = false;
#pragma unroll
  for (int i = 0; i < kSlices; ++i) {
    if (gids[i] < -1 || gids[i] >= T.num_tables) {
      bad_table = true;
      gids[i] = -1;
    }
  }
  // Row offsets: the fast paths keep rows 0..63 / 64..127 one per lane in
  // VGPRs (selects, not a branch, so the loads above are not sunk into one).
  const bool has_lo = rows_fast && wl < rows, has_hi = rows_fast && wl + 64 < rows;
  bool bad_row = (has_lo && (r_lo < 0 || r_lo >= T.n)) | (has_hi && (r_hi < 0 || r_hi >= T.n));
  const uint32_t rowoff_lo = has_lo ? (uint32_t)r_lo * (uint32_t)T.m + (uint32_t)c0 : 0u;
  const uint32_t rowoff_hi = has_hi ? (uint32_t)r_hi * (uint32_t)T.m + (uint32_t)c0 : 0u;
  // Offset of the lane's first bitstream words (loaded after the table
  // expansion), computed here: the wait for `pos` then falls before the table
  // loads are issued, not at the join of their two paths.
  uint32_t off0 = active ? ((pos >> 5) & ~1u) * 4u : kBsPast;
  __asm__ volatile("" : "+v"(off0));
  // Likewise the descriptor's bitstream fields (scalar loads).
  const uint8_t *bs_ptr = reinterpret_cast<const uint8_t *>(T.bitstream);
  int64_t bs_words = T.bitstream_words;
  __asm__ volatile("" : "+s"(bs_ptr), "+s"(bs_words));
  // The tables' contents (buffer loads when their byte offsets fit 31 bits).
  uint4 sv[kSlices];
  uint32_t nibs[kSlices];
  const int part = tid & 15;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(T.decode_syms) & 15u) == 0) &&
                      ((reinterpret_cast<uintptr_t>(T.decode_lens) & 3u) == 0);
  const bool tab_buffer = vec_ok && T.num_tables <= (1 << 22);
  if (tab_buffer) {
    const uint32_t ntab = (uint32_t)T.num_tables;
    const __amdgpu_buffer_rsrc_t r_syms = make_rsrc(T.decode_syms, ntab * (uint32_t)(kTable * 2));
    const __amdgpu_buffer_rsrc_t r_lens = make_rsrc(T.decode_lens, ntab * (uint32_t)kPacked);
#pragma unroll
    for (int i = 0; i < kSlices; ++i) {
      const bool has = gids[i] >= 0;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(
          r_syms, has ? (uint32_t)gids[i] * (uint32_t)(kTable * 2) + (uint32_t)part * 16u : 0x80000000u, 0, 0);
      sv[i] = make_uint4(v[0], v[1], v[2], v[3]);
      nibs[i] = __builtin_amdgcn_raw_buffer_load_b32(
          r_lens, has ? (uint32_t)gids[i] * (uint32_t)kPacked + (uint32_t)part * 4u : 0x80000000u, 0, 0);
    }
  }
  if (bad_table) flag(status, MPS_STATUS_BAD_TABLE);
  // The two fallbacks below load through global pointers (gload), so that the
  // waits after their join stay partial and the first bitstream words' loads
  // below can still be in flight during the expansion.
  if (!rows_fast) {
    for (int i = tid; i < rows; i += kBlock) {
      const int32_t r = gload(w.row_idx + i);
      bad_row |= r < 0 || r >= T.n;
      s_rows[i] = r;
    }
  }
#pragma unroll
  for (int i = 0; i < kSlices && !tab_buffer; ++i) {
    const int32_t g = gids[i];
    sv[i] = make_uint4(0u, 0u, 0u, 0u);
    nibs[i] = 0;
    if (g >= 0) {
      const uint16_t *sp = T.decode_syms + (int64_t)g * kTable + part * 8;
      const uint8_t *lp = T.decode_lens + (int64_t)g * kPacked + part * 4;
      if (vec_ok) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = gload(reinterpret_cast<const u32x4 *>(sp));
        sv[i] = make_uint4(v[0], v[1], v[2], v[3]);
        nibs[i] = gload(reinterpret_cast<const uint32_t *>(lp));
      } else {
        uint32_t h[8], b[4];
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = gload_single(sp + j);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = gload_single(lp + j);
        sv[i] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        nibs[i] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      }
    }
  }

#if MPS_TRACE_ITEMS
  __asm__ volatile("" ::"v"(sv[0].x), "v"(sv[3].w), "v"(nibs[0]), "v"(nibs[3]));
  const uint64_t tr_l2 = __builtin_amdgcn_s_memrealtime();
  tr[1] = ((tr_l1 - tr_start) & 0xFFFFFFFFull) | ((tr_l2 - tr_start) << 32);
  if ((tid & 63) == 0) s_wflag[32 + (tid >> 6)] = (uint32_t)(tr_l2 - tr_start);
#endif
  uint32_t esc_seen = 0;
#pragma unroll
  for (int i = 0; i < kSlices; ++i) {
    esc_seen |= nibs[i] & 0x88888888u;
    // Entry j = sym_j << 16 | (nib_j & 7) | (nib_j & 8 ? 16 : 0). The nibbles go
    // to bytes (even entries in `fl`, odd ones in `fh`), where nib + (nib & 8)
    // is the entry's low byte; one byte permute per entry then joins it with
    // the symbol (the high or low half of sv: entries 2c and 2c + 1 share word c).
    const uint32_t lo = nibs[i] & 0x0F0F0F0Fu, hi = (nibs[i] >> 4) & 0x0F0F0F0Fu;
    const uint32_t fl = lo + (lo & 0x08080808u), fh = hi + (hi & 0x08080808u);
    const uint32_t w4[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
    uint32_t e[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      e[2 * c] = __builtin_amdgcn_perm(w4[c], fl, 0x05040C00u | (uint32_t)c);      // [fl byte c, 0, sym lo]
      e[2 * c + 1] = __builtin_amdgcn_perm(w4[c], fh, 0x07060C00u | (uint32_t)c);  // [fh byte c, 0, sym hi]
    }
    const uint32_t qt = (uint32_t)((tid >> 4) + 64 * i);  // the table's FP8 byte
    uint32_t *tab = lut + qt * kTable;
    *reinterpret_cast<uint4 *>(tab + (uint32_t)part * 8u) = make_uint4(e[0], e[1], e[2], e[3]);
    *reinterpret_cast<uint4 *>(tab + (uint32_t)part * 8u + 4u) = make_uint4(e[4], e[5], e[6], e[7]);
  }
#if MPS_TRACE_ITEMS
  const uint64_t tr_exp = __builtin_amdgcn_s_memrealtime();
#endif
  // First four bitstream words of this lane (two 16-byte loads); the slab
  // path queues all four, the others three. A lane's words are scattered (64
  // lines a wave), and the CU's memory path takes its waves' loads in order:
  // issued with the table loads they held back the later waves' tables (and so
  // the barrier below); issued at the decode's start, their round trip added
  // to it. Issued here, once the wave's own tables are in LDS, they overlap
  // the other waves' expansion and the two barriers; the decode waits for them
  // after issuing its first FP8 loads.
  __builtin_amdgcn_sched_barrier(0);
  uint2 first[4];
  {
    const uint64_t bs_bytes = bs_words > 0 ? (uint64_t)bs_words * 8u : 0u;
    const uint64_t base_byte = base >> 3;
    const uint32_t win_bytes = rows_fast && base_byte < bs_bytes ? (uint32_t)(bs_bytes - base_byte) : 0u;
    const __amdgpu_buffer_rsrc_t r_bs = make_rsrc(bs_ptr + (base_byte < bs_bytes ? base_byte : 0), win_bytes);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r_bs, off0 + 16u * (uint32_t)i, 0, 0);
      first[2 * i] = make_uint2(v[0], v[1]);
      first[2 * i + 1] = make_uint2(v[2], v[3]);
    }
  }
  // Block-wide ORs of "a row index is out of range" (bit 0) and "a table has an
  // ESC entry" (bit 1): one word per wave; wave 0's also carries the ticket
  // (bits 2..31). Every wave gets its own copy of the 16 words, in its own
  // queue columns: wave w's lane i writes the word to column 64 i + w, and wave
  // i reads columns 64 i .. 64 i + 15. Only wave i writes those columns later
  // (its queue), after reading them, so no second barrier has to keep a fast
  // wave's queue from overwriting words a slower wave has not read yet.
  {
    const uint32_t wf = (__builtin_amdgcn_ballot_w64(bad_row) ? 1u : 0u) |
                        (__builtin_amdgcn_ballot_w64(esc_seen != 0) ? 2u : 0u) | (uni(tk) << 2);
    if ((tid & 63) < kBlock / 64) s_wflag[((tid & 63) << 6) | (tid >> 6)] = wf;
  }
  __syncthreads();
#if MPS_TRACE_ITEMS
  const uint64_t tr_b1 = __builtin_amdgcn_s_memrealtime();
  uint32_t tr_l2max = 0;
  for (int w = 0; w < kBlock / 64; ++w) tr_l2max = max(tr_l2max, s_wflag[32 + w]);
  tr[2] = ((tr_exp - tr_start) & 0xFFFFFFFFull) | ((tr_b1 - tr_start) << 32);
  tr[3] = tr_l2max;
#endif
  uint32_t bflags = 0;
  {
    const uint32_t *mine = s_wflag + (uni((uint32_t)tid) & ~63u);  // this wave's copy
#pragma unroll
    for (int w = 0; w < kBlock / 64; w += 4) {
      const uint4 f = *reinterpret_cast<const uint4 *>(mine + w);
      bflags |= f.x | f.y | f.z | f.w;
    }
  }
  bflags = uni(bflags);
  ticket = bflags >> 2;
  const bool has_esc = (bflags & 2u) != 0;
  const bool any_bad_row = (bflags & 1u) != 0;
#if MPS_TRACE_ITEMS
  tr[0] = __builtin_amdgcn_s_memrealtime();
#endif

  if (!bucket_ok || any_bad_row) {
    if (tid == 0) flag(status, !bucket_ok ? MPS_STATUS_BAD_BUCKET : MPS_STATUS_BAD_ROW);
    return;
  }
  if (!active) return;
  // A bucket shared by `wg_parts` workgroups (the single-tensor kernel, few
  // buckets for the CUs): every one expands the tables; on the k = 1024 paths
  // workgroup `wg_part` then decodes the substreams of waves
  // [16 wg_part / wg_parts, 16 (wg_part + 1) / wg_parts), on the others part 0 decodes all.
  if (wg_parts > 1) {
    const int32_t wv = (int32_t)(uni((uint32_t)tid) >> 6);
    if (k1024 ? (wv * wg_parts / (kBlock / 64) != wg_part) : (wg_part != 0)) return;
  }
  if (k1024) {
    const uint32_t P = (uint32_t)cl / 1024u;
    if (P >= 4) {
#define MPS_SLAB(WRAP, ESC)                                                                               \
  decode_slab4<WRAP, ESC, 10>(T, out, lut, qregion, (uint32_t)lane, (uint32_t)lane, 10u, (uint32_t)rows, P, \
                              rowoff_lo, rowoff_hi, base, first, pos, pos_end, status)
      if (P % 4 == 0) {
        if (has_esc) MPS_SLAB(0, true);
        else MPS_SLAB(0, false);
      } else {
        if (has_esc) MPS_SLAB(1, true);
        else MPS_SLAB(1, false);
      }
      return;
    }
    // P < 4: the same path, with groups that span two to four rows
    if (has_esc) MPS_SLAB(2, true);
    else MPS_SLAB(2, false);
#undef MPS_SLAB
  } else if (kSlabK && slab) {
    // k_eff 256 / 512 (col_len % k_eff == 0 on the fast path): work-item tid
    // decodes substream `col` of its range, over slabs of k_eff columns
    const uint32_t ks = k_eff == 512 ? 9u : 8u;
    const uint32_t P = (uint32_t)cl >> ks;
#define MPS_SLABK(WRAP, ESC)                                                                                   \
  decode_slab4<WRAP, ESC, 0>(T, out, lut, qregion, (uint32_t)tid, (uint32_t)lane, ks, (uint32_t)rows, P, rowoff_lo, \
                             rowoff_hi, base, first, pos, pos_end, status)
    if (P % 4 == 0) {
      if (has_esc) MPS_SLABK(0, true);
      else MPS_SLABK(0, false);
    } else if (P > 4) {
      if (has_esc) MPS_SLABK(1, true);
      else MPS_SLABK(1, false);
    } else {
      if (has_esc) MPS_SLABK(2, true);
      else MPS_SLABK(2, false);
    }
#undef MPS_SLABK
  } else if (fast) {
    decode_rows_fast(T, out, lut, qregion, (uint32_t)tid, (uint32_t)lane, (uint32_t)k_eff, (uint32_t)rows,
                     (uint32_t)(cl / k_eff), rowoff_lo, rowoff_hi, base, first, pos, pos_end, status);
  } else {
    const uint64_t pos0 = base + gload(sb + lane);
    const uint64_t pend = base + gload(w.endbits + lane);
    if (nm <= 0xFFFFFFFFull)
      decode_lane<uint32_t>(T, out, lut, s_rows, lane, k_eff, total, c0, cl, pos0, pend, status);
    else
      decode_lane<uint64_t>(T, out, lut, s_rows, lane, k_eff, total, c0, cl, pos0, pend, status);
  }
}

// End of a bucket: drain the wave's memory counters (its last stores and the
// FP8 and bitstream prefetches past its substream's end) before the barrier,
// where the wait overlaps the other waves' last groups. The next set-up then
// starts with nothing outstanding, and none of its loads waits behind these.
__device__ __forceinline__ void end_bucket() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // the next bucket's set-up overwrites the LDS
}

// Both kernels are persistent: one workgroup per CU (the LDS holds one
// bucket's tables) walks its share of the buckets, so a bucket's set-up does
// not also pay a workgroup launch. fp8_decode_one deals the buckets
// round-robin; every workgroup runs the same uniform loop to its end.
template <bool kSlabK>
//
// parts > 1 (k = 1024 tensors with fewer buckets than CUs): the grid is
// buckets x parts, and workgroup g decodes part g % parts of bucket g / parts
// (decode_bucket), so that a tensor of 8 buckets runs on 128 CUs instead of 8.
// A bucket's substreams are sequential chains, which only lane checkpoints (a
// plan's) cut into row ranges; fewer waves a CU run each chain faster.
__global__ __launch_bounds__(kBlock) void fp8_decode_one(mps_fp8_tensor T, uint32_t *status, int32_t parts) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
  uint32_t ticket;
#if MPS_TRACE_ITEMS
  uint64_t tr[4];
#endif
  if (parts > 1) {
    const int64_t b = (int64_t)blockIdx.x / parts;
    if (b < T.num_buckets)
      decode_bucket<false, kSlabK>(T, T.out, bucket_item(T, b), lds, status, nullptr, ticket,
                                   (int32_t)(blockIdx.x % parts), parts MPS_TR_ARG);
    return;
  }
  for (int64_t b = blockIdx.x; b < T.num_buckets; b += gridDim.x) {
    decode_bucket<false, kSlabK>(T, T.out, bucket_item(T, b), lds, status, nullptr, ticket, 0, 1 MPS_TR_ARG);
    end_bucket();
  }
}

// fp8_decode_plan takes its work items from a queue: workgroup g starts with
// item g; each item takes a ticket t from queue[0] (in its set-up, or with
// kEndTicket as it ends), and the workgroup's next item is gridDim.x + t. The items are sorted largest first,
// so the CUs that drew small items or ran fast take more of them, and all
// finish close together (a fixed deal would leave the CUs with the larger
// shares running alone at the end). The last workgroup to leave (queue[1]
// counts them) puts both words back to zero for the next launch: launches of
// one queue must not overlap.
//
// out_delta: elements every tensor's output moves by (a plan decoding into a
// buffer laid out like, but other than, the one it was created with).
//
// Tickets travel in 30 bits of the set-up's flag words: a launch holds fewer
// than kMaxQueueItems work items.
constexpr int64_t kMaxQueueItems = (int64_t(1) << 30) - 65536;

// The item trace (instrumented builds): workgroup g < kTraceWgs records its
// first kTraceItems items, kTraceWords words each: the real-time clock (100 MHz) at the
// item's start and after its end barrier, the item's path << 40 | rows << 20 |
// k_eff, its col_len, the clock after the set-up's last barrier, the clock
// when waves 0 and 15 finished their decode (before the end drain), and wave
// 0's ticks from its set-up start: to its level-1 loads' return (word 7 low
// half), its tables' return (word 7 high half), the end of its table expansion
// (word 8 low half), the set-up's first barrier (word 8 high half) and the
// last wave's tables (word 9). Threads 0 and 960 write them with ordinary
// stores after the barrier; words 10 and 11 are spare.
#if MPS_TRACE_ITEMS
constexpr int kTraceWgs = 256, kTraceItems = 128, kTraceWords = 12;
__device__ uint64_t g_item_trace[kTraceWgs * kTraceItems * kTraceWords];
#endif

template <bool kSlabK, bool kEndTicket>
__global__ __launch_bounds__(kBlock) void fp8_decode_plan(const mps_fp8_tensor *__restrict__ tensors,
                                                          const WorkItem *__restrict__ work, int64_t nwork,
                                                          uint32_t *status, int64_t out_delta, uint32_t *queue) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
  if ((int64_t)blockIdx.x < nwork) {
    WorkItem w = work[blockIdx.x];
#if MPS_TRACE_ITEMS
    int tr_it = 0;
#endif
    for (;;) {
      uint32_t ticket;
#if MPS_TRACE_ITEMS
      const uint64_t tr0 = __builtin_amdgcn_s_memrealtime();
      uint64_t tr[4] = {0, 0, 0, 0};
#endif
      const mps_fp8_tensor &T = tensors[w.tensor];
      decode_bucket<!kEndTicket, kSlabK>(T, T.out + out_delta, w, lds, status, queue, ticket, 0, 1 MPS_TR_ARG);
#if MPS_TRACE_ITEMS
      const uint64_t tr_wave = __builtin_amdgcn_s_memrealtime();
#endif
      if constexpr (kEndTicket) {
        // The ticket is taken once wave 0 is through with the item, so the
        // next item goes to a workgroup that is about to be free; thread 0
        // hands it out through the LDS once every wave is done with the
        // item's queue, and every wave reads it before the next set-up.
        uint32_t tq = 0;
        if (threadIdx.x == 0)
          tq = __hip_atomic_fetch_add((__attribute__((address_space(1))) uint32_t *)(queue), 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
        end_bucket();
        if (threadIdx.x == 0) lds[0] = tq;
        __syncthreads();
        ticket = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds[0]);
        __syncthreads();
      }
      const int64_t next = (int64_t)gridDim.x + ticket;
      // The next record (scalar registers); with the set-up's ticket it is
      // loaded before the drain of this item's stores, which covers its round trip.
      const WorkItem wn = work[next < nwork ? next : 0];
      if constexpr (!kEndTicket) end_bucket();
#if MPS_TRACE_ITEMS
      if (blockIdx.x < kTraceWgs && tr_it < kTraceItems) {
        uint64_t *tp = g_item_trace + ((size_t)blockIdx.x * kTraceItems + tr_it) * kTraceWords;
        if (threadIdx.x == 0) {
          tp[0] = tr0;
          tp[1] = __builtin_amdgcn_s_memrealtime();
          tp[2] = ((uint64_t)(uint32_t)w.path << 40) | ((uint64_t)(uint32_t)w.rows << 20) | (uint64_t)(uint32_t)w.k_eff;
          tp[3] = (uint64_t)(uint32_t)w.cl;
          tp[4] = tr[0];
          tp[5] = tr_wave;
          tp[7] = tr[1];
          tp[8] = tr[2];
          tp[9] = tr[3];
        } else if (threadIdx.x == 960) {
          tp[6] = tr_wave;
        }
      }
      ++tr_it;
#endif
      if (next >= nwork) break;
      w = wn;
    }
  }
  if (threadIdx.x == 0) {
    if (atomicAdd(queue + 1, 1u) == gridDim.x - 1) {
      atomicExch(queue, 0u);
      atomicExch(queue + 1, 0u);
    }
  }
}

// ---------------------------------------------------------------------------
// Lane checkpoints: where each substream of a bucket stands at the first row
// of each of its row ranges, so that a plan can decode the ranges as separate
// work items (more work items than buckets when a plan has few).
//
// One workgroup per bucket to split (k = 1024 and fast paths: substream t's
// i-th element is row i / P, column c0 + t + (i % P) * K). Thread t walks
// substream t through the code lengths only: the FP8 byte picks the table,
// the next 7 bits pick the length nibble, an ESC code skips 16 more bits (the
// lossless decode's semantics). It records its position after each range's
// last element. Row indices and table ids out of range stop the walk and mark
// the job failed (the plan then keeps the bucket whole, and its decode
// reports them).
// ---------------------------------------------------------------------------
struct SplitJob {
  int32_t tensor;
  int32_t K;           // substreams (k_eff)
  int32_t P;           // col_len / K
  int32_t rows;        // rows of the bucket
  int32_t c0;          // first column
  int32_t range_rows;  // rows per range (the last range may have fewer)
  int32_t ranges;
  int32_t full;        // also rows 0 (the lanes' start bits) and `ranges` (their end bits)
  int64_t bit_base;
  int64_t out;         // first u32 of the job's checkpoints: [ranges - 1][K], or [ranges + 1][K] when full
  const int32_t *table_ids;
  const uint32_t *startbits;
  const int32_t *row_idx;
};

__global__ __launch_bounds__(kBlock) void fp8_checkpoints(const mps_fp8_tensor *__restrict__ tensors,
                                                          const SplitJob *__restrict__ jobs,
                                                          uint32_t *__restrict__ ckpt, uint32_t *__restrict__ failed) {
  __shared__ int32_t s_gid[256];
  __shared__ uint32_t s_lens[256 * kPacked / 4];  // packed length nibbles of each FP8 byte's table
  const SplitJob J = jobs[blockIdx.x];
  const mps_fp8_tensor &T = tensors[J.tensor];
  const int tid = threadIdx.x;
  if (tid < 256) {
    int32_t g = J.table_ids[tid];
    if (g < -1 || g >= T.num_tables) {
      failed[blockIdx.x] = 1u;
      g = -1;
    }
    s_gid[tid] = g;
  }
  __syncthreads();
  for (int i = tid; i < 256 * kPacked; i += kBlock) {
    const int32_t g = s_gid[i / kPacked];
    reinterpret_cast<uint8_t *>(s_lens)[i] = g >= 0 ? T.decode_lens[(int64_t)g * kPacked + i % kPacked] : 0u;
  }
  __syncthreads();
  if (tid >= J.K) return;
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;
  const uint8_t *lens = reinterpret_cast<const uint8_t *>(s_lens);
  uint64_t pos = (uint64_t)J.bit_base + J.startbits[tid];
  const int64_t row0 = J.out + (J.full ? 0 : -(int64_t)J.K);  // where checkpoint row 0 would go
  if (J.full) {
    ckpt[row0 + tid] = J.startbits[tid];
    ckpt[row0 + (int64_t)J.ranges * J.K + tid] = J.startbits[tid + 1];
  }
  uint64_t cidx = ~0ull;
  uint32_t ca = 0, cb = 0;
  const int64_t per_range = (int64_t)J.range_rows * J.P;
  int64_t next = per_range;
  int32_t row_idx = 0;
  int32_t rr = -1, p = 0;  // element's row (within the bucket) and column block
  for (int j = 1; j < J.ranges; ++j, next += per_range) {
    for (int64_t i = next - per_range; i < next; ++i) {
      if (rr != (int32_t)(i / J.P)) {
        rr = (int32_t)(i / J.P);
        p = 0;
        row_idx = J.row_idx[rr];
        if (row_idx < 0 || row_idx >= T.n) {
          failed[blockIdx.x] = 1u;
          return;
        }
      }
      const uint8_t q = T.fp8[(int64_t)row_idx * T.m + J.c0 + tid + (int64_t)p * J.K];
      ++p;
      const uint64_t c = pos >> 5;
      if (c != cidx) {
        cidx = c;
        ca = chunk_at(bs32, nchunks, c);
        cb = chunk_at(bs32, nchunks, c + 1);
      }
      const uint32_t peek = (uint32_t)(((((uint64_t)ca << 32) | cb) << (pos & 31u)) >> 57);
      const uint32_t nib = (lens[q * kPacked + (peek >> 1)] >> ((peek & 1u) * 4u)) & 0xFu;
      pos += (nib & 7u) + ((nib & 8u) ? 16u : 0u);
    }
    ckpt[row0 + (int64_t)j * J.K + tid] = (uint32_t)(pos - (uint64_t)J.bit_base);
  }
}

// ---------------------------------------------------------------------------
// Allocation-free batched decode. Some callers cannot allocate device memory
// (code under graph capture, tight serving loops). For them
// mps_fp8_decode_batch_noalloc decodes a list of tensors in one persistent
// launch, like a plan, with its descriptors and work records in `scratch`, a
// static device array of kScratchBytes that each device holds from module
// load to the end of the process. Buckets are not split into row ranges
// (that needs lane checkpoints, which a plan computes once).
//
// Layout of `scratch`: the descriptors (at most kMaxBatchTensors), then one
// 64-byte work record per bucket (at most kMaxBatchWork), then the decode
// launch's queue words in the last 256 bytes (zero from module load; each
// launch leaves them zero).
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(4) << 20;
constexpr int64_t kMaxBatchTensors = 1024;
constexpr size_t kBatchWorkOff = ((sizeof(mps_fp8_tensor) * kMaxBatchTensors + 255) / 256) * 256;
constexpr size_t kBatchQueueOff = kScratchBytes - 256;
constexpr int64_t kMaxBatchWork = (int64_t)((kBatchQueueOff - kBatchWorkOff) / sizeof(WorkItem));

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// One work record per bucket, in tensor order. Every workgroup first scans the
// bucket counts of the (at most 1024) tensors in LDS, then each work-item
// writes the record of one bucket from that bucket's metadata.
__global__ __launch_bounds__(256) void fp8_batch_records(const mps_fp8_tensor *__restrict__ tensors, int32_t count,
                                                        int64_t total, WorkItem *__restrict__ work) {
  constexpr int kPer = kMaxBatchTensors / 256;  // tensors per work-item in the scan
  __shared__ int64_t s_first[kMaxBatchTensors + 1];
  __shared__ int64_t s_part[256];
  const int t = threadIdx.x;
  int64_t v[kPer], sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int32_t i = t * kPer + j;
    v[j] = i < count ? tensors[i].num_buckets : 0;
    sum += v[j];
  }
  s_part[t] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {  // inclusive scan of the 256 partial sums
    const int64_t add = t >= off ? s_part[t - off] : 0;
    __syncthreads();
    s_part[t] += add;
    __syncthreads();
  }
  int64_t acc = s_part[t] - sum;  // exclusive prefix of this work-item's tensors
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    s_first[t * kPer + j] = acc;
    acc += v[j];
  }
  if (t == 255) s_first[kMaxBatchTensors] = acc;
  __syncthreads();
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total) return;
  int32_t lo = 0, hi = count - 1;  // the tensor i with s_first[i] <= g < s_first[i + 1]
  while (lo < hi) {
    const int32_t mid = (lo + hi + 1) >> 1;
    if (s_first[mid] <= g) lo = mid;
    else hi = mid - 1;
  }
  const mps_fp8_tensor &T = tensors[lo];
  WorkItem w = bucket_item(T, g - s_first[lo]);
  w.tensor = lo;
  work[g] = w;
}

// The device address of `scratch` on the current device, looked up once per
// device (the host-side name of a device array is not its address).
int scratch_ptr(uint8_t **out) {
  static std::mutex mu;
  static uint8_t *ptrs[kMaxDevices] = {};
  int dev = 0;
  MPS_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(MPS_ERR_INVALID_ARGUMENT, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    ptrs[dev] = static_cast<uint8_t *>(p);
  }
  *out = ptrs[dev];
  return MPS_OK;
}

// Workgroups of a persistent launch on the current device: one per CU.
int persistent_grid(int64_t items, unsigned *grid) {
  int dev = 0, cus = 0;
  MPS_HIP_CHECK(hipGetDevice(&dev));
  MPS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (cus < 1) cus = 1;
  *grid = (unsigned)(items < cus ? items : cus);
  return MPS_OK;
}

int check_tensor(const mps_fp8_tensor *t) {
  if (!t) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor descriptor is NULL");
  if (t->n <= 0 || t->m <= 0) return fail(MPS_ERR_INVALID_ARGUMENT, "n,m must be > 0");
  if (t->k <= 0 || t->k > 1024)
    return fail(MPS_ERR_INVALID_ARGUMENT, "bucket_thread_startbit_u32 has invalid k (must be 1..1024)");
  if (t->num_buckets < 0 || t->num_buckets > INT32_MAX)
    return fail(MPS_ERR_INVALID_ARGUMENT, "invalid number of buckets");
  if (t->num_buckets > 0 && (!t->fp8 || !t->out || !t->bucket_table || !t->bucket_col_start || !t->bucket_col_len ||
                             !t->bucket_row_offsets || !t->bucket_thread_startbit || !t->bucket_bit_base))
    return fail(MPS_ERR_INVALID_ARGUMENT, "NULL sidecar pointer");
  return MPS_OK;
}

}  // namespace

// The status word of the single-tensor decodes (FP8 and AWQ) on a device: a
// module global, so each device holds its own copy, zero from module load to
// the end of the process, and no decode allocates it. It is per device, not
// per stream: decodes on different streams of one device OR into the same
// word (mps_fp8_read_status reads and clears it). Plans carry a word of their own.
static __device__ __align__(256) uint32_t g_status[64];

int status_word(int device, uint32_t **out) {
  static std::mutex mu;
  static uint32_t *words[kMaxDevices] = {};
  if (device < 0 || device >= kMaxDevices) return fail(MPS_ERR_INVALID_ARGUMENT, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!words[device]) {
    // The host-side name of a device global is not its device address: look
    // it up once per device, with that device current.
    int prev = 0;
    MPS_HIP_CHECK(hipGetDevice(&prev));
    if (prev != device) MPS_HIP_CHECK(hipSetDevice(device));
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_status));
    if (prev != device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(status word)");
    words[device] = static_cast<uint32_t *>(p);
  }
  *out = words[device];
  return MPS_OK;
}

std::string &last_error() {
  static thread_local std::string s;
  return s;
}

// Read a device status word and clear it, after `stream`'s work (synchronous).
int read_and_clear(int device, uint32_t *word, void *stream, const char *what, uint32_t *status_out) {
  int prev = 0;
  MPS_HIP_CHECK(hipGetDevice(&prev));
  if (prev != device) MPS_HIP_CHECK(hipSetDevice(device));
  uint32_t v = 0;
  const uint32_t zero = 0;
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e == hipSuccess) e = hipMemcpy(&v, word, sizeof(v), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice);
  if (prev != device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, what);
  *status_out = v;
  return MPS_OK;
}

}  // namespace mps

using namespace mps;

namespace {
constexpr size_t kAlign = 256;
// Work queues of a plan: one per stream that launches it (two u32 words each,
// 64 bytes apart), so that launches on different streams - a graph replay
// and an eager decode, a prefetch on a side stream - never share one.
constexpr int kPlanQueues = 32;
constexpr size_t kQueueStride = 64;
// A work item's set-up (tables into the LDS, the lanes' first loads, the
// pipeline's fill and drain) costs about as long as decoding this many
// elements; plans weigh items by their elements plus this. (Tuning builds:
// MPS_ITEM_SETUP.)
#ifndef MPS_ITEM_SETUP
#define MPS_ITEM_SETUP 65536
#endif
constexpr int64_t kItemSetup = MPS_ITEM_SETUP;
size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }
}  // namespace

// A plan owns one device allocation: its status word, the tensor descriptors,
// the lane checkpoints of the buckets it split, the work records and (during
// creation) the checkpoint jobs and their failure flags.
// Tensors with k 256 or 512 substreams may have buckets for the slab path at that k.
inline bool slab_k(int64_t k) { return k == 256 || k == 512; }

struct mps_fp8_plan {
  void *d_block = nullptr;
  uint32_t *d_status = nullptr;
  // kPlanQueues work queues (work counter and exit count, zero between
  // launches); queue i serves streams[i], assigned at the stream's first launch.
  uint32_t *d_queue = nullptr;
  std::mutex mu;
  std::vector<void *> streams;
  mps_fp8_tensor *d_tensors = nullptr;
  WorkItem *d_work = nullptr;
  uint16_t *first_out = nullptr;  // the first tensor's output at creation (decode_into moves all by one offset)
  int64_t count = 0;
  int64_t work_items = 0;
  int device = 0;
  bool slab_k = false;      // some tensor has k 256 or 512: launch fp8_decode_plan<true, ...>
  bool end_ticket = false;  // few work items a CU: tickets taken as items end (fp8_decode_plan<..., true>)
};

extern "C" {

#if MPS_TRACE_ITEMS
// The item trace's host side (instrumented builds only; not part of the product ABI).
int mps_item_trace_clear(void) {
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_item_trace)) != hipSuccess) return MPS_ERR_HIP;
  return hipMemset(p, 0, sizeof(g_item_trace)) == hipSuccess ? MPS_OK : MPS_ERR_HIP;
}
int mps_item_trace_read(uint64_t *dst, int64_t words) {
  if (!dst || words < (int64_t)(sizeof(g_item_trace) / 8)) return MPS_ERR_INVALID_ARGUMENT;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_item_trace), sizeof(g_item_trace)) == hipSuccess ? MPS_OK
                                                                                                  : MPS_ERR_HIP;
}
#endif


const char *mps_last_error(void) { return last_error().c_str(); }

int mps_clock_rate_khz(int device, int64_t *khz_out) {
  if (!khz_out) return fail(MPS_ERR_INVALID_ARGUMENT, "khz_out is NULL");
  int v = 0;
  MPS_HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeClockRate, device));
  *khz_out = v;
  return MPS_OK;
}

int mps_stream_capture_id(void *stream, uint64_t *id_out) {
  last_error().clear();
  if (!id_out) return fail(MPS_ERR_INVALID_ARGUMENT, "id_out is NULL");
  hipStreamCaptureStatus s = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  MPS_HIP_CHECK(hipStreamGetCaptureInfo(reinterpret_cast<hipStream_t>(stream), &s, &id));
  *id_out = s == hipStreamCaptureStatusActive ? (uint64_t)id : 0u;
  return MPS_OK;
}

int mps_fp8_decode(const mps_fp8_tensor *tensor, int64_t max_len, void *stream) {
  last_error().clear();
  if (max_len != kL) return fail(MPS_ERR_INVALID_ARGUMENT, "decode kernel is specialized: max_len must be 7");
  int rc = check_tensor(tensor);
  if (rc != MPS_OK) return rc;
  if (tensor->num_buckets == 0) return MPS_OK;
  int dev = 0;
  MPS_HIP_CHECK(hipGetDevice(&dev));
  uint32_t *status = nullptr;
  rc = status_word(dev, &status);
  if (rc != MPS_OK) return rc;
  unsigned grid = 0;
  rc = persistent_grid(tensor->num_buckets, &grid);
  if (rc != MPS_OK) return rc;
  // Few buckets for the CUs (k = 1024): each bucket shared by `parts`
  // workgroups, the largest power of two up to 16 (one wave each) that keeps
  // buckets x parts within the CUs.
  int32_t parts = 1;
  {
    int dev2 = 0, cus = 0;
    MPS_HIP_CHECK(hipGetDevice(&dev2));
    MPS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev2));
    if (tensor->k == kBlock)
      while (parts < kBlock / 64 && tensor->num_buckets * parts * 2 <= (int64_t)cus) parts *= 2;
    if (parts > 1) grid = (unsigned)(tensor->num_buckets * parts);
  }
  if (slab_k(tensor->k))
    hipLaunchKernelGGL(fp8_decode_one<true>, dim3(grid), dim3(kBlock), 0, reinterpret_cast<hipStream_t>(stream),
                       *tensor, status, parts);
  else
    hipLaunchKernelGGL(fp8_decode_one<false>, dim3(grid), dim3(kBlock), 0, reinterpret_cast<hipStream_t>(stream),
                       *tensor, status, parts);
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

int mps_fp8_plan_create(const mps_fp8_tensor *tensors, int64_t count, void *stream, mps_fp8_plan **plan_out) {
  last_error().clear();
  if (!plan_out) return fail(MPS_ERR_INVALID_ARGUMENT, "plan_out is NULL");
  *plan_out = nullptr;
  if (count < 0 || (count > 0 && !tensors)) return fail(MPS_ERR_INVALID_ARGUMENT, "invalid tensor list");
  for (int64_t i = 0; i < count; ++i) {
    const int rc = check_tensor(&tensors[i]);
    if (rc != MPS_OK) return rc;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // The sidecars may still be being written by work on the caller's stream:
  // everything below reads them after that work.
  MPS_HIP_CHECK(hipStreamSynchronize(st));
  // One work record per bucket.
  std::vector<WorkItem> bucket;
  std::vector<int64_t> elems;  // elements of each bucket (0: a bad bucket)
  std::vector<int32_t> roff, cstart, clen;
  std::vector<int64_t> bbase;
  for (int64_t i = 0; i < count; ++i) {
    const mps_fp8_tensor &T = tensors[i];
    const int64_t nb = T.num_buckets;
    if (nb == 0) continue;
    roff.resize((size_t)nb + 1);
    cstart.resize((size_t)nb);
    clen.resize((size_t)nb);
    bbase.resize((size_t)nb);
    MPS_HIP_CHECK(hipMemcpy(roff.data(), T.bucket_row_offsets, sizeof(int32_t) * (nb + 1), hipMemcpyDefault));
    MPS_HIP_CHECK(hipMemcpy(cstart.data(), T.bucket_col_start, sizeof(int32_t) * nb, hipMemcpyDefault));
    MPS_HIP_CHECK(hipMemcpy(clen.data(), T.bucket_col_len, sizeof(int32_t) * nb, hipMemcpyDefault));
    MPS_HIP_CHECK(hipMemcpy(bbase.data(), T.bucket_bit_base, sizeof(int64_t) * nb, hipMemcpyDefault));
    for (int64_t b = 0; b < nb; ++b) {
      const BucketShape s = bucket_shape(roff[b], roff[b + 1], cstart[b], clen[b], T);
      WorkItem w;
      w.tensor = (int32_t)i;
      w.c0 = cstart[b];
      w.cl = clen[b];
      w.rows = s.rows;
      w.k_eff = s.k_eff;
      w.path = s.path;
      w.bit_base = bbase[b];
      w.table_ids = T.bucket_table + b * 256;
      w.startbits = T.bucket_thread_startbit + b * (T.k + 1);
      w.endbits = w.startbits + 1;
      w.row_idx = T.row_indices + (s.path != kPathBad ? roff[b] : 0);
      bucket.push_back(w);
      elems.push_back(s.path != kPathBad ? (int64_t)s.rows * clen[b] : 0);
    }
  }
  if (bucket.size() > (size_t)INT32_MAX) return fail(MPS_ERR_INVALID_ARGUMENT, "too many buckets for one plan");
  int device = 0, cus = 0;
  MPS_HIP_CHECK(hipGetDevice(&device));
  MPS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));

  // Row ranges. A plan whose buckets are few or uneven for the CUs (a layer,
  // a single tensor) would leave CUs idle behind its largest buckets: buckets
  // on the k = 1024 and fast paths larger than total / (2 * CUs) elements are
  // split into row ranges of at most that size (and at least 64 elements per
  // substream, 16 groups, so that a range's set-up stays small beside its
  // decode). Each range starts from lane checkpoints (fp8_checkpoints).
  //
  // A fast-path bucket with k_eff 256 or 512 fills only k_eff of a
  // workgroup's 1024 work-items, and its tables allow one workgroup per CU. So
  // it is cut into a multiple of S = 1024 / k_eff row ranges, and each work
  // item runs S of them side by side over the same tables (kMultiRange): the
  // unit of splitting is then an item of S ranges.
  //
  // An item's cost is the time its work-items take: the elements each one
  // decodes times 1024 (the elements of a k = 1024 item; S ranges side by
  // side cost one range's), plus kItemSetup for its set-up.
  //
  // Then the tail. The launch's queue hands the items out largest first
  // (fp8_decode_plan), and an item handed out when R elements of work remain
  // (it and the items after it) can end up to about its size minus R / CUs
  // after the others. Every item past the first CUs that exceeds
  // kTailRatio * R / CUs has its bucket split twice as fine, until none does
  // or none can be. Coarse items keep the set-ups few (each costs about as
  // much as decoding kItemSetup elements); the fine ones at the end fill the
  // CUs' last gaps.
#ifndef MPS_SPLIT_DIV
#define MPS_SPLIT_DIV 2
#endif
#ifndef MPS_TAIL_RATIO
#define MPS_TAIL_RATIO 3
#endif
  constexpr int64_t kTailRatio = MPS_TAIL_RATIO;
  const int64_t ncu = std::max(cus, 1);
  // Per bucket: ranges per item (1, or S for a multi-range bucket), the most
  // items it may be cut into, and its cost as one item (elements + set-up).
  std::vector<int64_t> per_item(bucket.size(), 1), maxi(bucket.size(), 1), whole_cost(bucket.size());
  // cost of `rows` rows of split-capable bucket i decoded by one group of work-items
  auto rows_cost = [&](size_t i, int64_t rows) {
    return rows * (int64_t)(bucket[i].cl / bucket[i].k_eff) * 1024 + kItemSetup;
  };
  for (size_t i = 0; i < bucket.size(); ++i) {
    const WorkItem &w = bucket[i];
    const int64_t ke = std::max<int64_t>(w.k_eff, 1);
    whole_cost[i] = (elems[i] + ke - 1) / ke * 1024 + kItemSetup;
    if ((w.path != kPathK1024 && w.path != kPathFast) || w.rows < 2) continue;
    const int32_t P = w.cl / w.k_eff;
    const int32_t min_rows = std::max<int32_t>(1, (64 + P - 1) / P);
    const int64_t maxr = std::max<int64_t>(1, w.rows / min_rows);
    const int64_t S = w.path == kPathFast && (w.k_eff == 256 || w.k_eff == 512) ? 1024 / w.k_eff : 1;
    // range rows ride in 8 bits of the work record (fast buckets hold <= 128 rows)
    if (S > 1 && maxr >= S && w.rows <= 255) {
      per_item[i] = S;
      maxi[i] = maxr / S;
      whole_cost[i] = rows_cost(i, (w.rows + S - 1) / S);
    } else {
      maxi[i] = maxr;
    }
  }
  // Items of bucket i cut into ni items: their costs, largest first.
  auto for_items = [&](size_t i, int64_t ni, auto &&emit) {
    const int64_t rows = bucket[i].rows;
    if (ni <= 1 && per_item[i] == 1) {
      emit(whole_cost[i]);
      return;
    }
    const int64_t rr = (rows + ni * per_item[i] - 1) / (ni * per_item[i]);  // rows per range
    const int64_t step = rr * per_item[i];                                    // rows per item
    for (int64_t r0 = 0; r0 < rows; r0 += step) emit(rows_cost(i, std::min(rr, rows - r0)));
  };
  int64_t total = 0;
  for (size_t i = 0; i < bucket.size(); ++i) total += whole_cost[i] - kItemSetup;
  const int64_t cap = std::max<int64_t>(total / (MPS_SPLIT_DIV * ncu), 65536);
  std::vector<int64_t> ni(bucket.size(), 1);  // items of each bucket
  for (size_t i = 0; i < bucket.size(); ++i) {
    const int64_t c = whole_cost[i] - kItemSetup;
    if (c > cap) ni[i] = std::min<int64_t>((c + cap - 1) / cap, maxi[i]);
  }
  {
    struct Piece {
      int64_t cost;
      size_t b;
    };
    std::vector<Piece> pieces;
    std::vector<char> bump(bucket.size());
    for (int iter = 0; iter < 64; ++iter) {
      pieces.clear();
      for (size_t i = 0; i < bucket.size(); ++i) for_items(i, ni[i], [&](int64_t c) { pieces.push_back({c, i}); });
      std::stable_sort(pieces.begin(), pieces.end(), [](const Piece &a, const Piece &c) { return a.cost > c.cost; });
      std::fill(bump.begin(), bump.end(), 0);
      bool changed = false;
      int64_t rest = 0;
      for (size_t q = pieces.size(); q-- > 0;) {
        rest += pieces[q].cost;
        const size_t b = pieces[q].b;
        if ((int64_t)q < ncu || bump[b] || ni[b] >= maxi[b]) continue;
        if ((double)pieces[q].cost * (double)ncu > (double)kTailRatio * (double)rest) {
          bump[b] = 1;
          ni[b] = std::min(maxi[b], ni[b] * 2);
          changed = true;
        }
      }
      if (!changed) break;
    }
  }
  // Splitting pays only where it shortens the launch: a tensor whose buckets
  // about match the CUs (a 70B gate_proj: 224 buckets of 1 M elements for 256
  // CUs) already ends after one bucket per CU, and its ranges would only add
  // set-ups. So the plan predicts both launches (items largest first, each to
  // the CU that frees first) and keeps the buckets whole (multi-range buckets:
  // one item) unless the split one ends sooner.
  {
    auto makespan = [&](const std::vector<int64_t> &items_of) {
      std::vector<int64_t> items;
      for (size_t i = 0; i < bucket.size(); ++i) for_items(i, items_of[i], [&](int64_t c) { items.push_back(c); });
      std::sort(items.begin(), items.end(), std::greater<int64_t>());
      std::priority_queue<int64_t, std::vector<int64_t>, std::greater<int64_t>> cu;
      for (int64_t c = 0; c < ncu; ++c) cu.push(0);
      int64_t end = 0;
      for (int64_t x : items) {
        const int64_t t = cu.top() + x;
        cu.pop();
        cu.push(t);
        end = std::max(end, t);
      }
      return end;
    };
    const std::vector<int64_t> whole(bucket.size(), 1);
    if (std::any_of(ni.begin(), ni.end(), [](int64_t x) { return x > 1; }) && makespan(whole) <= makespan(ni))
      ni = whole;
  }
  // Ranges of each bucket.
  std::vector<int64_t> nr(bucket.size());
  for (size_t i = 0; i < bucket.size(); ++i) nr[i] = ni[i] * per_item[i];
  std::vector<SplitJob> jobs;
  std::vector<size_t> job_of(bucket.size(), SIZE_MAX);
  int64_t ck_words = 0, max_items = 0;
  for (size_t i = 0; i < bucket.size(); ++i) {
    const WorkItem &w = bucket[i];
    ++max_items;
    if (nr[i] < 2) continue;
    const int32_t P = w.cl / w.k_eff;
    int64_t ranges = nr[i];
    const int32_t range_rows = (int32_t)((w.rows + ranges - 1) / ranges);
    ranges = (w.rows + range_rows - 1) / range_rows;
    if (ranges < 2) continue;
    SplitJob j{};
    j.tensor = w.tensor;
    j.K = w.k_eff;
    j.P = P;
    j.rows = w.rows;
    j.c0 = w.c0;
    j.range_rows = range_rows;
    j.ranges = (int32_t)ranges;
    j.bit_base = w.bit_base;
    j.out = ck_words;
    j.table_ids = w.table_ids;
    j.startbits = w.startbits;
    j.row_idx = w.row_idx;
    j.full = per_item[i] > 1 ? 1 : 0;
    job_of[i] = jobs.size();
    jobs.push_back(j);
    ck_words += (per_item[i] > 1 ? ranges + 1 : ranges - 1) * w.k_eff;
    max_items += ranges - 1;
  }

  // The plan's device block: the status word at 0, the work queues from
  // kAlign, then the descriptors, checkpoints, split jobs, their flags and the
  // work records.
  if (max_items >= kMaxQueueItems) return fail(MPS_ERR_INVALID_ARGUMENT, "too many work items for one plan");
  const size_t o_queues = kAlign;
  const size_t o_tensors = o_queues + align_up(kQueueStride * kPlanQueues);
  const size_t o_ckpt = o_tensors + align_up(sizeof(mps_fp8_tensor) * (size_t)count);
  const size_t o_jobs = o_ckpt + align_up(sizeof(uint32_t) * (size_t)ck_words);
  const size_t o_failed = o_jobs + align_up(sizeof(SplitJob) * jobs.size());
  const size_t o_work = o_failed + align_up(sizeof(uint32_t) * jobs.size());
  const size_t bytes = o_work + sizeof(WorkItem) * (size_t)max_items;
  auto *p = new (std::nothrow) mps_fp8_plan();
  if (!p) return fail(MPS_ERR_NO_MEMORY, "out of memory");
  p->count = count;
  p->slab_k = std::any_of(tensors, tensors + count, [](const mps_fp8_tensor &t) { return slab_k(t.k); });
  p->device = device;
  p->first_out = count > 0 ? tensors[0].out : nullptr;
  hipError_t e = hipMalloc(&p->d_block, bytes);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "mps_fp8_plan_create");
  }
  auto cleanup = [&](hipError_t err) {
    (void)hipStreamSynchronize(st);
    (void)hipFree(p->d_block);
    delete p;
    return hip_fail(err, "mps_fp8_plan_create");
  };
  char *blk = static_cast<char *>(p->d_block);
  p->d_status = reinterpret_cast<uint32_t *>(blk);
  p->d_queue = reinterpret_cast<uint32_t *>(blk + o_queues);
  p->d_tensors = reinterpret_cast<mps_fp8_tensor *>(blk + o_tensors);
  p->d_work = reinterpret_cast<WorkItem *>(blk + o_work);
  uint32_t *d_ckpt = reinterpret_cast<uint32_t *>(blk + o_ckpt);
  // Status word and queues (zero), descriptors, jobs and their flags (zero): one copy, on the caller's stream.
  std::vector<char> head(o_work, 0);
  if (count > 0) std::memcpy(head.data() + o_tensors, tensors, sizeof(mps_fp8_tensor) * (size_t)count);
  if (!jobs.empty()) std::memcpy(head.data() + o_jobs, jobs.data(), sizeof(SplitJob) * jobs.size());
  e = hipMemcpyAsync(blk, head.data(), head.size(), hipMemcpyHostToDevice, st);
  std::vector<uint32_t> failed(jobs.size(), 0u);
  if (e == hipSuccess && !jobs.empty()) {
    hipLaunchKernelGGL(fp8_checkpoints, dim3((unsigned)jobs.size()), dim3(kBlock), 0, st, p->d_tensors,
                       reinterpret_cast<const SplitJob *>(blk + o_jobs), d_ckpt,
                       reinterpret_cast<uint32_t *>(blk + o_failed));
    e = hipGetLastError();
    if (e == hipSuccess)
      e = hipMemcpyAsync(failed.data(), blk + o_failed, sizeof(uint32_t) * jobs.size(), hipMemcpyDeviceToHost, st);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return cleanup(e);

  // Work items (buckets and ranges), largest first, the order in which the
  // launch's queue hands them out, by the cost above.
  std::vector<WorkItem> work;
  std::vector<int64_t> cost;
  for (size_t i = 0; i < bucket.size(); ++i) {
    const WorkItem &w = bucket[i];
    if (job_of[i] == SIZE_MAX || failed[job_of[i]]) {
      work.push_back(w);
      cost.push_back(per_item[i] > 1 ? rows_cost(i, w.rows) : whole_cost[i]);  // a failed walk: one range
      continue;
    }
    const SplitJob &j = jobs[job_of[i]];
    const uint32_t *ck = d_ckpt + j.out;
    if (j.full) {
      // S ranges an item; range r's start bits are checkpoint row r, its end bits row r + 1
      const int32_t S = 1024 / j.K;
      for (int32_t r = 0; r < j.ranges; r += S) {
        WorkItem x = w;
        x.path = kPathFast | kMultiRange | (j.range_rows << 8);
        x.rows = w.rows - r * j.range_rows;
        x.row_idx = w.row_idx + (int64_t)r * j.range_rows;
        x.startbits = ck + (int64_t)r * j.K;
        x.endbits = ck + (int64_t)(r + 1) * j.K;
        work.push_back(x);
        cost.push_back(rows_cost(i, std::min(j.range_rows, x.rows)));
      }
      continue;
    }
    for (int32_t r = 0; r < j.ranges; ++r) {
      WorkItem x = w;
      x.rows = std::min(j.range_rows, w.rows - r * j.range_rows);
      x.row_idx = w.row_idx + (int64_t)r * j.range_rows;
      x.startbits = r == 0 ? w.startbits : ck + (int64_t)(r - 1) * j.K;
      x.endbits = r + 1 == j.ranges ? w.endbits : ck + (int64_t)r * j.K;
      work.push_back(x);
      cost.push_back(rows_cost(i, x.rows));
    }
  }
  {
    std::vector<size_t> order(work.size());
    for (size_t j = 0; j < order.size(); ++j) order[j] = j;
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t c) { return cost[a] > cost[c]; });
    std::vector<WorkItem> sorted(work.size());
    for (size_t j = 0; j < order.size(); ++j) sorted[j] = work[order[j]];
    work.swap(sorted);
  }
  p->work_items = (int64_t)work.size();
  // Ticket mode. With the ticket taken in an item's set-up, a workgroup holds
  // its next item for the whole current one: right for many items of about one
  // size (a full model: ~100 a CU), where the next record then loads during the
  // drain. With few items a CU (a layer, a tensor: split items of mixed sizes),
  // a workgroup that drew a long item would keep its next one from a workgroup
  // that frees sooner, so the ticket is taken as the item ends (measured: 8B
  // layer -2.5%, 70B layer -4.7%; the full model +0.3% that way).
  p->end_ticket = p->work_items < 16 * (int64_t)ncu;
  if (!work.empty()) {
    e = hipMemcpyAsync(p->d_work, work.data(), sizeof(WorkItem) * work.size(), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return cleanup(e);
  }
  *plan_out = p;
  return MPS_OK;
}

namespace {
// The work queue of `stream` in the plan: the one it was given at its first
// launch, or the next free one. A launch leaves its queue as it found it, so
// launches on one stream (in stream order) can share one; launches on
// different streams may overlap and each has its own. A graph captured on a
// stream replays with that stream's queue.
int plan_queue(mps_fp8_plan *plan, void *stream, uint32_t **queue) {
  std::lock_guard<std::mutex> lock(plan->mu);
  size_t i = 0;
  while (i < plan->streams.size() && plan->streams[i] != stream) ++i;
  if (i == plan->streams.size()) {
    if (i >= (size_t)kPlanQueues)
      return fail(MPS_ERR_RUNTIME, "a decode plan serves at most %d streams", kPlanQueues);
    plan->streams.push_back(stream);
  }
  *queue = plan->d_queue + i * (kQueueStride / sizeof(uint32_t));
  return MPS_OK;
}

int plan_launch(mps_fp8_plan *plan, int64_t out_delta, uint32_t *status, void *stream) {
  if (plan->work_items == 0) return MPS_OK;
  unsigned grid = 0;
  int rc = persistent_grid(plan->work_items, &grid);
  if (rc != MPS_OK) return rc;
  uint32_t *queue = nullptr;
  rc = plan_queue(plan, stream, &queue);
  if (rc != MPS_OK) return rc;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, reinterpret_cast<hipStream_t>(stream), plan->d_tensors,
                       plan->d_work, plan->work_items, status, out_delta, queue);
  };
  if (plan->slab_k) {
    if (plan->end_ticket) launch(fp8_decode_plan<true, true>);
    else launch(fp8_decode_plan<true, false>);
  } else {
    if (plan->end_ticket) launch(fp8_decode_plan<false, true>);
    else launch(fp8_decode_plan<false, false>);
  }
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}
}  // namespace

int mps_fp8_plan_decode(mps_fp8_plan *plan, void *stream) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  return plan_launch(plan, 0, plan->d_status, stream);
}

int mps_fp8_plan_decode_into(mps_fp8_plan *plan, uint16_t *out, void *stream) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (!out) return fail(MPS_ERR_INVALID_ARGUMENT, "out is NULL");
  if (plan->count == 0) return MPS_OK;
  uint32_t *status = nullptr;
  const int rc = status_word(plan->device, &status);
  if (rc != MPS_OK) return rc;
  const intptr_t delta = reinterpret_cast<intptr_t>(out) - reinterpret_cast<intptr_t>(plan->first_out);
  if (delta % (intptr_t)sizeof(uint16_t) != 0)
    return fail(MPS_ERR_INVALID_ARGUMENT, "out must be 2-byte aligned like the plan's outputs");
  return plan_launch(plan, (int64_t)(delta / (intptr_t)sizeof(uint16_t)), status, stream);
}

int mps_fp8_plan_info(const mps_fp8_plan *plan, int64_t *work_items, int64_t *lds_bytes) {
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (work_items) *work_items = plan->work_items;
  if (lds_bytes) *lds_bytes = (int64_t)kLdsWords * 4;
  return MPS_OK;
}

int mps_fp8_plan_read_status(mps_fp8_plan *plan, void *stream, uint32_t *status_out) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (!status_out) return fail(MPS_ERR_INVALID_ARGUMENT, "status_out is NULL");
  return read_and_clear(plan->device, plan->d_status, stream, "mps_fp8_plan_read_status", status_out);
}

int mps_fp8_plan_destroy(mps_fp8_plan *plan) {
  if (!plan) return MPS_OK;
  if (plan->d_block) (void)hipFree(plan->d_block);
  delete plan;
  return MPS_OK;
}

int mps_fp8_read_status(int device, void *stream, uint32_t *status_out) {
  last_error().clear();
  if (!status_out) return fail(MPS_ERR_INVALID_ARGUMENT, "status_out is NULL");
  uint32_t *word = nullptr;
  const int rc = status_word(device, &word);
  if (rc != MPS_OK) return rc;
  return read_and_clear(device, word, stream, "mps_fp8_read_status", status_out);
}


int mps_fp8_decode_batch_noalloc(const mps_fp8_tensor *tensors, int64_t count, int64_t max_len, void *stream) {
  last_error().clear();
  if (max_len != kL) return fail(MPS_ERR_INVALID_ARGUMENT, "decode kernel is specialized: max_len must be 7");
  if (count < 0 || (count > 0 && !tensors)) return fail(MPS_ERR_INVALID_ARGUMENT, "invalid tensor list");
  if (count > kMaxBatchTensors)
    return fail(MPS_ERR_INVALID_ARGUMENT,
                "mps_fp8_decode_batch_noalloc: %lld tensors exceed its static scratch (at most %lld)",
                (long long)count, (long long)kMaxBatchTensors);
  int64_t total = 0;
  for (int64_t i = 0; i < count; ++i) {
    const int rc = check_tensor(&tensors[i]);
    if (rc != MPS_OK) return rc;
    total += tensors[i].num_buckets;
  }
  if (total > kMaxBatchWork)
    return fail(MPS_ERR_INVALID_ARGUMENT,
                "mps_fp8_decode_batch_noalloc: %lld buckets exceed its static scratch (at most %lld)",
                (long long)total, (long long)kMaxBatchWork);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // The descriptors travel by a copy from the caller's host array. Captured
  // into a graph, that copy would re-read the host address on every replay,
  // long after the array is gone: a capturing stream is refused, before any
  // copy or launch.
  {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess || cs != hipStreamCaptureStatusNone)
      return fail(MPS_ERR_INVALID_ARGUMENT,
                  "mps_fp8_decode_batch_noalloc cannot run on a capturing stream (its descriptors are copied "
                  "from host memory); create a decode plan before the capture and launch that instead");
  }
  if (total == 0) return MPS_OK;
  int dev = 0;
  MPS_HIP_CHECK(hipGetDevice(&dev));
  uint32_t *status = nullptr;
  int rc = status_word(dev, &status);
  if (rc != MPS_OK) return rc;
  uint8_t *base = nullptr;
  rc = scratch_ptr(&base);
  if (rc != MPS_OK) return rc;
  auto *d_tensors = reinterpret_cast<mps_fp8_tensor *>(base);
  auto *d_work = reinterpret_cast<WorkItem *>(base + kBatchWorkOff);
  // The descriptors are read from the caller's host array before this returns.
  MPS_HIP_CHECK(hipMemcpyAsync(d_tensors, tensors, sizeof(mps_fp8_tensor) * (size_t)count, hipMemcpyHostToDevice, st));
  hipLaunchKernelGGL(fp8_batch_records, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, d_tensors,
                     (int32_t)count, total, d_work);
  MPS_HIP_CHECK(hipGetLastError());
  unsigned grid = 0;
  rc = persistent_grid(total, &grid);
  if (rc != MPS_OK) return rc;
  const bool sk = std::any_of(tensors, tensors + count, [](const mps_fp8_tensor &t) { return slab_k(t.k); });
  if (sk)
    hipLaunchKernelGGL((fp8_decode_plan<true, false>), dim3(grid), dim3(kBlock), 0, st, d_tensors, d_work, total,
                       status, (int64_t)0, reinterpret_cast<uint32_t *>(base + kBatchQueueOff));
  else
    hipLaunchKernelGGL((fp8_decode_plan<false, false>), dim3(grid), dim3(kBlock), 0, st, d_tensors, d_work, total,
                       status, (int64_t)0, reinterpret_cast<uint32_t *>(base + kBatchQueueOff));
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

}  // extern "C"
