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
// element costs one ds_read_b32 for its code and none for its address. The
// bit supply is the FP8 generic lane's: a 64-bit MSB-aligned buffer topped up
// to >= 32 bits after every element from a 4-chunk register queue, whose
// loads (and the block's int4 bytes) are issued one block of kDepth elements
// ahead. kDepth = 4 keeps a block's codes (<= 44 bits) within the two chunks
// staged per block; ESC payloads can drain the queue, which then reads a chunk
// straight from memory.
#include <hip/hip_runtime.h>

#include <cstdint>

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
constexpr int kDepth = 4;

__device__ __forceinline__ void flag(uint32_t *status, unsigned int f) { atomicOr(status, f); }

// Stream chunk c (32 bits, stream order) of u64 words stored little-endian:
// word w's first 32 stream bits are u32 2w+1. Past the end the last chunk is
// re-read: a well-formed lane never consumes those bits, and an 11-bit peek
// that runs past its last code selects an entry whose low bits do not matter.
__device__ __forceinline__ uint32_t chunk_at(const uint32_t *__restrict__ bs32, uint64_t nchunks, uint64_t c) {
  const uint64_t cc = c < nchunks ? c : nchunks - 1;
  return bs32[cc ^ 1u];
}

__device__ uint32_t g_awq_zero_chunks[2];

// Element offset (row * m + column start) of row (group) rr of the bucket.
__device__ __forceinline__ uint32_t row_base(const mps_awq_tensor &T, const uint32_t *__restrict__ s_base,
                                             int32_t ra, int32_t rr, int32_t c0, int32_t cl) {
  if (rr < kRowSlots) return s_base[rr];
  const int64_t row = T.row_indices[ra + rr];
  const int64_t col = T.group_col_start ? (int64_t)T.group_col_start[ra + rr] : (int64_t)c0;
  if (row < 0 || row >= T.n || col < 0 || col + cl > T.m) return kBadBase;
  return (uint32_t)(row * T.m + col);
}

__global__ __launch_bounds__(kAwqBlock) void awq_decode_kernel(mps_awq_tensor T, uint32_t *status) {
  __shared__ uint32_t lut[kLutEntries];
  __shared__ uint32_t s_base[kRowSlots];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
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
  // is all ESC entries, as the reference decodes it.
  for (int i = tid; i < kLutEntries; i += kAwqBlock) {
    const int q = i >> kAwqL, p = i & (kAwqTable - 1);
    const int32_t gid = T.bucket_table[b * 16 + q];
    uint32_t ent = 15u;
    if (gid >= 0 && gid < T.num_tables) {
      const uint32_t v = T.decode_lens[(int64_t)gid * kAwqPacked + (p >> 1)];
      ent = ((uint32_t)T.decode_syms[(int64_t)gid * kAwqTable + p] << 16) | ((p & 1) ? (v >> 4) : (v & 15u));
    } else if (gid != -1 && p == 0) {
      flag(status, MPS_STATUS_BAD_TABLE);
    }
    lut[i] = ent;
  }
  const int32_t staged = rows < kRowSlots ? rows : kRowSlots;
  for (int r = tid; r < staged; r += kAwqBlock) {
    const int64_t row = T.row_indices[ra + r];
    const int64_t col = by_scale ? (int64_t)T.group_col_start[ra + r] : (int64_t)c0;
    uint32_t base = kBadBase;
    if (row >= 0 && row < T.n && col >= 0 && col + cl <= T.m) base = (uint32_t)(row * T.m + col);
    else flag(status, MPS_STATUS_BAD_ROW);
    s_base[r] = base;
  }
  __syncthreads();
  if (tid >= k_eff) return;

  const uint32_t *__restrict__ sb = T.bucket_thread_startbit + b * ((int64_t)k + 1);
  const uint64_t pos0 = (uint64_t)T.bucket_bit_base[b] + sb[tid];
  const uint64_t pos_end = (uint64_t)T.bucket_bit_base[b] + sb[tid + 1];
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_awq_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;

  // Initial fill: buffer from chunks cb, cb+1; queue = cb+2 .. cb+5; tail = cb+6.
  const uint64_t cb = pos0 >> 5;
  const int skip = (int)(pos0 & 31u);
  uint64_t buf = (((uint64_t)chunk_at(bs32, nchunks, cb) << 32) | chunk_at(bs32, nchunks, cb + 1)) << skip;
  int cnt = 64 - skip;
  uint32_t q0 = chunk_at(bs32, nchunks, cb + 2), q1 = chunk_at(bs32, nchunks, cb + 3);
  uint32_t q2 = chunk_at(bs32, nchunks, cb + 4), q3 = chunk_at(bs32, nchunks, cb + 5);
  int qn = 4;
  uint64_t tail = cb + 6;

  // Element walk e = tid + i*k_eff -> (rr, cc) = (e / cl, e % cl), incrementally.
  int32_t rr = tid / cl;
  int32_t cc = tid - rr * cl;
  const int32_t dr = k_eff / cl, dc = k_eff - dr * cl;
  const int32_t count = (int32_t)((total - tid + k_eff - 1) / k_eff);
  const uint8_t *__restrict__ qv = T.int4;
  uint16_t *__restrict__ out = T.out;
  const uint32_t first = row_base(T, s_base, ra, rr, c0, cl);
  const uint32_t safe = first == kBadBase ? 0u : first + (uint32_t)cc;  // an address every lane may read
  int32_t walked = 0;
  auto next_block = [&](uint32_t (&idx)[kDepth]) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      uint32_t v = kBadBase;
      if (walked + j < count) {
        const uint32_t base = row_base(T, s_base, ra, rr, c0, cl);
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
  uint32_t s0 = chunk_at(bs32, nchunks, tail), s1 = chunk_at(bs32, nchunks, tail + 1);
  bool stale = false;

  auto refill = [&]() {
    if (cnt < 32) {
      if (qn > 0) {
        buf |= (uint64_t)q0 << (32 - cnt);
        q0 = q1;
        q1 = q2;
        q2 = q3;
        --qn;
      } else {
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
    if (idx != kBadBase) out[idx] = (uint16_t)sym;
    refill();
  };
  auto block = [&](int32_t i0, uint32_t (&qc)[kDepth], uint32_t (&ic)[kDepth], uint32_t (&qnx)[kDepth],
                   uint32_t (&inx)[kDepth]) {
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
    for (int j = 0; j < kDepth; ++j) qnx[j] = qv[inx[j] == kBadBase ? safe : inx[j]];
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
  // The next unread bit must be where the next lane's substream begins.
  if (tail * 32u - (uint64_t)(cnt + 32 * qn) != pos_end) flag(status, MPS_STATUS_DESYNC);
}

int check_awq(const mps_awq_tensor *t) {
  if (!t) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor is NULL");
  if (t->n <= 0 || t->m <= 0) return fail(MPS_ERR_INVALID_ARGUMENT, "n,m must be > 0");
  if (t->n * t->m >= ((int64_t)1 << 32) - 1) return fail(MPS_ERR_INVALID_ARGUMENT, "tensor too large (n*m >= 2^32)");
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

extern "C" {

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
  hipLaunchKernelGGL(awq_decode_kernel, dim3((unsigned)tensor->num_buckets), dim3(kAwqBlock), 0,
                     reinterpret_cast<hipStream_t>(stream), *tensor, status);
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

}  // extern "C"
