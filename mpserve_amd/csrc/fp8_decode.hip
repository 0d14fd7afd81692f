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

#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "mps_common.h"

namespace mps {

namespace {

constexpr int kL = 7;
constexpr int kTable = 1 << kL;           // 128 entries per code table
constexpr int kPacked = kTable / 2;       // 64 bytes of packed 4-bit lengths
constexpr int kBlock = 1024;              // work-items per bucket workgroup (>= k)
constexpr int kRowsLds = 256;             // row indices staged in LDS
constexpr uint32_t kEscBit = 1u << 19;
constexpr int kMaxDevices = 64;

// Integrity flags go to a per-device status word passed to every launch.
__device__ __forceinline__ void flag(uint32_t *status, unsigned int f) { atomicOr(status, f); }

// Stream chunk c (32 bits, stream order) of a bitstream of u64 words stored
// little-endian: word w's high half (its first 32 stream bits) is u32 2w+1.
// Past the end the last chunk is re-read instead of zeros, so the load needs no
// branch: a well-formed stream never consumes those bits, and a 7-bit peek that
// runs past its last code selects a table entry whose low bits do not matter.
__device__ __forceinline__ uint32_t chunk_at(const uint32_t *__restrict__ bs32, uint64_t nchunks, uint64_t c) {
  const uint64_t cc = c < nchunks ? c : nchunks - 1;
  return bs32[cc ^ 1u];
}

__device__ uint32_t g_zero_chunks[2];

struct WorkItem {
  int32_t tensor;
  int32_t bucket;
};

// One lane: decode its substream. Elements are processed in blocks of kDepth;
// the FP8 bytes of block j+1 are loaded while block j decodes, so their memory
// latency overlaps the table lookups instead of stalling each element.
constexpr int kDepth = 8;

template <typename Idx>
__device__ __forceinline__ void decode_lane(const mps_fp8_tensor &T, const uint32_t *__restrict__ lut,
                                            const int32_t *__restrict__ s_rows, int32_t lane, int32_t k_eff,
                                            int64_t total, int32_t c0, int32_t cl, uint64_t pos0, uint64_t pos_end,
                                            uint32_t *status) {
  const bool empty = T.bitstream_words <= 0;
  const uint32_t *__restrict__ bs32 = empty ? g_zero_chunks : reinterpret_cast<const uint32_t *>(T.bitstream);
  const uint64_t nchunks = empty ? 2u : (uint64_t)T.bitstream_words * 2u;
  uint64_t c = pos0 >> 5;
  const int skip = (int)(pos0 & 31u);
  uint64_t buf = (((uint64_t)chunk_at(bs32, nchunks, c) << 32) | chunk_at(bs32, nchunks, c + 1)) << skip;
  int cnt = 64 - skip;
  c += 2;
  uint32_t nxt = chunk_at(bs32, nchunks, c);

  // Element walk e = lane + i*k_eff -> (rr, cc) = (e / cl, e % cl), incrementally.
  int32_t rr = lane / cl;
  int32_t cc = lane - rr * cl;
  const int32_t dr = k_eff / cl;
  const int32_t dc = k_eff - dr * cl;
  const int32_t count = (int32_t)((total - lane + k_eff - 1) / k_eff);
  const Idx m = (Idx)T.m;
  const int32_t last_row = (int32_t)((total - 1) / cl);
  Idx rowbase = (Idx)s_rows[rr] * m + (Idx)c0;
  auto step = [&]() -> Idx {
    const Idx v = rowbase + (Idx)cc;
    cc += dc;
    rr += dr;
    if (cc >= cl) {
      cc -= cl;
      rr += 1;
    }
    if (dr != 0 || cc < dc) rowbase = (Idx)s_rows[rr < last_row ? rr : last_row] * m + (Idx)c0;
    return v;
  };
  const uint8_t *__restrict__ fp8 = T.fp8;
  uint16_t *__restrict__ out = T.out;

  Idx idx_cur[kDepth], idx_nxt[kDepth];
  uint32_t q_cur[kDepth], q_nxt[kDepth];
  const Idx first = rowbase + (Idx)cc;
#pragma unroll
  for (int j = 0; j < kDepth; ++j) {
    idx_cur[j] = (j < count) ? step() : first;
    q_cur[j] = fp8[idx_cur[j]];
  }
  for (int32_t i0 = 0; i0 < count; i0 += kDepth) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      idx_nxt[j] = (i0 + kDepth + j < count) ? step() : first;
      q_nxt[j] = fp8[idx_nxt[j]];
    }
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      if (i0 + j < count) {
        const uint32_t peek = (uint32_t)(buf >> (64 - kL));
        const uint32_t ent = lut[(q_cur[j] << kL) | peek];
        const int len = (int)((ent >> 16) & 7u);
        buf <<= len;
        cnt -= len;
        uint32_t sym = ent & 0xFFFFu;
        if (ent & kEscBit) {
          sym = (uint32_t)(buf >> 48);
          buf <<= 16;
          cnt -= 16;
        }
        out[idx_cur[j]] = (uint16_t)sym;
        if (cnt < 32) {
          buf |= (uint64_t)nxt << (32 - cnt);
          cnt += 32;
          ++c;
          nxt = chunk_at(bs32, nchunks, c);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      idx_cur[j] = idx_nxt[j];
      q_cur[j] = q_nxt[j];
    }
  }
  // The next unread bit must be where the next lane's substream begins.
  if (c * 32u - (uint64_t)cnt != pos_end) flag(status, MPS_STATUS_DESYNC);
}

__device__ __forceinline__ void decode_bucket(const mps_fp8_tensor &T, int64_t b, uint32_t *lut, int32_t *s_gid,
                                              int32_t *s_rows, int *s_bad, uint32_t *status) {
  const int tid = threadIdx.x;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(T.decode_syms) & 15u) == 0) &&
                      ((reinterpret_cast<uintptr_t>(T.decode_lens) & 3u) == 0);
  if (tid == 0) *s_bad = 0;

  // fp8 byte -> table id, validated.
  for (int i = tid; i < 256; i += kBlock) {
    int32_t g = T.bucket_table[b * 256 + i];
    if (g < -1 || g >= T.num_tables) {
      flag(status, MPS_STATUS_BAD_TABLE);
      g = -1;
    }
    s_gid[i] = g;
  }
  const int32_t ra = T.bucket_row_offsets[b];
  const int32_t rb = T.bucket_row_offsets[b + 1];
  const int32_t c0 = T.bucket_col_start[b];
  const int32_t cl = T.bucket_col_len[b];
  const bool bucket_ok = ra >= 0 && rb >= ra && (int64_t)rb <= T.num_row_indices && rb - ra <= kRowsLds &&
                         cl > 0 && c0 >= 0 && (int64_t)c0 + cl <= T.m;
  const int32_t rows = bucket_ok ? rb - ra : 0;
  __syncthreads();
  for (int i = tid; i < rows; i += kBlock) {
    const int32_t r = T.row_indices[ra + i];
    if (r < 0 || r >= T.n) *s_bad = 1;
    s_rows[i] = r;
  }

  // Expand the 256 tables into 32-bit LDS entries, 8 entries per work item.
  for (int w = tid; w < 256 * (kTable / 8); w += kBlock) {
    const int f = w >> 4;
    const int part = w & 15;
    const int32_t g = s_gid[f];
    uint32_t syms[8];
    uint32_t nibs = 0;
    if (g >= 0) {
      const uint16_t *sp = T.decode_syms + (int64_t)g * kTable + part * 8;
      const uint8_t *lp = T.decode_lens + (int64_t)g * kPacked + part * 4;
      if (vec_ok) {
        const uint4 v = *reinterpret_cast<const uint4 *>(sp);
        syms[0] = v.x & 0xFFFFu; syms[1] = v.x >> 16; syms[2] = v.y & 0xFFFFu; syms[3] = v.y >> 16;
        syms[4] = v.z & 0xFFFFu; syms[5] = v.z >> 16; syms[6] = v.w & 0xFFFFu; syms[7] = v.w >> 16;
        nibs = *reinterpret_cast<const uint32_t *>(lp);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) syms[j] = sp[j];
        nibs = (uint32_t)lp[0] | ((uint32_t)lp[1] << 8) | ((uint32_t)lp[2] << 16) | ((uint32_t)lp[3] << 24);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) syms[j] = 0;
    }
    uint32_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t nib = (nibs >> (4 * j)) & 0xFu;
      e[j] = syms[j] | ((nib & 7u) << 16) | ((nib & 8u) ? kEscBit : 0u);
    }
    uint4 *dst = reinterpret_cast<uint4 *>(lut + f * kTable + part * 8);
    dst[0] = make_uint4(e[0], e[1], e[2], e[3]);
    dst[1] = make_uint4(e[4], e[5], e[6], e[7]);
  }
  __syncthreads();

  if (!bucket_ok || *s_bad) {
    if (tid == 0) flag(status, !bucket_ok ? MPS_STATUS_BAD_BUCKET : MPS_STATUS_BAD_ROW);
    return;
  }
  if (rows == 0) return;
  const int64_t total = (int64_t)rows * cl;
  const int32_t k_eff = (int32_t)(T.k < total ? T.k : total);
  const int lane = tid;
  if (lane >= k_eff) return;
  const uint32_t *sb = T.bucket_thread_startbit + b * (T.k + 1);
  const uint64_t base = (uint64_t)T.bucket_bit_base[b];
  const uint64_t pos0 = base + sb[lane];
  const uint64_t pos_end = base + sb[lane + 1];
  if ((uint64_t)T.n * (uint64_t)T.m <= 0xFFFFFFFFull)
    decode_lane<uint32_t>(T, lut, s_rows, lane, k_eff, total, c0, cl, pos0, pos_end, status);
  else
    decode_lane<uint64_t>(T, lut, s_rows, lane, k_eff, total, c0, cl, pos0, pos_end, status);
}

__global__ __launch_bounds__(kBlock) void fp8_decode_one(mps_fp8_tensor T, uint32_t *status) {
  __shared__ __attribute__((aligned(16))) uint32_t lut[256 * kTable];
  __shared__ int32_t s_gid[256];
  __shared__ int32_t s_rows[kRowsLds];
  __shared__ int s_bad;
  decode_bucket(T, blockIdx.x, lut, s_gid, s_rows, &s_bad, status);
}

__global__ __launch_bounds__(kBlock) void fp8_decode_plan(const mps_fp8_tensor *__restrict__ tensors,
                                                          const WorkItem *__restrict__ work, uint32_t *status) {
  __shared__ __attribute__((aligned(16))) uint32_t lut[256 * kTable];
  __shared__ int32_t s_gid[256];
  __shared__ int32_t s_rows[kRowsLds];
  __shared__ int s_bad;
  const WorkItem w = work[blockIdx.x];
  decode_bucket(tensors[w.tensor], w.bucket, lut, s_gid, s_rows, &s_bad, status);
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

// One 4-byte status word per device, allocated on first use and kept for the
// life of the process (it is cleared by mps_fp8_read_status).
int status_word(int device, uint32_t **out) {
  static std::mutex mu;
  static uint32_t *words[kMaxDevices] = {};
  if (device < 0 || device >= kMaxDevices) return fail(MPS_ERR_INVALID_ARGUMENT, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!words[device]) {
    int prev = 0;
    MPS_HIP_CHECK(hipGetDevice(&prev));
    if (prev != device) MPS_HIP_CHECK(hipSetDevice(device));
    uint32_t *p = nullptr;
    hipError_t e = hipMalloc(&p, 256);
    const uint32_t zero[64] = {};
    if (e == hipSuccess) e = hipMemcpy(p, zero, sizeof(zero), hipMemcpyHostToDevice);
    if (prev != device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(e, "status word allocation");
    words[device] = p;
  }
  *out = words[device];
  return MPS_OK;
}

std::string &last_error() {
  static thread_local std::string s;
  return s;
}

}  // namespace mps

using namespace mps;

struct mps_fp8_plan {
  mps_fp8_tensor *d_tensors = nullptr;
  WorkItem *d_work = nullptr;
  int64_t count = 0;
  int64_t work_items = 0;
  int device = 0;
};

extern "C" {

const char *mps_last_error(void) { return last_error().c_str(); }

int mps_clock_rate_khz(int device, int64_t *khz_out) {
  if (!khz_out) return fail(MPS_ERR_INVALID_ARGUMENT, "khz_out is NULL");
  int v = 0;
  MPS_HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeClockRate, device));
  *khz_out = v;
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
  hipLaunchKernelGGL(fp8_decode_one, dim3((unsigned)tensor->num_buckets), dim3(kBlock), 0,
                     reinterpret_cast<hipStream_t>(stream), *tensor, status);
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

int mps_fp8_plan_create(const mps_fp8_tensor *tensors, int64_t count, mps_fp8_plan **plan_out) {
  last_error().clear();
  if (!plan_out) return fail(MPS_ERR_INVALID_ARGUMENT, "plan_out is NULL");
  *plan_out = nullptr;
  if (count < 0 || (count > 0 && !tensors)) return fail(MPS_ERR_INVALID_ARGUMENT, "invalid tensor list");
  std::vector<WorkItem> work;
  for (int64_t i = 0; i < count; ++i) {
    int rc = check_tensor(&tensors[i]);
    if (rc != MPS_OK) return rc;
    for (int64_t b = 0; b < tensors[i].num_buckets; ++b) work.push_back({(int32_t)i, (int32_t)b});
  }
  if (work.size() > (size_t)INT32_MAX) return fail(MPS_ERR_INVALID_ARGUMENT, "too many buckets for one plan");
  auto *p = new mps_fp8_plan();
  p->count = count;
  p->work_items = (int64_t)work.size();
  hipError_t e = hipGetDevice(&p->device);
  if (e == hipSuccess && count > 0) e = hipMalloc(&p->d_tensors, sizeof(mps_fp8_tensor) * count);
  if (e == hipSuccess && !work.empty()) e = hipMalloc(&p->d_work, sizeof(WorkItem) * work.size());
  if (e == hipSuccess && count > 0)
    e = hipMemcpy(p->d_tensors, tensors, sizeof(mps_fp8_tensor) * count, hipMemcpyHostToDevice);
  if (e == hipSuccess && !work.empty())
    e = hipMemcpy(p->d_work, work.data(), sizeof(WorkItem) * work.size(), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    if (p->d_tensors) (void)hipFree(p->d_tensors);
    if (p->d_work) (void)hipFree(p->d_work);
    delete p;
    return hip_fail(e, "mps_fp8_plan_create");
  }
  *plan_out = p;
  return MPS_OK;
}

int mps_fp8_plan_decode(mps_fp8_plan *plan, void *stream) {
  last_error().clear();
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (plan->work_items == 0) return MPS_OK;
  uint32_t *status = nullptr;
  int rc = status_word(plan->device, &status);
  if (rc != MPS_OK) return rc;
  hipLaunchKernelGGL(fp8_decode_plan, dim3((unsigned)plan->work_items), dim3(kBlock), 0,
                     reinterpret_cast<hipStream_t>(stream), plan->d_tensors, plan->d_work, status);
  MPS_HIP_CHECK(hipGetLastError());
  return MPS_OK;
}

int mps_fp8_plan_info(const mps_fp8_plan *plan, int64_t *work_items, int64_t *lds_bytes) {
  if (!plan) return fail(MPS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (work_items) *work_items = plan->work_items;
  if (lds_bytes) *lds_bytes = (int64_t)(256 * kTable * 4 + 256 * 4 + kRowsLds * 4);
  return MPS_OK;
}

int mps_fp8_plan_destroy(mps_fp8_plan *plan) {
  if (!plan) return MPS_OK;
  if (plan->d_tensors) (void)hipFree(plan->d_tensors);
  if (plan->d_work) (void)hipFree(plan->d_work);
  delete plan;
  return MPS_OK;
}

int mps_fp8_read_status(int device, void *stream, uint32_t *status_out) {
  last_error().clear();
  if (!status_out) return fail(MPS_ERR_INVALID_ARGUMENT, "status_out is NULL");
  uint32_t *word = nullptr;
  int rc = status_word(device, &word);
  if (rc != MPS_OK) return rc;
  int prev = 0;
  MPS_HIP_CHECK(hipGetDevice(&prev));
  if (prev != device) MPS_HIP_CHECK(hipSetDevice(device));
  uint32_t v = 0;
  const uint32_t zero = 0;
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e == hipSuccess) e = hipMemcpy(&v, word, sizeof(v), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice);
  if (prev != device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, "mps_fp8_read_status");
  *status_out = v;
  return MPS_OK;
}

}  // extern "C"
