/*
 * mpserve_amd — MI355X (gfx950) FP8 + Huffman-sidecar weight path, C ABI.
 *
 * Plain pointers and sizes only. Every pointer named "device" is HIP device
 * memory on the current device; host pointers are named so. All entry points
 * return MPS_OK (0) or a negative MPS_ERR_* code; mps_last_error() gives the
 * message of the last failure on the calling thread.
 *
 * Sidecar format: the one MPServe's builder writes
 * (reference kernel/build_huffman.cu:292-969, scripts/compress_llm_fp8_huffman.py:284-306).
 */
#ifndef MPSERVE_AMD_H
#define MPSERVE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MPS_OK 0
#define MPS_ERR_INVALID_ARGUMENT (-1) /* maps to Python ValueError (std::invalid_argument in the reference) */
#define MPS_ERR_RUNTIME (-2)          /* maps to Python RuntimeError */
#define MPS_ERR_HIP (-3)              /* a HIP runtime call failed */
#define MPS_ERR_NO_MEMORY (-4)

/* Device-side integrity flags a decode records (see mps_fp8_read_status). */
#define MPS_STATUS_BAD_BUCKET 0x1u   /* row range / column range outside the tensor */
#define MPS_STATUS_BAD_ROW 0x2u      /* a row index outside [0, n) */
#define MPS_STATUS_BAD_TABLE 0x4u    /* a bucket_table gid outside [-1, G) */
#define MPS_STATUS_DESYNC 0x8u       /* a lane ended at a bit other than the next lane's start */

/* One FP8 tensor and its sidecar, all device pointers, as stored by the
 * reference's compress script (huff_* tensors) with the decode call's dtype
 * views (reference scripts/mpserve_vllm_fp8_huffman.py:457-472). */
typedef struct mps_fp8_tensor {
  const uint8_t *fp8;                    /* [n*m]            huff_fp8_u8 */
  const uint64_t *bitstream;             /* [bitstream_words] huff_bitstream_u64 */
  int64_t bitstream_words;
  const uint16_t *decode_syms;           /* [num_tables,128] huff_decode_syms_u16 */
  const uint8_t *decode_lens;            /* [num_tables,64]  huff_decode_lens_u8 (packed 4-bit) */
  int64_t num_tables;
  const int32_t *bucket_table;           /* [num_buckets,256] fp8 byte -> table id or -1 */
  const int32_t *bucket_col_start;       /* [num_buckets] */
  const int32_t *bucket_col_len;         /* [num_buckets] */
  const int32_t *bucket_row_offsets;     /* [num_buckets+1] into row_indices */
  const int32_t *row_indices;            /* [num_row_indices] */
  int64_t num_row_indices;
  const uint32_t *bucket_thread_startbit;/* [num_buckets, k+1] lane start bits, relative */
  const int64_t *bucket_bit_base;        /* [num_buckets+1] bucket base bits (64-aligned) */
  int64_t num_buckets;
  int64_t k;                             /* substreams (lanes) per bucket, 1..1024 */
  int64_t n, m;                          /* output shape [n, m] */
  uint16_t *out;                         /* [n*m] BF16 bit patterns (device) */
} mps_fp8_tensor;

/* Message of the last failed call on this thread ("" if none). */
const char *mps_last_error(void);

/* HIP clock rate (kHz) of `device`.
 * Replaces MPServe_cuda.cuda_clock_rate_khz (reference kernel/wrapper.cpp:133-141). */
int mps_clock_rate_khz(int device, int64_t *khz_out);

/* Decode one tensor: out[n,m] = BF16 rebuilt from FP8 bytes + sidecar, on `stream`
 * (a hipStream_t; NULL = the legacy default stream). Lossless: reads the raw
 * 16 bits after ESC codes, and walks columns as e % col_len.
 * Replaces huffman_cpp::huffman_decode_fp8_entry (reference kernel/decode_huffman.cu:591-758,
 * bound as MPServe_cuda.huffman_decode_fp8 at kernel/wrapper.cpp:456-503); the
 * shape/dtype checks of that entry are done by the caller, which knows dtypes.
 * max_len must be 7. Asynchronous: returns after the launch. */
int mps_fp8_decode(const mps_fp8_tensor *tensor, int64_t max_len, void *stream);

/* Batched decode plan: one launch decodes many tensors (a layer, a model).
 * Creation first synchronises `stream` (the caller's stream, which may still
 * be writing the sidecars), then reads each tensor's bucket row offsets,
 * column ranges and bit bases to order the work largest first and to build
 * one work record per bucket, and copies the descriptors into one device
 * allocation the plan owns (with its own status word). When the buckets are
 * few or uneven for the device's CUs, large buckets are split into row
 * ranges: a kernel on `stream` walks their substreams' code lengths once and
 * records each substream's bit position at every range's first row (the lane
 * checkpoints, also owned by the plan). A sidecar whose bucket metadata, row
 * indices, start bits, tables, FP8 bytes or bitstream is rewritten needs a
 * new plan in that case. The pointed-to sidecars must stay alive while the
 * plan is used. Launches are persistent: one workgroup per CU takes work
 * items from a queue in the plan's memory, which each launch leaves as it
 * found it. The plan holds 32 such queues and gives each stream that launches
 * it (mps_fp8_plan_decode and mps_fp8_plan_decode_into alike) its own at the
 * stream's first launch, so launches on different streams may overlap, and a
 * launch captured into a graph replays with the queue of the stream it was
 * captured on (a replay must then not overlap an eager launch on that same
 * stream). A 33rd stream is refused with MPS_ERR_RUNTIME. Decodes are
 * asynchronous on their stream and OR their MPS_STATUS_* flags into the
 * plan's status word (mps_fp8_plan_read_status).
 * No counterpart in the reference, which launches once per tensor
 * (kernel/decode_huffman.cu:739); it serves its apply() and model loading paths
 * (scripts/mpserve_vllm_fp8_huffman.py:491-557). */
typedef struct mps_fp8_plan mps_fp8_plan;
int mps_fp8_plan_create(const mps_fp8_tensor *tensors, int64_t count, void *stream, mps_fp8_plan **plan_out);
int mps_fp8_plan_decode(mps_fp8_plan *plan, void *stream);
/* Decode the plan into a buffer laid out like the outputs it was created
 * with, moved to `out`: every tensor's output moves by (out - the first
 * tensor's output at creation), in BF16 elements. A plan of one tensor decodes
 * into any n*m buffer; a plan whose tensors' outputs are row slices of one
 * weight decodes into any buffer of that weight's size. The flags go to the
 * device status word (mps_fp8_read_status), as a single-tensor decode's do.
 * This serves the drop-in decode op's per-sidecar plan cache and the vLLM
 * method's scratch slots. */
int mps_fp8_plan_decode_into(mps_fp8_plan *plan, uint16_t *out, void *stream);
/* The plan's work list (for profiling tools): work items (buckets, and the row
 * ranges of the buckets it split), bytes of LDS per workgroup. */
int mps_fp8_plan_info(const mps_fp8_plan *plan, int64_t *work_items, int64_t *lds_bytes);
/* Read and clear the plan's MPS_STATUS_* flags; synchronises `stream` first. */
int mps_fp8_plan_read_status(mps_fp8_plan *plan, void *stream, uint32_t *status_out);
int mps_fp8_plan_destroy(mps_fp8_plan *plan);

/* Allocation-free batched decode: decodes `count` tensors (at most 1024, with
 * at most 63,100 buckets in all) in one persistent launch, as a plan would,
 * but without creating one. It calls no hipMalloc, hipFree or other
 * allocating routine and does not synchronise: the descriptors (copied from
 * the host array on `stream`) and one work record per bucket go into a static
 * device array of 4 MiB that each device holds from library load to the end
 * of the process. Buckets are not split into row ranges. Flags go to the
 * device status word (mps_fp8_read_status). Calls that overlap on one device
 * share that array and race: issue them on one stream, or order them.
 * Larger inputs, and a `stream` that is capturing a graph (the descriptor
 * copy would replay from a host array that is gone), are rejected with
 * MPS_ERR_INVALID_ARGUMENT before any copy or launch.
 * No counterpart in the reference; it serves callers that cannot allocate
 * device memory in their decode loop (tight serving loops, harnesses that
 * forbid allocation). Code under graph capture launches a plan made before
 * the capture instead. */
int mps_fp8_decode_batch_noalloc(const mps_fp8_tensor *tensors, int64_t count, int64_t max_len, void *stream);

/* Capture id of `stream`: the id of the graph capture it is in, or 0 when it
 * is not capturing (hipStreamGetCaptureInfo). No counterpart in the
 * reference: the vLLM method uses it to tell a captured forward pass from an
 * eager one, so that a packed block's decoded weight is reused only within
 * one of them. */
int mps_stream_capture_id(void *stream, uint64_t *id_out);

/* Inputs of the GPU sidecar builder, all device pointers: BF16 bit patterns
 * and FP8 bytes of the same tensor (`numel` elements, shape dims[0..ndim)),
 * and the u16 scale keys (shape scale_dims[0..scale_ndim), scale_numel
 * values). */
typedef struct mps_fp8_encode_in {
  const uint16_t *bf16;
  const uint8_t *fp8;
  const uint16_t *scales;
  int64_t numel;
  int32_t ndim;
  int32_t scale_ndim;
  int64_t dims[8];
  int64_t scale_dims[8];
  int64_t scale_numel;
  int64_t max_len;           /* 1..15 (decoding needs 7) */
  int64_t threads_per_block; /* k: substreams per bucket, 1..1024 */
} mps_fp8_encode_in;

/* Build the Huffman sidecar of one tensor on the GPU, byte-identical to the
 * reference builder. Replaces huffman_cpp::huffman_build_fp8_decode_tables_entry
 * (reference kernel/build_huffman.cu:292-969, bound as
 * MPServe_cuda.huffman_build_fp8_decode_tables at kernel/wrapper.cpp:418-454),
 * which runs single-threaded on the host; same argument checks and messages.
 * Synchronises `stream` (output sizes are data dependent). The result lives in
 * device memory owned by the returned handle. */
typedef struct mps_fp8_sidecar mps_fp8_sidecar;
int mps_fp8_encode(const mps_fp8_encode_in *in, void *stream, mps_fp8_sidecar **out);
/* One AWQ int4 tensor and its sidecar, all device pointers, in either layout
 * of the reference's AWQ int4 builders (dtype views as for the FP8 tensor). */
typedef struct mps_awq_tensor {
  const uint8_t *int4;                   /* [n*m] int4 values, one per byte (low nibble) */
  const uint64_t *bitstream;             /* [bitstream_words] */
  int64_t bitstream_words;
  const uint16_t *decode_syms;           /* [num_tables,2048] */
  const uint8_t *decode_lens;            /* [num_tables,1024] packed 4-bit, 15 = ESC */
  int64_t num_tables;
  const int32_t *bucket_table;           /* [num_buckets,16] int4 value -> table id or -1 */
  const int32_t *bucket_col_start;       /* row layout: [num_buckets]; by-scale layout: NULL */
  const int32_t *bucket_col_len;         /* row layout: [num_buckets]; by-scale layout: NULL */
  const int32_t *bucket_row_offsets;     /* [num_buckets+1] bucket_row_offsets / bucket_group_offsets */
  const int32_t *row_indices;            /* [num_row_indices] row_indices / group_rows */
  int64_t num_row_indices;
  const int32_t *group_col_start;        /* by-scale layout: [num_row_indices]; row layout: NULL */
  int64_t group_size;                    /* by-scale layout: columns per group */
  const uint32_t *bucket_thread_startbit;/* [num_buckets, k+1] */
  const int64_t *bucket_bit_base;        /* [num_buckets+1] */
  int64_t num_buckets;
  int64_t k;                             /* 1..1024 */
  int64_t n, m;                          /* output shape [n, m], n*m < 2^31 */
  uint16_t *out;                         /* [n*m] BF16 bit patterns (device) */
} mps_awq_tensor;

/* Decode one AWQ int4 tensor: out[n,m] = BF16 rebuilt from int4 values + sidecar,
 * on `stream`. Replaces huffman_cpp::huffman_decode_awq_int4_bucket_entry
 * (group_col_start == NULL; reference kernel/decode_huffman.cu:877-1018 and
 * :378-475, bound at kernel/wrapper.cpp:324-369) and
 * ..._by_scale_entry (group_col_start != NULL; kernel/decode_huffman.cu:760-875
 * and :477-589, bound at kernel/wrapper.cpp:371-416). The shape/dtype checks
 * of those entries are done by the caller. max_len must be 11. Columns of a
 * row bucket are walked as e % col_len, as the builder lays them out.
 * Asynchronous: returns after the launch. */
int mps_awq_decode(const mps_awq_tensor *tensor, int64_t max_len, void *stream);

/* Batched AWQ decode plan: one launch decodes every bucket of many AWQ int4
 * tensors (either layout, mixed), largest work first. Runs of up to 1024 / k
 * consecutive buckets with identical table ids share one workgroup and its
 * tables. Creation synchronises `stream` first, then reads each tensor's
 * bucket row offsets, table ids (and column lengths) once and copies the
 * descriptors into one device allocation the plan owns (with its own status
 * word, mps_awq_plan_read_status); the pointed-to tensors must stay alive
 * while the plan is used, and a tensor whose bucket metadata is rewritten
 * needs a new plan. Decodes are asynchronous on `stream`. A launch runs one
 * workgroup per CU that takes the plan's work records from a queue in the
 * plan's memory; the plan holds 32 such queues and gives each stream that
 * launches it its own (a 33rd stream is refused with MPS_ERR_RUNTIME), so
 * launches on different streams may overlap. A graph replays with the queue
 * of the stream it was captured on.
 * No counterpart in the reference, which launches once per tensor
 * (kernel/decode_huffman.cu:857, :998). */
typedef struct mps_awq_plan mps_awq_plan;
int mps_awq_plan_create(const mps_awq_tensor *tensors, int64_t count, void *stream, mps_awq_plan **plan_out);
int mps_awq_plan_decode(mps_awq_plan *plan, void *stream);
/* Decode the plan into a buffer laid out like its outputs, moved to `out`, as
 * mps_fp8_plan_decode_into does (the move must keep 8-byte alignment); the
 * flags go to the device status word. No counterpart in the reference: it
 * serves the AWQ decode ops' per-sidecar plan cache. */
int mps_awq_plan_decode_into(mps_awq_plan *plan, uint16_t *out, void *stream);
int mps_awq_plan_info(const mps_awq_plan *plan, int64_t *work_items);
int mps_awq_plan_read_status(mps_awq_plan *plan, void *stream, uint32_t *status_out);
int mps_awq_plan_destroy(mps_awq_plan *plan);

/* Inputs of the AWQ int4 sidecar builders, all device pointers: BF16 bit
 * patterns and int4 values (one per byte, low nibble) of an [n, m] weight, and
 * the u16 (BF16 bit) scales: one value, [n] (scale_ndim 1) or block-wise
 * [n/bs0, m/bs1] (scale_ndim 2). by_scale = 0 builds row buckets, 1 builds
 * buckets of quantisation groups of one exact scale (at most group_cap each). */
typedef struct mps_awq_encode_in {
  const uint16_t *bf16;
  const uint8_t *int4;
  const uint16_t *scales;
  int64_t n, m;
  int32_t scale_ndim;
  int32_t by_scale;
  int64_t scale_dims[2];
  int64_t scale_numel;
  int64_t max_len;           /* 1..15 (decoding needs 11) */
  int64_t threads_per_block; /* k: substreams per bucket, 1..1024 */
  int64_t group_cap;         /* by_scale: groups per bucket, > 0 */
} mps_awq_encode_in;

/* Build the AWQ int4 sidecar of one weight on the GPU, byte-identical to the
 * reference builders, which run single-threaded on the host:
 *   by_scale = 0: huffman_cpp::huffman_build_awq_int4_bucket_decode_tables_entry
 *     (reference kernel/build_huffman.cu:1583-2126, bound as
 *     MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables at kernel/wrapper.cpp:258-288);
 *   by_scale = 1: ..._by_scale_entry (kernel/build_huffman.cu:1075-1580, bound as
 *     MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables_by_scale at kernel/wrapper.cpp:290-321).
 * Same argument checks and messages. The result uses the FP8 handle's 17
 * slots: slots 0-13 in the reference's order of the row-bucket dict (slot 3 is
 * table_qv_u16, slot 7 bucket_table_i32 [B,16]); by scale, slot 5 holds
 * bucket_group_offsets_i32, slot 6 group_rows_i32, slot 8 group_col_start_i32
 * and slot 13 shape_nmkg_i64 (slot 9 is empty). Slots 14-16 are empty. */
int mps_awq_encode(const mps_awq_encode_in *in, void *stream, mps_fp8_sidecar **out);

/* Element counts of the 17 outputs, in the reference's order (kernel/wrapper.cpp:429-446):
 * decode_syms_u16, decode_lens_u8, table_scale_u16, table_fp8_u16, bucket_scale_u16,
 * bucket_row_offsets_i32, row_indices_i32, bucket_table_i32, bucket_col_start_i32,
 * bucket_col_len_i32, bucket_thread_startbit_u32, bucket_bit_base_i64, bitstream_u64,
 * shape_nmk_i64, bucket_U_i32, bucket_unique_gid_i32, bucket_fp8_uidx_i16. */
int mps_fp8_sidecar_sizes(const mps_fp8_sidecar *sc, int64_t *sizes17);
/* Copy the 17 outputs into caller buffers (host or device; hipMemcpyDefault); synchronises. */
int mps_fp8_sidecar_copy(const mps_fp8_sidecar *sc, void *const *dst17, void *stream);
/* {keys coded with ESC, elements equal to their key's esc_sym, distinct (key, symbol) pairs, hash slots}. */
int mps_fp8_sidecar_stats(const mps_fp8_sidecar *sc, int64_t *stats4);
int mps_fp8_sidecar_free(mps_fp8_sidecar *sc);

/* Read and clear the MPS_STATUS_* flags the single-tensor decodes
 * (mps_fp8_decode, mps_awq_decode, mps_fp8_plan_decode_into) on `device`
 * recorded since the last call. The word is per device, not per stream:
 * flags of decodes on any stream of the device accumulate in it. It is a
 * module global of the library (no allocation). Synchronises `stream` first. */
int mps_fp8_read_status(int device, void *stream, uint32_t *status_out);

#ifdef __cplusplus
}
#endif

#endif /* MPSERVE_AMD_H */
