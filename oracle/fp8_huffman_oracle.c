/*
 * CPU restatement of MPServe's FP8 + Huffman-sidecar path. TEST INFRASTRUCTURE ONLY.
 *
 * This file is the parity oracle: tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may call it, as the checker. The product
 * (mpserve_amd) never links, loads or calls it.
 *
 * It restates, in plain C with no hashing containers, what the reference does:
 *   encoder  kernel/build_huffman.cu:292-969  (huffman_build_fp8_decode_tables_entry)
 *     histogram          :392-401     key = scale_u16<<16 | fp8, symbol = bf16 bits
 *     key order / gid    :403-412
 *     per-key items      :453-478     (count asc, sym asc)
 *     ESC selection      :485-535
 *     package-merge      :46-118
 *     canonical codes    :171-203     codes handed out in items order
 *     LUT fill + pack    :205-239, single-symbol case :464-472
 *     row bucketing      :611-656, block-2D bucketing :657-696
 *     bucket_table / U   :737-783
 *     bitstream          :786-925     MSB-first, 64-bit aligned bucket bases
 *   decoder  kernel/decode_huffman.cu:188-372 (semantics; the oracle is lossless:
 *     it reads the 16 raw bits after an ESC code, which the reference kernel
 *     skips at :348-353, and walks columns as e % col_len like the encoder at
 *     build_huffman.cu:837-841). Mode ORC_DECODE_REFERENCE_KERNEL reproduces the
 *     reference kernel's own walk (single row wrap, ESC ignored) for the lanes
 *     where that kernel stays in bounds.
 *
 * Parity pinning of each function is described in the header of oracle/__init__.py.
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_INVALID_ARGUMENT 1
#define ORC_RUNTIME_ERROR 2
#define ORC_NO_MEMORY 3

#define ORC_DECODE_LOSSLESS 0
#define ORC_DECODE_REFERENCE_KERNEL 1

typedef struct orc_sidecar {
  /* per-key tables */
  int64_t G;
  int64_t table_size;      /* 2^L */
  int64_t packed_len_size; /* 2^(L-1) */
  uint16_t *decode_syms;   /* [G, 2^L] */
  uint8_t *decode_lens;    /* [G, 2^(L-1)] */
  uint16_t *table_scale;   /* [G] */
  uint16_t *table_fp8;     /* [G] */
  /* buckets */
  int64_t B;
  uint16_t *bucket_scale;        /* [B] */
  int32_t *bucket_row_offsets;   /* [B+1] */
  int64_t R;
  int32_t *row_indices;          /* [R] */
  int32_t *bucket_table;         /* [B,256] */
  int32_t *bucket_col_start;     /* [B] */
  int32_t *bucket_col_len;       /* [B] */
  int64_t k;
  uint32_t *bucket_thread_startbit; /* [B,k+1] */
  int64_t *bucket_bit_base;      /* [B+1] */
  int64_t W;
  uint64_t *bitstream;           /* [W] */
  int64_t shape_nmk[3];
  int32_t *bucket_U;             /* [B] */
  int32_t *bucket_unique_gid;    /* [B,256] */
  int16_t *bucket_fp8_uidx;      /* [B,256] */
  /* diagnostics (not part of the reference output) */
  int64_t esc_keys;              /* keys coded with an ESC symbol */
  int64_t esc_collisions;        /* elements whose symbol equals its key's esc_sym but was not kept */
  int64_t esc_elements;          /* elements emitted as ESC + raw16 */
} orc_sidecar;

static char g_err[512];

const char *orc_last_error(void) { return g_err; }

static int set_err(int code, const char *msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

void orc_free(orc_sidecar *s) {
  if (!s) return;
  free(s->decode_syms); free(s->decode_lens); free(s->table_scale); free(s->table_fp8);
  free(s->bucket_scale); free(s->bucket_row_offsets); free(s->row_indices); free(s->bucket_table);
  free(s->bucket_col_start); free(s->bucket_col_len); free(s->bucket_thread_startbit);
  free(s->bucket_bit_base); free(s->bitstream); free(s->bucket_U); free(s->bucket_unique_gid);
  free(s->bucket_fp8_uidx);
  free(s);
}

/* ------------------------------------------------------------------------- */
/* Package-merge, restated from build_huffman.cu:46-118.                     */
/* weights must be sorted ascending (the caller's items are). Leaf ties are  */
/* resolved leaf-first in each merge (build_huffman.cu:81). Package weights  */
/* are summed in 32-bit two's complement, as the reference's int sums are on */
/* the x86-64 targets it is built for.                                       */
/* Returns 0, or an ORC_* error.                                             */
/* ------------------------------------------------------------------------- */
typedef struct { int32_t w; int32_t ref; } pm_item;

int orc_package_merge(const int32_t *weights_in, int n, int L, int32_t *lens_out) {
  if (L <= 0 || L > 30) return set_err(ORC_INVALID_ARGUMENT, "max_len must be in (0, 30]");
  if (n == 0) return ORC_OK;
  if (n == 1) { lens_out[0] = 1; return ORC_OK; }
  if ((int64_t)n > ((int64_t)1 << L)) return set_err(ORC_INVALID_ARGUMENT, "Too many symbols for max_len");

  /* stable sort of the weights: insertion sort keeps equal weights in order */
  int32_t *w = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
  if (!w) return set_err(ORC_NO_MEMORY, "out of memory");
  memcpy(w, weights_in, sizeof(int32_t) * (size_t)n);
  for (int i = 1; i < n; ++i) {
    int32_t v = w[i]; int j = i - 1;
    while (j >= 0 && w[j] > v) { w[j + 1] = w[j]; --j; }
    w[j + 1] = v;
  }

  const int K = 2 * (n - 1);
  const int keep = 2 * K;
  /* package node p has id n+p and children pl[p], pr[p] (leaf ids < n) */
  const int max_pk = (L > 1 ? (L - 1) : 1) * keep + 1;
  int32_t *pl = (int32_t *)malloc(sizeof(int32_t) * (size_t)max_pk);
  int32_t *pr = (int32_t *)malloc(sizeof(int32_t) * (size_t)max_pk);
  pm_item *cur = (pm_item *)malloc(sizeof(pm_item) * (size_t)(keep + n));
  pm_item *nxt = (pm_item *)malloc(sizeof(pm_item) * (size_t)(keep + n));
  pm_item *pk = (pm_item *)malloc(sizeof(pm_item) * (size_t)(keep + n));
  int32_t *stack = (int32_t *)malloc(sizeof(int32_t) * (size_t)(2 * max_pk + 8));
  if (!pl || !pr || !cur || !nxt || !pk || !stack) {
    free(w); free(pl); free(pr); free(cur); free(nxt); free(pk); free(stack);
    return set_err(ORC_NO_MEMORY, "out of memory");
  }
  int npk = 0;
  int ncur = n < keep ? n : keep;
  for (int i = 0; i < ncur; ++i) { cur[i].w = w[i]; cur[i].ref = i; }

  for (int round = 0; round < L - 1; ++round) {
    int t = ncur < keep ? ncur : keep;
    int np = 0;
    for (int i = 0; i + 1 < t; i += 2) {
      pl[npk] = cur[i].ref; pr[npk] = cur[i + 1].ref;
      pk[np].w = (int32_t)((uint32_t)cur[i].w + (uint32_t)cur[i + 1].w);
      pk[np].ref = n + npk;
      ++npk; ++np;
    }
    /* merge leaves (w[0..n)) with packages, leaf first on ties, cap at keep */
    int a = 0, b = 0, o = 0;
    while (o < keep && a < n && b < np) {
      if (w[a] <= pk[b].w) { nxt[o].w = w[a]; nxt[o].ref = a; ++a; }
      else { nxt[o] = pk[b]; ++b; }
      ++o;
    }
    while (o < keep && a < n) { nxt[o].w = w[a]; nxt[o].ref = a; ++a; ++o; }
    while (o < keep && b < np) { nxt[o] = pk[b]; ++b; ++o; }
    pm_item *tmp = cur; cur = nxt; nxt = tmp; ncur = o;
  }
  int rc = ORC_OK;
  if (ncur < K) {
    rc = set_err(ORC_RUNTIME_ERROR, "Internal error: not enough packages");
  } else {
    for (int i = 0; i < n; ++i) lens_out[i] = 0;
    for (int i = 0; i < K; ++i) {
      int sp = 0; stack[sp++] = cur[i].ref;
      while (sp > 0) {
        int r = stack[--sp];
        if (r < n) { lens_out[r]++; continue; }
        stack[sp++] = pl[r - n];
        stack[sp++] = pr[r - n];
      }
    }
  }
  free(w); free(pl); free(pr); free(cur); free(nxt); free(pk); free(stack);
  return rc;
}

/* ------------------------------------------------------------------------- */
/* Sorting helpers                                                            */
/* ------------------------------------------------------------------------- */
typedef struct { int32_t count; uint16_t sym; } orc_item;

static int item_cmp_asc(const void *pa, const void *pb) {
  const orc_item *a = (const orc_item *)pa, *b = (const orc_item *)pb;
  if (a->count != b->count) return a->count < b->count ? -1 : 1;
  return (int)a->sym - (int)b->sym;
}
static int item_cmp_desc(const void *pa, const void *pb) {
  const orc_item *a = (const orc_item *)pa, *b = (const orc_item *)pb;
  if (a->count != b->count) return a->count > b->count ? -1 : 1;
  return (int)a->sym - (int)b->sym;
}

/* LSD radix sort of 64-bit values on their low `bits` bits, 16 bits a pass. */
static int radix_sort_u64(uint64_t *v, int64_t n, int bits) {
  uint64_t *tmp = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(n > 0 ? n : 1));
  int64_t *cnt = (int64_t *)malloc(sizeof(int64_t) * 65536);
  if (!tmp || !cnt) { free(tmp); free(cnt); return -1; }
  uint64_t *src = v, *dst = tmp;
  for (int sh = 0; sh < bits; sh += 16) {
    memset(cnt, 0, sizeof(int64_t) * 65536);
    for (int64_t i = 0; i < n; ++i) cnt[(src[i] >> sh) & 0xFFFF]++;
    int64_t acc = 0;
    for (int d = 0; d < 65536; ++d) { int64_t c = cnt[d]; cnt[d] = acc; acc += c; }
    for (int64_t i = 0; i < n; ++i) dst[cnt[(src[i] >> sh) & 0xFFFF]++] = src[i];
    uint64_t *t = src; src = dst; dst = t;
  }
  if (src != v) memcpy(v, src, sizeof(uint64_t) * (size_t)n);
  free(tmp); free(cnt);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Encoder                                                                    */
/* ------------------------------------------------------------------------- */
typedef struct { uint16_t scale; int32_t row_start, row_count, col_start, col_len; } orc_bucket;

/* per-element code word: bits 0..15 code, 16..20 len, bit 24: append raw16 */
#define CW_RAW (1u << 24)

int orc_encode(const uint16_t *bf16, const uint8_t *fp8, int64_t numel,
               int ndim, const int64_t *dims,
               const uint16_t *scales, int64_t scale_numel, int scale_ndim, const int64_t *scale_dims,
               int64_t max_len, int64_t threads_per_block, orc_sidecar **out) {
  *out = NULL;
  g_err[0] = 0;
  /* validation: build_huffman.cu:298-366 */
  if (max_len <= 0 || max_len > 15) return set_err(ORC_INVALID_ARGUMENT, "max_len must be in [1, 15]");
  if (threads_per_block <= 0 || threads_per_block > 1024)
    return set_err(ORC_INVALID_ARGUMENT, "threads_per_block must be in [1, 1024]");
  const int L = (int)max_len;
  const int scale_scalar = (scale_numel == 1);
  const int scale_per_elem = (scale_numel == numel);
  int scale_per_row = 0, scale_block2d = 0;
  int64_t n_rows = -1, n_cols = -1, sb0 = -1, sb1 = -1, nb0 = -1, nb1 = -1;
  if (!scale_scalar && !scale_per_elem && ndim == 2) {
    n_rows = dims[0]; n_cols = dims[1];
    scale_per_row = (scale_numel == n_rows);
    if (!scale_per_row && scale_ndim == 2) {
      nb0 = scale_dims[0]; nb1 = scale_dims[1];
      if (nb0 > 0 && nb1 > 0 && (n_rows % nb0 == 0) && (n_cols % nb1 == 0)) {
        sb0 = n_rows / nb0; sb1 = n_cols / nb1;
        if (sb0 > 0 && sb1 > 0) scale_block2d = 1;
      }
    }
  }
  if (!scale_scalar && !scale_per_elem && !scale_per_row && !scale_block2d)
    return set_err(ORC_INVALID_ARGUMENT,
                   "unsupported scales shape: use scalar, per-row (n,), per-element (numel), or 2D block-wise [n/bs0,m/bs1]");

  /* scale of flat element i: build_huffman.cu:368-390 */
#define SCALE_OF(i) (scale_scalar ? scales[0] : scale_per_elem ? scales[(i)] : \
    scale_block2d ? scales[(((i) / n_cols) / sb0) * nb1 + (((i) % n_cols) / sb1)] : scales[(i) / n_cols])

  /* histogram: build_huffman.cu:392-401, as a sort of (key<<16 | sym) */
  uint64_t *comp = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(numel > 0 ? numel : 1));
  if (!comp) return set_err(ORC_NO_MEMORY, "out of memory");
  for (int64_t i = 0; i < numel; ++i) {
    uint64_t key = ((uint64_t)SCALE_OF(i) << 16) | fp8[i];
    comp[i] = (key << 16) | bf16[i];
  }
  if (radix_sort_u64(comp, numel, 48)) { free(comp); return set_err(ORC_NO_MEMORY, "out of memory"); }
  int64_t D = 0;
  for (int64_t i = 0; i < numel; ++i) if (i == 0 || comp[i] != comp[i - 1]) ++D;
  uint64_t *ucomp = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(D + 1));
  uint32_t *ucount = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(D + 1));
  uint32_t *ucode = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(D + 1));
  if (!ucomp || !ucount || !ucode) { free(comp); free(ucomp); free(ucount); free(ucode); return set_err(ORC_NO_MEMORY, "out of memory"); }
  {
    int64_t d = -1;
    for (int64_t i = 0; i < numel; ++i) {
      if (i == 0 || comp[i] != comp[i - 1]) { ++d; ucomp[d] = comp[i]; ucount[d] = 0; }
      ucount[d]++;
    }
  }
  free(comp);

  /* keys ascending -> gid: build_huffman.cu:403-412 */
  int64_t G = 0;
  for (int64_t d = 0; d < D; ++d) if (d == 0 || (ucomp[d] >> 16) != (ucomp[d - 1] >> 16)) ++G;
  int64_t *key_first = (int64_t *)malloc(sizeof(int64_t) * (size_t)(G + 1));
  uint32_t *keys = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(G + 1));
  orc_sidecar *s = (orc_sidecar *)calloc(1, sizeof(orc_sidecar));
  const int64_t table_size = (int64_t)1 << L;
  const int64_t packed = table_size / 2 > 0 ? table_size / 2 : 0;
  int rc = ORC_OK;
  uint8_t *unpacked = NULL;
  orc_item *items = NULL, *rebuilt = NULL;
  int32_t *wts = NULL, *lens = NULL;
  uint16_t *esc_sym_of = NULL;
  uint8_t *use_esc_of = NULL;
  if (!key_first || !keys || !s) { rc = set_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
  {
    int64_t g = -1;
    for (int64_t d = 0; d < D; ++d) {
      if (d == 0 || (ucomp[d] >> 16) != (ucomp[d - 1] >> 16)) { ++g; key_first[g] = d; keys[g] = (uint32_t)(ucomp[d] >> 16); }
    }
    key_first[G] = D;
  }
  s->G = G; s->table_size = table_size; s->packed_len_size = packed;
  s->decode_syms = (uint16_t *)calloc((size_t)(G * table_size + 1), sizeof(uint16_t));
  s->decode_lens = (uint8_t *)calloc((size_t)(G * packed + 1), 1);
  s->table_scale = (uint16_t *)calloc((size_t)G + 1, sizeof(uint16_t));
  s->table_fp8 = (uint16_t *)calloc((size_t)G + 1, sizeof(uint16_t));
  unpacked = (uint8_t *)malloc((size_t)table_size);
  esc_sym_of = (uint16_t *)calloc((size_t)G + 1, sizeof(uint16_t));
  use_esc_of = (uint8_t *)calloc((size_t)G + 1, 1);
  if (!s->decode_syms || !s->decode_lens || !s->table_scale || !s->table_fp8 || !unpacked || !esc_sym_of || !use_esc_of) {
    rc = set_err(ORC_NO_MEMORY, "out of memory"); goto fail;
  }

  /* per-key code books: build_huffman.cu:445-578 */
  {
    int64_t max_items = 1;
    for (int64_t g = 0; g < G; ++g) {
      int64_t c = key_first[g + 1] - key_first[g];
      if (c > max_items) max_items = c;
    }
    items = (orc_item *)malloc(sizeof(orc_item) * (size_t)max_items);
    rebuilt = (orc_item *)malloc(sizeof(orc_item) * (size_t)(table_size + 1));
    wts = (int32_t *)malloc(sizeof(int32_t) * (size_t)(table_size + 1));
    lens = (int32_t *)malloc(sizeof(int32_t) * (size_t)(table_size + 1));
    if (!items || !rebuilt || !wts || !lens) { rc = set_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
  }
  for (int64_t g = 0; g < G; ++g) {
    const int64_t d0 = key_first[g], d1 = key_first[g + 1];
    int64_t ni = d1 - d0;
    s->table_scale[g] = (uint16_t)(keys[g] >> 16);
    s->table_fp8[g] = (uint16_t)(keys[g] & 0xFFFF);
    uint16_t *syms_g = s->decode_syms + g * table_size;
    for (int64_t d = d0; d < d1; ++d) { items[d - d0].count = (int32_t)ucount[d]; items[d - d0].sym = (uint16_t)(ucomp[d] & 0xFFFF); }

    if (ni == 1) {
      /* single symbol: len 1, code 0 everywhere (build_huffman.cu:464-472) */
      for (int64_t j = 0; j < table_size; ++j) { syms_g[j] = items[0].sym; unpacked[j] = 1; }
      ucode[d0] = (1u << 16) | 0u;
    } else {
      qsort(items, (size_t)ni, sizeof(orc_item), item_cmp_asc);
      int use_esc = 0;
      uint16_t esc_sym = 0;
      orc_item *list = items;
      int64_t nl = ni;
      if (ni > table_size) {
        /* ESC: keep the 2^L-1 most frequent (count desc, sym asc) + ESC (:489-535) */
        use_esc = 1;
        qsort(items, (size_t)ni, sizeof(orc_item), item_cmp_desc);
        const int64_t keep_k = table_size - 1;
        uint32_t esc_freq = 0;
        for (int64_t i = keep_k; i < ni; ++i) esc_freq += (uint32_t)items[i].count;
        /* smallest u16 not kept: sort the kept symbols and find the first gap */
        uint16_t *ks = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)keep_k + 1);
        if (!ks) { rc = set_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
        for (int64_t i = 0; i < keep_k; ++i) ks[i] = items[i].sym;
        for (int64_t i = 1; i < keep_k; ++i) {
          uint16_t v = ks[i]; int64_t j = i - 1;
          while (j >= 0 && ks[j] > v) { ks[j + 1] = ks[j]; --j; }
          ks[j + 1] = v;
        }
        uint32_t cand = 0;
        for (int64_t i = 0; i < keep_k; ++i) { if (ks[i] == cand) ++cand; else if (ks[i] > cand) break; }
        free(ks);
        esc_sym = (uint16_t)cand;
        for (int64_t i = 0; i < keep_k; ++i) rebuilt[i] = items[i];
        rebuilt[keep_k].count = (int32_t)esc_freq;
        rebuilt[keep_k].sym = esc_sym;
        nl = keep_k + 1;
        qsort(rebuilt, (size_t)nl, sizeof(orc_item), item_cmp_asc);
        list = rebuilt;
        s->esc_keys++;
      }
      for (int64_t i = 0; i < nl; ++i) wts[i] = list[i].count;
      int prc = orc_package_merge(wts, (int)nl, L, lens);
      if (prc != ORC_OK) { rc = prc; goto fail; }
      /* canonical codes (build_huffman.cu:171-203): next_code recurrence over
         lengths, codes handed out in list order */
      int bl_count[17] = {0};
      uint32_t next_code[17] = {0};
      for (int64_t i = 0; i < nl; ++i) {
        if (lens[i] <= 0 || lens[i] > L) { rc = set_err(ORC_RUNTIME_ERROR, "invalid code length"); goto fail; }
        bl_count[lens[i]]++;
      }
      uint32_t code = 0;
      for (int bits = 1; bits < 16; ++bits) { code = (code + (uint32_t)bl_count[bits - 1]) << 1; next_code[bits] = code; }
      memset(unpacked, 0, (size_t)table_size);
      for (int64_t j = 0; j < table_size; ++j) syms_g[j] = 0;
      /* code of every item, and the LUT ranges (build_huffman.cu:205-228) */
      uint32_t esc_cw = 0;
      for (int64_t i = 0; i < nl; ++i) {
        const int len = lens[i];
        const uint32_t c = next_code[len]++;
        const uint32_t fill = 1u << (L - len);
        const uint32_t base = c << (L - len);
        const int is_esc = use_esc && list[i].sym == esc_sym;
        for (uint32_t f = 0; f < fill; ++f) {
          syms_g[base + f] = list[i].sym;
          unpacked[base + f] = (uint8_t)(is_esc ? (len | 0x8) : len);
        }
        /* record the code word on the matching histogram entry */
        const uint32_t cw = ((uint32_t)len << 16) | (c & 0xFFFFu);
        if (is_esc) esc_cw = cw;
        for (int64_t d = d0; d < d1; ++d) {
          if ((uint16_t)(ucomp[d] & 0xFFFF) == list[i].sym) { ucode[d] = cw; break; }
        }
      }
      if (use_esc) {
        /* The encoder map holds the kept symbols plus esc_sym. A symbol outside
           it is coded ESC code + raw16. A data symbol equal to esc_sym (never a
           kept one) finds the ESC code in the map and gets no raw16
           (build_huffman.cu:850-864): the decoder cannot tell it apart. */
        for (int64_t d = d0; d < d1; ++d) {
          uint16_t sy = (uint16_t)(ucomp[d] & 0xFFFF);
          int in_map = 0;
          for (int64_t i = 0; i < nl; ++i) if (list[i].sym == sy) { in_map = 1; break; }
          if (!in_map) ucode[d] = esc_cw | CW_RAW;
          else if (sy == esc_sym) s->esc_collisions += ucount[d];
        }
        esc_sym_of[g] = esc_sym; use_esc_of[g] = 1;
      }
    }
    /* pack 4-bit lengths low nibble first (build_huffman.cu:230-239) */
    uint8_t *lens_g = s->decode_lens + g * packed;
    for (int64_t j = 0; j < packed; ++j)
      lens_g[j] = (uint8_t)((unpacked[2 * j] & 0x0F) | ((unpacked[2 * j + 1] & 0x0F) << 4));
  }

  /* buckets: build_huffman.cu:582-696 */
  if (ndim != 2) { rc = set_err(ORC_INVALID_ARGUMENT, "bucket packing requires bf16_params to be 2D [n,m]"); goto fail; }
  {
    const int64_t n = dims[0], m = dims[1];
    if (n <= 0 || m <= 0) { rc = set_err(ORC_INVALID_ARGUMENT, "bf16_params shape must be non-empty"); goto fail; }
    orc_bucket *bk = NULL;
    int64_t nbk = 0, cap_bk = 0;
    int32_t *rows = NULL;
    int64_t nrows_out = 0, cap_rows = 0;
#define PUSH_BUCKET(SC, START, COUNT, C0, CLEN) do { \
      if (nbk == cap_bk) { cap_bk = cap_bk ? cap_bk * 2 : 64; bk = (orc_bucket *)realloc(bk, sizeof(orc_bucket) * (size_t)cap_bk); } \
      bk[nbk].scale = (SC); bk[nbk].row_start = (START); bk[nbk].row_count = (COUNT); \
      bk[nbk].col_start = (C0); bk[nbk].col_len = (CLEN); ++nbk; } while (0)
#define PUSH_ROW(R) do { \
      if (nrows_out == cap_rows) { cap_rows = cap_rows ? cap_rows * 2 : 1024; rows = (int32_t *)realloc(rows, sizeof(int32_t) * (size_t)cap_rows); } \
      rows[nrows_out++] = (R); } while (0)
    if (!scale_block2d) {
      if (!(scale_scalar || (!scale_per_elem && scale_per_row))) {
        rc = set_err(ORC_INVALID_ARGUMENT, "bucket packing requires scales to be scalar, per-row (n,), or 2D block-wise");
        goto fail;
      }
      /* rows grouped by row scale, scales ascending, rows ascending, <=128 rows each */
      uint64_t *rk = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)n);
      for (int64_t r = 0; r < n; ++r) {
        uint16_t sc = scale_scalar ? scales[0] : scales[r];
        rk[r] = ((uint64_t)sc << 32) | (uint64_t)r;
      }
      radix_sort_u64(rk, n, 48);
      int64_t i = 0;
      while (i < n) {
        int64_t j = i;
        while (j < n && (rk[j] >> 32) == (rk[i] >> 32)) ++j;
        uint16_t sc = (uint16_t)(rk[i] >> 32);
        for (int64_t off = i; off < j; off += 128) {
          int64_t take = (j - off) < 128 ? (j - off) : 128;
          int32_t start = (int32_t)nrows_out;
          for (int64_t q = 0; q < take; ++q) PUSH_ROW((int32_t)(rk[off + q] & 0xFFFFFFFFu));
          PUSH_BUCKET(sc, start, (int32_t)take, 0, (int32_t)m);
        }
        i = j;
      }
      free(rk);
    } else {
      for (int64_t br = 0; br < nb0; ++br) {
        for (int64_t bc = 0; bc < nb1; ++bc) {
          uint16_t sc = scales[br * nb1 + bc];
          for (int64_t off = 0; off < sb0; off += 128) {
            int64_t take = (sb0 - off) < 128 ? (sb0 - off) : 128;
            int32_t start = (int32_t)nrows_out;
            for (int64_t q = 0; q < take; ++q) PUSH_ROW((int32_t)(br * sb0 + off + q));
            PUSH_BUCKET(sc, start, (int32_t)take, (int32_t)(bc * sb1), (int32_t)sb1);
          }
        }
      }
    }
    const int64_t B = nbk;
    const int64_t k = threads_per_block;
    s->B = B; s->k = k; s->R = nrows_out;
    s->shape_nmk[0] = n; s->shape_nmk[1] = m; s->shape_nmk[2] = k;
    s->bucket_scale = (uint16_t *)calloc((size_t)B + 1, sizeof(uint16_t));
    s->bucket_row_offsets = (int32_t *)calloc((size_t)B + 1, sizeof(int32_t));
    s->row_indices = (int32_t *)calloc((size_t)nrows_out + 1, sizeof(int32_t));
    s->bucket_table = (int32_t *)calloc((size_t)B * 256 + 1, sizeof(int32_t));
    s->bucket_col_start = (int32_t *)calloc((size_t)B + 1, sizeof(int32_t));
    s->bucket_col_len = (int32_t *)calloc((size_t)B + 1, sizeof(int32_t));
    s->bucket_U = (int32_t *)calloc((size_t)B + 1, sizeof(int32_t));
    s->bucket_unique_gid = (int32_t *)calloc((size_t)B * 256 + 1, sizeof(int32_t));
    s->bucket_fp8_uidx = (int16_t *)calloc((size_t)B * 256 + 1, sizeof(int16_t));
    s->bucket_thread_startbit = (uint32_t *)calloc((size_t)(B * (k + 1)) + 1, sizeof(uint32_t));
    s->bucket_bit_base = (int64_t *)calloc((size_t)B + 1, sizeof(int64_t));
    if (nrows_out) memcpy(s->row_indices, rows, sizeof(int32_t) * (size_t)nrows_out);
    for (int64_t b = 0; b < B; ++b) {
      s->bucket_scale[b] = bk[b].scale;
      s->bucket_row_offsets[b] = bk[b].row_start;
      s->bucket_col_start[b] = bk[b].col_start;
      s->bucket_col_len[b] = bk[b].col_len;
    }
    s->bucket_row_offsets[B] = (int32_t)nrows_out;
    free(rows);

    /* bucket_table: gid of (bucket scale, fp8) or -1 (build_huffman.cu:737-746) */
    for (int64_t b = 0; b < B; ++b) {
      for (int c = 0; c < 256; ++c) {
        uint32_t key = ((uint32_t)bk[b].scale << 16) | (uint32_t)c;
        int64_t lo = 0, hi = G - 1, found = -1;
        while (lo <= hi) {
          int64_t mid = (lo + hi) / 2;
          if (keys[mid] == key) { found = mid; break; }
          if (keys[mid] < key) lo = mid + 1; else hi = mid - 1;
        }
        s->bucket_table[b * 256 + c] = (int32_t)found;
      }
      /* U / first-appearance unique gids / fp8 -> uidx (build_huffman.cu:748-783) */
      int32_t U = 0;
      for (int i = 0; i < 256; ++i) { s->bucket_unique_gid[b * 256 + i] = -1; s->bucket_fp8_uidx[b * 256 + i] = -1; }
      for (int i = 0; i < 256; ++i) {
        int32_t gid = s->bucket_table[b * 256 + i];
        if (gid < 0) continue;
        int32_t f = -1;
        for (int32_t j = 0; j < U; ++j) if (s->bucket_unique_gid[b * 256 + j] == gid) { f = j; break; }
        if (f < 0 && U < 256) { s->bucket_unique_gid[b * 256 + U] = gid; f = U; ++U; }
        s->bucket_fp8_uidx[b * 256 + i] = (int16_t)f;
      }
      s->bucket_U[b] = U;
    }

    /* per-element code word via the histogram entry (binary search) */
    uint32_t *cw = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)numel);
    if (!cw) { free(bk); rc = set_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
    for (int64_t i = 0; i < numel; ++i) {
      uint64_t c = (((((uint64_t)SCALE_OF(i)) << 16) | fp8[i]) << 16) | bf16[i];
      int64_t lo = 0, hi = D - 1, f = -1;
      while (lo <= hi) {
        int64_t mid = (lo + hi) / 2;
        if (ucomp[mid] == c) { f = mid; break; }
        if (ucomp[mid] < c) lo = mid + 1; else hi = mid - 1;
      }
      cw[i] = ucode[f];
    }

    /* bitstream (build_huffman.cu:786-925). Element order per lane t of bucket
       b: e = t, t+k_eff, ...; rr = e / col_len, cc = e % col_len. */
    int64_t cap_w = 1024, pos = 0;
    uint64_t *bs = (uint64_t *)calloc((size_t)cap_w, sizeof(uint64_t));
    for (int64_t b = 0; b < B && rc == ORC_OK; ++b) {
      if (pos & 63) pos = (pos + 63) & ~(int64_t)63;
      const int64_t base = pos;
      s->bucket_bit_base[b] = base;
      const int64_t total = (int64_t)bk[b].row_count * bk[b].col_len;
      int64_t k_eff = k < (total > 1 ? total : 1) ? k : (total > 1 ? total : 1);
      uint32_t *st = s->bucket_thread_startbit + b * (k + 1);
      /* pass 1: bit counts per lane -> relative u32 starts */
      int64_t rel = 0;
      st[0] = 0;
      for (int64_t t = 0; t < k_eff; ++t) {
        int64_t bits = 0;
        for (int64_t e = t; e < total; e += k_eff) {
          int64_t rr = e / bk[b].col_len, cc = e % bk[b].col_len;
          int64_t idx = (int64_t)s->row_indices[bk[b].row_start + rr] * m + bk[b].col_start + cc;
          uint32_t w = cw[idx];
          bits += ((w >> 16) & 0x1F) + ((w & CW_RAW) ? 16 : 0);
        }
        rel += bits;
        st[t + 1] = (uint32_t)rel;
      }
      for (int64_t t = k_eff + 1; t <= k; ++t) st[t] = st[k_eff];
      /* pass 2: append MSB-first */
      for (int64_t t = 0; t < k_eff; ++t) {
        for (int64_t e = t; e < total; e += k_eff) {
          int64_t rr = e / bk[b].col_len, cc = e % bk[b].col_len;
          int64_t idx = (int64_t)s->row_indices[bk[b].row_start + rr] * m + bk[b].col_start + cc;
          uint32_t w = cw[idx];
          int nb = (int)((w >> 16) & 0x1F);
          uint32_t v = w & 0xFFFFu;
          for (int pass = 0; pass < 2; ++pass) {
            if (nb > 0) {
              if ((pos >> 6) + 2 > cap_w) {
                int64_t nc = cap_w * 2;
                bs = (uint64_t *)realloc(bs, sizeof(uint64_t) * (size_t)nc);
                memset(bs + cap_w, 0, sizeof(uint64_t) * (size_t)(nc - cap_w));
                cap_w = nc;
              }
              for (int q = nb - 1; q >= 0; --q) {
                if ((v >> q) & 1u) bs[pos >> 6] |= (uint64_t)1 << (63 - (pos & 63));
                ++pos;
              }
            }
            if (pass == 0 && (w & CW_RAW)) { nb = 16; v = bf16[idx]; s->esc_elements++; }
            else break;
          }
        }
      }
      if ((uint32_t)(pos - base) != st[k_eff]) { rc = set_err(ORC_RUNTIME_ERROR, "internal error: bucket bit length mismatch"); }
    }
    s->bucket_bit_base[B] = pos;
    s->W = (pos + 63) >> 6;
    s->bitstream = (uint64_t *)calloc((size_t)s->W + 1, sizeof(uint64_t));
    if (s->W) memcpy(s->bitstream, bs, sizeof(uint64_t) * (size_t)s->W);
    free(bs); free(cw); free(bk);
    if (rc != ORC_OK) goto fail;
  }
  free(ucomp); free(ucount); free(ucode); free(key_first); free(keys); free(unpacked);
  free(items); free(rebuilt); free(wts); free(lens); free(esc_sym_of); free(use_esc_of);
  *out = s;
  return ORC_OK;
fail:
  free(ucomp); free(ucount); free(ucode); free(key_first); free(keys); free(unpacked);
  free(items); free(rebuilt); free(wts); free(lens); free(esc_sym_of); free(use_esc_of);
  orc_free(s);
  return rc;
#undef SCALE_OF
}

/* ------------------------------------------------------------------------- */
/* Decoder                                                                    */
/* ------------------------------------------------------------------------- */
static inline uint32_t peek_bits(const uint64_t *bs, int64_t W, int64_t pos, int nbits) {
  /* MSB-first bits [pos, pos+nbits), zeros past the end (decode_huffman.cu:82-88) */
  uint32_t v = 0;
  for (int i = 0; i < nbits; ++i) {
    int64_t p = pos + i;
    int64_t w = p >> 6;
    uint32_t bit = 0;
    if (w >= 0 && w < W) bit = (uint32_t)((bs[w] >> (63 - (p & 63))) & 1u);
    v = (v << 1) | bit;
  }
  return v;
}

typedef struct {
  const uint8_t *fp8; const uint64_t *bs; int64_t W; const uint16_t *syms; const uint8_t *lens;
  int64_t G; const int32_t *btab; const int32_t *col_start; const int32_t *col_len;
  const int32_t *row_off; const int32_t *row_idx; int64_t R; const uint32_t *startbit; int64_t k;
  const int64_t *bit_base; int64_t B; int64_t n, m; int L; int mode; uint16_t *out;
  int64_t *lane_prefix; /* [B+1] cumulative active lanes */
  int64_t lane_begin, lane_end;
  int status;
} dec_job;

static void decode_lane(const dec_job *j, int64_t b, int64_t t) {
  const int32_t ra = j->row_off[b], rb = j->row_off[b + 1];
  const int32_t rows = rb - ra;
  if (rows <= 0) return;
  const int32_t c0 = j->col_start[b], cl = j->col_len[b];
  if (cl <= 0) return;
  if (c0 < 0 || (int64_t)c0 + cl > j->m) return;
  const int64_t total = (int64_t)rows * cl;
  int64_t k_eff = j->k < total ? j->k : total;
  if (k_eff < 1) k_eff = 1;
  if (t >= k_eff) return;
  const int L = j->L;
  const int64_t tsz = (int64_t)1 << L, psz = tsz / 2;
  int64_t pos = j->bit_base[b] + (int64_t)j->startbit[b * (j->k + 1) + t];
  int64_t rr = 0, cc = t;
  for (int64_t e = t; e < total; e += k_eff) {
    if (j->mode == ORC_DECODE_LOSSLESS) { rr = e / cl; cc = e % cl; }
    if (rr >= rows || ra + rr >= j->R) return;
    const int64_t idx = (int64_t)j->row_idx[ra + rr] * j->m + c0 + cc;
    if (idx < 0 || idx >= j->n * j->m) return;
    const uint32_t q = j->fp8[idx];
    const int32_t gid = j->btab[b * 256 + q];
    const uint32_t p = peek_bits(j->bs, j->W, pos, L);
    uint16_t sym = 0; uint32_t nib = 0;
    if (gid >= 0 && gid < j->G) {
      sym = j->syms[gid * tsz + p];
      uint8_t v = j->lens[gid * psz + (p >> 1)];
      nib = (p & 1u) ? (uint32_t)(v >> 4) : (uint32_t)(v & 0x0F);
    }
    pos += nib & 7u;
    if (j->mode == ORC_DECODE_LOSSLESS && (nib & 8u)) {
      sym = (uint16_t)peek_bits(j->bs, j->W, pos, 16);
      pos += 16;
    }
    j->out[idx] = sym;
    if (j->mode == ORC_DECODE_REFERENCE_KERNEL) {
      /* decode_huffman.cu:363-370: one wrap per step */
      cc += k_eff;
      if (cc >= cl) { cc -= cl; rr += 1; }
    }
  }
}

static void *decode_worker(void *arg) {
  dec_job *j = (dec_job *)arg;
  int64_t b = 0;
  for (int64_t g = j->lane_begin; g < j->lane_end; ++g) {
    while (j->lane_prefix[b + 1] <= g) ++b;
    decode_lane(j, b, g - j->lane_prefix[b]);
  }
  return NULL;
}

int orc_decode(const uint8_t *fp8, const uint64_t *bs, int64_t W,
               const uint16_t *syms, const uint8_t *lens, int64_t G,
               const int32_t *bucket_table, const int32_t *col_start, const int32_t *col_len,
               const int32_t *row_off, const int32_t *row_idx, int64_t R,
               const uint32_t *startbit, int64_t k, const int64_t *bit_base, int64_t B,
               int64_t n, int64_t m, int max_len, int mode, int nthreads, uint16_t *out) {
  g_err[0] = 0;
  if (max_len < 1 || max_len > 7) return set_err(ORC_INVALID_ARGUMENT, "oracle decode supports max_len in [1,7]");
  if (k < 1 || k > 1024) return set_err(ORC_INVALID_ARGUMENT, "k must be in [1,1024]");
  if (nthreads < 1) nthreads = 1;
  dec_job base;
  memset(&base, 0, sizeof(base));
  base.fp8 = fp8; base.bs = bs; base.W = W; base.syms = syms; base.lens = lens; base.G = G;
  base.btab = bucket_table; base.col_start = col_start; base.col_len = col_len; base.row_off = row_off;
  base.row_idx = row_idx; base.R = R; base.startbit = startbit; base.k = k; base.bit_base = bit_base;
  base.B = B; base.n = n; base.m = m; base.L = max_len; base.mode = mode; base.out = out;
  int64_t *lp = (int64_t *)malloc(sizeof(int64_t) * (size_t)(B + 1));
  if (!lp) return set_err(ORC_NO_MEMORY, "out of memory");
  lp[0] = 0;
  for (int64_t b = 0; b < B; ++b) {
    int64_t rows = (int64_t)row_off[b + 1] - row_off[b];
    int64_t total = rows * (int64_t)col_len[b];
    int64_t ke = total < k ? total : k;
    if (ke < 1) ke = 1;
    if (rows <= 0 || col_len[b] <= 0) ke = 0;
    lp[b + 1] = lp[b] + ke;
  }
  base.lane_prefix = lp;
  const int64_t lanes = lp[B];
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  int ok[256];
  dec_job jobs[256];
  for (int i = 0; i < nthreads; ++i) {
    jobs[i] = base;
    jobs[i].lane_begin = lanes * i / nthreads;
    jobs[i].lane_end = lanes * (i + 1) / nthreads;
    ok[i] = 0;
    if (nthreads > 1 && pthread_create(&th[i], NULL, decode_worker, &jobs[i]) == 0) ok[i] = 1;
    else decode_worker(&jobs[i]);
  }
  for (int i = 0; i < nthreads; ++i) if (ok[i]) pthread_join(th[i], NULL);
  free(lp);
  return ORC_OK;
}
