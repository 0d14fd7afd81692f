/*
 * CPU restatement of MPServe's AWQ int4 + Huffman-sidecar path. TEST INFRASTRUCTURE ONLY.
 *
 * Like fp8_huffman_oracle.c, this file is the parity oracle: tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may call it, as
 * the checker. The product (mpserve_amd) never links, loads or calls it.
 *
 * It restates, in plain C with no hashing containers, the two AWQ int4 bucket
 * builders and their decoders:
 *   huffman_build_awq_int4_bucket_decode_tables_entry  kernel/build_huffman.cu:1583-2126
 *     validation :1589-1650; key = scale_u16<<16 | (qv & 0xF) :1667-1677
 *     per-key code book :1701-1836 (ESC: keep 2^L-1 by (count desc, sym asc),
 *       esc_sym = smallest u16 not kept, weight max(esc_freq,1), list re-sorted
 *       (count asc, sym asc); ESC length forced to L; ESC LUT nibbles = 15)
 *     row / block-2D bucketing :1868-1933 (<=128 rows a bucket)
 *     bucket_table [B,16] :1973-1982; bitstream :1984-2099
 *   huffman_build_awq_int4_bucket_decode_tables_by_scale_entry  kernel/build_huffman.cu:1075-1580
 *     code book :1217-1344 (ESC: esc_sym = smallest u16 absent from ALL of
 *       the key's symbols, 0xFFFF if none; the list stays in (count desc, sym
 *       asc) order with ESC last, while package-merge returns lengths by
 *       sorted position :46-118, so the lengths apply positionally)
 *     ragged buckets of quantisation groups (row, col_start) by exact scale,
 *       groups ordered (row, col), <= group_cap groups a bucket :1350-1385
 *   decoders kernel/decode_huffman.cu:378-589: L = 11, nibble 15 = ESC
 *     (consume L bits, then 16 raw bits), a table id < 0 decodes as ESC too.
 *     The int4 bucket kernel walks columns with one wrap per step
 *     (:462-468); this oracle walks e % col_len like the encoder (:2040-2042).
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

int orc_package_merge(const int32_t *weights_in, int n, int L, int32_t *lens_out);

typedef struct orc_awq_sidecar {
  int64_t G, table_size, packed_len_size;
  uint16_t *decode_syms;   /* [G, 2^L] */
  uint8_t *decode_lens;    /* [G, 2^(L-1)] */
  uint16_t *table_scale;   /* [G] */
  uint16_t *table_qv;      /* [G] */
  int64_t B;
  uint16_t *bucket_scale;  /* [B] */
  int32_t *row_offsets;    /* [B+1] bucket_row_offsets or bucket_group_offsets */
  int64_t R;
  int32_t *row_indices;    /* [R] row_indices or group_rows */
  int32_t *col_start;      /* [B] bucket_col_start, or [R] group_col_start (by scale) */
  int32_t *col_len;        /* [B] bucket_col_len (bucket layout only) */
  int32_t *bucket_table;   /* [B,16] */
  int64_t k;
  uint32_t *startbit;      /* [B,k+1] */
  int64_t *bit_base;       /* [B+1] */
  int64_t W;
  uint64_t *bitstream;     /* [W] */
  int64_t shape[4];        /* n, m, k (, group_size) */
  int64_t group_size;      /* by scale: columns per group; bucket layout: 0 */
  int64_t esc_keys, esc_collisions, esc_elements;
} orc_awq_sidecar;

static char g_awq_err[512];
const char *orc_awq_last_error(void) { return g_awq_err; }
static int awq_err(int code, const char *msg) {
  snprintf(g_awq_err, sizeof(g_awq_err), "%s", msg);
  return code;
}

void orc_awq_free(orc_awq_sidecar *s) {
  if (!s) return;
  free(s->decode_syms); free(s->decode_lens); free(s->table_scale); free(s->table_qv);
  free(s->bucket_scale); free(s->row_offsets); free(s->row_indices); free(s->col_start); free(s->col_len);
  free(s->bucket_table); free(s->startbit); free(s->bit_base); free(s->bitstream);
  free(s);
}

typedef struct { int32_t count; uint16_t sym; } awq_item;
static int awq_cmp_asc(const void *pa, const void *pb) {
  const awq_item *a = (const awq_item *)pa, *b = (const awq_item *)pb;
  if (a->count != b->count) return a->count < b->count ? -1 : 1;
  return (int)a->sym - (int)b->sym;
}
static int awq_cmp_desc(const void *pa, const void *pb) {
  const awq_item *a = (const awq_item *)pa, *b = (const awq_item *)pb;
  if (a->count != b->count) return a->count > b->count ? -1 : 1;
  return (int)a->sym - (int)b->sym;
}
static int cmp_u64(const void *pa, const void *pb) {
  uint64_t a = *(const uint64_t *)pa, b = *(const uint64_t *)pb;
  return a < b ? -1 : a > b;
}
static int cmp_i32(const void *pa, const void *pb) {
  int32_t a = *(const int32_t *)pa, b = *(const int32_t *)pb;
  return a < b ? -1 : a > b;
}

#define CW_RAW (1u << 24)

/* by_scale = 0: huffman_build_awq_int4_bucket_decode_tables_entry;
   by_scale = 1: huffman_build_awq_int4_bucket_decode_tables_by_scale_entry. */
int orc_awq_encode(const uint16_t *bf16, const uint8_t *qv, int64_t n, int64_t m,
                   const uint16_t *scales, int64_t scale_numel, int scale_ndim, const int64_t *scale_dims,
                   int64_t max_len, int64_t threads, int64_t group_cap, int by_scale, orc_awq_sidecar **out) {
  *out = NULL;
  g_awq_err[0] = 0;
  const int L = (int)max_len;
  if (L <= 0 || L > 15) return awq_err(ORC_INVALID_ARGUMENT, "max_len must be in (0,15]");
  if (threads <= 0 || threads > 1024) return awq_err(ORC_INVALID_ARGUMENT, "threads_per_block must be in [1,1024]");
  if (by_scale && group_cap <= 0) return awq_err(ORC_INVALID_ARGUMENT, "group_cap must be > 0");
  if (n <= 0 || m <= 0) return awq_err(ORC_INVALID_ARGUMENT, "bf16_params shape must be non-empty");
  /* scale modes (:1625-1650): scalar, per-row (1-D of n), block-2D */
  const int scalar = scale_numel == 1;
  const int per_row = !scalar && scale_ndim == 1 && scale_numel == n;
  int block2d = 0;
  int64_t nb0 = -1, nb1 = -1, sb0 = -1, sb1 = -1;
  if (!scalar && !per_row && scale_ndim == 2) {
    nb0 = scale_dims[0]; nb1 = scale_dims[1];
    if (nb0 > 0 && nb1 > 0 && n % nb0 == 0 && m % nb1 == 0) {
      sb0 = n / nb0; sb1 = m / nb1;
      if (sb0 > 0 && sb1 > 0) block2d = 1;
    }
  }
  if (!scalar && !per_row && !block2d)
    return awq_err(ORC_INVALID_ARGUMENT,
                   "unsupported scales_u16 shape: use scalar, per-row (n,), or 2D block-wise [n/bs0,m/bs1]");
#define SC_RC(r, c) (scalar ? scales[0] : per_row ? scales[(r)] : scales[((r) / sb0) * nb1 + (c) / sb1])
  const int64_t N = n * m;
  const int64_t T = (int64_t)1 << L;
  const int64_t P = T / 2;

  /* histogram as a sort of (key << 16 | sym), key = scale << 16 | qv */
  uint64_t *comp = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)N);
  if (!comp) return awq_err(ORC_NO_MEMORY, "out of memory");
  for (int64_t r = 0; r < n; ++r)
    for (int64_t c = 0; c < m; ++c) {
      const int64_t i = r * m + c;
      const uint64_t key = ((uint64_t)SC_RC(r, c) << 16) | (uint64_t)(qv[i] & 0x0Fu);
      comp[i] = (key << 16) | bf16[i];
    }
  qsort(comp, (size_t)N, sizeof(uint64_t), cmp_u64);
  int64_t D = 0;
  for (int64_t i = 0; i < N; ++i) if (i == 0 || comp[i] != comp[i - 1]) ++D;
  uint64_t *ucomp = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)D);
  uint32_t *ucount = (uint32_t *)calloc((size_t)D, sizeof(uint32_t));
  uint32_t *ucode = (uint32_t *)calloc((size_t)D, sizeof(uint32_t));
  orc_awq_sidecar *s = (orc_awq_sidecar *)calloc(1, sizeof(orc_awq_sidecar));
  int64_t *key_first = NULL;
  uint32_t *keys = NULL;
  awq_item *items = NULL, *list = NULL;
  int32_t *wts = NULL, *lens = NULL, *sorted_w = NULL;
  uint8_t *unpacked = NULL;
  int rc = ORC_OK;
  if (!ucomp || !ucount || !ucode || !s) { free(comp); rc = awq_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
  {
    int64_t d = -1;
    for (int64_t i = 0; i < N; ++i) {
      if (i == 0 || comp[i] != comp[i - 1]) { ++d; ucomp[d] = comp[i]; }
      ucount[d]++;
    }
  }
  free(comp);

  /* keys ascending -> gid */
  int64_t G = 0;
  for (int64_t d = 0; d < D; ++d) if (d == 0 || (ucomp[d] >> 16) != (ucomp[d - 1] >> 16)) ++G;
  key_first = (int64_t *)malloc(sizeof(int64_t) * (size_t)(G + 1));
  keys = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(G + 1));
  if (!key_first || !keys) { rc = awq_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
  {
    int64_t g = -1;
    for (int64_t d = 0; d < D; ++d)
      if (d == 0 || (ucomp[d] >> 16) != (ucomp[d - 1] >> 16)) { ++g; key_first[g] = d; keys[g] = (uint32_t)(ucomp[d] >> 16); }
    key_first[G] = D;
  }
  s->G = G; s->table_size = T; s->packed_len_size = P;
  s->decode_syms = (uint16_t *)calloc((size_t)(G * T + 1), 2);
  s->decode_lens = (uint8_t *)calloc((size_t)(G * P + 1), 1);
  s->table_scale = (uint16_t *)calloc((size_t)G + 1, 2);
  s->table_qv = (uint16_t *)calloc((size_t)G + 1, 2);
  items = (awq_item *)malloc(sizeof(awq_item) * (size_t)(D + 1));
  list = (awq_item *)malloc(sizeof(awq_item) * (size_t)(T + 1));
  wts = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T + 1));
  sorted_w = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T + 1));
  lens = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T + 1));
  unpacked = (uint8_t *)malloc((size_t)T);
  if (!s->decode_syms || !s->decode_lens || !s->table_scale || !s->table_qv || !items || !list || !wts ||
      !sorted_w || !lens || !unpacked) { rc = awq_err(ORC_NO_MEMORY, "out of memory"); goto fail; }

  for (int64_t g = 0; g < G; ++g) {
    const int64_t d0 = key_first[g], d1 = key_first[g + 1], ni = d1 - d0;
    s->table_scale[g] = (uint16_t)(keys[g] >> 16);
    s->table_qv[g] = (uint16_t)(keys[g] & 0xFFFF);
    uint16_t *syms_g = s->decode_syms + g * T;
    for (int64_t d = d0; d < d1; ++d) { items[d - d0].count = (int32_t)ucount[d]; items[d - d0].sym = (uint16_t)(ucomp[d] & 0xFFFF); }
    if (ni == 1) {
      /* one symbol: every entry, length 1, code 0 (:1731-1737) */
      for (int64_t j = 0; j < T; ++j) { syms_g[j] = items[0].sym; unpacked[j] = 1; }
      ucode[d0] = 1u << 16;
    } else {
      qsort(items, (size_t)ni, sizeof(awq_item), awq_cmp_asc);
      int use_esc = 0;
      uint16_t esc_sym = 0;
      int64_t nl = ni;
      if (ni > T) {
        use_esc = 1;
        qsort(items, (size_t)ni, sizeof(awq_item), awq_cmp_desc);
        const int64_t keep_k = T - 1;
        uint32_t esc_freq = 0;
        for (int64_t i = keep_k; i < ni; ++i) esc_freq += (uint32_t)items[i].count;
        /* smallest u16 outside a symbol set: sort the set, find the first gap */
        const int64_t nset = by_scale ? ni : keep_k;  /* all symbols (:1267-1273) or the kept ones (:1788-1794) */
        int32_t *set = (int32_t *)malloc(sizeof(int32_t) * (size_t)nset);
        if (!set) { rc = awq_err(ORC_NO_MEMORY, "out of memory"); goto fail; }
        for (int64_t i = 0; i < nset; ++i) set[i] = items[i].sym;
        qsort(set, (size_t)nset, sizeof(int32_t), cmp_i32);
        uint32_t cand = 0;
        for (int64_t i = 0; i < nset; ++i) { if ((uint32_t)set[i] == cand) ++cand; else if ((uint32_t)set[i] > cand) break; }
        free(set);
        if (cand > 0xFFFFu) cand = by_scale ? 0xFFFFu : 0u;  /* all 65536 present: :1274-1277 */
        esc_sym = (uint16_t)cand;
        for (int64_t i = 0; i < keep_k; ++i) list[i] = items[i];
        list[keep_k].sym = esc_sym;
        nl = keep_k + 1;
        if (by_scale) {
          list[keep_k].count = (int32_t)esc_freq;  /* stays last, list not re-sorted (:1279-1289) */
        } else {
          list[keep_k].count = (int32_t)esc_freq > 0 ? (int32_t)esc_freq : 1;  /* :1804 */
          qsort(list, (size_t)nl, sizeof(awq_item), awq_cmp_asc);
        }
        s->esc_keys++;
      } else {
        for (int64_t i = 0; i < ni; ++i) list[i] = items[i];
      }
      /* package-merge sorts the weights and returns lengths by sorted
         position; the callers apply them to their list positionally */
      for (int64_t i = 0; i < nl; ++i) { wts[i] = list[i].count; sorted_w[i] = list[i].count; }
      qsort(sorted_w, (size_t)nl, sizeof(int32_t), cmp_i32);
      int prc = orc_package_merge(sorted_w, (int)nl, L, lens);
      if (prc != ORC_OK) { rc = prc; goto fail; }
      for (int64_t i = 0; i < nl; ++i) {
        if (lens[i] <= 0 || lens[i] > L) { rc = awq_err(ORC_RUNTIME_ERROR, "invalid code length"); goto fail; }
        if (use_esc && list[i].sym == esc_sym) lens[i] = L;  /* ESC has length L (:1823-1827) */
      }
      int bl_count[17] = {0};
      uint32_t next_code[17] = {0};
      for (int64_t i = 0; i < nl; ++i) bl_count[lens[i]]++;
      uint32_t code = 0;
      for (int bits = 1; bits < 16; ++bits) { code = (code + (uint32_t)bl_count[bits - 1]) << 1; next_code[bits] = code; }
      memset(unpacked, 0, (size_t)T);
      for (int64_t j = 0; j < T; ++j) syms_g[j] = 0;
      uint32_t esc_cw = 0;
      for (int64_t i = 0; i < nl; ++i) {
        const int len = lens[i];
        const uint32_t c = next_code[len]++;
        const uint32_t fill = 1u << (L - len), base = c << (L - len);
        const int is_esc = use_esc && list[i].sym == esc_sym;
        for (uint32_t f = 0; f < fill; ++f) {
          syms_g[base + f] = list[i].sym;
          unpacked[base + f] = (uint8_t)(is_esc ? 15 : len);
        }
        const uint32_t cw = ((uint32_t)len << 16) | (c & 0xFFFFu);
        if (is_esc) esc_cw = cw;
        for (int64_t d = d0; d < d1; ++d)
          if ((uint16_t)(ucomp[d] & 0xFFFF) == list[i].sym) { ucode[d] = cw; break; }
      }
      if (use_esc) {
        /* symbols outside the map: ESC code + raw16; a data symbol equal to
           esc_sym finds the ESC code and gets no raw16 (:2075-2090) */
        for (int64_t d = d0; d < d1; ++d) {
          const uint16_t sy = (uint16_t)(ucomp[d] & 0xFFFF);
          int in_map = 0;
          for (int64_t i = 0; i < nl; ++i) if (list[i].sym == sy) { in_map = 1; break; }
          if (!in_map) ucode[d] = esc_cw | CW_RAW;
          else if (sy == esc_sym) s->esc_collisions += ucount[d];
        }
      }
    }
    uint8_t *lens_g = s->decode_lens + g * P;
    for (int64_t j = 0; j < P; ++j) lens_g[j] = (uint8_t)((unpacked[2 * j] & 0x0F) | ((unpacked[2 * j + 1] & 0x0F) << 4));
  }

  /* buckets */
  {
    int64_t cap = 64, B = 0, R = 0, capR = 1024;
    uint16_t *bsc = (uint16_t *)malloc(2 * (size_t)cap);
    int32_t *roff = (int32_t *)malloc(4 * (size_t)(cap + 1));
    int32_t *bcs = (int32_t *)malloc(4 * (size_t)cap);
    int32_t *bcl = (int32_t *)malloc(4 * (size_t)cap);
    int32_t *rows = (int32_t *)malloc(4 * (size_t)capR);
    int32_t *gcol = (int32_t *)malloc(4 * (size_t)capR);
    roff[0] = 0;
#define GROW_B() do { if (B + 1 >= cap) { cap *= 2; bsc = (uint16_t *)realloc(bsc, 2 * (size_t)cap); \
      roff = (int32_t *)realloc(roff, 4 * (size_t)(cap + 1)); bcs = (int32_t *)realloc(bcs, 4 * (size_t)cap); \
      bcl = (int32_t *)realloc(bcl, 4 * (size_t)cap); } } while (0)
#define PUSH_R(RW, GC) do { if (R == capR) { capR *= 2; rows = (int32_t *)realloc(rows, 4 * (size_t)capR); \
      gcol = (int32_t *)realloc(gcol, 4 * (size_t)capR); } rows[R] = (RW); gcol[R] = (GC); ++R; } while (0)
    int64_t gsz = 0;
    if (!by_scale) {
      if (!block2d) {
        /* rows grouped by scale, scales ascending, rows ascending (:1869-1905) */
        uint64_t *rk = (uint64_t *)malloc(8 * (size_t)n);
        for (int64_t r = 0; r < n; ++r) rk[r] = ((uint64_t)(scalar ? scales[0] : scales[r]) << 32) | (uint64_t)r;
        qsort(rk, (size_t)n, 8, cmp_u64);
        int64_t i = 0;
        while (i < n) {
          int64_t j = i;
          while (j < n && (rk[j] >> 32) == (rk[i] >> 32)) ++j;
          for (int64_t off = i; off < j; off += 128) {
            const int64_t take = (j - off) < 128 ? (j - off) : 128;
            for (int64_t q = 0; q < take; ++q) PUSH_R((int32_t)(rk[off + q] & 0xFFFFFFFFu), 0);
            GROW_B();
            bsc[B] = (uint16_t)(rk[i] >> 32); bcs[B] = 0; bcl[B] = (int32_t)m; ++B; roff[B] = (int32_t)R;
          }
          i = j;
        }
        free(rk);
      } else {
        /* (row block, column block), <= 128 rows a bucket (:1906-1933) */
        for (int64_t br = 0; br < nb0; ++br)
          for (int64_t bc = 0; bc < nb1; ++bc)
            for (int64_t off = 0; off < sb0; off += 128) {
              const int64_t take = (sb0 - off) < 128 ? (sb0 - off) : 128;
              for (int64_t q = 0; q < take; ++q) PUSH_R((int32_t)(br * sb0 + off + q), 0);
              GROW_B();
              bsc[B] = scales[br * nb1 + bc]; bcs[B] = (int32_t)(bc * sb1); bcl[B] = (int32_t)sb1; ++B; roff[B] = (int32_t)R;
            }
      }
    } else {
      /* groups (row, col_start) by exact scale, scales ascending, groups by (row, col) (:1350-1385) */
      gsz = block2d ? sb1 : m;
      const int64_t gpr = block2d ? nb1 : 1;
      const int64_t NG = n * gpr;
      uint64_t *gk = (uint64_t *)malloc(8 * (size_t)NG);
      for (int64_t r = 0; r < n; ++r)
        for (int64_t bc = 0; bc < gpr; ++bc) gk[r * gpr + bc] = ((uint64_t)SC_RC(r, bc * gsz) << 40) | (uint64_t)(r * gpr + bc);
      qsort(gk, (size_t)NG, 8, cmp_u64);
      int64_t i = 0;
      while (i < NG) {
        int64_t j = i;
        while (j < NG && (gk[j] >> 40) == (gk[i] >> 40)) ++j;
        for (int64_t off = i; off < j; off += group_cap) {
          const int64_t take = (j - off) < group_cap ? (j - off) : group_cap;
          for (int64_t q = 0; q < take; ++q) {
            const int64_t gi = (int64_t)(gk[off + q] & 0xFFFFFFFFFFull);
            PUSH_R((int32_t)(gi / gpr), (int32_t)((gi % gpr) * gsz));
          }
          GROW_B();
          bsc[B] = (uint16_t)(gk[i] >> 40); bcs[B] = 0; bcl[B] = (int32_t)gsz; ++B; roff[B] = (int32_t)R;
        }
        i = j;
      }
      free(gk);
    }
    const int64_t k = threads;
    s->B = B; s->R = R; s->k = k; s->group_size = gsz;
    s->shape[0] = n; s->shape[1] = m; s->shape[2] = k; s->shape[3] = gsz;
    s->bucket_scale = bsc; s->row_offsets = roff; s->row_indices = rows;
    s->col_start = by_scale ? gcol : bcs;
    s->col_len = bcl;
    if (by_scale) free(bcs); else free(gcol);
    s->bucket_table = (int32_t *)calloc((size_t)B * 16 + 1, 4);
    s->startbit = (uint32_t *)calloc((size_t)(B * (k + 1)) + 1, 4);
    s->bit_base = (int64_t *)calloc((size_t)B + 1, 8);
    for (int64_t b = 0; b < B; ++b)
      for (int q = 0; q < 16; ++q) {
        const uint32_t key = ((uint32_t)bsc[b] << 16) | (uint32_t)q;
        int64_t lo = 0, hi = G - 1, f = -1;
        while (lo <= hi) {
          const int64_t mid = (lo + hi) / 2;
          if (keys[mid] == key) { f = mid; break; }
          if (keys[mid] < key) lo = mid + 1; else hi = mid - 1;
        }
        s->bucket_table[b * 16 + q] = (int32_t)f;
      }

    /* bitstream: lane t of a bucket codes e = t, t+k_eff, ...; element e is
       (rr, cc) = (e / col_len, e % col_len) of the bucket's row (or group) list */
    int64_t cap_w = 1024, pos = 0;
    uint64_t *bs = (uint64_t *)calloc((size_t)cap_w, 8);
    for (int64_t b = 0; b < B && rc == ORC_OK; ++b) {
      if (pos & 63) pos = (pos + 63) & ~(int64_t)63;
      const int64_t base = pos;
      s->bit_base[b] = base;
      const int64_t ra = roff[b], cl = bcl[b];
      const int64_t total = (int64_t)(roff[b + 1] - ra) * cl;
      const int64_t k_eff = k < (total > 1 ? total : 1) ? k : (total > 1 ? total : 1);
      uint32_t *st = s->startbit + b * (k + 1);
      for (int pass = 0; pass < 2; ++pass) {
        int64_t rel = 0;
        for (int64_t t = 0; t < k_eff; ++t) {
          for (int64_t e = t; e < total; e += k_eff) {
            const int64_t rr = e / cl, cc = e % cl;
            const int64_t c = (by_scale ? s->col_start[ra + rr] : s->col_start[b]) + cc;
            const int64_t idx = (int64_t)rows[ra + rr] * m + c;
            const uint64_t key = ((uint64_t)bsc[b] << 16) | (uint64_t)(qv[idx] & 0x0Fu);
            const uint64_t want = (key << 16) | bf16[idx];
            int64_t lo = 0, hi = D - 1, f = -1;
            while (lo <= hi) {
              const int64_t mid = (lo + hi) / 2;
              if (ucomp[mid] == want) { f = mid; break; }
              if (ucomp[mid] < want) lo = mid + 1; else hi = mid - 1;
            }
            if (f < 0) { rc = awq_err(ORC_RUNTIME_ERROR, "missing enc table for (scale,qv) key"); break; }
            const uint32_t w = ucode[f];
            const int nb = (int)((w >> 16) & 0x1F);
            if (pass == 0) { rel += nb + ((w & CW_RAW) ? 16 : 0); continue; }
            for (int part = 0; part < 2; ++part) {
              const int bits = part == 0 ? nb : 16;
              const uint32_t v = part == 0 ? (w & 0xFFFFu) : bf16[idx];
              if (part == 1) { if (!(w & CW_RAW)) break; s->esc_elements++; }
              if ((pos >> 6) + 2 > cap_w) {
                const int64_t nc = cap_w * 2;
                bs = (uint64_t *)realloc(bs, 8 * (size_t)nc);
                memset(bs + cap_w, 0, 8 * (size_t)(nc - cap_w));
                cap_w = nc;
              }
              for (int q = bits - 1; q >= 0; --q) {
                if ((v >> q) & 1u) bs[pos >> 6] |= (uint64_t)1 << (63 - (pos & 63));
                ++pos;
              }
            }
          }
          if (rc != ORC_OK) break;
          if (pass == 0) st[t + 1] = (uint32_t)rel;
        }
        if (pass == 0) { st[0] = 0; for (int64_t t = k_eff + 1; t <= k; ++t) st[t] = st[k_eff]; }
      }
      if (rc == ORC_OK && (uint32_t)(pos - base) != st[k_eff])
        rc = awq_err(ORC_RUNTIME_ERROR, "internal error: bucket bit length mismatch");
    }
    s->bit_base[B] = pos;
    s->W = (pos + 63) >> 6;
    s->bitstream = (uint64_t *)calloc((size_t)s->W + 1, 8);
    if (s->W) memcpy(s->bitstream, bs, 8 * (size_t)s->W);
    free(bs);
    if (rc != ORC_OK) goto fail;
  }
  free(ucomp); free(ucount); free(ucode); free(key_first); free(keys); free(items); free(list);
  free(wts); free(sorted_w); free(lens); free(unpacked);
  *out = s;
  return ORC_OK;
fail:
  free(ucomp); free(ucount); free(ucode); free(key_first); free(keys); free(items); free(list);
  free(wts); free(sorted_w); free(lens); free(unpacked);
  orc_awq_free(s);
  return rc;
#undef SC_RC
}

/* ------------------------------------------------------------------------- */
/* Decoder (kernel/decode_huffman.cu:378-589)                                 */
/* ------------------------------------------------------------------------- */
static inline uint32_t awq_peek(const uint64_t *bs, int64_t W, int64_t pos, int nbits) {
  /* MSB-first bits [pos, pos+nbits), zeros past the end */
  uint32_t v = 0;
  for (int i = 0; i < nbits; ++i) {
    const int64_t p = pos + i, w = p >> 6;
    const uint32_t bit = (w >= 0 && w < W) ? (uint32_t)((bs[w] >> (63 - (p & 63))) & 1u) : 0u;
    v = (v << 1) | bit;
  }
  return v;
}

typedef struct {
  const uint8_t *qv; const uint64_t *bs; int64_t W; const uint16_t *syms; const uint8_t *lens; int64_t G;
  const int32_t *btab; const int32_t *col_start; const int32_t *col_len; const int32_t *row_off;
  const int32_t *row_idx; int64_t R; const int32_t *group_col; int64_t group_size;
  const uint32_t *startbit; int64_t k; const int64_t *bit_base; int64_t B; int64_t n, m; uint16_t *out;
  const int64_t *lane_prefix; int64_t lane_begin, lane_end;
} awq_dec_job;

/* rows (or groups) and column span of bucket b; 0 if the bucket decodes nothing */
static int awq_bucket(const awq_dec_job *j, int64_t b, int64_t *ra, int64_t *rows, int64_t *c0, int64_t *cl) {
  *ra = j->row_off[b];
  *rows = (int64_t)j->row_off[b + 1] - *ra;
  if (*rows <= 0) return 0;
  if (j->group_col) { *c0 = 0; *cl = j->group_size; return *cl > 0; }
  *c0 = j->col_start[b]; *cl = j->col_len[b];
  if (*cl <= 0 || *c0 < 0 || *c0 + *cl > j->m) return 0;
  return 1;
}

static void awq_decode_lane(const awq_dec_job *j, int64_t b, int64_t t) {
  int64_t ra, rows, c0, cl;
  if (!awq_bucket(j, b, &ra, &rows, &c0, &cl)) return;
  const int64_t total = rows * cl;
  int64_t k_eff = j->k < total ? j->k : total;
  if (k_eff < 1) k_eff = 1;
  if (t >= k_eff) return;
  const int L = 11;
  int64_t pos = j->bit_base[b] + (int64_t)j->startbit[b * (j->k + 1) + t];
  for (int64_t e = t; e < total; e += k_eff) {
    const int64_t rr = e / cl, cc = e % cl;
    if (ra + rr >= j->R) return;
    const int64_t col = (j->group_col ? j->group_col[ra + rr] : c0) + cc;
    const int64_t idx = (int64_t)j->row_idx[ra + rr] * j->m + col;
    if (idx < 0 || idx >= j->n * j->m) return;
    const int32_t gid = j->btab[b * 16 + (j->qv[idx] & 0x0F)];
    const uint32_t p = awq_peek(j->bs, j->W, pos, L);
    uint32_t nib = 15;
    uint16_t sym = 0;
    if (gid >= 0 && gid < j->G) {
      const uint8_t v = j->lens[gid * 1024 + (p >> 1)];
      nib = (p & 1u) ? (uint32_t)(v >> 4) : (uint32_t)(v & 0x0F);
      sym = j->syms[gid * 2048 + p];
    }
    if (nib != 15) {
      pos += nib;
    } else {
      /* ESC (and a bucket_table entry of -1): L bits, then 16 raw bits */
      pos += L;
      sym = (uint16_t)awq_peek(j->bs, j->W, pos, 16);
      pos += 16;
    }
    j->out[idx] = sym;
  }
}

static void *awq_decode_worker(void *arg) {
  awq_dec_job *j = (awq_dec_job *)arg;
  int64_t b = 0;
  for (int64_t g = j->lane_begin; g < j->lane_end; ++g) {
    while (j->lane_prefix[b + 1] <= g) ++b;
    awq_decode_lane(j, b, g - j->lane_prefix[b]);
  }
  return NULL;
}

/* group_col == NULL: bucket layout (col_start/col_len per bucket);
   otherwise by-scale layout (group_col per group, group_size columns each). */
int orc_awq_decode(const uint8_t *qv, const uint64_t *bs, int64_t W, const uint16_t *syms, const uint8_t *lens,
                   int64_t G, const int32_t *bucket_table, const int32_t *col_start, const int32_t *col_len,
                   const int32_t *row_off, const int32_t *row_idx, int64_t R, const int32_t *group_col,
                   int64_t group_size, const uint32_t *startbit, int64_t k, const int64_t *bit_base, int64_t B,
                   int64_t n, int64_t m, int nthreads, uint16_t *out) {
  g_awq_err[0] = 0;
  if (k < 1 || k > 1024) return awq_err(ORC_INVALID_ARGUMENT, "k must be in [1,1024]");
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  awq_dec_job base;
  memset(&base, 0, sizeof(base));
  base.qv = qv; base.bs = bs; base.W = W; base.syms = syms; base.lens = lens; base.G = G;
  base.btab = bucket_table; base.col_start = col_start; base.col_len = col_len; base.row_off = row_off;
  base.row_idx = row_idx; base.R = R; base.group_col = group_col; base.group_size = group_size;
  base.startbit = startbit; base.k = k; base.bit_base = bit_base; base.B = B; base.n = n; base.m = m;
  base.out = out;
  int64_t *lp = (int64_t *)malloc(sizeof(int64_t) * (size_t)(B + 1));
  if (!lp) return awq_err(ORC_NO_MEMORY, "out of memory");
  lp[0] = 0;
  for (int64_t b = 0; b < B; ++b) {
    int64_t ra, rows, c0, cl, ke = 0;
    if (awq_bucket(&base, b, &ra, &rows, &c0, &cl)) {
      const int64_t total = rows * cl;
      ke = total < k ? total : k;
      if (ke < 1) ke = 1;
    }
    lp[b + 1] = lp[b] + ke;
  }
  base.lane_prefix = lp;
  const int64_t lanes = lp[B];
  pthread_t th[256];
  int ok[256];
  awq_dec_job jobs[256];
  for (int i = 0; i < nthreads; ++i) {
    jobs[i] = base;
    jobs[i].lane_begin = lanes * i / nthreads;
    jobs[i].lane_end = lanes * (i + 1) / nthreads;
    ok[i] = 0;
    if (nthreads > 1 && pthread_create(&th[i], NULL, awq_decode_worker, &jobs[i]) == 0) ok[i] = 1;
    else awq_decode_worker(&jobs[i]);
  }
  for (int i = 0; i < nthreads; ++i) if (ok[i]) pthread_join(th[i], NULL);
  free(lp);
  return ORC_OK;
}
