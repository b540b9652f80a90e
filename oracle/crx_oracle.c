/*
 * crx_oracle.c -- CPU restatement of the crukx-sync update codec (format version 2).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the MI355X implementation in
 * crukx-sync_amd/.  Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * may load it, and only to check or to time the reference algorithm; the product never links,
 * loads or calls it.
 *
 * It restates, in plain sequential C, what the reference does with torch tensor ops.  Every
 * function cites the reference source it follows (paths relative to the reference repository).
 * Pinning (what checks each function against something other than this code):
 *   orc_weight / orc_checksum   published SplitMix64 outputs for seed 0 and the golden
 *                               checksums written by the reference (tests/golden).
 *   orc_huffman_lengths         golden vectors written by importing the reference
 *                               (codec.huffman_lengths), plus Kraft/optimality properties.
 *   orc_canonical_codes         golden vectors from codec.canonical_codes; prefix-freeness.
 *   orc_rice_param              golden vectors from codec._rice_params.
 *   orc_encode                  golden update bytes written by the reference's encode_update
 *                               on the same inputs (small cases byte-for-byte, large by SHA-256).
 *   orc_parse / orc_apply       the reference's hostile byte strings, golden updates applied
 *                               back to the new weights, every single-byte flip of a golden
 *                               update (reject-and-keep-old or still-exact).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_CORRUPT 1   /* CorruptUpdate in the reference */
#define ORC_VALUE 2     /* ValueError in the reference */
#define ORC_NOMEM 3

#define MAX_CODE_LEN 17   /* wire.py:10 */
#define MAX_SYMBOL 131070 /* wire.py:11 */
#define SYM_SPACE 131071  /* codec.py:18 */
#define MAX_RICE 30       /* wire.py:12 */
#define BLOCK 256         /* wire.py:13 */

static void set_err(char *err, size_t errlen, const char *msg) {
    if (err && errlen) {
        snprintf(err, errlen, "%s", msg);
    }
}

/* ------------------------------------------------------------------ checksum
 * codec.py:53-58 (_weights) and docs/FORMAT.md:61-64: w_i = splitmix64(i) | 1 with
 * z = (i+1)*0x9E3779B97F4A7C15, two xor-shift-multiply rounds, final xor-shift. */
uint64_t orc_weight(uint64_t i) {
    uint64_t z = (i + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return (z ^ (z >> 31)) | 1ULL;
}

/* codec.py:61-68: sum(u_i * w_i) mod 2^64 over the uint16 bit patterns. */
uint64_t orc_checksum(const uint16_t *u, uint64_t n) {
    uint64_t s = 0;
    for (uint64_t i = 0; i < n; i++) s += (uint64_t)u[i] * orc_weight(i);
    return s;
}

/* ------------------------------------------------------------------ Huffman
 * codec.py:81-98 (_huffman_unlimited): heapq over (count, id) pairs; leaves are ids 0..n-1 in
 * table order, merged nodes get ids n, n+1, ...; each pop takes the smallest (count, id) pair,
 * which is a total order, so any correct priority queue reproduces heapq's merge sequence.
 * Depth of a leaf = number of merges above it. */
typedef struct { unsigned __int128 c; int64_t id; } hnode; /* merged counts may pass 2^64; Python ints do not wrap */

static int hless(const hnode *a, const hnode *b) {
    return a->c < b->c || (a->c == b->c && a->id < b->id);
}

static void hpush(hnode *h, int64_t *n, hnode v) {
    int64_t i = (*n)++;
    while (i > 0) {
        int64_t p = (i - 1) / 2;
        if (!hless(&v, &h[p])) break;
        h[i] = h[p];
        i = p;
    }
    h[i] = v;
}

static hnode hpop(hnode *h, int64_t *n) {
    hnode top = h[0];
    hnode last = h[--(*n)];
    int64_t i = 0;
    for (;;) {
        int64_t l = 2 * i + 1, r = l + 1, m = i;
        const hnode *best = &last;
        if (l < *n && hless(&h[l], best)) { m = l; best = &h[l]; }
        if (r < *n && hless(&h[r], best)) { m = r; best = &h[r]; }
        if (m == i) break;
        h[i] = h[m];
        i = m;
    }
    if (*n > 0) h[i] = last;
    return top;
}

static int huffman_unlimited(const uint64_t *counts, int64_t n, int64_t *depth_out) {
    if (n == 1) { depth_out[0] = 1; return ORC_OK; }
    hnode *h = malloc(sizeof(hnode) * (size_t)n);
    int64_t *parent = malloc(sizeof(int64_t) * (size_t)(2 * n - 1));
    int64_t *depth = malloc(sizeof(int64_t) * (size_t)(2 * n - 1));
    if (!h || !parent || !depth) { free(h); free(parent); free(depth); return ORC_NOMEM; }
    int64_t hn = 0;
    for (int64_t i = 0; i < n; i++) { hnode v = {counts[i], i}; hpush(h, &hn, v); }
    int64_t nxt = n;
    while (hn > 1) {
        hnode a = hpop(h, &hn), b = hpop(h, &hn);
        parent[a.id] = parent[b.id] = nxt;
        hnode m = {a.c + b.c, nxt};
        hpush(h, &hn, m);
        nxt++;
    }
    depth[2 * n - 2] = 0; /* root: the last merged node */
    for (int64_t node = 2 * n - 3; node >= 0; node--) depth[node] = depth[parent[node]] + 1;
    for (int64_t i = 0; i < n; i++) depth_out[i] = depth[i];
    free(h); free(parent); free(depth);
    return ORC_OK;
}

/* codec.py:71-78 (huffman_lengths): up to 8 rounds of c -> max(1, c >> 2) while the longest code
 * exceeds MAX_CODE_LEN, then equal lengths max(1, bit_length(n-1)). */
int orc_huffman_lengths(const uint64_t *counts_in, int64_t n, int32_t *lengths) {
    uint64_t *c = malloc(sizeof(uint64_t) * (size_t)n);
    int64_t *d = malloc(sizeof(int64_t) * (size_t)n);
    if (!c || !d) { free(c); free(d); return ORC_NOMEM; }
    memcpy(c, counts_in, sizeof(uint64_t) * (size_t)n);
    for (int round = 0; round < 8; round++) {
        if (huffman_unlimited(c, n, d) != ORC_OK) { free(c); free(d); return ORC_NOMEM; }
        int64_t mx = 0;
        for (int64_t i = 0; i < n; i++) mx = d[i] > mx ? d[i] : mx;
        if (mx <= MAX_CODE_LEN) {
            for (int64_t i = 0; i < n; i++) lengths[i] = (int32_t)d[i];
            free(c); free(d);
            return ORC_OK;
        }
        for (int64_t i = 0; i < n; i++) { uint64_t v = c[i] >> 2; c[i] = v ? v : 1; }
    }
    int32_t bl = 0;
    for (uint64_t v = (uint64_t)(n - 1); v; v >>= 1) bl++;
    for (int64_t i = 0; i < n; i++) lengths[i] = bl > 1 ? bl : 1;
    free(c); free(d);
    return ORC_OK;
}

/* codec.py:101-111 (canonical_codes): codes in order of (length, position in the table). */
static const int32_t *g_sort_len;
static int cmp_len_pos(const void *a, const void *b) {
    int64_t i = *(const int64_t *)a, j = *(const int64_t *)b;
    if (g_sort_len[i] != g_sort_len[j]) return g_sort_len[i] < g_sort_len[j] ? -1 : 1;
    return i < j ? -1 : (i > j);
}

int orc_canonical_codes(const int32_t *lengths, int64_t n, uint32_t *codes) {
    int64_t *order = malloc(sizeof(int64_t) * (size_t)n);
    if (!order) return ORC_NOMEM;
    for (int64_t i = 0; i < n; i++) order[i] = i;
    g_sort_len = lengths;
    qsort(order, (size_t)n, sizeof(int64_t), cmp_len_pos);
    uint64_t code = 0;
    int32_t prev = lengths[order[0]];
    for (int64_t k = 0; k < n; k++) {
        int64_t i = order[k];
        if (k) code = (code + 1) << (lengths[i] - prev);
        codes[i] = (uint32_t)code;
        prev = lengths[i];
    }
    free(order);
    return ORC_OK;
}

/* ------------------------------------------------------------------ Rice parameter
 * codec.py:268-275 (_rice_params) for one group: mean gap in fp64, r0 = floor(log2(max(mean,1)))
 * clamped to [0, 30]; the cheapest of {r0-1, r0, r0+1} (clamped) by exact bit cost
 * sum((gap >> r) + 1 + r), first minimum wins (argmin). */
int32_t orc_rice_param(const int64_t *gaps, int64_t count) {
    int64_t s = 0;
    for (int64_t i = 0; i < count; i++) s += gaps[i];
    double mean = (double)s / (double)count;
    double m = mean < 1.0 ? 1.0 : mean;
    int64_t r0 = (int64_t)floor(log2(m));
    if (r0 < 0) r0 = 0;
    if (r0 > MAX_RICE) r0 = MAX_RICE;
    int64_t cand[3] = {r0 - 1 < 0 ? 0 : r0 - 1, r0, r0 + 1 > MAX_RICE ? MAX_RICE : r0 + 1};
    int64_t best = 0, best_cost = 0;
    for (int k = 0; k < 3; k++) {
        int64_t cost = 0;
        for (int64_t i = 0; i < count; i++) cost += (gaps[i] >> cand[k]) + 1 + cand[k];
        if (k == 0 || cost < best_cost) { best = k; best_cost = cost; }
    }
    return (int32_t)cand[best];
}

/* ------------------------------------------------------------------ byte buffer + varints */
typedef struct { uint8_t *p; size_t n, cap; int oom; } bbuf;

static void bb_reserve(bbuf *b, size_t extra) {
    if (b->oom) return;
    if (b->n + extra <= b->cap) return;
    size_t cap = b->cap ? b->cap : 256;
    while (cap < b->n + extra) cap *= 2;
    uint8_t *q = realloc(b->p, cap);
    if (!q) { b->oom = 1; return; }
    b->p = q;
    b->cap = cap;
}

static void bb_put(bbuf *b, const void *src, size_t n) {
    bb_reserve(b, n);
    if (b->oom) return;
    memcpy(b->p + b->n, src, n);
    b->n += n;
}

static void bb_u8(bbuf *b, uint8_t v) { bb_put(b, &v, 1); }

/* wire.py:55-61 (write_varint): unsigned LEB128, values must be < 2^63. */
static int bb_varint(bbuf *b, uint64_t v) {
    if (v >= (1ULL << 63)) return ORC_VALUE;
    while (v >= 0x80) { bb_u8(b, (uint8_t)((v & 0x7F) | 0x80)); v >>= 7; }
    bb_u8(b, (uint8_t)v);
    return ORC_OK;
}

static void bb_u32le(bbuf *b, uint32_t v) {
    uint8_t t[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    bb_put(b, t, 4);
}

static void bb_u64le(bbuf *b, uint64_t v) {
    uint8_t t[8];
    for (int k = 0; k < 8; k++) t[k] = (uint8_t)(v >> (8 * k));
    bb_put(b, t, 8);
}

/* MSB-first bit writer (docs/FORMAT.md:37-44; codec.py:218-257 writes the same bits). */
typedef struct { uint8_t *p; uint64_t nbits, capbits; int oom; } bitw;

static void bw_reserve(bitw *w, uint64_t extra) {
    if (w->oom) return;
    if (w->nbits + extra <= w->capbits) return;
    uint64_t cap = w->capbits ? w->capbits : 4096;
    while (cap < w->nbits + extra) cap *= 2;
    size_t oldbytes = w->capbits ? (size_t)(w->capbits / 8 + 8) : 0;
    size_t newbytes = (size_t)(cap / 8 + 8);
    uint8_t *q = realloc(w->p, newbytes);
    if (!q) { w->oom = 1; return; }
    memset(q + oldbytes, 0, newbytes - oldbytes);
    w->p = q;
    w->capbits = cap;
}

static void bw_bits(bitw *w, uint64_t v, int n) { /* n <= 64, MSB first */
    bw_reserve(w, (uint64_t)n);
    if (w->oom) return;
    for (int k = n - 1; k >= 0; k--) {
        if ((v >> k) & 1) w->p[w->nbits >> 3] |= (uint8_t)(0x80 >> (w->nbits & 7));
        w->nbits++;
    }
}

static void bw_ones(bitw *w, uint64_t q) {
    bw_reserve(w, q);
    if (w->oom) return;
    while (q && (w->nbits & 7)) { w->p[w->nbits >> 3] |= (uint8_t)(0x80 >> (w->nbits & 7)); w->nbits++; q--; }
    while (q >= 8) { w->p[w->nbits >> 3] = 0xFF; w->nbits += 8; q -= 8; }
    while (q) { w->p[w->nbits >> 3] |= (uint8_t)(0x80 >> (w->nbits & 7)); w->nbits++; q--; }
}

/* ------------------------------------------------------------------ encoder
 * codec.py:278-420 (encode) + wire.py:64-89 (serialize), restated per tensor:
 *  - tensors in the caller's order, only those with a changed element (codec.py:295-301);
 *  - changes taken in stable exponent order of old (codec.py:133-147, docs/FORMAT.md:21-24):
 *    local index = number of earlier elements with the same old exponent;
 *  - gap = local - previous local - 1 (first: local), residual zz = zigzag(new - old) on the
 *    sign-extended int16 bits (codec.py:317-330);
 *  - checksum delta sum((new_u - old_u) * w(pos)) (codec.py:325), new checksum = cache + delta or
 *    a full pass over new (codec.py:344-352);
 *  - one Rice parameter per group (codec.py:358-360), one Huffman table per exponent over all
 *    tensors, symbols ascending (codec.py:354-392), codes canonical (codec.py:388);
 *  - bits per change: Rice gap then Huffman code, MSB first; block_bits per 256 changes of a
 *    group; a block of 2^32 bits or more is a ValueError (codec.py:394-420). */
typedef struct { int32_t e; uint32_t zz; int64_t gap; } chg_rec;
typedef struct { uint64_t key; uint64_t count; } keycnt;

static int cmp_u64(const void *a, const void *b) {
    uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : (x > y);
}

static int64_t find_key(const keycnt *k, int64_t n, uint64_t key) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        int64_t mid = (lo + hi) / 2;
        if (k[mid].key < key) lo = mid + 1; else hi = mid;
    }
    return lo;
}

typedef struct {
    int64_t n_changes;   /* total changes in the tensor */
    chg_rec *recs;       /* in group order */
    int32_t n_groups;
    int32_t g_exp[256];
    int64_t g_count[256];
    int32_t g_rice[256];
    uint64_t checksum;
} tens_enc;

int orc_encode(int32_t n, const char *const *names, const uint64_t *name_lens,
               const uint16_t *const *olds, const uint16_t *const *news, const uint64_t *numels,
               const int32_t *has_cache, const uint64_t *cache_vals,
               uint8_t **out, uint64_t *out_len, uint64_t *new_chk, int32_t *present,
               char *err, uint64_t errlen) {
    *out = NULL;
    *out_len = 0;
    tens_enc *te = calloc((size_t)(n > 0 ? n : 1), sizeof(tens_enc));
    if (!te) return ORC_NOMEM;
    int rc = ORC_OK;
    int64_t total_changes = 0;
    for (int32_t t = 0; t < n; t++) {
        present[t] = 0;
        const uint16_t *a = olds[t], *b = news[t];
        uint64_t N = numels[t];
        int64_t nc = 0;
        for (uint64_t i = 0; i < N; i++) nc += a[i] != b[i];
        if (!nc) continue;
        present[t] = 1;
        /* stable exponent ranks of the changed elements, then bucket by exponent */
        int64_t seen[256] = {0}, chg_per_e[256] = {0};
        int64_t *rank = malloc(sizeof(int64_t) * (size_t)nc);
        int32_t *ex = malloc(sizeof(int32_t) * (size_t)nc);
        uint64_t *pos = malloc(sizeof(uint64_t) * (size_t)nc);
        chg_rec *recs = malloc(sizeof(chg_rec) * (size_t)nc);
        if (!rank || !ex || !pos || !recs) { free(rank); free(ex); free(pos); free(recs); rc = ORC_NOMEM; goto done; }
        int64_t k = 0;
        for (uint64_t i = 0; i < N; i++) {
            int32_t e = (a[i] >> 7) & 0xFF;
            if (a[i] != b[i]) { rank[k] = seen[e]; ex[k] = e; pos[k] = i; chg_per_e[e]++; k++; }
            seen[e]++;
        }
        int64_t start[257];
        start[0] = 0;
        for (int e = 0; e < 256; e++) start[e + 1] = start[e] + chg_per_e[e];
        int64_t fill[256];
        memcpy(fill, start, sizeof(fill));
        uint64_t delta = 0;
        int64_t prev_rank[256];
        for (int e = 0; e < 256; e++) prev_rank[e] = -1;
        /* position order within an exponent is rank order, so a stable bucket gives group order */
        for (int64_t j = 0; j < nc; j++) {
            int32_t e = ex[j];
            int64_t d = fill[e]++;
            int16_t va = (int16_t)a[pos[j]], vb = (int16_t)b[pos[j]];
            int64_t res = (int64_t)vb - (int64_t)va;
            recs[d].e = e;
            recs[d].zz = (uint32_t)(res >= 0 ? 2 * res : -2 * res - 1);
            recs[d].gap = rank[j] - prev_rank[e] - 1;
            prev_rank[e] = rank[j];
            delta += (uint64_t)((int64_t)b[pos[j]] - (int64_t)a[pos[j]]) * orc_weight(pos[j]);
        }
        free(rank); free(ex); free(pos);
        te[t].recs = recs;
        te[t].n_changes = nc;
        int32_t ng = 0;
        for (int e = 0; e < 256; e++) {
            if (!chg_per_e[e]) continue;
            te[t].g_exp[ng] = e;
            te[t].g_count[ng] = chg_per_e[e];
            int64_t *gg = malloc(sizeof(int64_t) * (size_t)chg_per_e[e]);
            if (!gg) { rc = ORC_NOMEM; goto done; }
            for (int64_t j = 0; j < chg_per_e[e]; j++) gg[j] = recs[start[e] + j].gap;
            te[t].g_rice[ng] = orc_rice_param(gg, chg_per_e[e]);
            free(gg);
            ng++;
        }
        te[t].n_groups = ng;
        te[t].checksum = (has_cache && has_cache[t]) ? cache_vals[t] + delta : orc_checksum(b, N);
        new_chk[t] = te[t].checksum;
        total_changes += nc;
    }
    {
        bbuf ob = {0};
        if (total_changes == 0) { /* codec.py:299-301: Update([], []) */
            bb_put(&ob, "CRXS", 4); bb_u8(&ob, 2); bb_varint(&ob, 0); bb_varint(&ob, 0); bb_varint(&ob, 0);
            if (ob.oom) { free(ob.p); rc = ORC_NOMEM; goto done; }
            *out = ob.p; *out_len = ob.n;
            goto done;
        }
        /* residual symbol counts per exponent over the whole update */
        uint64_t *keys = malloc(sizeof(uint64_t) * (size_t)total_changes);
        if (!keys) { rc = ORC_NOMEM; goto done; }
        int64_t kk = 0;
        for (int32_t t = 0; t < n; t++)
            for (int64_t j = 0; j < te[t].n_changes; j++)
                keys[kk++] = (uint64_t)te[t].recs[j].e * SYM_SPACE + te[t].recs[j].zz;
        qsort(keys, (size_t)total_changes, sizeof(uint64_t), cmp_u64);
        keycnt *kc = malloc(sizeof(keycnt) * (size_t)total_changes);
        if (!kc) { free(keys); rc = ORC_NOMEM; goto done; }
        int64_t nk = 0;
        for (int64_t j = 0; j < total_changes; j++) {
            if (nk && kc[nk - 1].key == keys[j]) kc[nk - 1].count++;
            else { kc[nk].key = keys[j]; kc[nk].count = 1; nk++; }
        }
        free(keys);
        uint32_t *code_of = malloc(sizeof(uint32_t) * (size_t)nk);
        int32_t *len_of = malloc(sizeof(int32_t) * (size_t)nk);
        uint64_t *cnts = malloc(sizeof(uint64_t) * (size_t)nk);
        if (!code_of || !len_of || !cnts) { free(kc); free(code_of); free(len_of); free(cnts); rc = ORC_NOMEM; goto done; }
        int32_t n_tables = 0;
        for (int64_t lo = 0; lo < nk;) {
            uint64_t e = kc[lo].key / SYM_SPACE;
            int64_t hi = lo;
            while (hi < nk && kc[hi].key / SYM_SPACE == e) hi++;
            for (int64_t j = lo; j < hi; j++) cnts[j - lo] = kc[j].count;
            if (orc_huffman_lengths(cnts, hi - lo, len_of + lo) != ORC_OK ||
                orc_canonical_codes(len_of + lo, hi - lo, code_of + lo) != ORC_OK) {
                free(kc); free(code_of); free(len_of); free(cnts); rc = ORC_NOMEM; goto done;
            }
            n_tables++;
            lo = hi;
        }
        free(cnts);
        /* header (wire.py:64-89) */
        bb_put(&ob, "CRXS", 4);
        bb_u8(&ob, 2);
        bb_varint(&ob, (uint64_t)n_tables);
        for (int64_t lo = 0; lo < nk;) {
            uint64_t e = kc[lo].key / SYM_SPACE;
            int64_t hi = lo;
            while (hi < nk && kc[hi].key / SYM_SPACE == e) hi++;
            bb_u8(&ob, (uint8_t)e);
            bb_varint(&ob, (uint64_t)(hi - lo));
            for (int64_t j = lo; j < hi; j++) { bb_varint(&ob, kc[j].key % SYM_SPACE); bb_u8(&ob, (uint8_t)len_of[j]); }
            lo = hi;
        }
        int32_t n_present = 0;
        for (int32_t t = 0; t < n; t++) n_present += present[t];
        bb_varint(&ob, (uint64_t)n_present);
        uint64_t n_blocks = 0;
        for (int32_t t = 0; t < n; t++) {
            if (!present[t]) continue;
            bb_varint(&ob, name_lens[t]);
            bb_put(&ob, names[t], (size_t)name_lens[t]);
            bb_varint(&ob, numels[t]);
            bb_u64le(&ob, te[t].checksum);
            bb_varint(&ob, (uint64_t)te[t].n_groups);
            for (int32_t g = 0; g < te[t].n_groups; g++) {
                bb_u8(&ob, (uint8_t)te[t].g_exp[g]);
                bb_varint(&ob, (uint64_t)te[t].g_count[g]);
                bb_u8(&ob, (uint8_t)te[t].g_rice[g]);
                n_blocks += (uint64_t)((te[t].g_count[g] + BLOCK - 1) / BLOCK);
            }
        }
        /* payload + block table */
        uint64_t *bb = malloc(sizeof(uint64_t) * (size_t)(n_blocks ? n_blocks : 1));
        bitw w = {0};
        uint64_t bi = 0;
        for (int32_t t = 0; t < n && bb; t++) {
            if (!present[t]) continue;
            int64_t j = 0;
            for (int32_t g = 0; g < te[t].n_groups; g++) {
                int32_t r = te[t].g_rice[g];
                for (int64_t c = 0; c < te[t].g_count[g]; c++, j++) {
                    if (c % BLOCK == 0) bb[bi++] = w.nbits;
                    const chg_rec *x = &te[t].recs[j];
                    int64_t kix = find_key(kc, nk, (uint64_t)x->e * SYM_SPACE + x->zz);
                    bw_ones(&w, (uint64_t)(x->gap >> r));
                    bw_bits(&w, 0, 1);
                    if (r) bw_bits(&w, (uint64_t)x->gap & ((1ULL << r) - 1), r);
                    bw_bits(&w, code_of[kix], len_of[kix]);
                }
            }
        }
        free(kc); free(code_of); free(len_of);
        if (!bb || w.oom) { free(bb); free(w.p); free(ob.p); rc = ORC_NOMEM; goto done; }
        for (uint64_t b2 = 0; b2 < n_blocks; b2++) {
            uint64_t endb = b2 + 1 < n_blocks ? bb[b2 + 1] : w.nbits;
            uint64_t len = endb - bb[b2];
            if (len >= (1ULL << 32)) {
                set_err(err, errlen, "a block exceeds 2^32 bits; the update cannot be represented");
                free(bb); free(w.p); free(ob.p); rc = ORC_VALUE; goto done;
            }
            bb_u32le(&ob, (uint32_t)len);
        }
        free(bb);
        uint64_t plen = (w.nbits + 7) / 8;
        bb_varint(&ob, plen);
        if (plen) bb_put(&ob, w.p, (size_t)plen);
        free(w.p);
        if (ob.oom) { free(ob.p); rc = ORC_NOMEM; goto done; }
        *out = ob.p;
        *out_len = ob.n;
    }
done:
    for (int32_t t = 0; t < n; t++) free(te[t].recs);
    free(te);
    return rc;
}

void orc_free(void *p) { free(p); }

/* ------------------------------------------------------------------ parser
 * wire.py:92-212 (_Reader, parse), every check in the same order; any failure is CorruptUpdate.
 * Kraft's inequality is checked exactly: every 2^-L with L <= 17 is a multiple of 2^-17, so the
 * reference's fp64 sum (wire.py:206) is exact and "> 1 + 1e-12" means "> 2^17 in units of 2^-17". */
typedef struct { int exponent; int64_t n_sym; uint64_t *syms; uint8_t *lens; } p_table;
typedef struct { int exponent; uint64_t count; int rice; } p_group;
typedef struct {
    const uint8_t *name; uint64_t name_len; uint64_t numel; uint64_t checksum;
    int n_groups; p_group groups[256];
} p_tensor;
typedef struct {
    int n_tables; p_table tables[256];
    int64_t n_tensors; p_tensor *tensors;
    uint64_t n_blocks; const uint8_t *block_bits; /* n_blocks u32 little-endian */
    uint64_t payload_len; const uint8_t *payload;
} p_update;

typedef struct { const uint8_t *d; uint64_t n, pos; } reader;

static int rd_take(reader *r, uint64_t n, const uint8_t **p) {
    if (n > r->n - r->pos) return ORC_CORRUPT;
    *p = r->d + r->pos;
    r->pos += n;
    return ORC_OK;
}

static int rd_u8(reader *r, int *v) {
    const uint8_t *p;
    if (rd_take(r, 1, &p)) return ORC_CORRUPT;
    *v = p[0];
    return ORC_OK;
}

static int rd_varint(reader *r, uint64_t *out) {
    uint64_t v = 0;
    int shift = 0;
    for (;;) {
        int b;
        if (rd_u8(r, &b)) return ORC_CORRUPT;
        uint64_t bits = (uint64_t)(b & 0x7F);
        if (bits) {
            if (shift >= 63) return ORC_CORRUPT;            /* v >= 2^63 */
            v |= bits << shift;
            if (v >= (1ULL << 63)) return ORC_CORRUPT;
        }
        if (!(b & 0x80)) { *out = v; return ORC_OK; }
        shift += 7;
        if (shift > 63) return ORC_CORRUPT;
    }
}

static void free_update(p_update *u) {
    for (int i = 0; i < u->n_tables; i++) { free(u->tables[i].syms); free(u->tables[i].lens); }
    free(u->tensors);
    free(u);
}

/* strict UTF-8 as Python's bytes.decode("utf-8") */
static int utf8_ok(const uint8_t *s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        uint8_t c = s[i];
        if (c < 0x80) { i++; continue; }
        int len;
        uint32_t cp, min;
        if (c >= 0xC2 && c <= 0xDF) { len = 2; cp = c & 0x1F; min = 0x80; }
        else if (c >= 0xE0 && c <= 0xEF) { len = 3; cp = c & 0x0F; min = 0x800; }
        else if (c >= 0xF0 && c <= 0xF4) { len = 4; cp = c & 0x07; min = 0x10000; }
        else return 0;
        if (i + (uint64_t)len > n) return 0;
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0) != 0x80) return 0;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return 0;
        i += (uint64_t)len;
    }
    return 1;
}

static int cmp_u64v(const void *a, const void *b) { return cmp_u64(a, b); }

static int parse_update(const uint8_t *data, uint64_t len, p_update **out, char *err, uint64_t errlen) {
    reader r = {data, len, 0};
    p_update *u = calloc(1, sizeof(p_update));
    if (!u) return ORC_NOMEM;
    const uint8_t *p;
    int b;

#define FAIL(msg) do { set_err(err, errlen, msg); free_update(u); return ORC_CORRUPT; } while (0)
    if (rd_take(&r, 4, &p)) FAIL("update is truncated");
    if (memcmp(p, "CRXS", 4)) FAIL("not a crukx-sync update");
    if (rd_u8(&r, &b)) FAIL("update is truncated");
    if (b != 2) FAIL("unsupported format version");
    uint64_t n_tables;
    if (rd_varint(&r, &n_tables)) FAIL("bad varint");
    if (n_tables > 256) FAIL("too many tables");
    int have_table[256] = {0};
    for (uint64_t ti = 0; ti < n_tables; ti++) {
        int exp;
        uint64_t n_sym;
        if (rd_u8(&r, &exp) || rd_varint(&r, &n_sym)) FAIL("bad table header");
        uint64_t lim = (uint64_t)(MAX_SYMBOL + 1);
        uint64_t half = (r.n - r.pos) / 2;
        if (half < lim) lim = half;
        if (have_table[exp] || !(n_sym > 0 && n_sym <= lim)) FAIL("bad table header");
        have_table[exp] = 1;
        p_table *tb = &u->tables[u->n_tables++];
        tb->exponent = exp;
        tb->n_sym = (int64_t)n_sym;
        tb->syms = malloc(sizeof(uint64_t) * (size_t)n_sym);
        tb->lens = malloc((size_t)n_sym);
        if (!tb->syms || !tb->lens) { free_update(u); return ORC_NOMEM; }
        for (uint64_t k = 0; k < n_sym; k++) {
            int L;
            if (rd_varint(&r, &tb->syms[k]) || rd_u8(&r, &L)) FAIL("update is truncated");
            tb->lens[k] = (uint8_t)L;
        }
        uint64_t *sorted = malloc(sizeof(uint64_t) * (size_t)n_sym);
        if (!sorted) { free_update(u); return ORC_NOMEM; }
        memcpy(sorted, tb->syms, sizeof(uint64_t) * (size_t)n_sym);
        qsort(sorted, (size_t)n_sym, sizeof(uint64_t), cmp_u64v);
        int bad = sorted[n_sym - 1] > MAX_SYMBOL;
        for (uint64_t k = 1; k < n_sym; k++) bad |= sorted[k] == sorted[k - 1];
        free(sorted);
        if (bad) FAIL("bad table symbols");
        int mn = 255, mx = 0;
        uint64_t kraft = 0;
        for (uint64_t k = 0; k < n_sym; k++) {
            int L = tb->lens[k];
            mn = L < mn ? L : mn;
            mx = L > mx ? L : mx;
        }
        if (mn < 1 || mx > MAX_CODE_LEN) FAIL("bad Huffman code lengths");
        for (uint64_t k = 0; k < n_sym; k++) kraft += 1ULL << (MAX_CODE_LEN - tb->lens[k]);
        if (kraft > (1ULL << MAX_CODE_LEN)) FAIL("bad Huffman code lengths");
    }
    uint64_t n_tensors;
    if (rd_varint(&r, &n_tensors)) FAIL("bad varint");
    if (n_tensors > r.n - r.pos) FAIL("too many tensors");
    u->tensors = calloc((size_t)(n_tensors ? n_tensors : 1), sizeof(p_tensor));
    if (!u->tensors) { free_update(u); return ORC_NOMEM; }
    uint64_t total_blocks = 0;
    uint64_t per_exp[256] = {0};
    for (uint64_t i = 0; i < n_tensors; i++) {
        p_tensor *t = &u->tensors[i];
        uint64_t nl;
        if (rd_varint(&r, &nl) || rd_take(&r, nl, &p)) FAIL("update is truncated");
        if (!utf8_ok(p, nl)) FAIL("tensor name is not valid UTF-8");
        for (uint64_t j = 0; j < i; j++)
            if (u->tensors[j].name_len == nl && !memcmp(u->tensors[j].name, p, (size_t)nl)) FAIL("tensor appears twice");
        t->name = p;
        t->name_len = nl;
        u->n_tensors = (int64_t)i + 1;
        if (rd_varint(&r, &t->numel)) FAIL("bad varint");
        if (rd_take(&r, 8, &p)) FAIL("update is truncated");
        t->checksum = 0;
        for (int k = 0; k < 8; k++) t->checksum |= (uint64_t)p[k] << (8 * k);
        uint64_t ng;
        if (rd_varint(&r, &ng)) FAIL("bad varint");
        if (!(ng > 0 && ng <= 256)) FAIL("bad group count");
        int seen[256] = {0};
        uint64_t sum = 0;
        for (uint64_t g = 0; g < ng; g++) {
            int e, rice;
            uint64_t cnt;
            if (rd_u8(&r, &e) || rd_varint(&r, &cnt) || rd_u8(&r, &rice)) FAIL("update is truncated");
            if (seen[e] || !have_table[e]) FAIL("bad group exponent");
            if (!(cnt > 0 && cnt <= t->numel) || rice > MAX_RICE) FAIL("bad group header");
            seen[e] = 1;
            t->groups[g].exponent = e;
            t->groups[g].count = cnt;
            t->groups[g].rice = rice;
            total_blocks += (cnt + BLOCK - 1) / BLOCK;      /* each term < 2^55 */
            if (total_blocks > (1ULL << 62)) total_blocks = 1ULL << 62;  /* Python ints do not wrap */
            sum += cnt;                                      /* cnt <= numel < 2^63 */
            if (sum > (1ULL << 63)) sum = 1ULL << 63;
        }
        t->n_groups = (int)ng;
        if (sum > t->numel) FAIL("more changes than elements");
        for (uint64_t g = 0; g < ng; g++) {
            uint64_t *pe = &per_exp[t->groups[g].exponent];
            *pe += t->groups[g].count;
            if (*pe > (1ULL << 63)) *pe = 1ULL << 63;
        }
    }
    for (int ti = 0; ti < u->n_tables; ti++)
        if ((uint64_t)u->tables[ti].n_sym > per_exp[u->tables[ti].exponent]) FAIL("table unused or larger than its changes");
    if (total_blocks > (r.n - r.pos) / 4) FAIL("block table longer than the update"); /* 4*blocks > remaining */
    if (rd_take(&r, 4 * total_blocks, &u->block_bits)) FAIL("update is truncated");
    u->n_blocks = total_blocks;
    uint64_t plen;
    if (rd_varint(&r, &plen)) FAIL("bad varint");
    if (rd_take(&r, plen, &u->payload)) FAIL("update is truncated");
    u->payload_len = plen;
    if (r.pos != r.n) FAIL("trailing bytes after the payload");
    uint64_t total_bits = 0;
    for (uint64_t k = 0; k < total_blocks; k++) {
        const uint8_t *q = u->block_bits + 4 * k;
        total_bits += (uint64_t)q[0] | (uint64_t)q[1] << 8 | (uint64_t)q[2] << 16 | (uint64_t)q[3] << 24;
    }
    if ((total_bits + 7) / 8 != plen) FAIL("payload length does not match its block table");
    if (total_bits % 8 && (u->payload[plen - 1] & ((1u << (8 - total_bits % 8)) - 1))) FAIL("non-zero padding bits");
    uint64_t bi = 0;
    for (int64_t i = 0; i < u->n_tensors; i++)
        for (int g = 0; g < u->tensors[i].n_groups; g++) {
            const p_group *gr = &u->tensors[i].groups[g];
            for (uint64_t k = 0; k < (gr->count + BLOCK - 1) / BLOCK; k++, bi++) {
                const uint8_t *q = u->block_bits + 4 * bi;
                uint64_t bits = (uint64_t)q[0] | (uint64_t)q[1] << 8 | (uint64_t)q[2] << 16 | (uint64_t)q[3] << 24;
                uint64_t m = gr->count - k * BLOCK;
                if (m > BLOCK) m = BLOCK;
                if (bits < m * (uint64_t)(2 + gr->rice)) FAIL("block shorter than its symbols could be");
            }
        }
#undef FAIL
    *out = u;
    return ORC_OK;
}

/* Parse only (the structural checks of wire.parse).  Returns ORC_OK or ORC_CORRUPT. */
int orc_parse_check(const uint8_t *data, uint64_t len, char *err, uint64_t errlen) {
    p_update *u = NULL;
    int rc = parse_update(data, len, &u, err, errlen);
    if (rc == ORC_OK) free_update(u);
    return rc;
}

/* ------------------------------------------------------------------ apply
 * codec.py:578-717 (apply) with the decoder semantics of codec.py:504-575 / _triton.py:33-88:
 *  - per block, `count` times: the symbol must start before the block end; unary run of ones
 *    (q), bounded by q_max = group size >> rice (codec.py:616); a zero; rice bits; a canonical
 *    Huffman code found by length 1..17 (codec.py:434-454,524-530); the block must end exactly at
 *    its declared length (codec.py:535).  Bits past the payload read as zero (codec.py:478-482).
 *  - local = running sum of (gap + 1) - 1 within the group (codec.py:640-642) and must stay below
 *    the group size (codec.py:696-697);
 *  - the change goes to the position holding the local-th element of the group in the stable
 *    exponent order of the receiver's old weights (codec.py:654-694, docs/FORMAT.md:21-24);
 *  - new_u = (old_u + unzigzag(zz)) mod 2^16 (codec.py:698); per tensor the cached or full old
 *    checksum plus sum((new_u - old_u) * w(pos)) must equal the header checksum
 *    (codec.py:699-708); any failure writes nothing (codec.py:709-714).
 * Acceptance is the reference's: its flags differ only in when they fire, not in the verdict
 * (every flagged condition ends in CorruptUpdate). */
typedef struct { const uint8_t *p; uint64_t nbytes; } bitsrc;

static inline int bit_at(const bitsrc *s, uint64_t pos) {
    uint64_t byte = pos >> 3;
    if (byte >= s->nbytes) return 0;
    return (s->p[byte] >> (7 - (pos & 7))) & 1;
}

static inline uint64_t bits_at(const bitsrc *s, uint64_t pos, int n) {
    uint64_t v = 0;
    for (int k = 0; k < n; k++) v = (v << 1) | (uint64_t)bit_at(s, pos + (uint64_t)k);
    return v;
}

typedef struct { uint64_t first[MAX_CODE_LEN + 1], count[MAX_CODE_LEN + 1], base[MAX_CODE_LEN + 1]; uint64_t *syms; } canon;

static int build_canon(const p_table *t, canon *c) {
    /* codec.py:434-454 */
    int64_t n = t->n_sym;
    int32_t *lens = malloc(sizeof(int32_t) * (size_t)n);
    int64_t *order = malloc(sizeof(int64_t) * (size_t)n);
    c->syms = malloc(sizeof(uint64_t) * (size_t)n);
    if (!lens || !order || !c->syms) { free(lens); free(order); free(c->syms); c->syms = NULL; return ORC_NOMEM; }
    uint64_t per_len[MAX_CODE_LEN + 1] = {0};
    for (int64_t i = 0; i < n; i++) { lens[i] = t->lens[i]; per_len[lens[i]]++; order[i] = i; }
    g_sort_len = lens;
    qsort(order, (size_t)n, sizeof(int64_t), cmp_len_pos);
    uint64_t code = 0, idx = 0;
    for (int L = 1; L <= MAX_CODE_LEN; L++) {
        c->first[L] = code;
        c->count[L] = per_len[L];
        c->base[L] = idx;
        code = (code + per_len[L]) << 1;
        idx += per_len[L];
    }
    for (int64_t i = 0; i < n; i++) c->syms[i] = t->syms[order[i]];
    free(lens); free(order);
    return ORC_OK;
}

int orc_apply(const uint8_t *data, uint64_t len, int32_t n_targets, const char *const *names,
              const uint64_t *name_lens, uint16_t *const *datas, const uint64_t *numels,
              const int32_t *has_cache, const uint64_t *cache_vals,
              uint64_t *changed_out, int32_t *n_tensors_out, int32_t *tensor_target,
              uint64_t *tensor_checksum, char *err, uint64_t errlen) {
    p_update *u = NULL;
    int rc = parse_update(data, len, &u, err, errlen);
    if (rc) return rc;
    *changed_out = 0;
    *n_tensors_out = (int32_t)u->n_tensors;
    if (u->n_tensors == 0) { free_update(u); return ORC_OK; }
    int64_t T = u->n_tensors;
    for (int64_t i = 0; i < T; i++) {
        int32_t found = -1;
        for (int32_t j = 0; j < n_targets; j++)
            if (name_lens[j] == u->tensors[i].name_len && !memcmp(names[j], u->tensors[i].name, (size_t)name_lens[j])) { found = j; break; }
        if (found < 0) { set_err(err, errlen, "update has a tensor that the receiver does not have"); free_update(u); return ORC_VALUE; }
        if (numels[found] != u->tensors[i].numel) { set_err(err, errlen, "numel mismatch"); free_update(u); return ORC_VALUE; }
        tensor_target[i] = found;
        tensor_checksum[i] = u->tensors[i].checksum;
    }
    canon *cn = calloc((size_t)u->n_tables, sizeof(canon));
    int table_of[256];
    for (int e = 0; e < 256; e++) table_of[e] = -1;
    for (int k = 0; k < u->n_tables; k++) {
        table_of[u->tables[k].exponent] = k;
        if (build_canon(&u->tables[k], &cn[k])) { rc = ORC_NOMEM; goto out; }
    }
    bitsrc src = {u->payload, u->payload_len};
    uint64_t cur = 0, bi = 0, total = 0;
    for (int64_t i = 0; i < T; i++)
        for (int g = 0; g < u->tensors[i].n_groups; g++) total += u->tensors[i].groups[g].count;
    uint64_t *idx = malloc(sizeof(uint64_t) * (size_t)(total ? total : 1));
    uint16_t *val = malloc(sizeof(uint16_t) * (size_t)(total ? total : 1));
    if (!idx || !val) { free(idx); free(val); rc = ORC_NOMEM; goto out; }
    int bad = 0;
    uint64_t el = 0;
    for (int64_t i = 0; i < T && !bad; i++) {
        const p_tensor *t = &u->tensors[i];
        const uint16_t *a = datas[tensor_target[i]];
        uint64_t N = t->numel;
        /* the receiver's exponent groups: sizes and positions in stable order */
        uint64_t size[256] = {0};
        for (uint64_t p2 = 0; p2 < N; p2++) size[(a[p2] >> 7) & 0xFF]++;
        uint64_t gstart[257];
        gstart[0] = 0;
        for (int e = 0; e < 256; e++) gstart[e + 1] = gstart[e] + size[e];
        uint64_t *ord = malloc(sizeof(uint64_t) * (size_t)(N ? N : 1));
        if (!ord) { rc = ORC_NOMEM; free(idx); free(val); goto out; }
        uint64_t fillp[256];
        memcpy(fillp, gstart, sizeof(fillp));
        for (uint64_t p2 = 0; p2 < N; p2++) ord[fillp[(a[p2] >> 7) & 0xFF]++] = p2;
        uint64_t dsum = 0;
        for (int g = 0; g < t->n_groups && !bad; g++) {
            const p_group *gr = &t->groups[g];
            const canon *c = &cn[table_of[gr->exponent]];
            uint64_t gsize = size[gr->exponent];
            if (gr->count > gsize) { bad = 1; break; }
            uint64_t qmax = gsize >> gr->rice;
            uint64_t local = 0;
            int first = 1;
            for (uint64_t k = 0; k < (gr->count + BLOCK - 1) / BLOCK && !bad; k++, bi++) {
                const uint8_t *q8 = u->block_bits + 4 * bi;
                uint64_t bbits = (uint64_t)q8[0] | (uint64_t)q8[1] << 8 | (uint64_t)q8[2] << 16 | (uint64_t)q8[3] << 24;
                uint64_t end = cur + bbits;
                uint64_t m = gr->count - k * BLOCK;
                if (m > BLOCK) m = BLOCK;
                for (uint64_t s = 0; s < m; s++) {
                    if (cur >= end) { bad = 1; break; }
                    uint64_t q = 0;
                    while (bit_at(&src, cur + q)) {
                        q++;
                        if (q > qmax) break;
                    }
                    if (q > qmax) { bad = 1; break; }
                    uint64_t c2 = cur + q + 1;
                    uint64_t rem = gr->rice ? bits_at(&src, c2, gr->rice) : 0;
                    c2 += (uint64_t)gr->rice;
                    uint64_t peek = bits_at(&src, c2, MAX_CODE_LEN);
                    int L = 0;
                    uint64_t sym = 0;
                    for (int l = 1; l <= MAX_CODE_LEN; l++) {
                        uint64_t code = peek >> (MAX_CODE_LEN - l);
                        if (code >= c->first[l] && code < c->first[l] + c->count[l]) {
                            L = l;
                            sym = c->syms[c->base[l] + code - c->first[l]];
                            break;
                        }
                    }
                    if (!L) { bad = 1; break; }
                    cur = c2 + (uint64_t)L;
                    uint64_t gap = (q << gr->rice) | rem;
                    if (gap >= gsize) { bad = 1; break; }
                    local = first ? gap : local + gap + 1;
                    first = 0;
                    if (local >= gsize) { bad = 1; break; }
                    uint64_t p2 = ord[gstart[gr->exponent] + local];
                    int64_t d = (int64_t)(sym >> 1) ^ -(int64_t)(sym & 1);
                    uint16_t old_u = a[p2];
                    uint16_t new_u = (uint16_t)(((int64_t)old_u + d) & 0xFFFF);
                    idx[el] = p2;
                    val[el] = new_u;
                    el++;
                    dsum += (uint64_t)((int64_t)new_u - (int64_t)old_u) * orc_weight(p2);
                }
                if (!bad && cur != end) bad = 1;
            }
        }
        free(ord);
        if (bad) break;
        uint64_t oldchk = (has_cache && has_cache[tensor_target[i]]) ? cache_vals[tensor_target[i]] : orc_checksum(a, N);
        if (oldchk + dsum != t->checksum) { bad = 1; set_err(err, errlen, "update does not verify (checksum mismatch)"); }
    }
    if (bad) {
        if (err && errlen && !err[0]) set_err(err, errlen, "update does not decode or verify");
        free(idx); free(val);
        rc = ORC_CORRUPT;
        goto out;
    }
    /* all verified: write */
    el = 0;
    for (int64_t i = 0; i < T; i++) {
        uint16_t *a = datas[tensor_target[i]];
        uint64_t n_i = 0;
        for (int g = 0; g < u->tensors[i].n_groups; g++) n_i += u->tensors[i].groups[g].count;
        for (uint64_t k = 0; k < n_i; k++, el++) a[idx[el]] = val[el];
    }
    *changed_out = total;
    free(idx); free(val);
out:
    if (cn) for (int k = 0; k < u->n_tables; k++) free(cn[k].syms);
    free(cn);
    free_update(u);
    return rc;
}
