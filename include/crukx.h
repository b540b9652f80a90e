/*
 * crukx.h -- C ABI of the MI355X (gfx950) implementation of the crukx-sync update codec,
 * wire format version 2 ("CRXS" 0x02).
 *
 * The reference (Crukx-dev/crukx-sync v0.2.0) is pure Python/torch and has no FFI; these entry
 * points replace the functions of its hot path, named per declaration below (paths relative to
 * the reference repository).  The Python package crukx_sync in crukx-sync_amd/ binds them with
 * ctypes (crukx_sync/_native.py) and keeps the reference's public API unchanged.
 *
 * Conventions
 *   - Status codes: CRX_OK, CRX_CORRUPT (-> crukx_sync.CorruptUpdate), CRX_INVALID (-> ValueError),
 *     CRX_DEVICE (HIP runtime error -> RuntimeError), CRX_NOMEM (-> MemoryError).  No C++
 *     exception crosses the ABI.  `err`/`errlen` receive a NUL-terminated message.
 *   - Tensors are passed as device pointers to 16-bit bit patterns (bf16 or int16), 2-byte
 *     aligned, contiguous, with an element count.
 *   - Device memory: the library calls `alloc(alloc_ctx, nbytes)` for every device buffer it
 *     needs (the Python layer hands out torch caching-allocator tensors); the caller frees them
 *     after the call (encode: when the crx_encoded handle is freed).  A call usually asks for one
 *     block sized from the previous call of its kind and carves its buffers from it.  Small
 *     host<->device transfers use pinned host memory the library allocates per host thread and
 *     keeps until the process ends.  Copies of an update's bytes between device memory and
 *     pageable host memory go through 64 MiB of pinned buffers (allocated once per process) on up
 *     to four threads that the call starts and joins.  Work runs on `stream` (a hipStream_t).
 *     Results are final on return.  crx_apply returns once its writes (or, for an update that does
 *     not verify, the restoring of what it wrote) are done: the host waits for the verdict's data,
 *     which the stream delivers after the last write.  crx_encoded_write's copies into device memory
 *     are left ordered on `stream`, so the buffers `alloc` handed out must stay usable by work
 *     already on `stream` after the call (a stream-ordered allocator such as torch's caching
 *     allocator does this).  Everything else is complete on return.
 *   - `slab` is the reference's codec._SLAB (codec.py:30; 0 = its default, 2^24).  As there, apply
 *     checks the group sizes of tensors of more than `slab` elements before decoding (codec.py:598-604,
 *     "group has more changes than elements").  It also bounds the elements ranked by one wavefront:
 *     min(slab, 65536) rounded down to a multiple of 128 (at least 128).  It never changes the bytes.
 */
#ifndef CRUKX_H
#define CRUKX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CRX_ABI_VERSION 1

#define CRX_OK 0
#define CRX_CORRUPT 1
#define CRX_INVALID 2
#define CRX_DEVICE 3
#define CRX_NOMEM 4

typedef void *(*crx_alloc_fn)(void *alloc_ctx, uint64_t nbytes);

typedef struct crx_update crx_update;   /* a parsed update (host header + block table) */
typedef struct crx_encoded crx_encoded; /* an encoded update (host header, device bits) */

/* ABI version of the loaded library (CRX_ABI_VERSION). */
int32_t crx_abi_version(void);

/* ------------------------------------------------------------------ wire format (host)
 * Replaces wire.parse (src/crukx_sync/wire.py:126-212): magic, version, every limit of
 * docs/FORMAT.md:46-57 in the reference's order.  `data` holds the whole update (host memory);
 * crx_apply uploads the payload from it unless given a device copy.  For an update held in
 * device memory, crx_parse_prefix parses a host copy of its leading bytes.  The handle refers to
 * the block table and payload in `data` / `prefix`: keep those bytes until crx_update_free. */
int32_t crx_parse(const uint8_t *data, uint64_t len, crx_update **out, char *err, uint64_t errlen);
/* Parses from a prefix of an update held elsewhere: `prefix` has `prefix_len` bytes of an update
 * of `total_len` bytes whose last byte is `last_byte`.  Returns CRX_OK, CRX_CORRUPT, or
 * CRX_INVALID with *need set to the prefix length required (then call again). */
int32_t crx_parse_prefix(const uint8_t *prefix, uint64_t prefix_len, uint64_t total_len, uint8_t last_byte,
                         crx_update **out, uint64_t *need, char *err, uint64_t errlen);
void crx_update_free(crx_update *u);

/* Accessors (wire.Update, wire.py:20-48). */
int64_t crx_update_n_tables(const crx_update *u);
int32_t crx_update_table(const crx_update *u, int64_t i, int32_t *exponent, int64_t *n_sym,
                         uint32_t *symbols /* n_sym or NULL */, uint8_t *lengths /* n_sym or NULL */);
int64_t crx_update_n_tensors(const crx_update *u);
int32_t crx_update_tensor(const crx_update *u, int64_t i, const uint8_t **name, uint64_t *name_len,
                          uint64_t *numel, uint64_t *checksum, int32_t *n_groups);
int32_t crx_update_group(const crx_update *u, int64_t i, int32_t g, int32_t *exponent, uint64_t *count,
                         int32_t *rice);
/* All tensor headers at once: names concatenated into `names` (capacity `names_cap`; the total
 * length is returned in *names_len), name_ends[i] = end offset of name i, plus numels and checksums
 * (n_tensors entries each).  Returns CRX_INVALID with *names_len set if `names_cap` is too small. */
int32_t crx_update_headers(const crx_update *u, char *names, uint64_t names_cap, uint64_t *names_len,
                           uint64_t *name_ends, uint64_t *numels, uint64_t *checksums);
uint64_t crx_update_n_blocks(const crx_update *u);
/* Copies the block table (n_blocks u32) into `out`. */
int32_t crx_update_block_bits(const crx_update *u, uint32_t *out);
uint64_t crx_update_payload_offset(const crx_update *u);
uint64_t crx_update_payload_len(const crx_update *u);
uint64_t crx_update_total_changes(const crx_update *u);

/* ------------------------------------------------------------------ apply (device)
 * Replaces codec.apply (src/crukx_sync/codec.py:578-717) including the block decoder
 * (codec.py:504-575, _triton.py:33-106): decode every block, locate every change in the stable
 * exponent order of the receiver's old weights and verify each tensor's checksum; the weights end
 * written only if the update verifies, as with the reference's verify-then-write (codec.py:703-707).
 * The pass that locates the changes writes most of them as it goes, before the verdict; a kernel
 * after the device's verdict makes the remaining writes if the update verifies, and otherwise puts
 * the old bits back (from the located changes), so later work on `stream` sees either all of the
 * update or none of it.  `targets[i]` is the receiver tensor for update tensor i (crx_update_tensor
 * order) with `numels[i]` elements (below 2^32: CRX_INVALID otherwise); the tensors must not
 * overlap.  An update of 2^32 or more changes is applied part by part, consecutive tensors of at
 * most 2^31 elements (a larger tensor alone) per part: every part is first verified without
 * writing anything, the verdict is taken on the whole update, then the parts are written one after
 * another (each verified again as it is; should that fail, because the weights changed between the
 * passes, or device memory runs out after the first part is written, CRX_DEVICE reports it with the
 * parts before it written).  `has_cache[i]`/`cache_vals[i]` give a trusted old checksum (else one is
 * computed from the weights).  `payload_dev` is NULL to upload the payload (and block table) from
 * the parsed host bytes, or the address of the payload inside a device-resident copy of the whole
 * update (the block table, which precedes the payload, is read from there too).  On
 * CRX_INVALID and CRX_NOMEM nothing is written; on CRX_CORRUPT the weights end as they were (for a
 * checksum mismatch, after the undo enqueued on `stream`); on CRX_OK the remaining writes are
 * enqueued on `stream`.  CRX_DEVICE (a HIP runtime error) leaves the weights unspecified: some writes
 * may have run and their undo may not.  Treat the weights, and any checksum cached for them, as
 * unknown then.
 * `*changed` receives the number of changed elements. */
int32_t crx_apply(const crx_update *u, const uint8_t *payload_dev, uint16_t *const *targets,
                  const uint64_t *numels, const int32_t *has_cache, const uint64_t *cache_vals, int32_t slab,
                  void *stream, crx_alloc_fn alloc, void *alloc_ctx, uint64_t *changed, char *err,
                  uint64_t errlen);

/* crx_apply with the receiver's per-slab exponent counts kept across updates.  These counts change
 * only when an element crosses a power of two, so the histogram pass (a full read of the weights)
 * is skipped for tensors whose counts are known.  hist_in[i] (device, crx_apply_hist_words(numel,
 * slab) u32, or NULL) holds tensor i's counts, valid only while its weights are unchanged since they
 * were recorded, only for the same slab size and only with a trusted cached checksum (has_cache[i]);
 * the library cannot check its size, so counts recorded with another slab size read out of bounds;
 * hist_out[i] (or NULL)
 * receives the counts after this update (it may equal hist_in[i]).  On any status but CRX_OK the
 * weights end as with crx_apply but hist_out may hold partial results: discard them.  No counterpart in
 * the reference (its analogue is the checksum cache, codec.py:457-460,713-716). */
int32_t crx_apply_cached(const crx_update *u, const uint8_t *payload_dev, uint16_t *const *targets,
                         const uint64_t *numels, const int32_t *has_cache, const uint64_t *cache_vals,
                         uint32_t *const *hist_in, uint32_t *const *hist_out, int32_t slab, void *stream,
                         crx_alloc_fn alloc, void *alloc_ctx, uint64_t *changed, char *err, uint64_t errlen);
/* Size in u32 of one tensor's counts for crx_apply_cached. */
uint64_t crx_apply_hist_words(uint64_t numel, int32_t slab);

/* ------------------------------------------------------------------ encode (device)
 * Replaces codec.encode (src/crukx_sync/codec.py:278-420): rank changes in stable exponent order,
 * gaps and residuals, per-group Rice parameters, one canonical Huffman table per exponent, bit
 * packing and the block table.  Tensors in caller order; `has_cache`/`cache_vals` give the
 * sender's cached checksum of old (new checksum = cache + delta), else the checksum of new is
 * computed in full.  Fails with CRX_INVALID if a block reaches 2^32 bits (codec.py:417-419).  An update
 * of 2^32 or more changes is encoded part by part, as the reference packs batches of changes
 * (codec.py:214,337-341,394-410): consecutive tensors of at most 2^31 elements per part, each ranked
 * once for the symbol counts of the whole update's tables and again to be coded at its bit offset in
 * the one payload; the bytes are those of a single pass.  The environment variable
 * CRX_PART_ELEMENTS (a positive element count) makes encode and apply split every update larger than
 * it into parts of that size, so that the part-wise path can be tested at small sizes. */
int32_t crx_encode(int32_t n, const uint16_t *const *olds, const uint16_t *const *news, const uint64_t *numels,
                   const int32_t *has_cache, const uint64_t *cache_vals, int32_t slab, void *stream,
                   crx_alloc_fn alloc, void *alloc_ctx, crx_encoded **out, char *err, uint64_t errlen);
/* Tensor t of the encode call is in the update (has a changed element). */
int32_t crx_encoded_present(const crx_encoded *e, int32_t t);
/* New checksum of tensor t (valid when present). */
uint64_t crx_encoded_checksum(const crx_encoded *e, int32_t t);
/* Both of the above for every tensor of the encode call (n entries each). */
void crx_encoded_checksums(const crx_encoded *e, int32_t *present, uint64_t *checksums);
uint64_t crx_encoded_total_changes(const crx_encoded *e);
/* Serialized size (wire.serialize, wire.py:64-89) given the names of the encode call's tensors. */
uint64_t crx_encoded_size(const crx_encoded *e, const char *const *names, const uint64_t *name_lens);
/* Writes the serialized update to `dst`: host memory (complete on return), or device memory when
 * dst_on_device (the copies are ordered on `stream`; the encoded handle must outlive them).  A host
 * destination of 8 MiB or more is advised for transparent huge pages (madvise MADV_HUGEPAGE on its
 * whole 2 MiB pages): a fresh buffer then takes one page fault per 2 MiB instead of per 4 KiB. */
int32_t crx_encoded_write(const crx_encoded *e, const char *const *names, const uint64_t *name_lens, uint8_t *dst,
                          int32_t dst_on_device, void *stream, char *err, uint64_t errlen);
/* Header pieces for wire.Update materialisation. */
int64_t crx_encoded_n_tables(const crx_encoded *e);
int32_t crx_encoded_table(const crx_encoded *e, int64_t i, int32_t *exponent, int64_t *n_sym, uint32_t *symbols,
                          uint8_t *lengths);
int32_t crx_encoded_n_groups(const crx_encoded *e, int32_t t);
int32_t crx_encoded_group(const crx_encoded *e, int32_t t, int32_t g, int32_t *exponent, uint64_t *count,
                          int32_t *rice);
uint64_t crx_encoded_n_blocks(const crx_encoded *e);
int32_t crx_encoded_block_bits(const crx_encoded *e, uint32_t *out, void *stream);
uint64_t crx_encoded_payload_len(const crx_encoded *e);
int32_t crx_encoded_payload(const crx_encoded *e, uint8_t *out, void *stream);
void crx_encoded_free(crx_encoded *e);

/* ------------------------------------------------------------------ checksum (device)
 * Replaces codec.checksum (src/crukx_sync/codec.py:61-68): sum(u_i * (splitmix64(i) | 1)) mod 2^64
 * over n 16-bit patterns, as a deterministic device reduction. */
int32_t crx_checksum(const uint16_t *data, uint64_t n, void *stream, crx_alloc_fn alloc, void *alloc_ctx,
                     uint64_t *out, char *err, uint64_t errlen);
/* crx_checksum without any allocation: no counterpart in the reference.  For callers that cannot
 * allocate (tight serving loops, harnesses that forbid hipMalloc): the per-workgroup partial sums live
 * in a static device array of 2049 u64 (16 KiB per device, held until the process ends) instead of
 * memory from an allocator, and the result goes to *out (host memory) through a plain copy; the call
 * waits for `stream`, so it cannot be used inside stream capture.  n must be below 2^32 (as for
 * crx_checksum; CRX_INVALID otherwise).  Calls that overlap on one device share that array and
 * race: serialize them. */
int32_t crx_checksum_noalloc(const uint16_t *data, uint64_t n, void *stream, uint64_t *out, char *err,
                             uint64_t errlen);

/* ------------------------------------------------------------------ host helpers
 * codec.huffman_lengths (codec.py:71-98): code lengths limited to 17 bits. */
int32_t crx_huffman_lengths(const uint64_t *counts, int64_t n, int32_t *lengths);
/* codec.canonical_codes (codec.py:101-111). */
int32_t crx_canonical_codes(const int32_t *lengths, int64_t n, uint32_t *codes);
/* codec._rice_params (codec.py:268-275) for one group from its sums: `count` changes whose gaps
 * sum to `gap_sum`; `shifted[k]` = sum(gap >> cand[k]) for the candidates written to `cand`
 * by crx_rice_candidates.  Returns the chosen parameter. */
void crx_rice_candidates(uint64_t count, uint64_t gap_sum, int32_t cand[3]);
int32_t crx_rice_choose(uint64_t count, const int32_t cand[3], const uint64_t shifted[3]);

/* ------------------------------------------------------------------ timing
 * When enabled, each kernel launch is bracketed by HIP events on its stream and the durations
 * accumulate per kernel name.  crx_timing_read writes "name calls total_ms\n" lines. */
void crx_timing_enable(int32_t on);
/* Limits the timing to the kernels named in `names` (comma-separated); NULL or "" times every kernel.
 * Host phases ("host:...") are recorded whenever timing is enabled. */
void crx_timing_only(const char *names);
void crx_timing_reset(void);
int32_t crx_timing_read(char *buf, uint64_t len);

#ifdef __cplusplus
}
#endif

#endif /* CRUKX_H */
