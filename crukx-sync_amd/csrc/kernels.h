// Device data layouts and kernel launchers of the gfx950 update codec.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace crx {

constexpr int kRow = 128;             // elements per wavefront row: 64 lanes x one 32-bit word
constexpr int kDense = 32;            // residual symbols below this are counted in a dense table
constexpr int kLocalGroups = 64;      // groups a statistics workgroup accumulates in LDS
constexpr uint32_t kScanTiles = 32;   // slabs per chunk of the per-tensor histogram scan
constexpr int kElemsPerThread = 16;   // change-order kernels: contiguous elements per thread
constexpr int kElemsPerWG = 256 * kElemsPerThread;
constexpr uint32_t kNone = 0xFFFFFFFFu;
constexpr int32_t kFar = 0x40000000;  // "no target in this slab" for the select pass
// bits of the apply verdict flag
constexpr unsigned int kBadDecode = 1;    // a block does not decode exactly to its length
constexpr unsigned int kBadLocal = 2;     // a change lies beyond its exponent group
constexpr unsigned int kBadUnplaced = 4;  // a change was not found in the receiver's weights
// a group has more changes than its tensor has elements of that exponent, in a tensor of more than
// `slab` elements (BlockArgs::group_check_numel; the reference raises this before decoding for tensors
// larger than its _SLAB, codec.py:598-604)
constexpr unsigned int kBadGroup = 8;

// One tensor of a call.  Elements are read as 32-bit words from `frame`, the 4-byte aligned address
// at or below the first element: tensor element i is 16-bit frame element i + lead.
struct TensorDesc {
    const uint32_t *frame;      // old weights (encode) / receiver weights (apply)
    const uint32_t *frame_new;  // encode: new weights, same lead as `frame`
    uint16_t *base;             // apply: receiver tensor, written by the scatter
    uint64_t numel;
    uint32_t lead;
    uint32_t tile_begin;        // first slab (global index)
    uint32_t n_tiles;
    uint32_t cold;              // 1: a full checksum is needed (new for encode, old for apply)
    const uint32_t *hist_in;    // apply: [n_tiles][256] exponent counts of these weights, or null
    uint32_t *hist_out;         // apply: receives the counts after the update, or null
};

// One (tensor, exponent) group.  Encode fills r0/rice/blk_base after the statistics pass;
// apply fills everything from the parsed header.
struct GroupDev {
    uint32_t tensor;
    uint32_t exponent;
    uint32_t count;
    uint32_t elem_base;  // first change of the group in update order
    uint32_t blk_base;   // first block of the group
    uint32_t rice;
    uint32_t r0;         // encode: floor(log2(mean gap)) clamped
    uint32_t table;      // apply: decoding table index
};

// Per change block of an update (apply): what the per-block kernels need, in one load.
struct BlockInfo {
    uint32_t g;         // group
    uint32_t eb;        // first change of the block in update order
    uint32_t cnt;       // changes in the block (1..256)
    uint32_t key;       // tensor << 8 | exponent of the group
    uint32_t blk_base;  // first block of the group
    uint32_t count;     // changes in the group
    uint32_t tensor;
    uint32_t pad;
};

struct EncRankArgs {
    const TensorDesc *descs;
    const uint32_t *tile_tensor;    // [tiles] tensor of each slab
    uint32_t n_tensors, slab;
    uint32_t *hall, *hchg;          // [tiles][256]
    uint64_t *rec;                  // change records, slab by slab
    const unsigned long long *rec_base;  // [tiles] first record of each slab, or null: slab t at t * rec_per_slab
    uint64_t rec_per_slab;          // records a slab may store when rec_base is null
    uint32_t *rec_count;            // [tiles] changes of each slab (counted past the capacity too)
    unsigned int *overflow;         // set when a slab has more changes than it may store
    uint64_t *delta, *full;         // [tiles]
};

struct HistArgs {
    const TensorDesc *descs;
    const uint32_t *tile_tensor;
    uint32_t n_tensors, slab;
    uint32_t *hall;                 // [tiles][256]
    uint64_t *full;                 // [tiles] cold slabs: the even rows' part of the old checksum
    const uint32_t *list;           // the slabs to process (one workgroup each), or null for all
};

struct ScanChunk {                  // SCAN_TILES consecutive slabs of one tensor
    uint32_t tile_begin, tile_end, tensor, pad;
};

struct StatsArgs {
    const uint64_t *sorted;         // (zz << 32) | group-local index, in update order
    uint64_t n;
    const GroupDev *groups;
    uint32_t n_groups;
    const uint32_t *cmap;           // [n / kElemsPerThread] group of every thread's first change
    uint32_t *dense;                // [256][kDense]
    uint32_t *rare;                 // (exponent << 17) | zz for zz >= kDense
    uint64_t rare_cap;
    unsigned long long *counters;   // [0] rare count, [1] rare overflow
    unsigned long long *cost;       // [groups][3]
};

struct CodeArgs {
    const uint64_t *sorted;
    uint64_t n;
    const GroupDev *groups;
    uint32_t n_groups;
    const uint32_t *lut;            // [256][kDense]: (code << 5) | length, 0 if absent
    const uint32_t *rare_keys;      // sorted (exponent << 17) | zz
    const uint32_t *rare_vals;
    uint32_t n_rare;
    const uint32_t *cmap;           // [n / kElemsPerThread] group of every thread's first change
    unsigned long long *tsum;       // [threads] bits per thread (kElemsPerThread changes)
    const unsigned long long *toff; // [threads] exclusive bit offsets
    uint32_t *words;                // payload as big-endian bytes in 32-bit words
    unsigned long long *bstart;     // [blocks + 1] bit offset of each block
    uint64_t n_words;               // words allocated: a workgroup whose bits end past them writes nothing
    unsigned int *overflow;         // |= 2 when that happens
    uint64_t bit_base;              // payload bit of these changes' first bit (a part of a chunked update)
};

struct DecodeArgs {
    const TensorDesc *descs;
    // the payload: a big-endian byte stream that starts bit0 bits into the 8-byte aligned word
    // payload[0] and ends in payload[n_words - 1] (bits past its end are never decisive)
    const uint64_t *payload;
    uint64_t n_words;
    const uint32_t *block_bits;
    const unsigned long long *block_off;
    uint64_t n_blocks;
    const GroupDev *groups;
    uint32_t n_groups;
    const uint32_t *bmap;           // [blocks] group of every block
    const uint32_t *lim;            // [tables][17]: end of length l's codes, left-justified to 17 bits
    const uint32_t *off;            // [tables][17]: symbol index of code 0 of length l (mod 2^32)
    const uint32_t *syms;
    uint32_t n_syms;
    unsigned long long *dz;         // [changes] zz | (block-relative local index << 32)
    unsigned long long *blk_sum;    // [blocks] sum of (gap + 1) per block
    unsigned int *bad;
    uint32_t n_tables;              // tables: lim and off hold 17 entries each
    uint32_t bit0;                  // first payload bit in payload[0] (0-56, a multiple of 8)
};

struct SelectArgs {
    const TensorDesc *descs;
    const uint32_t *tile_tensor;
    uint32_t n_tensors, slab;
    const uint32_t *pre;            // [tiles][256] exponent counts before the slab (in its tensor)
    const uint32_t *lb;             // [tiles + 1][256] first change of the group at or after the slab
    const int32_t *group_of;        // [tensor][256] group index or -1
    const GroupDev *groups;
    const uint32_t *local;          // group-local index of every change
    // [changes] the select pass's records, slab by slab (each slab's in row order): change index | offset
    // in the slab << 32 | old bits << 48
    unsigned long long *rec;
    uint32_t *rstart;               // [tiles + 1] first record of each slab (written by k_locate)
    const uint32_t *tchg;           // [tensors + 1] first change of each tensor
    unsigned int *bad;              // kBadUnplaced: a slab's targets were not all found
    uint2 *more;                    // [kSelMoreWindows tiles] (slab, first exponent) of windows after a slab's first
    unsigned int *n_more;           // their number (zero before k_locate)
    uint32_t n_front;               // listed windows taken by the front blocks of the select pass
    // A slab streamed in one window is written by its select wave once its records are complete:
    // new bits, checksum delta and exponent moves (k_commit undoes the writes if the update does not
    // verify).  Slabs with more windows (multi, set by k_locate) are left to k_verify and k_commit.
    const unsigned long long *dz;   // [changes] decoder output: zz in the low 32 bits
    uint64_t *sdelta;               // [tiles] checksum delta of each single-window slab's changes
    uint8_t *multi;                 // [tiles] the slab has more than one window (k_locate)
    uint32_t *done;                 // [tiles] records written through by the select pass (zeroed by k_locate)
    uint32_t n_changes;
    const unsigned long long *blk_prefix;  // [blocks + 1] sums of (gap + 1) over the blocks before each
    // [tiles] each slab's weighted sum for its tensor's checksum when the tensor is cold (no cached
    // checksum), else 0: completed by the slab's first window, which reads the weights before any
    // write (to the histogram pass's sum of the even rows, when that pass streamed the slab)
    uint64_t *full;
};

struct SlabArgs {                   // per-slab kernels over the select pass's records (one workgroup per slab)
    const TensorDesc *descs;
    const uint32_t *tile_tensor;
    uint32_t slab;
    const uint32_t *rstart;              // [tiles + 1]
    const unsigned long long *rec;       // [changes] as SelectArgs::rec
    const unsigned long long *dz;        // [changes] decoder output: zz in the low 32 bits
    uint32_t *pn;                        // [changes] offset in the slab | new bits << 16 (k_verify)
    uint64_t *sdelta;                    // [tiles] checksum delta of each slab's changes
    unsigned int *bad;
    const unsigned int *ok;              // the device's verdict (k_verdict), read by k_commit
    uint32_t n_changes;
    const uint8_t *multi;                // [tiles] as SelectArgs::multi
    const uint32_t *done;                // [tiles] as SelectArgs::done
};

struct BlockArgs {                  // per-block kernels over the change list (one workgroup per block)
    const GroupDev *groups;
    uint32_t n_groups, slab;
    const BlockInfo *binfo;         // [blocks]
    const TensorDesc *descs;
    const uint32_t *sizes;
    const unsigned long long *blk_prefix;
    uint32_t *local;                // [changes] group-local index (written by k_local_fix)
    const unsigned long long *dz;   // [changes] decoder output: zz | (block-relative local << 32)
    unsigned int *bad;
    uint64_t n_blocks;
    uint64_t group_check_numel;     // tensors of more elements report a group larger than its exponent's count as kBadGroup
};

void launch_enc_rank(const EncRankArgs &a, uint32_t tiles, hipStream_t s);
// Histograms of the listed slabs (all when a.list is null): n workgroups.
void launch_hist(const HistArgs &a, uint32_t n, hipStream_t s);
// Per-tensor exclusive scans over slabs of per-slab exponent tables, in place; slabs of tensors with
// cached counts (descs: hist_in and not cold) are read from those counts.  n_tabs (1 or 2) tables of
// the same layout are scanned by the same launches, each with its own chunk sums and totals.
struct ScanTabs {
    uint32_t *h[2];       // [tiles][256] tables, scanned in place
    uint32_t *csum[2];    // [chunks][256] chunk sums of each
    uint32_t *totals[2];  // [tensors][256] totals of each
};
void launch_scan_tables(const TensorDesc *descs, const ScanTabs &p, uint32_t n_tabs, const ScanChunk *chunks,
                        uint32_t n_chunks, const uint32_t *tensor_chunk_begin, uint32_t n_tensors, hipStream_t s);
void launch_enc_groups(const uint32_t *totals_chg, uint32_t n_tensors, GroupDev *groups, uint32_t *gbase,
                       unsigned long long *counters, hipStream_t s);
void launch_place(const EncRankArgs &a, uint32_t tiles, const uint32_t *tile_tensor,
                  const uint32_t *hall_pre, const uint32_t *hchg_pre, const uint32_t *gbase,
                  uint64_t *sorted, uint64_t n_sorted, hipStream_t s);
void launch_r0(GroupDev *groups, uint32_t n_groups, const uint64_t *sorted, hipStream_t s);
void launch_stats(const StatsArgs &a, hipStream_t s);
void launch_code_lengths(const CodeArgs &a, hipStream_t s);
// cmap[c] = group of change kElemsPerThread * c; bmap[b] = group of block b
void launch_chunk_map(const GroupDev *groups, uint32_t n_groups, uint32_t *cmap, hipStream_t s);
void launch_block_map(const GroupDev *groups, uint32_t n_groups, uint32_t *bmap, BlockInfo *binfo, hipStream_t s);
void launch_pack(const CodeArgs &a, hipStream_t s);
void launch_block_bits(const unsigned long long *bstart, uint64_t n_blocks, uint32_t *out, unsigned int *overflow,
                       hipStream_t s);
// Exclusive prefix sums with out[n] = total; `part` holds scan_parts(n) values of scratch.
uint64_t scan_parts(uint64_t n);
void launch_scan_u64(const unsigned long long *in, uint64_t n, unsigned long long *out, unsigned long long *part,
                     hipStream_t s);
void launch_scan_u32(const uint32_t *in, uint64_t n, unsigned long long *out, unsigned long long *part, hipStream_t s);
// ok = 1 iff *bad is 0 and every tensor's old checksum (cached[t] where has[t], else full[t]) plus
// its delta equals want[t]; 0 otherwise.  One workgroup.
void launch_verdict(uint32_t n, const unsigned long long *delta, const uint64_t *full, const int32_t *has,
                    const uint64_t *cached, const uint64_t *want, const unsigned int *bad, unsigned int *ok,
                    hipStream_t s);
void launch_tensor_sums(const TensorDesc *descs, uint32_t n_tensors, const uint64_t *per_tile, uint64_t *out,
                        hipStream_t s);
void launch_decode(const DecodeArgs &a, hipStream_t s);
constexpr uint32_t kDecSyms = 2048;  // decoding symbols staged in LDS when they fit (with the first indices)
// Dynamic LDS of the decoder for n_syms symbols.
inline uint32_t decode_lds_bytes(uint32_t n_syms, uint32_t n_tables) { return n_syms <= kDecSyms ? (n_syms + 17u * n_tables) * 4u : 0u; }
void launch_local_fix(const BlockArgs &a, uint64_t n_blocks, hipStream_t s);
void launch_locate(const SelectArgs &a, uint32_t tiles, hipStream_t s);
// tile_tensor[tile] = tensor of every slab of the layout
void launch_tile_map(const TensorDesc *descs, uint32_t n_tensors, uint32_t *tile_tensor, hipStream_t s);
// Exponents per window of the select pass (a slab is streamed once per window holding targets), and
// the most windows a slab can need after its first.
constexpr uint32_t kSelWin = 64;
constexpr uint32_t kSelMoreWindows = 256 / kSelWin - 1;
// dense: the larger LDS target list (for updates averaging over kSelectDenseTargets changes per slab);
// any_cold: some tensor has no cached checksum (its slabs' sums go to SelectArgs::full)
constexpr uint64_t kSelectDenseTargets = 800;
void launch_select(const SelectArgs &a, uint32_t tiles, bool dense, bool any_cold, hipStream_t s);
// New values and checksum deltas of the records of slabs with more than one window (one workgroup
// per slab; the select pass did the others' already).
void launch_verify(const SlabArgs &a, uint32_t tiles, hipStream_t s);
// After the device's verdict (one workgroup per slab): if the update verifies, the writes of slabs
// with more than one window; if not, the old bits back where the select pass wrote.
void launch_commit(const SlabArgs &a, uint32_t tiles, hipStream_t s);
void launch_checksum(const uint32_t *frame, uint32_t lead, uint64_t n, uint64_t *partial, uint32_t n_parts,
                     hipStream_t s);
// The full checksum of n 16-bit elements (frame words, lead as in TensorDesc) into *out (host
// memory), through a static per-device scratch array: no device or host allocation.  Waits for the
// stream.  Not timed by crx_timing (no events are created).
hipError_t checksum_noalloc(const uint32_t *frame, uint32_t lead, uint64_t n, hipStream_t s, uint64_t *out);

// Host-side timing of launches (events on the launch stream), enabled by crx_timing_enable and
// limited to the kernels named by crx_timing_only.  timing_begin and timing_end bracket one launch.
void timing_begin(const char *name, hipStream_t s);
void timing_end(const char *name, hipStream_t s);

}  // namespace crx
