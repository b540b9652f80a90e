// gfx950 kernels of the update codec (wave64, LDS, HBM-streaming; no MFMA: nothing here is a
// contraction).
//
// Ranking (encode) and selection (apply) work on slabs: one wavefront owns `slab` consecutive
// elements of one tensor and streams them as rows of 64 lanes x one 32-bit word (two bf16).  A
// running per-exponent histogram in LDS gives, for any element, the number of same-exponent
// elements before its row; the stable in-row rank comes from ballots and mbcnt.  Per-slab
// histograms are scanned per tensor afterwards, so a slab's ranks become tensor-wide ranks.
#include "kernels.h"

#include <crx_wave.h>

#include <algorithm>
#include <mutex>

namespace crx {
namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;
constexpr uint64_t kMix1 = 0xBF58476D1CE4E5B9ULL;
constexpr uint64_t kMix2 = 0x94D049BB133111EBULL;
constexpr int kRankRows = 8;    // rows per batch of the encode rank pass (two streams)
constexpr uint32_t kPlaceRecs = 12;  // records per lane per batch of the placement pass
constexpr int kChgCap = 256;    // changes the rank pass buffers in LDS; a flush leaves room for a row
constexpr uint32_t kRankCopies = 4;  // copies of each exponent count in the rank pass (2, 4 or 8; 4 measured best)
static_assert(kRankCopies == 2 || kRankCopies == 4 || kRankCopies == 8, "kRankCopies");
constexpr int kScanRows = 16;   // rows per batch of the apply histogram pass
constexpr int kSelectRows = 8;  // ... of the select pass (fewer registers: occupancy)

// splitmix64(i) | 1: the per-position checksum weight (docs/FORMAT.md:61-64).  mix_weight takes
// z = (i + 1) * golden, so that streaming passes can step z by a constant instead of multiplying.
__device__ __forceinline__ uint64_t mix_weight(uint64_t z) {
    z = (z ^ (z >> 30)) * kMix1;
    z = (z ^ (z >> 27)) * kMix2;
    return (z ^ (z >> 31)) | 1ULL;
}
__device__ __forceinline__ uint64_t weight(uint64_t i) { return mix_weight((i + 1) * kGolden); }

// sum of u * w mod 2^64 over 16-bit u: the products with the low word of w are summed in 64 bits, with
// the high word mod 2^32 in 32 bits, and combined once at the end (two 32-bit multiplies per element
// instead of a 16 x 64-bit product).
struct WeightedSum {
    uint64_t lo = 0;
    uint32_t hi = 0;
    __device__ __forceinline__ void add(uint32_t u, uint64_t w) {
        lo += (uint64_t)u * (uint32_t)w;
        hi += u * (uint32_t)(w >> 32);
    }
    __device__ __forceinline__ uint64_t total() const { return lo + ((uint64_t)hi << 32); }
};

__device__ __forceinline__ uint32_t lane() { return __lane_id(); }
// 64-bit integer min (the generic min template of the HIP headers goes through double precision)
__device__ __forceinline__ uint64_t min64(uint64_t a, uint64_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
// number of set bits of m below this lane
__device__ __forceinline__ uint32_t mbcnt(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ uint32_t rdlane(uint32_t v, uint32_t l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ uint64_t wave_sum(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint32_t zigzag(uint32_t o16, uint32_t n16) {
    int32_t res = (int32_t)(int16_t)n16 - (int32_t)(int16_t)o16;
    return res >= 0 ? (uint32_t)(2 * res) : (uint32_t)(-2 * res - 1);
}

__global__ __launch_bounds__(256) void k_tile_map(const TensorDesc *descs, uint32_t *tile_tensor) {
    const TensorDesc d = descs[blockIdx.x];
    for (uint32_t i = threadIdx.x; i < d.n_tiles; i += 256) tile_tensor[d.tile_begin + i] = blockIdx.x;
}

// One workgroup per group: the group of every kElemsPerThread-th change and of every block.
__global__ __launch_bounds__(256) void k_chunk_map(const GroupDev *groups, uint32_t *cmap) {
    const GroupDev g = groups[blockIdx.x];
    const uint64_t c0 = ((uint64_t)g.elem_base + kElemsPerThread - 1) / kElemsPerThread;
    const uint64_t c1 = ((uint64_t)g.elem_base + g.count + kElemsPerThread - 1) / kElemsPerThread;
    for (uint64_t c = c0 + threadIdx.x; c < c1; c += 256) cmap[c] = blockIdx.x;
}

__global__ __launch_bounds__(256) void k_block_map(const GroupDev *groups, uint32_t *bmap, BlockInfo *binfo) {
    const GroupDev g = groups[blockIdx.x];
    const uint32_t nb = (g.count + 255) / 256;
    for (uint32_t i = threadIdx.x; i < nb; i += 256) {
        bmap[g.blk_base + i] = blockIdx.x;
        binfo[g.blk_base + i] = BlockInfo{blockIdx.x, g.elem_base + 256 * i, min(256u, g.count - 256 * i),
                                          (g.tensor << 8) | g.exponent, g.blk_base, g.count, g.tensor, 0};
    }
}

// last group whose first change is <= i
__device__ uint32_t group_of_elem(const GroupDev *g, uint32_t n, uint64_t i) {
    uint32_t lo = 0, hi = n;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (g[mid].elem_base <= i) lo = mid;
        else hi = mid;
    }
    return lo;
}

// last group whose first block is <= b
__device__ uint32_t group_of_block(const GroupDev *g, uint32_t n, uint64_t b) {
    uint32_t lo = 0, hi = n;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (g[mid].blk_base <= b) lo = mid;
        else hi = mid;
    }
    return lo;
}

// ================================================================== slab streaming
// A wavefront reads its slab as rows of 64 lanes x one 32-bit word (two consecutive bf16), 32-bit
// offsets relative to the slab's first frame word.  Interior rows need no masking; only the first
// (odd start) and last (partial) rows do, and the rows past the end that complete the last batch
// (every lane outside [f_lo, f_hi)).
struct Slab {
    uint32_t first;   // frame word index of the slab's first word
    uint32_t nwords;  // words covering the slab
    uint32_t f_lo;    // valid 16-bit offsets within the slab's words: [f_lo, f_hi)
    uint32_t f_hi;
    uint32_t base;    // tensor index of offset 0 (mod 2^32): element f is tensor element base + f
    uint32_t nrows;
    uint32_t full_lo, full_n;  // rows [full_lo, full_lo + full_n) lie entirely in [f_lo, f_hi)
};

__device__ __forceinline__ Slab slab_of(const TensorDesc &td, uint32_t local, uint32_t slab) {
    const uint64_t lo = (uint64_t)local * slab, hi = min(lo + slab, td.numel);
    const uint64_t d_begin = (lo + td.lead) >> 1, d_end = (hi + td.lead + 1) >> 1;
    Slab s;
    s.first = (uint32_t)d_begin;
    s.nwords = (uint32_t)(d_end - d_begin);
    s.f_lo = (uint32_t)(lo + td.lead - 2 * d_begin);
    s.f_hi = (uint32_t)(hi + td.lead - 2 * d_begin);
    s.base = (uint32_t)(2 * d_begin - td.lead);
    s.nrows = (s.nwords + 63) / 64;
    s.full_lo = (s.f_lo + kRow - 1) / kRow;
    const uint32_t full_hi = s.f_hi / kRow;
    s.full_n = full_hi > s.full_lo ? full_hi - s.full_lo : 0;
    return s;
}

__device__ __forceinline__ bool row_full(const Slab &s, uint32_t r) { return r - s.full_lo < s.full_n; }

// Raw buffer resource over the slab's words [p, p + nwords): the hardware range check returns 0 for
// any load at or past the end, so rows fetched ahead of the slab's end need neither masks nor
// addresses inside the allocation.  Dword 3 is the gfx9-family default format.
using Rsrc = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ Rsrc slab_rsrc(const uint32_t *frame, const Slab &s) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(frame + s.first), (short)0,
                                             (int)(s.nwords * 4u), 0x00020000);
}

// Streams the slab's rows through `body(row, word of stream 0, word of stream S-1)`, U rows per batch
// with the next batch already in flight (U..2U rows of loads outstanding per wavefront while a batch
// is processed).  The two batches' registers alternate (the loop body holds two batches), so no
// registers are copied between batches.  Every batch is whole: rows at or past nrows read as zero
// and lie outside [f_lo, f_hi), so the body treats them as partial rows with no valid lane.
// CPOL is the cache policy of the loads of the first stream, CPOL_LAST that of the last stream
// (kStreamNT: non-temporal).  Measured: the select pass with non-temporal loads 5.08 -> 4.93 ms; the
// rank pass 6.50 -> 6.18 ms with them on one of its two streams, 6.71 ms with them on both.
constexpr int kStreamNT = 2;
template <int U, int S, int CPOL = 0, int CPOL_LAST = CPOL, typename Body>
__device__ __forceinline__ void stream_rows(const Slab &sl, const Rsrc (&src)[S], Body &&body) {
    static_assert(S == 1 || S == 2, "one or two streams");
    const uint32_t lb = lane() * 4u;
    uint32_t a[S][U], b[S][U];
    auto load = [&](uint32_t(&dst)[S][U], uint32_t r) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            dst[0][u] = __builtin_amdgcn_raw_buffer_load_b32(src[0], (r + u) * 256u + lb, 0, S == 1 ? CPOL_LAST : CPOL);
            if (S == 2) dst[S - 1][u] = __builtin_amdgcn_raw_buffer_load_b32(src[S - 1], (r + u) * 256u + lb, 0, CPOL_LAST);
        }
    };
    if (sl.nrows == 0) return;
    load(a, 0);
    for (uint32_t r0 = 0;; r0 += 2 * U) {  // r0 < nrows here
        load(b, r0 + U);
#pragma unroll
        for (int u = 0; u < U; ++u) body(r0 + u, a[0][u], a[S - 1][u]);
        if (r0 + U >= sl.nrows) break;
        load(a, r0 + 2 * U);
#pragma unroll
        for (int u = 0; u < U; ++u) body(r0 + U + u, b[0][u], b[S - 1][u]);
        if (r0 + 2 * U >= sl.nrows) break;
    }
}

// ================================================================== encode: rank pass
// One wavefront per slab; reads old and new once.  For every changed element it needs its rank among
// the slab's elements with the same old exponent (`rank`) and among the slab's changes with that
// exponent (`rc`).  The running per-exponent counts in LDS give the part of `rank` before the row,
// ballots and mbcnt the stable part inside the row.  Changed elements are buffered in LDS in slab
// order as (rank, offset, old, new) and finished in dense batches: `rc` from per-exponent
// change counts and ballots over the batch, zigzag residual, checksum delta, 64-bit record.  Records
// go to the slab's own region, [base, base + cap): no shared counter.
__device__ void flush_changes(const EncRankArgs &a, const Slab &sl, const uint32_t *meta, const uint32_t *vals,
                              uint32_t *hchg, uint32_t cnt, uint64_t base, uint64_t cap, uint64_t &written,
                              uint64_t &dacc) {
    wave_fence();
    const bool fits = written + cnt <= cap;
    const uint32_t ln = lane();
    for (uint32_t j0 = 0; j0 < cnt; j0 += 64) {
        const uint32_t j = j0 + ln;
        const bool v = j < cnt;
        const uint32_t m = v ? meta[j] : 0u;  // rank | (offset - f_lo) << 16
        const uint32_t val = v ? vals[j] : 0u;  // old | new << 16
        const uint32_t k = v ? (val >> 7) & 0xFF : 256u;
        // rc: the exponent's changes in earlier batches plus the earlier lanes of this batch
        uint32_t rc = 0;
        uint64_t P = ballot(v);
        while (P) {
            const uint32_t kk = rdlane(k, (uint32_t)__builtin_ctzll(P));
            const uint64_t M = ballot(k == kk);
            const uint32_t before = hchg[kk];
            if (k == kk) rc = before + mbcnt(M);
            wave_fence();
            if (ln == 0) hchg[kk] = before + (uint32_t)__popcll(M);
            wave_fence();
            P &= ~M;
        }
        if (v) {
            const uint32_t o16 = val & 0xFFFF, n16 = val >> 16;
            const uint32_t f = (m >> 16) + sl.f_lo;
            dacc += (uint64_t)((int64_t)n16 - (int64_t)o16) * weight(sl.base + f);
            if (fits)
                a.rec[base + written + j] = (uint64_t)(m & 0xFFFF) | ((uint64_t)rc << 17) | ((uint64_t)k << 34) |
                                            ((uint64_t)zigzag(o16, n16) << 42);
        }
    }
    if (!fits && ln == 0) *a.overflow = 1u;
    written += cnt;
    wave_fence();
}

// the exponent-k count of the encode rank pass: the sum of its copies
__device__ __forceinline__ uint32_t rank_count(const uint32_t *hall, uint32_t k) {
    if (kRankCopies == 2) {
        const uint2 h = *reinterpret_cast<const uint2 *>(&hall[2 * k]);
        return h.x + h.y;
    }
    uint32_t s = 0;
#pragma unroll
    for (uint32_t q = 0; q < kRankCopies; q += 4) {
        const uint4 h = *reinterpret_cast<const uint4 *>(&hall[kRankCopies * k + q]);
        s += h.x + h.y + h.z + h.w;
    }
    return s;
}

template <bool COLD>
__device__ __forceinline__ void enc_rank_slab(const EncRankArgs &a, const TensorDesc &td, uint32_t tau, const Slab &sl,
                              uint32_t *hall, uint32_t *hchg, uint32_t *meta, uint32_t *vals) {
    const uint32_t ln = lane(), rep = ln & (kRankCopies - 1);
    const Rsrc src[2] = {slab_rsrc(td.frame, sl), slab_rsrc(td.frame_new, sl)};
    const uint64_t rbase = a.rec_base ? a.rec_base[tau] : (uint64_t)tau * a.rec_per_slab;
    const uint64_t rcap = a.rec_base ? ~0ULL : a.rec_per_slab;
    uint64_t written = 0;
    uint32_t cnt = 0;
    uint64_t dacc = 0;
    WeightedSum full;  // cold: checksum of new
    // cold: z = (index + 1) * golden of this lane's first element in the current row (element index
    // 2 * first word - lead + offset, computed in 64 bits: it is -1 for the pad before an odd start)
    uint64_t z = COLD ? (uint64_t)(2 * (int64_t)sl.first - (int64_t)td.lead + 2 * ln + 1) * kGolden : 0;
    stream_rows<kRankRows, 2, 0, kStreamNT>(sl, src, [&](uint32_t r, uint32_t o, uint32_t nw) {
        // exponents; lanes outside the slab count into slot 256 and never change
        uint32_t k0 = (o >> 7) & 0xFF, k1 = (o >> 23) & 0xFF, x = o ^ nw, n = nw;
        if (!row_full(sl, r)) {
            const uint32_t f = r * kRow + 2 * ln;
            if (f < sl.f_lo || f >= sl.f_hi) {
                k0 = 256;
                x &= 0xFFFF0000u;
                n &= 0xFFFF0000u;
            }
            if (f + 1 < sl.f_lo || f + 1 >= sl.f_hi) {
                k1 = 256;
                x &= 0xFFFFu;
                n &= 0xFFFFu;
            }
        }
        const bool c0 = (x & 0xFFFF) != 0, c1 = x > 0xFFFF;
        const uint64_t C0 = ballot(c0), C1 = ballot(c1);
        if ((C0 | C1) && __popcll(C0) + __popcll(C1) == 1) {
            // one change in the row (about half the rows with changes at 1%): its rank and buffer
            // entry from scalar ballot arithmetic, written by its own lane
            const bool hi = C0 == 0;  // the change is the high element of its lane
            const uint32_t l = (uint32_t)__builtin_ctzll(hi ? C1 : C0);
            const uint32_t k = hi ? rdlane(k1, l) : rdlane(k0, l);
            const uint64_t M0 = ballot(k0 == k), M1 = ballot(k1 == k), lt = (1ULL << l) - 1;
            const uint32_t in_row = (uint32_t)(__popcll(M0 & lt) + __popcll(M1 & lt)) + (hi ? (uint32_t)(M0 >> l) & 1u : 0u);
            const uint32_t rk = rank_count(hall, k) + in_row;
            if (ln == l) {
                const uint32_t fr = (r * kRow + 2 * ln + (hi ? 1u : 0u) - sl.f_lo) << 16;
                meta[cnt] = rk | fr;
                vals[cnt] = hi ? (o >> 16) | (n & 0xFFFF0000u) : (o & 0xFFFF) | (n << 16);
            }
            cnt += 1;
            wave_fence();
        } else if (C0 | C1) {
            uint32_t rk0 = 0, rk1 = 0;  // meaningful for changed elements only
            uint64_t P0 = C0, P1 = C1;
            do {  // once per distinct exponent among this row's changes
                const uint32_t l = (uint32_t)__builtin_ctzll(P0 | P1);
                const uint32_t k = rdlane((P0 >> l) & 1 ? k0 : k1, l);
                const bool m0 = k0 == k, m1 = k1 == k;
                const uint64_t M0 = ballot(m0), M1 = ballot(m1);
                // exponent-k elements before this row, plus this row's before this lane
                const uint32_t before = rank_count(hall, k) +
                                        __builtin_amdgcn_mbcnt_hi((uint32_t)(M1 >> 32),
                                            __builtin_amdgcn_mbcnt_lo((uint32_t)M1, mbcnt(M0)));
                if (m0) rk0 = before;
                if (m1) rk1 = before + (m0 ? 1u : 0u);
                P0 &= ~M0;
                P1 &= ~M1;
            } while (P0 | P1);
            const uint32_t f = r * kRow + 2 * ln;
            const uint32_t cb = __builtin_amdgcn_mbcnt_hi((uint32_t)(C1 >> 32),
                                    __builtin_amdgcn_mbcnt_lo((uint32_t)C1, cnt + mbcnt(C0)));  // buffer slot
            const uint32_t fr = (f - sl.f_lo) << 16;  // slab offsets past f_lo fit 16 bits (slab <= 65536)
            if (c0) {
                meta[cb] = rk0 | fr;
                vals[cb] = (o & 0xFFFF) | (n << 16);
            }
            if (c1) {
                const uint32_t s = cb + (c0 ? 1u : 0u);
                meta[s] = rk1 | (fr + 0x10000u);
                vals[s] = (o >> 16) | (n & 0xFFFF0000u);
            }
            cnt += (uint32_t)(__popcll(C0) + __popcll(C1));
            wave_fence();
        }
        atomicAdd(&hall[kRankCopies * k0 + rep], 1u);
        atomicAdd(&hall[kRankCopies * k1 + rep], 1u);
        if (COLD) {  // elements outside the slab were zeroed in n
            full.add(n & 0xFFFF, mix_weight(z));
            full.add(n >> 16, mix_weight(z + kGolden));
            z += (uint64_t)kRow * kGolden;
        }
        if (cnt > kChgCap - kRow) {
            flush_changes(a, sl, meta, vals, hchg, cnt, rbase, rcap, written, dacc);
            cnt = 0;
        }
    });
    if (cnt) flush_changes(a, sl, meta, vals, hchg, cnt, rbase, rcap, written, dacc);
    wave_fence();
    for (uint32_t k = ln; k < 256; k += 64) {
        a.hall[(uint64_t)tau * 256 + k] = rank_count(hall, k);
        a.hchg[(uint64_t)tau * 256 + k] = hchg[k];
    }
    dacc = wave_sum(dacc);
    const uint64_t facc = wave_sum(full.total());
    if (ln == 0) {
        a.delta[tau] = dacc;
        a.full[tau] = facc;
        a.rec_count[tau] = (uint32_t)written;
    }
}

__global__ __launch_bounds__(64) void k_enc_rank(EncRankArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t hall[257 * kRankCopies];  // copies by lane; 256: outside
    __shared__ uint32_t hchg[256];
    __shared__ uint32_t meta[kChgCap];
    __shared__ uint32_t vals[kChgCap];
    const uint32_t tau = blockIdx.x;
    const TensorDesc td = a.descs[a.tile_tensor[tau]];
    const Slab sl = slab_of(td, tau - td.tile_begin, a.slab);
    for (uint32_t i = lane(); i < 257 * kRankCopies; i += 64) hall[i] = 0;
    for (uint32_t i = lane(); i < 256; i += 64) hchg[i] = 0;
    wave_fence();
    if (td.cold) enc_rank_slab<true>(a, td, tau, sl, hall, hchg, meta, vals);
    else enc_rank_slab<false>(a, td, tau, sl, hall, hchg, meta, vals);
}

// ================================================================== apply: histogram pass
// 8 copies of every exponent's count, copy = lane & 7, so the atomics of a row rarely collide.  Lanes
// outside the slab count into exponent slot 256.  The old weights' checksum, when not cached, is
// needed only by the verdict; it is arithmetic-bound and this pass is bound by its atomics, the select
// pass by memory, so the two split it: this pass sums a slab's even rows, the select pass its odd
// rows (all of them when this pass does not stream the slab: its counts are cached).
constexpr uint32_t kHistCopies = 8;

// The weighted sum of a cold slab's weights for its tensor's checksum (codec.py:61-68), over its odd
// rows (odd) or all of them: one stream of the slab, for slabs the select pass does not stream (no
// targets, or an update already rejected).
__device__ __forceinline__ uint64_t cold_sum(const TensorDesc &td, const Slab &sl, bool odd) {
    const uint32_t ln = lane();
    const Rsrc src[1] = {slab_rsrc(td.frame, sl)};
    WeightedSum acc;
    // z = (index + 1) * golden of this lane's first element in the current row
    uint64_t z = (uint64_t)(2 * (int64_t)sl.first - (int64_t)td.lead + 2 * ln + 1) * kGolden;
    // half the histogram pass's batch: this runs for few slabs, inside kernels whose occupancy its
    // registers would otherwise set
    stream_rows<kScanRows / 2>(sl, src, [&](uint32_t r, uint32_t o, uint32_t) {
        uint32_t v = o;
        if (!row_full(sl, r)) {
            const uint32_t f = r * kRow + 2 * ln;
            if (f < sl.f_lo || f >= sl.f_hi) v &= 0xFFFF0000u;
            if (f + 1 < sl.f_lo || f + 1 >= sl.f_hi) v &= 0xFFFFu;
        }
        if (!odd || (r & 1u)) {
            acc.add(v & 0xFFFF, mix_weight(z));
            acc.add(v >> 16, mix_weight(z + kGolden));
        }
        z += (uint64_t)kRow * kGolden;
    });
    return wave_sum(acc.total());
}

template <bool COLD>
__device__ void hist_slab(const HistArgs &a, const TensorDesc &td, uint32_t tau, const Slab &sl, uint32_t *hall) {
    const uint32_t ln = lane(), rep = ln & (kHistCopies - 1);
    const Rsrc src[1] = {slab_rsrc(td.frame, sl)};
    WeightedSum full;  // COLD: the even rows' part of the old checksum
    // COLD: z = (index + 1) * golden of this lane's first element in the current row
    uint64_t z = COLD ? (uint64_t)(2 * (int64_t)sl.first - (int64_t)td.lead + 2 * ln + 1) * kGolden : 0;
    stream_rows<kScanRows>(sl, src, [&](uint32_t r, uint32_t o, uint32_t) {
        const uint32_t f = r * kRow + 2 * ln;
        uint32_t k0 = (o >> 7) & 0xFF, k1 = (o >> 23) & 0xFF, v = o;
        if (!row_full(sl, r)) {
            if (f < sl.f_lo || f >= sl.f_hi) {
                k0 = 256;
                v &= 0xFFFF0000u;
            }
            if (f + 1 < sl.f_lo || f + 1 >= sl.f_hi) {
                k1 = 256;
                v &= 0xFFFFu;
            }
        }
        atomicAdd(&hall[k0 * kHistCopies + rep], 1u);
        atomicAdd(&hall[k1 * kHistCopies + rep], 1u);
        if (COLD) {
            if (!(r & 1u)) {
                full.add(v & 0xFFFF, mix_weight(z));
                full.add(v >> 16, mix_weight(z + kGolden));
            }
            z += (uint64_t)kRow * kGolden;
        }
    });
    wave_fence();
    uint32_t *out = td.hist_out ? td.hist_out + (uint64_t)(tau - td.tile_begin) * 256 : nullptr;
    for (uint32_t k = ln; k < 256; k += 64) {
        uint32_t sum = 0;
#pragma unroll
        for (uint32_t q = 0; q < kHistCopies; q += 4) {
            const uint4 h = *reinterpret_cast<const uint4 *>(&hall[k * kHistCopies + q]);
            sum += h.x + h.y + h.z + h.w;
        }
        a.hall[(uint64_t)tau * 256 + k] = sum;
        if (out) out[k] = sum;
    }
    if (COLD) {
        const uint64_t facc = wave_sum(full.total());
        if (ln == 0) a.full[tau] = facc;
    }
}

__global__ __launch_bounds__(64) void k_hist(HistArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t hall[257 * kHistCopies];
    const uint32_t tau = a.list ? a.list[blockIdx.x] : blockIdx.x;
    const TensorDesc td = a.descs[a.tile_tensor[tau]];
    if (td.hist_in) {  // counts recorded by the previous update: copied to a separate hist_out
        const uint64_t at = (uint64_t)(tau - td.tile_begin) * 256;
        for (uint32_t k = lane(); k < 256; k += 64) td.hist_out[at + k] = td.hist_in[at + k];
        return;
    }
    const Slab sl = slab_of(td, tau - td.tile_begin, a.slab);
    for (uint32_t i = lane(); i < 257 * kHistCopies; i += 64) hall[i] = 0;
    wave_fence();
    if (td.cold) hist_slab<true>(a, td, tau, sl, hall);
    else hist_slab<false>(a, td, tau, sl, hall);
}

// ================================================================== per-tensor histogram scan
// h[tile][256] -> exclusive prefix over the tensor's slabs, in place; totals[tensor][256].
// The loops below read a batch of values before writing any (the reads and writes alias as far as
// the compiler knows), so a batch costs one memory latency instead of one per value.
constexpr uint32_t kScanBatch = 32;  // = kScanTiles: a chunk in one batch

// Per-slab counts of slab t of a chunk's tensor: the receiver's cached counts when the apply uses
// them (the histogram pass skipped those slabs), else the table being scanned.
__device__ __forceinline__ const uint32_t *scan_src(const TensorDesc &td, const uint32_t *h, uint32_t t) {
    return td.hist_in ? td.hist_in + (uint64_t)(t - td.tile_begin) * 256 : h + (uint64_t)t * 256;
}

// One or two tables are scanned by the same launches: workgroup i takes table i / n (n chunks or
// tensors per table) and its chunk or tensor i mod n.
__global__ __launch_bounds__(256) void k_scan_sum(const TensorDesc *descs, ScanTabs p, const ScanChunk *ch,
                                                  uint32_t n_chunks) {
    const uint32_t tab = blockIdx.x >= n_chunks, i = blockIdx.x - tab * n_chunks;
    const ScanChunk c = ch[i];
    const TensorDesc td = descs[c.tensor];
    const uint32_t *const h = p.h[tab];
    const uint32_t k = threadIdx.x;
    uint32_t s = 0;
    for (uint32_t t0 = c.tile_begin; t0 < c.tile_end; t0 += kScanBatch) {  // a batch of loads in flight
        uint32_t x[kScanBatch];
#pragma unroll
        for (uint32_t j = 0; j < kScanBatch; ++j) x[j] = t0 + j < c.tile_end ? scan_src(td, h, t0 + j)[k] : 0u;
#pragma unroll
        for (uint32_t j = 0; j < kScanBatch; ++j) s += x[j];
    }
    p.csum[tab][(uint64_t)i * 256 + k] = s;
}

// exclusive running sums of src column k over rows i0 .. i0 + n into dst (which may be src);
// src(i) and dst(i) give row i.  Returns the total.
template <typename Src, typename Dst>
__device__ __forceinline__ uint32_t scan_column(Src src, Dst dst, uint32_t i0, uint32_t n, uint32_t k, uint32_t run) {
    for (uint32_t b = 0; b < n; b += kScanBatch) {
        uint32_t x[kScanBatch];
#pragma unroll
        for (uint32_t j = 0; j < kScanBatch; ++j)
            if (b + j < n) x[j] = src(i0 + b + j)[k];
#pragma unroll
        for (uint32_t j = 0; j < kScanBatch; ++j) {
            if (b + j < n) {
                dst(i0 + b + j)[k] = run;
                run += x[j];
            }
        }
    }
    return run;
}

__global__ __launch_bounds__(256) void k_scan_mid(ScanTabs p, const uint32_t *tcb, uint32_t n_tensors) {
    const uint32_t tab = blockIdx.x >= n_tensors, t = blockIdx.x - tab * n_tensors, k = threadIdx.x;
    uint32_t *const csum = p.csum[tab];
    auto row = [&](uint32_t i) { return csum + (uint64_t)i * 256; };
    p.totals[tab][(uint64_t)t * 256 + k] = scan_column(row, row, tcb[t], tcb[t + 1] - tcb[t], k, 0);
}

__global__ __launch_bounds__(256) void k_scan_fin(const TensorDesc *descs, ScanTabs p, const ScanChunk *ch,
                                                  uint32_t n_chunks) {
    const uint32_t tab = blockIdx.x >= n_chunks, i = blockIdx.x - tab * n_chunks;
    const ScanChunk c = ch[i];
    const TensorDesc td = descs[c.tensor];
    uint32_t *const h = p.h[tab];
    const uint32_t k = threadIdx.x;
    auto src = [&](uint32_t t) { return scan_src(td, h, t); };
    auto dst = [&](uint32_t t) { return h + (uint64_t)t * 256; };
    scan_column(src, dst, c.tile_begin, c.tile_end - c.tile_begin, k, p.csum[tab][(uint64_t)i * 256 + k]);
}

// ================================================================== encode: groups and placement
// Groups are the non-empty (tensor, exponent) pairs in (tensor, exponent) order (codec.py:317-333).

// Records -> update order: position = group start + changes of the group in earlier slabs + rank
// among the slab's changes of that exponent; value = zz and the group-local index.
// One wavefront per slab: its records -> (zz << 32 | group-local index) at the change's place in
// update order.
__global__ __launch_bounds__(64) void k_place(EncRankArgs a, const uint32_t *tile_tensor, const uint32_t *hall_pre,
                                              const uint32_t *hchg_pre, const uint32_t *gbase, uint64_t *sorted,
                                              uint64_t n_sorted) {
    // per exponent of this slab: first group-local index, first place in update order
    __shared__ uint32_t off_rank[256], off_dest[256];
    const uint32_t tau = blockIdx.x, ln = lane();
    const uint32_t t = tile_tensor[tau], count = a.rec_count[tau];
    const uint64_t base = a.rec_base ? a.rec_base[tau] : (uint64_t)tau * a.rec_per_slab;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t k = ln + 64 * q;
        off_rank[k] = hall_pre[(uint64_t)tau * 256 + k];
        off_dest[k] = gbase[(uint64_t)t * 256 + k] + hchg_pre[(uint64_t)tau * 256 + k];
    }
    wave_fence();
    // kPlaceRecs records per lane: all loads, then all LDS lookups, then all stores (a load issued
    // after a store would wait for the store too)
    constexpr uint32_t U = kPlaceRecs;
    for (uint32_t j0 = 0; j0 < count; j0 += 64 * U) {
        uint64_t r[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t j = j0 + 64 * u + ln;
            r[u] = j < count ? a.rec[base + j] : 0ULL;
        }
        uint32_t dest[U], lo[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t rank = (uint32_t)(r[u] & 0x1FFFF), rc = (uint32_t)((r[u] >> 17) & 0x1FFFF);
            const uint32_t k = (uint32_t)((r[u] >> 34) & 0xFF);
            dest[u] = off_dest[k] + rc;
            lo[u] = off_rank[k] + rank;
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t j = j0 + 64 * u + ln;
            if (j < count && dest[u] < n_sorted) sorted[dest[u]] = ((r[u] >> 42) << 32) | lo[u];
        }
    }
}

// r0 = floor(log2(max(mean gap, 1))) clamped to 30; the gaps of a group sum to last index + 1 - count.
__global__ __launch_bounds__(256) void k_r0(GroupDev *groups, uint32_t n_groups, const uint64_t *sorted) {
    const uint32_t g = blockIdx.x * 256 + threadIdx.x;
    if (g >= n_groups) return;
    const GroupDev gr = groups[g];
    const uint64_t last = (uint32_t)sorted[(uint64_t)gr.elem_base + gr.count - 1];
    const uint64_t s = last + 1 - gr.count;
    uint32_t r0 = 0;
    while (r0 < 30 && ((uint64_t)gr.count << (r0 + 1)) <= s) ++r0;
    groups[g].r0 = r0;
}

// Records of a workgroup's changes in LDS: thread t's kElemsPerThread records at t * kRecPad (the pad
// spreads one wavefront's reads of its threads' k-th records over the banks).
constexpr uint32_t kRecPad = kElemsPerThread + 1;

// All of a thread's loads are issued before any is stored (one memory latency per workgroup, not
// one per record).
__device__ __forceinline__ void stage_records(const uint64_t *sorted, uint64_t n, uint64_t wbase, uint64_t *rec) {
    constexpr uint32_t kPer = kElemsPerWG / 256;
    uint64_t v[kPer];
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        const uint64_t i = wbase + threadIdx.x + 256 * u;
        v[u] = i < n ? sorted[i] : 0ULL;
    }
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        const uint32_t j = threadIdx.x + 256 * u;
        rec[(j / kElemsPerThread) * kRecPad + (j % kElemsPerThread)] = v[u];
    }
    __syncthreads();
}

// group-local index of the change before this thread's first one (0 if it starts its group)
__device__ __forceinline__ uint64_t prev_index(const uint64_t *sorted, const uint64_t *rec, uint64_t ib, uint32_t elem_base) {
    if (ib <= elem_base) return 0;
    return (uint32_t)(threadIdx.x ? rec[(threadIdx.x - 1) * kRecPad + kElemsPerThread - 1] : sorted[ib - 1]);
}

__device__ __forceinline__ void rice_cands(uint32_t r0, uint32_t c[3]) {
    c[0] = r0 ? r0 - 1 : 0;
    c[1] = r0;
    c[2] = r0 < 30 ? r0 + 1 : 30;
}

// Per workgroup: 4096 consecutive changes, 16 contiguous per thread.  Sums of gap >> r for the
// three Rice candidates of each group, residual symbol counts per exponent (dense below kDense,
// the rest appended to a list the host sorts).
__global__ __launch_bounds__(256) void k_stats(StatsArgs a) {
    __shared__ uint32_t lhist[kLocalGroups * kDense];
    __shared__ unsigned long long lcost[kLocalGroups * 3];
    __shared__ uint64_t rec[256 * kRecPad];
    const uint32_t tid = threadIdx.x;
    const uint64_t wbase = (uint64_t)blockIdx.x * kElemsPerWG;
    for (uint32_t x = tid; x < kLocalGroups * kDense; x += 256) lhist[x] = 0;
    for (uint32_t x = tid; x < kLocalGroups * 3; x += 256) lcost[x] = 0;
    stage_records(a.sorted, a.n, wbase, rec);
    const uint32_t gf = a.cmap[wbase / kElemsPerThread];
    const uint64_t ib = wbase + (uint64_t)tid * kElemsPerThread;
    const bool any = ib < a.n;
    uint32_t g = any ? a.cmap[ib / kElemsPerThread] : 0;
    GroupDev gr = a.groups[g];
    uint32_t c[3];
    rice_cands(gr.r0, c);
    uint64_t prev = any ? prev_index(a.sorted, rec, ib, gr.elem_base) : 0;
    unsigned long long s0 = 0, s1 = 0, s2 = 0;
    auto flush_cost = [&](uint32_t gg) {
        if (!(s0 | s1 | s2)) return;
        const uint32_t lg = gg - gf;
        if (lg < kLocalGroups) {
            atomicAdd(&lcost[lg * 3 + 0], s0);
            atomicAdd(&lcost[lg * 3 + 1], s1);
            atomicAdd(&lcost[lg * 3 + 2], s2);
        } else {
            atomicAdd(&a.cost[(uint64_t)gg * 3 + 0], s0);
            atomicAdd(&a.cost[(uint64_t)gg * 3 + 1], s1);
            atomicAdd(&a.cost[(uint64_t)gg * 3 + 2], s2);
        }
        s0 = s1 = s2 = 0;
    };
    for (int k = 0; k < kElemsPerThread; ++k) {
        const uint64_t i = ib + k;
        const bool valid = i < a.n;
        uint32_t zz = 0, e = 0;
        if (valid) {
            while (i >= (uint64_t)gr.elem_base + gr.count) {
                flush_cost(g);
                gr = a.groups[++g];
                rice_cands(gr.r0, c);
            }
            const uint64_t v = rec[tid * kRecPad + k];
            const uint64_t gidx = (uint32_t)v;
            zz = (uint32_t)(v >> 32);
            e = gr.exponent;
            const uint64_t gap = i == gr.elem_base ? gidx : gidx - prev - 1;
            prev = gidx;
            s0 += gap >> c[0];
            s1 += gap >> c[1];
            s2 += gap >> c[2];
            if (zz < kDense) {
                const uint32_t lg = g - gf;
                if (lg < kLocalGroups) atomicAdd(&lhist[lg * kDense + zz], 1u);
                else atomicAdd(&a.dense[e * kDense + zz], 1u);
            }
        }
        const bool rare = valid && zz >= kDense;
        const uint64_t m = ballot(rare);
        if (m) {
            const uint32_t leader = (uint32_t)__builtin_ctzll(m);
            unsigned long long base = 0;
            if (lane() == leader) base = atomicAdd(&a.counters[0], (unsigned long long)__popcll(m));
            base = __shfl(base, leader, 64);
            if (rare) {
                const unsigned long long idx = base + mbcnt(m);
                if (idx < a.rare_cap) a.rare[idx] = (e << 17) | zz;
                else atomicOr(&a.counters[1], 1ULL);
            }
        }
    }
    if (any) flush_cost(g);
    __syncthreads();
    for (uint32_t x = tid; x < kLocalGroups * kDense; x += 256) {
        const uint32_t v = lhist[x];
        if (v) atomicAdd(&a.dense[a.groups[gf + x / kDense].exponent * kDense + x % kDense], v);
    }
    for (uint32_t x = tid; x < kLocalGroups * 3; x += 256) {
        const unsigned long long v = lcost[x];
        if (v) atomicAdd(&a.cost[(uint64_t)(gf + x / 3) * 3 + x % 3], v);
    }
}

// ================================================================== encode: code lengths and packing
// The change-order kernels give each thread kElemsPerThread consecutive changes.  A workgroup's
// records are first staged in LDS with coalesced loads (thread t's records at t * kRecPad: the pad
// spreads one wavefront's reads of its threads' k-th records over the banks); each thread then walks
// its records from LDS and issues its table lookups together.
// A thread's codes: gap, key = exponent << 22 | rice << 17 | zz, the Huffman entry and, when the
// change opens a block, the block index.
struct ThreadCodes {
    uint64_t gap[kElemsPerThread];
    uint32_t key[kElemsPerThread];
    uint32_t hv[kElemsPerThread];   // (code << 5) | length
    uint32_t blk[kElemsPerThread];  // block opened by the change, else kNone
    uint32_t n;
};

__device__ __forceinline__ uint32_t huff_entry(const CodeArgs &a, uint32_t e, uint32_t zz) {
    if (zz < kDense) return a.lut[e * kDense + zz];
    const uint32_t key = (e << 17) | zz;
    uint32_t lo = 0, hi = a.n_rare;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (a.rare_keys[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    return lo < a.n_rare ? a.rare_vals[lo] : 0u;
}

__device__ __forceinline__ void thread_codes(const CodeArgs &a, const uint64_t *rec, uint64_t wbase, ThreadCodes &tc) {
    const uint32_t t = threadIdx.x;
    const uint64_t ib = wbase + (uint64_t)t * kElemsPerThread;
    tc.n = ib < a.n ? (uint32_t)min64(kElemsPerThread, a.n - ib) : 0u;
    uint32_t g = tc.n ? a.cmap[ib / kElemsPerThread] : 0u;
    GroupDev gr = a.groups[g];
    uint64_t gend = (uint64_t)gr.elem_base + gr.count;
    uint64_t prev = tc.n ? prev_index(a.sorted, rec, ib, gr.elem_base) : 0;
#pragma unroll
    for (int k = 0; k < kElemsPerThread; ++k) {
        const uint64_t i = ib + k;
        tc.gap[k] = 0;
        tc.key[k] = 0;
        tc.blk[k] = kNone;
        if ((uint32_t)k < tc.n) {
            while (i >= gend) {
                gr = a.groups[++g];
                gend = (uint64_t)gr.elem_base + gr.count;
            }
            const uint64_t v = rec[t * kRecPad + k];
            const uint64_t gidx = (uint32_t)v;
            tc.gap[k] = i == gr.elem_base ? gidx : gidx - prev - 1;
            prev = gidx;
            tc.key[k] = (gr.exponent << 22) | (gr.rice << 17) | (uint32_t)(v >> 32);
            const uint64_t rel = i - gr.elem_base;
            if ((rel & 255) == 0) tc.blk[k] = gr.blk_base + (uint32_t)(rel >> 8);
        }
    }
#pragma unroll
    for (int k = 0; k < kElemsPerThread; ++k)
        tc.hv[k] = (uint32_t)k < tc.n ? huff_entry(a, tc.key[k] >> 22, tc.key[k] & 0x1FFFF) : 0u;
}

__device__ __forceinline__ uint64_t code_len(const ThreadCodes &tc, int k) {
    const uint32_t rice = (tc.key[k] >> 17) & 31;
    return (tc.gap[k] >> rice) + 1 + rice + (tc.hv[k] & 31);
}

// Exclusive sum over a 256-thread workgroup (4 wavefronts): wavefront scans by shuffles, then the
// 4 wavefront totals through `sh` (at least 4 entries).  *total receives the workgroup's sum.
__device__ unsigned long long block_exclusive_sum(unsigned long long v, unsigned long long *sh, unsigned long long *total) {
    const uint32_t ln = lane(), w = threadIdx.x >> 6;
    unsigned long long incl = v;
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long t = __shfl_up(incl, o, 64);
        if (ln >= (uint32_t)o) incl += t;
    }
    if (ln == 63) sh[w] = incl;
    __syncthreads();
    unsigned long long before = 0, tot = 0;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        const unsigned long long x = sh[q];
        if (q < w) before += x;
        tot += x;
    }
    __syncthreads();  // sh may be reused by the caller
    *total = tot;
    return before + incl - v;
}

// Groups from the (tensor, exponent) change totals, in that order: kGroupChunk totals per workgroup
// (16 consecutive per thread).  A workgroup first sums the totals before its chunk (coalesced, a few
// hundred KB at most), then scans its own.  gbase[i] = changes before entry i; counters[0] = groups,
// counters[1] = changes (written by the last workgroup).
constexpr uint32_t kGroupChunk = 4096;
__global__ __launch_bounds__(256) void k_enc_groups(const uint32_t *tot, uint32_t n_tensors, GroupDev *groups,
                                                    uint32_t *gbase, unsigned long long *counters) {
    __shared__ unsigned long long sh[8];
    const uint32_t tid = threadIdx.x;
    const uint64_t n = (uint64_t)n_tensors * 256, c0 = (uint64_t)blockIdx.x * kGroupChunk;
    unsigned long long pv = 0, pz = 0;  // totals before the chunk
    for (uint64_t i0 = tid; i0 < c0; i0 += 256 * 8) {
        uint32_t v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) v[u] = i0 + 256 * u < c0 ? tot[i0 + 256 * u] : 0u;
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            pv += v[u];
            pz += v[u] ? 1u : 0u;
        }
    }
    unsigned long long bv, bz;
    block_exclusive_sum(pv, sh, &bv);
    block_exclusive_sum(pz, sh, &bz);
    const uint64_t lo = min64(c0 + 16ull * tid, n), hi = min64(lo + 16, n);
    uint32_t v[16];
    unsigned long long sv = 0, sz = 0;
#pragma unroll
    for (uint32_t u = 0; u < 16; ++u) {
        v[u] = lo + u < hi ? tot[lo + u] : 0u;
        sv += v[u];
        sz += v[u] ? 1u : 0u;
    }
    unsigned long long tv, tz;
    unsigned long long ev = bv + block_exclusive_sum(sv, sh, &tv);
    unsigned long long ez = bz + block_exclusive_sum(sz, sh, &tz);
#pragma unroll
    for (uint32_t u = 0; u < 16; ++u) {
        const uint64_t i = lo + u;
        if (i < hi) {
            gbase[i] = (uint32_t)ev;  // meaningful while the total stays below 2^32 (checked by the host)
            if (v[u]) {
                GroupDev g{};
                g.tensor = (uint32_t)(i >> 8);
                g.exponent = (uint32_t)(i & 255);
                g.count = v[u];
                g.elem_base = (uint32_t)ev;
                groups[ez] = g;
                ++ez;
            }
            ev += v[u];
        }
    }
    if (blockIdx.x + 1 == gridDim.x && tid == 0) {
        counters[0] = bz + tz;  // groups
        counters[1] = bv + tv;  // changes
    }
}

__global__ __launch_bounds__(256) void k_code_lengths(CodeArgs a) {
    __shared__ uint64_t rec[256 * kRecPad];
    const uint64_t wbase = (uint64_t)blockIdx.x * kElemsPerWG;
    stage_records(a.sorted, a.n, wbase, rec);
    ThreadCodes tc;
    thread_codes(a, rec, wbase, tc);
    if (!tc.n) return;
    unsigned long long sum = 0;
#pragma unroll
    for (int k = 0; k < kElemsPerThread; ++k)
        if ((uint32_t)k < tc.n) sum += code_len(tc, k);
    a.tsum[(uint64_t)blockIdx.x * 256 + threadIdx.x] = sum;
}

// A thread's codes fill the contiguous bit range [off, off + its total): words wholly inside the
// range are written with plain stores; the first word (when the range starts inside it) and the
// last partial word are shared with the neighbouring threads and are ORed in.  The stream is
// big-endian bytes in 32-bit words and starts zeroed.
// A thread's codes fill the contiguous bit range [off, off + its total).  In LDS (the workgroup's
// words staged in `words`, indexed from word `w0`) every word is ORed in; in HBM, words wholly inside
// the range are written with plain stores and only the first (when the range starts inside it) and
// the last partial word, shared with the neighbouring threads, are ORed in.  Big-endian bytes in
// 32-bit words; the words start zeroed.
template <bool LDS>
struct BitWriter {
    uint32_t *words;
    uint64_t w;       // next word to write
    uint64_t acc;     // pending bits, right-aligned
    uint32_t n;       // number of pending bits (< 32 between calls)
    bool shared;      // the next word is shared with the previous thread

    __device__ BitWriter(uint32_t *words_, uint64_t w0, uint64_t off)
        : words(words_ - (LDS ? w0 : 0)), w(off >> 5), acc(0), n((uint32_t)(off & 31)), shared((off & 31) != 0) {}

    __device__ __forceinline__ void emit(uint32_t v) {
        if (LDS || shared) atomicOr(&words[w], __builtin_bswap32(v));
        else words[w] = __builtin_bswap32(v);
        shared = false;
        ++w;
    }
    // len <= 32 bits of v (right-aligned, no bits above len)
    __device__ __forceinline__ void put(uint64_t v, uint32_t len) {
        acc = (acc << len) | v;
        n += len;
        if (n >= 32) {
            n -= 32;
            emit((uint32_t)(acc >> n));
            acc &= (1ULL << n) - 1;
        }
    }
    __device__ __forceinline__ void ones(uint64_t q) {
        for (; q >= 32; q -= 32) put(0xFFFFFFFFULL, 32);
        if (q) put((1ULL << q) - 1, (uint32_t)q);
    }
    __device__ __forceinline__ void finish() {
        if (n) atomicOr(&words[w], __builtin_bswap32((uint32_t)(acc << (32 - n))));
    }
};

// 1^q 0 r-bit remainder, then the Huffman code (codec.py:214-257)
template <bool LDS>
__device__ __forceinline__ void put_code(BitWriter<LDS> &bw, uint64_t gap, uint32_t rice, uint32_t hv) {
    const uint64_t q = gap >> rice;
    const uint32_t hl = hv & 31;
    const uint64_t tail = ((gap & ((1ULL << rice) - 1)) << hl) | (hv >> 5);  // 0, r bits, Huffman code
    const uint32_t tail_len = 1 + rice + hl;                                  // <= 48
    if (q + tail_len <= 32) {
        bw.put(q ? (((1ULL << q) - 1) << tail_len) | tail : tail, (uint32_t)(q + tail_len));
    } else {
        bw.ones(q);
        if (tail_len > 32) {
            bw.put(tail >> 32, tail_len - 32);
            bw.put(tail & 0xFFFFFFFFULL, 32);
        } else {
            bw.put(tail, tail_len);
        }
    }
}

template <bool LDS>
__device__ __forceinline__ void pack_thread(const CodeArgs &a, const ThreadCodes &tc, uint32_t *words, uint64_t w0,
                                            unsigned long long off) {
    BitWriter<LDS> bw(words, w0, off);
#pragma unroll
    for (int k = 0; k < kElemsPerThread; ++k) {
        if ((uint32_t)k < tc.n) {
            if (tc.blk[k] != kNone) a.bstart[tc.blk[k]] = off;
            const uint32_t rice = (tc.key[k] >> 17) & 31;
            put_code(bw, tc.gap[k], rice, tc.hv[k]);
            off += code_len(tc, k);
        }
    }
    bw.finish();
}

// The workgroup's bits are assembled in LDS (the record staging area, free once the codes are in
// registers) and written out with coalesced stores; only its first and last words, which it may
// share with the neighbouring workgroups, are ORed into HBM.  A workgroup whose bits do not fit
// writes them directly.
constexpr uint32_t kPackLdsWords = 256 * kRecPad * 2;
__global__ __launch_bounds__(256) void k_pack(CodeArgs a) {
    __shared__ uint64_t rec[256 * kRecPad];
    const uint64_t wbase = (uint64_t)blockIdx.x * kElemsPerWG;
    stage_records(a.sorted, a.n, wbase, rec);
    ThreadCodes tc;
    thread_codes(a, rec, wbase, tc);
    const uint64_t t0 = (uint64_t)blockIdx.x * 256, n_thr = (a.n + kElemsPerThread - 1) / kElemsPerThread;
    const unsigned long long b_lo = a.bit_base + a.toff[t0], b_hi = a.bit_base + a.toff[min64(t0 + 256, n_thr)];
    const uint64_t w0 = b_lo >> 5, nw = ((b_hi + 31) >> 5) - w0;
    const unsigned long long off = tc.n ? a.bit_base + a.toff[t0 + threadIdx.x] : 0ULL;
    if (w0 + nw > a.n_words) {  // uniform: the payload was sized from other lengths than these
        if (threadIdx.x == 0) atomicOr(a.overflow, 2u);
        return;
    }
    if (nw > kPackLdsWords) {  // uniform across the workgroup
        if (tc.n) pack_thread<false>(a, tc, a.words, 0, off);
        return;
    }
    uint32_t *buf = reinterpret_cast<uint32_t *>(rec);
    __syncthreads();  // every thread has read its records
    for (uint32_t i = threadIdx.x; i < nw; i += 256) buf[i] = 0;
    __syncthreads();
    if (tc.n) pack_thread<true>(a, tc, buf, w0, off);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nw; i += 256) {
        const uint32_t v = buf[i];
        if (i == 0 || i + 1 == nw) {
            if (v) atomicOr(&a.words[w0 + i], v);
        } else {
            a.words[w0 + i] = v;
        }
    }
}

__global__ __launch_bounds__(256) void k_block_bits(const unsigned long long *bstart, uint64_t n_blocks, uint32_t *out,
                                                    unsigned int *overflow) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= n_blocks) return;
    const unsigned long long len = bstart[b + 1] - bstart[b];
    if (len >= (1ULL << 32)) atomicOr(overflow, 1u);
    out[b] = (uint32_t)len;
}

// ================================================================== generic scans and sums
// Exclusive prefix sums, out[i] = in[0] + ... + in[i-1] and out[n] = total, in three coalesced
// passes: per-chunk sums, a scan of the chunk sums (one workgroup), then the chunks themselves.
constexpr uint32_t kScanChunk = 4096;  // elements per workgroup: 256 threads x 16

template <typename T>
__global__ __launch_bounds__(256) void k_scan_reduce(const T *in, uint64_t n, unsigned long long *part) {
    __shared__ unsigned long long sh[4];
    const uint64_t b = (uint64_t)blockIdx.x * kScanChunk;
    unsigned long long s = 0;
    for (uint32_t j = threadIdx.x; j < kScanChunk; j += 256)
        if (b + j < n) s += in[b + j];
    unsigned long long tot;
    block_exclusive_sum(s, sh, &tot);
    if (threadIdx.x == 0) part[blockIdx.x] = tot;
}

// part[0..m) -> exclusive prefix in place, part[m] = total
__global__ __launch_bounds__(256) void k_scan_parts(unsigned long long *part, uint64_t m) {
    __shared__ unsigned long long sh[4];
    unsigned long long carry = 0;
    for (uint64_t base = 0; base < m; base += 256) {
        const uint64_t i = base + threadIdx.x;
        const unsigned long long v = i < m ? part[i] : 0ULL;
        unsigned long long tot;
        const unsigned long long ex = block_exclusive_sum(v, sh, &tot);
        if (i < m) part[i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) part[m] = carry;
}

template <typename T>
__global__ __launch_bounds__(256) void k_scan_down(const T *in, uint64_t n, const unsigned long long *part,
                                                  unsigned long long *out) {
    __shared__ unsigned long long buf[kScanChunk + kScanChunk / 16];  // element j at j + j / 16
    __shared__ unsigned long long sh[4];
    const uint32_t tid = threadIdx.x;
    const uint64_t b = (uint64_t)blockIdx.x * kScanChunk;
    for (uint32_t j = tid; j < kScanChunk; j += 256) buf[j + (j >> 4)] = b + j < n ? (unsigned long long)in[b + j] : 0ULL;
    __syncthreads();
    unsigned long long *mine = buf + tid * 17;  // this thread's 16 consecutive elements
    unsigned long long s = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) s += mine[k];
    unsigned long long tot;
    unsigned long long run = part[blockIdx.x] + block_exclusive_sum(s, sh, &tot);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const unsigned long long v = mine[k];
        mine[k] = run;
        run += v;
    }
    __syncthreads();
    for (uint32_t j = tid; j < kScanChunk; j += 256)
        if (b + j < n) out[b + j] = buf[j + (j >> 4)];
    if (blockIdx.x == gridDim.x - 1 && tid == 0) out[n] = part[gridDim.x];
}

__global__ void k_scan_empty(unsigned long long *out) { out[0] = 0; }

__global__ __launch_bounds__(256) void k_tensor_sums(const TensorDesc *descs, const uint64_t *per_tile, uint64_t *out) {
    __shared__ unsigned long long sh[256];
    const TensorDesc td = descs[blockIdx.x];
    unsigned long long s = 0;
    for (uint32_t t = threadIdx.x; t < td.n_tiles; t += 256) s += per_tile[td.tile_begin + t];
    unsigned long long total;
    block_exclusive_sum(s, sh, &total);
    if (threadIdx.x == 0) out[blockIdx.x] = total;
}

// Full checksum of one tensor: each workgroup sums a contiguous range into partial[blockIdx.x].
__global__ __launch_bounds__(256) void k_checksum(const uint32_t *frame, uint32_t lead, uint64_t n, uint64_t *partial,
                                                  uint32_t n_parts) {
    __shared__ unsigned long long sh[256];
    const uint64_t words = (n + lead + 1) >> 1;
    const uint64_t per = (words + n_parts - 1) / n_parts;
    const uint64_t wb = (uint64_t)blockIdx.x * per, we = min(wb + per, words);
    // the range's words (at most 2^31 bytes: per <= max(65536, words / 2048) words)
    const Rsrc src = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(frame + min64(wb, words)), (short)0,
                                                       (int)(we > wb ? (we - wb) * 4u : 0u), 0x00020000);
    WeightedSum acc;
    // z = (index + 1) * golden of the thread's first element of word d, stepped with d
    uint64_t z = (uint64_t)(2 * (int64_t)(wb + threadIdx.x) - (int64_t)lead + 1) * kGolden;
    for (uint64_t d = wb + threadIdx.x; d < we; d += 256, z += 512 * kGolden) {
        const uint32_t o = __builtin_amdgcn_raw_buffer_load_b32(src, (uint32_t)(d - wb) * 4u, 0, 0);
        const int64_t i0 = (int64_t)(2 * d) - (int64_t)lead;
        const uint32_t u0 = i0 >= 0 ? o & 0xFFFF : 0u, u1 = i0 + 1 < (int64_t)n ? o >> 16 : 0u;
        acc.add(u0, mix_weight(z));
        acc.add(u1, mix_weight(z + kGolden));
    }
    unsigned long long total;
    block_exclusive_sum(acc.total(), sh, &total);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// One workgroup: *out = part[0] + ... + part[n - 1] (mod 2^64).
__global__ __launch_bounds__(256) void k_sum_parts(const unsigned long long *part, uint32_t n, unsigned long long *out) {
    __shared__ unsigned long long sh[4];
    unsigned long long s = 0;
    for (uint32_t i = threadIdx.x; i < n; i += 256) s += part[i];
    unsigned long long total;
    block_exclusive_sum(s, sh, &total);
    if (threadIdx.x == 0) *out = total;
}

// ================================================================== apply: block decode
// One lane per 256-change block (codec.py:504-575), 64 consecutive blocks per wavefront.  Each lane
// reads its block's payload bits from HBM (BitReader below); the decoding symbols and each table's
// symbol index of the first code of every length are staged in LDS when they fit.  A change normally
// costs one 64-bit window of the stream (unary run, remainder and Huffman peek together) and two LDS
// reads (its length's first index, then its symbol); code lengths come from comparisons of the 17-bit
// peek with the canonical limits held in registers (the first indices in registers as well took 17
// more registers and a select tree per change: 0.63 ms against 0.56 with them in LDS and 16 changes
// per store burst).  The decoder does not read the receiver's weights or counts (positions are
// checked against those by k_local_fix), so it can run beside the exponent-count pass.  Each lane
// keeps kDecBuf decoded changes in registers and stores them together: storing one change at a time
// left each lane's output lines half-written in L2, and they reached HBM several times over; 16 at a
// time (128 bytes) also spaces out the stores that the next payload load waits behind.
constexpr uint32_t kDecBuf = 16;         // changes decoded per lane between stores
// s_waitcnt operand (gfx9 encoding) that waits for every vector memory operation: vmcnt 0, expcnt and
// lgkmcnt at their maxima (no wait)
constexpr int kWaitVmem = 0x0F70;

// dst[0, n) = src[0, n) by one wavefront, 16 loads per lane in flight before any LDS write (a loop that
// loads one value and writes it before the next load costs one memory latency per 64 values)
__device__ __forceinline__ void stage_lds(uint32_t *dst, const uint32_t *src, uint32_t n) {
    constexpr uint32_t U = 16;
    const uint32_t ln = lane();
    for (uint32_t i0 = 0; i0 < n; i0 += 64 * U) {
        uint32_t v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            v[u] = src[min(i0 + u * 64 + ln, n - 1)];  // clamped, not branched: all U loads issue
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = i0 + u * 64 + ln;
            if (i < n) dst[i] = v[u];
        }
    }
}

// A lane's reader of its block's bits: the two 64-bit words around the read position in registers
// (hi, lo) and the next one already loading (nx), so each word's load has the decoding of the 64 bits
// before it (about six changes) to arrive.  Staging a wavefront's payload in LDS instead took up to
// 28 KiB per wavefront: a quarter of the wavefronts fit, each alone on its SIMD with nothing to hide
// its dependent chain.  Read positions only move forward.  The words are kept as loaded (byte-swapped
// only when read), so nothing consumes a load before the read that needs it: swapping or testing it at
// the load made every load wait at once.  Past the stream's last word the last word is read again:
// bits past a block's end never decide a valid change (a canonical code's length does not depend on
// the bits after it, and unary runs stop at the block's end).
struct BitReader {
    const uint64_t *p;
    uint64_t n, w;  // words in the stream; index of hi
    uint64_t hi, lo, nx;
    __device__ __forceinline__ uint64_t word(uint64_t i) const { return p[min64(i, n - 1)]; }
    __device__ __forceinline__ void start(const uint64_t *payload, uint64_t n_words, uint64_t pos) {
        p = payload;
        n = n_words;
        w = pos >> 6;
        hi = word(w);
        lo = word(w + 1);
        nx = word(w + 2);
    }
    // the 64 bits from bit pos, which is at or past the previous read's
    __device__ __forceinline__ uint64_t bits(uint64_t pos) {
        const uint64_t t = pos >> 6;
        if (t >= w + 3) {  // a long jump (a long unary run): start over there
            w = t;
            hi = word(t);
            lo = word(t + 1);
            nx = word(t + 2);
        } else {
            while (w < t) {
                hi = lo;
                lo = nx;
                nx = word(w + 3);
                ++w;
            }
        }
        const uint32_t s = (uint32_t)(pos & 63);
        const uint64_t h = __builtin_bswap64(hi), l = __builtin_bswap64(lo);
        return s ? (h << s) | (l >> (64 - s)) : h;
    }
};

template <bool LDS_SYMS>
__device__ void decode_blocks(const DecodeArgs &a, const uint32_t *S_syms) {
    const uint32_t ln = lane();
    const uint64_t b = (uint64_t)blockIdx.x * 64 + ln;
    if (b >= a.n_blocks) return;
    uint32_t lim[17];
    const uint32_t g = a.bmap[b];
    const GroupDev gr = a.groups[g];
    const uint64_t kb = b - gr.blk_base;
    const uint32_t cnt = (uint32_t)min64(256, gr.count - kb * 256);
    const uint64_t eb = (uint64_t)gr.elem_base + kb * 256;
    // the decoder does not need the receiver's exponent counts (k_local_fix checks positions against
    // them): unary runs are bounded by the tensor's size, which bounds any valid gap
    const uint64_t size = a.descs[gr.tensor].numel;
    const uint32_t rice = gr.rice;
    const uint64_t qmax = size >> rice;
    uint64_t cur = a.bit0 + a.block_off[b];
    const uint64_t end = cur + a.block_bits[b];
    bool bad = false;
    BitReader R;
    R.start(a.payload, a.n_words, cur);
#pragma unroll
    for (int l = 0; l < 17; ++l) {
        lim[l] = a.lim[(uint64_t)gr.table * 17 + l];
    }
    // every load above is complete before the first change: otherwise the compiler, which cannot tell
    // the first pass through the loop from the others, waits for these limits inside each change, and
    // with them for every payload load and store issued since (vmcnt counts both, in order)
    __builtin_amdgcn_s_waitcnt(kWaitVmem);
    uint64_t rel = 0;  // sum of (gap + 1) so far in this block
    // decodes change s of the block into out: zz | (block-relative local << 32); false once bad
    auto step = [&](uint32_t s, unsigned long long &out) {
        uint64_t x = R.bits(cur);
        uint64_t q;
        if (~x) {  // the unary run ends inside this window
            q = (uint64_t)__builtin_clzll(~x);
        } else {
            q = 64;
            for (;;) {
                if (q > qmax || cur + q >= end) break;
                const uint64_t y = ~R.bits(cur + q);
                if (y) {
                    q += (uint64_t)__builtin_clzll(y);
                    break;
                }
                q += 64;
            }
        }
        const uint64_t c = cur + q + 1;
        // remainder and Huffman peek: from the same window when they fit in it, else a new read
        if (q + 1 + rice + 17 <= 64) x <<= (q + 1);
        else x = R.bits(c);
        const uint64_t rem = rice ? x >> (64 - rice) : 0ULL;
        const uint32_t peek = (uint32_t)((x << rice) >> (64 - 17));
        // code length: 1 + #{l : lim[l] <= peek} (lim is non-decreasing), summed as a tree; then the
        // symbol index base off[L - 1] through a 5-level select tree (short dependency chains)
        uint32_t t[17];
#pragma unroll
        for (int l = 0; l < 17; ++l) t[l] = lim[l] <= peek ? 1u : 0u;
#pragma unroll
        for (int w = 1; w < 17; w <<= 1)
#pragma unroll
            for (int l = 0; l + w < 17; l += 2 * w) t[l] += t[l + w];
        const uint32_t L = 1 + t[0], li = min(L - 1, 16u);
        const uint32_t oi = gr.table * 17 + li;
        const uint32_t o0 = LDS_SYMS ? S_syms[a.n_syms + oi] : a.off[oi];
        const uint32_t idx = o0 + (L <= 17 ? peek >> (17 - L) : 0u);
        const uint64_t gap = (q << rice) | rem;
        if (q > qmax || cur + q >= end || L > 17 || gap >= size) {
            bad = true;  // positions past the group's exponent count are caught by k_local_fix
        } else {
            rel += gap + 1;
            const uint32_t si = min(idx, a.n_syms - 1);
            const uint32_t zz = LDS_SYMS ? S_syms[si] : a.syms[si];
            out = (unsigned long long)zz | ((unsigned long long)min64(rel - 1, 0xFFFFFFFFULL) << 32);
            cur = c + rice + L;
        }
    };
    // kDecBuf changes at a time, kept in registers and stored together: the block's output lines
    // are written in few bursts instead of one 8-byte piece per change
    unsigned long long *const dst = a.dz + eb;
    for (uint32_t s0 = 0; s0 < cnt && !bad; s0 += kDecBuf) {
        unsigned long long buf[kDecBuf];
#pragma unroll
        for (uint32_t j = 0; j < kDecBuf; ++j)
            if (s0 + j < cnt && !bad) step(s0 + j, buf[j]);
        if (bad) break;
        if (s0 + kDecBuf <= cnt) {
#pragma unroll
            for (uint32_t j = 0; j < kDecBuf; ++j) dst[s0 + j] = buf[j];
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kDecBuf; ++j)
                if (s0 + j < cnt) dst[s0 + j] = buf[j];
        }
    }
    if (!bad && cur != end) bad = true;
    a.blk_sum[b] = rel;
    if (bad) atomicOr(a.bad, kBadDecode);
}

template <bool LDS_SYMS>
__global__ __launch_bounds__(64) void k_decode(DecodeArgs a) {
    CRX_DYNAMIC_LDS(uint32_t, dyn_lds);  // the symbols, then the tables' first indices, when they fit
    if (LDS_SYMS) {
        stage_lds(dyn_lds, a.syms, a.n_syms);
        stage_lds(dyn_lds + a.n_syms, a.off, 17 * a.n_tables);
    }
    wave_fence();
    decode_blocks<LDS_SYMS>(a, dyn_lds);
}

// Change blocks handled by one workgroup of the per-block kernels (fewer, longer workgroups; their
// loads are issued together).
constexpr uint32_t kBlocksPerWG = 4;

// Block b's changes [eb, eb + cnt) and its group (cnt 0 past the last block).
__device__ __forceinline__ BlockInfo block_info(const BlockArgs &a, uint64_t b) {
    if (b < a.n_blocks) return a.binfo[b];
    return BlockInfo{0, 0, 0, 0, 0, 0, 0, 0};
}

// local = (sum of (gap + 1) over earlier blocks of the group) + block-relative local; must stay
// below the group size (codec.py:640-642,696-697).  Also the group-size check (codec.py:598-604).
__global__ __launch_bounds__(256) void k_local_fix(BlockArgs a) {
    const bool failed = *a.bad;  // read before this kernel's own flags
    const uint32_t s = threadIdx.x;
    BlockInfo r[kBlocksPerWG];
    unsigned long long base[kBlocksPerWG];
    uint64_t size[kBlocksPerWG];
    uint32_t raw[kBlocksPerWG];
#pragma unroll
    for (uint32_t u = 0; u < kBlocksPerWG; ++u) r[u] = block_info(a, (uint64_t)blockIdx.x * kBlocksPerWG + u);
#pragma unroll
    for (uint32_t u = 0; u < kBlocksPerWG; ++u) {
        const uint64_t b = (uint64_t)blockIdx.x * kBlocksPerWG + u;
        size[u] = 0;
        base[u] = 0;
        raw[u] = 0;
        if (r[u].cnt) {
            size[u] = a.sizes[r[u].key];
            base[u] = a.blk_prefix[b] - a.blk_prefix[r[u].blk_base];
            if (s < r[u].cnt) raw[u] = (uint32_t)(a.dz[(uint64_t)r[u].eb + s] >> 32);
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < kBlocksPerWG; ++u) {
        const uint64_t b = (uint64_t)blockIdx.x * kBlocksPerWG + u;
        // a group with more changes than the receiver has elements of its exponent (checked even
        // after a failed decode: the reference checks it first)
        if (r[u].cnt && b == r[u].blk_base && r[u].count > size[u] && threadIdx.x == 0)
            atomicOr(a.bad, a.descs[r[u].tensor].numel > a.group_check_numel ? kBadGroup : kBadLocal);
    }
    if (failed) return;
#pragma unroll
    for (uint32_t u = 0; u < kBlocksPerWG; ++u) {
        if (s < r[u].cnt) {
            const unsigned long long local = base[u] + raw[u];
            if (local >= size[u]) atomicOr(a.bad, kBadLocal);
            a.local[(uint64_t)r[u].eb + s] = (uint32_t)min64(local, 0xFFFFFFFFULL);
        }
    }
}

// For every (slab, exponent): the first change of the group whose local index is at or after the
// number of same-exponent elements before the slab.  Also lists the slab's exponent windows after
// its first one (the select pass streams the slab once per window): windows of kSelWin exponents,
// each starting at the lowest exponent with targets past the previous window.
// The searches are chains of dependent loads, so the pass is bound by how many are in flight: each
// wavefront takes kLocTiles slabs, packs the (slab, exponent) pairs that have a group into a list,
// and each lane runs kLocPer of the list's searches side by side (their loads issued together).  The
// LDS footprint stays small (6 KiB) so that many wavefronts are resident.
constexpr uint32_t kLocTiles = 4;  // slabs per wavefront
constexpr uint32_t kLocPer = 2;    // searches per lane in flight
__global__ __launch_bounds__(64) void k_locate(SelectArgs a, uint32_t tiles) {
    __shared__ uint32_t arg_g[kLocTiles * 256];          // the searches, packed: group
    __shared__ uint16_t arg_s[kLocTiles * 256];          // and slot = 256 u + exponent
    __shared__ unsigned long long hasw[kLocTiles * 4];   // per slab: bit k % 64 of word k / 64, exponent k has targets
    __shared__ uint32_t before[kLocTiles];               // per slab: its tensor's changes positioned before it
    __shared__ uint32_t last_of[kLocTiles];               // per slab: the last of its tensor
    const uint32_t ln = lane(), tau0 = blockIdx.x * kLocTiles;
    // nothing written through yet, whether or not the select pass runs (k_commit reads these)
    if (ln < kLocTiles && tau0 + ln < tiles) {
        a.done[tau0 + ln] = 0;
        a.multi[tau0 + ln] = 0;
    }
    if (*a.bad) {  // an update already rejected: no records; rstart defined all the same
        if (ln < kLocTiles && tau0 + ln < tiles) a.rstart[tau0 + ln] = 0;
        if (ln == 0 && blockIdx.x == 0) a.rstart[tiles] = 0;
        return;
    }
    // slab u of the wavefront, exponents ln + 64 q: those with a group are packed into consecutive
    // entries; the others have no first change (kNone).  All loads are issued before any is used.
    uint32_t tt[kLocTiles];
#pragma unroll
    for (uint32_t u = 0; u < kLocTiles; ++u) tt[u] = a.tile_tensor[min(tau0 + u, tiles - 1)];
    int32_t g[kLocTiles][4];
#pragma unroll
    for (uint32_t u = 0; u < kLocTiles; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) g[u][q] = a.group_of[(uint64_t)tt[u] * 256 + ln + 64 * q];
    if (ln < kLocTiles) {
        const TensorDesc &d = a.descs[a.tile_tensor[min(tau0 + ln, tiles - 1)]];
        before[ln] = 0;
        last_of[ln] = tau0 + ln + 1 >= d.tile_begin + d.n_tiles ? 1u : 0u;
    }
    if (ln < kLocTiles * 4) hasw[ln] = 0;
    uint32_t n_act = 0;
#pragma unroll
    for (uint32_t u = 0; u < kLocTiles; ++u) {
        const uint32_t tau = tau0 + u;
        if (tau >= tiles) break;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t k = ln + 64 * q;
            if (g[u][q] < 0) ((uint32_t *)a.lb)[(uint64_t)tau * 256 + k] = kNone;
            const uint64_t m = ballot(g[u][q] >= 0);
            if (g[u][q] >= 0) {
                arg_g[n_act + mbcnt(m)] = (uint32_t)g[u][q];
                arg_s[n_act + mbcnt(m)] = (uint16_t)(256 * u + k);
            }
            n_act += (uint32_t)__popcll(m);
        }
    }
    wave_fence();
    for (uint32_t i0 = 0; i0 < n_act; i0 += 64 * kLocPer) {
        uint32_t lo[kLocPer], hi[kLocPer], end[kLocPer], vhi[kLocPer], gb[kLocPer], tgt[kLocPer], nxt[kLocPer],
            slot[kLocPer];
        bool on[kLocPer];
        uint32_t gcnt[kLocPer], gblk[kLocPer];  // the group's changes and first block
#pragma unroll
        for (uint32_t p = 0; p < kLocPer; ++p) {  // the searches' bounds: every load issued before any use
            const uint32_t j = i0 + 64 * p + ln;
            on[p] = j < n_act;
            const uint32_t jj = on[p] ? j : n_act - 1;
            slot[p] = arg_s[jj];
            const uint32_t u = slot[p] >> 8, k = slot[p] & 255u, tau = tau0 + u;
            const GroupDev *grp = &a.groups[arg_g[jj]];
            gb[p] = grp->elem_base;
            gcnt[p] = grp->count;
            gblk[p] = grp->blk_base;
            tgt[p] = a.pre[(uint64_t)tau * 256 + k];
            // the count before the next slab (kNone for a tensor's last slab, whose row is read in its place)
            nxt[p] = a.pre[(uint64_t)(last_of[u] ? tau : tau + 1) * 256 + k];
        }
        // Each search is first narrowed to one block of 256 changes.  Block j of a group holds the local
        // indices [base_j, base_{j+1}), base_j = the decoder's block sums before it (blk_prefix), so the
        // target lies in the last block with base_j <= target, and the first change at or past the target
        // in that block: the block is estimated from the target's share of the group's range and checked
        // with two loads (the blocks are bisected when the estimate misses), then bisected itself.
        // (the group's local indices are below 2^32, so the block bases are taken mod 2^32)
        uint32_t p0[kLocPer], span[kLocPer], nb[kLocPer], jlo[kLocPer], jhi[kLocPer];
#pragma unroll
        for (uint32_t p = 0; p < kLocPer; ++p) {
            if (last_of[slot[p] >> 8]) nxt[p] = kNone;
            end[p] = gb[p] + gcnt[p];
            vhi[p] = kNone;
            nb[p] = (gcnt[p] + 255u) / 256u;
            p0[p] = (uint32_t)a.blk_prefix[gblk[p]];
            span[p] = (uint32_t)a.blk_prefix[gblk[p] + nb[p]];
        }
        uint32_t e0[kLocPer], e1[kLocPer];
#pragma unroll
        for (uint32_t p = 0; p < kLocPer; ++p) {
            span[p] -= p0[p];  // the group's range: its last change's local index + 1
            const bool in = on[p] && tgt[p] < span[p];
            const uint32_t je = in ? (uint32_t)min64((uint64_t)tgt[p] * nb[p] / span[p], nb[p] - 1) : 0u;
            jlo[p] = je;
            jhi[p] = in ? je + 1 : 0u;  // in: the block is in [jlo, jhi) once the estimate is checked
            e0[p] = (uint32_t)a.blk_prefix[gblk[p] + je];
            e1[p] = (uint32_t)a.blk_prefix[gblk[p] + je + 1];
        }
#pragma unroll
        for (uint32_t p = 0; p < kLocPer; ++p) {
            if (jhi[p]) {  // the estimate's block, or the side of it that holds the target
                if (tgt[p] < e0[p] - p0[p]) {
                    jhi[p] = jlo[p];
                    jlo[p] = 0;
                } else if (tgt[p] >= e1[p] - p0[p]) {
                    jlo[p] = jlo[p] + 1;
                    jhi[p] = nb[p];
                }
            }
        }
        for (;;) {  // the last block with base <= target, in [jlo, jhi) (base_jlo <= target)
            bool any = false;
#pragma unroll
            for (uint32_t p = 0; p < kLocPer; ++p) any |= jhi[p] - jlo[p] > 1;
            if (!__any(any)) break;
            uint32_t mid[kLocPer], v[kLocPer];
#pragma unroll
            for (uint32_t p = 0; p < kLocPer; ++p) {
                mid[p] = jlo[p] + ((jhi[p] - jlo[p]) >> 1);
                v[p] = (uint32_t)a.blk_prefix[gblk[p] + mid[p]];
            }
#pragma unroll
            for (uint32_t p = 0; p < kLocPer; ++p) {
                if (jhi[p] - jlo[p] > 1) {
                    if (v[p] - p0[p] <= tgt[p]) jlo[p] = mid[p];
                    else jhi[p] = mid[p];
                }
            }
        }
#pragma unroll
        for (uint32_t p = 0; p < kLocPer; ++p) {
            if (jhi[p]) {  // the block's changes
                lo[p] = gb[p] + 256u * jlo[p];
                hi[p] = min(lo[p] + 256u, end[p]);
            } else {  // no search, or every change of the group lies before the target
                lo[p] = hi[p] = end[p];
            }
        }
        for (;;) {  // lower bounds of tgt in local[lo, hi), kLocPer at a time
            bool any = false;
#pragma unroll
            for (uint32_t p = 0; p < kLocPer; ++p) any |= lo[p] < hi[p];
            if (!__any(any)) break;
            // some search is open, so the update has changes: every index below is one of them
            uint32_t mid[kLocPer], v[kLocPer];
#pragma unroll
            for (uint32_t p = 0; p < kLocPer; ++p) {
                mid[p] = lo[p] + ((hi[p] - lo[p]) >> 1);
                v[p] = a.local[min(mid[p], a.n_changes - 1)];
            }
#pragma unroll
            for (uint32_t p = 0; p < kLocPer; ++p) {
                const bool open = lo[p] < hi[p], below = v[p] < tgt[p];
                lo[p] = open && below ? mid[p] + 1 : lo[p];
                vhi[p] = open && !below ? v[p] : vhi[p];  // local[hi] once hi has moved
                hi[p] = open && !below ? mid[p] : hi[p];
            }
        }
#pragma unroll
        for (uint32_t p = 0; p < kLocPer; ++p) {
            if (on[p]) {
                const uint32_t u = slot[p] >> 8, k = slot[p] & 255u;
                ((uint32_t *)a.lb)[(uint64_t)(tau0 + u) * 256 + k] = lo[p];
                if (lo[p] < end[p] && (nxt[p] == kNone || vhi[p] < nxt[p]))
                    atomicOr(&hasw[4 * u + (k >> 6)], 1ULL << (k & 63));
                atomicAdd(&before[u], lo[p] - gb[p]);  // the group's changes before the slab
            }
        }
    }
    wave_fence();
    if (ln == 0) {
        for (uint32_t u = 0; u < kLocTiles; ++u) {
            const uint32_t tau = tau0 + u;
            if (tau >= tiles) break;
            // the slab's records follow those of the slabs before it: of earlier tensors, then of its own
            a.rstart[tau] = a.tchg[tt[u]] + before[u];
            if (tau + 1 == tiles) a.rstart[tiles] = a.tchg[a.n_tensors];
            const unsigned long long *w = &hasw[4 * u];  // windows greedy from the lowest exponent with targets
            auto first_at = [&](uint32_t from) -> uint32_t {  // lowest set bit at or past `from` (256: none)
                for (uint32_t q = from >> 6; q < 4; ++q) {
                    const uint64_t x = q == (from >> 6) ? w[q] & (~0ULL << (from & 63)) : w[q];
                    if (x) return 64 * q + (uint32_t)__builtin_ctzll(x);
                }
                return 256u;
            };
            uint32_t kb = first_at(0);
            while (kb < 256 - kSelWin) {
                kb = first_at(kb + kSelWin);
                if (kb < 256) {
                    a.more[atomicAdd(a.n_more, 1u)] = make_uint2(tau, kb);
                    a.multi[tau] = 1;
                }
            }
        }
    }
}

// ================================================================== apply: select pass
// One wavefront per slab.  The slab's targets (group-local indices of its changes, minus the
// exponent's count before the slab = ranks within the slab) are copied to LDS, per exponent in
// order.  The slab is streamed once per window of kWin consecutive exponents holding targets
// (normally one window covers them all).  Every element adds one to its exponent's running count
// (kSelCopies copies, by lane, so few lanes share an address); elements outside the window go to a
// spare counter no other lane uses.  Lane e owns window exponent e: it sums that exponent's copies
// and compares the total with the exponent's next target, so one ballot names the exponents with
// targets in the row.  For each of them, ballots and mbcnt give every element of that exponent its
// stable in-row rank, and the lane holding the element whose rank matches the target records it;
// then the lanes of all those exponents read their next targets together.  A row with more targets
// of one exponent publishes that exponent's elements in LDS by rank and takes the rest one per lane.
// A slab streamed in one window is then written through by its wave (write_through).
//
// Cost (7.6e9 weights, 1% changed, counters per 128-element row): 35 vector and 31 scalar
// instructions, 4.3 LDS instructions; LDS bank and address conflicts of the atomics stall about a
// third of the time each.  Fewer vector instructions alone (42 -> 35 per row with the split-halves
// layout) or fewer conflicts alone (8 copies) left the time unchanged: issue, LDS and latency are
// all near their limits, with the LDS footprint setting occupancy.
// targets per window held in LDS (a multiple of 1024; more are read from HBM): the smaller list keeps
// the footprint small (occupancy) for sparse updates, the larger one serves denser updates
constexpr uint32_t kTgtCapSparse = 1024, kTgtCapDense = 2048;
constexpr uint32_t kWin = kSelWin;           // exponents per window: one per lane
constexpr uint32_t kSelCopies = 4;            // copies of each running count (4 or 8)
constexpr uint32_t kSpare = 64 / kSelCopies;  // spare counters: lane l uses copy l % kSelCopies of spare l / kSelCopies
constexpr uint32_t kCntShift = kSelCopies == 4 ? 3 : 2;  // (window index << 7) >> kCntShift = counter byte offset
static_assert(kSelCopies == 4 || kSelCopies == 8, "kSelCopies");
static_assert(kTgtCapSparse % 1024 == 0 && kTgtCapDense % 1024 == 0, "target list capacity");

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 as16(uint32_t v) { return __builtin_bit_cast(u16x2, v); }

// sum of the copies of count c
__device__ __forceinline__ uint32_t sel_count(const uint32_t *cnt, uint32_t c) {
    uint32_t s = 0;
#pragma unroll
    for (uint32_t q = 0; q < kSelCopies; q += 4) {
        const uint4 v = *reinterpret_cast<const uint4 *>(&cnt[kSelCopies * c + q]);
        s += v.x + v.y + v.z + v.w;
    }
    return s;
}

template <uint32_t CAP>
struct SelectLds {
    uint32_t cnt[(kWin + kSpare) * kSelCopies];  // running counts, kSelCopies copies (by lane)
    alignas(16) uint16_t list[CAP];                // slab ranks of the window's targets, per exponent in order
    union {
        uint32_t slot[2 * kRow];  // streaming: in-row rank -> record high word; [kRow, 2 kRow): per lane
        uint4 info[64];           // set-up, per lane (its window exponent; zero past kWin): {list begin, list end, change index - list
                                  // index, exponent count before the slab}
    };
};

// Streams the slab's rows like stream_rows (U rows per batch, the next batch in flight), but lane l
// holds elements l and l + 64 of each row (two 16-bit loads into the halves of one register, as
// lo | hi << 16).  Within a row the 64 low elements then come before the 64 high ones, each half in
// lane order, so the rank of an element among the row's elements of one kind needs the ballot of its
// own half only.
template <int U, int CPOL, typename Body>
__device__ __forceinline__ void stream_halves(const Slab &sl, const Rsrc &src, Body &&body) {
    const uint32_t lb = lane() * 2u;
    u16x2 cur[U], nxt[U];
    auto load = [&](u16x2(&dst)[U], uint32_t base) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            dst[u].x = __builtin_amdgcn_raw_buffer_load_b16(src, base + u * 256u, 0, CPOL);
            dst[u].y = __builtin_amdgcn_raw_buffer_load_b16(src, base + u * 256u + 128u, 0, CPOL);
        }
    };
    load(cur, lb);
    for (uint32_t r0 = 0; r0 < sl.nrows; r0 += U) {
        load(nxt, (r0 + U) * 256u + lb);
#pragma unroll
        for (int u = 0; u < U; ++u) body(r0 + u, __builtin_bit_cast(uint32_t, cur[u]));
#pragma unroll
        for (int u = 0; u < U; ++u) cur[u] = nxt[u];
    }
}

template <uint32_t CAP, bool LDS_LIST, bool COLD>
__device__ __forceinline__ uint32_t select_slab(const SelectArgs &a, const TensorDesc &td, const Slab &sl, uint32_t kbase, SelectLds<CAP> &S,
                            uint32_t nxt, uint32_t ci, const uint32_t cend, const uint32_t jofs, const uint32_t pre_k,
                            uint32_t j, uint64_t &fsum) {
    // lane e, for window exponent e: nxt = slab rank of its next target (kFar: none left), ci = that
    // target's change index, cend = the end of its changes, jofs = change index - list index (LDS
    // list), pre_k = its count before the slab (HBM list).  j (uniform): the window's next record.
    // COLD: the stream also sums the slab's weights for the tensor's checksum (codec.py:61-68) into
    // fsum, as it reads them before any write (the verdict's input when no checksum is cached): the odd
    // rows when the histogram pass streamed the slab (it summed the even ones), else every row.
    const uint32_t ln = lane();
    // Per 16-bit half, an element's key is (window index << 7) + (its lane's copy << 5): the counter's
    // byte offset << kCntShift, so one shift gives the address.  Exponents below the window wrap past
    // the spare's key (the copy term is below 128), those above it are clamped to the spare's.
    const uint32_t rep = (ln & (kSelCopies - 1)) << (kCntShift + 2);
    const uint32_t kb = (((kbase << 7) - rep) & 0xFFFFu) * 0x10001u;
    const uint32_t sp = (((kWin + ln / kSelCopies) << 7) + rep) * 0x10001u;
    char *const cnt = reinterpret_cast<char *>(S.cnt);
    // slab rank of the target with change index c (below its exponent's end)
    auto target = [&](uint32_t c, uint32_t jo, uint32_t pr) -> uint32_t {
        if (LDS_LIST) return S.list[min(c - jo, CAP - 1)];
        return a.local[c] - pr;
    };
    // Found targets become records, stored in the order found (rows in order) from record j on: the
    // change index c and the element's high word h = offset in the slab | bits << 16.  (Staging them
    // in LDS for one coalesced store per 64 measured slower than these sequential single stores: select
    // 4.84 -> 5.14 ms at 1% changed, 7.45 -> 8.8 ms at 2%.)
    auto record = [&](uint32_t c, uint32_t h) -> unsigned long long {
        return (unsigned long long)c | ((unsigned long long)h << 32);
    };

    uint32_t prev = 0;  // exponent ln's count before the row
    WeightedSum cs;     // COLD: the checksum sum
    const bool odd = td.hist_in == nullptr;  // COLD: the histogram pass summed the even rows
    // COLD: z = (index + 1) * golden of this lane's low element in the current row (its high element: + 64)
    uint64_t z = COLD ? (uint64_t)(2 * (int64_t)sl.first - (int64_t)td.lead + ln + 1) * kGolden : 0;
    stream_halves<kSelectRows, kStreamNT>(sl, slab_rsrc(td.frame, sl), [&](uint32_t r, uint32_t o) {
        // both elements' keys; outside the window or the slab: the spare's
        u16x2 c = __builtin_elementwise_min(as16(o & 0x7F807F80u) - as16(kb), as16(sp));
        const uint32_t f = r * kRow + ln;  // the low element's offset; the high one's is f + 64
        uint32_t v = o;                    // COLD: the slab's own elements (zero outside it)
        if (!row_full(sl, r)) {
            if (f < sl.f_lo || f >= sl.f_hi) {
                c.x = as16(sp).x;
                v &= 0xFFFF0000u;
            }
            if (f + 64 < sl.f_lo || f + 64 >= sl.f_hi) {
                c.y = as16(sp).y;
                v &= 0xFFFFu;
            }
        }
        if (COLD) {  // the odd rows, or all of them when the histogram pass did not stream the slab
            if (!odd || (r & 1u)) {
                cs.add(v & 0xFFFF, mix_weight(z));
                cs.add(v >> 16, mix_weight(z + 64 * kGolden));
            }
            z += (uint64_t)kRow * kGolden;
        }
        const uint32_t key = __builtin_bit_cast(uint32_t, c);
        atomicAdd(reinterpret_cast<uint32_t *>(cnt + ((key & 0xFFFFu) >> kCntShift)), 1u);
        atomicAdd(reinterpret_cast<uint32_t *>(cnt + (key >> (16 + kCntShift))), 1u);
        wave_fence();  // the counts every lane added
        const uint32_t s = sel_count(S.cnt, ln);  // exponent ln's count up to the row's end
        const uint32_t seen = prev;
        prev = s;
        uint64_t H = ballot(s > nxt);
        if (!H) return;
        wave_fence();
        // window index << 7 of both elements (the copy term cleared)
        const uint32_t kx = key & 0xFF80FF80u, c0 = kx & 0xFFFFu, c1 = kx >> 16;
        // this lane's elements as records' high words: offset in the slab | bits << 16
        const uint32_t w0 = (f - sl.f_lo) | (o << 16), w1 = (f + 64 - sl.f_lo) | (o & 0xFFFF0000u);
        const uint32_t q = nxt - seen;  // in-row rank of the next target, for the exponents in H
        const bool hit = s > nxt;       // this lane's exponent is in H
        do {  // the next target of each exponent with targets in this row: exactly one element
            const uint32_t k = (uint32_t)__builtin_ctzll(H), kk = k << 7;
            const uint32_t qk = rdlane(q, k), ck = rdlane(ci, k);
            const bool m0 = c0 == kk;
            const uint64_t M0 = ballot(m0);
            const uint32_t n0 = (uint32_t)__popcll(M0);  // exponent k's low elements in the row
            if (qk < n0) {  // a low element: the one whose rank among them is qk
                if (m0 && mbcnt(M0) == qk) a.rec[j] = record(ck, w0);
            } else {        // a high element: rank qk - n0 among the high ones
                const bool m1 = c1 == kk;
                const uint64_t M1 = ballot(m1);  // by every lane: a wave-wide vote
                if (m1 && mbcnt(M1) == qk - n0) a.rec[j] = record(ck, w1);
            }
            ++j;
            clear_bit(H, k);
        } while (H);
        if (hit) {  // every exponent that had one: its next target, lane-parallel
            ++ci;
            nxt = ci < cend ? target(ci, jofs, pre_k) : (uint32_t)kFar;
        }
        H = ballot(s > nxt);
        if (!H) return;
        // more targets of an exponent in this row (rare at low densities): publish its elements by
        // in-row rank (other lanes write a slot of their own past the ranks) and take the rest one per
        // lane
        wave_fence();
        do {
            const uint32_t k = (uint32_t)__builtin_ctzll(H);
            const uint32_t after = rdlane(s, k), seen_k = rdlane(seen, k), ke = rdlane(cend, k);
            const uint32_t jo = LDS_LIST ? rdlane(jofs, k) : 0u, pr = LDS_LIST ? 0u : rdlane(pre_k, k);
            uint32_t ck = rdlane(ci, k);
            const bool m0 = c0 == (k << 7), m1 = c1 == (k << 7);
            const uint64_t M0 = ballot(m0);
            const uint32_t rr0 = mbcnt(M0), rr1 = (uint32_t)__popcll(M0) + mbcnt(ballot(m1));  // in-row ranks
            S.slot[m0 ? rr0 : kRow + ln] = w0;
            S.slot[m1 ? rr1 : kRow + ln] = w1;
            wave_fence();
            uint32_t n, tl;
            do {  // one target per lane (64 more if all lanes take one); the takers are lanes 0 .. n-1
                const uint32_t c = ck + ln;
                tl = c < ke ? target(c, jo, pr) : (uint32_t)kFar;
                const bool take = c < ke && tl < after;  // never past the exponent's own targets
                n = (uint32_t)__popcll(ballot(take));
                if (take) a.rec[j + ln] = record(c, S.slot[tl - seen_k]);
                j += n;
                ck += n;
            } while (n == 64);
            const uint32_t tc = rdlane(tl, n);  // the first target not taken, or kFar
            wave_fence();
            if (ln == k) {
                nxt = tc;
                ci = ck;
            }
            clear_bit(H, k);
        } while (H);
    });
    // every target of this window's exponents is found once its rank is passed: one still pending
    // lies past the slab's elements of its exponent (never so when the local indices were in range)
    if (ci < cend) atomicOr(a.bad, kBadUnplaced);
    if (COLD) fsum = wave_sum(cs.total());
    return j;  // past the window's last record
}

// The writes of a slab streamed in one window, by its select wave once the window's records [r0, r1)
// are stored (those of a window not fully placed are the ones found): new = (old + unzigzag(zz)) mod
// 2^16 (codec.py:698-700) over the receiver's bits, the slab's checksum delta, and the exponent counts
// of elements that move between binades.  The update is not verified yet: k_commit puts the old bits
// back (they are in the records) if it does not verify, so a failed apply leaves the weights as they
// were, as the reference's verify-then-write does (codec.py:703-707).  Writing here, while the other
// waves of the chip are still streaming, takes the partial-sector writes off a pass of their own.
constexpr uint32_t kWritePer = 2;  // records per lane with their loads in flight together (registers: occupancy)

__device__ void write_through(const SelectArgs &a, const TensorDesc &td, uint32_t tau, uint32_t lt, uint32_t r0,
                              uint32_t r1) {
    // this wave's record stores are complete, and its loads below see them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const uint32_t ln = lane();
    const uint64_t first = (uint64_t)lt * a.slab;  // tensor index of the slab's first element
    const uint32_t extent = (uint32_t)min64(a.slab, td.numel - first);  // offsets of found targets lie below
    uint16_t *const base = td.base + first;
    uint32_t *const h = td.hist_out ? td.hist_out + (uint64_t)lt * 256 : nullptr;
    unsigned long long d = 0;
    for (uint32_t b = r0; b < r1; b += 64 * kWritePer) {
        unsigned long long rc[kWritePer], z[kWritePer];
#pragma unroll
        for (uint32_t u = 0; u < kWritePer; ++u) {
            const uint32_t i = b + ln + 64 * u;
            rc[u] = i < r1 ? a.rec[i] : 0ULL;
        }
#pragma unroll
        for (uint32_t u = 0; u < kWritePer; ++u) {
            const uint32_t i = b + ln + 64 * u;
            z[u] = i < r1 && (uint32_t)rc[u] < a.n_changes ? a.dz[(uint32_t)rc[u]] : 0ULL;
        }
#pragma unroll
        for (uint32_t u = 0; u < kWritePer; ++u) {
            const uint32_t i = b + ln + 64 * u;
            if (i < r1) {
                if ((uint32_t)rc[u] >= a.n_changes) atomicOr(a.bad, kBadUnplaced);  // never for found targets
                const uint32_t zz = (uint32_t)z[u];
                const uint32_t off = (uint32_t)(rc[u] >> 32) & 0xFFFFu, old = (uint32_t)(rc[u] >> 48);
                const int32_t delta = (int32_t)(zz >> 1) ^ -(int32_t)(zz & 1);
                const uint32_t nu = (uint32_t)((int32_t)old + delta) & 0xFFFF;
                if (off < extent) base[off] = (uint16_t)nu;
                d += (uint64_t)((int64_t)nu - (int64_t)old) * weight(first + off);
                const uint32_t eo = (old >> 7) & 0xFF, en = (nu >> 7) & 0xFF;
                if (eo != en && h) {  // the element moves between exponent counts of its slab
                    atomicSub(&h[eo], 1u);
                    atomicAdd(&h[en], 1u);
                }
            }
        }
    }
    d = wave_sum(d);
    if (ln == 0) {
        a.sdelta[tau] = d;
        a.done[tau] = r1 - r0;
    }
}

// One window of one slab: exponents [kfirst, kfirst + kWin), or from the slab's lowest exponent with
// targets when kfirst is 256.  The slab's targets are the group changes [lb(slab), lb(next slab)) of
// each exponent (to the group's end for a tensor's last slab).  ANYCOLD: some tensor of the update has
// no cached checksum (otherwise the checksum summing is left out of the kernel's code).
template <uint32_t CAP, bool ANYCOLD>
__device__ __forceinline__ void select_window(const SelectArgs &a, uint32_t tau, uint32_t kfirst, SelectLds<CAP> &S) {
    const uint32_t ln = lane();
    const uint32_t t = a.tile_tensor[tau];
    const TensorDesc td = a.descs[t];
    int32_t g4[4];
    uint32_t j0[4], j1[4], pr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // exponents 4 ln + q; independent loads, issued together
        const uint32_t k = 4 * ln + q;
        g4[q] = a.group_of[(uint64_t)t * 256 + k];
        j0[q] = a.lb[(uint64_t)tau * 256 + k];
        j1[q] = a.lb[(uint64_t)(tau + 1) * 256 + k];
        pr[q] = a.pre[(uint64_t)tau * 256 + k];
    }
    const uint32_t local_tile = tau - td.tile_begin;
    const bool last = local_tile + 1 >= td.n_tiles;
    uint32_t n4[4], klo = 256;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        n4[q] = 0;
        if (g4[q] >= 0) {
            uint32_t je = j1[q];
            if (last) {
                const GroupDev gr = a.groups[g4[q]];
                je = gr.elem_base + gr.count;
            }
            if (j0[q] < je) n4[q] = je - j0[q];
        }
        if (n4[q]) klo = min(klo, 4 * ln + q);
    }
    for (int o = 32; o > 0; o >>= 1) klo = min(klo, (uint32_t)__shfl_xor(klo, o, 64));
    const uint32_t kbase = kfirst < 256 ? kfirst : klo;
    if (kbase >= 256) {  // no targets in this slab: nothing to write, a checksum delta of zero
        if (kfirst == 256) {
            const bool cold = ANYCOLD && td.cold;
            const uint64_t f = cold ? cold_sum(td, slab_of(td, local_tile, a.slab), !td.hist_in) : 0;
            if (ln == 0) {
                a.sdelta[tau] = 0;
                a.full[tau] = f + (cold && !td.hist_in ? a.full[tau] : 0);
            }
        }
        return;
    }
    // the window's records follow the slab's records of lower exponents (other windows)
    uint32_t below = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) below += 4 * ln + q < kbase ? n4[q] : 0u;
    for (int o = 32; o > 0; o >>= 1) below += (uint32_t)__shfl_xor(below, o, 64);
    const uint32_t jbase = a.rstart[tau] + below;
    const Slab sl = slab_of(td, local_tile, a.slab);
    {
        uint32_t nw[4], mine = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            nw[q] = 4 * ln + q - kbase < kWin ? n4[q] : 0u;
            mine += nw[q];
        }
        uint32_t incl = mine;  // inclusive scan of per-lane totals across the wave
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t v = __shfl_up(incl, o, 64);
            if (ln >= (uint32_t)o) incl += v;
        }
        const uint32_t total = __shfl(incl, 63, 64);
        const bool in_lds = total <= CAP;
        S.info[ln] = make_uint4(0u, 0u, 0u, 0u);  // window exponents past 255
        wave_fence();
        uint32_t start[4], off = incl - mine;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t c = 4 * ln + q - kbase;
            start[q] = off;
            if (c < kWin) S.info[c] = make_uint4(off, off + nw[q], j0[q] - off, pr[q]);
            off += nw[q];
        }
        wave_fence();
        if (in_lds) {
            // list entry x belongs to the last exponent whose list starts at or before x: mark the starts
            // of the non-empty lists, then a running maximum over the entries, 1024 at a time (16 per
            // lane, in order)
            uint16_t *mark = S.list;  // each round reads its marks before its list entries overwrite them
            for (uint32_t x = ln; x < CAP; x += 64) mark[x] = 0;
            wave_fence();
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (nw[q]) mark[start[q]] = (uint16_t)(4 * ln + q - kbase + 1);
            wave_fence();
            uint32_t carry = 0;  // the maximum over earlier rounds
            for (uint32_t x0 = 0; x0 < total; x0 += 1024) {
                uint32_t v[16], run = 0;
#pragma unroll
                for (int i = 0; i < 16; i += 8) {
                    const uint4 m = *reinterpret_cast<const uint4 *>(&mark[x0 + 16 * ln + i]);
                    const uint32_t w4[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        v[i + 2 * h] = run = max(run, w4[h] & 0xFFFF);
                        v[i + 2 * h + 1] = run = max(run, w4[h] >> 16);
                    }
                }
                uint32_t incl = run;  // inclusive max-scan of the lane maxima
                for (int o = 1; o < 64; o <<= 1) {
                    const uint32_t w = __shfl_up(incl, o, 64);
                    if (ln >= (uint32_t)o) incl = max(incl, w);
                }
                uint32_t before = __shfl_up(incl, 1, 64);
                before = max(ln == 0 ? 0u : before, carry);
                carry = max(carry, (uint32_t)__shfl(incl, 63, 64));
                uint32_t idx[16], sub[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t c = max(before, v[i]);
                    const uint4 inf = S.info[c ? c - 1 : 0];
                    idx[i] = inf.z + x0 + 16 * ln + i;
                    sub[i] = inf.w;
                }
                wave_fence();
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t x = x0 + 16 * ln + i;
                    if (x < total) S.list[x] = (uint16_t)(a.local[idx[i]] - sub[i]);
                }
                wave_fence();
            }
        }
        wave_fence();
        const uint4 inf = S.info[ln];  // lane ln: window exponent ln
        uint32_t first = (uint32_t)kFar;
        if (inf.x < inf.y) first = in_lds ? S.list[inf.x] : a.local[inf.z + inf.x] - inf.w;
        wave_fence();
        for (uint32_t i = ln; i < (kWin + kSpare) * kSelCopies; i += 64) S.cnt[i] = 0;
        wave_fence();
        const uint32_t c_first = inf.x + inf.z, c_end = inf.y + inf.z;  // change indices
        const uint32_t j = __builtin_amdgcn_readfirstlane(jbase);  // uniform: kept in a scalar register
        // a slab's first window sums its weights for a cold tensor's checksum
        const bool cold = ANYCOLD && kfirst == 256 && td.cold;
        uint64_t fsum = 0;
        uint32_t jend;
        if (in_lds)
            jend = cold ? select_slab<CAP, true, ANYCOLD>(a, td, sl, kbase, S, first, c_first, c_end, inf.z, inf.w, j, fsum)
                        : select_slab<CAP, true, false>(a, td, sl, kbase, S, first, c_first, c_end, inf.z, inf.w, j, fsum);
        else
            jend = cold ? select_slab<CAP, false, ANYCOLD>(a, td, sl, kbase, S, first, c_first, c_end, inf.z, inf.w, j, fsum)
                        : select_slab<CAP, false, false>(a, td, sl, kbase, S, first, c_first, c_end, inf.z, inf.w, j, fsum);
        if (kfirst == 256 && ln == 0) a.full[tau] = fsum + (cold && !td.hist_in ? a.full[tau] : 0);
        // a slab streamed once (its first window is its only one) is written now
        if (kfirst == 256 && !a.multi[tau]) write_through(a, td, tau, local_tile, j, jend);
    }
}

// Blocks [0, n_front): the first n_front windows k_locate listed (started first, so they overlap
// the rest); then one block per slab for its first window.  ANYCOLD as for select_window.
template <uint32_t CAP, bool ANYCOLD>
__global__ __launch_bounds__(64) void k_select(SelectArgs a) {
    __shared__ __attribute__((aligned(16))) SelectLds<CAP> S;
    const uint32_t b = blockIdx.x;
    if (*a.bad) {  // positions will not be used; a cold slab's checksum still feeds the verdict
        if (b >= a.n_front) {
            const uint32_t tau = b - a.n_front;
            const TensorDesc td = a.descs[a.tile_tensor[tau]];
            const bool cold = ANYCOLD && td.cold;
            const uint64_t f = cold ? cold_sum(td, slab_of(td, tau - td.tile_begin, a.slab), !td.hist_in) : 0;
            if (lane() == 0) a.full[tau] = f + (cold && !td.hist_in ? a.full[tau] : 0);
        }
        return;
    }
    if (b < a.n_front) {
        if (b >= *a.n_more) return;
        const uint2 m = a.more[b];
        select_window<CAP, ANYCOLD>(a, m.x, m.y, S);
    } else {
        select_window<CAP, ANYCOLD>(a, b - a.n_front, 256u, S);
    }
}

// Listed windows past the first n_front (normally none); a fixed grid walks them.
template <uint32_t CAP>
__global__ __launch_bounds__(64) void k_select_more(SelectArgs a) {
    __shared__ __attribute__((aligned(16))) SelectLds<CAP> S;
    if (*a.bad) return;
    const uint32_t n = *a.n_more;
    for (uint32_t i = a.n_front + blockIdx.x; i < n; i += gridDim.x) {
        const uint2 m = a.more[i];
        select_window<CAP, false>(a, m.x, m.y, S);  // windows after a slab's first: no checksum
        wave_fence();
    }
}

// new = (old + unzigzag(zz)) mod 2^16 and the checksum delta (codec.py:698-700), slab by slab over the
// select pass's records; the exponent counts of elements that move between binades are updated.
constexpr uint32_t kVerifyPer = 4;  // records per thread with their loads in flight together

__global__ __launch_bounds__(256) void k_verify(SlabArgs a) {
    __shared__ unsigned long long sh[4];
    const uint32_t tau = blockIdx.x, tid = threadIdx.x;
    if (*a.bad) {  // positions were not all computed: deltas of zero, so the verdict is deterministic
        if (tid == 0) a.sdelta[tau] = 0;
        return;
    }
    if (!a.multi[tau]) return;  // streamed in one window: the select pass wrote its delta
    const uint32_t r0 = a.rstart[tau], r1 = a.rstart[tau + 1];
    const TensorDesc td = a.descs[a.tile_tensor[tau]];
    const uint32_t lt = tau - td.tile_begin;
    const uint32_t first = lt * a.slab;  // tensor index of the slab's first element
    uint32_t *const h = td.hist_out ? td.hist_out + (uint64_t)lt * 256 : nullptr;
    unsigned long long d = 0;
    for (uint32_t b = r0; b < r1; b += 256 * kVerifyPer) {
        unsigned long long rc[kVerifyPer], z[kVerifyPer];
#pragma unroll
        for (uint32_t u = 0; u < kVerifyPer; ++u) {
            const uint32_t i = b + tid + 256 * u;
            rc[u] = i < r1 ? a.rec[i] : 0ULL;
        }
#pragma unroll
        for (uint32_t u = 0; u < kVerifyPer; ++u) {
            const uint32_t i = b + tid + 256 * u;
            z[u] = i < r1 && (uint32_t)rc[u] < a.n_changes ? a.dz[(uint32_t)rc[u]] : 0ULL;
        }
#pragma unroll
        for (uint32_t u = 0; u < kVerifyPer; ++u) {
            const uint32_t i = b + tid + 256 * u;
            if (i < r1) {
                if ((uint32_t)rc[u] >= a.n_changes) atomicOr(a.bad, kBadUnplaced);  // never for found targets
                const uint32_t zz = (uint32_t)z[u];
                const uint32_t off = (uint32_t)(rc[u] >> 32) & 0xFFFFu, old = (uint32_t)(rc[u] >> 48);
                const int32_t delta = (int32_t)(zz >> 1) ^ -(int32_t)(zz & 1);
                const uint32_t nu = (uint32_t)((int32_t)old + delta) & 0xFFFF;
                d += (uint64_t)((int64_t)nu - (int64_t)old) * weight(first + off);
                a.pn[i] = off | (nu << 16);
                const uint32_t eo = (old >> 7) & 0xFF, en = (nu >> 7) & 0xFF;
                if (eo != en && h) {  // the element moves between exponent counts of its slab
                    atomicSub(&h[eo], 1u);
                    atomicAdd(&h[en], 1u);
                }
            }
        }
    }
    unsigned long long total;
    block_exclusive_sum(d, sh, &total);
    if (tid == 0) a.sdelta[tau] = total;
}

// The host's verdict (codec.py:598-604,696-712), computed on the device as well so that the scatter
// can follow it without a host round trip; the host still raises the errors from the same data.
__global__ __launch_bounds__(256) void k_verdict(uint32_t n, const unsigned long long *delta, const uint64_t *full,
                                                 const int32_t *has, const uint64_t *cached, const uint64_t *want,
                                                 const unsigned int *bad, unsigned int *ok) {
    __shared__ unsigned int miss;
    if (threadIdx.x == 0) miss = 0;
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < n; t += 256) {
        const uint64_t old = has[t] ? cached[t] : full[t];
        if (old + delta[t] != want[t]) atomicOr(&miss, 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) *ok = (miss == 0 && *bad == 0) ? 1u : 0u;
}

// After the device's verdict, one workgroup per slab.  A slab with more than one window: its writes,
// if the update verifies (its records are in row order per window, so the stores of a wavefront go to
// ascending addresses).  A slab the select pass wrote through: if the update does not verify, its old
// bits back from the records, so that the weights are as they were.
__global__ __launch_bounds__(256) void k_commit(SlabArgs a, uint32_t tiles) {
    const bool ok = *a.ok != 0;
    for (uint32_t tau = blockIdx.x; tau < tiles; tau += gridDim.x) {
        const bool multi = a.multi[tau] != 0;
        if (multi != ok) continue;  // verified and written through, or not verified and never written
        // done is zero unless the select pass wrote the slab (k_locate clears it first): nothing to undo,
        // and rstart is not read (k_locate does not locate the records of an update already rejected)
        const uint32_t done = multi ? 1u : a.done[tau];
        if (!done) continue;
        // the records [r0, r0 + n), within the record buffer whatever rstart holds; counted from 0 so
        // that no index wraps
        const uint32_t r0 = min(a.rstart[tau], a.n_changes);
        const uint32_t n = min(multi ? a.rstart[tau + 1] - r0 : done, a.n_changes - r0);
        const TensorDesc td = a.descs[a.tile_tensor[tau]];
        const uint64_t first = (uint64_t)(tau - td.tile_begin) * a.slab;
        const uint32_t extent = (uint32_t)min64(a.slab, td.numel - first);  // offsets of found targets lie below
        uint16_t *const base = td.base + first;
        if (multi) {
            for (uint32_t k = threadIdx.x; k < n; k += 256) {
                const uint32_t v = a.pn[r0 + k];
                if ((v & 0xFFFFu) < extent) base[v & 0xFFFFu] = (uint16_t)(v >> 16);
            }
        } else {
            for (uint32_t k = threadIdx.x; k < n; k += 256) {
                const unsigned long long rc = a.rec[r0 + k];
                const uint32_t off = (uint32_t)(rc >> 32) & 0xFFFFu;
                if (off < extent) base[off] = (uint16_t)(rc >> 48);
            }
        }
    }
}

inline uint32_t grid1(uint64_t n, uint32_t per) { return (uint32_t)((n + per - 1) / per); }

}  // namespace

// ================================================================== launchers
#define CRX_LAUNCH(name, kernel, grid, block, stream, ...)                                   \
    do {                                                                                     \
        if ((grid) > 0) {                                                                    \
            timing_begin(name, stream);                                                      \
            hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, stream, __VA_ARGS__);     \
            timing_end(name, stream);                                                        \
        }                                                                                    \
    } while (0)

void launch_enc_rank(const EncRankArgs &a, uint32_t tiles, hipStream_t s) {
    CRX_LAUNCH("enc_rank", k_enc_rank, tiles, 64, s, a);
}
void launch_hist(const HistArgs &a, uint32_t n, hipStream_t s) { CRX_LAUNCH("apply_hist", k_hist, n, 64, s, a); }

void launch_scan_tables(const TensorDesc *descs, const ScanTabs &p, uint32_t n_tabs, const ScanChunk *chunks,
                        uint32_t n_chunks, const uint32_t *tensor_chunk_begin, uint32_t n_tensors, hipStream_t s) {
    CRX_LAUNCH("scan_sum", k_scan_sum, n_tabs * n_chunks, 256, s, descs, p, chunks, n_chunks);
    CRX_LAUNCH("scan_mid", k_scan_mid, n_tabs * n_tensors, 256, s, p, tensor_chunk_begin, n_tensors);
    CRX_LAUNCH("scan_fin", k_scan_fin, n_tabs * n_chunks, 256, s, descs, p, chunks, n_chunks);
}

void launch_enc_groups(const uint32_t *totals_chg, uint32_t n_tensors, GroupDev *groups, uint32_t *gbase,
                       unsigned long long *counters, hipStream_t s) {
    CRX_LAUNCH("enc_groups", k_enc_groups, grid1((uint64_t)n_tensors * 256, kGroupChunk), 256, s, totals_chg, n_tensors,
               groups, gbase, counters);
}

void launch_place(const EncRankArgs &a, uint32_t tiles, const uint32_t *tile_tensor, const uint32_t *hall_pre,
                  const uint32_t *hchg_pre, const uint32_t *gbase, uint64_t *sorted, uint64_t n_sorted, hipStream_t s) {
    CRX_LAUNCH("place", k_place, tiles, 64, s, a, tile_tensor, hall_pre, hchg_pre, gbase, sorted, n_sorted);
}

void launch_tile_map(const TensorDesc *descs, uint32_t n_tensors, uint32_t *tile_tensor, hipStream_t s) {
    CRX_LAUNCH("tile_map", k_tile_map, n_tensors, 256, s, descs, tile_tensor);
}

void launch_r0(GroupDev *groups, uint32_t n_groups, const uint64_t *sorted, hipStream_t s) {
    CRX_LAUNCH("rice_r0", k_r0, grid1(n_groups, 256), 256, s, groups, n_groups, sorted);
}

void launch_stats(const StatsArgs &a, hipStream_t s) { CRX_LAUNCH("stats", k_stats, grid1(a.n, kElemsPerWG), 256, s, a); }

void launch_chunk_map(const GroupDev *groups, uint32_t n_groups, uint32_t *cmap, hipStream_t s) {
    CRX_LAUNCH("chunk_map", k_chunk_map, n_groups, 256, s, groups, cmap);
}

void launch_block_map(const GroupDev *groups, uint32_t n_groups, uint32_t *bmap, BlockInfo *binfo, hipStream_t s) {
    CRX_LAUNCH("block_map", k_block_map, n_groups, 256, s, groups, bmap, binfo);
}

void launch_code_lengths(const CodeArgs &a, hipStream_t s) {
    CRX_LAUNCH("code_lengths", k_code_lengths, grid1(a.n, kElemsPerWG), 256, s, a);
}

void launch_pack(const CodeArgs &a, hipStream_t s) { CRX_LAUNCH("pack", k_pack, grid1(a.n, kElemsPerWG), 256, s, a); }

void launch_block_bits(const unsigned long long *bstart, uint64_t n_blocks, uint32_t *out, unsigned int *overflow,
                       hipStream_t s) {
    CRX_LAUNCH("block_bits", k_block_bits, grid1(n_blocks, 256), 256, s, bstart, n_blocks, out, overflow);
}

uint64_t scan_parts(uint64_t n) { return (n + kScanChunk - 1) / kScanChunk + 1; }

template <typename T>
static void launch_scan(const char *name, const T *in, uint64_t n, unsigned long long *out, unsigned long long *part,
                        hipStream_t s) {
    if (!n) {
        CRX_LAUNCH(name, k_scan_empty, 1, 1, s, out);
        return;
    }
    const uint64_t m = (n + kScanChunk - 1) / kScanChunk;
    CRX_LAUNCH(name, k_scan_reduce<T>, (uint32_t)m, 256, s, in, n, part);
    CRX_LAUNCH(name, k_scan_parts, 1, 256, s, part, m);
    CRX_LAUNCH(name, k_scan_down<T>, (uint32_t)m, 256, s, in, n, part, out);
}

void launch_scan_u64(const unsigned long long *in, uint64_t n, unsigned long long *out, unsigned long long *part,
                     hipStream_t s) {
    launch_scan("scan_u64", in, n, out, part, s);
}

void launch_scan_u32(const uint32_t *in, uint64_t n, unsigned long long *out, unsigned long long *part, hipStream_t s) {
    launch_scan("scan_u32", in, n, out, part, s);
}

void launch_verdict(uint32_t n, const unsigned long long *delta, const uint64_t *full, const int32_t *has,
                    const uint64_t *cached, const uint64_t *want, const unsigned int *bad, unsigned int *ok,
                    hipStream_t s) {
    timing_begin("verdict", s);
    hipLaunchKernelGGL(k_verdict, dim3(1), dim3(256), 0, s, n, delta, full, has, cached, want, bad, ok);
    timing_end("verdict", s);
}

void launch_tensor_sums(const TensorDesc *descs, uint32_t n_tensors, const uint64_t *per_tile, uint64_t *out,
                        hipStream_t s) {
    CRX_LAUNCH("tensor_sums", k_tensor_sums, n_tensors, 256, s, descs, per_tile, out);
}

void launch_decode(const DecodeArgs &a, hipStream_t s) {
    const uint32_t grid = grid1(a.n_blocks, 64), lds = decode_lds_bytes(a.n_syms, a.n_tables);
    if (!grid) return;
    timing_begin("decode", s);
    if (a.n_syms <= kDecSyms) hipLaunchKernelGGL(k_decode<true>, dim3(grid), dim3(64), lds, s, a);
    else hipLaunchKernelGGL(k_decode<false>, dim3(grid), dim3(64), lds, s, a);
    timing_end("decode", s);
}

void launch_local_fix(const BlockArgs &a, uint64_t n_blocks, hipStream_t s) {
    CRX_LAUNCH("local_fix", k_local_fix, grid1(n_blocks, kBlocksPerWG), 256, s, a);
}

void launch_locate(const SelectArgs &a, uint32_t tiles, hipStream_t s) {
    CRX_LAUNCH("locate", k_locate, grid1(tiles, kLocTiles), 64, s, a, tiles);
}

void launch_select(const SelectArgs &a, uint32_t tiles, bool dense, bool any_cold, hipStream_t s) {
    if (dense) {
        if (any_cold) CRX_LAUNCH("select", (k_select<kTgtCapDense, true>), a.n_front + tiles, 64, s, a);
        else CRX_LAUNCH("select", (k_select<kTgtCapDense, false>), a.n_front + tiles, 64, s, a);
        CRX_LAUNCH("select_more", k_select_more<kTgtCapDense>, 256, 64, s, a);
    } else {
        if (any_cold) CRX_LAUNCH("select", (k_select<kTgtCapSparse, true>), a.n_front + tiles, 64, s, a);
        else CRX_LAUNCH("select", (k_select<kTgtCapSparse, false>), a.n_front + tiles, 64, s, a);
        CRX_LAUNCH("select_more", k_select_more<kTgtCapSparse>, 256, 64, s, a);
    }
}

void launch_verify(const SlabArgs &a, uint32_t tiles, hipStream_t s) { CRX_LAUNCH("verify", k_verify, tiles, 256, s, a); }

void launch_commit(const SlabArgs &a, uint32_t tiles, hipStream_t s) {
    CRX_LAUNCH("commit", k_commit, std::min<uint32_t>(tiles, 2048), 256, s, a, tiles);  // slabs strided over the grid
}

void launch_checksum(const uint32_t *frame, uint32_t lead, uint64_t n, uint64_t *partial, uint32_t n_parts,
                     hipStream_t s) {
    CRX_LAUNCH("checksum", k_checksum, n_parts, 256, s, frame, lead, n, partial, n_parts);
}

// ================================================================== allocation-free checksum
// The scratch memory of checksum_noalloc: k_checksum's partial sums and their total, in a static
// device array (each device holds its own copy until the process ends) instead of memory from the
// caller's allocator.  Every call overwrites what it reads, so nothing needs clearing between calls;
// calls that overlap on one device share the array and race.
constexpr uint32_t kNoAllocParts = 2048;
static __device__ __align__(256) unsigned long long scratch[kNoAllocParts + 1];

// The array's device address on the current device, looked up once per device with that device
// current.  In host code `scratch` names a host-side stand-in, not device memory: kernels and copies
// are given this address instead.
static hipError_t scratch_address(unsigned long long **out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static unsigned long long *addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = static_cast<unsigned long long *>(p);
    }
    *out = addr[dev];
    return hipSuccess;
}

hipError_t checksum_noalloc(const uint32_t *frame, uint32_t lead, uint64_t n, hipStream_t s, uint64_t *out) {
    unsigned long long *sc = nullptr;
    hipError_t e = scratch_address(&sc);
    if (e != hipSuccess) return e;
    const uint64_t words = (n + lead + 1) >> 1;
    const uint32_t parts = (uint32_t)std::min<uint64_t>(kNoAllocParts, (words + 65535) / 65536);
    hipLaunchKernelGGL(k_checksum, dim3(parts), dim3(256), 0, s, frame, lead, n, reinterpret_cast<uint64_t *>(sc),
                       parts);
    hipLaunchKernelGGL(k_sum_parts, dim3(1), dim3(256), 0, s, sc, parts, sc + kNoAllocParts);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(out, sc + kNoAllocParts, sizeof(uint64_t), hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return e;
    return hipStreamSynchronize(s);
}

}  // namespace crx
