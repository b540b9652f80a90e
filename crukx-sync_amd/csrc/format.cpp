// Host-side format code: parser, varints, Huffman lengths, canonical codes, Rice choice.
#include "format.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <string_view>
#include <unordered_set>

namespace crx {

namespace {

// Sequential reader over a prefix of the update (wire.py:92-123): every overrun of the whole
// update is Corrupt ("truncated"); an overrun of the available prefix only asks for more bytes.
struct Reader {
    const uint8_t *d;
    uint64_t avail, total, pos = 0;

    uint64_t remaining() const { return total - pos; }

    const uint8_t *take(uint64_t n) {
        if (n > total - pos) throw Corrupt("update is truncated");
        if (n > avail - std::min(avail, pos)) throw NeedMore{pos + n};
        const uint8_t *p = d + pos;
        pos += n;
        return p;
    }
    void skip(uint64_t n) {  // payload: length-checked, not read
        if (n > total - pos) throw Corrupt("update is truncated");
        pos += n;
    }
    int u8() { return take(1)[0]; }
    uint64_t varint() {
        const uint64_t lim = std::min(avail, total);
        if (pos + 1 < lim) {  // one- and two-byte values, the common case
            const uint64_t b0 = d[pos], b1 = d[pos + 1];
            if (!(b0 & 0x80)) {
                pos += 1;
                return b0;
            }
            if (!(b1 & 0x80)) {
                pos += 2;
                return (b0 & 0x7F) | (b1 << 7);
            }
        }
        uint64_t v = 0;
        int shift = 0;
        for (;;) {
            uint64_t b = (uint64_t)u8();
            uint64_t bits = b & 0x7F;
            if (bits) {
                if (shift >= 63 || (bits << shift) >> shift != bits || ((v | (bits << shift)) >> 63))
                    throw Corrupt("varint out of range");
                v |= bits << shift;
            }
            if (!(b & 0x80)) return v;
            shift += 7;
            if (shift > 63) throw Corrupt("varint too long");
        }
    }
};

// Strict UTF-8 as Python's bytes.decode("utf-8"): no overlongs, surrogates or code points past
// U+10FFFF.
bool valid_utf8(const uint8_t *s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint32_t cp, lo;
        if (c >= 0xC2 && c <= 0xDF) { len = 2; cp = c & 0x1F; lo = 0x80; }
        else if (c >= 0xE0 && c <= 0xEF) { len = 3; cp = c & 0x0F; lo = 0x800; }
        else if (c >= 0xF0 && c <= 0xF4) { len = 4; cp = c & 0x07; lo = 0x10000; }
        else return false;
        if (n - i < (uint64_t)len) return false;
        for (int k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if (cp < lo || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += (uint64_t)len;
    }
    return true;
}

// The sum of n little-endian u32 (block table entries), and whether any is below `lo`: plain
// loops the compiler vectorises.
// The sum of n little-endian u32 at p, and whether any of them is below lo, in one vectorised pass
// (an AVX2 clone is chosen at load time where the host has AVX2).
__attribute__((target_clones("avx2", "default")))
void sum_and_any_below(const uint8_t *p, uint64_t n, uint32_t lo, uint64_t &sum, bool &below) {
    uint64_t s = 0;
    uint32_t f = 0;
    for (uint64_t k = 0; k < n; ++k) {
        uint32_t v;
        std::memcpy(&v, p + 4 * k, 4);
        s += v;
        f |= v < lo;
    }
    sum += s;
    below |= f != 0;
}

inline uint64_t sat_add(uint64_t a, uint64_t b, uint64_t cap) {  // the reference's ints do not wrap
    uint64_t s = a + b;
    return (s < a || s > cap) ? cap : s;
}

}  // namespace

void put_varint(std::vector<uint8_t> &out, uint64_t v) {
    if (v >= (1ULL << 63)) throw Invalid("varint out of range");
    while (v >= 0x80) {
        out.push_back((uint8_t)((v & 0x7F) | 0x80));
        v >>= 7;
    }
    out.push_back((uint8_t)v);
}

uint64_t prefix_need(const uint8_t *d, uint64_t avail, uint64_t total) {
    const uint64_t lim = std::min(avail, total);
    uint64_t pos = 0;
    bool out = false;  // the walk needs a byte past lim
    auto byte = [&]() -> uint64_t {
        if (pos >= lim) {
            out = true;
            return 0;
        }
        return d[pos++];
    };
    auto varint = [&]() -> uint64_t {
        uint64_t v = 0;
        for (int shift = 0; shift < 70 && !out; shift += 7) {
            const uint64_t b = byte();
            if (shift < 64) v |= (b & 0x7F) << shift;
            if (!(b & 0x80)) return v;
        }
        return v;
    };
    auto skip = [&](uint64_t n) {
        if (n > lim - std::min(lim, pos)) out = true;
        else pos += n;
    };
    auto more = [&]() { return std::max(avail + 1, 2 * avail); };  // past the available bytes: at least this
    // a prefix that is not an update of this version is left to parse, which rejects it
    if (lim < 5 || std::memcmp(d, "CRXS", 4) != 0 || d[4] != kVersion) return avail;
    skip(5);
    const uint64_t n_tables = varint();
    if (out) return more();
    if (n_tables > 256) return avail;
    for (uint64_t t = 0; t < n_tables; ++t) {
        byte();
        const uint64_t n_sym = varint();
        if (out) return more();
        if (n_sym > total) return avail;
        for (uint64_t k = 0; k < n_sym && !out; ++k) {
            varint();
            byte();
        }
        if (out) return more();
    }
    const uint64_t n_tensors = varint();
    if (out) return more();
    if (n_tensors > total) return avail;
    uint64_t blocks = 0;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        skip(varint());  // name
        varint();        // numel
        skip(8);         // checksum
        const uint64_t n_groups = varint();
        if (out) return more();
        if (n_groups > 256) return avail;
        for (uint64_t g = 0; g < n_groups && !out; ++g) {
            byte();
            blocks = sat_add(blocks, n_blocks(varint()), total);
            byte();
        }
        if (out) return more();
    }
    if (blocks > total / 4) return avail;
    const uint64_t table_end = pos + 4 * blocks;
    if (table_end + 1 > lim) return std::max(table_end + 10, avail + 1);  // the table and the payload length
    pos = table_end;
    varint();  // payload length
    return out ? more() : pos;
}

// wire.py:126-212, check for check and in the same order.
void parse(const uint8_t *data, uint64_t avail, uint64_t total, uint8_t last, Update &u) {
    Reader r{data, avail, total};
    const uint8_t *magic = r.take(4);
    if (std::memcmp(magic, "CRXS", 4) != 0) throw Corrupt("not a crukx-sync update");
    int version = r.u8();
    if (version != kVersion) throw Corrupt("unsupported format version " + std::to_string(version));

    uint64_t n_tables = r.varint();
    if (n_tables > 256) throw Corrupt("too many tables");
    bool have_table[256] = {};
    u.tables.clear();
    for (uint64_t ti = 0; ti < n_tables; ++ti) {
        int exp = r.u8();
        uint64_t n_sym = r.varint();
        uint64_t lim = std::min<uint64_t>(kMaxSymbol + 1, r.remaining() / 2);
        if (have_table[exp] || !(n_sym > 0 && n_sym <= lim)) throw Corrupt("bad table header");
        have_table[exp] = true;
        Table t;
        t.exponent = exp;
        t.symbols.resize(n_sym);
        t.lengths.resize(n_sym);
        uint64_t max_sym = 0;
        for (uint64_t k = 0; k < n_sym; ++k) {
            uint64_t s = r.varint();
            t.lengths[k] = (uint8_t)r.u8();
            max_sym = std::max(max_sym, s);
            t.symbols[k] = (uint32_t)std::min<uint64_t>(s, 0xFFFFFFFFu);
        }
        std::vector<uint32_t> sorted(t.symbols);
        std::sort(sorted.begin(), sorted.end());
        bool dup = std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end();
        if (dup || max_sym > kMaxSymbol) throw Corrupt("bad table symbols");
        int mn = 255, mx = 0;
        for (uint8_t L : t.lengths) {
            mn = std::min<int>(mn, L);
            mx = std::max<int>(mx, L);
        }
        if (mn < 1 || mx > kMaxCodeLen) throw Corrupt("bad Huffman code lengths");
        // Kraft sum in units of 2^-17: every term 2^-L (L <= 17) is a whole number of units, so
        // the reference's fp64 sum (wire.py:206) is exact and "> 1 + 1e-12" is "> 2^17 units".
        uint64_t kraft = 0;
        for (uint8_t L : t.lengths) kraft += 1ULL << (kMaxCodeLen - L);
        if (kraft > (1ULL << kMaxCodeLen)) throw Corrupt("bad Huffman code lengths");
        u.tables.push_back(std::move(t));
    }

    uint64_t n_tensors = r.varint();
    if (n_tensors > r.remaining()) throw Corrupt("too many tensors");
    u.tensors.clear();
    u.tensors.reserve(n_tensors);
    uint64_t total_blocks = 0, per_exp[256] = {};
    const uint64_t kCap = 1ULL << 63;
    std::unordered_set<std::string_view> names;  // views into the parsed bytes
    names.reserve(std::min<uint64_t>(n_tensors, 1 << 16));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorHeader th;
        uint64_t name_len = r.varint();
        const uint8_t *name = r.take(name_len);
        if (!valid_utf8(name, name_len)) throw Corrupt("tensor name is not valid UTF-8");
        th.name.assign((const char *)name, name_len);
        if (!names.insert(std::string_view((const char *)name, name_len)).second)
            throw Corrupt("tensor '" + th.name + "' appears twice");
        th.numel = r.varint();
        const uint8_t *c = r.take(8);
        for (int k = 0; k < 8; ++k) th.checksum |= (uint64_t)c[k] << (8 * k);
        uint64_t n_groups = r.varint();
        if (!(n_groups > 0 && n_groups <= 256)) throw Corrupt("bad group count");
        bool exps[256] = {};
        uint64_t sum = 0;
        th.groups.reserve(n_groups);
        for (uint64_t g = 0; g < n_groups; ++g) {
            Group gr;
            gr.exponent = r.u8();
            gr.count = r.varint();
            gr.rice = r.u8();
            if (exps[gr.exponent] || !have_table[gr.exponent]) throw Corrupt("bad group exponent");
            if (!(gr.count > 0 && gr.count <= th.numel) || gr.rice > kMaxRice) throw Corrupt("bad group header");
            exps[gr.exponent] = true;
            total_blocks = sat_add(total_blocks, n_blocks(gr.count), 1ULL << 62);
            sum = sat_add(sum, gr.count, kCap);
            th.groups.push_back(gr);
        }
        if (sum > th.numel) throw Corrupt("more changes than elements");
        for (const Group &gr : th.groups) per_exp[gr.exponent] = sat_add(per_exp[gr.exponent], gr.count, kCap);
        u.tensors.push_back(std::move(th));
    }
    // every table used, and no larger than the changes with its exponent (wire.py:241-248)
    for (const Table &t : u.tables)
        if (t.symbols.size() > per_exp[t.exponent]) throw Corrupt("table unused or larger than its changes");

    if (total_blocks > r.remaining() / 4) throw Corrupt("block table longer than the update");
    u.block_table_offset = r.pos;
    u.block_table = r.take(4 * total_blocks);
    u.n_blocks = total_blocks;
    static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "the block table is little-endian u32");
    // one pass over the table: the total, and the check that each change has at least 2 + rice_r
    // bits (wire.py:261-268; its error is raised after the payload checks, as there)
    uint64_t total_bits = 0, b = 0, changes = 0;
    bool short_block = false;
    for (const TensorHeader &t : u.tensors)
        for (const Group &g : t.groups) {
            changes += g.count;
            const uint64_t nb = n_blocks(g.count), full = g.count / kBlock;
            sum_and_any_below(u.block_table + 4 * b, full, kBlock * (2 + (uint32_t)g.rice), total_bits, short_block);
            if (nb > full) {
                const uint32_t v = u.block_bits(b + full);
                total_bits += v;
                if ((uint64_t)v < (g.count - full * kBlock) * (uint64_t)(2 + g.rice)) short_block = true;
            }
            b += nb;
        }
    uint64_t payload_len = r.varint();
    u.payload_offset = r.pos;
    r.skip(payload_len);
    u.payload_len = payload_len;
    if (r.remaining()) throw Corrupt("trailing bytes after the payload");
    if ((total_bits + 7) / 8 != payload_len) throw Corrupt("payload length does not match its block table");
    if ((total_bits % 8) && (last & ((1u << (8 - total_bits % 8)) - 1))) throw Corrupt("non-zero padding bits");
    if (short_block) throw Corrupt("block shorter than its symbols could be");
    u.total_bits = total_bits;
    u.total_changes = changes;
}

// ------------------------------------------------------------------ Huffman
// Two-queue Huffman construction.  The reference pops (count, id) pairs from a heap
// (codec.py:85-94); leaves carry ids 0..n-1 in table order and merged nodes ids n, n+1, ....
// Merged nodes are created with non-decreasing counts and increasing ids, so the queue of merged
// nodes is already ordered by (count, id); with the leaves sorted by (count, id) the smallest
// pair is always at the head of one of the two queues, giving the same merges as the heap.
namespace {

using u128 = unsigned __int128;

std::vector<int> huffman_unlimited(const std::vector<uint64_t> &counts) {
    const int64_t n = (int64_t)counts.size();
    if (n == 1) return {1};
    std::vector<int64_t> leaves(n);
    std::iota(leaves.begin(), leaves.end(), 0);
    std::stable_sort(leaves.begin(), leaves.end(), [&](int64_t a, int64_t b) { return counts[a] < counts[b]; });
    struct Node {
        u128 c;
        int64_t id;
    };
    std::vector<Node> merged;
    merged.reserve(n - 1);
    std::vector<int64_t> parent(2 * n - 1);
    size_t li = 0, mi = 0;
    auto pick = [&]() -> Node {
        bool take_leaf;
        if (li >= leaves.size()) take_leaf = false;
        else if (mi >= merged.size()) take_leaf = true;
        else {
            const u128 lc = counts[leaves[li]];
            const Node &m = merged[mi];
            take_leaf = lc < m.c || (lc == m.c && leaves[li] < m.id);
        }
        if (take_leaf) {
            int64_t id = leaves[li++];
            return Node{counts[id], id};
        }
        return merged[mi++];
    };
    for (int64_t next = n; next < 2 * n - 1; ++next) {
        Node a = pick(), b = pick();
        parent[a.id] = parent[b.id] = next;
        merged.push_back(Node{a.c + b.c, next});
    }
    std::vector<int> depth(2 * n - 1, 0);
    for (int64_t node = 2 * n - 3; node >= 0; --node) depth[node] = depth[parent[node]] + 1;
    depth.resize(n);
    return depth;
}

}  // namespace

std::vector<int> huffman_lengths(const std::vector<uint64_t> &counts_in) {
    std::vector<uint64_t> c(counts_in);
    for (int round = 0; round < 8; ++round) {
        std::vector<int> L = huffman_unlimited(c);
        if (*std::max_element(L.begin(), L.end()) <= kMaxCodeLen) return L;
        for (uint64_t &x : c) x = std::max<uint64_t>(1, x >> 2);
    }
    int bits = 0;
    for (uint64_t v = c.size() - 1; v; v >>= 1) ++bits;
    return std::vector<int>(c.size(), std::max(1, bits));
}

// DEFLATE-style construction: the first code of length L is (first(L-1) + count(L-1)) << 1,
// codes within a length follow table position.  Identical to assigning codes in
// (length, position) order with code = (code + 1) << (len - prev_len).
std::vector<uint32_t> canonical_codes(const std::vector<int> &lengths) {
    int maxlen = 0;
    for (int L : lengths) maxlen = std::max(maxlen, L);
    std::vector<uint64_t> count(maxlen + 2, 0), next(maxlen + 2, 0);
    for (int L : lengths) count[L]++;
    uint64_t code = 0;
    int minlen = maxlen;
    for (int L : lengths) minlen = std::min(minlen, L);
    for (int L = minlen; L <= maxlen; ++L) {
        next[L] = code;
        code = (code + count[L]) << 1;
    }
    std::vector<uint32_t> out(lengths.size());
    for (size_t i = 0; i < lengths.size(); ++i) out[i] = (uint32_t)next[lengths[i]]++;
    return out;
}

// ------------------------------------------------------------------ Rice
// r0 = floor(log2(max(gap_sum / count, 1))) clamped to [0, 30], in fp64 as the reference computes it
// (codec.py:271-272).  The device computes the same r0 exactly in integers (the largest k with
// count * 2^k <= gap_sum); the two agree whenever gap_sum < 2^32, which always holds there because
// a group's gaps sum to less than its size.
void rice_candidates(uint64_t count, uint64_t gap_sum, int cand[3]) {
    const double mean = (double)gap_sum / (double)count;
    int r0 = (int)std::floor(std::log2(mean < 1.0 ? 1.0 : mean));
    r0 = std::min(std::max(r0, 0), kMaxRice);
    cand[0] = std::max(r0 - 1, 0);
    cand[1] = r0;
    cand[2] = std::min(r0 + 1, kMaxRice);
}

// cost(r) = sum((gap >> r) + 1 + r); the first minimum among the three wins (torch.argmin).
int rice_choose(uint64_t count, const int cand[3], const uint64_t shifted[3]) {
    int best = 0;
    u128 best_cost = 0;
    for (int k = 0; k < 3; ++k) {
        u128 cost = (u128)shifted[k] + (u128)count * (1 + (unsigned)cand[k]);
        if (k == 0 || cost < best_cost) {
            best = k;
            best_cost = cost;
        }
    }
    return cand[best];
}

}  // namespace crx
