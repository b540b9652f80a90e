// A CPU model of the apply's decoder (k_decode, decode_blocks in crukx-sync_amd/csrc/kernels.hip) and
// local-index pass (k_local_fix), with the decoding tables built as engine.cpp's apply() builds them,
// for tests only.  Every array access is bounds-checked (std::vector::at).  Built with AddressSanitizer
// and UBSan by tests/test_decode_model.py, which feeds it corrupted updates.
//
// Input file: u32 T, then T x 256 u32 receiver exponent counts (sizes[t][k]), then repeated (u64
// little-endian length, update bytes).  Output, one line per update: the value emu() returns.
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>
#include <algorithm>
#include "format.h"
#include <cstdio>
#include <fstream>
#include <iterator>
#include <memory>
using namespace crx;

static inline uint64_t min64(uint64_t a, uint64_t b) { return a < b ? a : b; }

struct Reader {
    const std::vector<uint64_t> *p;
    uint64_t n, w, hi, lo, nx;
    uint64_t word(uint64_t i) const { return p->at(min64(i, n - 1)); }
    void start(const std::vector<uint64_t> &pay, uint64_t nw, uint64_t pos) {
        p = &pay; n = nw; w = pos >> 6; hi = word(w); lo = word(w + 1); nx = word(w + 2);
    }
    uint64_t bits(uint64_t pos) {
        const uint64_t t = pos >> 6;
        if (t >= w + 3) { w = t; hi = word(t); lo = word(t + 1); nx = word(t + 2); }
        else { while (w < t) { hi = lo; lo = nx; nx = word(w + 3); ++w; } }
        const uint32_t s = (uint32_t)(pos & 63);
        const uint64_t h = __builtin_bswap64(hi), l = __builtin_bswap64(lo);
        return s ? (h << s) | (l >> (64 - s)) : h;
    }
};

struct G { uint32_t tensor, exponent, count, elem_base, blk_base, rice, table; };

// returns: -1 parse error, -2 out-of-bounds access, else flags: 1 decode bad, 2 local bad, 4 group bad,
// 8 locals not strictly increasing in a group while no flag is set, 16 a local past 2^32
static int emu(const uint8_t *data, uint64_t len, const uint32_t *sizes, uint32_t T, char *msg, uint64_t msglen) {
    Update u;
    try {
        parse(data, len, len, len ? data[len - 1] : 0, u);
    } catch (const std::exception &e) {
        std::strncpy(msg, e.what(), msglen - 1);
        return -1;
    }
    if (u.tensors.size() != T) return -1;
    try {
        int table_of[256];
        std::fill(table_of, table_of + 256, -1);
        std::vector<uint32_t> lim(u.tables.size() * 17, 0), off(u.tables.size() * 17, 0), syms;
        for (size_t ti = 0; ti < u.tables.size(); ++ti) {
            const Table &tb = u.tables[ti];
            table_of[tb.exponent] = (int)ti;
            uint32_t per_len[kMaxCodeLen + 1] = {};
            for (uint8_t l : tb.lengths) per_len[l]++;
            std::vector<uint32_t> order(tb.symbols.size());
            for (size_t k = 0; k < order.size(); ++k) order[k] = (uint32_t)k;
            std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return tb.lengths[a] < tb.lengths[b]; });
            uint32_t code = 0, idx = (uint32_t)syms.size();
            for (int l = 1; l <= kMaxCodeLen; ++l) {
                lim.at(ti * 17 + l - 1) = (code + per_len[l]) << (kMaxCodeLen - l);
                off.at(ti * 17 + l - 1) = idx - code;
                code = (code + per_len[l]) << 1;
                idx += per_len[l];
            }
            for (uint32_t k : order) syms.push_back(tb.symbols[k]);
        }
        std::vector<G> groups;
        uint64_t elem = 0, blk = 0;
        for (uint32_t t = 0; t < T; ++t)
            for (const Group &g : u.tensors[t].groups) {
                groups.push_back(G{t, (uint32_t)g.exponent, (uint32_t)g.count, (uint32_t)elem, (uint32_t)blk, (uint32_t)g.rice,
                                   (uint32_t)table_of[g.exponent]});
                elem += g.count;
                blk += n_blocks(g.count);
            }
        const uint64_t C = elem, B = blk;
        std::vector<uint32_t> bb(B);
        for (uint64_t b = 0; b < B; ++b) bb.at(b) = u.block_bits(b);
        std::vector<uint64_t> boff(B + 1, 0);
        for (uint64_t b = 0; b < B; ++b) boff.at(b + 1) = boff.at(b) + bb.at(b);
        const uint64_t pay_words = (u.payload_len + 7) / 8 + 2;
        std::vector<uint64_t> pay(pay_words, 0);
        std::memcpy(pay.data(), data + u.payload_offset, u.payload_len);
        std::vector<uint32_t> bmap(B);
        for (uint32_t g = 0; g < groups.size(); ++g)
            for (uint64_t k = 0; k < n_blocks(groups[g].count); ++k) bmap.at(groups[g].blk_base + k) = g;
        std::vector<uint64_t> dz(C, 0xDEADBEEFDEADBEEFull), blk_sum(B, 0);
        std::vector<uint8_t> written(C, 0);
        int flags = 0;
        for (uint64_t b = 0; b < B; ++b) {
            const G &gr = groups.at(bmap.at(b));
            const uint64_t kb = b - gr.blk_base;
            const uint32_t cnt = (uint32_t)min64(256, gr.count - kb * 256);
            const uint64_t eb = (uint64_t)gr.elem_base + kb * 256;
            uint64_t size = 0;  // the tensor's numel
            size = u.tensors.at(gr.tensor).numel;
            const uint32_t rice = gr.rice;
            const uint64_t qmax = size >> rice;
            uint64_t cur = boff.at(b);
            const uint64_t end = cur + bb.at(b);
            bool bad = false;
            Reader R;
            R.start(pay, pay_words, cur);
            uint32_t L17[17], O17[17];
            for (int l = 0; l < 17; ++l) { L17[l] = lim.at((uint64_t)gr.table * 17 + l); O17[l] = off.at((uint64_t)gr.table * 17 + l); }
            uint64_t rel = 0;
            for (uint32_t s = 0; s < cnt && !bad; ++s) {
                uint64_t x = R.bits(cur), q;
                if (~x) q = (uint64_t)__builtin_clzll(~x);
                else {
                    q = 64;
                    for (;;) {
                        if (q > qmax || cur + q >= end) break;
                        const uint64_t y = ~R.bits(cur + q);
                        if (y) { q += (uint64_t)__builtin_clzll(y); break; }
                        q += 64;
                    }
                }
                const uint64_t c = cur + q + 1;
                if (q + 1 + rice + 17 <= 64) x <<= (q + 1);
                else x = R.bits(c);
                const uint64_t rem = rice ? x >> (64 - rice) : 0ULL;
                const uint32_t peek = (uint32_t)((x << rice) >> (64 - 17));
                uint32_t Lc = 1;
                for (int l = 0; l < 17; ++l) Lc += L17[l] <= peek ? 1u : 0u;
                const uint32_t li = Lc - 1;
                const uint32_t idx = Lc <= 17 ? O17[li] + (peek >> (17 - Lc)) : 0u;
                const uint64_t gap = (q << rice) | rem;
                if (q > qmax || cur + q >= end || Lc > 17 || gap >= size) { bad = true; break; }
                rel += gap + 1;
                const uint32_t si = std::min<uint32_t>(idx, (uint32_t)syms.size() - 1);
                const uint32_t zz = syms.at(si);
                dz.at(eb + s) = (uint64_t)zz | ((uint64_t)min64(rel - 1, 0xFFFFFFFFULL) << 32);
                written.at(eb + s) = 1;
                cur = c + rice + Lc;
            }
            if (!bad && cur != end) bad = true;
            blk_sum.at(b) = rel;
            if (bad) flags |= 1;
        }
        // k_local_fix
        std::vector<uint64_t> pre(B + 1, 0);
        for (uint64_t b = 0; b < B; ++b) pre.at(b + 1) = pre.at(b) + blk_sum.at(b);
        std::vector<uint64_t> local(C, 0);
        for (uint64_t b = 0; b < B; ++b) {
            const G &gr = groups.at(bmap.at(b));
            const uint64_t kb = b - gr.blk_base;
            const uint32_t cnt = (uint32_t)min64(256, gr.count - kb * 256);
            const uint64_t eb = (uint64_t)gr.elem_base + kb * 256;
            const uint64_t sz = sizes[(uint64_t)gr.tensor * 256 + gr.exponent];
            if (b == gr.blk_base && gr.count > sz) flags |= 4;
            if (flags & 1) continue;
            const uint64_t base = pre.at(b) - pre.at(gr.blk_base);
            for (uint32_t s = 0; s < cnt; ++s) {
                const uint64_t raw = dz.at(eb + s) >> 32;
                const uint64_t l = base + raw;
                if (l >= sz) flags |= 2;
                if (l > 0xFFFFFFFFull) flags |= 16;
                local.at(eb + s) = l;
            }
        }
        if (!(flags & 7)) {
            for (const G &g : groups)
                for (uint64_t i = 1; i < g.count; ++i)
                    if (local.at(g.elem_base + i) <= local.at(g.elem_base + i - 1)) { flags |= 8; break; }
        }
        return flags;
    } catch (const std::out_of_range &e) {
        std::strncpy(msg, e.what(), msglen - 1);
        return -2;
    }
}

int main(int argc, char **argv) {
    if (argc != 2) return 2;
    std::ifstream f(argv[1], std::ios::binary);
    const std::vector<uint8_t> all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (all.size() < 4) return 3;
    uint32_t T = 0;
    std::memcpy(&T, all.data(), 4);
    size_t at = 4;
    if (all.size() < at + (size_t)T * 256 * 4) return 3;
    std::vector<uint32_t> sizes((size_t)T * 256);
    std::memcpy(sizes.data(), all.data() + at, sizes.size() * 4);
    at += sizes.size() * 4;
    char msg[256];
    while (at + 8 <= all.size()) {
        uint64_t n = 0;
        std::memcpy(&n, all.data() + at, 8);
        at += 8;
        if (n > all.size() - at) return 3;
        std::unique_ptr<uint8_t[]> in(new uint8_t[n ? n : 1]);  // exactly the input's size
        std::memcpy(in.get(), all.data() + at, n);
        at += n;
        msg[0] = 0;
        std::printf("%d\n", emu(in.get(), n, sizes.data(), T, msg, sizeof msg));
    }
    return at == all.size() ? 0 : 3;
}
