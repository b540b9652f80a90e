// Runs the product's update parser (crukx-sync_amd/csrc/format.cpp) over a batch of inputs, each
// parsed whole and as prefixes of several lengths (as crx_parse_prefix does: prefix_need first, parse
// when the prefix holds what it needs), and prints one line per input.  Built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_parse_sanitized.py, which compares
// the lines with the production library's crx_parse.
//
// Input file: repeated (u64 little-endian length, bytes).  Output line per input:
//   <whole> | <prefix cut 0> | <cut 1> | <cut len/2> | <cut len-1>
// where each outcome is "ok <tables> <tensors> <blocks> <changes> <payload offset> <payload len>"
// (the whole one followed by prefix_need of the whole input), "corrupt <message>", "invalid <message>"
// or "need <bytes>".
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <string>
#include <vector>

#include "format.h"

namespace {

std::string outcome(const uint8_t *data, uint64_t avail, uint64_t total, uint8_t last) {
    crx::Update u;
    try {
        crx::parse(data, avail, total, last, u);
    } catch (const crx::NeedMore &m) {
        return "need " + std::to_string(m.need);
    } catch (const crx::Corrupt &e) {
        return std::string("corrupt ") + e.what();
    } catch (const std::exception &e) {
        return std::string("invalid ") + e.what();
    }
    return "ok " + std::to_string(u.tables.size()) + " " + std::to_string(u.tensors.size()) + " " +
           std::to_string(u.n_blocks) + " " + std::to_string(u.total_changes) + " " +
           std::to_string(u.payload_offset) + " " + std::to_string(u.payload_len);
}

// crx_parse_prefix's order: the walk first, asking for more without parsing
std::string prefix_outcome(const uint8_t *data, uint64_t avail, uint64_t total, uint8_t last) {
    const uint64_t want = crx::prefix_need(data, avail, total);
    if (want > avail && avail < total) return "need " + std::to_string(std::min(want, total));
    return outcome(data, avail, total, last);
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s BATCH\n", argv[0]);
        return 2;
    }
    std::ifstream f(argv[1], std::ios::binary);
    const std::vector<uint8_t> all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    size_t at = 0;
    while (at + 8 <= all.size()) {
        uint64_t n = 0;
        for (int i = 0; i < 8; ++i) n |= (uint64_t)all[at + i] << (8 * i);
        at += 8;
        if (n > all.size() - at) return 3;
        // each input (and each prefix) in an allocation of exactly its size (non-null even when empty),
        // so that any read past it is reported
        std::unique_ptr<uint8_t[]> in(new uint8_t[n]);
        std::memcpy(in.get(), all.data() + at, n);
        at += n;
        const uint8_t last = n ? in[n - 1] : 0;
        std::string line = outcome(in.get(), n, n, last);
        if (line.rfind("ok ", 0) == 0) line += " " + std::to_string(crx::prefix_need(in.get(), n, n));
        for (uint64_t cut : {uint64_t(0), uint64_t(1), n / 2, n ? n - 1 : 0}) {
            if (cut > n) cut = n;
            std::unique_ptr<uint8_t[]> pre(new uint8_t[cut]);
            std::memcpy(pre.get(), in.get(), cut);
            line += " | " + prefix_outcome(pre.get(), cut, n, last);
        }
        std::printf("%s\n", line.c_str());
    }
    return at == all.size() ? 0 : 3;
}
