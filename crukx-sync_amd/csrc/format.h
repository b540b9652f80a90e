// Host-side pieces of the update format (docs/FORMAT.md of the reference, version 2):
// the parsed update, the parser with every receiver limit, header serialisation, Huffman code
// lengths, canonical codes and the Rice parameter choice.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace crx {

constexpr int kBlock = 256;          // changes per block (wire.py:13)
constexpr int kMaxCodeLen = 17;      // wire.py:10
constexpr uint32_t kMaxSymbol = 131070;  // wire.py:11
constexpr int kMaxRice = 30;         // wire.py:12
constexpr uint8_t kVersion = 2;      // wire.py:9

struct Corrupt : std::runtime_error {  // -> CorruptUpdate
    explicit Corrupt(const std::string &m) : std::runtime_error(m) {}
};
struct Invalid : std::runtime_error {  // -> ValueError
    explicit Invalid(const std::string &m) : std::runtime_error(m) {}
};
struct DeviceError : std::runtime_error {  // -> RuntimeError
    explicit DeviceError(const std::string &m) : std::runtime_error(m) {}
};
struct NeedMore {  // parse from a prefix: this many leading bytes are needed
    uint64_t need;
};

struct Table {
    int exponent = 0;
    std::vector<uint32_t> symbols;
    std::vector<uint8_t> lengths;
};

struct Group {
    int exponent = 0;
    uint64_t count = 0;
    int rice = 0;
};

struct TensorHeader {
    std::string name;
    uint64_t numel = 0;
    uint64_t checksum = 0;
    std::vector<Group> groups;
};

struct Update {
    std::vector<Table> tables;
    std::vector<TensorHeader> tensors;
    // the block table: n_blocks little-endian u32 inside the parsed bytes (which the caller keeps
    // alive for the life of the Update, as for the payload)
    const uint8_t *block_table = nullptr;
    uint64_t n_blocks = 0;
    uint64_t block_table_offset = 0;  // byte offset of the block table in the update
    uint32_t block_bits(uint64_t k) const {
        uint32_t v;
        std::memcpy(&v, block_table + 4 * k, 4);
        return v;
    }
    uint64_t payload_offset = 0;
    uint64_t payload_len = 0;
    const uint8_t *payload_host = nullptr;  // null when the payload lives on the device
    uint64_t total_bits = 0;
    uint64_t total_changes = 0;
};

inline uint64_t n_blocks(uint64_t count) { return (count + kBlock - 1) / kBlock; }

// Parses `avail` leading bytes of an update of `total` bytes whose last byte is `last`.  The
// payload bytes themselves are not read (only its length and final byte).  Throws Corrupt for any
// violation of the format's limits, NeedMore if the header or block table extends past `avail`.
void parse(const uint8_t *data, uint64_t avail, uint64_t total, uint8_t last, Update &u);

// The leading bytes that parse() reads of an update of `total` bytes (header, block table and payload
// length), found by walking the same fields without checking them and without throwing: when the
// first `avail` bytes do not hold them all, a number larger than `avail` (exact once the walk reaches
// the block table); `avail` or less when they do, or when the walk cannot be followed (parse then
// reports what it finds).  A first prefix that is too short then costs no exception (the process's
// first C++ exception is slow to unwind: the unwinder first indexes every loaded library).
uint64_t prefix_need(const uint8_t *data, uint64_t avail, uint64_t total);

// LEB128 varint (wire.py:55-61); throws Invalid for values >= 2^63.
void put_varint(std::vector<uint8_t> &out, uint64_t v);

// Huffman code lengths limited to 17 bits, with the reference's tie-breaks (codec.py:71-98).
std::vector<int> huffman_lengths(const std::vector<uint64_t> &counts);
// Canonical codes in order of (length, table position) (codec.py:101-111).
std::vector<uint32_t> canonical_codes(const std::vector<int> &lengths);
// Rice candidates around floor(log2(mean gap)) and the cheapest of them (codec.py:268-275).
void rice_candidates(uint64_t count, uint64_t gap_sum, int cand[3]);
int rice_choose(uint64_t count, const int cand[3], const uint64_t shifted[3]);

}  // namespace crx
