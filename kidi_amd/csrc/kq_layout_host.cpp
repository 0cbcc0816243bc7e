// Host-side conversion between Kidi's packed weight layout (ops/quantization.cpp:91, :113-114: row-major,
// element k of a row in bits (k % (8/bits)) * bits of byte k / (8/bits)) and the gfx950 tile layout of
// kq_layout.hpp. Runs once per weight at load time, multi-threaded over row blocks.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "kq_internal.hpp"

namespace kq {
namespace {

template <typename Body>
void parallel_blocks(std::int64_t count, Body body) {
    const std::int64_t hw = std::max<std::int64_t>(1, std::thread::hardware_concurrency());
    const std::int64_t workers = std::min<std::int64_t>(hw, std::max<std::int64_t>(1, count / 16));
    if (workers <= 1) {
        body(0, count);
        return;
    }
    std::vector<std::thread> pool;
    const std::int64_t chunk = (count + workers - 1) / workers;
    for (std::int64_t w = 0; w < workers; ++w) {
        const std::int64_t a = w * chunk, b = std::min(count, a + chunk);
        if (a < b) pool.emplace_back(body, a, b);
    }
    for (auto& t : pool) t.join();
}

}  // namespace

void encode_tiles(int bits, std::int64_t rows, std::int64_t cols, const std::uint8_t* values, std::uint8_t* tiles) {
    const Geometry g = Geometry::make(bits, 32, rows, cols);
    const std::int64_t row_bytes = cols / (8 / bits);
    const int off = sign_offset(bits);
    const int mask = (1 << bits) - 1;
    parallel_blocks(g.n_tiles, [&](std::int64_t nt0, std::int64_t nt1) {
        std::memset(tiles + nt0 * g.k_tiles * kTileBytes, 0, static_cast<std::size_t>((nt1 - nt0) * g.k_tiles * kTileBytes));
        for (std::int64_t nt = nt0; nt < nt1; ++nt)
            for (std::int64_t n = nt * kTileRows; n < (nt + 1) * kTileRows; ++n)
                for (std::int64_t k = 0; k < g.cols_p; ++k) {
                    // padding rows/columns carry code 0
                    const int c = (n < rows && k < cols) ? kidi_code(values + n * row_bytes, bits, k) : 0;
                    const CodePos p = code_position(bits, g.k_tiles, n, k);
                    if (bits == 8) tiles[p.byte] = static_cast<std::uint8_t>(c);
                    else tiles[p.byte] = static_cast<std::uint8_t>(tiles[p.byte] | (((c + off) & mask) << p.shift));
                }
    });
}

void decode_tiles(int bits, std::int64_t rows, std::int64_t cols, const std::uint8_t* tiles, std::int8_t* codes) {
    const Geometry g = Geometry::make(bits, 32, rows, cols);
    const int off = sign_offset(bits);
    const int mask = (1 << bits) - 1;
    for (std::int64_t n = 0; n < rows; ++n)
        for (std::int64_t k = 0; k < cols; ++k) {
            const CodePos p = code_position(bits, g.k_tiles, n, k);
            codes[n * cols + k] = bits == 8 ? static_cast<std::int8_t>(tiles[p.byte])
                                            : static_cast<std::int8_t>(((tiles[p.byte] >> p.shift) & mask) - off);
        }
}

}  // namespace kq
