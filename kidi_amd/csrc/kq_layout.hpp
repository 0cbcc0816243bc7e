// gfx950 weight layout of the quantized linear layer.
//
// A packed weight [N, K] with b-bit codes is stored as 1 KiB tiles. A tile covers 16 output rows and KT = 512/b
// input columns (64 bytes per row): KT = 256 (2-bit), 128 (4-bit), 64 (8-bit). Tiles are ordered row-block major:
// tile (nt, kt) lives at byte (nt * k_tiles + kt) * 1024, so one row block's K range is one contiguous stream.
//
// Inside a tile the 16-byte slot of lane l = nn + 16*L (nn = row within the tile, L = 0..3) is what wavefront
// lane l loads with one 128-bit access. Each 64-column block j of the tile gives every lane 16 codes, and byte
// position p = 8*h + i (h = 0..1, i = 0..7) of those 16 codes is column 64*j + 32*h + 8*L + i. The activation
// codes of a row use the same order inside every 64-column block (byte 16*L + 8*h + i of block j), so a lane's
// 16 weight bytes and 16 activation bytes pair up element by element: that is the operand order of
// v_mfma_i32_16x16x64_i8 (lane = row + 16 * k-quarter), of v_mfma_i32_16x16x32_i8 for one 32-column half h, and
// of v_dot4_i32_i8 on 4-byte pieces. A 32-column chunk (j, h) of a row is spread over the 4 lanes nn + 16*L.
//
// Codes are stored unsigned where they are narrower than a byte, so they unpack with a shift and a mask:
//   4-bit: u = c + 8 in [0, 15]. Dword 2*j + h of the slot holds the 8 codes of (j, h): the low nibble of byte r
//          is i = r, the high nibble of byte r is i = 4 + r. lo = d & 0x0F0F0F0F and hi = (d >> 4) & 0x0F0F0F0F are
//          then codes i = 0..3 and 4..7 in byte order.
//   2-bit: u = c + 2 in [0, 3]. Dword j holds block j; (d >> 2*s) & 0x03030303 is codes p = 4*s + 0..3.
//   8-bit: c as a signed byte at position p.
// Per-group metadata (scales, zero-points, code sums) is stored [n_tiles][groups][16], so the 16 values a tile
// row block needs for one group are adjacent.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define KQ_HD __host__ __device__
#else
#define KQ_HD
#endif

namespace kq {

constexpr int kTileBytes = 1024;
constexpr int kTileRows = 16;

KQ_HD constexpr int k_per_tile(int bits) { return 512 / bits; }
KQ_HD constexpr int sign_offset(int bits) { return bits == 8 ? 0 : (1 << (bits - 1)); }

KQ_HD inline std::int64_t round_up(std::int64_t v, std::int64_t m) { return (v + m - 1) / m * m; }

struct Geometry {
    int bits = 4;
    int group = 128;
    std::int64_t rows = 0, cols = 0;      // N, K
    std::int64_t rows_p = 0, cols_p = 0;  // padded to the tile
    std::int64_t n_tiles = 0, k_tiles = 0, groups_p = 0;

    KQ_HD static Geometry make(int bits, int group, std::int64_t rows, std::int64_t cols) {
        Geometry g;
        g.bits = bits;
        g.group = group;
        g.rows = rows;
        g.cols = cols;
        g.rows_p = round_up(rows, kTileRows);
        g.cols_p = round_up(cols, k_per_tile(bits));
        g.n_tiles = g.rows_p / kTileRows;
        g.k_tiles = g.cols_p / k_per_tile(bits);
        g.groups_p = group > 0 ? g.cols_p / group : 0;
        return g;
    }
    KQ_HD std::int64_t tile_bytes_total() const { return n_tiles * k_tiles * kTileBytes; }
    KQ_HD std::int64_t meta_count() const { return n_tiles * groups_p * kTileRows; }
    KQ_HD std::int64_t meta_index(std::int64_t n, std::int64_t b) const {
        return ((n / kTileRows) * groups_p + b) * kTileRows + (n % kTileRows);
    }
};

// The tiled fast layout needs every 32-column chunk inside one group and groups that tile the padded K exactly.
KQ_HD inline bool tiled_group_ok(int bits, int group) {
    const int kt = k_per_tile(bits);
    return group >= 32 && group % 32 == 0 && (kt % group == 0 || group % kt == 0);
}

// Position of code (n, k) inside the tiled layout: byte offset and bit shift of its field.
struct CodePos {
    std::int64_t byte;
    int shift;
};

KQ_HD inline CodePos code_position(int bits, std::int64_t k_tiles, std::int64_t n, std::int64_t k) {
    const int kt_cols = k_per_tile(bits);
    const std::int64_t nt = n / kTileRows, kt = k / kt_cols;
    const int nn = static_cast<int>(n % kTileRows);
    const int kk = static_cast<int>(k % kt_cols);
    const int j = kk / 64, r64 = kk % 64;
    const int h = r64 / 32, L = (r64 % 32) / 8, i = r64 % 8;
    const std::int64_t slot = (nt * k_tiles + kt) * kTileBytes + 16 * (nn + 16 * L);
    if (bits == 8) return {slot + 8 * h + i, 0};
    if (bits == 4) return {slot + 4 * (2 * j + h) + (i % 4), (i >= 4) ? 4 : 0};
    return {slot + 4 * j + (i % 4), 2 * (2 * h + i / 4)};
}

// Signed code of element k of a Kidi-layout row (ops/quantization.cpp:91, :113-114; eager_test.cpp:318-320).
KQ_HD inline int kidi_code(const std::uint8_t* row, int bits, std::int64_t k) {
    if (bits == 8) return static_cast<std::int8_t>(row[k]);
    const int per_byte = 8 / bits;
    const int raw = (row[k / per_byte] >> ((k % per_byte) * bits)) & ((1 << bits) - 1);
    const int sign = 1 << (bits - 1);
    return (raw ^ sign) - sign;
}

// Permuted position of activation column k inside its row (same order as the weight slots).
KQ_HD inline std::int64_t act_position(std::int64_t k) {
    const std::int64_t block = k / 64;
    const int r = static_cast<int>(k % 64);
    const int h = r / 32, L = (r % 32) / 8, i = r % 8;
    return block * 64 + 16 * L + 8 * h + i;
}

}  // namespace kq
