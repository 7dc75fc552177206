// m27q_layout.h -- GGUF block geometry and the TILED device layout.
//
// Shared by the host packer (m27q_layout.cpp) and the gfx950 kernels.  The
// GGUF block byte layouts are fixed by the file format (the reference's
// BlockQ4K / BlockQ5K / BlockQ6K / BlockQ8 structs, exec:18-36, :57-62, hold the same
// bytes); the TILED layout is this library's own.
#pragma once

#include <cstddef>
#include <cstdint>

namespace m27q {

// ggml type ids (include/mono27b_gguf.h:27-43).
constexpr uint32_t kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kIQ4_XS = 23;

// GGUF block sizes in bytes / weights (src/mono27b_gguf.cpp:167-195).
constexpr int kQ4KBytes = 144;   // f16 d, f16 dmin, u8 scales[12], u8 qs[128]
constexpr int kQ5KBytes = 176;   // f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
constexpr int kQ6KBytes = 210;   // u8 ql[128], u8 qh[64], i8 scales[16], f16 d
constexpr int kQ80Bytes = 34;    // f16 d, i8 qs[32]
constexpr int kIQ4XSBytes = 136; // f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128] (exec:44-49)

// Byte offsets inside one GGUF block.
constexpr int kQ4KHdr = 16;      // d, dmin, scales: bytes [0, 16)
constexpr int kQ5KQh = 16, kQ5KQs = 48;
constexpr int kIQ4XSQs = 8;       // d, scales_h, scales_l: bytes [0, 8)
constexpr int kQ6KQl = 0, kQ6KQh = 128, kQ6KSc = 192, kQ6KD = 208;

// ---------------------------------------------------------------- TILED --
// Rows are grouped in tiles of kTileRows.  For tile t and block column b the
// kTileRows blocks of that column are stored as consecutive planes, so a
// wavefront of 64 lanes (8 lanes per row) reads each plane with one
// 16-byte-per-lane load:
//
//  Q4_K  unit = one block column                          1152 B
//        [0, 128)      8 x 16 B headers (d, dmin, scales[12])  row i at 16 i
//        [128, 1152)   qs by 32-byte chunk pair g = 0..3, then row:
//                      qs[32 g, 32 g + 32) of row i at 128 + 256 g + 32 i
//  Q5_K  unit = one block column                          1408 B
//        [0, 128)      8 x 16 B headers (d, dmin, scales[12])  row i at 16 i
//        [128, 1152)   qs as for Q4_K
//        [1152, 1408)  8 x 32 B qh                             row i at 1152 + 32 i
//  Q6_K  unit = one block column                          1680 B
//        [0, 1024)     8 x 128 B ql                            row i at 128 i
//        [1024, 1536)  8 x 64 B qh                             row i at 1024 + 64 i
//        [1536, 1664)  8 x 16 B scales                         row i at 1536 + 16 i
//        [1664, 1680)  8 x 2 B d                               row i at 1664 + 2 i
//  IQ4_XS unit = one block column                         1088 B
//        [0, 1024)     8 x 128 B qs                            row i at 128 i
//        [1024, 1088)  8 x 8 B headers (d, scales_h, scales_l) row i at 1024 + 8 i
//  Q8_0  unit = four block columns (128 weights)          1088 B
//        [0, 1024)     8 rows x 4 blocks x 32 B qs             (i, k) at 128 i + 32 k
//        [1024, 1088)  8 rows x 4 blocks x 2 B d               (i, k) at 1024 + 8 i + 2 k
//
// Unit (t, u) starts at (t * units_per_row + u) * unit_bytes.  Rows past
// row_count in the last tile, and Q8_0 block columns past row_blocks in the
// last unit, are zero blocks (d = 0, so they contribute exactly 0).
//
// The Q4_K / Q5_K qs plane is ordered chunk pair first so that both of its
// readers get whole 128-byte lines per load: the M = 1 kernels read the 1 KiB
// plane with one 16-byte load per lane (lane l takes bytes 16 l, i.e. row
// (l / 2) % 8 and chunk 2 (l / 16) + l % 2), and the small-M MFMA kernels load
// their operands straight into registers, where a lane needs the same 16 bytes
// of 16 different rows: with one 128-byte row after another those loads touch
// a line per row and run at half the streaming rate (measured on gfx950 over
// 100 MB: 2.5-2.8 TB/s against 5.0-6.1 chunk pair first).
constexpr int kTileRows = 8;
constexpr int kLanesPerRow = 8;                    // GEMV: 8 lanes x 16 B per row and unit
constexpr int kWavesPerWG = 4;                     // GEMV workgroup = 4 waves ...
constexpr int kRowsPerWG = kWavesPerWG * kTileRows;  // ... = 32 output rows
constexpr int kQ4KUnit = kTileRows * kQ4KBytes;      // 1152
constexpr int kQ5KUnit = kTileRows * kQ5KBytes;      // 1408
constexpr int kQ5KTQh = 1152;
constexpr int kQ4KTQs = 128;
// Offset in a Q4_K / Q5_K unit of qs bytes [32 g, 32 g + 32) of row i.
constexpr int q4k_tqs(int i, int g) { return kQ4KTQs + 256 * g + 32 * i; }
constexpr int kQ6KUnit = kTileRows * kQ6KBytes;      // 1680
constexpr int kIQ4XSUnit = kTileRows * kIQ4XSBytes;  // 1088
constexpr int kIQ4XSTHdr = 1024;
constexpr int kQ80UnitBlocks = 4;
constexpr int kQ80Unit = kTileRows * kQ80UnitBlocks * kQ80Bytes;  // 1088

constexpr int kQ6KTQl = 0, kQ6KTQh = 1024, kQ6KTSc = 1536, kQ6KTD = 1664;
constexpr int kQ80TD = 1024;

static_assert(kQ4KUnit % 16 == 0 && kQ5KUnit % 16 == 0 && kQ6KUnit % 16 == 0 && kQ80Unit % 16 == 0 &&
                  kIQ4XSUnit % 16 == 0,
              "every tiled unit keeps 16-byte alignment");

inline int block_bytes(uint32_t type) {
    switch (type) {
        case kQ4_K: return kQ4KBytes;
        case kQ5_K: return kQ5KBytes;
        case kQ6_K: return kQ6KBytes;
        case kQ8_0: return kQ80Bytes;
        case kIQ4_XS: return kIQ4XSBytes;
        case kF16: return 2;
        case kF32: return 4;
        default: return 0;
    }
}

inline int block_elems(uint32_t type) {
    switch (type) {
        case kQ4_K: case kQ5_K: case kQ6_K: case kIQ4_XS: return 256;
        case kQ8_0: return 32;
        case kF16: case kF32: return 1;
        default: return 0;
    }
}

inline bool is_quant(uint32_t type) {
    return type == kQ4_K || type == kQ5_K || type == kQ6_K || type == kQ8_0 || type == kIQ4_XS;
}

inline int tiles_of(uint32_t rows) { return (int)((rows + kTileRows - 1) / kTileRows); }

inline int units_per_row(uint32_t type, uint32_t rb) {
    return type == kQ8_0 ? (int)((rb + kQ80UnitBlocks - 1) / kQ80UnitBlocks) : (int)rb;
}

inline int unit_bytes(uint32_t type) {
    switch (type) {
        case kQ4_K: return kQ4KUnit;
        case kQ5_K: return kQ5KUnit;
        case kQ6_K: return kQ6KUnit;
        case kQ8_0: return kQ80Unit;
        case kIQ4_XS: return kIQ4XSUnit;
        default: return 0;
    }
}

inline size_t tiled_bytes(uint32_t type, uint32_t rb, uint32_t rc) {
    if (!is_quant(type)) return 0;
    return (size_t)tiles_of(rc) * (size_t)units_per_row(type, rb) * (size_t)unit_bytes(type);
}

}  // namespace m27q
