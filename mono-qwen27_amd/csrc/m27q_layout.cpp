// m27q_layout.cpp -- host-side pack-time re-tiling (GGUF rows <-> TILED).
//
// The reference uploads raw GGUF bytes verbatim (lw(), exec:1695-1716).  This
// packer moves the same bytes into the TILED layout described in
// m27q_layout.h; it is byte-preserving per block and m27q_unpack inverts it.
#include <cstring>

#include "../../include/m27q.h"
#include "m27q_layout.h"

using namespace m27q;

namespace {

// Copy one GGUF block <-> its slots in a tiled unit.  dir = true: GGUF -> tiled.
// The 128 qs bytes of row i <-> their four 32-byte chunk pairs in the unit.
void move_qs_pairs(uint8_t *unit, int i, uint8_t *qs, bool to_tiled) {
    for (int g = 0; g < 4; ++g) {
        if (to_tiled) std::memcpy(unit + q4k_tqs(i, g), qs + 32 * g, 32);
        else std::memcpy(qs + 32 * g, unit + q4k_tqs(i, g), 32);
    }
}

void move_q4k(uint8_t *unit, int i, uint8_t *blk, bool to_tiled) {
    uint8_t *hdr = unit + 16 * i;
    if (to_tiled) std::memcpy(hdr, blk, kQ4KHdr);
    else std::memcpy(blk, hdr, kQ4KHdr);
    move_qs_pairs(unit, i, blk + kQ4KHdr, to_tiled);
}

void move_q5k(uint8_t *unit, int i, uint8_t *blk, bool to_tiled) {
    uint8_t *hdr = unit + 16 * i, *qh = unit + kQ5KTQh + 32 * i;
    if (to_tiled) {
        std::memcpy(hdr, blk, kQ4KHdr);
        std::memcpy(qh, blk + kQ5KQh, 32);
    } else {
        std::memcpy(blk, hdr, kQ4KHdr);
        std::memcpy(blk + kQ5KQh, qh, 32);
    }
    move_qs_pairs(unit, i, blk + kQ5KQs, to_tiled);
}

void move_q6k(uint8_t *unit, int i, uint8_t *blk, bool to_tiled) {
    struct Piece { int tiled, gguf, len; };
    const Piece pieces[4] = {
        {kQ6KTQl + 128 * i, kQ6KQl, 128},
        {kQ6KTQh + 64 * i, kQ6KQh, 64},
        {kQ6KTSc + 16 * i, kQ6KSc, 16},
        {kQ6KTD + 2 * i, kQ6KD, 2},
    };
    for (const Piece &p : pieces) {
        if (to_tiled) std::memcpy(unit + p.tiled, blk + p.gguf, p.len);
        else std::memcpy(blk + p.gguf, unit + p.tiled, p.len);
    }
}

void move_iq4xs(uint8_t *unit, int i, uint8_t *blk, bool to_tiled) {
    uint8_t *qs = unit + 128 * i, *hdr = unit + kIQ4XSTHdr + 8 * i;
    if (to_tiled) {
        std::memcpy(hdr, blk, kIQ4XSQs);
        std::memcpy(qs, blk + kIQ4XSQs, 128);
    } else {
        std::memcpy(blk, hdr, kIQ4XSQs);
        std::memcpy(blk + kIQ4XSQs, qs, 128);
    }
}

void move_q80(uint8_t *unit, int i, int k, uint8_t *blk, bool to_tiled) {
    uint8_t *qs = unit + 128 * i + 32 * k, *d = unit + kQ80TD + 8 * i + 2 * k;
    if (to_tiled) {
        std::memcpy(d, blk, 2);
        std::memcpy(qs, blk + 2, 32);
    } else {
        std::memcpy(blk, d, 2);
        std::memcpy(blk + 2, qs, 32);
    }
}

m27q_status convert(uint32_t type, uint32_t rb, uint32_t rc, const void *src, void *dst, bool to_tiled) {
    if (!src || !dst) return M27Q_ERR_NULL;
    if (!is_quant(type)) return M27Q_ERR_TYPE;
    if (rb == 0 || rc == 0 || rb > (1u << 20)) return M27Q_ERR_SHAPE;
    const size_t bb = (size_t)block_bytes(type);
    const size_t row_bytes = bb * rb;
    const int upr = units_per_row(type, rb);
    const size_t ub = (size_t)unit_bytes(type);
    uint8_t *tiled = (uint8_t *)(to_tiled ? dst : src);
    uint8_t *gguf = (uint8_t *)(to_tiled ? src : dst);
    if (to_tiled) std::memset(tiled, 0, tiled_bytes(type, rb, rc));  // padding rows / blocks
    for (uint32_t r = 0; r < rc; ++r) {
        const int t = (int)(r / kTileRows), i = (int)(r % kTileRows);
        uint8_t *row = gguf + (size_t)r * row_bytes;
        for (uint32_t b = 0; b < rb; ++b) {
            uint8_t *blk = row + (size_t)b * bb;
            if (type == kQ8_0) {
                uint8_t *unit = tiled + ((size_t)t * upr + b / kQ80UnitBlocks) * ub;
                move_q80(unit, i, (int)(b % kQ80UnitBlocks), blk, to_tiled);
            } else {
                uint8_t *unit = tiled + ((size_t)t * upr + b) * ub;
                if (type == kQ4_K) move_q4k(unit, i, blk, to_tiled);
                else if (type == kQ5_K) move_q5k(unit, i, blk, to_tiled);
                else if (type == kIQ4_XS) move_iq4xs(unit, i, blk, to_tiled);
                else move_q6k(unit, i, blk, to_tiled);
            }
        }
    }
    return M27Q_OK;
}

}  // namespace

extern "C" {

M27Q_API const char *m27q_status_string(m27q_status s) {
    switch (s) {
        case M27Q_OK: return "ok";
        case M27Q_ERR_NULL: return "null pointer";
        case M27Q_ERR_SHAPE: return "invalid shape";
        case M27Q_ERR_TYPE: return "unsupported ggml type";
        case M27Q_ERR_LAYOUT: return "unsupported layout or misaligned buffer";
        case M27Q_ERR_SCRATCH: return "scratch buffer too small";
        case M27Q_ERR_RANGE: return "index out of range";
        case M27Q_ERR_HIP: return "HIP launch failed";
        case M27Q_ERR_IO: return "file read/write failed, or not a .m27b blob";
    }
    return "unknown status";
}

M27Q_API size_t m27q_row_size(uint32_t ggml_type, uint32_t ne) {
    const int be = block_elems(ggml_type), bb = block_bytes(ggml_type);
    if (!be || !bb || ne == 0 || ne % (uint32_t)be) return 0;
    return (size_t)(ne / (uint32_t)be) * (size_t)bb;
}

M27Q_API size_t m27q_weight_bytes(uint32_t ggml_type, uint32_t row_blocks, uint32_t row_count, uint32_t layout) {
    if (layout == M27Q_LAYOUT_GGUF) {
        const int bb = block_bytes(ggml_type);
        return bb ? (size_t)bb * row_blocks * row_count : 0;
    }
    if (layout == M27Q_LAYOUT_TILED) return tiled_bytes(ggml_type, row_blocks, row_count);
    return 0;
}

M27Q_API m27q_status m27q_repack(uint32_t ggml_type, uint32_t row_blocks, uint32_t row_count,
                                 const void *gguf_rows, void *tiled) {
    return convert(ggml_type, row_blocks, row_count, gguf_rows, tiled, true);
}

M27Q_API m27q_status m27q_unpack(uint32_t ggml_type, uint32_t row_blocks, uint32_t row_count,
                                 const void *tiled, void *gguf_rows) {
    return convert(ggml_type, row_blocks, row_count, tiled, gguf_rows, false);
}

}  // extern "C"
