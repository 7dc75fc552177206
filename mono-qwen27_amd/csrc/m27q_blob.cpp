// m27q_blob.cpp -- pack-time re-tiling of a .m27b weight blob.
//
// The reference's blob (include/mono27b_format.h:30-84, written by
// mono27b_write_stub_blob, src/mono27b_blob.cpp:378-438) is a header, a
// section table, a tokenizer section and a weights section: a section header,
// one entry per tensor, then the tensors' bytes (entry offsets are relative to
// the weights section).  Its loader uploads those bytes verbatim (lw(),
// exec:1695-1716).  m27q_retile_blob writes a copy whose quantized matrix
// entries hold the TILED layout instead, with the layout tag in the entry's
// reserved field (0 GGUF, 1 TILED) and each tensor 256-byte aligned; every
// other byte (header fields, tokenizer, non-matrix tensors) is copied.  The
// result still passes the reference's own blob validation and entry reads.
// The record layouts below must stay byte-identical to the reference's
// structs: they are the file format.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/m27q.h"
#include "m27q_layout.h"

using namespace m27q;

namespace {

constexpr uint32_t kBlobMagic = 0x4237324dU;     // "M27B"
constexpr uint32_t kWeightsMagic = 0x5754324dU;  // "M2TW"
constexpr uint32_t kSectionWeights = 2U;

struct BlobHeader {
    uint32_t magic, schema_version, section_count, reserved0;
    uint64_t file_bytes, tensor_table_offset, section_table_offset, tokenizer_offset, tokenizer_bytes;
    uint32_t max_ctx_hint, target_layers, draft_layers;
    char target_arch[16], draft_arch[16], target_quant[16], draft_quant[16];
};
struct BlobSection {
    uint32_t kind, reserved;
    uint64_t offset, bytes;
};
struct WeightsSection {
    uint32_t magic, version, entry_count, reserved;
};
struct WeightEntry {
    char name[64];
    uint32_t ggml_type, source_model, role, row_elems, row_count, reserved;
    uint64_t data_offset, data_bytes;
};
static_assert(sizeof(BlobHeader) == 136 && sizeof(BlobSection) == 24 && sizeof(WeightsSection) == 16 &&
                  sizeof(WeightEntry) == 104,
              "the .m27b record sizes");

constexpr uint64_t kAlign = 256;
constexpr size_t kCopyChunk = 64u << 20;

struct File {
    FILE *f = nullptr;
    explicit File(const char *path, const char *mode) : f(std::fopen(path, mode)) {}
    ~File() {
        if (f) std::fclose(f);
    }
    bool seek(uint64_t off) const { return std::fseek(f, (long)off, SEEK_SET) == 0; }
    bool read(void *p, size_t n) const { return n == 0 || std::fread(p, 1, n, f) == n; }
    bool write(const void *p, size_t n) const { return n == 0 || std::fwrite(p, 1, n, f) == n; }
};

// Copy n bytes from in (at off) to the current position of out.
bool copy_range(const File &in, uint64_t off, uint64_t n, const File &out) {
    std::vector<uint8_t> buf((size_t)std::min<uint64_t>(n, kCopyChunk));
    if (!in.seek(off)) return false;
    while (n) {
        const size_t c = (size_t)std::min<uint64_t>(n, buf.size());
        if (!in.read(buf.data(), c) || !out.write(buf.data(), c)) return false;
        n -= c;
    }
    return true;
}

bool zeros(const File &out, uint64_t n) {
    static const uint8_t z[kAlign] = {};
    while (n) {
        const size_t c = (size_t)std::min<uint64_t>(n, kAlign);
        if (!out.write(z, c)) return false;
        n -= c;
    }
    return true;
}

// A matrix entry whose bytes are whole GGUF rows of a type with a TILED form.
bool retilable(const WeightEntry &e) {
    if (e.reserved != M27Q_LAYOUT_GGUF || !is_quant(e.ggml_type) || e.row_elems == 0 || e.row_count == 0) return false;
    const int be = block_elems(e.ggml_type);
    if (e.row_elems % (uint32_t)be) return false;
    return e.data_bytes == (uint64_t)e.row_count * (e.row_elems / be) * block_bytes(e.ggml_type);
}

}  // namespace

extern "C" {

M27Q_API m27q_status m27q_retile_blob(const char *in_path, const char *out_path) {
    if (!in_path || !out_path) return M27Q_ERR_NULL;
    if (!std::strcmp(in_path, out_path)) return M27Q_ERR_IO;
    const File in(in_path, "rb");
    if (!in.f) return M27Q_ERR_IO;
    BlobHeader h;
    if (!in.read(&h, sizeof(h)) || h.magic != kBlobMagic || h.section_count == 0 || h.section_count > 64)
        return M27Q_ERR_IO;
    std::vector<BlobSection> secs(h.section_count);
    if (!in.seek(h.section_table_offset) || !in.read(secs.data(), secs.size() * sizeof(BlobSection)))
        return M27Q_ERR_IO;
    int wi = -1;
    for (int i = 0; i < (int)secs.size(); ++i)
        if (secs[i].kind == kSectionWeights) wi = i;
    if (wi < 0) return M27Q_ERR_IO;
    const BlobSection ws = secs[wi];
    // The weights section must be the file's tail (as mono27b_write_stub_blob
    // lays it out), and the section table must sit before it.
    if (ws.offset + ws.bytes != h.file_bytes || h.section_table_offset + secs.size() * sizeof(BlobSection) > ws.offset)
        return M27Q_ERR_IO;
    WeightsSection wh;
    if (!in.seek(ws.offset) || !in.read(&wh, sizeof(wh)) || wh.magic != kWeightsMagic || wh.entry_count == 0 ||
        wh.entry_count > (1u << 20))
        return M27Q_ERR_IO;
    std::vector<WeightEntry> ents(wh.entry_count), outs;
    if (!in.read(ents.data(), ents.size() * sizeof(WeightEntry))) return M27Q_ERR_IO;
    for (const WeightEntry &e : ents)
        if (e.data_offset + e.data_bytes > ws.bytes) return M27Q_ERR_IO;

    // New entry table: offsets relative to the weights section, 256-aligned.
    outs = ents;
    uint64_t pos = sizeof(WeightsSection) + ents.size() * sizeof(WeightEntry);
    for (WeightEntry &e : outs) {
        pos = (pos + kAlign - 1) / kAlign * kAlign;
        if (retilable(e)) {
            e.reserved = M27Q_LAYOUT_TILED;
            e.data_bytes = tiled_bytes(e.ggml_type, e.row_elems / block_elems(e.ggml_type), e.row_count);
        }
        e.data_offset = pos;
        pos += e.data_bytes;
    }
    BlobSection ws2 = ws;
    ws2.bytes = pos;
    BlobHeader h2 = h;
    h2.file_bytes = ws.offset + pos;
    std::vector<BlobSection> secs2 = secs;
    secs2[wi] = ws2;

    const File out(out_path, "wb");
    if (!out.f) return M27Q_ERR_IO;
    // Everything before the weights section, with the updated header and table.
    if (!copy_range(in, 0, ws.offset, out) || !out.seek(0) || !out.write(&h2, sizeof(h2)) ||
        !out.seek(h.section_table_offset) || !out.write(secs2.data(), secs2.size() * sizeof(BlobSection)) ||
        !out.seek(ws.offset) || !out.write(&wh, sizeof(wh)) || !out.write(outs.data(), outs.size() * sizeof(WeightEntry)))
        return M27Q_ERR_IO;
    uint64_t at = sizeof(WeightsSection) + outs.size() * sizeof(WeightEntry);
    std::vector<uint8_t> src, dst;
    for (size_t i = 0; i < ents.size(); ++i) {
        const WeightEntry &e = ents[i], &o = outs[i];
        if (!zeros(out, o.data_offset - at)) return M27Q_ERR_IO;
        if (o.reserved == M27Q_LAYOUT_TILED && e.reserved != M27Q_LAYOUT_TILED) {
            src.resize((size_t)e.data_bytes);
            dst.resize((size_t)o.data_bytes);
            const uint32_t rb = e.row_elems / block_elems(e.ggml_type);
            if (!in.seek(ws.offset + e.data_offset) || !in.read(src.data(), src.size())) return M27Q_ERR_IO;
            const m27q_status st = m27q_repack(e.ggml_type, rb, e.row_count, src.data(), dst.data());
            if (st != M27Q_OK) return st;
            if (!out.write(dst.data(), dst.size())) return M27Q_ERR_IO;
        } else if (!copy_range(in, ws.offset + e.data_offset, e.data_bytes, out)) {
            return M27Q_ERR_IO;
        }
        at = o.data_offset + o.data_bytes;
    }
    return std::fflush(out.f) == 0 ? M27Q_OK : M27Q_ERR_IO;
}

}  // extern "C"
