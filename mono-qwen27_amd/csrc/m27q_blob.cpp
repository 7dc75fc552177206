// m27q_blob.cpp -- pack-time re-tiling of a .m27b weight blob.
//
// The reference's blob (include/mono27b_format.h:30-84, written by
// mono27b_write_stub_blob, src/mono27b_blob.cpp:378-438) is a header, a
// section table, a tokenizer section and a weights section: a section header,
// one entry per tensor, then the tensors' bytes (entry offsets are relative to
// the weights section).  Its loader uploads those bytes verbatim (lw(),
// exec:1695-1716).  m27q_retile_blob writes a copy whose quantized matrix
// entries hold the TILED layout instead, with the layout tag in the entry's
// reserved field (0 GGUF; TILED: 1 in the low 16 bits, the revision of the
// TILED byte order in the high 16) and each tensor 256-byte aligned; every
// other byte (header fields, tokenizer, non-matrix tensors) is copied.  The
// result still passes the reference's own blob validation and entry reads.
// m27q_blob_tensors / m27q_blob_load are the loader's side: the entry table
// as weight descriptors (the layout from the reserved field) and one
// tensor's bytes uploaded to caller-owned device memory, the role of lw()
// for a blob.  The record layouts below must stay byte-identical to the
// reference's structs: they are the file format.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>
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

// Revision 2: the Q4_K / Q5_K qs plane chunk pair first.  A TILED entry of
// another revision is listed with row_blocks 0, which m27q_blob_load refuses.
constexpr uint32_t kTiledRevision = 2;
constexpr uint32_t kTiledTag = M27Q_LAYOUT_TILED | kTiledRevision << 16;

constexpr uint32_t kMaxRows = 1u << 24;   // the products' row limit
constexpr uint32_t kMaxRowElems = 1u << 20;

// A matrix entry whose bytes are whole GGUF rows of a type with a TILED form.
bool retilable(const WeightEntry &e) {
    if (e.reserved != M27Q_LAYOUT_GGUF || !is_quant(e.ggml_type) || e.row_elems == 0 || e.row_count == 0 ||
        e.row_count > kMaxRows || e.row_elems > kMaxRowElems)
        return false;
    const int be = block_elems(e.ggml_type);
    if (e.row_elems % (uint32_t)be) return false;
    return e.data_bytes == (uint64_t)e.row_count * (e.row_elems / be) * block_bytes(e.ggml_type);
}

// The blob's table: header, section table, the weights section's header and
// entries.  Every offset read from the file is checked without overflow.
struct Table {
    BlobHeader h;
    std::vector<BlobSection> secs;
    int wi = -1;  // index of the weights section
    WeightsSection wh;
    std::vector<WeightEntry> ents;
};

m27q_status read_table(const File &in, Table &t) {
    if (!in.read(&t.h, sizeof(t.h)) || t.h.magic != kBlobMagic || t.h.section_count == 0 || t.h.section_count > 64)
        return M27Q_ERR_IO;
    t.secs.resize(t.h.section_count);
    if (!in.seek(t.h.section_table_offset) || !in.read(t.secs.data(), t.secs.size() * sizeof(BlobSection)))
        return M27Q_ERR_IO;
    for (int i = 0; i < (int)t.secs.size(); ++i)
        if (t.secs[i].kind == kSectionWeights) t.wi = i;
    if (t.wi < 0) return M27Q_ERR_IO;
    const BlobSection &ws = t.secs[t.wi];
    // The weights section is the file's tail (as mono27b_write_stub_blob lays
    // it out), and the section table sits before it.
    const uint64_t table_bytes = t.secs.size() * sizeof(BlobSection);
    if (ws.offset > t.h.file_bytes || ws.bytes != t.h.file_bytes - ws.offset || t.h.section_table_offset > ws.offset ||
        table_bytes > ws.offset - t.h.section_table_offset || ws.bytes < sizeof(WeightsSection))
        return M27Q_ERR_IO;
    if (!in.seek(ws.offset) || !in.read(&t.wh, sizeof(t.wh)) || t.wh.magic != kWeightsMagic ||
        t.wh.entry_count == 0 || t.wh.entry_count > (1u << 20) ||
        (uint64_t)t.wh.entry_count * sizeof(WeightEntry) > ws.bytes - sizeof(WeightsSection))
        return M27Q_ERR_IO;
    t.ents.resize(t.wh.entry_count);
    if (!in.read(t.ents.data(), t.ents.size() * sizeof(WeightEntry))) return M27Q_ERR_IO;
    for (const WeightEntry &e : t.ents)
        if (e.data_offset > ws.bytes || e.data_bytes > ws.bytes - e.data_offset) return M27Q_ERR_IO;
    return M27Q_OK;
}

m27q_status retile(const char *in_path, const char *out_path) {
    const File in(in_path, "rb");
    if (!in.f) return M27Q_ERR_IO;
    Table t;
    if (const m27q_status st = read_table(in, t); st != M27Q_OK) return st;
    const BlobSection ws = t.secs[t.wi];
    const std::vector<WeightEntry> &ents = t.ents;

    // New entry table: offsets relative to the weights section, 256-aligned.
    std::vector<WeightEntry> outs = ents;
    uint64_t pos = sizeof(WeightsSection) + ents.size() * sizeof(WeightEntry);
    for (WeightEntry &e : outs) {
        pos = (pos + kAlign - 1) / kAlign * kAlign;
        if (retilable(e)) {
            e.reserved = kTiledTag;
            e.data_bytes = tiled_bytes(e.ggml_type, e.row_elems / block_elems(e.ggml_type), e.row_count);
        }
        e.data_offset = pos;
        pos += e.data_bytes;
    }
    BlobSection ws2 = ws;
    ws2.bytes = pos;
    BlobHeader h2 = t.h;
    h2.file_bytes = ws.offset + pos;
    std::vector<BlobSection> secs2 = t.secs;
    secs2[t.wi] = ws2;

    const File out(out_path, "wb");
    if (!out.f) return M27Q_ERR_IO;
    // Everything before the weights section, with the updated header and table.
    if (!copy_range(in, 0, ws.offset, out) || !out.seek(0) || !out.write(&h2, sizeof(h2)) ||
        !out.seek(t.h.section_table_offset) || !out.write(secs2.data(), secs2.size() * sizeof(BlobSection)) ||
        !out.seek(ws.offset) || !out.write(&t.wh, sizeof(t.wh)) ||
        !out.write(outs.data(), outs.size() * sizeof(WeightEntry)))
        return M27Q_ERR_IO;
    uint64_t at = sizeof(WeightsSection) + outs.size() * sizeof(WeightEntry);
    std::vector<uint8_t> src, dst;
    for (size_t i = 0; i < ents.size(); ++i) {
        const WeightEntry &e = ents[i], &o = outs[i];
        if (!zeros(out, o.data_offset - at)) return M27Q_ERR_IO;
        if (o.reserved == kTiledTag && e.reserved == M27Q_LAYOUT_GGUF) {
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

// Row blocks of an entry as the products count them (K for F32 / F16), as
// lw() sets WeightView::row_blocks (exec:1706-1707); 0 if the entry's bytes
// are not whole rows of its type in its layout.
uint32_t entry_row_blocks(const WeightEntry &e) {
    if (e.row_elems == 0 || e.row_count == 0 || e.row_count > kMaxRows || e.row_elems > kMaxRowElems) return 0;
    const int be = block_elems(e.ggml_type);
    if (be == 0 || e.row_elems % (uint32_t)be) return 0;
    const uint32_t rb = e.row_elems / (uint32_t)be;
    uint64_t want = 0;
    if (e.reserved == kTiledTag) {
        if (!is_quant(e.ggml_type)) return 0;
        want = tiled_bytes(e.ggml_type, rb, e.row_count);
    } else if (e.reserved == M27Q_LAYOUT_GGUF) {
        want = (uint64_t)e.row_count * rb * (uint64_t)block_bytes(e.ggml_type);
    }
    return want != 0 && e.data_bytes == want ? rb : 0;
}

m27q_status tensors(const char *path, m27q_blob_tensor *out, int cap, int *count) {
    const File in(path, "rb");
    if (!in.f) return M27Q_ERR_IO;
    Table t;
    if (const m27q_status st = read_table(in, t); st != M27Q_OK) return st;
    *count = (int)t.ents.size();
    for (int i = 0; i < (int)t.ents.size() && i < cap; ++i) {
        const WeightEntry &e = t.ents[i];
        m27q_blob_tensor &o = out[i];
        std::memset(&o, 0, sizeof(o));
        std::memcpy(o.name, e.name, sizeof(o.name));
        o.name[sizeof(o.name) - 1] = '\0';
        o.ggml_type = e.ggml_type;
        o.source_model = e.source_model;
        o.role = e.role;
        o.row_elems = e.row_elems;
        o.row_count = e.row_count;
        o.layout = e.reserved & 0xffffu;
        o.row_blocks = entry_row_blocks(e);
        o.file_offset = t.secs[t.wi].offset + e.data_offset;
        o.bytes = e.data_bytes;
    }
    return M27Q_OK;
}

m27q_status load(const char *path, const m27q_blob_tensor *t, void *dst, size_t dst_bytes, m27q_weight *w) {
    if (t->row_blocks == 0 || block_elems(t->ggml_type) == 0 || t->row_count == 0) return M27Q_ERR_TYPE;
    if (t->layout != M27Q_LAYOUT_GGUF && t->layout != M27Q_LAYOUT_TILED) return M27Q_ERR_LAYOUT;
    if (t->layout == M27Q_LAYOUT_TILED && (uintptr_t)dst % 16) return M27Q_ERR_LAYOUT;
    if (t->bytes != m27q_weight_bytes(t->ggml_type, t->row_blocks, t->row_count, t->layout)) return M27Q_ERR_SHAPE;
    if (dst_bytes < t->bytes) return M27Q_ERR_SHAPE;
    const File in(path, "rb");
    if (!in.f || !in.seek(t->file_offset)) return M27Q_ERR_IO;
    // Staged through host memory in chunks, as lw() copies its mapped bytes
    // with one synchronous cudaMemcpy (exec:1712).
    std::vector<uint8_t> buf((size_t)std::min<uint64_t>(t->bytes, kCopyChunk));
    for (uint64_t off = 0; off < t->bytes;) {
        const size_t c = (size_t)std::min<uint64_t>(t->bytes - off, buf.size());
        if (!in.read(buf.data(), c)) return M27Q_ERR_IO;
        if (hipMemcpy((uint8_t *)dst + off, buf.data(), c, hipMemcpyHostToDevice) != hipSuccess) return M27Q_ERR_HIP;
        off += c;
    }
    *w = m27q_weight{dst, t->ggml_type, t->row_blocks, t->row_count, t->layout};
    return M27Q_OK;
}

}  // namespace

extern "C" {

M27Q_API m27q_status m27q_retile_blob(const char *in_path, const char *out_path) {
    if (!in_path || !out_path) return M27Q_ERR_NULL;
    if (!std::strcmp(in_path, out_path)) return M27Q_ERR_IO;
    try {
        return retile(in_path, out_path);
    } catch (const std::bad_alloc &) {
        return M27Q_ERR_IO;
    }
}

M27Q_API m27q_status m27q_blob_tensors(const char *path, m27q_blob_tensor *out, int cap, int *count) {
    if (!path || !count || (cap > 0 && !out)) return M27Q_ERR_NULL;
    try {
        return tensors(path, out, cap, count);
    } catch (const std::bad_alloc &) {
        return M27Q_ERR_IO;
    }
}

M27Q_API m27q_status m27q_blob_load(const char *path, const m27q_blob_tensor *t, void *device_dst, size_t dst_bytes,
                                    m27q_weight *w) {
    if (!path || !t || !device_dst || !w) return M27Q_ERR_NULL;
    try {
        return load(path, t, device_dst, dst_bytes, w);
    } catch (const std::bad_alloc &) {
        return M27Q_ERR_IO;
    }
}

}  // extern "C"
