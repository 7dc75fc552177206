// Test harness (oracle side): C entry points over the reference's own .m27b
// writer, validator and entry reader (src/mono27b_blob.cpp, compiled from the
// reference checkout into oracle/_ref/ by oracle/Makefile).  Used only by
// tests/test_blob.py to make blobs and to check the packer's output.
#include <cstdio>
#include <cstring>
#include <string>

#include "mono27b_format.h"

extern "C" {

static void put_error(const std::string &e, char *err, int cap) {
    if (err && cap > 0) std::snprintf(err, (size_t)cap, "%s", e.c_str());
}

// entries: n records laid out as Mono27BWeightEntry; payload: the tensor bytes
// the entries' data_offset values point into (relative to the weights section).
int refblob_write(const char *path, int n, const void *entries, const unsigned char *payload, unsigned long long bytes,
                  char *err, int cap) {
    Mono27BTokenizerSection tok{};
    tok.vocab_size = 8;
    const unsigned char tok_bytes[16] = {'m', '2', '7', 'q', ' ', 't', 'e', 's', 't'};
    Mono27BWeightsSection ws{};
    ws.entry_count = (uint32_t)n;
    std::string e;
    const bool ok = mono27b_write_stub_blob(path, 4096, tok, tok_bytes, sizeof(tok_bytes), ws,
                                           (const Mono27BWeightEntry *)entries, payload, bytes, e);
    if (!ok) put_error(e, err, cap);
    return ok ? 0 : 1;
}

int refblob_validate(const char *path, char *err, int cap) {
    std::string e;
    const bool ok = mono27b_validate_blob_file(path, e);
    if (!ok) put_error(e, err, cap);
    return ok ? 0 : 1;
}

// Entries as mono27b_read_weights_section returns them (bounds-checked there).
int refblob_read_entries(const char *path, void *out, int cap, char *err, int errcap) {
    Mono27BWeightsSection ws{};
    std::string e;
    if (!mono27b_read_weights_section(path, ws, (Mono27BWeightEntry *)out, (size_t)cap, e)) {
        put_error(e, err, errcap);
        return -1;
    }
    return (int)ws.entry_count;
}

int refblob_entry_size() { return (int)sizeof(Mono27BWeightEntry); }
int refblob_weights_offset(const char *path) {
    Mono27BBlobSection s[4] = {};
    std::string e;
    if (!mono27b_read_blob_sections(path, s, 4, e)) return -1;
    for (const auto &x : s)
        if (x.kind == MONO27B_SECTION_WEIGHTS) return (int)x.offset;
    return -1;
}

}  // extern "C"
