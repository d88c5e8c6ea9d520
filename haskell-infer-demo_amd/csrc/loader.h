/*
 * loader.h - Host-side pieces of the INT4 load path: SHA-256, a small JSON reader, and the
 * weights.manifest.json schema (internal to the library; the C ABI is in include/w4a16.h).
 */
#ifndef W4A16_LOADER_H
#define W4A16_LOADER_H

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace w4a16 {

struct Sha256 {
    Sha256() { reset(); }
    void reset();
    void update(const void *data, size_t len);
    std::string hex(); /* finishes the digest; lowercase hex */

  private:
    void block(const uint8_t *p);
    uint32_t h[8];
    uint64_t total;
    uint8_t buf[64];
    size_t fill;
};

/* A parsed JSON value. Objects keep their members in document order. */
struct JValue {
    enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
    bool boolean = false;
    double number = 0.0;
    std::string text;
    std::vector<JValue> items;
    std::vector<std::pair<std::string, JValue>> members;

    const JValue *find(const char *key) const;
};

/* Manifest status codes, the reader's refusal classes (values as reference
 * csrc/include/quant_manifest.h:55-63). */
enum ManifestStatus {
    kManifestOk = 0,
    kManifestErrArg = 1,
    kManifestErrSyntax = 2,
    kManifestErrFormat = 3,
    kManifestErrShape = 4,
    kManifestErrIo = 5,
    kManifestErrHash = 6,
};

/* Parse a JSON document (RFC 8259 subset: ASCII strings, duplicate keys refused). */
int json_parse(const std::string &text, JValue *out);

struct Artifact {
    std::string file, dtype, sha256;
    long long bytes = 0;
    long long count = -1; /* scale element count; -1 for a packed payload */
};

struct Entry {
    std::string role;
    int role_index = -1;
    int layer = 0;
    long long n = 0, k = 0, group = 0;
    Artifact packed, scales;
};

struct PairEntry {
    std::string name;
    int layer = 0;
    std::string member_role[2];
    int member_role_index[2] = {-1, -1};
    long long n = 0, k = 0, group = 0;
    Artifact packed, scales;
};

struct Manifest {
    int version = 0;
    std::string converter_name;
    int converter_version = 0;
    std::string source_model_dir;
    std::vector<Entry> entries;
    std::vector<PairEntry> pairs;
    int int4_cells = 0, bf16_cells = 0;

    int find_entry(int layer, const char *role) const;
    int find_pair(const char *name, int layer) const;
};

/* Parse and validate a sidecar; returns a ManifestStatus, the reason via set_error. */
int manifest_parse(const std::string &json, Manifest *out);

/* Read root/artifact.file, requiring the recorded byte count, dtype and SHA-256. */
int artifact_read(const std::string &root, const Artifact &a, const char *want_dtype,
                  std::vector<uint8_t> *out);

}  // namespace w4a16

/* Grows the current device's split-K scratch to the worst case of every FFN call of 1..max_rows
 * rows at this hidden/intermediate (kernels.hip), so the store's forwards never allocate. */
int reserve_split_scratch(int max_rows, int hidden, int inter);

#endif /* W4A16_LOADER_H */
