/*
 * manifest.cpp - Reader and validator of the weights.manifest.json sidecar.
 *
 * The schema is the one the reference converter writes (reference
 * scripts/quantize_weights.py:219-318) and its reader enforces (reference csrc/quant_manifest.c);
 * the refusal classes and their status values are the reader's (quant_manifest.h:55-63), so a
 * caller that maps statuses sees the same behaviour. The document is parsed into a tree first
 * and then validated section by section in document order, which keeps the reference's rule
 * that "precision_map" and "pairs" must follow "entries" (quant_manifest.c:999-1024).
 */
#include <sys/stat.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "loader.h"

namespace w4a16 {

const JValue *JValue::find(const char *key) const {
    for (const auto &m : members)
        if (m.first == key) return &m.second;
    return nullptr;
}

/* ----------------------------------------------------------------------------------------- */
/* JSON                                                                                       */
/* ----------------------------------------------------------------------------------------- */

namespace {

constexpr int kMaxDepth = 32;
constexpr size_t kMaxEntries = 256; /* reference quant_manifest.h:47-51 */
constexpr size_t kMaxPairs = 128;

struct Parser {
    const char *p, *end, *begin;

    int err(const char *what) {
        return set_error(kManifestErrSyntax, "manifest: %s at byte %lld", what,
                         (long long)(p - begin));
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    int string(std::string *out) {
        if (p >= end || *p != '"') return err("expected a string");
        ++p;
        out->clear();
        while (p < end && *p != '"') {
            char ch = *p++;
            if ((unsigned char)ch < 0x20) return err("a control character inside a string");
            if (ch == '\\') {
                if (p >= end) return err("unterminated escape");
                const char e = *p++;
                switch (e) {
                    case '"': ch = '"'; break;
                    case '\\': ch = '\\'; break;
                    case '/': ch = '/'; break;
                    case 'b': ch = '\b'; break;
                    case 'f': ch = '\f'; break;
                    case 'n': ch = '\n'; break;
                    case 'r': ch = '\r'; break;
                    case 't': ch = '\t'; break;
                    case 'u': {
                        unsigned v = 0;
                        for (int i = 0; i < 4; ++i) {
                            if (p >= end) return err("truncated \\u escape");
                            const char hch = *p++;
                            int d = (hch >= '0' && hch <= '9') ? hch - '0'
                                    : (hch >= 'a' && hch <= 'f') ? hch - 'a' + 10
                                    : (hch >= 'A' && hch <= 'F') ? hch - 'A' + 10 : -1;
                            if (d < 0) return err("malformed \\u escape");
                            v = v * 16 + (unsigned)d;
                        }
                        /* the schema's strings are paths, role names and hex digests */
                        if (v > 0x7F) return err("a string outside ASCII");
                        ch = (char)v;
                        break;
                    }
                    default: return err("unknown escape");
                }
            }
            out->push_back(ch);
        }
        if (p >= end) return err("unterminated string");
        ++p;
        return kManifestOk;
    }
    int number(double *out) {
        const char *start = p;
        if (p < end && *p == '-') ++p;
        int digits = 0;
        while (p < end && *p >= '0' && *p <= '9') ++p, ++digits;
        if (p < end && *p == '.') {
            ++p;
            while (p < end && *p >= '0' && *p <= '9') ++p, ++digits;
        }
        if (!digits) return err("expected a value");
        if (p < end && (*p == 'e' || *p == 'E')) {
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            int ed = 0;
            while (p < end && *p >= '0' && *p <= '9') ++p, ++ed;
            if (!ed) return err("malformed exponent");
        }
        const std::string lit(start, (size_t)(p - start));
        char *stop = nullptr;
        errno = 0;
        *out = std::strtod(lit.c_str(), &stop);
        if (!stop || *stop != '\0' || errno == ERANGE) return err("malformed number");
        return kManifestOk;
    }
    int value(JValue *v, int depth) {
        if (depth > kMaxDepth) return err("nesting is too deep");
        ws();
        if (p >= end) return err("expected a value");
        const char ch = *p;
        if (ch == '"') {
            v->kind = JValue::kString;
            return string(&v->text);
        }
        if (ch == '{') {
            v->kind = JValue::kObject;
            ++p;
            ws();
            if (p < end && *p == '}') return ++p, kManifestOk;
            for (;;) {
                ws();
                std::string key;
                int st = string(&key);
                if (st) return st;
                for (const auto &m : v->members)
                    if (m.first == key) return set_error(kManifestErrSyntax, "manifest: duplicate key \"%s\"", key.c_str());
                ws();
                if (p >= end || *p != ':') return err("expected ':'");
                ++p;
                v->members.emplace_back(key, JValue());
                st = value(&v->members.back().second, depth + 1);
                if (st) return st;
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == '}') return ++p, kManifestOk;
                return err("expected ',' or '}'");
            }
        }
        if (ch == '[') {
            v->kind = JValue::kArray;
            ++p;
            ws();
            if (p < end && *p == ']') return ++p, kManifestOk;
            for (;;) {
                v->items.emplace_back();
                int st = value(&v->items.back(), depth + 1);
                if (st) return st;
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == ']') return ++p, kManifestOk;
                return err("expected ',' or ']'");
            }
        }
        auto word = [&](const char *w) {
            const size_t n = std::strlen(w);
            if ((size_t)(end - p) >= n && std::memcmp(p, w, n) == 0) { p += n; return true; }
            return false;
        };
        if (word("true")) { v->kind = JValue::kBool; v->boolean = true; return kManifestOk; }
        if (word("false")) { v->kind = JValue::kBool; v->boolean = false; return kManifestOk; }
        if (word("null")) { v->kind = JValue::kNull; return kManifestOk; }
        v->kind = JValue::kNumber;
        return number(&v->number);
    }
};

/* ---- typed field access: a missing field is a syntax error, a wrongly typed one too ------ */

int need(const JValue &obj, const char *key, const JValue **out, const char *where) {
    *out = obj.find(key);
    if (!*out) return set_error(kManifestErrSyntax, "manifest: %s is missing \"%s\"", where, key);
    return kManifestOk;
}

int as_int(const JValue &v, long long *out, const char *what) {
    if (v.kind != JValue::kNumber || v.number != std::floor(v.number) || std::fabs(v.number) > 9e15)
        return set_error(kManifestErrSyntax, "manifest: %s is not an integer", what);
    *out = (long long)v.number;
    return kManifestOk;
}

int as_str(const JValue &v, std::string *out, const char *what) {
    if (v.kind != JValue::kString) return set_error(kManifestErrSyntax, "manifest: %s is not a string", what);
    *out = v.text;
    return kManifestOk;
}

int as_shape2(const JValue &v, long long *n, long long *k, const char *what) {
    if (v.kind != JValue::kArray || v.items.size() != 2)
        return set_error(kManifestErrSyntax, "manifest: %s is not a two-element shape", what);
    int st = as_int(v.items[0], n, what);
    return st ? st : as_int(v.items[1], k, what);
}

bool lower_hex64(const std::string &s) {
    if (s.size() != 64) return false;
    for (char c : s)
        if (!((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'))) return false;
    return true;
}

/* {"bytes", "count" (scales only), "dtype", "file", "sha256"} */
int parse_artifact(const JValue &v, Artifact *a, bool scale, const std::string &where) {
    if (v.kind != JValue::kObject)
        return set_error(kManifestErrSyntax, "manifest: %s artifact is not an object", where.c_str());
    const JValue *f;
    int st;
    if ((st = need(v, "bytes", &f, where.c_str())) || (st = as_int(*f, &a->bytes, "bytes"))) return st;
    if ((st = need(v, "dtype", &f, where.c_str())) || (st = as_str(*f, &a->dtype, "dtype"))) return st;
    if ((st = need(v, "file", &f, where.c_str())) || (st = as_str(*f, &a->file, "file"))) return st;
    if ((st = need(v, "sha256", &f, where.c_str())) || (st = as_str(*f, &a->sha256, "sha256"))) return st;
    const JValue *count = v.find("count");
    if (scale && !count)
        return set_error(kManifestErrSyntax, "manifest: %s scale artifact has no count", where.c_str());
    if (!scale && count)
        return set_error(kManifestErrSyntax, "manifest: %s packed payload carries a count",
                         where.c_str());
    a->count = -1;
    if (count && (st = as_int(*count, &a->count, "count"))) return st;
    return kManifestOk;
}

/* The artifact's own rules (reference quant_manifest.c:340-362). */
int require_artifact(const Artifact &a, const char *dtype, const std::string &where, bool scale) {
    if (!lower_hex64(a.sha256))
        return set_error(kManifestErrFormat, "manifest: %s has a malformed sha256", where.c_str());
    if (a.bytes <= 0)
        return set_error(kManifestErrFormat, "manifest: %s has a nonpositive byte count", where.c_str());
    if (a.file.empty()) return set_error(kManifestErrFormat, "manifest: %s has no file", where.c_str());
    if (a.dtype != dtype)
        return set_error(kManifestErrFormat, "manifest: %s is %s, the frozen format is %s",
                         where.c_str(), a.dtype.c_str(), dtype);
    if (scale != (a.count >= 0))
        return set_error(kManifestErrFormat, "manifest: %s %s a scale count", where.c_str(),
                         scale ? "is missing" : "carries");
    return kManifestOk;
}

int parse_format(const JValue &v) {
    if (v.kind != JValue::kObject) return set_error(kManifestErrSyntax, "manifest: format is not an object");
    static const char *const keys[] = {"name", "abi_version", "group", "qmin", "qmax",
                                       "zero_point", "invalid_code", "packed_dtype", "scale_dtype"};
    for (const char *k : keys)
        if (!v.find(k)) return set_error(kManifestErrSyntax, "manifest: the format block is incomplete");
    long long abi = 0, group = 0, qmin = 0, qmax = 0, zero = 0, invalid = 0;
    std::string pd, sd, name;
    int st;
    if ((st = as_str(*v.find("name"), &name, "format name")) ||
        (st = as_int(*v.find("abi_version"), &abi, "abi_version")) ||
        (st = as_int(*v.find("group"), &group, "group")) ||
        (st = as_int(*v.find("qmin"), &qmin, "qmin")) || (st = as_int(*v.find("qmax"), &qmax, "qmax")) ||
        (st = as_int(*v.find("zero_point"), &zero, "zero_point")) ||
        (st = as_int(*v.find("invalid_code"), &invalid, "invalid_code")) ||
        (st = as_str(*v.find("packed_dtype"), &pd, "packed_dtype")) ||
        (st = as_str(*v.find("scale_dtype"), &sd, "scale_dtype")))
        return st;
    if (abi != 1)
        return set_error(kManifestErrFormat, "manifest: format abi_version %lld, this reader speaks 1", abi);
    if (group != W4A16_GROUP || qmin != -7 || qmax != 7 || zero != 0 || invalid != -8)
        return set_error(kManifestErrFormat,
                         "manifest: the format block is not the frozen format (group %lld, q [%lld, "
                         "%lld], zero_point %lld, invalid_code %lld)", group, qmin, qmax, zero, invalid);
    if (pd != "u8" || sd != "bf16")
        return set_error(kManifestErrFormat, "manifest: packed/scales dtype %s/%s, the frozen format is u8/bf16",
                         pd.c_str(), sd.c_str());
    return kManifestOk;
}

int check_entry(const Entry &e) {
    if (e.role.empty()) return set_error(kManifestErrFormat, "manifest: an entry has no role");
    if (e.layer < 0) return set_error(kManifestErrFormat, "manifest: %s has a negative layer", e.role.c_str());
    long long pbytes = 0, nscales = 0;
    if (w4a16_layout_init(e.n, e.k, e.group, &pbytes, &nscales) != W4A16_OK)
        return set_error(kManifestErrShape, "manifest: %s layer %d is not a shape the format holds: [%lld, %lld] group %lld",
                         e.role.c_str(), e.layer, e.n, e.k, e.group);
    char buf[160];
    std::snprintf(buf, sizeof(buf), "%s layer %d", e.role.c_str(), e.layer);
    const std::string where(buf);
    int st = require_artifact(e.packed, "u8", where, false);
    if (st) return st;
    if ((st = require_artifact(e.scales, "bf16", where, true))) return st;
    if (e.packed.bytes != pbytes)
        return set_error(kManifestErrShape, "manifest: %s records %lld packed bytes, the shape holds %lld",
                         where.c_str(), e.packed.bytes, pbytes);
    if (e.scales.count != nscales)
        return set_error(kManifestErrShape, "manifest: %s records %lld scales, the shape holds %lld",
                         where.c_str(), e.scales.count, nscales);
    if (e.scales.bytes != 2 * e.scales.count)
        return set_error(kManifestErrShape, "manifest: %s records %lld scale bytes for %lld scales",
                         where.c_str(), e.scales.bytes, e.scales.count);
    return kManifestOk;
}

int parse_entries(const JValue &v, Manifest *m) {
    if (v.kind != JValue::kArray) return set_error(kManifestErrSyntax, "manifest: entries is not an array");
    if (v.items.empty()) return set_error(kManifestErrFormat, "manifest: entries is empty");
    if (v.items.size() > kMaxEntries)
        return set_error(kManifestErrFormat, "manifest: more than %zu entries", kMaxEntries);
    for (const JValue &item : v.items) {
        if (item.kind != JValue::kObject) return set_error(kManifestErrSyntax, "manifest: an entry is not an object");
        static const char *const req[] = {"role", "layer", "logical_shape", "packed", "scales", "group"};
        for (const char *k : req)
            if (!item.find(k))
                return set_error(kManifestErrSyntax, "manifest: an entry is missing one of role/layer/"
                                 "logical_shape/packed/scales/group");
        Entry e;
        long long layer = 0, ri = -1;
        int st;
        if ((st = as_str(*item.find("role"), &e.role, "role")) ||
            (st = as_int(*item.find("layer"), &layer, "layer")) ||
            (st = as_shape2(*item.find("logical_shape"), &e.n, &e.k, "logical_shape")) ||
            (st = as_int(*item.find("group"), &e.group, "group")))
            return st;
        e.layer = (int)layer;
        if (const JValue *r = item.find("role_index")) {
            if ((st = as_int(*r, &ri, "role_index"))) return st;
        }
        e.role_index = (int)ri;
        if ((st = parse_artifact(*item.find("packed"), &e.packed, false, e.role)) ||
            (st = parse_artifact(*item.find("scales"), &e.scales, true, e.role)))
            return st;
        if (const JValue *axis = item.find("group_axis")) {
            std::string a;
            if ((st = as_str(*axis, &a, "group_axis"))) return st;
            if (a != "k")
                return set_error(kManifestErrFormat, "manifest: the group axis is %s, the format groups K", a.c_str());
        }
        if ((st = check_entry(e))) return st;
        m->entries.push_back(e);
    }
    return kManifestOk;
}

/* A precision cell per (layer, role); every entry is an int4 cell and only entries are
 * (reference quant_manifest.c:715-810). */
int parse_precision_map(const JValue &v, Manifest *m) {
    if (v.kind != JValue::kArray) return set_error(kManifestErrSyntax, "manifest: precision_map is not an array");
    if (v.items.empty()) return set_error(kManifestErrFormat, "manifest: the precision map is empty");
    std::vector<char> seen(m->entries.size(), 0);
    for (const JValue &cell : v.items) {
        if (cell.kind != JValue::kObject || !cell.find("role") || !cell.find("layer") || !cell.find("precision"))
            return set_error(kManifestErrSyntax, "manifest: a precision cell is missing role/layer/precision");
        std::string role, prec;
        long long layer = 0;
        int st;
        if ((st = as_str(*cell.find("role"), &role, "role")) || (st = as_int(*cell.find("layer"), &layer, "layer")) ||
            (st = as_str(*cell.find("precision"), &prec, "precision")))
            return st;
        if (prec == "int4") {
            const int idx = m->find_entry((int)layer, role.c_str());
            if (idx < 0)
                return set_error(kManifestErrShape, "manifest: the precision map calls %s layer %lld int4, "
                                 "which has no entry", role.c_str(), layer);
            if (seen[idx]) return set_error(kManifestErrShape, "manifest: %s layer %lld appears twice as int4", role.c_str(), layer);
            seen[idx] = 1;
            ++m->int4_cells;
        } else if (prec == "bf16") {
            ++m->bf16_cells;
        } else {
            return set_error(kManifestErrFormat, "manifest: a precision cell is %s, expected int4 or bf16", prec.c_str());
        }
    }
    for (size_t i = 0; i < seen.size(); ++i)
        if (!seen[i])
            return set_error(kManifestErrShape, "manifest: %s layer %d has an entry but no int4 precision cell",
                             m->entries[i].role.c_str(), m->entries[i].layer);
    return kManifestOk;
}

/* A pair is its members' rows, in the recorded order (reference quant_manifest.c:520-576). */
int check_pair(const Manifest &m, const PairEntry &p) {
    char buf[200];
    std::snprintf(buf, sizeof(buf), "pair %s layer %d", p.name.c_str(), p.layer);
    const std::string where(buf);
    int st = require_artifact(p.packed, "u8", where, false);
    if (st || (st = require_artifact(p.scales, "bf16", where, true))) return st;
    if (p.n <= 0 || p.k <= 0) return set_error(kManifestErrShape, "manifest: %s has a nonpositive shape", where.c_str());
    long long rows = 0, bytes = 0, scales = 0, k = -1;
    for (int i = 0; i < 2; ++i) {
        const int idx = m.find_entry(p.layer, p.member_role[i].c_str());
        if (idx < 0)
            return set_error(kManifestErrShape, "manifest: %s names member %s, which is not an entry of layer %d",
                             where.c_str(), p.member_role[i].c_str(), p.layer);
        const Entry &e = m.entries[idx];
        if (p.member_role_index[i] >= 0 && p.member_role_index[i] != e.role_index)
            return set_error(kManifestErrShape, "manifest: %s records member %s as role_index %d, the entry is %d",
                             where.c_str(), e.role.c_str(), p.member_role_index[i], e.role_index);
        if (k < 0) k = e.k;
        else if (e.k != k)
            return set_error(kManifestErrShape, "manifest: %s concatenates members of different K", where.c_str());
        rows += e.n;
        bytes += e.packed.bytes;
        scales += e.scales.count;
    }
    if (p.k != k || p.n != rows)
        return set_error(kManifestErrShape, "manifest: %s is [%lld, %lld], its members are [%lld, %lld]",
                         where.c_str(), p.n, p.k, rows, k);
    if (p.packed.bytes != bytes)
        return set_error(kManifestErrShape, "manifest: %s records %lld packed bytes, its members hold %lld",
                         where.c_str(), p.packed.bytes, bytes);
    if (p.scales.count != scales || p.scales.bytes != 2 * scales)
        return set_error(kManifestErrShape, "manifest: %s records %lld scales, its members hold %lld",
                         where.c_str(), p.scales.count, scales);
    if (p.group != W4A16_GROUP)
        return set_error(kManifestErrFormat, "manifest: %s groups %lld, the format groups %d", where.c_str(),
                         p.group, W4A16_GROUP);
    return kManifestOk;
}

int parse_pairs(const JValue &v, Manifest *m) {
    if (v.kind != JValue::kArray) return set_error(kManifestErrSyntax, "manifest: pairs is not an array");
    if (v.items.size() > kMaxPairs) return set_error(kManifestErrFormat, "manifest: more than %zu pairs", kMaxPairs);
    for (const JValue &item : v.items) {
        static const char *const req[] = {"name", "layer", "members", "logical_shape", "packed", "scales", "group"};
        if (item.kind != JValue::kObject) return set_error(kManifestErrSyntax, "manifest: a pair is not an object");
        for (const char *k : req)
            if (!item.find(k))
                return set_error(kManifestErrSyntax, "manifest: a pair is missing one of name/layer/members/"
                                 "logical_shape/packed/scales/group");
        PairEntry p;
        long long layer = 0;
        int st;
        if ((st = as_str(*item.find("name"), &p.name, "name")) || (st = as_int(*item.find("layer"), &layer, "layer")) ||
            (st = as_shape2(*item.find("logical_shape"), &p.n, &p.k, "logical_shape")) ||
            (st = as_int(*item.find("group"), &p.group, "group")))
            return st;
        p.layer = (int)layer;
        const JValue &mem = *item.find("members");
        if (mem.kind != JValue::kArray || mem.items.size() != 2)
            return set_error(kManifestErrSyntax, "manifest: a pair does not have two members");
        for (int i = 0; i < 2; ++i) {
            const JValue &mi = mem.items[i];
            if (mi.kind != JValue::kObject || !mi.find("role"))
                return set_error(kManifestErrSyntax, "manifest: a pair member has no role");
            if ((st = as_str(*mi.find("role"), &p.member_role[i], "member role"))) return st;
            if (const JValue *ri = mi.find("role_index")) {
                long long v2 = -1;
                if ((st = as_int(*ri, &v2, "member role_index"))) return st;
                p.member_role_index[i] = (int)v2;
            }
        }
        if ((st = parse_artifact(*item.find("packed"), &p.packed, false, p.name)) ||
            (st = parse_artifact(*item.find("scales"), &p.scales, true, p.name)))
            return st;
        if ((st = check_pair(*m, p))) return st;
        m->pairs.push_back(p);
    }
    return kManifestOk;
}

}  // namespace

int json_parse(const std::string &text, JValue *out) {
    Parser ps{text.data(), text.data() + text.size(), text.data()};
    *out = JValue();
    int st = ps.value(out, 0);
    if (st) return st;
    ps.ws();
    if (ps.p != ps.end) return ps.err("trailing bytes after the document");
    return kManifestOk;
}

int Manifest::find_entry(int layer, const char *role) const {
    for (size_t i = 0; i < entries.size(); ++i)
        if (entries[i].layer == layer && entries[i].role == role) return (int)i;
    return -1;
}

int Manifest::find_pair(const char *name, int layer) const {
    for (size_t i = 0; i < pairs.size(); ++i)
        if (pairs[i].layer == layer && pairs[i].name == name) return (int)i;
    return -1;
}

int manifest_parse(const std::string &json, Manifest *out) {
    *out = Manifest();
    JValue doc;
    int st = json_parse(json, &doc);
    if (st) return st;
    if (doc.kind != JValue::kObject) return set_error(kManifestErrSyntax, "manifest: the document is not an object");
    if (doc.members.empty()) return set_error(kManifestErrSyntax, "manifest: the document is empty");
    bool seen_version = false, seen_format = false, seen_conv = false, seen_source = false;
    bool seen_entries = false, seen_prec = false;
    for (const auto &kv : doc.members) {
        const std::string &key = kv.first;
        const JValue &v = kv.second;
        if (key == "manifest_version") {
            long long ver = 0;
            if ((st = as_int(v, &ver, "manifest_version"))) return st;
            out->version = (int)ver;
            seen_version = true;
        } else if (key == "format") {
            if ((st = parse_format(v))) return st;
            seen_format = true;
        } else if (key == "converter") {
            if (v.kind != JValue::kObject) return set_error(kManifestErrSyntax, "manifest: converter is not an object");
            if (const JValue *n = v.find("name"))
                if ((st = as_str(*n, &out->converter_name, "converter name"))) return st;
            if (const JValue *n = v.find("version")) {
                long long cv = 0;
                if ((st = as_int(*n, &cv, "converter version"))) return st;
                out->converter_version = (int)cv;
            }
            seen_conv = true;
        } else if (key == "source") {
            if (v.kind != JValue::kObject) return set_error(kManifestErrSyntax, "manifest: source is not an object");
            if (const JValue *d = v.find("model_dir"))
                if ((st = as_str(*d, &out->source_model_dir, "model_dir"))) return st;
            seen_source = true;
        } else if (key == "entries") {
            if ((st = parse_entries(v, out))) return st;
            seen_entries = true;
        } else if (key == "precision_map") {
            if (!seen_entries)
                return set_error(kManifestErrSyntax, "manifest: precision_map precedes entries, so it cannot be checked against them");
            if ((st = parse_precision_map(v, out))) return st;
            seen_prec = true;
        } else if (key == "pairs") {
            if (!seen_entries)
                return set_error(kManifestErrSyntax, "manifest: pairs precede entries, so a pair cannot be checked against its members");
            if ((st = parse_pairs(v, out))) return st;
        }
    }
    if (!seen_version || !seen_format || !seen_conv || !seen_source || !seen_entries || !seen_prec)
        return set_error(kManifestErrSyntax, "manifest: missing one of manifest_version/format/converter/source/entries/precision_map");
    if (out->version != 1) return set_error(kManifestErrFormat, "manifest: version %d, this reader speaks 1", out->version);
    if (out->converter_name.empty() || out->converter_version <= 0)
        return set_error(kManifestErrFormat, "manifest: the converter is unnamed or unversioned");
    if (out->source_model_dir.empty()) return set_error(kManifestErrFormat, "manifest: no source model directory");
    if ((int)out->entries.size() != out->int4_cells)
        return set_error(kManifestErrShape, "manifest: %d int4 cells for %zu entries", out->int4_cells, out->entries.size());
    return kManifestOk;
}

/* reference csrc/quant_manifest.c:1085-1139 */
int artifact_read(const std::string &root, const Artifact &a, const char *want_dtype,
                  std::vector<uint8_t> *out) {
    out->clear();
    if (want_dtype && a.dtype != want_dtype)
        return set_error(kManifestErrFormat, "manifest: %s is %s, expected %s", a.file.c_str(), a.dtype.c_str(), want_dtype);
    const std::string path = root + "/" + a.file;
    struct stat info;
    if (stat(path.c_str(), &info) != 0)
        return set_error(kManifestErrIo, "manifest: %s: %s", path.c_str(), std::strerror(errno));
    if ((long long)info.st_size != a.bytes)
        return set_error(kManifestErrIo, "manifest: %s is %lld bytes, the manifest records %lld", path.c_str(),
                         (long long)info.st_size, a.bytes);
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) return set_error(kManifestErrIo, "manifest: %s: %s", path.c_str(), std::strerror(errno));
    std::vector<uint8_t> buf((size_t)a.bytes);
    const size_t got = std::fread(buf.data(), 1, buf.size(), f);
    std::fclose(f);
    if (got != buf.size())
        return set_error(kManifestErrIo, "manifest: %s read %zu of %lld bytes", path.c_str(), got, a.bytes);
    Sha256 h;
    h.update(buf.data(), buf.size());
    const std::string digest = h.hex();
    if (digest != a.sha256)
        return set_error(kManifestErrHash, "manifest: %s hashes to %s, the manifest records %s", path.c_str(),
                         digest.c_str(), a.sha256.c_str());
    out->swap(buf);
    return kManifestOk;
}

}  // namespace w4a16

using namespace w4a16;

extern "C" int w4a16_manifest_check(const char *json, int *entries, int *pairs) {
    if (!json) return set_error(kManifestErrArg, "manifest: null argument");
    Manifest m;
    const int st = manifest_parse(std::string(json), &m);
    if (st) return st;
    if (entries) *entries = (int)m.entries.size();
    if (pairs) *pairs = (int)m.pairs.size();
    return kManifestOk;
}

extern "C" int w4a16_artifact_verify(const char *root, const char *file, const char *dtype,
                                     long long bytes, const char *sha256_hex,
                                     const char *want_dtype) {
    if (!root || !file || !dtype || !sha256_hex) return set_error(kManifestErrArg, "manifest: null argument");
    Artifact a;
    a.file = file;
    a.dtype = dtype;
    a.bytes = bytes;
    a.sha256 = sha256_hex;
    std::vector<uint8_t> data;
    return artifact_read(root, a, want_dtype, &data);
}
