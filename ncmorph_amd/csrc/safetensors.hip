// Safetensors header and sharded-index reader and the direct bf16 upload
// (packages/safetensors/root.zig; the loader's weight path, src/loader.zig:
// 95-202, 339-342, without the widen to f32: tensor bytes go to the device
// as they are stored). Host code; the upload streams the mapped file through
// two pinned staging buffers on the context's stream.
//
// Checks, in the reference's order (root.zig:148-193): the 8-byte
// little-endian length prefix (>= 8 bytes, <= 100 000 000), the JSON slice
// present, valid UTF-8, a JSON object whose "__metadata__" (if any) maps to
// strings and whose other members are {"dtype", "shape", "data_offsets"}
// (non-negative integers; two offsets), known dtypes; then, in data-offset
// order, contiguous offsets from 0, shape products and bit sizes without
// overflow, whole bytes, byte sizes matching shapes, and the file size equal
// to prefix + header + data. A failure returns NCM_E_FORMAT and
// ncm_last_error() names the reference's error.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ncmorph_amd.h"
#include "status.h"

namespace {

// ------------------------------------------------------------------ JSON

struct JValue {
    enum Kind { Null, Bool, Int, Float, BigInt, String, Array, Object } kind = Null;
    int64_t i = 0;
    std::string s;
    std::vector<JValue> items;                              // Array
    std::vector<std::pair<std::string, JValue>> members;    // Object, in document order
    // A repeated key keeps its first position and its last value (the
    // behaviour of an insertion-ordered map that is assigned to). Keys are
    // compared as whole strings: a key may hold U+0000 (a "\u0000" escape),
    // so it must never be looked up through its c_str().
    const JValue* get(const std::string& key) const {
        for (size_t k = members.size(); k-- > 0;)
            if (members[k].first == key) return &members[k].second;
        return nullptr;
    }
};

// Strict RFC 8259 parser (no trailing commas, no comments, no leading zeros,
// no control characters in strings). Integers that fit int64 are Int, other
// integers BigInt, numbers with a fraction or exponent Float.
struct JParser {
    const char* p;
    const char* e;
    int depth = 0;
    bool ok = true;

    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail() { ok = false; return false; }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(e - p) < n || memcmp(p, w, n) != 0) return fail();
        p += n;
        return true;
    }
    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (e - p < 4) return fail();
        v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail();
        }
        return true;
    }
    bool str(std::string& out) {
        if (p >= e || *p != '"') return fail();
        ++p;
        while (p < e) {
            const unsigned char c = (unsigned char)*p;
            if (c == '"') { ++p; return true; }
            if (c < 0x20) return fail();
            if (c != '\\') { out += (char)c; ++p; continue; }
            ++p;
            if (p >= e) return fail();
            const char x = *p++;
            switch (x) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp <= 0xDBFF) {  // high surrogate: a low one follows
                        uint32_t lo;
                        if (e - p < 2 || p[0] != '\\' || p[1] != 'u') return fail();
                        p += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo > 0xDFFF) return fail();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                        return fail();
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail();
            }
        }
        return fail();
    }
    bool num(JValue& v) {
        const char* s0 = p;
        bool neg = false, frac = false;
        if (p < e && *p == '-') { neg = true; ++p; }
        if (p >= e || *p < '0' || *p > '9') return fail();
        if (*p == '0') {
            ++p;
        } else {
            while (p < e && *p >= '0' && *p <= '9') ++p;
        }
        const char* int_end = p;
        if (p < e && *p == '.') {
            ++p;
            if (p >= e || *p < '0' || *p > '9') return fail();
            while (p < e && *p >= '0' && *p <= '9') ++p;
            frac = true;
        }
        if (p < e && (*p == 'e' || *p == 'E')) {
            ++p;
            if (p < e && (*p == '+' || *p == '-')) ++p;
            if (p >= e || *p < '0' || *p > '9') return fail();
            while (p < e && *p >= '0' && *p <= '9') ++p;
            frac = true;
        }
        if (frac) { v.kind = JValue::Float; return true; }
        // Integer: int64 when it fits.
        const char* d = s0 + (neg ? 1 : 0);
        unsigned __int128 acc = 0;
        bool big = false;
        for (const char* q = d; q < int_end; ++q) {
            acc = acc * 10 + (unsigned)(*q - '0');
            if (acc > ((unsigned __int128)1 << 64)) { big = true; break; }
        }
        const unsigned __int128 lim = neg ? ((unsigned __int128)1 << 63) : (((unsigned __int128)1 << 63) - 1);
        if (big || acc > lim) { v.kind = JValue::BigInt; return true; }
        v.kind = JValue::Int;
        v.i = neg ? (int64_t)(-(__int128)acc) : (int64_t)acc;
        return true;
    }
    bool value(JValue& v) {
        if (++depth > 512) return fail();
        ws();
        if (p >= e) return fail();
        bool r;
        switch (*p) {
            case '{': r = object(v); break;
            case '[': r = array(v); break;
            case '"': v.kind = JValue::String; r = str(v.s); break;
            case 't': v.kind = JValue::Bool; v.i = 1; r = lit("true"); break;
            case 'f': v.kind = JValue::Bool; v.i = 0; r = lit("false"); break;
            case 'n': v.kind = JValue::Null; r = lit("null"); break;
            default: r = num(v); break;
        }
        --depth;
        return r;
    }
    bool array(JValue& v) {
        v.kind = JValue::Array;
        ++p;
        ws();
        if (p < e && *p == ']') { ++p; return true; }
        while (true) {
            v.items.emplace_back();
            if (!value(v.items.back())) return false;
            ws();
            if (p < e && *p == ',') { ++p; continue; }
            if (p < e && *p == ']') { ++p; return true; }
            return fail();
        }
    }
    bool object(JValue& v) {
        v.kind = JValue::Object;
        ++p;
        ws();
        if (p < e && *p == '}') { ++p; return true; }
        while (true) {
            ws();
            std::string key;
            if (!str(key)) return false;
            ws();
            if (p >= e || *p != ':') return fail();
            ++p;
            JValue val;
            if (!value(val)) return false;
            v.members.emplace_back(std::move(key), std::move(val));
            ws();
            if (p < e && *p == ',') { ++p; continue; }
            if (p < e && *p == '}') { ++p; return true; }
            return fail();
        }
    }
};

bool parse_json(const char* b, size_t n, JValue& out) {
    JParser jp{b, b + n};
    if (!jp.value(out)) return false;
    jp.ws();
    return jp.ok && jp.p == jp.e;
}

// Well-formed UTF-8: no overlong forms, no surrogates, nothing above U+10FFFF.
bool utf8_valid(const unsigned char* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const unsigned char c = s[i];
        if (c < 0x80) { ++i; continue; }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000))
            return false;
        if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += len;
    }
    return true;
}

// ------------------------------------------------------------- dtypes

// Names and bit sizes in the order of the reference's Dtype enum
// (root.zig:33-68, 75-98): the codes are that order.
struct DtypeEntry {
    const char* name;
    int bits;
};
const DtypeEntry kDtypes[] = {
    {"BOOL", 8},     {"U8", 8},      {"I8", 8},          {"U16", 16},         {"I16", 16},
    {"U32", 32},     {"I32", 32},    {"U64", 64},        {"I64", 64},         {"F4", 4},
    {"F6_E2M3", 6},  {"F6_E3M2", 6}, {"F8_E5M2", 8},     {"F8_E4M3", 8},      {"F8_E8M0", 8},
    {"F8_E4M3FNUZ", 8}, {"F8_E5M2FNUZ", 8}, {"F16", 16}, {"BF16", 16},        {"F32", 32},
    {"F64", 64},     {"C64", 64},
};
constexpr int kNumDtypes = (int)(sizeof(kDtypes) / sizeof(kDtypes[0]));

int dtype_code(const std::string& name) {
    for (int k = 0; k < kNumDtypes; ++k)
        if (name == kDtypes[k].name) return k;
    return -1;
}

struct Tensor {
    std::string name;
    int dtype;
    std::vector<uint64_t> shape;
    uint64_t begin, end;
};

int format_error(const char* what) {
    ncm_set_error_detail(what);
    return NCM_E_FORMAT;
}

bool non_negative(const JValue& v, uint64_t& out) {
    if (v.kind != JValue::Int || v.i < 0) return false;
    out = (uint64_t)v.i;
    return true;
}

}  // namespace

struct ncm_st_file {
    uint64_t header_len = 0, data_len = 0;
    std::vector<Tensor> tensors;  // data-offset order
    // Mapped file (ncm_st_open only).
    const unsigned char* map = nullptr;
    size_t map_len = 0;
};

struct ncm_st_index {
    std::vector<std::pair<std::string, std::string>> weight_map;  // tensor -> shard
    bool has_total = false;
    uint64_t total_size = 0;
};

namespace {

int parse_header(const unsigned char* bytes, size_t len, uint64_t file_size, ncm_st_file* f) {
    constexpr uint64_t kMaxHeader = 100000000ull;
    if (len < 8) return format_error("HeaderTooSmall");
    uint64_t hl = 0;
    for (int k = 7; k >= 0; --k) hl = (hl << 8) | bytes[k];
    if (hl > kMaxHeader) return format_error("HeaderTooLarge");
    if (len < 8 + hl) return format_error("InvalidHeaderLength");
    const unsigned char* js = bytes + 8;
    if (!utf8_valid(js, (size_t)hl)) return format_error("InvalidUtf8");
    JValue root;
    if (!parse_json((const char*)js, (size_t)hl, root)) return format_error("SyntaxError");
    if (root.kind != JValue::Object) return format_error("InvalidHeader");

    std::vector<Tensor> ts;
    for (size_t mi = 0; mi < root.members.size(); ++mi) {
        const auto& m = root.members[mi];
        bool seen = false;
        for (size_t k = 0; k < mi; ++k) seen = seen || root.members[k].first == m.first;
        if (seen) continue;  // handled at its first position, with its last value
        const JValue& v = *root.get(m.first);
        if (m.first == "__metadata__") {
            if (v.kind != JValue::Object) return format_error("InvalidHeader");
            for (const auto& mm : v.members)
                if (mm.second.kind != JValue::String) return format_error("InvalidHeader");
            continue;
        }
        if (v.kind != JValue::Object) return format_error("InvalidHeader");
        const JValue* dt = v.get("dtype");
        if (!dt || dt->kind != JValue::String) return format_error("InvalidHeader");
        const int code = dtype_code(dt->s);
        if (code < 0) return format_error("UnknownDtype");
        const JValue* sh = v.get("shape");
        if (!sh || sh->kind != JValue::Array) return format_error("InvalidHeader");
        Tensor t;
        t.name = m.first;
        t.dtype = code;
        for (const auto& it : sh->items) {
            uint64_t d;
            if (!non_negative(it, d)) return format_error("InvalidHeader");
            t.shape.push_back(d);
        }
        const JValue* off = v.get("data_offsets");
        if (!off || off->kind != JValue::Array) return format_error("InvalidHeader");
        if (off->items.size() != 2) return format_error("InvalidHeader");
        if (!non_negative(off->items[0], t.begin) || !non_negative(off->items[1], t.end))
            return format_error("InvalidHeader");
        ts.push_back(std::move(t));
    }
    std::stable_sort(ts.begin(), ts.end(), [](const Tensor& a, const Tensor& b) {
        return a.begin != b.begin ? a.begin < b.begin : a.end < b.end;
    });
    uint64_t expected = 0;
    for (const Tensor& t : ts) {
        if (t.begin != expected || t.end < t.begin) return format_error("InvalidOffsets");
        expected = t.end;
        uint64_t count = 1;
        for (uint64_t d : t.shape)
            if (__builtin_mul_overflow(count, d, &count)) return format_error("ShapeOverflow");
        uint64_t bits;
        if (__builtin_mul_overflow(count, (uint64_t)kDtypes[t.dtype].bits, &bits))
            return format_error("ShapeOverflow");
        if (bits % 8 != 0) return format_error("MisalignedBits");
        if (t.end - t.begin != bits / 8) return format_error("SizeMismatch");
    }
    if (8 + hl + expected != file_size) return format_error("FileSizeMismatch");
    f->header_len = hl;
    f->data_len = expected;
    f->tensors = std::move(ts);
    return NCM_OK;
}

bool plain_file_name(const std::string& s) {
    if (s.empty() || s == "." || s == "..") return false;
    for (char c : s)
        if (c == '/' || c == '\\' || c == 0) return false;
    return true;
}

void fill_info(const Tensor& t, ncm_st_tensor_t* out) {
    out->name = t.name.c_str();
    out->dtype = t.dtype;
    out->ndim = (int32_t)t.shape.size();
    for (int k = 0; k < NCM_ST_MAX_DIMS; ++k)
        out->shape[k] = k < (int)t.shape.size() ? t.shape[k] : 0;
    out->data_begin = t.begin;
    out->data_end = t.end;
}

}  // namespace

extern "C" {

int ncm_st_parse(const void* bytes, size_t len, uint64_t file_size, ncm_st_file_t** out) {
    if (!out || (len > 0 && !bytes)) return NCM_E_NULL;
    *out = nullptr;
    ncm_st_file* f = new (std::nothrow) ncm_st_file;
    if (!f) return NCM_E_NOMEM;
    const int rc = parse_header((const unsigned char*)bytes, len, file_size, f);
    if (rc) { delete f; return rc; }
    *out = f;
    return NCM_OK;
}

int ncm_st_open(const char* path, ncm_st_file_t** out) {
    if (!path || !out) return NCM_E_NULL;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) { ncm_set_error_detail(std::string("open: ") + strerror(errno)); return NCM_E_ARG; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return NCM_E_ARG; }
    const size_t size = (size_t)st.st_size;
    void* map = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
    close(fd);
    if (size && map == MAP_FAILED) { ncm_set_error_detail("mmap failed"); return NCM_E_NOMEM; }
    ncm_st_file* f = new (std::nothrow) ncm_st_file;
    if (!f) { if (map) munmap(map, size); return NCM_E_NOMEM; }
    const int rc = parse_header((const unsigned char*)map, size, size, f);
    if (rc) { if (map) munmap(map, size); delete f; return rc; }
    f->map = (const unsigned char*)map;
    f->map_len = size;
    *out = f;
    return NCM_OK;
}

int ncm_st_close(ncm_st_file_t* f) {
    if (!f) return NCM_E_NULL;
    if (f->map) munmap((void*)f->map, f->map_len);
    delete f;
    return NCM_OK;
}

int ncm_st_summary(const ncm_st_file_t* f, uint64_t* header_len, uint64_t* data_len,
                   int64_t* tensor_count) {
    if (!f) return NCM_E_NULL;
    if (header_len) *header_len = f->header_len;
    if (data_len) *data_len = f->data_len;
    if (tensor_count) *tensor_count = (int64_t)f->tensors.size();
    return NCM_OK;
}

int ncm_st_tensor(const ncm_st_file_t* f, int64_t index, ncm_st_tensor_t* out) {
    if (!f || !out) return NCM_E_NULL;
    if (index < 0 || index >= (int64_t)f->tensors.size()) return NCM_E_ARG;
    const Tensor& t = f->tensors[(size_t)index];
    fill_info(t, out);
    return t.shape.size() > NCM_ST_MAX_DIMS ? NCM_E_SHAPE : NCM_OK;
}

int ncm_st_find(const ncm_st_file_t* f, const char* name, ncm_st_tensor_t* out) {
    if (!f || !name || !out) return NCM_E_NULL;
    for (const Tensor& t : f->tensors)
        if (t.name == name) {
            fill_info(t, out);
            return t.shape.size() > NCM_ST_MAX_DIMS ? NCM_E_SHAPE : NCM_OK;
        }
    ncm_set_error_detail(std::string("no tensor named ") + name);
    return NCM_E_ARG;
}

const char* ncm_st_dtype_name(int dtype) {
    return dtype >= 0 && dtype < kNumDtypes ? kDtypes[dtype].name : "";
}

int ncm_st_dtype_bits(int dtype) { return dtype >= 0 && dtype < kNumDtypes ? kDtypes[dtype].bits : 0; }

int ncm_st_upload(ncm_ctx_t* ctx, const ncm_st_file_t* f, const char* name, void* dst,
                  size_t dst_bytes) {
    if (!ctx || !f || !name || !dst) return NCM_E_NULL;
    if (!f->map) { ncm_set_error_detail("file was parsed from memory, not opened"); return NCM_E_ARG; }
    const Tensor* t = nullptr;
    for (const Tensor& x : f->tensors)
        if (x.name == name) { t = &x; break; }
    if (!t) { ncm_set_error_detail(std::string("no tensor named ") + name); return NCM_E_ARG; }
    const uint64_t n = t->end - t->begin;
    if (dst_bytes != n) return NCM_E_LENGTH;
    if (n == 0) return NCM_OK;
    const unsigned char* src = f->map + 8 + f->header_len + t->begin;
    return ncm_upload_host_bytes(ctx, src, dst, (size_t)n);
}

int ncm_st_parse_index(const char* json, size_t len, ncm_st_index_t** out) {
    if (!out || (len > 0 && !json)) return NCM_E_NULL;
    *out = nullptr;
    JValue root;
    if (!parse_json(json, len, root)) return format_error("SyntaxError");
    if (root.kind != JValue::Object) return format_error("InvalidIndex");
    const JValue* wm = root.get("weight_map");
    if (!wm || wm->kind != JValue::Object) return format_error("InvalidIndex");
    ncm_st_index* ix = new (std::nothrow) ncm_st_index;
    if (!ix) return NCM_E_NOMEM;
    for (size_t mi = 0; mi < wm->members.size(); ++mi) {
        const std::string& key = wm->members[mi].first;
        bool seen = false;
        for (size_t k = 0; k < mi; ++k) seen = seen || wm->members[k].first == key;
        if (seen) continue;
        const JValue& val = *wm->get(key);
        if (val.kind != JValue::String) { delete ix; return format_error("InvalidIndex"); }
        if (!plain_file_name(val.s)) { delete ix; return format_error("UnsafeShardName"); }
        ix->weight_map.emplace_back(key, val.s);
    }
    if (const JValue* md = root.get("metadata")) {
        if (md->kind != JValue::Object) { delete ix; return format_error("InvalidIndex"); }
        if (const JValue* ts = md->get("total_size")) {
            if (!non_negative(*ts, ix->total_size)) { delete ix; return format_error("InvalidHeader"); }
            ix->has_total = true;
        }
    }
    *out = ix;
    return NCM_OK;
}

int ncm_st_index_close(ncm_st_index_t* ix) {
    if (!ix) return NCM_E_NULL;
    delete ix;
    return NCM_OK;
}

int64_t ncm_st_index_count(const ncm_st_index_t* ix) {
    return ix ? (int64_t)ix->weight_map.size() : -1;
}

int ncm_st_index_entry(const ncm_st_index_t* ix, int64_t i, const char** tensor,
                       const char** shard) {
    if (!ix || !tensor || !shard) return NCM_E_NULL;
    if (i < 0 || i >= (int64_t)ix->weight_map.size()) return NCM_E_ARG;
    *tensor = ix->weight_map[(size_t)i].first.c_str();
    *shard = ix->weight_map[(size_t)i].second.c_str();
    return NCM_OK;
}

int ncm_st_index_total_size(const ncm_st_index_t* ix, uint64_t* total) {
    if (!ix || !total) return NCM_E_NULL;
    if (!ix->has_total) return NCM_E_ARG;
    *total = ix->total_size;
    return NCM_OK;
}

}  // extern "C"
