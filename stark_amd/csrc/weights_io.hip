// Weight files feeding the quantized products: Stark's converted artifact
// (safetensors, read as the engine's ParameterLoader reads it) and GGUF v3
// checkpoints (read as the hybrid engine's Weights::open reads them), plus
// WeightMatrix::load, which turns an artifact's `<prefix>.weights / .scales /
// .biases | .zero_points` tensors into a stark_qmm_b ready for
// stark_qmm_encode. Host code only: files are mapped read-only, tensors are
// copied to the device on request.
//
// Reference behaviour restated here (paths under crates/stark-engine/src/):
//   parameters/safetensors_metadata.rs:113-128   header size (8-byte LE) + JSON, 100 MB bound
//   parameters/loader.rs:80-127                    index: offsets checked against the file
//   parameters/loader.rs:272-305                   ParameterLeaf::validate (shape, dtype, byte size)
//   encodable_block/weight_matrix.rs:53-216        parse_spec + WeightMatrix::load
//   backends/common/kernel/matmul/mod.rs:78-157    QuantParams shapes, source output widths
//   engine/hybrid/weights.rs:815-900               Weights::open (GGUF splits)
//   engine/hybrid/weights.rs:2556-2595             product, block_layout, encoded_size
//   engine/hybrid/weights.rs:2686-2865             GGUF header reader and read_gguf
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "qmm_common.h"

namespace {

thread_local std::string g_last_error;

stark_qmm_status fail(stark_qmm_status st, const std::string& msg) {
    g_last_error = msg;
    return st;
}

// ------------------------------------------------------------------ JSON
// The subset a safetensors header uses: objects, arrays, strings, integers
// (and, for __metadata__ values, any scalar kept as text).
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    std::string text;  // STR: the string; NUM: the literal
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;

    const Json* get(const std::string& k) const {
        for (const auto& m : members)
            if (m.first == k) return &m.second;
        return nullptr;
    }
    bool as_u64(uint64_t* out) const {
        if (kind != NUM || text.empty()) return false;
        uint64_t v = 0;
        for (char c : text) {
            if (c < '0' || c > '9') return false;
            const uint64_t d = (uint64_t)(c - '0');
            if (v > (UINT64_MAX - d) / 10) return false;
            v = v * 10 + d;
        }
        *out = v;
        return true;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    int depth = 0;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n)) return false;
        p += n;
        return true;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 63));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 63));
            out += (char)(0x80 | (cp & 63));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 63));
            out += (char)(0x80 | ((cp >> 6) & 63));
            out += (char)(0x80 | (cp & 63));
        }
    }
    bool hex4(uint32_t* v) {
        if (end - p < 4) return false;
        *v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& out) {
        if (p >= end || *p != '"') return false;
        ++p;
        while (p < end && *p != '"') {
            const unsigned char c = (unsigned char)*p++;
            if (c < 0x20) return false;
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (p >= end) return false;
            const char e = *p++;
            switch (e) {
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
                if (!hex4(&cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {
                    uint32_t lo;
                    if (!lit("\\u") || !hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, cp);
                break;
            }
            default: return false;
            }
        }
        if (p >= end) return false;
        ++p;
        return true;
    }
    bool value(Json& v) {
        if (++depth > 64) return false;
        ws();
        if (p >= end) return false;
        bool ok = true;
        if (*p == '{') {
            v.kind = Json::OBJ;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
            } else {
                for (;;) {
                    ws();
                    std::string k;
                    if (!string(k)) return false;
                    ws();
                    if (p >= end || *p != ':') return false;
                    ++p;
                    Json m;
                    if (!value(m)) return false;
                    v.members.emplace_back(std::move(k), std::move(m));
                    ws();
                    if (p < end && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        ++p;
                        break;
                    }
                    return false;
                }
            }
        } else if (*p == '[') {
            v.kind = Json::ARR;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
            } else {
                for (;;) {
                    Json m;
                    if (!value(m)) return false;
                    v.items.push_back(std::move(m));
                    ws();
                    if (p < end && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        ++p;
                        break;
                    }
                    return false;
                }
            }
        } else if (*p == '"') {
            v.kind = Json::STR;
            ok = string(v.text);
        } else if (lit("true")) {
            v.kind = Json::BOOL;
            v.text = "true";
        } else if (lit("false")) {
            v.kind = Json::BOOL;
            v.text = "false";
        } else if (lit("null")) {
            v.kind = Json::NUL;
        } else {
            v.kind = Json::NUM;
            const char* s = p;
            if (p < end && *p == '-') ++p;
            while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' ||
                               *p == '-'))
                ++p;
            v.text.assign(s, p);
            ok = p > s;
        }
        --depth;
        return ok;
    }
};

bool parse_json(const char* data, size_t n, Json& out) {
    JsonParser ps{data, data + n};
    if (!ps.value(out)) return false;
    ps.ws();
    return ps.p == ps.end;
}

// ------------------------------------------------------------------ files

struct Mapping {
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t length = 0;
    ~Mapping() {
        if (base && length) munmap((void*)base, length);
        if (fd >= 0) close(fd);
    }
};

stark_qmm_status map_file(const std::string& path, Mapping& m) {
    m.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (m.fd < 0) return fail(STARK_QMM_IO_ERROR, "cannot open " + path);
    struct stat st;
    if (fstat(m.fd, &st) != 0) return fail(STARK_QMM_IO_ERROR, "cannot stat " + path);
    m.length = (uint64_t)st.st_size;
    if (m.length) {
        void* p = mmap(nullptr, m.length, PROT_READ, MAP_PRIVATE, m.fd, 0);
        if (p == MAP_FAILED) return fail(STARK_QMM_IO_ERROR, "cannot map " + path);
        m.base = (const uint8_t*)p;
    }
    return STARK_QMM_OK;
}

struct Tensor {
    uint32_t dtype = 0;            // safetensors: STARK_QMM_* data type; GGUF: ggml kind
    std::vector<uint64_t> shape;   // outermost first
    size_t file = 0;               // index into the mappings
    uint64_t offset = 0, size = 0;
};

bool checked_mul(uint64_t a, uint64_t b, uint64_t* r) { return !__builtin_mul_overflow(a, b, r); }
bool checked_add(uint64_t a, uint64_t b, uint64_t* r) { return !__builtin_add_overflow(a, b, r); }

// engine DataType byte sizes (data_type.rs); 0 = not a tensor dtype the engine loads
uint64_t dtype_bytes(uint32_t dt) {
    switch (dt) {
    case STARK_QMM_F32: case STARK_QMM_U32: case STARK_QMM_I32: return 4;
    case STARK_QMM_F16: case STARK_QMM_BF16: return 2;
    case STARK_QMM_U8: case STARK_QMM_I8: return 1;
    case STARK_QMM_I64: case STARK_QMM_U64: return 8;
    default: return 0;
    }
}

// Dtype::data_type (safetensors_metadata.rs:95-110)
bool safetensors_dtype(const std::string& s, uint32_t* dt) {
    static const std::pair<const char*, uint32_t> table[] = {
        {"F16", STARK_QMM_F16}, {"BF16", STARK_QMM_BF16}, {"F32", STARK_QMM_F32}, {"I8", STARK_QMM_I8},
        {"U8", STARK_QMM_U8},   {"I32", STARK_QMM_I32},   {"U32", STARK_QMM_U32}, {"I64", STARK_QMM_I64},
        {"U64", STARK_QMM_U64}};
    for (const auto& e : table)
        if (s == e.first) {
            *dt = e.second;
            return true;
        }
    return false;
}

// block_layout (weights.rs:2565-2584): GGML kind -> (values, bytes) per block.
bool gguf_block(uint32_t kind, uint64_t* values, uint64_t* bytes) {
    switch (kind) {
    case 0: *values = 1; *bytes = 4; return true;
    case 1: case 30: *values = 1; *bytes = 2; return true;
    case 8: *values = 32; *bytes = 34; return true;
    case 10: *values = 256; *bytes = 84; return true;
    case 11: *values = 256; *bytes = 110; return true;
    case 12: *values = 256; *bytes = 144; return true;
    case 13: *values = 256; *bytes = 176; return true;
    case 14: *values = 256; *bytes = 210; return true;
    case 16: *values = 256; *bytes = 66; return true;
    case 17: *values = 256; *bytes = 74; return true;
    case 18: *values = 256; *bytes = 98; return true;
    case 23: *values = 256; *bytes = 136; return true;
    default: return false;
    }
}

// encoded_size (weights.rs:2586-2595)
stark_qmm_status gguf_encoded_size(uint32_t kind, uint64_t count, uint64_t* out) {
    uint64_t values, bytes;
    if (!gguf_block(kind, &values, &bytes)) return fail(STARK_QMM_UNSUPPORTED, "unsupported weight block format");
    if (count % values) return fail(STARK_QMM_INVALID_ARGUMENT, "weight dimension is not block aligned");
    if (!checked_mul(count / values, bytes, out)) return fail(STARK_QMM_INVALID_ARGUMENT, "encoded weight size overflow");
    return STARK_QMM_OK;
}

}  // namespace

struct stark_qmm_file {
    uint32_t kind = STARK_QMM_FILE_SAFETENSORS;
    std::vector<std::unique_ptr<Mapping>> maps;
    std::map<std::string, Tensor> tensors;
    std::vector<std::string> names;                     // sorted
    std::map<std::string, std::string> metadata;        // values as text
};

namespace {

// ---- Stark artifact: read_metadata + ParameterLoader::new
constexpr uint64_t kMaxSafetensorsHeader = 100000000;  // safetensors_metadata.rs:111

stark_qmm_status open_safetensors(const std::string& path, stark_qmm_file& f) {
    auto m = std::make_unique<Mapping>();
    stark_qmm_status st = map_file(path, *m);
    if (st != STARK_QMM_OK) return st;
    if (m->length < 8) return fail(STARK_QMM_HEADER_ERROR, "Unable to read safetensors header bytes");
    uint64_t hsize;
    memcpy(&hsize, m->base, 8);
    if (hsize > kMaxSafetensorsHeader) return fail(STARK_QMM_HEADER_ERROR, "The header is too large.");
    if (hsize > m->length - 8) return fail(STARK_QMM_HEADER_ERROR, "Unable to read safetensors header JSON");
    Json root;
    if (!parse_json((const char*)m->base + 8, hsize, root) || root.kind != Json::OBJ)
        return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
    const uint64_t global = 8 + hsize;
    for (const auto& mem : root.members) {
        if (mem.first == "__metadata__") {
            if (mem.second.kind != Json::OBJ) return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
            for (const auto& kv : mem.second.members) {
                if (kv.second.kind != Json::STR)
                    return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
                f.metadata[kv.first] = kv.second.text;
            }
            continue;
        }
        const Json& v = mem.second;
        const Json* dt = v.get("dtype");
        const Json* sh = v.get("shape");
        const Json* off = v.get("data_offsets");
        if (v.kind != Json::OBJ || !dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !off ||
            off->kind != Json::ARR || off->items.size() != 2)
            return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
        Tensor t;
        if (!safetensors_dtype(dt->text, &t.dtype))
            return fail(STARK_QMM_HEADER_ERROR, "Unsupported safetensors dtype: " + dt->text);
        for (const Json& d : sh->items) {
            uint64_t x;
            if (!d.as_u64(&x) || x > 0xffffffffull) return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
            t.shape.push_back(x);
        }
        uint64_t begin, end;
        if (!off->items[0].as_u64(&begin) || !off->items[1].as_u64(&end))
            return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
        if (end < begin)
            return fail(STARK_QMM_HEADER_ERROR, "Invalid data offsets for tensor " + mem.first + ": begin=" +
                                                    std::to_string(begin) + ", end=" + std::to_string(end));
        t.size = end - begin;
        if (!checked_add(global, begin, &t.offset))
            return fail(STARK_QMM_HEADER_ERROR, "Tensor offset overflow for tensor " + mem.first);
        uint64_t absolute_end;
        if (!checked_add(global, end, &absolute_end) || absolute_end > m->length)
            return fail(STARK_QMM_HEADER_ERROR, "Tensor payload exceeds file length");
        if (!f.tensors.emplace(mem.first, std::move(t)).second)
            return fail(STARK_QMM_HEADER_ERROR, "The header is not valid UTF-8 JSON");
    }
    f.kind = STARK_QMM_FILE_SAFETENSORS;
    f.maps.push_back(std::move(m));
    return STARK_QMM_OK;
}

// ---- GGUF v3: HeaderReader + read_gguf (weights.rs:2686-2865)
constexpr uint64_t kMaxGgufHeader = 128ull * 1024 * 1024;  // weights.rs:40
constexpr uint64_t kMaxCount = 2000000;                      // weights.rs:41

struct GgufReader {
    const uint8_t* base;
    uint64_t length, pos = 0;
    stark_qmm_status st = STARK_QMM_OK;

    bool take(uint64_t n, const uint8_t** out) {
        if (st != STARK_QMM_OK) return false;
        uint64_t np;
        if (!checked_add(pos, n, &np)) {
            st = fail(STARK_QMM_INVALID_ARGUMENT, "GGUF header overflow");
            return false;
        }
        if (np > kMaxGgufHeader) {
            st = fail(STARK_QMM_INVALID_ARGUMENT, "GGUF header too large");
            return false;
        }
        if (np > length) {
            st = fail(STARK_QMM_IO_ERROR, "failed to fill whole buffer");
            return false;
        }
        *out = base + pos;
        pos = np;
        return true;
    }
    template <class T>
    bool scalar(T* v) {
        const uint8_t* p;
        if (!take(sizeof(T), &p)) return false;
        memcpy(v, p, sizeof(T));
        return true;
    }
    bool count(uint64_t* c) {
        if (!scalar(c)) return false;
        if (*c > kMaxCount) {
            st = fail(STARK_QMM_INVALID_ARGUMENT, "GGUF count exceeds bounds");
            return false;
        }
        return true;
    }
    bool text(std::string* s) {
        uint64_t n;
        const uint8_t* p;
        if (!count(&n) || !take(n, &p)) return false;
        s->assign((const char*)p, n);
        // UTF-8 validity (String::from_utf8)
        for (size_t i = 0; i < n;) {
            const unsigned char c = p[i];
            const int len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
            if (!len || i + len > n) {
                st = fail(STARK_QMM_INVALID_ARGUMENT, "invalid GGUF text encoding");
                return false;
            }
            for (int k = 1; k < len; ++k)
                if ((p[i + k] & 0xC0) != 0x80) {
                    st = fail(STARK_QMM_INVALID_ARGUMENT, "invalid GGUF text encoding");
                    return false;
                }
            i += len;
        }
        return true;
    }
    // One metadata value as text (arrays as [a,b,...]); numbers in decimal.
    bool value(uint32_t kind, std::string* out, int depth = 0) {
        switch (kind) {
        case 0: { uint8_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 1: { int8_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 2: { uint16_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 3: { int16_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 4: { uint32_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 5: { int32_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 6: case 12: {
            double d;
            if (kind == 6) { float v; if (!scalar(&v)) return false; d = v; }
            else if (!scalar(&d)) return false;
            if (!std::isfinite(d)) { st = fail(STARK_QMM_INVALID_ARGUMENT, "nonfinite GGUF metadata"); return false; }
            char buf[64];
            snprintf(buf, sizeof buf, "%.17g", d);
            *out = buf;
            return true;
        }
        case 7: {
            uint8_t v;
            if (!scalar(&v)) return false;
            if (v > 1) { st = fail(STARK_QMM_INVALID_ARGUMENT, "invalid GGUF boolean"); return false; }
            *out = v ? "true" : "false";
            return true;
        }
        case 8: return text(out);
        case 9: {
            uint32_t sub;
            uint64_t n;
            if (!scalar(&sub)) return false;
            if (sub == 9 || depth > 0) { st = fail(STARK_QMM_UNSUPPORTED, "nested GGUF arrays"); return false; }
            if (!count(&n)) return false;
            *out = "[";
            for (uint64_t i = 0; i < n; ++i) {
                std::string e;
                if (!value(sub, &e, depth + 1)) return false;
                if (i) *out += ",";
                *out += e;
            }
            *out += "]";
            return true;
        }
        case 10: { uint64_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        case 11: { int64_t v; if (!scalar(&v)) return false; *out = std::to_string(v); return true; }
        default: st = fail(STARK_QMM_UNSUPPORTED, "unsupported GGUF metadata type"); return false;
        }
    }
};

bool meta_u64(const std::map<std::string, std::string>& md, const char* key, uint64_t* v) {
    auto it = md.find(key);
    if (it == md.end()) return false;
    Json j;
    j.kind = Json::NUM;
    j.text = it->second;
    return j.as_u64(v);
}

stark_qmm_status read_gguf(Mapping& m, size_t file, std::map<std::string, Tensor>& tensors,
                           std::map<std::string, std::string>& metadata) {
    GgufReader r{m.base, m.length};
    const uint8_t* magic;
    uint32_t version = 0;
    if (!r.take(4, &magic)) return r.st;
    if (memcmp(magic, "GGUF", 4) || !r.scalar(&version) || version != 3)
        return r.st != STARK_QMM_OK ? r.st : fail(STARK_QMM_UNSUPPORTED, "GGUF version three is required");
    uint64_t tensor_count, metadata_count;
    if (!r.count(&tensor_count) || !r.count(&metadata_count)) return r.st;
    for (uint64_t i = 0; i < metadata_count; ++i) {
        std::string name, value;
        uint32_t kind;
        if (!r.text(&name) || !r.scalar(&kind) || !r.value(kind, &value)) return r.st;
        if (name.empty() || !metadata.emplace(name, value).second)
            return fail(STARK_QMM_INVALID_ARGUMENT, "duplicate GGUF metadata");
    }
    uint64_t alignment = 32;
    if (metadata.count("general.alignment") && !meta_u64(metadata, "general.alignment", &alignment)) alignment = 32;
    if (alignment == 0 || (alignment & (alignment - 1)) || alignment > 4096)
        return fail(STARK_QMM_INVALID_ARGUMENT, "invalid GGUF alignment");
    std::vector<std::string> order;
    for (uint64_t i = 0; i < tensor_count; ++i) {
        std::string name;
        uint32_t rank;
        if (!r.text(&name) || !r.scalar(&rank)) return r.st;
        if (name.empty() || rank < 1 || rank > 4) return fail(STARK_QMM_INVALID_ARGUMENT, "invalid GGUF tensor identity or rank");
        Tensor t;
        t.file = file;
        for (uint32_t d = 0; d < rank; ++d) {
            uint64_t x;
            if (!r.scalar(&x)) return r.st;
            t.shape.push_back(x);
        }
        if (!r.scalar(&t.dtype)) return r.st;
        // the safetensors-only integer tags are never GGML kinds
        static const uint32_t admitted[] = {0, 1, 30, 8, 10, 11, 12, 13, 14, 16, 17, 18, 23};
        if (std::find(std::begin(admitted), std::end(admitted), t.dtype) == std::end(admitted))
            return fail(STARK_QMM_UNSUPPORTED, "unsupported GGUF tensor type");
        if (!r.scalar(&t.offset)) return r.st;
        uint64_t count = 1;
        for (uint64_t d : t.shape) {
            if (d == 0) return fail(STARK_QMM_INVALID_ARGUMENT, "empty tensor dimension");
            if (!checked_mul(count, d, &count)) return fail(STARK_QMM_INVALID_ARGUMENT, "tensor size overflow");
        }
        stark_qmm_status st = gguf_encoded_size(t.dtype, count, &t.size);
        if (st != STARK_QMM_OK) return st;
        uint64_t row;
        st = gguf_encoded_size(t.dtype, t.shape[0], &row);  // whole blocks per row
        if (st != STARK_QMM_OK) return st;
        if (t.offset % alignment) return fail(STARK_QMM_INVALID_ARGUMENT, "unaligned GGUF tensor");
        std::reverse(t.shape.begin(), t.shape.end());  // GGML lists the innermost dimension first
        if (!tensors.emplace(name, std::move(t)).second) return fail(STARK_QMM_INVALID_ARGUMENT, "duplicate GGUF tensor");
        order.push_back(name);
    }
    uint64_t start;
    if (!checked_add(r.pos, alignment - 1, &start)) return fail(STARK_QMM_INVALID_ARGUMENT, "GGUF offset overflow");
    start &= ~(alignment - 1);
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    for (const std::string& n : order) {
        Tensor& t = tensors[n];
        uint64_t end;
        if (!checked_add(t.offset, start, &t.offset)) return fail(STARK_QMM_INVALID_ARGUMENT, "GGUF offset overflow");
        if (!checked_add(t.offset, t.size, &end) || end > m.length)
            return fail(STARK_QMM_INVALID_ARGUMENT, "truncated GGUF tensor");
        spans.emplace_back(t.offset, end);
    }
    std::sort(spans.begin(), spans.end());
    uint64_t end = start;
    for (const auto& s : spans) {
        if (s.first < end) return fail(STARK_QMM_INVALID_ARGUMENT, "overlapping GGUF tensors");
        end = s.second;
    }
    if (start > m.length) return fail(STARK_QMM_INVALID_ARGUMENT, "truncated GGUF header");
    return STARK_QMM_OK;
}

bool has_suffix(const std::string& s, const char* suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// Weights::open for GGUF (weights.rs:815-895): one file, or a directory of
// split files (names starting "._" are skipped) whose split.no / split.count
// form a complete set; metadata comes from split 0.
stark_qmm_status open_gguf(const std::string& path, bool dir, stark_qmm_file& f) {
    std::vector<std::string> paths;
    if (dir) {
        DIR* d = opendir(path.c_str());
        if (!d) return fail(STARK_QMM_IO_ERROR, "cannot read directory " + path);
        while (dirent* e = readdir(d)) {
            const std::string n = e->d_name;
            if (n.rfind("._", 0) == 0) continue;
            if (has_suffix(n, ".gguf") || has_suffix(n, ".safetensors")) paths.push_back(path + "/" + n);
        }
        closedir(d);
        std::sort(paths.begin(), paths.end());
    } else {
        paths.push_back(path);
    }
    if (paths.empty() || paths.size() > 512) return fail(STARK_QMM_INVALID_ARGUMENT, "missing or excessive weight shards");
    for (const std::string& p : paths)
        if (!has_suffix(p, ".gguf")) return fail(STARK_QMM_INVALID_ARGUMENT, "mixed weight containers");
    std::map<uint64_t, uint64_t> splits;
    for (const std::string& p : paths) {
        auto m = std::make_unique<Mapping>();
        stark_qmm_status st = map_file(p, *m);
        if (st != STARK_QMM_OK) return st;
        std::map<std::string, Tensor> tensors;
        std::map<std::string, std::string> md;
        st = read_gguf(*m, f.maps.size(), tensors, md);
        if (st != STARK_QMM_OK) return st;
        uint64_t count = 1, index = 0;
        if (md.count("split.count") && !meta_u64(md, "split.count", &count)) count = 1;
        if (md.count("split.no") && !meta_u64(md, "split.no", &index)) index = 0;
        if (count == 0 || count > 512 || index >= count || !splits.emplace(index, count).second)
            return fail(STARK_QMM_INVALID_ARGUMENT, "invalid or duplicate GGUF split");
        if (index == 0) f.metadata = md;
        for (auto& t : tensors)
            if (!f.tensors.emplace(t.first, std::move(t.second)).second)
                return fail(STARK_QMM_INVALID_ARGUMENT, "duplicate tensor across weight shards");
        f.maps.push_back(std::move(m));
    }
    const uint64_t n = paths.size();
    if (splits.size() != n) return fail(STARK_QMM_INVALID_ARGUMENT, "incomplete GGUF split set");
    for (const auto& s : splits)
        if (s.first >= n || s.second != n) return fail(STARK_QMM_INVALID_ARGUMENT, "incomplete GGUF split set");
    uint64_t total;
    if (f.metadata.count("split.tensors.count") && meta_u64(f.metadata, "split.tensors.count", &total) &&
        total != f.tensors.size())
        return fail(STARK_QMM_INVALID_ARGUMENT, "incomplete GGUF tensor inventory");
    f.kind = STARK_QMM_FILE_GGUF;
    return STARK_QMM_OK;
}

const Tensor* find(const stark_qmm_file* f, const std::string& key) {
    auto it = f->tensors.find(key);
    return it == f->tensors.end() ? nullptr : &it->second;
}

stark_qmm_status upload(const stark_qmm_file* f, const Tensor& t, void** dev, void* stream) {
    void* d = nullptr;
    if (hipMalloc(&d, std::max<uint64_t>(t.size, 1)) != hipSuccess) return fail(STARK_QMM_OUT_OF_MEMORY, "hipMalloc failed");
    const uint8_t* src = f->maps[t.file]->base + t.offset;
    if (t.size && (hipMemcpyAsync(d, src, t.size, hipMemcpyHostToDevice, (hipStream_t)stream) != hipSuccess ||
                   hipStreamSynchronize((hipStream_t)stream) != hipSuccess)) {
        (void)hipFree(d);
        return fail(STARK_QMM_DEVICE_FAILURE, "copy to the device failed");
    }
    *dev = d;
    return STARK_QMM_OK;
}

std::string shape_text(const std::vector<uint64_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// ParameterLeaf::validate (loader.rs:272-305) on tree.leaf(name)
stark_qmm_status leaf(const stark_qmm_file* f, const std::string& key, std::vector<uint64_t> shape, uint32_t dtype,
                      const Tensor** out) {
    const Tensor* t = find(f, key);
    if (!t) return fail(STARK_QMM_KEY_NOT_FOUND, "Array with key \"" + key + "\" not found.");
    if (t->shape != shape || t->dtype != dtype)
        return fail(STARK_QMM_INVALID_TENSOR, "Invalid tensor " + key + ": got " + shape_text(t->shape) + ", expected " +
                                                  shape_text(shape));
    uint64_t expected = dtype_bytes(dtype);
    for (uint64_t d : shape) expected *= d;
    if (t->size != expected)
        return fail(STARK_QMM_INVALID_TENSOR, "Invalid tensor byte size: got " + std::to_string(t->size) + " bytes for " +
                                                  key + ", expected " + std::to_string(expected) + " bytes");
    *out = t;
    return STARK_QMM_OK;
}

uint32_t round_up(uint32_t v, uint32_t m) { return (v + m - 1) / m * m; }

}  // namespace

extern "C" {

const char* stark_qmm_last_error(void) { return g_last_error.c_str(); }

stark_qmm_status stark_qmm_file_open(const char* path, stark_qmm_file** out) {
    if (!path || !out) return fail(STARK_QMM_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    g_last_error.clear();
    std::unique_ptr<stark_qmm_file> f(new (std::nothrow) stark_qmm_file);
    if (!f) return fail(STARK_QMM_OUT_OF_MEMORY, "out of memory");
    const std::string p = path;
    struct stat st;
    if (stat(path, &st) != 0) return fail(STARK_QMM_IO_ERROR, "cannot open " + p);
    stark_qmm_status s;
    if (S_ISDIR(st.st_mode)) s = open_gguf(p, true, *f);
    else if (has_suffix(p, ".gguf")) s = open_gguf(p, false, *f);
    else s = open_safetensors(p, *f);
    if (s != STARK_QMM_OK) return s;
    for (const auto& t : f->tensors) f->names.push_back(t.first);
    *out = f.release();
    return STARK_QMM_OK;
}

void stark_qmm_file_close(stark_qmm_file* f) { delete f; }

uint32_t stark_qmm_file_kind(const stark_qmm_file* f) { return f ? f->kind : 0; }

uint64_t stark_qmm_file_tensor_count(const stark_qmm_file* f) { return f ? f->names.size() : 0; }

const char* stark_qmm_file_tensor_name(const stark_qmm_file* f, uint64_t index) {
    return f && index < f->names.size() ? f->names[index].c_str() : nullptr;
}

stark_qmm_status stark_qmm_file_tensor(const stark_qmm_file* f, const char* name, stark_qmm_tensor_info* info) {
    if (!f || !name || !info) return fail(STARK_QMM_INVALID_ARGUMENT, "null argument");
    const Tensor* t = find(f, name);
    if (!t) return fail(STARK_QMM_KEY_NOT_FOUND, std::string("Array with key \"") + name + "\" not found.");
    if (t->shape.size() > 8) return fail(STARK_QMM_INVALID_ARGUMENT, "unsupported weight rank");
    memset(info, 0, sizeof *info);
    info->dtype = t->dtype;
    info->rank = (uint32_t)t->shape.size();
    for (size_t i = 0; i < t->shape.size(); ++i) info->shape[i] = t->shape[i];
    info->offset = t->offset;
    info->size = t->size;
    info->host = f->maps[t->file]->base + t->offset;
    return STARK_QMM_OK;
}

stark_qmm_status stark_qmm_file_metadata(const stark_qmm_file* f, const char* key, const char** value) {
    if (!f || !key || !value) return fail(STARK_QMM_INVALID_ARGUMENT, "null argument");
    auto it = f->metadata.find(key);
    if (it == f->metadata.end()) return fail(STARK_QMM_KEY_NOT_FOUND, std::string("metadata key ") + key + " not found");
    *value = it->second.c_str();
    return STARK_QMM_OK;
}

stark_qmm_status stark_qmm_file_upload(const stark_qmm_file* f, const char* name, void** device, void* stream) {
    if (!f || !name || !device) return fail(STARK_QMM_INVALID_ARGUMENT, "null argument");
    const Tensor* t = find(f, name);
    if (!t) return fail(STARK_QMM_KEY_NOT_FOUND, std::string("Array with key \"") + name + "\" not found.");
    return upload(f, *t, device, stream);
}

stark_qmm_status stark_qmm_device_free(void* device) {
    return device && hipFree(device) != hipSuccess ? STARK_QMM_DEVICE_FAILURE : STARK_QMM_OK;
}

stark_qmm_status stark_qmm_weight_matrix_load(const stark_qmm_file* f, const char* prefix,
                                              const stark_qmm_weight_spec* spec, uint32_t required_layout,
                                              uint32_t output_dim, uint32_t input_dim, uint32_t data_type,
                                              stark_qmm_weight_matrix* out, void* stream) {
    if (!f || !prefix || !spec || !out) return fail(STARK_QMM_INVALID_ARGUMENT, "null argument");
    if (spec->struct_size != sizeof(stark_qmm_weight_spec) || out->struct_size != sizeof(stark_qmm_weight_matrix))
        return STARK_QMM_ABI_MISMATCH;
    const uint32_t out_size = out->struct_size;
    memset(out, 0, sizeof *out);
    out->struct_size = out_size;
    const std::string pre = std::string(prefix) + (prefix[0] ? "." : "");
    const auto U = [](const std::string& m) { return fail(STARK_QMM_UNSUPPORTED_CONFIGURATION, m); };
    if (data_type != STARK_QMM_F32 && data_type != STARK_QMM_F16 && data_type != STARK_QMM_BF16)
        return U("unsupported weights data type");
    const bool materialize = spec->kind == STARK_QMM_SPEC_MLX && spec->materialize_affine_input_sum;
    if (materialize && !(spec->bits == 4 && data_type == STARK_QMM_BF16))
        return U("materialized affine input sums require BF16 W4 matrices");
    // parse_spec (weight_matrix.rs:53-96)
    uint32_t layout = spec->layout, method = 0, mode = 0;
    bool quantized = true;
    if (layout > STARK_QMM_WEIGHT_INPUT_OUTPUT) return U("unknown weight layout");
    switch (spec->kind) {
    case STARK_QMM_SPEC_FULL_PRECISION: quantized = false; break;
    case STARK_QMM_SPEC_MLX: method = STARK_QMM_CORRECTION_BIASES; break;
    case STARK_QMM_SPEC_INT:
        method = spec->is_symmetric ? STARK_QMM_CORRECTION_SYMMETRIC : STARK_QMM_CORRECTION_ZERO_POINTS;
        break;
    default: return U("unsupported weight matrix spec");
    }
    if (quantized) {
        if (spec->bits == 4) mode = STARK_QMM_MODE_U4;
        else if (spec->bits == 5 && method == STARK_QMM_CORRECTION_BIASES) mode = STARK_QMM_MODE_U5;
        else if (spec->bits == 6 && method == STARK_QMM_CORRECTION_BIASES) mode = STARK_QMM_MODE_U6;
        else if (spec->bits == 8) mode = STARK_QMM_MODE_U8;
        else return U("bits=" + std::to_string(spec->bits) + ", group_size=" + std::to_string(spec->group_size));
        if (spec->group_size == 0) return U("group size must be non-zero");
        if ((mode == STARK_QMM_MODE_U5 || mode == STARK_QMM_MODE_U6) &&
            (spec->group_size != 64 || layout != STARK_QMM_WEIGHT_OUTPUT_INPUT))
            return U("packed five/six-bit affine matrices require group64 and output-input layout");
    }
    if (layout != required_layout) return U("expected weight layout " + std::to_string(required_layout) + ", got " +
                                            std::to_string(layout));
    // physical_shape (weight_matrix.rs:321-330)
    const uint32_t rows = layout == STARK_QMM_WEIGHT_OUTPUT_INPUT ? output_dim : input_dim;
    const uint32_t columns = layout == STARK_QMM_WEIGHT_OUTPUT_INPUT ? input_dim : output_dim;
    out->rows = rows;
    out->columns = columns;
    // QuantParams::with_source_output_widths (mod.rs:78-92)
    if (spec->source_output_count) {
        if (spec->source_output_count > 4) return U("source output widths require one to four nonzero contiguous spans");
        uint64_t sum = 0;
        for (uint32_t i = 0; i < spec->source_output_count; ++i) {
            if (!spec->source_output_widths[i]) return U("source output widths require one to four nonzero contiguous spans");
            sum += spec->source_output_widths[i];
        }
        if (sum != rows) return U("source output widths must exactly cover the weight matrix rows");
        out->source_output_count = spec->source_output_count;
        memcpy(out->source_output_widths, spec->source_output_widths, sizeof out->source_output_widths);
    }
    const Tensor* tw = nullptr;
    stark_qmm_status st;
    if (!quantized) {
        st = leaf(f, pre + "weights", {rows, columns}, data_type, &tw);
        if (st != STARK_QMM_OK) return st;
        st = upload(f, *tw, &out->device[0], stream);
        if (st != STARK_QMM_OK) return st;
        out->b.values = out->device[0];
        return STARK_QMM_OK;
    }
    const uint32_t bits = spec->bits, gs = spec->group_size;
    if ((mode == STARK_QMM_MODE_U5 || mode == STARK_QMM_MODE_U6) && (columns % gs || data_type != STARK_QMM_BF16))
        return U("packed five/six-bit affine matrices require output-input layout, complete group-64 rows and BF16 "
                 "coefficients");
    if (mode == STARK_QMM_MODE_U4 && columns % 2)
        return U("stored columns " + std::to_string(columns) + " do not contain complete packed bytes");
    const uint32_t groups = (columns + gs - 1) / gs;
    const uint64_t row_bytes = ((uint64_t)columns * bits + 7) / 8;
    if (row_bytes > 0xffffffffull) return U("packed row size overflow");
    // params layout: output-input stores [G, N] (GroupOutput), input-output [N, G]
    const uint32_t pl = layout == STARK_QMM_WEIGHT_OUTPUT_INPUT ? STARK_QMM_LAYOUT_GROUP_OUTPUT : STARK_QMM_LAYOUT_OUTPUT_GROUP;
    const auto plane_shape = [&](uint32_t pd) -> std::vector<uint64_t> {  // QuantParams::shape (mod.rs:119-128)
        if (pl == STARK_QMM_LAYOUT_OUTPUT_GROUP) return {rows, round_up(groups, pd) / pd};
        return {groups, round_up(rows, 4) / pd};
    };
    const Tensor *ts = nullptr, *tc = nullptr;
    st = leaf(f, pre + "weights", {rows, row_bytes}, STARK_QMM_U8, &tw);
    if (st != STARK_QMM_OK) return st;
    st = leaf(f, pre + "scales", plane_shape(1), data_type, &ts);
    if (st != STARK_QMM_OK) return st;
    if (method == STARK_QMM_CORRECTION_BIASES) st = leaf(f, pre + "biases", plane_shape(1), data_type, &tc);
    else if (method == STARK_QMM_CORRECTION_ZERO_POINTS) st = leaf(f, pre + "zero_points", plane_shape(8 / bits), STARK_QMM_U8, &tc);
    if (st != STARK_QMM_OK) return st;
    const Tensor* parts[3] = {tw, ts, tc};
    for (int i = 0; i < 3; ++i) {
        if (!parts[i]) continue;
        st = upload(f, *parts[i], &out->device[i], stream);
        if (st != STARK_QMM_OK) {
            stark_qmm_weight_matrix_free(out);
            return st;
        }
    }
    stark_qmm_b& b = out->b;
    b.codes = out->device[0];
    b.codes_size = tw->size;
    b.scales = out->device[1];
    b.correction = method;
    b.correction_data = out->device[2];
    b.params.layout = pl;
    b.params.row_count = rows;
    b.params.group_count = groups;
    b.params.materialize_affine_input_sum = materialize ? 1u : 0u;
    b.mode = mode;
    b.group_size = gs;
    b.signed_codes = 0;
    return STARK_QMM_OK;
}

void stark_qmm_weight_matrix_free(stark_qmm_weight_matrix* m) {
    if (!m) return;
    for (void*& d : m->device) {
        if (d) (void)hipFree(d);
        d = nullptr;
    }
}

}  // extern "C"
