// safetensors container parser and dtype conversion for the checkpoint loader.
//
// Container format: the one the reference reads with safetensors.safe_open
// (speccheck/specimpl.py:70-86): u64 little-endian header size, UTF-8 JSON header, data.
// The JSON parser below accepts the general grammar (objects, arrays, strings with escapes,
// numbers, true/false/null) and keeps only what the tensor entries need.
#include "q35_safetensors.h"

#include <cstring>

namespace q35 {
namespace {

struct Json {
    const char* p;
    const char* end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool lit(char c) {
        ws();
        if (p < end && *p == c) { ++p; return true; }
        return false;
    }
    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (end - p < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string& s) {
        ws();
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        s.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if ((unsigned char)c < 0x20) return fail("control character in string");
            if (c != '\\') { s += c; continue; }
            if (p >= end) return fail("truncated escape");
            c = *p++;
            switch (c) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {          // surrogate pair
                        uint32_t lo;
                        if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
                        p += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool integer(int64_t& v) {
        ws();
        const char* s = p;
        if (p < end && *p == '-') return fail("negative size or offset");
        uint64_t x = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p - '0');
            if (x > (UINT64_C(0x7FFFFFFFFFFFFFFF) - d) / 10) return fail("integer overflow");
            x = x * 10 + d;
            ++p;
        }
        if (p == s) return fail("expected an integer");
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return fail("expected an integer");
        v = (int64_t)x;
        return true;
    }
    bool skip_value(int depth = 0) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("truncated header");
        if (*p == '"') { std::string s; return str(s); }
        if (*p == '{') {
            ++p;
            if (lit('}')) return true;
            do {
                std::string k;
                if (!str(k) || !lit(':') || !skip_value(depth + 1)) return fail("bad object");
            } while (lit(','));
            return lit('}') || fail("expected '}'");
        }
        if (*p == '[') {
            ++p;
            if (lit(']')) return true;
            do {
                if (!skip_value(depth + 1)) return false;
            } while (lit(','));
            return lit(']') || fail("expected ']'");
        }
        for (const char* w : {"true", "false", "null"}) {
            const size_t n = std::strlen(w);
            if ((size_t)(end - p) >= n && std::memcmp(p, w, n) == 0) { p += n; return true; }
        }
        const char* s = p;
        if (p < end && (*p == '-' || *p == '+')) ++p;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) ++p;
        return p > s || fail("bad value");
    }
    bool int_array(std::vector<int64_t>& v) {
        v.clear();
        if (!lit('[')) return fail("expected an array");
        if (lit(']')) return true;
        do {
            int64_t x;
            if (!integer(x)) return false;
            v.push_back(x);
        } while (lit(','));
        return lit(']') || fail("expected ']'");
    }
};

int dtype_size(const std::string& d) {
    if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

uint16_t f32_bits_to_bf16(uint32_t b) {
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x0040u);   // quiet NaN
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

uint32_t f16_bits_to_f32_bits(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    if (exp == 0x1F) return sign | 0x7F800000u | (man << 13);                   // inf / NaN
    if (exp == 0) {
        if (man == 0) return sign;                                              // +-0
        int e = -1;                                                             // subnormal
        do { man <<= 1; ++e; } while (!(man & 0x400u));
        return sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    return sign | ((exp + 127 - 15) << 23) | (man << 13);
}

}  // namespace

bool parse_safetensors(const void* file, size_t n, std::vector<StTensor>& out, std::string& err) {
    out.clear();
    const uint8_t* b = (const uint8_t*)file;
    if (!b || n < 8) { err = "file shorter than the 8-byte header size"; return false; }
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i) hl = (hl << 8) | b[i];
    if (hl < 2 || hl > n - 8) { err = "header size out of range"; return false; }
    const uint8_t* data = b + 8 + hl;
    const size_t data_bytes = n - 8 - (size_t)hl;
    Json j{(const char*)b + 8, (const char*)b + 8 + hl, {}};
    if (!j.lit('{')) { err = "header is not a JSON object"; return false; }
    if (!j.lit('}')) {
        do {
            std::string key;
            if (!j.str(key) || !j.lit(':')) { err = j.err.empty() ? "bad header key" : j.err; return false; }
            if (key == "__metadata__") {
                if (!j.skip_value()) { err = j.err; return false; }
                continue;
            }
            StTensor t;
            t.name = key;
            int64_t off0 = -1, off1 = -1;
            bool have_dtype = false, have_shape = false;
            if (!j.lit('{')) { err = "tensor entry is not an object: " + key; return false; }
            if (!j.lit('}')) {
                do {
                    std::string f;
                    if (!j.str(f) || !j.lit(':')) { err = "bad field in " + key; return false; }
                    if (f == "dtype") {
                        if (!j.str(t.dtype)) { err = "bad dtype in " + key; return false; }
                        have_dtype = true;
                    } else if (f == "shape") {
                        if (!j.int_array(t.shape)) { err = "bad shape in " + key; return false; }
                        have_shape = true;
                    } else if (f == "data_offsets") {
                        std::vector<int64_t> o;
                        if (!j.int_array(o) || o.size() != 2) { err = "bad data_offsets in " + key; return false; }
                        off0 = o[0];
                        off1 = o[1];
                    } else if (!j.skip_value()) {
                        err = j.err;
                        return false;
                    }
                } while (j.lit(','));
                if (!j.lit('}')) { err = "expected '}' after " + key; return false; }
            }
            if (!have_dtype || !have_shape || off0 < 0) { err = "incomplete tensor entry: " + key; return false; }
            const int es = dtype_size(t.dtype);
            if (es == 0) { err = "unknown dtype " + t.dtype + " of " + key; return false; }
            uint64_t numel = 1;
            for (int64_t d : t.shape) {
                if (d != 0 && numel > UINT64_C(0x0FFFFFFFFFFFFFFF) / (uint64_t)d) { err = "shape overflow in " + key; return false; }
                numel *= (uint64_t)d;
            }
            if (off1 < off0 || (uint64_t)off1 > data_bytes) { err = "data_offsets out of range in " + key; return false; }
            if ((uint64_t)(off1 - off0) != numel * (uint64_t)es) { err = "byte count does not match shape in " + key; return false; }
            t.data = data + off0;
            t.bytes = (size_t)(off1 - off0);
            out.push_back(std::move(t));
        } while (j.lit(','));
        if (!j.lit('}')) { err = j.err.empty() ? "expected '}' closing the header" : j.err; return false; }
    }
    j.ws();
    if (j.p != j.end) { err = "trailing bytes after the header object"; return false; }
    for (size_t i = 0; i < out.size(); ++i)
        for (size_t k = i + 1; k < out.size(); ++k)
            if (out[i].name == out[k].name) { err = "duplicate tensor " + out[i].name; return false; }
    return true;
}

bool to_bf16(const StTensor& t, std::vector<uint16_t>& out, std::string& err) {
    if (t.dtype == "BF16") {
        out.resize(t.bytes / 2);
        std::memcpy(out.data(), t.data, t.bytes);
    } else if (t.dtype == "F32") {
        out.resize(t.bytes / 4);
        for (size_t i = 0; i < out.size(); ++i) {
            uint32_t v;
            std::memcpy(&v, t.data + 4 * i, 4);
            out[i] = f32_bits_to_bf16(v);
        }
    } else if (t.dtype == "F16") {
        out.resize(t.bytes / 2);
        for (size_t i = 0; i < out.size(); ++i) {
            uint16_t h;
            std::memcpy(&h, t.data + 2 * i, 2);
            out[i] = f32_bits_to_bf16(f16_bits_to_f32_bits(h));
        }
    } else {
        err = "tensor " + t.name + " has dtype " + t.dtype + " (BF16, F16 or F32 expected)";
        return false;
    }
    return true;
}

}  // namespace q35
