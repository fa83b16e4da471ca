// flkv_codec.h — the FLKV bundle frame (src/kv_cache/bundle.rs:1-22) on the host: header
// encoding and decoding for the cache layer (kv_cache.cpp). Not part of the C-ABI.
//
// Frame: "FLKV", version u16 LE (1), header_len u32 LE, the header as JSON, then the payload.
// The header is KvBundleMeta (bundle.rs:71-81) as serde_json writes it: a compact object with
// the fields in declaration order (model_id, token_count, token_ids, block_size, num_layers,
// num_kv_heads, head_dim, dtype), unsigned integers in decimal, the dtype as the variant name
// ("F32" / "F16" / "BF16"), strings escaped as serde_json does (quote, backslash, \b \f \n \r \t,
// other control characters as \u00xx, everything else verbatim). The reader accepts what
// serde_json::from_slice accepts for that struct: any field order, whitespace, unknown fields
// (skipped), and rejects missing fields, non-integer or negative sizes, token ids above u32,
// unknown dtypes, malformed strings and trailing characters.
#pragma once

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "flour_hip.h"

namespace flour {
namespace flkv {

constexpr char MAGIC[4] = {'F', 'L', 'K', 'V'};
constexpr uint16_t VERSION = 1;
constexpr size_t PREFIX = 4 + 2 + 4;

struct Meta {
    std::string model_id;
    uint64_t token_count = 0;
    std::vector<uint32_t> token_ids;
    uint64_t block_size = 0, num_layers = 0, num_kv_heads = 0, head_dim = 0;
    int dtype = FLOUR_DTYPE_F32;
};

inline const char* dtype_name(int dt) {
    return dt == FLOUR_DTYPE_F32 ? "F32" : dt == FLOUR_DTYPE_F16 ? "F16" : "BF16";
}
inline int dtype_bytes(int dt) { return dt == FLOUR_DTYPE_F32 ? 4 : 2; }

inline void put_json_string(std::string& o, const std::string& s) {
    static const char hex[] = "0123456789abcdef";
    o += '"';
    for (unsigned char ch : s) {
        switch (ch) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\b': o += "\\b"; break;
            case '\f': o += "\\f"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if (ch < 0x20) {
                    o += "\\u00";
                    o += hex[ch >> 4];
                    o += hex[ch & 15];
                } else {
                    o += (char)ch;
                }
        }
    }
    o += '"';
}

inline std::string encode_header(const Meta& m) {
    std::string o = "{\"model_id\":";
    put_json_string(o, m.model_id);
    o += ",\"token_count\":" + std::to_string(m.token_count);
    o += ",\"token_ids\":[";
    for (size_t i = 0; i < m.token_ids.size(); i++) {
        if (i) o += ',';
        o += std::to_string(m.token_ids[i]);
    }
    o += "],\"block_size\":" + std::to_string(m.block_size);
    o += ",\"num_layers\":" + std::to_string(m.num_layers);
    o += ",\"num_kv_heads\":" + std::to_string(m.num_kv_heads);
    o += ",\"head_dim\":" + std::to_string(m.head_dim);
    o += ",\"dtype\":\"";
    o += dtype_name(m.dtype);
    o += "\"}";
    return o;
}

// ---- reader
class Reader {
  public:
    Reader(const char* p, size_t n) : p_(p), e_(p + n) {}
    std::string err;

    bool parse(Meta& m) {
        bool have[8] = {};
        static const char* names[8] = {"model_id",     "token_count", "token_ids",
                                       "block_size",   "num_layers",  "num_kv_heads",
                                       "head_dim",     "dtype"};
        if (!expect('{')) return fail("expected a JSON object");
        ws();
        if (!peek('}')) {
            for (;;) {
                std::string key;
                ws();
                if (!string(key)) return false;
                if (!expect(':')) return fail("expected `:`");
                int f = -1;
                for (int i = 0; i < 8; i++)
                    if (key == names[i]) f = i;
                bool ok = true;
                switch (f) {
                    case 0: ws(); ok = string(m.model_id); break;
                    case 1: ok = usize(m.token_count); break;
                    case 2: ok = u32_array(m.token_ids); break;
                    case 3: ok = usize(m.block_size); break;
                    case 4: ok = usize(m.num_layers); break;
                    case 5: ok = usize(m.num_kv_heads); break;
                    case 6: ok = usize(m.head_dim); break;
                    case 7: ok = dtype(m.dtype); break;
                    default: ok = skip_value(0); break;
                }
                if (!ok) return false;
                if (f >= 0 && have[f]) return fail(std::string("duplicate field `") + names[f] + "`");
                if (f >= 0) have[f] = true;
                if (expect(',')) continue;
                if (expect('}')) break;
                return fail("expected `,` or `}`");
            }
        } else {
            p_++;
        }
        ws();
        if (p_ != e_) return fail("trailing characters");
        for (int i = 0; i < 8; i++)
            if (!have[i]) return fail(std::string("missing field `") + names[i] + "`");
        return true;
    }

  private:
    const char* p_;
    const char* e_;

    bool fail(const std::string& m) {
        if (err.empty()) err = m;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool peek(char c) {
        ws();
        return p_ < e_ && *p_ == c;
    }
    bool expect(char c) {
        if (!peek(c)) return false;
        p_++;
        return true;
    }
    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) {
            o += (char)cp;
        } else if (cp < 0x800) {
            o += (char)(0xc0 | (cp >> 6));
            o += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            o += (char)(0xe0 | (cp >> 12));
            o += (char)(0x80 | ((cp >> 6) & 0x3f));
            o += (char)(0x80 | (cp & 0x3f));
        } else {
            o += (char)(0xf0 | (cp >> 18));
            o += (char)(0x80 | ((cp >> 12) & 0x3f));
            o += (char)(0x80 | ((cp >> 6) & 0x3f));
            o += (char)(0x80 | (cp & 0x3f));
        }
    }
    bool hex4(uint32_t& v) {
        if (e_ - p_ < 4) return fail("EOF while parsing a string");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("invalid escape");
        }
        return true;
    }
    // length of a valid UTF-8 sequence starting at p (0 if invalid)
    static int utf8_len(const unsigned char* p, const unsigned char* e) {
        const unsigned c = p[0];
        int n = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (n == 0 || e - p < n) return 0;
        uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1f) : n == 3 ? (c & 0x0f) : (c & 0x07);
        for (int i = 1; i < n; i++) {
            if ((p[i] & 0xc0) != 0x80) return 0;
            cp = (cp << 6) | (p[i] & 0x3f);
        }
        const uint32_t min[5] = {0, 0, 0x80, 0x800, 0x10000};
        if (cp < min[n] || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return 0;
        return n;
    }
    bool string(std::string& out) {
        out.clear();
        if (p_ >= e_ || *p_ != '"') return fail("expected a string");
        p_++;
        while (p_ < e_) {
            const unsigned char c = (unsigned char)*p_;
            if (c == '"') {
                p_++;
                return true;
            }
            if (c < 0x20) return fail("control character (\\u0000-\\u001F) found while parsing a string");
            if (c != '\\') {
                const int n = utf8_len((const unsigned char*)p_, (const unsigned char*)e_);
                if (n == 0) return fail("invalid unicode code point");
                out.append(p_, n);
                p_ += n;
                continue;
            }
            if (++p_ >= e_) break;
            const char x = *p_++;
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
                    if (cp >= 0xdc00 && cp <= 0xdfff) return fail("lone leading surrogate in hex escape");
                    if (cp >= 0xd800 && cp <= 0xdbff) {
                        uint32_t lo;
                        if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u')
                            return fail("unexpected end of hex escape");
                        p_ += 2;
                        if (!hex4(lo)) return false;
                        if (lo < 0xdc00 || lo > 0xdfff) return fail("lone leading surrogate in hex escape");
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
        return fail("EOF while parsing a string");
    }
    // a JSON number that must be a non-negative integer no larger than `max`
    bool integer(uint64_t& v, uint64_t max, const char* what) {
        ws();
        const char* s = p_;
        if (p_ < e_ && *p_ == '-') return fail(std::string("invalid value: integer, expected ") + what);
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail(std::string("invalid type, expected ") + what);
        if (*p_ == '0' && p_ + 1 < e_ && p_[1] >= '0' && p_[1] <= '9') return fail("invalid number");
        v = 0;
        bool over = false;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_++ - '0');
            if (v > (UINT64_MAX - d) / 10) over = true;
            v = v * 10 + d;
        }
        if (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E'))
            return fail(std::string("invalid type: floating point, expected ") + what);
        if (over || v > max) return fail(std::string("invalid value: integer, expected ") + what);
        (void)s;
        return true;
    }
    bool usize(uint64_t& v) { return integer(v, UINT64_MAX, "usize"); }
    bool u32_array(std::vector<uint32_t>& out) {
        out.clear();
        if (!expect('[')) return fail("invalid type, expected a sequence");
        if (expect(']')) return true;
        for (;;) {
            uint64_t v;
            if (!integer(v, 0xffffffffull, "u32")) return false;
            out.push_back((uint32_t)v);
            if (expect(',')) continue;
            if (expect(']')) return true;
            return fail("expected `,` or `]`");
        }
    }
    bool dtype(int& dt) {
        std::string s;
        ws();
        if (!string(s)) return false;
        if (s == "F32") dt = FLOUR_DTYPE_F32;
        else if (s == "F16") dt = FLOUR_DTYPE_F16;
        else if (s == "BF16") dt = FLOUR_DTYPE_BF16;
        else return fail("unknown variant `" + s + "`, expected one of `F32`, `F16`, `BF16`");
        return true;
    }
    bool skip_value(int depth) {
        if (depth > 128) return fail("recursion limit exceeded");
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        const char c = *p_;
        if (c == '"') {
            std::string tmp;
            return string(tmp);
        }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            p_++;
            if (expect(close)) return true;
            for (;;) {
                if (c == '{') {
                    std::string k;
                    ws();
                    if (!string(k) || !expect(':')) return fail("expected `:`");
                }
                if (!skip_value(depth + 1)) return false;
                if (expect(',')) continue;
                if (expect(close)) return true;
                return fail("expected `,` or a closing bracket");
            }
        }
        for (const char* lit : {"true", "false", "null"}) {
            const size_t n = strlen(lit);
            if ((size_t)(e_ - p_) >= n && memcmp(p_, lit, n) == 0) {
                p_ += n;
                return true;
            }
        }
        if (c == '-' || (c >= '0' && c <= '9')) {  // any JSON number
            if (*p_ == '-') p_++;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("invalid number");
            while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' ||
                               *p_ == 'E' || *p_ == '+' || *p_ == '-'))
                p_++;
            return true;
        }
        return fail("expected value");
    }
};

}  // namespace flkv
}  // namespace flour
