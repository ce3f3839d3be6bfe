// Parser of the JSON header of a safetensors file, the reference's on-disk
// weight format (scripts/phone_pipeline_nd.py:15-43 reads it in Python,
// vulkan/safetensors_reader.h:33-70 in C++): a u64 little-endian header
// length, then a JSON object mapping tensor names to {dtype, shape,
// data_offsets}, plus an optional "__metadata__" object.
//
// Host-only C++17 with no HIP dependency, so the same code is compiled into
// the library (weights.hip) and into a sanitizer build for the CPU tests.
// Every read is bounded by the header's end, nesting is capped, and every
// size product is checked for overflow before it is used; a malformed
// header yields an error message, never a crash.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace anima_hip {
namespace st {

// dtype codes as the reference's vk_weight_add takes them (phone_pipeline_nd.py:31).
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

inline int dtype_code(const std::string &s)
{
    if (s == "F32")
        return kF32;
    if (s == "F16")
        return kF16;
    if (s == "BF16")
        return kBF16;
    return -1;
}

inline int dtype_bytes(int code) { return code == kF32 ? 4 : 2; }

// Deepest nesting of arrays and objects accepted in values the parser skips
// (__metadata__ and unknown fields).  Real headers nest two levels.
constexpr int kMaxDepth = 64;

// A small JSON reader for the header: objects, strings, integers and arrays;
// anything else in a value (floats, booleans, null) is skipped.
class Json {
public:
    Json(const char *p, const char *end) : p_(p), end_(end) {}

    bool ok() const { return err_.empty(); }
    const std::string &error() const { return err_; }

    void ws()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r'))
            ++p_;
    }
    bool peek(char c)
    {
        ws();
        return p_ < end_ && *p_ == c;
    }
    bool expect(char c)
    {
        ws();
        if (p_ < end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return bad(std::string("expected '") + c + "'");
    }
    bool string(std::string &out)
    {
        if (!expect('"'))
            return false;
        out.clear();
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\') {
                if (p_ >= end_)
                    break;
                c = *p_++;
                switch (c) {
                case 'n': c = '\n'; break;
                case 't': c = '\t'; break;
                case 'r': c = '\r'; break;
                case 'b': c = '\b'; break;
                case 'f': c = '\f'; break;
                case 'u':  // keep the escape as text; names here are ASCII
                    out += "\\u";
                    continue;
                default: break;
                }
            }
            out += c;
        }
        if (p_ >= end_)
            return bad("unterminated string");
        ++p_;
        return true;
    }
    bool integer(int64_t &v)
    {
        ws();
        bool neg = false;
        if (p_ < end_ && *p_ == '-') {
            neg = true;
            ++p_;
        }
        if (p_ >= end_ || *p_ < '0' || *p_ > '9')
            return bad("expected an integer");
        v = 0;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            if (v > (INT64_MAX - 9) / 10)
                return bad("integer overflow");
            v = v * 10 + (*p_++ - '0');
        }
        if (neg)
            v = -v;
        return true;
    }
    bool int_array(std::vector<int64_t> &out)
    {
        out.clear();
        if (!expect('['))
            return false;
        if (peek(']'))
            return expect(']');
        for (;;) {
            int64_t v;
            if (!integer(v))
                return false;
            out.push_back(v);
            if (peek(','))
                expect(',');
            else
                return expect(']');
        }
    }
    // Skip any JSON value nested at most kMaxDepth levels deep.  Iterative:
    // one byte of state per open bracket, so a hostile header cannot exhaust
    // the stack.
    bool skip()
    {
        std::string open;  // closing bracket of every enclosing array/object
        for (;;) {
            ws();
            if (p_ >= end_)
                return bad("unexpected end");
            // One value.
            if (*p_ == '"') {
                std::string s;
                if (!string(s))
                    return false;
            } else if (*p_ == '{' || *p_ == '[') {
                if (open.size() >= size_t(kMaxDepth))
                    return bad("nesting deeper than " + std::to_string(kMaxDepth));
                const bool obj = *p_ == '{';
                open.push_back(obj ? '}' : ']');
                ++p_;
                if (peek(open.back())) {
                    ++p_;
                    open.pop_back();
                } else {
                    if (obj && !key())
                        return false;
                    continue;  // first member's value
                }
            } else {
                const char *start = p_;
                while (p_ < end_ && *p_ != ',' && *p_ != '}' && *p_ != ']')
                    ++p_;
                if (p_ == start)
                    return bad("empty value");
            }
            // After a value: next member, or close enclosing containers.
            for (;;) {
                if (open.empty())
                    return true;
                if (peek(',')) {
                    ++p_;
                    if (open.back() == '}' && !key())
                        return false;
                    break;
                }
                if (!expect(open.back()))
                    return false;
                open.pop_back();
            }
        }
    }
    bool at_end()
    {
        ws();
        return p_ >= end_;
    }

private:
    // An object member's key and colon.
    bool key()
    {
        std::string k;
        return string(k) && expect(':');
    }
    bool bad(const std::string &m)
    {
        if (err_.empty())
            err_ = m;
        return false;
    }
    const char *p_, *end_;
    std::string err_;
};

// One tensor of the header.
struct Entry {
    std::string name;  // as in the file
    int dtype = -1;
    std::vector<int64_t> shape;
    size_t begin = 0, bytes = 0;  // inside the data region
};

// Parse and validate the header [p, end) of a file whose data region holds
// data_len bytes.  On failure returns false with the reason in `err`.
inline bool parse_header(const char *p, const char *end, size_t data_len, std::vector<Entry> &out,
                         std::string &err)
{
    out.clear();
    Json js(p, end);
    const auto fail = [&err](const std::string &m) {
        err = m;
        return false;
    };
    if (!js.expect('{'))
        return fail("weights: header is not a JSON object: " + js.error());
    if (!js.peek('}')) {
        for (;;) {
            std::string key;
            if (!js.string(key) || !js.expect(':'))
                return fail("weights: bad header entry: " + js.error());
            if (key == "__metadata__") {
                if (!js.skip())
                    return fail("weights: bad __metadata__: " + js.error());
            } else {
                Entry t;
                t.name = key;
                std::vector<int64_t> offs;
                bool has_dtype = false, has_shape = false, has_offs = false;
                if (!js.expect('{'))
                    return fail("weights: tensor '" + key + "' is not an object");
                if (!js.peek('}')) {
                    for (;;) {
                        std::string f;
                        if (!js.string(f) || !js.expect(':'))
                            return fail("weights: bad field in '" + key + "': " + js.error());
                        if (f == "dtype") {
                            std::string d;
                            if (!js.string(d))
                                return fail("weights: bad dtype of '" + key + "'");
                            t.dtype = dtype_code(d);
                            if (t.dtype < 0)
                                return fail("weights: tensor '" + key +
                                            "' has unsupported dtype " + d);
                            has_dtype = true;
                        } else if (f == "shape") {
                            if (!js.int_array(t.shape))
                                return fail("weights: bad shape of '" + key + "': " + js.error());
                            has_shape = true;
                        } else if (f == "data_offsets") {
                            if (!js.int_array(offs) || offs.size() != 2)
                                return fail("weights: bad data_offsets of '" + key + "'");
                            has_offs = true;
                        } else if (!js.skip()) {
                            return fail("weights: bad field in '" + key + "': " + js.error());
                        }
                        if (js.peek(','))
                            js.expect(',');
                        else if (!js.expect('}'))
                            return fail("weights: bad tensor entry '" + key + "': " + js.error());
                        else
                            break;
                    }
                } else {
                    js.expect('}');
                }
                if (!has_dtype || !has_shape || !has_offs)
                    return fail("weights: tensor '" + key +
                                "' lacks dtype, shape or data_offsets");
                // Element count, then byte count, each checked against
                // overflow before the product is formed.
                const size_t esz = size_t(dtype_bytes(t.dtype));
                uint64_t n = 1;
                for (int64_t d : t.shape) {
                    if (d < 0 || (d > 0 && n > uint64_t(INT64_MAX) / uint64_t(d)))
                        return fail("weights: bad shape of '" + key + "'");
                    n *= uint64_t(d);
                }
                if (n > uint64_t(SIZE_MAX) / esz)
                    return fail("weights: shape of '" + key + "' is too large");
                if (offs[0] < 0 || offs[1] < offs[0] || uint64_t(offs[1]) > uint64_t(data_len))
                    return fail("weights: data_offsets of '" + key + "' lie outside the file");
                t.begin = size_t(offs[0]);
                t.bytes = size_t(offs[1] - offs[0]);
                const size_t need = size_t(n) * esz;
                if (t.bytes != need)
                    return fail("weights: '" + key + "' holds " + std::to_string(t.bytes) +
                                " bytes, its dtype and shape need " + std::to_string(need));
                out.push_back(std::move(t));
            }
            if (js.peek(','))
                js.expect(',');
            else if (!js.expect('}'))
                return fail("weights: bad header: " + js.error());
            else
                break;
        }
    } else {
        js.expect('}');
    }
    if (!js.at_end())
        return fail("weights: trailing bytes after the header object");
    return true;
}

}  // namespace st
}  // namespace anima_hip
