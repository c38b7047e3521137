// The reference's serialization format: FieldValue tree, binary "TS_B" v1 and
// JSON.  Citations are paths under train-station/src/serialization/.
#include "ts_serial.h"

#include <algorithm>
#include <cctype>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <thread>

#include "ts_host.h"

namespace ts {
namespace ser {

// ---- values ----------------------------------------------------------------------

Value Value::boolean(bool v) {
    Value x;
    x.kind = Kind::Bool;
    x.u = v ? 1 : 0;
    return x;
}
Value Value::usize(uint64_t v) {
    Value x;
    x.kind = Kind::Usize;
    x.u = v;
    return x;
}
Value Value::f32(float v) {
    Value x;
    x.kind = Kind::F32;
    uint32_t b;
    std::memcpy(&b, &v, 4);
    x.u = b;
    return x;
}
Value Value::string(std::string v) {
    Value x;
    x.kind = Kind::String;
    x.s = std::move(v);
    return x;
}
Value Value::array(std::vector<Value> v) {
    Value x;
    x.kind = Kind::Array;
    x.items = std::move(v);
    return x;
}
Value Value::none() { return Value(); }
Value Value::some(Value v) {
    Value x;
    x.kind = Kind::Optional;
    x.items.push_back(std::move(v));
    return x;
}
Value Value::object(Fields f) {
    Value x;
    x.kind = Kind::Object;
    x.fields = std::move(f);
    return x;
}
Value Value::enum_unit(std::string variant) {
    Value x;
    x.kind = Kind::Enum;
    x.s = std::move(variant);
    return x;
}
Value Value::binary_object(std::vector<uint8_t> b) {
    Value x;
    x.kind = Kind::BinaryObject;
    x.bytes = std::move(b);
    return x;
}
Value Value::float_values(std::vector<float> v) {
    Value x;
    x.kind = Kind::Array;
    x.form = ArrayForm::Floats;
    x.count = v.size();
    x.floats = std::move(v);
    return x;
}

size_t Value::array_size() const { return form == ArrayForm::Items ? items.size() : count; }

const Value *Value::member(const std::string &name) const {
    const Value *found = nullptr;
    for (const auto &kv : fields)
        if (kv.first == name) found = &kv.second;
    return found;
}

namespace {

const char *kind_name(Kind k) {
    static const char *names[] = {"Bool",   "I8",     "I16",        "I32",          "I64",
                                  "U8",     "U16",    "U32",        "U64",          "Usize",
                                  "F32",    "F64",    "String",     "Bytes",        "JsonObject",
                                  "BinaryObject", "Array", "Optional", "Object",     "Enum"};
    const unsigned i = static_cast<unsigned>(k);
    return i < 20 ? names[i] : "?";
}

[[noreturn]] void fail(const std::string &field, const std::string &msg) {
    throw Error("Validation failed for field '" + field + "': " + msg);
}

int64_t as_signed(const Value &v) {
    switch (v.kind) {
        case Kind::I8: return static_cast<int8_t>(v.u);
        case Kind::I16: return static_cast<int16_t>(v.u);
        case Kind::I32: return static_cast<int32_t>(v.u);
        default: return static_cast<int64_t>(v.u);
    }
}

// The FieldValue the JSON reader makes of a number (json/structs.rs:232-256).
// Integral values are cast to i64 (Rust `as`: saturating) and take the
// narrowest signed type; the branch meant to prefer usize compares against
// `usize::MAX as i64`, which is -1, so it never applies.  Other values are F64.
Value number_value(double n) {
    Value x;
    if (n - std::trunc(n) == 0.0) {
        int64_t i;
        if (n >= 9223372036854775807.0) i = std::numeric_limits<int64_t>::max();
        else if (n <= -9223372036854775808.0) i = std::numeric_limits<int64_t>::min();
        else i = static_cast<int64_t>(n);
        if (i >= -128 && i <= 127) x.kind = Kind::I8;
        else if (i >= -32768 && i <= 32767) x.kind = Kind::I16;
        else if (i >= -2147483648LL && i <= 2147483647LL) x.kind = Kind::I32;
        else x.kind = Kind::I64;
        x.u = static_cast<uint64_t>(i);
    } else {
        x.kind = Kind::F64;
        std::memcpy(&x.u, &n, 8);
    }
    return x;
}

float f32_of_number(double n) {  // as_f32(number_value(n))
    const Value v = number_value(n);
    if (v.kind == Kind::F64) return static_cast<float>(n);
    return static_cast<float>(as_signed(v));
}

}  // namespace

bool as_bool(const Value &v, const std::string &field) {
    if (v.kind != Kind::Bool) fail(field, std::string("Expected bool, found ") + kind_name(v.kind));
    return v.u != 0;
}

uint64_t as_usize(const Value &v, const std::string &field) {
    switch (v.kind) {
        case Kind::Usize:
        case Kind::U8:
        case Kind::U16:
        case Kind::U32:
        case Kind::U64: return v.u;
        case Kind::I8:
        case Kind::I16:
        case Kind::I32:
        case Kind::I64: {
            const int64_t i = as_signed(v);
            if (i < 0) fail(field, "Cannot convert negative " + std::string(kind_name(v.kind)) + " " +
                                       std::to_string(i) + " to usize");
            return static_cast<uint64_t>(i);
        }
        default: fail(field, std::string("Expected usize, found ") + kind_name(v.kind));
    }
}

float as_f32(const Value &v, const std::string &field) {
    switch (v.kind) {
        case Kind::F32: {
            const uint32_t b = static_cast<uint32_t>(v.u);
            float f;
            std::memcpy(&f, &b, 4);
            return f;
        }
        case Kind::F64: {
            double d;
            std::memcpy(&d, &v.u, 8);
            return static_cast<float>(d);
        }
        case Kind::I8:
        case Kind::I16:
        case Kind::I32:
        case Kind::I64: return static_cast<float>(as_signed(v));
        case Kind::U8:
        case Kind::U16:
        case Kind::U32:
        case Kind::U64:
        case Kind::Usize: return static_cast<float>(v.u);
        default: fail(field, std::string("Expected f32, found ") + kind_name(v.kind));
    }
}

const std::string &as_json_object(const Value &v, const std::string &field) {
    if (v.kind != Kind::JsonObject) fail(field, std::string("Expected JSON object, found ") + kind_name(v.kind));
    return v.s;
}

void array_to_f32(const Value &v, const std::string &field, float *out) {
    if (v.kind != Kind::Array) fail(field, std::string("Expected Vec<f32>, found ") + kind_name(v.kind));
    switch (v.form) {
        case ArrayForm::Items:
            for (size_t i = 0; i < v.items.size(); ++i)
                out[i] = as_f32(v.items[i], field + "[" + std::to_string(i) + "]");
            return;
        case ArrayForm::Records: {
            const uint8_t *r = v.buf->data() + v.offset;
            for (size_t i = 0; i < v.count; ++i) std::memcpy(out + i, r + 5 * i + 1, 4);
            return;
        }
        case ArrayForm::Numbers:
            for (size_t i = 0; i < v.count; ++i) out[i] = f32_of_number(v.numbers[i]);
            return;
        case ArrayForm::Floats: std::memcpy(out, v.floats.data(), 4 * v.count); return;
    }
}

std::vector<uint64_t> array_to_usize(const Value &v, const std::string &field) {
    if (v.kind != Kind::Array) fail(field, std::string("Expected Vec<usize>, found ") + kind_name(v.kind));
    std::vector<uint64_t> out(v.array_size());
    switch (v.form) {
        case ArrayForm::Items:
            for (size_t i = 0; i < out.size(); ++i) out[i] = as_usize(v.items[i], field);
            break;
        case ArrayForm::Numbers:
            for (size_t i = 0; i < out.size(); ++i) out[i] = as_usize(number_value(v.numbers[i]), field);
            break;
        default: fail(field, "Expected usize in array, found F32");
    }
    return out;
}

// ---- binary ------------------------------------------------------------------------

namespace {

constexpr uint32_t kMagic = 0x54535F42;  // "TS_B" (binary/types.rs:13)
constexpr uint32_t kVersion = 1;         // binary/types.rs:20
constexpr uint32_t kTensorType = 0x1001; // binary/types.rs:44
constexpr size_t kHeaderBytes = 24;      // magic, version, checksum, data length (u64), type

struct BinWriter {
    std::vector<uint8_t> &out;
    void raw(const void *p, size_t n) {
        const uint8_t *b = static_cast<const uint8_t *>(p);
        out.insert(out.end(), b, b + n);
    }
    void u8(uint8_t v) { out.push_back(v); }
    void u16(uint16_t v) { uint8_t b[2] = {uint8_t(v), uint8_t(v >> 8)}; raw(b, 2); }
    void u32(uint32_t v) {
        uint8_t b[4];
        for (int i = 0; i < 4; ++i) b[i] = uint8_t(v >> (8 * i));
        raw(b, 4);
    }
    void u64(uint64_t v) {
        uint8_t b[8];
        for (int i = 0; i < 8; ++i) b[i] = uint8_t(v >> (8 * i));
        raw(b, 8);
    }
    // binary/writer.rs write_string: u32 byte length + UTF-8 bytes
    void str(const std::string &s) {
        u32(static_cast<uint32_t>(s.size()));
        raw(s.data(), s.size());
    }
    // write_vec_u8: u64 length + bytes
    void vec(const std::vector<uint8_t> &b) {
        u64(b.size());
        raw(b.data(), b.size());
    }
};

void write_value(BinWriter &w, const Value &v);

void write_number_value(BinWriter &w, double n) { write_value(w, number_value(n)); }

// binary/structs.rs:147-290
void write_value(BinWriter &w, const Value &v) {
    w.u8(static_cast<uint8_t>(v.kind));
    switch (v.kind) {
        case Kind::Bool: w.u8(v.u ? 1 : 0); break;
        case Kind::I8:
        case Kind::U8: w.u8(static_cast<uint8_t>(v.u)); break;
        case Kind::I16:
        case Kind::U16: w.u16(static_cast<uint16_t>(v.u)); break;
        case Kind::I32:
        case Kind::U32:
        case Kind::F32: w.u32(static_cast<uint32_t>(v.u)); break;
        case Kind::I64:
        case Kind::U64:
        case Kind::Usize:
        case Kind::F64: w.u64(v.u); break;
        case Kind::String:
        case Kind::JsonObject: w.str(v.s); break;
        case Kind::Bytes:
        case Kind::BinaryObject: w.vec(v.bytes); break;
        case Kind::Array:
            w.u64(v.array_size());
            switch (v.form) {
                case ArrayForm::Items:
                    for (const Value &e : v.items) write_value(w, e);
                    break;
                case ArrayForm::Records:
                    if (v.buf) w.raw(v.buf->data() + v.offset, 5 * v.count);
                    else w.out.resize(w.out.size() + 5 * v.count);  // filled in by the caller
                    break;
                case ArrayForm::Numbers:
                    for (double n : v.numbers) write_number_value(w, n);
                    break;
                case ArrayForm::Floats:
                    for (float f : v.floats) {
                        uint32_t b;
                        std::memcpy(&b, &f, 4);
                        w.u8(static_cast<uint8_t>(Kind::F32));
                        w.u32(b);
                    }
                    break;
            }
            break;
        case Kind::Optional:
            w.u8(v.items.empty() ? 0 : 1);
            if (!v.items.empty()) write_value(w, v.items[0]);
            break;
        case Kind::Object:
            w.u64(v.fields.size());
            for (const auto &kv : v.fields) {
                w.str(kv.first);
                write_value(w, kv.second);
            }
            break;
        case Kind::Enum:
            w.str(v.s);
            w.u8(v.items.empty() ? 0 : 1);
            if (!v.items.empty()) write_value(w, v.items[0]);
            break;
    }
}

struct BinReader {
    const uint8_t *p;
    size_t n, pos;
    const std::shared_ptr<const std::vector<uint8_t>> &buf;

    [[noreturn]] void err(const std::string &msg) const {
        throw Error("Binary format error: " + msg + " (at byte " + std::to_string(pos) + ")");
    }
    void need(size_t k) const {
        if (n - pos < k) err("unexpected end of data (failed to fill whole buffer)");
    }
    uint8_t u8() {
        need(1);
        return p[pos++];
    }
    uint16_t u16() {
        need(2);
        uint16_t v = uint16_t(p[pos] | (p[pos + 1] << 8));
        pos += 2;
        return v;
    }
    uint32_t u32() {
        need(4);
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) v |= uint32_t(p[pos + i]) << (8 * i);
        pos += 4;
        return v;
    }
    uint64_t u64() {
        need(8);
        uint64_t v = 0;
        for (int i = 0; i < 8; ++i) v |= uint64_t(p[pos + i]) << (8 * i);
        pos += 8;
        return v;
    }
    bool boolean() {  // reader.rs read_bool: 0 or 1
        const uint8_t b = u8();
        if (b > 1) {
            --pos;
            err("Invalid boolean value: " + std::to_string(b));
        }
        return b == 1;
    }
    std::string str() {  // reader.rs read_string: at most 1,000,000 bytes of UTF-8
        const uint32_t len = u32();
        if (len > 1000000u) {
            pos -= 4;
            err("String length " + std::to_string(len) + " exceeds maximum allowed");
        }
        need(len);
        std::string s(reinterpret_cast<const char *>(p + pos), len);
        if (!valid_utf8(p + pos, len)) err("Invalid UTF-8 string");
        pos += len;
        return s;
    }
    std::vector<uint8_t> vec() {  // read_vec_u8: at most 100,000,000 bytes
        const uint64_t len = u64();
        if (len > 100000000ull) {
            pos -= 8;
            err("Collection length " + std::to_string(len) + " exceeds maximum allowed");
        }
        need(len);
        std::vector<uint8_t> b(p + pos, p + pos + len);
        pos += len;
        return b;
    }
    static bool valid_utf8(const uint8_t *s, size_t n) {
        size_t i = 0;
        while (i < n) {
            const uint8_t c = s[i];
            if (c < 0x80) { ++i; continue; }
            size_t k;
            uint32_t cp;
            if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; }
            else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; }
            else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; }
            else return false;
            if (n - i <= k) return false;
            for (size_t j = 1; j <= k; ++j) {
                if ((s[i + j] & 0xC0) != 0x80) return false;
                cp = (cp << 6) | (s[i + j] & 0x3F);
            }
            static const uint32_t min_cp[4] = {0, 0x80, 0x800, 0x10000};
            if (cp < min_cp[k] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
            i += k + 1;
        }
        return true;
    }
};

Value read_value(BinReader &r, int depth);

Value read_array(BinReader &r, int depth) {
    Value v;
    v.kind = Kind::Array;
    const uint64_t count = r.u64();
    // All-F32 arrays (tensor data) stay as records inside the buffer.
    if (count > 0 && (r.n - r.pos) / 5 >= count) {
        const uint8_t *q = r.p + r.pos;
        bool all = true;
        for (uint64_t i = 0; i < count && all; ++i) all = q[5 * i] == static_cast<uint8_t>(Kind::F32);
        if (all) {
            v.form = ArrayForm::Records;
            v.count = count;
            v.buf = r.buf;
            v.offset = r.pos;
            r.pos += 5 * count;
            return v;
        }
    }
    for (uint64_t i = 0; i < count; ++i) v.items.push_back(read_value(r, depth + 1));
    return v;
}

// binary/structs.rs:349-460
Value read_value(BinReader &r, int depth) {
    if (depth > 256) r.err("nesting deeper than 256 levels");
    const uint8_t tag = r.u8();
    Value v;
    if (tag > static_cast<uint8_t>(Kind::Enum)) {
        --r.pos;
        r.err("Unknown type tag: " + std::to_string(tag));
    }
    v.kind = static_cast<Kind>(tag);
    switch (v.kind) {
        case Kind::Bool: v.u = r.boolean() ? 1 : 0; break;
        case Kind::I8: v.u = static_cast<uint64_t>(static_cast<int64_t>(static_cast<int8_t>(r.u8()))); break;
        case Kind::U8: v.u = r.u8(); break;
        case Kind::I16: v.u = static_cast<uint64_t>(static_cast<int64_t>(static_cast<int16_t>(r.u16()))); break;
        case Kind::U16: v.u = r.u16(); break;
        case Kind::I32: v.u = static_cast<uint64_t>(static_cast<int64_t>(static_cast<int32_t>(r.u32()))); break;
        case Kind::U32:
        case Kind::F32: v.u = r.u32(); break;
        case Kind::I64:
        case Kind::U64:
        case Kind::Usize:
        case Kind::F64: v.u = r.u64(); break;
        case Kind::String:
        case Kind::JsonObject: v.s = r.str(); break;
        case Kind::Bytes:
        case Kind::BinaryObject: v.bytes = r.vec(); break;
        case Kind::Array: return read_array(r, depth);
        case Kind::Optional:
            if (r.boolean()) v.items.push_back(read_value(r, depth + 1));
            break;
        case Kind::Object: {
            const uint64_t count = r.u64();
            for (uint64_t i = 0; i < count; ++i) {
                std::string key = r.str();
                Value val = read_value(r, depth + 1);
                bool replaced = false;  // a HashMap keeps the last value of a repeated key
                for (auto &kv : v.fields)
                    if (kv.first == key) {
                        kv.second = std::move(val);
                        replaced = true;
                        break;
                    }
                if (!replaced) v.fields.emplace_back(std::move(key), std::move(val));
            }
            break;
        }
        case Kind::Enum:
            v.s = r.str();
            if (r.boolean()) v.items.push_back(read_value(r, depth + 1));
            break;
    }
    return v;
}

}  // namespace

// binary/header.rs:41-53 and :120-162, binary/structs.rs:90-120
std::vector<uint8_t> to_binary(const Fields &fields) {
    std::vector<uint8_t> out;
    BinWriter w{out};
    w.u32(kMagic);
    w.u32(kVersion);
    w.u32(0);  // checksum placeholder, never filled in by the reference
    w.u64(0);  // data length, patched below
    w.u32(kTensorType);
    w.u64(fields.size());
    for (const auto &kv : fields) {
        w.str(kv.first);
        write_value(w, kv.second);
    }
    const uint64_t len = out.size() - kHeaderBytes;
    for (int i = 0; i < 8; ++i) out[12 + i] = uint8_t(len >> (8 * i));
    return out;
}

// binary/header.rs:76-106 and :178-215, binary/structs.rs:293-312
Fields from_binary(std::shared_ptr<const std::vector<uint8_t>> data) {
    BinReader r{data->data(), data->size(), 0, data};
    const uint32_t magic = r.u32();
    if (magic != kMagic) {
        char msg[96];
        std::snprintf(msg, sizeof msg, "Invalid magic number: expected 0x%08X, found 0x%08X", kMagic, magic);
        throw Error(msg);
    }
    const uint32_t version = r.u32();
    if (version != kVersion)
        throw Error("Version mismatch: expected " + std::to_string(kVersion) + ", found " +
                    std::to_string(version));
    (void)r.u32();  // checksum, not validated (header.rs:99)
    const uint64_t data_length = r.u64();
    const uint32_t type = r.u32();
    if (type < 0x1001 || type > 0x1005) {
        char msg[64];
        std::snprintf(msg, sizeof msg, "Unknown object type: 0x%08X", type);
        r.err(msg);
    }
    if (type != kTensorType) r.err("Object type mismatch: expected Tensor");
    if (data_length > r.n - r.pos)
        r.err("Data length mismatch: header claims " + std::to_string(data_length) +
              " bytes of data, but only " + std::to_string(r.n - r.pos) + " bytes available");
    const uint64_t count = r.u64();
    Fields f;
    for (uint64_t i = 0; i < count; ++i) {
        std::string name = r.str();
        Value v = read_value(r, 0);
        bool replaced = false;
        for (auto &kv : f)
            if (kv.first == name) {
                kv.second = std::move(v);
                replaced = true;
                break;
            }
        if (!replaced) f.emplace_back(std::move(name), std::move(v));
    }
    return f;
}

// ---- JSON writer -------------------------------------------------------------------

namespace {

// Rust's Display of a finite non-zero float: the shortest digits that read
// back as the same value (std::to_chars gives them), laid out in fixed
// notation without an exponent.
template <class F>
void append_display(std::string &out, F v) {
    if (std::isnan(v)) {
        out += "NaN";
        return;
    }
    if (std::isinf(v)) {
        out += v < 0 ? "-inf" : "inf";
        return;
    }
    if (v == 0) {
        out += std::signbit(v) ? "-0" : "0";
        return;
    }
    char buf[64];
    auto res = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
    const char *s = buf, *end = res.ptr;
    if (*s == '-') {
        out += '-';
        ++s;
    }
    const char *e = std::find(s, end, 'e');
    std::string digits;
    for (const char *c = s; c < e; ++c)
        if (*c != '.') digits += *c;
    int exp = 0;  // value = d.ddd * 10^exp; to_chars does not terminate the text
    if (e < end) std::from_chars(e + 1 + (e[1] == '+' ? 1 : 0), end, exp);
    const int k = static_cast<int>(digits.size());
    if (exp >= k - 1) {
        out += digits;
        out.append(static_cast<size_t>(exp - (k - 1)), '0');
    } else if (exp >= 0) {
        out.append(digits, 0, static_cast<size_t>(exp + 1));
        out += '.';
        out.append(digits, static_cast<size_t>(exp + 1), std::string::npos);
    } else {
        out += "0.";
        out.append(static_cast<size_t>(-exp - 1), '0');
        out += digits;
    }
}

// json/structs.rs:80-95: integral values get ".0" (fract() == 0.0 holds for
// finite integral values, false for NaN and infinities)
template <class F>
void append_json_float(std::string &out, F v) {
    append_display(out, v);
    if (std::isfinite(v) && std::trunc(v) == v) out += ".0";
}

// json/escape.rs escape_string
void append_escaped(std::string &out, const std::string &s) {
    size_t i = 0;
    while (i < s.size()) {
        const unsigned char c = static_cast<unsigned char>(s[i]);
        switch (c) {
            case '"': out += "\\\""; ++i; continue;
            case '\\': out += "\\\\"; ++i; continue;
            case 0x08: out += "\\b"; ++i; continue;
            case 0x0c: out += "\\f"; ++i; continue;
            case '\n': out += "\\n"; ++i; continue;
            case '\r': out += "\\r"; ++i; continue;
            case '\t': out += "\\t"; ++i; continue;
            default: break;
        }
        // char::is_control: U+0000-U+001F and U+007F-U+009F (the latter are
        // two-byte sequences); other characters are copied whole
        size_t len = 1;
        if (c >= 0xF0) len = 4;
        else if (c >= 0xE0) len = 3;
        else if (c >= 0xC0) len = 2;
        if (i + len > s.size()) len = s.size() - i;
        uint32_t cp = c;
        if (len == 2) cp = ((c & 0x1Fu) << 6) | (static_cast<unsigned char>(s[i + 1]) & 0x3Fu);
        if (len <= 2 && (cp < 0x20 || (cp >= 0x7F && cp <= 0x9F))) {
            char b[8];
            std::snprintf(b, sizeof b, "\\u%04x", cp);
            out += b;
        } else {
            out.append(s, i, len);
        }
        i += len;
    }
}

void append_hex(std::string &out, const std::vector<uint8_t> &b) {
    static const char *hex = "0123456789abcdef";
    out += '"';
    for (uint8_t x : b) {
        out += hex[x >> 4];
        out += hex[x & 15];
    }
    out += '"';
}

void append_f32_list(std::string &out, const float *v, size_t n) {
    // large arrays are formatted in parallel, in order
    const size_t kPer = 1 << 18;
    unsigned threads = std::thread::hardware_concurrency();
    if (threads > 16) threads = 16;
    if (n < 2 * kPer || threads < 2) {
        for (size_t i = 0; i < n; ++i) {
            if (i) out += ',';
            append_json_float(out, v[i]);
        }
        return;
    }
    std::vector<std::string> parts(threads);
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t)
        pool.emplace_back([&, t] {
            const size_t lo = n * t / threads, hi = n * (t + 1) / threads;
            std::string &s = parts[t];
            s.reserve((hi - lo) * 12);
            for (size_t i = lo; i < hi; ++i) {
                if (i) s += ',';
                append_json_float(s, v[i]);
            }
        });
    for (auto &th : pool) th.join();
    for (auto &s : parts) out += s;
}

void json_value(std::string &out, const Value &v) {
    switch (v.kind) {
        case Kind::Bool: out += v.u ? "true" : "false"; break;
        case Kind::I8:
        case Kind::I16:
        case Kind::I32:
        case Kind::I64: out += std::to_string(as_signed(v)); break;
        case Kind::U8:
        case Kind::U16:
        case Kind::U32:
        case Kind::U64:
        case Kind::Usize: out += std::to_string(v.u); break;
        case Kind::F32: append_json_float(out, as_f32(v, "")); break;
        case Kind::F64: {
            double d;
            std::memcpy(&d, &v.u, 8);
            append_json_float(out, d);
            break;
        }
        case Kind::String:
            out += '"';
            append_escaped(out, v.s);
            out += '"';
            break;
        case Kind::JsonObject: out += v.s; break;  // embedded as it is
        case Kind::Bytes:
        case Kind::BinaryObject: append_hex(out, v.bytes); break;
        case Kind::Array:
            out += '[';
            switch (v.form) {
                case ArrayForm::Items:
                    for (size_t i = 0; i < v.items.size(); ++i) {
                        if (i) out += ',';
                        json_value(out, v.items[i]);
                    }
                    break;
                case ArrayForm::Floats: append_f32_list(out, v.floats.data(), v.count); break;
                case ArrayForm::Records: {
                    std::vector<float> tmp(v.count);
                    array_to_f32(v, "", tmp.data());
                    append_f32_list(out, tmp.data(), v.count);
                    break;
                }
                case ArrayForm::Numbers:
                    for (size_t i = 0; i < v.count; ++i) {
                        if (i) out += ',';
                        json_value(out, number_value(v.numbers[i]));
                    }
                    break;
            }
            out += ']';
            break;
        case Kind::Optional:
            if (v.items.empty()) out += "null";
            else json_value(out, v.items[0]);
            break;
        case Kind::Object:
            out += '{';
            for (size_t i = 0; i < v.fields.size(); ++i) {
                if (i) out += ',';
                out += '"';
                append_escaped(out, v.fields[i].first);
                out += "\":";
                json_value(out, v.fields[i].second);
            }
            out += '}';
            break;
        case Kind::Enum:  // {"variant":"Name","data":...}, json/structs.rs:138-160
            out += "{\"variant\":\"";
            append_escaped(out, v.s);
            out += "\",\"data\":";
            if (v.items.empty()) out += "null";
            else json_value(out, v.items[0]);
            out += '}';
            break;
    }
}

}  // namespace

std::string format_f32(float v) {
    std::string s;
    append_json_float(s, v);
    return s;
}

void append_f32(std::string &out, float v) { append_json_float(out, v); }

// json/structs.rs:32-43: top-level names are written without escaping
std::string to_json(const Fields &fields) {
    std::string out = "{";
    for (size_t i = 0; i < fields.size(); ++i) {
        if (i) out += ',';
        out += '"';
        out += fields[i].first;
        out += "\":";
        json_value(out, fields[i].second);
    }
    out += '}';
    return out;
}

// ---- JSON parser -------------------------------------------------------------------

namespace {

struct JsonParser {
    const char *p, *end, *begin;

    [[noreturn]] void err(const std::string &msg) const {
        size_t line = 1, col = 1;
        for (const char *c = begin; c < p; ++c) {
            if (*c == '\n') {
                ++line;
                col = 1;
            } else {
                ++col;
            }
        }
        throw Error("JSON format error: " + msg + " at line " + std::to_string(line) + ", column " +
                    std::to_string(col));
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool lit(const char *w) {
        const size_t n = std::strlen(w);
        if (static_cast<size_t>(end - p) >= n && std::memcmp(p, w, n) == 0) {
            p += n;
            return true;
        }
        return false;
    }
    static void put_utf8(std::string &s, uint32_t cp) {
        if (cp < 0x80) s += char(cp);
        else if (cp < 0x800) {
            s += char(0xC0 | (cp >> 6));
            s += char(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += char(0xE0 | (cp >> 12));
            s += char(0x80 | ((cp >> 6) & 0x3F));
            s += char(0x80 | (cp & 0x3F));
        } else {
            s += char(0xF0 | (cp >> 18));
            s += char(0x80 | ((cp >> 12) & 0x3F));
            s += char(0x80 | ((cp >> 6) & 0x3F));
            s += char(0x80 | (cp & 0x3F));
        }
    }
    std::string string() {  // at the opening quote
        ++p;
        std::string s;
        while (true) {
            if (p >= end) err("Unterminated string");
            const char c = *p++;
            if (c == '"') break;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p >= end) err("Unterminated string");
            const char e = *p++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\x08'; break;
                case 'f': s += '\x0c'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        if (p >= end) err("Incomplete Unicode escape sequence");
                        const char h = *p++;
                        uint32_t d;
                        if (h >= '0' && h <= '9') d = h - '0';
                        else if (h >= 'a' && h <= 'f') d = h - 'a' + 10;
                        else if (h >= 'A' && h <= 'F') d = h - 'A' + 10;
                        else err(std::string("Invalid hex digit in Unicode escape: ") + h);
                        cp = cp * 16 + d;
                    }
                    if (cp >= 0xD800 && cp <= 0xDFFF)  // char::from_u32 rejects surrogates
                        err("Invalid Unicode code point: " + std::to_string(cp));
                    put_utf8(s, cp);
                    break;
                }
                default: err(std::string("Invalid escape sequence: \\") + e);
            }
        }
        return s;
    }
    double number() {  // json/parser.rs:290-365 grammar, value as Rust's f64 parse
        const char *start = p;
        if (p < end && *p == '-') ++p;
        if (p < end && *p == '0') ++p;
        else if (p < end && *p >= '0' && *p <= '9') {
            while (p < end && *p >= '0' && *p <= '9') ++p;
        } else err("Expected digit");
        if (p < end && *p == '.') {
            ++p;
            if (p >= end || *p < '0' || *p > '9') err("Expected digit after decimal point");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            if (p >= end || *p < '0' || *p > '9') err("Expected digit in exponent");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        const std::string tok(start, p);
        return std::strtod(tok.c_str(), nullptr);
    }
    bool at_number() const { return p < end && (*p == '-' || (*p >= '0' && *p <= '9')); }

    Value value(int depth) {
        if (depth > 256) err("nesting deeper than 256 levels");
        ws();
        if (p >= end) err("Unexpected end of input");
        const char c = *p;
        if (c == '{') return object(depth);
        if (c == '[') return array(depth);
        if (c == '"') {
            std::string s = string();
            // json/structs.rs:257-279: "0x" + an even number of hex digits becomes Bytes
            if (s.size() > 2 && s[0] == '0' && s[1] == 'x' && (s.size() - 2) % 2 == 0 &&
                std::all_of(s.begin() + 2, s.end(), [](char h) { return std::isxdigit(static_cast<unsigned char>(h)); })) {
                Value v;
                v.kind = Kind::Bytes;
                for (size_t i = 2; i < s.size(); i += 2)
                    v.bytes.push_back(static_cast<uint8_t>(std::stoi(s.substr(i, 2), nullptr, 16)));
                return v;
            }
            return Value::string(std::move(s));
        }
        if (lit("true")) return Value::boolean(true);
        if (lit("false")) return Value::boolean(false);
        if (lit("null")) return Value::none();
        if (at_number()) return number_value(number());
        err(std::string("Unexpected character '") + c + "'");
    }
    Value array(int depth) {
        ++p;
        Value v;
        v.kind = Kind::Array;
        ws();
        if (p < end && *p == ']') {
            ++p;
            return v;
        }
        // numbers are kept as f64 until an element of another type appears
        bool numeric = true;
        while (true) {
            ws();
            if (numeric && at_number()) {
                v.numbers.push_back(number());
            } else {
                if (numeric) {
                    numeric = false;
                    for (double n : v.numbers) v.items.push_back(number_value(n));
                    v.numbers.clear();
                }
                v.items.push_back(value(depth + 1));
            }
            ws();
            if (p >= end) err("Unterminated array");
            if (*p == ',') {
                ++p;
                continue;
            }
            if (*p == ']') {
                ++p;
                break;
            }
            err("Expected ',' or ']' in array");
        }
        if (numeric) {
            v.form = ArrayForm::Numbers;
            v.count = v.numbers.size();
        }
        return v;
    }
    Value object(int depth) {
        ++p;
        Value v;
        v.kind = Kind::Object;
        ws();
        if (p < end && *p == '}') {
            ++p;
        } else {
            while (true) {
                ws();
                if (p >= end || *p != '"') err("Expected string key in object");
                std::string key = string();
                ws();
                if (p >= end || *p != ':') err("Expected ':' after object key");
                ++p;
                Value val = value(depth + 1);
                bool replaced = false;
                for (auto &kv : v.fields)
                    if (kv.first == key) {
                        kv.second = std::move(val);
                        replaced = true;
                        break;
                    }
                if (!replaced) v.fields.emplace_back(std::move(key), std::move(val));
                ws();
                if (p >= end) err("Unterminated object");
                if (*p == ',') {
                    ++p;
                    continue;
                }
                if (*p == '}') {
                    ++p;
                    break;
                }
                err("Expected ',' or '}' in object");
            }
        }
        // json/structs.rs:283-307: exactly {"variant", "data"} is an enum
        if (v.fields.size() == 2 && v.member("variant") && v.member("data")) {
            const Value &var = *v.member("variant");
            if (var.kind != Kind::String) err("Enum variant must be a string");
            Value e = Value::enum_unit(var.s);
            Value data = *v.member("data");
            if (!(data.kind == Kind::Optional && data.items.empty())) e.items.push_back(std::move(data));
            return e;
        }
        return v;
    }
};

}  // namespace

// json/structs.rs:186-200
Fields from_json(const std::string &text) {
    JsonParser j{text.data(), text.data() + text.size(), text.data()};
    Value root = j.value(0);
    j.ws();
    if (j.p != j.end) j.err("Unexpected trailing characters");
    if (root.kind != Kind::Object) throw Error("JSON format error: Expected JSON object at root");
    return std::move(root.fields);
}

// ---- files ---------------------------------------------------------------------------

std::vector<uint8_t> read_file(const std::string &path) {
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) throw Error("IO error: cannot open " + path);
    std::vector<uint8_t> data;
    std::fseek(f, 0, SEEK_END);
    const long size = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    if (size > 0) {
        data.resize(static_cast<size_t>(size));
        if (std::fread(data.data(), 1, data.size(), f) != data.size()) {
            std::fclose(f);
            throw Error("IO error: short read from " + path);
        }
    }
    std::fclose(f);
    return data;
}

void write_file(const std::string &path, const void *data, size_t len) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) throw Error("IO error: cannot create " + path);
    const bool ok = std::fwrite(data, 1, len, f) == len;
    const bool closed = std::fclose(f) == 0;
    if (!ok || !closed) throw Error("IO error: short write to " + path);
}

}  // namespace ser
}  // namespace ts
