// The reference's serialization format, restated for the device-side Tensor
// and Adam: the FieldValue tree (serialization/core/types.rs), its binary
// encoding "TS_B" v1 (serialization/binary/{types,header,writer,reader,
// structs}.rs) and its JSON encoding (serialization/json/{structs,parser,
// escape}.rs).  Readers apply the reference's conversions and limits, so a
// file either side can read, both read the same way.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace ts {
namespace ser {

// FieldValue variants; the values are the binary type tags
// (binary/structs.rs:147-290).
enum class Kind : uint8_t {
    Bool = 0, I8 = 1, I16 = 2, I32 = 3, I64 = 4, U8 = 5, U16 = 6, U32 = 7, U64 = 8, Usize = 9,
    F32 = 10, F64 = 11, String = 12, Bytes = 13, JsonObject = 14, BinaryObject = 15,
    Array = 16, Optional = 17, Object = 18, Enum = 19,
};

struct Value;
using Fields = std::vector<std::pair<std::string, Value>>;

// How an Array holds its elements.  Tensor data is large, so besides a list
// of Values an Array can hold, without one Value per element:
//   Records - n binary F32 records ([10][f32 LE], 5 bytes each) inside `buf`
//   Numbers - JSON numbers as parsed (f64), converted on use as the reference does
//   Floats  - f32 values to be written
enum class ArrayForm : uint8_t { Items, Records, Numbers, Floats };

struct Value {
    Kind kind = Kind::Optional;  // default: Optional(None)
    uint64_t u = 0;              // Bool / integers (two's complement) / F32 and F64 bits
    std::string s;               // String, JsonObject, Enum variant
    std::vector<uint8_t> bytes;  // Bytes, BinaryObject
    std::vector<Value> items;    // Array items; Optional and Enum payload (0 or 1 item)
    Fields fields;               // Object, in order (a repeated key: the last one counts)
    ArrayForm form = ArrayForm::Items;
    size_t count = 0;                                   // element count of the compact forms
    std::shared_ptr<const std::vector<uint8_t>> buf;    // Records: the buffer they live in
    size_t offset = 0;                                  // Records: byte offset in buf
    std::vector<double> numbers;                        // Numbers
    std::vector<float> floats;                          // Floats

    static Value boolean(bool v);
    static Value usize(uint64_t v);
    static Value f32(float v);
    static Value string(std::string v);
    static Value array(std::vector<Value> v);
    static Value none();
    static Value some(Value v);
    static Value object(Fields f);
    static Value enum_unit(std::string variant);
    static Value binary_object(std::vector<uint8_t> b);
    static Value float_values(std::vector<float> v);

    size_t array_size() const;
    // Object member by name (the last occurrence), or nullptr
    const Value *member(const std::string &name) const;
};

// FieldValue::as_* with the reference's conversions (core/types.rs:525-1263).
bool as_bool(const Value &v, const std::string &field);
uint64_t as_usize(const Value &v, const std::string &field);
float as_f32(const Value &v, const std::string &field);
const std::string &as_json_object(const Value &v, const std::string &field);
// Elements of an Array as f32 (Vec<f32>::from_field_value, core/impls.rs:687-710)
// into host memory; out must hold array_size() floats.
void array_to_f32(const Value &v, const std::string &field, float *out);
std::vector<uint64_t> array_to_usize(const Value &v, const std::string &field);

// Binary: header (magic "TS_B", version 1, checksum 0, data length, object
// type 0x1001 -- the StructSerializer path always writes Tensor's type,
// binary/structs.rs:90-120) followed by the field count and the fields.
std::vector<uint8_t> to_binary(const Fields &fields);
// Parses a whole buffer; Records arrays keep a reference to it.
Fields from_binary(std::shared_ptr<const std::vector<uint8_t>> data);

// JSON: the reference's mapping (json/structs.rs:32-184) and parser
// (json/parser.rs, json/structs.rs:186-300).
std::string to_json(const Fields &fields);
Fields from_json(const std::string &text);

// An f32 as the JSON writer prints it: Rust's Display (shortest digits that
// round-trip, fixed notation) with ".0" appended to integral values
// (json/structs.rs:80-87): 1 -> "1.0", 1e-7 -> "0.0000001", NaN -> "NaN".
std::string format_f32(float v);
// Appends the same text to out.
void append_f32(std::string &out, float v);

std::vector<uint8_t> read_file(const std::string &path);
void write_file(const std::string &path, const void *data, size_t len);

}  // namespace ser
}  // namespace ts
