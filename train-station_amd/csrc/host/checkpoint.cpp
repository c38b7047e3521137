// Checkpoint and resume of device tensors and of Adam's state in the
// reference's formats: Tensor (tensor/core/serialization.rs:179-288), Adam,
// AdamConfig and the per-parameter state (optimizers/adam/serialization.rs:
// 40-235), binary "TS_B" v1 and JSON (ts_serial.h).
//
// The binary data array of a tensor is encoded and decoded on the device
// (ts_hip_encode_f32_records / ts_hip_decode_f32_records), so saving is one
// device->host copy of the finished bytes and loading one host->device copy.
#include <cstring>

#include "ts_hip.h"
#include "ts_host.h"
#include "ts_serial.h"

namespace ts {

using ser::Fields;
using ser::Kind;
using ser::Value;

namespace {

void *stream() { return Runtime::get().stream(); }

size_t product(const std::vector<size_t> &dims) {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    return n;
}

std::vector<size_t> contiguous_strides(const std::vector<size_t> &dims) {  // shape.rs:318-331
    std::vector<size_t> s(dims.size());
    size_t stride = 1;
    for (size_t i = dims.size(); i-- > 0;) {
        s[i] = stride;
        stride *= dims[i];
    }
    return s;
}

Value usize_array(const std::vector<size_t> &v) {
    std::vector<Value> items;
    for (size_t x : v) items.push_back(Value::usize(x));
    return Value::array(std::move(items));
}

// Shape (tensor/core/serialization.rs:128-138): dims, size, strides, layout
Value shape_value(const std::vector<size_t> &dims) {
    Fields f;
    f.emplace_back("dims", usize_array(dims));
    f.emplace_back("size", Value::usize(product(dims)));
    f.emplace_back("strides", usize_array(contiguous_strides(dims)));
    f.emplace_back("layout", Value::enum_unit("Contiguous"));
    return Value::object(std::move(f));
}

// Device (serialization.rs:56-64).  Recorded as the CPU device: the
// reference's loader refuses any other (tensor/core/utils.rs:331-335 panics
// for CUDA), and this loader places every tensor on the GPU whatever it says.
Value device_value() {
    Fields f;
    f.emplace_back("type", Value::enum_unit("Cpu"));
    f.emplace_back("index", Value::usize(0));
    return Value::object(std::move(f));
}

const Value &need(const Fields &f, const std::string &name) {
    const Value *v = nullptr;
    for (const auto &kv : f)
        if (kv.first == name) v = &kv.second;
    if (!v) throw Error("Validation failed for field '" + name + "': Field not found");
    return *v;
}

const Value &need_member(const Value &obj, const std::string &name, const std::string &field,
                         const std::string &what) {
    const Value *v = obj.member(name);
    if (!v) throw Error("Validation failed for field '" + field + "': Missing " + what);
    return *v;
}

std::string enum_unit_variant(const Value &v, const std::string &field, const char *what) {
    if (v.kind != Kind::Enum)
        throw Error("Validation failed for field '" + field + "': Expected enum value for " + what);
    if (!v.items.empty())
        throw Error("Validation failed for field '" + field + "': " + std::string(what) +
                    " variants should not have associated data");
    return v.s;
}

// Bytes of the data array: header (24) + field count (8) + name "data"
// (4 + 4) + Array tag (1) + element count (8).  The data field comes first.
constexpr size_t kDataRecordsAt = 24 + 8 + 4 + 4 + 1 + 8;

// The binary form of a device buffer as a Tensor of `dims`.
std::vector<uint8_t> device_to_binary(const float *dev, const std::vector<size_t> &dims, bool requires_grad) {
    refuse_while_recording("checkpoint");
    const size_t n = product(dims);
    Value data;
    data.kind = Kind::Array;
    data.form = ser::ArrayForm::Records;  // no buffer: a hole of 5n bytes filled below
    data.count = n;
    Fields f;
    f.emplace_back("data", std::move(data));
    f.emplace_back("shape", shape_value(dims));
    f.emplace_back("device", device_value());
    f.emplace_back("requires_grad", Value::boolean(requires_grad));
    std::vector<uint8_t> out = ser::to_binary(f);
    if (n) {
        std::unique_ptr<Allocation> aligned;
        const float *src = dev;
        if (reinterpret_cast<uintptr_t>(src) & 15u) {
            aligned = std::make_unique<Allocation>(n);
            check(ts_hip_copy(dev, aligned->get(), n, stream()), "ts_hip_copy");
            src = aligned->get();
        }
        Allocation records((5 * n + 3) / 4);
        check(ts_hip_encode_f32_records(src, n, records.get(), stream()), "ts_hip_encode_f32_records");
        check(ts_hip_memcpy_bytes(out.data() + kDataRecordsAt, records.get(), 5 * n, 1, stream()),
              "ts_hip_memcpy_bytes");
        Runtime::get().sync();
    }
    return out;
}

std::vector<float> device_to_host(const float *dev, size_t n) {
    refuse_while_recording("checkpoint");
    std::vector<float> h(n);
    if (n) {
        check(ts_hip_memcpy_async(h.data(), dev, n, 1, stream()), "ts_hip_memcpy_async");
        Runtime::get().sync();
    }
    return h;
}

std::string device_to_json(const float *dev, const std::vector<size_t> &dims, bool requires_grad) {
    Fields f;
    f.emplace_back("data", Value::float_values(device_to_host(dev, product(dims))));
    f.emplace_back("shape", shape_value(dims));
    f.emplace_back("device", device_value());
    f.emplace_back("requires_grad", Value::boolean(requires_grad));
    return ser::to_json(f);
}

// Writes the values of a data Array into device memory (n floats).
void upload_array(const Value &data, size_t n, float *dev) {
    refuse_while_recording("checkpoint");
    if (!n) return;
    if (data.form == ser::ArrayForm::Records) {
        Allocation records((5 * n + 3) / 4);
        check(ts_hip_memcpy_bytes(records.get(), data.buf->data() + data.offset, 5 * n, 0, stream()),
              "ts_hip_memcpy_bytes");
        check(ts_hip_decode_f32_records(records.get(), n, dev, nullptr, stream()),
              "ts_hip_decode_f32_records");
        Runtime::get().sync();
        return;
    }
    std::vector<float> host(n);
    ser::array_to_f32(data, "data", host.data());
    check(ts_hip_memcpy_async(dev, host.data(), n, 0, stream()), "ts_hip_memcpy_async");
    Runtime::get().sync();
}

// Tensor::from_deserializer (tensor/core/serialization.rs:201-248)
Tensor tensor_from_fields(const Fields &f) {
    const Value &data = need(f, "data");
    if (data.kind != Kind::Array)
        throw Error("Validation failed for field 'data': Expected Vec<f32>, found a non-array value");
    if (data.form == ser::ArrayForm::Items) {  // element types are checked before the shape
        for (size_t i = 0; i < data.items.size(); ++i) (void)ser::as_f32(data.items[i], "data[" + std::to_string(i) + "]");
    }
    const Value &shape = need(f, "shape");
    if (shape.kind != Kind::Object)
        throw Error("Validation failed for field 'shape': Expected object for shape");
    const auto dims64 = ser::array_to_usize(need_member(shape, "dims", "shape", "dims field in shape"), "dims");
    const uint64_t size = ser::as_usize(need_member(shape, "size", "shape", "size field in shape"), "size");
    const auto strides64 =
        ser::array_to_usize(need_member(shape, "strides", "shape", "strides field in shape"), "strides");
    const std::string layout =
        enum_unit_variant(need_member(shape, "layout", "shape", "layout field in shape"), "layout", "memory layout");
    if (layout != "Contiguous" && layout != "Strided" && layout != "View")
        throw Error("Validation failed for field 'layout': Unknown memory layout variant: " + layout);
    std::vector<size_t> dims(dims64.begin(), dims64.end());
    const size_t expected = product(dims);
    if (size != expected)
        throw Error("Validation failed for field 'shape': Shape size " + std::to_string(size) +
                    " doesn't match computed size " + std::to_string(expected));
    if (dims.size() != strides64.size())
        throw Error("Validation failed for field 'shape': Dimensions and strides must have same length");
    const Value &device = need(f, "device");
    if (device.kind != Kind::Object)
        throw Error("Validation failed for field 'device': Expected object for device");
    const std::string dtype =
        enum_unit_variant(need_member(device, "type", "device", "device type field"), "type", "device type");
    if (dtype != "Cpu" && dtype != "Cuda")
        throw Error("Validation failed for field 'type': Unknown device type variant: " + dtype);
    (void)ser::as_usize(need_member(device, "index", "device", "device index field"), "index");
    const bool requires_grad = ser::as_bool(need(f, "requires_grad"), "requires_grad");
    if (data.array_size() != size)
        throw Error("Validation failed for field 'tensor': Data length " + std::to_string(data.array_size()) +
                    " doesn't match shape size " + std::to_string(size));
    if (std::vector<size_t>(strides64.begin(), strides64.end()) != contiguous_strides(dims))
        throw Error("Validation failed for field 'tensor': Reconstructed tensor shape doesn't match "
                    "serialized shape");
    Tensor t = Tensor::new_uninit(dims);
    upload_array(data, size, t.dev_mut());
    t.set_requires_grad(requires_grad);
    return t;
}

Tensor tensor_from_binary_buffer(std::shared_ptr<const std::vector<uint8_t>> buf) {
    return tensor_from_fields(ser::from_binary(std::move(buf)));
}

// Tensor::from_field_value (serialization.rs:251-288): a nested binary
// object, JSON text, or an object of the four fields
Tensor tensor_from_value(const Value &v, const std::string &field) {
    try {
        if (v.kind == Kind::BinaryObject)
            return tensor_from_binary_buffer(std::make_shared<const std::vector<uint8_t>>(v.bytes));
        if (v.kind == Kind::JsonObject) return tensor_from_fields(ser::from_json(v.s));
        if (v.kind == Kind::Object) return tensor_from_fields(v.fields);
    } catch (const Error &e) {
        throw Error("Validation failed for field '" + field + "': Failed to deserialize tensor: " + e.what());
    }
    throw Error("Validation failed for field '" + field +
                "': Expected binary object, JSON object, or structured object for tensor field");
}

// ---- AdamConfig (adam/serialization.rs:40-95) -------------------------------------------

Fields config_fields(const AdamConfig &c) {
    Fields f;
    f.emplace_back("learning_rate", Value::f32(c.learning_rate));
    f.emplace_back("beta1", Value::f32(c.beta1));
    f.emplace_back("beta2", Value::f32(c.beta2));
    f.emplace_back("eps", Value::f32(c.eps));
    f.emplace_back("weight_decay", Value::f32(c.weight_decay));
    f.emplace_back("amsgrad", Value::boolean(c.amsgrad));
    return f;
}

AdamConfig config_from_fields(const Fields &f) {
    AdamConfig c;
    c.learning_rate = ser::as_f32(need(f, "learning_rate"), "learning_rate");
    c.beta1 = ser::as_f32(need(f, "beta1"), "beta1");
    c.beta2 = ser::as_f32(need(f, "beta2"), "beta2");
    c.eps = ser::as_f32(need(f, "eps"), "eps");
    c.weight_decay = ser::as_f32(need(f, "weight_decay"), "weight_decay");
    c.amsgrad = ser::as_bool(need(f, "amsgrad"), "amsgrad");
    return c;
}

// Rust's str::parse::<usize> on a states key: optional '+', then decimal digits
bool parse_usize_key(const std::string &s, size_t &out) {
    size_t i = (!s.empty() && s[0] == '+') ? 1 : 0;
    if (i == s.size()) return false;
    unsigned long long v = 0;
    for (; i < s.size(); ++i) {
        if (s[i] < '0' || s[i] > '9') return false;
        const unsigned d = static_cast<unsigned>(s[i] - '0');
        if (v > (~0ull - d) / 10) return false;
        v = v * 10 + d;
    }
    out = static_cast<size_t>(v);
    return true;
}

}  // namespace

// ---- Tensor -------------------------------------------------------------------------------

std::vector<uint8_t> Tensor::to_binary() const { return device_to_binary(dev(), dims_, requires_grad_); }

Tensor Tensor::from_binary(const uint8_t *data, size_t len) {
    return tensor_from_binary_buffer(std::make_shared<const std::vector<uint8_t>>(data, data + len));
}

std::string Tensor::to_json() const { return device_to_json(dev(), dims_, requires_grad_); }

Tensor Tensor::from_json(const std::string &json) { return tensor_from_fields(ser::from_json(json)); }

void Tensor::save_binary(const std::string &path) const {
    const std::vector<uint8_t> b = to_binary();
    ser::write_file(path, b.data(), b.size());
}

void Tensor::save_json(const std::string &path) const {
    const std::string s = to_json();
    ser::write_file(path, s.data(), s.size());
}

Tensor Tensor::load_binary(const std::string &path) {
    return tensor_from_binary_buffer(std::make_shared<const std::vector<uint8_t>>(ser::read_file(path)));
}

Tensor Tensor::load_json(const std::string &path) {
    const std::vector<uint8_t> b = ser::read_file(path);
    return from_json(std::string(b.begin(), b.end()));
}

// ---- AdamConfig -----------------------------------------------------------------------------

std::vector<uint8_t> adam_config_to_binary(const AdamConfig &c) { return ser::to_binary(config_fields(c)); }
std::string adam_config_to_json(const AdamConfig &c) { return ser::to_json(config_fields(c)); }
AdamConfig adam_config_from_binary(const uint8_t *data, size_t len) {
    return config_from_fields(ser::from_binary(std::make_shared<const std::vector<uint8_t>>(data, data + len)));
}
AdamConfig adam_config_from_json(const std::string &json) { return config_from_fields(ser::from_json(json)); }

// ---- Adam (adam/serialization.rs:140-235) ----------------------------------------------------

// Nested tensors (m, v, v_hat_max) are written as binary objects in the
// binary form and as embedded JSON in the JSON form.  The reference embeds
// JSON text in both; its binary reader accepts either, and refuses strings
// over 1,000,000 bytes (binary/reader.rs:79-94), which JSON text of more than
// about 10^5 values exceeds, while a binary object may hold 10^8 bytes.
Fields Adam::to_fields(bool binary) const {
    settle();
    Fields states;
    auto nested = [&](const float *dev, const std::vector<size_t> &dims) {
        return binary ? Value::binary_object(device_to_binary(dev, dims, false))
                      : [&] {
                            Value j;
                            j.kind = Kind::JsonObject;
                            j.s = device_to_json(dev, dims, false);
                            return j;
                        }();
    };
    for (size_t id : insertion_order_) {
        const State &s = states_.at(id);
        Fields st;
        st.emplace_back("m", nested(s.m ? s.m->get() : nullptr, s.dims));
        st.emplace_back("v", nested(s.v ? s.v->get() : nullptr, s.dims));
        st.emplace_back("v_hat_max", s.v_hat_max ? Value::some(nested(s.v_hat_max->get(), s.dims)) : Value::none());
        st.emplace_back("step", Value::usize(s.step));
        states.emplace_back(std::to_string(id), Value::object(std::move(st)));
    }
    std::vector<Value> order;
    for (size_t id : insertion_order_) order.push_back(Value::usize(id));
    Fields f;
    f.emplace_back("config", Value::object(config_fields(config_)));
    f.emplace_back("states", Value::object(std::move(states)));
    f.emplace_back("step_count", Value::usize(ledger_->step_count));
    f.emplace_back("insertion_order", Value::array(std::move(order)));
    return f;
}

Adam Adam::from_fields(const ser::Fields &f) {
    Adam a;
    const Value &config = need(f, "config");
    if (config.kind != Kind::Object)
        throw Error("Validation failed for field 'config': Expected Object for AdamConfig");
    a.config_ = config_from_fields(config.fields);
    const Value &states = need(f, "states");
    if (states.kind != Kind::Object)
        throw Error("Validation failed for field 'states': Expected Object for "
                    "HashMap<usize, SerializableParameterState>");
    for (const auto &kv : states.fields) {
        size_t id = 0;
        if (!parse_usize_key(kv.first, id))
            throw Error("Validation failed for field 'states': Invalid key '" + kv.first +
                        "' in parameter states map");
        const Value &sv = kv.second;
        if (sv.kind != Kind::Object)
            throw Error("Validation failed for field '" + kv.first +
                        "': Expected Object for SerializableParameterState");
        Tensor m = tensor_from_value(need(sv.fields, "m"), "m");
        Tensor v = tensor_from_value(need(sv.fields, "v"), "v");
        const Value &vm = need(sv.fields, "v_hat_max");
        State s;
        s.dims = m.dims();
        s.n = m.size();
        if (vm.kind == Kind::Optional) {
            if (!vm.items.empty()) {
                Tensor t = tensor_from_value(vm.items[0], "v_hat_max");
                s.v_hat_max = t.allocation();
            }
        } else {  // Option<T>::from_field_value also takes a bare value
            Tensor t = tensor_from_value(vm, "v_hat_max");
            s.v_hat_max = t.allocation();
        }
        s.step = ser::as_usize(need(sv.fields, "step"), "step");
        if (v.size() != s.n) throw Error("Momentum and velocity size mismatch in saved state " + kv.first);
        s.m = m.allocation();
        s.v = v.allocation();
        a.states_[id] = std::move(s);
    }
    a.ledger_->step_count = ser::as_usize(need(f, "step_count"), "step_count");
    const auto order = ser::array_to_usize(need(f, "insertion_order"), "insertion_order");
    a.insertion_order_.assign(order.begin(), order.end());
    return a;
}

std::vector<uint8_t> Adam::to_binary() const { return ser::to_binary(to_fields(true)); }
std::string Adam::to_json() const { return ser::to_json(to_fields(false)); }

Adam Adam::from_binary(const uint8_t *data, size_t len) {
    return from_fields(ser::from_binary(std::make_shared<const std::vector<uint8_t>>(data, data + len)));
}

Adam Adam::from_json(const std::string &json) { return from_fields(ser::from_json(json)); }

void Adam::save_binary(const std::string &path) const {
    const std::vector<uint8_t> b = to_binary();
    ser::write_file(path, b.data(), b.size());
}

void Adam::save_json(const std::string &path) const {
    const std::string s = to_json();
    ser::write_file(path, s.data(), s.size());
}

Adam Adam::load_binary(const std::string &path) {
    return from_fields(ser::from_binary(std::make_shared<const std::vector<uint8_t>>(ser::read_file(path))));
}

Adam Adam::load_json(const std::string &path) {
    const std::vector<uint8_t> b = ser::read_file(path);
    return from_json(std::string(b.begin(), b.end()));
}

// adam/mod.rs:396-454
void Adam::relink_parameters(const std::vector<const Tensor *> &params) {
    settle();  // replayed steps land on the states under their old ids first
    for (size_t i = 0; i < params.size(); ++i)
        if (!params[i]->requires_grad())
            throw Error("Parameter at index " + std::to_string(i) + " must require gradients");
    if (params.size() != insertion_order_.size())
        throw Error("Parameter count mismatch: expected " + std::to_string(insertion_order_.size()) +
                    " parameters, got " + std::to_string(params.size()));
    std::unordered_map<size_t, State> fresh;
    std::vector<size_t> order;
    std::unordered_map<size_t, int> used;  // saved ids already mapped (copied on a repeat)
    for (size_t i = 0; i < params.size(); ++i) {
        auto it = states_.find(insertion_order_[i]);
        if (it == states_.end())
            throw Error("No saved state found for parameter at position " + std::to_string(i));
        const State &saved = it->second;
        if (params[i]->dims() != saved.dims)
            throw Error("Shape mismatch for parameter at position " + std::to_string(i) + ": expected " +
                        dims_str(saved.dims) + ", got " + dims_str(params[i]->dims()));
        State s = saved;  // the device state moves over; the reference clones it
        if (used[insertion_order_[i]]++) {
            auto dup = [&](const std::shared_ptr<Allocation> &a) -> std::shared_ptr<Allocation> {
                if (!a) return a;
                auto b = std::make_shared<Allocation>(s.n);
                check(ts_hip_copy(a->get(), b->get(), s.n, stream()), "ts_hip_copy");
                return b;
            };
            s.m = dup(s.m);
            s.v = dup(s.v);
            s.v_hat_max = dup(s.v_hat_max);
        }
        fresh[params[i]->id()] = std::move(s);
        order.push_back(params[i]->id());
    }
    states_ = std::move(fresh);
    insertion_order_ = std::move(order);
}

}  // namespace ts
