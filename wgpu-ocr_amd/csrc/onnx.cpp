// ONNX protobuf reader (the wire format by hand; no protobuf library). Semantics of
// src/onnx.rs:57-133: float / int64 tensors from raw_data or the typed fields.
#include "onnx.h"

#include <cstring>
#include <fstream>
#include <iterator>

#include "common.h"

namespace ocr {

namespace {

struct Reader {
    const uint8_t *p, *end;

    bool done() const { return p >= end; }
    uint64_t varint() {
        uint64_t v = 0;
        for (int shift = 0; shift < 64; shift += 7) {
            if (p >= end) fail("onnx: truncated varint");
            uint8_t b = *p++;
            v |= uint64_t(b & 0x7f) << shift;
            if (b < 0x80) return v;
        }
        fail("onnx: varint too long");
    }
    // Next field: number, wire type, and for wire type 2 the payload range.
    bool next(uint32_t &field, uint32_t &wire, uint64_t &val, Reader &sub) {
        if (done()) return false;
        uint64_t key = varint();
        field = uint32_t(key >> 3);
        wire = uint32_t(key & 7);
        switch (wire) {
        case 0: val = varint(); break;
        case 1:
            if (end - p < 8) fail("onnx: truncated fixed64");
            std::memcpy(&val, p, 8);
            p += 8;
            break;
        case 2: {
            uint64_t n = varint();
            if (uint64_t(end - p) < n) fail("onnx: truncated field");
            sub = Reader{p, p + n};
            p += n;
            break;
        }
        case 5: {
            if (end - p < 4) fail("onnx: truncated fixed32");
            uint32_t v32;
            std::memcpy(&v32, p, 4);
            val = v32;
            p += 4;
            break;
        }
        default: fail("onnx: unsupported wire type " + std::to_string(wire));
        }
        return true;
    }
    std::string str() const { return std::string(reinterpret_cast<const char *>(p), size_t(end - p)); }
};

void read_ints(uint32_t wire, uint64_t val, Reader sub, std::vector<int64_t> &out) {
    if (wire == 0) {
        out.push_back(int64_t(val));
        return;
    }
    while (!sub.done()) out.push_back(int64_t(sub.varint()));  // packed
}

void read_floats(uint32_t wire, uint64_t val, Reader sub, std::vector<float> &out) {
    if (wire == 5) {
        uint32_t v = uint32_t(val);
        float f;
        std::memcpy(&f, &v, 4);
        out.push_back(f);
        return;
    }
    size_t n = size_t(sub.end - sub.p) / 4;
    size_t at = out.size();
    out.resize(at + n);
    std::memcpy(out.data() + at, sub.p, n * 4);
}

constexpr int FLOAT = 1, INT64 = 7;

struct TensorVal {
    std::string name;
    std::vector<int64_t> dims;
    int dtype = 0;
    bool has_raw = false;
    Reader raw{nullptr, nullptr};
    std::vector<float> floats;
    std::vector<int64_t> int64s;
};

TensorVal parse_tensor(Reader r) {
    TensorVal t;
    uint32_t f, w;
    uint64_t v;
    Reader sub{nullptr, nullptr};
    while (r.next(f, w, v, sub)) {
        if (f == 1) read_ints(w, v, sub, t.dims);
        else if (f == 2) t.dtype = int(v);
        else if (f == 8) t.name = sub.str();
        else if (f == 9) { t.has_raw = true; t.raw = sub; }
        else if (f == 4) read_floats(w, v, sub, t.floats);
        else if (f == 7) read_ints(w, v, sub, t.int64s);
    }
    return t;
}

// onnx.rs:57-85 (values) and 93-104 (add): floats become weights, int64 become integer lists.
void add_tensor(Onnx &m, const std::string &name, const TensorVal &t) {
    size_t count = 1;
    for (int64_t d : t.dims) {
        if (d < 0) fail("onnx: negative dimension in " + name);
        count *= size_t(d);
    }
    if (t.dtype == FLOAT) {
        Weight w;
        w.dims = t.dims;
        if (t.has_raw) {
            size_t n = size_t(t.raw.end - t.raw.p) / 4;
            w.data.resize(n);
            std::memcpy(w.data.data(), t.raw.p, n * 4);
        } else {
            w.data = t.floats;
        }
        if (w.data.size() != count)
            fail("onnx: " + name + ": " + std::to_string(w.data.size()) + " values for " + std::to_string(count));
        m.weights[name] = std::move(w);
    } else if (t.dtype == INT64) {
        std::vector<int64_t> v;
        if (t.has_raw) {
            size_t n = size_t(t.raw.end - t.raw.p) / 8;
            v.resize(n);
            std::memcpy(v.data(), t.raw.p, n * 8);
        } else {
            v = t.int64s;
        }
        m.ints[name] = std::move(v);
    }
}

Attr parse_attr(Reader r, TensorVal *tensor_out, bool *has_tensor) {
    Attr a;
    uint32_t f, w;
    uint64_t v;
    Reader sub{nullptr, nullptr};
    while (r.next(f, w, v, sub)) {
        switch (f) {
        case 1: a.name = sub.str(); break;
        case 2: {
            uint32_t v32 = uint32_t(v);
            std::memcpy(&a.f, &v32, 4);
            a.has_f = true;
            break;
        }
        case 3: a.i = int64_t(v); a.has_i = true; break;
        case 4: a.s = sub.str(); a.has_s = true; break;
        case 5:
            if (tensor_out) { *tensor_out = parse_tensor(sub); *has_tensor = true; }
            break;
        case 7: read_floats(w, v, sub, a.floats); break;
        case 8: read_ints(w, v, sub, a.ints); break;
        case 20: a.type = int(v); break;
        default: break;
        }
    }
    return a;
}

std::string value_info_name(Reader r) {
    uint32_t f, w;
    uint64_t v;
    Reader sub{nullptr, nullptr};
    while (r.next(f, w, v, sub))
        if (f == 1) return sub.str();
    return {};
}

}  // namespace

const Attr *Node::attr(const std::string &name) const {
    for (const Attr &a : attrs)
        if (a.name == name) return &a;
    return nullptr;
}

std::optional<std::vector<int64_t>> Node::ints(const std::string &name) const {
    const Attr *a = attr(name);
    if (!a) return std::nullopt;
    return a->ints;
}

std::optional<int64_t> Node::int_(const std::string &name) const {
    const Attr *a = attr(name);
    if (!a || !a->has_i) return std::nullopt;
    return a->i;
}

std::optional<std::string> Node::str(const std::string &name) const {
    const Attr *a = attr(name);
    if (!a || !a->has_s) return std::nullopt;
    return a->s;
}

std::optional<float> Node::f32(const std::string &name) const {
    const Attr *a = attr(name);
    if (!a || !a->has_f) return std::nullopt;
    return a->f;
}

Onnx Onnx::parse(const uint8_t *data, size_t size) {
    Reader model{data, data + size};
    uint32_t f, w;
    uint64_t v;
    Reader sub{nullptr, nullptr}, graph{nullptr, nullptr};
    bool has_graph = false;
    while (model.next(f, w, v, sub))
        if (f == 7 && w == 2) { graph = sub; has_graph = true; }
    if (!has_graph) fail("model has no graph");
    Onnx m;
    std::vector<std::string> inputs, outputs;
    while (graph.next(f, w, v, sub)) {
        if (f == 1) {
            Node n;
            TensorVal constant;
            bool has_const = false;
            uint32_t g, gw;
            uint64_t gv;
            Reader s2{nullptr, nullptr};
            Reader nr = sub;
            while (nr.next(g, gw, gv, s2)) {
                if (g == 1) n.inputs.push_back(s2.str());
                else if (g == 2) n.outputs.push_back(s2.str());
                else if (g == 4) n.op = s2.str();
                else if (g == 5) n.attrs.push_back(parse_attr(s2, &constant, &has_const));
            }
            // onnx.rs:111-117: Constants become weights or integer lists, like initializers.
            if (n.op == "Constant") {
                if (!n.outputs.empty() && has_const) add_tensor(m, n.outputs[0], constant);
                continue;
            }
            m.nodes.push_back(std::move(n));
        } else if (f == 5) {
            TensorVal t = parse_tensor(sub);
            add_tensor(m, t.name, t);
        } else if (f == 11) {
            inputs.push_back(value_info_name(sub));
        } else if (f == 12) {
            outputs.push_back(value_info_name(sub));
        }
    }
    for (const std::string &i : inputs)
        if (!m.weights.count(i) && !m.ints.count(i)) { m.input = i; break; }
    if (m.input.empty()) fail("no graph input");
    if (outputs.empty()) fail("no graph output");
    m.output = outputs[0];
    return m;
}

Onnx Onnx::load(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail(path + ": cannot open");
    std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    return parse(bytes.data(), bytes.size());
}

const Weight &Onnx::weight(const std::string &name) const {
    auto it = weights.find(name);
    if (it == weights.end()) fail("missing weight " + name);
    return it->second;
}

int Onnx::readers(const std::string &name) const {
    int n = 0;
    for (const Node &nd : nodes)
        for (const std::string &i : nd.inputs)
            if (i == name) { n++; break; }
    return n;
}

}  // namespace ocr
