// ONNX model reader: the graph and weights straight from the .onnx file (src/onnx.rs:1-133).
#pragma once

#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <vector>

namespace ocr {

// A float tensor: its dimensions and row-major data (onnx.rs:8-13).
struct Weight {
    std::vector<int64_t> dims;
    std::vector<float> data;
};

struct Attr {
    std::string name;
    int type = 0;  // AttributeProto.AttributeType
    float f = 0.f;
    int64_t i = 0;
    std::string s;
    std::vector<int64_t> ints;
    std::vector<float> floats;
    bool has_f = false, has_i = false, has_s = false;
};

struct Node {
    std::string op;
    std::vector<std::string> inputs, outputs;
    std::vector<Attr> attrs;

    const Attr *attr(const std::string &name) const;
    std::optional<std::vector<int64_t>> ints(const std::string &name) const;  // onnx.rs:28-30
    std::optional<int64_t> int_(const std::string &name) const;               // onnx.rs:32-34
    std::optional<std::string> str(const std::string &name) const;            // onnx.rs:36-38
    std::optional<float> f32(const std::string &name) const;                  // onnx.rs:40-42
};

struct Onnx {
    std::vector<Node> nodes;
    std::map<std::string, Weight> weights;              // float initializers and Constants
    std::map<std::string, std::vector<int64_t>> ints;   // int64 initializers and Constants
    std::string input, output;

    // Onnx::load (onnx.rs:88-123): initializers and Constant nodes become weights or integer
    // lists; the input is the first graph input that is not an initializer; the output is the
    // first graph output.
    static Onnx load(const std::string &path);
    static Onnx parse(const uint8_t *data, size_t size);
    const Weight &weight(const std::string &name) const;  // onnx.rs:125-127
    int readers(const std::string &name) const;           // onnx.rs:130-132
};

}  // namespace ocr
