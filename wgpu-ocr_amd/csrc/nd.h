// The N-D ONNX executor for the PP-OCRv6 models (the reference's NdGraph, src/nd.rs:428-1394).
// Float tensors live on the device, row-major (ONNX's layout); integer tensors (shapes,
// indices) stay on the host, as the reference keeps them (nd.rs:436-440).
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "kernels.h"
#include "nd_kernels.h"
#include "nd_plan.h"
#include "onnx.h"
#include "runtime.h"

namespace ocr {

struct NdTensor {
    std::shared_ptr<DBuf> buf;  // owner (null for weights and caller memory)
    float *p = nullptr;
    std::vector<int64_t> shape;
    size_t count() const;
};

struct NdValue {
    bool is_int = false;
    NdTensor t;
    std::vector<int64_t> iv, ishape;
};

// One step of the plan (nd_plan.h) with its weights on the device: a node, or a node with the
// ones fused into it.
struct NdOp {
    NdKind kind = NdKind::Generic;
    int node = 0;  // the first node's index
    std::vector<std::string> inputs;
    std::string output;
    int act = ACT_NONE;
    // Conv / ConvTranspose
    int cin = 0, cout = 0, cin_g = 0, group = 1, kh = 0, kw = 0, sh = 1, sw = 1;
    int pads[4] = {0, 0, 0, 0};
    bool same_upper = false, mfma = false;
    ConvPack pk;
    const uint16_t *whi = nullptr, *wlo = nullptr;
    const float *w = nullptr, *b = nullptr, *affine = nullptr;
    std::string residual, in_scale;
    // Linear: [k] -> [n]
    int k = 0, n = 0;
    // LayerNorm
    const float *gb = nullptr;
    int len = 0;
    float eps = 1e-5f;
    // Affine
    const float *st = nullptr;
    // Attention: inputs are the QKV projection, the first and the last Reshape's shapes
    float scale = 1.f;
};

class NdGraph {
  public:
    // nd.rs:505: `stop_before_softmax` returns the logits a final Softmax would read.
    static NdGraph build(Ctx &ctx, const Onnx &onnx, bool stop_before_softmax);

    // nd.rs:834: the graph on x (device memory, row-major); returns the output tensor.
    NdTensor run(Ctx &ctx, const NdTensor &x) const;
    // The arg-max over the last axis of the output per row (first index on ties, nd.rs:383).
    // When the graph ends in a Linear (the CTC head), its logits are never written: the GEMM
    // keeps per-block (max, index) pairs that one more kernel reduces.
    void run_argmax(Ctx &ctx, const NdTensor &x, uint32_t *d_best, std::vector<int64_t> *out_shape) const;
    // Output shape for an input shape: every op's shape rule on the host, nothing launched.
    std::vector<int64_t> output_shape(const std::vector<int64_t> &in) const;

    std::string input, output;
    std::vector<NdOp> ops;

  private:
    struct DevW {
        const float *p = nullptr;
        std::vector<int64_t> shape;
        std::vector<float> host;  // small constants (scales, exponents), up to 16 values
    };
    std::vector<Node> nodes_;
    std::map<std::string, DevW> weights_;
    std::map<std::string, std::vector<int64_t>> ints_;
    std::map<std::string, size_t> last_use_;
    NdTensor run_ops(Ctx *ctx, const NdTensor &x, size_t nops, std::map<std::string, NdValue> *vals) const;
    NdValue get(const std::map<std::string, NdValue> &vals, const std::string &name) const;
};

}  // namespace ocr
