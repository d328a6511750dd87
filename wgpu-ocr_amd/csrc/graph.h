// Executor for convolutional ONNX graphs (the reference's Graph, src/gpu.rs:1058-1378).
#pragma once

#include <array>
#include <functional>
#include <string>
#include <vector>

#include "kernels.h"
#include "onnx.h"
#include "runtime.h"

namespace ocr {

enum class OpKind { Conv, Direct, ConvT, MaxPool, Slice, Concat, Act, Identity };

struct Step {
    OpKind kind = OpKind::Identity;
    std::vector<std::string> inputs;
    std::string output;
    // Conv / Direct / ConvT
    int cin = 0, cout = 0, kh = 0, kw = 0, pt = 0, pl = 0, pb = 0, pr = 0, sh = 1, sw = 1, group = 1;
    int act = ACT_NONE;
    bool mfma = false;        // dense conv on the matrix cores (else conv_generic)
    ConvPack pk;
    const uint16_t *whi = nullptr, *wlo = nullptr, *wfrag = nullptr;  // wfrag: conv_igemm's packing
    const float *w = nullptr, *b = nullptr;  // float32 weights (direct, transpose, generic) and bias
    const uint16_t *w1frag = nullptr;        // direct 3 x 3 with float16-exact weights: conv1_mfma's
    int ph = 1, pw = 1;                       // a fused MaxPool's kernel, or MaxPool's kernel
    // A MaxPool fused into a dense conv: pool_only when it was the conv's only reader (output is
    // then the pooled value); otherwise pool_output names the pooled value next to the full one.
    bool pool_only = false;
    std::string pool_output;
    // ConvTranspose with stride s as s x s sub-pixel phases: phase (py, px) is a stride-1
    // ty x tx conv of the input written to output pixels (s * i + py, s * j + px), on the matrix
    // cores. Empty when the kernel is smaller than the stride or a phase would exceed 3 x 3.
    struct TPhase {
        int py = 0, px = 0, ty = 0, tx = 0;
        ConvPack pk;
        const uint16_t *whi = nullptr, *wlo = nullptr, *wfrag = nullptr;
    };
    std::vector<TPhase> phases;
    // All phases as one conv of the input over ceil(kh / s) x ceil(kw / s) taps (zero weights
    // where a phase has fewer): output channel k * cout + c is channel c of phase k (py = k / s,
    // px = k % s); whi unset when it does not apply.
    TPhase allph;
    std::vector<int64_t> starts, ends, axes;  // Slice
};

// Shape of an activation: n, h, w, c.
using Shape = std::array<int, 4>;

class Graph {
  public:
    // The graph of `onnx` up to (not including) the first node of type `stop`, if given
    // (gpu.rs:1102-1240). The stop node, if found, is copied to *stop_node.
    static Graph build(Ctx &ctx, const Onnx &onnx, const char *stop, Node *stop_node, bool *found_stop);

    // Output shape for an input of shape `in` (throws on an invalid shape).
    Shape infer(const Shape &in) const;

    struct Out {
        DBuf buf;
        Act act;
    };
    // Record the graph on `x` on the context's stream; returns the output (gpu.rs:1243-1377).
    Out run(Ctx &ctx, const Act &x) const;
    // The same on several inputs of one height and channel count (any widths and image counts):
    // each step for all of them before the next, a dense 3 x 3 conv as one launch over all.
    std::vector<Out> run_multi(Ctx &ctx, const std::vector<Act> &xs) const;
    // The same, where the graph's output (a 2 x 1 MaxPool of a conv with 4 output rows) is
    // followed by an AveragePool (kh, 1) to one row written time-major into X[t][ntot][c] at line
    // offsets 0, n0, n0 + n1, ...: when the last layer can do that in its own epilogue it does,
    // returns true and the outputs are left empty; otherwise returns false with the outputs.
    // after_step, if given, is called with each step's index once its kernels are queued (the
    // fused last layer excepted).
    bool run_multi_time_major(Ctx &ctx, const std::vector<Act> &xs, int kh, float *X, int ntot,
                              std::vector<Out> &outs, const std::function<void(int)> &after_step = {}) const;

    std::string input, output;
    std::vector<Step> steps;

  private:
    struct Exec;
    bool run_multi_tm(Ctx &ctx, const std::vector<Act> &xs, int kh, float *X, int ntot, std::vector<Out> &outs,
                      const std::function<void(int)> &after_step) const;
    std::vector<Shape> shapes(const Shape &in) const;  // output shape of every step
};

}  // namespace ocr
