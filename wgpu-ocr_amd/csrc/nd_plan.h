// The fusion plan of the N-D executor: which ONNX nodes of a graph run as one launch. Pure host
// code (no device work), so the plan can be made and inspected without a GPU (ocr_nd_plan).
//
// The graph is viewed as a def-use graph: every value has one producing node and a list of
// consuming nodes (the graph output counts as one more consumer). A step starts at an anchor
// node (a dense or grouped Conv, a ConvTranspose, a MatMul by a 2-D initializer, the first
// ReduceMean of a LayerNorm, a BatchNormalization, or any other node on its own) and grows along
// the anchor's result through a fixed sequence of epilogue slots, each slot a small pattern of
// nodes matched over the def-use edges (operand order free for Add and Mul). A pattern is taken
// only when every value it swallows has no consumer outside it, so no fused value is ever needed
// by another step. The step runs at the place of its last node, which in a topologically ordered
// graph comes after every value the step reads.
//
// What is fused matches the operator contract of the reference's NdGraph::new (src/nd.rs:505-817):
// Identity nodes are dropped (their readers read the input), a final Softmax can be cut off, a
// squeeze-excitation Mul by a HardSigmoid gate read only by a dense Conv becomes that conv's input
// scale, the exporter's LayerNorm chain becomes one op, Conv takes a constant bias Add, a ReLU or
// the exporter's GELU chain and a residual Add, a MatMul by a weight takes a bias Add and SiLU,
// a ConvTranspose takes a bias Add and ReLU or Sigmoid, and a lone BatchNormalization becomes a
// channel affine. This library adds three: a BatchNormalization right after a Conv's bias becomes
// the conv's epilogue affine, a MatMul by a weight takes a residual Add after its bias and
// activation, and the exporter's multi-head self-attention chain (from the QKV projection's
// reshape to the output's reshape) becomes one step.
#pragma once

#include <string>
#include <vector>

#include "common.h"
#include "onnx.h"

namespace ocr {

enum class NdKind { Generic, Conv, ConvT, Linear, LayerNorm, Affine, Attention };

struct NdStep {
    NdKind kind = NdKind::Generic;
    int anchor = 0;                 // the node whose kernel the step runs
    int last = 0;                   // the node whose output the step writes (it runs at that place)
    std::vector<int> nodes;         // every node of the step, anchor first
    std::string output;
    int act = ACT_NONE;
    std::vector<std::string> bias;  // constant bias tensors added in the epilogue (in order)
    int batch_norm = -1;            // BatchNormalization node folded into a Conv's epilogue
    std::string residual;           // computed tensor added after the activation
    std::string in_scale;           // per (image, channel) scale of a Conv's input
    std::string conv_input;         // a Conv's input once its input scale is taken out
    // LayerNorm
    std::string gamma, beta;
    float eps = 1e-5f;
    // Attention (its input is conv_input: the fused QKV projection [n, T, 3 H d])
    std::string attn_shape, attn_out_shape;  // the first and the last Reshape's shape operands
    float attn_scale = 1.f;
};

struct NdPlan {
    std::vector<Node> nodes;  // the graph's nodes with Identity nodes removed and their readers redirected
    std::string input, output;
    std::vector<NdStep> steps;  // in the order they run
};

NdPlan plan_nd(const Onnx &onnx, bool stop_before_softmax);
// One line per step: kind, anchor op and index, nodes, epilogue and output (for tests and logs).
std::string describe(const NdPlan &plan);

}  // namespace ocr
