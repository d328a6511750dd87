// The ocrs detection and recognition models on the GPU (src/gpu.rs:1380-1603).
#pragma once

#include <functional>
#include <memory>
#include <vector>

#include "graph.h"

namespace ocr {

constexpr int DET_MH = 800, DET_MW = 600;  // the detector's fixed input size (gpu.rs:1394)

class Detector {
  public:
    Detector(Ctx &ctx, const Onnx &onnx);  // Detector::new (gpu.rs:1385-1387)

    // Detector::detect_page (gpu.rs:1393-1422) for `count` pages at once, all on the device:
    // RGB bytes (h x w x 3 each) -> ocrs grey, padded to at least the model size and resized to
    // it -> the model (one batched pass) -> the valid part resized back to the page,
    // thresholded and bit-packed into h rows of ceil(w / 32) words.
    void detect_pages_device(const uint8_t *const *rgb, const int *w, const int *h, int count, float thr,
                             uint32_t *const *bits);
    // Detector::detect (gpu.rs:1425-1430): the probability map of a [1, 1, h, w] host input.
    std::vector<float> detect(const float *input, int h, int w);

  private:
    Ctx &ctx_;
    Graph graph_;
};

class Recognizer {
  public:
    Recognizer(Ctx &ctx, const Onnx &onnx, uint32_t lines);  // Recognizer::new (gpu.rs:1452-1506)
    ~Recognizer();

    struct Batch {
        const float *data;  // [n][64][w] line images (host or device memory, see below)
        int n, w;
    };
    struct Dims {
        int tmax, ntot, classes;
    };
    Dims dims(const Batch *batches, int count) const;
    // Recognizer::recognize (gpu.rs:1510-1602) with the batches' data in device memory.
    // logits: device [tmax][ntot][classes] raw logits (rows t >= lens[line] are not defined);
    // best: device [tmax][ntot] arg-max per row (last index on ties), may be null; lens: host
    // [ntot], every line's step count (its batch's trunk width, gpu.rs:1552). between, if given,
    // is called after the first half of the trunk's layers, after the trunk's and after each GRU
    // layer's kernels are queued (a caller that interleaves other work on the stream).
    // gru_stream, if given, runs the two recurrences and everything after the second (the output
    // layer and the arg-max): each recurrence waits for its input projection on the context's
    // stream, which waits for the first only before the second projection and returns without
    // waiting for the second. What the caller queues meanwhile (from between(), or its next
    // pass's trunk) runs beside the recurrence, whose workgroups occupy one CU per 8 lines and
    // direction. logits and best are then written in gru_stream's order: the caller orders its
    // reads after that stream and marks the buffers as used on it.
    void recognize_device(const Batch *batches, int count, float *logits, uint32_t *best, uint32_t *lens,
                          const std::function<void()> &between = {}, hipStream_t gru_stream = nullptr);
    int classes() const { return classes_; }
    bool recurrent_exact() const { return r_exact_; }
    uint32_t lines() const { return lines_; }

  private:
    struct Layer {
        ConvPack pk;  // the input projection as a 1 x 1 convolution: [1536][input]
        const uint16_t *w_hi = nullptr, *w_lo = nullptr, *w_frag = nullptr;
        const float *wb = nullptr;  // [2][768]
        const uint16_t *r = nullptr;  // [2][768][256] float16
        const float *r32 = nullptr;   // [2][256][768] float32 (R transposed), when R stays float32
        const float *rb = nullptr;    // [2][768]
        int input = 0;
    };
    Ctx &ctx_;
    Graph trunk_;
    int pool_kh_ = 0;
    Layer layers_[2];
    ConvPack lin_pk_;
    const uint16_t *lin_hi_ = nullptr, *lin_lo_ = nullptr, *lin_frag_ = nullptr;
    const float *lin_b_ = nullptr;
    int classes_ = 0;
    uint32_t lines_ = 8;
    bool r_exact_ = true;
};

}  // namespace ocr
