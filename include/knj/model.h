// include/knj/model.h -- C++ host interface of the device decode step.
//
// Keeps the shape of the reference's model-step interface
// (/root/reference/src/model/model.h:32-163): ModelGeometry, Model::Options,
// Model::open -> forward(tokens, n) -> logits of the last token, reset(),
// pos(), geom(), threads().  The weights and the KV cache live on the GPU; the
// arithmetic runs in the gfx950 kernels behind include/knj_capi.h, which this
// class calls.  Errors are std::runtime_error, as in the reference (context
// exhausted, token out of range, bad geometry).
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../knj_capi.h"
#include "profiler.h"

namespace knj {

struct ModelGeometry {
  int n_layer = 0;
  int n_embd = 0;
  int n_head = 0;
  int n_head_kv = 0;
  int head_dim = 0;
  int n_ff_exp = 0;
  int n_expert = 0;
  int n_expert_used = 0;
  int n_vocab = 0;
  int n_ctx_train = 0;
  float rms_eps = 1e-6f;
  float rope_base = 1e6f;
  bool rope_split_halves = true;  // ggml NEOX pairing (i, i + d/2), the only one qwen3moe uses

  int q_dim() const { return n_head * head_dim; }
  int kv_dim() const { return n_head_kv * head_dim; }
  std::string describe() const;
};

class Model {
 public:
  struct Options {
    int n_ctx = 2048;
    int threads = 0;  // accepted for interface compatibility; the step runs on the GPU
  };

  // A qwen3moe GGUF file (reference src/model/model.cpp:174): geometry and
  // weights from the file, throws on a missing key or tensor, a shape that
  // disagrees with the geometry, a weight type the device path lacks, or
  // opt.n_ctx above the trained context.
  static std::unique_ptr<Model> open(const std::string& path, const Options& opt);
  // Synthetic weights (seeded, include/knj_synth.h) of the given geometry and
  // quantisation, generated on the GPU.
  static std::unique_ptr<Model> open_synthetic(const knj_model_config& cfg, uint64_t seed,
                                               const Options& opt);
  // A weight image laid out as include/knj_model.h describes.
  static std::unique_ptr<Model> open_image(const knj_model_config& cfg, const void* image,
                                           uint64_t bytes, const Options& opt);

  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  const ModelGeometry& geom() const { return g_; }
  int n_ctx() const { return n_ctx_; }
  int pos() const;
  int threads() const { return 1; }

  // Drops the KV cache and returns to position 0.
  void reset();

  // Fills cache slots [0, n_pos) with seeded f16 values and moves to n_pos:
  // a long context without running its prefill (knj_model_fill_kv).
  void fill_kv(int n_pos, uint64_t seed);

  // Runs `n` tokens starting at the current position; returns n_vocab logits
  // of the last token, valid until the next call.
  const float* forward(const int32_t* tokens, int n);

  // Greedy decode on the device: feeds `first`, returns `steps` argmax tokens.
  std::vector<int32_t> decode_greedy(int32_t first, int steps);

  // The same decode with every kernel launch timed by dispatch-recorded events
  // (knj_model_profile), one step per call.  Each step's launches go to `prof`
  // as device spans named "class:layer:kernel" after prof.step_done() has seen
  // its warmup; steps are laid end to end on one timeline, so the host time
  // between steps is not counted as device idle.  Same tokens as decode_greedy.
  std::vector<int32_t> decode_greedy_profiled(int32_t first, int steps, Profiler& prof);

  // Host<->device bytes copied so far (knj_model_transfer_bytes).
  TransferStats transfer_stats() const;

  knj_model* handle() const { return m_; }

 private:
  Model() = default;
  knj_model* m_ = nullptr;
  ModelGeometry g_;
  int n_ctx_ = 0;
  std::vector<float> logits_;
};

// Throws std::runtime_error with knj_last_error() when rc != KNJ_OK.
void check(int rc, const char* what);

}  // namespace knj
