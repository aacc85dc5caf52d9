#pragma once

// Greedy decoding over a decode-step graph, in C++.
//
// The reference has no decode loop: its examples run one full forward per Engine::run
// (examples/qwen2/main.py:56-61, tests/test_models.py:61-71). This driver runs a
// dli.graph.v1 decode step (one new token per sequence, e.g. the graphs python/dli_qwen2
// builds) once per position:
//
//   inputs   input_ids int64 [B], positions int64 [B] (slot of each row's new token), plus the
//            weights given at construction
//   outputs  next_ids int64 [B] (argmax of the step's logits), anything else the graph lists
//
// The prompt is fed one position per step through the same graph (its KV entries are written by
// the step's own cache appends), then each step's next_ids becomes the next input.
//
// On a device, the first step runs eagerly with its real ids and positions (creating operators,
// caches and workspaces) and is then captured into a HIP graph (ATen's graph capture, so
// operator outputs come from a private memory pool that stays valid across replays) that every
// later step replays; the ids and positions are copied into the graph's static input buffers
// first. With capture off, or for host tensors, every step is an eager Engine::run.
//
// A graph that lists an output named "status" (the decoder_stack launch status, non-zero when a
// wait in the persistent launch gave up and the step's outputs are invalid) is checked where the
// driver synchronizes with the device anyway: at the start of step() (for earlier steps) and at
// the end of generate(). A failure raises std::runtime_error and clears the word.

#include <cstdint>
#include <memory>

#include "dli/engine.h"

namespace dli {

struct GreedyOptions {
  std::int64_t block_size = 64;     // KV cache block size (tokens)
  std::int64_t max_seq_len = 4096;  // KV capacity per sequence; later positions are rejected
  bool capture = true;              // HIP graph capture/replay of the step (device weights)
};

class GreedyDecoder {
 public:
  // engine: loaded plugin, outlives the decoder. weights: every graph input except input_ids and
  // positions. batch: rows per step.
  GreedyDecoder(Engine& engine, Graph graph, TensorMap weights, std::int64_t batch,
                GreedyOptions options = {});
  ~GreedyDecoder();
  GreedyDecoder(const GreedyDecoder&) = delete;
  GreedyDecoder& operator=(const GreedyDecoder&) = delete;

  std::int64_t batch() const;
  bool captured() const;

  // One step for ids [B] at positions [B] (int64, host or device). Returns the step's outputs
  // (next_ids and the graph's other outputs). Captured outputs are the graph's static buffers:
  // the next step overwrites them.
  TensorMap step(const Tensor& ids, const Tensor& positions);

  // prompt int64 [B, S] (host or device): positions start .. start + S - 1 take the prompt, then
  // `steps` greedy tokens follow. Returns the generated ids, int64 [B, steps], on the host. No
  // step synchronizes with the host (the position range is checked once up front).
  Tensor generate(const Tensor& prompt, std::int64_t steps, std::int64_t start = 0);

  // Synchronizes, then raises if a step since the last check reported a failed launch.
  void checkStatus();

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

}  // namespace dli
