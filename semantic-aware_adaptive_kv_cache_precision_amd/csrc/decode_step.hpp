// A whole decode step of a Qwen2 / Llama-shaped decoder as one HIP graph,
// replayed once a token.
//
// The reference sequences a step from the host, a device call at a time
// (src/microinfer/model.py:332-403 Model.run, engine.py:1180-1206 greedy
// generation). Here the step's token, position and seq_k live in device
// memory and every kernel reads them there: the store writes its row at the
// device's position, the decode reads the device's seq_k, the head's argmax
// writes the next token and moves the position on. So one graph, captured
// for the most positions a run attends, serves every step of the run with
// nothing from the host between steps; the host reserves the run's pages
// first (allocation is a host operation) and records what was stored after.
//
// Layers as the reference's (model.py:366-403): RMSNorm of the fp32
// residual, q/k/v projections (k without its bias when attention adds the
// rotated bias, ADR-0009), RoPE, the store, the paged decode, the output
// projection added into the residual, RMSNorm, gate/up with SwiGLU, the down
// projection added into the residual; then the final RMSNorm, the head's
// logits, and the greedy token. With scores, each layer keeps its page
// statistics and one launch a step folds every layer's into the scores.

#pragma once

#include "runtime.hpp"

#include <cstdint>
#include <memory>
#include <vector>

namespace mi
{
  struct ModelShape
  {
    int layers;
    int hidden;
    int intermediate;
    int heads;
    int kv_heads;
    int head_dim;
    int vocab;
    float rms_eps;
    double rope_theta;
  };

  // One layer's tensors, fp16 on the device, [out][in] row-major; a bias
  // may be null.
  struct LayerWeights
  {
    const std::uint16_t *input_norm;
    const std::uint16_t *q_w;
    const std::uint16_t *q_b;
    const std::uint16_t *k_w;
    const std::uint16_t *k_b;
    const std::uint16_t *v_w;
    const std::uint16_t *v_b;
    const std::uint16_t *o_w;
    const std::uint16_t *post_norm;
    const std::uint16_t *gate_w;
    const std::uint16_t *up_w;
    const std::uint16_t *down_w;
  };

  struct ModelWeights
  {
    const std::uint16_t *embed;      // [vocab][hidden]
    const std::uint16_t *final_norm; // [hidden]
    const std::uint16_t *head;       // [vocab][hidden]
    std::vector<LayerWeights> layers;
  };

  class DecodeStep
  {
  public:
    // `cache` (a sealing cache of shape.layers layers) must outlive the
    // step. `scores`, if not null, takes each step's masses at the cadence
    // `score_every` (a step whose seq_k is a multiple of it).
    DecodeStep(KVPages &cache, const ModelShape &shape, ModelWeights weights,
               ImportanceScores *scores, int score_every);
    ~DecodeStep();
    DecodeStep(const DecodeStep &) = delete;
    DecodeStep &operator=(const DecodeStep &) = delete;

    // The prompt `tokens` (n of them) at positions [position, position + n)
    // in chunks of `chunk` rows, each chunk a layer at a time as the
    // reference's Model.run takes them (model.py:332-403): RMSNorm, the
    // q/k/v projections (hipBLASLt), RoPE, the store (sealing pages as they
    // fill), the chunk's attention (the matrix-core kernel over the pages
    // before each query's own at their tiers), the output projection into
    // the fp32 residual, RMSNorm, gate and up, SwiGLU, down. Then the last
    // row's logits and greedy token: the first decode token, returned in
    // *first. Returns the device milliseconds of the whole prefill.
    double prefill(const std::int32_t *tokens, int n, int position, int chunk,
                   std::int32_t *first);
    // `steps` greedy steps: the first feeds `token` at `position` (the cache
    // holds every position before it), each later one the token before it.
    // The chosen tokens go to `tokens` (host, `steps` of them). Returns the
    // device milliseconds of the graph's replays (the run's steps). With
    // `graphed` false the same launches are made from the host, a step at a
    // time (bit-identical; for tools that follow individual launches).
    double run(int token, int position, int steps, std::int32_t *tokens, bool graphed = true);
    // The last step's logits (fp32, vocab of them) to host memory.
    void logits(float *host, std::size_t count) const;
    // Launches a step makes (the graph's kernel nodes).
    int launches() const { return launches_; }
    // The plans the last step's GEMVs ran as, seven ints each: which
    // projection (kPlanOutput, kPlanGateUp, kPlanDown: layer 0's; kPlanHead),
    // its rows, its input length, the waves a row is split over, whether the
    // grid was the resident one (several rows a wave), the waves a
    // workgroup, the workgroups.
    static constexpr int kPlanOutput = 0, kPlanGateUp = 1, kPlanDown = 2, kPlanHead = 3;
    static constexpr int kPlanInts = 7;
    const std::vector<int> &plans() const { return plans_; }

  private:
    void size_buffers(int steps);
    void prepare_launches(int max_seq_k);
    void capture(int max_seq_k);
    void enqueue_step(int max_seq_k, hipStream_t stream);

    KVPages &cache_;
    ModelShape shape_;
    ModelWeights weights_;
    ImportanceScores *scores_;
    int score_every_;
    bool key_bias_; // every layer has a key bias: attention adds it rotated
    RopeTable rope_;
    hipStream_t stream_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
    hipEvent_t begin_ = nullptr;
    hipEvent_t end_ = nullptr;
    int launches_ = 0;
    std::vector<int> plans_;
    int head_blocks_ = 0;
    int token_room_ = 0;
    // Device buffers: the step's state (four ints), the residual (fp32),
    // the normed input, [q | k] after RoPE, v, the attention's
    // output, the MLP's activation, the logits, the head's block bests, the
    // kept page statistics, and the run's tokens.
    std::unique_ptr<DeviceBuffer> state_;
    std::unique_ptr<DeviceBuffer> residual_;
    std::unique_ptr<DeviceBuffer> normed_;
    std::unique_ptr<DeviceBuffer> qk_;
    std::unique_ptr<DeviceBuffer> v_;
    std::unique_ptr<DeviceBuffer> attended_;
    std::unique_ptr<DeviceBuffer> activated_;
    std::unique_ptr<DeviceBuffer> logits_;
    std::unique_ptr<DeviceBuffer> best_value_;
    std::unique_ptr<DeviceBuffer> best_index_;
    std::unique_ptr<DeviceBuffer> kept_;
    std::unique_ptr<DeviceBuffer> tokens_;
    // A prefill's chunk buffers (rows of `chunk_room_`), its token ids and
    // positions, and the attention's partials.
    void size_chunk(int rows, int prompt);
    int chunk_room_ = 0;
    int prompt_room_ = 0;
    std::unique_ptr<DeviceBuffer> c_residual_, c_normed_, c_q_raw_, c_q_, c_k_raw_, c_k_, c_v_,
        c_attended_, c_gate_, c_up_, c_act_, c_partials_, c_ids_, c_positions_;
  };

} // namespace mi
