// A decode step captured as one HIP graph (the design is described in
// decode_step.hpp).

#include "decode_step.hpp"

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <string>
#include <vector>

namespace mi
{
  namespace
  {
    std::unique_ptr<DeviceBuffer> device_bytes(std::size_t bytes)
    {
      return std::make_unique<DeviceBuffer>(std::max<std::size_t>(bytes, 256));
    }

    void require(bool ok, const std::string &what)
    {
      if (!ok)
      {
        throw InvalidArgument(what);
      }
    }
  } // namespace

  DecodeStep::DecodeStep(KVPages &cache, const ModelShape &shape, ModelWeights weights,
                         ImportanceScores *scores, int score_every)
      : cache_(cache), shape_(shape), weights_(std::move(weights)), scores_(scores),
        score_every_(score_every), rope_(shape.head_dim, shape.rope_theta)
  {
    const ModelShape &s = shape_;
    require(s.layers > 0 && s.hidden > 0 && s.intermediate > 0 && s.heads > 0 && s.kv_heads > 0 &&
                s.head_dim > 0 && s.vocab > 0,
            "a model's layers, widths, heads and vocabulary are positive");
    require(s.heads % s.kv_heads == 0, "query heads are a multiple of KV heads");
    require(s.hidden % 8 == 0 && s.intermediate % 8 == 0 && (s.heads * s.head_dim) % 8 == 0,
            "a step's projections take inputs of a multiple of 8 values");
    require(cache.layers() == s.layers && cache.kv_heads() == s.kv_heads &&
                cache.head_dim() == s.head_dim,
            "the cache holds " + std::to_string(cache.layers()) + " layers of " +
                std::to_string(cache.kv_heads()) + " x " + std::to_string(cache.head_dim()) +
                "; the model has " + std::to_string(s.layers) + " of " +
                std::to_string(s.kv_heads) + " x " + std::to_string(s.head_dim));
    require(cache.seals() && cache.halves() == Halves::kBoth,
            "a graphed decode step runs on a cache that seals its pages (a tier map, a quantised "
            "tier or always_seal), with both halves at their tiers");
    require(weights_.embed != nullptr && weights_.final_norm != nullptr && weights_.head != nullptr &&
                static_cast<int>(weights_.layers.size()) == s.layers,
            "the model's embedding, final norm, head and every layer's weights are needed");
    require(score_every >= 1, "score_every is a count of steps, at least 1");
    require(scores == nullptr || scores->layers() == s.layers,
            "the scores hold a row a layer of the cache");
    int biased = 0;
    for (const LayerWeights &w : weights_.layers)
    {
      require(w.input_norm && w.q_w && w.k_w && w.v_w && w.o_w && w.post_norm && w.gate_w &&
                  w.up_w && w.down_w,
              "every layer needs its norms and its seven projection weights");
      biased += w.k_b != nullptr ? 1 : 0;
    }
    require(biased == 0 || biased == s.layers, "a key bias on every layer or on none");
    key_bias_ = biased == s.layers;

    const std::size_t q_width = static_cast<std::size_t>(s.heads) * s.head_dim;
    const std::size_t kv_width = static_cast<std::size_t>(s.kv_heads) * s.head_dim;
    state_ = device_bytes(4 * sizeof(int));
    residual_ = device_bytes(static_cast<std::size_t>(s.hidden) * sizeof(float));
    normed_ = device_bytes(static_cast<std::size_t>(s.hidden) * 2);
    qk_ = device_bytes((q_width + kv_width) * 2);
    v_ = device_bytes(kv_width * 2);
    attended_ = device_bytes(q_width * 2);
    activated_ = device_bytes(static_cast<std::size_t>(s.intermediate) * 2);
    logits_ = device_bytes(static_cast<std::size_t>(s.vocab) * sizeof(float));
    ProjectArgs head{};
    head.segments = 1;
    head.seg[0].rows = s.vocab;
    head.in = s.hidden;
    head.mode = ProjectMode::kLogits;
    head_blocks_ = project_blocks(head);
    best_value_ = device_bytes(static_cast<std::size_t>(head_blocks_) * sizeof(float));
    best_index_ = device_bytes(static_cast<std::size_t>(head_blocks_) * sizeof(int));
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate step");
    hip_check(hipEventCreate(&begin_), "hipEventCreate");
    hip_check(hipEventCreate(&end_), "hipEventCreate");
  }

  DecodeStep::~DecodeStep()
  {
    if (stream_ != nullptr)
    {
      (void)hipStreamSynchronize(stream_);
    }
    if (exec_ != nullptr)
    {
      (void)hipGraphExecDestroy(exec_);
    }
    if (begin_ != nullptr)
    {
      (void)hipEventDestroy(begin_);
    }
    if (end_ != nullptr)
    {
      (void)hipEventDestroy(end_);
    }
    if (stream_ != nullptr)
    {
      (void)hipStreamDestroy(stream_);
    }
  }

  void DecodeStep::size_buffers(int steps)
  {
    if (steps > token_room_)
    {
      tokens_ = device_bytes(static_cast<std::size_t>(steps) * sizeof(std::int32_t));
      token_room_ = steps;
    }
  }

  void DecodeStep::enqueue_step(int max_seq_k, hipStream_t stream)
  {
    const ModelShape &s = shape_;
    const int q_width = s.heads * s.head_dim;
    int *state = state_->as<int>();
    float *residual = residual_->as<float>();
    auto *normed = normed_->as<std::uint16_t>();
    auto *qk = qk_->as<std::uint16_t>();
    auto *v = v_->as<std::uint16_t>();
    auto *attended = attended_->as<std::uint16_t>();
    auto *activated = activated_->as<std::uint16_t>();
    float *kept = scores_ != nullptr ? kept_->as<float>() : nullptr;
    int launches = 0;
    plans_.clear();
    // The plan each of the step's GEMVs ran as (layer 0's and the head's),
    // for tools and tests that check which variant a shape takes.
    const auto record = [&](int what, const ProjectArgs &p, ProjectPlanInfo info) {
      plans_.insert(plans_.end(), {what, p.seg[0].rows, p.in, info.split, info.pipelined,
                                   info.waves, info.blocks});
    };

    // RMSNorm rides in the projection that reads its output (each workgroup
    // forms the normed row from the fp32 residual, to the RMSNorm kernel's
    // bits), RoPE and the open page's row in the q/k/v launch, the page's
    // seal in the decode's combine: six launches a layer.
    const auto normed_input = [&](ProjectArgs &p, const std::uint16_t *norm) {
      p.residual = residual;
      p.norm_weight = norm;
      p.eps = s.rms_eps;
      p.x = normed; // unused with a norm
    };
    launch_embed(state + kStepToken, 1, weights_.embed, residual, true, s.hidden, s.vocab, stream);
    ++launches;
    for (int l = 0; l < s.layers; ++l)
    {
      const LayerWeights &w = weights_.layers[l];
      // q, k and v with the input's RMSNorm, RoPE and the open page's row in
      // one launch; the page's seal, when the row is its last, rides in the
      // decode's combine.
      const StepStore target = cache_.step_store(l, qk + q_width, v, state + kStepPosition);
      QkvStep qkv{};
      qkv.w[0] = w.q_w;
      qkv.w[1] = w.k_w;
      qkv.w[2] = w.v_w;
      qkv.b[0] = w.q_b;
      // The key bias, when attention adds it rotated, stays out of k.
      qkv.b[1] = key_bias_ ? nullptr : w.k_b;
      qkv.b[2] = w.v_b;
      qkv.in = s.hidden;
      qkv.residual = residual;
      qkv.norm_weight = w.input_norm;
      qkv.eps = s.rms_eps;
      qkv.heads = s.heads;
      qkv.kv_heads = s.kv_heads;
      qkv.head_dim = s.head_dim;
      qkv.rope = rope_.data();
      qkv.position = state + kStepPosition;
      qkv.qk = qk;
      qkv.v = v;
      qkv.open = target.open;
      launch_qkv_step(qkv, stream);
      cache_.attention_step(l, qk, key_bias_ ? w.k_b : nullptr, &rope_, attended,
                            state + kStepSeqK, max_seq_k, s.heads, s.kv_heads, s.head_dim,
                            qk + q_width, v, kept, &target);
      ProjectArgs o{};
      o.segments = 1;
      o.seg[0] = {w.o_w, nullptr, residual, s.hidden};
      o.in = q_width;
      o.x = attended;
      o.mode = ProjectMode::kAccumulate;
      const ProjectPlanInfo o_plan = launch_project(o, stream);
      ProjectArgs mlp{};
      mlp.segments = 2;
      mlp.seg[0] = {w.gate_w, nullptr, activated, s.intermediate};
      mlp.seg[1] = {w.up_w, nullptr, nullptr, s.intermediate};
      mlp.in = s.hidden;
      mlp.mode = ProjectMode::kSwiglu;
      normed_input(mlp, w.post_norm);
      const ProjectPlanInfo mlp_plan = launch_project(mlp, stream);
      ProjectArgs down{};
      down.segments = 1;
      down.seg[0] = {w.down_w, nullptr, residual, s.hidden};
      down.in = s.intermediate;
      down.x = activated;
      down.mode = ProjectMode::kAccumulate;
      const ProjectPlanInfo down_plan = launch_project(down, stream);
      if (l == 0)
      {
        record(kPlanOutput, o, o_plan);
        record(kPlanGateUp, mlp, mlp_plan);
        record(kPlanDown, down, down_plan);
      }
      launches += 6; // norm + qkv + RoPE + store, decode + combine (+ seal), o, norm + gate/up,
                     // down
    }
    ProjectArgs head{};
    head.segments = 1;
    head.seg[0] = {weights_.head, nullptr, logits_->as<float>(), s.vocab};
    head.in = s.hidden;
    head.mode = ProjectMode::kLogits;
    normed_input(head, weights_.final_norm);
    head.best_value = best_value_->as<float>();
    head.best_index = best_index_->as<int>();
    head.best_count = head_blocks_;
    record(kPlanHead, head, launch_project(head, stream));
    ++launches;
    if (scores_ != nullptr)
    {
      cache_.fold_step(kept, state + kStepSeqK, max_seq_k, s.heads, s.kv_heads, s.head_dim,
                       score_every_, scores_->layer_scores(0), scores_->max_pages(),
                       scores_->alpha());
      ++launches;
    }
    launch_advance(best_value_->as<float>(), best_index_->as<int>(), head_blocks_, s.vocab, state,
                   tokens_->as<std::int32_t>(), token_room_, stream);
    ++launches;
    launches_ = launches;
  }

  void DecodeStep::prepare_launches(int max_seq_k)
  {
    const ModelShape &s = shape_;
    // Everything the launches use is made before the capture: the tables
    // and scratch at max_seq_k, the RoPE table, the kept statistics.
    rope_.cover(std::max(max_seq_k, RopeTable::kAngleRows));
    cache_.prepare_step(max_seq_k, s.heads, s.head_dim);
    if (scores_ != nullptr)
    {
      const int pages = (max_seq_k + cache_.page_tokens() - 1) / cache_.page_tokens();
      require(pages <= scores_->max_pages(),
              "the scores hold " + std::to_string(scores_->max_pages()) + " pages a layer; the "
              "run reaches " + std::to_string(pages));
      const std::size_t floats = decode_kept_floats(s.heads, s.kv_heads, max_seq_k) * s.layers;
      if (kept_ == nullptr || kept_->bytes() < floats * sizeof(float))
      {
        kept_ = device_bytes(floats * sizeof(float));
      }
    }
    // The step's stream does not wait for other streams: whatever the cache
    // launched on them (table edits, allocations) is finished first.
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize before capture");
  }

  void DecodeStep::capture(int max_seq_k)
  {
    prepare_launches(max_seq_k);
    if (exec_ != nullptr)
    {
      hip_check(hipGraphExecDestroy(exec_), "hipGraphExecDestroy");
      exec_ = nullptr;
    }
    const hipStream_t previous = runtime_stream();
    set_runtime_stream(stream_);
    hipGraph_t graph = nullptr;
    hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal),
              "hipStreamBeginCapture step");
    try
    {
      enqueue_step(max_seq_k, stream_);
    }
    catch (...)
    {
      (void)hipStreamEndCapture(stream_, &graph);
      if (graph != nullptr)
      {
        (void)hipGraphDestroy(graph);
      }
      set_runtime_stream(previous);
      throw;
    }
    const hipError_t ended = hipStreamEndCapture(stream_, &graph);
    set_runtime_stream(previous);
    hip_check(ended, "hipStreamEndCapture step");
    const hipError_t made = hipGraphInstantiate(&exec_, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    hip_check(made, "hipGraphInstantiate step");
  }

  double DecodeStep::run(int token, int position, int steps, std::int32_t *tokens, bool graphed)
  {
    require(steps > 0 && position >= 0, "a run takes at least one step from a position >= 0");
    require(tokens != nullptr, "a run writes its tokens to host memory");
    const int end = position + steps;
    // The run's pages, then a graph for the most positions it attends (or,
    // eager, the same launches made from the host a step at a time).
    cache_.reserve(end);
    size_buffers(steps);
    if (graphed)
    {
      capture(end);
    }
    else
    {
      prepare_launches(end);
    }
    const int state[4] = {token, position, position + 1, 0};
    hip_check(hipMemcpyAsync(state_->raw(), state, sizeof(state), hipMemcpyHostToDevice, stream_),
              "hipMemcpyAsync step state");
    hip_check(hipEventRecord(begin_, stream_), "hipEventRecord");
    if (graphed)
    {
      for (int i = 0; i < steps; ++i)
      {
        hip_check(hipGraphLaunch(exec_, stream_), "hipGraphLaunch step");
      }
    }
    else
    {
      const hipStream_t previous = runtime_stream();
      set_runtime_stream(stream_);
      try
      {
        for (int i = 0; i < steps; ++i)
        {
          enqueue_step(end, stream_);
        }
      }
      catch (...)
      {
        set_runtime_stream(previous);
        throw;
      }
      set_runtime_stream(previous);
    }
    hip_check(hipEventRecord(end_, stream_), "hipEventRecord");
    hip_check(hipMemcpyAsync(tokens, tokens_->raw(), static_cast<std::size_t>(steps) * 4,
                             hipMemcpyDeviceToHost, stream_),
              "hipMemcpyAsync tokens");
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize step run");
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, begin_, end_), "hipEventElapsedTime");
    cache_.stored_on_device(end);
    return ms;
  }

  void DecodeStep::size_chunk(int rows, int prompt)
  {
    const ModelShape &s = shape_;
    const std::size_t q_width = static_cast<std::size_t>(s.heads) * s.head_dim;
    const std::size_t kv_width = static_cast<std::size_t>(s.kv_heads) * s.head_dim;
    if (rows > chunk_room_)
    {
      const std::size_t r = rows;
      c_residual_ = device_bytes(r * s.hidden * sizeof(float));
      c_normed_ = device_bytes(r * s.hidden * 2);
      c_q_raw_ = device_bytes(r * q_width * 2);
      c_q_ = device_bytes(r * q_width * 2);
      c_k_raw_ = device_bytes(r * kv_width * 2);
      c_k_ = device_bytes(r * kv_width * 2);
      c_v_ = device_bytes(r * kv_width * 2);
      c_attended_ = device_bytes(r * q_width * 2);
      c_gate_ = device_bytes(r * s.intermediate * 2);
      c_up_ = device_bytes(r * s.intermediate * 2);
      c_act_ = device_bytes(r * s.intermediate * 2);
      chunk_room_ = rows;
    }
    if (c_partials_ == nullptr)
    {
      c_partials_ = device_bytes(attention_partials_floats(s.head_dim) * sizeof(float));
    }
    if (prompt > prompt_room_)
    {
      c_ids_ = device_bytes(static_cast<std::size_t>(prompt) * sizeof(std::int32_t));
      c_positions_ = device_bytes(static_cast<std::size_t>(prompt) * sizeof(std::int32_t));
      prompt_room_ = prompt;
    }
  }

  double DecodeStep::prefill(const std::int32_t *tokens, int n, int position, int chunk,
                             std::int32_t *first)
  {
    const ModelShape &s = shape_;
    require(n > 0 && position >= 0 && chunk > 0, "a prefill takes at least one token, a position "
                                                 ">= 0 and chunks of at least one row");
    require(tokens != nullptr && first != nullptr, "a prefill reads its tokens from host memory "
                                                   "and writes the first decode token there");
    const int q_width = s.heads * s.head_dim;
    const int kv_width = s.kv_heads * s.head_dim;
    const int rows_most = std::min(chunk, n);
    cache_.reserve(position + n);
    rope_.cover(std::max(position + n, RopeTable::kAngleRows));
    size_chunk(rows_most, n);
    size_buffers(1);
    std::vector<std::int32_t> at(static_cast<std::size_t>(n));
    for (int i = 0; i < n; ++i)
    {
      at[i] = position + i;
    }
    const int state[4] = {0, position + n - 1, position + n, 0};
    // Whatever the cache launched elsewhere (table edits, the reservation's
    // pages) is done before this stream starts.
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize before a prefill");
    const hipStream_t stream = stream_;
    hip_check(hipMemcpyAsync(c_ids_->raw(), tokens, static_cast<std::size_t>(n) * 4,
                             hipMemcpyHostToDevice, stream),
              "hipMemcpyAsync prompt");
    hip_check(hipMemcpyAsync(c_positions_->raw(), at.data(), static_cast<std::size_t>(n) * 4,
                             hipMemcpyHostToDevice, stream),
              "hipMemcpyAsync positions");
    hip_check(hipMemcpyAsync(state_->raw(), state, sizeof(state), hipMemcpyHostToDevice, stream),
              "hipMemcpyAsync step state");
    const hipStream_t previous = runtime_stream();
    set_runtime_stream(stream);
    float *residual = c_residual_->as<float>();
    auto *normed = c_normed_->as<std::uint16_t>();
    auto *q_raw = c_q_raw_->as<std::uint16_t>();
    auto *q = c_q_->as<std::uint16_t>();
    auto *k_raw = c_k_raw_->as<std::uint16_t>();
    auto *k = c_k_->as<std::uint16_t>();
    auto *v = c_v_->as<std::uint16_t>();
    auto *attended = c_attended_->as<std::uint16_t>();
    auto *gate = c_gate_->as<std::uint16_t>();
    auto *up = c_up_->as<std::uint16_t>();
    auto *act = c_act_->as<std::uint16_t>();
    const auto *ids = c_ids_->as<const std::int32_t>();
    const auto *positions = c_positions_->as<const std::int32_t>();
    float ms = 0.0f;
    try
    {
      hip_check(hipEventRecord(begin_, stream), "hipEventRecord");
      int last_rows = 0;
      for (int c0 = 0; c0 < n; c0 += chunk)
      {
        const int rows = std::min(chunk, n - c0);
        const int p0 = position + c0;
        launch_embed(ids + c0, rows, weights_.embed, residual, true, s.hidden, s.vocab, stream);
        for (int l = 0; l < s.layers; ++l)
        {
          const LayerWeights &w = weights_.layers[l];
          launch_rmsnorm(residual, true, w.input_norm, normed, rows, s.hidden, s.rms_eps, stream);
          linear_half(normed, w.q_w, w.q_b, q_raw, rows, s.hidden, q_width, stream);
          // The key bias, when attention adds it rotated, stays out of k.
          linear_half(normed, w.k_w, key_bias_ ? nullptr : w.k_b, k_raw, rows, s.hidden,
                      kv_width, stream);
          linear_half(normed, w.v_w, w.v_b, v, rows, s.hidden, kv_width, stream);
          // RoPE of q and k in one launch, the angles from the step's table
          // (the RoPE kernel's rows to the bit).
          RopeRows rope{};
          rope.x[0] = q_raw;
          rope.out[0] = q;
          rope.heads[0] = s.heads;
          rope.x[1] = k_raw;
          rope.out[1] = k;
          rope.heads[1] = s.kv_heads;
          rope.positions = positions + c0;
          rope.table = rope_.data();
          rope.table_positions = rope_.positions();
          rope.seq = rows;
          rope.head_dim = s.head_dim;
          launch_rope_rows(rope, stream);
          cache_.store(l, k, v, p0, rows);
          cache_.attention(l, q, key_bias_ ? w.k_b : nullptr, &rope_, attended, rows, p0 + rows,
                           s.heads, s.kv_heads, s.head_dim, k, v, nullptr, nullptr, 0.0f,
                           c_partials_->as<float>());
          linear_float(attended, w.o_w, residual, true, rows, q_width, s.hidden, stream);
          launch_rmsnorm(residual, true, w.post_norm, normed, rows, s.hidden, s.rms_eps, stream);
          linear_half(normed, w.gate_w, nullptr, gate, rows, s.hidden, s.intermediate, stream);
          linear_half(normed, w.up_w, nullptr, up, rows, s.hidden, s.intermediate, stream);
          launch_swiglu(gate, up, act, static_cast<std::size_t>(rows) * s.intermediate, stream);
          linear_float(act, w.down_w, residual, true, rows, s.intermediate, s.hidden, stream);
        }
        last_rows = rows;
      }
      // The last row's logits, its RMSNorm formed in the head's projection,
      // and the greedy token: the state moves to the first decode step.
      ProjectArgs head{};
      head.segments = 1;
      head.seg[0] = {weights_.head, nullptr, logits_->as<float>(), s.vocab};
      head.in = s.hidden;
      head.mode = ProjectMode::kLogits;
      head.residual = residual + static_cast<std::size_t>(last_rows - 1) * s.hidden;
      head.norm_weight = weights_.final_norm;
      head.eps = s.rms_eps;
      head.x = normed;
      head.best_value = best_value_->as<float>();
      head.best_index = best_index_->as<int>();
      head.best_count = head_blocks_;
      launch_project(head, stream);
      launch_advance(best_value_->as<float>(), best_index_->as<int>(), head_blocks_, s.vocab,
                     state_->as<int>(), tokens_->as<std::int32_t>(), token_room_, stream);
      hip_check(hipEventRecord(end_, stream), "hipEventRecord");
      hip_check(hipMemcpyAsync(first, state_->as<int>() + kStepToken, sizeof(std::int32_t),
                               hipMemcpyDeviceToHost, stream),
                "hipMemcpyAsync first token");
      hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize prefill");
      hip_check(hipEventElapsedTime(&ms, begin_, end_), "hipEventElapsedTime");
    }
    catch (...)
    {
      set_runtime_stream(previous);
      throw;
    }
    set_runtime_stream(previous);
    return ms;
  }

  void DecodeStep::logits(float *host, std::size_t count) const
  {
    require(count <= static_cast<std::size_t>(shape_.vocab),
            "the logits are " + std::to_string(shape_.vocab) + " values");
    hip_check(hipMemcpyAsync(host, logits_->raw(), count * sizeof(float), hipMemcpyDeviceToHost,
                             stream_),
              "hipMemcpyAsync logits");
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize logits");
  }

} // namespace mi
