// The importance scores and the RoPE table: device buffers of the runtime
// with their fill, fold and table launches (reference:
// src/core_kernels/importance_scores.{h,cu}, rope_table.{h,cu}).

#include "runtime.hpp"

#include <algorithm>
#include <cmath>

namespace mi
{
  // ---- ImportanceScores -----------------------------------------------------------

  ImportanceScores::ImportanceScores(int layers, int max_pages, float alpha)
      : layers_(layers), max_pages_(max_pages), alpha_(alpha)
  {
    if (layers <= 0 || max_pages <= 0)
    {
      throw InvalidArgument("layers and max_pages must be positive");
    }
    if (!(alpha > 0.0f && alpha <= 1.0f))
    {
      throw InvalidArgument("alpha, the newest observation's weight, is in (0, 1]; got " +
                            std::to_string(alpha));
    }
    const std::size_t count = static_cast<std::size_t>(layers) * max_pages;
    scores_ = std::make_unique<DeviceBuffer>(count * sizeof(float));
    launch_fill(scores_->as<float>(), count, NAN, runtime_stream());
  }

  float *ImportanceScores::layer_scores(int layer) const
  {
    if (layer < 0 || layer >= layers_)
    {
      throw OutOfRange("layer " + std::to_string(layer) + " of " + std::to_string(layers_));
    }
    return scores_->as<float>() + static_cast<std::size_t>(layer) * max_pages_;
  }

  void ImportanceScores::fold(int layer, const float *mass, int heads, int pages,
                              hipStream_t stream)
  {
    float *row = layer_scores(layer);
    if (pages < 0 || pages > max_pages_ || heads <= 0)
    {
      throw InvalidArgument(std::to_string(pages) + " pages of " + std::to_string(heads) +
                            " heads; the scores hold up to " + std::to_string(max_pages_) +
                            " pages, and a mass has a head at least");
    }
    launch_fold(row, mass, heads, pages, alpha_, stream);
  }

  std::vector<float> ImportanceScores::download()
  {
    std::vector<float> host(static_cast<std::size_t>(layers_) * max_pages_);
    hip_check(hipMemcpy(host.data(), scores_->raw(), host.size() * sizeof(float),
                        hipMemcpyDeviceToHost),
              "hipMemcpy importance scores device-to-host");
    ++downloads_;
    return host;
  }

  void ImportanceScores::upload(const float *host, int layers, int max_pages)
  {
    if (layers != layers_ || max_pages != max_pages_)
    {
      throw InvalidArgument("scores to put back are (layers, max_pages), (" +
                            std::to_string(layers_) + ", " + std::to_string(max_pages_) +
                            "); got (" + std::to_string(layers) + ", " +
                            std::to_string(max_pages) + ")");
    }
    hip_check(hipMemcpy(scores_->raw(), host, nbytes(), hipMemcpyHostToDevice),
              "hipMemcpy importance scores host-to-device");
  }

  // ---- RopeTable --------------------------------------------------------------------

  RopeTable::RopeTable(int head_dim, double theta) : head_dim_(head_dim), theta_(theta)
  {
    if (head_dim <= 0 || head_dim % 2 != 0)
    {
      throw InvalidArgument("head_dim must be positive and even, got " + std::to_string(head_dim));
    }
    if (!(theta > 0.0))
    {
      throw InvalidArgument("theta must be positive, got " + std::to_string(theta));
    }
  }

  void RopeTable::cover(int count)
  {
    if (count <= positions_)
    {
      return;
    }
    const int grown = std::max({count, 2 * positions_, kAngleRows});
    auto table = std::make_unique<DeviceBuffer>(static_cast<std::size_t>(grown) * head_dim_ *
                                                sizeof(float));
    launch_rope_table(table->as<float>(), grown, head_dim_, theta_, runtime_stream());
    auto angles = std::make_unique<DeviceBuffer>(static_cast<std::size_t>(kAngleRows) * head_dim_ *
                                                 2 * sizeof(std::uint16_t));
    launch_rope_angles(table->as<const float>(), angles->as<std::uint16_t>(), kAngleRows,
                       head_dim_, runtime_stream());
    table_ = std::move(table);
    angles_ = std::move(angles);
    positions_ = grown;
  }

} // namespace mi
