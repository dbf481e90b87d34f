// The small kernels around the dense projections: the embedding gather, the
// greedy argmax over logits, and the bias rows of an empty projection.
//
// Reference: embed.cu:17-76 (a gather, bit for bit; fp32 output is the fp16
// row widened exactly; an id outside the vocabulary reads as a zero row),
// argmax.cu:17-81 (the largest logit, the lowest index on a tie, NaN never
// chosen; a row with no value >= -FLT_MAX, all -inf or NaN, gives `cols`,
// one past its last index).

#include "common.hpp"
#include "kernels.hpp"

#include <cfloat>

namespace mi
{
  namespace
  {

    constexpr int kThreads = 256;

    __device__ inline void store_row_element(std::uint16_t *out, std::uint16_t v) { *out = v; }
    __device__ inline void store_row_element(float *out, std::uint16_t v) { *out = h2f(v); }

    // A workgroup per token, its row copied element by element (a step
    // gathers a few rows of a few KB). An unknown id's row is never read.
    template <typename Out>
    __global__ void __launch_bounds__(kThreads)
        embed_kernel(const std::int32_t *__restrict__ ids, const std::uint16_t *__restrict__ table,
                     Out *__restrict__ out, int hidden, int vocab)
    {
      const std::int32_t id = ids[blockIdx.x];
      const bool known = id >= 0 && id < vocab;
      const std::uint16_t *row = table + static_cast<std::size_t>(known ? id : 0) * hidden;
      Out *dst = out + static_cast<std::size_t>(blockIdx.x) * hidden;
      for (int c = threadIdx.x; c < hidden; c += blockDim.x)
      {
        const std::uint16_t v = known ? row[c] : std::uint16_t(0);
        store_row_element(dst + c, v);
      }
    }

    // The better of two (value, index) candidates: the larger value, the
    // lower index on equal values; a NaN compares false and never wins.
    // Commutative and associative, so any reduction order gives one answer.
    __device__ inline void keep_better(float &best, int &at, float value, int index)
    {
      if (value > best || (value == best && index < at))
      {
        best = value;
        at = index;
      }
    }

    __global__ void __launch_bounds__(kThreads)
        argmax_kernel(const float *__restrict__ x, int cols, std::int32_t *__restrict__ out)
    {
      __shared__ float s_best[kThreads / 64];
      __shared__ int s_at[kThreads / 64];
      const float *row = x + static_cast<std::size_t>(blockIdx.x) * cols;
      float best = -FLT_MAX;
      int at = cols;
      for (int c = threadIdx.x; c < cols; c += blockDim.x)
      {
        keep_better(best, at, row[c], c);
      }
      for (int offset = 32; offset > 0; offset >>= 1)
      {
        const float b = __shfl_xor(best, offset);
        const int a = __shfl_xor(at, offset);
        keep_better(best, at, b, a);
      }
      const int wave = threadIdx.x / 64;
      if (threadIdx.x % 64 == 0)
      {
        s_best[wave] = best;
        s_at[wave] = at;
      }
      __syncthreads();
      if (threadIdx.x == 0)
      {
        for (int w = 1; w < kThreads / 64; ++w)
        {
          keep_better(best, at, s_best[w], s_at[w]);
        }
        out[blockIdx.x] = at;
      }
    }

    __global__ void __launch_bounds__(kThreads)
        broadcast_rows_kernel(const std::uint16_t *__restrict__ row, std::uint16_t *__restrict__ out,
                              int cols, std::size_t count)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        out[i] = row != nullptr ? row[i % cols] : std::uint16_t(0);
      }
    }

  } // namespace

  void launch_embed(const std::int32_t *ids, int count, const void *table, void *out,
                    bool out_is_f32, int hidden, int vocab, hipStream_t stream)
  {
    if (count < 0 || hidden < 0 || vocab < 0)
    {
      throw InvalidArgument("embed's count, hidden and vocab are >= 0");
    }
    if (count == 0 || hidden == 0)
    {
      return;
    }
    const auto *t = static_cast<const std::uint16_t *>(table);
    if (out_is_f32)
    {
      hipLaunchKernelGGL(embed_kernel<float>, dim3(count), dim3(kThreads), 0, stream, ids, t,
                         static_cast<float *>(out), hidden, vocab);
    }
    else
    {
      hipLaunchKernelGGL(embed_kernel<std::uint16_t>, dim3(count), dim3(kThreads), 0, stream, ids,
                         t, static_cast<std::uint16_t *>(out), hidden, vocab);
    }
    hip_check(hipGetLastError(), "embed kernel launch");
  }

  void launch_argmax_rows(const float *x, int rows, int cols, std::int32_t *out,
                          hipStream_t stream)
  {
    if (rows <= 0 || cols <= 0)
    {
      return;
    }
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kThreads), 0, stream, x, cols, out);
    hip_check(hipGetLastError(), "argmax kernel launch");
  }

  void launch_broadcast_rows(const void *row, void *out, int rows, int cols, hipStream_t stream)
  {
    const std::size_t count = static_cast<std::size_t>(rows) * cols;
    if (count == 0)
    {
      return;
    }
    const int blocks = static_cast<int>(std::min<std::size_t>((count + kThreads - 1) / kThreads, 4096));
    hipLaunchKernelGGL(broadcast_rows_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                       static_cast<const std::uint16_t *>(row), static_cast<std::uint16_t *>(out),
                       cols, count);
    hip_check(hipGetLastError(), "bias broadcast launch");
  }

} // namespace mi
