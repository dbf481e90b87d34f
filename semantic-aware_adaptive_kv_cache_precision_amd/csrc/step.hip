// The dense half of a decode step on gfx950: one token's projections as
// matrix-vector products streamed from HBM, the greedy choice over the
// vocabulary, and the step's advance. Every kernel that needs the step's
// token or position reads it from device memory, so that one captured graph
// serves every step of a run.
//
// Semantics are the reference's projections and their neighbours
// (linear.cu:85-142: fp16 operands, fp32 accumulation, a bias added in fp32
// before the one rounding to fp16, the residual stream accumulated in fp32
// and never rounded; swiglu.cu:26-38: silu(g) * u in fp32 from the fp16 gate
// and up; argmax.cu:17-81: the largest logit, the lowest index on a tie, NaN
// never chosen, `cols` when no value is >= -FLT_MAX).
//
// Work layout (MI355X-first): a decode step's projections are one row of
// activations against a weight matrix, so they are bound by the weight bytes
// streamed from HBM, not by arithmetic. A wave owns a weight row: the row's
// 16-byte runs go to the lanes in turn (one coalesced 1 KiB load a
// wave-instruction, several loads in flight before any is used), the
// products are v_dot2 of fp16 pairs into fp32 (each product exact), and a
// wave reduction leaves the row's dot in every lane. Eight rows a workgroup,
// so that even the 1536-row projections launch 192 workgroups and the
// vocabulary's ~19K. The projections a step makes from one input run in one
// launch: q, k and v (three weight matrices, one grid over their rows), gate
// and up (a wave both rows of one output, the SwiGLU in the epilogue).

#include "common.hpp"
#include "kernels.hpp"

#include <cfloat>
#include <climits>

namespace mi
{
  namespace
  {
    constexpr int kWaves = 8;
    constexpr int kThreads = 64 * kWaves;
    constexpr int kAhead = 4; // 16-byte runs a lane has in flight
    constexpr int kAdvanceThreads = 1024;

    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(1))) u32x4 *g_u32x4;

    __device__ inline float dot_run(const u32x4 &w, const u32x4 &x, float acc)
    {
#pragma unroll
      for (int i = 0; i < 4; ++i)
      {
        const unsigned wi = w[i], xi = x[i];
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, wi), __builtin_bit_cast(half2v, xi),
                                     acc, false);
      }
      return acc;
    }

    __device__ inline float wave_total(float v)
    {
#pragma unroll
      for (int offset = 32; offset > 0; offset >>= 1)
      {
        v += __shfl_xor(v, offset);
      }
      return v;
    }

    // The dot of a weight row with x (both `in` fp16 values, in a multiple
    // of 8, 16-byte aligned), in every lane of the wave.
    __device__ inline float row_dot(const std::uint16_t *w, const std::uint16_t *x, int in, int lane)
    {
      const int runs = in / 8;
      float acc = 0.0f;
      for (int r0 = lane; r0 < runs; r0 += 64 * kAhead)
      {
        u32x4 wv[kAhead], xv[kAhead];
#pragma unroll
        for (int i = 0; i < kAhead; ++i)
        {
          const int r = r0 + 64 * i;
          const int at = r < runs ? r : r0; // a lane past the row re-reads its first run, unused
          wv[i] = *((g_u32x4)(w + 8 * static_cast<std::size_t>(at)));
          xv[i] = *((g_u32x4)(x + 8 * static_cast<std::size_t>(at)));
        }
#pragma unroll
        for (int i = 0; i < kAhead; ++i)
        {
          if (r0 + 64 * i < runs)
          {
            acc = dot_run(wv[i], xv[i], acc);
          }
        }
      }
      return wave_total(acc);
    }

    __device__ inline std::uint16_t to_half(float v) { return __half_as_ushort(__float2half(v)); }

    // The better of two (value, index) candidates, as argmax.cu chooses: the
    // larger value, the lower index on equal values; NaN never wins.
    __device__ inline void keep_better(float &best, int &at, float value, int index)
    {
      if (value > best || (value == best && index < at))
      {
        best = value;
        at = index;
      }
    }

    // Rows of every segment in turn; a wave a row (two rows, gate and up,
    // for SwiGLU).
    __global__ void __launch_bounds__(kThreads) project_kernel(ProjectArgs p)
    {
      __shared__ float s_best[kWaves];
      __shared__ int s_at[kWaves];
      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      int row = blockIdx.x * kWaves + wave;
      int seg = 0;
      // SwiGLU's grid covers gate's rows only (up's ride with them).
      const int walked = p.mode == ProjectMode::kSwiglu ? 1 : p.segments;
      while (seg + 1 < walked && row >= p.seg[seg].rows)
      {
        row -= p.seg[seg].rows;
        ++seg;
      }
      const bool live = row < p.seg[seg].rows;
      const ProjectSegment &s = p.seg[seg];
      float best = -FLT_MAX;
      int at = INT_MAX;
      if (live)
      {
        const std::uint16_t *w = s.w + static_cast<std::size_t>(row) * p.in;
        const float acc = row_dot(w, p.x, p.in, lane);
        switch (p.mode)
        {
        case ProjectMode::kHalf:
          if (lane == 0)
          {
            const float b = s.bias != nullptr ? h2f(s.bias[row]) : 0.0f;
            static_cast<std::uint16_t *>(s.out)[row] = to_half(acc + b);
          }
          break;
        case ProjectMode::kAccumulate:
          if (lane == 0)
          {
            float *out = static_cast<float *>(s.out) + row;
            *out = *out + acc;
          }
          break;
        case ProjectMode::kSwiglu:
        {
          // seg[1] is up, with gate's rows: the same row of it.
          const std::uint16_t *wu = p.seg[1].w + static_cast<std::size_t>(row) * p.in;
          const float up = row_dot(wu, p.x, p.in, lane);
          if (lane == 0)
          {
            const float g = h2f(to_half(acc));
            const float u = h2f(to_half(up));
            const float silu = g / (1.0f + expf(-g));
            static_cast<std::uint16_t *>(s.out)[row] = to_half(silu * u);
          }
          break;
        }
        case ProjectMode::kLogits:
          if (lane == 0)
          {
            static_cast<float *>(s.out)[row] = acc;
          }
          keep_better(best, at, acc, row);
          break;
        }
      }
      if (p.mode == ProjectMode::kLogits)
      {
        // The workgroup's best logit, for the advance to choose from.
        if (lane == 0)
        {
          s_best[wave] = best;
          s_at[wave] = at;
        }
        __syncthreads();
        if (threadIdx.x == 0)
        {
          for (int w2 = 0; w2 < kWaves; ++w2)
          {
            keep_better(best, at, s_best[w2], s_at[w2]);
          }
          p.best_value[blockIdx.x] = best;
          p.best_index[blockIdx.x] = at;
        }
      }
    }

    // The step's greedy token from the head's per-block bests, then the
    // step's state moved on: the token is the next step's input and the
    // run's output, the position and seq_k advance by one.
    __global__ void __launch_bounds__(kAdvanceThreads)
        advance_kernel(const float *__restrict__ best_value, const int *__restrict__ best_index,
                       int blocks, int vocab, int *__restrict__ state,
                       std::int32_t *__restrict__ tokens, int max_tokens)
    {
      __shared__ float s_best[kAdvanceThreads / 64];
      __shared__ int s_at[kAdvanceThreads / 64];
      float best = -FLT_MAX;
      int at = INT_MAX;
      for (int b = threadIdx.x; b < blocks; b += kAdvanceThreads)
      {
        keep_better(best, at, best_value[b], best_index[b]);
      }
#pragma unroll
      for (int offset = 32; offset > 0; offset >>= 1)
      {
        const float v = __shfl_xor(best, offset);
        const int i = __shfl_xor(at, offset);
        keep_better(best, at, v, i);
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
        for (int w = 1; w < kAdvanceThreads / 64; ++w)
        {
          keep_better(best, at, s_best[w], s_at[w]);
        }
        const int token = at < vocab ? at : vocab; // no value >= -FLT_MAX: one past the last
        const int step = state[kStepIndex];
        if (step < max_tokens)
        {
          tokens[step] = token;
        }
        state[kStepToken] = token;
        state[kStepPosition] = state[kStepPosition] + 1;
        state[kStepSeqK] = state[kStepPosition] + 1;
        state[kStepIndex] = step + 1;
      }
    }

    // Uniform values in [-scale, scale) from a counter hash (splitmix64), as
    // fp16: synthetic weights of a given shape, made on the device.
    __global__ void random_half_kernel(std::uint16_t *__restrict__ out, std::size_t count,
                                       unsigned long long seed, float scale)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        unsigned long long z = seed + 0x9E3779B97F4A7C15ull * (i + 1);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        const float u = static_cast<float>(z >> 40) * (1.0f / 16777216.0f); // [0, 1)
        out[i] = to_half((2.0f * u - 1.0f) * scale);
      }
    }

  } // namespace

  int project_blocks(const ProjectArgs &p)
  {
    long long rows = 0;
    for (int i = 0; i < p.segments; ++i)
    {
      rows += p.seg[i].rows;
    }
    if (p.mode == ProjectMode::kSwiglu)
    {
      rows = p.seg[0].rows; // up's rows ride with gate's
    }
    return static_cast<int>((rows + kWaves - 1) / kWaves);
  }

  void launch_project(const ProjectArgs &p, hipStream_t stream)
  {
    if (p.segments < 1 || p.segments > kProjectSegments || p.in <= 0 || p.in % 8 != 0 ||
        reinterpret_cast<std::uintptr_t>(p.x) % 16 != 0)
    {
      throw InvalidArgument("a projection takes 1 to 3 weight matrices and an input of a multiple "
                            "of 8 fp16 values, 16-byte aligned; got " +
                            std::to_string(p.segments) + " and " + std::to_string(p.in));
    }
    if (p.mode == ProjectMode::kSwiglu && (p.segments != 2 || p.seg[0].rows != p.seg[1].rows))
    {
      throw InvalidArgument("SwiGLU projects gate and up, of the same rows");
    }
    for (int i = 0; i < p.segments; ++i)
    {
      if (p.seg[i].w == nullptr || (p.mode != ProjectMode::kSwiglu || i == 0) != (p.seg[i].out != nullptr) ||
          reinterpret_cast<std::uintptr_t>(p.seg[i].w) % 16 != 0 || p.seg[i].rows <= 0)
      {
        throw InvalidArgument("projection segment " + std::to_string(i) +
                              " needs 16-byte aligned weights, rows and an output");
      }
    }
    const int blocks = project_blocks(p);
    if (p.mode == ProjectMode::kLogits && (p.best_value == nullptr || p.best_index == nullptr))
    {
      throw InvalidArgument("the head's projection keeps each block's best logit");
    }
    hipLaunchKernelGGL(project_kernel, dim3(blocks), dim3(kThreads), 0, stream, p);
    hip_check(hipGetLastError(), "projection kernel launch");
  }

  void launch_advance(const float *best_value, const int *best_index, int blocks, int vocab,
                      int *state, std::int32_t *tokens, int max_tokens, hipStream_t stream)
  {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(kAdvanceThreads), 0, stream, best_value,
                       best_index, blocks, vocab, state, tokens, max_tokens);
    hip_check(hipGetLastError(), "advance kernel launch");
  }

  void launch_random_half(void *out, std::size_t count, unsigned long long seed, float scale,
                          hipStream_t stream)
  {
    if (count == 0)
    {
      return;
    }
    const int blocks = static_cast<int>(std::min<std::size_t>((count + 255) / 256, 65536));
    hipLaunchKernelGGL(random_half_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<std::uint16_t *>(out), count, seed, scale);
    hip_check(hipGetLastError(), "random fill kernel launch");
  }

} // namespace mi
