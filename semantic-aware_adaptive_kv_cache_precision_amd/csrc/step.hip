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
// streamed from HBM, not by arithmetic. A wave owns a weight row at a time:
// the row's 16-byte runs go to the lanes in turn (one coalesced 1 KiB load a
// wave-instruction), a batch of runs in flight while the one before it is
// used, the products v_dot2 of fp16 pairs into fp32 (each product exact),
// and a wave reduction leaves the row's dot in every lane. The input row is
// staged once a workgroup in LDS -- or, where an RMSNorm feeds the
// projection, formed there from the fp32 residual to the RMSNorm kernel's
// bits -- after each wave's first weight loads are already on their way.
// Eight rows a workgroup at a time; past 2048 workgroups (the head's
// vocabulary) each wave takes several rows. The projections a step makes
// from one input run in one launch: q, k and v (three weight matrices, one
// grid over their rows), gate and up (a wave both rows of one output, the
// SwiGLU in the epilogue).

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cfloat>
#include <climits>

namespace mi
{
  namespace
  {
    constexpr int kWaves = 8;
    constexpr int kThreads = 64 * kWaves;
    constexpr int kAdvanceThreads = 1024;
    constexpr long long kMaxBlocks = 2048;

    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(1))) u32x4 *g_u32x4;

    __device__ inline std::uint16_t to_half(float v) { return __half_as_ushort(__float2half(v)); }

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

    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(1))) f32x4 *g_f32x4;

    // RMSNorm's scale of the residual row, summed as the RMSNorm kernel sums
    // it (256 lanes, each over its stride, a wave reduction, the four waves
    // in order), so that the normed row is that kernel's to the bit.
    __device__ inline float norm_scale(const float *x, int hidden, float eps, float *partial)
    {
      float acc = 0.0f;
      if (threadIdx.x < 256)
      {
        for (int i = threadIdx.x; i < hidden; i += 256)
        {
          const float v = x[i];
          acc += v * v;
        }
      }
      for (int offset = 32; offset > 0; offset >>= 1)
      {
        acc += __shfl_xor(acc, offset);
      }
      if (threadIdx.x < 256 && threadIdx.x % 64 == 0)
      {
        partial[threadIdx.x / 64] = acc;
      }
      __syncthreads();
      float total = 0.0f;
      for (int w = 0; w < 4; ++w)
      {
        total += partial[w];
      }
      return rsqrtf(total / static_cast<float>(hidden) + eps);
    }

    // Run r (eight values) of RMSNorm of the residual: x * scale * w, one
    // rounding to fp16, as the RMSNorm kernel stores it.
    __device__ inline u32x4 normed_run(const float *residual, const std::uint16_t *weight,
                                       float scale, int r)
    {
      const f32x4 a = *((g_f32x4)(residual + 8 * static_cast<std::size_t>(r)));
      const f32x4 b = *((g_f32x4)(residual + 8 * static_cast<std::size_t>(r) + 4));
      const u32x4 wv = *((g_u32x4)(weight + 8 * static_cast<std::size_t>(r)));
      const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      u32x4 out;
#pragma unroll
      for (int i = 0; i < 4; ++i)
      {
        const unsigned wi = wv[i];
        const unsigned lo = to_half(v[2 * i] * scale * h2f(static_cast<std::uint16_t>(wi)));
        const unsigned hi = to_half(v[2 * i + 1] * scale * h2f(static_cast<std::uint16_t>(wi >> 16)));
        out[i] = lo | (hi << 16);
      }
      return out;
    }

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

    // A wave's Ahead runs of one or two weight rows (run lane + 64 i of the
    // batch at r0), clamped into the row; a lane past the row re-reads a run
    // it does not use.
    template <int Ahead, bool Two>
    __device__ inline void load_batch(u32x4 (&a)[Ahead], u32x4 (&b)[Ahead],
                                      const std::uint16_t *w0, const std::uint16_t *w1, int r0,
                                      int runs)
    {
#pragma unroll
      for (int i = 0; i < Ahead; ++i)
      {
        const int r = r0 + 64 * i;
        const std::size_t at = 8 * static_cast<std::size_t>(r < runs ? r : 0);
        a[i] = *((g_u32x4)(w0 + at));
        if constexpr (Two)
        {
          b[i] = *((g_u32x4)(w1 + at));
        }
      }
    }

    // The dots of one weight row (two, gate and up, with Two) with the input
    // staged in LDS; the row's first batch was loaded before the input was.
    // Each batch's successor is in flight while it is used.
    template <int Ahead, bool Two>
    __device__ inline void row_dots(float &d0, float &d1, const std::uint16_t *w0,
                                    const std::uint16_t *w1, const u32x4 *x, int runs, int lane,
                                    u32x4 (&a)[Ahead], u32x4 (&b)[Ahead])
    {
      float acc0 = 0.0f, acc1 = 0.0f;
      for (int r0 = lane; r0 < runs; r0 += 64 * Ahead)
      {
        u32x4 na[Ahead], nb[Ahead];
        const int next = r0 + 64 * Ahead;
        if (next < runs)
        {
          load_batch<Ahead, Two>(na, nb, w0, w1, next, runs);
        }
#pragma unroll
        for (int i = 0; i < Ahead; ++i)
        {
          const int r = r0 + 64 * i;
          if (r < runs)
          {
            const u32x4 xv = x[r];
            acc0 = dot_run(a[i], xv, acc0);
            if constexpr (Two)
            {
              acc1 = dot_run(b[i], xv, acc1);
            }
          }
        }
        if (next < runs)
        {
#pragma unroll
          for (int i = 0; i < Ahead; ++i)
          {
            a[i] = na[i];
            if constexpr (Two)
            {
              b[i] = nb[i];
            }
          }
        }
      }
      d0 = wave_total(acc0);
      d1 = Two ? wave_total(acc1) : 0.0f;
    }

    // A wave a row at a time over its rows (row = block's wave + k * the
    // grid's waves), every segment's rows in turn, or gate's and up's rows
    // together for SwiGLU. The input -- x, or RMSNorm of the residual -- is
    // staged once a workgroup in LDS, after each wave's first weight loads
    // are on their way.
    template <int Ahead, bool Two>
    __global__ void __launch_bounds__(kThreads) project_kernel(ProjectArgs p)
    {
      extern __shared__ u32x4 x_lds[];
      __shared__ float s_best[kWaves];
      __shared__ int s_at[kWaves];
      __shared__ float s_partial[4];
      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int runs = p.in / 8;
      int total = 0;
      for (int i = 0; i < (Two ? 1 : p.segments); ++i)
      {
        total += p.seg[i].rows;
      }
      const int stride = gridDim.x * kWaves;
      // The wave's first row and its first batch, before the input.
      const auto locate = [&](int row, int &seg) {
        seg = 0;
        while (!Two && seg + 1 < p.segments && row >= p.seg[seg].rows)
        {
          row -= p.seg[seg].rows;
          ++seg;
        }
        return row;
      };
      int g = blockIdx.x * kWaves + wave;
      u32x4 a[Ahead], b[Ahead];
      if (g < total)
      {
        int seg;
        const int row = locate(g, seg);
        load_batch<Ahead, Two>(a, b, p.seg[seg].w + static_cast<std::size_t>(row) * p.in,
                               Two ? p.seg[1].w + static_cast<std::size_t>(row) * p.in : nullptr,
                               lane, runs);
      }
      if (p.norm_weight != nullptr)
      {
        const float scale = norm_scale(p.residual, p.in, p.eps, s_partial);
        for (int r = threadIdx.x; r < runs; r += kThreads)
        {
          x_lds[r] = normed_run(p.residual, p.norm_weight, scale, r);
        }
      }
      else
      {
        for (int r = threadIdx.x; r < runs; r += kThreads)
        {
          x_lds[r] = *((g_u32x4)(p.x + 8 * static_cast<std::size_t>(r)));
        }
      }
      __syncthreads();
      float best = -FLT_MAX;
      int at = INT_MAX;
      for (bool first = true; g < total; g += stride, first = false)
      {
        int seg;
        const int row = locate(g, seg);
        const ProjectSegment &s = p.seg[seg];
        const std::uint16_t *w0 = s.w + static_cast<std::size_t>(row) * p.in;
        const std::uint16_t *w1 = Two ? p.seg[1].w + static_cast<std::size_t>(row) * p.in : nullptr;
        if (!first)
        {
          load_batch<Ahead, Two>(a, b, w0, w1, lane, runs);
        }
        float acc, up;
        row_dots<Ahead, Two>(acc, up, w0, w1, x_lds, runs, lane, a, b);
        if (lane != 0)
        {
          keep_better(best, at, acc, row);
          continue;
        }
        switch (p.mode)
        {
        case ProjectMode::kHalf:
        {
          const float bias = s.bias != nullptr ? h2f(s.bias[row]) : 0.0f;
          static_cast<std::uint16_t *>(s.out)[row] = to_half(acc + bias);
          break;
        }
        case ProjectMode::kAccumulate:
        {
          float *out = static_cast<float *>(s.out) + row;
          *out = *out + acc;
          break;
        }
        case ProjectMode::kSwiglu:
        {
          const float gv = h2f(to_half(acc));
          const float uv = h2f(to_half(up));
          const float silu = gv / (1.0f + expf(-gv));
          static_cast<std::uint16_t *>(s.out)[row] = to_half(silu * uv);
          break;
        }
        case ProjectMode::kLogits:
          static_cast<float *>(s.out)[row] = acc;
          break;
        }
        keep_better(best, at, acc, row);
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
    // A wave a row, up to kMaxBlocks workgroups; past that the waves take
    // several rows each (the head's vocabulary), so that the staging of the
    // input is paid once for many rows.
    return static_cast<int>(std::min<long long>((rows + kWaves - 1) / kWaves, kMaxBlocks));
  }

  void launch_project(const ProjectArgs &p, hipStream_t stream)
  {
    const bool normed = p.norm_weight != nullptr;
    if (p.segments < 1 || p.segments > kProjectSegments || p.in <= 0 || p.in % 8 != 0 ||
        reinterpret_cast<std::uintptr_t>(normed ? static_cast<const void *>(p.residual)
                                                : static_cast<const void *>(p.x)) % 16 != 0 ||
        (normed && reinterpret_cast<std::uintptr_t>(p.norm_weight) % 16 != 0))
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
    // The input in LDS: in fp16 values. Long rows (the down projection's)
    // keep more of a row in flight.
    const std::size_t lds = static_cast<std::size_t>(p.in) * 2;
    if (lds > 64 * 1024)
    {
      throw InvalidArgument("a projection's input is at most 32768 values; got " +
                            std::to_string(p.in));
    }
    const bool two = p.mode == ProjectMode::kSwiglu;
    if (p.in > 4096)
    {
      if (two)
      {
        hipLaunchKernelGGL((project_kernel<8, true>), dim3(blocks), dim3(kThreads), lds, stream, p);
      }
      else
      {
        hipLaunchKernelGGL((project_kernel<8, false>), dim3(blocks), dim3(kThreads), lds, stream, p);
      }
    }
    else if (two)
    {
      hipLaunchKernelGGL((project_kernel<4, true>), dim3(blocks), dim3(kThreads), lds, stream, p);
    }
    else
    {
      hipLaunchKernelGGL((project_kernel<4, false>), dim3(blocks), dim3(kThreads), lds, stream, p);
    }
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
