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
// bits -- its reads asked for before the weights', in one trip that does
// not queue behind them.
// A row a wave (a long row split over four or eight waves) when the
// device holds the whole grid at once; otherwise as many workgroups as it
// holds, each wave taking several rows with the next row's runs in flight
// while one is used (the head's vocabulary). The projections a step makes
// from one input run in one launch: q, k and v (three weight matrices, one
// grid over their rows), gate and up (a wave both rows of one output, the
// SwiGLU in the epilogue).

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cfloat>
#include <climits>
#include <map>
#include <mutex>

namespace mi
{
  namespace
  {
    constexpr int kAdvanceThreads = 1024;

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

    // RMSNorm of the fp32 residual row staged in LDS as fp16 runs, with the
    // RMSNorm kernel's bits (inv_rms's sum in its order, then x * scale * w
    // rounded once), every global read asked for in one trip: `ask` reads
    // the values inv_rms sums (thread t < 256: t + 256 k) and the runs the
    // thread forms (t + Threads m) of the residual and the norm weight; a
    // kernel asks before its weights' loads, so that these do not queue
    // behind them. `stage` sums, meets the workgroup at a barrier and writes
    // the runs (the caller's barrier publishes them). The input is at most
    // 512 Ahead values (Ahead runs a lane of a wave).
    template <int Threads, int Ahead>
    struct NormedInput
    {
      static constexpr int kSquares = 2 * Ahead;
      static constexpr int kRuns = (64 * Ahead + Threads - 1) / Threads;
      float sq[kSquares];
      f32x4 lo[kRuns], hi[kRuns];
      u32x4 w[kRuns];

      __device__ void ask(const float *residual, const std::uint16_t *weight, int in)
      {
        const int t = threadIdx.x;
#pragma unroll
        for (int k = 0; k < kSquares; ++k)
        {
          const int i = t + 256 * k;
          sq[k] = t < 256 && i < in ? residual[i] : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < kRuns; ++m)
        {
          const int r = t + Threads * m;
          if (r < in / 8)
          {
            lo[m] = *((g_f32x4)(residual + 8 * static_cast<std::size_t>(r)));
            hi[m] = *((g_f32x4)(residual + 8 * static_cast<std::size_t>(r) + 4));
            w[m] = *((g_u32x4)(weight + 8 * static_cast<std::size_t>(r)));
          }
        }
      }

      __device__ void stage(int in, float eps, float *partial, u32x4 *x_lds)
      {
        // inv_rms's sum: the zeros past the row add nothing.
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kSquares; ++k)
        {
          acc += sq[k] * sq[k];
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
        const float total = ((partial[0] + partial[1]) + partial[2]) + partial[3];
        const float scale = rsqrtf(total / static_cast<float>(in) + eps);
#pragma unroll
        for (int m = 0; m < kRuns; ++m)
        {
          const int r = threadIdx.x + Threads * m;
          if (r < in / 8)
          {
            const float v[8] = {lo[m][0], lo[m][1], lo[m][2], lo[m][3],
                                hi[m][0], hi[m][1], hi[m][2], hi[m][3]};
            u32x4 out;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
              const unsigned wi = w[m][i];
              const unsigned l = to_half(v[2 * i] * scale * h2f(static_cast<std::uint16_t>(wi)));
              const unsigned h =
                  to_half(v[2 * i + 1] * scale * h2f(static_cast<std::uint16_t>(wi >> 16)));
              out[i] = l | (h << 16);
            }
            x_lds[r] = out;
          }
        }
      }
    };

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

    // The runs of a wave's part of one or two weight rows: run
    // begin + lane + 64 i for i < Ahead, clamped into the part (a lane past
    // its part re-reads the part's first run, which it does not use).
    template <int Ahead, bool Two>
    __device__ inline void load_part(u32x4 (&a)[Ahead], u32x4 (&b)[Ahead],
                                     const std::uint16_t *w0, const std::uint16_t *w1, int begin,
                                     int end, int lane)
    {
      if (begin >= end)
      {
        return; // an empty part reads nothing (not even its row's next run)
      }
#pragma unroll
      for (int i = 0; i < Ahead; ++i)
      {
        const int r = begin + lane + 64 * i;
        const std::size_t at = 8 * static_cast<std::size_t>(r < end ? r : begin);
        a[i] = *((g_u32x4)(w0 + at));
        if constexpr (Two)
        {
          b[i] = *((g_u32x4)(w1 + at));
        }
      }
    }

    // Which segment a row (counted over the segments in turn) falls in.
    __device__ inline int locate(const ProjectArgs &p, bool two, int row, int &seg)
    {
      seg = 0;
      while (!two && seg + 1 < p.segments && row >= p.seg[seg].rows)
      {
        row -= p.seg[seg].rows;
        ++seg;
      }
      return row;
    }

    // A weight row (gate's and up's rows together with Two) is read by
    // Split consecutive waves of a workgroup (of Waves waves), each a
    // contiguous part of its 16-byte runs, every run of the part in flight
    // at once (Ahead a lane);
    // the parts' dots meet in LDS and are summed in part order. A
    // workgroup holds Waves / Split rows at a time; with Pipe a wave's next
    // row is loaded while the current one is used (the head: many rows a
    // wave). The input -- x, or RMSNorm of the residual -- is staged once a
    // workgroup in LDS, its reads asked for before the wave's first loads.
    template <int Waves, int Ahead, bool Two, int Split, bool Pipe>
    __global__ void __launch_bounds__(64 * Waves) project_kernel(ProjectArgs p)
    {
      constexpr int kSlots = Waves / Split;
      constexpr int kBlockThreads = 64 * Waves;
      extern __shared__ u32x4 x_lds[];
      __shared__ float s_best[Waves];
      __shared__ int s_at[Waves];
      __shared__ float s_partial[4];
      __shared__ float s_dot[Waves];
      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int slot = wave / Split;
      const int part = wave % Split;
      const int runs = p.in / 8;
      const int part_runs = (runs + Split - 1) / Split;
      const int begin = min(runs, part * part_runs);
      const int end = min(runs, begin + part_runs);
      int total = 0;
      for (int i = 0; i < (Two ? 1 : p.segments); ++i)
      {
        total += p.seg[i].rows;
      }
      const int stride = gridDim.x * kSlots;
      const auto row_weights = [&](int g, int &seg, int &row) {
        row = locate(p, Two, g, seg);
        return p.seg[seg].w + static_cast<std::size_t>(row) * p.in;
      };
      const auto up_weights = [&](int row) {
        return Two ? p.seg[1].w + static_cast<std::size_t>(row) * p.in : nullptr;
      };
      // The input is asked for first, then the wave's first row's runs (and
      // with Pipe its second's): the input's one trip does not queue behind
      // the weights'. A row split over waves reads x (no RMSNorm) straight
      // from global memory, a lane its own runs: staging a long input once a
      // workgroup would read it more times than the weights' bytes.
      // Otherwise x, or RMSNorm of the residual, is staged in LDS.
      constexpr bool kDirect = Split > 1;
      constexpr int kStagedRuns = (64 * Ahead + kBlockThreads - 1) / kBlockThreads;
      const bool normed = !kDirect && p.norm_weight != nullptr;
      u32x4 xd[kDirect ? Ahead : 1];
      u32x4 xs[kDirect ? 1 : kStagedRuns];
      NormedInput<kBlockThreads, kDirect ? 1 : Ahead> norm;
      if constexpr (kDirect)
      {
#pragma unroll
        for (int i = 0; i < Ahead; ++i)
        {
          const int r = begin + lane + 64 * i;
          xd[i] = r < end ? *((g_u32x4)(p.x + 8 * static_cast<std::size_t>(r)))
                          : u32x4{0u, 0u, 0u, 0u};
        }
      }
      else if (normed)
      {
        norm.ask(p.residual, p.norm_weight, p.in);
      }
      else
      {
#pragma unroll
        for (int m = 0; m < kStagedRuns; ++m)
        {
          const int r = threadIdx.x + kBlockThreads * m;
          if (r < runs)
          {
            xs[m] = *((g_u32x4)(p.x + 8 * static_cast<std::size_t>(r)));
          }
        }
      }
      int g = blockIdx.x * kSlots + slot;
      u32x4 a[Ahead], b[Ahead];
      u32x4 na[Pipe ? Ahead : 1], nb[Pipe ? Ahead : 1];
      if (g < total)
      {
        int seg, row;
        const std::uint16_t *w0 = row_weights(g, seg, row);
        load_part<Ahead, Two>(a, b, w0, up_weights(row), begin, end, lane);
      }
      if constexpr (Pipe)
      {
        if (g + stride < total)
        {
          int nseg, nrow;
          const std::uint16_t *w0 = row_weights(g + stride, nseg, nrow);
          load_part<Ahead, Two>(na, nb, w0, up_weights(nrow), begin, end, lane);
        }
      }
      if constexpr (!kDirect)
      {
        if (normed)
        {
          norm.stage(p.in, p.eps, s_partial, x_lds);
        }
        else
        {
#pragma unroll
          for (int m = 0; m < kStagedRuns; ++m)
          {
            const int r = threadIdx.x + kBlockThreads * m;
            if (r < runs)
            {
              x_lds[r] = xs[m];
            }
          }
        }
        __syncthreads();
      }
      float best = -FLT_MAX;
      int at = INT_MAX;
      // One turn: the row g the registers (wa, wb) hold, its dot (the parts
      // of a split row meet at a barrier), its output; then wa and wb take
      // the row `ahead` turns on (the next, or with Pipe the one after: the
      // other buffer holds the next, in flight meanwhile).
      const auto turn = [&](u32x4 (&wa)[Ahead], u32x4 (&wb)[Ahead], int ahead) {
        const bool live = g < total;
        int seg = 0, row = 0;
        if (live)
        {
          row = locate(p, Two, g, seg);
        }
        float acc0 = 0.0f, acc1 = 0.0f;
        if (live)
        {
#pragma unroll
          for (int i = 0; i < Ahead; ++i)
          {
            const int r = begin + lane + 64 * i;
            if (r < end)
            {
              u32x4 xv;
              if constexpr (kDirect)
              {
                xv = xd[i];
              }
              else
              {
                xv = x_lds[r];
              }
              acc0 = dot_run(wa[i], xv, acc0);
              if constexpr (Two)
              {
                acc1 = dot_run(wb[i], xv, acc1);
              }
            }
          }
        }
        float dot = wave_total(acc0);
        const float up = Two ? wave_total(acc1) : 0.0f;
        if constexpr (Split > 1)
        {
          if (lane == 0)
          {
            s_dot[wave] = dot;
          }
          __syncthreads();
          dot = 0.0f;
#pragma unroll
          for (int q = 0; q < Split; ++q)
          {
            dot += s_dot[slot * Split + q];
          }
          __syncthreads();
        }
        if (g + ahead * stride < total)
        {
          int nseg, nrow;
          const std::uint16_t *w0 = row_weights(g + ahead * stride, nseg, nrow);
          load_part<Ahead, Two>(wa, wb, w0, up_weights(nrow), begin, end, lane);
        }
        if (!live || part != 0)
        {
          return;
        }
        if (lane != 0)
        {
          keep_better(best, at, dot, row);
          return;
        }
        const ProjectSegment &sg = p.seg[seg];
        switch (p.mode)
        {
        case ProjectMode::kHalf:
        {
          const float bias = sg.bias != nullptr ? h2f(sg.bias[row]) : 0.0f;
          static_cast<std::uint16_t *>(sg.out)[row] = to_half(dot + bias);
          break;
        }
        case ProjectMode::kAccumulate:
        {
          float *out = static_cast<float *>(sg.out) + row;
          *out = *out + dot;
          break;
        }
        case ProjectMode::kSwiglu:
        {
          const float gv = h2f(to_half(dot));
          const float uv = h2f(to_half(up));
          const float silu = gv / (1.0f + expf(-gv));
          static_cast<std::uint16_t *>(sg.out)[row] = to_half(silu * uv);
          break;
        }
        case ProjectMode::kLogits:
          static_cast<float *>(sg.out)[row] = dot;
          break;
        }
        keep_better(best, at, dot, row);
      };
      // Every wave of the workgroup takes the same number of turns (the
      // parts of a row meet at a barrier); a slot past the rows idles. With
      // Pipe the two buffers alternate, so that a turn waits only for its
      // own row.
      for (int base = blockIdx.x * kSlots; base < total; base += stride, g += stride)
      {
        if constexpr (Pipe)
        {
          turn(a, b, 2);
          base += stride;
          g += stride;
          if (base >= total)
          {
            break;
          }
          turn(na, nb, 2);
        }
        else
        {
          turn(a, b, 1);
        }
      }
      if (p.mode == ProjectMode::kLogits)
      {
        // The workgroup's best logit, for the advance to choose from (parts
        // other than the first hold no candidate).
        if (lane == 0)
        {
          s_best[wave] = best;
          s_at[wave] = at;
        }
        __syncthreads();
        if (threadIdx.x == 0)
        {
          for (int w2 = 0; w2 < Waves; ++w2)
          {
            keep_better(best, at, s_best[w2], s_at[w2]);
          }
          p.best_value[blockIdx.x] = best;
          p.best_index[blockIdx.x] = at;
        }
      }
    }

    // A decode step's q, k and v of a layer (QkvStep): an item a wave, the
    // rotation pair j of unit u (q's heads, then k's, then v's), its two
    // weight rows' dots with the normed input staged in LDS (the
    // projection's runs and order, so the same bits), then the bias, the
    // rounding, RoPE for q and k, and the open page's row for k and v.
    template <int Waves, int Ahead>
    __global__ void __launch_bounds__(64 * Waves) qkv_step_kernel(QkvStep p)
    {
      constexpr int kBlockThreads = 64 * Waves;
      constexpr int kPage = 32;
      extern __shared__ u32x4 x_lds[];
      __shared__ float s_partial[4];
      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int half = p.head_dim / 2;
      const int total = (p.heads + 2 * p.kv_heads) * half;
      const int runs = p.in / 8;
      const int stride = gridDim.x * Waves;
      const auto item_rows = [&](int item, int &seg, int &head, int &j) {
        const int u = item / half;
        j = item % half;
        seg = u < p.heads ? 0 : u < p.heads + p.kv_heads ? 1 : 2;
        head = seg == 0 ? u : seg == 1 ? u - p.heads : u - p.heads - p.kv_heads;
      };
      u32x4 a[Ahead], b[Ahead];
      const auto load = [&](int item) {
        int seg, head, j;
        item_rows(item, seg, head, j);
        const std::size_t r0 = static_cast<std::size_t>(head) * p.head_dim + j;
        load_part<Ahead, true>(a, b, p.w[seg] + r0 * p.in, p.w[seg] + (r0 + half) * p.in, 0,
                               runs, lane);
      };
      // The input's RMSNorm reads first, then the first item's weights.
      NormedInput<kBlockThreads, Ahead> norm;
      norm.ask(p.residual, p.norm_weight, p.in);
      int item = blockIdx.x * Waves + wave;
      if (item < total)
      {
        load(item);
      }
      // The position, and the first item's bias and angle, asked for with
      // its weights, before the input's norm is staged: none waits behind
      // the dots.
      const int position = *p.position;
      const int first_item = item;
      const auto epilogue_inputs = [&](int it, float &b0, float &b1, float &c, float &sn) {
        int seg, head, j;
        item_rows(it, seg, head, j);
        const std::size_t r0 = static_cast<std::size_t>(head) * p.head_dim + j;
        const std::uint16_t *bias = p.b[seg];
        b0 = bias != nullptr ? h2f(bias[r0]) : 0.0f;
        b1 = bias != nullptr ? h2f(bias[r0 + half]) : 0.0f;
        c = 1.0f;
        sn = 0.0f;
        if (seg != 2)
        {
          const float *cs = p.rope + (static_cast<std::size_t>(position) * half + j) * 2;
          c = cs[0];
          sn = cs[1];
        }
      };
      float first_b0 = 0.0f, first_b1 = 0.0f, first_c = 1.0f, first_sn = 0.0f;
      if (item < total && lane == 0)
      {
        epilogue_inputs(item, first_b0, first_b1, first_c, first_sn);
      }
      norm.stage(p.in, p.eps, s_partial, x_lds);
      __syncthreads();
      const int row = position % kPage;
      const std::size_t W = static_cast<std::size_t>(p.kv_heads) * p.head_dim;
      for (; item < total; item += stride)
      {
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int i = 0; i < Ahead; ++i)
        {
          const int r = lane + 64 * i;
          if (r < runs)
          {
            const u32x4 xv = x_lds[r];
            acc0 = dot_run(a[i], xv, acc0);
            acc1 = dot_run(b[i], xv, acc1);
          }
        }
        const float d0 = wave_total(acc0);
        const float d1 = wave_total(acc1);
        if (item + stride < total)
        {
          load(item + stride);
        }
        if (lane != 0)
        {
          continue;
        }
        int seg, head, j;
        item_rows(item, seg, head, j);
        const std::size_t r0 = static_cast<std::size_t>(head) * p.head_dim + j;
        const std::size_t r1 = r0 + half;
        float b0 = first_b0, b1 = first_b1, c = first_c, sn = first_sn;
        if (item != first_item)
        {
          epilogue_inputs(item, b0, b1, c, sn);
        }
        const unsigned h0 = to_half(d0 + b0);
        const unsigned h1 = to_half(d1 + b1);
        if (seg == 2)
        {
          p.v[r0] = static_cast<std::uint16_t>(h0);
          p.v[r1] = static_cast<std::uint16_t>(h1);
          if (row < kPage - 1)
          {
            std::uint16_t *at = p.open + (kPage + row) * W;
            at[r0] = static_cast<std::uint16_t>(h0);
            at[r1] = static_cast<std::uint16_t>(h1);
          }
          continue;
        }
        // RoPE of the rounded pair, as the RoPE kernel rotates it.
        std::uint16_t o1, o2;
        rope_pair(h2f(static_cast<std::uint16_t>(h0)), h2f(static_cast<std::uint16_t>(h1)), c, sn,
                  o1, o2);
        const std::size_t at = static_cast<std::size_t>(seg == 0 ? head : p.heads + head) *
                                   p.head_dim + j;
        p.qk[at] = o1;
        p.qk[at + half] = o2;
        if (seg == 1 && row < kPage - 1)
        {
          std::uint16_t *keys = p.open + row * W;
          keys[r0] = o1;
          keys[r1] = o2;
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

  namespace
  {
    // The waves a row is split over: one, unless a part of more than 512
    // runs (8 a lane) would be left, as a long input (the down projection)
    // gives; then 4 or 8, which also puts more waves on the bytes.
    int project_split(int in)
    {
      const int runs = in / 8;
      return runs <= 512 ? 1 : runs <= 4 * 512 ? 4 : 8;
    }

    using ProjectFn = void (*)(ProjectArgs);

    template <int Waves, int Ahead>
    ProjectFn project_variant(bool two, int split, bool pipe)
    {
      if (two)
      {
        return pipe ? project_kernel<Waves, Ahead, true, 1, true>
                    : project_kernel<Waves, Ahead, true, 1, false>;
      }
      if (split == 1)
      {
        return pipe ? project_kernel<Waves, Ahead, false, 1, true>
                    : project_kernel<Waves, Ahead, false, 1, false>;
      }
      return split == 4 ? project_kernel<Waves, Ahead, false, 4, false>
                        : project_kernel<Waves, Ahead, false, 8, false>;
    }

    template <int Ahead>
    ProjectFn project_variant(int waves, bool two, int split, bool pipe)
    {
      return waves == 8 ? project_variant<8, Ahead>(two, split, pipe)
                        : project_variant<4, Ahead>(two, split, pipe);
    }

    ProjectFn project_variant(int ahead, int waves, bool two, int split, bool pipe)
    {
      switch (ahead)
      {
      case 1: return project_variant<1>(waves, two, split, pipe);
      case 2: return project_variant<2>(waves, two, split, pipe);
      case 3: return project_variant<3>(waves, two, split, pipe);
      case 4: return project_variant<4>(waves, two, split, pipe);
      case 5: return project_variant<5>(waves, two, split, pipe);
      case 6: return project_variant<6>(waves, two, split, pipe);
      case 7: return project_variant<7>(waves, two, split, pipe);
      default: return project_variant<8>(waves, two, split, pipe);
      }
    }

    // Workgroups of a kernel the device holds at once, queried once a
    // (kernel, LDS) pair.
    int resident_blocks(ProjectFn fn, int threads, std::size_t lds)
    {
      static std::mutex lock;
      static std::map<std::pair<const void *, std::size_t>, int> known;
      const std::pair<const void *, std::size_t> key{reinterpret_cast<const void *>(fn), lds};
      {
        std::lock_guard<std::mutex> hold(lock);
        const auto it = known.find(key);
        if (it != known.end())
        {
          return it->second;
        }
      }
      int per_cu = 0;
      hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, key.first, threads, lds),
                "hipOccupancyMaxActiveBlocksPerMultiprocessor projection");
      const int blocks = std::max(per_cu, 1) * device_multiprocessors();
      std::lock_guard<std::mutex> hold(lock);
      known[key] = blocks;
      return blocks;
    }

    struct ProjectPlan
    {
      ProjectFn fn;
      int waves;
      int blocks;
      std::size_t lds;
      int split;
      bool pipelined;
    };

    // A wave a row (Split waves with a long input) in one grid when the
    // device holds that many workgroups at once -- for gate/up when it
    // holds four fifths of them, the rest a short second round (faster
    // than the resident grid, whose waves hold two rows' registers and so
    // fit fewer a SIMD); otherwise as many workgroups as it holds,
    // each wave over several rows with the next row's runs in flight while
    // one is used.
    ProjectPlan plan_projection(const ProjectArgs &p)
    {
      const bool two = p.mode == ProjectMode::kSwiglu;
      long long rows = 0;
      for (int i = 0; i < (two ? 1 : p.segments); ++i)
      {
        rows += p.seg[i].rows;
      }
      const int split = two ? 1 : project_split(p.in);
      const int waves = split == 8 ? 8 : 4;
      const int slots = waves / split;
      const int runs = p.in / 8;
      const int ahead = ((runs + split - 1) / split + 63) / 64;
      if (ahead > (two ? 4 : 8))
      {
        throw InvalidArgument("a SwiGLU projection's input is at most 2048 values; got " +
                              std::to_string(p.in));
      }
      if (split > 1 && p.norm_weight != nullptr)
      {
        throw InvalidArgument("an input of more than 4096 values is projected as it comes, "
                              "without an RMSNorm formed in the launch");
      }
      // A split row reads x as it comes; otherwise x (or its RMSNorm) is
      // staged in LDS, in fp16 values.
      const std::size_t lds = split > 1 ? 0 : static_cast<std::size_t>(p.in) * 2;
      const long long needed = (rows + slots - 1) / slots;
      ProjectFn plain = project_variant(ahead, waves, two, split, false);
      const long long held_plain = resident_blocks(plain, 64 * waves, lds);
      if (split > 1 || needed <= held_plain || (two && 4 * needed <= 5 * held_plain))
      {
        return {plain, waves, static_cast<int>(needed), lds, split, false};
      }
      ProjectFn pipe = project_variant(ahead, waves, two, split, true);
      const int held = resident_blocks(pipe, 64 * waves, lds);
      return {pipe, waves, static_cast<int>(std::min<long long>(needed, held)), lds, split, true};
    }
  } // namespace

  int project_blocks(const ProjectArgs &p)
  {
    if (p.in <= 0 || p.in % 8 != 0 || p.segments < 1 || p.segments > kProjectSegments)
    {
      throw InvalidArgument("a projection's plan needs its input length (a positive multiple "
                            "of 8) and 1 to 3 segments; got " + std::to_string(p.in) + " and " +
                            std::to_string(p.segments));
    }
    return plan_projection(p).blocks;
  }

  ProjectPlanInfo launch_project(const ProjectArgs &p, hipStream_t stream)
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
    if (p.mode == ProjectMode::kLogits && (p.best_value == nullptr || p.best_index == nullptr))
    {
      throw InvalidArgument("the head's projection keeps each block's best logit");
    }
    // The input in LDS: in fp16 values.
    if (static_cast<std::size_t>(p.in) * 2 > 64 * 1024)
    {
      throw InvalidArgument("a projection's input is at most 32768 values; got " +
                            std::to_string(p.in));
    }
    const ProjectPlan plan = plan_projection(p);
    // Each workgroup of the head writes its best logit: the arrays must hold
    // one an entry a workgroup.
    if (p.mode == ProjectMode::kLogits && plan.blocks > p.best_count)
    {
      throw InvalidArgument("the head's projection runs " + std::to_string(plan.blocks) +
                            " workgroups; its best arrays hold " + std::to_string(p.best_count));
    }
    ProjectArgs args = p;
    void *params[] = {&args};
    hip_check(hipLaunchKernel(reinterpret_cast<const void *>(plan.fn), dim3(plan.blocks),
                              dim3(64 * plan.waves), params, plan.lds, stream),
              "projection kernel launch");
    return {plan.split, plan.pipelined ? 1 : 0, plan.waves, plan.blocks};
  }

  void launch_qkv_step(const QkvStep &s, hipStream_t stream)
  {
    const int runs = s.in / 8;
    const int ahead = (runs + 63) / 64;
    const bool aligned = reinterpret_cast<std::uintptr_t>(s.residual) % 16 == 0 &&
                         reinterpret_cast<std::uintptr_t>(s.norm_weight) % 16 == 0;
    if ((s.head_dim != 64 && s.head_dim != 128) || s.in <= 0 || s.in % 8 != 0 || ahead > 4 ||
        !aligned || s.heads <= 0 || s.kv_heads <= 0 || s.rope == nullptr ||
        s.position == nullptr || s.open == nullptr)
    {
      throw InvalidArgument("a step's q/k/v projection takes head_dim 64 or 128, an input of a "
                            "multiple of 8 up to 2048 values, 16-byte aligned, a RoPE table, the "
                            "device position and the open page; got head_dim " +
                            std::to_string(s.head_dim) + ", input " + std::to_string(s.in));
    }
    for (int i = 0; i < 3; ++i)
    {
      if (s.w[i] == nullptr || reinterpret_cast<std::uintptr_t>(s.w[i]) % 16 != 0)
      {
        throw InvalidArgument("a step's q/k/v projection needs 16-byte aligned weights");
      }
    }
    constexpr int kStepWaves = 4;
    const int items = (s.heads + 2 * s.kv_heads) * (s.head_dim / 2);
    const int blocks = (items + kStepWaves - 1) / kStepWaves;
    const std::size_t lds = static_cast<std::size_t>(s.in) * 2;
    const auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(blocks), dim3(64 * kStepWaves), lds, stream, s);
    };
    switch (ahead)
    {
    case 1: go(qkv_step_kernel<kStepWaves, 1>); break;
    case 2: go(qkv_step_kernel<kStepWaves, 2>); break;
    case 3: go(qkv_step_kernel<kStepWaves, 3>); break;
    default: go(qkv_step_kernel<kStepWaves, 4>); break;
    }
    hip_check(hipGetLastError(), "step q/k/v kernel launch");
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
