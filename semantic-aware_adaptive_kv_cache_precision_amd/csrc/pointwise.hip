// RoPE, the RoPE cos/sin table, RMSNorm, SwiGLU and the fp16 add, for gfx950.
//
// Arithmetic follows the reference:
//   - RoPE rotate-half with the angle pos * theta^(-2j/hd) formed and reduced
//     in fp64 (rope.cu:32-54, rope_angle.cuh:15-21), per pair, or read from a
//     table of those angles' fp32 cos and sin (the same bits, without the
//     fp64 pow and sincos a pair: a 2048-token Llama chunk's q and k in
//     12.5 us against 50);
//   - RMSNorm in fp32 from fp16 or fp32 input, one fp16 rounding at the store
//     (rmsnorm.cu:33-84);
//   - SwiGLU as g / (1 + expf(-g)) * up in fp32 (swiglu.cu:26-38).
// Reductions are wave64: a wave's partial by DPP/shuffle, then one LDS step.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace mi
{
  namespace
  {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

    __device__ inline void rope_angle(double position, int j, int head_dim, double theta,
                                      double *s, double *c)
    {
      const double inv_freq = pow(theta, -2.0 * static_cast<double>(j) / head_dim);
      sincos(position * inv_freq, s, c);
    }

    // Rotates pair j of the row at `row` (channels j and j + half) by the
    // angle whose fp32 cosine and sine are cs, writing the fp16 results to
    // `out` (and to `also`, where given): each product and difference
    // rounded in fp32, then to fp16 (reference arithmetic: rope.cu:32-54).
    __device__ inline void rotate_pair(const std::uint16_t *row, int j, int half, float2 cs,
                                       std::uint16_t *out, std::uint16_t *also = nullptr)
    {
      std::uint16_t lo, hi;
      rope_pair(h2f(row[j]), h2f(row[j + half]), cs.x, cs.y, lo, hi);
      out[j] = lo;
      out[j + half] = hi;
      if (also != nullptr)
      {
        also[j] = lo;
        also[j + half] = hi;
      }
    }

    // RoPE with the angle formed per pair in fp64: a thread a rotation pair
    // of every (token, head) row, the grid striding over them.
    __global__ void rope_kernel(const std::uint16_t *__restrict__ x,
                                const std::int32_t *__restrict__ positions,
                                std::uint16_t *__restrict__ out, int heads, int head_dim,
                                double theta, std::size_t pairs)
    {
      const int half = head_dim / 2;
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < pairs; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const std::size_t row = i / half;
        const int j = static_cast<int>(i % half);
        double s, c;
        rope_angle(static_cast<double>(positions[row / heads]), j, head_dim, theta, &s, &c);
        const std::size_t base = row * head_dim;
        rotate_pair(x + base, j, half, make_float2(static_cast<float>(c), static_cast<float>(s)),
                    out + base);
      }
    }

    // RoPE of up to two row sets (a chunk's q and k) with the angles read
    // from a RopeTable ({cos, sin} in fp32 per (position, j), filled by
    // rope_table_kernel from the same double-precision angle rope_kernel
    // forms): a thread a rotation pair, the rotation rope_kernel's, so the
    // rows are its to the bit. A position past the table reads its last row
    // (the launcher's caller covers every position first).
    __global__ void rope_rows_kernel(RopeRows r)
    {
      const int half = r.head_dim / 2;
      const std::size_t first = static_cast<std::size_t>(r.seq) * r.heads[0] * half;
      const std::size_t total = first + static_cast<std::size_t>(r.seq) * r.heads[1] * half;
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < total; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const int set = i < first ? 0 : 1;
        const std::size_t k = set == 0 ? i : i - first;
        const std::size_t row = k / half; // (token, head)
        const int j = static_cast<int>(k % half);
        const int token = static_cast<int>(row / r.heads[set]);
        const int position = min(max(r.positions[token], 0), r.table_positions - 1);
        const float2 cs = *reinterpret_cast<const float2 *>(
            r.table + 2 * (static_cast<std::size_t>(position) * half + j));
        const std::size_t base = row * r.head_dim;
        rotate_pair(static_cast<const std::uint16_t *>(r.x[set]) + base, j, half, cs,
                    static_cast<std::uint16_t *>(r.out[set]) + base);
      }
    }

    __global__ void rope_table_kernel(float *__restrict__ table, int half, int head_dim,
                                      double theta, std::size_t count)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        double s, c;
        rope_angle(static_cast<double>(i / half), static_cast<int>(i % half), head_dim, theta, &s,
                   &c);
        table[2 * i] = static_cast<float>(c);
        table[2 * i + 1] = static_cast<float>(s);
      }
    }

    // The table's angles as fp16 high and low parts, a row a position:
    // channel c < half holds cos of angle c, channel c >= half sin of angle
    // c - half; high parts (head_dim halves), then low parts (the fp32 value
    // less the high part, rounded again). hi + lo carries the fp32 value to
    // within 2^-22 of it, for matrix-core products that need fp32 accuracy.
    __global__ void rope_angles_kernel(const float *__restrict__ table,
                                       std::uint16_t *__restrict__ angles, int half, int head_dim,
                                       std::size_t count)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const std::size_t t = i / head_dim;
        const int c = static_cast<int>(i % head_dim);
        const int j = c < half ? c : c - half;
        const float value = table[2 * (t * half + j) + (c < half ? 0 : 1)];
        const __half hi = __float2half_rn(value);
        const __half lo = __float2half_rn(value - __half2float(hi));
        angles[2 * t * head_dim + c] = __half_as_ushort(hi);
        angles[(2 * t + 1) * head_dim + c] = __half_as_ushort(lo);
      }
    }

    // RMSNorm: a 256-thread workgroup a row, the scale by inv_rms.
    template <typename In>
    __global__ void __launch_bounds__(256)
        rmsnorm_kernel(const In *__restrict__ x, const std::uint16_t *__restrict__ weight,
                       std::uint16_t *__restrict__ out, int hidden, float eps)
    {
      __shared__ float partial[4];
      const std::size_t row = static_cast<std::size_t>(blockIdx.x) * hidden;
      const float scale = inv_rms(x + row, hidden, eps, partial);
      normed_row(x + row, weight, out + row, hidden, scale);
    }

    // One decode row's work that precedes its attention, as one launch:
    // workgroup 0 the RMSNorm of r.x (when given); the rest a thread a
    // rotation pair of the q and k heads at *position (angles from the
    // table), the k heads' rotated pairs also written into the layer's FP16
    // page at that position, then a thread a value channel into the page's
    // value row. A position outside [0, r.positions) stores nothing.
    __global__ void __launch_bounds__(256) row_prep_kernel(RowPrep r)
    {
      int block = blockIdx.x;
      if (r.x != nullptr)
      {
        if (block == 0)
        {
          __shared__ float partial[4];
          const float scale = inv_rms(r.x, r.hidden, r.eps, partial);
          normed_row(r.x, r.norm_weight, r.normed, r.hidden, scale);
          return;
        }
        --block;
      }
      const int half = r.head_dim / 2;
      const int width = r.kv_heads * r.head_dim;
      const int pairs = (r.q_heads + r.kv_heads) * half;
      const int i = block * 256 + static_cast<int>(threadIdx.x);
      const int position = *r.position;
      const bool stored = position >= 0 && position < r.positions;
      std::uint16_t *page = nullptr;
      if (stored)
      {
        page = reinterpret_cast<std::uint16_t *>(r.pages[position / r.page_tokens]) +
               static_cast<std::size_t>(position % r.page_tokens) * width;
      }
      if (i < pairs)
      {
        const int head = i / half;
        const int j = i % half;
        const int at = min(max(position, 0), r.table_positions - 1);
        const float2 cs =
            *reinterpret_cast<const float2 *>(r.table + 2 * (static_cast<std::size_t>(at) * half + j));
        const std::size_t base = static_cast<std::size_t>(head) * r.head_dim;
        std::uint16_t *key_row =
            stored && head >= r.q_heads ? page + (head - r.q_heads) * r.head_dim : nullptr;
        rotate_pair(r.qk + base, j, half, cs, r.qk_out + base, key_row);
      }
      else if (i < pairs + width && stored)
      {
        const int c = i - pairs;
        page[static_cast<std::size_t>(r.page_tokens) * width + c] = r.values[c];
      }
    }

    // SiLU(g) * u of one fp16 pair (reference arithmetic: swiglu.cu:26-38):
    // g / (1 + e^-g) and the product in fp32, one rounding to fp16.
    __device__ inline std::uint16_t swiglu_value(std::uint16_t g, std::uint16_t u)
    {
      const float gf = h2f(g);
      const float silu = gf / (1.0f + expf(-gf));
      return __half_as_ushort(__float2half(silu * h2f(u)));
    }

    // SwiGLU over `count` values: with Wide, eight a thread through 16-byte
    // loads and stores for the first count / 8 * 8 and one a thread for the
    // rest; else one a thread throughout.
    template <bool Wide>
    __global__ void swiglu_kernel(const std::uint16_t *__restrict__ gate,
                                  const std::uint16_t *__restrict__ up,
                                  std::uint16_t *__restrict__ out, std::size_t count)
    {
      const std::size_t groups = Wide ? count / 8 : 0;
      const std::size_t items = groups + (count - 8 * groups);
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < items; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        if (i < groups)
        {
          const u32x4 g = *reinterpret_cast<const u32x4 *>(gate + 8 * i);
          const u32x4 u = *reinterpret_cast<const u32x4 *>(up + 8 * i);
          u32x4 o;
#pragma unroll
          for (int k = 0; k < 4; ++k)
          {
            o[k] = static_cast<unsigned>(swiglu_value(static_cast<std::uint16_t>(g[k]),
                                                      static_cast<std::uint16_t>(u[k]))) |
                   (static_cast<unsigned>(swiglu_value(static_cast<std::uint16_t>(g[k] >> 16),
                                                       static_cast<std::uint16_t>(u[k] >> 16)))
                    << 16);
          }
          *reinterpret_cast<u32x4 *>(out + 8 * i) = o;
        }
        else
        {
          const std::size_t e = 8 * groups + (i - groups);
          out[e] = swiglu_value(gate[e], up[e]);
        }
      }
    }

    __global__ void add_kernel(const std::uint16_t *a, const std::uint16_t *b, std::uint16_t *out,
                               std::size_t count)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        out[i] = __half_as_ushort(__float2half(h2f(a[i]) + h2f(b[i])));
      }
    }

    int grid_for(std::size_t count, int threads)
    {
      return static_cast<int>(std::max<std::size_t>(
          1, std::min<std::size_t>((count + threads - 1) / threads, 65536)));
    }

  } // namespace

  void launch_rope(const void *x, const std::int32_t *positions, void *out, int seq, int heads,
                   int head_dim, double theta, hipStream_t stream)
  {
    if (seq <= 0 || heads <= 0 || head_dim <= 0)
    {
      return;
    }
    const std::size_t pairs = static_cast<std::size_t>(seq) * heads * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0, stream,
                       static_cast<const std::uint16_t *>(x), positions,
                       static_cast<std::uint16_t *>(out), heads, head_dim, theta, pairs);
    hip_check(hipGetLastError(), "rope kernel launch");
  }

  void launch_row_prep(const RowPrep &r, hipStream_t stream)
  {
    if (r.head_dim <= 0 || r.head_dim % 2 != 0 || r.table == nullptr || r.table_positions <= 0 ||
        r.q_heads < 0 || r.kv_heads <= 0 || r.page_tokens <= 0 || r.pages == nullptr)
    {
      throw InvalidArgument("the row launch takes an even head_dim, a filled RoPE table and the "
                            "layer's pages");
    }
    const int items = (r.q_heads + r.kv_heads) * (r.head_dim / 2) + r.kv_heads * r.head_dim;
    const int blocks = (items + 255) / 256 + (r.x != nullptr ? 1 : 0);
    hipLaunchKernelGGL(row_prep_kernel, dim3(blocks), dim3(256), 0, stream, r);
    hip_check(hipGetLastError(), "row prep kernel launch");
  }

  void launch_rope_rows(const RopeRows &r, hipStream_t stream)
  {
    if (r.head_dim <= 0 || r.head_dim % 2 != 0 || r.table == nullptr || r.table_positions <= 0 ||
        r.seq < 0 || r.heads[0] < 0 || r.heads[1] < 0)
    {
      throw InvalidArgument("RoPE from a table takes an even head_dim and a filled table");
    }
    const std::size_t pairs =
        static_cast<std::size_t>(r.seq) * (r.heads[0] + r.heads[1]) * (r.head_dim / 2);
    if (pairs == 0)
    {
      return;
    }
    hipLaunchKernelGGL(rope_rows_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0, stream, r);
    hip_check(hipGetLastError(), "rope rows kernel launch");
  }

  void launch_rope_table(float *table, int positions, int head_dim, double theta,
                         hipStream_t stream)
  {
    const std::size_t entries = static_cast<std::size_t>(positions) * (head_dim / 2);
    if (entries == 0)
    {
      return;
    }
    hipLaunchKernelGGL(rope_table_kernel, dim3(grid_for(entries, 256)), dim3(256), 0, stream,
                       table, head_dim / 2, head_dim, theta, entries);
    hip_check(hipGetLastError(), "rope table kernel launch");
  }

  void launch_rope_angles(const float *table, std::uint16_t *angles, int positions, int head_dim,
                          hipStream_t stream)
  {
    const std::size_t count = static_cast<std::size_t>(positions) * head_dim;
    if (count == 0)
    {
      return;
    }
    hipLaunchKernelGGL(rope_angles_kernel, dim3(grid_for(count, 256)), dim3(256), 0, stream, table,
                       angles, head_dim / 2, head_dim, count);
    hip_check(hipGetLastError(), "rope angles kernel launch");
  }

  void launch_rmsnorm(const void *x, bool x_is_f32, const void *weight, void *out, int rows,
                      int hidden, float eps, hipStream_t stream)
  {
    if (rows <= 0 || hidden <= 0)
    {
      return;
    }
    const auto *w = static_cast<const std::uint16_t *>(weight);
    auto *o = static_cast<std::uint16_t *>(out);
    if (x_is_f32)
    {
      hipLaunchKernelGGL(rmsnorm_kernel<float>, dim3(rows), dim3(256), 0, stream,
                         static_cast<const float *>(x), w, o, hidden, eps);
    }
    else
    {
      hipLaunchKernelGGL(rmsnorm_kernel<std::uint16_t>, dim3(rows), dim3(256), 0, stream,
                         static_cast<const std::uint16_t *>(x), w, o, hidden, eps);
    }
    hip_check(hipGetLastError(), "rmsnorm kernel launch");
  }

  void launch_swiglu(const void *gate, const void *up, void *out, std::size_t count,
                     hipStream_t stream)
  {
    if (count == 0)
    {
      return;
    }
    const auto aligned = [](const void *p) {
      return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0;
    };
    const auto *g = static_cast<const std::uint16_t *>(gate);
    const auto *u = static_cast<const std::uint16_t *>(up);
    auto *o = static_cast<std::uint16_t *>(out);
    if (aligned(gate) && aligned(up) && aligned(out))
    {
      const std::size_t items = count / 8 + count % 8;
      hipLaunchKernelGGL(swiglu_kernel<true>, dim3(grid_for(items, 256)), dim3(256), 0, stream, g,
                         u, o, count);
    }
    else
    {
      hipLaunchKernelGGL(swiglu_kernel<false>, dim3(grid_for(count, 256)), dim3(256), 0, stream, g,
                         u, o, count);
    }
    hip_check(hipGetLastError(), "swiglu kernel launch");
  }

  void launch_add(const void *a, const void *b, void *out, std::size_t count, hipStream_t stream)
  {
    if (count == 0)
    {
      return;
    }
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(count, 256)), dim3(256), 0, stream,
                       static_cast<const std::uint16_t *>(a), static_cast<const std::uint16_t *>(b),
                       static_cast<std::uint16_t *>(out), count);
    hip_check(hipGetLastError(), "add kernel launch");
  }

} // namespace mi
