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

    __device__ inline void rope_angle(double position, int j, int head_dim, double theta,
                                      double *s, double *c)
    {
      const double inv_freq = pow(theta, -2.0 * static_cast<double>(j) / head_dim);
      sincos(position * inv_freq, s, c);
    }

    // One workgroup per (token, head); a lane per rotation pair.
    __global__ void rope_kernel(const std::uint16_t *__restrict__ x,
                                const std::int32_t *__restrict__ positions,
                                std::uint16_t *__restrict__ out, int heads, int head_dim,
                                double theta)
    {
      const int token = blockIdx.x / heads;
      const std::size_t base = static_cast<std::size_t>(blockIdx.x) * head_dim;
      const int half = head_dim / 2;
      const double pos = static_cast<double>(positions[token]);
      for (int j = threadIdx.x; j < half; j += blockDim.x)
      {
        double s, c;
        rope_angle(pos, j, head_dim, theta, &s, &c);
        const float sf = static_cast<float>(s);
        const float cf = static_cast<float>(c);
        const float x1 = h2f(x[base + j]);
        const float x2 = h2f(x[base + j + half]);
        out[base + j] = __half_as_ushort(__float2half(x1 * cf - x2 * sf));
        out[base + j + half] = __half_as_ushort(__float2half(x2 * cf + x1 * sf));
      }
    }

    // RoPE of up to two row sets (a chunk's q and k) with the angles read
    // from a RopeTable ({cos, sin} in fp32 per (position, j), filled by
    // rope_table_kernel from the same double-precision angle rope_kernel
    // forms): a thread a rotation pair, the rotation the RoPE kernel's fp32
    // arithmetic, so the rows are rope_kernel's to the bit. A position past
    // the table reads its last row (the launcher's caller covers every
    // position first).
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
        const auto *x = static_cast<const std::uint16_t *>(r.x[set]);
        auto *out = static_cast<std::uint16_t *>(r.out[set]);
        const float x1 = h2f(x[base + j]);
        const float x2 = h2f(x[base + j + half]);
        out[base + j] = __half_as_ushort(__float2half(x1 * cs.x - x2 * cs.y));
        out[base + j + half] = __half_as_ushort(__float2half(x2 * cs.x + x1 * cs.y));
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

    __device__ inline float widen(const std::uint16_t *x, std::size_t i)
    {
      return h2f(x[i]);
    }
    __device__ inline float widen(const float *x, std::size_t i) { return x[i]; }

    template <typename In>
    __global__ void __launch_bounds__(256)
        rmsnorm_kernel(const In *__restrict__ x, const std::uint16_t *__restrict__ weight,
                       std::uint16_t *__restrict__ out, int hidden, float eps)
    {
      __shared__ float partial[256 / 64];
      __shared__ float scale;
      const std::size_t row = static_cast<std::size_t>(blockIdx.x) * hidden;
      float acc = 0.0f;
      for (int i = threadIdx.x; i < hidden; i += blockDim.x)
      {
        const float v = widen(x, row + i);
        acc += v * v;
      }
      for (int offset = warpSize / 2; offset > 0; offset /= 2)
      {
        acc += __shfl_xor(acc, offset);
      }
      const int wave = threadIdx.x / warpSize;
      if (threadIdx.x % warpSize == 0)
      {
        partial[wave] = acc;
      }
      __syncthreads();
      if (threadIdx.x == 0)
      {
        float total = 0.0f;
        for (int w = 0; w < static_cast<int>(blockDim.x / warpSize); ++w)
        {
          total += partial[w];
        }
        scale = rsqrtf(total / static_cast<float>(hidden) + eps);
      }
      __syncthreads();
      for (int i = threadIdx.x; i < hidden; i += blockDim.x)
      {
        const float v = widen(x, row + i) * scale * h2f(weight[i]);
        out[row + i] = __half_as_ushort(__float2half(v));
      }
    }

    __global__ void swiglu_kernel(const std::uint16_t *__restrict__ gate,
                                  const std::uint16_t *__restrict__ up,
                                  std::uint16_t *__restrict__ out, std::size_t count)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const float g = h2f(gate[i]);
        const float silu = g / (1.0f + expf(-g));
        out[i] = __half_as_ushort(__float2half(silu * h2f(up[i])));
      }
    }

    // The same, eight values a thread through 16-byte loads and stores.
    __global__ void swiglu8_kernel(const uint4 *__restrict__ gate, const uint4 *__restrict__ up,
                                   uint4 *__restrict__ out, std::size_t groups)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < groups; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const uint4 gw = gate[i];
        const uint4 uw = up[i];
        const unsigned gs[4] = {gw.x, gw.y, gw.z, gw.w};
        const unsigned us[4] = {uw.x, uw.y, uw.z, uw.w};
        unsigned os[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
          unsigned word = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h)
          {
            const float g = h2f(static_cast<std::uint16_t>(gs[k] >> (16 * h)));
            const float silu = g / (1.0f + expf(-g));
            const float u = h2f(static_cast<std::uint16_t>(us[k] >> (16 * h)));
            word |= static_cast<unsigned>(__half_as_ushort(__float2half(silu * u))) << (16 * h);
          }
          os[k] = word;
        }
        out[i] = uint4{os[0], os[1], os[2], os[3]};
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
    hipLaunchKernelGGL(rope_kernel, dim3(seq * heads), dim3(64), 0, stream,
                       static_cast<const std::uint16_t *>(x), positions,
                       static_cast<std::uint16_t *>(out), heads, head_dim, theta);
    hip_check(hipGetLastError(), "rope kernel launch");
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
    if (count % 8 == 0 && aligned(gate) && aligned(up) && aligned(out))
    {
      const std::size_t groups = count / 8;
      hipLaunchKernelGGL(swiglu8_kernel, dim3(grid_for(groups, 256)), dim3(256), 0, stream,
                         static_cast<const uint4 *>(gate), static_cast<const uint4 *>(up),
                         static_cast<uint4 *>(out), groups);
    }
    else
    {
      hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(count, 256)), dim3(256), 0, stream,
                         static_cast<const std::uint16_t *>(gate),
                         static_cast<const std::uint16_t *>(up), static_cast<std::uint16_t *>(out),
                         count);
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
