// Dense projections through hipBLASLt: y = x W^T (+ bias), fp16 operands,
// fp32 accumulation (reference: linear.cu:85-142).
//
// The checkpoint stores W as (out_features, in_features) row-major and the
// rows of x are tokens. hipBLASLt is column-major, where a row-major matrix
// reads as its transpose, so the call computes y^T (out, rows) =
// op(W) (out, in) * x^T (in, rows) with op(W) = T over W's column-major
// (in, out) view and x^T read as stored; y^T column-major is y row-major.
//
// Three forms, as the reference has them:
//   - fp16 out, the bias (if any) added in the epilogue in fp32 before the one
//     rounding to fp16 (the reference seeds the output with the bias and
//     takes beta = 1: the same single rounding of acc + bias);
//   - fp32 out (the LM head's logits);
//   - fp32 accumulate, out += x W^T with beta = 1, never rounded to fp16
//     (the residual stream).
// Each shape's descriptors and algorithm are looked up once and kept. The
// workspace is fixed and generous, so an algorithm that splits the reduction
// reduces its partials in fp32 in the workspace rather than in the output
// type (the reference forbids reduced-precision split-K reductions for the
// same reason).

#include "common.hpp"
#include "kernels.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

namespace mi
{
  namespace
  {

    constexpr std::size_t kWorkspaceBytes = 64ull << 20;

    void blas_check(hipblasStatus_t s, const char *what)
    {
      if (s != HIPBLAS_STATUS_SUCCESS)
      {
        throw DeviceError(std::string(what) + " failed: hipblas status " + std::to_string(s));
      }
    }

    enum class Form : int
    {
      kHalf = 0,
      kHalfBias = 1,
      kFloat = 2,
      kFloatAccumulate = 3,
    };

    struct Plan
    {
      hipblasLtMatmulDesc_t desc = nullptr;
      hipblasLtMatrixLayout_t a = nullptr; // W, column-major (in, out)
      hipblasLtMatrixLayout_t b = nullptr; // x, column-major (in, rows)
      hipblasLtMatrixLayout_t d = nullptr; // y, column-major (out, rows)
      hipblasLtMatmulAlgo_t algo{};
      std::size_t workspace = 0;
    };

    // One handle and workspace for the life of the process, made on first
    // use and never destroyed (a destructor at exit could run after the HIP
    // runtime is gone; the driver reclaims both).
    struct Blas
    {
      hipblasLtHandle_t handle = nullptr;
      void *workspace = nullptr;
      std::mutex lock;
      std::map<std::tuple<int, int, int, int>, Plan> plans;

      Blas()
      {
        blas_check(hipblasLtCreate(&handle), "hipblasLtCreate");
        hip_check(hipMalloc(&workspace, kWorkspaceBytes), "hipMalloc GEMM workspace");
      }
    };

    Blas &blas()
    {
      static Blas *b = new Blas();
      return *b;
    }

    Plan make_plan(Blas &bl, Form form, int rows, int in_features, int out_features)
    {
      Plan p;
      const bool half_out = form == Form::kHalf || form == Form::kHalfBias;
      const hipDataType out_type = half_out ? HIP_R_16F : HIP_R_32F;
      blas_check(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F),
                 "hipblasLtMatmulDescCreate");
      const hipblasOperation_t op_w = HIPBLAS_OP_T;
      const hipblasOperation_t op_x = HIPBLAS_OP_N;
      blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_w,
                                                 sizeof(op_w)),
                 "set TRANSA");
      blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_x,
                                                 sizeof(op_x)),
                 "set TRANSB");
      if (form == Form::kHalfBias)
      {
        const hipblasLtEpilogue_t epilogue = HIPBLASLT_EPILOGUE_BIAS;
        const hipDataType bias_type = HIP_R_16F;
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE,
                                                   &epilogue, sizeof(epilogue)),
                   "set EPILOGUE");
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE,
                                                   &bias_type, sizeof(bias_type)),
                   "set BIAS_DATA_TYPE");
      }
      blas_check(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, in_features, out_features,
                                             in_features),
                 "hipblasLtMatrixLayoutCreate W");
      blas_check(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, in_features, rows, in_features),
                 "hipblasLtMatrixLayoutCreate x");
      blas_check(hipblasLtMatrixLayoutCreate(&p.d, out_type, out_features, rows, out_features),
                 "hipblasLtMatrixLayoutCreate y");

      hipblasLtMatmulPreference_t pref = nullptr;
      blas_check(hipblasLtMatmulPreferenceCreate(&pref), "hipblasLtMatmulPreferenceCreate");
      const std::uint64_t ws = kWorkspaceBytes;
      blas_check(hipblasLtMatmulPreferenceSetAttribute(
                     pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)),
                 "set MAX_WORKSPACE_BYTES");
      hipblasLtMatmulHeuristicResult_t found[1];
      int count = 0;
      const hipblasStatus_t s = hipblasLtMatmulAlgoGetHeuristic(
          bl.handle, p.desc, p.a, p.b, p.d, p.d, pref, 1, found, &count);
      hipblasLtMatmulPreferenceDestroy(pref);
      if (s != HIPBLAS_STATUS_SUCCESS || count < 1 || found[0].state != HIPBLAS_STATUS_SUCCESS)
      {
        throw DeviceError("hipBLASLt has no algorithm for a (" + std::to_string(rows) + ", " +
                          std::to_string(in_features) + ") x (" + std::to_string(out_features) +
                          ", " + std::to_string(in_features) + ")^T projection (status " +
                          std::to_string(s) + ")");
      }
      p.algo = found[0].algo;
      p.workspace = found[0].workspaceSize;
      return p;
    }

    void gemm(Form form, const void *x, const void *weight, const void *bias, void *out, int rows,
              int in_features, int out_features, hipStream_t stream)
    {
      Blas &bl = blas();
      std::lock_guard<std::mutex> guard(bl.lock);
      const auto key = std::make_tuple(static_cast<int>(form), rows, in_features, out_features);
      auto it = bl.plans.find(key);
      if (it == bl.plans.end())
      {
        it = bl.plans.emplace(key, make_plan(bl, form, rows, in_features, out_features)).first;
      }
      Plan &p = it->second;
      if (form == Form::kHalfBias)
      {
        blas_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER,
                                                   &bias, sizeof(bias)),
                   "set BIAS_POINTER");
      }
      const float alpha = 1.0f;
      const float beta = form == Form::kFloatAccumulate ? 1.0f : 0.0f;
      blas_check(hipblasLtMatmul(bl.handle, p.desc, &alpha, weight, p.a, x, p.b, &beta, out, p.d,
                                 out, p.d, &p.algo, bl.workspace, p.workspace, stream),
                 "hipblasLtMatmul");
    }

    void check_shape(int rows, int in_features, int out_features)
    {
      if (rows < 0 || in_features < 0 || out_features < 0)
      {
        throw InvalidArgument("a projection's rows, in_features and out_features are >= 0; got " +
                              std::to_string(rows) + ", " + std::to_string(in_features) + ", " +
                              std::to_string(out_features));
      }
    }

  } // namespace

  void linear_half(const void *x, const void *weight, const void *bias, void *out, int rows,
                   int in_features, int out_features, hipStream_t stream)
  {
    check_shape(rows, in_features, out_features);
    if (rows == 0 || out_features == 0)
    {
      return;
    }
    if (in_features == 0)
    {
      // An empty sum: the output is the bias, or zero.
      launch_broadcast_rows(bias, out, rows, out_features, stream);
      return;
    }
    gemm(bias != nullptr ? Form::kHalfBias : Form::kHalf, x, weight, bias, out, rows, in_features,
         out_features, stream);
  }

  void linear_float(const void *x, const void *weight, float *out, bool accumulate, int rows,
                    int in_features, int out_features, hipStream_t stream)
  {
    check_shape(rows, in_features, out_features);
    if (rows == 0 || out_features == 0)
    {
      return;
    }
    if (in_features == 0)
    {
      if (!accumulate)
      {
        launch_fill(out, static_cast<std::size_t>(rows) * out_features, 0.0f, stream);
      }
      return;
    }
    gemm(accumulate ? Form::kFloatAccumulate : Form::kFloat, x, weight, nullptr, out, rows,
         in_features, out_features, stream);
  }

} // namespace mi
