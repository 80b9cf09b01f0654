// Operator API: the fused decode kernels one at a time, on a caller stream.
// Counterparts of the TileLang factories in
// soraku_inference/acceleration/tilelang_kernels.py (same operands and
// meaning; masking uses -inf as the native path does, model.py:582-584,
// instead of the -1e30 of tilelang_kernels.py:31).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sk_error.h"
#include "sk_kernels.h"
#include "sk_launch.h"
#include "soraku_mi355x.h"

using namespace sk;

namespace {

int check_wdtype(int32_t wdtype) {
  SK_CHECK(wdtype == SK_F32 || wdtype == SK_BF16, SK_EINVAL, "wdtype must be SK_F32 or SK_BF16");
  return SK_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Runs a GEMV over B activation rows in chunks of at most 4 rows.
template <int PRO, int EPI>
int gemv_rows(hipStream_t st, int wdtype, int B, GemvArgs a, int ldres) {
  for (int b0 = 0; b0 < B; b0 += 4) {
    const int m = (B - b0) < 4 ? (B - b0) : 4;
    GemvArgs c = a;
    c.x = a.x + (size_t)b0 * a.ldx;
    c.out = a.out + (size_t)b0 * a.ldo;
    if (a.res) c.res = a.res + (size_t)b0 * ldres;
    SK_HIP((launch_gemv<PRO, EPI>(wdtype, m, c, st)));
  }
  return SK_OK;
}

}  // namespace

extern "C" {

int sk_op_add_rmsnorm(void* stream, int32_t B, int32_t D, float eps, const float* hidden,
                      const float* prefix, const float* weight, float* out) {
  SK_CHECK(B > 0 && D > 0, SK_EINVAL, "B and D must be positive");
  SK_CHECK(hidden && prefix && weight && out, SK_EINVAL, "NULL operand");
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(B), dim3(NT), 0, (hipStream_t)stream, hidden, prefix,
                     weight, eps, D, out, nullptr);
  SK_HIP(hipGetLastError());
  return SK_OK;
}

int sk_op_rmsnorm(void* stream, int32_t B, int32_t D, float eps, const float* x, const float* weight,
                  float* out) {
  SK_CHECK(B > 0 && D > 0, SK_EINVAL, "B and D must be positive");
  SK_CHECK(x && weight && out, SK_EINVAL, "NULL operand");
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(B), dim3(NT), 0, (hipStream_t)stream, x, nullptr,
                     weight, eps, D, out, nullptr);
  SK_HIP(hipGetLastError());
  return SK_OK;
}

int sk_op_swiglu_gemv(void* stream, int32_t B, int32_t I, int32_t D, int32_t wdtype, const float* x,
                      const void* wg, const void* wu, float* out) {
  int rc = check_wdtype(wdtype);
  if (rc) return rc;
  SK_CHECK(B > 0 && I > 0 && D > 0 && D % 8 == 0, SK_EINVAL, "B, I > 0 and D a positive multiple of 8");
  SK_CHECK(x && wg && wu && out, SK_EINVAL, "NULL operand");
  SK_CHECK(aligned16(x) && aligned16(wg) && aligned16(wu), SK_EINVAL, "operands must be 16-byte aligned");
  GemvArgs a = gemv_args(wg, I, D, x, D, out, I);
  a.w[1] = wu;
  return gemv_rows<PRO_NONE, EPI_SWIGLU>((hipStream_t)stream, wdtype, B, a, 0);
}

int sk_op_down_residual_gemv(void* stream, int32_t B, int32_t D, int32_t I, int32_t wdtype,
                             const float* act, const void* wd, const float* residual, float* out) {
  int rc = check_wdtype(wdtype);
  if (rc) return rc;
  SK_CHECK(B > 0 && D > 0 && I > 0 && I % 8 == 0, SK_EINVAL, "B, D > 0 and I a positive multiple of 8");
  SK_CHECK(act && wd && residual && out, SK_EINVAL, "NULL operand");
  SK_CHECK(aligned16(act) && aligned16(wd), SK_EINVAL, "operands must be 16-byte aligned");
  GemvArgs a = gemv_args(wd, D, I, act, I, out, D);
  a.res = residual; a.ldr = D;
  return gemv_rows<PRO_NONE, EPI_RESID>((hipStream_t)stream, wdtype, B, a, D);
}

int sk_op_classifier_gemv(void* stream, int32_t B, int32_t V, int32_t D, int32_t wdtype,
                          const float* body, const void* wq, const float* bias, float* out) {
  int rc = check_wdtype(wdtype);
  if (rc) return rc;
  SK_CHECK(B > 0 && V > 0 && D > 0 && D % 8 == 0, SK_EINVAL, "B, V > 0 and D a positive multiple of 8");
  SK_CHECK(body && wq && bias && out, SK_EINVAL, "NULL operand");
  SK_CHECK(aligned16(body) && aligned16(wq), SK_EINVAL, "operands must be 16-byte aligned");
  GemvArgs a = gemv_args(wq, V, D, body, D, out, V);
  a.bias = bias;
  return gemv_rows<PRO_NONE, EPI_BIAS>((hipStream_t)stream, wdtype, B, a, 0);
}

int sk_op_frame_embed(void* stream, int32_t R, int32_t Q, int32_t V, int32_t D, float scale,
                      const int64_t* codes, const float* table, float* out) {
  SK_CHECK(R > 0 && Q > 0 && V > 0 && D > 0, SK_EINVAL, "R, Q, V, D must be positive");
  SK_CHECK(codes && table && out, SK_EINVAL, "NULL operand");
  hipLaunchKernelGGL(frame_embed_op_kernel, dim3(R), dim3(NT), 0, (hipStream_t)stream, codes, table, Q, V,
                     D, scale, out);
  SK_HIP(hipGetLastError());
  return SK_OK;
}

int sk_op_prefix_add(void* stream, int32_t B, int32_t V, int32_t D, float scale, const float* prefix,
                     const float* table_q, const int64_t* code, float* out) {
  SK_CHECK(B > 0 && V > 0 && D > 0, SK_EINVAL, "B, V, D must be positive");
  SK_CHECK(prefix && table_q && code && out, SK_EINVAL, "NULL operand");
  hipLaunchKernelGGL(prefix_add_op_kernel, dim3(B), dim3(NT), 0, (hipStream_t)stream, prefix, table_q,
                     code, V, D, scale, out);
  SK_HIP(hipGetLastError());
  return SK_OK;
}

int sk_op_sampling_prep(void* stream, int32_t V, int32_t bos_id, int32_t pad_id, int32_t eos_id,
                        const float* logits, const float* temperature, const int32_t* mask_eos,
                        float* out) {
  SK_CHECK(V > 0, SK_EINVAL, "V must be positive");
  SK_CHECK(logits && temperature && mask_eos && out, SK_EINVAL, "NULL operand");
  hipLaunchKernelGGL(sampling_prep_op_kernel, dim3((V + NT - 1) / NT), dim3(NT), 0, (hipStream_t)stream,
                     logits, temperature, mask_eos, V, bos_id, pad_id, eos_id, out);
  SK_HIP(hipGetLastError());
  return SK_OK;
}

int sk_op_sample(void* stream, int32_t rows, int32_t V, const float* logits, float cfg_scale, int32_t q,
                 int32_t mask_eos_q0, int32_t bos_id, int32_t eos_id, int32_t pad_id, float temperature,
                 int32_t top_k, float top_p, double u, int64_t* code_out) {
  SK_CHECK(rows == 1 || rows == 2, SK_EINVAL, "rows must be 1 or 2");
  SK_CHECK(V > 3 && V <= MAX_V, SK_EINVAL, "V must be in [4, %d]", MAX_V);
  SK_CHECK(logits && code_out, SK_EINVAL, "NULL operand");
  SK_CHECK(u >= 0.0 && u < 1.0, SK_EINVAL, "u must lie in [0, 1)");
  SK_CHECK(q >= 0, SK_EINVAL, "q must be non-negative");
  SK_HIP(prepare_sampler());
  SK_HIP(with_vpt(V, [&](auto vpt) {
    hipLaunchKernelGGL((sample_op_kernel<decltype(vpt)::value>), dim3(1), dim3(SNT), SAMPLE_SMEM,
                       (hipStream_t)stream, logits, rows, V, cfg_scale, q, mask_eos_q0, bos_id, eos_id, pad_id,
                       temperature, top_k, top_p, u, code_out);
    return hipGetLastError();
  }));
  return SK_OK;
}

}  // extern "C"
