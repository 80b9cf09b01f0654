// Host-side launch helpers shared by the engine and the operator API.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "sk_kernels.h"
#include "soraku_mi355x.h"

namespace sk {

template <int M, int RPW, int PRO, int EPI, typename WL>
static hipError_t launch_gemv_t(const GemvArgs& a, hipStream_t st) {
  constexpr int rows_per_block = WAVES * RPW;
  const int grid = (a.N + rows_per_block - 1) / rows_per_block;
  const size_t smem = (size_t)M * a.K * sizeof(float);
  auto fn = gemv_kernel<M, RPW, PRO, EPI, WL>;
  if (smem > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(grid), dim3(NT), smem, st, a);
  return hipGetLastError();
}

// Rows per wave: 2 when that still yields >= 512 workgroups, else 1, so every
// GEMV of the decode step spreads over all 256 CUs.
template <int PRO, int EPI, typename WL>
static hipError_t launch_gemv_m(int M, const GemvArgs& a, hipStream_t st) {
  const bool wide = (a.N / (WAVES * 2)) >= 512;
  switch (M) {
    case 1: return wide ? launch_gemv_t<1, 2, PRO, EPI, WL>(a, st) : launch_gemv_t<1, 1, PRO, EPI, WL>(a, st);
    case 2: return wide ? launch_gemv_t<2, 2, PRO, EPI, WL>(a, st) : launch_gemv_t<2, 1, PRO, EPI, WL>(a, st);
    case 3: return wide ? launch_gemv_t<3, 2, PRO, EPI, WL>(a, st) : launch_gemv_t<3, 1, PRO, EPI, WL>(a, st);
    case 4: return wide ? launch_gemv_t<4, 2, PRO, EPI, WL>(a, st) : launch_gemv_t<4, 1, PRO, EPI, WL>(a, st);
    default: return hipErrorInvalidValue;
  }
}

// ---- compile-time-K GEMV (all of a wave's loads issued up front) ----------
template <int M, int KT, int RW, int PRO, int EPI, typename WL>
static hipError_t launch_fast_t(const GemvArgs& a, hipStream_t st) {
  constexpr int NS = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int NV = KT / (64 * WL::VEC);
  if constexpr (RW > 1 && RW * NS * NV > 16) {
    return launch_fast_t<M, KT, RW / 2, PRO, EPI, WL>(a, st);
  } else {
    const int grid = (a.N + WAVES * RW - 1) / (WAVES * RW);
    hipLaunchKernelGGL((gemv_fast_kernel<M, KT, RW, PRO, EPI, WL>), dim3(grid), dim3(NT), 0, st, a);
    return hipGetLastError();
  }
}

// Rows per wave: as many as keep <= 16 loads per lane in flight while the
// grid still has >= 256 workgroups (one per CU).
template <int M, int KT, int PRO, int EPI, typename WL>
static hipError_t launch_fast_k(const GemvArgs& a, hipStream_t st) {
  constexpr int NS = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int NV = KT / (64 * WL::VEC);
  int rw = 4;
  while (rw > 1 && (rw * NS * NV > 16 || a.N / (WAVES * rw) < 256)) rw /= 2;
  // Prefer a grid that spreads evenly over the 256 CUs: N = 3072 with SwiGLU
  // is 384 workgroups at 2 rows per wave (half the CUs stream twice the
  // bytes) but 768 at 1 row (3 per CU).
  if (rw > 1) {
    const int g = (a.N + WAVES * rw - 1) / (WAVES * rw), g2 = (a.N + WAVES * (rw / 2) - 1) / (WAVES * (rw / 2));
    if (g % 256 != 0 && g2 % 256 == 0) rw /= 2;
  }
  switch (rw) {
    case 4: return launch_fast_t<M, KT, 4, PRO, EPI, WL>(a, st);
    case 2: return launch_fast_t<M, KT, 2, PRO, EPI, WL>(a, st);
    default: return launch_fast_t<M, KT, 1, PRO, EPI, WL>(a, st);
  }
}

// K-sliced residual GEMV (4 rows per workgroup, K split over its waves), for
// the K whose slice is a whole number of 64-lane loads.
template <int M, int KT, typename WL>
static bool try_kslice(const GemvArgs& a, hipStream_t st, hipError_t* err) {
  if constexpr ((KT / WAVES) % (64 * WL::VEC) == 0) {
    constexpr int RG = 4;
    const int grid = (a.N + RG - 1) / RG;
    hipLaunchKernelGGL((gemv_kslice_kernel<M, KT, RG, WL>), dim3(grid), dim3(NT), 0, st, a);
    *err = hipGetLastError();
    return true;
  } else {
    return false;
  }
}
// Residual GEMVs that take the K-sliced form: BF16 weights (measured at the
// 1.7B shape: K = 2048, 4096, 6144 all faster); with FP32 weights the full-K
// form with activations shared through LDS is faster (0.6B: K = 2048, 3072).
template <typename WL>
static inline bool use_kslice(int K) {
  return std::is_same<WL, WBF16>::value && (K == 2048 || K == 4096 || K == 6144);
}

// K values with a specialised kernel: the decode shapes' hidden sizes for
// GEMVs fed by a norm / SwiGLU / classifier, and the inner sizes for the
// down / output projections.  Returns false when no specialisation applies.
template <int M, int PRO, int EPI, typename WL>
static bool launch_fast(const GemvArgs& a, hipStream_t st, hipError_t* err) {
  if constexpr (PRO == PRO_NONE && EPI == EPI_RESID) {
    if (use_kslice<WL>(a.K)) {
      switch (a.K) {
        case 2048: if (try_kslice<M, 2048, WL>(a, st, err)) return true; break;
        case 3072: if (try_kslice<M, 3072, WL>(a, st, err)) return true; break;
        case 4096: if (try_kslice<M, 4096, WL>(a, st, err)) return true; break;
        case 6144: if (try_kslice<M, 6144, WL>(a, st, err)) return true; break;
        default: break;
      }
    }
    switch (a.K) {
      case 2048: *err = launch_fast_k<M, 2048, PRO, EPI, WL>(a, st); return true;
      case 3072: *err = launch_fast_k<M, 3072, PRO, EPI, WL>(a, st); return true;
      case 4096: *err = launch_fast_k<M, 4096, PRO, EPI, WL>(a, st); return true;
      case 6144: *err = launch_fast_k<M, 6144, PRO, EPI, WL>(a, st); return true;
      default: return false;
    }
  } else {
    switch (a.K) {
      case 1024: *err = launch_fast_k<M, 1024, PRO, EPI, WL>(a, st); return true;
      case 2048: *err = launch_fast_k<M, 2048, PRO, EPI, WL>(a, st); return true;
      default: return false;
    }
  }
}

template <int PRO, int EPI, typename WL>
static hipError_t launch_gemv_w(int M, const GemvArgs& a, hipStream_t st) {
  hipError_t err = hipSuccess;
  if (M == 1 && launch_fast<1, PRO, EPI, WL>(a, st, &err)) return err;
  if (M == 2 && launch_fast<2, PRO, EPI, WL>(a, st, &err)) return err;
  return launch_gemv_m<PRO, EPI, WL>(M, a, st);
}

template <int PRO, int EPI>
static hipError_t launch_gemv(int wdtype, int M, const GemvArgs& a, hipStream_t st) {
  return wdtype == SK_BF16 ? launch_gemv_w<PRO, EPI, WBF16>(M, a, st)
                           : launch_gemv_w<PRO, EPI, WF32>(M, a, st);
}

static inline GemvArgs gemv_args(const void* w, int N, int K, const float* x, int ldx, float* out,
                                 int ldo) {
  GemvArgs a{};
  a.w[0] = w; a.w[1] = nullptr; a.w[2] = nullptr;
  a.seg_rows[0] = N; a.seg_rows[1] = 0; a.seg_rows[2] = 0;
  a.N = N; a.K = K;
  a.x = x; a.ldx = ldx;
  a.out = out; a.ldo = ldo;
  return a;
}

// Sampler launches pick the instantiation with the fewest logits per thread
// that covers V: 1, 2, 3, 5 or 8 per thread of SNT (V <= MAX_V).
static_assert(8 * SNT >= MAX_V, "sampler instantiations must cover MAX_V");
template <typename F>
static hipError_t with_vpt(int V, F&& f) {
  const int need = (V + SNT - 1) / SNT;
  if (need <= 1) return f(std::integral_constant<int, 1>{});
  if (need <= 2) return f(std::integral_constant<int, 2>{});
  if (need <= 3) return f(std::integral_constant<int, 3>{});
  if (need <= 5) return f(std::integral_constant<int, 5>{});
  return f(std::integral_constant<int, 8>{});
}

template <typename TL>
static hipError_t launch_sample_step(const SampleArgs& a, int q, int n_utts, hipStream_t st, int slices = 1) {
  return with_vpt(a.V, [&](auto vpt) {
    constexpr int VPT = decltype(vpt)::value;
    const dim3 grid(n_utts, slices);
    if (a.d <= SNT)
      hipLaunchKernelGGL((sample_step_kernel<TL, VPT, 1>), grid, dim3(SNT), SAMPLE_SMEM, st, a, q);
    else if (a.d <= 2 * SNT)
      hipLaunchKernelGGL((sample_step_kernel<TL, VPT, 2>), grid, dim3(SNT), SAMPLE_SMEM, st, a, q);
    else if (a.d <= 4 * SNT)
      hipLaunchKernelGGL((sample_step_kernel<TL, VPT, 4>), grid, dim3(SNT), SAMPLE_SMEM, st, a, q);
    else
      hipLaunchKernelGGL((sample_step_kernel<TL, VPT, DEPTH_DPT>), grid, dim3(SNT), SAMPLE_SMEM, st, a, q);
    return hipGetLastError();
  });
}
// Workgroups per utterance for a many-row sampler that forms the next depth
// step's inputs: the most (up to 16, within 256 in all) that divide d and the
// inner size evenly.
static inline int sample_slices(int n_utts, int d, int ki) {
  int s = 16;
  while (s > 1 && (n_utts * s > 256 || d % s != 0 || ki % s != 0)) s /= 2;
  return s;
}

// Depth step with the previous codebook's sampler folded in
// (depth_sample_gemv_kernel): one utterance, d = 1024 or 2048, 1 or 2 rows.
static inline bool depth_fused_fits(int d, int rows, int depth_inner, int V) {
  const int rw = depth_inner >= 4096 ? 2 : 1;
  return (d == 1024 || d == 2048) && (rows == 1 || rows == 2) && depth_inner % (SWAVES * rw) == 0 &&
         V <= MAX_V && depth_sample_smem(V) <= 65536;
}
template <typename TL, int VPT, int M, int KT>
static hipError_t launch_depth_fused_t(const SampleArgs& s, const GemvArgs& g, int q, hipStream_t st) {
  const size_t smem = depth_sample_smem(s.V);
  if (g.N >= 4096)
    hipLaunchKernelGGL((depth_sample_gemv_kernel<TL, VPT, M, KT, 2>), dim3(g.N / (SWAVES * 2)), dim3(SNT), smem, st,
                       s, g, q);
  else
    hipLaunchKernelGGL((depth_sample_gemv_kernel<TL, VPT, M, KT, 1>), dim3(g.N / SWAVES), dim3(SNT), smem, st, s, g,
                       q);
  return hipGetLastError();
}
template <typename TL>
static hipError_t launch_depth_fused(const SampleArgs& s, const GemvArgs& g, int rows, int q, hipStream_t st) {
  return with_vpt(s.V, [&](auto vpt) {
    constexpr int P = decltype(vpt)::value;
    if (g.K == 1024)
      return rows == 2 ? launch_depth_fused_t<TL, P, 2, 1024>(s, g, q, st) : launch_depth_fused_t<TL, P, 1, 1024>(s, g, q, st);
    return rows == 2 ? launch_depth_fused_t<TL, P, 2, 2048>(s, g, q, st) : launch_depth_fused_t<TL, P, 1, 2048>(s, g, q, st);
  });
}

// Depth steps by code tables (depth_step_kernel): CFG rows (2), the Qwen3-0.6B
// shape with FP32 weights (d 1024, inner 2048) or the 1.7B shape with BF16
// weights (d 2048, inner 4096) -- the shapes whose inner dimension is eight
// waves' 16-byte loads.
static inline bool code_tables_fit(int d, int rows, int depth_inner, int V, int wdtype) {
  const int vec = wdtype == SK_BF16 ? 8 : 4;
  return rows == 2 && ((d == 1024 && wdtype == SK_F32) || (d == 2048 && wdtype == SK_BF16)) &&
         depth_step_fits(d, depth_inner, vec) && V <= MAX_V && depth_sample_smem(V) <= 65536;
}
template <typename TL, int KD, int KI, int MODE>
static hipError_t launch_depth_step_t(const SampleArgs& s, const DepthArgs& g, int q, hipStream_t st) {
  if constexpr (MODE == 2) {   // with a sampler
    return with_vpt(s.V, [&](auto vpt) {
      hipLaunchKernelGGL((depth_step_kernel<TL, decltype(vpt)::value, 2, KD, KI, MODE>), dim3(DEPTH_WGS), dim3(SNT),
                         depth_sample_smem(s.V), st, s, g, q);
      return hipGetLastError();
    });
  } else {
    hipLaunchKernelGGL((depth_step_kernel<TL, 1, 2, KD, KI, MODE>), dim3(DEPTH_WGS), dim3(SNT), 0, st, s, g, q);
    return hipGetLastError();
  }
}
template <int MODE>
static hipError_t launch_depth_step(int wdtype, int d, const SampleArgs& s, const DepthArgs& g, int q,
                                    hipStream_t st) {
  if (wdtype == SK_BF16 && d == 2048) return launch_depth_step_t<WBF16, 2048, 4096, MODE>(s, g, q, st);
  if (wdtype == SK_F32 && d == 1024) return launch_depth_step_t<WF32, 1024, 2048, MODE>(s, g, q, st);
  return hipErrorInvalidConfiguration;   // not selected at capture
}

static inline hipError_t prepare_sampler() {
  static bool done = false;
  if (done) return hipSuccess;
  hipError_t e = hipSuccess;
  auto set = [&](const void* fn) {
    if (e == hipSuccess)
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)SAMPLE_SMEM);
  };
  for (int V : {SNT, 2 * SNT, 3 * SNT, 5 * SNT, 8 * SNT})
    with_vpt(V, [&](auto vpt) {
      constexpr int P = decltype(vpt)::value;
      set(reinterpret_cast<const void*>(sample_step_kernel<WF32, P, 1>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WF32, P, 2>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WF32, P, 4>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WF32, P, DEPTH_DPT>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WBF16, P, 1>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WBF16, P, 2>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WBF16, P, 4>));
      set(reinterpret_cast<const void*>(sample_step_kernel<WBF16, P, DEPTH_DPT>));
      set(reinterpret_cast<const void*>(sample_op_kernel<P>));
      return e;
    });
  if (e == hipSuccess) done = true;
  return e;
}

}  // namespace sk
