// Decode kernels for many rows (more than the GEMV kernels' 4): several
// utterances with CFG decoded together, up to 32 rows (the reference decodes
// one utterance's two CFG rows; fast_generate.py:232-328 batches those).
//
// The projections run as skinny GEMMs on the FP32 matrix cores: each
// workgroup owns 16 outputs for all rows and splits K over its 8 or 16 waves;
// the per-wave partial tiles are summed through LDS in fixed wave order
// (deterministic).  RMSNorms that feed a projection are folded into it.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "sk_kernels.h"

namespace sk {

struct SkinnyArgs {
  const void* w[3]; int seg_rows[3];   // weight segments (q / k / v), rows of each
  const void* w2;                      // SwiGLU: up weights
  const float* x; int ldx;             // [R][K]
  const float* norm_w; float eps;      // optional RMSNorm of x rows (gain [K])
  float* out; int ldo;                 // [R][N]
  const float* res; int ldr;           // residual (may alias out)
  const float* bias;                   // [N]
  int R, N, K;
  int ksplit;                          // K slices per output tile (1, 2 or 4; BF16 form)
  float* partial;                      // [tiles][ksplit][SK_PSZ] slice partials (ksplit > 1)
  unsigned* arrive;                    // [tiles] slice arrival counts, zero between launches
  // BF16 form only:
  const uint16_t* xs;                  // x in split form (xsplit_index), gain applied; null: FP32 x
  const float* ss_in; int n_ss;        // NORM with xs: [32][n_ss] partial sums of x^2 per row
  uint16_t* xs_out;                    // out again in split form for the next GEMM; null: none
  const float* xs_gain;                // gain applied before that split (the next RMSNorm); null: 1
  float* ss_out;                       // [32][N/16] sums of out^2 per row and output tile; null: none
  float* pre_out; int ld_pre;          // SwiGLU: gate and up before the activation, [R][ld_pre]
                                       // (gate at o, up at N + o); null: none
  // Split-K merge by tagged words (null tpart: the arrival-count merge):
  // slices 1.. store their partials as 8-byte words (value, tag) and leave;
  // slice 0 reads them until every tag is this launch's, *fc * 256 + tag_idx
  // + 1 (fc: the frame counter, constant over a frame; tag_idx: the launch's
  // place among the frame's GEMM launches), so a word left by an earlier
  // launch never carries it (the host clears the words wherever the frame
  // counter restarts at 0).  A wait past `spin` ticks sets err bit 1.
  unsigned long long* tpart;           // [tiles][SK_MAX_SPLIT][SK_PSZ]
  const int* fc; int tag_idx;
  unsigned* err; unsigned long long spin;
};

// Floats per slice partial: two epilogue values per thread (SwiGLU) + 32 row
// sums of squares.
constexpr int SK_PSZ = 2 * 512 + 32;
constexpr int SK_MAX_SPLIT = 4;          // largest K split a launch may use

constexpr int SK_ROWS = 32;             // rows covered (two 16-row MFMA tiles)

typedef float sv4f __attribute__((ext_vector_type(4)));

// out[r][o] for 16 outputs o of this workgroup and all rows r < R.  Lane l of
// a wave holds weights of output o0 + l % 16 and rows (l % 16) (+16) of x for
// VEC consecutive k at kb + VEC (l / 16); MFMA j pairs weight and x at the
// same k, so every k of the block enters the sum exactly once.  Wave w takes
// blocks w, w + W, ...; the next block's loads are in flight while one is
// multiplied.  NORM: x is taken through RMSNorm -- the gain is applied per k,
// the row's sum of squares is gathered on the way and 1 / rms scales the sum
// at the end (out = inv_rms * sum_k w_k g_k x_k).  EPI is one of the GEMV
// epilogues (store, bias, residual, SwiGLU).
template <int EPI, typename WL, int W, bool NORM>
__global__ __launch_bounds__(W * 64) void skinny_gemm_kernel(SkinnyArgs a) {
  constexpr int NA = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int VEC = WL::VEC;          // 4 (FP32) or 8 (BF16) k per lane per block
  constexpr int BK = 4 * VEC;           // k per block
  __shared__ float red[W][NA * 2 * 4][64];
  __shared__ float ssq[NORM ? W : 1][2][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, kq = lane >> 4;
  const int o0 = blockIdx.x * 16;
  const int o = min(o0 + i16, a.N - 1);
  const void* wb;
  int wr;
  if (o < a.seg_rows[0]) { wb = a.w[0]; wr = o; }
  else if (o < a.seg_rows[0] + a.seg_rows[1]) { wb = a.w[1]; wr = o - a.seg_rows[0]; }
  else { wb = a.w[2]; wr = o - a.seg_rows[0] - a.seg_rows[1]; }
  const size_t woff = (size_t)wr * a.K + VEC * kq;
  const size_t w2off = (size_t)o * a.K + VEC * kq;
  const float* xr0 = a.x + (size_t)min(i16, a.R - 1) * a.ldx + VEC * kq;
  const float* xr1 = a.x + (size_t)min(16 + i16, a.R - 1) * a.ldx + VEC * kq;
  const float* gp = NORM ? a.norm_w + VEC * kq : nullptr;
  struct Stage { float w[NA][VEC], x0[VEC], x1[VEC], g[NORM ? VEC : 1]; };
  auto load = [&](int kb, Stage& st) {
    WL::load(wb, woff + kb, st.w[0]);
    if constexpr (NA == 2) WL::load(a.w2, w2off + kb, st.w[NA - 1]);
#pragma unroll
    for (int j = 0; j < VEC; j += 4) {
      const float4 p = *reinterpret_cast<const float4*>(xr0 + kb + j);
      const float4 q = *reinterpret_cast<const float4*>(xr1 + kb + j);
      st.x0[j] = p.x; st.x0[j + 1] = p.y; st.x0[j + 2] = p.z; st.x0[j + 3] = p.w;
      st.x1[j] = q.x; st.x1[j + 1] = q.y; st.x1[j + 2] = q.z; st.x1[j + 3] = q.w;
      if constexpr (NORM) {
        const float4 g = *reinterpret_cast<const float4*>(gp + kb + j);
        st.g[j] = g.x; st.g[j + 1] = g.y; st.g[j + 2] = g.z; st.g[j + 3] = g.w;
      }
    }
  };
  sv4f acc[NA][2];
#pragma unroll
  for (int n = 0; n < NA; ++n) acc[n][0] = acc[n][1] = sv4f{0.f, 0.f, 0.f, 0.f};
  float ss0 = 0.f, ss1 = 0.f;
  auto comp = [&](const Stage& st) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      float x0 = st.x0[j], x1 = st.x1[j];
      if constexpr (NORM) {
        ss0 = fmaf(x0, x0, ss0);
        ss1 = fmaf(x1, x1, ss1);
        x0 *= st.g[j];
        x1 *= st.g[j];
      }
#pragma unroll
      for (int n = 0; n < NA; ++n) {
        acc[n][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(st.w[n][j], x0, acc[n][0], 0, 0, 0);
        acc[n][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(st.w[n][j], x1, acc[n][1], 0, 0, 0);
      }
    }
  };
  Stage sa, sb;
  constexpr int STEP = W * BK;
  int kb = wave * BK;
  if (kb < a.K) load(kb, sa);
  for (; kb < a.K; kb += 2 * STEP) {
    const int k1 = kb + STEP, k2 = k1 + STEP;
    if (k1 < a.K) load(k1, sb);
    comp(sa);
    if (k1 < a.K) {
      if (k2 < a.K) load(k2, sa);
      comp(sb);
    }
  }
#pragma unroll
  for (int n = 0; n < NA; ++n)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][(n * 2 + t) * 4 + v][lane] = acc[n][t][v];
  if constexpr (NORM) { ssq[wave][0][lane] = ss0; ssq[wave][1][lane] = ss1; }
  __syncthreads();
  if (tid >= 512) return;
  // thread -> (row tile t, v, lane): output o0 + 4 (lane / 16) + v, row 16 t + lane % 16
  const int t = tid >> 8, v = (tid >> 6) & 3, l = tid & 63;
  const int oo = o0 + 4 * (l >> 4) + v, r = 16 * t + (l & 15);
  float c[NA];
#pragma unroll
  for (int n = 0; n < NA; ++n) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) s += red[w][(n * 2 + t) * 4 + v][l];
    c[n] = s;
  }
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) ss += ssq[w][t][k4 * 16 + (l & 15)];
    const float inv = 1.0f / sqrtf(ss / (float)a.K + a.eps);
#pragma unroll
    for (int n = 0; n < NA; ++n) c[n] *= inv;
  }
  if (oo < a.N && r < a.R) {
    float y = c[0];
    if constexpr (EPI == EPI_BIAS) y = y + a.bias[oo];
    if constexpr (EPI == EPI_RESID) y = a.res[(size_t)r * a.ldr + oo] + y;
    if constexpr (EPI == EPI_SWIGLU) {
      if (a.pre_out) {
        a.pre_out[(size_t)r * a.ld_pre + oo] = y;
        a.pre_out[(size_t)r * a.ld_pre + a.N + oo] = c[NA - 1];
      }
      y = y / (1.0f + expf(-y)) * c[NA - 1];
    }
    a.out[(size_t)r * a.ldo + oo] = y;
  }
}

// BF16 weights: the same GEMM on the BF16 matrix cores
// (v_mfma_f32_16x16x32_bf16).  A lane's 8 consecutive BF16 weights are the A
// fragment as loaded; each x value (times the norm gain) is split into x_hi =
// bf16(x) and x_lo = bf16(x - x_hi), and both halves go through the MFMA, so
// the products are exact in FP32 and x keeps ~16 mantissa bits (relative
// error <= 2^-16).  Sums in FP32 as in the FP32 form.
typedef __bf16 sbf8 __attribute__((ext_vector_type(8)));

//
// Split K (ksplit S > 1, for outputs too few to fill the GPU): the S slices of
// an output tile are workgroups tile % 8 + 8 (S (tile / 8) + s), so all run on
// XCD tile % 8 (workgroups are dispatched to the 8 XCDs round-robin) and share
// its L2.  Each slice stores its partial tile, waits until the stores are
// acknowledged, and counts itself in arrive[tile] (an L2 atomic); the last
// slice to arrive adds the S partials in slice order, applies the epilogue and
// resets the count.  No workgroup waits for another.  The arrival count and
// the partials are workgroup-scope operations: they are coherent only because
// every slice of a tile runs on one XCD.  sk_create checks that mapping with
// xcd_probe_kernel and launches without split K when it does not hold.
//
// Split input (XS): x arrives in split form, written by the kernel that
// produced it with this GEMM's norm gain applied, so a stage is four 16-byte
// fragment loads per lane and no conversion; with NORM the row's sum of
// squares is the sum of the producer's per-tile partials (ss_in).  Outputs
// can be written in split form for the next GEMM (xs_out, with that GEMM's
// gain) together with their per-tile sums of squares (ss_out).
// XCC_ID hardware register of each workgroup (one 64-thread wave each): the
// XCD it runs on.  Split K needs workgroups whose ids agree modulo 8 to share
// an XCD (and so an L2).
__global__ __launch_bounds__(64) void xcd_probe_kernel(unsigned* ids) {
  const unsigned xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);   // hwreg(HW_REG_XCC_ID)
  if (threadIdx.x == 0) ids[blockIdx.x] = xcc;
}
constexpr int XCD_PROBE_WGS = 2048;

template <int EPI, int W, bool NORM, bool XS>
__global__ __launch_bounds__(W * 64) void skinny_bf16_kernel(SkinnyArgs a) {
  static_assert(!XS || W == 8, "split input: one thread per (row, 16th of the partial sums)");
  constexpr int NA = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int BK = 32;                // k per block: 8 per lane
  constexpr bool XNORM = NORM && !XS;   // gain and sum of squares taken from FP32 x here
  __shared__ float red[W][NA * 2 * 4][64];
  __shared__ float ssq[XNORM ? W : 1][2][64];
  __shared__ float ssr[XS_ROWS];
  __shared__ float sso[2][4][64];
  __shared__ int last_slice;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, kq = lane >> 4;
  const int S = a.ksplit;
  const bool tagged = S > 1 && a.tpart != nullptr;
  const int fcv = tagged ? *a.fc : 0;
  int tile = blockIdx.x, slice = 0;
  if (S > 1) {
    const int xcd = blockIdx.x & 7, q = blockIdx.x >> 3;
    slice = q % S;
    tile = (q / S) * 8 + xcd;
  }
  const int kbeg = slice * (a.K / S), kend = kbeg + a.K / S;
  const int o0 = tile * 16;
  const int o = min(o0 + i16, a.N - 1);
  const void* wb;
  int wr;
  if (o < a.seg_rows[0]) { wb = a.w[0]; wr = o; }
  else if (o < a.seg_rows[0] + a.seg_rows[1]) { wb = a.w[1]; wr = o - a.seg_rows[0]; }
  else { wb = a.w[2]; wr = o - a.seg_rows[0] - a.seg_rows[1]; }
  const uint16_t* wp = static_cast<const uint16_t*>(wb) + (size_t)wr * a.K + 8 * kq;
  const uint16_t* w2p = NA == 2 ? static_cast<const uint16_t*>(a.w2) + (size_t)o * a.K + 8 * kq : nullptr;
  const float* xr0 = a.x + (size_t)min(i16, a.R - 1) * a.ldx + 8 * kq;
  const float* xr1 = a.x + (size_t)min(16 + i16, a.R - 1) * a.ldx + 8 * kq;
  const float* gp = XNORM ? a.norm_w + 8 * kq : nullptr;
  const uint4* xsp = XS ? reinterpret_cast<const uint4*>(a.xs) + lane : nullptr;
  struct StageF { uint4 w[NA]; float4 x0[2], x1[2], g[XNORM ? 2 : 1]; };
  struct StageS { uint4 w[NA]; uint4 xs[4]; };   // hi/lo of row tiles 0 and 1
  using Stage = typename std::conditional<XS, StageS, StageF>::type;
  auto load = [&](int kb, Stage& st) {
    st.w[0] = *reinterpret_cast<const uint4*>(wp + kb);
    if constexpr (NA == 2) st.w[NA - 1] = *reinterpret_cast<const uint4*>(w2p + kb);
    if constexpr (XS) {
#pragma unroll
      for (int j = 0; j < 4; ++j) st.xs[j] = xsp[((size_t)(kb >> 5) * 4 + j) * 64];
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        st.x0[h] = *reinterpret_cast<const float4*>(xr0 + kb + 4 * h);
        st.x1[h] = *reinterpret_cast<const float4*>(xr1 + kb + 4 * h);
        if constexpr (XNORM) st.g[h] = *reinterpret_cast<const float4*>(gp + kb + 4 * h);
      }
    }
  };
  sv4f acc[NA][2];
#pragma unroll
  for (int n = 0; n < NA; ++n) acc[n][0] = acc[n][1] = sv4f{0.f, 0.f, 0.f, 0.f};
  float ss0 = 0.f, ss1 = 0.f;
  auto split = [&](const float4 (&xv)[2], const float4 (&gv)[XNORM ? 2 : 1], float& ss, sbf8& hi, sbf8& lo) {
    const float v[8] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float x = v[j];
      if constexpr (XNORM) {
        const float g[8] = {gv[0].x, gv[0].y, gv[0].z, gv[0].w, gv[XNORM ? 1 : 0].x, gv[XNORM ? 1 : 0].y,
                            gv[XNORM ? 1 : 0].z, gv[XNORM ? 1 : 0].w};
        ss = fmaf(x, x, ss);
        x *= g[j];
      }
      const __bf16 h = (__bf16)x;
      hi[j] = h;
      lo[j] = (__bf16)(x - (float)h);
    }
  };
  auto comp = [&](const Stage& st) {
    sbf8 h0, l0, h1, l1;
    if constexpr (XS) {
      h0 = __builtin_bit_cast(sbf8, st.xs[0]);
      l0 = __builtin_bit_cast(sbf8, st.xs[1]);
      h1 = __builtin_bit_cast(sbf8, st.xs[2]);
      l1 = __builtin_bit_cast(sbf8, st.xs[3]);
    } else {
      split(st.x0, st.g, ss0, h0, l0);
      split(st.x1, st.g, ss1, h1, l1);
    }
#pragma unroll
    for (int n = 0; n < NA; ++n) {
      const sbf8 wa = __builtin_bit_cast(sbf8, st.w[n]);
      acc[n][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, h0, acc[n][0], 0, 0, 0);
      acc[n][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, l0, acc[n][0], 0, 0, 0);
      acc[n][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, h1, acc[n][1], 0, 0, 0);
      acc[n][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, l1, acc[n][1], 0, 0, 0);
    }
  };
  // Split input with NORM: the producer's partial sums of squares of row
  // tid / 16, 16 threads per row, loaded ahead of the first stage.
  constexpr int SSP = 16;               // partials per thread: n_ss <= 256
  float ssp[(XS && NORM) ? SSP : 1];
  if constexpr (XS && NORM) {
    // index clamped in bounds, value masked: no branch between the loads
    const float* sp = a.ss_in + (size_t)(tid >> 4) * a.n_ss;
#pragma unroll
    for (int i = 0; i < SSP; ++i) {
      const int j = (tid & 15) + 16 * i;
      const float v = sp[min(j, a.n_ss - 1)];
      ssp[i] = j < a.n_ss ? v : 0.f;
    }
  }
  // Epilogue operands of this thread's output (row r, column oo), loaded at
  // entry: they do not depend on the sums.
  const bool et = tid < 512;            // threads 0..511 own one (row tile, v, lane) each
  const int t = (tid >> 8) & 1, v = (tid >> 6) & 3, l = tid & 63;
  const int oo = o0 + 4 * (l >> 4) + v, r = 16 * t + (l & 15);
  const bool ok = et && oo < a.N && r < a.R;
  float epi_in = 0.f;
  if constexpr (EPI == EPI_BIAS) epi_in = ok ? a.bias[oo] : 0.f;
  if constexpr (EPI == EPI_RESID) epi_in = ok ? a.res[(size_t)r * a.ldr + oo] : 0.f;
  // the split-form output's gain too (index clamped: no branch around the load)
  const float gain_in = a.xs_gain ? a.xs_gain[min(oo, a.N - 1)] : 1.f;
  constexpr int STEP = W * BK;
  // This wave's stages: k = kw0 + i * STEP for i < nst.  Up to 4 stages
  // (every K / split of the 0.6B shapes) the wave issues all of its loads up
  // front, in straight-line code for its exact stage count, then multiplies
  // the stages in order: each multiply waits for its own stage only.  (In a
  // loop with conditional loads the compiler cannot count the loads in flight
  // and waited for all of them.)  Longer slices use the two-stage ring.
  const int kw0 = kbeg + wave * BK;
  const int nst = kw0 < kend ? (kend - kw0 + STEP - 1) / STEP : 0;
  auto upfront = [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    Stage st[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) load(kw0 + i * STEP, st[i]);
    asm volatile("" ::: "memory");   // not sunk towards the multiplies
#pragma unroll
    for (int i = 0; i < NC; ++i) comp(st[i]);
  };
  if (nst == 1) {
    upfront(std::integral_constant<int, 1>{});
  } else if (nst == 2) {
    upfront(std::integral_constant<int, 2>{});
  } else if (nst == 3) {
    upfront(std::integral_constant<int, 3>{});
  } else if (nst == 4) {
    upfront(std::integral_constant<int, 4>{});
  } else if (nst > 4) {
    Stage sa, sb;
    int kb = kw0;
    load(kb, sa);
    for (; kb < kend; kb += 2 * STEP) {
      const int k1 = kb + STEP, k2 = k1 + STEP;
      if (k1 < kend) load(k1, sb);
      comp(sa);
      if (k1 < kend) {
        if (k2 < kend) load(k2, sa);
        comp(sb);
      }
    }
  }
  // The row's sum of squares is needed only by the epilogue: summed after the
  // stream, so waiting for the partials never holds back a stage's loads.
  if constexpr (XS && NORM) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < SSP; ++i) t += ssp[i];
    t += __shfl_xor(t, 8, 64);          // the row's 16 threads; each pair adds in both orders alike
    t += __shfl_xor(t, 4, 64);
    t += __shfl_xor(t, 2, 64);
    t += __shfl_xor(t, 1, 64);
    if ((tid & 15) == 0) ssr[tid >> 4] = t;
  }
#pragma unroll
  for (int n = 0; n < NA; ++n)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][(n * 2 + t) * 4 + v][lane] = acc[n][t][v];
  if constexpr (XNORM) { ssq[wave][0][lane] = ss0; ssq[wave][1][lane] = ss1; }
  __syncthreads();
  // With 16 waves the upper half only takes part in the barriers.
  float c[NA];
#pragma unroll
  for (int n = 0; n < NA; ++n) {
    float sacc = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) sacc += red[w][(n * 2 + t) * 4 + v][l];
    c[n] = sacc;
  }
  float ss = 0.f;
  if constexpr (XNORM) {
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) ss += ssq[w][t][k4 * 16 + (l & 15)];
  }
  if constexpr (XS && NORM) ss = ssr[r];
  if (tagged) {
    const unsigned long long tag = (unsigned long long)((unsigned)fcv * 256u + (unsigned)a.tag_idx + 1u) << 32;
    unsigned long long* tp = a.tpart + (size_t)tile * SK_MAX_SPLIT * SK_PSZ;
    auto put = [&](unsigned long long* p, float x) {
      __hip_atomic_store(p, tag | __float_as_uint(x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    if (slice != 0) {
      if (et) {
#pragma unroll
        for (int n = 0; n < NA; ++n) put(tp + (size_t)slice * SK_PSZ + n * 512 + tid, c[n]);
        if (XNORM && v == 0 && (l >> 4) == 0) put(tp + (size_t)slice * SK_PSZ + 2 * 512 + r, ss);
      }
      return;
    }
    if (et) {
      // slices 1 .. S-1 (unrolled to SK_MAX_SPLIT, slice index clamped):
      // word (q - 1) * NA + n, then the row sums of squares
      constexpr int NW = (NA + (XNORM ? 1 : 0)) * (SK_MAX_SPLIT - 1);
      auto addr = [&](int i) {
        const int q = i < NA * (SK_MAX_SPLIT - 1) ? i / NA + 1 : i - NA * (SK_MAX_SPLIT - 1) + 1;
        const size_t qo = (size_t)min(q, S - 1) * SK_PSZ;
        return i < NA * (SK_MAX_SPLIT - 1) ? tp + qo + (i % NA) * 512 + tid : tp + qo + 2 * 512 + r;
      };
      unsigned long long w[NW];
#pragma unroll
      for (int i = 0; i < NW; ++i) w[i] = *addr(i);
      const unsigned long long deadline = __builtin_amdgcn_s_memrealtime() + a.spin;
      for (;;) {
        bool miss = false;
#pragma unroll
        for (int i = 0; i < NW; ++i) miss |= (w[i] & 0xffffffff00000000ull) != tag;
        if (!miss) break;
        if (__builtin_amdgcn_s_memrealtime() > deadline) {
          __hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          break;
        }
#pragma unroll
        for (int i = 0; i < NW; ++i)
          if ((w[i] & 0xffffffff00000000ull) != tag)
            w[i] = __hip_atomic_load(addr(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // in slice order, as the arrival-count merge adds them
#pragma unroll
      for (int n = 0; n < NA; ++n)
#pragma unroll
        for (int q = 1; q < SK_MAX_SPLIT; ++q)
          if (q < S) c[n] += __uint_as_float((unsigned)w[(q - 1) * NA + n]);
      if constexpr (XNORM) {
#pragma unroll
        for (int q = 1; q < SK_MAX_SPLIT; ++q)
          if (q < S) ss += __uint_as_float((unsigned)w[NA * (SK_MAX_SPLIT - 1) + q - 1]);
      }
    }
  } else if (S > 1) {
    float* mine = a.partial + ((size_t)tile * S + slice) * SK_PSZ;
    if (et) {
#pragma unroll
      for (int n = 0; n < NA; ++n) mine[n * 512 + tid] = c[n];
      if (XNORM && v == 0 && (l >> 4) == 0) mine[2 * 512 + r] = ss;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's partials are in L2
    __syncthreads();
    if (tid == 0)
      last_slice = __hip_atomic_fetch_add(a.arrive + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) + 1u ==
                   (unsigned)S;
    __syncthreads();
    if (!last_slice) return;
    if (tid == 0) __hip_atomic_store(a.arrive + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (et) {
      // All slices' partials loaded together (slice index clamped, unrolled
      // to SK_MAX_SPLIT), then summed in slice order: a loop over the runtime
      // S waited for each load before issuing the next.
      const float* all = a.partial + (size_t)tile * S * SK_PSZ;
      float pv[NA][SK_MAX_SPLIT], sv[XNORM ? SK_MAX_SPLIT : 1];
#pragma unroll
      for (int q = 0; q < SK_MAX_SPLIT; ++q) {
        const size_t qo = (size_t)min(q, S - 1) * SK_PSZ;
#pragma unroll
        for (int n = 0; n < NA; ++n) pv[n][q] = all[qo + n * 512 + tid];
        if constexpr (XNORM) sv[q] = all[qo + 2 * 512 + r];
      }
#pragma unroll
      for (int n = 0; n < NA; ++n) {
        float sacc = 0.f;
#pragma unroll
        for (int q = 0; q < SK_MAX_SPLIT; ++q)
          if (q < S) sacc += pv[n][q];
        c[n] = sacc;
      }
      if constexpr (XNORM) {
        ss = 0.f;
#pragma unroll
        for (int q = 0; q < SK_MAX_SPLIT; ++q)
          if (q < S) ss += sv[q];
      }
    }
  }
  if constexpr (NORM) {
    const float inv = 1.0f / sqrtf(ss / (float)a.K + a.eps);
#pragma unroll
    for (int n = 0; n < NA; ++n) c[n] *= inv;
  }
  float y = 0.f;
  if (ok) {
    y = c[0];
    if constexpr (EPI == EPI_BIAS) y = y + epi_in;
    if constexpr (EPI == EPI_RESID) y = epi_in + y;
    if constexpr (EPI == EPI_SWIGLU) {
      if (a.pre_out) {
        a.pre_out[(size_t)r * a.ld_pre + oo] = y;
        a.pre_out[(size_t)r * a.ld_pre + a.N + oo] = c[NA - 1];
      }
      y = y / (1.0f + expf(-y)) * c[NA - 1];
    }
    a.out[(size_t)r * a.ldo + oo] = y;
    if (a.xs_out) xsplit_store(a.xs_out, r, oo, a.xs_gain ? y * gain_in : y);
  }
  if (a.ss_out) {                       // uniform over the workgroup
    if (et) sso[t][v][l] = y * y;
    __syncthreads();
    if (et && v == 0 && (l >> 4) == 0 && r < a.R) {
      float sq = 0.f;
#pragma unroll
      for (int v2 = 0; v2 < 4; ++v2)
#pragma unroll
        for (int q = 0; q < 4; ++q) sq += sso[t][v2][q * 16 + (l & 15)];
      a.ss_out[(size_t)r * (a.N / 16) + tile] = sq;
    }
  }
}

}  // namespace sk
