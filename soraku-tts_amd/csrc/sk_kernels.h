// Device kernels of the soraku-TTS per-frame decode engine for gfx950 (CDNA4).
//
// Every kernel runs 256-thread workgroups = 4 wave64s.  Matrices are the
// reference's nn.Linear layout [out_rows][in_cols] (row-major, K contiguous),
// read with 16-byte vector loads so one wave streams 1 KiB per instruction.
// Activation vectors are tiny (M <= 4 rows) and are staged once per workgroup
// in LDS, where the fused RMSNorm prologues also run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

namespace sk {
// Internal linkage: both translation units include these kernels.
namespace {

constexpr int NT = 256;      // threads per workgroup
constexpr int WAVES = NT / 64;
constexpr int ATT_CHUNK = 32; // KV tokens per attention workgroup
constexpr int MAX_V = 4096;   // sampler LDS capacity (audio vocab)

// ------------------------------------------------------------ reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Sum of `v` over the workgroup; every thread gets the result.  `red` holds
// WAVES floats of LDS; the call ends with the workgroup synchronised.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) t += red[w];
  return t;
}

// ------------------------------------------------------------ weight loads
// FP32 matrices: 4 elements per 16-byte load.
struct WF32 {
  static constexpr int VEC = 4;
  using elem = float;
  __device__ __forceinline__ static void load(const void* base, size_t off, float (&o)[VEC]) {
    const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
  __device__ __forceinline__ static float get(const void* base, size_t off) {
    return static_cast<const float*>(base)[off];
  }
  __device__ __forceinline__ static uint4 raw(const void* base, size_t off) {
    return *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + off);
  }
  __device__ __forceinline__ static void widen(const uint4& v, float (&o)[VEC]) {
    o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y); o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
  }
};
// BF16 matrices: 8 elements per 16-byte load, widened to FP32 exactly.
struct WBF16 {
  static constexpr int VEC = 8;
  using elem = uint16_t;
  __device__ __forceinline__ static void load(const void* base, size_t off, float (&o)[VEC]) {
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static float get(const void* base, size_t off) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[off]) << 16);
  }
  __device__ __forceinline__ static uint4 raw(const void* base, size_t off) {
    return *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
  }
  __device__ __forceinline__ static void widen(const uint4& v, float (&o)[VEC]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

// ------------------------------------------------------------ GEMV family
// y[m][n] = sum_k x[m][k] * W[n][k] for M activation rows (decode rows).
// PRO_ADDGATHER: x + (x2 + scale * table[code]) -- the depth head's codebook
// prefix advanced by the previous step's code (model.py:600-605) inside the
// consumer of the prefix; block 0 writes the advanced prefix to gout.
enum { PRO_NONE = 0, PRO_NORM = 1, PRO_ADDNORM = 2, PRO_ADDGATHER = 3 };
enum { EPI_STORE = 0, EPI_BIAS = 1, EPI_RESID = 2, EPI_SWIGLU = 3 };

struct GemvArgs {
  // Up to three row segments concatenated (q/k/v projections share a launch).
  // EPI_SWIGLU: w[0] = gate, w[1] = up, both with N rows.
  const void* w[3];
  int seg_rows[3];
  int N, K;
  const float* x;  int ldx;    // [M][K] input rows
  const float* x2; int ldx2;   // PRO_ADDNORM: added to x before the norm
  const float* norm_w; float eps;
  float* norm_out; int ldno;   // optional copy of the prologue output (block 0 writes it)
  float* out; int ldo;
  const float* res; int ldr;   // EPI_RESID (may alias out: one lane owns each element)
  const float* bias;           // EPI_BIAS
  // PRO_ADDGATHER: row m takes code gcode[(m / g_rpu) * gstride] of table
  // gtable ([V][K], weight dtype); the advanced prefix goes to gout[m][K].
  const int* gcode; int g_rpu, gstride;
  const void* gtable; float gscale;
  float* gout; int ldgo;
};

// Stage x (+ x2) into LDS xs[M][K], applying the RMSNorm prologue if asked.
template <int M, int PRO, typename WL>
__device__ __forceinline__ void stage_x(const GemvArgs& a, int K, float* xs, float (*red)[WAVES]) {
  const int tid = threadIdx.x;
  for (int m = 0; m < M; ++m) {
    const size_t trow = (PRO == PRO_ADDGATHER) ? (size_t)a.gcode[(m / a.g_rpu) * a.gstride] * K : 0;
    for (int k = tid * 4; k < K; k += NT * 4) {
      float4 v = *reinterpret_cast<const float4*>(a.x + (size_t)m * a.ldx + k);
      if (PRO == PRO_ADDNORM || PRO == PRO_ADDGATHER) {
        float4 w = *reinterpret_cast<const float4*>(a.x2 + (size_t)m * a.ldx2 + k);
        if (PRO == PRO_ADDGATHER) {
          w.x = __fadd_rn(w.x, __fmul_rn(WL::get(a.gtable, trow + k), a.gscale));
          w.y = __fadd_rn(w.y, __fmul_rn(WL::get(a.gtable, trow + k + 1), a.gscale));
          w.z = __fadd_rn(w.z, __fmul_rn(WL::get(a.gtable, trow + k + 2), a.gscale));
          w.w = __fadd_rn(w.w, __fmul_rn(WL::get(a.gtable, trow + k + 3), a.gscale));
          if (blockIdx.x == 0) *reinterpret_cast<float4*>(a.gout + (size_t)m * a.ldgo + k) = w;
        }
        v.x = __fadd_rn(v.x, w.x); v.y = __fadd_rn(v.y, w.y); v.z = __fadd_rn(v.z, w.z); v.w = __fadd_rn(v.w, w.w);
      }
      *reinterpret_cast<float4*>(&xs[m * K + k]) = v;
    }
  }
  if (PRO != PRO_NONE) {
    __syncthreads();
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = 0.f;
      for (int k = tid; k < K; k += NT) { const float v = xs[m * K + k]; s += v * v; }
      ss[m] = wave_sum(s);
    }
    if ((tid & 63) == 0) {
#pragma unroll
      for (int m = 0; m < M; ++m) red[m][tid >> 6] = ss[m];
    }
    __syncthreads();
    float inv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) t += red[m][w];
      inv[m] = 1.0f / sqrtf(t / (float)K + a.eps);
    }
    for (int m = 0; m < M; ++m)
      for (int k = tid; k < K; k += NT) {
        const float v = a.norm_w[k] * (xs[m * K + k] * inv[m]);
        xs[m * K + k] = v;
        if (a.norm_out && blockIdx.x == 0) a.norm_out[(size_t)m * a.ldno + k] = v;
      }
  }
  __syncthreads();
}

// Workgroup: 4 waves, each wave owns RPW output rows and streams those rows'
// full K with 16-byte loads; x comes from LDS.  With RMSNorm prologues each
// workgroup normalises the (tiny) input itself, which saves a launch.
// Norm form: w * (x * (1 / sqrt(mean(x^2) + eps))) (Qwen3RMSNorm, nn.RMSNorm).
template <int M, int RPW, int PRO, int EPI, typename WL>
__global__ __launch_bounds__(NT) void gemv_kernel(GemvArgs a) {
  extern __shared__ float smem[];
  float* xs = smem;                 // [M][K]
  __shared__ float red[M][WAVES];
  const int tid = threadIdx.x;
  const int K = a.K;
  stage_x<M, PRO, WL>(a, K, xs, red);

  constexpr int VEC = WL::VEC;
  constexpr int NS = (EPI == EPI_SWIGLU) ? 2 : 1;
  const int wave = tid >> 6, lane = tid & 63;
  const int row0 = (blockIdx.x * WAVES + wave) * RPW;

  const void* wp[RPW][NS];
  size_t woff[RPW][NS];
  bool live[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int n = row0 + r;
    live[r] = n < a.N;
    if (EPI == EPI_SWIGLU) {
      wp[r][0] = a.w[0];
      if (NS > 1) wp[r][NS - 1] = a.w[1];
#pragma unroll
      for (int s = 0; s < NS; ++s) woff[r][s] = (size_t)(live[r] ? n : 0) * K;
    } else {
      int seg = 0, local = live[r] ? n : 0;
      while (seg < 2 && local >= a.seg_rows[seg]) { local -= a.seg_rows[seg]; ++seg; }
      wp[r][0] = a.w[seg];
      woff[r][0] = (size_t)local * K;
    }
  }

  float acc[RPW][NS][M];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][s][m] = 0.f;

#pragma unroll 2
  for (int k = lane * VEC; k < K; k += 64 * VEC) {
    float wv[RPW][NS][VEC];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (live[r]) WL::load(wp[r][s], woff[r][s] + k, wv[r][s]);
        else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) wv[r][s][j] = 0.f;
        }
      }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float xv[VEC];
#pragma unroll
      for (int j = 0; j < VEC; j += 4) {
        const float4 t = *reinterpret_cast<const float4*>(&xs[m * K + k + j]);
        xv[j] = t.x; xv[j + 1] = t.y; xv[j + 2] = t.z; xv[j + 3] = t.w;
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int j = 0; j < VEC; ++j) acc[r][s][m] = fmaf(wv[r][s][j], xv[j], acc[r][s][m]);
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][s][m] = wave_sum(acc[r][s][m]);

  if (lane < M) {
    const int m = lane;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int n = row0 + r;
      if (!live[r]) continue;
      float v = acc[r][0][m];
      if (EPI == EPI_BIAS) v += a.bias[n];
      if (EPI == EPI_RESID) v += a.res[(size_t)m * a.ldr + n];
      if (EPI == EPI_SWIGLU) {
        const float g = v, u = acc[r][NS - 1][m];
        v = g / (1.0f + expf(-g)) * u;
      }
      a.out[(size_t)m * a.ldo + n] = v;
    }
  }
}

// Full-wave sum via DPP (row_shr / row_bcast); the total lands in lane 63
// and is broadcast with readlane.  Fixed order, so replays are bitwise equal.
template <int CTRL, int ROW_MASK, bool BOUND0>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, BOUND0));
}
// Workgroup barrier for LDS: waits for this wave's LDS (and scalar memory)
// operations only.  A fenced __syncthreads also waits for every global load
// the wave has in flight; the samplers and the depth steps share data
// between waves through LDS alone, while their weight loads stay in flight.
__device__ __forceinline__ void sk_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp<0xb1, 0xf, true>(v);    // quad_perm [1,0,3,2]
  v += dpp<0x4e, 0xf, true>(v);    // quad_perm [2,3,0,1]
  v += dpp<0x114, 0xf, true>(v);   // row_shr:4
  v += dpp<0x118, 0xf, true>(v);   // row_shr:8
  v += dpp<0x142, 0xa, false>(v);  // row_bcast:15
  v += dpp<0x143, 0xc, false>(v);  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// GEMV for a compile-time K with no LDS and no barriers.  Each wave owns RW
// output rows (x NS sources for SwiGLU).  It first loads the activations it
// needs straight into registers in its own lane layout (lane l holds
// x[m][(j*64 + l)*VEC ..+VEC) for every j: the whole K across the wave), then
// issues every 16-byte weight load of its rows, so the HBM stream starts
// before any arithmetic and waits only on the (L2-resident) activations.  The
// RMSNorm prologue is computed per wave from those registers with a DPP
// reduction.  Rows past N re-read row N-1 (in bounds) and are discarded.
template <int M, int KT, int RW, int PRO, int EPI, typename WL>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemv_fast_kernel(GemvArgs a) {
  constexpr int VEC = WL::VEC;
  constexpr int NV = KT / (64 * VEC);
  constexpr int NS = (EPI == EPI_SWIGLU) ? 2 : 1;
  static_assert(KT % (64 * VEC) == 0, "K must be a multiple of 64 * VEC");
  // wave index as a scalar, so row and segment selection stay in SGPRs and
  // no weight load waits on a vector-loaded pointer
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int row0 = (blockIdx.x * WAVES + wave) * RW;

  constexpr bool ADD = (PRO == PRO_ADDNORM || PRO == PRO_ADDGATHER);
  // The workgroup's waves share the activations: each thread loads CH
  // consecutive elements of x per chunk (1/NT of it, plus its share of the norm
  // gain, and of x2 for an add prologue) before the weight stream, finishes its
  // chunks once its own loads are in (x2 + table row * scale, then x + x2, the
  // per-element order of the unshared path), stores them to LDS, and after one
  // barrier -- with the weights still in flight -- every wave reads the whole
  // vectors from LDS.  The cache serves x once per workgroup instead of once per
  // wave, and no wave holds x2 or the table rows for the whole K in registers.
  // Capped at 32 KB of LDS: a 48 KB buffer (M = 2, K = 6144) leaves too few
  // workgroups per CU and is slower than per-wave loads.
  constexpr int CH = ADD ? VEC : 4;                                         // elements per chunk
  constexpr bool SHARE = M * KT * 4 <= 32768 && (M * KT) % (NT * CH) == 0;
  constexpr int XQ = SHARE ? (M * KT) / (NT * CH) : 1;                      // chunks of x per thread
  // The gain is loaded up front unless a gathered table row follows the
  // weights anyway (then it is loaded with that row, straight into LDS).
  constexpr bool GEARLY = SHARE && PRO != PRO_NONE && PRO != PRO_ADDGATHER;
  constexpr int GQ = GEARLY ? KT / (NT * 4) : 1;                            // float4 of the gain
  static_assert(!SHARE || PRO == PRO_NONE || KT % (NT * 4) == 0, "shared gain: K a multiple of 1024");
  __shared__ __attribute__((aligned(16))) float xsh[SHARE ? M * KT : 4];
  __shared__ __attribute__((aligned(16))) float gsh[(SHARE && PRO != PRO_NONE) ? KT : 4];
  float xq[XQ][CH], x2q[(SHARE && ADD) ? XQ : 1][CH];
  float4 gq[GQ];
  if constexpr (SHARE) {
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int f = (tid + NT * q) * CH, m = f / KT, k = f % KT;
#pragma unroll
      for (int i = 0; i < CH; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(a.x + (size_t)m * a.ldx + k + i);
        xq[q][i] = t.x; xq[q][i + 1] = t.y; xq[q][i + 2] = t.z; xq[q][i + 3] = t.w;
        if constexpr (ADD) {
          const float4 w = *reinterpret_cast<const float4*>(a.x2 + (size_t)m * a.ldx2 + k + i);
          x2q[q][i] = w.x; x2q[q][i + 1] = w.y; x2q[q][i + 2] = w.z; x2q[q][i + 3] = w.w;
        }
      }
    }
    if constexpr (GEARLY) {
#pragma unroll
      for (int q = 0; q < GQ; ++q) gq[q] = *reinterpret_cast<const float4*>(a.norm_w + (tid + NT * q) * 4);
    }
  }
  // Codes of the gathered table rows first, as vector loads (an opaque zero
  // lane offset keeps them off the scalar path): waiting on them later then
  // never waits on the weight stream issued after them.
  int gc[M];
  if (PRO == PRO_ADDGATHER) {
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
#pragma unroll
    for (int m = 0; m < M; ++m) gc[m] = a.gcode[(m / a.g_rpu) * a.gstride + zero];
  }
  float xv[M][NV][VEC];
  float x2v[(ADD && !SHARE) ? M : 1][(ADD && !SHARE) ? NV : 1][VEC];
  if constexpr (!SHARE) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; i += 4) {
          const size_t k = (size_t)(j * 64 + lane) * VEC + i;
          const float4 t = *reinterpret_cast<const float4*>(a.x + (size_t)m * a.ldx + k);
          xv[m][j][i] = t.x; xv[m][j][i + 1] = t.y; xv[m][j][i + 2] = t.z; xv[m][j][i + 3] = t.w;
          if (ADD) {
            const float4 w = *reinterpret_cast<const float4*>(a.x2 + (size_t)m * a.ldx2 + k);
            x2v[m][j][i] = w.x; x2v[m][j][i + 1] = w.y; x2v[m][j][i + 2] = w.z; x2v[m][j][i + 3] = w.w;
          }
        }
  }

  // Small operands next (norm gains, residual / bias for this lane's
  // outputs), so waiting on them never waits on the weight stream.
  float gw[(PRO != PRO_NONE) ? NV : 1][VEC];
  if (PRO != PRO_NONE && !SHARE) {
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const float4 g = *reinterpret_cast<const float4*>(a.norm_w + (j * 64 + lane) * VEC + i);
        gw[j][i] = g.x; gw[j][i + 1] = g.y; gw[j][i + 2] = g.z; gw[j][i + 3] = g.w;
      }
  }
  float epi[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = min(row0 + r, a.N - 1);
    const int m = lane < M ? lane : 0;
    epi[r] = (EPI == EPI_BIAS) ? a.bias[n] : (EPI == EPI_RESID) ? a.res[(size_t)m * a.ldr + n] : 0.f;
  }

  float wv[RW][NS][NV][VEC];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = min(row0 + r, a.N - 1);
    const void* base[NS];
    size_t off;
    if (EPI == EPI_SWIGLU) {
      base[0] = a.w[0];
      if (NS > 1) base[NS - 1] = a.w[1];
      off = (size_t)n * KT;
    } else {
      const int s0 = a.seg_rows[0], s1 = a.seg_rows[1];
      base[0] = n < s0 ? a.w[0] : (n - s0 < s1 ? a.w[1] : a.w[2]);
      off = (size_t)(n < s0 ? n : (n - s0 < s1 ? n - s0 : n - s0 - s1)) * KT;
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int j = 0; j < NV; ++j) WL::load(base[s], off + (size_t)(j * 64 + lane) * VEC, wv[r][s][j]);
  }

  if constexpr (SHARE) {
    // nothing issued below may be scheduled above the weight stream
    if constexpr (PRO == PRO_ADDGATHER) __builtin_amdgcn_sched_barrier(0);
    // gathered table rows and the gain: every load before the first store
    // (a store may alias them), so they take one round trip together
    constexpr int TQ = (PRO == PRO_ADDGATHER) ? XQ : 1;
    float tq[TQ][CH];
    if constexpr (PRO == PRO_ADDGATHER) {
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const int f = (tid + NT * q) * CH, m = f / KT, k = f % KT;
        int code = gc[0];
#pragma unroll
        for (int mm = 1; mm < M; ++mm) code = (m == mm) ? gc[mm] : code;
        WL::load(a.gtable, (size_t)code * KT + k, tq[q]);
      }
#pragma unroll
      for (int q = 0; q < KT / (NT * 4); ++q)   // LDS cannot alias the global stores below
        *reinterpret_cast<float4*>(&gsh[(tid + NT * q) * 4]) =
            *reinterpret_cast<const float4*>(a.norm_w + (tid + NT * q) * 4);
    }
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int f = (tid + NT * q) * CH, m = f / KT, k = f % KT;
      if constexpr (PRO == PRO_ADDGATHER) {
#pragma unroll
        for (int i = 0; i < CH; ++i) x2q[q][i] = __fadd_rn(x2q[q][i], __fmul_rn(tq[q][i], a.gscale));
        if (blockIdx.x == 0)
#pragma unroll
          for (int i = 0; i < CH; i += 4)
            *reinterpret_cast<float4*>(a.gout + (size_t)m * a.ldgo + k + i) =
                make_float4(x2q[q][i], x2q[q][i + 1], x2q[q][i + 2], x2q[q][i + 3]);
      }
      if constexpr (ADD) {
#pragma unroll
        for (int i = 0; i < CH; ++i) xq[q][i] = __fadd_rn(xq[q][i], x2q[q][i]);
      }
#pragma unroll
      for (int i = 0; i < CH; i += 4)
        *reinterpret_cast<float4*>(&xsh[f + i]) = make_float4(xq[q][i], xq[q][i + 1], xq[q][i + 2], xq[q][i + 3]);
    }
    if constexpr (GEARLY) {
#pragma unroll
      for (int q = 0; q < GQ; ++q) *reinterpret_cast<float4*>(&gsh[(tid + NT * q) * 4]) = gq[q];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; i += 4) {
          const float4 t = *reinterpret_cast<const float4*>(&xsh[m * KT + (j * 64 + lane) * VEC + i]);
          xv[m][j][i] = t.x; xv[m][j][i + 1] = t.y; xv[m][j][i + 2] = t.z; xv[m][j][i + 3] = t.w;
        }
    if constexpr (PRO != PRO_NONE) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; i += 4) {
          const float4 g = *reinterpret_cast<const float4*>(&gsh[(j * 64 + lane) * VEC + i]);
          gw[j][i] = g.x; gw[j][i + 1] = g.y; gw[j][i + 2] = g.z; gw[j][i + 3] = g.w;
        }
    }
  }

  // Unshared: the gathered rows are loaded after the weights (their address
  // waits on the code), and x + x2 is formed only now, so neither holds the
  // weight stream back.
  if constexpr (PRO == PRO_ADDGATHER && !SHARE) {
    float tv[M][NV][VEC];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < NV; ++j) WL::load(a.gtable, (size_t)gc[m] * KT + (size_t)(j * 64 + lane) * VEC, tv[m][j]);
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) x2v[m][j][i] = __fadd_rn(x2v[m][j][i], __fmul_rn(tv[m][j][i], a.gscale));
        if (blockIdx.x == 0 && wave == 0)
#pragma unroll
          for (int i = 0; i < VEC; i += 4)
            *reinterpret_cast<float4*>(a.gout + (size_t)m * a.ldgo + (size_t)(j * 64 + lane) * VEC + i) =
                make_float4(x2v[m][j][i], x2v[m][j][i + 1], x2v[m][j][i + 2], x2v[m][j][i + 3]);
      }
  }
  if constexpr (ADD && !SHARE) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[m][j][i] = __fadd_rn(xv[m][j][i], x2v[m][j][i]);
  }
  if (PRO != PRO_NONE) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) ss = fmaf(xv[m][j][i], xv[m][j][i], ss);
      const float inv = 1.0f / sqrtf(wave_sum_dpp(ss) / (float)KT + a.eps);
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; i += 4) {
          const int k = (j * 64 + lane) * VEC + i;
          xv[m][j][i] = gw[j][i] * (xv[m][j][i] * inv);
          xv[m][j][i + 1] = gw[j][i + 1] * (xv[m][j][i + 1] * inv);
          xv[m][j][i + 2] = gw[j][i + 2] * (xv[m][j][i + 2] * inv);
          xv[m][j][i + 3] = gw[j][i + 3] * (xv[m][j][i + 3] * inv);
          if (a.norm_out && blockIdx.x == 0 && wave == 0)
            *reinterpret_cast<float4*>(a.norm_out + (size_t)m * a.ldno + k) =
                make_float4(xv[m][j][i], xv[m][j][i + 1], xv[m][j][i + 2], xv[m][j][i + 3]);
        }
    }
  }

  float acc[RW][NS][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
          for (int i = 0; i < VEC; ++i) t = fmaf(wv[r][s][j][i], xv[m][j][i], t);
        acc[r][s][m] = wave_sum_dpp(t);
      }

  if (lane < M) {
    const int m = lane;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = row0 + r;
      if (n >= a.N) continue;
      float v = acc[r][0][0];
#pragma unroll
      for (int mm = 1; mm < M; ++mm)
        if (mm == m) v = acc[r][0][mm];
      float u = v;
#pragma unroll
      for (int mm = 0; mm < M; ++mm)
        if (mm == m) u = acc[r][NS - 1][mm];
      if (EPI == EPI_BIAS || EPI == EPI_RESID) v += epi[r];
      if (EPI == EPI_SWIGLU) v = v / (1.0f + expf(-v)) * u;
      a.out[(size_t)m * a.ldo + n] = v;
    }
  }
}

// Residual GEMV with K split over the workgroup's waves (down and output
// projections): wave w multiplies the K slice [w KT/WAVES, (w+1) KT/WAVES) of
// all RG rows of the workgroup, so each wave loads only its slice of the
// activations -- the full-K form loads all of x in every wave, 4x the cache
// traffic and, at large K, more registers than the weight stream leaves.
// The WAVES partial sums of an output are added in wave order after one
// barrier: out[m][n] = res[m][n] + sum_k w[n][k] x[m][k].  Rows past N re-read
// row N-1 (in bounds) and are not stored.
template <int M, int KT, int RG, typename WL>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemv_kslice_kernel(GemvArgs a) {
  constexpr int VEC = WL::VEC;
  constexpr int KS = KT / WAVES;
  constexpr int NV = KS / (64 * VEC);
  static_assert(KT % WAVES == 0 && KS % (64 * VEC) == 0, "K slice must be a multiple of 64 * VEC");
  static_assert(RG * M <= NT, "one epilogue thread per output");
  __shared__ float red[WAVES][RG * M];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n0 = blockIdx.x * RG;
  const int kw = wave * KS;
  // this wave's activation slice, the residual of this thread's output, then
  // every weight load: the stream waits only on the small loads before it
  float xv[M][NV][VEC];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(a.x + (size_t)m * a.ldx + kw + (j * 64 + lane) * VEC + i);
        xv[m][j][i] = t.x; xv[m][j][i + 1] = t.y; xv[m][j][i + 2] = t.z; xv[m][j][i + 3] = t.w;
      }
  const int eo = tid < RG * M ? tid : 0;
  const int er = eo / M, em = eo % M;
  const int en = min(n0 + er, a.N - 1);
  const float resv = a.res[(size_t)em * a.ldr + en];
  float wv[RG][NV][VEC];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const size_t off = (size_t)min(n0 + r, a.N - 1) * KT + kw;
#pragma unroll
    for (int j = 0; j < NV; ++j) WL::load(a.w[0], off + (size_t)(j * 64 + lane) * VEC, wv[r][j]);
  }
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) t = fmaf(wv[r][j][i], xv[m][j][i], t);
      t = wave_sum_dpp(t);
      if (lane == 0) red[wave][r * M + m] = t;
    }
  __syncthreads();
  if (tid < RG * M && n0 + er < a.N) {
    float sum = red[0][tid];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += red[w][tid];
    a.out[(size_t)em * a.ldo + n0 + er] = sum + resv;
  }
}

// ------------------------------------------------------------ RMSNorm rows
// out[b] = w * (x[b] (+ x2[b]) * 1/sqrt(mean(.^2) + eps)); grid = rows.
// Rows with active[b] == 0 are left untouched (prefill of ragged rows).
__global__ __launch_bounds__(NT) void rmsnorm_rows_kernel(const float* x, const float* x2,
                                                          const float* w, float eps, int D,
                                                          float* out, const int* active) {
  __shared__ float red[WAVES];
  const int b = blockIdx.x;
  if (active && !active[b]) return;
  const float* xr = x + (size_t)b * D;
  const float* x2r = x2 ? x2 + (size_t)b * D : nullptr;
  float s = 0.f;
  for (int k = threadIdx.x; k < D; k += NT) {
    const float v = x2r ? xr[k] + x2r[k] : xr[k];
    s += v * v;
  }
  const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
  for (int k = threadIdx.x; k < D; k += NT) {
    const float v = x2r ? xr[k] + x2r[k] : xr[k];
    out[(size_t)b * D + k] = w[k] * (v * inv);
  }
}

// ------------------------------------------------------------ split activations
// Split form of a GEMM input x [rows <= 32][K] for the BF16 matrix cores:
// for each 32-k block, row tile t (rows 16t .. 16t+15) and half (hi, lo), the
// 64 lanes' B fragments of v_mfma_f32_16x16x32_bf16, 8 BF16 each (lane 16q+i:
// row 16t+i, k = 32*block + 8q .. 8q+7), 1 KiB per (block, t, half).  x_hi =
// bf16(x g), x_lo = bf16(x g - x_hi), with g the consumer's RMSNorm gain (1
// without): the pair keeps ~16 mantissa bits of x g.  The kernel that produces
// x writes it, so a consumer's workgroups load ready fragments instead of
// each re-reading FP32 x and splitting it again.
constexpr int XS_ROWS = 32;
__host__ __device__ constexpr size_t xsplit_elems(int K) { return (size_t)K * XS_ROWS * 2; }
__device__ __forceinline__ size_t xsplit_index(int r, int k) {   // hi half; lo at + 512
  return ((size_t)(k >> 5) * 2 + (r >> 4)) * 1024 + (size_t)(16 * ((k & 31) >> 3) + (r & 15)) * 8 + (k & 7);
}
__device__ __forceinline__ void xsplit_store(uint16_t* xs, int r, int k, float v) {
  const __bf16 hi = (__bf16)v;
  const __bf16 lo = (__bf16)(v - (float)hi);
  const size_t i = xsplit_index(r, k);
  xs[i] = __builtin_bit_cast(uint16_t, hi);
  xs[i + 512] = __builtin_bit_cast(uint16_t, lo);
}

// ------------------------------------------------------------ attention
// One decode token per row against that row's own cache (per-row length and
// RoPE position; CFG rows differ in length).  Grid (chunks, Hkv, rows); the
// workgroup of chunk c handles KV tokens [c*32, c*32+32).
//
// Round trips are what cost here, so a workgroup issues every load that does
// not depend on the row's length at entry: its raw q/k/v, norm gains and RoPE
// frequencies first, then the K and V rows of its whole chunk (16 dims of one
// token per lane).  The chunk rows are read speculatively (the cache is
// allocated to max_ctx, so they are in bounds); tokens at or past the row's
// length are masked once kv_len arrives.  Queries and the new key get Qwen3's
// per-head RMSNorm then rotate-half RoPE with the row's (cos, sin) table
// (rope_cs, written when the position last moved).  The workgroup owning the new
// token appends it to the cache.  Partial (max, sum, o) per chunk go to
// scratch, merged by attention_combine_kernel.
struct AttnArgs {
  const float* qkv; int ldqkv;           // [rows][(Hq + 2 Hkv) hd] raw projections
  void* kc; void* vc;                    // this layer: [rows][Hkv][max_ctx][hd], FP32 or BF16
  const float* qn_w; const float* kn_w; float eps;
  const float2* rope;                    // [rows][hd/2] (cos, sin) at the row's position
  const int* kv_len; const int* active;
  float* part;                           // [rows][Hq][max_chunks][part_stride(hd)]: o[hd], max, sum
  float* out; int ldo;                   // [rows][Hq hd]
  int Hq, Hkv, hd, max_ctx, max_chunks;
  float scale;
  int nparts;                            // > 0: partials per (row, q head) to merge (stream kernel splits)
  int row_chunks[4];                     // attn_o_kernel: an upper bound on each row's chunk count
                                         // (the host's count for the frame; >= the row's own)
  uint16_t* xs_out;                      // output again in split form (null: none)
};

constexpr int ATT_DPL = 16;      // head dims per lane
// Floats per chunk partial: the hd outputs, the chunk's max and sum, padded
// so every partial starts 16-byte aligned (hd is a multiple of 16).
__host__ __device__ constexpr int part_stride(int hd) { return hd + 4; }

__host__ __device__ constexpr size_t attn_smem_floats(int G, int hd) {
  return ((size_t)G * hd + 4 * (size_t)hd + 3 * (size_t)(hd / 2) + (size_t)G * ATT_CHUNK + (size_t)G * 2 + 3) /
             4 * 4 +
         (size_t)ATT_CHUNK * hd;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_keep(float v) {   // disabled lanes keep v
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_keep<0xb1, 0xf>(v));
  v = fmaxf(v, dpp_keep<0x4e, 0xf>(v));
  v = fmaxf(v, dpp_keep<0x114, 0xf>(v));
  v = fmaxf(v, dpp_keep<0x118, 0xf>(v));
  v = fmaxf(v, dpp_keep<0x142, 0xa>(v));
  v = fmaxf(v, dpp_keep<0x143, 0xc>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Sum over each aligned group of `lpt` lanes (1..16); valid in the group's
// first lane.
__device__ __forceinline__ float group_sum_first(float v, int lpt) {
  if (lpt >= 2) v += dpp<0xb1, 0xf, true>(v);   // quad_perm [1,0,3,2]
  if (lpt >= 4) v += dpp<0x4e, 0xf, true>(v);   // quad_perm [2,3,0,1]
  if (lpt >= 8) v += dpp<0x12c, 0xf, true>(v);  // row_ror:12 (lane i reads lane i+4 of its row)
  if (lpt >= 16) v += dpp<0x128, 0xf, true>(v); // row_ror:8  (lane i reads lane i+8 of its row)
  return v;
}

// Grid (chunks, Hkv, rows); the workgroup of chunk c handles KV tokens
// [c*32, c*32+32) of one (row, kv head) and writes that chunk's (o, max, sum)
// for the G query heads; attention_combine_kernel merges the chunks.  Every
// load that does not depend on the row's length is issued at entry: raw
// q/k/v, norm gains, RoPE frequencies, then the chunk's K and V rows (16 dims
// of one token per lane; in bounds because the cache is allocated to max_ctx)
// -- tokens at or past the length are masked once kv_len arrives.  Queries
// and the new key get Qwen3's per-head RMSNorm then rotate-half RoPE with
// angle = fp32(pos * inv_freq) and cos/sin evaluated in double, rounded once;
// the workgroup owning the new token appends its K/V to the cache.
// FP32 -> BF16 bits, round to nearest even (the KV cache's BF16 storage).
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(bf16_bits(x) << 16); }

// KT: element type of the KV cache, float or uint16_t (BF16 bits).
template <typename KT>
__global__ __launch_bounds__(NT) void attention_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int c = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  const int G = a.Hq / a.Hkv, hd = a.hd, half = hd / 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t_begin = c * ATT_CHUNK;
  const size_t head_base = ((size_t)r * a.Hkv + h) * a.max_ctx;

  float* qs = sm;                        // [G][hd]
  float* knew = qs + G * hd;             // [hd]
  float* vnew = knew + hd;               // [hd]
  float* qw = vnew + hd;                 // [hd] q_norm gain
  float* kw = qw + hd;                   // [hd] k_norm gain
  float* fq = kw + hd;                   // [hd/2] inv_freq
  float* fcs = fq + half;                // [hd/2] cos
  float* fsn = fcs + half;               // [hd/2] sin
  float* sc = fsn + half;                // [G][CHUNK]
  float* st = sc + G * ATT_CHUNK;        // [G][2]
  float* vs = sm + attn_smem_floats(G, hd) - (size_t)ATT_CHUNK * hd;  // [CHUNK][hd]

  const int T = a.kv_len[r];
  const int act = a.active[r];
  // Every load goes to registers first (one element per thread: G*hd <= NT
  // and hd <= NT), then the chunk's K/V rows; LDS is written only once all of
  // them are in flight, so no load waits behind another's round trip.
  const float* row = a.qkv + (size_t)r * a.ldqkv;
  // Indices clamped instead of branched: with no branch around them the
  // compiler issues these loads, and the argument loads they need, together.
  const int tq = min(tid, G * hd - 1), th = min(tid, hd - 1), tr = min(tid, half - 1);
  const float q_r = row[(size_t)h * G * hd + tq];
  const float kn_r = row[(size_t)a.Hq * hd + (size_t)h * hd + th];
  const float vn_r = row[(size_t)(a.Hq + a.Hkv) * hd + (size_t)h * hd + th];
  const float qw_r = a.qn_w[th];
  const float kw_r = a.kn_w[th];
  const float2 cs_r = a.rope[(size_t)r * half + tr];

  const int LPT = hd / ATT_DPL;
  const int TPP = NT / LPT;              // tokens per pass
  const int npass = (ATT_CHUNK + TPP - 1) / TPP;
  const int sub = tid % LPT, tok = tid / LPT;
  constexpr bool KBF = sizeof(KT) == 2;
  constexpr int NLD = ATT_DPL * (int)sizeof(KT) / 16;   // 16-byte loads per row slice
  uint4 kraw[NLD], vraw[NLD];
  // Unconditional (token index clamped into the cache), so the compiler can
  // count these loads exactly and wait on the small ones above separately.
  auto load_tok = [&](int pass) {
    const int tl = min(pass * TPP + tok, ATT_CHUNK - 1);
    const int t = min(t_begin + tl, a.max_ctx - 1);
    const uint4* kp = reinterpret_cast<const uint4*>(static_cast<const KT*>(a.kc) + (head_base + t) * hd + sub * ATT_DPL);
    const uint4* vp = reinterpret_cast<const uint4*>(static_cast<const KT*>(a.vc) + (head_base + t) * hd + sub * ATT_DPL);
#pragma unroll
    for (int i = 0; i < NLD; ++i) { kraw[i] = kp[i]; vraw[i] = vp[i]; }
  };
  // raw cache words -> 16 FP32 values
  auto widen = [&](const uint4 (&raw)[NLD], float4 (&out)[ATT_DPL / 4]) {
    if constexpr (KBF) {
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
        for (int j = 0; j < 2; ++j)
          out[2 * i + j] = make_float4(__uint_as_float(w[2 * j] << 16), __uint_as_float(w[2 * j] & 0xffff0000u),
                                       __uint_as_float(w[2 * j + 1] << 16), __uint_as_float(w[2 * j + 1] & 0xffff0000u));
      }
    } else {
#pragma unroll
      for (int i = 0; i < NLD; ++i)
        out[i] = make_float4(__uint_as_float(raw[i].x), __uint_as_float(raw[i].y), __uint_as_float(raw[i].z),
                             __uint_as_float(raw[i].w));
    }
  };
  load_tok(0);
  // Keep the chunk's K/V loads above the exit test below: sunk past it, they
  // waited for kv_len and active to arrive first.
  asm volatile("" ::: "memory");
  const int ctx = T + 1;
  const int nch = (ctx + ATT_CHUNK - 1) / ATT_CHUNK;
  if (!act || c >= nch) return;
  const bool last = (c == nch - 1);
  const int n_t = min(ATT_CHUNK, ctx - t_begin);
  if (tid < G * hd) qs[tid] = q_r;
  if (tid < hd) { knew[tid] = kn_r; vnew[tid] = vn_r; qw[tid] = qw_r; kw[tid] = kw_r; }
  if (tid < half) { fcs[tid] = cs_r.x; fsn[tid] = cs_r.y; }
  __syncthreads();
  // Per-head RMSNorm over hd, then rotate-half RoPE; one wave per head.
  const int nheads = G + (last ? 1 : 0);
  for (int j = wave; j < nheads; j += WAVES) {
    float* v = (j < G) ? qs + j * hd : knew;
    const float* w = (j < G) ? qw : kw;
    float s = 0.f;
    for (int d = lane; d < hd; d += 64) s += v[d] * v[d];
    const float inv = 1.0f / sqrtf(wave_sum_dpp(s) / (float)hd + a.eps);
    for (int d = lane; d < half; d += 64) {
      const float x1 = w[d] * (v[d] * inv);
      const float x2 = w[d + half] * (v[d + half] * inv);
      v[d] = x1 * fcs[d] - x2 * fsn[d];
      v[d + half] = x2 * fcs[d] + x1 * fsn[d];
    }
  }
  __syncthreads();
  // Append the new token.  A BF16 cache stores it rounded, and this step then
  // attends to the rounded values too, as every later step will.
  if (last) {
    for (int d = tid; d < hd; d += NT) {
      if constexpr (KBF) {
        static_cast<KT*>(a.kc)[(head_base + T) * hd + d] = (KT)bf16_bits(knew[d]);
        static_cast<KT*>(a.vc)[(head_base + T) * hd + d] = (KT)bf16_bits(vnew[d]);
      } else {
        static_cast<KT*>(a.kc)[(head_base + T) * hd + d] = knew[d];
        static_cast<KT*>(a.vc)[(head_base + T) * hd + d] = vnew[d];
      }
    }
    if constexpr (KBF) {
      for (int d = tid; d < hd; d += NT) { knew[d] = bf16_round(knew[d]); vnew[d] = bf16_round(vnew[d]); }
      __syncthreads();                   // `last` is uniform over the workgroup
    }
  }

  for (int pass = 0; pass < npass; ++pass) {
    const int tl = pass * TPP + tok;
    const int t = t_begin + tl;
    if (pass > 0) load_tok(pass);
    float4 kr[ATT_DPL / 4], vr[ATT_DPL / 4];
    widen(kraw, kr);
    widen(vraw, vr);
    if (tl < n_t && t == T) {
#pragma unroll
      for (int i = 0; i < ATT_DPL / 4; ++i) {
        const int d = sub * ATT_DPL + 4 * i;
        kr[i] = make_float4(knew[d], knew[d + 1], knew[d + 2], knew[d + 3]);
        vr[i] = make_float4(vnew[d], vnew[d + 1], vnew[d + 2], vnew[d + 3]);
      }
    }
    for (int g = 0; g < G; ++g) {
      const float* qg = qs + g * hd + sub * ATT_DPL;
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < ATT_DPL / 4; ++i) {
        s = fmaf(qg[4 * i], kr[i].x, s);
        s = fmaf(qg[4 * i + 1], kr[i].y, s);
        s = fmaf(qg[4 * i + 2], kr[i].z, s);
        s = fmaf(qg[4 * i + 3], kr[i].w, s);
      }
      s = group_sum_first(s, LPT);
      if (sub == 0 && tl < n_t) sc[g * ATT_CHUNK + tl] = s * a.scale;
    }
    if (tl < ATT_CHUNK) {
      float4* vd = reinterpret_cast<float4*>(vs + (size_t)tl * hd + sub * ATT_DPL);
      const bool ok = tl < n_t;
#pragma unroll
      for (int i = 0; i < ATT_DPL / 4; ++i) vd[i] = ok ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __syncthreads();
  // Chunk softmax statistics: one wave per q head, one lane per token.
  for (int g = wave; g < G; g += WAVES) {
    const float v = (lane < n_t) ? sc[g * ATT_CHUNK + lane] : -INFINITY;
    const float m = wave_max_dpp(v);
    const float e = (lane < n_t) ? expf(v - m) : 0.f;
    const float l = wave_sum_dpp(e);
    if (lane < ATT_CHUNK) sc[g * ATT_CHUNK + lane] = e;
    if (lane == 0) { st[2 * g] = m; st[2 * g + 1] = l; }
  }
  __syncthreads();
  const int stride = part_stride(hd);
  for (int i = tid; i < G * hd; i += NT) {
    const int g = i / hd, d = i - g * hd;
    const float* eg = sc + g * ATT_CHUNK;
    float o = 0.f;
#pragma unroll 8
    for (int tl = 0; tl < ATT_CHUNK; ++tl) o = fmaf(eg[tl], vs[(size_t)tl * hd + d], o);
    float* pp = a.part + (((size_t)r * a.Hq + h * G + g) * a.max_chunks + c) * stride;
    pp[d] = o;
    if (d == 0) { pp[hd] = st[2 * g]; pp[hd + 1] = st[2 * g + 1]; }
  }
}

// One block of up to MERGE_CB chunks [c0, c0 + MERGE_CB) of one (row, q head,
// dim): the running (M, L, O) are rescaled to the block's max, then the
// block's chunks are added in chunk order.  Both merge forms use it, so they
// round identically.
constexpr int MERGE_CB = 16;
__device__ __forceinline__ void merge_block(const float (&mv)[MERGE_CB], const float (&lv)[MERGE_CB],
                                            const float (&ov)[MERGE_CB], int c0, int nch, float& M, float& L,
                                            float& O) {
  float Mb = M;
#pragma unroll
  for (int j = 0; j < MERGE_CB; ++j)
    if (c0 + j < nch) Mb = fmaxf(Mb, mv[j]);
  const float rescale = expf(M - Mb);   // 0 on the first block (M = -inf)
  L *= rescale;
  O *= rescale;
#pragma unroll
  for (int j = 0; j < MERGE_CB; ++j)
    if (c0 + j < nch) {
      const float f = expf(mv[j] - Mb);
      L = fmaf(lv[j], f, L);
      O = fmaf(ov[j], f, O);
    }
  M = Mb;
}

// Merge the chunk partials of one (row, q head) in chunk order: one thread
// per head dim.  The partials of up to 16 chunks are loaded together with
// kv_len (speculatively, in bounds) and masked once the chunk count is known.
// A kernel of its own, so the partials need no device-scope fence.
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a) {
  const int hq = blockIdx.x, r = blockIdx.y, d = threadIdx.x;
  const int hd = a.hd, stride = part_stride(hd);
  const int dd = min(d, hd - 1);         // lanes past hd mirror the last dim, no branch
  const float* pp = a.part + ((size_t)r * a.Hq + hq) * a.max_chunks * stride;
  constexpr int CB = MERGE_CB;
  float mv[CB], lv[CB], ov[CB];
  auto load_block = [&](int c0) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int cc = min(c0 + j, a.max_chunks - 1);
      mv[j] = pp[cc * stride + hd];
      lv[j] = pp[cc * stride + hd + 1];
      ov[j] = pp[cc * stride + dd];
    }
  };
  // Row length and state first: issued ahead of the partials, they arrive
  // with them instead of costing a round trip of their own afterwards.
  const int kvl = a.kv_len[r];
  const int act = a.active[r];
  load_block(0);
  asm volatile("" ::: "memory");
  const int nch = a.nparts > 0 ? a.nparts : (kvl + 1 + ATT_CHUNK - 1) / ATT_CHUNK;
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int c0 = 0; c0 < nch; c0 += CB) {
    if (c0 > 0) load_block(c0);
    merge_block(mv, lv, ov, c0, nch, M, L, O);
  }
  if (act && d < hd) {
    a.out[(size_t)r * a.ldo + (size_t)hq * hd + d] = O / L;
    if (a.xs_out) xsplit_store(a.xs_out, r, hq * hd + d, O / L);
  }
}

// Output projection with the chunk merge of attention_kernel in its prologue
// (few decode rows), in place of attention_combine_kernel + a residual GEMV:
// out[m][n] = res[m][n] + sum_k W[n][k] attn[m][k].  A workgroup issues its
// weight rows' loads, then the first AO_CB chunk partials (o, max, sum) of
// the (row, query head) each thread merges -- VPTH consecutive outputs --
// with the chunk index clamped to the row's chunk count from the launch
// arguments (at.row_chunks, set by the host), so these loads wait on no
// memory round trip; the row's length, loaded beside them, then gives the
// exact count that masks the merge and bounds the later blocks (a bound
// below it would reload the first block).  (Bounding the first block by the largest row's count
// instead read colder lines for the shorter row: 1.5 us slower per launch.)  The merge is in chunk order with a running max and rescale;
// attn = O / L goes to LDS, and after one barrier the waves multiply.
// Every workgroup re-reads the partials of all rows and heads, and each load
// instruction costs its CU's load pipe even when it hits in L1, so blocks are
// small (16 measured 2.5 us slower per launch) and the grid is small: one
// output row per wave, 8 waves.  Inactive rows read zeros.
constexpr int AO_NT = 512;
constexpr int AO_CB = 8;                     // chunks per merge block
template <int M, int KT, int RW, typename WL>
__global__ __launch_bounds__(AO_NT) __attribute__((amdgpu_waves_per_eu(1, 2))) void attn_o_kernel(GemvArgs g,
                                                                                                  AttnArgs at) {
  constexpr int VEC = WL::VEC;
  constexpr int NV = KT / (64 * VEC);
  constexpr int NW = AO_NT / 64;
  constexpr int VPTH = M * KT / AO_NT;          // merged outputs per thread
  constexpr int CB = AO_CB;
  static_assert(KT % (64 * VEC) == 0 && (M * KT) % AO_NT == 0 && VPTH % 4 == 0, "attn_o_kernel shape");
  __shared__ __attribute__((aligned(16))) float xsh[M * KT];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int row0 = (blockIdx.x * NW + wave) * RW;

  const int f = tid * VPTH, m = f / KT, k = f - m * KT, head = k / at.hd, d0 = k - head * at.hd;
  const int kvl = at.kv_len[m], act = at.active[m];
  const int rc = max(1, at.row_chunks[m]);
  float epi[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = min(row0 + r, g.N - 1);
    epi[r] = g.res[(size_t)(lane < M ? lane : 0) * g.ldr + n];
  }
  float wv[RW][NV][VEC];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const size_t off = (size_t)min(row0 + r, g.N - 1) * KT;
#pragma unroll
    for (int j = 0; j < NV; ++j) WL::load(g.w[0], off + (size_t)(j * 64 + lane) * VEC, wv[r][j]);
  }
  const int stride = part_stride(at.hd);
  const float* pp = at.part + ((size_t)m * at.Hq + head) * at.max_chunks * stride;
  float2 ml[CB];
  float4 ov[CB][VPTH / 4];
  auto load_block = [&](int c0, int bound) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {            // past the bound: re-read its last chunk
      const float* pc = pp + (size_t)min(c0 + j, bound - 1) * stride;
      ml[j] = *reinterpret_cast<const float2*>(pc + at.hd);
#pragma unroll
      for (int i = 0; i < VPTH / 4; ++i) ov[j][i] = *reinterpret_cast<const float4*>(pc + d0 + 4 * i);
    }
  };
  load_block(0, rc);
  const int nch = act ? (kvl + 1 + ATT_CHUNK - 1) / ATT_CHUNK : 0;
  if (nch > rc) load_block(0, nch);           // a bound below the row's count: reload (never expected)
  float Mr = -INFINITY, L = 0.f, O[VPTH];
#pragma unroll
  for (int v = 0; v < VPTH; ++v) O[v] = 0.f;
  for (int c0 = 0; c0 < nch; c0 += CB) {
    if (c0 > 0) load_block(c0, nch);
    float Mb = Mr;
#pragma unroll
    for (int j = 0; j < CB; ++j)
      if (c0 + j < nch) Mb = fmaxf(Mb, ml[j].x);
    const float sc = expf(Mr - Mb);           // 0 on the first block (Mr = -inf)
    L *= sc;
#pragma unroll
    for (int v = 0; v < VPTH; ++v) O[v] *= sc;
#pragma unroll
    for (int j = 0; j < CB; ++j)
      if (c0 + j < nch) {
        const float e = expf(ml[j].x - Mb);
        L = fmaf(ml[j].y, e, L);
#pragma unroll
        for (int i = 0; i < VPTH / 4; ++i) {
          O[4 * i] = fmaf(ov[j][i].x, e, O[4 * i]);
          O[4 * i + 1] = fmaf(ov[j][i].y, e, O[4 * i + 1]);
          O[4 * i + 2] = fmaf(ov[j][i].z, e, O[4 * i + 2]);
          O[4 * i + 3] = fmaf(ov[j][i].w, e, O[4 * i + 3]);
        }
      }
    Mr = Mb;
  }
#pragma unroll
  for (int i = 0; i < VPTH / 4; ++i)
    *reinterpret_cast<float4*>(&xsh[f + 4 * i]) =
        nch ? make_float4(O[4 * i] / L, O[4 * i + 1] / L, O[4 * i + 2] / L, O[4 * i + 3] / L)
            : make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();

  float acc[RW][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;
#pragma unroll
  for (int mm = 0; mm < M; ++mm)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float xv[VEC];
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(&xsh[mm * KT + (j * 64 + lane) * VEC + i]);
        xv[i] = t.x; xv[i + 1] = t.y; xv[i + 2] = t.z; xv[i + 3] = t.w;
      }
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[r][mm] = fmaf(wv[r][j][i], xv[i], acc[r][mm]);
    }
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int mm = 0; mm < M; ++mm) acc[r][mm] = wave_sum_dpp(acc[r][mm]);
  if (lane < M) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = row0 + r;
      if (n >= g.N) continue;
      float v = acc[r][0];
#pragma unroll
      for (int mm = 1; mm < M; ++mm)
        if (mm == lane) v = acc[r][mm];
      g.out[(size_t)lane * g.ldo + n] = v + epi[r];
    }
  }
}

// ------------------------------------------------------------ many-row attention
// All-reduce over each aligned group of n lanes (n = 1, 2, 4, 8, 16); every
// lane of the group gets the same bits (each step adds a commutative pair).
__device__ __forceinline__ float group_allsum(float v, int n) {
  if (n >= 2) v += dpp_keep<0xb1, 0xf>(v);    // quad_perm [1,0,3,2]
  if (n >= 4) v += dpp_keep<0x4e, 0xf>(v);    // quad_perm [2,3,0,1]
  if (n >= 8) v += dpp_keep<0x141, 0xf>(v);   // row_half_mirror: lane i <-> 7 - i
  if (n >= 16) v += dpp_keep<0x140, 0xf>(v);  // row_mirror: lane i <-> 15 - i
  return v;
}
// The same groups' maximum.
__device__ __forceinline__ float group_allmax(float v, int n) {
  if (n >= 2) v = fmaxf(v, dpp_keep<0xb1, 0xf>(v));
  if (n >= 4) v = fmaxf(v, dpp_keep<0x4e, 0xf>(v));
  if (n >= 8) v = fmaxf(v, dpp_keep<0x141, 0xf>(v));
  if (n >= 16) v = fmaxf(v, dpp_keep<0x140, 0xf>(v));
  return v;
}

// Two online-softmax states (max, sum, output) of one query head -> one.
// An empty state has max -inf and contributes nothing.
__device__ __forceinline__ float merge_weight(float m, float M) { return m == -INFINITY ? 0.f : expf(m - M); }

// smem floats of attention_stream_kernel
__host__ __device__ constexpr size_t attn_stream_smem_floats(int G, int hd, int nth) {
  return (size_t)G * hd + 4 * (size_t)hd + (size_t)hd + (size_t)(nth / 64) * G * (hd + 2);
}

// Decode attention for many rows.  Grid (S, Hkv, rows), NTH threads.  A group
// of LPT = hd/16 lanes (a slot) holds one token at a time, 16 dims per lane; slot
// `slot` of split s reads the tokens t = s*TPP + slot + j*S*TPP, j = 0, 1, ...
// (TPP = NTH/LPT slots), so each load instruction of a workgroup covers TPP
// consecutive cache rows.  Every slot runs its own online softmax over its
// tokens (running max, sum and 16 output dims per query head, all in
// registers): the loop has no LDS traffic and no barrier, and D tokens are in
// flight per slot.  The slots are merged once at the end, across lanes by
// shuffles and across waves in LDS.  Queries and the new key get Qwen3's
// per-head RMSNorm then rotate-half RoPE (as attention_kernel); the split that
// owns token T appends the new K/V and attends to it from registers.
// S == 1 writes the attention output; S > 1 writes one partial (o, max, sum)
// per split in the chunk-partial layout for attention_combine_kernel
// (nparts = S).  Requires G*hd <= NTH.
template <typename KT, int G, int NTH, int D>
__global__ __launch_bounds__(NTH) void attention_stream_kernel(AttnArgs a, int S) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  constexpr int NW = NTH / 64;
  const int s = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  const int hd = a.hd, half = hd / 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int LPT = hd / ATT_DPL, TPP = NTH / LPT;
  const int sub = tid % LPT, slot = tid / LPT;
  const size_t head_base = ((size_t)r * a.Hkv + h) * a.max_ctx;
  const int t0 = s * TPP + slot, tstep = S * TPP;

  float* qs = sm;                        // [G][hd]
  float* knew = qs + G * hd;             // [hd]
  float* vnew = knew + hd;               // [hd]
  float* qw = vnew + hd;                 // [hd]
  float* kw = qw + hd;                   // [hd]
  float* fcs = kw + hd;                  // [hd/2]
  float* fsn = fcs + half;               // [hd/2]
  float* mo = fsn + half;                // [NW][G][hd] merged outputs
  float* mls = mo + (size_t)NW * G * hd; // [NW][G][2] merged (max, sum)

  constexpr bool KBF = sizeof(KT) == 2;
  constexpr int EPV = 16 / (int)sizeof(KT);    // cache elements per 16-byte load
  constexpr int NLD = ATT_DPL / EPV;           // loads per token and lane
  // Load i of a slot covers 16-byte pieces i*LPT .. i*LPT+LPT-1 of the row, so
  // each load instruction reads whole cache lines; the lane's register e holds
  // head dim dim_of(e).
  auto dim_of = [&](int e) { return ((e / EPV) * LPT + sub) * EPV + e % EPV; };
  struct Tok { uint4 k[NLD], v[NLD]; };
  int t_last = 0;                        // last cached row of this (row, kv head)
  auto load = [&](int j, Tok& b) {       // token index clamped into the cache: always in bounds
    const int t = min(t0 + j * tstep, t_last);
    const uint4* kp = reinterpret_cast<const uint4*>(static_cast<const KT*>(a.kc) + (head_base + t) * hd) + sub;
    const uint4* vp = reinterpret_cast<const uint4*>(static_cast<const KT*>(a.vc) + (head_base + t) * hd) + sub;
#pragma unroll
    for (int i = 0; i < NLD; ++i) { b.k[i] = kp[i * LPT]; b.v[i] = vp[i * LPT]; }
  };
  auto widen = [&](const uint4 (&raw)[NLD], float (&out)[ATT_DPL]) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (KBF) {
          out[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
          out[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        } else {
          out[4 * i + j] = __uint_as_float(w[j]);
        }
      }
    }
  };

  // Issue order, kept by compiler barriers: the row's length and state, the
  // raw q / k / v of this head, norm gains and RoPE entry (indices clamped
  // instead of branched, so they go as one batch), then the first D tokens
  // of every slot, clamped to the last cached row so that no row past the
  // context is fetched (the new token T comes from registers).  All are
  // vector loads, which retire in order: the stream waits for the length
  // alone, and the exit test for the state alone.  (Scalar loads of the
  // length would make the q loads wait for it: the compiler can only wait for
  // all outstanding scalar loads at once.)  The exit test must not move above
  // the stream: hoisted, it put the row's state and a second round of
  // argument loads in front of it.
  asm volatile("" ::: "memory");
  const int T_raw = a.kv_len[r];
  const int act = a.active[r];
  const float* row = a.qkv + (size_t)r * a.ldqkv;
  const int tq = min(tid, G * hd - 1), th = min(tid, hd - 1), tr = min(tid, half - 1);
  const float q_r = row[(size_t)h * G * hd + tq];
  const float kn_r = row[(size_t)a.Hq * hd + (size_t)h * hd + th];
  const float vn_r = row[(size_t)(a.Hq + a.Hkv) * hd + (size_t)h * hd + th];
  const float qw_r = a.qn_w[th];
  const float kw_r = a.kn_w[th];
  const float2 cs_r = a.rope[(size_t)r * half + tr];
  __builtin_amdgcn_sched_barrier(0);
  const int T = __builtin_amdgcn_readfirstlane(T_raw);
  t_last = max(min(T, a.max_ctx) - 1, 0);
  Tok ring[D];
#pragma unroll
  for (int u = 0; u < D; ++u) load(u, ring[u]);
  asm volatile("" ::: "memory");
  if (!act) return;
  const int ctx = T + 1;
  const int n_iter = ctx > s * TPP ? (ctx - s * TPP + tstep - 1) / tstep : 0;
  const bool owner = ((T / TPP) % S) == s;
  if (tid < G * hd) qs[tid] = q_r;
  if (tid < hd) { knew[tid] = kn_r; vnew[tid] = vn_r; qw[tid] = qw_r; kw[tid] = kw_r; }
  if (tid < half) { fcs[tid] = cs_r.x; fsn[tid] = cs_r.y; }
  __syncthreads();
  const int nheads = G + (owner ? 1 : 0);
  for (int j = wave; j < nheads; j += NW) {
    float* v = (j < G) ? qs + j * hd : knew;
    const float* w = (j < G) ? qw : kw;
    float ss = 0.f;
    for (int d = lane; d < hd; d += 64) ss += v[d] * v[d];
    const float inv = 1.0f / sqrtf(wave_sum_dpp(ss) / (float)hd + a.eps);
    for (int d = lane; d < half; d += 64) {
      const float x1 = w[d] * (v[d] * inv);
      const float x2 = w[d + half] * (v[d + half] * inv);
      v[d] = x1 * fcs[d] - x2 * fsn[d];
      v[d + half] = x2 * fcs[d] + x1 * fsn[d];
    }
  }
  __syncthreads();
  // Append the new token.  A BF16 cache stores it rounded, and this step then
  // attends to the rounded values too, as every later step will.
  if (owner) {
    for (int d = tid; d < hd; d += NTH) {
      if constexpr (KBF) {
        static_cast<KT*>(a.kc)[(head_base + T) * hd + d] = (KT)bf16_bits(knew[d]);
        static_cast<KT*>(a.vc)[(head_base + T) * hd + d] = (KT)bf16_bits(vnew[d]);
      } else {
        static_cast<KT*>(a.kc)[(head_base + T) * hd + d] = knew[d];
        static_cast<KT*>(a.vc)[(head_base + T) * hd + d] = vnew[d];
      }
    }
    if constexpr (KBF) {
      for (int d = tid; d < hd; d += NTH) { knew[d] = bf16_round(knew[d]); vnew[d] = bf16_round(vnew[d]); }
      __syncthreads();                   // `owner` is uniform over the workgroup
    }
  }
  float q[G][ATT_DPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < ATT_DPL; ++i) q[g][i] = qs[g * hd + dim_of(i)];

  float m[G], l[G], o[G][ATT_DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY; l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < ATT_DPL; ++i) o[g][i] = 0.f;
  }
  // The trip count is padded to a multiple of D, and every iteration consumes
  // one ring entry and refills it after its last use with an unconditional
  // load (clamped; the last round's refills are not used).  Conditional
  // refills left the compiler unsure which loads were in flight, and it then
  // waited for all of them before each token.  Tokens past the context are
  // masked.
  const int n_pad = (n_iter + D - 1) / D * D;
  for (int j0 = 0; j0 < n_pad; j0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int j = j0 + u;
      const int t = t0 + j * tstep;
      float kr[ATT_DPL], vr[ATT_DPL];
      widen(ring[u].k, kr);
      widen(ring[u].v, vr);
      if (t == T) {
#pragma unroll
        for (int i = 0; i < ATT_DPL; ++i) { kr[i] = knew[dim_of(i)]; vr[i] = vnew[dim_of(i)]; }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < ATT_DPL; ++i) dot = fmaf(q[g][i], kr[i], dot);
        const float sc = group_allsum(dot, LPT) * a.scale;
        if (t < ctx) {
          const float mn = fmaxf(m[g], sc);
          const float f = expf(m[g] - mn);   // 0 while the slot is empty (m = -inf)
          const float p = expf(sc - mn);
          l[g] = fmaf(l[g], f, p);
#pragma unroll
          for (int i = 0; i < ATT_DPL; ++i) o[g][i] = fmaf(o[g][i], f, p * vr[i]);
          m[g] = mn;
        }
      }
      load(j + D, ring[u]);
    }
  }
  // Merge the slots of the wave (lanes with the same sub), then the waves.
  for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m2 = __shfl_xor(m[g], off, 64), l2 = __shfl_xor(l[g], off, 64);
      const float M = fmaxf(m[g], m2);
      const float f1 = merge_weight(m[g], M), f2 = merge_weight(m2, M);
      l[g] = l[g] * f1 + l2 * f2;
#pragma unroll
      for (int i = 0; i < ATT_DPL; ++i) {
        const float o2 = __shfl_xor(o[g][i], off, 64);
        o[g][i] = o[g][i] * f1 + o2 * f2;
      }
      m[g] = M;
    }
  }
  if (lane < LPT) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < ATT_DPL; ++i) mo[((size_t)wave * G + g) * hd + dim_of(i)] = o[g][i];
      if (lane == 0) { mls[(wave * G + g) * 2] = m[g]; mls[(wave * G + g) * 2 + 1] = l[g]; }
    }
  }
  __syncthreads();
  if (tid < G * hd) {
    const int g = tid / hd, d = tid - g * hd;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, mls[(w * G + g) * 2]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = merge_weight(mls[(w * G + g) * 2], M);
      L = fmaf(mls[(w * G + g) * 2 + 1], f, L);
      O = fmaf(mo[((size_t)w * G + g) * hd + d], f, O);
    }
    if (S == 1) {
      a.out[(size_t)r * a.ldo + (size_t)(h * G + g) * hd + d] = O / L;
      if (a.xs_out) xsplit_store(a.xs_out, r, (h * G + g) * hd + d, O / L);
    } else {
      float* pp = a.part + (((size_t)r * a.Hq + h * G + g) * a.max_chunks + s) * part_stride(hd);
      pp[d] = O;
      if (d == 0) { pp[hd] = M; pp[hd + 1] = L; }
    }
  }
}

// ------------------------------------------------------------ sampler
// Device-resident sampling parameters (rewritten between replays).
struct SkParams {
  float cfg_scale;
  float temperature; int top_k; float top_p;
  int has_q0; float temperature_q0; int top_k_q0; float top_p_q0;
  int record_logits;
  int pad[3];
};

// Order key of an FP32 value: larger value -> larger key; -0 and +0 equal.
__device__ __forceinline__ uint32_t fkey(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Sampler workgroups: SNT threads, two waves per SIMD, so the latency of
// one wave's reduction chains is hidden behind the other's.
constexpr int SNT = 512;
constexpr int SWAVES = SNT / 64;

struct SampleSmem {
  int hist[SWAVES][4][256];   // radix histograms, private per (wave, lane & 3)
  int scan[SWAVES];
  int wcount[SWAVES];
  unsigned lvc[SWAVES][8];    // per-wave distance-level counts, 16 levels x 16 bits
  float4 bst[SWAVES];          // per-wave (max, sum, finite count as int bits, -)
  unsigned long long bk[SWAVES];
  int prk[SWAVES][64];        // per-wave partial ranks of the first 64 keys
  int code;
  int sel_digit;
  int sel_excl;
  int sel_cnt;
};

// Sort key of candidate (value, index): a larger key comes first in the
// order value desc, index asc.  Key 0 sorts after every real candidate.
__device__ __forceinline__ unsigned long long skey(float v, int idx) {
  return ((unsigned long long)fkey(v) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ float key_value(unsigned long long k) {
  const uint32_t u = (uint32_t)(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ int key_index(unsigned long long k) {
  return (int)(0xffffffffu - (uint32_t)k);
}

template <int CTRL, int ROW_MASK, bool BOUND0>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, BOUND0);
}
// Inclusive prefix sum of an int over the 64 lanes (DPP row shifts + row broadcasts).
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += dpp_i<0x111, 0xf, true>(x);   // row_shr:1
  x += dpp_i<0x112, 0xf, true>(x);   // row_shr:2
  x += dpp_i<0x114, 0xf, true>(x);   // row_shr:4
  x += dpp_i<0x118, 0xf, true>(x);   // row_shr:8
  x += dpp_i<0x142, 0xa, false>(x);  // row_bcast:15
  x += dpp_i<0x143, 0xc, false>(x);  // row_bcast:31
  return x;
}
// Sum of an int over the 64 lanes, returned to every lane.
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i<0xb1, 0xf, true>(v);
  v += dpp_i<0x4e, 0xf, true>(v);
  v += dpp_i<0x114, 0xf, true>(v);
  v += dpp_i<0x118, 0xf, true>(v);
  v += dpp_i<0x142, 0xa, false>(v);
  v += dpp_i<0x143, 0xc, false>(v);
  return __builtin_amdgcn_readlane(v, 63);
}
// Sums of 8 words over the 64 lanes at once: every lane gets the total of
// word (lane >> 3).  Halving steps over lane bits 5 and 4 (permlane swaps)
// and 3 (row mirror), then plain sums within each group of 8 lanes.
__device__ __forceinline__ unsigned wave_reduce8(const unsigned (&w)[8], int lane) {
  unsigned v[4], t[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(w[i], w[i + 4], false, false);
    v[i] = r[0] + r[1];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(v[i], v[i + 2], false, false);
    t[i] = r[0] + r[1];
  }
  const bool hi = (lane >> 3) & 1;
  const unsigned keep = hi ? t[1] : t[0], send = hi ? t[0] : t[1];
  unsigned x = keep + (unsigned)dpp_i<0x140, 0xf, false>((int)send);   // row_mirror
  x += (unsigned)dpp_i<0x141, 0xf, false>((int)x);                    // row_half_mirror
  x += (unsigned)dpp_i<0x4e, 0xf, false>((int)x);                     // quad_perm [2,3,0,1]
  x += (unsigned)dpp_i<0xb1, 0xf, false>((int)x);                     // quad_perm [1,0,3,2]
  return x;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long t = __shfl_xor(k, o, 64);
    k = t > k ? t : k;
  }
  return k;
}

template <int CTRL, int ROW_MASK, bool BOUND0>
__device__ __forceinline__ double dpp_f64(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(b & 0xffffffffll), CTRL, ROW_MASK, 0xf, BOUND0);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROW_MASK, 0xf, BOUND0);
  return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}
// Inclusive prefix sum in float64 over the 64 lanes, in this fixed order:
// within each row of 16 lanes add the value 1, 2, 4, 8 lanes below (same
// row); then rows 1 and 3 add the last lane of the row before; then rows 2
// and 3 add lane 31.  The oracle repeats exactly these additions, so both
// sides round identically.
__device__ __forceinline__ double wave_scan_f64(double w) {
  w += dpp_f64<0x111, 0xf, true>(w);
  w += dpp_f64<0x112, 0xf, true>(w);
  w += dpp_f64<0x114, 0xf, true>(w);
  w += dpp_f64<0x118, 0xf, true>(w);
  w += dpp_f64<0x142, 0xa, false>(w);
  w += dpp_f64<0x143, 0xc, false>(w);
  return w;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}

// Inverse-CDF draw over the first n keys of a sorted list (value desc,
// index asc), run by one wave: w_i = exp(x_i - x_0) in float64, W = prefix
// sums (wave_scan_f64 per group of 64, plus the running total of the earlier
// groups); n_keep = first i with W_i > p * W_{n-1}, plus one (top-p, first
// always kept); the code is the first candidate with W_j > u * W_{n_keep-1}.
// Wg: n doubles of LDS (used when n > 64).
__device__ __forceinline__ int draw_sorted(const unsigned long long* sk, int n, float top_p, double u,
                                           double* Wg) {
  const int lane = threadIdx.x & 63;
  const double top = (double)key_value(sk[0]);
  if (n <= 64) {
    const unsigned long long k = sk[min(lane, n - 1)];
    const double w = (lane < n) ? exp((double)key_value(k) - top) : 0.0;
    const double W = wave_scan_f64(w);
    const double S = readlane_f64(W, n - 1);
    int nk = n;
    if (top_p > 0.f && top_p < 1.f) {
      const unsigned long long b = __ballot(lane + 1 < n && W > (double)top_p * S);
      if (b) nk = __ffsll((long long)b);
    }
    const double target = u * readlane_f64(W, nk - 1);
    const unsigned long long b = __ballot(lane < nk && W > target);
    const int j = b ? __ffsll((long long)b) - 1 : nk - 1;
    return key_index(sk[j]);
  }
  double carry = 0.0;
  for (int g0 = 0; g0 < n; g0 += 64) {
    const unsigned long long k = sk[min(g0 + lane, n - 1)];
    const double w = (g0 + lane < n) ? exp((double)key_value(k) - top) : 0.0;
    const double sc = wave_scan_f64(w);
    if (g0 + lane < n) Wg[g0 + lane] = carry + sc;
    carry = carry + readlane_f64(sc, 63);
  }
  __builtin_amdgcn_wave_barrier();
  const double S = Wg[n - 1];
  int nk = n;
  if (top_p > 0.f && top_p < 1.f) {
    const double thr = (double)top_p * S;
    for (int g0 = 0; g0 + 1 < n; g0 += 64) {
      const unsigned long long b = __ballot(g0 + lane + 1 < n && Wg[min(g0 + lane, n - 1)] > thr);
      if (b) { nk = g0 + __ffsll((long long)b); break; }
    }
  }
  const double target = u * Wg[nk - 1];
  int j = nk - 1;
  for (int g0 = 0; g0 < nk; g0 += 64) {
    const unsigned long long b = __ballot(g0 + lane < nk && Wg[min(g0 + lane, nk - 1)] > target);
    if (b) { j = g0 + __ffsll((long long)b) - 1; break; }
  }
  return key_index(sk[j]);
}

// Rank of key K among ck[0, n2) (n2 even, padded with key 0): the number of
// keys that sort before it.
__device__ __forceinline__ int key_rank(const unsigned long long* ck, int n2, unsigned long long K) {
  int rank = 0;
  int j = 0;
  for (; j + 8 <= n2; j += 8) {          // four 16-byte reads in flight per step
    ulonglong2 kk[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) kk[t] = *reinterpret_cast<const ulonglong2*>(ck + j + 2 * t);
#pragma unroll
    for (int t = 0; t < 4; ++t) rank += (kk[t].x > K ? 1 : 0) + (kk[t].y > K ? 1 : 0);
  }
  for (; j < n2; j += 2) {
    const ulonglong2 kk = *reinterpret_cast<const ulonglong2*>(ck + j);
    rank += (kk.x > K ? 1 : 0) + (kk.y > K ? 1 : 0);
  }
  return rank;
}

// Number of leading sorted candidates that survive top-k with ties kept:
// every value >= the k-th largest (model.py:697-699); k <= 0 keeps all.
__device__ __forceinline__ int topk_count(const unsigned long long* sk, int n, int k) {
  if (k <= 0 || k >= n) return n;
  const uint32_t kth = (uint32_t)(sk[k - 1] >> 32);
  const int lane = threadIdx.x & 63;
  int cnt = k;
  for (int g0 = k; g0 < n; g0 += 64) {
    const unsigned long long b =
        __ballot(g0 + lane < n && (uint32_t)(sk[min(g0 + lane, n - 1)] >> 32) >= kth);
    cnt += __popcll(b);
    if (b != ~0ull) break;
  }
  return cnt;
}

constexpr int FILTER_MAX = 256;          // largest candidate set the distance filter ranks directly

// xr[i] = value of logit v = threadIdx.x + i*SNT (registers; -inf past V):
// CFG-merged, masked and, when temperature > 0, divided by the temperature.
// Follows model.py:686-708: greedy argmax when temperature <= 0; else top-k
// (ties kept), top-p (shift-by-one, first kept) and the explicit-uniform
// inverse-CDF draw in float64 over candidates ordered by value desc, index
// asc.  ck: MAX_V keys of LDS; sk: FILTER_MAX keys of LDS; W: MAX_V doubles
// of LDS.  The code is valid in every lane of wave 0.
//
// Top-k selection.  One barrier gives the block maximum M and mean; a
// second gives, per wave, how many values fall in each of 16 distance levels
// lvl(x) = min(15, floor((M - x) * 16 / (M - mean))) (monotone in x, so
// {lvl <= L} is a set {x >= t}).  With L the first level whose cumulative
// count reaches k, that set holds every top-k member; when it has at most
// FILTER_MAX entries it is compacted and ranked exactly (one wave when it
// has at most 64).  Otherwise (flat distributions, top-k off) an exact
// 8-bit radix select finds the k-th key and the candidates are sorted.
template <int VPT>
__device__ __forceinline__ int sample_core(const float (&xr)[VPT], int V, float temp, int top_k, float top_p,
                                           double u, unsigned long long* ck, unsigned long long* sk,
                                           double* W, SampleSmem& s) {
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (!(temp > 0.f)) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const unsigned long long k = skey(xr[i], tid + i * SNT);
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) s.bk[wave] = best;
    sk_sync();
    unsigned long long b = s.bk[0];
#pragma unroll
    for (int w = 1; w < SWAVES; ++w) b = s.bk[w] > b ? s.bk[w] : b;
    return key_index(b);
  }

  // ---- block maximum, sum and count of the finite values (count by ballot)
  float mx = -INFINITY, sm = 0.f;
  int nf = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const bool f = isfinite(xr[i]);
    mx = f ? fmaxf(mx, xr[i]) : mx;
    sm += f ? xr[i] : 0.f;
    nf += __popcll(__ballot(f));
  }
  mx = wave_max_dpp(mx);
  sm = wave_sum_dpp(sm);
  if (lane == 0) s.bst[wave] = make_float4(mx, sm, __int_as_float(nf), 0.f);
  sk_sync();
  float4 b0 = s.bst[0];
  float M = b0.x, S = b0.y;
  int nfin = __float_as_int(b0.z);
#pragma unroll
  for (int w = 1; w < SWAVES; ++w) {
    const float4 bw = s.bst[w];
    M = fmaxf(M, bw.x); S += bw.y; nfin += __float_as_int(bw.z);
  }
  if (nfin == 0) return 0;               // every entry masked: nothing to draw

  // ---- distance levels lvl = min(15, floor((M - x) * 16 / (M - mean))),
  // counted in 4-bit fields (two accumulators when a thread holds > 15)
  // Any monotone level function keeps the selection exact: approximate
  // reciprocals suffice.
  const float spread = M - S * __builtin_amdgcn_rcpf((float)nfin);
  const float inv_step = spread > 0.f ? 16.f * __builtin_amdgcn_rcpf(spread) : 0.f;
  int lvl[VPT];
  unsigned long long cnt[2] = {0ull, 0ull};
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const bool f = isfinite(xr[i]);
    lvl[i] = f ? (int)fminf((M - xr[i]) * inv_step, 15.f) : 16;
    const unsigned long long one = f ? (1ull << (4 * (lvl[i] & 15))) : 0ull;
    cnt[VPT > 15 ? (i & 1) : 0] += one;
  }
  unsigned w8[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    unsigned t = 0;
#pragma unroll
    for (int a = 0; a < (VPT > 15 ? 2 : 1); ++a) {
      const unsigned byte = (unsigned)(cnt[a] >> (8 * m)) & 0xffu;
      t += (byte & 0xfu) | ((byte >> 4) << 16);
    }
    w8[m] = t;
  }
  const unsigned red = wave_reduce8(w8, lane);
  if ((lane & 7) == 0) s.lvc[wave][lane >> 3] = red;
  sk_sync();
  // Lane j (of every row of 16 lanes) owns level j: its count over all waves
  // and over the waves before this one, then inclusive scans over the 16
  // levels.  L = the first level whose cumulative count reaches keff (15 if
  // none does): {lvl <= L} holds every top-k member.
  const bool use_k = top_k > 0 && top_k < V;
  const int keff = use_k ? min(top_k, nfin) : nfin;
  int L, cum, wbase;
  {
    const int j = lane & 15;
    int t = 0, b = 0;
#pragma unroll
    for (int w = 0; w < SWAVES; ++w) {
      const int f = (int)((s.lvc[w][j >> 1] >> (16 * (j & 1))) & 0xffffu);
      t += f;
      b += (w < wave) ? f : 0;
    }
    t += dpp_i<0x111, 0xf, true>(t);   // row_shr:1
    t += dpp_i<0x112, 0xf, true>(t);   // row_shr:2
    t += dpp_i<0x114, 0xf, true>(t);   // row_shr:4
    t += dpp_i<0x118, 0xf, true>(t);   // row_shr:8
    b += dpp_i<0x111, 0xf, true>(b);
    b += dpp_i<0x112, 0xf, true>(b);
    b += dpp_i<0x114, 0xf, true>(b);
    b += dpp_i<0x118, 0xf, true>(b);
    const unsigned long long reach = __ballot(lane < 16 && t >= keff);
    L = reach ? min(__ffsll((long long)reach) - 1, 15) : 15;
    cum = __builtin_amdgcn_readlane(t, L);
    wbase = __builtin_amdgcn_readlane(b, L);
  }

  if (cum <= FILTER_MAX) {
    // ---- compact {lvl <= L} as sort keys in the deterministic order (wave,
    // slot i, lane): a ballot per slot, the lane's offset by mbcnt.
    int pos = wbase;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const bool in = lvl[i] <= L;
      const unsigned long long bm = __ballot(in);
      if (in)
        ck[pos + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bm >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bm, 0u))] =
            skey(xr[i], tid + i * SNT);
      pos += __popcll(bm);
    }
    const int n = cum;
    const int n2 = (n + 1) & ~1;
    if (tid == n && n < n2) ck[n] = 0ull;
    sk_sync();
    if (n <= 64) {
      // Wave w counts, for each of the first 64 keys (one per lane), the keys
      // of its slice [8w, 8w + 8) that sort before it; wave 0 adds the slices.
      static_assert(SWAVES * 8 >= 64, "rank slices must cover 64 keys");
      const unsigned long long K = (lane < n) ? ck[lane] : 0ull;
      int part = 0;
      if (8 * wave < n2) {
        const ulonglong2* kp = reinterpret_cast<const ulonglong2*>(ck + 8 * wave);
        ulonglong2 kk[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) kk[t] = kp[t];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int j = 8 * wave + 2 * t;
          part += (j < n2 && kk[t].x > K ? 1 : 0) + (j + 1 < n2 && kk[t].y > K ? 1 : 0);
        }
      }
      s.prk[wave][lane] = part;
      sk_sync();
      if (wave == 0) {
        int rank = 0;
#pragma unroll
        for (int w = 0; w < SWAVES; ++w) rank += s.prk[w][lane];
        if (lane < n) sk[rank] = K;
        __builtin_amdgcn_wave_barrier();
        return draw_sorted(sk, use_k ? topk_count(sk, n, top_k) : n, top_p, u, W);
      }
      return 0;
    }
    if (tid < n) {
      const unsigned long long K = ck[tid];
      sk[key_rank(ck, n2, K)] = K;
    }
    sk_sync();
    if (wave == 0) return draw_sorted(sk, use_k ? topk_count(sk, n, top_k) : n, top_p, u, W);
    return 0;
  }

  // ---- general path: exact radix select of the k-th key, then sort
  uint32_t key[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) key[i] = fkey(xr[i]);
  uint32_t cut = 0u;
  if (use_k) {
    int* H = &s.hist[0][0][0];
    int* Hw = H + (wave * 4 + (lane & 3)) * 256;
    uint32_t prefix = 0u, pmask = 0u;
    int kr = top_k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid * 4; i < SWAVES * 4 * 256; i += SNT * 4)
        *reinterpret_cast<int4*>(&H[i]) = make_int4(0, 0, 0, 0);
      sk_sync();
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        if (tid + i * SNT < V && (key[i] & pmask) == prefix) atomicAdd(&Hw[(key[i] >> shift) & 255u], 1);
      sk_sync();
      // bin 255 - tid (threads below 256) summed over the private copies,
      // then a scan over bins.
      int cnt = 0;
      if (tid < 256) {
#pragma unroll
        for (int j = 0; j < SWAVES * 4; ++j) cnt += H[j * 256 + (255 - tid)];
      }
      int incl = wave_incl_scan(cnt);
      if (lane == 63) s.scan[wave] = incl;
      sk_sync();
      for (int w = 0; w < wave; ++w) incl += s.scan[w];
      const int excl = incl - cnt;
      if (cnt > 0 && excl < kr && kr <= incl) { s.sel_digit = 255 - tid; s.sel_excl = excl; s.sel_cnt = cnt; }
      sk_sync();
      prefix |= (uint32_t)s.sel_digit << shift;
      pmask |= 255u << shift;
      kr -= s.sel_excl;
      const bool done = (s.sel_cnt == kr);
      sk_sync();
      if (done) break;
    }
    cut = prefix;
  }

  // Compact the candidates (finite, key >= cut) as sort keys.
  bool keep[VPT];
  int myc = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    keep[i] = isfinite(xr[i]) && key[i] >= cut;
    myc += keep[i] ? 1 : 0;
  }
  const int wincl = wave_incl_scan(myc);
  if (lane == 63) s.wcount[wave] = wincl;
  sk_sync();
  int base = 0, n = 0;
#pragma unroll
  for (int w = 0; w < SWAVES; ++w) {
    if (w < wave) base += s.wcount[w];
    n += s.wcount[w];
  }
  base += wincl - myc;
#pragma unroll
  for (int i = 0; i < VPT; ++i)
    if (keep[i]) ck[base++] = skey(xr[i], tid + i * SNT);
  int P = 1;
  while (P < n) P <<= 1;
  sk_sync();
  for (int i = n + tid; i < P; i += SNT) ck[i] = 0ull;
  sk_sync();
  // Bitonic sort of the keys in LDS, largest first.
  for (int k = 2; k <= P; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P; i += SNT) {
        const int l = i ^ j;
        if (l > i) {
          const unsigned long long ki = ck[i], kl = ck[l];
          const bool swap = ((i & k) == 0) ? (kl > ki) : (ki > kl);
          if (swap) { ck[i] = kl; ck[l] = ki; }
        }
      }
      sk_sync();
    }
  if (wave == 0) return draw_sorted(ck, n, top_p, u, W);
  return 0;
}

// CFG merge u + s (c - u) without contraction, then BOS/PAD (and EOS) -> -inf
// (model.py:579-584).  EOS is masked when force_mask is set or bit mask_bit
// (the utterance) of *mask_flag is set.  The merged row is optionally recorded, then kept in
// registers divided by the temperature when sampling (model.py:696).  Loads
// are clamped into the row and entries past V become -inf afterwards, so no
// load sits behind a branch (without an uncond row the cond row is loaded
// twice and the copy ignored: a load under `lu ?` made each one wait for the
// one before).
template <int VPT>
__device__ __forceinline__ void load_logits(const float* lc, const float* lu, int V, float (&cvv)[VPT],
                                            float (&uvv)[VPT]) {
  const float* lu2 = lu ? lu : lc;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int v = min((int)threadIdx.x + i * SNT, V - 1);
    cvv[i] = lc[v];
    uvv[i] = lu2[v];
  }
}
template <int VPT>
__device__ __forceinline__ void merge_mask_loaded(const float (&cvv)[VPT], const float (&uvv)[VPT], bool lu, float s,
                                                  int V, int bos, int eos, int pad, const int* mask_flag,
                                                  int mask_bit, bool force_mask, float temp, float* dbg,
                                                  float (&xr)[VPT]);
template <int VPT>
__device__ __forceinline__ void merge_mask(const float* lc, const float* lu, float s, int V, int bos, int eos,
                                           int pad, const int* mask_flag, int mask_bit, bool force_mask, float temp,
                                           float* dbg, float (&xr)[VPT]) {
  float cvv[VPT], uvv[VPT];
  load_logits<VPT>(lc, lu, V, cvv, uvv);
  merge_mask_loaded<VPT>(cvv, uvv, lu != nullptr, s, V, bos, eos, pad, mask_flag, mask_bit, force_mask, temp, dbg,
                         xr);
}
// The CFG merge and masks of loaded logits (see merge_mask).
template <int VPT>
__device__ __forceinline__ void merge_mask_loaded(const float (&cvv)[VPT], const float (&uvv)[VPT], bool lu, float s,
                                                  int V, int bos, int eos, int pad, const int* mask_flag,
                                                  int mask_bit, bool force_mask, float temp, float* dbg,
                                                  float (&xr)[VPT]) {
  const bool mask_eos = force_mask || (mask_flag && ((*mask_flag >> mask_bit) & 1));
  const bool divide = temp > 0.f;
  // Chunks below the lowest special id need no mask compares (uniform test).
  const int lo_special = min(min(bos, pad), mask_eos ? min(eos, V) : V);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int v = threadIdx.x + i * SNT;
    float m = cvv[i];
    if (lu) m = __fadd_rn(uvv[i], __fmul_rn(s, __fsub_rn(m, uvv[i])));
    if ((i + 1) * SNT > lo_special)
      if (v == bos || v == pad || (mask_eos && v == eos) || v >= V) m = -INFINITY;
    if (dbg && v < V) dbg[v] = m;
    xr[i] = divide ? m / temp : m;
  }
}

struct SampleArgs {
  const float* logits; int ldl; int rows_per_utt; int V;
  const SkParams* params;
  const int* fc;                       // device frame counter -> ring slot
  const double* u_cur;                 // [n_utts][Q] this frame's draws
  const int* flag_cur;                 // [2] this frame's (mask_eos_q0, forced)
  const int64_t* forced_ring;          // [frames][n_utts][Q]
  int64_t* codes_ring;                 // [frames][n_utts][Q]
  int* codes_cur;                      // [n_utts][Q] this frame's codes
  float* dbg;                          // [n_utts][Q][V]
  const void* table;                   // [Q][V][d]
  float* prefix; float* xnext;         // [rows][d]
  int d, Q; float scale;
  int bos, eos, pad;
  int n_utts;
  // Next depth step's input (q < Q-1): abuf = RMSNorm_in(hidden + prefix) per
  // row, and its split form for the many-row GEMMs (xs_abuf, may be null).
  const float* hidden; const float* w_in; float eps_in;
  float* abuf; uint16_t* xs_abuf;
  // Many rows with code tables (ptab set): the next depth step's SwiGLU
  // output as well, act = SwiGLU(r G_{q+1}) with G_{q+1} = G_q + scale
  // P_q[code] (G_q = W_gu (w_in * x_q)), so that step needs no gate/up GEMM.
  const float* ptab; int ki;           // [Q-1][V][2 ki] code tables; depth inner size (<= 4 SNT)
  const float* g_in; float* g_out;     // [rows][2 ki] G_q, G_{q+1} (gate | up); g_out null: not needed
  int g_in_normed;                     // g_in holds r_0 G_0 (codebook 0's GEMM): scaled by rms(hidden)
  float* act; int ld_act; uint16_t* xs_act;   // SwiGLU output [rows][ld_act] and its split form
  // The last codebook, one utterance with code tables: the prefix through
  // codebook Q-2 as the depth steps left it (scale * table rows summed in
  // codebook order), so the frame embedding is one more row (null: the rows
  // are gathered and summed here).
  const float* prefix_last;
  // Where the advanced prefix goes (null: back into prefix).  Set when the
  // sampler of an utterance runs in several workgroups (gridDim.y > 1), which
  // all read the whole prefix while each writes its slice.
  float* prefix_out;
};

// The depth input rows of one utterance after its code q (sample_step_kernel,
// SNT threads): prefix += table[q][code] * scale, x = hidden + prefix,
// abuf = w_in * (x * inv_rms(x)); with code tables also the next step's
// SwiGLU output (SampleArgs.ptab).  The loads are issued together once the
// code is known (all threads hold it).
constexpr int DEPTH_DPT = 8;             // d <= SNT * DEPTH_DPT
constexpr int DEPTH_API = 4;             // code-table inner indices per thread: ki <= SNT * DEPTH_API
// DPT: elements of d per thread (d <= SNT * DPT).  The outputs are split over
// the ns workgroups of the utterance (slice sl): each forms the whole x for
// the norm but writes d / ns of the prefix and abuf and ki / ns of G and act.
template <typename TL, int DPT>
__device__ __forceinline__ void depth_input_rows(const SampleArgs& a, int r0, int q, int code, int sl, int ns) {
  __shared__ float red[2][2][SWAVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nr = a.rows_per_utt;         // 1 or 2
  const size_t trow = ((size_t)q * a.V + code) * a.d;
  const bool tables = a.ptab != nullptr;   // uniform
  const int ds = a.d / ns, db = sl * ds;      // this slice's hidden indices
  const int kis = a.ki / ns, kb = sl * kis;   // and inner indices
  float* pout = a.prefix_out ? a.prefix_out : a.prefix;
  // Every operand first, indices clamped in bounds (rows past nr re-read row
  // 0, dims past d re-read d-1): one round trip, no branch between the
  // loads, and no load behind the prefix stores that might alias it.
  float tv[DPT], gv[DPT], pv[2][DPT], hv[2][DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) {
    const int k = min(tid + i * SNT, a.d - 1);
    tv[i] = TL::get(a.table, trow + k);
    gv[i] = a.w_in[k];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const size_t ro = (size_t)(r0 + (rr < nr ? rr : 0)) * a.d;
      pv[rr][i] = a.prefix[ro + k];
      hv[rr][i] = a.hidden[ro + k];
    }
  }
  // G_q of the rows and P_q[code] at this thread's inner indices (gate, up)
  float gq[2][2][DEPTH_API], pq[2][DEPTH_API];
  if (tables) {
    const float* pr = a.ptab + ((size_t)q * a.V + code) * 2 * a.ki;
#pragma unroll
    for (int i = 0; i < DEPTH_API; ++i) {
      if (i * SNT >= kis) break;         // uniform
      const int k = kb + min(tid + i * SNT, kis - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        pq[h][i] = pr[h * a.ki + k];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
          gq[rr][h][i] = a.g_in[(size_t)(r0 + (rr < nr ? rr : 0)) * 2 * a.ki + h * a.ki + k];
      }
    }
  }
  float xv[2][DPT];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const size_t ro = (size_t)(r0 + rr) * a.d;
    float ss = 0.f, sh = 0.f;
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
      const int k = tid + i * SNT;
      const float p = __fadd_rn(pv[rr][i], __fmul_rn(tv[i], a.scale));
      const float x = __fadd_rn(hv[rr][i], p);
      xv[rr][i] = x;
      if (k < a.d) {
        if (rr < nr && k - db >= 0 && k - db < ds) pout[ro + k] = p;
        ss = fmaf(x, x, ss);
        sh = fmaf(hv[rr][i], hv[rr][i], sh);
      }
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[0][rr][wave] = ss;
    if (tables) {
      sh = wave_sum_dpp(sh);
      if (lane == 0) red[1][rr][wave] = sh;
    }
  }
  sk_sync();
  for (int rr = 0; rr < nr; ++rr) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < SWAVES; ++w) t += red[0][rr][w];
    const float inv = 1.0f / sqrtf(t / (float)a.d + a.eps_in);
    const size_t ro = (size_t)(r0 + rr) * a.d;
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
      const int k = tid + i * SNT;
      if (k - db >= 0 && k - db < ds) {
        const float y = gv[i] * (xv[rr][i] * inv);
        a.abuf[ro + k] = y;
        if (a.xs_abuf) xsplit_store(a.xs_abuf, r0 + rr, k, y);
      }
    }
    if (tables) {
      // G_{q+1} = G_q + scale P_q[code] (after codebook 0's GEMM, G_0 = its
      // r_0 G_0 times rms(hidden)); act = SwiGLU(r_{q+1} G_{q+1}) as the GEMM
      // epilogue forms it
      float rms0 = 1.f;
      if (a.g_in_normed) {
        float th = 0.f;
#pragma unroll
        for (int w = 0; w < SWAVES; ++w) th += red[1][rr][w];
        rms0 = sqrtf(th / (float)a.d + a.eps_in);
      }
      const size_t go = (size_t)(r0 + rr) * 2 * a.ki;
#pragma unroll
      for (int i = 0; i < DEPTH_API; ++i) {
        if (i * SNT >= kis) break;       // uniform
        const int j = tid + i * SNT, k = kb + j;
        if (j < kis) {
          const float gt = fmaf(a.scale, pq[0][i], gq[rr][0][i] * rms0);
          const float up = fmaf(a.scale, pq[1][i], gq[rr][1][i] * rms0);
          if (a.g_out) {
            a.g_out[go + k] = gt;
            a.g_out[go + a.ki + k] = up;
          }
          const float xg = gt * inv, xu = up * inv;
          const float y = xg / (1.0f + expf(-xg)) * xu;
          a.act[(size_t)(r0 + rr) * a.ld_act + k] = y;
          if (a.xs_act) xsplit_store(a.xs_act, r0 + rr, k, y);
        }
      }
    }
  }
}

// One workgroup per utterance, launched once per codebook q.  Samples the
// code and records it.  Before the last codebook it advances the rows' prefix
// with it (prefix += table[q][code] / sqrt(Q), model.py:600-605) and writes the
// next depth step's input, abuf = RMSNorm_in(hidden + prefix) (eps
// FLT_EPSILON) -- the depth MLP input and its residual -- so the depth GEMVs
// take it ready-made.  After the last codebook it writes the frame embedding
// (model.py:105-114) as the next trunk input and clears the prefix the next
// frame starts from.  Every input that does not depend on the code
// is loaded in the first round trip (this frame's draws and flags sit at
// fixed addresses, so nothing waits on the frame counter).  VPT = logits per
// thread, ceil(V / SNT).
template <typename TL, int VPT, int DPT>
__global__ __launch_bounds__(SNT) void sample_step_kernel(SampleArgs a, int q) {
  extern __shared__ unsigned char raw[];
  double* W = reinterpret_cast<double*>(raw);
  unsigned long long* ck = reinterpret_cast<unsigned long long*>(W + MAX_V);
  unsigned long long* sk = ck + MAX_V;
  __shared__ SampleSmem s;
  __shared__ int codes_l[64];

  const int ut = blockIdx.x;
  // Workgroups (ut, sl) for sl < gridDim.y all draw the utterance's code
  // from the same inputs (so the same code); slice 0 records it, and each
  // forms its slice of the next depth step's inputs.
  const int sl = blockIdx.y, ns = gridDim.y;
  const int r0 = ut * a.rows_per_utt;
  const float* lc = a.logits + (size_t)r0 * a.ldl;
  const float* lu = (a.rows_per_utt == 2) ? lc + a.ldl : nullptr;
  const double u = a.u_cur[(size_t)ut * a.Q + q];
  const int forced = a.flag_cur[1];
  const int slot = *a.fc;
  const SkParams P = *a.params;
  const bool last = (q + 1 == a.Q);
  // The last codebook's frame embedding: from the prefix the depth steps
  // accumulated (prefix_last), else from the table rows of every code.
  constexpr int EI = 4, EQ = 16;        // d <= EI * SNT, 2 <= Q <= EQ
  const bool from_prefix = last && a.prefix_last != nullptr && a.d <= EI * SNT;
  // The codes drawn so far, for the table rows: with prefix_last they are not
  // needed, and the load (whose test makes the logits wait for it) is skipped.
  if (last && !from_prefix && threadIdx.x < a.Q && threadIdx.x != q)
    codes_l[threadIdx.x] = a.codes_cur[(size_t)ut * a.Q + threadIdx.x];
  const bool q0 = (q == 0) && P.has_q0;
  const float temp = q0 ? P.temperature_q0 : P.temperature;
  const int topk = q0 ? P.top_k_q0 : P.top_k;
  const float topp = q0 ? P.top_p_q0 : P.top_p;
  float xr[VPT];
  merge_mask<VPT>(lc, lu, P.cfg_scale, a.V, a.bos, a.eos, a.pad, a.flag_cur, ut, q != 0, temp,
                  (P.record_logits && sl == 0) ? a.dbg + ((size_t)ut * a.Q + q) * a.V : nullptr, xr);
  // The last codebook's frame embedding: the table rows of codebooks
  // 0 .. Q-2 do not depend on the draw, so they are in flight during it
  // (issued once the logits are in, so the sampler does not wait for them).
  // With prefix_last the depth steps have summed them already.
  const bool early = last && !from_prefix && a.d <= EI * SNT && a.Q >= 2 && a.Q <= EQ;
  float pl[EI];
  if (from_prefix) {
#pragma unroll
    for (int i = 0; i < EI; ++i) pl[i] = a.prefix_last[min((int)threadIdx.x + i * SNT, a.d - 1)];
  }
  const size_t row_stride = (size_t)a.V * a.d;
  float te[EI][EQ - 1];
  if (early) {
#pragma unroll
    for (int i = 0; i < EI; ++i)
#pragma unroll
      for (int j = 0; j < EQ - 1; ++j) {
        const int dd = min((int)threadIdx.x + i * SNT, a.d - 1), jj = min(j, a.Q - 2);
        const int cj = a.codes_cur[(size_t)ut * a.Q + jj];
        te[i][j] = TL::get(a.table, (size_t)jj * row_stride + (size_t)cj * a.d + dd);
      }
  }
  int code = sample_core<VPT>(xr, a.V, temp, topk, topp, u, ck, sk, W, s);
  const size_t uoff = ((size_t)slot * a.n_utts + ut) * a.Q + q;
  if (threadIdx.x == 0) {
    if (forced) code = (int)a.forced_ring[uoff];
    code = min(max(code, 0), a.V - 1);
    if (sl == 0) {
      a.codes_ring[uoff] = code;
      a.codes_cur[(size_t)ut * a.Q + q] = code;
    }
    codes_l[q] = code;
  }
  if (!last) {
    if (a.abuf) {
      sk_sync();                   // codes_l[q] from thread 0
      depth_input_rows<TL, DPT>(a, r0, q, codes_l[q], sl, ns);
    }
    return;
  }
  if (sl != 0) return;               // the last codebook runs one workgroup per utterance

  sk_sync();
  if (from_prefix) {
    // x = prefix_{Q-1} + scale * table[Q-1][code]: the prefix update's own
    // order (model.py:600-605), the same sum as the frame embedding
    // (model.py:105-114) up to FP32 rounding
    const int cq = codes_l[q];
    float tq[EI];
#pragma unroll
    for (int i = 0; i < EI; ++i)
      tq[i] = TL::get(a.table, (size_t)q * row_stride + (size_t)cq * a.d + min((int)threadIdx.x + i * SNT, a.d - 1));
#pragma unroll
    for (int i = 0; i < EI; ++i) {
      const int dd = threadIdx.x + i * SNT;
      if (dd >= a.d) continue;
      const float e = __fadd_rn(pl[i], __fmul_rn(tq[i], a.scale));
      for (int rr = 0; rr < a.rows_per_utt; ++rr) {
        a.xnext[(size_t)(r0 + rr) * a.d + dd] = e;
        a.prefix[(size_t)(r0 + rr) * a.d + dd] = 0.f;
      }
    }
    return;
  }
  if (early) {
    const int cq = codes_l[q];
    float tq[EI];
#pragma unroll
    for (int i = 0; i < EI; ++i)
      tq[i] = TL::get(a.table, (size_t)q * row_stride + (size_t)cq * a.d + min((int)threadIdx.x + i * SNT, a.d - 1));
#pragma unroll
    for (int i = 0; i < EI; ++i) {
      const int dd = threadIdx.x + i * SNT;
      if (dd >= a.d) continue;
      float e = te[i][0];                 // codebooks in order: the same fold as below
#pragma unroll
      for (int j = 1; j < EQ - 1; ++j)
        if (j < a.Q - 1) e = __fadd_rn(e, te[i][j]);
      e = __fmul_rn(__fadd_rn(e, tq[i]), a.scale);
      for (int rr = 0; rr < a.rows_per_utt; ++rr) {
        a.xnext[(size_t)(r0 + rr) * a.d + dd] = e;
        a.prefix[(size_t)(r0 + rr) * a.d + dd] = 0.f;
      }
    }
    return;
  }
  for (int dd = threadIdx.x; dd < a.d; dd += SNT) {
    float e = 0.f;
    for (int j0 = 0; j0 < a.Q; j0 += 16) {
      // unconditional loads (codebook index clamped), masked afterwards: a
      // load inside the bound test was waited for before the next was issued
      float t[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int jj = min(j0 + j, a.Q - 1);
        t[j] = TL::get(a.table, (size_t)jj * row_stride + (size_t)codes_l[jj] * a.d + dd);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (j0 + j < a.Q) e = (j0 + j == 0) ? t[j] : __fadd_rn(e, t[j]);
    }
    e = __fmul_rn(e, a.scale);
    for (int rr = 0; rr < a.rows_per_utt; ++rr) {
      a.xnext[(size_t)(r0 + rr) * a.d + dd] = e;
      a.prefix[(size_t)(r0 + rr) * a.d + dd] = 0.f;
    }
  }
}

// One depth step of one utterance (few decode rows): the sampler of codebook
// q-1, the prefix advance prefix += table[q-1][code] * scale (model.py:600-605),
// the depth input a = RMSNorm_in(hidden + prefix) and codebook q's gate/up
// GEMV with the SwiGLU epilogue -- one launch instead of a sampler launch and
// a GEMV launch.  Every workgroup draws the code itself from the same logits,
// uniform and parameters (the draw is deterministic, so all agree) while its
// weight rows stream in; workgroup 0 records the code, the advanced prefix
// (into the other buffer of the ping-pong pair, g.gout) and a (g.norm_out, the
// depth MLP's residual).  g: gate/up weights (w[0], w[1]), N = depth inner
// rows, K = KT = d, x = hidden, x2 = the prefix before code q-1, out = act.
// Dynamic LDS: the sampler's W (V doubles), compaction keys (V rounded up to a
// power of two) and sorted filter keys (FILTER_MAX).
__host__ __device__ constexpr int pow2_ceil(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}
__host__ __device__ constexpr size_t depth_sample_smem(int V) {
  return (size_t)V * sizeof(double) + ((size_t)pow2_ceil(V) + FILTER_MAX) * 8;
}
template <typename TL, int VPT, int M, int KT, int RW>
__global__ __launch_bounds__(SNT) void depth_sample_gemv_kernel(SampleArgs a, GemvArgs g, int q) {
  extern __shared__ unsigned char raw[];
  double* W = reinterpret_cast<double*>(raw);
  unsigned long long* ck = reinterpret_cast<unsigned long long*>(W + a.V);
  unsigned long long* sk = ck + pow2_ceil(a.V);
  __shared__ SampleSmem s;
  __shared__ __attribute__((aligned(16))) float xsh[M * KT];
  __shared__ float red[M][SWAVES];
  __shared__ int code_sh;
  constexpr int VEC = TL::VEC;
  constexpr int NV = KT / (64 * VEC);
  constexpr int DPT = KT / SNT;                 // input elements per thread
  static_assert(KT % (64 * VEC) == 0 && KT % SNT == 0 && M <= 2, "depth_sample_gemv_kernel shape");
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qs = q - 1;                         // the codebook sampled here
  const bool lead = blockIdx.x == 0;

  // Loads that do not depend on the code, before the weight stream: the
  // draw's inputs, then hidden, the prefix and the norm gain.
  const double u = a.u_cur[qs];
  const int forced = a.flag_cur[1];
  const int slot = *a.fc;
  const SkParams P = *a.params;
  float hv[M][DPT], pv[M][DPT], gv[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) {
    const int k = tid + i * SNT;
    gv[i] = g.norm_w[k];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      hv[m][i] = g.x[(size_t)m * g.ldx + k];
      pv[m][i] = g.x2[(size_t)m * g.ldx2 + k];
    }
  }
  const bool q0 = (qs == 0) && P.has_q0;
  const float temp = q0 ? P.temperature_q0 : P.temperature;
  const int topk = q0 ? P.top_k_q0 : P.top_k;
  const float topp = q0 ? P.top_p_q0 : P.top_p;
  float xr[VPT];
  merge_mask<VPT>(a.logits, M == 2 ? a.logits + a.ldl : nullptr, P.cfg_scale, a.V, a.bos, a.eos, a.pad,
                  a.flag_cur, 0, qs != 0, temp, (lead && P.record_logits) ? a.dbg + (size_t)qs * a.V : nullptr, xr);
  // this wave's gate and up rows
  const int n0 = (blockIdx.x * SWAVES + wave) * RW;
  uint4 wraw[RW][2][NV];                        // raw 16-byte words, widened where multiplied
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const size_t off = (size_t)min(n0 + r, g.N - 1) * KT;
#pragma unroll
    for (int sidx = 0; sidx < 2; ++sidx)
#pragma unroll
      for (int j = 0; j < NV; ++j) wraw[r][sidx][j] = TL::raw(g.w[sidx], off + (size_t)(j * 64 + lane) * VEC);
  }

  int code = sample_core<VPT>(xr, a.V, temp, topk, topp, u, ck, sk, W, s);
  const size_t uoff = (size_t)slot * a.Q + qs;
  if (tid == 0) {
    if (forced) code = (int)a.forced_ring[uoff];
    code = min(max(code, 0), a.V - 1);
    code_sh = code;
    if (lead) {
      a.codes_ring[uoff] = code;
      a.codes_cur[qs] = code;
    }
  }
  sk_sync();
  code = code_sh;

  // prefix += table[q-1][code] * scale; x = hidden + prefix; a = w * (x / rms(x))
  const size_t trow = ((size_t)qs * a.V + code) * KT;
  float tv[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) tv[i] = TL::get(a.table, trow + tid + i * SNT);
  float xv[M][DPT];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
      const float p = __fadd_rn(pv[m][i], __fmul_rn(tv[i], a.scale));
      xv[m][i] = __fadd_rn(hv[m][i], p);
      if (lead) g.gout[(size_t)m * g.ldgo + tid + i * SNT] = p;
      ss = fmaf(xv[m][i], xv[m][i], ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[m][wave] = ss;
  }
  sk_sync();
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < SWAVES; ++w) t += red[m][w];
    const float inv = 1.0f / sqrtf(t / (float)KT + g.eps);
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
      const float y = gv[i] * (xv[m][i] * inv);
      xsh[m * KT + tid + i * SNT] = y;
      if (lead) g.norm_out[(size_t)m * g.ldno + tid + i * SNT] = y;
    }
  }
  sk_sync();

  float acc[RW][2][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int sidx = 0; sidx < 2; ++sidx)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][sidx][m] = 0.f;
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float x[VEC];
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(&xsh[m * KT + (j * 64 + lane) * VEC + i]);
        x[i] = t.x; x[i + 1] = t.y; x[i + 2] = t.z; x[i + 3] = t.w;
      }
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int sidx = 0; sidx < 2; ++sidx) {
          float w[VEC];
          TL::widen(wraw[r][sidx][j], w);
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[r][sidx][m] = fmaf(w[i], x[i], acc[r][sidx][m]);
        }
    }
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int sidx = 0; sidx < 2; ++sidx)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][sidx][m] = wave_sum_dpp(acc[r][sidx][m]);
  if (lane < M) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = n0 + r;
      if (n >= g.N) continue;
      float gt = acc[r][0][0], up = acc[r][1][0];
#pragma unroll
      for (int m = 1; m < M; ++m)
        if (m == lane) { gt = acc[r][0][m]; up = acc[r][1][m]; }
      g.out[(size_t)lane * g.ldo + n] = gt / (1.0f + expf(-gt)) * up;
    }
  }
}

// Totals of N words over the 64 lanes of a wave (N = 4, 8 or 16): lane l
// returns the total of word l / (64 / N).  Halving steps: each exchange keeps
// one word of a pair in each half of the lanes it pairs (permlane32 / 16
// swaps for lane bits 5 and 4, DPP row mirror and half mirror for bits 3 and
// 2), so N words cost about N adds instead of N full reductions; then the
// lanes left holding one word sum within their group.  Every step adds a pair
// of lanes' values in both lanes, so all lanes of a group get the same bits.
template <int N>
__device__ __forceinline__ float wave_reduce_words(float (&w)[N], int lane) {
  static_assert(N == 4 || N == 8 || N == 16, "wave_reduce_words: N");
  float v[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {          // lane bit 5
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(w[i]), __float_as_uint(w[i + N / 2]), false,
                                                   false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float t[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {          // lane bit 4
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + N / 4]), false,
                                                   false);
    t[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float x;
  if constexpr (N == 4) {
    x = t[0];
    x += dpp_keep<0x140, 0xf>(x);            // row mirror: lane i <-> 15 - i
  } else {
    const bool b3 = (lane >> 3) & 1;         // lane bit 3: row mirror pairs it
    float c[N / 8];
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const float a0 = t[i] + dpp_keep<0x140, 0xf>(t[i]);
      const float a1 = t[i + N / 8] + dpp_keep<0x140, 0xf>(t[i + N / 8]);
      c[i] = b3 ? a1 : a0;
    }
    if constexpr (N == 8) {
      x = c[0];
    } else {                                 // lane bit 2: half mirror pairs it
      const bool b2 = (lane >> 2) & 1;
      const float a0 = c[0] + dpp_keep<0x141, 0xf>(c[0]);
      const float a1 = c[1] + dpp_keep<0x141, 0xf>(c[1]);
      x = b2 ? a1 : a0;
    }
  }
  if constexpr (N <= 8) x += dpp_keep<0x141, 0xf>(x);   // half mirror: lane i <-> 7 - i
  x += dpp_keep<0x4e, 0xf>(x);               // quad_perm [2,3,0,1]
  x += dpp_keep<0xb1, 0xf>(x);               // quad_perm [1,0,3,2]
  return x;
}

// RoPE (cos, sin) of position p for frequency fq: angle = fp32(p * fq), cos
// and sin evaluated in double and rounded once (modeling_qwen3.py:116-122).
__device__ __forceinline__ float2 rope_cs(int p, float fq) {
  const float ang = (float)p * fq;
  return make_float2((float)cos((double)ang), (float)sin((double)ang));
}

// ------------------------------------------------------------ depth step (code tables)
// One utterance's depth step with the SwiGLU input taken apart by linearity.
// The gate/up input of codebook q is a_q = w_in * x_q * r_q, with x_q = hidden +
// prefix_q, r_q = 1 / rms(x_q), and x_q = x_{q-1} + scale * table[q-1][c] once
// code c of codebook q-1 is drawn.  So
//
//   W_gu a_q = r_q * (G_q + scale * P_{q-1}[c]),   G_q = W_gu (w_in * x_{q-1}),
//                                                  P_j[c] = W_gu (w_in * table[j][c]),
//
// where P_j is a weight-only table of every code's contribution, built when
// the frame is captured, and G_q, by the same linearity, is G_1 plus the table
// entries of the codes drawn so far: G_{q+1} = G_q + scale * P_{q-1}[c], the
// very sum the SwiGLU input scales.  Only G_1 = W_gu (w_in * hidden) is a
// GEMV.  Once c is known every workgroup forms the whole SwiGLU output
// elementwise, so codebook q-1's sampler, the prefix advance, the SwiGLU, the
// down projection with its residual (y_q = a_q + W_d act_q, model.py:163-170)
// and G_{q+1} fit one launch, and the classifier follows.  Launches per
// codebook: two instead of three.
//
// Work of one launch (256 workgroups of SNT threads): for G_1 each wave owns
// RWG gate rows and the same RWG up rows of W_gu (whole rows, K = KD); for the
// down projection the workgroup owns RD = KD / 256 output rows while its 8
// waves split the inner dimension KI into 8 chunks of 64 * VEC (one 16-byte
// weight load per lane and row).  Every weight load is issued before the
// sampler runs.
//   MODE 0: G_1 = W_gu (w_in * hidden) only (x_0 = hidden; no sampler).
//   MODE 1: codebook 0's SwiGLU + down: act_0 = SwiGLU(r_0 G_1), y_0.
//   MODE 2: codebooks 1 .. Q-1: sampler of q-1, prefix, act_q, y_q, and
//           G_{q+1} = G_q + scale P_{q-1}[c] (workgroup 0 stores it; for
//           codebook Q-1 into a buffer nothing reads before it is rewritten).
//   MODE 4, 5: the frame's end: the trunk's final RMSNorm of each active row
//           (hidden, written by workgroup 0) from its fixed-point (4) or FP32
//           (5) output, then MODE 0 on it -- G_1 of the next frame -- and the
//           rows' step bookkeeping (lengths, positions, RoPE entries, frame
//           counter, the next frame's draws and flags), so the next frame
//           starts at codebook 0's SwiGLU.  (A final-norm launch of its own and
//           MODE 0 at the next frame's start were two launches; G_1 needs the
//           whole normed row in every workgroup anyway.)
struct DepthArgs {
  const void* w_gate; const void* w_up;    // [KI][KD]
  const void* w_down;                      // [KD][KI]
  const float* hidden;                     // [M][KD]
  const float* prefix_in; float* prefix_out;   // [M][KD] before / after code q-1 (MODE 2)
  const float* norm_w; float eps;          // norm_in gain [KD], FLT_EPSILON
  const float* g_in;                       // [M][2 KI] G_q (gate | up), MODE 1, 2
  float* g_out;                            // [M][2 KI] G_1 (MODE 0) or G_{q+1} (MODE 2)
  const float* ptab;                       // [Q-1][V][2 KI] code tables, MODE 2
  float* y;                                // [M][KD] depth MLP output, MODE 1, 2
  float scale;                             // frame scale 1/sqrt(Q)
  // MODE 4, 5: the trunk's last output, fixed point (xfix, 2^-32 units, MODE
  // 4) or FP32 (xf32, MODE 5); the accumulator that is zeroed, every row (fix_clear); the
  // final norm; hidden (written for active rows; inactive rows keep theirs);
  // the bookkeeping buffers, as final_norm_kernel's.
  const long long* xfix; const float* xf32; unsigned long long* fix_clear;
  const float* fnorm_w; float fnorm_eps; float* hidden_out;
  int* kv_len; int* pos; const int* active; int* counter;
  const double* u_ring; const int* flag_ring; double* u_cur; int* flag_cur; int nq; int max_frames;
  const float* inv_freq; int half; float2* rope; const float2* rope_tab; int tab_n;
};
constexpr int DEPTH_WGS = 256;

template <typename TL, int VPT, int M, int KD, int KI, int MODE>
__global__ __launch_bounds__(SNT) void depth_step_kernel(SampleArgs a, DepthArgs g, int q) {
  extern __shared__ unsigned char raw[];
  double* W = reinterpret_cast<double*>(raw);
  unsigned long long* ck = reinterpret_cast<unsigned long long*>(W + a.V);
  unsigned long long* sk = ck + pow2_ceil(a.V);
  constexpr bool SAMPLE = MODE == 2, GPART = MODE == 0 || MODE >= 4;
  constexpr bool DPART = MODE == 1 || MODE == 2, TAIL = MODE >= 4, TFIX = MODE == 4;
  constexpr int VEC = TL::VEC;
  constexpr int NV = KD / (64 * VEC);           // 16-byte loads per lane of one W_gu row
  constexpr int DPT = KD / SNT;                 // elements of x per thread
  constexpr int RWG = KI / (DEPTH_WGS * SWAVES);
  constexpr int RD = KD / DEPTH_WGS;
  static_assert(KD % (64 * VEC) == 0 && KD % SNT == 0 && KD % DEPTH_WGS == 0 && M <= 2, "depth_step shape");
  static_assert(RWG >= 1 && RWG * DEPTH_WGS * SWAVES == KI && KI == SWAVES * 64 * VEC, "depth_step inner");
  __shared__ SampleSmem s;
  __shared__ __attribute__((aligned(16))) float xsh[M * KD];
  __shared__ __attribute__((aligned(16))) float gsh[KD];
  __shared__ float red[M][SWAVES];
  __shared__ float dsum[SWAVES][RD][M];
  __shared__ int code_sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qs = q - 1;                         // the codebook sampled here (MODE 2)
  const bool lead = blockIdx.x == 0;

  // Loads that do not depend on the code, before the weight stream: the
  // logits first (the sampler waits for them), then the draw's inputs, the
  // hidden rows, the prefix and the norm gain.
  float xr[VPT], cvv[VPT], uvv[VPT];
  if constexpr (SAMPLE) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = min(tid + i * SNT, a.V - 1);
      cvv[i] = a.logits[v];
      uvv[i] = M == 2 ? a.logits[a.ldl + v] : 0.f;
    }
  }
  double u = 0.0;
  int forced = 0, slot = 0, mflag = 0;
  int64_t fcode = 0;
  SkParams P{};
  if constexpr (SAMPLE) {
    u = a.u_cur[qs];
    mflag = a.flag_cur[0];
    forced = a.flag_cur[1];
    P = *a.params;
  }
  float hv[M][DPT], pv[M][DPT], gv[DPT];
  // MODE 4, 5: the trunk's output rows (hv: fixed point in MODE 4, FP32 in
  // MODE 5), the final norm's gain (fw) and the rows' current hidden (kept by
  // inactive rows, in pv) -- loaded without branches, so they go out as one
  // batch ahead of the weight stream.
  float fw[TAIL ? DPT : 1];
  int act[M];
#pragma unroll
  for (int m = 0; m < M; ++m) act[m] = TAIL ? g.active[m] : 1;
  // ... and the step bookkeeping's independent inputs (every workgroup loads
  // them at clamped indices, only workgroup 0 uses them): thread t < M the
  // row's length and position, t < M * half the position of its RoPE row,
  // the frame counter.  The loads that depend on them (the RoPE table entry,
  // the next frame's draws and flags) follow the weight stream.
  int bk_kv = 0, bk_pos = 0, bk_cnt = 0, rp_row = 0, rp_t = 0, rp_pos = 0, rp_act = 0;
  if constexpr (TAIL) {
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    bk_cnt = g.counter[zero];
    const int rb = min(tid, M - 1);
    bk_kv = g.kv_len[rb];
    bk_pos = g.pos[rb];
    rp_row = min(tid / g.half, M - 1);
    rp_t = min(tid - rp_row * g.half, g.half - 1);
    rp_pos = g.pos[rp_row] + 1;
    rp_act = g.active[rp_row];
  }
#pragma unroll
  for (int i = 0; i < DPT; ++i) {
    const int k = tid + i * SNT;
    gv[i] = g.norm_w[k];
    if constexpr (TAIL) fw[i] = g.fnorm_w[k];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if constexpr (TFIX) hv[m][i] = (float)g.xfix[(size_t)m * KD + k] * 0x1p-32f;
      else if constexpr (TAIL) hv[m][i] = g.xf32[(size_t)m * KD + k];
      else hv[m][i] = g.hidden[(size_t)m * KD + k];
      pv[m][i] = TAIL ? g.hidden[(size_t)m * KD + k] : SAMPLE ? g.prefix_in[(size_t)m * KD + k] : 0.f;
    }
  }
  // G_q at this lane's inner indices of its wave's chunk (gate and up): at
  // entry without a sampler, else with the code's table entries after it
  // (they are needed only then, and they do not hold registers through it).
  const int kc = (wave * 64 + lane) * VEC;
  float gq[M][2][VEC];
  auto load_gq = [&]() {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < VEC; i += 4) {
          const float4 t = *reinterpret_cast<const float4*>(g.g_in + (size_t)m * 2 * KI + h * KI + kc + i);
          gq[m][h][i] = t.x; gq[m][h][i + 1] = t.y; gq[m][h][i + 2] = t.z; gq[m][h][i + 3] = t.w;
        }
  };
  if constexpr (MODE == 1) load_gq();
  // Weights: this wave's gate / up rows, this workgroup's down rows at the
  // chunk -- issued behind the logits and before any of them is used (the
  // scheduling barrier below keeps them there: sunk under the CFG merge they
  // started only once the logits had arrived).
  const int n0 = (blockIdx.x * SWAVES + wave) * RWG;
  uint4 wgu[GPART ? RWG : 1][2][NV];
  if constexpr (GPART) {
#pragma unroll
    for (int r = 0; r < RWG; ++r)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const size_t off = (size_t)(n0 + r) * KD + (size_t)(j * 64 + lane) * VEC;
        wgu[r][0][j] = TL::raw(g.w_gate, off);
        wgu[r][1][j] = TL::raw(g.w_up, off);
      }
  }
  // The down rows: at entry without a sampler; with one, once the logits
  // are merged (issued at entry, they delayed the logits the sampler waits
  // for: at the 1.7B shape its 16.8 MB held them back ~1.6 us), so they
  // stream while the sampler runs.
  const int row0 = blockIdx.x * RD;
  uint4 wd[DPART ? RD : 1];
  if constexpr (DPART && !SAMPLE) {
#pragma unroll
    for (int i = 0; i < RD; ++i) wd[i] = TL::raw(g.w_down, (size_t)(row0 + i) * KI + kc);
  }
  __builtin_amdgcn_sched_barrier(0);
  // MODE 4, 5: the bookkeeping loads that depend on a position or the frame
  // counter, behind the weights (their inputs were loaded ahead of them)
  double bk_u = 0.0;
  int bk_flag = 0;
  float2 bk_rp = make_float2(0.f, 0.f);
  if constexpr (TAIL) {
    bk_rp = g.rope_tab[(size_t)min(rp_pos, g.tab_n - 1) * g.half + rp_t];
    const int nx = min(bk_cnt + 1, g.max_frames - 1);
    bk_u = g.u_ring[(size_t)nx * g.nq + min(tid, g.nq - 1)];
    bk_flag = g.flag_ring[2 * nx + min(tid, 1)];
  }
  // The ring slot and the forced code as scalar loads behind the weights: a
  // vector load here would be waited for behind the whole weight stream, and
  // ahead of the weights its address chain held them back.
  if constexpr (SAMPLE) {
    slot = *a.fc;
    fcode = a.forced_ring[(size_t)slot * a.Q + qs];
  }
  if constexpr (SAMPLE) {
    const bool q0 = (qs == 0) && P.has_q0;
    merge_mask_loaded<VPT>(cvv, uvv, M == 2, P.cfg_scale, a.V, a.bos, a.eos, a.pad, &mflag, 0, qs != 0,
                           q0 ? P.temperature_q0 : P.temperature,
                           (lead && P.record_logits) ? a.dbg + (size_t)qs * a.V : nullptr, xr);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RD; ++i) wd[i] = TL::raw(g.w_down, (size_t)(row0 + i) * KI + kc);
    __builtin_amdgcn_sched_barrier(0);
  }

  // The code of codebook q-1 (every workgroup draws the same one), then its
  // table row and its code-table entries at this lane's chunk.
  int code = 0;
  float tv[DPT], pr[2][VEC];
  if constexpr (SAMPLE) {
    const bool q0 = (qs == 0) && P.has_q0;
    code = sample_core<VPT>(xr, a.V, q0 ? P.temperature_q0 : P.temperature, q0 ? P.top_k_q0 : P.top_k,
                            q0 ? P.top_p_q0 : P.top_p, u, ck, sk, W, s);
    const size_t uoff = (size_t)slot * a.Q + qs;
    if (tid == 0) {
      if (forced) code = (int)fcode;
      code = min(max(code, 0), a.V - 1);
      code_sh = code;
      if (lead) {
        a.codes_ring[uoff] = code;
        a.codes_cur[qs] = code;
      }
    }
    sk_sync();
    code = code_sh;
    const size_t trow = ((size_t)qs * a.V + code) * KD;
#pragma unroll
    for (int i = 0; i < DPT; ++i) tv[i] = TL::get(a.table, trow + tid + i * SNT);
    load_gq();
    const float* pp = g.ptab + ((size_t)qs * a.V + code) * 2 * KI + kc;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(pp + h * KI + i);
        pr[h][i] = t.x; pr[h][i + 1] = t.y; pr[h][i + 2] = t.z; pr[h][i + 3] = t.w;
      }
  }

  // MODE 4, 5: hidden = final_norm(trunk output) for active rows (the same
  // form as final_norm_kernel, w * (x * (1 / sqrt(mean(x^2) + eps)))); the
  // inactive rows keep their hidden.  Workgroup 0 stores it; every
  // workgroup zeroes its share of the accumulator the next frame's first
  // trunk launch adds into (a different buffer from xfix).
  if constexpr (TAIL) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < DPT; ++i) ss = fmaf(hv[m][i], hv[m][i], ss);
      ss = wave_sum_dpp(ss);
      if (lane == 0) red[m][wave] = ss;
    }
    sk_sync();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < SWAVES; ++w) t += red[m][w];
      const float invf = 1.0f / sqrtf(t / (float)KD + g.fnorm_eps);
#pragma unroll
      for (int i = 0; i < DPT; ++i) {
        const float h = fw[i] * (hv[m][i] * invf);
        hv[m][i] = act[m] ? h : pv[m][i];
        pv[m][i] = 0.f;
        if (lead && act[m]) g.hidden_out[(size_t)m * KD + tid + i * SNT] = h;
      }
    }
    if (g.fix_clear) {
      constexpr int CPW = M * KD / DEPTH_WGS;   // accumulator entries per workgroup
      if (tid < CPW) {
        g.fix_clear[blockIdx.x * CPW + tid] = 0ull;   // every row: a refill may make a retired row active again
      }
    }
    sk_sync();   // red is reused below
  }

  // x = hidden + (prefix + table row * scale), in the oracle's order; r = 1/rms(x)
#pragma unroll
  for (int i = 0; i < DPT; ++i) gsh[tid + i * SNT] = gv[i];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
      float x = hv[m][i];
      if constexpr (SAMPLE) {
        const float p = __fadd_rn(pv[m][i], __fmul_rn(tv[i], g.scale));
        x = __fadd_rn(hv[m][i], p);
        if (lead) g.prefix_out[(size_t)m * KD + tid + i * SNT] = p;
      }
      xsh[m * KD + tid + i * SNT] = x;
      ss = fmaf(x, x, ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[m][wave] = ss;
  }
  sk_sync();
  float inv[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < SWAVES; ++w) t += red[m][w];
    inv[m] = 1.0f / sqrtf(t / (float)KD + g.eps);
  }

  // G_{q+1} = W_gu (w_in * x_q): this wave's gate and up rows
  if constexpr (GPART) {
    float acc[RWG][2][M];
#pragma unroll
    for (int r = 0; r < RWG; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][h][m] = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int k0 = (j * 64 + lane) * VEC;
      float gw[VEC];
#pragma unroll
      for (int i = 0; i < VEC; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(&gsh[k0 + i]);
        gw[i] = t.x; gw[i + 1] = t.y; gw[i + 2] = t.z; gw[i + 3] = t.w;
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float x[VEC];
#pragma unroll
        for (int i = 0; i < VEC; i += 4) {
          const float4 t = *reinterpret_cast<const float4*>(&xsh[m * KD + k0 + i]);
          x[i] = __fmul_rn(gw[i], t.x); x[i + 1] = __fmul_rn(gw[i + 1], t.y);
          x[i + 2] = __fmul_rn(gw[i + 2], t.z); x[i + 3] = __fmul_rn(gw[i + 3], t.w);
        }
#pragma unroll
        for (int r = 0; r < RWG; ++r)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float w[VEC];
            TL::widen(wgu[r][h][j], w);
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[r][h][m] = fmaf(w[i], x[i], acc[r][h][m]);
          }
      }
    }
    // word (r * 2 + h) * M + m; its total lands in lanes word * (64 / NG) ...
    constexpr int NG = RWG * 2 * M;
    float wv[NG];
#pragma unroll
    for (int r = 0; r < RWG; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int m = 0; m < M; ++m) wv[(r * 2 + h) * M + m] = acc[r][h][m];
    const float tot = wave_reduce_words<NG>(wv, lane);
    if (lane % (64 / NG) == 0) {
      const int word = lane / (64 / NG), m = word % M, h = (word / M) % 2, r = word / (2 * M);
      g.g_out[(size_t)m * 2 * KI + h * KI + n0 + r] = tot;
    }
  }
  // MODE 4, 5, workgroup 0: the step bookkeeping from the values loaded
  // above (every read of them came before these writes: the barriers above
  // separate them).
  if constexpr (TAIL) {
    if (lead) {
      if (tid < M && act[tid]) { g.kv_len[tid] = bk_kv + 1; g.pos[tid] = bk_pos + 1; }
      if (tid < M * g.half && rp_act)
        g.rope[(size_t)rp_row * g.half + rp_t] = rp_pos < g.tab_n ? bk_rp : rope_cs(rp_pos, g.inv_freq[rp_t]);
      const int next = bk_cnt + 1;
      if (tid == 0) *g.counter = next;
      if (next < g.max_frames) {
        if (tid < g.nq) g.u_cur[tid] = bk_u;
        if (tid < 2) g.flag_cur[tid] = bk_flag;
      }
    }
  }

  // act = SwiGLU(r (G_q + scale P[c])) at this lane's chunk; y = a + W_d act
  if constexpr (DPART) {
    float act[M][VEC];
    float gnext[MODE == 2 ? M : 1][2][VEC];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float gt = gq[m][0][i], up = gq[m][1][i];
        if constexpr (SAMPLE) {
          gt = fmaf(g.scale, pr[0][i], gt);
          up = fmaf(g.scale, pr[1][i], up);
        }
        if constexpr (MODE == 2) {   // G_{q+1} = G_q + scale P_{q-1}[c]
          gnext[m][0][i] = gt;
          gnext[m][1][i] = up;
        }
        gt *= inv[m];
        up *= inv[m];
        // SwiGLU with the hardware exp2 and reciprocal (~1 ulp each): every
        // workgroup forms all of the step's inner activations, so their cost
        // is paid 256 times over.
        act[m][i] = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt)) * up;
      }
    if constexpr (MODE == 2) {
      if (lead) {   // every workgroup holds the same G_{q+1}; workgroup 0 stores it
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < VEC; i += 4)
              *reinterpret_cast<float4*>(g.g_out + (size_t)m * 2 * KI + h * KI + kc + i) =
                  make_float4(gnext[m][h][i], gnext[m][h][i + 1], gnext[m][h][i + 2], gnext[m][h][i + 3]);
      }
    }
    constexpr int ND = RD * M;                  // word i * M + m
    float dw[ND];
#pragma unroll
    for (int i = 0; i < RD; ++i) {
      float w[VEC];
      TL::widen(wd[i], w);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float t = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) t = fmaf(w[e], act[m][e], t);
        dw[i * M + m] = t;
      }
    }
    const float dt = wave_reduce_words<ND>(dw, lane);
    if (lane % (64 / ND) == 0) {
      const int word = lane / (64 / ND);
      dsum[wave][word / M][word % M] = dt;
    }
    sk_sync();
    if (tid < RD * M) {
      const int i = tid / M, m = tid - i * M, row = row0 + i;
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < SWAVES; ++w) t += dsum[w][i][m];
      const float av = gsh[row] * (xsh[m * KD + row] * inv[m]);   // residual a = w_in * (x * r)
      g.y[(size_t)m * KD + row] = av + t;
    }
  }
}

__host__ __device__ constexpr bool depth_step_fits(int d, int inner, int vec) {
  return (d == 1024 || d == 2048) && inner == SWAVES * 64 * vec && inner % (DEPTH_WGS * SWAVES) == 0;
}

// Code tables P_j[c] = W_gu (w_in * table[j][c]) are built with the prefill
// GEMM from rows of table[j] times the norm gain (FP32).
template <typename TL>
__global__ void scale_rows_kernel(const void* table, const float* gain, int rows, int d, float* out) {
  const size_t n = (size_t)rows * d;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = TL::get(table, i) * gain[i % d];
}

// Standalone sampler (operator API): one utterance, parameters by value.
template <int VPT>
__global__ __launch_bounds__(SNT) void sample_op_kernel(const float* logits, int rows, int V, float cfg, int q,
                                                       int mask_eos_q0, int bos, int eos, int pad, float temp,
                                                       int top_k, float top_p, double u, int64_t* code_out) {
  extern __shared__ unsigned char raw[];
  double* W = reinterpret_cast<double*>(raw);
  unsigned long long* ck = reinterpret_cast<unsigned long long*>(W + MAX_V);
  unsigned long long* sk = ck + MAX_V;
  __shared__ SampleSmem s;
  float xr[VPT];
  merge_mask<VPT>(logits, rows == 2 ? logits + V : nullptr, cfg, V, bos, eos, pad, nullptr, 0,
                  (q != 0) || mask_eos_q0 != 0, temp, nullptr, xr);
  const int code = sample_core<VPT>(xr, V, temp, top_k, top_p, u, ck, sk, W, s);
  if (threadIdx.x == 0) *code_out = code;
}

// Dynamic LDS of the samplers: W (MAX_V doubles), compaction / sort keys
// (MAX_V), sorted filter keys (FILTER_MAX).
constexpr size_t SAMPLE_SMEM = (size_t)MAX_V * sizeof(double) + (size_t)(MAX_V + FILTER_MAX) * 8;

// ------------------------------------------------------------ small kernels

// (cos, sin) table of rows row0 + blockIdx.x at their current positions.
__global__ __launch_bounds__(NT) void rope_rows_kernel(const int* pos, const float* inv_freq, int half, int row0,
                                                       float2* rope) {
  const int b = row0 + blockIdx.x;
  const int p = pos[b];
  for (int t = threadIdx.x; t < half; t += NT) rope[(size_t)b * half + t] = rope_cs(p, inv_freq[t]);
}

// Final trunk norm + per-row step bookkeeping after a decode trunk step: every
// active row advances its length and position (and its RoPE (cos, sin) to the
// new position), the frame counter moves on and the next frame's draws and flags
// are copied from the ring to the fixed current-frame slots.  With abuf set it
// also writes depth step 0's input, RMSNorm_in(hidden) (the codebook prefix is
// zero when a frame starts), and its split form when xs_abuf is set.  With
// xfix set the input row is the XCD-resident layers' fixed-point residual
// stream [rows][D] (2^-32 units) instead of x, and fix_clear (set with it) is
// the accumulator whose row this workgroup zeroes (an active row once the
// input is read, a retired row at once: the next frame's first layer adds
// into it for every row, and a refill may make the row active again).
__global__ __launch_bounds__(NT) void final_norm_kernel(const float* x, const long long* xfix,
                                                        unsigned long long* fix_clear, const float* w, float eps,
                                                        int D, float* hidden, int* kv_len, int* pos,
                                                        const int* active, int* counter,
                                                        const double* u_ring, const int* flag_ring,
                                                        double* u_cur, int* flag_cur, int nq,
                                                        int max_frames, const float* inv_freq, int half,
                                                        float2* rope, const float2* rope_tab, int tab_n,
                                                        const float* w_in, float eps_in, float* abuf,
                                                        uint16_t* xs_abuf) {
  __shared__ float red[WAVES];
  const int b = blockIdx.x, tx = threadIdx.x;
  // The bookkeeping's loads (step counters, the RoPE table row, the next
  // frame's draws and flags) are issued before the row's stores and held in
  // registers: issued where they are used, after those stores, each waited
  // for the stores and for the load before it.  The table row, draws and
  // flags are loaded right behind the row's loads (book()), unconditionally
  // at clamped indices (a load under a branch makes the join wait for it), so
  // rope_tab, u_ring and flag_ring must be valid buffers, and max_frames,
  // half, tab_n and nq at least 1 (the engine's config checks ensure both);
  // only the stores are conditional.  The frame counter is a vector load (opaque zero offset):
  // the first use of a scalar load waits for every scalar load in flight, and
  // the compiler puts that use ahead of the row's loads.  The asm statement
  // follows the scalar loads, since loads after it become vector loads too.
  // Every thread reads pos, kv_len and the counter before thread 0 writes
  // them (after the barriers in block_sum, or the one below); every
  // workgroup loads the counter, only workgroup 0 uses it.
  const int p0 = pos[b], kv0 = kv_len[b], np = p0 + 1;
  const bool act = active[b] != 0;
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  const int cnt = counter[zero];   // the frame counter; the next frame is cnt + 1
  int f0 = 0;
  double u0 = 0.0;
  float2 rp = make_float2(0.f, 0.f);
  auto book = [&]() {
    const int nx = min(cnt + 1, max_frames - 1);
    rp = rope_tab[(size_t)min(np, tab_n - 1) * half + min(tx, half - 1)];
    u0 = u_ring[(size_t)nx * nq + min(tx, nq - 1)];
    f0 = flag_ring[2 * nx + min(tx, 1)];
  };
  if (!act) book();
  if (!act && fix_clear)   // a retired row's entries too: a refill may make it active again
    for (int i = tx; i < D; i += NT) fix_clear[(size_t)b * D + i] = 0ull;
  if (act) {
    const float* xr = x + (size_t)b * D;
    const size_t ro = (size_t)b * D;
    constexpr int PER = 16;              // D <= 4096 in registers, all loads issued at once
    const bool al16 = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(xfix) |
                        reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(w_in) |
                        reinterpret_cast<uintptr_t>(hidden)) & 15u) == 0;
    if (al16 && D % (4 * NT) == 0 && D <= NT * PER) {
      // 16-byte loads: thread t holds elements 4 (t + i NT) .. + 3
      constexpr int P4 = PER / 4;
      const int n4 = D / (4 * NT);
      const float4* x4 = reinterpret_cast<const float4*>(xr);
      const float4* w4 = reinterpret_cast<const float4*>(w);
      const ulonglong2* f2 = xfix ? reinterpret_cast<const ulonglong2*>(xfix + ro) : nullptr;
      float4 xv[P4], wv[P4], gv[P4];
      ulonglong2 fv[P4][2];
      // every load first, then the bookkeeping's, then the sums; chunks past
      // n4 re-read the last element (no branch, so no wait between the
      // chunks' loads) and are discarded
#pragma unroll
      for (int i = 0; i < P4; ++i) {
        const int k4 = min(tx + i * NT, D / 4 - 1);
        if (xfix) {
          fv[i][0] = f2[2 * k4];
          fv[i][1] = f2[2 * k4 + 1];
        } else {
          xv[i] = x4[k4];
        }
        wv[i] = w4[k4];
        gv[i] = abuf ? reinterpret_cast<const float4*>(w_in)[k4] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      book();
      if (xfix) {   // the XCD-resident layers' fixed-point residual stream (2^-32 units)
#pragma unroll
        for (int i = 0; i < P4; ++i)
          xv[i] = make_float4((float)(long long)fv[i][0].x * 0x1p-32f, (float)(long long)fv[i][0].y * 0x1p-32f,
                              (float)(long long)fv[i][1].x * 0x1p-32f, (float)(long long)fv[i][1].y * 0x1p-32f);
      }
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < P4; ++i)
        if (i < n4) s += xv[i].x * xv[i].x + xv[i].y * xv[i].y + xv[i].z * xv[i].z + xv[i].w * xv[i].w;
      const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
      if (fix_clear) {   // every thread's loads are consumed: the row may be the one read
        ulonglong2* c2 = reinterpret_cast<ulonglong2*>(fix_clear + ro);
#pragma unroll
        for (int i = 0; i < P4; ++i)
          if (i < n4) {
            c2[2 * (tx + i * NT)] = make_ulonglong2(0ull, 0ull);
            c2[2 * (tx + i * NT) + 1] = make_ulonglong2(0ull, 0ull);
          }
      }
      float s2 = 0.f;
      float4* h4 = reinterpret_cast<float4*>(hidden + ro);
#pragma unroll
      for (int i = 0; i < P4; ++i) {
        const float4 y = make_float4(wv[i].x * (xv[i].x * inv), wv[i].y * (xv[i].y * inv), wv[i].z * (xv[i].z * inv),
                                     wv[i].w * (xv[i].w * inv));
        xv[i] = y;
        if (i < n4) {
          h4[threadIdx.x + i * NT] = y;
          s2 = fmaf(y.x, y.x, fmaf(y.y, y.y, fmaf(y.z, y.z, fmaf(y.w, y.w, s2))));
        }
      }
      // Depth step 0's input: the prefix is zero at the start of a frame.
      if (abuf) {
        const float inv2 = 1.0f / sqrtf(block_sum(s2, red) / (float)D + eps_in);
#pragma unroll
        for (int i = 0; i < P4; ++i) {
          if (i < n4) {
            const int k = 4 * ((int)threadIdx.x + i * NT);
            const float y[4] = {gv[i].x * (xv[i].x * inv2), gv[i].y * (xv[i].y * inv2), gv[i].z * (xv[i].z * inv2),
                                gv[i].w * (xv[i].w * inv2)};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              abuf[ro + k + c] = y[c];
              if (xs_abuf) xsplit_store(xs_abuf, b, k + c, y[c]);
            }
          }
        }
      }
    } else if (D <= NT * PER) {
      float xv[PER], wv[PER], gv[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int k = min((int)threadIdx.x + i * NT, D - 1);
        xv[i] = xfix ? (float)xfix[ro + k] * 0x1p-32f : xr[k];
        wv[i] = w[k];
        gv[i] = abuf ? w_in[k] : 0.f;
      }
      book();
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if ((int)threadIdx.x + i * NT < D) s += xv[i] * xv[i];
      const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
      if (fix_clear) {
#pragma unroll
        for (int i = 0; i < PER; ++i)
          if ((int)threadIdx.x + i * NT < D) fix_clear[ro + threadIdx.x + i * NT] = 0ull;
      }
      float s2 = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int k = threadIdx.x + i * NT;
        xv[i] = wv[i] * (xv[i] * inv);
        if (k < D) {
          hidden[ro + k] = xv[i];
          s2 = fmaf(xv[i], xv[i], s2);
        }
      }
      // Depth step 0's input: the prefix is zero at the start of a frame.
      if (abuf) {
        const float inv2 = 1.0f / sqrtf(block_sum(s2, red) / (float)D + eps_in);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int k = threadIdx.x + i * NT;
          if (k < D) {
            const float y = gv[i] * (xv[i] * inv2);
            abuf[ro + k] = y;
            if (xs_abuf) xsplit_store(xs_abuf, b, k, y);
          }
        }
      }
    } else {   // (the fixed-point input is only used with D <= NT * PER)
      book();
      float s = 0.f;
      for (int k = threadIdx.x; k < D; k += NT) s += xr[k] * xr[k];
      const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
      float s2 = 0.f;
      for (int k = threadIdx.x; k < D; k += NT) {
        const float h = w[k] * (xr[k] * inv);
        hidden[ro + k] = h;
        s2 = fmaf(h, h, s2);
      }
      if (abuf) {
        const float inv2 = 1.0f / sqrtf(block_sum(s2, red) / (float)D + eps_in);
        for (int k = threadIdx.x; k < D; k += NT) {
          const float y = w_in[k] * (hidden[ro + k] * inv2);
          abuf[ro + k] = y;
          if (xs_abuf) xsplit_store(xs_abuf, b, k, y);
        }
      }
    }
    if (tx == 0) { kv_len[b] = kv0 + 1; pos[b] = np; }
    // (cos, sin) of the new position: from the per-position table, computed
    // only for positions past it
    for (int t = tx; t < half; t += NT)
      rope[(size_t)b * half + t] = np < tab_n ? (t == tx ? rp : rope_tab[(size_t)np * half + t])
                                              : rope_cs(np, inv_freq[t]);
  }
  if (b == 0) {
    __syncthreads();
    const int next = cnt + 1;
    if (tx == 0) *counter = next;
    if (next < max_frames) {
      for (int i = tx; i < nq; i += NT) u_cur[i] = i == tx ? u0 : u_ring[(size_t)next * nq + i];
      if (tx < 2) flag_cur[tx] = f0;
    }
  }
}

// Prefix embeddings of one row: text rows (language rows replaced,
// model.py:326-338), then frame embeddings (model.py:105-114).
template <typename TL>
__global__ __launch_bounds__(NT) void embed_prefix_kernel(const int64_t* ids, int n_text,
                                                          const int64_t* codes, const void* embed,
                                                          const float* lang_table, int n_lang,
                                                          int l0, int l1, int l2, int l3,
                                                          const void* table, int Q, int V, int D,
                                                          float scale, float* out) {
  const int i = blockIdx.x;
  float* o = out + (size_t)i * D;
  if (i < n_text) {
    const int64_t id = ids[i];
    int lj = -1;
    if (n_lang > 0) lj = (id == l0) ? 0 : (id == l1) ? 1 : (id == l2) ? 2 : (id == l3) ? 3 : -1;
    for (int k = threadIdx.x; k < D; k += NT)
      o[k] = (lj >= 0) ? lang_table[(size_t)lj * D + k] : TL::get(embed, (size_t)id * D + k);
  } else {
    const int64_t* c = codes + (size_t)(i - n_text) * Q;
    for (int k = threadIdx.x; k < D; k += NT) {
      float e = 0.f;
      for (int j = 0; j < Q; ++j) {
        const float t = TL::get(table, ((size_t)j * V + (size_t)c[j]) * D + k);
        e = (j == 0) ? t : __fadd_rn(e, t);
      }
      o[k] = __fmul_rn(e, scale);
    }
  }
}

// ---- operator-API elementwise kernels (tilelang_kernels.py:176-254) ----
__global__ __launch_bounds__(NT) void frame_embed_op_kernel(const int64_t* codes, const float* table,
                                                            int Q, int V, int D, float scale,
                                                            float* out) {
  const int r = blockIdx.x;
  for (int k = threadIdx.x; k < D; k += NT) {
    float e = 0.f;
    for (int j = 0; j < Q; ++j) {
      const int64_t cj = codes[(size_t)r * Q + j];
      const int64_t c = cj < 0 ? 0 : (cj >= V ? V - 1 : cj);
      const float t = table[((size_t)j * V + (size_t)c) * D + k];
      e = (j == 0) ? t : __fadd_rn(e, t);
    }
    out[(size_t)r * D + k] = __fmul_rn(e, scale);
  }
}

__global__ __launch_bounds__(NT) void prefix_add_op_kernel(const float* prefix, const float* table_q,
                                                           const int64_t* code, int V, int D,
                                                           float scale, float* out) {
  const int b = blockIdx.x;
  const int64_t c = *code < 0 ? 0 : (*code >= V ? V - 1 : *code);
  for (int k = threadIdx.x; k < D; k += NT)
    out[(size_t)b * D + k] =
        __fadd_rn(prefix[(size_t)b * D + k], __fmul_rn(table_q[(size_t)c * D + k], scale));
}

__global__ __launch_bounds__(NT) void sampling_prep_op_kernel(const float* logits, const float* temp,
                                                              const int* mask_eos, int V, int bos,
                                                              int pad, int eos, float* out) {
  const int v = blockIdx.x * NT + threadIdx.x;
  if (v >= V) return;
  float x = logits[v] / temp[0];
  if (v == bos || v == pad || (mask_eos[0] > 0 && v == eos)) x = -INFINITY;
  out[v] = x;
}

}  // namespace
}  // namespace sk
