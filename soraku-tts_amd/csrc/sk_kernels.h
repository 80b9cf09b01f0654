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
constexpr int ATT_CHUNK = 64; // KV tokens per attention workgroup
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
};

// ------------------------------------------------------------ GEMV family
// y[m][n] = sum_k x[m][k] * W[n][k] for M activation rows (decode rows).
enum { PRO_NONE = 0, PRO_NORM = 1, PRO_ADDNORM = 2 };
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
};

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

  for (int m = 0; m < M; ++m)
    for (int k = tid; k < K; k += NT) {
      float v = a.x[(size_t)m * a.ldx + k];
      if (PRO == PRO_ADDNORM) v += a.x2[(size_t)m * a.ldx2 + k];
      xs[m * K + k] = v;
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

// ------------------------------------------------------------ attention
// One decode token per row against that row's own cache (per-row length and
// RoPE position; CFG rows differ in length).  Grid (chunks, Hkv, rows); the
// workgroup of chunk c handles KV tokens [c*64, c*64+64).  Each workgroup
// applies q_norm/k_norm + RoPE itself (Qwen3 norms per head before RoPE); the
// workgroup owning the new token also appends it to the cache.  Partial
// (max, sum, o) per chunk go to scratch; the last workgroup of a (row, kv head)
// to finish merges them in chunk order, so results do not depend on timing.
struct AttnArgs {
  const float* qkv; int ldqkv;           // [rows][(Hq + 2 Hkv) hd] raw projections
  float* kc; float* vc;                  // this layer: [rows][Hkv][max_ctx][hd]
  const float* qn_w; const float* kn_w; float eps;
  const float* rope_cos; const float* rope_sin;  // [max_ctx][hd/2]
  const int* kv_len; const int* pos; const int* active;
  float* part; int* counters;            // [rows][Hq][max_chunks][hd+2], [rows][Hkv]
  float* out; int ldo;                   // [rows][Hq hd]
  int Hq, Hkv, hd, max_ctx, max_chunks;
  float scale;
};

__global__ __launch_bounds__(NT) void attention_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int c = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  if (!a.active[r]) return;
  const int T = a.kv_len[r];             // cached tokens; the new one goes to slot T
  const int ctx = T + 1;
  const int nch = (ctx + ATT_CHUNK - 1) / ATT_CHUNK;
  if (c >= nch) return;
  const int G = a.Hq / a.Hkv, hd = a.hd, half = hd / 2;
  const int p = a.pos[r];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool last = (c == nch - 1);

  float* qs = sm;                        // [G][hd]
  float* knew = qs + G * hd;             // [hd]
  float* vnew = knew + hd;               // [hd]
  float* sc = vnew + hd;                 // [G][CHUNK]
  float* mls = sc + G * ATT_CHUNK;       // [G][2]
  __shared__ int is_last;

  const float* row = a.qkv + (size_t)r * a.ldqkv;
  for (int i = tid; i < G * hd; i += NT) qs[i] = row[(size_t)h * G * hd + i];
  if (last)
    for (int i = tid; i < hd; i += NT) {
      knew[i] = row[(size_t)a.Hq * hd + (size_t)h * hd + i];
      vnew[i] = row[(size_t)(a.Hq + a.Hkv) * hd + (size_t)h * hd + i];
    }
  __syncthreads();

  // Per-head RMSNorm over hd, then rotate-half RoPE; one wave per head.
  const int nheads = G + (last ? 1 : 0);
  const float* cs = a.rope_cos + (size_t)p * half;
  const float* sn = a.rope_sin + (size_t)p * half;
  for (int j = wave; j < nheads; j += WAVES) {
    float* v = (j < G) ? qs + j * hd : knew;
    const float* w = (j < G) ? a.qn_w : a.kn_w;
    float s = 0.f;
    for (int d = lane; d < hd; d += 64) s += v[d] * v[d];
    const float inv = 1.0f / sqrtf(wave_sum(s) / (float)hd + a.eps);
    for (int d = lane; d < half; d += 64) {
      const float x1 = w[d] * (v[d] * inv);
      const float x2 = w[d + half] * (v[d + half] * inv);
      v[d] = x1 * cs[d] - x2 * sn[d];
      v[d + half] = x2 * cs[d] + x1 * sn[d];
    }
  }
  __syncthreads();

  const size_t head_base = ((size_t)r * a.Hkv + h) * a.max_ctx;
  if (last)
    for (int d = tid; d < hd; d += NT) {
      a.kc[(head_base + T) * hd + d] = knew[d];
      a.vc[(head_base + T) * hd + d] = vnew[d];
    }

  // Scores: LPT lanes per token, 8 dims per lane.
  const int LPT = hd / 8;
  const int TPI = NT / LPT;
  const int grp = tid / LPT, sub = tid % LPT;
  const int t_begin = c * ATT_CHUNK;
  const int n_t = min(ATT_CHUNK, ctx - t_begin);
  for (int t0 = 0; t0 < ATT_CHUNK; t0 += TPI) {
    const int tl = t0 + grp;
    const int t = t_begin + tl;
    float kv8[8];
    if (tl < n_t) {
      if (t == T) {
#pragma unroll
        for (int j = 0; j < 8; ++j) kv8[j] = knew[sub * 8 + j];
      } else {
        const float4* kp = reinterpret_cast<const float4*>(a.kc + (head_base + t) * hd + sub * 8);
        const float4 k0 = kp[0], k1 = kp[1];
        kv8[0] = k0.x; kv8[1] = k0.y; kv8[2] = k0.z; kv8[3] = k0.w;
        kv8[4] = k1.x; kv8[5] = k1.y; kv8[6] = k1.z; kv8[7] = k1.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) kv8[j] = 0.f;
    }
    for (int g = 0; g < G; ++g) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s = fmaf(qs[g * hd + sub * 8 + j], kv8[j], s);
      for (int o = LPT / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      if (sub == 0 && tl < n_t) sc[g * ATT_CHUNK + tl] = s * a.scale;
    }
  }
  __syncthreads();

  // Chunk softmax statistics: one wave per q head, one lane per token.
  for (int g = wave; g < G; g += WAVES) {
    const float v = (lane < n_t) ? sc[g * ATT_CHUNK + lane] : -INFINITY;
    const float m = wave_max(v);
    const float e = (lane < n_t) ? expf(v - m) : 0.f;
    const float l = wave_sum(e);
    sc[g * ATT_CHUNK + lane] = e;
    if (lane == 0) { mls[2 * g] = m; mls[2 * g + 1] = l; }
  }
  __syncthreads();

  const int stride = hd + 2;
  for (int i = tid; i < G * hd; i += NT) {
    const int g = i / hd, d = i - g * hd;
    float o = 0.f;
    for (int tl = 0; tl < n_t; ++tl) {
      const int t = t_begin + tl;
      const float v = (t == T) ? vnew[d] : a.vc[(head_base + t) * hd + d];
      o = fmaf(sc[g * ATT_CHUNK + tl], v, o);
    }
    float* pp = a.part + (((size_t)r * a.Hq + h * G + g) * a.max_chunks + c) * stride;
    pp[d] = o;
    if (d == 0) { pp[hd] = mls[2 * g]; pp[hd + 1] = mls[2 * g + 1]; }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int old = atomicAdd(&a.counters[r * a.Hkv + h], 1);
    is_last = (old == nch - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int i = tid; i < G * hd; i += NT) {
    const int g = i / hd, d = i - g * hd;
    const float* pp = a.part + (((size_t)r * a.Hq + h * G + g) * a.max_chunks) * stride;
    float M = -INFINITY;
    for (int cc = 0; cc < nch; ++cc) M = fmaxf(M, __builtin_nontemporal_load(&pp[cc * stride + hd]));
    float L = 0.f, O = 0.f;
    for (int cc = 0; cc < nch; ++cc) {
      const float f = expf(__builtin_nontemporal_load(&pp[cc * stride + hd]) - M);
      L = fmaf(__builtin_nontemporal_load(&pp[cc * stride + hd + 1]), f, L);
      O = fmaf(__builtin_nontemporal_load(&pp[cc * stride + d]), f, O);
    }
    a.out[(size_t)r * a.ldo + (size_t)(h * G + g) * hd + d] = O / L;
  }
  if (tid == 0) a.counters[r * a.Hkv + h] = 0;
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

struct SampleSmem {
  int hist[256];
  int scan[WAVES];
  int n;
  int code;
  uint32_t prefix;
  int sel_digit;
  int sel_excl;
  float bv[WAVES];
  int bi[WAVES];
};

// x[0..V) in LDS (already CFG-merged and masked).  Follows model.py:686-708:
// greedy argmax when temperature <= 0; else x / T, top-k (ties kept), top-p
// (shift-by-one, first kept) and the explicit-uniform inverse-CDF draw in
// float64 over candidates ordered by value desc, index asc.
// cv/ci: candidate arrays of MAX_V entries; W: MAX_V doubles.
__device__ int sample_core(float* x, int V, float temp, int top_k, float top_p, double u,
                           float* cv, int* ci, double* W, SampleSmem& s) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (!(temp > 0.f)) {
    float bv = -INFINITY; int bi = 0x7fffffff;
    for (int v = tid; v < V; v += NT) {
      const float f = x[v];
      if (f > bv || bi == 0x7fffffff) { bv = f; bi = v; }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { s.bv[wave] = bv; s.bi[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
      float b = s.bv[0]; int i = s.bi[0];
      for (int w = 1; w < WAVES; ++w)
        if (s.bv[w] > b || (s.bv[w] == b && s.bi[w] < i)) { b = s.bv[w]; i = s.bi[w]; }
      s.code = i;
    }
    __syncthreads();
    return s.code;
  }
  for (int v = tid; v < V; v += NT) x[v] = x[v] / temp;
  __syncthreads();

  // k-th largest key by 8-bit radix select (MSB first).
  uint32_t cut = 0u;
  if (top_k > 0 && top_k < V) {
    uint32_t prefix = 0u, pmask = 0u;
    int kr = top_k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      s.hist[tid] = 0;
      __syncthreads();
      for (int v = tid; v < V; v += NT) {
        const uint32_t key = fkey(x[v]);
        if ((key & pmask) == prefix) atomicAdd(&s.hist[(key >> shift) & 255u], 1);
      }
      __syncthreads();
      // Inclusive scan over bins 255..0 (thread t holds bin 255 - t).
      const int cnt = s.hist[255 - tid];
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      if (lane == 63) s.scan[wave] = incl;
      __syncthreads();
      for (int w = 0; w < wave; ++w) incl += s.scan[w];
      const int excl = incl - cnt;
      if (cnt > 0 && excl < kr && kr <= incl) { s.sel_digit = 255 - tid; s.sel_excl = excl; }
      __syncthreads();
      prefix |= (uint32_t)s.sel_digit << shift;
      pmask |= 255u << shift;
      kr -= s.sel_excl;
      __syncthreads();
    }
    cut = prefix;
  }

  if (tid == 0) s.n = 0;
  __syncthreads();
  for (int v = tid; v < V; v += NT) {
    const float f = x[v];
    if (isfinite(f) && fkey(f) >= cut) {
      const int slot = atomicAdd(&s.n, 1);
      cv[slot] = f; ci[slot] = v;
    }
  }
  __syncthreads();
  const int n = s.n;
  int P = 1;
  while (P < n) P <<= 1;
  for (int i = n + tid; i < P; i += NT) { cv[i] = -INFINITY; ci[i] = 0x7fffffff; }
  __syncthreads();
  // Bitonic sort: "before" = larger value, then smaller index.
  for (int k = 2; k <= P; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P; i += NT) {
        const int l = i ^ j;
        if (l > i) {
          const float vi = cv[i], vl = cv[l];
          const int ii = ci[i], il = ci[l];
          const bool l_before = (vl > vi) || (vl == vi && il < ii);
          const bool i_before = (vi > vl) || (vi == vl && ii < il);
          const bool swap = ((i & k) == 0) ? l_before : i_before;
          if (swap) { cv[i] = vl; cv[l] = vi; ci[i] = il; ci[l] = ii; }
        }
      }
      __syncthreads();
    }
  const double top = (double)cv[0];
  for (int i = tid; i < n; i += NT) W[i] = exp((double)cv[i] - top);
  __syncthreads();
  if (tid == 0 && n == 0) s.code = 0;  // no finite logit (non-finite input): fixed, in-range code
  if (tid == 0 && n > 0) {
    double acc = 0.0;
    for (int i = 0; i < n; ++i) { acc += W[i]; W[i] = acc; }
    int nk = n;
    if (top_p > 0.f && top_p < 1.f) {
      const double pp = (double)top_p;
      for (int i = 0; i + 1 < n; ++i)
        if (W[i] / acc > pp) { nk = i + 1; break; }
    }
    const double target = u * W[nk - 1];
    int j = nk - 1;
    for (int i = 0; i < nk; ++i)
      if (W[i] > target) { j = i; break; }
    s.code = ci[j];
  }
  __syncthreads();
  return s.code;
}

// CFG merge u + s (c - u) without contraction, then BOS/PAD (and EOS) -> -inf
// (model.py:579-584).
__device__ __forceinline__ void merge_mask(const float* lc, const float* lu, float s, int V,
                                           int bos, int eos, int pad, bool mask_eos, float* x) {
  for (int v = threadIdx.x; v < V; v += NT) {
    float m = lc[v];
    if (lu) {
      const float uu = lu[v];
      m = __fadd_rn(uu, __fmul_rn(s, __fsub_rn(m, uu)));
    }
    if (v == bos || v == pad || (mask_eos && v == eos)) m = -INFINITY;
    x[v] = m;
  }
}

struct SampleArgs {
  const float* logits; int ldl; int rows_per_utt; int V;
  const SkParams* params;
  const int* fc;                       // device frame counter -> ring slot
  const double* u_ring;                // [frames][n_utts][Q]
  const int* flag_ring;                // [frames][2] (mask_eos_q0, forced)
  const int64_t* forced_ring;          // [frames][n_utts][Q]
  int64_t* codes_ring;                 // [frames][n_utts][Q]
  float* dbg;                          // [n_utts][Q][V]
  const void* table;                   // [Q][V][d]
  float* prefix; float* xnext;         // [rows][d]
  int d, Q; float scale;
  int bos, eos, pad;
  int n_utts;
};

// One workgroup per utterance, launched once per codebook q.  Samples the
// code, records it, advances both rows' prefix (model.py:600-605) and, after
// the last codebook, writes the frame embedding (model.py:105-114) as the next
// trunk input and clears the prefix.
template <typename TL>
__global__ __launch_bounds__(NT) void sample_step_kernel(SampleArgs a, int q) {
  extern __shared__ unsigned char raw[];
  double* W = reinterpret_cast<double*>(raw);
  float* x = reinterpret_cast<float*>(W + MAX_V);
  float* cv = x + MAX_V;
  int* ci = reinterpret_cast<int*>(cv + MAX_V);
  __shared__ SampleSmem s;
  __shared__ int64_t codes_l[64];

  const int ut = blockIdx.x;
  const SkParams P = *a.params;
  const int slot = *a.fc;
  const int* flags = a.flag_ring + 2 * slot;
  const int r0 = ut * a.rows_per_utt;
  const float* lc = a.logits + (size_t)r0 * a.ldl;
  const float* lu = (a.rows_per_utt == 2) ? lc + a.ldl : nullptr;
  const bool mask_eos = (q != 0) || flags[0] != 0;
  merge_mask(lc, lu, P.cfg_scale, a.V, a.bos, a.eos, a.pad, mask_eos, x);
  __syncthreads();
  if (P.record_logits)
    for (int v = threadIdx.x; v < a.V; v += NT)
      a.dbg[((size_t)ut * a.Q + q) * a.V + v] = x[v];
  const bool q0 = (q == 0) && P.has_q0;
  const float temp = q0 ? P.temperature_q0 : P.temperature;
  const int topk = q0 ? P.top_k_q0 : P.top_k;
  const float topp = q0 ? P.top_p_q0 : P.top_p;
  const size_t uoff = ((size_t)slot * a.n_utts + ut) * a.Q + q;
  int code = sample_core(x, a.V, temp, topk, topp, a.u_ring[uoff], cv, ci, W, s);
  if (flags[1]) code = (int)a.forced_ring[uoff];
  code = min(max(code, 0), a.V - 1);
  if (threadIdx.x == 0) a.codes_ring[uoff] = code;

  const size_t row_stride = (size_t)a.V * a.d;
  if (q + 1 < a.Q) {
    const size_t base = (size_t)q * row_stride + (size_t)code * a.d;
    for (int dd = threadIdx.x; dd < a.d; dd += NT) {
      const float t = __fmul_rn(TL::get(a.table, base + dd), a.scale);
      for (int rr = 0; rr < a.rows_per_utt; ++rr) {
        float* pr = a.prefix + (size_t)(r0 + rr) * a.d;
        pr[dd] = __fadd_rn(pr[dd], t);
      }
    }
  } else {
    if (threadIdx.x < a.Q)
      codes_l[threadIdx.x] = (threadIdx.x == q) ? (int64_t)code
                                                : a.codes_ring[((size_t)slot * a.n_utts + ut) * a.Q + threadIdx.x];
    __syncthreads();
    for (int dd = threadIdx.x; dd < a.d; dd += NT) {
      float e = 0.f;
      for (int j = 0; j < a.Q; ++j) {
        const float t = TL::get(a.table, (size_t)j * row_stride + (size_t)codes_l[j] * a.d + dd);
        e = (j == 0) ? t : __fadd_rn(e, t);
      }
      e = __fmul_rn(e, a.scale);
      for (int rr = 0; rr < a.rows_per_utt; ++rr) {
        a.xnext[(size_t)(r0 + rr) * a.d + dd] = e;
        a.prefix[(size_t)(r0 + rr) * a.d + dd] = 0.f;
      }
    }
  }
}

// Standalone sampler (operator API): one utterance, parameters by value.
__global__ __launch_bounds__(NT) void sample_op_kernel(const float* logits, int rows, int V,
                                                       float cfg, int q, int mask_eos_q0, int bos,
                                                       int eos, int pad, float temp, int top_k,
                                                       float top_p, double u, int64_t* code_out) {
  extern __shared__ unsigned char raw[];
  double* W = reinterpret_cast<double*>(raw);
  float* x = reinterpret_cast<float*>(W + MAX_V);
  float* cv = x + MAX_V;
  int* ci = reinterpret_cast<int*>(cv + MAX_V);
  __shared__ SampleSmem s;
  merge_mask(logits, rows == 2 ? logits + V : nullptr, cfg, V, bos, eos, pad,
             (q != 0) || mask_eos_q0 != 0, x);
  __syncthreads();
  const int code = sample_core(x, V, temp, top_k, top_p, u, cv, ci, W, s);
  if (threadIdx.x == 0) *code_out = code;
}

constexpr size_t SAMPLE_SMEM = (size_t)MAX_V * (sizeof(double) + 2 * sizeof(float) + sizeof(int));

// ------------------------------------------------------------ small kernels
// Final trunk norm + per-row step bookkeeping.  mode 0: decode frame (every
// row advances, frame counter += 1); mode 1: prefill token (active rows only,
// prefill step += 1).
__global__ __launch_bounds__(NT) void final_norm_kernel(const float* x, const float* w, float eps,
                                                        int D, float* hidden, int* kv_len, int* pos,
                                                        const int* active, int* counter) {
  __shared__ float red[WAVES];
  const int b = blockIdx.x;
  if (active[b]) {
    const float* xr = x + (size_t)b * D;
    float s = 0.f;
    for (int k = threadIdx.x; k < D; k += NT) s += xr[k] * xr[k];
    const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
    for (int k = threadIdx.x; k < D; k += NT) hidden[(size_t)b * D + k] = w[k] * (xr[k] * inv);
    if (threadIdx.x == 0) { kv_len[b] += 1; pos[b] += 1; }
  }
  if (b == 0 && threadIdx.x == 0) *counter += 1;
}

// Prefill token t = *step: row b takes embeds[b][t] if t < len[b].
__global__ __launch_bounds__(NT) void prefill_load_kernel(const float* embeds, int max_len,
                                                          const int* len, const int* step, int D,
                                                          float* x, int* active) {
  const int b = blockIdx.x;
  const int t = *step;
  const bool on = t < len[b];
  for (int k = threadIdx.x; k < D; k += NT)
    x[(size_t)b * D + k] = on ? embeds[((size_t)b * max_len + t) * D + k] : 0.f;
  if (threadIdx.x == 0) active[b] = on ? 1 : 0;
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
