// Batched prefill kernels: every prefix token of every row goes through the
// trunk at once (model.py:623-656 over Qwen3Model.forward,
// modeling_qwen3.py:367-427).  Tokens are packed row after row: token m is
// row tok_row[m] at position tok_pos[m]; row r's tokens start at row_start[r].
//
//   X = embeds -> per layer: Xn = RMSNorm(X); QKV = Xn Wqkv^T (MFMA GEMM);
//   QK-norm + RoPE, K/V written into the decode cache; causal attention per
//   row; X += Att Wo^T; Xn = RMSNorm(X); Act = silu(Xn Wg^T) * (Xn Wu^T);
//   X += Act Wd^T -> hidden = RMSNorm_final(X[last token of each row]).
#pragma once

#include <hip/hip_runtime.h>

#include "sk_kernels.h"

namespace sk {

// ------------------------------------------------------------ GEMM
// C[M][N] = A[M][K] . B[N][K]^T on the FP32 matrix cores
// (v_mfma_f32_16x16x4f32), 64 x 64 tiles, K in steps of 16 through LDS.  B
// (weights, FP32 or BF16 widened on load) may be split into up to three row
// segments (q / k / v projections).  Epilogues: store, residual add
// (out = res + C, res may alias out), SwiGLU (out = silu(A Bg^T) * (A Bu^T),
// B2 = up weights).  M, N arbitrary (rows past the end are clamped on load and
// not stored); K a multiple of 16.
enum { GEPI_STORE = 0, GEPI_RESID = 1, GEPI_SWIGLU = 2 };

struct GemmArgs {
  const float* A; int lda;
  const void* B[3]; int seg_rows[3];
  const void* B2;
  float* out; int ldo;
  const float* res; int ldr;
  int M, N, K;
};

constexpr int GBM = 64, GBN = 64, GBK = 16;
constexpr int GLD = GBM + 16;   // LDS row stride (floats): lanes 16 apart in k land 16 banks apart

typedef float v4f __attribute__((ext_vector_type(4)));

template <typename WL>
__device__ __forceinline__ float4 load_w4(const void* base, size_t off) {
  if constexpr (sizeof(typename WL::elem) == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
    return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                       __uint_as_float(v.y & 0xffff0000u));
  } else {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
  }
}

template <int EPI, typename WL>
__global__ __launch_bounds__(256) void gemm_nt_kernel(GemmArgs a) {
  constexpr int NB = (EPI == GEPI_SWIGLU) ? 2 : 1;
  __shared__ __attribute__((aligned(16))) float As[GBK][GLD];
  __shared__ __attribute__((aligned(16))) float Bs[NB][GBK][GLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * GBM;
  // loader: thread -> (tile row lr, k offset lk)
  const int lr = tid >> 2, lk = (tid & 3) * 4;
  const int am = min(m0 + lr, a.M - 1);
  const float* arow = a.A + (size_t)am * a.lda + lk;
  const int bn = min(n0 + lr, a.N - 1);
  const void* bbase;
  int brow;
  if (bn < a.seg_rows[0]) { bbase = a.B[0]; brow = bn; }
  else if (bn < a.seg_rows[0] + a.seg_rows[1]) { bbase = a.B[1]; brow = bn - a.seg_rows[0]; }
  else { bbase = a.B[2]; brow = bn - a.seg_rows[0] - a.seg_rows[1]; }
  const size_t boff = (size_t)brow * a.K + lk;
  const size_t b2off = (size_t)bn * a.K + lk;
  // wave tile: 32 x 32 at (wm, wn), 2 x 2 MFMA tiles of 16 x 16
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  v4f acc[NB][2][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[b][i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < a.K; k0 += GBK) {
    const float4 av = *reinterpret_cast<const float4*>(arow + k0);
    const float4 bv = load_w4<WL>(bbase, boff + k0);
    float4 bv2 = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (NB == 2) bv2 = load_w4<WL>(a.B2, b2off + k0);
    __syncthreads();   // previous step's reads are done
    As[lk + 0][lr] = av.x; As[lk + 1][lr] = av.y; As[lk + 2][lr] = av.z; As[lk + 3][lr] = av.w;
    Bs[0][lk + 0][lr] = bv.x; Bs[0][lk + 1][lr] = bv.y; Bs[0][lk + 2][lr] = bv.z; Bs[0][lk + 3][lr] = bv.w;
    if constexpr (NB == 2) {
      Bs[1][lk + 0][lr] = bv2.x; Bs[1][lk + 1][lr] = bv2.y; Bs[1][lk + 2][lr] = bv2.z; Bs[1][lk + 3][lr] = bv2.w;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < GBK; ks += 4) {
      const int kk = ks + (lane >> 4), ii = lane & 15;
      float af[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = As[kk][wm + i * 16 + ii];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float bf = Bs[b][kk][wn + j * 16 + ii];
#pragma unroll
          for (int i = 0; i < 2; ++i) acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf, acc[b][i][j], 0, 0, 0);
        }
    }
  }
  // lane holds C[row = 4 (lane / 16) + v][col = lane % 16] of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + j * 16 + (lane & 15);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm + i * 16 + 4 * (lane >> 4) + v;
        if (m < a.M && n < a.N) {
          float c = acc[0][i][j][v];
          if constexpr (EPI == GEPI_RESID) c = a.res[(size_t)m * a.ldr + n] + c;
          if constexpr (EPI == GEPI_SWIGLU) {
            const float u = acc[NB - 1][i][j][v];
            c = c / (1.0f + expf(-c)) * u;
          }
          a.out[(size_t)m * a.ldo + n] = c;
        }
      }
    }
}

// ------------------------------------------------------------ per-token kernels
// X[m] = embeds[tok_row[m]][tok_pos[m]].
__global__ __launch_bounds__(NT) void pf_gather_kernel(const float* embeds, int max_ctx, const int* tok_row,
                                                       const int* tok_pos, int D, float* X) {
  const int m = blockIdx.x;
  const float* src = embeds + ((size_t)tok_row[m] * max_ctx + tok_pos[m]) * D;
  for (int k = threadIdx.x; k < D; k += NT) X[(size_t)m * D + k] = src[k];
}

// (cos, sin) of positions 0..n-1 (rope_cs), one block per position.
__global__ __launch_bounds__(NT) void pf_rope_table_kernel(const float* inv_freq, int half, float2* tab) {
  const int p = blockIdx.x;
  for (int t = threadIdx.x; t < half; t += NT) tab[(size_t)p * half + t] = rope_cs(p, inv_freq[t]);
}

// Token m: per-head RMSNorm of q and k (gains qn_w / kn_w), rotate-half RoPE
// at the token's position, q -> Q[m][Hq][hd]; k, v -> this layer's cache at
// (row, kv head, position), rounded to BF16 when KT is.  One wave per head.
template <typename KT>
__global__ __launch_bounds__(NT) void pf_qkv_kernel(const float* qkv, int ldqkv, const int* tok_row,
                                                    const int* tok_pos, const float* qn_w, const float* kn_w,
                                                    float eps, const float2* rope_tab, int Hq, int Hkv, int hd,
                                                    int max_ctx, float* Q, KT* kc, KT* vc) {
  const int m = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = tok_row[m], p = tok_pos[m];
  const int half = hd / 2;
  const float* row = qkv + (size_t)m * ldqkv;
  for (int h = wave; h < Hq + 2 * Hkv; h += WAVES) {
    const float* src = row + (size_t)h * hd;
    if (h >= Hq + Hkv) {                       // v: copy
      const int kh = h - Hq - Hkv;
      KT* dst = vc + (((size_t)r * Hkv + kh) * max_ctx + p) * hd;
      for (int d = lane; d < hd; d += 64) {
        if constexpr (sizeof(KT) == 2) dst[d] = (KT)bf16_bits(src[d]);
        else dst[d] = src[d];
      }
      continue;
    }
    const bool isq = h < Hq;
    const float* w = isq ? qn_w : kn_w;
    float s = 0.f;
    for (int d = lane; d < hd; d += 64) s += src[d] * src[d];
    const float inv = 1.0f / sqrtf(wave_sum_dpp(s) / (float)hd + eps);
    for (int i = lane; i < half; i += 64) {
      const float2 cs = rope_tab[(size_t)p * half + i];
      const float x1 = w[i] * (src[i] * inv);
      const float x2 = w[i + half] * (src[i + half] * inv);
      const float y1 = x1 * cs.x - x2 * cs.y;
      const float y2 = x2 * cs.x + x1 * cs.y;
      if (isq) {
        float* dq = Q + ((size_t)m * Hq + h) * hd;
        dq[i] = y1;
        dq[i + half] = y2;
      } else {
        KT* dst = kc + (((size_t)r * Hkv + (h - Hq)) * max_ctx + p) * hd;
        if constexpr (sizeof(KT) == 2) { dst[i] = (KT)bf16_bits(y1); dst[i + half] = (KT)bf16_bits(y2); }
        else { dst[i] = y1; dst[i + half] = y2; }
      }
    }
  }
}

// ------------------------------------------------------------ causal attention
// Grid (query blocks, Hkv, rows); the workgroup holds PF_NQ = 32 query
// vectors: the G heads of kv head h for QB = 32 / G consecutive positions of
// the row, and walks the row's keys 0 .. (last query position) in chunks of
// 32 with an online softmax (scale hd^-1/2, keys after the query masked).
// K / V come from the cache just written (BF16 widened), so attention sees
// exactly what decode steps will see.
constexpr int PF_NQ = 32, PF_KC = 32;

__host__ __device__ constexpr size_t pf_attn_smem_floats(int hd) {
  return (size_t)PF_NQ * (hd + 4) + 2 * (size_t)PF_KC * (hd + 4) + (size_t)PF_NQ * PF_KC + 3 * (size_t)PF_NQ;
}

template <typename KT>
__global__ __launch_bounds__(NT) void pf_attention_kernel(const float* Q, const KT* kc, const KT* vc,
                                                          const int* row_start, const int* len, int Hq, int Hkv,
                                                          int hd, int max_ctx, float scale, float* out, int ldo) {
  extern __shared__ __attribute__((aligned(16))) float psm[];
  const int G = Hq / Hkv, QB = PF_NQ / G;
  const int qb = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  const int n = len[r];
  const int p0 = qb * QB;
  if (p0 >= n) return;
  const int tid = threadIdx.x;
  const int ld = hd + 4;
  float* Qs = psm;                              // [NQ][ld]
  float* Ks = Qs + PF_NQ * ld;                  // [KC][ld]
  float* Vs = Ks + PF_KC * ld;                  // [KC][ld]
  float* S = Vs + PF_KC * ld;                   // [NQ][KC]
  float* Msc = S + PF_NQ * PF_KC;               // [NQ] rescale of this chunk
  float* Ml = Msc + PF_NQ;                      // [NQ] final sums
  const size_t head_base = ((size_t)r * Hkv + h) * max_ctx;
  const int m0 = row_start[r];
  // query vector qv = g * QB + tq: head h * G + g at position p0 + tq
  for (int i = tid; i < PF_NQ * hd; i += NT) {
    const int qv = i / hd, d = i - qv * hd;
    const int g = qv / QB, tq = qv - g * QB;
    const int p = min(p0 + tq, n - 1);
    Qs[qv * ld + d] = Q[((size_t)(m0 + p) * Hq + h * G + g) * hd + d];
  }
  // scores: thread -> query tid / 8, keys (tid % 8) + 8 j
  const int sq = tid >> 3, sj = tid & 7;
  const int sg = sq / QB, spos = p0 + (sq - sg * QB);
  // PV: thread -> query tid / 8, dims (tid % 8) * hd / 8 ...
  const int dpt = hd / 8;
  const int od0 = (tid & 7) * dpt;
  float o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;       // threads < NQ: their query's running max / sum
  const int last_p = min(p0 + QB, n) - 1;
  for (int k0 = 0; k0 <= last_p; k0 += PF_KC) {
    __syncthreads();
    for (int i = tid; i < PF_KC * hd; i += NT) {
      const int j = i / hd, d = i - j * hd;
      const int t = min(k0 + j, n - 1);
      const size_t off = (head_base + t) * hd + d;
      float kv, vv;
      if constexpr (sizeof(KT) == 2) {
        kv = __uint_as_float((uint32_t)kc[off] << 16);
        vv = __uint_as_float((uint32_t)vc[off] << 16);
      } else {
        kv = kc[off];
        vv = vc[off];
      }
      Ks[j * ld + d] = kv;
      Vs[j * ld + d] = vv;
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < PF_KC / 8; ++jj) {
      const int j = sj + 8 * jj;
      const float* qp = Qs + sq * ld;
      const float* kp = Ks + j * ld;
      float s = 0.f;
      for (int d = 0; d < hd; d += 4) {
        const float4 qa = *reinterpret_cast<const float4*>(qp + d);
        const float4 ka = *reinterpret_cast<const float4*>(kp + d);
        s = fmaf(qa.x, ka.x, s); s = fmaf(qa.y, ka.y, s); s = fmaf(qa.z, ka.z, s); s = fmaf(qa.w, ka.w, s);
      }
      const bool ok = (k0 + j <= spos) && (spos < n);
      S[sq * PF_KC + j] = ok ? s * scale : -INFINITY;
    }
    __syncthreads();
    if (tid < PF_NQ) {
      float mx = m_run;
      for (int j = 0; j < PF_KC; ++j) mx = fmaxf(mx, S[tid * PF_KC + j]);
      const float sc = (mx == -INFINITY) ? 1.f : expf(m_run - mx);
      float l = l_run * sc;
      for (int j = 0; j < PF_KC; ++j) {
        const float e = (mx == -INFINITY) ? 0.f : expf(S[tid * PF_KC + j] - mx);
        S[tid * PF_KC + j] = e;
        l += e;
      }
      m_run = mx;
      l_run = l;
      Msc[tid] = sc;
    }
    __syncthreads();
    const float sc = Msc[sq];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < dpt) o[i] *= sc;
    for (int j = 0; j < PF_KC; ++j) {
      const float pj = S[sq * PF_KC + j];
      const float* vp = Vs + j * ld + od0;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (i < dpt) o[i] = fmaf(pj, vp[i], o[i]);
    }
  }
  if (tid < PF_NQ) Ml[tid] = l_run;
  __syncthreads();
  if (spos < n) {
    const float inv = 1.0f / Ml[sq];
    float* dst = out + (size_t)(m0 + spos) * ldo + (size_t)(h * G + sg) * hd + od0;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < dpt) dst[i] = o[i] * inv;
  }
}

// Row r after its prefix: hidden = RMSNorm_final(X[last token]); kv_len and
// position = prefix length, RoPE (cos, sin) at that position, row active.
__global__ __launch_bounds__(NT) void pf_finish_kernel(const float* X, const int* row_start, const int* len,
                                                       const float* w, float eps, int D, float* hidden,
                                                       int* kv_len, int* pos, int* active, const float* inv_freq,
                                                       int half, float2* rope) {
  __shared__ float red[WAVES];
  const int r = blockIdx.x;
  const int n = len[r];
  const float* xr = X + (size_t)(row_start[r] + n - 1) * D;
  float s = 0.f;
  for (int k = threadIdx.x; k < D; k += NT) s += xr[k] * xr[k];
  const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
  for (int k = threadIdx.x; k < D; k += NT) hidden[(size_t)r * D + k] = w[k] * (xr[k] * inv);
  for (int t = threadIdx.x; t < half; t += NT) rope[(size_t)r * half + t] = rope_cs(n, inv_freq[t]);
  if (threadIdx.x == 0) { kv_len[r] = n; pos[r] = n; active[r] = 1; }
}

}  // namespace sk
