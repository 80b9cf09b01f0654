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
// (v_mfma_f32_16x16x4f32).  Workgroup tile BM x 64 (BM = 64, or 32 when
// 64-row tiles would leave CUs idle), K in steps of 32 through LDS; the next
// step's A / B tiles are loaded into registers while the current one is
// multiplied.  B (weights, FP32 or BF16 widened on load) may be split into up
// to three row segments (q / k / v projections).  Epilogues: store, residual
// add (out = res + C, res may alias out), SwiGLU (out = silu(A Bg^T) *
// (A Bu^T), B2 = up weights).  M, N arbitrary (rows past the end are clamped
// on load and not stored); K a multiple of 32.
enum { GEPI_STORE = 0, GEPI_RESID = 1, GEPI_SWIGLU = 2 };

struct GemmArgs {
  const float* A; int lda;
  const void* B[3]; int seg_rows[3];
  const void* B2;
  float* out; int ldo;
  const float* res; int ldr;
  int M, N, K;
};

constexpr int GBN = 64, GBK = 32;

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

template <int EPI, typename WL, int BM>
__global__ __launch_bounds__(256) void gemm_nt_kernel(GemmArgs a) {
  constexpr int NB = (EPI == GEPI_SWIGLU) ? 2 : 1;
  // Odd k-row strides: the loader's 8 k groups x 4 rows per 32 lanes store to
  // 32 distinct banks, and an MFMA fragment read (16 rows x 2 k per 32 lanes)
  // shifts 17 banks per k.
  constexpr int LDA = BM + 17, LDB = GBN + 17;
  constexpr int AL = BM * GBK / 4 / 256;         // float4 of A per thread per step (1 or 2)
  constexpr int BL = GBN * GBK / 4 / 256;        // float4 of B per thread per step (2)
  constexpr int TM = BM / 32;                    // 16-row MFMA tiles per wave (wave tile (BM/2) x 32)
  __shared__ __attribute__((aligned(16))) float As[GBK][LDA];
  __shared__ __attribute__((aligned(16))) float Bs[NB][GBK][LDB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * BM;
  // loader: float4 i of a thread covers tile row (tid >> 3) + 32 i, k offset (tid & 7) * 4
  const int lr = tid >> 3, lk = (tid & 7) * 4;
  const float* arow[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) arow[i] = a.A + (size_t)min(m0 + lr + 32 * i, a.M - 1) * a.lda + lk;
  const void* bbase[BL];
  size_t boff[BL], b2off[BL];
#pragma unroll
  for (int i = 0; i < BL; ++i) {
    const int bn = min(n0 + lr + 32 * i, a.N - 1);
    int brow;
    if (bn < a.seg_rows[0]) { bbase[i] = a.B[0]; brow = bn; }
    else if (bn < a.seg_rows[0] + a.seg_rows[1]) { bbase[i] = a.B[1]; brow = bn - a.seg_rows[0]; }
    else { bbase[i] = a.B[2]; brow = bn - a.seg_rows[0] - a.seg_rows[1]; }
    boff[i] = (size_t)brow * a.K + lk;
    b2off[i] = (size_t)bn * a.K + lk;
  }
  float4 ra[AL], rb[BL], rb2[BL];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < AL; ++i) ra[i] = *reinterpret_cast<const float4*>(arow[i] + k0);
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      rb[i] = load_w4<WL>(bbase[i], boff[i] + k0);
      if constexpr (NB == 2) rb2[i] = load_w4<WL>(a.B2, b2off[i] + k0);
    }
  };
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * 32;
  v4f acc[NB][TM][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[b][i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  fetch(0);
  for (int k0 = 0; k0 < a.K; k0 += GBK) {
    __syncthreads();   // the previous step's LDS reads are done
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const int rr = lr + 32 * i;
      As[lk + 0][rr] = ra[i].x; As[lk + 1][rr] = ra[i].y; As[lk + 2][rr] = ra[i].z; As[lk + 3][rr] = ra[i].w;
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      const int rr = lr + 32 * i;
      Bs[0][lk + 0][rr] = rb[i].x; Bs[0][lk + 1][rr] = rb[i].y; Bs[0][lk + 2][rr] = rb[i].z; Bs[0][lk + 3][rr] = rb[i].w;
      if constexpr (NB == 2) {
        Bs[1][lk + 0][rr] = rb2[i].x; Bs[1][lk + 1][rr] = rb2[i].y; Bs[1][lk + 2][rr] = rb2[i].z;
        Bs[1][lk + 3][rr] = rb2[i].w;
      }
    }
    __syncthreads();
    if (k0 + GBK < a.K) fetch(k0 + GBK);   // in flight while this step multiplies
#pragma unroll
    for (int ks = 0; ks < GBK; ks += 4) {
      const int kk = ks + (lane >> 4), ii = lane & 15;
      float af[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[kk][wm + i * 16 + ii];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float bf = Bs[b][kk][wn + j * 16 + ii];
#pragma unroll
          for (int i = 0; i < TM; ++i) acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf, acc[b][i][j], 0, 0, 0);
        }
    }
  }
  // lane holds C[row = 4 (lane / 16) + v][col = lane % 16] of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < TM; ++i)
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

typedef __bf16 pbf8 __attribute__((ext_vector_type(8)));

// FP32 -> (hi, lo) BF16 pair of 4 values, packed 4 x 16 bits each.
__device__ __forceinline__ void split4(const float4 v, uint2& hi, uint2& lo) {
  const float x[4] = {v.x, v.y, v.z, v.w};
  uint16_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const __bf16 b = (__bf16)x[i];
    h[i] = __builtin_bit_cast(uint16_t, b);
    l[i] = __builtin_bit_cast(uint16_t, (__bf16)(x[i] - (float)b));
  }
  hi = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
  lo = make_uint2((uint32_t)l[0] | ((uint32_t)l[1] << 16), (uint32_t)l[2] | ((uint32_t)l[3] << 16));
}

// The same GEMM for BF16 weights on the BF16 matrix cores
// (v_mfma_f32_16x16x32_bf16).  Each 32-k step stores the A tile to LDS
// already split into x_hi = bf16(x) and x_lo = bf16(x - x_hi), in MFMA
// fragment order (per 16-row tile and half: 64 lanes x 8 BF16, lane 16q + i =
// row i, k 8q .. 8q+7), so a wave reads a fragment with one 16-byte LDS load;
// the weights are stored as fragments unchanged.  Two MFMAs per product
// (A_hi W, A_lo W): the products are exact in FP32 and A keeps ~16 mantissa
// bits.  The output layout is the FP32 form's, and so is the epilogue.
template <int EPI, int BM>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(GemmArgs a) {
  constexpr int NB = (EPI == GEPI_SWIGLU) ? 2 : 1;
  constexpr int TA = BM / 16, TB = GBN / 16;     // 16-row tiles of A, 16-column tiles of B
  constexpr int TM = BM / 32;                    // A tiles per wave (wave tile (BM/2) x 32)
  constexpr int AL = BM * 8 / 256;               // float4 of A per thread per step (1 or 2)
  __shared__ __attribute__((aligned(16))) uint16_t As[2][TA * 512];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[NB][TB * 512];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * BM;
  // fragment slot (in BF16 elements) of element k of row r within a 32-k step
  auto slot = [](int r, int k) { return ((r >> 4) * 64 + (k >> 3) * 16 + (r & 15)) * 8 + (k & 7); };

  const float* arow[AL];
  int adst[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    const int idx = tid + 256 * i, r = idx >> 3, k4 = (idx & 7) * 4;
    arow[i] = a.A + (size_t)min(m0 + r, a.M - 1) * a.lda + k4;
    adst[i] = slot(r, k4);
  }
  // weights: 64 rows x 32 k = 256 pieces of 8 BF16, one per thread
  const int bn_l = tid >> 2, bk = (tid & 3) * 8;
  const int bn = min(n0 + bn_l, a.N - 1);
  const void* bbase;
  int brow;
  if (bn < a.seg_rows[0]) { bbase = a.B[0]; brow = bn; }
  else if (bn < a.seg_rows[0] + a.seg_rows[1]) { bbase = a.B[1]; brow = bn - a.seg_rows[0]; }
  else { bbase = a.B[2]; brow = bn - a.seg_rows[0] - a.seg_rows[1]; }
  const uint16_t* bp = static_cast<const uint16_t*>(bbase) + (size_t)brow * a.K + bk;
  const uint16_t* b2p = NB == 2 ? static_cast<const uint16_t*>(a.B2) + (size_t)bn * a.K + bk : nullptr;
  const int bdst = slot(bn_l, bk);
  // next step's A and B pieces.  The two B pieces are named registers: as a
  // two-element array the compiler kept them in memory, which put a wait on
  // each prefetch in front of the step's MFMAs.
  float4 ra[AL];
  uint4 rb0, rb1 = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < AL; ++i) ra[i] = *reinterpret_cast<const float4*>(arow[i]);
  rb0 = *reinterpret_cast<const uint4*>(bp);
  if constexpr (NB == 2) rb1 = *reinterpret_cast<const uint4*>(b2p);
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * 32;
  v4f acc[NB][TM][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[b][i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < a.K; k0 += GBK) {
    __syncthreads();   // the previous step's LDS reads are done
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      uint2 hi, lo;
      split4(ra[i], hi, lo);
      *reinterpret_cast<uint2*>(&As[0][adst[i]]) = hi;
      *reinterpret_cast<uint2*>(&As[1][adst[i]]) = lo;
    }
    *reinterpret_cast<uint4*>(&Bs[0][bdst]) = rb0;
    if constexpr (NB == 2) *reinterpret_cast<uint4*>(&Bs[NB - 1][bdst]) = rb1;
    __syncthreads();
    if (k0 + GBK < a.K) {   // in flight while this step multiplies
      const int kn = k0 + GBK;
#pragma unroll
      for (int i = 0; i < AL; ++i) ra[i] = *reinterpret_cast<const float4*>(arow[i] + kn);
      rb0 = *reinterpret_cast<const uint4*>(bp + kn);
      if constexpr (NB == 2) rb1 = *reinterpret_cast<const uint4*>(b2p + kn);
    }
    pbf8 ah[TM], al[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int t = wm / 16 + i;
      ah[i] = __builtin_bit_cast(pbf8, *reinterpret_cast<const uint4*>(&As[0][(t * 64 + lane) * 8]));
      al[i] = __builtin_bit_cast(pbf8, *reinterpret_cast<const uint4*>(&As[1][(t * 64 + lane) * 8]));
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = wn / 16 + j;
        const pbf8 bw = __builtin_bit_cast(pbf8, *reinterpret_cast<const uint4*>(&Bs[b][(t * 64 + lane) * 8]));
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bw, acc[b][i][j], 0, 0, 0);
          acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bw, acc[b][i][j], 0, 0, 0);
        }
      }
  }
  // lane holds C[row = 4 (lane / 16) + v][col = lane % 16] of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < TM; ++i)
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
// Per chunk: S = Q K^T on the matrix cores (one 16 x 16 tile per wave, Q
// fragments kept in registers), softmax over each query's 32 scores by 8
// threads (DPP all-reduce), O += P V on the matrix cores.  K / V come from
// the cache just written (BF16 widened), so attention sees exactly what
// decode steps will see.
constexpr int PF_NQ = 32, PF_KC = 32;

__host__ __device__ constexpr int pf_ldk(int hd) { return hd + 2; }    // lanes 0-15: 16 rows, 2 banks apart
__host__ __device__ constexpr int pf_ldv(int hd) { return hd + 16; }   // lanes 16-31: next row, 16 banks on
constexpr int PF_LDS = PF_KC + 1;
__host__ __device__ constexpr size_t pf_attn_smem_floats(int hd) {
  return (size_t)PF_KC * pf_ldk(hd) + (size_t)PF_KC * pf_ldv(hd) + (size_t)PF_NQ * PF_LDS + 2 * (size_t)PF_NQ;
}

// all-reduce over each aligned group of 8 lanes
__device__ __forceinline__ float grp8_max(float v) {
  v = fmaxf(v, dpp_keep<0xb1, 0xf>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_keep<0x4e, 0xf>(v));    // quad_perm [2,3,0,1]
  return fmaxf(v, dpp_keep<0x141, 0xf>(v));  // row_half_mirror: lane i <-> 7 - i
}
__device__ __forceinline__ float grp8_sum(float v) {
  v += dpp_keep<0xb1, 0xf>(v);
  v += dpp_keep<0x4e, 0xf>(v);
  return v + dpp_keep<0x141, 0xf>(v);
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
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ldk = pf_ldk(hd), ldv = pf_ldv(hd);
  float* Ks = psm;                              // [KC][ldk]
  float* Vs = Ks + PF_KC * ldk;                 // [KC][ldv]
  float* P = Vs + PF_KC * ldv;                  // [NQ][PF_LDS] scores, then probabilities
  float* Msc = P + PF_NQ * PF_LDS;              // [NQ] rescale of this chunk
  float* Ml = Msc + PF_NQ;                      // [NQ] final sums
  const size_t head_base = ((size_t)r * Hkv + h) * max_ctx;
  const int m0 = row_start[r];
  // query vector qv = g * QB + tq: head h * G + g at position p0 + tq
  auto qpos = [&](int qv) { return p0 + (qv - (qv / QB) * QB); };
  auto qhead = [&](int qv) { return h * G + qv / QB; };
  const int i16 = lane & 15, k4 = lane >> 4;
  // S tile of this wave: queries [16 qi, +16), keys [16 ki, +16)
  const int qi = wave >> 1, ki = wave & 1;
  float qf[32];                                 // A fragments over hd / 4 k-steps
  {
    const int qv = qi * 16 + i16;
    const int p = min(qpos(qv), n - 1);
    const float* qrow = Q + ((size_t)(m0 + p) * Hq + qhead(qv)) * hd;
#pragma unroll
    for (int ks = 0; ks < 32; ++ks) qf[ks] = (ks * 4 < hd) ? qrow[ks * 4 + k4] : 0.f;
  }
  // softmax role: query tid / 8, keys (tid % 8) * 4 .. + 4
  const int sq = tid >> 3, sk0 = (tid & 7) * 4;
  const int sp = qpos(sq);
  float m_run = -INFINITY, l_run = 0.f;
  // PV tiles of this wave: (query tile, d tile) pairs t = wave, wave + 4, ...
  const int ndt = hd / 16, ntile = 2 * ndt;
  v4f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
  const int last_p = min(p0 + QB, n) - 1;
  // K / V chunk staging: groups of 4 dims, up to 4 per thread (hd <= 128),
  // loaded one chunk ahead into registers.
  const int q4 = hd / 4, n4 = PF_KC * q4;
  float4 kr[4], vr[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(tid + u * NT, n4 - 1);
      const int j = i / q4, d = (i - j * q4) * 4;
      const size_t off = (head_base + min(k0 + j, n - 1)) * hd + d;
      if constexpr (sizeof(KT) == 2) {
        const uint2 kb = *reinterpret_cast<const uint2*>(kc + off);
        const uint2 vb = *reinterpret_cast<const uint2*>(vc + off);
        kr[u] = make_float4(__uint_as_float(kb.x << 16), __uint_as_float(kb.x & 0xffff0000u),
                            __uint_as_float(kb.y << 16), __uint_as_float(kb.y & 0xffff0000u));
        vr[u] = make_float4(__uint_as_float(vb.x << 16), __uint_as_float(vb.x & 0xffff0000u),
                            __uint_as_float(vb.y << 16), __uint_as_float(vb.y & 0xffff0000u));
      } else {   // built element-wise like the BF16 form, which keeps kr / vr in registers
        const float4 kb = *reinterpret_cast<const float4*>(kc + off);
        const float4 vb = *reinterpret_cast<const float4*>(vc + off);
        kr[u] = make_float4(kb.x, kb.y, kb.z, kb.w);
        vr[u] = make_float4(vb.x, vb.y, vb.z, vb.w);
      }
    }
  };
  fetch(0);
  for (int k0 = 0; k0 <= last_p; k0 += PF_KC) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = tid + u * NT;
      if (i < n4) {
        const int j = i / q4, d = (i - j * q4) * 4;
        float2* kd = reinterpret_cast<float2*>(Ks + j * ldk + d);
        kd[0] = make_float2(kr[u].x, kr[u].y);
        kd[1] = make_float2(kr[u].z, kr[u].w);
        *reinterpret_cast<float4*>(Vs + j * ldv + d) = vr[u];
      }
    }
    __syncthreads();
    if (k0 + PF_KC <= last_p) fetch(k0 + PF_KC);
    // S tile = Q K^T
    {
      v4f sacc = v4f{0.f, 0.f, 0.f, 0.f};
      const float* kp = Ks + (ki * 16 + i16) * ldk + k4;
#pragma unroll
      for (int ks = 0; ks < 32; ++ks)
        if (ks * 4 < hd) sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[ks], kp[ks * 4], sacc, 0, 0, 0);
      const int key = k0 + ki * 16 + i16;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int qv = qi * 16 + 4 * k4 + v;
        const int pq = qpos(qv);
        const bool ok = key <= pq && pq < n;
        P[qv * PF_LDS + ki * 16 + i16] = ok ? sacc[v] * scale : -INFINITY;
      }
    }
    __syncthreads();
    // online softmax of query sq over its 32 scores (8 threads, 4 each)
    {
      float sv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[j] = P[sq * PF_LDS + sk0 + j];
      const float mx = grp8_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
      const float mn = fmaxf(m_run, mx);
      const bool none = (mn == -INFINITY);
      const float sc = none ? 1.f : expf(m_run - mn);
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = none ? 0.f : expf(sv[j] - mn);
        P[sq * PF_LDS + sk0 + j] = e;
        part += e;
      }
      l_run = l_run * sc + grp8_sum(part);
      m_run = mn;
      if ((tid & 7) == 0) Msc[sq] = sc;
    }
    __syncthreads();
    // O = O * rescale + P V
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
      const int t = wave + 4 * t4;
      if (t < ntile) {
        const int tq = t / ndt, td = t - tq * ndt;
#pragma unroll
        for (int v = 0; v < 4; ++v) o[t4][v] *= Msc[tq * 16 + 4 * k4 + v];
        const float* pp = P + (tq * 16 + i16) * PF_LDS + k4;
        const float* vp = Vs + k4 * ldv + td * 16 + i16;
#pragma unroll
        for (int ks = 0; ks < PF_KC / 4; ++ks)
          o[t4] = __builtin_amdgcn_mfma_f32_16x16x4f32(pp[ks * 4], vp[ks * 4 * ldv], o[t4], 0, 0, 0);
      }
    }
  }
  if ((tid & 7) == 0) Ml[sq] = l_run;
  __syncthreads();
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4) {
    const int t = wave + 4 * t4;
    if (t < ntile) {
      const int tq = t / ndt, td = t - tq * ndt;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int qv = tq * 16 + 4 * k4 + v;
        const int pq = qpos(qv);
        if (pq < n)
          out[(size_t)(m0 + pq) * ldo + (size_t)qhead(qv) * hd + td * 16 + i16] = o[t4][v] / Ml[qv];
      }
    }
  }
}

// Row r after its prefix: hidden = RMSNorm_final(X[last token]); kv_len and
// position = prefix length, RoPE (cos, sin) at that position, row active; the
// first depth step's input abuf = RMSNorm_in(hidden) (and its split form).
// Rows with no tokens in this prefill keep their state.
__global__ __launch_bounds__(NT) void pf_finish_kernel(const float* X, const int* row_start, const int* len,
                                                       const float* w, float eps, int D, float* hidden,
                                                       int* kv_len, int* pos, int* active, const float* inv_freq,
                                                       int half, float2* rope, const float* w_in, float eps_in,
                                                       float* abuf, uint16_t* xs_abuf) {
  __shared__ float red[WAVES];
  const int r = blockIdx.x;
  const int n = len[r];
  if (n == 0) return;                    // not in this prefill: the row keeps its state
  const float* xr = X + (size_t)(row_start[r] + n - 1) * D;
  const size_t ro = (size_t)r * D;
  float s = 0.f;
  for (int k = threadIdx.x; k < D; k += NT) s += xr[k] * xr[k];
  const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + eps);
  float s2 = 0.f;
  for (int k = threadIdx.x; k < D; k += NT) {
    const float h = w[k] * (xr[k] * inv);
    hidden[ro + k] = h;
    s2 = fmaf(h, h, s2);
  }
  // The first frame's depth step 0 input, RMSNorm_in(hidden) (zero prefix).
  const float inv2 = 1.0f / sqrtf(block_sum(s2, red) / (float)D + eps_in);
  for (int k = threadIdx.x; k < D; k += NT) {
    const float y = w_in[k] * (hidden[ro + k] * inv2);
    abuf[ro + k] = y;
    if (xs_abuf) xsplit_store(xs_abuf, r, k, y);
  }
  for (int t = threadIdx.x; t < half; t += NT) rope[(size_t)r * half + t] = rope_cs(n, inv_freq[t]);
  if (threadIdx.x == 0) { kv_len[r] = n; pos[r] = n; active[r] = 1; }
}

}  // namespace sk
