// XCD-resident trunk layer for one utterance with CFG (two decode rows) and
// eight KV heads: two launches per layer instead of five.
//
// MI355X has 8 XCDs of 32 CUs; each XCD has its own L2, and the workgroups of
// a launch are dealt to the XCDs round-robin (lx_xcd).  KV head g's work goes
// to XCD g, so the dependencies inside a layer that are local to
// a head -- q/k/v rows -> attention chunks -> chunk merge -> that head pair's
// columns of the O projection -- and local to an eighth of the SwiGLU inner
// dimension -- gate/up rows -> those columns of the down projection -- stay on
// one XCD and pass through its L2:
//
//   lx_attn_kernel: x -> RMSNorm -> q/k/v rows of KV head g -> (tagged) ->
//     QK-norm, RoPE, KV append, 32-token attention chunks of head g ->
//     barrier -> chunk merge -> O[:, head g's 256 columns] . attn = this
//     XCD's partial of the residual update;
//   lx_mlp_kernel (lx_mlp8_kernel at the 1.7B shape): x -> RMSNorm ->
//     gate/up rows of inner slice g -> SwiGLU -> (tagged) -> down[:, slice
//     g] . act = this XCD's partial.
//
// The residual stream between the launches is 64-bit fixed point (2^-32
// units): each launch reads x whole from one accumulator and adds its
// partials (XCD 0 also adds x itself) into the next with integer atomics,
// which commute, so the sum is exact and replays stay bitwise equal.  Every
// launch thus reads its input in one load, with no exchange before its first
// projection.  Three accumulators rotate: launch i reads acc[i % 3] (the
// first layer reads the FP32 frame embedding), adds into acc[(i + 1) % 3] and
// clears acc[(i + 2) % 3], which launch i - 1 read; the final norm reads the
// last one and clears the first layer's target for the next frame.
//
// Barrier among the 32 workgroups of an XCD (lx_xcd_barrier): each workgroup
// stores its epoch in its own word of the XCD's flag line and one wave polls
// the 32 words with agent-scope loads, which read the L2 (0.5 us measured,
// against 1.6 us for a kernel boundary).  Data exchanged through it (the
// chunk partials) is written with plain stores whose completion the writer
// waits for, and read after it with plain loads; the q/k/v rows and the
// SwiGLU output pass without a barrier, as tagged words (lx_put, lx_settle).
// The epochs advance by one per launch (the attention half's chunk barrier,
// or a plain store in the MLP half), and the tags are the launch's epoch.
// On gfx9 one counter (vmcnt) covers loads and stores and
// retires in issue order, so waiting for a store also waits for every load
// issued before it, and a load's data is usable only once every earlier load
// of the wave has arrived.  Each workgroup therefore splits its 8 waves:
//   * exchange waves (0-3) issue the first phase's weights and do the q/k/v
//     or SwiGLU exchange; they hold no prefetch across an exchange (in the
//     attention half they issue the O projection's rows once the q/k/v
//     exchange is done, then only pass the attention's LDS barriers, and
//     project after the chunk merge);
//   * stream waves (4-7) load the input into LDS, then issue the later
//     phases' K/V and weights ahead of use, take their inputs from LDS and
//     poll the chunk partials' barrier, so nothing they wait for is behind
//     an exchange.
// Each role is straight-line code and both execute the same sequence of LDS
// barriers (lx_sync); none of them waits for global loads.
//
// Every spin is bounded (spin_ticks of the 100 MHz real-time counter): a
// workgroup that times out sets err bit 0 and leaves the launch (so would a
// dispatch that gave an XCD other than 32 of the workgroups).  The host
// reports err after a frame.  A set bit ends the barrier waits that see it
// (a long wait reads the error word every 64th poll), and every barrier of a
// later launch, which finds it set at entry, returns at once without polling:
// a failed frame costs at most about one spin limit, and the frames queued
// behind it run through without waiting.
#pragma once

#include <type_traits>
#include "sk_kernels.h"

namespace sk {
namespace {

constexpr int LX_XCDS = 8;
constexpr int LX_PER = 32;                      // workgroups per XCD
constexpr int LX_WGS = LX_XCDS * LX_PER;
constexpr int LX_NT = 512;                      // 4 exchange + 4 stream waves
constexpr int LX_FLAGS = 64;                    // flag words per XCD (32 used; 256 B apart)
constexpr int LX_M = 2, LX_HD = 128, LX_G = 2, LX_HKV = 8, LX_HQ = LX_G * LX_HKV;
// A barrier wait longer than this (50 ms of the 100 MHz real-time counter)
// ends the launch with an error instead of waiting further.
constexpr unsigned long long LX_SPIN_TICKS = 5000000ull;
constexpr int LX_MAXCH = 128;                   // attention chunks per row (max_ctx <= 4096)

struct LxArgs {
  const void* wq; const void* wk; const void* wv; const void* wo;   // [out][in], weight dtype
  const void* wg; const void* wu; const void* wd;
  const float* gain;                 // RMSNorm gain of the launch's input (in_norm / post_norm)
  const float* q_norm; const float* k_norm;
  const float* xin;                  // [M][D] FP32 input (the first layer: the frame embedding)
  const long long* acc_in;           // [M][D] fixed-point input (every later launch)
  unsigned long long* acc_out;       // [M][D] accumulator this launch adds x + its partials into
  unsigned long long* acc_clear;     // [M][D] accumulator this launch clears
  uint2* qkv;                        // [M][(HQ + 2 HKV) HD] raw projections, tagged (exchanged)
  float* part;                       // [M][HQ][max_chunks][HD + 4] chunk partials (exchanged)
  uint2* act; int ld_act;            // [M][ld_act] SwiGLU output, tagged (exchanged)
  void* kc; void* vc;                // this layer's cache, [M][HKV][max_ctx][HD]
  const float2* rope;                // [M][HD / 2] (cos, sin) at each row's position
  const int* kv_len; const int* active;
  unsigned* flags;                   // [8][LX_FLAGS] barrier epochs
  unsigned* err;
  int max_ctx, max_chunks;
  float eps, scale;
  unsigned long long spin_ticks;
};

// At d = 1024 the waves that issue the weight rows at entry first sleep 8
// units of 64 clocks (~0.2 us), so the launch's input loads, issued at entry
// by the other waves, reach the CU's memory queue ahead of the weight
// requests.  A wave that issues more loads than the queue holds stalls at
// issue until earlier ones return, and the input used to arrive behind the
// weight rows.  Measured on the 0.6B frame: 818 -> 785 us (each half alone
// -14 / -17 us; 6, 10 or 12 units 788-790 us); no change at d = 2048.
constexpr int LX_WEIGHT_DELAY = 8;

// The XCD this workgroup runs on (the XCC_ID hardware register).  The
// dispatcher deals a launch's workgroups to the 8 XCDs round-robin, starting
// at an XCD that can differ between launches (it did with two streams in
// use), so the XCD is read, not derived from blockIdx.x; the workgroups of one
// XCD are those with one blockIdx.x mod 8, so blockIdx.x / 8 numbers them
// 0..31 within it (sk_create checks the round-robin with xcd_probe_kernel).
__device__ __forceinline__ int lx_xcd() { return (int)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 7u); }

// Workgroup barrier for LDS only: waits for this wave's LDS operations, never
// for its global loads (a fenced __syncthreads would wait for the prefetches).
__device__ __forceinline__ void lx_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void lx_wait_stores() {
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
  asm volatile("" ::: "memory");
}
// Exchanged data (written in this launch by other workgroups of the XCD) is
// read with plain loads: the L1 starts every launch empty, a CU reads each
// exchanged line once, after the barrier, and L1 does not allocate on stores,
// so the loads miss in L1 and read the XCD's L2 (0.36 us after a barrier,
// against 0.96 us for agent-scope loads).
__device__ __forceinline__ float lx_ld(const float* p) { return *p; }

// Tagged exchange words (the q/k/v rows and the SwiGLU output): the value's
// bits in the low half, the launch's tag in the high half, written with one
// 8-byte store (naturally aligned 8-byte accesses are single-copy atomic), so
// a reader that sees the tag sees the value.  The writer neither waits for its
// stores nor raises a flag: the reader loads the words once with plain loads
// (the lines are first touched then, so they miss in L1 and read the L2) and
// reloads those whose tag is not yet the launch's with agent-scope loads,
// which skip the L1 line the first load left.  The tag is the launch's input
// barrier epoch, which grows with every launch, so a word from an earlier
// launch never carries the current one.  (For the input sums, gathered by
// every workgroup from all 32, the barrier with plain words measured faster:
// 8 words per thread from writers up to microseconds apart make many reloads.)
__device__ __forceinline__ void lx_put(uint2* p, float v, unsigned tag) {
  const unsigned long long wv = (unsigned long long)__float_as_uint(v) | ((unsigned long long)tag << 32);
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), wv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ unsigned long long lx_get(const uint2* p) {
  return *reinterpret_cast<const unsigned long long*>(p);
}
__device__ __forceinline__ float lx_val(unsigned long long v) { return __uint_as_float((unsigned)v); }
// Reloads until every word of v carries tag; false if the deadline passes
// first.  addr(i) is word i's address.
template <int N, typename Addr>
__device__ __forceinline__ bool lx_settle(unsigned long long (&v)[N], Addr addr, unsigned tag,
                                          unsigned long long deadline) {
  for (;;) {
    bool miss = false;
#pragma unroll
    for (int i = 0; i < N; ++i) miss |= (unsigned)(v[i] >> 32) != tag;
    if (!miss) return true;
    if (__builtin_amdgcn_s_memrealtime() > deadline) return false;
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((unsigned)(v[i] >> 32) != tag)
        v[i] = __hip_atomic_load(reinterpret_cast<const unsigned long long*>(addr(i)), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
  }
}
// A wave's verdict on its exchange (all lanes settled) into ok[w]; a failing
// wave sets err bit 0.  Read back with lx_all_ok after the next LDS barrier.
__device__ __forceinline__ void lx_report(bool good, int* ok, int w, unsigned* err) {
  const bool all = __builtin_amdgcn_ballot_w64(!good) == 0ull;
  if ((threadIdx.x & 63) == 0) {
    ok[w] = all ? 1 : 0;
    if (!all) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}
__device__ __forceinline__ bool lx_all_ok(const int* ok) { return (ok[0] & ok[1] & ok[2] & ok[3]) != 0; }

// The 32 workgroups of this XCD meet.  The waves that stored the data being
// exchanged have waited for their stores; wave `poller` (one with no load in
// flight) stores this workgroup's epoch and polls all 32, the other waves
// only pass the two LDS barriers.  Returns false (uniformly) on a timeout,
// when the error word is seen set during a long wait (it is read every 64th
// poll, ~30 us apart, so the fast path polls the epochs alone), or at once,
// without polling, when err0 (the error word as the launch found it) is set.
// The epoch is stored in every case, so the XCD's other workgroups are not
// held by this one.
__device__ __forceinline__ bool lx_xcd_barrier(unsigned* fl, int j, unsigned target, unsigned long long deadline,
                                               unsigned err0, unsigned* err, int* okf, int poller) {
  lx_sync();
  const int tid = threadIdx.x;
  if ((tid >> 6) == poller) {
    const int lane = tid & 63;
    if (lane == 0) __hip_atomic_store(fl + j, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    int good = err0 == 0u;
    for (unsigned it = 1; good; ++it) {
      const unsigned v = __hip_atomic_load(fl + (lane & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__builtin_amdgcn_ballot_w64((int)(v - target) < 0) == 0ull) break;
      if (__builtin_amdgcn_s_memrealtime() > deadline)
        good = 0;
      else if ((it & 63u) == 0u && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
        good = 0;
    }
    if (lane == 0) {
      *okf = good;
      if (!good) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  lx_sync();
  return *okf != 0;
}

// Fixed-point residual stream: value * 2^32 in a 64-bit integer.  FP32 to
// fixed point drops only bits below 2^-32; fixed point to FP32 rounds once.
constexpr float LX_FIX_ONE = 4294967296.0f;
__device__ __forceinline__ long long lx_fix(float v) { return (long long)(v * LX_FIX_ONE); }
__device__ __forceinline__ float lx_unfix(long long q) { return (float)q * (1.0f / LX_FIX_ONE); }
// Partial v of output (m, n), plus x (fixed point) on XCD 0, into the next
// accumulator.
__device__ __forceinline__ void lx_accum(unsigned long long* acc, size_t idx, float v, long long x) {
  __hip_atomic_fetch_add(acc + idx, (unsigned long long)(lx_fix(v) + x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Input of a launch, loaded by the stream waves (threads 256..511): stream
// thread st holds elements st * EPT .. st * EPT + EPT - 1 of x [M][D] (so
// stream waves 2m and 2m + 1 hold row m), fixed point (FIX) or FP32 (the
// first layer), and its 1/256 share of the norm gain.  finish() writes x to
// LDS as FP32 with each stream wave's sum of squares (ssq[w4]) and the gain
// to gsh.  clear() zeroes this workgroup's 1/256 share of acc_clear.  xo()
// is x[m][n] in fixed point, for the XCD-0 workgroups' accumulation.
template <int D, bool FIX>
struct LxIn {
  static constexpr int EPT = LX_M * D / 256;     // elements per stream thread
  static constexpr int GPT = D / 256;            // gain elements per stream thread
  static constexpr int CPW = LX_M * D / LX_WGS;  // accumulator entries each workgroup clears
  static_assert(EPT % 4 == 0 && GPT % 4 == 0 && CPW % 2 == 0 && 64 * EPT <= D, "LxIn shape");
  ulonglong2 xq[FIX ? EPT / 2 : 1];
  float4 xf[FIX ? 1 : EPT / 4];
  float4 gv[GPT / 4];
  __device__ __forceinline__ void issue(const LxArgs& a, int st) {
    if constexpr (FIX) {
      const ulonglong2* src = reinterpret_cast<const ulonglong2*>(a.acc_in + (size_t)st * EPT);
#pragma unroll
      for (int i = 0; i < EPT / 2; ++i) xq[i] = src[i];
    } else {
      const float4* src = reinterpret_cast<const float4*>(a.xin + (size_t)st * EPT);
#pragma unroll
      for (int i = 0; i < EPT / 4; ++i) xf[i] = src[i];
    }
#pragma unroll
    for (int i = 0; i < GPT / 4; ++i) gv[i] = *reinterpret_cast<const float4*>(a.gain + st * GPT + 4 * i);
  }
  __device__ __forceinline__ static long long xo(const LxArgs& a, int m, int n) {
    if constexpr (FIX) return a.acc_in[(size_t)m * D + n];
    else return lx_fix(a.xin[(size_t)m * D + n]);
  }
  // by wave 0 before its first load (lanes past the share repeat its last
  // store): its first wait, for its weights, comes long after the store is
  // done.  (Issued by the stream waves after their input loads, the stores
  // made the compiler spill the gain to scratch.)
  __device__ __forceinline__ static void clear(const LxArgs& a, int wave, int lane) {
    if (wave == 0)
      reinterpret_cast<ulonglong2*>(a.acc_clear + (size_t)blockIdx.x * CPW)[min(lane, CPW / 2 - 1)] =
          make_ulonglong2(0ull, 0ull);
  }
  __device__ __forceinline__ void finish(int st, int w4, float* xsh, float* gsh, float* ssq) {
#pragma unroll
    for (int i = 0; i < GPT / 4; ++i) *reinterpret_cast<float4*>(gsh + st * GPT + 4 * i) = gv[i];
    float v[EPT];
#pragma unroll
    for (int i = 0; i < EPT / 4; ++i) {
      if constexpr (FIX) {
        v[4 * i] = lx_unfix((long long)xq[2 * i].x); v[4 * i + 1] = lx_unfix((long long)xq[2 * i].y);
        v[4 * i + 2] = lx_unfix((long long)xq[2 * i + 1].x); v[4 * i + 3] = lx_unfix((long long)xq[2 * i + 1].y);
      } else {
        v[4 * i] = xf[i].x; v[4 * i + 1] = xf[i].y; v[4 * i + 2] = xf[i].z; v[4 * i + 3] = xf[i].w;
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < EPT / 4; ++i) {
      *reinterpret_cast<float4*>(xsh + st * EPT + 4 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
#pragma unroll
      for (int k = 0; k < 4; ++k) ss = fmaf(v[4 * i + k], v[4 * i + k], ss);
    }
    ss = wave_sum_dpp(ss);
    if ((st & 63) == 0) ssq[w4] = ss;
  }
};

// 1 / rms of row m from the stream waves' sums (stream waves 2m, 2m+1 hold row m).
template <int D>
__device__ __forceinline__ float lx_inv_rms(const float* ssq, int m, float eps) {
  return 1.0f / sqrtf((ssq[2 * m] + ssq[2 * m + 1]) / (float)D + eps);
}

// RW rows of a GEMV over K = D against the normalized input rows held in LDS:
// acc[r][m] = sum_k w[r][k] gain[k] (x[m][k] inv[m]).  Weights are raw 16-byte
// words in registers (BF16 widened where multiplied), in the lane layout of
// gemv_fast_kernel (lane l holds k = (jj*64 + l)*VEC + i); x is read from LDS
// one slice at a time.  acc holds this lane's partial sums; the caller
// reduces them together (wave_reduce_words).
template <int D, int RW, typename WL>
__device__ __forceinline__ void lx_dots(const uint4 (&w)[RW][D / (64 * WL::VEC)], const float* xsh, const float* gsh,
                                        const float (&inv)[LX_M], int lane, float (&acc)[RW][LX_M]) {
  constexpr int VEC = WL::VEC, NV = D / (64 * VEC);
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < LX_M; ++m) acc[r][m] = 0.f;
#pragma unroll
  for (int jj = 0; jj < NV; ++jj) {
    float xv[LX_M][VEC];
    const int k0 = (jj * 64 + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; i += 4) {
      const float4 gg = *reinterpret_cast<const float4*>(gsh + k0 + i);
#pragma unroll
      for (int m = 0; m < LX_M; ++m) {
        const float4 t = *reinterpret_cast<const float4*>(xsh + m * D + k0 + i);
        xv[m][i] = gg.x * (t.x * inv[m]);
        xv[m][i + 1] = gg.y * (t.y * inv[m]);
        xv[m][i + 2] = gg.z * (t.z * inv[m]);
        xv[m][i + 3] = gg.w * (t.w * inv[m]);
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float wf[VEC];
      WL::widen(w[r][jj], wf);
#pragma unroll
      for (int m = 0; m < LX_M; ++m)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[r][m] = fmaf(wf[i], xv[m][i], acc[r][m]);
    }
  }
}

// Wave sums of R x M per-lane partials at once: word w = r * M + m (padded to
// N words with zeros) ends in lanes [w * 64 / N, (w + 1) * 64 / N).
template <int N, int R>
__device__ __forceinline__ float lx_reduce(const float (&acc)[R][LX_M], int lane) {
  static_assert(R * LX_M <= N, "lx_reduce: too many words");
  float w[N];
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = i < R * LX_M ? acc[i / LX_M][i % LX_M] : 0.f;
  return wave_reduce_words<N>(w, lane);
}

// E consecutive elements of a weight row (the O and down projections' column
// slices): FP32 E = 2 (8 bytes; 4, 16 bytes, for the O projection's 256
// columns); BF16 E = 4 (8 bytes) or 2 (4 bytes) when the slice is not a
// multiple of 256 columns.  Held raw from the load and widened
// to FP32 where multiplied, so no conversion waits for a prefetch.
template <typename WL, int E> struct LxCols;
template <> struct LxCols<WF32, 2> {
  using raw_t = uint2;
  __device__ __forceinline__ static raw_t load(const void* base, size_t off) {
    return *reinterpret_cast<const uint2*>(static_cast<const float*>(base) + off);
  }
  __device__ __forceinline__ static void widen(raw_t t, float (&o)[2]) { o[0] = __uint_as_float(t.x); o[1] = __uint_as_float(t.y); }
};
template <> struct LxCols<WF32, 4> {
  using raw_t = uint4;
  __device__ __forceinline__ static raw_t load(const void* base, size_t off) {
    return *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + off);
  }
  __device__ __forceinline__ static void widen(raw_t t, float (&o)[4]) {
    o[0] = __uint_as_float(t.x); o[1] = __uint_as_float(t.y); o[2] = __uint_as_float(t.z); o[3] = __uint_as_float(t.w);
  }
};
template <> struct LxCols<WBF16, 4> {
  using raw_t = uint2;
  __device__ __forceinline__ static raw_t load(const void* base, size_t off) {
    return *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
  }
  __device__ __forceinline__ static void widen(raw_t t, float (&o)[4]) {
    o[0] = __uint_as_float(t.x << 16); o[1] = __uint_as_float(t.x & 0xffff0000u);
    o[2] = __uint_as_float(t.y << 16); o[3] = __uint_as_float(t.y & 0xffff0000u);
  }
};
template <> struct LxCols<WBF16, 2> {
  using raw_t = uint32_t;
  __device__ __forceinline__ static raw_t load(const void* base, size_t off) {
    return *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(base) + off);
  }
  __device__ __forceinline__ static void widen(raw_t t, float (&o)[2]) {
    o[0] = __uint_as_float(t << 16); o[1] = __uint_as_float(t & 0xffff0000u);
  }
};
template <typename WL>
__host__ __device__ constexpr int lx_col_elems(int ncols) {
  return sizeof(typename WL::elem) == 4 ? 2 : (ncols % 256 == 0 ? 4 : 2);
}

// ---------------------------------------------------------------------------
// Attention half of a layer.  Grid LX_WGS, block LX_NT.
// KT: KV cache element (float or uint16_t BF16 bits).
template <typename WL, typename KT, int D, bool FIX>
__global__ __launch_bounds__(LX_NT) void lx_attn_kernel(LxArgs a) {
  constexpr int M = LX_M, HD = LX_HD, G = LX_G, HQ = LX_HQ, HKV = LX_HKV;
  constexpr int VEC = WL::VEC, NVQ = D / (64 * VEC);
  constexpr int QRW = (G + 2) * HD / LX_PER / 4;        // q/k/v rows per exchange wave
  constexpr int OROWS = D / LX_PER, ORW = OROWS / 4;     // W_o rows per workgroup / exchange wave
  constexpr int OCOL = G * HD;                           // W_o columns of one KV head
  // 16-byte FP32 slices: half the load instructions of 8-byte ones (the
  // waves that issue them stall at issue while the CU's memory queue is full)
  constexpr int OE = sizeof(typename WL::elem) == 4 ? 4 : lx_col_elems<WL>(OCOL);
  using NL = LxCols<WL, OE>;
  constexpr int OU = OCOL / (64 * OE);                   // column units per lane per W_o row
  constexpr int LPT = HD / ATT_DPL;                      // lanes per token
  constexpr int NLD = ATT_DPL * (int)sizeof(KT) / 16;    // 16-byte K (and V) loads per lane
  constexpr bool KBF = sizeof(KT) == 2;
  constexpr int PS = part_stride(HD);
  static_assert(QRW == 4 && OCOL % (64 * OE) == 0 && LX_NT / 2 / LPT == ATT_CHUNK, "lx_attn_kernel shape");
  static_assert(D % (64 * VEC) == 0 && ORW * 4 == OROWS, "lx_attn_kernel shape");

  __shared__ __attribute__((aligned(16))) float xsh[M * D];
  __shared__ __attribute__((aligned(16))) float gsh[D];
  __shared__ float ssq[8];
  __shared__ __attribute__((aligned(16))) float qs[M][G * HD];   // raw, then normalized + rotated
  __shared__ __attribute__((aligned(16))) float kn[M][HD];
  __shared__ __attribute__((aligned(16))) float vn[M][HD];
  __shared__ float sc[G][ATT_CHUNK];
  __shared__ float stt[G][2];
  __shared__ __attribute__((aligned(16))) float vs[ATT_CHUNK * HD];
  __shared__ __attribute__((aligned(16))) float ash[M][OCOL];
  __shared__ float qwn[HD], kwn[HD];
  __shared__ float2 csh[M][HD / 2];
  __shared__ int stsh[2][6];   // row 0: kv_len[0..1], active[0..1], barrier epoch, error word
  __shared__ int okf;
  __shared__ int okq[4];   // per-wave verdicts on the q/k/v exchange

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lx_xcd(), j = blockIdx.x >> 3;
  const unsigned long long deadline = __builtin_amdgcn_s_memrealtime() + a.spin_ticks;
  unsigned* fl = a.flags + g * LX_FLAGS;
  // Row lengths decide the chunk slots: slot s is row 0's chunk s, then row
  // 1's chunk s - nch0; workgroup j takes slots j, j + 32, ...  The loads sit
  // where each role first needs them (see the role sections).
  // The stream waves load them (they need the lengths first, for their K/V
  // loads) together with the barrier epoch and the error word, and pass all
  // six to the exchange waves through LDS (stsh), whose own loads would sit
  // behind their weight stream.
  int T0, T1, nch0, nch1, nsl, nit;
  auto rows_state = [&](int t0, int t1, int a0, int a1) {
    T0 = t0; T1 = t1;
    nch0 = a0 ? (T0 + ATT_CHUNK) / ATT_CHUNK : 0;   // chunks holding T + 1 tokens
    nch1 = a1 ? (T1 + ATT_CHUNK) / ATT_CHUNK : 0;
    nsl = nch0 + nch1;
    nit = (nsl + LX_PER - 1) / LX_PER;              // slots per workgroup (one bound for all)
  };
  // Chunk merge after the chunk barrier, by all 8 waves; each wave serves one
  // (row, head) pair (row tid >> 8, head (tid >> 7) & 1 of the pair, dim
  // tid & 127).  Every thread issues its output's first 16 chunk partials,
  // lanes c = lane & 15 (each 16-lane row alike) the pair's chunk maxima and
  // sums; 16-lane DPP trees give every lane the maximum M and the weights'
  // sum, each lane its chunk's weight exp(m_c - M), and readlane hands weight
  // q to the whole wave as a scalar; then O = sum_c w_c o_c in chunk order.
  // (LDS shuffles in place of the DPP steps and readlanes cost ~0.4 us more:
  // some 24 dependent LDS round trips.)
  auto merge = [&]() {
    const int m = tid >> 8, gi = (tid >> 7) & 1, d = tid & (HD - 1);
    const int nch = m == 0 ? nch0 : nch1;   // uniform in the wave
    const float* pp = a.part + (((size_t)m * HQ + g * G + gi) * a.max_chunks) * PS;
    constexpr int CB = 16;
    float ov[CB];
#pragma unroll
    for (int q = 0; q < CB; ++q) ov[q] = lx_ld(pp + (size_t)min(q, max(nch - 1, 0)) * PS + d);
    const int c = lane & 15;
    const float2 v0 = *reinterpret_cast<const float2*>(pp + (size_t)min(c, max(nch - 1, 0)) * PS + HD);
    float mx = c < nch ? v0.x : -INFINITY;
    for (int c0 = CB; c0 < nch; c0 += CB)
      if (c0 + c < nch) mx = fmaxf(mx, lx_ld(pp + (size_t)(c0 + c) * PS + HD));
    mx = group_allmax(mx, 16);
    const float e0 = c < nch ? expf(v0.x - mx) : 0.f;
    float l = v0.y * e0;
    float O = 0.f;
#pragma unroll
    for (int q = 0; q < CB; ++q) {
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), q));
      if (q < nch) O = fmaf(w, ov[q], O);
    }
    for (int c0 = CB; c0 < nch; c0 += CB) {
      float e = 0.f;
      if (c0 + c < nch) {
        const float2 v = *reinterpret_cast<const float2*>(pp + (size_t)(c0 + c) * PS + HD);
        e = expf(v.x - mx);
        l = fmaf(v.y, e, l);
      }
#pragma unroll
      for (int q = 0; q < CB; ++q) {
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), q));
        if (c0 + q < nch) O = fmaf(w, lx_ld(pp + (size_t)(c0 + q) * PS + d), O);
      }
    }
    l = group_allsum(l, 16);
    ash[m][gi * HD + d] = O * (nch ? 1.0f / l : 0.f);
  };

  if (wave >= 4) {
    // ===================== stream waves =====================
    __builtin_amdgcn_sched_barrier(1);
    const int w4 = wave - 4, st = tid - 256;
    const int tok = st / LPT, sub = st % LPT;
    LxIn<D, FIX> in;
    unsigned ep, er;
    {
      const int t0 = a.kv_len[0], t1 = a.kv_len[1], a0 = a.active[0], a1 = a.active[1];
      ep = fl[j]; er = *a.err;
      in.issue(a, st);
      rows_state(t0, t1, a0, a1);
      // every stream thread writes (thread 0 to row 0, the rest to row 1):
      // no branch for the compiler to sink these loads into
      int* sd = stsh[st == 0 ? 0 : 1];
      sd[0] = t0; sd[1] = t1; sd[2] = a0; sd[3] = a1; sd[4] = (int)ep; sd[5] = (int)er;
    }
    // K/V of this workgroup's first slot (clamped into the cache when the
    // slot does not exist; then unused)
    const int s0 = j < nsl ? j : 0;
    const int m0 = s0 < nch0 ? 0 : 1, c0s = s0 < nch0 ? s0 : s0 - nch0;
    uint4 kraw[NLD], vraw[NLD];
    auto load_kv = [&](int m, int c) {
      const int tt = min(c * ATT_CHUNK + tok, a.max_ctx - 1);
      const size_t off = (((size_t)m * HKV + g) * a.max_ctx + tt) * HD + sub * ATT_DPL;
      const uint4* kp = reinterpret_cast<const uint4*>(static_cast<const KT*>(a.kc) + off);
      const uint4* vp = reinterpret_cast<const uint4*>(static_cast<const KT*>(a.vc) + off);
#pragma unroll
      for (int i = 0; i < NLD; ++i) { kraw[i] = kp[i]; vraw[i] = vp[i]; }
    };
    in.finish(st, w4, xsh, gsh, ssq);
    lx_sync();                                                   // 1
    // The first slot's K/V, issued once the exchange waves' q/k/v weights
    // are in flight (the projections are on the critical path; the cache rows
    // are needed only after the q/k/v exchange)
    load_kv(m0, c0s);
    lx_sync();                                                   // 4
    if (!lx_all_ok(okq)) return;
    if constexpr (KBF) lx_sync();                                // 6 (the rounded new token)
    // One slot: scores, chunk softmax, partial (o, max, sum) into pb.
    auto attend = [&](int it) {
      const int s = j + it * LX_PER;
      const bool live = s < nsl;
      const int m = s < nch0 ? 0 : 1, c = s < nch0 ? s : s - nch0;
      const int Tm = m == 0 ? T0 : T1;
      const int ctx = Tm + 1, tb = c * ATT_CHUNK;
      const int n_t = live ? min(ATT_CHUNK, ctx - tb) : 0;
      float4 kr[ATT_DPL / 4], vr[ATT_DPL / 4];
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        if constexpr (KBF) {
          const uint32_t wk[4] = {kraw[i].x, kraw[i].y, kraw[i].z, kraw[i].w};
          const uint32_t wv[4] = {vraw[i].x, vraw[i].y, vraw[i].z, vraw[i].w};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            kr[2 * i + h] = make_float4(__uint_as_float(wk[2 * h] << 16), __uint_as_float(wk[2 * h] & 0xffff0000u),
                                        __uint_as_float(wk[2 * h + 1] << 16), __uint_as_float(wk[2 * h + 1] & 0xffff0000u));
            vr[2 * i + h] = make_float4(__uint_as_float(wv[2 * h] << 16), __uint_as_float(wv[2 * h] & 0xffff0000u),
                                        __uint_as_float(wv[2 * h + 1] << 16), __uint_as_float(wv[2 * h + 1] & 0xffff0000u));
          }
        } else {
          kr[i] = make_float4(__uint_as_float(kraw[i].x), __uint_as_float(kraw[i].y), __uint_as_float(kraw[i].z),
                              __uint_as_float(kraw[i].w));
          vr[i] = make_float4(__uint_as_float(vraw[i].x), __uint_as_float(vraw[i].y), __uint_as_float(vraw[i].z),
                              __uint_as_float(vraw[i].w));
        }
      }
      if (live && tb + tok == Tm) {   // the new token: not in the cache yet when loaded
#pragma unroll
        for (int i = 0; i < ATT_DPL / 4; ++i) {
          const int d = sub * ATT_DPL + 4 * i;
          kr[i] = make_float4(kn[m][d], kn[m][d + 1], kn[m][d + 2], kn[m][d + 3]);
          vr[i] = make_float4(vn[m][d], vn[m][d + 1], vn[m][d + 2], vn[m][d + 3]);
        }
      }
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        const float* qg = &qs[m][gi * HD + sub * ATT_DPL];
        float sdot = 0.f;
#pragma unroll
        for (int i = 0; i < ATT_DPL / 4; ++i) {
          sdot = fmaf(qg[4 * i], kr[i].x, sdot);
          sdot = fmaf(qg[4 * i + 1], kr[i].y, sdot);
          sdot = fmaf(qg[4 * i + 2], kr[i].z, sdot);
          sdot = fmaf(qg[4 * i + 3], kr[i].w, sdot);
        }
        sdot = group_sum_first(sdot, LPT);
        if (sub == 0) sc[gi][tok] = tok < n_t ? sdot * a.scale : -INFINITY;
      }
      {
        float4* vd = reinterpret_cast<float4*>(vs + (size_t)tok * HD + sub * ATT_DPL);
        const bool ok = tok < n_t;
#pragma unroll
        for (int i = 0; i < ATT_DPL / 4; ++i) vd[i] = ok ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      lx_sync();                                                 // A
      if (w4 < G) {   // chunk softmax statistics: one wave per q head, one lane per token
        const float v = lane < ATT_CHUNK ? sc[w4][lane] : -INFINITY;
        const float mx = wave_max_dpp(v);
        const float ex = (lane < n_t) ? expf(v - mx) : 0.f;
        const float l = wave_sum_dpp(ex);
        if (lane < ATT_CHUNK) sc[w4][lane] = ex;
        if (lane == 0) { stt[w4][0] = mx; stt[w4][1] = l; }
      }
      lx_sync();                                                 // B
      {   // the chunk's partial (o, max, sum) straight to the XCD's L2
        const int gi = st / HD, d = st - gi * HD;
        float o = 0.f;
#pragma unroll 8
        for (int tl = 0; tl < ATT_CHUNK; ++tl) o = fmaf(sc[gi][tl], vs[(size_t)tl * HD + d], o);
        if (live) {
          float* dst = a.part + (((size_t)m * HQ + g * G + gi) * a.max_chunks + c) * PS;
          dst[d] = o;
          if (d < 2) dst[HD + d] = stt[gi][d];
        }
      }
      lx_sync();                                                 // C: sc, vs free for the next slot
    };
    attend(0);   // the first slot apart, so waiting for its K/V does not wait for W_o
    for (int it = 1; it < nit; ++it) {
      const int s = j + it * LX_PER;
      const bool live = s < nsl;
      load_kv(live ? (s < nch0 ? 0 : 1) : 0, live ? (s < nch0 ? s : s - nch0) : 0);
      attend(it);
    }
    // the partials are out once this wave's stores are (its K/V loads,
    // issued before them, are in by now); stream wave 4 polls
    lx_wait_stores();
    if (!lx_xcd_barrier(fl, j, ep + 1, deadline, er, a.err, &okf, 4)) return;   // 7, 8
    merge();
    lx_sync();                                                   // 9 (the exchange waves project)
  } else {
    // ===================== exchange waves =====================
    // (the two roles start with different scheduling barriers, so no code of
    // either is hoisted above the branch and made to wait for the other's loads)
    __builtin_amdgcn_sched_barrier(0);
    const int w4 = wave;
    LxIn<D, FIX>::clear(a, wave, lane);
    if constexpr (D == 1024) __builtin_amdgcn_s_sleep(LX_WEIGHT_DELAY);   // the input first
    // norm gains and RoPE entries (needed after the q/k/v exchange)
    const int t = tid, tr = t & 127, trow = t >> 7;
    const float qw_r = a.q_norm[tr], kw_r = a.k_norm[tr];
    const float2 cs_r = a.rope[(size_t)trow * (HD / 2) + (tr & (HD / 2 - 1))];
    // this wave's q/k/v rows (the 512 rows of KV head g: q heads gG.., k, v)
    const int r0 = j * (QRW * 4) + w4 * QRW;
    const void* wb;
    int wrow, ocol;
    if (r0 < G * HD) { wb = a.wq; wrow = g * G * HD + r0; ocol = wrow; }
    else if (r0 < (G + 1) * HD) { wb = a.wk; wrow = g * HD + r0 - G * HD; ocol = HQ * HD + wrow; }
    else { wb = a.wv; wrow = g * HD + r0 - (G + 1) * HD; ocol = (HQ + HKV) * HD + wrow; }
    uint4 w[QRW][NVQ];
#pragma unroll
    for (int r = 0; r < QRW; ++r)
#pragma unroll
      for (int jj = 0; jj < NVQ; ++jj) w[r][jj] = WL::raw(wb, (size_t)(wrow + r) * D + (size_t)(jj * 64 + lane) * VEC);
    if (trow == 0) { qwn[tr] = qw_r; kwn[tr] = kw_r; }
    if (tr < HD / 2) csh[trow][tr] = cs_r;
    lx_sync();                                                   // 1 (input in LDS)
    const unsigned ep0 = (unsigned)stsh[0][4], err0 = (unsigned)stsh[0][5], tag = ep0 + 1;
    rows_state(stsh[0][0], stsh[0][1], stsh[0][2], stsh[0][3]);
    const float inv[M] = {lx_inv_rms<D>(ssq, 0, a.eps), lx_inv_rms<D>(ssq, 1, a.eps)};
    float acc[QRW][M];
    lx_dots<D, QRW, WL>(w, xsh, gsh, inv, lane, acc);
    {
      const float v = lx_reduce<8, QRW>(acc, lane);   // word r * M + m in lanes [8 w, 8 w + 8)
      const int wd = lane >> 3;
      if ((lane & 7) == 0) lx_put(a.qkv + (size_t)(wd & 1) * (HQ + 2 * HKV) * HD + ocol + (wd >> 1), v, tag);
    }
    // Wave w4 takes two whole vectors of 128 as their tags arrive -- q heads
    // 0 and 1 of row 0 (wave 0) or of row 1 (wave 1), k of rows 0 and 1
    // (wave 2), v of rows 0 and 1 (wave 3) -- lane l dims l and l + 64 of
    // each, so the Qwen3 per-head RMSNorm (a wave sum) and the rotate-half
    // RoPE (pairs l, l + 64) run on the settled registers and only their
    // results go through LDS.
    {
      const int ldq = (HQ + 2 * HKV) * HD;
      auto src = [&](int i) -> const uint2* {
        const int vv = i >> 1, dd = lane + (i & 1) * 64;
        return w4 < 2 ? a.qkv + (size_t)w4 * ldq + g * G * HD + vv * HD + dd
                      : a.qkv + (size_t)vv * ldq + (w4 == 2 ? HQ * HD : (HQ + HKV) * HD) + g * HD + dd;
      };
      unsigned long long v[4];
      // ~0.3 us before the first load: loaded right after the own store,
      // most words were not yet there and each reload is an L2 round trip
      // (0.6B frame -8 us; 5 or 20 instead of 10: -5 us, 30: 0)
      __builtin_amdgcn_s_sleep(10);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = lx_get(src(i));
      lx_report(lx_settle(v, src, tag, deadline), okq, w4, a.err);
#pragma unroll
      for (int vv = 0; vv < 2; ++vv) {
        const float x1 = lx_val(v[2 * vv]), x2 = lx_val(v[2 * vv + 1]);
        if (w4 == 3) {
          vn[vv][lane] = x1;
          vn[vv][lane + 64] = x2;
        } else {
          const int m = w4 < 2 ? w4 : vv;
          const float ssum = wave_sum_dpp(fmaf(x1, x1, x2 * x2));
          const float rinv = 1.0f / sqrtf(ssum / (float)HD + a.eps);
          const float* wn = w4 < 2 ? qwn : kwn;
          const float g1 = wn[lane], g2 = wn[lane + 64];
          const float2 cs = csh[m][lane];
          const float y1 = g1 * (x1 * rinv), y2 = g2 * (x2 * rinv);
          float* o = w4 < 2 ? &qs[m][vv * HD] : kn[m];
          o[lane] = y1 * cs.x - y2 * cs.y;
          o[lane + 64] = y2 * cs.x + y1 * cs.y;
        }
      }
    }
    lx_sync();                                                   // 4
    if (!lx_all_ok(okq)) return;
    // This wave's W_o rows (head g's columns) and, on XCD 0, x at its
    // outputs, needed after the merge.  Issued here, by waves that then only
    // pass the attention's LDS barriers: a wave that issues them stalls at
    // issue while the CU's memory queue is full, and in the stream waves that
    // stall delayed the chunk scores.  Lanes with (lane & 3) == 0 own outputs
    // (m, n) = (wd & 1, n0 + 8 h + (wd >> 1)), wd = lane >> 2, h < OH.
    const int n0 = j * OROWS + w4 * ORW, wd = lane >> 2;
    constexpr int OH = ORW * M / 16;
    typename NL::raw_t wo[ORW][OU];
    auto load_wo = [&](auto rb, auto re) {
#pragma unroll
      for (int r = decltype(rb)::value; r < decltype(re)::value; ++r)
#pragma unroll
        for (int u = 0; u < OU; ++u)
          wo[r][u] = NL::load(a.wo, (size_t)(n0 + r) * (HQ * HD) + g * OCOL + (size_t)(u * 64 + lane) * OE);
    };
    // more than 8 loads per lane (the 1.7B shape's 16) go out in two halves,
    // the second after the first slot's scores: 1,140 -> 1,136 us per 1.7B
    // frame; at 8 loads the split cost 3 us per 0.6B frame
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, (ORW * OU > 8 ? ORW / 2 : ORW)>;
    using H2 = std::integral_constant<int, ORW>;
    load_wo(H0{}, H1{});
    long long xo[OH];
#pragma unroll
    for (int h = 0; h < OH; ++h) xo[h] = g == 0 ? LxIn<D, FIX>::xo(a, wd & 1, n0 + 8 * h + (wd >> 1)) : 0ll;
    // append the new token (workgroup owning each row's last chunk); a BF16
    // cache stores it rounded and this step attends to the rounded values
    {
      const int m = trow, d = tr;
      const int nchm = m == 0 ? nch0 : nch1, Tm = m == 0 ? T0 : T1;
      const int slast = (m == 0 ? 0 : nch0) + nchm - 1;
      if (nchm > 0 && slast % LX_PER == j) {
        const size_t off = (((size_t)m * HKV + g) * a.max_ctx + Tm) * HD + d;
        if constexpr (KBF) {
          static_cast<uint16_t*>(a.kc)[off] = (uint16_t)bf16_bits(kn[m][d]);
          static_cast<uint16_t*>(a.vc)[off] = (uint16_t)bf16_bits(vn[m][d]);
        } else {
          static_cast<float*>(a.kc)[off] = kn[m][d];
          static_cast<float*>(a.vc)[off] = vn[m][d];
        }
      }
      if constexpr (KBF) {   // each thread rounds the element it appended
        kn[m][d] = bf16_round(kn[m][d]);
        vn[m][d] = bf16_round(vn[m][d]);
      }
    }
    if constexpr (KBF) lx_sync();                                // 6 (the rounded new token)
    // the second half of the W_o rows (if split) once the first slot's scores are in
    if (nit > 0) {
      lx_sync();                                                 // A: scores, V in LDS
      load_wo(H1{}, H2{});
      lx_sync();                                                 // B: softmax
      lx_sync();                                                 // C: partials stored
    } else {
      load_wo(H1{}, H2{});
    }
    for (int it = 1; it < nit; ++it) {
      lx_sync();                                                 // A
      lx_sync();                                                 // B
      lx_sync();                                                 // C
    }
    if (!lx_xcd_barrier(fl, j, tag, deadline, err0, a.err, &okf, 4)) return;   // 7, 8 (stream wave 4 polls)
    merge();
    lx_sync();                                                   // 9
    float oacc[ORW][M];
#pragma unroll
    for (int r = 0; r < ORW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) oacc[r][m] = 0.f;
#pragma unroll
    for (int u = 0; u < OU; ++u) {
      const int k0 = (u * 64 + lane) * OE;
      float xv[M][OE];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < OE; ++i) xv[m][i] = ash[m][k0 + i];
#pragma unroll
      for (int r = 0; r < ORW; ++r) {
        float wf[OE];
        NL::widen(wo[r][u], wf);
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int i = 0; i < OE; ++i) oacc[r][m] = fmaf(wf[i], xv[m][i], oacc[r][m]);
      }
    }
    static_assert(ORW * M == 16 || ORW * M == 32, "O rows per exchange wave");
#pragma unroll
    for (int h = 0; h < OH; ++h) {
      float part[8][M];
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) part[r][m] = oacc[h * 8 + r][m];
      const float v = lx_reduce<16, 8>(part, lane);   // word r * M + m in lanes [4 w, 4 w + 4)
      if ((lane & 3) == 0) lx_accum(a.acc_out, (size_t)(wd & 1) * D + n0 + 8 * h + (wd >> 1), v, xo[h]);
    }
  }
}

// ---------------------------------------------------------------------------
// MLP half of a layer.  Grid LX_WGS, block LX_NT.  XCD g owns inner indices
// [g I/8, (g+1) I/8); workgroup j of it IW = I/256 of them, IPW per
// exchange wave; the stream waves hold the down projection's rows.
template <typename WL, int D, int I>
__global__ __launch_bounds__(LX_NT) void lx_mlp_kernel(LxArgs a) {
  constexpr bool FIX = true;
  constexpr int M = LX_M, VEC = WL::VEC, NV = D / (64 * VEC);
  constexpr int IX = I / LX_XCDS, IW = IX / LX_PER;
  constexpr int GUW = 4;
  constexpr int IPW = IW / GUW;                       // inner indices per gate/up wave
  constexpr int DROWS = D / LX_PER, DRW = DROWS / 4;  // down rows per workgroup / stream wave
  constexpr int DE = lx_col_elems<WL>(IX);
  using NL = LxCols<WL, DE>;
  constexpr int DU = IX / (64 * DE);                  // column units per lane per down row
  static_assert(IW % 4 == 0 && IPW * GUW == IW && IX % (64 * DE) == 0 && DRW * 4 == DROWS, "lx_mlp_kernel shape");

  __shared__ __attribute__((aligned(16))) float xsh[M * D];
  __shared__ __attribute__((aligned(16))) float gsh[D];
  __shared__ float ssq[8];
  __shared__ __attribute__((aligned(16))) float ash[M][IX];   // the XCD's slice
  __shared__ int stsh[2];   // [0]: the epoch (loaded by the stream waves)
  __shared__ int oka[4];   // per-wave verdicts on the SwiGLU exchange

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lx_xcd(), j = blockIdx.x >> 3;
  const unsigned long long deadline = __builtin_amdgcn_s_memrealtime() + a.spin_ticks;
  unsigned* fl = a.flags + g * LX_FLAGS;
  const int i0 = g * IX + j * IW;                     // first inner index of this workgroup
  // gate/up wave gw (0..GUW-1): its weight rows are issued, then it waits
  // at the LDS barrier after which the input is in LDS
  auto gate_up = [&](int gw, float& act) {
    uint4 w[2 * IPW][NV];
    const int ib = i0 + gw * IPW;
#pragma unroll
    for (int r = 0; r < IPW; ++r)
#pragma unroll
      for (int jj = 0; jj < NV; ++jj) {
        w[2 * r][jj] = WL::raw(a.wg, (size_t)(ib + r) * D + (size_t)(jj * 64 + lane) * VEC);
        w[2 * r + 1][jj] = WL::raw(a.wu, (size_t)(ib + r) * D + (size_t)(jj * 64 + lane) * VEC);
      }
    lx_sync();                                                   // 1 (input in LDS)
    const float inv[M] = {lx_inv_rms<D>(ssq, 0, a.eps), lx_inv_rms<D>(ssq, 1, a.eps)};
    float acc[2 * IPW][M];
    lx_dots<D, 2 * IPW, WL>(w, xsh, gsh, inv, lane, acc);
    // word (2 i + gate/up) M + m = 4 i + 2 gu + m: lanes [4 w, 4 w + 4); the
    // up word of a gate word sits 8 lanes further on
    static_assert(2 * IPW * M <= 16, "gate/up rows per wave");
    const float x = lx_reduce<16, 2 * IPW>(acc, lane);
    const float u = __shfl(x, (lane + 8) & 63, 64);
    const int wd = lane >> 2;
    act = x / (1.0f + expf(-x)) * u;   // valid in lanes with (wd & 2) == 0: i = wd >> 2, m = wd & 1
    return true;
  };

  if (wave < 4) {
    // ===================== exchange waves =====================
    // (the two roles start with different scheduling barriers, so no code of
    // either is hoisted above the branch and made to wait for the other's loads)
    __builtin_amdgcn_sched_barrier(0);
    LxIn<D, FIX>::clear(a, wave, lane);
    if constexpr (D == 1024) __builtin_amdgcn_s_sleep(LX_WEIGHT_DELAY);   // the input first
    float act;
    if (!gate_up(wave, act)) return;
    const unsigned tag = (unsigned)stsh[0] + 1;   // this launch's epoch
    // stored for the next launch (no barrier here); every lane of wave 0
    // stores the same word, so the store needs no per-lane branch
    if (wave == 0) __hip_atomic_store(fl + j, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    {
      const int wd = lane >> 2, i = wd >> 2, m = wd & 1;
      if ((lane & 3) == 0 && (wd & 2) == 0 && i < IPW) lx_put(a.act + (size_t)m * a.ld_act + i0 + wave * IPW + i, act, tag);
    }
    {
      constexpr int PT = M * IX / 256;                           // loads per thread, all issued first
      static_assert(M * IX % 256 == 0, "act slice per exchange thread");
      auto src = [&](int q) -> const uint2* {
        const int e = tid + 256 * q, m = e / IX, k = e - m * IX;
        return a.act + (size_t)m * a.ld_act + g * IX + k;
      };
      unsigned long long v[PT];
      __builtin_amdgcn_s_sleep(10);   // as before the q/k/v loads
#pragma unroll
      for (int q = 0; q < PT; ++q) v[q] = lx_get(src(q));
      lx_report(lx_settle(v, src, tag, deadline), oka, wave, a.err);
#pragma unroll
      for (int q = 0; q < PT; ++q) {
        const int e = tid + 256 * q, m = e / IX, k = e - m * IX;
        ash[m][k] = lx_val(v[q]);
      }
    }
    lx_sync();                                                   // 4
  } else {
    // ===================== stream waves =====================
    __builtin_amdgcn_sched_barrier(1);
    const int w4 = wave - 4;
    // down rows of this wave, slice g's columns; lanes with (lane & 3) == 0
    // own outputs (m, n) = (wo & 1, n0 + 8 h + (wo >> 1)), wo = lane >> 2
    const int n0 = j * DROWS + w4 * DRW, wo = lane >> 2;
    constexpr int OH = DRW * M / 16;
    typename NL::raw_t wd[DRW][DU];
    auto load_down = [&]() {
#pragma unroll
      for (int r = 0; r < DRW; ++r)
#pragma unroll
        for (int u = 0; u < DU; ++u)
          wd[r][u] = NL::load(a.wd, (size_t)(n0 + r) * I + g * IX + (size_t)(u * 64 + lane) * DE);
    };
    long long xo[OH];
    {
      const int st = tid - 256;
      LxIn<D, FIX> in;
      const unsigned ep = fl[j];
      in.issue(a, st);
#pragma unroll
      for (int h = 0; h < OH; ++h) xo[h] = LxIn<D, FIX>::xo(a, wo & 1, n0 + 8 * h + (wo >> 1));
      stsh[st == 0 ? 0 : 1] = (int)ep;   // no branch to sink the loads into
      in.finish(st, w4, xsh, gsh, ssq);
      lx_sync();                                                 // 1
    }
    // issued at entry, beside the gate/up rows, they slowed the 0.6B frame
    // by 22 us (they share the HBM queues with the rows the dots wait for)
    load_down();
    lx_sync();                                                   // 4
    if (!lx_all_ok(oka)) return;
    float acc[DRW][M];
#pragma unroll
    for (int r = 0; r < DRW; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
#pragma unroll
    for (int u = 0; u < DU; ++u) {
      const int k0 = (u * 64 + lane) * DE;
      float xv[M][DE];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < DE; ++i) xv[m][i] = ash[m][k0 + i];
#pragma unroll
      for (int r = 0; r < DRW; ++r) {
        float wf[DE];
        NL::widen(wd[r][u], wf);
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int i = 0; i < DE; ++i) acc[r][m] = fmaf(wf[i], xv[m][i], acc[r][m]);
      }
    }
    static_assert(DRW * M == 16 || DRW * M == 32, "down rows per stream wave");
#pragma unroll
    for (int h = 0; h < DRW * M / 16; ++h) {
      float part[8][M];
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) part[r][m] = acc[h * 8 + r][m];
      const float v = lx_reduce<16, 8>(part, lane);   // word r * M + m in lanes [4 w, 4 w + 4)
      if ((lane & 3) == 0) lx_accum(a.acc_out, (size_t)(wo & 1) * D + n0 + 8 * h + (wo >> 1), v, g == 0 ? xo[h] : 0ll);
    }
  }
}

// ---------------------------------------------------------------------------
// MLP half for the wider shape (Qwen3-1.7B: d 2048, SwiGLU 6144): 24 inner
// indices per workgroup are 48 gate/up rows of 4 KB (BF16), more than 4 waves
// can hold, so all 8 waves take 3 inner indices each and then 8 down rows
// each.  The stream waves (4-7) also sum the input (their store wait before
// the input barrier then includes their own gate/up rows, which the dots after
// it need anyway); the SwiGLU output is exchanged as tagged words behind the
// down rows.
template <typename WL, int D, int I>
__global__ __launch_bounds__(LX_NT) void lx_mlp8_kernel(LxArgs a) {
  constexpr bool FIX = true;
  constexpr int M = LX_M, VEC = WL::VEC, NV = D / (64 * VEC);
  constexpr int IX = I / LX_XCDS, IW = IX / LX_PER;
  constexpr int IPW = IW / 8;                         // inner indices per wave
  constexpr int DROWS = D / LX_PER, DRW = DROWS / 8;  // down rows per workgroup / wave
  constexpr int DE = lx_col_elems<WL>(IX);
  using NL = LxCols<WL, DE>;
  constexpr int DU = IX / (64 * DE);                  // column units per lane per down row
  constexpr int PT = M * IX / LX_NT;                  // SwiGLU outputs per thread in the exchange
  static_assert(IPW * 8 == IW && 2 * IPW * M <= 16 && DRW * 8 == DROWS && DRW * M == 16, "lx_mlp8_kernel shape");
  static_assert(IX % (64 * DE) == 0 && M * IX % LX_NT == 0, "lx_mlp8_kernel shape");

  __shared__ __attribute__((aligned(16))) float xsh[M * D];
  __shared__ __attribute__((aligned(16))) float gsh[D];
  __shared__ float ssq[8];
  __shared__ __attribute__((aligned(16))) float ash[M][IX];   // the XCD's slice
  __shared__ int stsh[2];      // [0]: the epoch (loaded by the stream waves)
  __shared__ int oka[8];       // per-wave verdicts on the SwiGLU exchange

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lx_xcd(), j = blockIdx.x >> 3;
  const unsigned long long deadline = __builtin_amdgcn_s_memrealtime() + a.spin_ticks;
  unsigned* fl = a.flags + g * LX_FLAGS;
  const int i0 = g * IX + j * IW;                     // first inner index of this workgroup
  const int ib = i0 + wave * IPW;
  uint4 w[2 * IPW][NV];
  auto load_gate_up = [&]() {
#pragma unroll
    for (int r = 0; r < IPW; ++r)
#pragma unroll
      for (int jj = 0; jj < NV; ++jj) {
        w[2 * r][jj] = WL::raw(a.wg, (size_t)(ib + r) * D + (size_t)(jj * 64 + lane) * VEC);
        w[2 * r + 1][jj] = WL::raw(a.wu, (size_t)(ib + r) * D + (size_t)(jj * 64 + lane) * VEC);
      }
  };
  // this wave's down rows, slice g's columns; lanes with (lane & 3) == 0
  // own outputs (m, n) = (wo & 1, n0 + (wo >> 1)), wo = lane >> 2
  const int n0 = j * DROWS + wave * DRW, wo = lane >> 2;
  typename NL::raw_t wdn[DRW][DU];
  auto load_down = [&]() {
#pragma unroll
    for (int r = 0; r < DRW; ++r)
#pragma unroll
      for (int u = 0; u < DU; ++u)
        wdn[r][u] = NL::load(a.wd, (size_t)(n0 + r) * I + g * IX + (size_t)(u * 64 + lane) * DE);
  };
  long long xo;
  if (wave < 4) {
    // gate/up rows, then the down rows behind them
    __builtin_amdgcn_sched_barrier(0);
    LxIn<D, FIX>::clear(a, wave, lane);
    xo = LxIn<D, FIX>::xo(a, wo & 1, n0 + (wo >> 1));
    load_gate_up();
    load_down();
    lx_sync();                                                   // 1
  } else {
    // the input first (so waiting for it waits for nothing else), then the
    // gate/up rows, then the down rows
    __builtin_amdgcn_sched_barrier(1);
    const int st = tid - 256, w4 = wave - 4;
    LxIn<D, FIX> in;
    const unsigned ep = fl[j];
    in.issue(a, st);
    xo = LxIn<D, FIX>::xo(a, wo & 1, n0 + (wo >> 1));
    load_gate_up();
    stsh[st == 0 ? 0 : 1] = (int)ep;   // no branch to sink the loads into
    in.finish(st, w4, xsh, gsh, ssq);
    lx_sync();                                                   // 1
    load_down();
  }
  const unsigned tag = (unsigned)stsh[0] + 1;                 // this launch's epoch
  // stored for the next launch (no barrier here); every lane of wave 0 stores
  // the same word, so the store needs no per-lane branch
  if (wave == 0) __hip_atomic_store(fl + j, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  {
    const float inv[M] = {lx_inv_rms<D>(ssq, 0, a.eps), lx_inv_rms<D>(ssq, 1, a.eps)};
    float acc[2 * IPW][M];
    lx_dots<D, 2 * IPW, WL>(w, xsh, gsh, inv, lane, acc);
    // word (2 i + gate/up) M + m = 4 i + 2 gu + m: lanes [4 w, 4 w + 4); the
    // up word of a gate word sits 8 lanes further on
    const float x = lx_reduce<16, 2 * IPW>(acc, lane);
    const float u = __shfl(x, (lane + 8) & 63, 64);
    const int wd = lane >> 2, i = wd >> 2, m = wd & 1;
    const float act = x / (1.0f + expf(-x)) * u;
    if ((lane & 3) == 0 && (wd & 2) == 0 && i < IPW) lx_put(a.act + (size_t)m * a.ld_act + ib + i, act, tag);
  }
  {
    auto src = [&](int q) -> const uint2* {
      const int e = tid + LX_NT * q, m = e / IX, k = e - m * IX;
      return a.act + (size_t)m * a.ld_act + g * IX + k;
    };
    unsigned long long v[PT];
#pragma unroll
    for (int q = 0; q < PT; ++q) v[q] = lx_get(src(q));
    lx_report(lx_settle(v, src, tag, deadline), oka, wave, a.err);
#pragma unroll
    for (int q = 0; q < PT; ++q) {
      const int e = tid + LX_NT * q, m = e / IX, k = e - m * IX;
      ash[m][k] = lx_val(v[q]);
    }
  }
  lx_sync();                                                     // 2
  if (!(lx_all_ok(oka) && lx_all_ok(oka + 4))) return;
  float acc[DRW][M];
#pragma unroll
  for (int r = 0; r < DRW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
#pragma unroll
  for (int u = 0; u < DU; ++u) {
    const int k0 = (u * 64 + lane) * DE;
    float xv[M][DE];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < DE; ++i) xv[m][i] = ash[m][k0 + i];
#pragma unroll
    for (int r = 0; r < DRW; ++r) {
      float wf[DE];
      NL::widen(wdn[r][u], wf);
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < DE; ++i) acc[r][m] = fmaf(wf[i], xv[m][i], acc[r][m]);
    }
  }
  const float v = lx_reduce<16, DRW>(acc, lane);   // word r * M + m in lanes [4 w, 4 w + 4)
  if ((lane & 3) == 0) lx_accum(a.acc_out, (size_t)(wo & 1) * D + n0 + (wo >> 1), v, g == 0 ? xo : 0ll);
}

}  // namespace
}  // namespace sk
