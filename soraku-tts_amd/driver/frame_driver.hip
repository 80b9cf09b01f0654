// Stand-alone frame driver: runs the decode engine through the C ABI alone
// (no Python, no PyTorch) with synthetic weights, so hardware-counter
// profilers can attach to a plain process.
//
//   sk_frame_driver [options] [frames] [warmup]
//     --model q06b|q17b   Qwen3-0.6B shape with FP32 weights (default), or the
//                         Qwen3-1.7B shape (hidden 2048, SwiGLU 6144) with BF16
//                         weights; FP32 KV either way
//     --utts N            N utterances with CFG decoded together (2N rows),
//                         Qwen3-0.6B shape with BF16 weights, KV capacity 512,
//                         prefixes of 120-240 positions drawn per utterance
//     --prefix T P        prefill T text ids + BOS frame + P prompt frames
//                         (default 96 + 144; 95 + 144 for q17b; per utterance
//                         with --utts when given)
//     --kv C U            one utterance: after the prefill, the cond / uncond
//                         rows' KV lengths jump to C / U
//     --kv-mid M          --utts: after the prefill, every row's KV length jumps
//                         to its drawn prefix length + M
//     --kv-bf16           BF16 KV cache (default FP32)
//     --max-ctx N         KV capacity per row (default: the prefix and the
//                         frames exactly, or 512 with --utts)
//   sk_frame_driver --copy MiB   (only a device copy of MiB MiB, 4 times: the
//                                 reference for HBM byte counters)
//
// The KV jumps let a short prefill stand in for a long one (the cache is
// zeroed first, so the skipped entries hold zeros; the frame's work depends
// only on the lengths).  Sampling: CFG 1.5, temperature 0.9, top-k 50, top-p
// 0.95, seeded uniforms; weights drawn uniform with std 0.02, unit norm gains,
// zero bias.  Prints one line with frames/s.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "soraku_mi355x.h"

#define HIPCHECK(x)                                                                  \
  do {                                                                               \
    hipError_t e_ = (x);                                                             \
    if (e_ != hipSuccess) {                                                          \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));                 \
      return 1;                                                                      \
    }                                                                                \
  } while (0)
#define SKCHECK(x)                                                                   \
  do {                                                                               \
    int r_ = (x);                                                                    \
    if (r_ != SK_OK) {                                                               \
      fprintf(stderr, "%s failed (%d): %s\n", #x, r_, sk_last_error());              \
      return 1;                                                                      \
    }                                                                                \
  } while (0)

__device__ __forceinline__ float hashed_value(size_t i, uint32_t seed, float scale, float offset) {
  uint32_t h = (uint32_t)i * 2654435761u ^ (seed * 0x9e3779b9u);
  h ^= h >> 15; h *= 2246822519u; h ^= h >> 13; h *= 3266489917u; h ^= h >> 16;
  return ((float)(h >> 8) * (1.0f / 16777216.0f) - 0.5f) * scale + offset;
}

// value = (uniform in [-0.5, 0.5)) * scale + offset, from a hash of the index
__global__ void fill_kernel(float* p, size_t n, uint32_t seed, float scale, float offset) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = hashed_value(i, seed, scale, offset);
}

// The same values rounded to BF16 (nearest, ties to even).
__global__ void fill_bf16_kernel(uint16_t* p, size_t n, uint32_t seed, float scale, float offset) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t b = __float_as_uint(hashed_value(i, seed, scale, offset));
    b += 0x7fffu + ((b >> 16) & 1u);
    p[i] = (uint16_t)(b >> 16);
  }
}

__global__ void copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

static int copy_probe(int mib) {
  const size_t n = (size_t)mib * (1 << 20) / 16;
  float4 *a = nullptr, *b = nullptr;
  HIPCHECK(hipMalloc(&a, n * 16));
  HIPCHECK(hipMalloc(&b, n * 16));
  hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, 0, reinterpret_cast<float*>(a), n * 4, 7u, 1.f, 0.f);
  for (int i = 0; i < 4; ++i) hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, 0, a, b, n);
  HIPCHECK(hipDeviceSynchronize());
  printf("{\"copy_bytes_each_way\": %zu, \"copies\": 4}\n", n * 16);
  HIPCHECK(hipFree(a));
  HIPCHECK(hipFree(b));
  return 0;
}

static uint64_t rng_state = 0x853c49e6748fea9bull;
static uint32_t rnd() {
  rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(rng_state >> 33);
}

static int usage() {
  fprintf(stderr, "usage: sk_frame_driver [--model q06b|q17b] [--utts N] [--prefix T P] [--kv C U] "
                  "[--kv-mid M] [--kv-bf16] [--max-ctx N] [frames] [warmup]\n       sk_frame_driver --copy MiB\n");
  return 2;
}

int main(int argc, char** argv) {
  if (argc > 2 && std::string(argv[1]) == "--copy") return copy_probe(atoi(argv[2]));
  bool big = false;
  int utts = 1, p_text = -1, p_prompt = -1, kv_c = -1, kv_u = -1, kv_mid = -1;
  bool kv_bf16 = false;
  int max_ctx = -1;
  std::vector<int> pos;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto need = [&](int k) { return i + k < argc; };
    if (a == "--model" && need(1)) { big = std::string(argv[++i]) == "q17b"; }
    else if (a == "--utts" && need(1)) { utts = atoi(argv[++i]); }
    else if (a == "--prefix" && need(2)) { p_text = atoi(argv[i + 1]); p_prompt = atoi(argv[i + 2]); i += 2; }
    else if (a == "--kv" && need(2)) { kv_c = atoi(argv[i + 1]); kv_u = atoi(argv[i + 2]); i += 2; }
    else if (a == "--kv-mid" && need(1)) { kv_mid = atoi(argv[++i]); }
    else if (a == "--kv-bf16") { kv_bf16 = true; }
    else if (a == "--max-ctx" && need(1)) { max_ctx = atoi(argv[++i]); }
    else if (!a.empty() && a[0] != '-') { pos.push_back(atoi(argv[i])); }
    else return usage();
  }
  const int frames = pos.size() > 0 ? pos[0] : 40;
  const int warmup = pos.size() > 1 ? pos[1] : 4;
  const bool wide = utts > 1;
  const int max_frames = big ? 480 : 240;
  const int def_text = big ? 95 : 96, def_prompt = 144;
  if (utts < 1 || utts > 16 || (wide && big) || frames < 1 || warmup < 0 || frames + warmup > max_frames ||
      (p_text >= 0 && (p_text < 1 || p_prompt < 0 || p_text + p_prompt > def_text + def_prompt)))
    return usage();

  sk_config c{};
  c.d_model = big ? 2048 : 1024; c.n_layers = 28; c.n_q_heads = 16; c.n_kv_heads = 8; c.head_dim = 128;
  c.trunk_inter = big ? 6144 : 3072; c.depth_inner = 2 * c.d_model; c.n_codebooks = 16; c.audio_vocab = 2051;
  c.text_vocab = 151936; c.bos_id = 2048; c.eos_id = 2049; c.pad_id = 2050;
  c.trunk_eps = 1e-6f; c.depth_eps = 1.1920929e-07f; c.rope_theta = 1e6f; c.frame_scale = 0.25f;
  c.weight_dtype = (big || wide) ? SK_BF16 : SK_F32; c.kv_dtype = kv_bf16 ? SK_BF16 : SK_F32;
  c.n_utts = utts; c.cfg_rows = 2;
  c.max_ctx = max_ctx > 0 ? max_ctx : wide ? 512 : def_text + 1 + def_prompt + max_frames + 8;
  c.max_frames = max_frames; c.n_language = 0;
  for (int i = 0; i < 4; ++i) c.language_ids[i] = -1;
  sk_engine* e = nullptr;
  SKCHECK(sk_create(&c, nullptr, &e));

  // ---- weights
  struct W { std::string key; std::vector<int64_t> shape; float scale, offset; bool matrix; };
  std::vector<W> ws;
  const int64_t d = c.d_model, hq = c.n_q_heads * c.head_dim, hkv = c.n_kv_heads * c.head_dim;
  const float sw = 0.02f * 3.4641016f;   // uniform width for std 0.02
  ws.push_back({"trunk.embed_tokens.weight", {c.text_vocab, d}, sw, 0.f, true});
  for (int l = 0; l < c.n_layers; ++l) {
    const std::string p = "trunk.layers." + std::to_string(l) + ".";
    ws.push_back({p + "input_layernorm.weight", {d}, 0.f, 1.f, false});
    ws.push_back({p + "self_attn.q_proj.weight", {hq, d}, sw, 0.f, true});
    ws.push_back({p + "self_attn.k_proj.weight", {hkv, d}, sw, 0.f, true});
    ws.push_back({p + "self_attn.v_proj.weight", {hkv, d}, sw, 0.f, true});
    ws.push_back({p + "self_attn.o_proj.weight", {d, hq}, sw, 0.f, true});
    ws.push_back({p + "self_attn.q_norm.weight", {c.head_dim}, 0.f, 1.f, false});
    ws.push_back({p + "self_attn.k_norm.weight", {c.head_dim}, 0.f, 1.f, false});
    ws.push_back({p + "post_attention_layernorm.weight", {d}, 0.f, 1.f, false});
    ws.push_back({p + "mlp.gate_proj.weight", {c.trunk_inter, d}, sw, 0.f, true});
    ws.push_back({p + "mlp.up_proj.weight", {c.trunk_inter, d}, sw, 0.f, true});
    ws.push_back({p + "mlp.down_proj.weight", {d, c.trunk_inter}, sw, 0.f, true});
  }
  ws.push_back({"trunk.norm.weight", {d}, 0.f, 1.f, false});
  ws.push_back({"audio_codebooks.table", {c.n_codebooks, c.audio_vocab, d}, sw, 0.f, true});
  ws.push_back({"depth_head.norm_in.weight", {d}, 0.f, 1.f, false});
  ws.push_back({"depth_head.mlp.gate_proj.weight", {c.depth_inner, d}, sw, 0.f, true});
  ws.push_back({"depth_head.mlp.up_proj.weight", {c.depth_inner, d}, sw, 0.f, true});
  ws.push_back({"depth_head.mlp.down_proj.weight", {d, c.depth_inner}, sw, 0.f, true});
  ws.push_back({"depth_head.norm_out.weight", {d}, 0.f, 1.f, false});
  ws.push_back({"depth_head.bias", {c.n_codebooks, c.audio_vocab}, 0.f, 0.f, false});
  std::vector<void*> bufs;
  uint32_t seed = 1;
  for (const W& w : ws) {
    size_t n = 1;
    for (int64_t v : w.shape) n *= (size_t)v;
    const bool bf = w.matrix && c.weight_dtype == SK_BF16;
    void* p = nullptr;
    HIPCHECK(hipMalloc(&p, n * (bf ? 2 : 4)));
    if (bf)
      hipLaunchKernelGGL(fill_bf16_kernel, dim3(1024), dim3(256), 0, 0, static_cast<uint16_t*>(p), n, seed++,
                         w.scale, w.offset);
    else
      hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, 0, static_cast<float*>(p), n, seed++, w.scale,
                         w.offset);
    HIPCHECK(hipGetLastError());
    bufs.push_back(p);
    SKCHECK(sk_bind_weight(e, w.key.c_str(), p, bf ? SK_BF16 : SK_F32, w.shape.data(), (int32_t)w.shape.size()));
  }
  HIPCHECK(hipDeviceSynchronize());
  for (int l = 0; l < c.n_layers; ++l)
    for (int kv = 0; kv < 2; ++kv) {
      void* p = nullptr;
      SKCHECK(sk_kv_ptr(e, l, kv, &p));
      HIPCHECK(hipMemset(p, 0, (size_t)2 * utts * c.n_kv_heads * c.max_ctx * c.head_dim * (kv_bf16 ? 2 : 4)));
    }

  // ---- prefixes: cond = text ids + BOS frame + prompt frames; uncond = one text id + the same frames
  const int Q = c.n_codebooks;
  const int64_t unc = 151643;
  std::vector<int> full_len(2 * utts);   // drawn prefix lengths (--utts) or the prefilled ones
  for (int u = 0; u < utts; ++u) {
    int nt = p_text >= 0 ? p_text : def_text, np_ = p_text >= 0 ? p_prompt : def_prompt;
    if (wide) {   // ragged prefixes: 120-240 positions, ~60% prompt frames
      const int plen = 120 + (int)(rnd() % 121);
      const int npr = (int)(0.6 * plen + 0.5);
      full_len[2 * u] = plen;
      full_len[2 * u + 1] = npr + 2;
      if (p_text < 0) { nt = plen - 1 - npr; np_ = npr; }
    } else {
      full_len[0] = nt + 1 + np_;
      full_len[1] = 2 + np_;
    }
    std::vector<int64_t> text(nt), frames_in((size_t)(1 + np_) * Q);
    text[0] = 151643;
    for (int i = 1; i < nt; ++i) text[i] = rnd() % 151643;
    for (int q = 0; q < Q; ++q) frames_in[q] = c.bos_id;
    for (size_t i = Q; i < frames_in.size(); ++i) frames_in[i] = rnd() % 2048;
    SKCHECK(sk_prefill_row(e, 2 * u, text.data(), nt, frames_in.data(), 1 + np_));
    SKCHECK(sk_prefill_row(e, 2 * u + 1, &unc, 1, frames_in.data(), 1 + np_));
  }
  SKCHECK(sk_prefill_run(e));
  if (!wide && kv_c >= 0) {
    SKCHECK(sk_set_row_state(e, 0, kv_c, kv_c));
    SKCHECK(sk_set_row_state(e, 1, kv_u, kv_u));
  }
  if (wide && kv_mid >= 0)
    for (int r = 0; r < 2 * utts; ++r) SKCHECK(sk_set_row_state(e, r, full_len[r] + kv_mid, full_len[r] + kv_mid));
  // the rows' KV lengths at the first decoded frame (what byte counts depend on)
  fprintf(stderr, "kv_lens:");
  for (int r = 0; r < 2 * utts; ++r) {
    int kv = full_len[r];
    if (!wide && kv_c >= 0) kv = r == 0 ? kv_c : kv_u;
    if (wide && kv_mid >= 0) kv += kv_mid;
    fprintf(stderr, " %d", kv);
  }
  fprintf(stderr, "\n");
  SKCHECK(sk_set_sampling(e, 1.5f, 0.9f, 50, 0.95f, 0, 0.f, 0, 0.f));
  SKCHECK(sk_capture(e));

  const int total = warmup + frames;
  std::vector<double> uvals((size_t)total * utts * Q);
  for (double& v : uvals) v = (rnd() >> 8) * (1.0 / 16777216.0);
  std::vector<int32_t> mask(total, -1);   // EOS masked for every utterance
  SKCHECK(sk_queue_frames(e, total, uvals.data(), mask.data()));
  hipStream_t st = static_cast<hipStream_t>(sk_stream(e));
  if (warmup) SKCHECK(sk_replay(e, warmup));
  SKCHECK(sk_synchronize(e));
  hipEvent_t a, b;
  HIPCHECK(hipEventCreate(&a));
  HIPCHECK(hipEventCreate(&b));
  HIPCHECK(hipEventRecord(a, st));
  SKCHECK(sk_replay(e, frames));
  HIPCHECK(hipEventRecord(b, st));
  HIPCHECK(hipEventSynchronize(b));
  float ms = 0.f;
  HIPCHECK(hipEventElapsedTime(&ms, a, b));
  std::vector<int64_t> codes((size_t)frames * utts * Q);
  SKCHECK(sk_read_codes(e, frames, codes.data()));
  printf("{\"model\": \"%s\", \"utterances\": %d, \"frames\": %d, \"us_per_frame\": %.2f, \"frames_per_s\": %.1f, "
         "\"first_codes\": [%lld, %lld, %lld]}\n",
         big ? "q17b" : "q06b", utts, frames, ms * 1e3 / frames, frames / (ms * 1e-3), (long long)codes[0],
         (long long)codes[1], (long long)codes[2]);
  SKCHECK(sk_destroy(e));
  for (void* p : bufs) hipFree(p);
  return 0;
}
