// Stand-alone frame driver: runs the decode engine through the C ABI alone
// (no Python, no PyTorch), on a Qwen3-0.6B-shaped model with synthetic
// weights, so hardware-counter profilers can attach to a plain process.
//
//   sk_frame_driver [frames] [warmup] [text_ids] [prompt_frames] [cond_len uncond_len]
//
// With cond_len / uncond_len, the rows' KV lengths jump to those values after
// the prefill (the cache is zeroed first, so the skipped entries hold zeros):
// a short prefill then stands in for a long one, for profilers that cannot
// follow the thousands of launches of a long prefill.
//   sk_frame_driver --copy MiB     (only a device copy of MiB MiB, 4 times:
//                                   the reference for HBM byte counters)
//
// Workload: one utterance with CFG (rows cond + uncond), 96 text ids + BOS +
// 144 prompt frames by default (uncond: one text id), CFG 1.5, temperature 0.9, top-k
// 50, top-p 0.95, seeded uniforms; FP32 weights drawn uniform with std 0.02,
// unit norm gains, zero bias.  Prints one line with frames/s.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
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

// value = (uniform in [-0.5, 0.5)) * scale + offset, from a hash of the index
__global__ void fill_kernel(float* p, size_t n, uint32_t seed, float scale, float offset) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t h = (uint32_t)i * 2654435761u ^ (seed * 0x9e3779b9u);
    h ^= h >> 15; h *= 2246822519u; h ^= h >> 13; h *= 3266489917u; h ^= h >> 16;
    p[i] = ((float)(h >> 8) * (1.0f / 16777216.0f) - 0.5f) * scale + offset;
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

int main(int argc, char** argv) {
  if (argc > 2 && std::string(argv[1]) == "--copy") return copy_probe(atoi(argv[2]));
  const int frames = argc > 1 ? atoi(argv[1]) : 40;
  const int warmup = argc > 2 ? atoi(argv[2]) : 4;
  const int n_text = argc > 3 ? atoi(argv[3]) : 96, n_prompt = argc > 4 ? atoi(argv[4]) : 144;
  const int max_frames = 240;
  if (frames < 1 || warmup < 0 || frames + warmup > max_frames || n_text < 1 || n_prompt < 0 ||
      n_text + n_prompt > 96 + 144) {
    fprintf(stderr, "need frames >= 1, frames + warmup <= %d, text_ids >= 1, prompt_frames >= 0, "
                    "text_ids + prompt_frames <= 240\n", max_frames);
    return 2;
  }
  sk_config c{};
  c.d_model = 1024; c.n_layers = 28; c.n_q_heads = 16; c.n_kv_heads = 8; c.head_dim = 128;
  c.trunk_inter = 3072; c.depth_inner = 2048; c.n_codebooks = 16; c.audio_vocab = 2051;
  c.text_vocab = 151936; c.bos_id = 2048; c.eos_id = 2049; c.pad_id = 2050;
  c.trunk_eps = 1e-6f; c.depth_eps = 1.1920929e-07f; c.rope_theta = 1e6f; c.frame_scale = 0.25f;
  c.weight_dtype = SK_F32; c.n_utts = 1; c.cfg_rows = 2;
  c.max_ctx = 96 + 1 + 144 + max_frames + 8; c.max_frames = max_frames; c.n_language = 0;
  sk_engine* e = nullptr;
  SKCHECK(sk_create(&c, nullptr, &e));

  // ---- weights
  struct W { std::string key; std::vector<int64_t> shape; float scale, offset; };
  std::vector<W> ws;
  const int64_t d = c.d_model, hq = c.n_q_heads * c.head_dim, hkv = c.n_kv_heads * c.head_dim;
  const float sw = 0.02f * 3.4641016f;   // uniform width for std 0.02
  ws.push_back({"trunk.embed_tokens.weight", {c.text_vocab, d}, sw, 0.f});
  for (int l = 0; l < c.n_layers; ++l) {
    const std::string p = "trunk.layers." + std::to_string(l) + ".";
    ws.push_back({p + "input_layernorm.weight", {d}, 0.f, 1.f});
    ws.push_back({p + "self_attn.q_proj.weight", {hq, d}, sw, 0.f});
    ws.push_back({p + "self_attn.k_proj.weight", {hkv, d}, sw, 0.f});
    ws.push_back({p + "self_attn.v_proj.weight", {hkv, d}, sw, 0.f});
    ws.push_back({p + "self_attn.o_proj.weight", {d, hq}, sw, 0.f});
    ws.push_back({p + "self_attn.q_norm.weight", {c.head_dim}, 0.f, 1.f});
    ws.push_back({p + "self_attn.k_norm.weight", {c.head_dim}, 0.f, 1.f});
    ws.push_back({p + "post_attention_layernorm.weight", {d}, 0.f, 1.f});
    ws.push_back({p + "mlp.gate_proj.weight", {c.trunk_inter, d}, sw, 0.f});
    ws.push_back({p + "mlp.up_proj.weight", {c.trunk_inter, d}, sw, 0.f});
    ws.push_back({p + "mlp.down_proj.weight", {d, c.trunk_inter}, sw, 0.f});
  }
  ws.push_back({"trunk.norm.weight", {d}, 0.f, 1.f});
  ws.push_back({"audio_codebooks.table", {c.n_codebooks, c.audio_vocab, d}, sw, 0.f});
  ws.push_back({"depth_head.norm_in.weight", {d}, 0.f, 1.f});
  ws.push_back({"depth_head.mlp.gate_proj.weight", {c.depth_inner, d}, sw, 0.f});
  ws.push_back({"depth_head.mlp.up_proj.weight", {c.depth_inner, d}, sw, 0.f});
  ws.push_back({"depth_head.mlp.down_proj.weight", {d, c.depth_inner}, sw, 0.f});
  ws.push_back({"depth_head.norm_out.weight", {d}, 0.f, 1.f});
  ws.push_back({"depth_head.bias", {c.n_codebooks, c.audio_vocab}, 0.f, 0.f});
  std::vector<float*> bufs;
  uint32_t seed = 1;
  for (const W& w : ws) {
    size_t n = 1;
    for (int64_t v : w.shape) n *= (size_t)v;
    float* p = nullptr;
    HIPCHECK(hipMalloc(&p, n * sizeof(float)));
    hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, 0, p, n, seed++, w.scale, w.offset);
    HIPCHECK(hipGetLastError());
    bufs.push_back(p);
    SKCHECK(sk_bind_weight(e, w.key.c_str(), p, SK_F32, w.shape.data(), (int32_t)w.shape.size()));
  }
  HIPCHECK(hipDeviceSynchronize());

  // ---- prefix: cond = text ids + BOS frame + prompt frames; uncond = one text id + same frames
  const int Q = c.n_codebooks;
  std::vector<int64_t> text(n_text), frames_in((size_t)(1 + n_prompt) * Q);
  text[0] = 151643;
  for (int i = 1; i < n_text; ++i) text[i] = rnd() % 151643;
  for (int q = 0; q < Q; ++q) frames_in[q] = c.bos_id;
  for (size_t i = Q; i < frames_in.size(); ++i) frames_in[i] = rnd() % 2048;
  const int64_t unc = 151643;
  for (int l = 0; l < c.n_layers; ++l)
    for (int kv = 0; kv < 2; ++kv) {
      void* p = nullptr;
      SKCHECK(sk_kv_ptr(e, l, kv, &p));
      HIPCHECK(hipMemset(p, 0, (size_t)2 * c.n_kv_heads * c.max_ctx * c.head_dim * sizeof(float)));
    }
  SKCHECK(sk_prefill_row(e, 0, text.data(), n_text, frames_in.data(), 1 + n_prompt));
  SKCHECK(sk_prefill_row(e, 1, &unc, 1, frames_in.data(), 1 + n_prompt));
  SKCHECK(sk_prefill_run(e));
  if (argc > 6) {
    const int lc = atoi(argv[5]), lu = atoi(argv[6]);
    SKCHECK(sk_set_row_state(e, 0, lc, lc));
    SKCHECK(sk_set_row_state(e, 1, lu, lu));
  }
  SKCHECK(sk_set_sampling(e, 1.5f, 0.9f, 50, 0.95f, 0, 0.f, 0, 0.f));
  SKCHECK(sk_capture(e));

  const int total = warmup + frames;
  std::vector<double> u((size_t)total * Q);
  for (double& v : u) v = (rnd() >> 8) * (1.0 / 16777216.0);
  std::vector<int32_t> mask(total, 1);
  SKCHECK(sk_queue_frames(e, total, u.data(), mask.data()));
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
  std::vector<int64_t> codes((size_t)frames * Q);
  SKCHECK(sk_read_codes(e, frames, codes.data()));
  printf("{\"frames\": %d, \"us_per_frame\": %.2f, \"frames_per_s\": %.1f, \"first_codes\": [%lld, %lld, %lld]}\n",
         frames, ms * 1e3 / frames, frames / (ms * 1e-3), (long long)codes[0], (long long)codes[1],
         (long long)codes[2]);
  SKCHECK(sk_destroy(e));
  for (float* p : bufs) hipFree(p);
  return 0;
}
