// Per-frame CFG decode engine: device state, weight binding, prefill,
// whole-frame hipGraph capture and replay (GraphFrameEngine counterpart,
// soraku_inference/acceleration/graph_frame.py:23-328).
//
// HBM layout (all FP32 unless the matrices are BF16):
//   x, hidden, prefix, abuf, ybuf  [rows][d]       residual stream / depth state
//   qkv                            [rows][(Hq+2Hkv) hd]
//   attn                           [rows][Hq hd]
//   act                            [rows][max(I, depth_inner)]
//   logits                         [rows][V]
//   K cache, V cache               [L][rows][Hkv][max_ctx][hd]
//   rope cos/sin                   [max_ctx][hd/2]
//   per-frame ring                 uniforms [F][n_utts][Q] f64, flags [F][2],
//                                  forced/codes [F][n_utts][Q] i64
// Row r = 2u is utterance u's cond row, 2u+1 its uncond row (cfg_rows = 2).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "sk_error.h"
#include "sk_kernels.h"
#include "sk_launch.h"
#include "sk_layer.h"
#include "sk_prefill.h"
#include "sk_wide.h"
#include "soraku_mi355x.h"

using namespace sk;

namespace {

struct LayerW {
  const void *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
  const void *gate = nullptr, *up = nullptr, *down = nullptr;
  const float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

template <typename T>
hipError_t dalloc(T** p, size_t n) {
  return hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T) + 256);
}

// Activation buffers of the batched prefill, M = packed prefix tokens.
struct PrefillBufs {
  float *X = nullptr, *Xn = nullptr, *QKV = nullptr, *Q = nullptr, *ATT = nullptr, *ACT = nullptr;
  int *tok_row = nullptr, *tok_pos = nullptr;
};

// Scratch of sk_prefill_run_noalloc: the prefill's activation buffers for up
// to SK_NOALLOC_SCRATCH_BYTES, in device memory the code object brings with
// it.  Host code never uses the symbol itself, only the address
// hipGetSymbolAddress returns for each device (scratch_ptr below).
static __device__ __align__(256) float scratch[SK_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// Looks up this device's copy of `scratch` once (the device must be current).
hipError_t scratch_ptr(int device, void** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return err;
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

// Bytes of PrefillBufs for M tokens, each buffer 256-byte aligned.
size_t prefill_bytes(const sk_config& c, int nqkv, size_t M) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t hq = (size_t)c.n_q_heads * c.head_dim;
  return up(M * c.d_model * 4) * 2 + up(M * nqkv * 4) + up(M * hq * 4) * 2 + up(M * c.trunk_inter * 4) +
         up(M * 4) * 2;
}

// Carves PrefillBufs for M tokens out of `base` (prefill_bytes(M) bytes).
PrefillBufs carve_prefill(const sk_config& c, int nqkv, size_t M, void* base) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t hq = (size_t)c.n_q_heads * c.head_dim;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* q = p; p += up(bytes); return q; };
  PrefillBufs b;
  b.X = reinterpret_cast<float*>(take(M * c.d_model * 4));
  b.Xn = reinterpret_cast<float*>(take(M * c.d_model * 4));
  b.QKV = reinterpret_cast<float*>(take(M * nqkv * 4));
  b.Q = reinterpret_cast<float*>(take(M * hq * 4));
  b.ATT = reinterpret_cast<float*>(take(M * hq * 4));
  b.ACT = reinterpret_cast<float*>(take(M * c.trunk_inter * 4));
  b.tok_row = reinterpret_cast<int*>(take(M * 4));
  b.tok_pos = reinterpret_cast<int*>(take(M * 4));
  return b;
}

}  // namespace

struct sk_engine {
  sk_config c{};
  int rows = 0, G = 0, nqkv = 0, inner_max = 0, max_chunks = 0;
  bool wide = false;          // more rows than the GEMV kernels take: skinny MFMA GEMMs
  int attn_splits = 0;        // > 0: attention_stream_kernel with this many splits per (row, kv head)
  bool split_k = false;       // many-row BF16 GEMMs may split K (workgroups i, i + 8, ... share an XCD)
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t order_ev = nullptr;   // recorded on `stream` when another engine's frames follow this one's

  // weights (borrowed)
  std::vector<LayerW> L;
  const float* final_norm = nullptr;
  const void* embed_tokens = nullptr;
  const void* table = nullptr;
  const void* out_proj = nullptr;   // untied classifier [Q][V][d]; the table when null
  const float *d_norm_in = nullptr, *d_norm_out = nullptr, *d_bias = nullptr, *lang = nullptr;
  const void *d_gate = nullptr, *d_up = nullptr, *d_down = nullptr;

  // device buffers (owned)
  float *x = nullptr, *hidden = nullptr, *prefix = nullptr, *prefix2 = nullptr, *abuf = nullptr,
        *ybuf = nullptr;
  float *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
  char *kc = nullptr, *vc = nullptr;   // KV caches, cfg.kv_dtype elements
  float *inv_freq = nullptr;
  float *part = nullptr, *dbg = nullptr, *embeds = nullptr;
  float2* rope = nullptr;     // [rows][hd/2] (cos, sin) at each row's position
  float* sk_partial = nullptr;  // many-row path: split-K slice partials
  unsigned* sk_arrive = nullptr;
  unsigned long long* sk_tpart = nullptr;   // split-K partials as tagged words
  size_t sk_tpart_bytes = 0;
  unsigned* sk_err = nullptr;              // bit 1: a split-K merge wait timed out
  int sk_tags = 0;                         // GEMM launches enqueued so far in the frame
  // Many-row path with BF16 weights: GEMM inputs in split form (written by
  // their producers) and per-tile sums of squares for the RMSNorms.
  uint16_t *xs_x = nullptr, *xs_attn = nullptr, *xs_act = nullptr, *xs_abuf = nullptr, *xs_y = nullptr;
  float *ss_x = nullptr, *ss_y = nullptr;   // [32][d_model / 16]
  int *kv_len = nullptr, *pos = nullptr, *active = nullptr, *plen = nullptr;
  int *fc = nullptr, *flag_ring = nullptr, *flag_cur = nullptr;
  double *u_ring = nullptr, *u_cur = nullptr;
  int64_t *forced_ring = nullptr, *codes_ring = nullptr, *stage_ids = nullptr, *stage_codes = nullptr;
  int* codes_cur = nullptr;
  SkParams* params = nullptr;

  // host mirrors
  int fc_host = 0;
  std::vector<int> active_host;   // rows decoding (advance each frame); retired rows do not
  bool prefilled = false;      // every row holds a prefix; cleared while a row is staged
  bool ran_full = false;       // an sk_prefill_run has completed (refills may follow)
  std::vector<int> kv_host, len_host;
  std::vector<char> staged;
  SkParams p_host{};

  // The frame graph.  Its chunk-attention nodes launch `grid_chunks` chunks
  // per (row, kv head), and its attn_o nodes take each row's chunk count as
  // an argument; before each replay the host sets both to the chunks the
  // rows hold (only when they change).  A larger grid or bound is always
  // correct (chunks past a row's length exit at once / are masked by its
  // length), and the counts only grow between prefills, so replays already
  // queued stay correct.
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<hipGraphNode_t> attn_nodes, o_nodes;
  std::vector<hipKernelNodeParams> attn_params, o_params;
  std::vector<GemvArgs> o_gargs;
  std::vector<AttnArgs> o_aargs;
  std::vector<void*> o_kp;           // kernelParams of the attn_o nodes: 2 per node
  int grid_chunks = 0;
  int row_chunks[4] = {0, 0, 0, 0};

  // One utterance's depth steps by code tables (depth_step_kernel): the
  // tables P_j[c] = W_gu (norm_in gain * table[j][c]) for j < Q-1, built when
  // the frame is captured, and the ping-pong G buffers [rows][2 * depth_inner].
  bool code_tables = false;
  bool wide_tables = false;          // many rows: the samplers form the next depth step's SwiGLU output
  float* ptab = nullptr;
  float* gbuf[2] = {nullptr, nullptr};

  // XCD-resident trunk layers (lx_attn_kernel + lx_mlp_kernel per layer, one
  // utterance with CFG, 8 KV heads): the residual stream's three rotating
  // fixed-point accumulators, barrier epochs and the error word (nonzero: a
  // barrier timed out).
  bool lx = false;
  unsigned long long spin_ticks = LX_SPIN_TICKS;   // bound of every barrier / exchange wait, in 10 ns ticks
  unsigned long long* lx_acc = nullptr;   // [3][rows][d], 2^-32 units
  uint2 *lx_qkv = nullptr, *lx_act = nullptr;   // tagged exchange words (zeroed at creation)
  unsigned *lx_flags = nullptr, *lx_err = nullptr;

  // batched prefill activations, sized for the largest packed prefix so far
  int pf_cap = 0;
  void* pf_mem = nullptr;
  PrefillBufs pf;
  int* p_row_start = nullptr;
  float2* p_rope = nullptr;   // [max_ctx + 1][hd/2] (cos, sin) by position, filled at creation
};

namespace {

size_t kv_layer_elems(const sk_engine* e) {
  return (size_t)e->rows * e->c.n_kv_heads * e->c.max_ctx * e->c.head_dim;
}
size_t kv_layer_bytes(const sk_engine* e) {
  return kv_layer_elems(e) * (e->c.kv_dtype == SK_BF16 ? 2 : 4);
}

void drop_graphs(sk_engine* e) {
  if (e->exec) hipGraphExecDestroy(e->exec);
  if (e->graph) hipGraphDestroy(e->graph);
  e->exec = nullptr; e->graph = nullptr;
  e->attn_nodes.clear();
  e->attn_params.clear();
  e->o_nodes.clear();
  e->o_params.clear();
  e->o_gargs.clear();
  e->o_aargs.clear();
  e->o_kp.clear();
  e->grid_chunks = 0;
  for (int& v : e->row_chunks) v = 0;
}

// Each row's chunk count for the frame `ahead` frames after the host's
// state, once that frame's token is appended (1 for inactive rows).
int row_frame_chunks(const sk_engine* e, int r, int ahead) {
  if (!e->active_host[r]) return 1;
  return std::min(e->max_chunks, (e->kv_host[r] + ahead + 1 + ATT_CHUNK - 1) / ATT_CHUNK);
}

// Point the graph's chunk-attention nodes and attn_o nodes at the frame's
// chunk counts (no-op when unchanged).
hipError_t set_frame_chunks(sk_engine* e, int ahead) {
  if (!e->exec) return hipSuccess;
  int rc[4] = {1, 1, 1, 1}, nch = 1;
  for (int r = 0; r < e->rows && r < 4; ++r) nch = std::max(nch, rc[r] = row_frame_chunks(e, r, ahead));
  for (int r = 4; r < e->rows; ++r) nch = std::max(nch, row_frame_chunks(e, r, ahead));
  hipError_t err = hipSuccess;
  if (nch != e->grid_chunks) {
    for (size_t i = 0; i < e->attn_nodes.size() && err == hipSuccess; ++i) {
      e->attn_params[i].gridDim.x = nch;
      err = hipGraphExecKernelNodeSetParams(e->exec, e->attn_nodes[i], &e->attn_params[i]);
    }
    if (err != hipSuccess) return err;
    e->grid_chunks = nch;
  }
  if (!std::equal(rc, rc + 4, e->row_chunks)) {
    for (size_t i = 0; i < e->o_nodes.size() && err == hipSuccess; ++i) {
      for (int r = 0; r < 4; ++r) e->o_aargs[i].row_chunks[r] = rc[r];
      err = hipGraphExecKernelNodeSetParams(e->exec, e->o_nodes[i], &e->o_params[i]);
    }
    if (err != hipSuccess) return err;
    std::copy(rc, rc + 4, e->row_chunks);
  }
  return hipSuccess;
}

// The captured frame is a chain; collect its chunk-attention kernel nodes.
hipError_t find_attn_nodes(sk_engine* e) {
  size_t n = 0;
  hipError_t err = hipGraphGetNodes(e->graph, nullptr, &n);
  if (err != hipSuccess) return err;
  std::vector<hipGraphNode_t> nodes(n);
  if ((err = hipGraphGetNodes(e->graph, nodes.data(), &n)) != hipSuccess) return err;
  const void* fns[2] = {reinterpret_cast<const void*>(attention_kernel<float>),
                        reinterpret_cast<const void*>(attention_kernel<uint16_t>)};
  const void* ofns[6] = {reinterpret_cast<const void*>(attn_o_kernel<1, 2048, 1, WF32>),
                         reinterpret_cast<const void*>(attn_o_kernel<2, 2048, 1, WF32>),
                         reinterpret_cast<const void*>(attn_o_kernel<4, 2048, 1, WF32>),
                         reinterpret_cast<const void*>(attn_o_kernel<1, 2048, 1, WBF16>),
                         reinterpret_cast<const void*>(attn_o_kernel<2, 2048, 1, WBF16>),
                         reinterpret_cast<const void*>(attn_o_kernel<4, 2048, 1, WBF16>)};
  for (hipGraphNode_t node : nodes) {
    hipGraphNodeType t;
    if ((err = hipGraphNodeGetType(node, &t)) != hipSuccess) return err;
    if (t != hipGraphNodeTypeKernel) continue;
    hipKernelNodeParams p{};
    if ((err = hipGraphKernelNodeGetParams(node, &p)) != hipSuccess) return err;
    if (p.func == fns[0] || p.func == fns[1]) {
      e->attn_nodes.push_back(node);
      e->attn_params.push_back(p);
    } else if (std::find(ofns, ofns + 6, p.func) != ofns + 6) {
      // own copies of the (GemvArgs, AttnArgs) arguments, to rewrite row_chunks
      e->o_nodes.push_back(node);
      e->o_params.push_back(p);
      e->o_gargs.push_back(*static_cast<const GemvArgs*>(p.kernelParams[0]));
      e->o_aargs.push_back(*static_cast<const AttnArgs*>(p.kernelParams[1]));
    }
  }
  e->o_kp.resize(2 * e->o_nodes.size());
  for (size_t i = 0; i < e->o_nodes.size(); ++i) {
    e->o_kp[2 * i] = &e->o_gargs[i];
    e->o_kp[2 * i + 1] = &e->o_aargs[i];
    e->o_params[i].kernelParams = &e->o_kp[2 * i];
    e->o_params[i].extra = nullptr;
  }
  e->grid_chunks = e->max_chunks;   // as captured
  for (int r = 0; r < 4; ++r) e->row_chunks[r] = e->max_chunks;
  return hipSuccess;
}

int validate_config(const sk_config* c) {
  SK_CHECK(c != nullptr, SK_EINVAL, "config is NULL");
  SK_CHECK(c->d_model > 0 && c->d_model % 32 == 0, SK_EINVAL, "d_model must be a positive multiple of 32");
  SK_CHECK(c->n_layers > 0, SK_EINVAL, "n_layers must be positive");
  SK_CHECK(c->n_q_heads > 0 && c->n_kv_heads > 0 && c->n_q_heads % c->n_kv_heads == 0, SK_EINVAL,
           "n_q_heads must be a positive multiple of n_kv_heads");
  const int hd = c->head_dim;
  SK_CHECK(hd == 16 || hd == 32 || hd == 64 || hd == 128,
           SK_EINVAL, "head_dim must be a power of two in [16, 128]");
  SK_CHECK(32 % (c->n_q_heads / c->n_kv_heads) == 0, SK_EINVAL, "n_q_heads / n_kv_heads must divide 32");
  SK_CHECK(c->trunk_inter > 0 && c->trunk_inter % 32 == 0, SK_EINVAL, "trunk_inter must be a positive multiple of 32");
  SK_CHECK(c->n_q_heads * hd % 32 == 0, SK_EINVAL, "n_q_heads * head_dim must be a multiple of 32");
  SK_CHECK(c->depth_inner > 0 && c->depth_inner % 8 == 0, SK_EINVAL, "depth_inner must be a positive multiple of 8");
  SK_CHECK(c->n_codebooks > 0 && c->n_codebooks <= 64, SK_EINVAL, "n_codebooks must be in [1, 64]");
  SK_CHECK(c->audio_vocab > 3 && c->audio_vocab <= MAX_V, SK_EINVAL, "audio_vocab must be in [4, %d]", MAX_V);
  SK_CHECK(c->text_vocab > 0, SK_EINVAL, "text_vocab must be positive");
  SK_CHECK(c->bos_id >= 0 && c->bos_id < c->audio_vocab && c->eos_id >= 0 && c->eos_id < c->audio_vocab &&
               c->pad_id >= 0 && c->pad_id < c->audio_vocab,
           SK_EINVAL, "special ids must lie inside the audio vocabulary");
  SK_CHECK(c->trunk_eps > 0.f && c->depth_eps > 0.f && c->rope_theta > 0.f, SK_EINVAL,
           "eps and rope_theta must be positive");
  SK_CHECK(c->weight_dtype == SK_F32 || c->weight_dtype == SK_BF16, SK_EINVAL, "weight_dtype must be SK_F32 or SK_BF16");
  SK_CHECK(c->kv_dtype == SK_F32 || c->kv_dtype == SK_BF16, SK_EINVAL, "kv_dtype must be SK_F32 or SK_BF16");
  SK_CHECK(c->cfg_rows == 1 || c->cfg_rows == 2, SK_EINVAL, "cfg_rows must be 1 or 2");
  SK_CHECK(c->n_utts >= 1 && c->n_utts * c->cfg_rows <= SK_ROWS, SK_EINVAL,
           "n_utts * cfg_rows must be in [1, %d] (decode rows)", SK_ROWS);
  SK_CHECK(c->n_utts * c->cfg_rows <= 4 || c->depth_inner % 32 == 0, SK_EINVAL,
           "depth_inner must be a multiple of 32 for more than 4 decode rows");
  // The many-row sampler writes the next depth input with DEPTH_DPT values
  // per thread (depth_input_rows): d_model <= DEPTH_DPT * SNT = 4096.
  SK_CHECK(c->n_utts * c->cfg_rows <= 4 || c->d_model <= DEPTH_DPT * SNT, SK_EINVAL,
           "d_model must be at most %d for more than 4 decode rows", DEPTH_DPT * SNT);
  SK_CHECK(c->max_ctx >= 2 && c->max_ctx <= 65536, SK_EINVAL, "max_ctx must be in [2, 65536]");
  SK_CHECK(c->max_frames >= 1, SK_EINVAL, "max_frames must be positive");
  SK_CHECK(c->n_language == 0 || c->n_language == 4, SK_EINVAL, "n_language must be 0 or 4");
  SK_CHECK((c->n_q_heads / c->n_kv_heads) * hd <= 256 && c->n_q_heads / c->n_kv_heads <= 8, SK_EINVAL,
           "GQA group too large (<= 8 q heads per kv head, q heads x head_dim <= 256)");
  return SK_OK;
}

// FP32 RoPE inverse frequencies 1 / theta^(2i/hd) (modeling_qwen3.py:116-122);
// the kernels form the FP32 angle pos * inv_freq and its cos/sin
// (modeling_qwen3.py:126-137).
std::vector<float> rope_inv_freq(const sk_config& c) {
  const int half = c.head_dim / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i) {
    const float ex = (float)(2 * i) / (float)c.head_dim;
    inv[i] = 1.0f / powf(c.rope_theta, ex);
  }
  return inv;
}

int check_decode_weights(const sk_engine* e) {
  for (int i = 0; i < e->c.n_layers; ++i) {
    const LayerW& w = e->L[i];
    SK_CHECK(w.q && w.k && w.v && w.o && w.gate && w.up && w.down && w.in_norm && w.post_norm &&
                 w.q_norm && w.k_norm,
             SK_ENOWEIGHT, "trunk.layers.%d is not fully bound", i);
  }
  SK_CHECK(e->final_norm, SK_ENOWEIGHT, "trunk.norm.weight is not bound");
  SK_CHECK(e->table, SK_ENOWEIGHT, "audio_codebooks.table is not bound");
  SK_CHECK(e->d_norm_in && e->d_norm_out && e->d_bias && e->d_gate && e->d_up && e->d_down,
           SK_ENOWEIGHT, "depth_head is not fully bound");
  return SK_OK;
}

// ---- graph bodies -------------------------------------------------------

// ---- many-row path: skinny MFMA GEMMs ---------------------------------------

// 16 waves per workgroup (K split 16 ways) when there are few workgroups
// (N <= 1024 outputs, one weight matrix), else 8.  NORM: RMSNorm of x folded in.
template <int EPI, bool NORM, typename WL>
hipError_t launch_skinny_w(const SkinnyArgs& a, hipStream_t st) {
  const dim3 grid((a.N + 15) / 16);
  if (EPI != EPI_SWIGLU && a.N <= 1024)
    hipLaunchKernelGGL((skinny_gemm_kernel<EPI, WL, 16, NORM>), grid, dim3(16 * 64), 0, st, a);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<EPI, WL, 8, NORM>), grid, dim3(8 * 64), 0, st, a);
  return hipGetLastError();
}
// BF16 weights: K split over 4 or 2 workgroups per output tile when the
// tiles alone would fill fewer than 256 CUs (tiles a multiple of 8, K slices
// a multiple of 32); the slice partials live in `partial`, the arrival counts
// in `arrive` (zero between launches).
template <int EPI, bool NORM>
hipError_t launch_skinny_bf16(SkinnyArgs a, float* partial, unsigned* arrive, bool allow_split, hipStream_t st) {
  const int tiles = (a.N + 15) / 16;
  a.ksplit = 1;
  if (allow_split && tiles % 8 == 0) {
    if (tiles <= 64 && a.K % (4 * 32) == 0) a.ksplit = 4;
    else if (tiles <= 128 && a.K % (2 * 32) == 0) a.ksplit = 2;
  }
  static_assert(SK_MAX_SPLIT >= 4, "the kernel's split-K merge covers the splits chosen here");
  a.partial = partial; a.arrive = arrive;
  const dim3 grid(tiles * a.ksplit);
  if (a.xs)
    hipLaunchKernelGGL((skinny_bf16_kernel<EPI, 8, NORM, true>), grid, dim3(8 * 64), 0, st, a);
  else
    hipLaunchKernelGGL((skinny_bf16_kernel<EPI, 8, NORM, false>), grid, dim3(8 * 64), 0, st, a);
  return hipGetLastError();
}
template <int EPI, bool NORM = false>
hipError_t launch_skinny(sk_engine* e, const SkinnyArgs& a0) {
  SkinnyArgs a = a0;
  if (e->sk_tags < 255) {   // a distinct tag per launch of the frame (tag_idx < 255)
    a.tpart = e->sk_tpart; a.fc = e->fc; a.tag_idx = e->sk_tags++;
    a.err = e->sk_err; a.spin = e->spin_ticks;
  }
  return e->c.weight_dtype == SK_BF16 ? launch_skinny_bf16<EPI, NORM>(a, e->sk_partial, e->sk_arrive, e->split_k,
                                                                      e->stream)
                                      : launch_skinny_w<EPI, NORM, WF32>(a, e->stream);
}

SkinnyArgs skinny_args(const void* w, int N, int K, const float* x, int ldx, float* out, int ldo, int R) {
  SkinnyArgs a{};
  a.w[0] = w; a.w[1] = nullptr; a.w[2] = nullptr;
  a.seg_rows[0] = N; a.seg_rows[1] = 0; a.seg_rows[2] = 0;
  a.x = x; a.ldx = ldx; a.out = out; a.ldo = ldo;
  a.R = R; a.N = N; a.K = K;
  return a;
}

// Chunked decode attention: one workgroup per 32-token chunk of each (row,
// kv head), merged by attention_combine_kernel.  Few rows: the chunks fill
// the chip.
hipError_t launch_attn_chunks(sk_engine* e, const AttnArgs& at, bool merge = true) {
  const size_t asmem = attn_smem_floats(e->G, at.hd) * sizeof(float);
  const dim3 grid(e->max_chunks, at.Hkv, e->rows);   // replays set it to the live chunks
  if (e->c.kv_dtype == SK_BF16)
    hipLaunchKernelGGL(attention_kernel<uint16_t>, grid, dim3(NT), asmem, e->stream, at);
  else
    hipLaunchKernelGGL(attention_kernel<float>, grid, dim3(NT), asmem, e->stream, at);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !merge) return err;
  hipLaunchKernelGGL(attention_combine_kernel, dim3(at.Hq, e->rows), dim3(NT), 0, e->stream, at);
  return hipGetLastError();
}

// Output projection + residual with the attention chunk merge folded in
// (attn_o_kernel): instantiated for K = Hq * hd = 2048 and 1, 2 or 4 decode
// rows; attn_o_fits says whether an engine takes it, otherwise the chunk
// merge kernel + residual GEMV run instead.
template <int M, typename WL>
hipError_t launch_attn_o_m(const GemvArgs& g, const AttnArgs& at, hipStream_t st) {
  constexpr int RW = 1;
  const int grid = (g.N + (AO_NT / 64) * RW - 1) / ((AO_NT / 64) * RW);
  hipLaunchKernelGGL((attn_o_kernel<M, 2048, RW, WL>), dim3(grid), dim3(AO_NT), 0, st, g, at);
  return hipGetLastError();
}
bool attn_o_fits(const sk_engine* e) {
  const int K = e->c.n_q_heads * e->c.head_dim, M = e->rows;
  const int vpth = M * K / AO_NT;
  return !e->wide && e->attn_splits == 0 && K == 2048 && (M == 1 || M == 2 || M == 4) && e->c.head_dim % vpth == 0;
}
template <typename WL>
hipError_t launch_attn_o_w(int M, const GemvArgs& g, const AttnArgs& at, hipStream_t st) {
  switch (M) {
    case 1: return launch_attn_o_m<1, WL>(g, at, st);
    case 2: return launch_attn_o_m<2, WL>(g, at, st);
    default: return launch_attn_o_m<4, WL>(g, at, st);
  }
}

// Streaming decode attention (many rows): attn_splits workgroups per (row,
// kv head); with one split the kernel writes the output itself.
constexpr int ATTN_STREAM_NTH = 512;
constexpr int ATTN_STREAM_DEPTH = 2;   // tokens in flight per slot
template <typename KT, int G>
hipError_t launch_attn_stream_g(sk_engine* e, AttnArgs at) {
  const int S = e->attn_splits;
  at.nparts = S > 1 ? S : 0;
  const size_t smem = attn_stream_smem_floats(G, at.hd, ATTN_STREAM_NTH) * sizeof(float);
  // 4 query heads: one token in flight keeps the state in registers
  constexpr int D = G >= 4 ? 1 : ATTN_STREAM_DEPTH;
  hipLaunchKernelGGL((attention_stream_kernel<KT, G, ATTN_STREAM_NTH, D>), dim3(S, at.Hkv, e->rows),
                     dim3(ATTN_STREAM_NTH), smem, e->stream, at, S);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || S == 1) return err;
  hipLaunchKernelGGL(attention_combine_kernel, dim3(at.Hq, e->rows), dim3(NT), 0, e->stream, at);
  return hipGetLastError();
}
template <typename KT>
hipError_t launch_attn_stream_kt(sk_engine* e, const AttnArgs& at) {
  switch (e->G) {
    case 1: return launch_attn_stream_g<KT, 1>(e, at);
    case 2: return launch_attn_stream_g<KT, 2>(e, at);
    case 4: return launch_attn_stream_g<KT, 4>(e, at);
    default: return hipErrorInvalidConfiguration;   // not selected at creation
  }
}
hipError_t launch_attn_stream(sk_engine* e, const AttnArgs& at) {
  return e->c.kv_dtype == SK_BF16 ? launch_attn_stream_kt<uint16_t>(e, at) : launch_attn_stream_kt<float>(e, at);
}

// XCD-resident layers (sk_layer.h): one utterance with CFG, 16 q / 8 KV heads
// of 128, at the Qwen3-0.6B trunk shape (d 1024, SwiGLU 3072) or the
// Qwen3-1.7B one (d 2048, SwiGLU 6144), FP32 or BF16 weights and cache.
bool lx_fits(const sk_engine* e) {
  const sk_config& c = e->c;
  const bool shape = (c.d_model == 1024 && c.trunk_inter == 3072) || (c.d_model == 2048 && c.trunk_inter == 6144);
  // n_layers % 3 == 2 would leave the trunk's output in accumulator 1, the
  // next frame's first-layer target, which the frame's last launch must zero
  // after every workgroup has read the whole output: one kernel cannot order
  // that, so such trunks keep the five-kernel layers.
  return e->rows == LX_M && !e->wide && e->attn_splits == 0 && c.n_kv_heads == LX_HKV && c.n_q_heads == LX_HQ &&
         c.head_dim == LX_HD && shape && e->max_chunks <= LX_MAXCH && c.n_layers % 3 != 2;
}

template <typename WL, typename KT>
hipError_t launch_lx(int d, bool first, const LxArgs& A, const LxArgs& C, hipStream_t st) {
  if (d == 1024) {
    if (first) hipLaunchKernelGGL((lx_attn_kernel<WL, KT, 1024, false>), dim3(LX_WGS), dim3(LX_NT), 0, st, A);
    else hipLaunchKernelGGL((lx_attn_kernel<WL, KT, 1024, true>), dim3(LX_WGS), dim3(LX_NT), 0, st, A);
    hipLaunchKernelGGL((lx_mlp_kernel<WL, 1024, 3072>), dim3(LX_WGS), dim3(LX_NT), 0, st, C);
  } else {
    if (first) hipLaunchKernelGGL((lx_attn_kernel<WL, KT, 2048, false>), dim3(LX_WGS), dim3(LX_NT), 0, st, A);
    else hipLaunchKernelGGL((lx_attn_kernel<WL, KT, 2048, true>), dim3(LX_WGS), dim3(LX_NT), 0, st, A);
    hipLaunchKernelGGL((lx_mlp8_kernel<WL, 2048, 6144>), dim3(LX_WGS), dim3(LX_NT), 0, st, C);
  }
  return hipGetLastError();
}

// Fixed-point accumulator k % 3 of the XCD-resident layers (sk_layer.h).
unsigned long long* lx_acc(const sk_engine* e, int k) {
  return e->lx_acc + (size_t)(k % 3) * e->rows * e->c.d_model;
}

// Each layer as two launches: attention half (x -> q/k/v -> attention -> O
// partials) and MLP half (x -> SwiGLU -> down partials).  Launch i = 2 l + h
// reads accumulator i (the first one the FP32 frame embedding), adds x and
// its partials into accumulator i + 1 and clears accumulator i + 2; the final
// norm reads accumulator 2 L and clears accumulator 1, the first launch's
// target of the next frame.
hipError_t enqueue_trunk_lx(sk_engine* e) {
  const sk_config& c = e->c;
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = e->L[l];
    const int i = 2 * l;
    LxArgs A{};
    A.wq = w.q; A.wk = w.k; A.wv = w.v; A.wo = w.o;
    A.gain = w.in_norm; A.q_norm = w.q_norm; A.k_norm = w.k_norm;
    A.xin = e->x;
    A.acc_in = reinterpret_cast<const long long*>(lx_acc(e, i));
    A.acc_out = lx_acc(e, i + 1);
    A.acc_clear = lx_acc(e, i + 2);
    A.qkv = e->lx_qkv; A.part = e->part; A.act = e->lx_act; A.ld_act = c.trunk_inter;
    A.kc = e->kc + (size_t)l * kv_layer_bytes(e);
    A.vc = e->vc + (size_t)l * kv_layer_bytes(e);
    A.rope = e->rope; A.kv_len = e->kv_len; A.active = e->active;
    A.flags = e->lx_flags; A.err = e->lx_err;
    A.max_ctx = c.max_ctx; A.max_chunks = e->max_chunks;
    A.eps = c.trunk_eps; A.scale = 1.0f / sqrtf((float)c.head_dim);
    A.spin_ticks = e->spin_ticks;
    LxArgs C = A;
    C.wg = w.gate; C.wu = w.up; C.wd = w.down; C.gain = w.post_norm;
    C.acc_in = reinterpret_cast<const long long*>(lx_acc(e, i + 1));
    C.acc_out = lx_acc(e, i + 2);
    C.acc_clear = lx_acc(e, i + 3);
    const bool wbf = c.weight_dtype == SK_BF16, kbf = c.kv_dtype == SK_BF16;
    const int d = c.d_model;
    const bool first = l == 0;
    const hipError_t err = wbf ? (kbf ? launch_lx<WBF16, uint16_t>(d, first, A, C, e->stream)
                                      : launch_lx<WBF16, float>(d, first, A, C, e->stream))
                               : (kbf ? launch_lx<WF32, uint16_t>(d, first, A, C, e->stream)
                                      : launch_lx<WF32, float>(d, first, A, C, e->stream));
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

hipError_t enqueue_trunk(sk_engine* e) {
  if (e->lx) return enqueue_trunk_lx(e);
  const sk_config& c = e->c;
  const int d = c.d_model, hd = c.head_dim, M = e->rows;
  const int wt = c.weight_dtype;
  hipError_t err;
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = e->L[l];
    GemvArgs a = gemv_args(w.q, e->nqkv, d, e->x, d, e->qkv, e->nqkv);
    a.w[1] = w.k; a.w[2] = w.v;
    a.seg_rows[0] = c.n_q_heads * hd; a.seg_rows[1] = c.n_kv_heads * hd; a.seg_rows[2] = c.n_kv_heads * hd;
    a.norm_w = w.in_norm; a.eps = c.trunk_eps;
    if (e->wide) {
      SkinnyArgs k = skinny_args(w.q, e->nqkv, d, e->x, d, e->qkv, e->nqkv, M);
      k.w[1] = w.k; k.w[2] = w.v;
      k.seg_rows[0] = a.seg_rows[0]; k.seg_rows[1] = a.seg_rows[1]; k.seg_rows[2] = a.seg_rows[2];
      k.norm_w = w.in_norm; k.eps = c.trunk_eps;
      if (e->xs_x && l > 0) { k.xs = e->xs_x; k.ss_in = e->ss_x; k.n_ss = d / 16; }   // from the last down
      if ((err = launch_skinny<EPI_STORE, true>(e, k)) != hipSuccess) return err;
    } else if ((err = launch_gemv<PRO_NORM, EPI_STORE>(wt, M, a, e->stream)) != hipSuccess) {
      return err;
    }

    AttnArgs at{};
    at.qkv = e->qkv; at.ldqkv = e->nqkv;
    at.kc = e->kc + (size_t)l * kv_layer_bytes(e);
    at.vc = e->vc + (size_t)l * kv_layer_bytes(e);
    at.qn_w = w.q_norm; at.kn_w = w.k_norm; at.eps = c.trunk_eps;
    at.rope = e->rope;
    at.part = e->part; at.max_chunks = e->max_chunks;
    at.kv_len = e->kv_len; at.active = e->active;
    at.out = e->attn; at.ldo = c.n_q_heads * hd;
    at.Hq = c.n_q_heads; at.Hkv = c.n_kv_heads; at.hd = hd; at.max_ctx = c.max_ctx;

    at.scale = 1.0f / sqrtf((float)hd);
    at.xs_out = e->xs_attn;
    for (int& rc : at.row_chunks) rc = e->max_chunks;   // replays set each row's count
    const bool fused_o = attn_o_fits(e);
    if ((err = e->attn_splits > 0 ? launch_attn_stream(e, at) : launch_attn_chunks(e, at, !fused_o)) != hipSuccess)
      return err;

    if (e->wide) {
      const int hq = c.n_q_heads * hd, I = c.trunk_inter;
      const bool xs = e->xs_x != nullptr;
      SkinnyArgs k = skinny_args(w.o, d, hq, e->attn, hq, e->x, d, M);
      k.res = e->x; k.ldr = d;
      if (xs) { k.xs = e->xs_attn; k.xs_out = e->xs_x; k.xs_gain = w.post_norm; k.ss_out = e->ss_x; }
      if ((err = launch_skinny<EPI_RESID>(e, k)) != hipSuccess) return err;
      k = skinny_args(w.gate, I, d, e->x, d, e->act, e->inner_max, M);
      k.w2 = w.up; k.norm_w = w.post_norm; k.eps = c.trunk_eps;
      if (xs) { k.xs = e->xs_x; k.ss_in = e->ss_x; k.n_ss = d / 16; k.xs_out = e->xs_act; }
      if ((err = launch_skinny<EPI_SWIGLU, true>(e, k)) != hipSuccess) return err;
      k = skinny_args(w.down, d, I, e->act, e->inner_max, e->x, d, M);
      k.res = e->x; k.ldr = d;
      if (xs) {
        k.xs = e->xs_act;
        if (l + 1 < c.n_layers) { k.xs_out = e->xs_x; k.xs_gain = e->L[l + 1].in_norm; k.ss_out = e->ss_x; }
      }
      if ((err = launch_skinny<EPI_RESID>(e, k)) != hipSuccess) return err;
      continue;
    }
    a = gemv_args(w.o, d, c.n_q_heads * hd, e->attn, c.n_q_heads * hd, e->x, d);
    a.res = e->x; a.ldr = d;
    err = fused_o ? (wt == SK_BF16 ? launch_attn_o_w<WBF16>(M, a, at, e->stream)
                                   : launch_attn_o_w<WF32>(M, a, at, e->stream))
                  : launch_gemv<PRO_NONE, EPI_RESID>(wt, M, a, e->stream);
    if (err != hipSuccess) return err;

    a = gemv_args(w.gate, c.trunk_inter, d, e->x, d, e->act, e->inner_max);
    a.w[1] = w.up; a.norm_w = w.post_norm; a.eps = c.trunk_eps;
    if ((err = launch_gemv<PRO_NORM, EPI_SWIGLU>(wt, M, a, e->stream)) != hipSuccess) return err;

    a = gemv_args(w.down, d, c.trunk_inter, e->act, e->inner_max, e->x, d);
    a.res = e->x; a.ldr = d;
    if ((err = launch_gemv<PRO_NONE, EPI_RESID>(wt, M, a, e->stream)) != hipSuccess) return err;
  }
  return hipSuccess;
}

// Depth step q of the many-row path: prefix advance + norm_in, SwiGLU, down +
// residual, norm_out, classifier + bias (the sampler follows).
hipError_t enqueue_depth_wide(sk_engine* e, int q) {
  const sk_config& c = e->c;
  const int d = c.d_model, M = e->rows, V = c.audio_vocab, wt = c.weight_dtype;
  const size_t tsz = (wt == SK_BF16) ? 2 : 4;
  hipError_t err;
  const bool xs = e->xs_abuf != nullptr;
  SkinnyArgs k;
  // With code tables only codebook 0 runs the gate/up GEMM (its gate and up
  // before the activation, r_0 G_0, kept for the samplers); codebook q's
  // SwiGLU output comes from the sampler of q - 1.
  if (!e->wide_tables || q == 0) {
    k = skinny_args(e->d_gate, c.depth_inner, d, e->abuf, d, e->act, e->inner_max, M);
    k.w2 = e->d_up;
    if (xs) { k.xs = e->xs_abuf; k.xs_out = e->xs_act; }
    if (e->wide_tables) { k.pre_out = e->gbuf[0]; k.ld_pre = 2 * c.depth_inner; }
    if ((err = launch_skinny<EPI_SWIGLU>(e, k)) != hipSuccess) return err;
  }
  k = skinny_args(e->d_down, d, c.depth_inner, e->act, e->inner_max, e->ybuf, d, M);
  k.res = e->abuf; k.ldr = d;
  if (xs) { k.xs = e->xs_act; k.xs_out = e->xs_y; k.xs_gain = e->d_norm_out; k.ss_out = e->ss_y; }
  if ((err = launch_skinny<EPI_RESID>(e, k)) != hipSuccess) return err;
  const void* tq = static_cast<const char*>(e->out_proj ? e->out_proj : e->table) + (size_t)q * V * d * tsz;
  k = skinny_args(tq, V, d, e->ybuf, d, e->logits, V, M);
  k.bias = e->d_bias + (size_t)q * V; k.norm_w = e->d_norm_out; k.eps = c.depth_eps;
  if (xs) { k.xs = e->xs_y; k.ss_in = e->ss_y; k.n_ss = d / 16; }
  return launch_skinny<EPI_BIAS, true>(e, k);
}

hipError_t enqueue_tail(sk_engine* e);

// Depth-step arguments of the code-table path (the per-step buffers are set
// by the caller).
DepthArgs depth_args(sk_engine* e) {
  const sk_config& c = e->c;
  DepthArgs g{};
  g.w_gate = e->d_gate; g.w_up = e->d_up; g.w_down = e->d_down; g.hidden = e->hidden;
  g.norm_w = e->d_norm_in; g.eps = c.depth_eps; g.ptab = e->ptab; g.y = e->ybuf; g.scale = c.frame_scale;
  return g;
}
// G_1 = W_gu (w_in * hidden) of the code-table path into gbuf[0], where
// codebook 0's step reads it: after a prefill and at capture (a frame
// computes it for the next one at its end).
hipError_t launch_g1(sk_engine* e) {
  DepthArgs g = depth_args(e);
  g.g_out = e->gbuf[0];
  SampleArgs s{};
  return launch_depth_step<0>(e->c.weight_dtype, e->c.d_model, s, g, 0, e->stream);
}

hipError_t enqueue_frame(sk_engine* e) {
  const sk_config& c = e->c;
  const int d = c.d_model, M = e->rows, V = c.audio_vocab;
  e->sk_tags = 0;
  const int wt = c.weight_dtype;
  const size_t tsz = (wt == SK_BF16) ? 2 : 4;
  hipError_t err;
  SampleArgs s{};
  s.logits = e->logits; s.ldl = V; s.rows_per_utt = c.cfg_rows; s.V = V;
  s.params = e->params; s.fc = e->fc;
  s.u_cur = e->u_cur; s.flag_cur = e->flag_cur; s.forced_ring = e->forced_ring;
  s.codes_ring = e->codes_ring; s.codes_cur = e->codes_cur; s.dbg = e->dbg; s.table = e->table;
  s.prefix = e->prefix; s.xnext = e->x; s.d = d; s.Q = c.n_codebooks; s.scale = c.frame_scale;
  s.bos = c.bos_id; s.eos = c.eos_id; s.pad = c.pad_id; s.n_utts = c.n_utts;
  // Depth step inputs.  Many rows: step 0's abuf = RMSNorm_in(hidden) comes
  // from the trunk's final norm (or the prefill), and the sampler launch of
  // step q advances its rows' codebook prefix with code q and writes step
  // q+1's abuf -- no separate launch.  Few rows: the gate/up GEMV's prologue
  // forms it; step q >= 1 reads the previous step's prefix, adds the embedding
  // of code q-1 and writes the result to the other buffer of the pair (readers
  // of one launch never see its own writes).  Either way the last sampler
  // launch writes the frame embedding and zeroes `prefix` again.
  if (e->wide) {
    s.hidden = e->hidden; s.w_in = e->d_norm_in; s.eps_in = c.depth_eps;
    s.abuf = e->abuf; s.xs_abuf = e->xs_abuf;
  }
  // One utterance with code tables: per codebook one depth_step_kernel launch
  // (codebook q-1's sampler, the prefix, SwiGLU, down projection and the next
  // step's G) and the classifier; codebook 0 takes G_1, then SwiGLU + down.
  if (e->code_tables) {
    DepthArgs g = depth_args(e);
    for (int q = 0; q < c.n_codebooks; ++q) {
      if (q == 0) {   // G_1 is in gbuf[0]: from the previous frame's end, the prefill or the capture
        g.g_in = e->gbuf[0];
        if ((err = launch_depth_step<1>(wt, d, s, g, 0, e->stream)) != hipSuccess) return err;
      } else {
        g.prefix_in = (q % 2 == 1) ? e->prefix : e->prefix2;
        g.prefix_out = (q % 2 == 1) ? e->prefix2 : e->prefix;
        g.g_in = e->gbuf[(q - 1) % 2];
        g.g_out = e->gbuf[q % 2];
        // the last codebook too: its G_{q+1} lands in gbuf[1], which codebook
        // 1 of the next frame rewrites before codebook 2 reads it (a variant
        // without that store ran ~1.3 us (0.6B) / ~2.5 us (1.7B) slower)
        err = launch_depth_step<2>(wt, d, s, g, q, e->stream);
        if (err != hipSuccess) return err;
      }
      const void* tq = static_cast<const char*>(e->out_proj ? e->out_proj : e->table) + (size_t)q * V * d * tsz;
      GemvArgs a = gemv_args(tq, V, d, e->ybuf, d, e->logits, V);
      a.norm_w = e->d_norm_out; a.eps = c.depth_eps; a.bias = e->d_bias + (size_t)q * V;
      if ((err = launch_gemv<PRO_NORM, EPI_BIAS>(wt, M, a, e->stream)) != hipSuccess) return err;
    }
    // the prefix through codebook Q-2, written by the last depth step
    s.prefix_last = (c.n_codebooks - 1) % 2 == 1 ? e->prefix2 : e->prefix;
    err = (wt == SK_BF16) ? launch_sample_step<WBF16>(s, c.n_codebooks - 1, 1, e->stream)
                          : launch_sample_step<WF32>(s, c.n_codebooks - 1, 1, e->stream);
    if (err != hipSuccess) return err;
    return enqueue_tail(e);
  }
  // One utterance: codebook q-1's sampler runs inside codebook q's gate/up
  // launch (depth_sample_gemv_kernel); only the last codebook's has its own.
  const bool fuse = !e->wide && c.n_utts == 1 && depth_fused_fits(d, M, c.depth_inner, V);
  for (int q = 0; q < c.n_codebooks; ++q) {
    if (e->wide) {
      if ((err = enqueue_depth_wide(e, q)) != hipSuccess) return err;
      int slices = 1;
      if (e->wide_tables) {   // G_q in gbuf[q % 2] (after codebook 0: r_0 G_0), G_{q+1} into the other
        s.ptab = e->ptab; s.ki = c.depth_inner;
        s.g_in = e->gbuf[q % 2];
        s.g_out = q + 2 < c.n_codebooks ? e->gbuf[(q + 1) % 2] : nullptr;
        s.g_in_normed = q == 0;
        s.act = e->act; s.ld_act = e->inner_max; s.xs_act = e->xs_act;
        // Several workgroups per utterance (each draws the code, each writes
        // a slice), reading the prefix from one buffer and writing the other;
        // the last codebook's sampler clears `prefix`, where codebook 0 reads.
        if (q + 1 < c.n_codebooks) {
          slices = sample_slices(c.n_utts, d, c.depth_inner);
          s.prefix = q % 2 == 0 ? e->prefix : e->prefix2;
          s.prefix_out = q % 2 == 0 ? e->prefix2 : e->prefix;
        } else {
          s.prefix = e->prefix;
          s.prefix_out = nullptr;
        }
      }
      err = (wt == SK_BF16) ? launch_sample_step<WBF16>(s, q, c.n_utts, e->stream, slices)
                            : launch_sample_step<WF32>(s, q, c.n_utts, e->stream, slices);
      if (err != hipSuccess) return err;
      continue;
    }
    // The depth input is formed in the gate/up GEMV's prologue, which loads
    // the gathered table row of code q-1 behind its own weight stream.
    GemvArgs a = gemv_args(e->d_gate, c.depth_inner, d, e->hidden, d, e->act, e->inner_max);
    a.w[1] = e->d_up; a.ldx2 = d;
    a.norm_w = e->d_norm_in; a.eps = c.depth_eps; a.norm_out = e->abuf; a.ldno = d;
    if (q == 0) {
      a.x2 = e->prefix;
      if ((err = launch_gemv<PRO_ADDNORM, EPI_SWIGLU>(wt, M, a, e->stream)) != hipSuccess) return err;
    } else if (fuse) {
      a.x2 = (q % 2 == 1) ? e->prefix : e->prefix2;
      a.gout = (q % 2 == 1) ? e->prefix2 : e->prefix; a.ldgo = d;
      err = (wt == SK_BF16) ? launch_depth_fused<WBF16>(s, a, M, q, e->stream)
                            : launch_depth_fused<WF32>(s, a, M, q, e->stream);
      if (err != hipSuccess) return err;
    } else {
      a.x2 = (q % 2 == 1) ? e->prefix : e->prefix2;
      a.gout = (q % 2 == 1) ? e->prefix2 : e->prefix; a.ldgo = d;
      a.gcode = e->codes_cur + (q - 1); a.g_rpu = c.cfg_rows; a.gstride = c.n_codebooks;
      a.gtable = static_cast<const char*>(e->table) + (size_t)(q - 1) * V * d * tsz;
      a.gscale = c.frame_scale;
      if ((err = launch_gemv<PRO_ADDGATHER, EPI_SWIGLU>(wt, M, a, e->stream)) != hipSuccess) return err;
    }

    a = gemv_args(e->d_down, d, c.depth_inner, e->act, e->inner_max, e->ybuf, d);
    a.res = e->abuf; a.ldr = d;
    if ((err = launch_gemv<PRO_NONE, EPI_RESID>(wt, M, a, e->stream)) != hipSuccess) return err;

    const void* tq = static_cast<const char*>(e->out_proj ? e->out_proj : e->table) + (size_t)q * V * d * tsz;
    a = gemv_args(tq, V, d, e->ybuf, d, e->logits, V);
    a.norm_w = e->d_norm_out; a.eps = c.depth_eps; a.bias = e->d_bias + (size_t)q * V;
    if ((err = launch_gemv<PRO_NORM, EPI_BIAS>(wt, M, a, e->stream)) != hipSuccess) return err;

    if (fuse && q + 1 < c.n_codebooks) continue;   // sampled inside the next gate/up launch
    err = (wt == SK_BF16) ? launch_sample_step<WBF16>(s, q, c.n_utts, e->stream)
                          : launch_sample_step<WF32>(s, q, c.n_utts, e->stream);
    if (err != hipSuccess) return err;
  }
  return enqueue_tail(e);
}

// The frame's trunk step and final norm (after its depth steps).
hipError_t enqueue_tail(sk_engine* e) {
  const sk_config& c = e->c;
  const int d = c.d_model, M = e->rows;
  hipError_t err;
  if ((err = enqueue_trunk(e)) != hipSuccess) return err;
  if (e->code_tables) {   // final norm, bookkeeping and the next frame's G_1 in one launch
    DepthArgs g = depth_args(e);
    g.g_out = e->gbuf[0];
    g.xfix = e->lx ? reinterpret_cast<const long long*>(lx_acc(e, 2 * c.n_layers)) : nullptr;
    g.xf32 = e->x;
    g.fix_clear = e->lx ? lx_acc(e, 1) : nullptr;
    g.fnorm_w = e->final_norm; g.fnorm_eps = c.trunk_eps; g.hidden_out = e->hidden;
    g.kv_len = e->kv_len; g.pos = e->pos; g.active = e->active; g.counter = e->fc;
    g.u_ring = e->u_ring; g.flag_ring = e->flag_ring; g.u_cur = e->u_cur; g.flag_cur = e->flag_cur;
    g.nq = c.n_utts * c.n_codebooks; g.max_frames = c.max_frames;
    g.inv_freq = e->inv_freq; g.half = c.head_dim / 2; g.rope = e->rope;
    g.rope_tab = (const float2*)e->p_rope; g.tab_n = c.max_ctx + 1;
    SampleArgs s{};
    return e->lx ? launch_depth_step<4>(c.weight_dtype, d, s, g, 0, e->stream)    // fixed-point trunk output
                 : launch_depth_step<5>(c.weight_dtype, d, s, g, 0, e->stream);   // FP32 trunk output
  }
  hipLaunchKernelGGL(final_norm_kernel, dim3(M), dim3(NT), 0, e->stream, e->x,
                     e->lx ? reinterpret_cast<const long long*>(lx_acc(e, 2 * c.n_layers)) : nullptr,
                     e->lx ? lx_acc(e, 1) : nullptr, e->final_norm,
                     c.trunk_eps, d, e->hidden, e->kv_len, e->pos, e->active, e->fc, e->u_ring,
                     e->flag_ring, e->u_cur, e->flag_cur, c.n_utts * c.n_codebooks, c.max_frames,
                     e->inv_freq, c.head_dim / 2, e->rope, (const float2*)e->p_rope, c.max_ctx + 1,
                     e->d_norm_in, c.depth_eps, e->wide ? e->abuf : nullptr, e->xs_abuf);
  return hipGetLastError();
}

// Code tables of the depth steps (depth_step_kernel): P_j = (table[j] * norm_in
// gain) W_gu^T for j < Q-1, [V][gate | up] per codebook, on the FP32 matrix
// cores (BF16 weights widened exactly); derived from the weights bound when the
// frame is captured.
template <typename TL>
hipError_t build_code_tables_t(sk_engine* e, float* tmp) {
  const sk_config& c = e->c;
  const int d = c.d_model, KI = c.depth_inner, V = c.audio_vocab;
  const size_t tsz = sizeof(typename TL::elem);
  for (int j = 0; j + 1 < c.n_codebooks; ++j) {
    const void* tj = static_cast<const char*>(e->table) + (size_t)j * V * d * tsz;
    hipLaunchKernelGGL(scale_rows_kernel<TL>, dim3(1024), dim3(256), 0, e->stream, tj, e->d_norm_in, V, d, tmp);
    GemmArgs g{};
    g.A = tmp; g.lda = d;
    g.B[0] = e->d_gate; g.B[1] = e->d_up; g.B[2] = nullptr;
    g.seg_rows[0] = KI; g.seg_rows[1] = KI; g.seg_rows[2] = 0;
    g.out = e->ptab + (size_t)j * V * 2 * KI; g.ldo = 2 * KI;
    g.M = V; g.N = 2 * KI; g.K = d;
    hipLaunchKernelGGL((gemm_nt_kernel<GEPI_STORE, TL, 64>), dim3((2 * KI + GBN - 1) / GBN, (V + 63) / 64), dim3(256),
                       0, e->stream, g);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}
int build_code_tables(sk_engine* e) {
  const sk_config& c = e->c;
  const size_t KI = c.depth_inner, V = c.audio_vocab, d = c.d_model;
  if (!e->ptab) {
    SK_HIP(dalloc(&e->ptab, (size_t)(c.n_codebooks - 1) * V * 2 * KI));
    SK_HIP(dalloc(&e->gbuf[0], (size_t)e->rows * 2 * KI));
    SK_HIP(dalloc(&e->gbuf[1], (size_t)e->rows * 2 * KI));
  }
  float* tmp = nullptr;
  SK_HIP(dalloc(&tmp, V * d));
  const hipError_t err = c.weight_dtype == SK_BF16 ? build_code_tables_t<WBF16>(e, tmp)
                                                   : build_code_tables_t<WF32>(e, tmp);
  const hipError_t serr = hipStreamSynchronize(e->stream);
  hipFree(tmp);
  SK_HIP(err);
  SK_HIP(serr);
  return SK_OK;
}

// ---- batched prefill -------------------------------------------------------

// 64-row tiles unless they leave more than half the CUs idle, then 32-row tiles.
template <int EPI>
hipError_t launch_gemm(int wdtype, const GemmArgs& g, hipStream_t st) {
  const int nt = (g.N + GBN - 1) / GBN;
  const bool small = nt * ((g.M + 63) / 64) < 128;
  const dim3 grid(nt, small ? (g.M + 31) / 32 : (g.M + 63) / 64);
  if (wdtype == SK_BF16) {
    if (small) hipLaunchKernelGGL((gemm_bf16_kernel<EPI, 32>), grid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL((gemm_bf16_kernel<EPI, 64>), grid, dim3(256), 0, st, g);
  } else {   // FP32 weights stay on the FP32 matrix cores: exact FP32 products
    if (small) hipLaunchKernelGGL((gemm_nt_kernel<EPI, WF32, 32>), grid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL((gemm_nt_kernel<EPI, WF32, 64>), grid, dim3(256), 0, st, g);
  }
  return hipGetLastError();
}

GemmArgs gemm_args(const float* A, int lda, const void* B, int M, int N, int K, float* out, int ldo) {
  GemmArgs g{};
  g.A = A; g.lda = lda;
  g.B[0] = B; g.B[1] = nullptr; g.B[2] = nullptr;
  g.seg_rows[0] = N; g.seg_rows[1] = 0; g.seg_rows[2] = 0;
  g.out = out; g.ldo = ldo;
  g.M = M; g.N = N; g.K = K;
  return g;
}

hipError_t ensure_prefill_bufs(sk_engine* e, int M) {
  if (M <= e->pf_cap) return hipSuccess;
  if (e->pf_mem) hipFree(e->pf_mem);
  e->pf_mem = nullptr;
  e->pf = PrefillBufs{};
  e->pf_cap = 0;
  const hipError_t err = hipMalloc(&e->pf_mem, prefill_bytes(e->c, e->nqkv, M));
  if (err != hipSuccess) return err;
  e->pf = carve_prefill(e->c, e->nqkv, M, e->pf_mem);
  e->pf_cap = M;
  return hipSuccess;
}

// All staged prefix tokens through the trunk at once (M = total tokens).
hipError_t enqueue_batched_prefill(sk_engine* e, int M, int max_len, const PrefillBufs& b) {
  const sk_config& c = e->c;
  const int d = c.d_model, hd = c.head_dim, wt = c.weight_dtype;
  const int hq = c.n_q_heads * hd, I = c.trunk_inter;
  const bool bf = c.kv_dtype == SK_BF16;
  hipStream_t st = e->stream;
  hipError_t err;
  hipLaunchKernelGGL(pf_gather_kernel, dim3(M), dim3(NT), 0, st, e->embeds, c.max_ctx, b.tok_row,
                     b.tok_pos, d, b.X);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const size_t asmem = pf_attn_smem_floats(hd) * sizeof(float);
  const int G = c.n_q_heads / c.n_kv_heads, QB = PF_NQ / G;
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& w = e->L[l];
    char* kc = e->kc + (size_t)l * kv_layer_bytes(e);
    char* vc = e->vc + (size_t)l * kv_layer_bytes(e);
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(M), dim3(NT), 0, st, b.X, (const float*)nullptr, w.in_norm,
                       c.trunk_eps, d, b.Xn, (const int*)nullptr);
    GemmArgs g = gemm_args(b.Xn, d, w.q, M, e->nqkv, d, b.QKV, e->nqkv);
    g.B[1] = w.k; g.B[2] = w.v;
    g.seg_rows[0] = hq; g.seg_rows[1] = c.n_kv_heads * hd; g.seg_rows[2] = c.n_kv_heads * hd;
    if ((err = launch_gemm<GEPI_STORE>(wt, g, st)) != hipSuccess) return err;
    if (bf)
      hipLaunchKernelGGL(pf_qkv_kernel<uint16_t>, dim3(M), dim3(NT), 0, st, b.QKV, e->nqkv, b.tok_row,
                         b.tok_pos, w.q_norm, w.k_norm, c.trunk_eps, e->p_rope, c.n_q_heads, c.n_kv_heads, hd,
                         c.max_ctx, b.Q, reinterpret_cast<uint16_t*>(kc), reinterpret_cast<uint16_t*>(vc));
    else
      hipLaunchKernelGGL(pf_qkv_kernel<float>, dim3(M), dim3(NT), 0, st, b.QKV, e->nqkv, b.tok_row,
                         b.tok_pos, w.q_norm, w.k_norm, c.trunk_eps, e->p_rope, c.n_q_heads, c.n_kv_heads, hd,
                         c.max_ctx, b.Q, reinterpret_cast<float*>(kc), reinterpret_cast<float*>(vc));
    const dim3 agrid((max_len + QB - 1) / QB, c.n_kv_heads, e->rows);
    const float scale = 1.0f / sqrtf((float)hd);
    if (bf)
      hipLaunchKernelGGL(pf_attention_kernel<uint16_t>, agrid, dim3(NT), asmem, st, b.Q,
                         reinterpret_cast<const uint16_t*>(kc), reinterpret_cast<const uint16_t*>(vc),
                         e->p_row_start, e->plen, c.n_q_heads, c.n_kv_heads, hd, c.max_ctx, scale, b.ATT, hq);
    else
      hipLaunchKernelGGL(pf_attention_kernel<float>, agrid, dim3(NT), asmem, st, b.Q,
                         reinterpret_cast<const float*>(kc), reinterpret_cast<const float*>(vc), e->p_row_start,
                         e->plen, c.n_q_heads, c.n_kv_heads, hd, c.max_ctx, scale, b.ATT, hq);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    g = gemm_args(b.ATT, hq, w.o, M, d, hq, b.X, d);
    g.res = b.X; g.ldr = d;
    if ((err = launch_gemm<GEPI_RESID>(wt, g, st)) != hipSuccess) return err;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(M), dim3(NT), 0, st, b.X, (const float*)nullptr, w.post_norm,
                       c.trunk_eps, d, b.Xn, (const int*)nullptr);
    g = gemm_args(b.Xn, d, w.gate, M, I, d, b.ACT, I);
    g.B2 = w.up;
    if ((err = launch_gemm<GEPI_SWIGLU>(wt, g, st)) != hipSuccess) return err;
    g = gemm_args(b.ACT, I, w.down, M, d, I, b.X, d);
    g.res = b.X; g.ldr = d;
    if ((err = launch_gemm<GEPI_RESID>(wt, g, st)) != hipSuccess) return err;
  }
  hipLaunchKernelGGL(pf_finish_kernel, dim3(e->rows), dim3(NT), 0, st, b.X, e->p_row_start, e->plen,
                     e->final_norm, c.trunk_eps, d, e->hidden, e->kv_len, e->pos, e->active, e->inv_freq, hd / 2,
                     e->rope, e->d_norm_in, c.depth_eps, e->abuf, e->xs_abuf);
  const hipError_t fe = hipGetLastError();
  if (fe != hipSuccess || !e->code_tables) return fe;
  return launch_g1(e);
}

int capture(sk_engine* e, hipError_t (*body)(sk_engine*), hipGraph_t* g, hipGraphExec_t* x) {
  SK_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  const hipError_t err = body(e);
  hipGraph_t graph = nullptr;
  const hipError_t end = hipStreamEndCapture(e->stream, &graph);
  if (err != hipSuccess) {
    if (graph) hipGraphDestroy(graph);
    return fail(SK_EHIP, "kernel launch during capture failed: %s", hipGetErrorString(err));
  }
  SK_CHECK(end == hipSuccess, SK_EHIP, "hipStreamEndCapture failed: %s", hipGetErrorString(end));
  hipGraphExec_t exec = nullptr;
  const hipError_t ins = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (ins != hipSuccess) {
    hipGraphDestroy(graph);
    return fail(SK_EHIP, "hipGraphInstantiate failed: %s", hipGetErrorString(ins));
  }
  // Upload now, so the first replay of a context bucket's graph (mid-decode)
  // does not pay for it.
  const hipError_t up = hipGraphUpload(exec, e->stream);
  if (up != hipSuccess) {
    hipGraphExecDestroy(exec);
    hipGraphDestroy(graph);
    return fail(SK_EHIP, "hipGraphUpload failed: %s", hipGetErrorString(up));
  }
  *g = graph;
  *x = exec;
  return SK_OK;
}

// Whether workgroups whose ids agree modulo 8 run on one XCD (read from the
// XCC_ID register of 2048 probe workgroups): the split-K merge of the
// many-row GEMMs relies on it.  Single-XCD partitions pass trivially.
hipError_t probe_xcd_mapping(hipStream_t st, bool* ok) {
  *ok = false;
  unsigned* d = nullptr;
  hipError_t err = hipMalloc(reinterpret_cast<void**>(&d), XCD_PROBE_WGS * sizeof(unsigned));
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(xcd_probe_kernel, dim3(XCD_PROBE_WGS), dim3(64), 0, st, d);
  std::vector<unsigned> ids(XCD_PROBE_WGS);
  err = hipGetLastError();
  if (err == hipSuccess) err = hipMemcpyAsync(ids.data(), d, ids.size() * sizeof(unsigned), hipMemcpyDeviceToHost, st);
  if (err == hipSuccess) err = hipStreamSynchronize(st);
  hipFree(d);
  if (err != hipSuccess) return err;
  bool same = true;
  for (int i = 8; i < XCD_PROBE_WGS; ++i) same = same && ids[i] == ids[i % 8];
  *ok = same;
  return hipSuccess;
}

bool parse_layer(const char* key, int* layer, const char** rest) {
  const char* pre = "trunk.layers.";
  const size_t n = strlen(pre);
  if (strncmp(key, pre, n) != 0) return false;
  const char* p = key + n;
  if (*p < '0' || *p > '9') return false;
  int v = 0;
  while (*p >= '0' && *p <= '9') { v = v * 10 + (*p - '0'); ++p; if (v > 100000) return false; }
  if (*p != '.') return false;
  *layer = v;
  *rest = p + 1;
  return true;
}

}  // namespace

extern "C" {

const char* sk_last_error(void) { return last_error().c_str(); }

// ---- frame order between engines on one device ------------------------------
// Frames (and prefills) of different engines on one device run one after
// another.  The
// XCD-resident layers and the tagged split-K merge wait inside a launch for
// other workgroups of the same launch, so all of its workgroups must be
// resident at once; another engine's frame running beside it would hold CUs
// those workgroups need, and both would wait until their spin limits end the
// frames with an error.  When a device's frames pass from one engine to
// another, the new engine's stream first waits for everything the previous
// engine had queued (an event recorded on that engine's stream at the
// switch), so an engine that steps alone pays nothing.  The lock is held
// while frames or a prefill are enqueued and while a graph is captured, so
// no event is ever recorded on a stream that is capturing.
namespace {
struct FrameOrder {
  std::mutex mu;
  sk_engine* last = nullptr;   // the engine whose frames were enqueued last on this device
};
FrameOrder g_frame_order[MAX_DEVICES];
}  // namespace

// With g_frame_order[e->device].mu held, before e enqueues frames.
static hipError_t order_after_previous(sk_engine* e) {
  FrameOrder& fo = g_frame_order[e->device];
  sk_engine* p = fo.last;
  fo.last = e;
  if (!p || p == e) return hipSuccess;
  hipError_t err = hipEventRecord(p->order_ev, p->stream);
  if (err == hipSuccess) err = hipStreamWaitEvent(e->stream, p->order_ev, 0);
  return err;
}

static void leave_frame_order(sk_engine* e) {
  if (!e->stream) return;   // never got as far as launching anything
  FrameOrder& fo = g_frame_order[e->device];
  std::lock_guard<std::mutex> lk(fo.mu);
  if (fo.last == e) fo.last = nullptr;
}

int sk_create(const sk_config* cfg, void* hip_stream, sk_engine** out) {
  SK_CHECK(out != nullptr, SK_EINVAL, "out is NULL");
  *out = nullptr;
  int rc = validate_config(cfg);
  if (rc != SK_OK) return rc;
  sk_engine* e = new sk_engine();
  e->c = *cfg;
  const sk_config& c = e->c;
  e->rows = c.n_utts * c.cfg_rows;
  e->wide = e->rows > 4;
  e->G = c.n_q_heads / c.n_kv_heads;
  e->nqkv = (c.n_q_heads + 2 * c.n_kv_heads) * c.head_dim;
  e->inner_max = c.trunk_inter > c.depth_inner ? c.trunk_inter : c.depth_inner;
  e->max_chunks = (c.max_ctx + ATT_CHUNK - 1) / ATT_CHUNK;
  // Many rows: streaming attention with enough splits per (row, kv head) for
  // ~256 workgroups (one per CU); its partials reuse the chunk-partial buffer.
  if (e->wide && (e->G == 1 || e->G == 2 || e->G == 4) && e->G * c.head_dim <= ATTN_STREAM_NTH) {
    const int pairs = e->rows * c.n_kv_heads;
    e->attn_splits = std::max(1, std::min(e->max_chunks, (256 + pairs - 1) / pairs));
  }
  e->L.resize(c.n_layers);
  e->kv_host.assign(e->rows, 0);
  e->active_host.assign(e->rows, 0);
  e->len_host.assign(e->rows, 0);
  e->staged.assign(e->rows, 0);
  auto bail = [&](int code) { sk_destroy(e); return code; };
#define ALLOC(ptr, n)                                                                   \
  do {                                                                                  \
    const hipError_t _a = dalloc(&(ptr), (n));                                          \
    if (_a != hipSuccess) {                                                             \
      fail(SK_EHIP, "hipMalloc(%s) failed: %s", #ptr, hipGetErrorString(_a));           \
      return bail(SK_EHIP);                                                             \
    }                                                                                   \
  } while (0)
  if (hipGetDevice(&e->device) != hipSuccess) { fail(SK_EHIP, "no HIP device"); return bail(SK_EHIP); }
  {
    void* sp = nullptr;   // this device's copy of the no-alloc prefill scratch, looked up once
    const hipError_t se = scratch_ptr(e->device, &sp);
    if (se != hipSuccess) { fail(SK_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(se)); return bail(SK_EHIP); }
  }
  if (hip_stream) {
    const hipError_t se = hipStreamSynchronize(static_cast<hipStream_t>(hip_stream));
    if (se != hipSuccess) { fail(SK_EHIP, "caller stream: %s", hipGetErrorString(se)); return bail(SK_EHIP); }
  }
  if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
    fail(SK_EHIP, "hipStreamCreateWithFlags failed");
    return bail(SK_EHIP);
  }
  if (hipEventCreateWithFlags(&e->order_ev, hipEventDisableTiming) != hipSuccess) {
    fail(SK_EHIP, "hipEventCreateWithFlags failed");
    return bail(SK_EHIP);
  }
  const size_t R = e->rows, d = c.d_model, Q = c.n_codebooks, V = c.audio_vocab;
  ALLOC(e->x, R * d); ALLOC(e->hidden, R * d); ALLOC(e->prefix, R * d); ALLOC(e->prefix2, R * d);
  ALLOC(e->abuf, R * d); ALLOC(e->ybuf, R * d);
  ALLOC(e->qkv, R * e->nqkv); ALLOC(e->attn, R * c.n_q_heads * c.head_dim);
  ALLOC(e->act, R * e->inner_max); ALLOC(e->logits, R * V);
  ALLOC(e->kc, (size_t)c.n_layers * kv_layer_bytes(e));
  ALLOC(e->vc, (size_t)c.n_layers * kv_layer_bytes(e));
  ALLOC(e->inv_freq, (size_t)c.head_dim / 2);
  ALLOC(e->rope, R * (size_t)c.head_dim / 2);
  {
    const size_t nmax = std::max({(size_t)e->nqkv, (size_t)c.trunk_inter, (size_t)c.depth_inner,
                                  (size_t)c.audio_vocab, (size_t)c.d_model});
    ALLOC(e->sk_partial, (nmax / 16 + 1) * 4 * SK_PSZ);
    ALLOC(e->sk_arrive, nmax / 16 + 1);
    ALLOC(e->sk_tpart, (nmax / 16 + 1) * SK_MAX_SPLIT * SK_PSZ);
    e->sk_tpart_bytes = (nmax / 16 + 1) * SK_MAX_SPLIT * SK_PSZ * sizeof(unsigned long long);
    ALLOC(e->sk_err, 1);
  }
  ALLOC(e->part, R * c.n_q_heads * e->max_chunks * part_stride(c.head_dim));
  const bool split_in = e->wide && c.weight_dtype == SK_BF16;
  if (split_in) {
    ALLOC(e->xs_x, xsplit_elems(d)); ALLOC(e->xs_attn, xsplit_elems(c.n_q_heads * c.head_dim));
    ALLOC(e->xs_act, xsplit_elems(e->inner_max)); ALLOC(e->xs_abuf, xsplit_elems(d)); ALLOC(e->xs_y, xsplit_elems(d));
    ALLOC(e->ss_x, (size_t)XS_ROWS * d / 16); ALLOC(e->ss_y, (size_t)XS_ROWS * d / 16);
  }
  ALLOC(e->kv_len, R); ALLOC(e->pos, R); ALLOC(e->active, R); ALLOC(e->plen, R);
  ALLOC(e->fc, 1);
  ALLOC(e->p_rope, (size_t)(c.max_ctx + 1) * (c.head_dim / 2));
  ALLOC(e->p_row_start, R);
  ALLOC(e->u_ring, (size_t)c.max_frames * c.n_utts * Q);
  ALLOC(e->flag_ring, (size_t)c.max_frames * 2);
  ALLOC(e->u_cur, (size_t)c.n_utts * Q);
  ALLOC(e->flag_cur, 2);
  ALLOC(e->codes_cur, (size_t)c.n_utts * Q);
  ALLOC(e->forced_ring, (size_t)c.max_frames * c.n_utts * Q);
  ALLOC(e->codes_ring, (size_t)c.max_frames * c.n_utts * Q);
  ALLOC(e->dbg, (size_t)c.n_utts * Q * V);
  ALLOC(e->embeds, R * c.max_ctx * d);
  ALLOC(e->stage_ids, (size_t)c.max_ctx);
  ALLOC(e->stage_codes, (size_t)c.max_ctx * Q);
  ALLOC(e->params, 1);
#undef ALLOC
  const std::vector<float> inv = rope_inv_freq(c);
  hipError_t he = hipMemcpy(e->inv_freq, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice);
  if (he == hipSuccess) he = hipMemset(e->u_cur, 0, (size_t)c.n_utts * Q * sizeof(double));
  if (he == hipSuccess) he = hipMemset(e->flag_cur, 0, 2 * sizeof(int));
  if (he == hipSuccess) he = hipMemset(e->x, 0, R * d * sizeof(float));
  if (he == hipSuccess) he = hipMemset(e->prefix, 0, R * d * sizeof(float));
  if (he == hipSuccess) he = hipMemset(e->prefix2, 0, R * d * sizeof(float));
  if (he == hipSuccess) he = hipMemset(e->kv_len, 0, R * sizeof(int));
  if (he == hipSuccess) he = hipMemset(e->sk_err, 0, sizeof(unsigned));
  if (he == hipSuccess) he = hipMemset(e->sk_tpart, 0, e->sk_tpart_bytes);   // tag 0 is never a launch's
  if (he == hipSuccess)
    he = hipMemset(e->sk_arrive, 0,
                   (std::max({(size_t)e->nqkv, (size_t)c.trunk_inter, (size_t)c.depth_inner, (size_t)c.audio_vocab,
                              (size_t)c.d_model}) / 16 + 1) * sizeof(unsigned));
  if (he == hipSuccess) he = hipMemset(e->pos, 0, R * sizeof(int));
  if (split_in) {   // rows past R are never written; keep them finite
    uint16_t* xs[] = {e->xs_x, e->xs_attn, e->xs_act, e->xs_abuf, e->xs_y};
    const size_t xk[] = {d, (size_t)c.n_q_heads * c.head_dim, (size_t)e->inner_max, d, d};
    for (int i = 0; i < 5 && he == hipSuccess; ++i) he = hipMemset(xs[i], 0, xsplit_elems((int)xk[i]) * sizeof(uint16_t));
    if (he == hipSuccess) he = hipMemset(e->ss_x, 0, (size_t)XS_ROWS * d / 16 * sizeof(float));
    if (he == hipSuccess) he = hipMemset(e->ss_y, 0, (size_t)XS_ROWS * d / 16 * sizeof(float));
  }
  if (he == hipSuccess) he = hipMemset(e->fc, 0, sizeof(int));
  if (he == hipSuccess) he = hipMemset(e->flag_ring, 0, (size_t)c.max_frames * 2 * sizeof(int));
  if (he == hipSuccess) he = hipMemset(e->u_ring, 0, (size_t)c.max_frames * c.n_utts * Q * sizeof(double));
  e->p_host.cfg_scale = 1.0f;
  e->p_host.temperature = 0.0f;
  if (he == hipSuccess) he = hipMemcpy(e->params, &e->p_host, sizeof(SkParams), hipMemcpyHostToDevice);
  if (he == hipSuccess) {
    hipLaunchKernelGGL(pf_rope_table_kernel, dim3(c.max_ctx + 1), dim3(NT), 0, e->stream, e->inv_freq,
                       c.head_dim / 2, e->p_rope);
    he = hipGetLastError();
    if (he == hipSuccess) he = hipStreamSynchronize(e->stream);
  }
  if (he == hipSuccess) he = prepare_sampler();
  if (he == hipSuccess && e->wide && c.weight_dtype == SK_BF16) he = probe_xcd_mapping(e->stream, &e->split_k);
  // XCD-resident layers: the shape fits, the device has 8 x 32 CUs, workgroups
  // whose ids agree mod 8 share an XCD, and SORAKU_XCD_LAYERS is not "0"
  if (he == hipSuccess && lx_fits(e)) {
    const char* env = getenv("SORAKU_XCD_LAYERS");
    int cus = 0;
    he = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e->device);
    bool mapped = false;
    if (he == hipSuccess && cus == LX_WGS && !(env && strcmp(env, "0") == 0)) he = probe_xcd_mapping(e->stream, &mapped);
    e->lx = he == hipSuccess && mapped;
  }
  if (he == hipSuccess && e->lx) {
    he = dalloc(&e->lx_acc, 3 * (size_t)R * d);
    if (he == hipSuccess) he = dalloc(&e->lx_flags, (size_t)LX_XCDS * LX_FLAGS);
    if (he == hipSuccess) he = dalloc(&e->lx_err, 1);
    const size_t nqkv = (size_t)R * (c.n_q_heads + 2 * c.n_kv_heads) * c.head_dim, nact = (size_t)R * c.trunk_inter;
    if (he == hipSuccess) he = dalloc(&e->lx_qkv, nqkv);
    if (he == hipSuccess) he = dalloc(&e->lx_act, nact);
    if (he == hipSuccess) he = hipMemset(e->lx_qkv, 0, nqkv * sizeof(uint2));
    if (he == hipSuccess) he = hipMemset(e->lx_act, 0, nact * sizeof(uint2));
    // all zero at creation: the first frame's first launch adds into
    // accumulator 1 (and a frame whose layer launches left early, after a
    // barrier timeout, still reads finite values)
    if (he == hipSuccess) he = hipMemset(e->lx_acc, 0, 3 * (size_t)R * d * sizeof(unsigned long long));
    if (he == hipSuccess) he = hipMemset(e->lx_flags, 0, (size_t)LX_XCDS * LX_FLAGS * sizeof(unsigned));
    if (he == hipSuccess) he = hipMemset(e->lx_err, 0, sizeof(unsigned));
  }
  if (he == hipSuccess)
    he = hipFuncSetAttribute(c.kv_dtype == SK_BF16 ? reinterpret_cast<const void*>(attention_kernel<uint16_t>)
                                                   : reinterpret_cast<const void*>(attention_kernel<float>),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)(attn_smem_floats(e->G, c.head_dim) * sizeof(float)));
  if (he != hipSuccess) { fail(SK_EHIP, "engine init: %s", hipGetErrorString(he)); return bail(SK_EHIP); }
  *out = e;
  return SK_OK;
}

int sk_destroy(sk_engine* e) {
  if (!e) return SK_OK;
  leave_frame_order(e);
  if (e->stream) hipStreamSynchronize(e->stream);
  drop_graphs(e);
  void* bufs[] = {e->sk_partial, e->sk_arrive, e->sk_tpart, e->sk_err, e->xs_x, e->xs_attn, e->xs_act, e->xs_abuf, e->xs_y, e->ss_x, e->ss_y, e->x, e->hidden, e->prefix, e->prefix2, e->abuf, e->ybuf, e->qkv, e->attn, e->act, e->logits,
                  e->kc, e->vc, e->inv_freq, e->rope, e->part, e->dbg, e->embeds, e->u_cur, e->flag_cur, e->codes_cur,
                  e->kv_len, e->pos, e->active, e->plen, e->fc, e->flag_ring, e->u_ring,
                  e->pf_mem, e->ptab, e->gbuf[0], e->gbuf[1],
                  e->lx_acc, e->lx_qkv, e->lx_act,
                  e->lx_flags, e->lx_err,
                  e->p_row_start, e->p_rope,
                  e->forced_ring, e->codes_ring, e->stage_ids, e->stage_codes, e->params};
  for (void* p : bufs)
    if (p) hipFree(p);
  if (e->order_ev) hipEventDestroy(e->order_ev);
  if (e->stream) hipStreamDestroy(e->stream);
  delete e;
  return SK_OK;
}

int sk_bind_weight(sk_engine* e, const char* key, const void* dev_ptr, int32_t dtype,
                   const int64_t* shape, int32_t ndim) {
  SK_CHECK(e && key && shape, SK_EINVAL, "engine, key and shape must be non-NULL");
  SK_CHECK(dev_ptr != nullptr, SK_EINVAL, "%s: device pointer is NULL", key);
  SK_CHECK(((uintptr_t)dev_ptr & 15) == 0, SK_EINVAL, "%s: device pointer must be 16-byte aligned", key);
  const sk_config& c = e->c;
  const int64_t d = c.d_model, hd = c.head_dim, wt = c.weight_dtype;
  auto want = [&](std::initializer_list<int64_t> dims, int32_t dt) -> int {
    SK_CHECK(dtype == dt, SK_EINVAL, "%s: dtype %d, expected %d", key, dtype, dt);
    SK_CHECK(ndim == (int32_t)dims.size(), SK_EINVAL, "%s: ndim %d, expected %d", key, ndim, (int)dims.size());
    int i = 0;
    for (int64_t v : dims) {
      SK_CHECK(shape[i] == v, SK_EINVAL, "%s: dim %d is %lld, expected %lld", key, i,
               (long long)shape[i], (long long)v);
      ++i;
    }
    return SK_OK;
  };
  int rc = SK_OK;
  int layer = -1;
  const char* rest = nullptr;
  if (parse_layer(key, &layer, &rest)) {
    SK_CHECK(layer < c.n_layers, SK_EINVAL, "%s: layer index out of range", key);
    LayerW& w = e->L[layer];
    const std::string r(rest);
    if (r == "input_layernorm.weight") { if (!(rc = want({d}, SK_F32))) w.in_norm = (const float*)dev_ptr; }
    else if (r == "post_attention_layernorm.weight") { if (!(rc = want({d}, SK_F32))) w.post_norm = (const float*)dev_ptr; }
    else if (r == "self_attn.q_norm.weight") { if (!(rc = want({hd}, SK_F32))) w.q_norm = (const float*)dev_ptr; }
    else if (r == "self_attn.k_norm.weight") { if (!(rc = want({hd}, SK_F32))) w.k_norm = (const float*)dev_ptr; }
    else if (r == "self_attn.q_proj.weight") { if (!(rc = want({c.n_q_heads * hd, d}, wt))) w.q = dev_ptr; }
    else if (r == "self_attn.k_proj.weight") { if (!(rc = want({c.n_kv_heads * hd, d}, wt))) w.k = dev_ptr; }
    else if (r == "self_attn.v_proj.weight") { if (!(rc = want({c.n_kv_heads * hd, d}, wt))) w.v = dev_ptr; }
    else if (r == "self_attn.o_proj.weight") { if (!(rc = want({d, c.n_q_heads * hd}, wt))) w.o = dev_ptr; }
    else if (r == "mlp.gate_proj.weight") { if (!(rc = want({c.trunk_inter, d}, wt))) w.gate = dev_ptr; }
    else if (r == "mlp.up_proj.weight") { if (!(rc = want({c.trunk_inter, d}, wt))) w.up = dev_ptr; }
    else if (r == "mlp.down_proj.weight") { if (!(rc = want({d, c.trunk_inter}, wt))) w.down = dev_ptr; }
    else return fail(SK_EINVAL, "unknown weight key %s", key);
  } else {
    const std::string k(key);
    if (k == "trunk.norm.weight") { if (!(rc = want({d}, SK_F32))) e->final_norm = (const float*)dev_ptr; }
    else if (k == "trunk.embed_tokens.weight") { if (!(rc = want({c.text_vocab, d}, wt))) e->embed_tokens = dev_ptr; }
    else if (k == "audio_codebooks.table") { if (!(rc = want({c.n_codebooks, c.audio_vocab, d}, wt))) e->table = dev_ptr; }
    else if (k == "depth_head.out_proj") { if (!(rc = want({c.n_codebooks, c.audio_vocab, d}, wt))) e->out_proj = dev_ptr; }
    else if (k == "depth_head.norm_in.weight") { if (!(rc = want({d}, SK_F32))) e->d_norm_in = (const float*)dev_ptr; }
    else if (k == "depth_head.norm_out.weight") { if (!(rc = want({d}, SK_F32))) e->d_norm_out = (const float*)dev_ptr; }
    else if (k == "depth_head.mlp.gate_proj.weight") { if (!(rc = want({c.depth_inner, d}, wt))) e->d_gate = dev_ptr; }
    else if (k == "depth_head.mlp.up_proj.weight") { if (!(rc = want({c.depth_inner, d}, wt))) e->d_up = dev_ptr; }
    else if (k == "depth_head.mlp.down_proj.weight") { if (!(rc = want({d, c.depth_inner}, wt))) e->d_down = dev_ptr; }
    else if (k == "depth_head.bias") { if (!(rc = want({c.n_codebooks, c.audio_vocab}, SK_F32))) e->d_bias = (const float*)dev_ptr; }
    else if (k == "language_embeddings.weight") {
      SK_CHECK(c.n_language == 4, SK_EINVAL, "language_embeddings.weight bound but n_language is 0");
      if (!(rc = want({4, d}, SK_F32))) e->lang = (const float*)dev_ptr;
    } else return fail(SK_EINVAL, "unknown weight key %s", key);
  }
  if (rc == SK_OK) drop_graphs(e);  // captured graphs hold the old addresses
  return rc;
}

int sk_prefill_row(sk_engine* e, int32_t row, const int64_t* text_ids, int32_t n_text,
                   const int64_t* frame_codes, int32_t n_frames) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  const sk_config& c = e->c;
  SK_CHECK(row >= 0 && row < e->rows, SK_EINVAL, "row %d out of range [0, %d)", row, e->rows);
  SK_CHECK(n_text >= 0 && n_frames >= 0 && n_text + n_frames >= 1, SK_EINVAL, "empty prefix");
  SK_CHECK(n_text == 0 || text_ids, SK_EINVAL, "text_ids is NULL");
  SK_CHECK(n_frames == 0 || frame_codes, SK_EINVAL, "frame_codes is NULL");
  SK_CHECK(n_text + n_frames < c.max_ctx, SK_EKVFULL, "prefix of %d tokens does not fit max_ctx=%d",
           n_text + n_frames, c.max_ctx);
  for (int i = 0; i < n_text; ++i)
    SK_CHECK(text_ids[i] >= 0 && text_ids[i] < c.text_vocab, SK_EINVAL, "text id %lld out of range",
             (long long)text_ids[i]);
  for (int i = 0; i < n_frames * c.n_codebooks; ++i)
    SK_CHECK(frame_codes[i] >= 0 && frame_codes[i] < c.audio_vocab, SK_EINVAL, "frame code %lld out of range",
             (long long)frame_codes[i]);
  SK_CHECK(n_text == 0 || e->embed_tokens, SK_ENOWEIGHT, "trunk.embed_tokens.weight is not bound");
  SK_CHECK(n_frames == 0 || e->table, SK_ENOWEIGHT, "audio_codebooks.table is not bound");
  SK_CHECK(c.n_language == 0 || n_text == 0 || e->lang, SK_ENOWEIGHT, "language_embeddings.weight is not bound");
  if (n_text) SK_HIP(hipMemcpyAsync(e->stage_ids, text_ids, n_text * sizeof(int64_t), hipMemcpyHostToDevice, e->stream));
  if (n_frames)
    SK_HIP(hipMemcpyAsync(e->stage_codes, frame_codes, (size_t)n_frames * c.n_codebooks * sizeof(int64_t),
                          hipMemcpyHostToDevice, e->stream));
  float* dst = e->embeds + (size_t)row * c.max_ctx * c.d_model;
  const int n = n_text + n_frames;
  if (c.weight_dtype == SK_BF16)
    hipLaunchKernelGGL(embed_prefix_kernel<WBF16>, dim3(n), dim3(NT), 0, e->stream, e->stage_ids, n_text,
                       e->stage_codes, e->embed_tokens, e->lang, c.n_language, c.language_ids[0],
                       c.language_ids[1], c.language_ids[2], c.language_ids[3], e->table, c.n_codebooks,
                       c.audio_vocab, c.d_model, c.frame_scale, dst);
  else
    hipLaunchKernelGGL(embed_prefix_kernel<WF32>, dim3(n), dim3(NT), 0, e->stream, e->stage_ids, n_text,
                       e->stage_codes, e->embed_tokens, e->lang, c.n_language, c.language_ids[0],
                       c.language_ids[1], c.language_ids[2], c.language_ids[3], e->table, c.n_codebooks,
                       c.audio_vocab, c.d_model, c.frame_scale, dst);
  SK_HIP(hipGetLastError());
  SK_HIP(hipStreamSynchronize(e->stream));
  e->len_host[row] = n;
  e->staged[row] = 1;
  e->prefilled = false;
  return SK_OK;
}

// Prefill the staged rows.  all: every row must be staged and the frame
// counter and codebook prefixes start over; otherwise (refill) only the staged
// rows are touched -- the other rows' caches, lengths and hidden states and
// the frame counter stay as they are (unstaged rows get length 0 here, which
// every prefill kernel skips).
// The split-K merge's tagged words carry frame counter * 256 + launch + 1.
// Where the frame counter restarts at 0, a word an earlier run's frame left
// could carry the tag a launch of the new run waits for (slice 0 would then
// take a stale partial): the words are cleared there, since tag 0 is never a
// launch's.
static hipError_t clear_split_tags(sk_engine* e) {
  return e->wide ? hipMemsetAsync(e->sk_tpart, 0, e->sk_tpart_bytes, e->stream) : hipSuccess;
}

static int prefill_staged(sk_engine* e, bool all, bool noalloc) {
  const int R = e->rows;
  int n_staged = 0;
  for (int r = 0; r < R; ++r) {
    if (all) SK_CHECK(e->staged[r], SK_ESTATE, "row %d has no staged prefix", r);
    n_staged += e->staged[r] ? 1 : 0;
  }
  SK_CHECK(n_staged > 0, SK_ESTATE, "no row has a staged prefix");
  int rc = check_decode_weights(e);
  if (rc != SK_OK) return rc;
  // Pack the staged rows' prefix tokens row after row.
  std::vector<int> row_start(R), row_len(R), tok_row, tok_pos;
  int M = 0, max_len = 0;
  for (int r = 0; r < R; ++r) {
    row_start[r] = M;
    row_len[r] = e->staged[r] ? e->len_host[r] : 0;
    for (int p = 0; p < row_len[r]; ++p) { tok_row.push_back(r); tok_pos.push_back(p); }
    M += row_len[r];
    max_len = row_len[r] > max_len ? row_len[r] : max_len;
  }
  PrefillBufs bufs;
  if (noalloc) {
    const size_t need = prefill_bytes(e->c, e->nqkv, M);
    SK_CHECK(need <= SK_NOALLOC_SCRATCH_BYTES, SK_EINVAL,
             "prefill of %d packed tokens needs %zu bytes of scratch, more than the %zu of "
             "sk_prefill_run_noalloc (use sk_prefill_run)", M, need, (size_t)SK_NOALLOC_SCRATCH_BYTES);
    void* base = nullptr;
    SK_HIP(scratch_ptr(e->device, &base));
    bufs = carve_prefill(e->c, e->nqkv, M, base);
  } else {
    const hipError_t ae = ensure_prefill_bufs(e, M);
    SK_CHECK(ae == hipSuccess, SK_EHIP, "prefill buffers for %d tokens: %s", M, hipGetErrorString(ae));
    bufs = e->pf;
  }
  {
    // in the device's order of engines, like frames: no other engine's frame
    // runs beside the prefill, and prefills of different engines (which share
    // the no-alloc scratch) take turns
    std::lock_guard<std::mutex> lk(g_frame_order[e->device].mu);
    SK_HIP(order_after_previous(e));
    SK_HIP(hipMemcpyAsync(e->plen, row_len.data(), R * sizeof(int), hipMemcpyHostToDevice, e->stream));
    SK_HIP(hipMemcpyAsync(e->p_row_start, row_start.data(), R * sizeof(int), hipMemcpyHostToDevice, e->stream));
    SK_HIP(hipMemcpyAsync(bufs.tok_row, tok_row.data(), M * sizeof(int), hipMemcpyHostToDevice, e->stream));
    SK_HIP(hipMemcpyAsync(bufs.tok_pos, tok_pos.data(), M * sizeof(int), hipMemcpyHostToDevice, e->stream));
    if (all) {
      SK_HIP(hipMemsetAsync(e->fc, 0, sizeof(int), e->stream));
      SK_HIP(clear_split_tags(e));
      SK_HIP(hipMemsetAsync(e->prefix, 0, (size_t)R * e->c.d_model * sizeof(float), e->stream));
      SK_HIP(hipMemsetAsync(e->prefix2, 0, (size_t)R * e->c.d_model * sizeof(float), e->stream));
    }
    SK_HIP(enqueue_batched_prefill(e, M, max_len, bufs));
  }
  SK_HIP(hipStreamSynchronize(e->stream));
  for (int r = 0; r < R; ++r)
    if (e->staged[r]) { e->kv_host[r] = e->len_host[r]; e->active_host[r] = 1; e->staged[r] = 0; }
  if (all) { e->fc_host = 0; e->ran_full = true; }
  e->prefilled = true;
  return SK_OK;
}

int sk_prefill_run(sk_engine* e) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  return prefill_staged(e, true, false);
}

int sk_prefill_run_noalloc(sk_engine* e) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  // The prefill copies host-side tables and waits for its stream: it cannot
  // be recorded into a graph.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  SK_HIP(hipStreamIsCapturing(e->stream, &cs));
  SK_CHECK(cs == hipStreamCaptureStatusNone, SK_ESTATE, "sk_prefill_run_noalloc on a capturing stream");
  return prefill_staged(e, true, true);
}

int sk_prefill_refill(sk_engine* e) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_CHECK(e->ran_full, SK_ESTATE, "refill before the first sk_prefill_run");
  return prefill_staged(e, false, false);
}

int sk_retire_row(sk_engine* e, int32_t row) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_CHECK(row >= 0 && row < e->rows, SK_EINVAL, "row %d out of range", row);
  const int zero = 0;
  SK_HIP(hipMemcpyAsync(e->active + row, &zero, sizeof(int), hipMemcpyHostToDevice, e->stream));
  SK_HIP(hipStreamSynchronize(e->stream));
  e->active_host[row] = 0;
  return SK_OK;
}

int sk_reset_frames(sk_engine* e) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_HIP(hipMemsetAsync(e->fc, 0, sizeof(int), e->stream));
  SK_HIP(clear_split_tags(e));
  SK_HIP(hipStreamSynchronize(e->stream));
  e->fc_host = 0;
  return SK_OK;
}

int sk_set_row_state(sk_engine* e, int32_t row, int32_t kv_len, int32_t position) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_CHECK(row >= 0 && row < e->rows, SK_EINVAL, "row %d out of range", row);
  SK_CHECK(kv_len >= 0 && kv_len < e->c.max_ctx, SK_EKVFULL, "kv_len %d outside [0, max_ctx)", kv_len);
  SK_CHECK(position >= 0 && position < e->c.max_ctx, SK_EINVAL, "position %d outside [0, max_ctx)", position);
  // Queued replays advance kv_len / pos on the device: let them finish before
  // the row's state is overwritten, and write it on the engine's stream.
  SK_HIP(hipStreamSynchronize(e->stream));
  const int one = 1;
  SK_HIP(hipMemcpyAsync(e->kv_len + row, &kv_len, sizeof(int), hipMemcpyHostToDevice, e->stream));
  SK_HIP(hipMemcpyAsync(e->pos + row, &position, sizeof(int), hipMemcpyHostToDevice, e->stream));
  SK_HIP(hipMemcpyAsync(e->active + row, &one, sizeof(int), hipMemcpyHostToDevice, e->stream));
  hipLaunchKernelGGL(rope_rows_kernel, dim3(1), dim3(NT), 0, e->stream, e->pos, e->inv_freq,
                     e->c.head_dim / 2, row, e->rope);
  SK_HIP(hipGetLastError());
  SK_HIP(hipStreamSynchronize(e->stream));
  e->kv_host[row] = kv_len;
  e->active_host[row] = 1;
  return SK_OK;
}

int sk_kv_ptr(sk_engine* e, int32_t layer, int32_t kv, void** out) {
  SK_CHECK(e && out, SK_EINVAL, "engine and out must be non-NULL");
  SK_CHECK(layer >= 0 && layer < e->c.n_layers, SK_EINVAL, "layer out of range");
  SK_CHECK(kv == 0 || kv == 1, SK_EINVAL, "kv must be 0 (K) or 1 (V)");
  *out = (kv ? e->vc : e->kc) + (size_t)layer * kv_layer_bytes(e);
  return SK_OK;
}

int sk_get_hidden(sk_engine* e, float* host_out) {
  SK_CHECK(e && host_out, SK_EINVAL, "engine and host_out must be non-NULL");
  SK_HIP(hipStreamSynchronize(e->stream));
  SK_HIP(hipMemcpy(host_out, e->hidden, (size_t)e->rows * e->c.d_model * sizeof(float), hipMemcpyDeviceToHost));
  return SK_OK;
}

int sk_set_sampling(sk_engine* e, float cfg_scale, float temperature, int32_t top_k, float top_p,
                    int32_t has_q0, float temperature_q0, int32_t top_k_q0, float top_p_q0) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_CHECK(isfinite(cfg_scale) && isfinite(temperature) && isfinite(top_p), SK_EINVAL, "non-finite sampling parameter");
  SK_CHECK(!has_q0 || (isfinite(temperature_q0) && isfinite(top_p_q0)), SK_EINVAL, "non-finite q0 parameter");
  SK_CHECK(e->c.cfg_rows == 2 || cfg_scale == 1.0f, SK_EINVAL, "cfg_scale != 1 needs cfg_rows == 2");
  SkParams p = e->p_host;
  p.cfg_scale = cfg_scale;
  p.temperature = temperature; p.top_k = top_k; p.top_p = top_p;
  p.has_q0 = has_q0 ? 1 : 0;
  p.temperature_q0 = has_q0 ? temperature_q0 : temperature;
  p.top_k_q0 = has_q0 ? top_k_q0 : top_k;
  p.top_p_q0 = has_q0 ? top_p_q0 : top_p;
  SK_HIP(hipStreamSynchronize(e->stream));
  SK_HIP(hipMemcpy(e->params, &p, sizeof(SkParams), hipMemcpyHostToDevice));
  e->p_host = p;
  return SK_OK;
}

int sk_debug_set_spin_ticks(sk_engine* e, uint64_t ticks) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_CHECK(e->exec == nullptr, SK_ESTATE, "the spin limit is set before sk_capture");
  SK_CHECK(ticks <= LX_SPIN_TICKS, SK_EINVAL, "spin limit above %llu ticks", LX_SPIN_TICKS);
  e->spin_ticks = ticks;
  return SK_OK;
}

int sk_set_debug(sk_engine* e, int32_t record_logits) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SkParams p = e->p_host;
  p.record_logits = record_logits ? 1 : 0;
  SK_HIP(hipStreamSynchronize(e->stream));
  SK_HIP(hipMemcpy(e->params, &p, sizeof(SkParams), hipMemcpyHostToDevice));
  e->p_host = p;
  return SK_OK;
}

int sk_capture(sk_engine* e) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  int rc = check_decode_weights(e);
  if (rc != SK_OK) return rc;
  if (e->exec) return SK_OK;
  SK_HIP(hipStreamSynchronize(e->stream));
  e->code_tables = !e->wide && e->c.n_utts == 1 &&
                   code_tables_fit(e->c.d_model, e->rows, e->c.depth_inner, e->c.audio_vocab, e->c.weight_dtype);
  e->wide_tables = e->wide && e->c.depth_inner <= SNT * DEPTH_API && e->c.d_model <= SNT * DEPTH_DPT;
  if ((e->code_tables || e->wide_tables) && (rc = build_code_tables(e)) != SK_OK) return rc;
  if (e->code_tables && e->prefilled) SK_HIP(launch_g1(e));   // a prefill before the capture did not compute G_1
  {
    std::lock_guard<std::mutex> lk(g_frame_order[e->device].mu);
    rc = capture(e, enqueue_frame, &e->graph, &e->exec);
  }
  if (rc != SK_OK) return rc;
  const hipError_t fe = find_attn_nodes(e);
  if (fe != hipSuccess) {
    drop_graphs(e);
    return fail(SK_EHIP, "frame graph nodes: %s", hipGetErrorString(fe));
  }
  SK_HIP(hipStreamSynchronize(e->stream));
  return SK_OK;
}

// The XCD-resident layers' error word (read after the stream is drained).
static int check_lx(sk_engine* e) {
  unsigned w = 0;
  if (e->sk_err) {
    SK_HIP(hipMemcpy(&w, e->sk_err, sizeof(w), hipMemcpyDeviceToHost));
    SK_CHECK(w == 0u, SK_EHIP, "split-K merge wait timed out (error word 0x%x); the engine must be recreated", w);
  }
  if (!e->lx) return SK_OK;
  SK_HIP(hipMemcpy(&w, e->lx_err, sizeof(w), hipMemcpyDeviceToHost));
  SK_CHECK(w == 0u, SK_EHIP, "trunk layer barrier timed out (error word 0x%x); the engine must be recreated", w);
  return SK_OK;
}

static int check_step(sk_engine* e, int n) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_CHECK(e->exec != nullptr, SK_ENOCAPTURE, "step before capture");
  SK_CHECK(e->prefilled, SK_ESTATE, "step before prefill");
  SK_CHECK(n >= 1, SK_EINVAL, "frame count must be positive");
  SK_CHECK(e->fc_host + n <= e->c.max_frames, SK_EKVFULL, "frame ring full (max_frames=%d)", e->c.max_frames);
  for (int r = 0; r < e->rows; ++r)
    SK_CHECK(!e->active_host[r] || e->kv_host[r] + n <= e->c.max_ctx, SK_EKVFULL,
             "KV cache full on row %d (max_ctx=%d)", r, e->c.max_ctx);
  return SK_OK;
}

int sk_step_frame(sk_engine* e, int32_t mask_eos_q0, const double* uniforms,
                  const int64_t* forced_codes, int64_t* codes_out, float* logits_dbg) {
  int rc = check_step(e, 1);
  if (rc != SK_OK) return rc;
  SK_CHECK(codes_out != nullptr, SK_EINVAL, "codes_out is NULL");
  SK_CHECK(!logits_dbg || e->p_host.record_logits, SK_ESTATE, "logits_dbg needs sk_set_debug(e, 1)");
  const sk_config& c = e->c;
  const size_t nq = (size_t)c.n_utts * c.n_codebooks;
  if (uniforms)
    for (size_t i = 0; i < nq; ++i)
      SK_CHECK(uniforms[i] >= 0.0 && uniforms[i] < 1.0, SK_EINVAL, "uniform %zu outside [0,1)", i);
  if (forced_codes)
    for (size_t i = 0; i < nq; ++i)
      SK_CHECK(forced_codes[i] >= 0 && forced_codes[i] < c.audio_vocab, SK_EINVAL, "forced code out of range");
  const int slot = e->fc_host;
  std::vector<double> u(nq, 0.0);
  if (uniforms) memcpy(u.data(), uniforms, nq * sizeof(double));
  const int flags[2] = {mask_eos_q0, forced_codes ? 1 : 0};
  SK_HIP(hipMemcpyAsync(e->u_ring + slot * nq, u.data(), nq * sizeof(double), hipMemcpyHostToDevice, e->stream));
  SK_HIP(hipMemcpyAsync(e->flag_ring + 2 * slot, flags, sizeof(flags), hipMemcpyHostToDevice, e->stream));
  SK_HIP(hipMemcpyAsync(e->u_cur, u.data(), nq * sizeof(double), hipMemcpyHostToDevice, e->stream));
  SK_HIP(hipMemcpyAsync(e->flag_cur, flags, sizeof(flags), hipMemcpyHostToDevice, e->stream));
  if (forced_codes)
    SK_HIP(hipMemcpyAsync(e->forced_ring + slot * nq, forced_codes, nq * sizeof(int64_t), hipMemcpyHostToDevice,
                          e->stream));
  {
    std::lock_guard<std::mutex> lk(g_frame_order[e->device].mu);
    SK_HIP(order_after_previous(e));
    SK_HIP(set_frame_chunks(e, 0));
    SK_HIP(hipGraphLaunch(e->exec, e->stream));
  }
  SK_HIP(hipMemcpyAsync(codes_out, e->codes_ring + slot * nq, nq * sizeof(int64_t), hipMemcpyDeviceToHost, e->stream));
  if (logits_dbg)
    SK_HIP(hipMemcpyAsync(logits_dbg, e->dbg, nq * c.audio_vocab * sizeof(float), hipMemcpyDeviceToHost, e->stream));
  SK_HIP(hipStreamSynchronize(e->stream));
  e->fc_host += 1;
  for (int r = 0; r < e->rows; ++r) e->kv_host[r] += e->active_host[r];
  return check_lx(e);
}

int sk_queue_frames(sk_engine* e, int32_t n, const double* uniforms, const int32_t* mask_eos_q0) {
  int rc = check_step(e, n);
  if (rc != SK_OK) return rc;
  const sk_config& c = e->c;
  const size_t nq = (size_t)c.n_utts * c.n_codebooks;
  std::vector<double> u((size_t)n * nq, 0.0);
  if (uniforms) {
    for (size_t i = 0; i < u.size(); ++i)
      SK_CHECK(uniforms[i] >= 0.0 && uniforms[i] < 1.0, SK_EINVAL, "uniform %zu outside [0,1)", i);
    memcpy(u.data(), uniforms, u.size() * sizeof(double));
  }
  std::vector<int> flags((size_t)2 * n, 0);
  for (int i = 0; i < n; ++i) flags[2 * i] = mask_eos_q0 ? mask_eos_q0[i] : 0;
  SK_HIP(hipStreamSynchronize(e->stream));
  SK_HIP(hipMemcpy(e->u_ring + (size_t)e->fc_host * nq, u.data(), u.size() * sizeof(double), hipMemcpyHostToDevice));
  SK_HIP(hipMemcpy(e->flag_ring + 2 * (size_t)e->fc_host, flags.data(), flags.size() * sizeof(int),
                   hipMemcpyHostToDevice));
  SK_HIP(hipMemcpy(e->u_cur, u.data(), nq * sizeof(double), hipMemcpyHostToDevice));
  SK_HIP(hipMemcpy(e->flag_cur, flags.data(), 2 * sizeof(int), hipMemcpyHostToDevice));
  return SK_OK;
}

int sk_replay(sk_engine* e, int32_t n) {
  int rc = check_step(e, n);
  if (rc != SK_OK) return rc;
  {
    std::lock_guard<std::mutex> lk(g_frame_order[e->device].mu);
    SK_HIP(order_after_previous(e));
    for (int i = 0; i < n; ++i) {
      SK_HIP(set_frame_chunks(e, i));
      SK_HIP(hipGraphLaunch(e->exec, e->stream));
    }
  }
  e->fc_host += n;
  for (int r = 0; r < e->rows; ++r) e->kv_host[r] += n * e->active_host[r];
  return SK_OK;
}

int sk_read_codes(sk_engine* e, int32_t n, int64_t* codes_out) {
  SK_CHECK(e && codes_out, SK_EINVAL, "engine and codes_out must be non-NULL");
  SK_CHECK(n >= 1 && n <= e->fc_host, SK_EINVAL, "only %d frames were decoded", e->fc_host);
  const size_t nq = (size_t)e->c.n_utts * e->c.n_codebooks;
  SK_HIP(hipStreamSynchronize(e->stream));
  SK_HIP(hipMemcpy(codes_out, e->codes_ring + (size_t)(e->fc_host - n) * nq, (size_t)n * nq * sizeof(int64_t),
                   hipMemcpyDeviceToHost));
  return check_lx(e);
}

int sk_synchronize(sk_engine* e) {
  SK_CHECK(e != nullptr, SK_EINVAL, "engine is NULL");
  SK_HIP(hipStreamSynchronize(e->stream));
  return check_lx(e);
}

void* sk_stream(sk_engine* e) { return e ? (void*)e->stream : nullptr; }

int32_t sk_frames_done(sk_engine* e) { return e ? e->fc_host : -1; }
int32_t sk_xcd_layers(sk_engine* e) { return e ? (e->lx ? 1 : 0) : -1; }

}  // extern "C"
