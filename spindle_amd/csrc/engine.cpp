// The decode / verify engine: a C++ restatement of SmolLm2Engine's hot API
// (smollm_chat.rs:1574-1668, forward_slice :3364-3552, forward_batch_slice :3142-3362,
// compute_logits_batch :3588-3602, the greedy speculative loop of generate_reply :4205-4348)
// over one GPU. The whole model and the f16 KV cache stay resident in HBM; one forward pass
// of m <= 16 rows is a fixed launch sequence of fused kernels (fused.hip), captured once per
// m into a HIP graph and replayed with the step record (token ids, start position) in device
// memory.
//
// Residual stream: two buffers alternate so that no kernel reads what it writes. The q/k/v
// kernel reads xA (+ the previous layer's FFN output) and writes the sum to xB; the router
// (or the dense gate/up kernel) reads xB (+ the attention output) and writes the sum to xA.
#include <string.h>

#include <chrono>
#include <cmath>
#include <cstdlib>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/spx.h"
#include "decode.h"
#include "fused.h"
#include "internal.h"
#include "persist.h"
#include "kv.h"
#include "sample.h"
#include "spec.h"

using namespace spx;

namespace {

// kernel classes of the profile (spx_engine_profile_read)
enum {
  PC_EMBED, PC_QKV, PC_ATTN, PC_QUANT, PC_WO, PC_ROUTER, PC_GATEUP, PC_DOWN, PC_NORM, PC_LMHEAD, PC_ARGMAX, PROF_NCLS
};
const char *PROF_NAMES[PROF_NCLS] = {"embed", "qkv_matvec", "attention", "q8k_quantize", "attn_output_matvec", "router_route",
                                     "gate_up_swiglu", "down_combine", "final_norm", "lm_head_matvec", "argmax"};

struct LayerW {
  const float *attn_norm = nullptr, *ffn_norm = nullptr;
  const float *q_bias = nullptr, *k_bias = nullptr, *v_bias = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  spx_tensor *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
  bool moe = false;
  spx_tensor *gate = nullptr, *up = nullptr, *down = nullptr, *router = nullptr;
  int *njobs = nullptr;  // device: [0] jobs of this layer's last pass, [2] experts with users (passes of > 16 rows)
};

bool is_kq(const spx_tensor *t) { return t && (t->v.dtype == T_Q4K || t->v.dtype == T_Q6K); }
bool is_fq(const spx_tensor *t) { return t && (t->v.dtype == T_Q8_0 || t->v.dtype == T_Q5_0 || t->v.dtype == T_Q5K); }
int bucket(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16; }

int64_t now_us() {
  return std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

struct spx_engine {
  spx_ctx *ctx = nullptr;
  spx_model_config c{};
  int q_dim = 0, kv_dim = 0, n_ff = 0, nch = 1, lm_grid = 2048, nbest = 1;
  int lm_dec_grid = 256;  // decode pipeline: LM head workgroups (SPX_LM_DEC_GRID), one per CU
  int n_cu = 256;         // compute units of the device
  bool mq = true;          // passes of 2..16 rows on the int8 matrix cores (SPX_MQ, spx_engine_set_mfma)
  // passes of 2..16 rows: the matrix-core kernels from this many rows, per projection (q|k|v,
  // attention output, gate/up, routed down, LM head; SPX_MQ_ROWS "a,b,c,d,e"); below, the
  // lane-exact kernels (the same bits). Qwen3-30B-A3B shapes, us per launch (matrix cores vs
  // lane-exact): rows 2: 11.2/8.2, 9.9/6.4, 17.4/14.9, 9.4 (lane), 114/93; rows 9: 12.0/13.5,
  // 12.6/11.3, 23.0/31.5, 19.8/16.8, 117/191; rows 16: 12.4/27.7, 13.9/15.1, 26.2/72.8,
  // 22.0/25.4, 119/420.
  enum { MQ_QKV, MQ_WO, MQ_GATEUP, MQ_DOWN, MQ_LM, MQ_KINDS };
  int mq_rows[MQ_KINDS] = {6, 12, 5, 12, 4};
  bool mq_shapes = true;   // every K-quant matrix's blocks-a-row count is one the matrix-core kernels take (dec_mq_nb_ok)
  int mv_mode = -1, lm_mode = -1, tail_max = 2, down_mode = 0;  // launch-shape overrides (SPX_MV_MODE, SPX_LM_MODE, SPX_TAIL_MAX, SPX_DOWN_MODE)
  int pf_attn = 4;          // prefill passes: 4 K / V rows prepared + the position slices (k_attn_fs: bits of its own, no partials), 3 the chunk loop (k_attn_fl), 2 the multi-tile
                            // kernels (the bits verify and decode rows get; at least 2 query heads a kv head), 1 k_rows_prep +
                            // k_attn_pf + merge, 0 k_rows_prep + k_attn (SPX_PF_ATTN)
  int pf_min_rows = MAX_M + 1;  // passes of this many rows or more prepare their attention rows once (SPX_PF_MIN)
  bool att_merge = false;  // one-row passes: attention chunks merged inside the attention launch (SPX_ATT_MERGE)
  int att_mt_min = 2;      // unprepared passes of this many rows (up to 16) take the multi-tile attention (SPX_ATT_MT; 0: never)
  std::map<std::string, spx_tensor *> mats;
  std::map<std::string, float *> vecs;
  std::map<std::string, int64_t> vec_len;
  std::vector<LayerW> L;
  spx_tensor *embed = nullptr, *lm_head = nullptr;
  const float *out_norm = nullptr;
  bool prepared = false, use_graphs = true;
  bool dec_ok = false, dec_on = true;  // one-row passes on the decode pipeline (decode.hip)
  bool dec2 = true;                    // two-row passes on it too (SPX_DEC2; enqueue_decode with nv = 2)
  // one-row passes of a Q8_0 model on the fused kernels with the norms in the consumers'
  // prologues and the residual adds in the producers' epilogues instead of last-workgroup
  // tails (the same bits; SPX_FPRO=0 keeps the tails)
  bool fpro = false;
  // one-row passes with their layers as cooperative launches (persist.hip), where the model
  // fits its tiles; off by default: measured slower than the pipeline (SPX_PERSIST=1 or
  // spx_engine_set_persist turns it on)
  bool persist_ok = false, persist_on = false;
  int persist_grid_n = 0;
  PersistArgs pa{};
  std::vector<PLayer> players;  // the layers' tensors, passed to each layer's launch
  int *perr_host = nullptr;  // pinned: the launch's error word, copied back with the pick
  std::unique_ptr<spx::Sampler> smp;  // spx_engine_generate's sampler (none: plain greedy)
  spx_engine *draft = nullptr;        // draft model for spx_engine_generate (none: prompt lookup)
  std::vector<float> inv_freq;        // RoPE inverse frequencies (host), for the window's slide
  __half *kv_stage = nullptr;         // the slide's staging rows: one layer's K and V [2][max_seq][kv_dim]
  float2 *kv_cs = nullptr;
  std::vector<void *> allocs;
  // device state
  __half *kc = nullptr, *vc = nullptr;
  float2 *rope = nullptr;
  StepRec *st_dev = nullptr, *st_host = nullptr;
  float *xA = nullptr, *xB = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *proj = nullptr, *ffn = nullptr;
  float *xn2 = nullptr, *h = nullptr, *rlog = nullptr, *logits = nullptr, *xn = nullptr, *part_ml = nullptr, *part_o = nullptr;
  Q8KP aq{}, xq2{}, hq{}, xq{};
  int *amax = nullptr, *att_cnt = nullptr, *rt_cnt = nullptr, *gu_cnt = nullptr, *tail_cnt = nullptr, *dn_cnt = nullptr;
  unsigned long long *best = nullptr;
  int *hist = nullptr;  // token history of back-to-back decode passes [max_seq]
  int *chosen = nullptr, *nkeep = nullptr, *expert_count = nullptr;
  float *weights = nullptr;
  Job *jobs = nullptr;
  float *yd = nullptr;  // [PMAX * n_used][dim]: expert outputs of a multi-row pass, combined by the next norm
  float *qp = nullptr;  // [PMAX][q_dim]: prepared queries of a prefill pass
  int last_m = 0;       // rows of the last pass
  // layer snapshots (spx_engine_debug_layers): [n_layers + 1][MAX_M][dbg_off[DBG_NF]] floats
  bool dbg_on = false;
  float *dbg = nullptr;
  int64_t dbg_off[13] = {};
  // captured passes by LM-head selection and rows: [0] every row's logits and pick, [1] the
  // last row's only, [2] none (spx_engine_feed's chunks)
  hipGraphExec_t graph[3][PMAX + 1] = {};
  int lm_sel = 0;       // LM-head selection of the pass being enqueued (as graph's first index)
  int n_used = 0;
  // kernel-class timing (eager passes only): event pairs recorded around each launch
  struct ProfRec { int cls, layer; double bytes; bool per_expert; hipEvent_t a, b; };
  bool profiling = false;
  std::vector<ProfRec> prof;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_next = 0;
  double prof_us[PROF_NCLS] = {}, prof_bytes[PROF_NCLS] = {};
  int64_t prof_n[PROF_NCLS] = {};

  template <class T>
  T *dalloc(size_t n) {
    void *p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(n * sizeof(T), 16)) != hipSuccess) return nullptr;
    allocs.push_back(p);
    // the context's stream does not wait for the null stream: finish the clear before any
    // launch on it can touch the buffer
    if (hipMemset(p, 0, std::max<size_t>(n * sizeof(T), 16)) != hipSuccess || hipDeviceSynchronize() != hipSuccess) return nullptr;
    return static_cast<T *>(p);
  }
  // permuted Q8_K buffer for nv vectors of cols columns
  bool q8alloc(Q8KP &b, int nv, int64_t cols) {
    const int64_t nb = cols / 256;
    b.q = dalloc<uint32_t>((size_t)nv * cols / 4 + 16);
    b.d = dalloc<float>((size_t)nv * nb + 16);
    b.bs = dalloc<int2>((size_t)nv * nb * 8 + 16);
    return b.q && b.d && b.bs;
  }
};

namespace {

// ---------------------------------------------------------------- profiling
struct ProfScope {
  spx_engine *E;
  int idx = -1;
  ProfScope(spx_engine *e, int cls, double bytes, int layer = -1, bool per_expert = false) : E(e) {
    if (!E->profiling) return;
    if (E->ev_next + 2 > E->ev_pool.size()) {
      for (int i = 0; i < 256; i++) { hipEvent_t ev; if (hipEventCreate(&ev) == hipSuccess) E->ev_pool.push_back(ev); }
    }
    if (E->ev_next + 2 > E->ev_pool.size()) return;
    spx_engine::ProfRec r{cls, layer, bytes, per_expert, E->ev_pool[E->ev_next], E->ev_pool[E->ev_next + 1]};
    E->ev_next += 2;
    (void)hipEventRecord(r.a, E->ctx->stream);
    E->prof.push_back(r);
    idx = (int)E->prof.size() - 1;
  }
  ~ProfScope() {
    if (idx >= 0) (void)hipEventRecord(E->prof[idx].b, E->ctx->stream);
  }
};

double wbytes(const spx_tensor *t) { return (double)row_bytes(t->v.dtype, t->v.cols) * (double)t->v.rows; }

// Row r of an m-row Q8_K image of cols values a row.
Q8KP q8kp_row(Q8KP y, int r, int64_t cols) {
  y.q += (int64_t)r * (cols >> 2);
  y.d += (int64_t)r * (cols >> 8);
  y.bs += (int64_t)r * (cols >> 8) * 8;
  return y;
}

Seg seg_of(const spx_tensor *t, float *out, int64_t ld_out, int m, int mode, int R) {
  Seg s{};
  s.w = t->v;
  s.out = out;
  s.ld_out = ld_out;
  s.r0 = 0;
  s.r1 = t->v.rows;
  s.expert = 0;
  s.wgs = mv_wgs(t->v.rows, m, mode, t->v.dtype, R);
  return s;
}

// Launch mode of a matrix pass: row-parallel for integer weights (all m), unless forced to
// eight rows per wavefront (SPX_MV_MODE=0).
int mode_of(const spx_engine *E, const spx_tensor *t, int m) {
  (void)m;
  if (!is_kq(t)) return 0;
  return E->mv_mode >= 0 ? E->mv_mode : 1;
}

// Residual add + RMSNorm feeding the next consumer: the attn_norm of layer l's q/k/v (fp32
// for float-activation weights, Q8_K for integer ones), or for l == n_layers the
// output_norm (fp32 hidden state, and Q8_K for an integer LM head).
NormTail norm_next(spx_engine *E, int l, const float *x, const float *add, float *x_out) {
  NormTail t{};
  t.x = x;
  t.add = add;
  t.rscale = E->c.residual_scale;
  t.eps = E->c.rms_eps;
  t.x_out = x_out;
  t.dim = E->c.dim;
  t.counter = E->tail_cnt;
  if (l < E->c.n_layers) {
    const LayerW &ly = E->L[l];
    t.nw = ly.attn_norm;
    if (is_kq(ly.wq)) t.q_out = E->xq2; else t.xn_out = E->xn2;
  } else {
    t.nw = E->out_norm;
    t.xn_out = E->xn;
    if (is_kq(E->lm_head)) t.q_out = E->xq;
  }
  return t;
}

// ffn_norm of layer l: fp32 for the router or float gate/up, Q8_K for integer gate/up.
NormTail norm_ffn(spx_engine *E, int l, const float *x, const float *add, float *x_out) {
  const LayerW &ly = E->L[l];
  NormTail t{};
  t.x = x;
  t.add = add;
  t.rscale = E->c.residual_scale;
  t.eps = E->c.rms_eps;
  t.x_out = x_out;
  t.dim = E->c.dim;
  t.counter = E->tail_cnt;
  t.nw = ly.ffn_norm;
  if (ly.moe || !is_kq(ly.gate)) t.xn_out = E->xn2;
  if (is_kq(ly.gate)) t.q_out = E->xq2;
  return t;
}

int mv_run(spx_engine *E, MVArgs &a, int m, int mode, int grid_cap = 0) {
  int total = 0;
  for (int i = 0; i < a.nseg; i++) total += a.seg[i].wgs;
  int grid = total;
  if (grid_cap > 0 && grid > grid_cap) grid = grid_cap;
  a.m = m;
  a.nbest = grid;
  a.fq = E->mq ? 1 : 0;
  SPX_HIP(launch_mv(a, m, mode, E->st_dev, grid, E->ctx->stream));
  return 0;
}

// Matrix pass over one tensor; with a norm tail when `tail` has weights and tails are on for
// this pass, else followed by a standalone norm launch.
int mv_one(spx_engine *E, const spx_tensor *w, int m, const float *x, int64_t ld_x, Q8KP y, float *out, int64_t ld_out,
           const NormTail *tail, bool tails, int cls_norm) {
  const int mode = mode_of(E, w, m);
  int G = 8, R = 1;
  rp_shape(w->v.nb, G, R);
  MVArgs a{};
  a.seg[0] = seg_of(w, out, ld_out, m, mode, R);
  a.nseg = 1;
  a.x = x;
  a.ld_x = ld_x;
  a.y = y;
  a.G = G;
  a.R = R;
  a.lscale = E->c.logit_scale;
  const bool fused = tail && tails && (mode == 1 || !is_kq(w));  // the tile kernel takes no tail
  if (fused) a.tail = *tail;
  if (int r = mv_run(E, a, m, mode)) return r;
  if (tail && !fused) {
    ProfScope ps(E, cls_norm, 0);
    SPX_HIP(launch_norm(*tail, E->st_dev, m, E->ctx->stream));
  }
  return 0;
}

// One-row Q8_0 matvec with the residual epilogue res_out = res_in + rscale * y (k_mv_f1):
// the producer's half of a pass without norm tails.
int mv_res(spx_engine *E, const spx_tensor *w, const float *x, int64_t ld_x, float *out, const float *res_in, float *res_out) {
  MVArgs a{};
  a.seg[0] = seg_of(w, out, w->v.rows, 1, 0, 1);
  a.nseg = 1;
  a.x = x;
  a.ld_x = ld_x;
  a.lscale = E->c.logit_scale;
  a.res_in = res_in;
  a.res_out = res_out;
  a.rscale = E->c.residual_scale;
  return mv_run(E, a, 1, 0);
}

// One forward pass of m rows at the step record's start position: embeddings through the
// LM head and the greedy pick (forward_slice / forward_batch_slice + compute_logits_batch).
// Residual stream: the embedding writes xA; attn_output's norm tail adds its output to xA
// and writes xB; the FFN's tail adds its output to xB and writes xA.
// Attention of a pass of m unprepared rows: the multi-tile kernels (launch_attention_mt) from
// att_mt_min rows, else the tile-per-workgroup kernel; both give the same bits.
hipError_t attn_launch(spx_engine *E, const AttnArgs &aa, int m, hipStream_t s) {
  if (E->att_mt_min > 0 && m >= E->att_mt_min && m <= MAX_M && !aa.prepped && (aa.hd == 64 || aa.hd == 128) &&
      (!aa.q_bias || (aa.n_heads / aa.n_kv) * aa.hd <= 2048))
    return launch_attention_mt(aa, m, E->st_dev, s);
  return launch_attention(aa, m, E->st_dev, s);
}

// layer snapshot fields (spx_engine_debug_layers)
enum { DBG_XIN, DBG_Q, DBG_K, DBG_V, DBG_ATT, DBG_PROJ, DBG_XMID, DBG_RLOG, DBG_H, DBG_CHOSEN, DBG_WEIGHTS, DBG_NKEEP, DBG_NF };

// Copies m rows of len words (source rows len words apart, or ld) into field f of layer l's
// snapshot record.
int snap(spx_engine *E, int l, int f, const void *src, int64_t len, int m, int64_t ld = 0) {
  if (!E->dbg_on) return 0;
  const int64_t R = E->dbg_off[DBG_NF];
  SPX_HIP(hipMemcpy2DAsync(E->dbg + (int64_t)l * MAX_M * R + E->dbg_off[f], (size_t)R * 4, src, (size_t)(ld ? ld : len) * 4,
                           (size_t)len * 4, (size_t)m, hipMemcpyDeviceToDevice, E->ctx->stream));
  return 0;
}

// The routed experts' (or the dense FFN's) snapshot fields of layer l after its gate/up.
int snap_ffn(spx_engine *E, int l, int m) {
  if (!E->dbg_on) return 0;
  const LayerW &ly = E->L[l];
  const int64_t nff = ly.gate->v.rows;
  if (int r = snap(E, l, DBG_H, E->h, (ly.moe ? E->n_used : 1) * nff, m)) return r;
  if (!ly.moe) return 0;
  if (int r = snap(E, l, DBG_RLOG, E->rlog, E->c.n_expert, m)) return r;
  if (int r = snap(E, l, DBG_CHOSEN, E->chosen, 32, m)) return r;
  if (int r = snap(E, l, DBG_WEIGHTS, E->weights, 32, m)) return r;
  return snap(E, l, DBG_NKEEP, E->nkeep, 1, m);
}

int enqueue_forward(spx_engine *E, int m, bool advance = false) {
  const auto &c = E->c;
  hipStream_t s = E->ctx->stream;
  const int dim = c.dim, hd = c.head_dim;
  const bool tails = m <= E->tail_max;
  // one-row passes of a Q8_0 model: each consumer normalises its input row itself (pro), each
  // producer adds its residual itself (res): no tails, no norm launches
  const bool pro = E->fpro && m == 1;
  auto pro_of = [&](const float *x, const float *nw, float *xn_out) {
    NormTail t{};
    t.x = x; t.nw = nw; t.eps = c.rms_eps; t.dim = dim; t.xn_out = xn_out;
    return t;
  };
  {
    ProfScope ps(E, PC_EMBED, 0);
    NormTail t = norm_next(E, 0, E->xA, nullptr, nullptr);
    if (pro) t.nw = nullptr;  // the embedding row only
    SPX_HIP(launch_embed(E->embed->v, E->st_dev, c.embedding_scale, t, m, s));
  }
  for (int l = 0; l < c.n_layers; l++) {
    const LayerW &ly = E->L[l];
    {  // q, k, v in one launch
      ProfScope ps(E, PC_QKV, wbytes(ly.wq) + wbytes(ly.wk) + wbytes(ly.wv));
      const int mode = mode_of(E, ly.wq, m);
      int G = 8, R = 1;
      rp_shape(ly.wq->v.nb, G, R);
      MVArgs a{};
      a.seg[0] = seg_of(ly.wq, E->q, E->q_dim, m, mode, R);
      a.seg[1] = seg_of(ly.wk, E->k, E->kv_dim, m, mode, R);
      a.seg[2] = seg_of(ly.wv, E->v, E->kv_dim, m, mode, R);
      a.nseg = 3;
      a.y = E->xq2;
      a.x = E->xn2;
      a.ld_x = dim;
      a.G = G;
      a.R = R;
      if (pro) a.pro = pro_of(E->xA, ly.attn_norm, nullptr);
      if (int r = mv_run(E, a, m, mode)) return r;
    }
    // attention (+ Q8_K of its output for an integer attn_output)
    const bool wo_int = is_kq(ly.wo);
    const bool att_q_fused = wo_int && ((c.n_heads / c.n_kv_heads) * hd) % 256 == 0;
    {
      ProfScope ps(E, PC_ATTN, -1.0 - l);
      AttnArgs aa{};
      aa.q = E->q; aa.k = E->k; aa.v = E->v;
      aa.q_bias = ly.q_bias; aa.k_bias = ly.k_bias; aa.v_bias = ly.v_bias; aa.q_norm = ly.q_norm; aa.k_norm = ly.k_norm;
      aa.rope = E->rope; aa.kc = E->kc; aa.vc = E->vc; aa.part_ml = E->part_ml; aa.part_o = E->part_o; aa.counter = E->att_cnt; aa.att = E->att;
      if (att_q_fused) aa.aq = E->aq;
      aa.layer = l; aa.max_seq = c.max_seq; aa.kv_dim = E->kv_dim; aa.hd = hd; aa.n_heads = c.n_heads; aa.n_kv = c.n_kv_heads;
      aa.neox = c.rope_neox; aa.nch = E->nch; aa.nslot = E->nch + ATT_GMAX; aa.eps = c.rms_eps;
      aa.scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt((float)hd);
      SPX_HIP(attn_launch(E, aa, m, s));
    }
    if (wo_int && !att_q_fused) { ProfScope ps(E, PC_QUANT, 0); SPX_HIP(launch_q8kp_quantize(E->att, E->q_dim, E->q_dim, m, E->aq, s)); }
    {  // attn_output + residual + ffn_norm
      ProfScope ps(E, PC_WO, wbytes(ly.wo));
      const NormTail t = norm_ffn(E, l, E->xA, E->proj, E->xB);
      if (pro) {
        if (int r = mv_res(E, ly.wo, E->att, E->q_dim, E->proj, E->xA, E->xB)) return r;
      } else {
        if (int r = mv_one(E, ly.wo, m, E->att, E->q_dim, E->aq, E->proj, dim, &t, tails, PC_NORM)) return r;
      }
    }
    const int nff = (int)ly.gate->v.rows;
    const bool d_int = is_kq(ly.down);
    const NormTail tn = norm_next(E, l + 1, E->xB, E->ffn, E->xA);
    const int gmode = m <= 2 ? mode_of(E, ly.gate, m) : 0;  // grouped experts: row-parallel at decode, tiles for verify
    if (ly.moe) {  // moe_forward / moe_forward_batch (:925-1392)
      const int nu = c.n_expert_used, ne = c.n_expert;
      {
        ProfScope ps(E, PC_ROUTER, wbytes(ly.router));
        RouterArgs ra{};
        ra.w = ly.router->v; ra.x = E->xn2; ra.logits = E->rlog; ra.dim = dim;
        ra.n_expert = ne; ra.n_used = nu; ra.norm = c.expert_norm; ra.moe_prune = c.moe_prune; ra.counter = E->rt_cnt;
        ra.chosen = E->chosen; ra.weights = E->weights; ra.nkeep = E->nkeep; ra.jobs = E->jobs; ra.njobs = ly.njobs;
        ra.expert_count = E->expert_count + (size_t)l * ne;
        if (pro) { ra.pro = pro_of(E->xB, ly.ffn_norm, nullptr); ra.logits_only = 1; }
        SPX_HIP(launch_router(ra, m, E->st_dev, s));
      }
      const int max_gu_jobs = std::min(256, m * nu);  // jobs of at most GU_USERS users
      // Q8_0 experts, 2..16 rows: gate/up and down on the fp32 matrix cores, a job per expert
      const bool fq = E->mq && m >= FQ_MIN_ROWS && m <= MAX_M && ly.gate->v.dtype == T_Q8_0 && ly.up->v.dtype == T_Q8_0 &&
                      ly.down->v.dtype == T_Q8_0;
      const int max_dn_jobs = std::min(ne, m * nu);
      {
        ProfScope ps(E, PC_GATEUP, wbytes(ly.gate) + wbytes(ly.up), l, true);  // one expert's slabs
        GUArgs ga{};
        ga.gate = ly.gate->v; ga.up = ly.up->v; ga.y = E->xq2; ga.x = E->xn2;
        ga.jobs = E->jobs; ga.njobs = ly.njobs + 1; ga.h = E->h; ga.counter = E->gu_cnt; ga.n_ff = nff;
        if (d_int) ga.hq = E->hq;
        if (pro) {  // the routing in the gate/up prologue (one job per kept choice)
          ga.pro = pro_of(E->xB, ly.ffn_norm, nullptr);
          F1Route &rt = ga.rt;
          rt.logits = E->rlog; rt.n_expert = ne; rt.n_used = nu; rt.norm = c.expert_norm; rt.moe_prune = c.moe_prune;
          rt.chosen = E->chosen; rt.weights = E->weights; rt.nkeep = E->nkeep; rt.jobs = E->jobs + 256; rt.njobs = ly.njobs;
          rt.expert_count = E->expert_count + (size_t)l * ne;
        }
        if (fq) {
          ga.jobs = E->jobs + 256; ga.njobs = ly.njobs; ga.vdiv = nu; ga.fq = 1;
          SPX_HIP(launch_gateup(ga, m, 0, E->st_dev, max_dn_jobs, s));
        } else {
          SPX_HIP(launch_gateup(ga, std::min(m, GU_USERS), mode_of(E, ly.gate, m), E->st_dev, max_gu_jobs, s));
        }
      }
      {
        ProfScope ps(E, PC_DOWN, wbytes(ly.down), l, true);
        DownArgs da{};
        da.w = ly.down->v; da.y = E->hq; da.x = E->h; da.jobs = E->jobs + 256; da.njobs = ly.njobs; da.weights = E->weights;
        da.nkeep = E->nkeep; da.n_used = nu; da.out = E->ffn;
        if (pro) { da.res_in = E->xB; da.res_out = E->xA; da.rscale = c.residual_scale; }
        else if (tails) da.tail = tn;
        if (fq) {
          da.yd = E->yd; da.counter = E->dn_cnt;
          SPX_HIP(launch_down_fq(da, max_dn_jobs, E->st_dev, s));
        } else {
          SPX_HIP(launch_down(da, m, m > 2 && d_int && E->down_mode == 1 ? 1 : 0, E->st_dev, s));
        }
      }
      if (!tails && !pro) { ProfScope ps(E, PC_NORM, 0); SPX_HIP(launch_norm(tn, E->st_dev, m, s)); }
    } else {  // ffn_forward / ffn_forward_multi (:590-646): k = 1, w = 1
      {
        ProfScope ps(E, PC_GATEUP, wbytes(ly.gate) + wbytes(ly.up));
        GUArgs ga{};
        ga.gate = ly.gate->v; ga.up = ly.up->v; ga.y = E->xq2; ga.x = E->xn2; ga.h = E->h; ga.counter = E->gu_cnt; ga.n_ff = nff;
        ga.fq = E->mq && m >= FQ_MIN_ROWS ? 1 : 0;
        if (d_int) ga.hq = E->hq;
        if (pro) ga.pro = pro_of(E->xB, ly.ffn_norm, nullptr);
        SPX_HIP(launch_gateup(ga, m, gmode, E->st_dev, 1, s));
      }
      {
        ProfScope ps(E, PC_DOWN, wbytes(ly.down));
        if (pro) {
          if (int r = mv_res(E, ly.down, E->h, nff, E->ffn, E->xB, E->xA)) return r;
        } else {
          if (int r = mv_one(E, ly.down, m, E->h, nff, E->hq, E->ffn, dim, &tn, tails, PC_NORM)) return r;
        }
      }
    }
  }
  if (E->lm_sel == 2) return 0;  // feed's earlier chunks: no logits
  // feed's last chunk: the last row's logits and pick only (row 0 of logits / amax; its
  // normalised row stays at row m - 1 of xn)
  const bool last = E->lm_sel == 1 && m > 1;
  const int lm = last ? 1 : m;
  {
    ProfScope ps(E, PC_LMHEAD, wbytes(E->lm_head));
    const int mode = E->lm_mode >= 0 && is_kq(E->lm_head) ? E->lm_mode : 0;
    int G = 8, R = 1;
    rp_shape(E->lm_head->v.nb, G, R);
    MVArgs a{};
    a.seg[0] = seg_of(E->lm_head, E->logits, c.vocab, lm, mode, R);
    a.nseg = 1;
    a.x = E->xn + (int64_t)(m - lm) * dim;
    a.ld_x = dim;
    a.y = q8kp_row(E->xq, m - lm, dim);
    if (pro) a.pro = pro_of(E->xA, E->out_norm, E->xn);  // (one row: xn written by workgroup 0)
    a.G = G;
    a.R = R;
    a.best = E->best;
    a.lscale = c.logit_scale;
    if (last) {  // one vector: no step record (its m is the pass's)
      int grid = a.seg[0].wgs;
      if (mode == 0 && E->lm_grid > 0 && grid > E->lm_grid) grid = E->lm_grid;
      a.m = 1;
      a.nbest = grid;
      SPX_HIP(launch_mv(a, 1, mode, nullptr, grid, s));
      E->nbest = grid;
    } else {
      if (int r = mv_run(E, a, m, mode, mode == 0 ? E->lm_grid : 0)) return r;
      E->nbest = a.nbest;
    }
  }
  {
    ProfScope ps(E, PC_ARGMAX, 0);
    SPX_HIP(launch_argmax_final(E->best, E->nbest, E->amax, last ? nullptr : E->st_dev, advance ? E->hist : nullptr, lm, s));
  }
  return 0;
}

// One-row pass on the decode pipeline (decode.hip): the same values as enqueue_forward(E, 1),
// computed by kernels that meet only at kernel boundaries. Residual stream: the embedding
// writes xA; attn_output writes xB = xA + rscale * proj; the FFN writes xA = xB + rscale * y.
// nv = 2: a two-row pass (verify of a one-token draft) on the same kernels, each taking both
// rows (kd_mv2, kd_router<2>, kd_gateup<.., 2>, kd_down<.., 2>: every row the bits of its
// one-row pass, the weights read once), attention on the multi-row kernels; no step-record
// advance, no layer snapshots (those passes take enqueue_pass_m).
int enqueue_decode(spx_engine *E, bool advance, int nv = 1) {
  const auto &c = E->c;
  hipStream_t s = E->ctx->stream;
  const int dim = c.dim, hd = c.head_dim;
  auto tiles_g = [](const spx_tensor *t, int G) { return (int)((t->v.rows + DEC_MV_NW * (8 / G) - 1) / (DEC_MV_NW * (8 / G))); };
  auto gshape = [](const spx_tensor *t) { int G, R; rp_shape(t->v.nb, G, R); return G; };
  auto tiles = [&](const spx_tensor *t) { return tiles_g(t, gshape(t)); };
  {
    ProfScope ps(E, PC_EMBED, 0);
    NormTail t{};
    t.x = E->xA;
    t.dim = dim;
    SPX_HIP(launch_embed(E->embed->v, E->st_dev, c.embedding_scale, t, nv, s));
  }
  for (int l = 0; l < c.n_layers; l++) {
    const LayerW &ly = E->L[l];
    if (int r = snap(E, l, DBG_XIN, E->xA, dim, 1)) return r;
    {
      ProfScope ps(E, PC_QKV, wbytes(ly.wq) + wbytes(ly.wk) + wbytes(ly.wv));
      DecMVArgs a{};
      const spx_tensor *w3[3] = {ly.wq, ly.wk, ly.wv};
      float *o3[3] = {E->q, E->k, E->v};
      // row groups: rp_shape's unless twice the rows a workgroup (G / 2, two blocks a group)
      // keeps the launch within one workgroup a CU (a second one on a CU doubles its prologue)
      int G = gshape(ly.wq), total = 0;
      if (G >= 2 && (ly.wq->v.nb + G / 2 - 1) / (G / 2) <= 2 && tiles_g(ly.wq, G) + tiles_g(ly.wk, G) + tiles_g(ly.wv, G) > E->n_cu &&
          tiles_g(ly.wq, G / 2) + tiles_g(ly.wk, G / 2) + tiles_g(ly.wv, G / 2) <= E->n_cu)
        G /= 2;
      for (int i = 0; i < 3; i++) { a.w[i] = w3[i]->v; a.out[i] = o3[i]; a.tiles[i] = tiles_g(w3[i], G); total += a.tiles[i]; }
      a.nseg = 3;
      a.G = G;
      a.in = DecIn{E->xA, ly.attn_norm, c.rms_eps, dim};
      a.nv = nv;
      SPX_HIP(launch_dec_mv(a, total, s));
    }
    if (int r = snap(E, l, DBG_Q, E->q, E->q_dim, 1) || snap(E, l, DBG_K, E->k, E->kv_dim, 1) || snap(E, l, DBG_V, E->v, E->kv_dim, 1)) return r;
    {
      ProfScope ps(E, PC_ATTN, -1.0 - l);
      AttnArgs aa{};
      aa.q = E->q; aa.k = E->k; aa.v = E->v;
      aa.q_bias = ly.q_bias; aa.k_bias = ly.k_bias; aa.v_bias = ly.v_bias; aa.q_norm = ly.q_norm; aa.k_norm = ly.k_norm;
      aa.rope = E->rope; aa.kc = E->kc; aa.vc = E->vc; aa.part_ml = E->part_ml; aa.part_o = E->part_o; aa.counter = E->att_cnt; aa.att = E->att;
      aa.layer = l; aa.max_seq = c.max_seq; aa.kv_dim = E->kv_dim; aa.hd = hd; aa.n_heads = c.n_heads; aa.n_kv = c.n_kv_heads;
      aa.neox = c.rope_neox; aa.nch = E->nch; aa.nslot = E->nch + ATT_GMAX; aa.eps = c.rms_eps;
      aa.scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt((float)hd);
      if (nv > 1) {
        SPX_HIP(attn_launch(E, aa, nv, s));
      } else if (E->att_merge) {
        SPX_HIP(launch_attention(aa, 1, E->st_dev, s));
      } else {
        SPX_HIP(launch_attention_partials(aa, E->st_dev, s));
        DecMergeArgs ma{E->part_ml, E->part_o, E->att, aa.nslot, hd, c.n_heads, c.n_kv_heads};
        SPX_HIP(launch_dec_merge(ma, E->st_dev, s));
      }
    }
    if (int r = snap(E, l, DBG_ATT, E->att, E->q_dim, 1)) return r;
    {
      ProfScope ps(E, PC_WO, wbytes(ly.wo));
      DecMVArgs a{};
      a.w[0] = ly.wo->v; a.out[0] = E->proj; a.tiles[0] = tiles(ly.wo); a.nseg = 1; a.G = gshape(ly.wo);
      a.in = DecIn{E->att, nullptr, 0.0f, E->q_dim};
      a.res_in = E->xA; a.res_out = E->xB; a.rscale = c.residual_scale;
      a.nv = nv;
      SPX_HIP(launch_dec_mv(a, a.tiles[0], s));
    }
    if (int r = snap(E, l, DBG_PROJ, E->proj, dim, 1) || snap(E, l, DBG_XMID, E->xB, dim, 1)) return r;
    const int nff = (int)ly.gate->v.rows;
    const DecIn fin{E->xB, ly.ffn_norm, c.rms_eps, dim};
    DecGateUpArgs ga{};
    ga.gate = ly.gate->v; ga.up = ly.up->v; ga.in = fin; ga.h = E->h; ga.n_ff = nff; ga.nv = nv;
    if (ly.moe) {  // moe_forward (:1176-1392)
      {
        ProfScope ps(E, PC_ROUTER, wbytes(ly.router));
        DecRouterArgs ra{ly.router->v, fin, E->rlog, c.n_expert, nv};
        SPX_HIP(launch_dec_router(ra, s));
      }
      {
        ProfScope ps(E, PC_GATEUP, wbytes(ly.gate) + wbytes(ly.up), l, true);  // one expert's slabs
        ga.logits = E->rlog; ga.n_expert = c.n_expert; ga.n_used = c.n_expert_used; ga.norm = c.expert_norm; ga.moe_prune = c.moe_prune;
        ga.chosen = E->chosen; ga.weights = E->weights; ga.nkeep = E->nkeep; ga.njobs = ly.njobs;
        ga.expert_count = E->expert_count + (size_t)l * c.n_expert;
        SPX_HIP(launch_dec_gateup(ga, s));
      }
      if (int r = snap_ffn(E, l, 1)) return r;
      {
        ProfScope ps(E, PC_DOWN, wbytes(ly.down), l, true);
        DecDownArgs da{ly.down->v, E->h, E->chosen, E->weights, E->nkeep, c.n_expert_used, E->xB, E->xA, c.residual_scale, nv};
        SPX_HIP(launch_dec_down(da, s));
      }
    } else {  // ffn_forward (:590-614)
      {
        ProfScope ps(E, PC_GATEUP, wbytes(ly.gate) + wbytes(ly.up));
        SPX_HIP(launch_dec_gateup(ga, s));
      }
      if (int r = snap_ffn(E, l, 1)) return r;
      {
        ProfScope ps(E, PC_DOWN, wbytes(ly.down));
        DecMVArgs a{};
        a.w[0] = ly.down->v; a.out[0] = E->ffn; a.tiles[0] = tiles(ly.down); a.nseg = 1; a.G = gshape(ly.down);
        a.in = DecIn{E->h, nullptr, 0.0f, nff};
        a.res_in = E->xB; a.res_out = E->xA; a.rscale = c.residual_scale;
        a.nv = nv;
        SPX_HIP(launch_dec_mv(a, a.tiles[0], s));
      }
    }
  }
  if (int r = snap(E, c.n_layers, DBG_XIN, E->xA, dim, 1)) return r;
  if (nv > 1 && E->lm_sel == 2) return 0;  // feed's earlier chunks: no logits
  const bool last = nv > 1 && E->lm_sel == 1;  // the last row only (row 0 of xn / logits / amax)
  const int nl = last ? 1 : nv;
  int grid = 1;
  {
    ProfScope ps(E, PC_LMHEAD, wbytes(E->lm_head));
    DecMVArgs a{};
    a.w[0] = E->lm_head->v; a.out[0] = E->logits; a.tiles[0] = tiles(E->lm_head); a.nseg = 1; a.G = gshape(E->lm_head);
    a.in = DecIn{E->xA + (int64_t)(nv - nl) * dim, E->out_norm, c.rms_eps, dim};
    a.best = E->best; a.lscale = c.logit_scale; a.xn_out = E->xn;
    a.nv = nl;
    grid = std::min(a.tiles[0], E->lm_dec_grid);
    SPX_HIP(launch_dec_mv(a, grid, s));
  }
  E->nbest = grid;
  {
    ProfScope ps(E, PC_ARGMAX, 0);
    SPX_HIP(launch_argmax_final(E->best, grid, E->amax, last ? nullptr : E->st_dev, advance ? E->hist : nullptr, nl, s));
  }
  return 0;
}

// A pass of 2 <= m <= 16 rows on the decode pipeline's multi-row kernels: the same values as
// enqueue_forward(E, m). Per layer: attn_norm (Q8_K of the rows), q/k/v, attention (the fused
// multi-row kernel, its merge and the Q8_K of its output included), attn_output + residual,
// ffn_norm, then router / routing + jobs / grouped gate-up / Q8_K of h / grouped down +
// combine + residual (dense: gate-up / Q8_K of h / down + residual).
int enqueue_pass_m(spx_engine *E, int m) {
  const auto &c = E->c;
  hipStream_t s = E->ctx->stream;
  const int dim = c.dim, hd = c.head_dim, nu = E->n_used;
  auto mtiles = [](const spx_tensor *t) {
    int G, R;
    rp_shape(t->v.nb, G, R);
    return (int)((t->v.rows + DEC_MM_NW * R - 1) / (DEC_MM_NW * R));
  };
  auto gshape = [](const spx_tensor *t) { int G, R; rp_shape(t->v.nb, G, R); return G; };
  auto qtiles = [](const spx_tensor *t) { return (int)((t->v.rows + 15) / 16); };
  // passes of more than 16 rows (prefill; matrix cores only): the matvecs take the rows in
  // groups of 16 per workgroup, the attention rows are prepared once (launch_rows_prep), the
  // MoE jobs hold at most 16 users (kp_route) and are staged job by job (kp_gateup_mq)
  const bool big = m > MAX_M;
  const bool mq = E->mq && E->mq_shapes;  // (the lane-exact kernels where a matrix's shape has no matrix-core kernel)
  if (big && !mq) return fail("passes of more than 16 rows run on the matrix cores only (blocks-a-row counts 1, 2, 3, 4, 8, 16)");
  auto mqk = [&](int kind) { return mq && (big || m >= E->mq_rows[kind]); };
  auto mq_grid = [&](int tiles) { return dec_mq_grid(tiles, m); };
  const int maxj = std::min(512, std::min(c.n_expert, m * nu) + (m * nu) / MAX_M);  // jobs of <= 16 users
  bool combine = false;  // the last MoE layer's expert outputs wait in yd for the next norm
  auto norm = [&](const float *x, const float *nw, float *xn_out, Q8KP q) {
    DecNormArgs na{};
    na.x = x; na.nw = nw; na.eps = c.rms_eps; na.dim = dim; na.xn_out = xn_out; na.q_out = q;
    if (combine) {  // x = xB + combine, written back to xA (= x)
      na.yd = E->yd; na.cw = E->weights; na.nkeep = E->nkeep; na.res_in = E->xB; na.x_out = E->xA;
      na.n_used = nu; na.rscale = c.residual_scale;
      combine = false;
    }
    return launch_dec_norm(na, m, s);
  };
  {
    ProfScope ps(E, PC_EMBED, 0);
    NormTail t{};
    t.x = E->xA;
    t.dim = dim;
    SPX_HIP(launch_embed(E->embed->v, E->st_dev, c.embedding_scale, t, m, s));
  }
  for (int l = 0; l < c.n_layers; l++) {
    const LayerW &ly = E->L[l];
    {
      ProfScope ps(E, PC_NORM, 0);
      SPX_HIP(norm(E->xA, ly.attn_norm, nullptr, E->xq2));
    }
    if (int r = snap(E, l, DBG_XIN, E->xA, dim, m)) return r;
    {
      ProfScope ps(E, PC_QKV, wbytes(ly.wq) + wbytes(ly.wk) + wbytes(ly.wv));
      DecMMArgs a{};
      const spx_tensor *w3[3] = {ly.wq, ly.wk, ly.wv};
      float *o3[3] = {E->q, E->k, E->v};
      const int64_t ld3[3] = {E->q_dim, E->kv_dim, E->kv_dim};
      int total = 0;
      for (int i = 0; i < 3; i++) { a.w[i] = w3[i]->v; a.out[i] = o3[i]; a.ld_out[i] = ld3[i]; a.tiles[i] = mqk(spx_engine::MQ_QKV) ? qtiles(w3[i]) : mtiles(w3[i]); total += a.tiles[i]; }
      a.nseg = 3; a.G = gshape(ly.wq); a.y = E->xq2; a.cols = dim; a.m = m;
      SPX_HIP(mqk(spx_engine::MQ_QKV) ? launch_dec_mq(a, mq_grid(total), s) : launch_dec_mm(a, dec_mm_grid(total), s));
    }
    if (int r = snap(E, l, DBG_Q, E->q, E->q_dim, m) || snap(E, l, DBG_K, E->k, E->kv_dim, m) || snap(E, l, DBG_V, E->v, E->kv_dim, m)) return r;
    const bool att_q_fused = ((c.n_heads / c.n_kv_heads) * hd) % 256 == 0;
    {
      ProfScope ps(E, PC_ATTN, -1.0 - l);
      AttnArgs aa{};
      aa.q = E->q; aa.k = E->k; aa.v = E->v;
      aa.q_bias = ly.q_bias; aa.k_bias = ly.k_bias; aa.v_bias = ly.v_bias; aa.q_norm = ly.q_norm; aa.k_norm = ly.k_norm;
      aa.rope = E->rope; aa.kc = E->kc; aa.vc = E->vc; aa.part_ml = E->part_ml; aa.part_o = E->part_o; aa.counter = E->att_cnt; aa.att = E->att;
      if (att_q_fused) aa.aq = E->aq;
      aa.layer = l; aa.max_seq = c.max_seq; aa.kv_dim = E->kv_dim; aa.hd = hd; aa.n_heads = c.n_heads; aa.n_kv = c.n_kv_heads;
      aa.neox = c.rope_neox; aa.nch = E->nch; aa.nslot = E->nch + ATT_GMAX; aa.eps = c.rms_eps;
      aa.scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt((float)hd);
      if (m >= E->pf_min_rows && E->pf_attn >= 3 && m > MAX_M && (hd == 64 || hd == 128)) {
        // rows prepared once, then a chunk loop with bits of its own (prefill rows share no
        // bits with verify rows: a row's attention differs from its 16-row pass's in the last bits)
        if (E->pf_attn == 4) {  // K / V rows prepared, the queries in the attention kernel
          SPX_HIP(launch_rows_prep(aa, nullptr, m, E->st_dev, s));
          aa.prepped = 2;
          SPX_HIP(launch_attention_fs(aa, m, E->st_dev, s));
        } else {
          SPX_HIP(launch_rows_prep(aa, E->qp, m, E->st_dev, s));
          aa.q = E->qp;
          aa.prepped = 1;
          SPX_HIP(launch_attention_fl(aa, m, E->st_dev, s));
        }
      } else if (m >= E->pf_min_rows && E->pf_attn >= 2 && m > MAX_M && c.n_heads / c.n_kv_heads >= 2 &&
          (!ly.q_bias || (c.n_heads / c.n_kv_heads) * hd <= 2048)) {
        SPX_HIP(launch_attention_mt(aa, m, E->st_dev, s));
      } else if (m >= E->pf_min_rows) {  // rows prepared once (for 2..16 rows the fused kernel is faster: M = 9 4.46 vs 4.69 ms a pass)
        SPX_HIP(launch_rows_prep(aa, E->qp, m, E->st_dev, s));
        aa.q = E->qp;
        aa.prepped = 1;
        SPX_HIP(E->pf_attn ? launch_attention_pf(aa, m, E->st_dev, s) : attn_launch(E, aa, m, s));
      } else {
        SPX_HIP(attn_launch(E, aa, m, s));
      }
    }
    if (!att_q_fused) { ProfScope ps(E, PC_QUANT, 0); SPX_HIP(launch_q8kp_quantize(E->att, E->q_dim, E->q_dim, m, E->aq, s)); }
    if (int r = snap(E, l, DBG_ATT, E->att, E->q_dim, m)) return r;
    {
      ProfScope ps(E, PC_WO, wbytes(ly.wo));
      DecMMArgs a{};
      a.w[0] = ly.wo->v; a.out[0] = E->proj; a.ld_out[0] = dim; a.tiles[0] = mqk(spx_engine::MQ_WO) ? qtiles(ly.wo) : mtiles(ly.wo); a.nseg = 1; a.G = gshape(ly.wo);
      a.y = E->aq; a.cols = E->q_dim; a.m = m;
      a.res_in = E->xA; a.res_out = E->xB; a.rscale = c.residual_scale;
      SPX_HIP(mqk(spx_engine::MQ_WO) ? launch_dec_mq(a, mq_grid(a.tiles[0]), s) : launch_dec_mm(a, dec_mm_grid(a.tiles[0]), s));
    }
    if (int r = snap(E, l, DBG_PROJ, E->proj, dim, m) || snap(E, l, DBG_XMID, E->xB, dim, m)) return r;
    const int nff = (int)ly.gate->v.rows;
    {
      ProfScope ps(E, PC_NORM, 0);
      SPX_HIP(norm(E->xB, ly.ffn_norm, ly.moe ? E->xn2 : nullptr, E->xq2));
    }
    DecGateUpMArgs ga{};
    ga.gate = ly.gate->v; ga.up = ly.up->v; ga.y = E->xq2; ga.h = E->h; ga.n_ff = nff; ga.m = m;
    if (ly.moe) {  // moe_forward_batch (:925-1174)
      {
        ProfScope ps(E, PC_ROUTER, wbytes(ly.router));
        DecRouterMArgs ra{ly.router->v, E->xn2, E->rlog, c.n_expert, dim, m};
        SPX_HIP(launch_dec_router_m(ra, s));
      }
      {  // routing + jobs (every workgroup) and the grouped gate/up
        ProfScope ps(E, PC_GATEUP, wbytes(ly.gate) + wbytes(ly.up), l, true);
        ga.rt = DecRouteArgs{E->rlog, c.n_expert, c.n_expert_used, c.expert_norm, m, c.moe_prune, E->chosen, E->weights, E->nkeep,
                             E->jobs, ly.njobs, E->expert_count + (size_t)l * c.n_expert};
        if (big) {
          SPX_HIP(launch_kp_route(ga.rt, s));
          SPX_HIP(launch_kp_gateup_mq(ga, E->jobs, ly.njobs, maxj, s));
        } else {
          SPX_HIP(mqk(spx_engine::MQ_GATEUP) ? launch_dec_gateup_mq(ga, std::min(m * nu, c.n_expert), s) : launch_dec_gateup_m(ga, std::min(m * nu, c.n_expert), s));
        }
      }
      if (int r = snap_ffn(E, l, m)) return r;
      {
        ProfScope ps(E, PC_DOWN, wbytes(ly.down), l, true);
        DecDownMArgs da{ly.down->v, E->h, E->jobs, ly.njobs, E->yd, big ? maxj : std::min(m * nu, c.n_expert)};
        SPX_HIP(mqk(spx_engine::MQ_DOWN) ? launch_dec_down_mq(da, s) : launch_dec_down_m(da, s));
        combine = true;  // + weighted combine + residual in the next norm (xB -> xA)
      }
    } else {  // ffn_forward_multi (:616-646)
      {
        ProfScope ps(E, PC_GATEUP, wbytes(ly.gate) + wbytes(ly.up));
        if (big) SPX_HIP(launch_kp_gateup_mq(ga, nullptr, nullptr, 1, s));
        else SPX_HIP(mqk(spx_engine::MQ_GATEUP) ? launch_dec_gateup_mq(ga, 1, s) : launch_dec_gateup_m(ga, 1, s));
        SPX_HIP(launch_q8kp_quantize(E->h, nff, nff, m, E->hq, s));
      }
      if (int r = snap_ffn(E, l, m)) return r;
      {
        ProfScope ps(E, PC_DOWN, wbytes(ly.down));
        DecMMArgs a{};
        a.w[0] = ly.down->v; a.out[0] = E->ffn; a.ld_out[0] = dim; a.tiles[0] = mqk(spx_engine::MQ_DOWN) ? qtiles(ly.down) : mtiles(ly.down); a.nseg = 1;
        a.G = gshape(ly.down); a.y = E->hq; a.cols = nff; a.m = m;
        a.res_in = E->xB; a.res_out = E->xA; a.rscale = c.residual_scale;
        SPX_HIP(mqk(spx_engine::MQ_DOWN) ? launch_dec_mq(a, mq_grid(a.tiles[0]), s) : launch_dec_mm(a, dec_mm_grid(a.tiles[0]), s));
      }
    }
  }
  if (E->lm_sel == 2) return 0;  // feed's earlier chunks: no logits
  int grid = 1;
  if (E->lm_sel == 1) {  // feed's last chunk: the last row's output_norm, logits and pick (row 0 of xn / logits / amax)
    ProfScope ps(E, PC_LMHEAD, wbytes(E->lm_head));
    SPX_HIP(norm(E->xA, E->out_norm, E->xn, E->xq));  // (also the last layer's expert combine into xA)
    const int G = gshape(E->lm_head), R = 8 / G;
    DecMVArgs a{};
    a.w[0] = E->lm_head->v; a.out[0] = E->logits; a.tiles[0] = (int)((E->lm_head->v.rows + DEC_MV_NW * R - 1) / (DEC_MV_NW * R));
    a.nseg = 1; a.G = G;
    a.in = DecIn{E->xA + (int64_t)(m - 1) * dim, E->out_norm, c.rms_eps, dim};
    a.best = E->best; a.lscale = c.logit_scale; a.xn_out = E->xn;
    grid = std::min(a.tiles[0], E->lm_dec_grid);
    SPX_HIP(launch_dec_mv(a, grid, s));
    E->nbest = grid;
    ProfScope pa(E, PC_ARGMAX, 0);
    SPX_HIP(launch_argmax_final(E->best, grid, E->amax, nullptr, nullptr, 1, s));
    return 0;
  }
  {
    ProfScope ps(E, PC_LMHEAD, wbytes(E->lm_head));
    SPX_HIP(norm(E->xA, E->out_norm, E->xn, E->xq));
    if (int r = snap(E, c.n_layers, DBG_XIN, E->xA, dim, m)) return r;
    DecMMArgs a{};
    a.w[0] = E->lm_head->v; a.out[0] = E->logits; a.ld_out[0] = c.vocab; a.tiles[0] = mqk(spx_engine::MQ_LM) ? qtiles(E->lm_head) : mtiles(E->lm_head); a.nseg = 1;
    a.G = gshape(E->lm_head); a.y = E->xq; a.cols = dim; a.m = m;
    grid = mqk(spx_engine::MQ_LM) ? mq_grid(a.tiles[0]) : std::min(a.tiles[0], 512);
    a.best = E->best; a.nbest = grid; a.lscale = c.logit_scale;
    SPX_HIP(mqk(spx_engine::MQ_LM) ? launch_dec_mq(a, grid, s) : launch_dec_mm(a, grid, s));
  }
  E->nbest = grid;
  {
    ProfScope ps(E, PC_ARGMAX, 0);
    SPX_HIP(launch_argmax_final(E->best, grid, E->amax, E->st_dev, nullptr, m, s));
  }
  return 0;
}

// A one-row pass with its layers as cooperative launches of the persistent kernel (barrier
// counters zeroed first) between the decode pipeline's embedding and its LM head and pick.
int enqueue_persist(spx_engine *E, bool advance) {
  const auto &c = E->c;
  hipStream_t s = E->ctx->stream;
  {
    ProfScope ps(E, PC_EMBED, 0);
    NormTail t{};
    t.x = E->xA;
    t.dim = c.dim;
    SPX_HIP(launch_embed(E->embed->v, E->st_dev, c.embedding_scale, t, 1, s));
  }
  SPX_HIP(hipMemsetAsync(E->pa.bar, 0, PERSIST_BAR_WORDS * sizeof(unsigned), s));
  unsigned epoch = 0;
  for (int l = 0; l < c.n_layers; l++) {
    SPX_HIP(launch_persist_layer(E->pa, E->players[l], l, epoch, E->persist_grid_n, s));
    epoch += persist_layer_barriers(E->L[l].moe);
  }
  int grid = 1;
  {
    ProfScope ps(E, PC_LMHEAD, wbytes(E->lm_head));
    auto tiles = [](const spx_tensor *t) { int G, R; rp_shape(t->v.nb, G, R); return (int)((t->v.rows + DEC_MV_NW * R - 1) / (DEC_MV_NW * R)); };
    DecMVArgs a{};
    int G, R;
    rp_shape(E->lm_head->v.nb, G, R);
    a.w[0] = E->lm_head->v; a.out[0] = E->logits; a.tiles[0] = tiles(E->lm_head); a.nseg = 1; a.G = G;
    a.in = DecIn{E->xA, E->out_norm, c.rms_eps, c.dim};
    a.best = E->best; a.lscale = c.logit_scale; a.xn_out = E->xn;
    grid = std::min(a.tiles[0], E->lm_dec_grid);
    SPX_HIP(launch_dec_mv(a, grid, s));
  }
  E->nbest = grid;
  {
    ProfScope ps(E, PC_ARGMAX, 0);
    SPX_HIP(launch_argmax_final(E->best, grid, E->amax, E->st_dev, advance ? E->hist : nullptr, 1, s));
  }
  return 0;
}

bool persist_used(const spx_engine *E, int m) {
  return m == 1 && E->dec_ok && E->dec_on && E->persist_ok && E->persist_on && !E->profiling && !E->dbg_on;
}

// After a synchronised pass on the persistent kernel: a barrier that timed out voids the pass;
// the engine then falls back to the decode pipeline for good.
int persist_check(spx_engine *E) {
  if (*E->perr_host == 0) return 0;
  *E->perr_host = 0;
  (void)hipMemsetAsync(E->pa.err, 0, sizeof(int), E->ctx->stream);
  E->persist_ok = false;
  return fail("persistent decode pass: a device-wide barrier timed out, the pass is void; one-row passes run on the decode "
              "pipeline from now on");
}

// Graph slot m (1..16): a pass of m rows; slot 0: a one-row decode pass that advances the
// step record itself (back-to-back greedy decoding without host round trips).
void drop_graphs(spx_engine *E) {
  for (auto &row : E->graph)
    for (auto &g : row)
      if (g) { (void)hipGraphExecDestroy(g); g = nullptr; }
}

int run_forward(spx_engine *E, int m, bool advance = false) {
  hipStream_t s = E->ctx->stream;
  const bool dec = E->dec_ok && E->dec_on;
  if (persist_used(E, m)) return enqueue_persist(E, advance);
  auto enqueue = [&]() {
    if (!dec) return enqueue_forward(E, m, advance);
    if (m == 1) return enqueue_decode(E, advance);
    return m == 2 && E->dec2 && !E->dbg_on ? enqueue_decode(E, false, 2) : enqueue_pass_m(E, m);
  };
  if (!E->use_graphs || E->profiling || E->dbg_on) return enqueue();
  const int slot = advance ? 0 : m;
  hipGraphExec_t &gx = E->graph[advance ? 0 : E->lm_sel][slot];
  if (!gx) {
    SPX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int r = enqueue();
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (r) { if (g) (void)hipGraphDestroy(g); return r; }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&gx, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) { gx = nullptr; return hip_fail(e, "hipGraphInstantiate"); }
  }
  SPX_HIP(hipGraphLaunch(gx, s));
  return 0;
}

}  // namespace

extern "C" {

int spx_engine_create(spx_ctx *ctx, const spx_model_config *cfg, spx_engine **out) {
  if (!ctx || !cfg || !out) return fail("spx_engine_create: null argument");
  const spx_model_config &c = *cfg;
  if (c.dim <= 0 || c.dim > 256 * NORM_NT || c.dim % 16)
    return fail("spx_engine_create: dim must be a positive multiple of 16, at most " + std::to_string(256 * NORM_NT));
  if (c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads) return fail("spx_engine_create: n_heads must be a multiple of n_kv_heads");
  if (c.head_dim != 64 && c.head_dim != 128) return fail("spx_engine_create: the attention kernel supports head_dim 64 or 128");
  if (16 * (c.n_heads / c.n_kv_heads) > ATT_QMAX) return fail("spx_engine_create: at most 8 query heads per kv head");
  if (c.n_layers <= 0 || c.vocab <= 0 || c.max_seq <= 0) return fail("spx_engine_create: bad layer count, vocab or max_seq");
  if (c.max_seq > 64 * ATT_GRP * ATT_GMAX) return fail("spx_engine_create: max_seq above " + std::to_string(64 * ATT_GRP * ATT_GMAX));
  if (c.n_expert < 0 || c.n_expert > 256 || c.n_expert_used < 0 || c.n_expert_used > 32 || (c.n_expert && !c.n_expert_used))
    return fail("spx_engine_create: unsupported expert counts (n_expert <= 256, n_expert_used in 1..32)");
  spx_engine *E = new spx_engine();
  E->ctx = ctx;
  E->c = c;
  if (E->c.embedding_scale == 0.0f) E->c.embedding_scale = 1.0f;
  if (E->c.residual_scale == 0.0f) E->c.residual_scale = 1.0f;
  if (E->c.logit_scale == 0.0f) E->c.logit_scale = 1.0f;
  E->q_dim = c.n_heads * c.head_dim;
  E->kv_dim = c.n_kv_heads * c.head_dim;
  E->L.resize(c.n_layers);
  E->nch = (c.max_seq + 63) / 64;
  {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) E->n_cu = n;
  }
  if (const char *v = std::getenv("SPX_LM_GRID")) E->lm_grid = std::max(1, atoi(v));
  if (const char *v = std::getenv("SPX_LM_DEC_GRID")) E->lm_dec_grid = std::max(1, std::min(atoi(v), 2048));
  if (const char *v = std::getenv("SPX_MV_MODE")) E->mv_mode = std::max(0, std::min(1, atoi(v)));
  if (const char *v = std::getenv("SPX_LM_MODE")) E->lm_mode = std::max(0, std::min(1, atoi(v)));
  if (const char *v = std::getenv("SPX_TAIL_MAX")) E->tail_max = std::max(0, std::min(MAX_M, atoi(v)));
  if (const char *v = std::getenv("SPX_DOWN_MODE")) E->down_mode = std::max(0, std::min(1, atoi(v)));
  if (const char *v = std::getenv("SPX_ATT_MERGE")) E->att_merge = atoi(v) != 0;
  if (const char *v = std::getenv("SPX_PF_ATTN")) E->pf_attn = std::max(0, std::min(4, atoi(v)));
  if (const char *v = std::getenv("SPX_DEC2")) E->dec2 = atoi(v) != 0;
  if (const char *v = std::getenv("SPX_ATT_MT")) E->att_mt_min = std::max(0, std::min(MAX_M + 1, atoi(v)));
  if (const char *v = std::getenv("SPX_PF_MIN")) E->pf_min_rows = std::max(2, std::min(MAX_M + 1, atoi(v)));
  *out = E;
  return 0;
}

int spx_engine_set_tensor(spx_engine *E, const char *name, int dtype, int64_t cols, int64_t rows, int n_expert, const void *data) {
  if (!E || !name || !data) return fail("spx_engine_set_tensor: null argument");
  if (E->prepared) return fail("spx_engine_set_tensor: engine already prepared");
  const std::string n(name);
  SPX_HIP(hipSetDevice(E->ctx->device));
  const bool is_vec = n.find("_norm.weight") != std::string::npos || n.find(".bias") != std::string::npos;
  if (is_vec) {
    if (dtype != T_F32) return fail(n + ": norms and biases must be F32 (resolve_layers, smollm_chat.rs:220-226)");
    const int64_t len = cols * rows * n_expert;
    float *d = E->dalloc<float>((size_t)len);
    if (!d) return fail("out of device memory for " + n);
    SPX_HIP(hipMemcpy(d, data, sizeof(float) * len, hipMemcpyHostToDevice));
    E->vecs[n] = d;
    E->vec_len[n] = len;
    return 0;
  }
  spx_tensor *t = nullptr;
  if (int r = spx_tensor_upload(E->ctx, dtype, cols, rows, n_expert, data, &t)) return r;
  auto it = E->mats.find(n);
  if (it != E->mats.end()) spx_tensor_free(E->ctx, it->second);
  E->mats[n] = t;
  return 0;
}

int spx_engine_prepare(spx_engine *E) {
  if (!E) return fail("spx_engine_prepare: null engine");
  if (E->prepared) return 0;
  auto &c = E->c;
  auto mat = [&](const std::string &n) -> spx_tensor * { auto it = E->mats.find(n); return it == E->mats.end() ? nullptr : it->second; };
  auto vec = [&](const std::string &n, int64_t len) -> const float * {
    auto it = E->vecs.find(n);
    if (it == E->vecs.end() || E->vec_len[n] != len) return nullptr;
    return it->second;
  };
  auto need_mat = [&](const std::string &n, int64_t cols, int64_t rows, int ne, spx_tensor **dst) -> int {
    spx_tensor *t = mat(n);
    if (!t) return fail("missing tensor " + n);
    if (t->v.cols != cols || t->v.rows != rows || t->v.n_expert != ne)
      return fail(n + ": expected " + std::to_string(rows) + "x" + std::to_string(cols) + "x" + std::to_string(ne) + ", got " +
                  std::to_string(t->v.rows) + "x" + std::to_string(t->v.cols) + "x" + std::to_string(t->v.n_expert));
    if (!is_kq(t) && !is_fq(t)) return fail(n + ": weight matrices must be Q4_K, Q6_K, Q8_0, Q5_0 or Q5_K for the GPU kernels");
    *dst = t;
    return 0;
  };
  E->embed = mat("token_embd.weight");
  if (!E->embed || E->embed->v.cols != c.dim || E->embed->v.rows != c.vocab) return fail("missing or misshaped token_embd.weight");
  E->lm_head = mat("output.weight") ? mat("output.weight") : E->embed;  // tied embeddings (:1921)
  if (E->lm_head->v.cols != c.dim || E->lm_head->v.rows != c.vocab) return fail("misshaped output.weight");
  if (!is_kq(E->lm_head) && !is_fq(E->lm_head)) return fail("the LM head must be Q4_K, Q6_K, Q8_0, Q5_0 or Q5_K");
  if (!(E->out_norm = vec("output_norm.weight", c.dim))) return fail("missing output_norm.weight");
  int nff_max = 0;
  for (int l = 0; l < c.n_layers; l++) {
    LayerW &ly = E->L[l];
    const std::string p = "blk." + std::to_string(l) + ".";
    if (!(ly.attn_norm = vec(p + "attn_norm.weight", c.dim))) return fail("missing " + p + "attn_norm.weight");
    if (!(ly.ffn_norm = vec(p + "ffn_norm.weight", c.dim))) return fail("missing " + p + "ffn_norm.weight");
    if (int r = need_mat(p + "attn_q.weight", c.dim, E->q_dim, 1, &ly.wq)) return r;
    if (int r = need_mat(p + "attn_k.weight", c.dim, E->kv_dim, 1, &ly.wk)) return r;
    if (int r = need_mat(p + "attn_v.weight", c.dim, E->kv_dim, 1, &ly.wv)) return r;
    if (int r = need_mat(p + "attn_output.weight", E->q_dim, c.dim, 1, &ly.wo)) return r;
    if (is_kq(ly.wq) != is_kq(ly.wk) || is_kq(ly.wq) != is_kq(ly.wv))
      return fail(p + "attn_q/k/v: integer (Q4_K/Q6_K) and float-activation (Q8_0/Q5_0) formats cannot be mixed");
    ly.q_bias = vec(p + "attn_q.bias", E->q_dim);
    ly.k_bias = vec(p + "attn_k.bias", E->kv_dim);
    ly.v_bias = vec(p + "attn_v.bias", E->kv_dim);
    ly.q_norm = vec(p + "attn_q_norm.weight", c.head_dim);
    ly.k_norm = vec(p + "attn_k_norm.weight", c.head_dim);
    if ((E->vecs.count(p + "attn_q_norm.weight") && !ly.q_norm) || (E->vecs.count(p + "attn_k_norm.weight") && !ly.k_norm))
      return fail(p + "attn_q_norm/attn_k_norm: only per-head norms (head_dim entries) are supported");
    if (mat(p + "ffn_gate_inp.weight")) {
      if (!c.n_expert) return fail("MoE tensors present but expert_count is 0");
      ly.moe = true;
      spx_tensor *r = mat(p + "ffn_gate_inp.weight");
      if (r->v.dtype != T_F32 || r->v.cols != c.dim || r->v.rows != c.n_expert) return fail(p + "ffn_gate_inp.weight: expected F32 " + std::to_string(c.n_expert) + "x" + std::to_string(c.dim));
      ly.router = r;
      spx_tensor *g = mat(p + "ffn_gate_exps.weight");
      if (!g) return fail("missing " + p + "ffn_gate_exps.weight");
      const int64_t nff = g->v.rows;
      if (int rr = need_mat(p + "ffn_gate_exps.weight", c.dim, nff, c.n_expert, &ly.gate)) return rr;
      if (int rr = need_mat(p + "ffn_up_exps.weight", c.dim, nff, c.n_expert, &ly.up)) return rr;
      if (int rr = need_mat(p + "ffn_down_exps.weight", nff, c.dim, c.n_expert, &ly.down)) return rr;
      nff_max = std::max<int>(nff_max, (int)nff);
    } else {
      spx_tensor *g = mat(p + "ffn_gate.weight");
      if (!g) return fail("missing " + p + "ffn_gate.weight");
      const int64_t nff = g->v.rows;
      if (int rr = need_mat(p + "ffn_gate.weight", c.dim, nff, 1, &ly.gate)) return rr;
      if (int rr = need_mat(p + "ffn_up.weight", c.dim, nff, 1, &ly.up)) return rr;
      if (int rr = need_mat(p + "ffn_down.weight", nff, c.dim, 1, &ly.down)) return rr;
      nff_max = std::max<int>(nff_max, (int)nff);
    }
    if (ly.gate->v.dtype != ly.up->v.dtype) return fail(p + "ffn_gate and ffn_up must share a format");
    if (is_kq(ly.down) && ly.gate->v.rows % 256) return fail(p + "a Q4_K/Q6_K ffn_down needs a feed-forward width that is a multiple of 256");
    if (ly.gate->v.rows % 16) return fail(p + "the feed-forward width must be a multiple of 16");
  }
  if (nff_max > 4096) return fail("feed-forward width above 4096");
  E->n_ff = nff_max;
  for (auto &ly : E->L)
    for (spx_tensor *t : {ly.wq, ly.wk, ly.wv, ly.wo, ly.gate, ly.up, ly.down, E->lm_head})
      if (t && is_kq(t) && t->v.cols % 256) return fail("K-quant tensors need cols % 256 == 0");
  // device buffers
  const int M = PMAX, nu = std::max(1, c.n_expert_used), nv = M * nu;
  const int64_t kvn = (int64_t)c.n_layers * c.max_seq * E->kv_dim;
  const int qmax = std::max({c.dim, E->q_dim});
  const int nff = std::max(256, E->n_ff);
  bool ok = (E->kc = E->dalloc<__half>(kvn)) && (E->vc = E->dalloc<__half>(kvn)) &&
            (E->rope = E->dalloc<float2>((size_t)c.max_seq * (c.head_dim / 2))) && (E->st_dev = E->dalloc<StepRec>(1)) &&
            (E->xA = E->dalloc<float>((size_t)M * c.dim)) && (E->xB = E->dalloc<float>((size_t)M * c.dim)) &&
            (E->q = E->dalloc<float>((size_t)M * E->q_dim)) && (E->k = E->dalloc<float>((size_t)M * E->kv_dim)) &&
            (E->v = E->dalloc<float>((size_t)M * E->kv_dim)) && (E->att = E->dalloc<float>((size_t)M * E->q_dim)) &&
            (E->proj = E->dalloc<float>((size_t)M * c.dim)) && (E->ffn = E->dalloc<float>((size_t)M * c.dim)) &&
            (E->xn2 = E->dalloc<float>((size_t)M * qmax)) && (E->xn = E->dalloc<float>((size_t)M * c.dim)) &&
            (E->qp = E->dalloc<float>((size_t)M * E->q_dim)) &&
            (E->h = E->dalloc<float>((size_t)nv * nff)) && (E->yd = E->dalloc<float>((size_t)nv * c.dim)) && (E->rlog = E->dalloc<float>((size_t)M * std::max(1, c.n_expert))) &&
            (E->logits = E->dalloc<float>((size_t)M * c.vocab)) && (E->amax = E->dalloc<int>(M)) &&
            (E->best = E->dalloc<unsigned long long>((size_t)M * std::max<int64_t>(E->lm_grid, c.vocab / 4 + 1))) &&
            (E->tail_cnt = E->dalloc<int>((size_t)(1 + CNT_SUB) * CNT_STRIDE)) && (E->dn_cnt = E->dalloc<int>((size_t)(2 + c.dim / 32) * CNT_STRIDE)) && (E->hist = E->dalloc<int>((size_t)c.max_seq)) &&
            (E->part_ml = E->dalloc<float>((size_t)c.n_kv_heads * (E->nch + ATT_GMAX) * ATT_QMAX * 2)) &&
            (E->part_o = E->dalloc<float>((size_t)c.n_kv_heads * (E->nch + ATT_GMAX) * ATT_QMAX * c.head_dim)) &&
            (E->att_cnt = E->dalloc<int>((size_t)c.n_kv_heads * ATT_QT * (1 + ATT_GMAX) * CNT_STRIDE)) && (E->rt_cnt = E->dalloc<int>((size_t)(1 + CNT_SUB) * CNT_STRIDE)) &&
            (E->gu_cnt = E->dalloc<int>((size_t)MAX_M * nu * (nff / 256 + 1) * (1 + GU_SUB) * CNT_STRIDE)) && (E->chosen = E->dalloc<int>(M * 32)) &&
            (E->nkeep = E->dalloc<int>(M)) && (E->weights = E->dalloc<float>(M * 32)) && (E->jobs = E->dalloc<Job>(512)) &&
            (E->expert_count = E->dalloc<int>((size_t)c.n_layers * std::max(1, c.n_expert))) &&
            E->q8alloc(E->aq, M, ((E->q_dim + 255) / 256) * 256) && E->q8alloc(E->xq2, M, ((c.dim + 255) / 256) * 256) &&
            E->q8alloc(E->xq, M, ((c.dim + 255) / 256) * 256) && E->q8alloc(E->hq, nv, nff) &&
            (E->kv_stage = E->dalloc<__half>((size_t)2 * c.max_seq * E->kv_dim)) && (E->kv_cs = E->dalloc<float2>((size_t)c.head_dim / 2));
  if (!ok) return fail("spx_engine_prepare: out of device memory");
  for (auto &ly : E->L)
    if (ly.moe && !(ly.njobs = E->dalloc<int>(3))) return fail("out of device memory");
  SPX_HIP(hipHostMalloc(&E->st_host, sizeof(StepRec)));
  // RoPE table: inv_freq = 1/theta^(2i/hd) (Rope::new :1399-1402); angle = pos * inv_freq.
  const int half = c.head_dim / 2;
  std::vector<float2> tab((size_t)c.max_seq * half);
  std::vector<float> inv(half);
  for (int i = 0; i < half; i++) inv[i] = 1.0f / powf(c.rope_theta, 2.0f * (float)i / (float)c.head_dim);
  E->inv_freq = inv;
  for (int p = 0; p < c.max_seq; p++)
    for (int i = 0; i < half; i++) {
      const float ang = (float)p * inv[i];
      tab[(size_t)p * half + i] = make_float2(cosf(ang), sinf(ang));
    }
  SPX_HIP(hipMemcpy(E->rope, tab.data(), sizeof(float2) * tab.size(), hipMemcpyHostToDevice));
  SPX_HIP(hipDeviceSynchronize());
  E->n_used = nu;
  // the decode pipeline takes models whose matrices are all K-quants (integer path)
  bool dok = is_kq(E->lm_head) && c.dim % 256 == 0 && E->q_dim % 256 == 0 && c.dim <= 256 * DEC_MAXNB &&
             E->q_dim <= 256 * DEC_MAXNB && E->n_ff <= 256 * DEC_MAXNB;
  for (auto &ly : E->L) {
    for (spx_tensor *t : {ly.wq, ly.wk, ly.wv, ly.wo, ly.gate, ly.up, ly.down}) dok = dok && is_kq(t);
    if (ly.moe) dok = dok && (int64_t)nu * ly.gate->v.rows <= DEC_DOWN_Q;
  }
  E->dec_ok = dok;
  // two-row passes on it: both rows' kept slots in the down kernel's LDS image and row groups
  for (auto &ly : E->L)
    if (ly.moe && (2 * nu > 32 || (int64_t)2 * nu * ly.gate->v.rows > DEC_DOWN_Q)) E->dec2 = false;
  {  // every one-row consumer of a normalised row must be a kernel with the prologue
    auto q8 = [](const spx_tensor *t) { return t->v.dtype == T_Q8_0 && t->v.cols <= 4096; };
    bool fp = !dok && q8(E->lm_head) && c.dim <= 256 * NORM_NT;
    for (auto &ly : E->L) {
      fp = fp && q8(ly.wq) && q8(ly.wk) && q8(ly.wv) && q8(ly.wo) && ly.wk->v.cols == ly.wq->v.cols && ly.wv->v.cols == ly.wq->v.cols;
      fp = fp && !is_kq(ly.gate) && !is_kq(ly.up);
      fp = fp && (ly.moe ? ly.router->v.dtype == T_F32 && !is_kq(ly.down) : q8(ly.down));
    }
    if (const char *v = std::getenv("SPX_FPRO")) fp = fp && atoi(v) != 0;
    E->fpro = fp;
  }
  // passes of 2..16 rows: expert down rows of at most 4 blocks (n_ff <= 1024)
  // the down kernel stages every user's Q8_K h row in LDS: 16 rows x n_used users
  for (auto &ly : E->L) {
    if (ly.moe && (ly.down->v.nb > 4 || downm_lds_bytes((int)ly.down->v.cols) > 64 * 1024)) E->dec_ok = false;
    if (gum_lds_bytes(MAX_M, (int)ly.gate->v.cols, ly.moe ? std::min(MAX_M * nu, c.n_expert) : 1) > 160 * 1024) E->dec_ok = false;
  }
  if (E->dec_ok) {  // the persistent decode pass: per-layer tensor table, barrier words
    std::vector<PLayer> pl(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
      const LayerW &ly = E->L[l];
      PLayer &d = pl[l];
      d.wq = ly.wq->v; d.wk = ly.wk->v; d.wv = ly.wv->v; d.wo = ly.wo->v;
      d.gate = ly.gate->v; d.up = ly.up->v; d.down = ly.down->v;
      if (ly.router) d.router = ly.router->v;
      d.attn_norm = ly.attn_norm; d.ffn_norm = ly.ffn_norm; d.q_norm = ly.q_norm; d.k_norm = ly.k_norm;
      d.q_bias = ly.q_bias; d.k_bias = ly.k_bias; d.v_bias = ly.v_bias;
      d.moe = ly.moe ? 1 : 0;
      d.njobs = ly.njobs;
      d.expert_count = ly.moe ? E->expert_count + (size_t)l * c.n_expert : nullptr;
    }
    E->players = pl;
    unsigned *bar = E->dalloc<unsigned>(PERSIST_BAR_WORDS);
    int *err = E->dalloc<int>(1);
    if (!bar || !err) return fail("out of device memory");
    SPX_HIP(hipHostMalloc(&E->perr_host, sizeof(int)));
    *E->perr_host = 0;
    PersistArgs &a = E->pa;
    a.n_layers = c.n_layers; a.lm_head = E->lm_head->v; a.out_norm = E->out_norm;
    a.dim = c.dim; a.q_dim = E->q_dim; a.kv_dim = E->kv_dim; a.hd = c.head_dim; a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads;
    a.n_ff = E->n_ff; a.n_expert = c.n_expert; a.n_used = nu; a.expert_norm = c.expert_norm; a.moe_prune = c.moe_prune;
    a.eps = c.rms_eps; a.rscale = c.residual_scale; a.lscale = c.logit_scale;
    a.attn_scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt((float)c.head_dim);
    a.neox = c.rope_neox; a.max_seq = c.max_seq; a.nch = E->nch; a.nslot = E->nch + ATT_GMAX;
    a.xa = E->xA; a.xb = E->xB; a.q = E->q; a.k = E->k; a.v = E->v; a.att = E->att; a.h = E->h; a.rlog = E->rlog;
    a.logits = E->logits; a.xn = E->xn; a.part_ml = E->part_ml; a.part_o = E->part_o; a.kc = E->kc; a.vc = E->vc; a.rope = E->rope;
    a.best = E->best; a.chosen = E->chosen; a.nkeep = E->nkeep; a.weights = E->weights; a.st = E->st_dev; a.hist = E->hist;
    a.amax = E->amax; a.bar = bar; a.err = err;
    E->persist_grid_n = persist_grid(c.head_dim, E->n_cu);
    bool uniform = true;  // one feed-forward width for every layer
    for (auto &ly : E->L) uniform = uniform && ly.gate->v.rows == E->n_ff;
    E->persist_ok = uniform && E->persist_grid_n > 0 && persist_fits(a, E->persist_grid_n);
  }
  for (const auto &kv : E->mats) {
    const TensorView &v = kv.second->v;
    if ((v.dtype == T_Q4K || v.dtype == T_Q6K) && !dec_mq_nb_ok((int)v.nb)) E->mq_shapes = false;
  }
  if (const char *v = std::getenv("SPX_PERSIST")) E->persist_on = atoi(v) != 0;
  if (std::getenv("SPX_PERSIST_TSTAMP") && E->dec_ok) E->pa.tstamp = E->dalloc<uint64_t>(4096);
  if (const char *v = std::getenv("SPX_DECODE")) E->dec_on = atoi(v) != 0;
  if (const char *v = std::getenv("SPX_MQ")) E->mq = atoi(v) != 0;
  if (const char *v = std::getenv("SPX_MQ_ROWS")) {
    int k = 0;
    for (const char *p = v; *p && k < spx_engine::MQ_KINDS; k++) {
      E->mq_rows[k] = std::max(2, atoi(p));
      while (*p && *p != ',') p++;
      if (*p == ',') p++;
    }
  }
  E->prepared = true;
  return 0;
}

int spx_engine_set_graphs(spx_engine *E, int on) {
  if (!E) return fail("null engine");
  E->use_graphs = on != 0;
  return 0;
}

int spx_engine_set_decode(spx_engine *E, int on) {
  if (!E) return fail("null engine");
  if (E->dec_on != (on != 0)) {  // the captured graphs hold the other pipeline: capture again
    SPX_HIP(hipStreamSynchronize(E->ctx->stream));
    drop_graphs(E);
  }
  E->dec_on = on != 0;
  return 0;
}

int spx_engine_set_mfma(spx_engine *E, int on) {
  if (!E) return fail("null engine");
  if (E->mq != (on != 0)) {  // the captured multi-row graphs hold the other kernels: capture again
    SPX_HIP(hipStreamSynchronize(E->ctx->stream));
    drop_graphs(E);
  }
  E->mq = on != 0;
  return 0;
}

int spx_engine_decode_pipeline(spx_engine *E, int *active) {
  if (!E || !active) return fail("null argument");
  if (!E->prepared) return fail("spx_engine_decode_pipeline: call spx_engine_prepare first");
  *active = E->dec_ok && E->dec_on ? 1 : 0;
  return 0;
}

int spx_engine_set_persist(spx_engine *E, int on) {
  if (!E) return fail("null engine");
  E->persist_on = on != 0;
  return 0;
}

int spx_engine_persist_active(spx_engine *E, int *active) {
  if (!E || !active) return fail("null argument");
  *active = E->dec_ok && E->dec_on && E->persist_ok && E->persist_on ? 1 : 0;
  return 0;
}

}  // extern "C"

namespace {
// One pass of m rows (spx_engine_forward) with LM-head selection sel (0: every row, 1: the last
// row's logits / pick / normalised row into row 0 of logits / argmax / hidden, 2: none).
int forward_sel(spx_engine *E, const int32_t *ids, int m, int start_pos, float *hidden, float *logits, int32_t *argmax, int sel) {
  if (!E || !ids) return fail("spx_engine_forward: null argument");
  if (m == 1) sel = sel == 2 ? 2 : 0;
  if (!E->prepared) return fail("spx_engine_forward: call spx_engine_prepare first");
  if (m < 1 || m > PMAX) return fail("spx_engine_forward: m must be in 1.." + std::to_string(PMAX));
  if (start_pos < 0 || start_pos + m > E->c.max_seq) return fail("spx_engine_forward: positions beyond max_seq (the KV window is full)");
  for (int i = 0; i < m; i++)
    if (ids[i] < 0 || ids[i] >= E->c.vocab) return fail("spx_engine_forward: token id out of range");
  if (m > MAX_M && !(E->dec_ok && E->dec_on && E->mq && E->mq_shapes)) {
    // no prefill kernels for this model / setting: passes of at most 16 rows, one after the
    // other (a row's results do not depend on the rows that share its pass)
    for (int r0 = 0; r0 < m; r0 += MAX_M) {
      const int n = std::min(MAX_M, m - r0);
      if (sel) {  // feed: only the last pass's last row
        const bool fin = r0 + n == m;
        if (int r = forward_sel(E, ids + r0, n, start_pos + r0, fin ? hidden : nullptr, fin ? logits : nullptr, fin ? argmax : nullptr,
                                fin ? sel : 2))
          return r;
        continue;
      }
      if (int r = forward_sel(E, ids + r0, n, start_pos + r0, hidden ? hidden + (int64_t)r0 * E->c.dim : nullptr,
                              logits ? logits + (int64_t)r0 * E->c.vocab : nullptr, argmax ? argmax + r0 : nullptr, 0))
        return r;
    }
    return 0;
  }
  hipStream_t s = E->ctx->stream;
  SPX_HIP(hipSetDevice(E->ctx->device));
  SPX_HIP(hipStreamSynchronize(s));
  E->st_host->m = m;
  E->st_host->start = start_pos;
  E->st_host->step = 0;
  for (int i = 0; i < m; i++) E->st_host->ids[i] = ids[i];
  E->last_m = m;
  SPX_HIP(hipMemcpyAsync(E->st_dev, E->st_host, sizeof(StepRec), hipMemcpyHostToDevice, s));
  E->lm_sel = sel;
  const int rf = run_forward(E, m);
  E->lm_sel = 0;
  if (rf) return rf;
  const int nr = sel ? 1 : m;  // rows copied out (sel 1: the last row's, at row 0; the decode pipeline's norm writes row 0)
  const int64_t hrow = sel && !(E->dec_ok && E->dec_on) ? m - 1 : 0;
  if (sel != 2) {
    if (hidden) SPX_HIP(hipMemcpyAsync(hidden, E->xn + hrow * E->c.dim, sizeof(float) * nr * E->c.dim, hipMemcpyDeviceToHost, s));
    if (logits) SPX_HIP(hipMemcpyAsync(logits, E->logits, sizeof(float) * nr * E->c.vocab, hipMemcpyDeviceToHost, s));
    if (argmax) SPX_HIP(hipMemcpyAsync(argmax, E->amax, sizeof(int) * nr, hipMemcpyDeviceToHost, s));
  }
  const bool pers = persist_used(E, m);
  if (pers) SPX_HIP(hipMemcpyAsync(E->perr_host, E->pa.err, sizeof(int), hipMemcpyDeviceToHost, s));
  SPX_HIP(hipStreamSynchronize(s));
  if (pers)
    if (int r = persist_check(E)) return r;
  if (E->profiling && !E->prof.empty()) {
    std::vector<int32_t> nj(E->c.n_layers, 0);  // experts run per layer (their slabs' bytes)
    for (int l = 0; l < E->c.n_layers; l++)
      if (E->L[l].moe) SPX_HIP(hipMemcpy(&nj[l], E->L[l].njobs + (m > MAX_M ? 2 : 0), sizeof(int), hipMemcpyDeviceToHost));
    const int64_t kv_pos_bytes = (int64_t)E->kv_dim * 2 * 2;  // K and V, f16
    for (auto &r : E->prof) {
      float ms = 0.0f;
      SPX_HIP(hipEventElapsedTime(&ms, r.a, r.b));
      double bytes = r.bytes;
      if (r.per_expert) bytes = r.bytes * nj[r.layer];  // one expert's slab per selected expert
      if (r.cls == PC_ATTN) bytes = (double)kv_pos_bytes * (start_pos + m);  // KV bytes read once per pass
      E->prof_us[r.cls] += 1000.0 * ms;
      E->prof_bytes[r.cls] += bytes;
      E->prof_n[r.cls] += 1;
    }
    E->prof.clear();
    E->ev_next = 0;
  }
  return 0;
}

}  // namespace

extern "C" {

int spx_engine_forward(spx_engine *E, const int32_t *ids, int m, int start_pos, float *hidden, float *logits, int32_t *argmax) {
  return forward_sel(E, ids, m, start_pos, hidden, logits, argmax, 0);
}

int spx_engine_feed(spx_engine *E, const int32_t *ids, int n, int start_pos, float *hidden_last, float *logits_last, int32_t *argmax_last) {
  if (!E || !ids) return fail("spx_engine_feed: null argument");
  if (n < 1) return fail("spx_engine_feed: n must be at least 1");
  for (int s0 = 0; s0 < n; s0 += PMAX) {
    const int cnt = std::min(PMAX, n - s0);
    const bool fin = s0 + cnt == n;
    if (int r = forward_sel(E, ids + s0, cnt, start_pos + s0, fin ? hidden_last : nullptr, fin ? logits_last : nullptr,
                            fin ? argmax_last : nullptr, fin ? 1 : 2))
      return r;
  }
  return 0;
}

int spx_engine_profile(spx_engine *E, int on) {
  if (!E) return fail("null engine");
  E->profiling = on != 0;
  if (on) { for (int i = 0; i < PROF_NCLS; i++) { E->prof_us[i] = 0; E->prof_bytes[i] = 0; E->prof_n[i] = 0; } }
  return 0;
}

int spx_engine_profile_read(spx_engine *E, int cls, const char **name, int64_t *launches, double *total_us, double *bytes) {
  if (!E || cls < 0 || cls >= PROF_NCLS) return fail("spx_engine_profile_read: bad class");
  if (name) *name = PROF_NAMES[cls];
  if (launches) *launches = E->prof_n[cls];
  if (total_us) *total_us = E->prof_us[cls];
  if (bytes) *bytes = E->prof_bytes[cls];
  return 0;
}

int spx_engine_decode(spx_engine *E, int32_t token, int start_pos, int n, int32_t *out) {
  if (!E || !out || n < 0) return fail("spx_engine_decode: bad argument");
  if (!E->use_graphs || E->profiling || E->dbg_on) {
    int32_t tok = token;
    for (int i = 0; i < n; i++) {  // step_token (:3106-3132) + greedy sample, one token per pass
      int32_t am = 0;
      if (int r = spx_engine_forward(E, &tok, 1, start_pos + i, nullptr, nullptr, &am)) return r;
      out[i] = am;
      tok = am;
    }
    return 0;
  }
  // the same passes replayed back to back: each pass's pick becomes the next pass's token on
  // the device (the step record advances), the picks are copied out once at the end
  if (!E->prepared) return fail("spx_engine_decode: call spx_engine_prepare first");
  if (token < 0 || token >= E->c.vocab) return fail("spx_engine_decode: token id out of range");
  if (start_pos < 0 || start_pos + n > E->c.max_seq) return fail("spx_engine_decode: positions beyond max_seq (the KV window is full)");
  if (n == 0) return 0;
  hipStream_t s = E->ctx->stream;
  SPX_HIP(hipSetDevice(E->ctx->device));
  SPX_HIP(hipStreamSynchronize(s));
  E->st_host->m = 1;
  E->st_host->start = start_pos;
  E->st_host->ids[0] = token;
  E->st_host->step = 0;
  E->last_m = 1;
  SPX_HIP(hipMemcpyAsync(E->st_dev, E->st_host, sizeof(StepRec), hipMemcpyHostToDevice, s));
  const bool pers = persist_used(E, 1);
  for (int i = 0; i < n; i++)
    if (int r = run_forward(E, 1, true)) return r;
  SPX_HIP(hipMemcpyAsync(out, E->hist, sizeof(int32_t) * n, hipMemcpyDeviceToHost, s));
  if (pers) SPX_HIP(hipMemcpyAsync(E->perr_host, E->pa.err, sizeof(int), hipMemcpyDeviceToHost, s));
  SPX_HIP(hipStreamSynchronize(s));
  if (pers)
    if (int r = persist_check(E)) return r;
  return 0;
}

int spx_engine_debug_read(spx_engine *E, const char *what, void *host, int64_t bytes) {
  if (!E || !what || !host) return fail("null argument");
  const std::string w(what);
  if (w == "sampler_rng") {  // the engine sampler's SplitMix64 state (host memory)
    if (!E->smp || bytes != 8) return fail("spx_engine_debug_read: no sampler, or bytes != 8");
    memcpy(host, &E->smp->rng, 8);
    return 0;
  }
  if (w == "layers") {
    if (!E->dbg) return fail("spx_engine_debug_read: layer snapshots are off (spx_engine_debug_layers)");
    const int64_t have = (int64_t)(E->c.n_layers + 1) * MAX_M * E->dbg_off[DBG_NF] * 4;
    if (bytes > have) return fail("spx_engine_debug_read: the layer record holds " + std::to_string(have) + " bytes");
    SPX_HIP(hipStreamSynchronize(E->ctx->stream));
    SPX_HIP(hipMemcpy(host, E->dbg, (size_t)bytes, hipMemcpyDeviceToHost));
    return 0;
  }
  const void *src = w == "tstamp" ? (const void *)E->pa.tstamp : w == "x" ? (const void *)E->xA : w == "xn" ? (const void *)E->xn : w == "q" ? (const void *)E->q : w == "k" ? (const void *)E->k : w == "v" ? (const void *)E->v
                  : w == "att" ? (const void *)E->att : w == "proj" ? (const void *)E->proj : w == "rlog" ? (const void *)E->rlog
                  : w == "chosen" ? (const void *)E->chosen : w == "weights" ? (const void *)E->weights
                  : w == "nkeep" ? (const void *)E->nkeep : w == "h" ? (const void *)E->h : w == "y" ? (const void *)E->ffn : nullptr;
  if (!src) return fail("spx_engine_debug_read: unknown buffer " + w);
  SPX_HIP(hipStreamSynchronize(E->ctx->stream));
  SPX_HIP(hipMemcpy(host, src, (size_t)bytes, hipMemcpyDeviceToHost));
  return 0;
}

int spx_engine_debug_layout(spx_engine *E, int64_t *off) {
  if (!E || !off) return fail("null argument");
  if (!E->prepared) return fail("spx_engine_debug_layout: call spx_engine_prepare first");
  const auto &c = E->c;
  int64_t nff = 0;
  for (const auto &ly : E->L) nff = std::max<int64_t>(nff, ly.gate->v.rows);
  const int64_t len[DBG_NF] = {c.dim, E->q_dim, E->kv_dim, E->kv_dim, E->q_dim, c.dim, c.dim, std::max(1, c.n_expert),
                               std::max(1, E->n_used) * nff, 32, 32, 1};
  int64_t o = 0;
  for (int f = 0; f < DBG_NF; f++) { off[f] = o; o += len[f]; }
  off[DBG_NF] = o;
  return 0;
}

int spx_engine_debug_layers(spx_engine *E, int on) {
  if (!E) return fail("null engine");
  if (!on) { E->dbg_on = false; return 0; }
  if (!E->prepared) return fail("spx_engine_debug_layers: call spx_engine_prepare first");
  if (!(E->dec_ok && E->dec_on)) return fail("spx_engine_debug_layers: layer snapshots need the decode pipelines (a K-quant model)");
  if (int r = spx_engine_debug_layout(E, E->dbg_off)) return r;
  if (!E->dbg && !(E->dbg = E->dalloc<float>((size_t)(E->c.n_layers + 1) * MAX_M * E->dbg_off[DBG_NF])))
    return fail("spx_engine_debug_layers: out of device memory");
  E->dbg_on = true;
  return 0;
}

int spx_engine_last_experts(spx_engine *E, int32_t *njobs_per_layer) {
  if (!E || !njobs_per_layer) return fail("null argument");
  SPX_HIP(hipStreamSynchronize(E->ctx->stream));
  for (int l = 0; l < E->c.n_layers; l++) {
    njobs_per_layer[l] = 0;
    if (E->L[l].moe) SPX_HIP(hipMemcpy(&njobs_per_layer[l], E->L[l].njobs + (E->last_m > MAX_M ? 2 : 0), sizeof(int), hipMemcpyDeviceToHost));
  }
  return 0;
}

int spx_engine_expert_counts(spx_engine *E, int32_t *counts) {
  if (!E || !counts) return fail("null argument");
  SPX_HIP(hipStreamSynchronize(E->ctx->stream));
  SPX_HIP(hipMemcpy(counts, E->expert_count, sizeof(int) * E->c.n_layers * std::max(1, E->c.n_expert), hipMemcpyDeviceToHost));
  return 0;
}

int spx_engine_kv_download(spx_engine *E, void *k_host, void *v_host) {
  if (!E || !k_host || !v_host) return fail("null argument");
  const size_t n = (size_t)E->c.n_layers * E->c.max_seq * E->kv_dim * sizeof(__half);
  SPX_HIP(hipStreamSynchronize(E->ctx->stream));
  SPX_HIP(hipMemcpy(k_host, E->kc, n, hipMemcpyDeviceToHost));
  SPX_HIP(hipMemcpy(v_host, E->vc, n, hipMemcpyDeviceToHost));
  return 0;
}

// ---------------------------------------------------------------- speculation
// lookup_draft (:2982-3015): latest earlier occurrence of the corpus's last n tokens, n from
// max_ngram down to min_ngram; a 2-token match proposes at most 2; drafts stop at stop ids.
int spx_lookup_draft(const int32_t *c, int n, int k, const int32_t *stop, int n_stop, int min_ng, int max_ng, int32_t *draft, int *ngram) {
  *ngram = 0;
  if (k <= 0) return 0;
  for (int ng = max_ng; ng >= min_ng; ng--) {
    if (n <= ng) continue;
    const int32_t *pat = c + n - ng;
    for (int i = n - ng - 1; i >= 0; i--) {
      if (c[i + ng - 1] != pat[ng - 1] || memcmp(c + i, pat, sizeof(int32_t) * ng) != 0) continue;
      const int s = i + ng, kk = ng == 2 ? std::min(k, 2) : k, e = std::min(s + kk, n);
      int len = 0;
      for (int j = s; j < e; j++) {
        bool is_stop = false;
        for (int q = 0; q < n_stop; q++) is_stop |= stop[q] == c[j];
        if (is_stop) break;
        draft[len++] = c[j];
      }
      if (len > 0) { *ngram = ng; return len; }
    }
  }
  return 0;
}

}  // extern "C"

namespace {

constexpr int CORPUS_MAX = 16 * 1024;  // LOOKUP_CORPUS_MAX (:28)

void remember(std::vector<int32_t> &corpus, const int32_t *ids, int n) {
  corpus.insert(corpus.end(), ids, ids + n);
  if ((int)corpus.size() > CORPUS_MAX) corpus.erase(corpus.begin(), corpus.begin() + (corpus.size() - CORPUS_MAX / 2));
}

}  // namespace

extern "C" {

// The attention block of a pass (forward_batch_slice :3226-3300, forward_slice :3432-3470) for
// m rows at start_pos..start_pos+m-1 of layer `layer`: q / k / v are the projections' outputs
// (device [m][q_dim], [m][kv_dim], [m][kv_dim]); biases, Q/K RMSNorm and RoPE are applied here,
// the rows' K / V written to the cache, and each row attends causally to positions <= its own.
int spx_engine_attention(spx_engine *E, int layer, const float *q, const float *k, const float *v, int m, int start_pos, float *att) {
  if (!E || !q || !k || !v || !att) return fail("spx_engine_attention: null argument");
  if (!E->prepared) return fail("spx_engine_attention: call spx_engine_prepare first");
  if (layer < 0 || layer >= E->c.n_layers) return fail("spx_engine_attention: layer out of range");
  if (m < 1 || m > MAX_M || start_pos < 0 || start_pos + m > E->c.max_seq) return fail("spx_engine_attention: rows / positions out of range");
  const auto &c = E->c;
  const LayerW &ly = E->L[layer];
  const int hd = c.head_dim;
  hipStream_t s = E->ctx->stream;
  SPX_HIP(hipSetDevice(E->ctx->device));
  SPX_HIP(hipStreamSynchronize(s));
  E->st_host->m = m;
  E->st_host->start = start_pos;
  E->st_host->step = 0;
  SPX_HIP(hipMemcpyAsync(E->st_dev, E->st_host, sizeof(StepRec), hipMemcpyHostToDevice, s));
  AttnArgs aa{};
  aa.q = q; aa.k = k; aa.v = v;
  aa.q_bias = ly.q_bias; aa.k_bias = ly.k_bias; aa.v_bias = ly.v_bias; aa.q_norm = ly.q_norm; aa.k_norm = ly.k_norm;
  aa.rope = E->rope; aa.kc = E->kc; aa.vc = E->vc; aa.part_ml = E->part_ml; aa.part_o = E->part_o; aa.counter = E->att_cnt; aa.att = att;
  aa.layer = layer; aa.max_seq = c.max_seq; aa.kv_dim = E->kv_dim; aa.hd = hd; aa.n_heads = c.n_heads; aa.n_kv = c.n_kv_heads;
  aa.neox = c.rope_neox; aa.nch = E->nch; aa.nslot = E->nch + ATT_GMAX; aa.eps = c.rms_eps;
  aa.scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt((float)hd);
  SPX_HIP(attn_launch(E, aa, m, s));
  SPX_HIP(hipStreamSynchronize(s));  // the step record is the engine's
  return 0;
}

// shift_kv (:2944-2971): n_discard (at most cur_pos - n_keep) positions after the n_keep pinned
// ones leave the window; the rest move down with their keys re-rotated by -n_discard.
int spx_engine_shift_kv(spx_engine *E, int n_keep, int n_discard, int cur_pos, int *new_pos) {
  if (!E || !new_pos) return fail("spx_engine_shift_kv: null argument");
  if (!E->prepared) return fail("spx_engine_shift_kv: call spx_engine_prepare first");
  if (n_keep < 0 || cur_pos < 0 || cur_pos > E->c.max_seq || n_discard < 0) return fail("spx_engine_shift_kv: bad positions");
  const int n_ctx = cur_pos > n_keep ? cur_pos - n_keep : 0;
  n_discard = std::min(n_discard, n_ctx);
  *new_pos = cur_pos;
  if (n_discard == 0) return 0;
  const auto &c = E->c;
  SPX_HIP(hipSetDevice(E->ctx->device));
  if (!E->kv_stage || !E->kv_cs) return fail("spx_engine_shift_kv: no staging rows (engine not prepared)");
  // Rope::rotate's angle (pos * inv_freq, f32) at pos = -n_discard, sin / cos in f32
  const int half = c.head_dim / 2;
  std::vector<float2> cs(half);
  for (int i = 0; i < half; i++) {
    const float ang = -(float)n_discard * E->inv_freq[i];
    cs[i] = make_float2(cosf(ang), sinf(ang));
  }
  hipStream_t s = E->ctx->stream;
  SPX_HIP(hipMemcpyAsync(E->kv_cs, cs.data(), sizeof(float2) * half, hipMemcpyHostToDevice, s));
  // one layer at a time through one layer's staging rows (allocated by spx_engine_prepare: a
  // slide in the middle of a generation allocates nothing)
  for (int l = 0; l < c.n_layers; l++) {
    KVShiftArgs a{};
    a.kc = E->kc + (size_t)l * c.max_seq * E->kv_dim; a.vc = E->vc + (size_t)l * c.max_seq * E->kv_dim;
    a.kt = E->kv_stage; a.vt = E->kv_stage + (size_t)c.max_seq * E->kv_dim;
    a.cs = E->kv_cs;
    a.n_layers = 1; a.max_seq = c.max_seq; a.kv_dim = E->kv_dim; a.head_dim = c.head_dim; a.neox = c.rope_neox;
    a.n_keep = n_keep; a.n_discard = n_discard; a.n_move = n_ctx - n_discard;
    SPX_HIP(launch_kv_shift(a, s));
  }
  SPX_HIP(hipStreamSynchronize(s));  // the host copy of cs goes out of scope
  *new_pos = cur_pos - n_discard;
  return 0;
}

// ensure_kv_room (:2924-2940): when cur_pos + needed passes max_seq, slides the window by the
// overflow or half the unpinned context, whichever is more (at most all of it).
int spx_engine_ensure_kv_room(spx_engine *E, int n_keep, int cur_pos, int needed, int *new_pos) {
  if (!E || !new_pos) return fail("spx_engine_ensure_kv_room: null argument");
  if (needed < 0 || cur_pos < 0) return fail("spx_engine_ensure_kv_room: bad positions");
  *new_pos = cur_pos;
  if (cur_pos + needed <= E->c.max_seq) return 0;
  const int n_ctx = cur_pos - n_keep;
  const int want = std::max(cur_pos + needed - E->c.max_seq, n_ctx / 2);
  if (int r = spx_engine_shift_kv(E, n_keep, std::min(want, std::max(n_ctx, 0)), cur_pos, new_pos)) return r;
  if (*new_pos + needed > E->c.max_seq) return fail("spx_engine_ensure_kv_room: the pinned positions leave no room");
  return 0;
}

int spx_engine_set_draft(spx_engine *E, spx_engine *D) {
  if (!E) return fail("spx_engine_set_draft: null engine");
  if (D == E) return fail("spx_engine_set_draft: an engine cannot draft for itself");
  if (D && D->c.vocab != E->c.vocab) return fail("spx_engine_set_draft: the draft model needs the same vocabulary");
  E->draft = D;
  return 0;
}

int spx_engine_set_sampler(spx_engine *E, const spx_sampler_params *p) {
  if (!E) return fail("spx_engine_set_sampler: null engine");
  if (!p) {
    E->smp.reset();
    return 0;
  }
  std::unique_ptr<spx::Sampler> s(new (std::nothrow) spx::Sampler());
  if (!s) return fail("spx_engine_set_sampler: out of memory");
  if (int r = s->init(p, E->c.vocab, E->ctx->device, E->ctx->stream)) return r;
  E->smp = std::move(s);
  return 0;
}

// generate_reply's speculative loop (:4205-4348) without chat framing: greedy decoding of up
// to max_new tokens after the prompt. Invariant at the top of the loop: `tok` is sampled but
// not yet in the KV cache; a verify pass feeds [tok, drafts...], the longest matching prefix
// of drafts is accepted, and the first mismatch (or the bonus token) becomes the next tok.
int spx_engine_generate(spx_engine *E, const int32_t *prompt, int n_prompt, int max_new, const spx_gen_params *p, int32_t *out,
                        spx_gen_stats *st) {
  if (!E || !prompt || !p || !out || !st) return fail("spx_engine_generate: null argument");
  if (n_prompt < 1 || max_new < 1) return fail("spx_engine_generate: empty prompt or max_new < 1");
  const int chunk = p->prefill_chunk > 0 ? p->prefill_chunk : PMAX;  // feed's chunks of 128 (:3090)
  if (chunk > PMAX) return fail("spx_engine_generate: prefill_chunk must be at most " + std::to_string(PMAX));
  if (p->kv_keep < 0 || p->kv_keep + std::max(chunk, MAX_M) + MAX_M > E->c.max_seq)
    return fail("spx_engine_generate: kv_keep must leave room for a prompt chunk and a pass");
  if (p->speculate && (p->draft_len < 1 || p->draft_len > MAX_M - 1)) return fail("spx_engine_generate: draft_len must be in 1..15");
  if (p->n_cached < 0 || p->n_cached >= n_prompt) return fail("spx_engine_generate: n_cached must be in 0..n_prompt-1");
  memset(st, 0, sizeof(*st));
  std::vector<int32_t> corpus;
  remember(corpus, prompt, n_prompt);
  int pos = p->n_cached;
  int32_t am[PMAX];
  int64_t t0 = now_us();
  for (int s = p->n_cached; s < n_prompt; s += chunk) {  // feed (:3041-3104): the last row's logits only
    const int cnt = std::min(chunk, n_prompt - s);
    if (int r = spx_engine_ensure_kv_room(E, p->kv_keep, pos, cnt, &pos)) return r;  // feed (:3089-3090)
    if (int r = forward_sel(E, prompt + s, cnt, pos, nullptr, nullptr, am, s + cnt == n_prompt ? 1 : 2)) return r;
    pos += cnt;
  }
  // a draft model is fed the same turn (:4141-4143); drafting stops for the reply once either
  // engine's window slides after this point (kv_shifts checks :4245, :4255)
  spx_engine *D = E->draft;
  int d_pos = p->n_cached;
  bool shifted = false;
  if (D) {
    int32_t dam[PMAX];
    for (int s = p->n_cached; s < n_prompt; s += chunk) {
      const int cnt = std::min(chunk, n_prompt - s);
      if (int r = spx_engine_ensure_kv_room(D, p->kv_keep, d_pos, cnt, &d_pos)) return r;
      if (int r = forward_sel(D, prompt + s, cnt, d_pos, nullptr, nullptr, dam, 2)) return r;
      d_pos += cnt;
    }
  }
  st->prefill_us = (double)(now_us() - t0);
  const int reply_start = pos;
  // pos = ensure_kv_room(pos, need), noting a slide of the target's window
  auto room = [&](int need) -> int {
    const int before = pos;
    if (int r = spx_engine_ensure_kv_room(E, p->kv_keep, pos, need, &pos)) return r;
    if (pos < before) shifted = true;
    return 0;
  };
  spx::Sampler *dsmp = D && D->smp && !D->smp->greedy_plain() ? D->smp.get() : nullptr;
  // the sampler (sample_next_token / sample_from_batch :3574-3621) over the tokens of this
  // reply, stop ids forbidden while fewer than 2 are out (:4220); without one, the greedy picks
  spx::Sampler *smp = E->smp && !E->smp->greedy_plain() ? E->smp.get() : nullptr;
  const int32_t *stop = smp ? smp->stop.data() : nullptr;
  const int n_stop = smp ? (int)smp->stop.size() : 0;
  const int V = E->c.vocab;
  const float lsc = E->c.logit_scale;
  int gen = 0;
  int tok = am[0];  // (the last prompt row's pick; its logits are row 0)
  if (smp) {
    if (int r = smp->prepare(E->logits, V, 1, lsc, out, 0, 1u, false)) return r;
    tok = smp->pick(0);
  }
  int backoff = 0, skip = 0, k_dyn = p->draft_len;
  spx::SpecModel sm;
  sm.fixed = p->fixed != 0;
  for (;;) {
    bool is_stop = false;
    for (int i = 0; i < n_stop; i++) is_stop |= stop[i] == tok;
    if (is_stop) break;  // :4226
    out[gen++] = tok;  // emit!
    remember(corpus, &tok, 1);
    if (gen >= max_new) break;
    const int budget = max_new - gen, k = std::min(k_dyn, budget - 1);
    int32_t draft[MAX_M];
    int nd = 0, cls = 3;
    const bool use_lookup = p->speculate && !D;
    if (k > 0 && (skip == 0 || use_lookup)) {
      if (D) {  // draft_engine (:4244-4269)
        if (!shifted && d_pos >= reply_start) {
          // catch the draft model up on the committed tokens it has not seen (tok at least),
          // then let it autoregress k proposals (its own greedy pick or sampler, no penalty)
          bool have = false, dshift = false;
          int32_t dam[MAX_M];
          auto dstep = [&](int32_t t) -> int {
            const int before = d_pos;
            if (int r = spx_engine_ensure_kv_room(D, p->kv_keep, d_pos, 1, &d_pos)) return r;
            if (d_pos < before) dshift = true;
            if (int r = spx_engine_forward(D, &t, 1, d_pos, nullptr, nullptr, dam)) return r;
            d_pos++;
            return 0;
          };
          for (int i = std::min(d_pos - reply_start, gen); i < gen; i++) {
            if (int r = dstep(out[i])) return r;
            have = true;
          }
          const int32_t *dstop = dsmp ? dsmp->stop.data() : nullptr;
          const int n_dstop = dsmp ? (int)dsmp->stop.size() : 0;
          for (int j = 0; have && !dshift && j < std::min(k, MAX_M - 1); j++) {
            int32_t x = dam[0];
            if (dsmp) {
              if (int r = dsmp->prepare(D->logits, D->c.vocab, 1, D->c.logit_scale, nullptr, 0, 0u, false)) return r;
              x = dsmp->pick(0);
            }
            bool ds = false;
            for (int q = 0; q < n_dstop; q++) ds |= dstop[q] == x;
            if (ds) break;
            draft[nd++] = x;
            if (j + 1 < k)
              if (int r = dstep(x)) return r;
          }
          if (dshift) nd = 0, shifted = true;  // the draft's window slid: no drafts from here on
        }
      } else if (use_lookup) {
        int32_t d[MAX_M];
        int ng = 0;
        const int len = spx_lookup_draft(corpus.data(), (int)corpus.size(), std::min(k, MAX_M - 1), stop, n_stop, p->min_ngram, p->max_ngram, d, &ng);
        if (skip == 0 || ng > 2) { memcpy(draft, d, sizeof(int32_t) * len); nd = len; cls = spx::SpecModel::cls(ng); }
      }
    }
    nd = sm.best_len(cls, nd);
    if (skip > 0) skip--;
    if (nd == 0) {
      if (int r = room(1)) return r;  // (:4283)
      const int64_t ts = now_us();
      if (int r = spx_engine_forward(E, &tok, 1, pos, nullptr, nullptr, am)) return r;
      const double us = (double)(now_us() - ts);
      pos++;
      tok = am[0];
      if (smp) {
        if (int r = smp->prepare(E->logits, V, 1, lsc, out, gen, gen < 2 ? 1u : 0u, false)) return r;
        tok = smp->pick(0);
      }
      sm.record_step((uint64_t)us);
      st->steps++;
      st->step_us += us;
      continue;
    }
    int32_t batch[MAX_M];
    batch[0] = tok;
    memcpy(batch + 1, draft, sizeof(int32_t) * nd);
    if (int r = room(nd + 1)) return r;  // (:4298)
    const int start = pos;
    const int64_t tv = now_us();
    if (int r = spx_engine_forward(E, batch, nd + 1, start, nullptr, nullptr, am)) return r;
    const double us = (double)(now_us() - tv);
    sm.record_verify(nd + 1, (uint64_t)us);
    st->verify_us += us;
    st->drafted += nd;
    st->verifies++;
    if (smp) {  // rows 0..nd over the reply + draft[0..i) (sample_from_batch :4311)
      std::vector<int32_t> win(out, out + gen);
      win.insert(win.end(), draft, draft + nd);
      uint32_t fs = 0;
      for (int i = 0; i <= nd; i++)
        if (gen + i < 2) fs |= 1u << i;
      if (int r = smp->prepare(E->logits, V, nd + 1, lsc, win.data(), gen, fs, false)) return r;
    }
    int accepted = 0, correction = -1;
    bool done = false;
    for (int i = 0; i < nd; i++) {
      const int s = smp ? smp->pick(i) : am[i];
      if (s != draft[i]) { correction = s; break; }
      accepted++;
      out[gen++] = s;
      remember(corpus, &s, 1);
      if (gen >= max_new) { done = true; break; }
    }
    st->accepted += accepted;
    sm.record_draft(cls, nd, accepted);
    pos = start + 1 + accepted;
    if (D) d_pos = std::min(d_pos, reply_start + gen);  // (:4334-4336)
    if (done) break;
    if (accepted == 0) { backoff = std::min(std::max(backoff * 2, 1), 16); skip = backoff; }
    else backoff = 0;
    if (p->adaptive_k) k_dyn = accepted == nd ? std::max(std::min(k_dyn + 2, 7), p->draft_len) : p->draft_len;
    tok = correction >= 0 ? correction : smp ? smp->pick(nd) : am[nd];
  }
  return gen;
}

int spx_engine_destroy(spx_engine *E) {
  if (!E) return 0;
  (void)hipSetDevice(E->ctx->device);
  (void)hipStreamSynchronize(E->ctx->stream);
  drop_graphs(E);
  for (auto ev : E->ev_pool) (void)hipEventDestroy(ev);
  for (auto &kv : E->mats) spx_tensor_free(E->ctx, kv.second);
  for (void *p : E->allocs) (void)hipFree(p);
  if (E->st_host) (void)hipHostFree(E->st_host);
  if (E->perr_host) (void)hipHostFree(E->perr_host);
  delete E;
  return 0;
}

}  // extern "C"
