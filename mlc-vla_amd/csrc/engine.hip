// Engine: parameter binding, activation buffers, the ordered kernel sequences of
// prefill / denoise_step_kv / denoise_loop_kv / chunk, hipGraph capture, and the
// exported C ABI (include/mlcvla.h).
#include "kernels.h"
#include "../../include/mlcvla.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <vector>

namespace mlcv {

static thread_local std::string g_err;
void set_error(const std::string& m) { g_err = m; }
const char* get_error() { return g_err.c_str(); }

namespace {

struct Lin {
  const _Float16* w = nullptr;
  const _Float16* wt = nullptr;  // tile-major copy for the prefill's 32-k tiles (TgArgs::bt) or null
  const uint32_t* qw = nullptr;
  const _Float16* qs = nullptr;
  const _Float16* b = nullptr;
  int N = 0, K = 0;
};

struct Layer {
  Lin q[2], k[2], v[2], o[2], gu[2], dn[2], mod_in, mod_post;
  const _Float16* ln_in0 = nullptr;
  const _Float16* ln_post0 = nullptr;
};

struct OpDesc {
  int seg_off = 0, nseg = 0, ntiles = 0, K = 0, epi = 0, seg_tiles = 0;
  int tr = 64, splits = 0;  // weight rows per tile, K slices (0: planner's choice)
  int mg = 1;               // m groups per weight slab (fragment-major 16-row tiles)
  bool q4 = false;
  bool frag = false;  // fragment-major X and weights (16-row tiles)
  bool xrow = false;  // row-major X with M <= 16, fragment-major weights (16-row tiles)
};

// Tiling of the step's layer GEMMs.  With fragment-major operands (M < 64): 16-row tiles
// whose waves load their operand fragments straight into registers; q/k/v, o_proj and
// gate_up take the whole K per workgroup (no split-K exchange), down splits K in 4.
// o_proj (64 weight slabs) shares each slab out over 4 workgroups of one m tile each, so
// that it runs on 256 workgroups with a quarter of X each.  fp16 gate_up runs on 32-row tiles
// (256 workgroups, X loaded once for both slabs: -11 us per step, bit-identical); q4f16_1
// gate_up stays on 16-row tiles (32-row: +5 us).
// Otherwise (M >= 64) the row-major kernels stage X through LDS with 16/32-row tiles.
// Everything else uses 64-row tiles and the planner's split.
struct Tiling {
  int tr, splits;
  int mg = 1;  // m groups: workgroups sharing a weight slab, each with 4 / mg m tiles
};
struct LayerTilings {
  Tiling qkv = {16, 1}, o = {16, 1, 4}, gu = {16, 1}, down = {16, 4};
  Tiling head = {16, 1}, tmlp = {16, 1};  // action_out and the time MLP (16-row tiles)
  Tiling mod = {16, 1};                   // the adaRMS modulation GEMV (16, 32 or 64 rows)
};
constexpr Tiling ROWMAJOR_QKV = {16, 1}, ROWMAJOR_O = {32, 4}, ROWMAJOR_GU = {32, 1}, ROWMAJOR_DOWN = {32, 8};
constexpr int TR_AIN = 32, SPLIT_AIN = 1;
constexpr int ATTN_TARGET = 128;  // workgroups of the step's attention (row blocks x key splits)
constexpr int MOD_SPLITS = 1;   // K slices of the modulation GEMV's 16-row tiles (1: whole K per tile)
// prefetch assignments (which launch of a layer fetches which later operand into the
// memory-side cache): the attention runs on half the CUs for the longest span of the layer
enum : unsigned {
  PF_QKV_KV = 1,       // q/k/v fetches the layer's prefix K / V
  PF_ATTN_O = 2,       // attention fetches the o_proj weights
  PF_ATTN_GU = 4,      // ... the gate_up weights
  PF_ATTN_DOWN = 8,    // ... the down weights
  PF_ATTN_QKV = 16,    // ... the next layer's q/k/v weights
  PF_O_DOWN = 32,      // o_proj fetches the down weights
  PF_DOWN_QKV = 64,    // down fetches the next layer's q/k/v weights
  PF_ATTN_KV = 128,    // attention fetches the next layer's prefix K / V (each line once)
};
constexpr unsigned PF_DEFAULT = PF_ATTN_O | PF_ATTN_GU;

// MLCV_TILING="qkv=16:S[:G],o=TR:S[:G],gu=TR:S[:G],down=TR:S[:G],head=16:S[:G],tmlp=16:S,mod=TR:1"
// overrides the tile rows (16, or 32 for o / gate_up / down), K slices and, for 16-row
// tiles, the m groups (1, 2 or 4) of the fragment-major GEMMs (the time MLP's K slices apply
// to its small-M tiles) for tuning (read at context creation; 0 = planner).
LayerTilings read_tilings(bool q4) {
  LayerTilings lt;
  if (!q4) lt.gu = {32, 1};
  // q4 modulations on 64-row tiles: 4x the weight bytes per workgroup (one tile is only 9 KB of
  // nibbles and scales at 16 rows): 33 vs 39 us per step; fp16 stays on 16 rows (39 vs 62 us)
  if (q4) lt.mod = {64, 1};
  const char* e = std::getenv("MLCV_TILING");
  if (!e) return lt;
  std::string spec(e);
  size_t pos = 0;
  while (pos < spec.size()) {
    size_t end = spec.find(',', pos);
    if (end == std::string::npos) end = spec.size();
    const std::string item = spec.substr(pos, end - pos);
    const size_t eq = item.find('='), colon = item.find(':');
    if (eq != std::string::npos && colon != std::string::npos && colon > eq) {
      const std::string name = item.substr(0, eq);
      const int tr = std::atoi(item.substr(eq + 1, colon - eq - 1).c_str());
      const int sp = std::atoi(item.substr(colon + 1).c_str());
      const size_t colon2 = item.find(':', colon + 1);
      int mg = colon2 == std::string::npos ? 1 : std::atoi(item.substr(colon2 + 1).c_str());
      if (!(mg == 2 || mg == 4) || tr != 16 || name == "tmlp") mg = 1;
      if (name == "mod" && (tr == 16 || tr == 32 || tr == 64)) lt.mod = Tiling{tr, 1};
      else if (tr == 16 || (tr == 32 && (name == "o" || name == "gu" || name == "down"))) {
        Tiling t{tr, sp, mg};
        if (name == "qkv") lt.qkv = t;
        else if (name == "head") lt.head = t;
        else if (name == "tmlp") lt.tmlp = t;
        else if (name == "o") lt.o = t;
        else if (name == "gu") lt.gu = t;
        else if (name == "down") lt.down = t;
      }
    }
    pos = end + 1;
  }
  return lt;
}
constexpr int RSS_COLS = 16;  // residual row statistics: one partial per 16 columns

struct Graph {
  hipGraphExec_t exec = nullptr;
  std::vector<const void*> key;
};

template <typename T>
int dalloc(T** p, size_t count, std::vector<void*>& owned) {
  void* q = nullptr;
  if (count == 0) count = 1;
  MLCV_HIP(hipMalloc(&q, count * sizeof(T)));
  owned.push_back(q);
  *p = reinterpret_cast<T*>(q);
  return 0;
}

}  // namespace

struct Ctx {
  mlcv_config cfg{};
  bool q4 = false;
  int dev = 0;
  int W0, F0, W1, F1, D, H, KV, HD, P, T, A, NS, NM;
  bool bound = false;
  bool use_graph = true, hoist = true;
  bool step_graph = false;  // denoise_step_kv as a graph replay (else direct launches)

  std::vector<Layer> layers;
  Lin final_mod, ain, aout, tin, tout;

  std::vector<void*> owned;       // buffers allocated at create
  std::vector<void*> bind_owned;  // buffers allocated at bind (q4 -> fp16 prefill weights)

  // suffix path
  _Float16 *x16, *q, *k, *v, *attn, *h, *cond, *tmp, *mod, *te, *xin16;
  // pre-scaled adaRMS input [T + 1][W1]: fp16(x * (1 + scale)) of the next norm, its
  // shift in row T (written by the producer of x; used when T < 64)
  _Float16* xu = nullptr;
  bool prescaled = false;
  // fragment-major path: q roped + scaled as fp16 hi/lo in the attention's fragment order
  // (attn_qf_index, zero outside the written rows) and the suffix k roped in fp32
  _Float16* qf = nullptr;
  float* k32 = nullptr;
  int attn_rpad = 64;
  // fragment-major operands for the layer GEMMs (M < 64, widths % 128 == 0): xu, attn
  // and h are [64][K] in the xf_index layout; the action expert's layer and head weights
  // get pre-shuffled copies at bind time
  bool frag = false;
  // the time MLP and modulation GEMVs (M = steps <= 16) on 16-row register-direct tiles
  // with pre-shuffled weights
  bool small_m = false;
  float *x32, *x0, *vout, *cos, *sin, *mask, *rowss;
  int rss_tiles = 1;
  // prefill path
  _Float16 *px, *pxn, *pqkv, *pctx, *ph, *pvalues;
  float *pcos, *psin, *pkeys;
  // the prefill attention's q in fragment order (q_frag_launch; head dims a multiple of 64,
  // else null and the attention ropes the raw q in its loader)
  _Float16* pqf = nullptr;
  // the head_dim-256 prefill attention (attn_prefill.hip: per-chunk K/V images from the layer's
  // writer, 32-row MFMA tiles, splits balanced over the valid chunks and combined in-kernel);
  // MLCV_PF_ATTN=0 runs the general attention instead
  bool pa_on = false;
  bool pf_wtile = true;  // prefill gate_up / down on tile-major weight copies (MLCV_PF_WTILE=0: row-major)
  PaPlan pa{};
  char* pa_img = nullptr;
  _Float16 *pa_qf = nullptr, *pa_part = nullptr;
  float* pa_ml = nullptr;
  unsigned* pa_ctr = nullptr;
  // the joint forward (denoise_step): suffix RoPE tables at positions P..P+T-1, all-valid mask
  float *m0cos = nullptr, *m0sin = nullptr, *m0mask = nullptr;
  // workspaces
  float* skws = nullptr;
  size_t skws_floats = 0;
  float* zero = nullptr;  // 64*64 zero floats, never written
  unsigned* counters = nullptr;
  size_t ncounters = 0;
  float* attn_ws = nullptr;
  // split-K partials and meeting counters of the prefill GEMMs (256-row tiles)
  float* gemm_ws = nullptr;
  size_t gemm_ws_floats = 0;
  unsigned* gemm_sync = nullptr;
  size_t gemm_sync_words = 0;
  // error word of the prefill GEMMs' split-K meetings (pinned host memory; status_dev is its
  // device address), read back by mlcv_sync; meet_polls bounds each meeting's wait
  unsigned* status = nullptr;
  unsigned* status_dev = nullptr;
  unsigned meet_polls = TG_MEET_POLLS;
  bool gemm_small = false;  // MLCV_PREFILL_SMALL_TILES=1: the 128 x 128 tile kernel only
  // prefix K/V chunk images of every layer (built once per call from keys / values)
  char* kvimg = nullptr;
  size_t img_layer_bytes = 0;
  // the enqueued sequence built the images and the attention reads them
  bool use_img = false;
  // MLCV_LOOP_IMG=1: the loop builds the images once and every step reads them.  Off by
  // default: the chunk copy from an image costs about what the conversion of the f32
  // keys costs (both are bound by the chunk's bytes), so the build is pure overhead
  bool loop_img = false;
  size_t attn_ws_floats_n = 0;
  int st_nsplit = 1, st_kps = 32, pf_nsplit = 1, pf_kps = 32;
  // the step attention in the XCD-grouped order: with plain K/V loads the 7 row blocks of a key
  // split share its K/V in one XCD's L2 (step 808 vs 821 us); MLCV_ATTN_XG=0 deals the tasks
  // over the XCDs in grid order instead
  bool attn_xg = true;

  SkSeg* d_segs = nullptr;
  std::vector<SkSeg> h_segs;
  std::vector<OpDesc> layer_ops;  // 4 per layer: qkv, o, gate_up, down
  OpDesc op_tin, op_tout, op_ain, op_aout;
  // for the side stream, the adaRMS modulations in 2 pieces: layer 0's two norms, then every
  // other norm (one launch over a segment table).  With fork_mod the step runs them on `side`
  // so that the second piece streams while layer 0 runs; ops wait for their piece (mod_ev).
  std::vector<OpDesc> mod_ops;
  OpDesc mod_all;  // every modulation in one launch (16-row tiles, used without the side stream)
  hipStream_t side = nullptr;
  hipEvent_t cond_ev = nullptr;
  std::vector<hipEvent_t> mod_ev;
  bool fork_mod = false;
  LayerTilings tilings;  // fragment-major layer GEMM tiles (MLCV_TILING at creation)
  // prefetch of later ops' operands by spare workgroups of the step's launches
  // (fragment-major path), PF_* bits: which launch fetches what
  unsigned prefetch = PF_DEFAULT;
  // prefetch workgroups per hosting launch (more slow the host, fewer stretch it): 80 keeps
  // the warm step and takes 12 us off the cold one against 64; 32 and 160 are much slower
  int pf_blocks = 80;
  float* skws_side = nullptr;  // split-K workspace / counters of the side stream
  unsigned* counters_side = nullptr;
  size_t ncounters_side = 0;

  // persistent step (step_persistent.hip): one launch per step after the modulations, for
  // the fragment-major shapes it is built for; off by default (MLCV_PERSIST=1 or
  // MLCV_OPT_PERSIST turns it on); activations are per layer so every launch writes each
  // buffer once
  bool pk_ok = false;   // the shapes allow it (decided at create)
  bool pk_on = false;   // ... and it is enabled
  PkArgs pk{};          // buffers, dims and plan; weights filled at bind
  PkLin* d_pklin = nullptr;
  // XCD tensor-parallel step (step_xtp.hip): two launches per layer for the pi0.5 action
  // expert's shape on a part of 8 XCDs x 32 CUs; on by default where it applies (MLCV_XTP=0 or
  // MLCV_OPT_XTP = 0 turns it off); activations are per layer and XCD
  bool xt_ok = false;  // the shapes and the device allow it (decided at create)
  bool xt_on = false;  // ... and it is enabled
  bool attn_noskip = false;  // MLCV_OPT_MASK_SKIP = 0: the attentions compute fully masked key chunks too
  XtArgs xt{};         // buffers and dims; weights filled at bind
  float* nscale = nullptr;  // [steps][2D+1] prescale of each norm's pre-scaled input
  _Float16* ain16 = nullptr;  // action_in weights in fp16 (q4 models: dequantized at bind)
  _Float16* aout16 = nullptr;  // action_out weights in fp16 (the XCD step's head; q4: dequantized at bind)

  hipStream_t cap = nullptr;
  Graph g_step, g_loop, g_prefill, g_chunk, g_m0;

  void drop_graphs() {
    for (Graph* g : {&g_step, &g_loop, &g_prefill, &g_chunk, &g_m0}) {
      if (g->exec) (void)hipGraphExecDestroy(g->exec);
      g->exec = nullptr;
      g->key.clear();
    }
  }
  ~Ctx() {
    drop_graphs();
    for (void* p : bind_owned) (void)hipFree(p);
    for (void* p : owned) (void)hipFree(p);
    if (cap) (void)hipStreamDestroy(cap);
    if (side) (void)hipStreamDestroy(side);
    if (cond_ev) (void)hipEventDestroy(cond_ev);
    for (hipEvent_t e : mod_ev)
      if (e) (void)hipEventDestroy(e);
    if (d_segs) (void)hipFree(d_segs);
    if (d_pklin) (void)hipFree(d_pklin);
    if (status) (void)hipHostFree(status);
  }
};

namespace {

size_t kv_slice(const Ctx& c) { return (size_t)c.KV * c.P * c.HD; }

// Workgroup target of the prefill's attention plan: as many key splits as let every workgroup
// (one per CU) run in one round -- at P = 968, 121 row blocks x 2 splits on 256 CUs (-0.18 ms
// against 3 splits in 1.4 rounds); MLCV_PF_ATTN_TARGET sets it instead (tuning).
int prefill_attn_target(int rows) {
  const int rb = (rows + 63) / 64;
  int target = std::max(1, std::max(device_cus(), 1) / rb) * rb;
  if (const char* e = std::getenv("MLCV_PF_ATTN_TARGET"))
    if (std::atoi(e) > 0) target = std::atoi(e);
  return target;
}

SkOp make_op(const Ctx& c, const OpDesc& d, const _Float16* x, int ldx, int M) {
  SkOp op{};
  op.x = x;
  op.ldx = ldx;
  op.M = M;
  op.K = d.K;
  op.eps = c.cfg.rms_norm_eps;
  op.epi = d.epi;
  op.segs = c.d_segs + d.seg_off;
  op.nseg = d.nseg;
  op.seg_tiles = d.seg_tiles;
  for (int i = 0; i < d.nseg && i < 3; ++i) op.inl[i] = c.h_segs[d.seg_off + i];
  op.ntiles = d.ntiles;
  op.tr = d.tr;
  op.mg = d.frag ? d.mg : 1;
  const SkPlan p = sk_plan(d.ntiles, d.K, (M + 63) / 64, d.splits);
  op.splitk = p.splitk;
  op.kper = p.kper;
  op.ws = c.skws;
  op.zero = c.zero;
  op.counters = c.counters;
  op.rowss_ld = c.rss_tiles;
  op.rowss_tiles = c.rss_tiles;
  op.frag = d.frag;
  op.xrow = d.xrow;
  return op;
}

int run_op(const Ctx& c, const OpDesc& d, SkOp op, hipStream_t st) { return sk_launch(op, d.q4, st); }

// ---- time MLP + all adaRMS modulations for M steps --------------------------
// fork: the modulation pieces go to the side stream after the time MLP, each followed by
// its event; the caller waits for piece p (wait_mod) before the first op that reads it.
int enqueue_time_mod(Ctx& c, const _Float16* te, int M, hipStream_t st, bool fork) {
  MLCV_TRY(run_op(c, c.op_tin, make_op(c, c.op_tin, te, c.W1, M), st));
  MLCV_TRY(run_op(c, c.op_tout, make_op(c, c.op_tout, c.tmp, c.W1, M), st));
  if (c.pk_on || c.xt_on) fork = false;  // the one-launch / XCD steps start after every modulation
  hipStream_t ms = st;
  if (fork) {
    MLCV_HIP(hipEventRecord(c.cond_ev, st));
    MLCV_HIP(hipStreamWaitEvent(c.side, c.cond_ev, 0));
    ms = c.side;
  }
  // with each piece of modulations, the power-of-two prescale of its norms' pre-scaled inputs
  // (piece 0: layer 0's two norms; piece 1: the others)
  const bool nsc = c.prescaled || c.pk_on || c.xt_on;
  if (!fork && c.mod_all.nseg > 0) {
    MLCV_TRY(run_op(c, c.mod_all, make_op(c, c.mod_all, c.cond, c.W1, M), st));
    if (nsc) MLCV_TRY(nscale_launch(c.mod, c.W1, c.NM, M, 0, c.NM, c.nscale, st));
  } else {
    for (int p = 0; p < (int)c.mod_ops.size(); ++p) {
      SkOp op = make_op(c, c.mod_ops[p], c.cond, c.W1, M);
      if (fork) {
        op.ws = c.skws_side;
        op.counters = c.counters_side;
      }
      MLCV_TRY(run_op(c, c.mod_ops[p], op, ms));
      if (nsc) MLCV_TRY(nscale_launch(c.mod, c.W1, c.NM, M, p == 0 ? 0 : 2, p == 0 ? 2 : c.NM - 2, c.nscale, ms));
      if (fork) MLCV_HIP(hipEventRecord(c.mod_ev[p], ms));
    }
  }
  return 0;
}

// before the first op that reads the modulations of layer p (p == D: the final norm)
int wait_mod(Ctx& c, int p, bool forked, hipStream_t st) {
  if (forked) MLCV_HIP(hipStreamWaitEvent(st, c.mod_ev[p == 0 ? 0 : 1], 0));
  return 0;
}

Tiling tile_qkv(const Ctx& c) { return c.frag ? c.tilings.qkv : ROWMAJOR_QKV; }
Tiling tile_o(const Ctx& c) { return c.frag ? c.tilings.o : ROWMAJOR_O; }
Tiling tile_gu(const Ctx& c) { return c.frag ? c.tilings.gu : ROWMAJOR_GU; }
Tiling tile_down(const Ctx& c) { return c.frag ? c.tilings.down : ROWMAJOR_DOWN; }
Tiling tile_head(const Ctx& c) { return c.frag ? c.tilings.head : Tiling{64, 0}; }

// ---- the ops of one decoder layer of the suffix path (modulations in modp) ------
const _Float16* mod_of(const Ctx& c, const _Float16* modp, int idx) { return modp + (size_t)idx * 3 * c.W1; }

// adaRMS consumer: pre-scaled X (T < 64) or the per-element prologue; m = [scale|shift|gate]
// the prescale of the norm whose modulation vector is m (a norm of c.mod)
const float* nsc_of(const Ctx& c, const _Float16* m) { return c.nscale + (m - c.mod) / (3 * c.W1); }

void set_norm(const Ctx& c, SkOp& op, const _Float16* m) {
  op.rowss_in = c.rowss;
  if (c.prescaled) {
    op.prescaled = true;
    op.nsc = nsc_of(c, m);
  } else {
    op.scale = m;
    op.shift = m + c.W1;
  }
}

// producer of x: also write the next adaRMS's pre-scaled input
void set_next_norm(const Ctx& c, SkOp& op, const _Float16* m) {
  if (!c.prescaled) return;
  op.xu_out = c.xu;
  op.xu_scale = m;
  op.xu_shift = m + c.W1;
  op.xu_nsc = nsc_of(c, m);
  op.frag_out = c.frag;
}

// ---- L2 prefetch descriptors --------------------------------------------------
void pf_add(Prefetch& pf, const void* base, size_t slab_bytes, int nslabs, int xoff, int every_xcd) {
  if (pf.nreg >= PF_MAX_REGIONS || nslabs <= 0 || base == nullptr) return;
  pf.r[pf.nreg++] = PfRegion{static_cast<const char*>(base), (int)slab_bytes, nslabs, xoff & 7, every_xcd};
}
// the weights of a fragment-major layer op: one tile's slabs (tr / 16 consecutive 16-row
// slabs) per region slab, read by the tile's workgroups on XCD tile % 8
void pf_weights(const Ctx& c, Prefetch& pf, const OpDesc& d, unsigned bit) {
  if (!(c.prefetch & bit) || !d.frag) return;
  pf.nblocks = c.pf_blocks;
  const size_t sl = d.tr / 16;
  for (int i = 0; i < d.nseg; ++i) {
    const SkSeg& sg = c.h_segs[d.seg_off + i];
    const int tiles = (i + 1 < d.nseg ? c.h_segs[d.seg_off + i + 1].tile0 : d.ntiles) - sg.tile0;
    if (d.q4) {
      pf_add(pf, sg.qw, sl * 8 * d.K, tiles, sg.tile0, 0);  // 16 rows x K/8 words per slab
      pf_add(pf, sg.qs, sl * d.K, tiles, sg.tile0, 0);      // 16 rows x K/32 scales per slab
    } else {
      pf_add(pf, sg.w, sl * 32 * d.K, tiles, sg.tile0, 0);  // 16 rows x K halfs per slab
    }
  }
}
// the prefix K / V of layer L (or its chunk images), read by the attention (every XCD
// reads every split's keys: every_xcd fills each XCD's L2, otherwise each line is read once)
void pf_kv(const Ctx& c, Prefetch& pf, int L, const float* keys, const _Float16* values, unsigned bit,
           int every_xcd) {
  if (!(c.prefetch & bit) || !c.frag || keys == nullptr) return;
  pf.nblocks = c.pf_blocks;
  if (c.use_img) {
    const int chunks = (c.P + 31) / 32;
    pf_add(pf, c.kvimg + (size_t)L * c.img_layer_bytes, c.img_layer_bytes / ((size_t)c.KV * chunks), c.KV * chunks,
           0, every_xcd);
  } else {
    const int slabs = (int)(kv_slice(c) / ((size_t)8 * c.HD));  // 8 keys per slab
    pf_add(pf, keys + L * kv_slice(c), (size_t)8 * c.HD * sizeof(float), slabs, 0, every_xcd);
    pf_add(pf, values + L * kv_slice(c), (size_t)8 * c.HD * sizeof(_Float16), slabs, 0, every_xcd);
  }
}

int enqueue_qkv(Ctx& c, int L, const _Float16* modp, hipStream_t st, const float* keys = nullptr,
                const _Float16* values = nullptr) {  // adaRMS (input) + q/k/v
  const _Float16* m_in = mod_of(c, modp, 2 * L);
  SkOp op = make_op(c, c.layer_ops[4 * L + 0], c.prescaled ? c.xu : c.x16, c.W1, c.T);
  pf_kv(c, op.pf, L, keys, values, PF_QKV_KV, 1);
  set_norm(c, op, m_in);
  op.rope_cos = c.cos;
  op.rope_sin = c.sin;
  op.rope_scale = 1.0f / std::sqrt((float)c.HD);
  op.rope_hd = c.HD;
  op.rope_grp = c.H / c.KV;
  op.rope_rpad = c.attn_rpad;
  return run_op(c, c.layer_ops[4 * L + 0], op, st);
}

// the chunk images of every layer's prefix K/V (once per call; read by enqueue_attn)
int enqueue_kv_prep(Ctx& c, const float* keys, const _Float16* values, hipStream_t st) {
  return attn_img_prep_launch(keys, 1, values, c.mask, c.D, c.KV, c.P, c.HD, c.kvimg, st);
}

int enqueue_attn(Ctx& c, int L, const float* keys, const _Float16* values, hipStream_t st) {
  AttnArgs a{};
  a.noskip = c.attn_noskip ? 1 : 0;
  a.q = c.q;
  a.q_ld = c.H * c.HD;
  a.cos = c.cos;
  a.sin = c.sin;
  a.q_scale = 1.0f / std::sqrt((float)c.HD);
  a.Tq = c.T;
  a.H = c.H;
  a.KV = c.KV;
  a.hd = c.HD;
  a.kp = keys + L * kv_slice(c);
  a.kp_f32 = 1;
  a.vp = values + L * kv_slice(c);
  a.Sp = c.P;
  a.mask = c.mask;
  a.ks = c.k;
  a.ks_ld = c.KV * c.HD;
  a.vs = c.v;
  a.vs_ld = c.KV * c.HD;
  a.Ts = c.T;
  a.ks_roped = 0;
  a.out = c.attn;
  a.out_ld = c.H * c.HD;
  a.out_frag = c.frag;
  if (c.frag) {
    a.qf = c.qf;
    a.ks32 = c.k32;
  }
  a.nsplit = c.st_nsplit;
  a.kps = c.st_kps;
  a.kimg = c.use_img ? c.kvimg + (size_t)L * c.img_layer_bytes : nullptr;
  a.img_chunks = (c.P + 31) / 32;
  a.rows = c.T * (c.H / c.KV);
  a.rpad = ((a.rows + 63) / 64) * 64;
  a.part_o = c.attn_ws;
  a.part_ml = c.attn_ws + (size_t)c.KV * a.nsplit * a.rpad * c.HD;
  pf_weights(c, a.pf, c.layer_ops[4 * L + 1], PF_ATTN_O);
  pf_weights(c, a.pf, c.layer_ops[4 * L + 2], PF_ATTN_GU);
  pf_weights(c, a.pf, c.layer_ops[4 * L + 3], PF_ATTN_DOWN);
  if (L + 1 < c.D) pf_weights(c, a.pf, c.layer_ops[4 * (L + 1)], PF_ATTN_QKV);
  if (L + 1 < c.D) pf_kv(c, a.pf, L + 1, keys, values, PF_ATTN_KV, 0);
  a.xgroup = c.attn_xg && a.qf && !a.kimg ? 1 : 0;
  return attn_launch(a, st);
}

int enqueue_oproj(Ctx& c, int L, const _Float16* modp, hipStream_t st) {  // o_proj + gated residual
  SkOp op = make_op(c, c.layer_ops[4 * L + 1], c.attn, c.H * c.HD, c.T);
  op.gate = mod_of(c, modp, 2 * L) + 2 * c.W1;
  op.rowss_out = c.rowss;
  set_next_norm(c, op, mod_of(c, modp, 2 * L + 1));
  pf_weights(c, op.pf, c.layer_ops[4 * L + 3], PF_O_DOWN);
  return run_op(c, c.layer_ops[4 * L + 1], op, st);
}

int enqueue_gateup(Ctx& c, int L, const _Float16* modp, hipStream_t st) {  // adaRMS (post) + gate_up + GeGLU
  const _Float16* m_post = mod_of(c, modp, 2 * L + 1);
  SkOp op = make_op(c, c.layer_ops[4 * L + 2], c.prescaled ? c.xu : c.x16, c.W1, c.T);
  set_norm(c, op, m_post);
  op.geglu_F = c.F1;
  op.frag_out = c.frag;
  return run_op(c, c.layer_ops[4 * L + 2], op, st);
}

int enqueue_down(Ctx& c, int L, const _Float16* modp, hipStream_t st) {  // down + gated residual
  SkOp op = make_op(c, c.layer_ops[4 * L + 3], c.h, c.F1, c.T);
  op.gate = mod_of(c, modp, 2 * L + 1) + 2 * c.W1;
  op.rowss_out = c.rowss;
  set_next_norm(c, op, mod_of(c, modp, L + 1 < c.D ? 2 * (L + 1) : 2 * c.D));
  if (L + 1 < c.D) pf_weights(c, op.pf, c.layer_ops[4 * (L + 1)], PF_DOWN_QKV);
  return run_op(c, c.layer_ops[4 * L + 3], op, st);
}

int enqueue_head(Ctx& c, const _Float16* modp, bool euler, hipStream_t st) {  // final adaRMS + action_out
  const _Float16* m_fin = mod_of(c, modp, 2 * c.D);
  SkOp op = make_op(c, c.op_aout, c.prescaled ? c.xu : c.x16, c.W1, c.T);
  set_norm(c, op, m_fin);
  if (euler) {
    op.epi = EPI_EULER;
    op.dt = (float)(-1.0 / c.NS);
    op.x32 = c.x32;
    op.x16 = c.xin16;
  }
  return run_op(c, c.op_aout, op, st);
}

int enqueue_action_in(Ctx& c, const _Float16* modp, hipStream_t st) {  // action_in_proj -> x, layer 0's norm input
  SkOp ain = make_op(c, c.op_ain, c.xin16, c.A, c.T);
  ain.rowss_out = c.rowss;
  set_next_norm(c, ain, mod_of(c, modp, 0));
  return run_op(c, c.op_ain, ain, st);
}

// the caller's own step inputs and output, read and written in place by the XCD step when it is
// launched directly (no graph holds the pointers); null members: the context's staged copies
struct StepIO {
  const _Float16* x_t = nullptr;
  const float* cos = nullptr;
  const float* sin = nullptr;
  const float* mask = nullptr;
  float* vout = nullptr;
};

// ---- one suffix-only velocity evaluation (modulations already in modp) -------
// forked: the modulation pieces run on the side stream (enqueue_time_mod with fork)
int enqueue_step(Ctx& c, const float* keys, const _Float16* values, const _Float16* modp, bool euler,
                 hipStream_t st, bool forked = false, const StepIO& io = StepIO{}) {
  if (c.xt_on) {
    // the XCD tensor-parallel layers, then the launch chain's head on the residual stream
    XtArgs a = c.xt;
    const size_t mi = (size_t)(modp - c.mod) / ((size_t)3 * c.W1);  // first norm of this step
    a.modp = modp;
    a.nscale = c.nscale + mi;
    a.keys = keys;
    a.values = values;
    a.mask = io.mask ? io.mask : c.mask;
    a.cos = io.cos ? io.cos : c.cos;
    a.sin = io.sin ? io.sin : c.sin;
    a.xin = io.x_t ? io.x_t : c.xin16;
    a.vout_user = io.vout;
    for (int L = 0; L < c.D; ++L) {
      a.L = L;
      MLCV_TRY(xt_attn_launch(a, st));
      MLCV_TRY(xt_mlp_launch(a, st));
    }
    // the final reduce, the final norm and action_out_proj (or the Euler update) in one launch
    a.vout = c.vout;
    a.x32 = c.x32;
    a.xnext = c.xin16;
    a.dt = (float)(-1.0 / c.NS);
    a.euler = euler ? 1 : 0;
    return xt_head_launch(a, st);
  }
  if (c.pk_on) {
    PkArgs p = c.pk;
    const size_t mi = (size_t)(modp - c.mod) / ((size_t)3 * c.W1);  // first norm of this step
    p.modp = modp;
    p.nscale = c.nscale + mi;
    p.keys = keys;
    p.values = values;
    p.mask = c.mask;
    p.cos = c.cos;
    p.sin = c.sin;
    p.xin = c.xin16;
    p.vout = c.vout;
    p.x32 = c.x32;
    p.x16 = c.xin16;
    p.dt = (float)(-1.0 / c.NS);
    p.euler = euler ? 1 : 0;
    return pk_launch(p, c.q4, st);
  }
  MLCV_TRY(wait_mod(c, 0, forked, st));
  MLCV_TRY(enqueue_action_in(c, modp, st));
  for (int L = 0; L < c.D; ++L) {
    MLCV_TRY(enqueue_qkv(c, L, modp, st, keys, values));
    MLCV_TRY(enqueue_attn(c, L, keys, values, st));
    MLCV_TRY(enqueue_oproj(c, L, modp, st));
    MLCV_TRY(enqueue_gateup(c, L, modp, st));
    MLCV_TRY(wait_mod(c, L + 1, forked, st));  // down writes the next norm's input
    MLCV_TRY(enqueue_down(c, L, modp, st));
  }
  return enqueue_head(c, modp, euler, st);
}

// The prefill's attention (attn_prefill_e0, gemma_dual.py:236-253,334-341): q straight from
// the q/k/v GEMM (roped and scaled in the attention's loader), the layer's roped fp32 keys and
// fp16 values from the cache, the prefix pad mask, no suffix block.
AttnArgs prefill_attn_args(const _Float16* q, int q_ld, const float* cos, const float* sin, int P, int H, int KV,
                           int HD, const float* keys, const _Float16* values, const float* mask, _Float16* out,
                           int nsplit, int kps, float* ws) {
  AttnArgs a{};
  a.q = q;
  a.q_ld = q_ld;
  a.cos = cos;
  a.sin = sin;
  a.q_scale = 1.0f / std::sqrt((float)HD);
  a.Tq = P;
  a.H = H;
  a.KV = KV;
  a.hd = HD;
  a.kp = keys;
  a.kp_f32 = 1;
  a.vp = values;
  a.Sp = P;
  a.mask = mask;
  a.Ts = 0;
  a.out = out;
  a.out_ld = H * HD;
  a.nsplit = nsplit;
  a.kps = kps;
  a.rows = P * (H / KV);
  a.rpad = ((a.rows + 63) / 64) * 64;
  a.part_o = ws;
  a.part_ml = ws + (size_t)KV * nsplit * a.rpad * HD;
  return a;
}

// the prefill GEMMs' split-K workspace (shared: the launches are ordered on one stream)
void gemm_ws_args(const Ctx& c, TgArgs& g) {
  g.ws = c.gemm_ws;
  g.ws_floats = c.gemm_ws_floats;
  g.sync = c.gemm_sync;
  g.sync_tiles = (int)(c.gemm_sync_words / 32);
  g.small_tiles = c.gemm_small ? 1 : 0;
  g.err = c.status_dev;
  g.meet_polls = c.meet_polls;
}

PaArgs pa_args(const PaPlan& plan, const _Float16* qf, const char* img, const float* mask, _Float16* out, int out_ld,
               int P, int H, int KV, _Float16* part, float* ml, unsigned* ctr, bool noskip) {
  PaArgs a{};
  a.qf = qf;
  a.img = img;
  a.mask = mask;
  a.out = out;
  a.out_ld = out_ld;
  a.P = P;
  a.H = H;
  a.KV = KV;
  a.rows = P * (H / KV);
  a.nch = plan.nch;
  a.nrb = plan.nrb;
  a.nsplit = plan.nsplit;
  a.part = part;
  a.part_ml = ml;
  a.ctr = ctr;
  a.noskip = noskip ? 1 : 0;
  // MLCV_PA_DEV_COMBINE=1: the device-scope combine (the path taken when a split runs on another
  // XCD than the dispatch order places it on), for the tests
  const char* dc = std::getenv("MLCV_PA_DEV_COMBINE");
  a.dev_combine = dc && std::atoi(dc) != 0 ? 1 : 0;
  return a;
}

// ---- prefill: expert-0 over the prefix, K/V written per layer ----------------
int enqueue_prefill(Ctx& c, float* keys, _Float16* values, hipStream_t st) {
  const int W0 = c.W0, P = c.P, HD = c.HD;
  const int nq = c.H * HD, nkv = c.KV * HD, nqkv = nq + 2 * nkv;
  for (int L = 0; L < c.D; ++L) {
    const Layer& ly = c.layers[L];
    float* kL = keys + L * kv_slice(c);
    _Float16* vL = values + L * kv_slice(c);
    MLCV_TRY(rmsnorm_launch(c.px, ly.ln_in0, c.pxn, P, W0, c.cfg.rms_norm_eps, st));
    TgArgs g{};
    g.a = c.pxn;
    g.lda = W0;
    g.b0 = ly.q[0].w;
    g.b1 = ly.k[0].w;
    g.b2 = ly.v[0].w;
    g.n1 = nq;
    g.n2 = nq + nkv;
    g.ldb = W0;
    g.c = c.pqkv;
    g.ldc = nqkv;
    g.M = P;
    g.N = nqkv;
    g.K = W0;
    g.epi = TG_STORE;
    gemm_ws_args(c, g);
    MLCV_TRY(tg_launch(g, st));
    // the cache slices of this layer, and (but for the last layer, whose attention feeds no
    // output) q roped, scaled and split into the attention's fragment order, in one launch
    const bool last = L == c.D - 1;
    if (c.pa_on && !last) {
      MLCV_TRY(pa_writer_launch(c.pqkv, nqkv, nq, nq + nkv, c.pcos, c.psin, P, c.H, c.KV, 1.0f / std::sqrt((float)HD),
                                kL, vL, c.pa, c.pa_img, c.pa_qf, 0, st));
      MLCV_TRY(pa_attn_launch(pa_args(c.pa, c.pa_qf, c.pa_img, c.mask, c.pctx, c.H * HD, P, c.H, c.KV, c.pa_part,
                                      c.pa_ml, c.pa_ctr, c.attn_noskip),
                              st));
    } else {
      AttnArgs pa = prefill_attn_args(c.pqkv, nqkv, c.pcos, c.psin, P, c.H, c.KV, HD, kL, vL, c.mask, c.pctx,
                                      c.pf_nsplit, c.pf_kps, c.attn_ws);
      pa.noskip = c.attn_noskip ? 1 : 0;
      MLCV_TRY(kvq_writer_launch(c.pqkv, nqkv, nq, nq + nkv, c.pcos, c.psin, P, c.H, c.KV, HD, kL, vL, pa.q_scale,
                                 pa.rpad, last ? nullptr : c.pqf, st));
      if (last) break;
      pa.qf = c.pqf;  // null: the attention ropes the raw q in its loader
      MLCV_TRY(attn_launch(pa, st));
    }
    TgArgs o{};
    o.a = c.pctx;
    o.lda = nq;
    o.b0 = o.b1 = o.b2 = ly.o[0].w;
    o.n1 = o.n2 = W0;
    o.ldb = nq;
    o.c = c.px;
    o.ldc = W0;
    o.M = P;
    o.N = W0;
    o.K = nq;
    o.epi = TG_RESIDUAL;
    gemm_ws_args(c, o);
    MLCV_TRY(tg_launch(o, st));
    TgArgs gu{};
    gu.a = c.pxn;
    gu.lda = W0;
    gu.b0 = gu.b1 = gu.b2 = ly.gu[0].w;
    gu.n1 = gu.n2 = 2 * c.F0;
    gu.ldb = W0;
    gu.c = c.ph;
    gu.ldc = c.F0;
    gu.M = P;
    gu.N = c.F0;
    gu.K = W0;
    gu.epi = TG_GEGLU;
    gu.F = c.F0;
    gu.bt = ly.gu[0].wt;
    gemm_ws_args(c, gu);
    TgArgs dn{};
    dn.a = c.ph;
    dn.lda = c.F0;
    dn.b0 = dn.b1 = dn.b2 = ly.dn[0].w;
    dn.n1 = dn.n2 = W0;
    dn.ldb = c.F0;
    dn.c = c.px;
    dn.ldc = W0;
    dn.M = P;
    dn.N = W0;
    dn.K = c.F0;
    dn.epi = TG_RESIDUAL;
    dn.bt = ly.dn[0].wt;
    gemm_ws_args(c, dn);
    // with the weights tile-major, the MLP's activations are too: the post-attention norm writes
    // gate_up's X and gate_up writes down's X in the 32-k tiles' layout (whole 1 KB per DMA
    // instruction on both operands), when both GEMMs run on those tiles
    const bool xtile = c.pf_wtile && gu.bt && dn.bt && tg_plan_k32(gu) && tg_plan_k32(dn);
    gu.at = gu.ct = dn.at = xtile ? 1 : 0;
    MLCV_TRY(rmsnorm_launch(c.px, ly.ln_post0, c.pxn, P, W0, c.cfg.rms_norm_eps, st, xtile));
    MLCV_TRY(tg_launch(gu, st));
    MLCV_TRY(tg_launch(dn, st));
  }
  return 0;
}

int enqueue_loop(Ctx& c, const float* keys, const _Float16* values, hipStream_t st) {
  const size_t modstep = (size_t)c.NM * 3 * c.W1;
  MLCV_TRY(euler_init_launch(c.x0, c.x32, c.xin16, c.T * c.A, st));
  if (c.loop_img) MLCV_TRY(enqueue_kv_prep(c, keys, values, st));
  c.use_img = c.loop_img;
  if (c.hoist) MLCV_TRY(enqueue_time_mod(c, c.te, c.NS, st, c.fork_mod));
  for (int i = 0; i < c.NS; ++i) {
    if (c.hoist) {
      // step 0 waits for each piece; later steps follow it on the same stream
      MLCV_TRY(enqueue_step(c, keys, values, c.mod + i * modstep, true, st, c.fork_mod && i == 0));
    } else {
      MLCV_TRY(enqueue_time_mod(c, c.te + (size_t)i * c.W1, 1, st, c.fork_mod));
      MLCV_TRY(enqueue_step(c, keys, values, c.mod, true, st, c.fork_mod));
    }
  }
  return 0;
}

int run_graph(Ctx& c, Graph& g, const std::vector<const void*>& key, const std::function<int(hipStream_t)>& body,
              hipStream_t user) {
  if (!c.use_graph) return body(user);
  if (!g.exec || g.key != key) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    g.exec = nullptr;
    MLCV_HIP(hipStreamBeginCapture(c.cap, hipStreamCaptureModeThreadLocal));
    const int r = body(c.cap);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(c.cap, &graph);
    if (r != 0) {
      if (e == hipSuccess && graph) (void)hipGraphDestroy(graph);
      return r;
    }
    MLCV_HIP(e);
    const hipError_t ie = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    MLCV_HIP(ie);
    g.key = key;
  }
  MLCV_HIP(hipGraphLaunch(g.exec, user));
  return 0;
}

int seg_ops(Ctx& c, OpDesc& d, const std::vector<SkSeg>& segs, int K, int epi, bool q4, int tr, int splits) {
  const int tile_rows = epi == EPI_GEGLU ? tr / 2 : tr;  // output columns per tile
  d.seg_off = (int)c.h_segs.size();
  d.nseg = (int)segs.size();
  d.K = K;
  d.epi = epi;
  d.q4 = q4;
  d.tr = tr;
  d.splits = splits;
  int t = 0;
  d.seg_tiles = segs.empty() ? 0 : (segs[0].n + tile_rows - 1) / tile_rows;
  for (SkSeg s : segs) {
    s.tile0 = t;
    const int nt = (s.n + tile_rows - 1) / tile_rows;
    if (nt != d.seg_tiles) d.seg_tiles = 0;
    t += nt;
    c.h_segs.push_back(s);
  }
  d.ntiles = t;
  return 0;
}

SkSeg seg_of(const Lin& l, void* out, int n, int ldo) {
  SkSeg s{};
  s.w = l.w;
  s.qw = l.qw;
  s.qs = l.qs;
  s.bias = l.b;
  s.out = out;
  s.n = n;
  s.ldo = ldo;
  return s;
}

}  // namespace
}  // namespace mlcv

using namespace mlcv;

struct mlcv_ctx {
  Ctx c;
  F32Model* f32 = nullptr;  // a float32 model: the generic fp32 kernels of model_f32.hip
  ~mlcv_ctx() {
    if (f32) f32_destroy(f32);
  }
};

// ---- scratch of mlcv_linear_noalloc -------------------------------------------------------
// One static device array per GPU, laid out as the zero page the skinny GEMM clamps its
// padding loads to, the split-K arrival counters (one per output tile; the last arrival
// resets its counter, so they are zero between calls) and the split-K partials.  8 MiB of
// partials hold every split plan of sk_plan for 64-row tiles (ceil(256 / tiles) splits of
// fewer than 256 tiles: under 512 x 4096 floats).
namespace {
constexpr size_t NA_ZERO_FLOATS = 64 * 64;
constexpr size_t NA_COUNTERS = (size_t)1 << 16;
constexpr size_t NA_PART_FLOATS = (size_t)1 << 21;
constexpr size_t NA_SCRATCH_BYTES = (NA_ZERO_FLOATS + NA_COUNTERS + NA_PART_FLOATS) * 4;
}  // namespace
static __device__ __align__(256) unsigned char scratch[NA_SCRATCH_BYTES];

namespace {
__global__ __launch_bounds__(256) void na_clear_kernel(unsigned* p, unsigned n) {
  for (unsigned i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) p[i] = 0u;
}

// This device's address of `scratch` (host code only ever passes this address to kernels);
// at the first call on a device its zero page and counters are cleared on `st`, ahead of
// the call's own kernels.
int noalloc_scratch(hipStream_t st, char** base) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  MLCV_HIP(hipGetDevice(&dev));
  MLCV_REQUIRE(dev >= 0 && dev < 64, "device index");
  std::lock_guard<std::mutex> lk(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    MLCV_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MLCV_REQUIRE(p != nullptr, "no device address for the linear scratch");
    na_clear_kernel<<<64, 256, 0, st>>>(static_cast<unsigned*>(p), (unsigned)(NA_ZERO_FLOATS + NA_COUNTERS));
    MLCV_HIP(hipGetLastError());
    addr[dev] = p;
  }
  *base = static_cast<char*>(addr[dev]);
  return 0;
}
}  // namespace

extern "C" {

const char* mlcv_last_error(void) { return get_error(); }

int mlcv_param_count(const mlcv_config* cfg, int32_t* count) {
  MLCV_REQUIRE(cfg && count, "null argument");
  const int per_layer_lin = 12 + 2;  // 8 attn + 4 mlp + 2 modulation linears
  const int n_fp = 18 * cfg->depth + 11;
  const int n_lin = per_layer_lin * cfg->depth + 1 + 4;  // + final modulation + 4 head linears
  *count = cfg->quant == MLCV_QUANT_Q4F16_1 ? n_fp + n_lin : n_fp;
  return 0;
}

int mlcv_create(const mlcv_config* cfg, mlcv_ctx** out) {
  MLCV_REQUIRE(cfg && out, "null argument");
  MLCV_REQUIRE(cfg->dtype == MLCV_DTYPE_F16 || cfg->dtype == MLCV_DTYPE_F32, "dtype: MLCV_DTYPE_F16 or MLCV_DTYPE_F32");
  if (cfg->dtype == MLCV_DTYPE_F32) {
    MLCV_REQUIRE(cfg->quant == MLCV_QUANT_NONE, "float32 models are not quantized");
    MLCV_REQUIRE(cfg->depth >= 1 && cfg->prefix_len >= 1 && cfg->suffix_len >= 1 && cfg->num_steps >= 1 &&
                     cfg->num_heads >= 1 && cfg->num_kv_heads >= 1,
                 "depth / lengths / steps / heads must be positive");
    auto* h = new (std::nothrow) mlcv_ctx();
    if (!h) {
      set_error("out of host memory");
      return -1;
    }
    h->c.cfg = *cfg;
    if (const int rc = f32_create(*cfg, &h->f32)) {
      delete h;
      return rc;
    }
    *out = h;
    return 0;
  }
  MLCV_REQUIRE(cfg->quant == MLCV_QUANT_NONE || cfg->quant == MLCV_QUANT_Q4F16_1, "unknown quantization");
  const int hd = cfg->head_dim;
  MLCV_REQUIRE(hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256, "head_dim must be 16/32/64/128/256");
  MLCV_REQUIRE(cfg->num_kv_heads == 1 || cfg->num_kv_heads == cfg->num_heads, "num_kv_heads must be 1 or num_heads");
  MLCV_REQUIRE(cfg->vlm_width % 32 == 0 && cfg->ae_width % 32 == 0, "widths must be multiples of 32");
  MLCV_REQUIRE(cfg->ae_mlp % 32 == 0 && cfg->vlm_mlp % 64 == 0, "mlp dims: ae % 32, vlm % 64");
  MLCV_REQUIRE(cfg->action_dim % 32 == 0, "action_dim must be a multiple of 32");
  MLCV_REQUIRE((cfg->num_heads * hd) % 32 == 0, "num_heads * head_dim must be a multiple of 32");
  MLCV_REQUIRE(cfg->depth >= 1 && cfg->prefix_len >= 1 && cfg->suffix_len >= 1 && cfg->num_steps >= 1,
               "depth / lengths / steps must be positive");
  MLCV_REQUIRE(cfg->num_steps <= 64, "num_steps must be <= 64");

  auto* h = new (std::nothrow) mlcv_ctx();
  if (!h) {
    set_error("out of host memory");
    return -1;
  }
  Ctx& c = h->c;
  c.tilings = read_tilings(cfg->quant == MLCV_QUANT_Q4F16_1);
  c.cfg = *cfg;
  c.q4 = cfg->quant == MLCV_QUANT_Q4F16_1;
  c.W0 = cfg->vlm_width;
  c.F0 = cfg->vlm_mlp;
  c.W1 = cfg->ae_width;
  c.F1 = cfg->ae_mlp;
  c.D = cfg->depth;
  c.H = cfg->num_heads;
  c.KV = cfg->num_kv_heads;
  c.HD = hd;
  c.P = cfg->prefix_len;
  c.T = cfg->suffix_len;
  c.A = cfg->action_dim;
  c.NS = cfg->num_steps;
  c.NM = 2 * c.D + 1;

  auto fail = [&](int r) {
    delete h;
    return r;
  };
  if (hipGetDevice(&c.dev) != hipSuccess) {
    set_error("no HIP device");
    return fail(-1);
  }
  const int T = c.T, W1 = c.W1, nq = c.H * hd, nkv = c.KV * hd;
  std::vector<void*>& o = c.owned;
  int r = 0;
#define ALLOC(ptr, n) \
  if ((r = dalloc(&(ptr), (size_t)(n), o)) != 0) return fail(r)
  ALLOC(c.x16, T * W1);
  ALLOC(c.q, T * nq);
  ALLOC(c.k, T * nkv);
  ALLOC(c.v, T * nkv);
  ALLOC(c.attn, (size_t)std::max(T, 64) * nq);
  ALLOC(c.h, (size_t)std::max(T, 64) * c.F1);
  ALLOC(c.cond, c.NS * W1);
  ALLOC(c.tmp, c.NS * W1);
  ALLOC(c.mod, (size_t)c.NS * c.NM * 3 * W1);
  ALLOC(c.nscale, (size_t)c.NS * c.NM);
  {  // prescale 1 until the first modulations (the per-op hooks may run a GEMM before them)
    const std::vector<float> ones((size_t)c.NS * c.NM, 1.0f);
    if (hipMemcpy(c.nscale, ones.data(), ones.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
      set_error("prescale initialisation failed");
      return fail(-1);
    }
  }
  ALLOC(c.te, c.NS * W1);
  ALLOC(c.xin16, T * c.A);
  ALLOC(c.x32, T * c.A);
  ALLOC(c.x0, T * c.A);
  ALLOC(c.vout, T * c.A);
  ALLOC(c.cos, T * hd / 2);
  ALLOC(c.sin, T * hd / 2);
  ALLOC(c.mask, c.P);
  MLCV_REQUIRE(W1 % 64 == 0, "ae_width must be a multiple of 64");
  c.rss_tiles = W1 / RSS_COLS;
  ALLOC(c.rowss, (size_t)T * c.rss_tiles);
  c.frag = T < 64 && W1 % 128 == 0 && nq % 128 == 0 && c.F1 % 128 == 0 && nkv % 16 == 0 && c.A % 16 == 0;
  c.prescaled = c.frag;
  c.small_m = c.frag && c.NS <= 16;
  ALLOC(c.xu, (size_t)64 * W1);
  c.attn_rpad = ((T * (c.H / c.KV) + 63) / 64) * 64;
  const size_t qf_halfs = (size_t)c.KV * c.attn_rpad * ((hd + 31) / 32) * 64;
  ALLOC(c.qf, qf_halfs);
  ALLOC(c.k32, (size_t)T * nkv);
  const size_t P = c.P;
  ALLOC(c.px, P * c.W0);
  const size_t P16 = (P + 15) / 16 * 16;  // whole 16-row blocks of the tile-major MLP activations
  ALLOC(c.pxn, P16 * c.W0);
  ALLOC(c.pqkv, P * (nq + 2 * nkv));
  ALLOC(c.pctx, P * nq);
  if (hd % 64 == 0) ALLOC(c.pqf, q_frag_halfs(c.KV, (int)((P * (c.H / c.KV) + 63) / 64 * 64), hd));
  {
    const char* e = std::getenv("MLCV_PF_ATTN");
    c.pa_on = pa_supported(hd, c.P, c.H, c.KV) && !(e && std::atoi(e) == 0);
  }
  if (c.pa_on) {
    c.pa = pa_plan(c.P, c.H, c.KV);
    ALLOC(c.pa_img, c.pa.img_bytes);
    ALLOC(c.pa_qf, c.pa.qf_halfs);
    ALLOC(c.pa_part, c.pa.part_halfs);
    ALLOC(c.pa_ml, c.pa.ml_floats);
    ALLOC(c.pa_ctr, c.pa.counters);
    if (hipMemset(c.pa_ctr, 0, c.pa.counters * sizeof(unsigned)) != hipSuccess) {
      set_error("prefill attention counters: hipMemset failed");
      return fail(-1);
    }
  }
  ALLOC(c.ph, P16 * c.F0);
  // rows past P of the tile-major blocks are read (their products are never stored): keep them finite
  if (hipMemset(c.pxn, 0, P16 * c.W0 * 2) != hipSuccess || hipMemset(c.ph, 0, P16 * c.F0 * 2) != hipSuccess) {
    set_error("prefill activations: hipMemset failed");
    return fail(-1);
  }
  ALLOC(c.pcos, P * hd / 2);
  ALLOC(c.psin, P * hd / 2);
  ALLOC(c.pkeys, (size_t)c.D * kv_slice(c));
  ALLOC(c.pvalues, (size_t)c.D * kv_slice(c));

  ALLOC(c.m0cos, (size_t)T * hd / 2);
  ALLOC(c.m0sin, (size_t)T * hd / 2);
  ALLOC(c.m0mask, P);
  // RoPE tables of positions 0..P+T-1: radians = pos / theta^((2/hd) i) in float64, cast to
  // float32; rows 0..P-1 are the prefill's, rows P..P+T-1 the joint forward's suffix rows
  {
    std::vector<float> hc((P + T) * hd / 2), hs((P + T) * hd / 2);
    for (size_t p = 0; p < P + T; ++p)
      for (int i = 0; i < hd / 2; ++i) {
        const double ts = std::pow((double)cfg->rope_theta, (2.0 / hd) * i);
        const double rad = (double)p / ts;
        hc[p * (hd / 2) + i] = (float)std::cos(rad);
        hs[p * (hd / 2) + i] = (float)std::sin(rad);
      }
    const size_t np = (size_t)P * hd / 2, ns = (size_t)T * hd / 2;
    if (hipMemcpy(c.pcos, hc.data(), np * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(c.psin, hs.data(), np * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(c.m0cos, hc.data() + np, ns * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(c.m0sin, hs.data() + np, ns * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(c.m0mask, 0, (size_t)P * 4) != hipSuccess) {
      set_error("copy of rope tables failed");
      return fail(-1);
    }
  }
  // attention split plans and workspace
  const int st_rows = T * (c.H / c.KV), pf_rows = c.P * (c.H / c.KV);
  // the step's attention: about ATTN_TARGET workgroups (MLCV_ATTN_TARGET overrides, tuning)
  const int attn_target = std::getenv("MLCV_ATTN_TARGET") ? std::atoi(std::getenv("MLCV_ATTN_TARGET")) : ATTN_TARGET;
  attn_plan(st_rows, c.P, T, attn_target > 0 ? attn_target : ATTN_TARGET, &c.st_nsplit, &c.st_kps);
  attn_plan(pf_rows, c.P, 0, prefill_attn_target(pf_rows), &c.pf_nsplit, &c.pf_kps);
  c.attn_ws_floats_n = std::max(attn_ws_floats(c.KV, st_rows, hd, c.st_nsplit),
                                attn_ws_floats(c.KV, pf_rows, hd, c.pf_nsplit));
  ALLOC(c.attn_ws, c.attn_ws_floats_n);
  c.gemm_ws_floats = tg_ws_floats();
  c.gemm_sync_words = tg_sync_words();
  ALLOC(c.gemm_ws, c.gemm_ws_floats);
  ALLOC(c.gemm_sync, c.gemm_sync_words);
  c.img_layer_bytes = attn_img_bytes(c.KV, c.P, hd);
  ALLOC(c.kvimg, (size_t)c.D * c.img_layer_bytes);

  // persistent step: shapes it is built for, its plan and its per-layer activations
  {
    auto env_int = [](const char* name, int dflt) {
      const char* e = std::getenv(name);
      return e ? std::atoi(e) : dflt;
    };
    // K slices of o_proj / down: the largest power of two up to 4 whose slices are whole
    // 128-column chunks per wave (q4: 512) of at most 1024 columns
    const int unit = c.q4 ? 512 : 128;
    auto pick = [&](int K, int want) {
      for (int s = want; s >= 1; s >>= 1)
        if (K % (s * unit) == 0 && K / s / 128 <= 8) return s;
      return 0;
    };
    const int so = pick(nq, env_int("MLCV_PK_SO", 4)), sd = pick(c.F1, env_int("MLCV_PK_SD", 4));
    const int G = device_cus();
    c.pk_ok = c.frag && pk_head_dim_ok(hd) && c.A % 32 == 0 && W1 / 128 <= 8 && so > 0 && sd > 0 && G > 0 &&
              G <= 512 && (c.KV == 1 || c.KV == c.H) && c.st_nsplit <= 32 &&
              (!c.q4 || (W1 / 128) % 4 == 0) && c.NS * c.NM <= 65536;
    c.pk_on = c.pk_ok && env_int("MLCV_PERSIST", 0) != 0;
    if (c.pk_ok) {
      PkArgs& p = c.pk;
      p.D = c.D;
      p.T = T;
      p.A = c.A;
      p.W1 = W1;
      p.F1 = c.F1;
      p.H = c.H;
      p.KV = c.KV;
      p.HD = hd;
      p.P = c.P;
      p.nq = nq;
      p.nkv = nkv;
      p.eps = cfg->rms_norm_eps;
      p.G = G;
      p.so = so;
      p.sd = sd;
      p.gu_sw = env_int("MLCV_PK_GUSW", 2) == 1 || c.F1 % 16 != 0 ? 1 : 2;
      p.nsplit = c.st_nsplit;
      p.kps = c.st_kps;
      p.rows = T * (c.H / c.KV);
      p.rpad = c.attn_rpad;
      p.spin = (unsigned)env_int("MLCV_PK_SPIN", 1 << 22);
      // idle workgroups of the attention phase prefetching the layer's later weights: measured
      // slower (they compete with the attention), so off unless asked for
      p.prefetch = env_int("MLCV_PK_PREFETCH", 0);
      p.merge_comb = (p.rpad / 64) * c.st_nsplit * c.KV <= G && env_int("MLCV_PK_MERGE_COMB", 1) != 0;
      auto al = [](size_t n) { return (n + 127) / 128 * 128; };  // whole 256-byte lines per layer
      p.s_x = al((size_t)T * W1);
      p.s_r = al((size_t)T * (W1 / 16));
      p.s_u = al((size_t)64 * W1);
      p.s_qf = al(qf_halfs);
      p.s_k = al((size_t)T * nkv);
      p.s_part = al(attn_ws_floats(c.KV, p.rows, hd, c.st_nsplit));
      p.s_attn = al((size_t)64 * nq);
      p.s_h = al((size_t)64 * c.F1);
      p.s_sko = al((size_t)(W1 / 16) * so * 4 * 64 * 4);
      p.s_skd = al((size_t)(W1 / 16) * sd * 4 * 64 * 4);
      const size_t D1 = (size_t)c.D + 1, Dn = (size_t)c.D;
      ALLOC(p.xres, D1 * p.s_x);
      ALLOC(p.rres, D1 * p.s_r);
      ALLOC(p.ures, D1 * p.s_u);
      ALLOC(p.xmid, Dn * p.s_x);
      ALLOC(p.rmid, Dn * p.s_r);
      ALLOC(p.umid, Dn * p.s_u);
      ALLOC(p.qf, Dn * p.s_qf);
      ALLOC(p.k32, Dn * p.s_k);
      ALLOC(p.vs, Dn * p.s_k);
      ALLOC(p.part, Dn * p.s_part);
      ALLOC(p.attn, Dn * p.s_attn);
      ALLOC(p.h, Dn * p.s_h);
      ALLOC(p.sko, Dn * p.s_sko);
      ALLOC(p.skd, Dn * p.s_skd);
      ALLOC(p.cnto, Dn * (W1 / 16));
      ALLOC(p.cntd, Dn * (W1 / 16));
      ALLOC(p.cntm, Dn * c.KV * (p.rpad / 64));
      ALLOC(p.prog, (size_t)G);
      ALLOC(p.err, 1);
      const std::pair<void*, size_t> zero_fill[] = {
          {p.xres, D1 * p.s_x * 2}, {p.rres, D1 * p.s_r * 4}, {p.ures, D1 * p.s_u * 2}, {p.xmid, Dn * p.s_x * 2},
          {p.rmid, Dn * p.s_r * 4}, {p.umid, Dn * p.s_u * 2}, {p.qf, Dn * p.s_qf * 2}, {p.k32, Dn * p.s_k * 4},
          {p.vs, Dn * p.s_k * 2}, {p.part, Dn * p.s_part * 4}, {p.attn, Dn * p.s_attn * 2}, {p.h, Dn * p.s_h * 2},
          {p.cnto, Dn * (W1 / 16) * 4}, {p.cntd, Dn * (W1 / 16) * 4}, {p.cntm, Dn * c.KV * (p.rpad / 64) * 4},
          {p.prog, (size_t)G * 4}, {p.err, 4}};
      for (const auto& z : zero_fill)
        if (hipMemset(z.first, 0, z.second) != hipSuccess) {
          set_error("persistent step buffers: memset failed");
          return fail(-1);
        }
    }
  }

  // XCD tensor-parallel step: the shape it is built for, on a part of 8 XCDs x 32 CUs
  {
    const char* e = std::getenv("MLCV_XTP");
    c.xt_ok = c.frag && xt_shape_ok(W1, c.F1, c.H, c.KV, hd, T, (int)P, c.A) && device_cus() == 256;
    c.xt_on = c.xt_ok && !(e && std::atoi(e) == 0) && !c.pk_on;
    if (c.xt_ok) {
      XtArgs& x = c.xt;
      x.D = c.D;
      x.T = T;
      x.P = (int)P;
      x.A = c.A;
      x.eps = cfg->rms_norm_eps;
      x.q4 = c.q4 ? 1 : 0;
      x.spin = 1u << 22;
      const size_t D8 = (size_t)c.D * 8, TW = (size_t)T * W1;
      ALLOC(x.x, D8 * TW);
      ALLOC(x.xm, D8 * TW);
      ALLOC(x.qf, D8 * XT_QF);
      ALLOC(x.k32, D8 * T * hd);
      ALLOC(x.v, D8 * T * hd);
      ALLOC(x.attn, D8 * 64 * hd);
      ALLOC(x.h, D8 * 64 * (c.F1 / 8));
      ALLOC(x.u, (size_t)8 * 64 * W1);
      ALLOC(x.rss, (size_t)8 * T * (W1 / 16));
      ALLOC(x.ap, (size_t)8 * 32 * 64 * hd);
      ALLOC(x.aml, (size_t)8 * 32 * 64 * 2);
      ALLOC(x.opart, (size_t)8 * 32 * T * 32);
      ALLOC(x.dpart, (size_t)8 * 32 * T * 32);
      ALLOC(x.flags, (size_t)8 * 32);
      ALLOC(x.err, 1);
      x.x16 = c.x16;
      const std::pair<void*, size_t> zero_fill[] = {
          {x.x, D8 * TW * 2}, {x.xm, D8 * TW * 2}, {x.qf, D8 * XT_QF * 2}, {x.k32, D8 * T * hd * 4},
          {x.v, D8 * T * hd * 2}, {x.attn, D8 * 64 * hd * 2}, {x.h, D8 * 64 * (c.F1 / 8) * 2},
          {x.u, (size_t)8 * 64 * W1 * 2}, {x.rss, (size_t)8 * T * (W1 / 16) * 4}, {x.ap, (size_t)8 * 32 * 64 * hd * 2},
          {x.aml, (size_t)8 * 32 * 64 * 2 * 4}, {x.opart, (size_t)8 * 32 * T * 32 * 4},
          {x.dpart, (size_t)8 * 32 * T * 32 * 4}, {x.flags, (size_t)8 * 32 * 4}, {x.err, 4}};
      for (const auto& z : zero_fill)
        if (hipMemset(z.first, 0, z.second) != hipSuccess) {
          set_error("XCD step buffers: memset failed");
          return fail(-1);
        }
    }
  }

  // skinny-GEMM op descriptions (segments are filled at bind time; shapes now)
  const int mb_t = (T + 63) / 64, mb_s = (c.NS + 63) / 64;
  struct Shape {
    int ntiles, K, mb, tr, splits;  // mb: m blocks times m groups
  };
  auto tiles = [](int n, int cols) { return (n + cols - 1) / cols; };
  std::vector<Shape> shapes = {
      {tiles(nq, tile_qkv(c).tr) + 2 * tiles(nkv, tile_qkv(c).tr), W1, mb_t * tile_qkv(c).mg, tile_qkv(c).tr,
       tile_qkv(c).splits},
      {tiles(W1, tile_o(c).tr), nq, mb_t * tile_o(c).mg, tile_o(c).tr, tile_o(c).splits},
      {tiles(c.F1, tile_gu(c).tr / 2), W1, mb_t * tile_gu(c).mg, tile_gu(c).tr, tile_gu(c).splits},
      {tiles(W1, tile_down(c).tr), c.F1, mb_t * tile_down(c).mg, tile_down(c).tr, tile_down(c).splits},
      {tiles(W1, 16), W1, mb_s, 16, c.tilings.tmlp.splits},                      // time mlp
      {tiles(W1, 64), W1, mb_s, 64, 0},
      {std::max(2, c.NM - 2) * tiles(3 * W1, 64), W1, mb_s, 64, 0},              // modulation pieces
      {std::max(2, c.NM) * tiles(3 * W1, 16), W1, mb_s, 16, MOD_SPLITS},
      {tiles(W1, TR_AIN), c.A, mb_t, TR_AIN, SPLIT_AIN},                         // action_in
      {tiles(c.A, tile_head(c).tr), W1, mb_t * tile_head(c).mg, tile_head(c).tr, tile_head(c).splits},  // action_out
  };
  for (const Shape& s : shapes) {
    const SkPlan p = sk_plan(s.ntiles, s.K, s.mb, s.splits);
    c.skws_floats = std::max(c.skws_floats, sk_ws_floats(s.ntiles, s.mb, p, s.tr));
    c.ncounters = std::max(c.ncounters, (size_t)s.ntiles * s.mb);
  }
  ALLOC(c.skws, c.skws_floats);
  ALLOC(c.counters, c.ncounters);
  {
    // modulation pieces: up to NM - 2 segments of 3 W1 rows; 16-row tiles take one split,
    // 64-row tiles the planner's
    const int segs = std::max(2, c.NM - 2);
    const int nt = segs * tiles(3 * W1, 16);
    const SkPlan p = sk_plan(segs * tiles(3 * W1, 64), W1, mb_s, 0);
    ALLOC(c.skws_side, std::max<size_t>(1, sk_ws_floats(segs * tiles(3 * W1, 64), mb_s, p, 64)));
    ALLOC(c.counters_side, (size_t)nt * mb_s);
    c.ncounters_side = (size_t)nt * mb_s;
  }
  ALLOC(c.zero, 64 * 64);
#undef ALLOC
  c.mod_ev.assign(2, nullptr);
  // measured: the forked modulation slows the layer chain more than it hides, so it is
  // off unless MLCV_FORK_MOD=1 (tuning)
  c.fork_mod = std::getenv("MLCV_FORK_MOD") != nullptr && std::atoi(std::getenv("MLCV_FORK_MOD")) != 0;
  if (const char* e = std::getenv("MLCV_LOOP_IMG")) c.loop_img = std::atoi(e) != 0;
  if (const char* e = std::getenv("MLCV_ATTN_XG")) c.attn_xg = std::atoi(e) != 0;
  if (const char* e = std::getenv("MLCV_PREFILL_SMALL_TILES")) c.gemm_small = std::atoi(e) != 0;
  if (const char* e = std::getenv("MLCV_PREFETCH")) c.prefetch = (unsigned)std::strtoul(e, nullptr, 0);
  if (const char* e = std::getenv("MLCV_PF_BLOCKS")) c.pf_blocks = std::max(8, std::atoi(e));
  bool ev_ok = hipEventCreateWithFlags(&c.cond_ev, hipEventDisableTiming) == hipSuccess;
  for (hipEvent_t& e : c.mod_ev) ev_ok = ev_ok && hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
  if (!ev_ok || hipStreamCreateWithFlags(&c.side, hipStreamNonBlocking) != hipSuccess) {
    set_error("modulation stream / event setup failed");
    return fail(-1);
  }
  if (hipHostMalloc(reinterpret_cast<void**>(&c.status), sizeof(unsigned), hipHostMallocMapped | hipHostMallocCoherent) !=
          hipSuccess ||
      hipHostGetDevicePointer(reinterpret_cast<void**>(&c.status_dev), c.status, 0) != hipSuccess) {
    set_error("status word setup failed");
    return fail(-1);
  }
  *c.status = 0;
  if (hipMemset(c.counters, 0, c.ncounters * sizeof(unsigned)) != hipSuccess ||
      hipMemset(c.gemm_sync, 0, c.gemm_sync_words * sizeof(unsigned)) != hipSuccess ||
      hipMemset(c.counters_side, 0, c.ncounters_side * sizeof(unsigned)) != hipSuccess ||
      hipMemset(c.xu, 0, (size_t)64 * W1 * 2) != hipSuccess ||
      hipMemset(c.qf, 0, qf_halfs * 2) != hipSuccess ||
      hipMemset(c.attn, 0, (size_t)std::max(T, 64) * nq * 2) != hipSuccess ||
      hipMemset(c.h, 0, (size_t)std::max(T, 64) * c.F1 * 2) != hipSuccess ||
      hipMemset(c.zero, 0, 64 * 64 * sizeof(float)) != hipSuccess ||
      hipStreamCreateWithFlags(&c.cap, hipStreamNonBlocking) != hipSuccess) {
    set_error("context setup failed");
    return fail(-1);
  }
  if (hipDeviceSynchronize() != hipSuccess) {
    set_error("context setup sync failed");
    return fail(-1);
  }
  *out = h;
  return 0;
}

int mlcv_destroy(mlcv_ctx* ctx) {
  if (!ctx) return 0;
  (void)hipDeviceSynchronize();
  delete ctx;
  return 0;
}

int mlcv_set_option(mlcv_ctx* ctx, int32_t key, int64_t value) {
  MLCV_REQUIRE(ctx, "null context");
  if (ctx->f32) {  // the float32 model runs eager launches; the step-form options do not apply
    MLCV_REQUIRE(key == MLCV_OPT_USE_GRAPH || key == MLCV_OPT_HOIST_MODULATION || key == MLCV_OPT_MASK_SKIP ||
                     key == MLCV_OPT_STEP_GRAPH,
                 "this option is not built for float32 models");
    return 0;
  }
  Ctx& c = ctx->c;
  if (key == MLCV_OPT_USE_GRAPH) c.use_graph = value != 0;
  else if (key == MLCV_OPT_STEP_GRAPH) c.step_graph = value != 0;
  else if (key == MLCV_OPT_HOIST_MODULATION) c.hoist = value != 0;
  else if (key == MLCV_OPT_PERSIST) {
    MLCV_REQUIRE(value == 0 || c.pk_ok, "the persistent step is not built for this configuration");
    c.pk_on = value != 0;
    if (c.pk_on) c.xt_on = false;
  } else if (key == MLCV_OPT_XTP) {
    MLCV_REQUIRE(value == 0 || c.xt_ok, "the XCD tensor-parallel step is not built for this configuration");
    MLCV_REQUIRE(value >= 0 && value <= 2, "XCD step option: 0, 1 or 2");
    c.xt_on = value != 0;
    c.xt.noskip = value == 2 || c.attn_noskip ? 1 : 0;
    if (c.xt_on) c.pk_on = false;
  } else if (key == MLCV_OPT_MASK_SKIP) {
    MLCV_REQUIRE(value == 0 || value == 1, "mask skip option: 0 or 1");
    c.attn_noskip = value == 0;
    c.pk.noskip = c.attn_noskip ? 1 : 0;
    c.xt.noskip = c.attn_noskip ? 1 : 0;
  } else if (key == MLCV_OPT_XTP_KEEP) {
    c.xt.ls = value != 0 ? 1 : 0;
  } else if (key == MLCV_OPT_SYNC_WORDS) {
    MLCV_HIP(hipDeviceSynchronize());
    if (c.pk_ok) {
      const std::vector<unsigned> w((size_t)c.pk.G, (unsigned)value);
      MLCV_HIP(hipMemcpy(c.pk.prog, w.data(), w.size() * 4, hipMemcpyHostToDevice));
    }
    if (c.xt_ok) {
      const std::vector<unsigned> w((size_t)8 * 32, (unsigned)value);
      MLCV_HIP(hipMemcpy(c.xt.flags, w.data(), w.size() * 4, hipMemcpyHostToDevice));
    }
  } else if (key == MLCV_OPT_PERSIST_SPIN) {
    MLCV_REQUIRE(value >= 0 && value <= 0x7FFFFFFF, "spin limit");
    c.pk.spin = (unsigned)value;
    c.xt.spin = (unsigned)value;
  } else if (key == MLCV_OPT_MEET_POLLS) {
    MLCV_REQUIRE(value >= 0 && value <= 0x7FFFFFFF, "meeting poll limit");
    c.meet_polls = (unsigned)value;
  } else MLCV_REQUIRE(false, "unknown option");
  c.drop_graphs();
  return 0;
}

int mlcv_bind_params(mlcv_ctx* ctx, const void* const* ptrs, int32_t count, void* stream) {
  MLCV_REQUIRE(ctx, "null argument");
  if (ctx->f32) {
    MLCV_REQUIRE(ptrs, "null argument");
    int32_t want = 0;
    MLCV_TRY(mlcv_param_count(&ctx->c.cfg, &want));
    MLCV_REQUIRE(count == want, "parameter count mismatch (expected " + std::to_string(want) + ")");
    MLCV_HIP(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
    return f32_bind(*ctx->f32, ptrs, count);
  }
  Ctx& c = ctx->c;
  // unbound until this call has finished: any failure below (a rejected list included) leaves
  // the context refusing every entry point ("parameters not bound") instead of pointing at
  // freed copies or at a half-built set of layers
  c.bound = false;
  c.drop_graphs();
  MLCV_REQUIRE(ptrs, "null argument");
  int32_t want = 0;
  MLCV_TRY(mlcv_param_count(&c.cfg, &want));
  MLCV_REQUIRE(count == want, "parameter count mismatch (expected " + std::to_string(want) + ")");
  for (int i = 0; i < count; ++i) MLCV_REQUIRE(ptrs[i] != nullptr, "null parameter pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  MLCV_HIP(hipStreamSynchronize(st));
  for (void* p : c.bind_owned) (void)hipFree(p);
  c.bind_owned.clear();

  int idx = 0;
  auto half_ptr = [&]() { return reinterpret_cast<const _Float16*>(ptrs[idx++]); };
  auto lin = [&](Lin& l, int N, int K, bool bias) {
    l = Lin{};
    l.N = N;
    l.K = K;
    if (c.q4) {
      l.qw = reinterpret_cast<const uint32_t*>(ptrs[idx++]);
      l.qs = half_ptr();
    } else {
      l.w = half_ptr();
    }
    if (bias) l.b = half_ptr();
  };
  const int nq = c.H * c.HD, nkv = c.KV * c.HD;
  const int widths[2] = {c.W0, c.W1}, mlps[2] = {c.F0, c.F1};
  c.layers.assign(c.D, Layer{});
  for (int L = 0; L < c.D; ++L) {
    Layer& ly = c.layers[L];
    for (int e = 0; e < 2; ++e) {
      lin(ly.q[e], nq, widths[e], false);
      lin(ly.k[e], nkv, widths[e], false);
      lin(ly.v[e], nkv, widths[e], false);
      lin(ly.o[e], widths[e], nq, false);
    }
    for (int e = 0; e < 2; ++e) {
      lin(ly.gu[e], 2 * mlps[e], widths[e], false);
      lin(ly.dn[e], widths[e], mlps[e], false);
    }
    ly.ln_in0 = half_ptr();
    lin(ly.mod_in, 3 * c.W1, c.W1, true);
    ly.ln_post0 = half_ptr();
    lin(ly.mod_post, 3 * c.W1, c.W1, true);
  }
  idx++;  // backbone.final_norm.0.weight (unused on the M1 path)
  lin(c.final_mod, 3 * c.W1, c.W1, true);
  lin(c.ain, c.W1, c.A, true);
  lin(c.aout, c.A, c.W1, true);
  lin(c.tin, c.W1, c.W1, true);
  lin(c.tout, c.W1, c.W1, true);
  MLCV_REQUIRE(idx == count, "internal: parameter walk mismatch");

  // q4: expert-0 (prefill, compute-bound) runs on an fp16 copy dequantized once
  if (c.q4) {
    for (int L = 0; L < c.D; ++L) {
      Layer& ly = c.layers[L];
      Lin* ls[6] = {&ly.q[0], &ly.k[0], &ly.v[0], &ly.o[0], &ly.gu[0], &ly.dn[0]};
      for (Lin* l : ls) {
        _Float16* w = nullptr;
        MLCV_TRY(dalloc(&w, (size_t)l->N * l->K, c.bind_owned));
        MLCV_TRY(q4_dequant_launch(l->qw, l->qs, w, l->N, l->K, st));
        l->w = w;
      }
    }
  }

  // tile-major copies of the prefill's gate_up and down weights: the 256 x 256 tiles read them
  // 32 k at a time, 64 bytes per weight row; in this layout one DMA instruction of 16 rows reads
  // one contiguous 1 KB (whole 128-byte lines) instead of 16 half lines
  if (const char* e = std::getenv("MLCV_PF_WTILE")) c.pf_wtile = std::atoi(e) != 0;
  if (c.pf_wtile && c.W0 % 32 == 0 && c.F0 % 32 == 0 && c.W0 % 16 == 0) {
    for (int L = 0; L < c.D; ++L) {
      for (Lin* l : {&c.layers[L].gu[0], &c.layers[L].dn[0]}) {
        _Float16* t = nullptr;
        MLCV_TRY(dalloc(&t, (size_t)l->N * l->K, c.bind_owned));
        MLCV_TRY(wtile_shuffle_launch(l->w, t, l->N, l->K, st));
        l->wt = t;
      }
    }
  }

  // fragment-major copies of the action expert's layer and head weights
  auto frag_copy = [&](const Lin& l, int geglu_F, int rope_hd = 0) -> Lin {
    if (!c.frag) return l;
    Lin f = l;
    if (c.q4) {
      uint32_t* qwf = nullptr;
      _Float16* qsf = nullptr;
      if (dalloc(&qwf, (size_t)l.N * l.K / 8, c.bind_owned) || dalloc(&qsf, (size_t)l.N * l.K / 32, c.bind_owned) ||
          wf_shuffle_q4_launch(l.qw, l.qs, qwf, qsf, l.N, l.K, geglu_F, rope_hd, st))
        f.N = -1;
      f.qw = qwf;
      f.qs = qsf;
    } else {
      _Float16* wf = nullptr;
      if (dalloc(&wf, (size_t)l.N * l.K, c.bind_owned) || wf_shuffle_launch(l.w, wf, l.N, l.K, geglu_F, rope_hd, st))
        f.N = -1;
      f.w = wf;
    }
    return f;
  };

  // skinny op tables
  c.h_segs.clear();
  c.layer_ops.assign(4 * c.D, OpDesc{});
  const int W1 = c.W1;
  std::vector<PkLin> pklin;  // the persistent step's weight table [D][PK_NLIN]
  auto pkl = [](const Lin& l) { return PkLin{l.w, l.qw, l.qs, l.b}; };
  for (int L = 0; L < c.D; ++L) {
    Layer& ly = c.layers[L];
    OpDesc* ops = &c.layer_ops[4 * L];
    // q and k with their rows paired for RoPE in the store epilogue (q then goes to the
    // attention's fragment buffer, the suffix k to fp32 rows)
    const Lin fq = frag_copy(ly.q[1], 0, c.HD), fk = frag_copy(ly.k[1], 0, c.HD), fv = frag_copy(ly.v[1], 0);
    const Lin fo = frag_copy(ly.o[1], 0), fgu = frag_copy(ly.gu[1], c.F1), fdn = frag_copy(ly.dn[1], 0);
    for (const Lin* l : {&fq, &fk, &fv, &fo, &fgu, &fdn}) MLCV_REQUIRE(l->N >= 0, get_error());
    for (const Lin* l : {&fq, &fk, &fv, &fo, &fgu, &fdn}) pklin.push_back(pkl(*l));
    {
      SkSeg sq = seg_of(fq, c.q, nq, nq), sk = seg_of(fk, c.k, nkv, nkv);
      if (c.frag) {
        sq.out = c.qf;
        sq.rope = 1;
        sk.out = c.k32;
        sk.rope = 2;
      }
      seg_ops(c, ops[0], {sq, sk, seg_of(fv, c.v, nkv, nkv)}, W1, EPI_STORE, c.q4, tile_qkv(c).tr,
              tile_qkv(c).splits);
    }
    seg_ops(c, ops[1], {seg_of(fo, c.x16, W1, W1)}, nq, EPI_GATED_RES, c.q4, tile_o(c).tr, tile_o(c).splits);
    seg_ops(c, ops[2], {seg_of(fgu, c.h, c.F1, c.F1)}, W1, EPI_GEGLU, c.q4, tile_gu(c).tr, tile_gu(c).splits);
    seg_ops(c, ops[3], {seg_of(fdn, c.x16, W1, W1)}, c.F1, EPI_GATED_RES, c.q4, tile_down(c).tr, tile_down(c).splits);
    for (int i = 0; i < 4; ++i) ops[i].frag = c.frag;
    ops[0].mg = c.frag ? tile_qkv(c).mg : 1;
    ops[1].mg = c.frag ? tile_o(c).mg : 1;
    ops[2].mg = c.frag ? tile_gu(c).mg : 1;
    ops[3].mg = c.frag ? tile_down(c).mg : 1;
  }
  {
    // small-M GEMVs: 16-row register-direct tiles on shuffled weights, or 64-row tiles
    auto gemv_copy = [&](const Lin& l) -> Lin { return c.small_m ? frag_copy(l, 0) : l; };
    const int gtr = c.small_m ? 16 : 64;
    const Lin ftin = gemv_copy(c.tin), ftout = gemv_copy(c.tout);
    MLCV_REQUIRE(ftin.N >= 0 && ftout.N >= 0, get_error());
    const int tsp = c.small_m ? c.tilings.tmlp.splits : 0;
    seg_ops(c, c.op_tin, {seg_of(ftin, c.tmp, W1, W1)}, W1, EPI_STORE_SILU, c.q4, gtr, tsp);
    seg_ops(c, c.op_tout, {seg_of(ftout, c.cond, W1, W1)}, W1, EPI_STORE_SILU, c.q4, gtr, tsp);
    c.op_tin.xrow = c.op_tout.xrow = c.small_m;
    const int ldo = c.NM * 3 * W1;
    std::vector<SkSeg> first, rest;
    for (int L = 0; L <= c.D; ++L) {
      std::vector<const Lin*> ls;
      if (L < c.D) ls = {&c.layers[L].mod_in, &c.layers[L].mod_post};
      else ls = {&c.final_mod};
      for (size_t i = 0; i < ls.size(); ++i) {
        const Lin f = gemv_copy(*ls[i]);
        MLCV_REQUIRE(f.N >= 0, get_error());
        (L == 0 ? first : rest).push_back(seg_of(f, c.mod + (size_t)(2 * L + i) * 3 * W1, 3 * W1, ldo));
      }
    }
    c.mod_ops.assign(2, OpDesc{});
    const int mtr = c.small_m ? c.tilings.mod.tr : gtr;  // modulation tile rows
    seg_ops(c, c.mod_ops[0], first, W1, EPI_STORE, c.q4, mtr, c.small_m ? MOD_SPLITS : 0);
    seg_ops(c, c.mod_ops[1], rest, W1, EPI_STORE, c.q4, mtr, c.small_m ? MOD_SPLITS : 0);
    for (OpDesc& d : c.mod_ops) d.xrow = c.small_m;
    // one launch instead of two: the second piece's grid waits for the first anyway without
    // the side stream, and each tile's arithmetic is the same in either grouping
    c.mod_all = OpDesc{};
    if (c.small_m && MOD_SPLITS == 1) {
      std::vector<SkSeg> all(first);
      all.insert(all.end(), rest.begin(), rest.end());
      seg_ops(c, c.mod_all, all, W1, EPI_STORE, c.q4, mtr, MOD_SPLITS);
      c.mod_all.xrow = true;
    }
  }
  seg_ops(c, c.op_ain, {seg_of(c.ain, c.x16, W1, W1)}, c.A, EPI_STORE, c.q4, TR_AIN, SPLIT_AIN);
  {
    const Lin fa = frag_copy(c.aout, 0);
    MLCV_REQUIRE(fa.N >= 0, get_error());
    seg_ops(c, c.op_aout, {seg_of(fa, c.vout, c.A, c.A)}, W1, EPI_VOUT, c.q4, tile_head(c).tr, tile_head(c).splits);
    c.op_aout.frag = c.frag;
    c.op_aout.mg = c.frag ? tile_head(c).mg : 1;
    c.pk.aout = pkl(fa);
  }
  if (c.pk_ok || c.xt_ok) {
    // action_in as fp16 rows (a q4 model's copy is dequantized once here)
    c.ain16 = const_cast<_Float16*>(c.ain.w);
    if (c.q4) {
      MLCV_TRY(dalloc(&c.ain16, (size_t)W1 * c.A, c.bind_owned));
      MLCV_TRY(q4_dequant_launch(c.ain.qw, c.ain.qs, c.ain16, W1, c.A, st));
    }
    c.pk.ain_w = c.ain16;
    c.pk.ain_b = c.ain.b;
    if (!c.d_pklin) MLCV_HIP(hipMalloc(&c.d_pklin, (size_t)c.D * PK_NLIN * sizeof(PkLin)));
    MLCV_HIP(hipMemcpy(c.d_pklin, pklin.data(), pklin.size() * sizeof(PkLin), hipMemcpyHostToDevice));
    c.pk.lw = c.d_pklin;
    c.xt.lw = c.d_pklin;
    c.xt.ain_w = c.ain16;
    c.xt.ain_b = c.ain.b;
    c.aout16 = const_cast<_Float16*>(c.aout.w);
    if (c.q4) {
      MLCV_TRY(dalloc(&c.aout16, (size_t)c.A * W1, c.bind_owned));
      MLCV_TRY(q4_dequant_launch(c.aout.qw, c.aout.qs, c.aout16, c.A, W1, st));
    }
    c.xt.aout_w = c.aout16;
    c.xt.aout_b = c.aout.b;
  }

  if (c.d_segs) {
    (void)hipFree(c.d_segs);
    c.d_segs = nullptr;
  }
  MLCV_HIP(hipMalloc(&c.d_segs, c.h_segs.size() * sizeof(SkSeg)));
  MLCV_HIP(hipMemcpy(c.d_segs, c.h_segs.data(), c.h_segs.size() * sizeof(SkSeg), hipMemcpyHostToDevice));
  MLCV_HIP(hipStreamSynchronize(st));
  c.bound = true;
  return 0;
}

int mlcv_prefill(mlcv_ctx* ctx, const void* prefix_embs, const float* prefix_mask, float* keys, void* values,
                 void* stream) {
  MLCV_REQUIRE(ctx && prefix_embs && prefix_mask && keys && values, "null argument");
  if (ctx->f32) return f32_prefill(*ctx->f32, prefix_embs, prefix_mask, keys, values, reinterpret_cast<hipStream_t>(stream));
  Ctx& c = ctx->c;
  MLCV_REQUIRE(c.bound, "parameters not bound");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const CopyJob in[] = {{prefix_embs, c.px, (size_t)c.P * c.W0 * 2}, {prefix_mask, c.mask, (size_t)c.P * 4}};
  MLCV_TRY(copy_list_launch(in, 2, st));
  MLCV_TRY(run_graph(c, c.g_prefill, {}, [&](hipStream_t s) { return enqueue_prefill(c, c.pkeys, c.pvalues, s); },
                     st));
  const size_t n = (size_t)c.D * kv_slice(c);
  const CopyJob out[] = {{c.pkeys, keys, n * 4}, {c.pvalues, values, n * 2}};
  return copy_list_launch(out, 2, st);
}

// the suffix RoPE tables and the prefix mask, staged with the entry point's other inputs
static void suffix_jobs(const Ctx& c, const float* cos, const float* sin, const float* mask, std::vector<CopyJob>& jobs) {
  const size_t half = c.HD / 2;
  jobs.push_back({cos, c.cos, (size_t)c.T * half * 4});
  jobs.push_back({sin, c.sin, (size_t)c.T * half * 4});
  jobs.push_back({mask, c.mask, (size_t)c.P * 4});
}

int mlcv_embed_language(const int32_t* input_ids, int32_t n, const void* table, int32_t vocab, int32_t width,
                        void* out, void* stream) {
  MLCV_REQUIRE(input_ids && table && out && n > 0 && vocab > 0 && width > 0, "bad argument");
  return embed_language_launch(input_ids, n, reinterpret_cast<const _Float16*>(table), vocab, width,
                               reinterpret_cast<_Float16*>(out), reinterpret_cast<hipStream_t>(stream));
}

int mlcv_denoise_step(mlcv_ctx* ctx, const void* prefix_embs, const void* x_t, const void* time_emb, float* v_out,
                      void* stream) {
  MLCV_REQUIRE(ctx && prefix_embs && x_t && time_emb && v_out, "null argument");
  MLCV_REQUIRE(!ctx->f32, "the joint forward (denoise_step) is not built for float32 models");
  Ctx& c = ctx->c;
  MLCV_REQUIRE(c.bound, "parameters not bound");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  std::vector<CopyJob> jobs = {{prefix_embs, c.px, (size_t)c.P * c.W0 * 2},
                               {x_t, c.xin16, (size_t)c.T * c.A * 2},
                               {time_emb, c.te, (size_t)c.W1 * 2}};
  suffix_jobs(c, c.m0cos, c.m0sin, c.m0mask, jobs);
  MLCV_TRY(copy_list_launch(jobs.data(), (int)jobs.size(), st));
  MLCV_TRY(run_graph(c, c.g_m0, {},
                     [&](hipStream_t s) {
                       MLCV_TRY(enqueue_prefill(c, c.pkeys, c.pvalues, s));
                       c.use_img = false;
                       MLCV_TRY(enqueue_time_mod(c, c.te, 1, s, c.fork_mod));
                       return enqueue_step(c, c.pkeys, c.pvalues, c.mod, false, s, c.fork_mod);
                     },
                     st));
  {  // a kernel, not hipMemcpyAsync: its copy started about 8 us after the graph had ended
    const CopyJob out{c.vout, v_out, (size_t)c.T * c.A * 4};
    MLCV_TRY(copy_list_launch(&out, 1, st));
  }
  return 0;
}

int mlcv_denoise_step_kv(mlcv_ctx* ctx, const float* keys, const void* values, const void* x_t, const void* time_emb,
                         const float* suffix_cos, const float* suffix_sin, const float* prefix_mask, float* v_out,
                         void* stream) {
  MLCV_REQUIRE(ctx && keys && values && x_t && time_emb && suffix_cos && suffix_sin && prefix_mask && v_out,
               "null argument");
  if (ctx->f32)
    return f32_step(*ctx->f32, keys, values, x_t, time_emb, suffix_cos, suffix_sin, prefix_mask, v_out,
                    reinterpret_cast<hipStream_t>(stream));
  Ctx& c = ctx->c;
  MLCV_REQUIRE(c.bound, "parameters not bound");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // launched directly, the XCD step reads the caller's inputs and writes its output in place
  // (its vector loads and stores need 16-byte alignment); otherwise they are staged
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool in_place = !c.step_graph && c.xt_on && a16(x_t) && a16(time_emb) && a16(suffix_cos) &&
                        a16(suffix_sin) && a16(prefix_mask) && a16(v_out);
  StepIO io;
  if (in_place) {
    io.x_t = reinterpret_cast<const _Float16*>(x_t);
    io.cos = suffix_cos;
    io.sin = suffix_sin;
    io.mask = prefix_mask;
    io.vout = v_out;
  } else {
    std::vector<CopyJob> jobs = {{x_t, c.xin16, (size_t)c.T * c.A * 2}, {time_emb, c.te, (size_t)c.W1 * 2}};
    suffix_jobs(c, suffix_cos, suffix_sin, prefix_mask, jobs);
    MLCV_TRY(copy_list_launch(jobs.data(), (int)jobs.size(), st));
  }
  const _Float16* vals = reinterpret_cast<const _Float16*>(values);
  const _Float16* te = in_place ? reinterpret_cast<const _Float16*>(time_emb) : c.te;
  auto body = [&](hipStream_t s) {
    c.use_img = false;
    MLCV_TRY(enqueue_time_mod(c, te, 1, s, c.fork_mod));
    return enqueue_step(c, keys, vals, c.mod, false, s, c.fork_mod, io);
  };
  if (c.step_graph) MLCV_TRY(run_graph(c, c.g_step, {keys, values}, body, st));
  else MLCV_TRY(body(st));
  if (in_place) return 0;  // the head wrote v_out
  {  // a kernel, not hipMemcpyAsync: its copy started about 8 us after the graph had ended
    const CopyJob out{c.vout, v_out, (size_t)c.T * c.A * 4};
    MLCV_TRY(copy_list_launch(&out, 1, st));
  }
  return 0;
}

int mlcv_denoise_loop_kv(mlcv_ctx* ctx, const float* keys, const void* values, const float* x0,
                         const void* time_embs, const float* suffix_cos, const float* suffix_sin,
                         const float* prefix_mask, float* x_out, void* stream) {
  MLCV_REQUIRE(ctx && keys && values && x0 && time_embs && suffix_cos && suffix_sin && prefix_mask && x_out,
               "null argument");
  if (ctx->f32)
    return f32_loop(*ctx->f32, keys, values, x0, time_embs, suffix_cos, suffix_sin, prefix_mask, x_out,
                    reinterpret_cast<hipStream_t>(stream));
  Ctx& c = ctx->c;
  MLCV_REQUIRE(c.bound, "parameters not bound");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  std::vector<CopyJob> jobs = {{x0, c.x0, (size_t)c.T * c.A * 4}, {time_embs, c.te, (size_t)c.NS * c.W1 * 2}};
  suffix_jobs(c, suffix_cos, suffix_sin, prefix_mask, jobs);
  MLCV_TRY(copy_list_launch(jobs.data(), (int)jobs.size(), st));
  const _Float16* vals = reinterpret_cast<const _Float16*>(values);
  MLCV_TRY(run_graph(c, c.g_loop, {keys, values}, [&](hipStream_t s) { return enqueue_loop(c, keys, vals, s); },
                     st));
  {  // a kernel, not hipMemcpyAsync: its copy started about 8 us after the graph had ended
    const CopyJob out{c.x32, x_out, (size_t)c.T * c.A * 4};
    MLCV_TRY(copy_list_launch(&out, 1, st));
  }
  return 0;
}

int mlcv_chunk(mlcv_ctx* ctx, const void* prefix_embs, const float* prefix_mask, const float* x0,
               const void* time_embs, const float* suffix_cos, const float* suffix_sin, float* x_out, void* stream) {
  MLCV_REQUIRE(ctx && prefix_embs && prefix_mask && x0 && time_embs && suffix_cos && suffix_sin && x_out,
               "null argument");
  if (ctx->f32)
    return f32_chunk(*ctx->f32, prefix_embs, prefix_mask, x0, time_embs, suffix_cos, suffix_sin, x_out,
                     reinterpret_cast<hipStream_t>(stream));
  Ctx& c = ctx->c;
  MLCV_REQUIRE(c.bound, "parameters not bound");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  std::vector<CopyJob> jobs = {{prefix_embs, c.px, (size_t)c.P * c.W0 * 2},
                               {x0, c.x0, (size_t)c.T * c.A * 4},
                               {time_embs, c.te, (size_t)c.NS * c.W1 * 2}};
  suffix_jobs(c, suffix_cos, suffix_sin, prefix_mask, jobs);
  MLCV_TRY(copy_list_launch(jobs.data(), (int)jobs.size(), st));
  MLCV_TRY(run_graph(c, c.g_chunk, {},
                     [&](hipStream_t s) {
                       MLCV_TRY(enqueue_prefill(c, c.pkeys, c.pvalues, s));
                       return enqueue_loop(c, c.pkeys, c.pvalues, s);
                     },
                     st));
  {  // a kernel, not hipMemcpyAsync: its copy started about 8 us after the graph had ended
    const CopyJob out{c.x32, x_out, (size_t)c.T * c.A * 4};
    MLCV_TRY(copy_list_launch(&out, 1, st));
  }
  return 0;
}

int mlcv_sync(mlcv_ctx* ctx, void* stream) {
  MLCV_REQUIRE(ctx, "null context");
  Ctx& c = ctx->c;
  MLCV_HIP(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
  if (ctx->f32) return 0;  // no bounded device-side waits in the float32 model
  // every error word is read and reset before returning, so that one cause does not leave
  // another's words inconsistent for the calls after this sync
  std::string why;
  if (const unsigned e = __atomic_load_n(c.status, __ATOMIC_ACQUIRE)) {
    __atomic_store_n(c.status, 0u, __ATOMIC_RELEASE);
    why += "a split-K meeting of the prefill GEMMs gave up (error word " + std::to_string(e) +
           "; other work held the CUs the split workgroups need)";
  }
  if (c.xt_ok) {
    unsigned xerr = 0;
    MLCV_HIP(hipMemcpy(&xerr, c.xt.err, 4, hipMemcpyDeviceToHost));
    if (xerr != 0) {
      // the barrier words are no longer equal after an abandoned launch: start over
      MLCV_HIP(hipMemset(c.xt.flags, 0, (size_t)8 * 32 * 4));
      MLCV_HIP(hipMemset(c.xt.err, 0, 4));
      why += std::string(why.empty() ? "" : "; ") + "XCD step: a barrier wait gave up (error word " +
             std::to_string(xerr) + ")";
    }
  }
  if (c.pk_ok) {
    unsigned err = 0;
    MLCV_HIP(hipMemcpy(&err, c.pk.err, 4, hipMemcpyDeviceToHost));
    if (err != 0) {
      // progress words and counters are inconsistent after an abandoned launch: start over
      const size_t Dn = (size_t)c.D, W16 = (size_t)c.W1 / 16;
      MLCV_HIP(hipMemset(c.pk.prog, 0, (size_t)c.pk.G * 4));
      MLCV_HIP(hipMemset(c.pk.cnto, 0, Dn * W16 * 4));
      MLCV_HIP(hipMemset(c.pk.cntd, 0, Dn * W16 * 4));
      MLCV_HIP(hipMemset(c.pk.cntm, 0, Dn * c.KV * (c.pk.rpad / 64) * 4));
      MLCV_HIP(hipMemset(c.pk.err, 0, 4));
      why += std::string(why.empty() ? "" : "; ") + "persistent step: a wait between phases gave up (error word " +
             std::to_string(err) + ")";
    }
  }
  if (why.empty()) return 0;
  MLCV_HIP(hipDeviceSynchronize());
  set_error(why + "; the outputs of the calls since the last successful sync are invalid");
  return -4;
}

int mlcv_step_probe(mlcv_ctx* ctx, int32_t what, int32_t layer, void* out, size_t bytes, void* stream) {
  MLCV_REQUIRE(ctx && out, "null argument");
  MLCV_REQUIRE(!ctx->f32, "step probes are not built for float32 models");
  Ctx& c = ctx->c;
  // the persistent and XCD steps keep every layer's intermediates; the launch chain reuses one
  // set of buffers, which hold the outputs of the last operation run (layer 0 names them)
  const bool xt = c.xt_on;
  const bool chain = !c.pk_on && !xt;
  MLCV_REQUIRE(!chain || c.frag, "probes of the launch chain need its fragment-major form (T < 64)");
  const PkArgs& p = c.pk;
  const int T = c.T, W1 = c.W1, nq = c.H * c.HD, nkv = c.KV * c.HD;
  const int last = what == MLCV_PROBE_XCD_X ? 8 * c.D - 1 : chain ? 0 : what == MLCV_PROBE_X ? c.D : c.D - 1;
  MLCV_REQUIRE(layer >= 0 && layer <= last, "probe layer out of range");
  MLCV_REQUIRE(what != MLCV_PROBE_XCD_X || xt, "the per-XCD copies exist only in the XCD step");
  MLCV_REQUIRE(!xt || c.xt.ls == 1 || what == MLCV_PROBE_VOUT || what == MLCV_PROBE_MOD ||
                   (what == MLCV_PROBE_X && layer == c.D),
               "the XCD step keeps per-layer intermediates only with MLCV_OPT_XTP_KEEP = 1");
  MLCV_TRY(mlcv_sync(ctx, stream));
  auto fetch = [&](const void* src, size_t n, std::vector<char>& h) -> int {
    h.resize(n);
    MLCV_HIP(hipMemcpy(h.data(), src, n, hipMemcpyDeviceToHost));
    return 0;
  };
  std::vector<char> raw;
  const size_t L = (size_t)layer;
  auto frag_rows = [&](const _Float16* src, int K) -> int {  // fragment-major [64][K] -> [T][K]
    MLCV_REQUIRE(bytes == (size_t)T * K * 2, "probe output size");
    MLCV_TRY(fetch(src, (size_t)64 * K * 2, raw));
    const _Float16* f = reinterpret_cast<const _Float16*>(raw.data());
    _Float16* o = static_cast<_Float16*>(out);
    for (int m = 0; m < T; ++m)
      for (int k = 0; k < K; ++k) o[(size_t)m * K + k] = f[xf_index(m, k)];
    return 0;
  };
  const size_t qf_halfs = (size_t)c.KV * c.attn_rpad * ((c.HD + 31) / 32) * 64;
  if (xt && what != MLCV_PROBE_VOUT && what != MLCV_PROBE_MOD && !(what == MLCV_PROBE_X && layer == c.D)) {
    // XCD 0's copy of the residual stream; head / MLP-column blocks gathered from the 8 XCDs
    const XtArgs& x = c.xt;
    const size_t TW = (size_t)T * W1, hd = (size_t)c.HD, FX = (size_t)c.F1 / 8;
    auto gather_frag = [&](const _Float16* base, size_t per, int K, int ld) -> int {  // 8 x [64][K] -> [T][8K]
      MLCV_REQUIRE(bytes == (size_t)T * ld * 2, "probe output size");
      MLCV_TRY(fetch(base, 8 * per * 2, raw));
      const _Float16* f = reinterpret_cast<const _Float16*>(raw.data());
      _Float16* o = static_cast<_Float16*>(out);
      for (int xc = 0; xc < 8; ++xc)
        for (int m = 0; m < T; ++m)
          for (int k = 0; k < K; ++k) o[(size_t)m * ld + xc * K + k] = f[xc * per + xf_index(m, k)];
      return 0;
    };
    switch (what) {
      case MLCV_PROBE_X:
      case MLCV_PROBE_X_MID:
        MLCV_REQUIRE(bytes == TW * 2, "probe output size");
        MLCV_HIP(hipMemcpy(out, (what == MLCV_PROBE_X ? x.x : x.xm) + L * 8 * TW, bytes, hipMemcpyDeviceToHost));
        return 0;
      case MLCV_PROBE_XCD_X:  // layer = 8 L + XCD
        MLCV_REQUIRE(bytes == TW * 2, "probe output size");
        MLCV_HIP(hipMemcpy(out, x.x + L * TW, bytes, hipMemcpyDeviceToHost));
        return 0;
      case MLCV_PROBE_K:
        MLCV_REQUIRE(bytes == (size_t)T * nkv * 4, "probe output size");
        MLCV_HIP(hipMemcpy(out, x.k32 + L * 8 * T * hd, bytes, hipMemcpyDeviceToHost));
        return 0;
      case MLCV_PROBE_V:
        MLCV_REQUIRE(bytes == (size_t)T * nkv * 2, "probe output size");
        MLCV_HIP(hipMemcpy(out, x.v + L * 8 * T * hd, bytes, hipMemcpyDeviceToHost));
        return 0;
      case MLCV_PROBE_ATTN: return gather_frag(x.attn + L * 8 * 64 * hd, 64 * hd, (int)hd, nq);
      case MLCV_PROBE_H: return gather_frag(x.h + L * 8 * 64 * FX, 64 * FX, (int)FX, c.F1);
      case MLCV_PROBE_Q: {  // hi + lo of each XCD's head -> [T][H*hd] f32
        MLCV_REQUIRE(bytes == (size_t)T * nq * 4, "probe output size");
        MLCV_TRY(fetch(x.qf + L * 8 * XT_QF, (size_t)8 * XT_QF * 2, raw));
        const _Float16* f = reinterpret_cast<const _Float16*>(raw.data());
        float* o = static_cast<float*>(out);
        for (int hh = 0; hh < 8; ++hh)
          for (int t = 0; t < T; ++t)
            for (int d = 0; d < c.HD; ++d)
              o[(size_t)t * nq + hh * c.HD + d] = (float)f[hh * XT_QF + attn_qf_index(0, 4, c.HD / 32, t, d, 0)] +
                                                  (float)f[hh * XT_QF + attn_qf_index(0, 4, c.HD / 32, t, d, 1)];
        return 0;
      }
      default: MLCV_REQUIRE(false, "unknown probe");
    }
  }
  switch (what) {
    case MLCV_PROBE_X:
      MLCV_REQUIRE(bytes == (size_t)T * W1 * 2, "probe output size");
      MLCV_HIP(hipMemcpy(out, chain || xt ? c.x16 : p.xres + L * p.s_x, bytes, hipMemcpyDeviceToHost));
      return 0;
    case MLCV_PROBE_X_MID:
      MLCV_REQUIRE(bytes == (size_t)T * W1 * 2, "probe output size");
      MLCV_HIP(hipMemcpy(out, chain ? c.x16 : p.xmid + L * p.s_x, bytes, hipMemcpyDeviceToHost));
      return 0;
    case MLCV_PROBE_K:
      MLCV_REQUIRE(bytes == (size_t)T * nkv * 4, "probe output size");
      MLCV_HIP(hipMemcpy(out, chain ? c.k32 : p.k32 + L * p.s_k, bytes, hipMemcpyDeviceToHost));
      return 0;
    case MLCV_PROBE_V:
      MLCV_REQUIRE(bytes == (size_t)T * nkv * 2, "probe output size");
      MLCV_HIP(hipMemcpy(out, chain ? c.v : p.vs + L * p.s_k, bytes, hipMemcpyDeviceToHost));
      return 0;
    case MLCV_PROBE_ATTN: return frag_rows(chain ? c.attn : p.attn + L * p.s_attn, nq);
    case MLCV_PROBE_H: return frag_rows(chain ? c.h : p.h + L * p.s_h, c.F1);
    case MLCV_PROBE_VOUT:
      MLCV_REQUIRE(layer == 0 && bytes == (size_t)T * c.A * 4, "probe output size");
      MLCV_HIP(hipMemcpy(out, c.vout, bytes, hipMemcpyDeviceToHost));
      return 0;
    case MLCV_PROBE_Q: {  // hi + lo of the roped, scaled q fragments -> [T][H*hd] f32
      MLCV_REQUIRE(bytes == (size_t)T * nq * 4, "probe output size");
      MLCV_TRY(fetch(chain ? c.qf : p.qf + L * p.s_qf, qf_halfs * 2, raw));
      const _Float16* f = reinterpret_cast<const _Float16*>(raw.data());
      float* o = static_cast<float*>(out);
      const int grp = c.H / c.KV, ntiles = c.attn_rpad / 16, nks = (c.HD + 31) / 32;
      for (int t = 0; t < T; ++t)
        for (int h = 0; h < c.H; ++h)
          for (int d = 0; d < c.HD; ++d) {
            const int kvh = h / grp, row = (h % grp) * T + t;
            o[(size_t)t * nq + h * c.HD + d] = (float)f[attn_qf_index(kvh, ntiles, nks, row, d, 0)] +
                                              (float)f[attn_qf_index(kvh, ntiles, nks, row, d, 1)];
          }
      return 0;
    }
    case MLCV_PROBE_MOD: {  // the modulations [2D+1][3 W1] of the last step (first step of a loop)
      MLCV_REQUIRE(layer == 0 && bytes == (size_t)c.NM * 3 * W1 * 2, "probe output size");
      MLCV_HIP(hipMemcpy(out, c.mod, bytes, hipMemcpyDeviceToHost));
      return 0;
    }
    default: MLCV_REQUIRE(false, "unknown probe");
  }
}

int mlcv_bench_op(mlcv_ctx* ctx, int32_t op, int32_t layer, int32_t iters, const float* keys, const void* values,
                  void* stream) {
  MLCV_REQUIRE(ctx && iters >= 0, "bad argument");
  MLCV_REQUIRE(!ctx->f32, "step ops are not built for float32 models");
  Ctx& c = ctx->c;
  MLCV_REQUIRE(c.bound, "parameters not bound");
  MLCV_REQUIRE(layer >= 0 && layer < c.D, "layer out of range");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const _Float16* vals = reinterpret_cast<const _Float16*>(values);
  if (op == MLCV_OP_ATTENTION || op == MLCV_OP_ATTENTION_ONLY) MLCV_REQUIRE(keys && values, "attention needs keys and values");
  for (int i = 0; i < iters; ++i) {
    switch (op) {
      case MLCV_OP_TIME_MOD: MLCV_TRY(enqueue_time_mod(c, c.te, 1, st, false)); break;
      case MLCV_OP_MODULATION:
        if (c.mod_all.nseg > 0) {
          MLCV_TRY(run_op(c, c.mod_all, make_op(c, c.mod_all, c.cond, c.W1, 1), st));
        } else {
          for (const OpDesc& d : c.mod_ops) MLCV_TRY(run_op(c, d, make_op(c, d, c.cond, c.W1, 1), st));
        }
        break;
      case MLCV_OP_QKV: MLCV_TRY(enqueue_qkv(c, layer, c.mod, st)); break;
      case MLCV_OP_ATTENTION:
        c.use_img = false;
        MLCV_TRY(enqueue_attn(c, layer, keys, vals, st));
        break;
      case MLCV_OP_ATTENTION_ONLY: {
        c.use_img = false;
        const unsigned pf = c.prefetch;
        c.prefetch = 0;
        const int r = enqueue_attn(c, layer, keys, vals, st);
        c.prefetch = pf;
        MLCV_TRY(r);
        break;
      }
      case MLCV_OP_OPROJ: MLCV_TRY(enqueue_oproj(c, layer, c.mod, st)); break;
      case MLCV_OP_GATEUP: MLCV_TRY(enqueue_gateup(c, layer, c.mod, st)); break;
      case MLCV_OP_DOWN: MLCV_TRY(enqueue_down(c, layer, c.mod, st)); break;
      case MLCV_OP_HEAD:
        if (c.xt_on) {  // the XCD step's head: final reduce + norm + action_out_proj in one launch
          XtArgs x = c.xt;
          x.modp = c.mod;
          x.nscale = c.nscale;
          x.vout = c.vout;
          x.euler = 0;
          MLCV_TRY(xt_head_launch(x, st));
        } else {
          MLCV_TRY(enqueue_head(c, c.mod, false, st));
        }
        break;
      case MLCV_OP_ACTION_IN: MLCV_TRY(enqueue_action_in(c, c.mod, st)); break;
      case MLCV_OP_XT_ATTN:
      case MLCV_OP_XT_MLP: {
        MLCV_REQUIRE(c.xt_on, "the XCD step is off");
        XtArgs x = c.xt;  // the inputs of a single step, as enqueue_step sets them
        x.modp = c.mod;
        x.nscale = c.nscale;
        x.mask = c.mask;
        x.cos = c.cos;
        x.sin = c.sin;
        x.xin = c.xin16;
        x.L = layer;
        MLCV_REQUIRE(keys && values, "the XCD launches need keys and values");
        x.keys = keys;
        x.values = vals;
        if (op == MLCV_OP_XT_ATTN) MLCV_TRY(xt_attn_launch(x, st));
        else MLCV_TRY(xt_mlp_launch(x, st));
        break;
      }
      default: MLCV_REQUIRE(false, "unknown op");
    }
  }
  return 0;
}

// ---- kernel-level entry points ------------------------------------------------

namespace {
struct Scratch {
  std::mutex mu;
  float* ws = nullptr;
  size_t ws_n = 0;
  unsigned* meet = nullptr;  // meeting words of the one-launch attention (32 per row block, zeroed)
  size_t meet_n = 0;
  unsigned* counters = nullptr;
  size_t counters_n = 0;
  SkSeg* seg = nullptr;
  float* zero = nullptr;
};
Scratch g_scratch;

int scratch_reserve(size_t ws_n, size_t counters_n, size_t meet_n = 0) {
  if (!g_scratch.seg) MLCV_HIP(hipMalloc(&g_scratch.seg, sizeof(SkSeg)));
  if (!g_scratch.zero) {
    MLCV_HIP(hipMalloc(&g_scratch.zero, 64 * 64 * sizeof(float)));
    MLCV_HIP(hipMemset(g_scratch.zero, 0, 64 * 64 * sizeof(float)));
  }
  if (ws_n > g_scratch.ws_n) {
    if (g_scratch.ws) MLCV_HIP(hipFree(g_scratch.ws));
    MLCV_HIP(hipMalloc(&g_scratch.ws, ws_n * sizeof(float)));
    g_scratch.ws_n = ws_n;
  }
  if (meet_n > g_scratch.meet_n) {
    if (g_scratch.meet) MLCV_HIP(hipFree(g_scratch.meet));
    MLCV_HIP(hipMalloc(&g_scratch.meet, meet_n * sizeof(unsigned)));
    MLCV_HIP(hipMemset(g_scratch.meet, 0, meet_n * sizeof(unsigned)));
    g_scratch.meet_n = meet_n;
  }
  if (counters_n > g_scratch.counters_n) {
    if (g_scratch.counters) MLCV_HIP(hipFree(g_scratch.counters));
    MLCV_HIP(hipMalloc(&g_scratch.counters, counters_n * sizeof(unsigned)));
    MLCV_HIP(hipMemset(g_scratch.counters, 0, counters_n * sizeof(unsigned)));
    g_scratch.counters_n = counters_n;
  }
  return 0;
}
}  // namespace

static int tile_scratch(float** ws_out, unsigned** sync_out, unsigned** err_out, unsigned** err_dev_out);
static int tile_meet_failed(unsigned* err, const char* what);

int mlcv_joint_attention(const void* q, int32_t Tq, int32_t H, int32_t KV, int32_t hd, const void* kp,
                         int32_t k_f32, const void* vp, int32_t Sp, const float* mask, const void* ks,
                         const void* vs, int32_t Ts, void* out, void* stream) {
  MLCV_REQUIRE(q && kp && vp && out && Tq > 0 && H > 0 && KV > 0 && Sp >= 0 && Ts >= 0, "bad argument");
  MLCV_REQUIRE(Ts == 0 || (ks && vs), "suffix k/v missing");
  MLCV_REQUIRE(Sp + Ts > 0, "no keys");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  AttnArgs a{};
  a.q = reinterpret_cast<const _Float16*>(q);
  a.q_ld = H * hd;
  a.q_scale = 1.0f;
  a.Tq = Tq;
  a.H = H;
  a.KV = KV;
  a.hd = hd;
  a.kp = kp;
  a.kp_f32 = k_f32;
  a.vp = reinterpret_cast<const _Float16*>(vp);
  a.Sp = Sp;
  a.mask = mask;
  a.ks = reinterpret_cast<const _Float16*>(ks);
  a.ks_ld = KV * hd;
  a.vs = reinterpret_cast<const _Float16*>(vs);
  a.vs_ld = KV * hd;
  a.Ts = Ts;
  a.ks_roped = 1;
  a.out = reinterpret_cast<_Float16*>(out);
  a.out_ld = H * hd;
  a.rows = Tq * (H / KV);
  a.rpad = ((a.rows + 63) / 64) * 64;
  // decode shapes (head_dim 256, every workgroup resident at once): the attention and its split
  // combine in one launch, one 32-key chunk per prefix split (more when that gives more than 31),
  // the suffix keys as the last split
  {
    const int nch = (Sp + 31) / 32;
    const char* ke = std::getenv("MLCV_ATTN_FUSED_KPS");  // keys per prefix split (tuning)
    const int kps = ke ? std::max(32, std::atoi(ke) / 32 * 32) : 32 * std::max(1, (nch + 30) / 31);
    const int nsplit = (Sp + kps - 1) / kps + (Ts > 0 ? 1 : 0), nrb = a.rpad / 64 * KV;
    const char* fe = std::getenv("MLCV_ATTN_FUSED");
    if (hd == 256 && nsplit >= 2 && nsplit <= 32 && (nrb + 7) / 8 * nsplit * 8 <= device_cus() &&
        !(fe && std::atoi(fe) == 0)) {
      a.nsplit = nsplit;
      a.kps = kps;
      float* tws = nullptr;
      unsigned *tsync = nullptr, *err = nullptr, *err_dev = nullptr;
      MLCV_TRY(tile_scratch(&tws, &tsync, &err, &err_dev));
      MLCV_TRY(tile_meet_failed(err, "mlcv_joint_attention (an earlier call)"));
      std::lock_guard<std::mutex> lk(g_scratch.mu);
      MLCV_TRY(scratch_reserve(attn_ws_floats(KV, a.rows, hd, nsplit), 1, (size_t)32 * nrb));
      a.part_o = g_scratch.ws;
      a.part_ml = g_scratch.ws + (size_t)KV * a.nsplit * a.rpad * hd;
      return attn_fused_launch(a, g_scratch.meet, TG_MEET_POLLS, err_dev, st);
    }
  }
  attn_plan(a.rows, Sp, Ts, 128, &a.nsplit, &a.kps);
  std::lock_guard<std::mutex> lk(g_scratch.mu);
  const size_t need = attn_ws_floats(KV, a.rows, hd, a.nsplit);
  // the production path: prefix chunk images, then the attention over them
  const size_t img_floats = Sp > 0 ? (attn_img_bytes(KV, Sp, hd) + 3) / 4 : 0;
  MLCV_TRY(scratch_reserve(need + img_floats + 4, 1));
  a.part_o = g_scratch.ws;
  a.part_ml = g_scratch.ws + (size_t)KV * a.nsplit * a.rpad * hd;
  if (Sp > 0) {
    char* img = reinterpret_cast<char*>(g_scratch.ws + ((need + 3) / 4) * 4);
    MLCV_TRY(attn_img_prep_launch(kp, k_f32, a.vp, mask, 1, KV, Sp, hd, img, st));
    a.kimg = img;
    a.img_chunks = (Sp + 31) / 32;
  }
  return attn_launch(a, st);
}

int mlcv_prefill_attention(const void* q, int32_t q_ld, const float* cos, const float* sin, int32_t P, int32_t H,
                           int32_t KV, int32_t hd, const float* keys, const void* values, const float* mask, void* out,
                           void* stream) {
  MLCV_REQUIRE(q && cos && sin && keys && values && out && P > 0 && H > 0 && KV > 0 && hd > 0, "bad argument");
  MLCV_REQUIRE(q_ld >= H * hd && q_ld % 8 == 0, "q row stride");
  const int rows = P * (H / KV);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const char* pe = std::getenv("MLCV_PF_ATTN");
  if (pa_supported(hd, P, H, KV) && !(pe && std::atoi(pe) == 0)) {
    // the prefill's head_dim-256 attention: chunk images and q fragments from the cache slices
    const PaPlan plan = pa_plan(P, H, KV);
    auto up = [](size_t bytes) { return (bytes + 255) / 256 * 64; };  // floats, 256-byte multiples
    const size_t o_img = 0, o_qf = o_img + up(plan.img_bytes), o_part = o_qf + up(plan.qf_halfs * 2),
                 o_ml = o_part + up(plan.part_halfs * 2), n = o_ml + up(plan.ml_floats * 4);
    std::lock_guard<std::mutex> lk(g_scratch.mu);
    MLCV_TRY(scratch_reserve(n, plan.counters));
    float* ws = g_scratch.ws;
    char* img = reinterpret_cast<char*>(ws + o_img);
    _Float16* qf = reinterpret_cast<_Float16*>(ws + o_qf);
    MLCV_TRY(pa_writer_launch(reinterpret_cast<const _Float16*>(q), q_ld, 0, 0, cos, sin, P, H, KV,
                              1.0f / std::sqrt((float)hd), const_cast<float*>(keys),
                              reinterpret_cast<_Float16*>(const_cast<void*>(values)), plan, img, qf, 1, st));
    return pa_attn_launch(pa_args(plan, qf, img, mask, reinterpret_cast<_Float16*>(out), H * hd, P, H, KV,
                                  reinterpret_cast<_Float16*>(ws + o_part), ws + o_ml, g_scratch.counters, false),
                          st);
  }
  int nsplit = 1, kps = 32;
  attn_plan(rows, P, 0, prefill_attn_target(rows), &nsplit, &kps);
  std::lock_guard<std::mutex> lk(g_scratch.mu);
  // the attention's split partials, then (head dims a multiple of 64) q in fragment order,
  // 16-byte aligned -- the prefill's own sequence of launches
  const size_t ws_n = (attn_ws_floats(KV, rows, hd, nsplit) + 4 + 3) / 4 * 4;
  const int rpad = (rows + 63) / 64 * 64;
  const bool frag = hd % 64 == 0;
  MLCV_TRY(scratch_reserve(ws_n + (frag ? q_frag_halfs(KV, rpad, hd) / 2 : 0), 1));
  AttnArgs a = prefill_attn_args(reinterpret_cast<const _Float16*>(q), q_ld, cos, sin, P, H, KV, hd, keys,
                                 reinterpret_cast<const _Float16*>(values), mask, reinterpret_cast<_Float16*>(out),
                                 nsplit, kps, g_scratch.ws);
  if (frag) {
    _Float16* qf = reinterpret_cast<_Float16*>(g_scratch.ws + ws_n);
    MLCV_TRY(q_frag_launch(reinterpret_cast<const _Float16*>(q), q_ld, cos, sin, P, H, KV, hd, a.q_scale, a.rpad, qf,
                           st));
    a.qf = qf;
  }
  return attn_launch(a, st);
}

int mlcv_q4_quantize(const void* w, uint32_t* q_weight, void* q_scale, int32_t N, int32_t K, void* stream) {
  MLCV_REQUIRE(w && q_weight && q_scale && N > 0 && K > 0, "bad argument");
  return q4_quantize_launch(reinterpret_cast<const _Float16*>(w), q_weight, reinterpret_cast<_Float16*>(q_scale), N,
                            K, reinterpret_cast<hipStream_t>(stream));
}

int mlcv_q4_dequantize(const uint32_t* q_weight, const void* q_scale, void* w, int32_t N, int32_t K, void* stream) {
  MLCV_REQUIRE(w && q_weight && q_scale && N > 0 && K > 0, "bad argument");
  return q4_dequant_launch(q_weight, reinterpret_cast<const _Float16*>(q_scale), reinterpret_cast<_Float16*>(w), N,
                           K, reinterpret_cast<hipStream_t>(stream));
}

// split-K workspace and meeting counters of the standalone tile-GEMM entry points (per
// device, kept until the process ends; the callers serialize on tile_mu)
static std::mutex tile_mu;
// Per-device split-K scratch of the tile GEMM entry points (mlcv_tile_linear, mlcv_embed_image):
// partials, meeting counters and the meetings' error word (pinned host memory: *err_out its
// host address, *err_dev_out its device address).
static int tile_scratch(float** ws_out, unsigned** sync_out, unsigned** err_out, unsigned** err_dev_out) {
  static float* ws[64] = {};
  static unsigned* sync[64] = {};
  static unsigned* err[64] = {};
  static unsigned* err_dev[64] = {};
  int dev = 0;
  MLCV_HIP(hipGetDevice(&dev));
  MLCV_REQUIRE(dev >= 0 && dev < 64, "device index");
  if (!err[dev]) {
    MLCV_HIP(hipHostMalloc(reinterpret_cast<void**>(&err[dev]), sizeof(unsigned),
                           hipHostMallocMapped | hipHostMallocCoherent));
    MLCV_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&err_dev[dev]), err[dev], 0));
    *err[dev] = 0;
  }
  if (!ws[dev]) {
    MLCV_HIP(hipMalloc(&ws[dev], tg_ws_floats() * sizeof(float)));
    MLCV_HIP(hipMalloc(&sync[dev], tg_sync_words() * sizeof(unsigned)));
    MLCV_HIP(hipMemset(sync[dev], 0, tg_sync_words() * sizeof(unsigned)));
  }
  *ws_out = ws[dev];
  *sync_out = sync[dev];
  *err_out = err[dev];
  *err_dev_out = err_dev[dev];
  return 0;
}

// a split-K meeting of an earlier call on this device's scratch gave up: report it once
static int tile_meet_failed(unsigned* err, const char* what) {
  const unsigned e = __atomic_load_n(err, __ATOMIC_ACQUIRE);
  if (e == 0) return 0;
  __atomic_store_n(err, 0u, __ATOMIC_RELEASE);
  set_error(std::string(what) + ": a meeting of split workgroups gave up (error word " + std::to_string(e) +
            "; other work held the CUs the split workgroups need); that output is invalid");
  return -4;
}

static VisionCfg vision_cfg(const mlcv_vision_config& c) {
  return VisionCfg{c.image_size, c.patch_size, c.num_channels, c.hidden_size, c.intermediate_size,
                   c.num_hidden_layers, c.num_attention_heads, c.projection_dim, c.layer_norm_eps};
}

int mlcv_vision_param_count(const mlcv_vision_config* cfg, int32_t* count) {
  MLCV_REQUIRE(cfg && count && cfg->num_hidden_layers >= 0, "bad argument");
  *count = 3 + 16 * cfg->num_hidden_layers + 4;
  return 0;
}

// the caller's workspace: [image copy | output | the tower's buffers], 256-byte aligned parts
static size_t vis_io_bytes(const mlcv_vision_config& c, size_t* img_b, size_t* out_b) {
  const size_t np = (size_t)(c.image_size / c.patch_size) * (c.image_size / c.patch_size);
  *img_b = ((size_t)c.image_size * c.image_size * c.num_channels * 2 + 255) / 256 * 256;
  *out_b = (np * c.projection_dim * 2 + 255) / 256 * 256;
  return *img_b + *out_b + 256;
}

int mlcv_embed_image_workspace(const mlcv_vision_config* cfg, size_t* bytes) {
  MLCV_REQUIRE(cfg && bytes && cfg->patch_size > 0, "bad argument");
  size_t ib = 0, ob = 0;
  *bytes = vis_io_bytes(*cfg, &ib, &ob) + vision_ws_bytes(vision_cfg(*cfg));
  return 0;
}

int mlcv_embed_image(const mlcv_vision_config* cfg, const void* const* params, int32_t count, const void* image,
                     void* out, void* workspace, size_t workspace_bytes, void* stream) {
  MLCV_REQUIRE(cfg && params && image && out && workspace, "null argument");
  MLCV_REQUIRE(cfg->image_size > 0 && cfg->patch_size > 0 && cfg->num_channels > 0 && cfg->hidden_size > 0 &&
                   cfg->intermediate_size > 0 && cfg->num_hidden_layers >= 0 && cfg->num_attention_heads > 0 &&
                   cfg->projection_dim > 0,
               "bad vision config");
  MLCV_REQUIRE(count == 3 + 16 * cfg->num_hidden_layers + 4, "vision parameter count");
  for (int i = 0; i < count; ++i) MLCV_REQUIRE(params[i] != nullptr, "null vision parameter");
  std::lock_guard<std::mutex> lk(tile_mu);
  float* gws = nullptr;
  unsigned *gsync = nullptr, *gerr = nullptr, *gerr_dev = nullptr;
  MLCV_TRY(tile_scratch(&gws, &gsync, &gerr, &gerr_dev));
  // an earlier image whose GEMM meeting gave up is reported here (this call is not run)
  MLCV_TRY(tile_meet_failed(gerr, "an earlier mlcv_embed_image or mlcv_tile_linear call"));
  // the ~330 launches of one image run as a hipGraph, captured on a private stream and kept
  // per device; a call with other pointers or another config captures again
  struct VisGraph {
    std::vector<const void*> key;
    hipGraphExec_t exec = nullptr;
    hipStream_t cap = nullptr;
  };
  static VisGraph graphs[64];
  int dev = 0;
  MLCV_HIP(hipGetDevice(&dev));
  MLCV_REQUIRE(dev >= 0 && dev < 64, "device index");
  VisGraph& G = graphs[dev];
  if (!G.cap) MLCV_HIP(hipStreamCreateWithFlags(&G.cap, hipStreamNonBlocking));
  size_t img_b = 0, out_b = 0;
  const size_t io = vis_io_bytes(*cfg, &img_b, &out_b);
  MLCV_REQUIRE(workspace_bytes >= io, "vision workspace too small");
  char* wbase = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(workspace) + 255) & ~uintptr_t(255));
  _Float16* wimg = reinterpret_cast<_Float16*>(wbase);
  _Float16* wout = reinterpret_cast<_Float16*>(wbase + img_b);
  char* wrest = wbase + img_b + out_b;
  const size_t rest_bytes = workspace_bytes - (size_t)(wrest - static_cast<char*>(workspace));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  std::vector<const void*> key(params, params + count);
  key.push_back(workspace);
  for (int f : {cfg->image_size, cfg->patch_size, cfg->num_channels, cfg->hidden_size, cfg->intermediate_size,
                cfg->num_hidden_layers, cfg->num_attention_heads, cfg->projection_dim})
    key.push_back(reinterpret_cast<const void*>((intptr_t)f));
  key.push_back(reinterpret_cast<const void*>((intptr_t)__builtin_bit_cast(int32_t, cfg->layer_norm_eps)));
  key.push_back(reinterpret_cast<const void*>((uintptr_t)workspace_bytes));
  if (!G.exec || G.key != key) {
    if (G.exec) (void)hipGraphExecDestroy(G.exec);
    G.exec = nullptr;
    G.key.clear();
    MLCV_HIP(hipStreamBeginCapture(G.cap, hipStreamCaptureModeThreadLocal));
    const int r = embed_image_enqueue(vision_cfg(*cfg), reinterpret_cast<const _Float16* const*>(params), wimg,
                                      wout, wrest, rest_bytes, gws, tg_ws_floats(), gsync,
                                      (int)(tg_sync_words() / 32), gerr_dev, G.cap);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(G.cap, &graph);
    if (r != 0) {
      if (e == hipSuccess && graph) (void)hipGraphDestroy(graph);
      return r;
    }
    MLCV_HIP(e);
    const hipError_t ie = hipGraphInstantiate(&G.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    MLCV_HIP(ie);
    G.key = key;
  }
  const size_t img_bytes = (size_t)cfg->image_size * cfg->image_size * cfg->num_channels * 2;
  const size_t out_bytes = (size_t)(cfg->image_size / cfg->patch_size) * (cfg->image_size / cfg->patch_size) *
                           cfg->projection_dim * 2;
  MLCV_HIP(hipMemcpyAsync(wimg, image, img_bytes, hipMemcpyDeviceToDevice, st));
  MLCV_HIP(hipGraphLaunch(G.exec, st));
  MLCV_HIP(hipMemcpyAsync(out, wout, out_bytes, hipMemcpyDeviceToDevice, st));
  return 0;
}

int mlcv_tile_linear(const void* x, int32_t M, int32_t K, const void* w, int32_t N, void* y, int32_t epi,
                     int32_t small_tiles, int32_t meet_polls, void* stream) {
  MLCV_REQUIRE(x && w && y && M > 0 && K > 0 && N > 0, "bad argument");
  MLCV_REQUIRE(epi == TG_STORE || epi == TG_RESIDUAL || epi == TG_GEGLU, "unknown epilogue");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> lk(tile_mu);
  float* gws = nullptr;
  unsigned *gsync = nullptr, *gerr = nullptr, *gerr_dev = nullptr;
  MLCV_TRY(tile_scratch(&gws, &gsync, &gerr, &gerr_dev));
  TgArgs g{};
  g.a = reinterpret_cast<const _Float16*>(x);
  g.lda = K;
  g.b0 = g.b1 = g.b2 = reinterpret_cast<const _Float16*>(w);
  g.n1 = g.n2 = epi == TG_GEGLU ? 2 * N : N;
  g.ldb = K;
  g.c = reinterpret_cast<_Float16*>(y);
  g.ldc = N;
  g.M = M;
  g.N = N;
  g.K = K;
  g.epi = epi;
  g.F = N;
  g.ws = gws;
  g.ws_floats = tg_ws_floats();
  g.sync = gsync;
  g.sync_tiles = (int)(tg_sync_words() / 32);
  g.small_tiles = small_tiles ? 1 : 0;
  g.err = gerr_dev;
  g.meet_polls = meet_polls < 0 ? TG_MEET_POLLS : (unsigned)meet_polls;
  MLCV_HIP(hipStreamSynchronize(st));
  MLCV_TRY(tile_meet_failed(gerr, "an earlier mlcv_embed_image call"));
  MLCV_TRY(tg_launch(g, st));
  MLCV_HIP(hipStreamSynchronize(st));
  return tile_meet_failed(gerr, "mlcv_tile_linear");
}

int mlcv_linear(const void* x, int32_t M, int32_t K, const void* w, const uint32_t* q_weight, const void* q_scale,
                const void* bias, void* y, int32_t N, void* stream) {
  MLCV_REQUIRE(x && y && M > 0 && K > 0 && N > 0, "bad argument");
  MLCV_REQUIRE((w != nullptr) != (q_weight != nullptr && q_scale != nullptr), "pass either w or q_weight+q_scale");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  SkSeg s{};
  s.w = reinterpret_cast<const _Float16*>(w);
  s.qw = q_weight;
  s.qs = reinterpret_cast<const _Float16*>(q_scale);
  s.bias = reinterpret_cast<const _Float16*>(bias);
  s.out = y;
  s.n = N;
  s.ldo = N;
  s.tile0 = 0;
  const int ntiles = (N + 63) / 64, mb = (M + 63) / 64;
  const SkPlan p = sk_plan(ntiles, K, mb, 0);
  std::lock_guard<std::mutex> lk(g_scratch.mu);
  MLCV_TRY(scratch_reserve(sk_ws_floats(ntiles, mb, p, 64), (size_t)ntiles * mb));
  MLCV_HIP(hipStreamSynchronize(st));
  MLCV_HIP(hipMemcpy(g_scratch.seg, &s, sizeof(SkSeg), hipMemcpyHostToDevice));
  SkOp op{};
  op.x = reinterpret_cast<const _Float16*>(x);
  op.ldx = K;
  op.M = M;
  op.K = K;
  op.epi = EPI_STORE;
  op.segs = g_scratch.seg;
  op.nseg = 1;
  op.inl[0] = s;
  op.ntiles = ntiles;
  op.tr = 64;
  op.splitk = p.splitk;
  op.kper = p.kper;
  op.ws = g_scratch.ws;
  op.zero = g_scratch.zero;
  op.counters = g_scratch.counters;
  MLCV_TRY(sk_launch(op, q_weight != nullptr, st));
  MLCV_HIP(hipStreamSynchronize(st));
  return 0;
}

int mlcv_linear_noalloc(const void* x, int32_t M, int32_t K, const void* w, const uint32_t* q_weight,
                        const void* q_scale, const void* bias, void* y, int32_t N, void* stream) {
  MLCV_REQUIRE(x && y && M > 0 && K > 0 && N > 0, "bad argument");
  MLCV_REQUIRE((w != nullptr) != (q_weight != nullptr && q_scale != nullptr), "pass either w or q_weight+q_scale");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int ntiles = (N + 63) / 64, mb = (M + 63) / 64;
  const SkPlan p = sk_plan(ntiles, K, mb, 0);
  MLCV_REQUIRE((size_t)ntiles * mb <= NA_COUNTERS,
               "mlcv_linear_noalloc: ceil(M/64) * ceil(N/64) = " + std::to_string((size_t)ntiles * mb) +
                   " output tiles, above its maximum of " + std::to_string(NA_COUNTERS));
  MLCV_REQUIRE(sk_ws_floats(ntiles, mb, p, 64) <= NA_PART_FLOATS,
               "mlcv_linear_noalloc: the split-K partials exceed its scratch of " + std::to_string(NA_PART_FLOATS * 4) +
                   " bytes");
  char* base = nullptr;
  MLCV_TRY(noalloc_scratch(st, &base));
  SkSeg s{};
  s.w = reinterpret_cast<const _Float16*>(w);
  s.qw = q_weight;
  s.qs = reinterpret_cast<const _Float16*>(q_scale);
  s.bias = reinterpret_cast<const _Float16*>(bias);
  s.out = y;
  s.n = N;
  s.ldo = N;
  s.tile0 = 0;
  SkOp op{};
  op.x = reinterpret_cast<const _Float16*>(x);
  op.ldx = K;
  op.M = M;
  op.K = K;
  op.epi = EPI_STORE;
  op.nseg = 1;  // one segment: passed inline, no segment table
  op.inl[0] = s;
  op.ntiles = ntiles;
  op.tr = 64;
  op.splitk = p.splitk;
  op.kper = p.kper;
  op.zero = reinterpret_cast<float*>(base);
  op.counters = reinterpret_cast<unsigned*>(base + NA_ZERO_FLOATS * 4);
  op.ws = reinterpret_cast<float*>(base + (NA_ZERO_FLOATS + NA_COUNTERS) * 4);
  return sk_launch(op, q_weight != nullptr, st);
}

}  // extern "C"
