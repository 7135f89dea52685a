// Kernel launch interfaces shared by the engine (host side).
#pragma once

#include "common.h"
#include "plan.h"

struct mlcv_config;  // include/mlcvla.h

namespace mlcv {

// ---------------------------------------------------------------------------
// Prefetch by spare workgroups.  A launch can append `nblocks` workgroups that only read
// the regions a later kernel of the sequence will read, so that the later kernel finds
// them in the memory-side cache (and, where the XCD's L2 keeps them across the launch
// boundary, in the L2 of the XCD its workgroups run on: workgroups are dealt to the 8
// XCDs round-robin by linear id, and a consumer tile t of a grid whose x extent is a
// multiple of 8 runs on XCD t % 8).  The loads touch one dword per 64-byte line and
// change nothing; a wrong guess of the placement costs only the extra reads.
// ---------------------------------------------------------------------------
struct PfRegion {
  const char* base;
  int slab_bytes;  // a multiple of 64
  int nslabs;
  int xoff;        // slab j is read on XCD (j + xoff) % 8 ...
  int every_xcd;   // ... or, when set, on every XCD
};
constexpr int PF_MAX_REGIONS = 6;
struct Prefetch {
  PfRegion r[PF_MAX_REGIONS];
  int nreg;
  int nblocks;     // prefetch workgroups (the launch rounds this up to whole grid rows)
  unsigned* sink;  // null: the loaded values are discarded (a non-null sink keeps them)
};

// In a prefetch workgroup: `lin` = its linear workgroup id, `lin0` = the linear id of the
// launch's first prefetch workgroup.  The lines of the slabs this XCD reads are spread
// over the XCD's prefetch workgroups, 16 loads in flight per lane (any workgroup size).
// prefetch_ranked: the workgroup of rank `rank` among the `nrank` prefetch workgroups of XCD
// `xcd`.
__device__ inline void prefetch_ranked(const Prefetch& pf, int xcd, int rank, int nrank) {
  const int tid = threadIdx.x, nt = blockDim.x;
  unsigned acc = 0;
  for (int ri = 0; ri < pf.nreg; ++ri) {
    const PfRegion R = pf.r[ri];
    const int lps = R.slab_bytes >> 6;
    const int first = R.every_xcd ? 0 : (xcd - R.xoff) & 7;
    const int step = R.every_xcd ? 1 : 8;
    const int nsl = R.every_xcd ? R.nslabs : (R.nslabs - first + 7) >> 3;
    const int nlines = nsl * lps;
    const int gstep = nrank * nt;
    for (int g = rank * nt + tid; g < nlines; g += 16 * gstep) {
      unsigned v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int gg = min(g + u * gstep, nlines - 1);
        const int j = gg / lps, off = gg - j * lps;
        v[u] = load_global(reinterpret_cast<const unsigned*>(R.base + (size_t)(first + step * j) * R.slab_bytes +
                                                             (size_t)off * 64));
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) acc ^= v[u];
    }
  }
  if (pf.sink) pf.sink[tid] = acc;
}
__device__ inline void prefetch_run(const Prefetch& pf, int lin, int lin0) {
  const int xcd = lin & 7;
  const int p = lin - lin0;
  const int p0 = (xcd - lin0) & 7;  // the first prefetch workgroup on this XCD
  prefetch_ranked(pf, xcd, (p - p0) >> 3, (pf.nblocks - p0 + 7) >> 3);
}

// ---------------------------------------------------------------------------
// skinny GEMM: Y[M, N] = X[M, K] . W[N, K]^T for M <= 64 per m-block, fp16 or
// q4f16_1 weights, fp32 accumulation on MFMA 16x16x32, fused prologue/epilogue.
// ---------------------------------------------------------------------------
enum SkEpi : int {
  EPI_STORE = 0,       // out = fp16(acc) [+ fp16 bias]
  EPI_STORE_SILU = 1,  // out = fp16(silu(fp16(acc) + bias))
  EPI_GATED_RES = 2,   // x = fp16(x + fp16(fp16(acc) * gate))      (in place)
  EPI_GEGLU = 3,       // h = fp16(fp16(gelu(fp16(acc_gate))) * fp16(acc_up))
  EPI_VOUT = 4,        // v = f32(fp16(fp16(acc) + bias))
  EPI_EULER = 5,       // x32 += dt * f32(fp16(fp16(acc) + bias)); x16 = fp16(x32)
};

// One weight matrix (segment) of a skinny GEMM launch; tiles of 64 output rows.
struct SkSeg {
  const _Float16* w;     // [n][K] fp16 row-major (null for q4)
  const uint32_t* qw;    // [n][K/8] packed nibbles (q4)
  const _Float16* qs;    // [n][K/32] fp16 group scales (q4)
  const _Float16* bias;  // [n] or null
  void* out;             // output base (element type depends on the epilogue)
  int n;                 // output rows of this segment
  int tile0;             // first tile id of this segment
  int ldo;               // output stride between m rows (elements)
  // RoPE in the store epilogue (fragment-major 16-row tiles whose weight rows are paired
  // (d, d + hd/2), see wf_shuffle_launch): 1 = q, written scaled as fp16 hi/lo in the
  // attention's B-fragment order (attn_qf_index); 2 = k, written as fp32 [m][ldo]
  int rope;
};

struct SkOp {
  const _Float16* x;     // X [M][ldx]
  int ldx, M, K;
  // adaRMS prologue: xn = fp16((x / sqrt(mean(x^2)+eps)) * (1 + scale) + shift)
  const _Float16* scale; // [K] or null (no per-element prologue)
  const _Float16* shift; // [K]
  float eps;
  // row sums of squares of the residual stream, one partial per 16-column group:
  // read by the prologue (rowss_in, rowss_tiles partials) and written by epilogues
  // that produce x (rowss_out); element [m * rowss_ld + group]
  const float* rowss_in;
  float* rowss_out;
  int rowss_ld, rowss_tiles;
  // pre-scaled adaRMS (consumer, M < 64): X rows [0, M) hold fp16(x * (1 + scale)) and
  // row M holds the shift, so the product needs no per-element prologue; the epilogue
  // forms y = acc[m] / sqrt(mean(x^2) + eps) + acc[M] from the row statistics
  bool prescaled;
  // producer side: with xu_out set, the STORE / GATED_RES epilogues also write
  // xu_out[m][n] = fp16(x[m][n] * (1 + xu_scale[n])) and xu_out[M][n] = xu_shift[n]
  // (stride ldo, M < 64): the next adaRMS GEMM's pre-scaled X
  _Float16* xu_out;
  const _Float16* xu_scale;
  const _Float16* xu_shift;
  // power-of-two prescale of that norm (nscale_launch), or null for 1: the pre-scaled copy
  // is fp16(x * (1 + scale) * c) with |1 + scale| c <= 1, so it stays as finite as x itself;
  // the consumer (prescaled, nsc) divides its row factor by the same c
  const float* xu_nsc;
  const float* nsc;
  // fragment-major operands (16-row tiles, M < 64, K % 128 == 0): X in the xf_index
  // layout, the weights pre-shuffled by wf_shuffle_launch
  bool frag;
  // the GeGLU output and xu_out are written in the xf_index layout (M < 64)
  bool frag_out;
  // row-major X with M <= 16 and fragment-major weights (16-row tiles, no prologue):
  // the small-M time MLP and modulation GEMVs
  bool xrow;
  // RoPE segments (SkSeg::rope): tables [M][hd/2] fp32, q scale, head dim, q heads per
  // kv head and the attention's padded rows per kv head
  const float* rope_cos;
  const float* rope_sin;
  float rope_scale;
  int rope_hd, rope_grp, rope_rpad;
  int epi;
  const _Float16* gate;  // [N] (EPI_GATED_RES)
  int geglu_F;           // EPI_GEGLU: rows [0,F) gate, [F,2F) up
  SkSeg inl[3];          // segments passed by value (nseg <= 3)
  const SkSeg* segs;     // device table when nseg > 3
  int nseg, ntiles;
  int seg_tiles;         // > 0: every segment has this many tiles (direct table index)
  int tr;                // weight rows per tile: 16, 32 or 64 (GeGLU: half gate, half up)
  int mg;                // m groups per 64-row block (0 or 1: none; 2 or 4: fragment-major
                         // 16-row tiles, 4 / mg m tiles per workgroup, plus the shift row's
                         // tile with pre-scaled input); the split-K workspace and counters
                         // then cover ntiles * mblocks * mg
  int splitk, kper;
  float* ws;             // split-K partials
  const float* zero;     // >= 64*64 zero floats, never written (absent bias)
  unsigned* counters;    // per (tile, m-block), zero between launches
  float dt;              // EPI_EULER
  float* x32;            // EPI_EULER state [M][ldo]
  _Float16* x16;         // EPI_EULER fp16 copy
  Prefetch pf;           // prefetch workgroups appended as grid rows y >= splitk
};

int sk_launch(const SkOp& op, bool q4, hipStream_t st);
// Prescale of pre-scaled adaRMS inputs: for steps x norms_n modulation vectors [3 W1] (scale,
// shift, gate) at mod + (step * NM + norm_lo + j) * 3 W1, out[step * NM + norm_lo + j] = 2^-e
// with e >= 0 the least such that max_k |1 + scale_k| 2^-e <= 1 (1 for a non-finite scale).
int nscale_launch(const _Float16* mod, int W1, int NM, int steps, int norm_lo, int norms_n, float* out,
                  hipStream_t st);

// fragment-major copies of the weights of 16-row slabs for the 16-row skinny tiles:
// fp16 block (slab s, k step ks) = 1 KB, lane 16 g + r holding W[row(s, r)][32 ks + 8 g ..
// +7]; q4 block (s, 128-k chunk c) = 1 KB of words, lane 16 g + r holding the 4 words of
// row(s, r) for k = 128 c + 32 g .. +31, and 64 scales in lane order.  row(s, r) = 16 s + r;
// with geglu_F > 0 gate row 8 s + r (r < 8) and up row F + 8 s + r - 8; with rope_hd > 0
// (heads of rope_hd rows, slab j of head h) h hd + 8 j + r (r < 8) and h hd + hd/2 + 8 j + r - 8.
int wf_shuffle_launch(const _Float16* w, _Float16* wf, int N, int K, int geglu_F, int rope_hd, hipStream_t st);
int wf_shuffle_q4_launch(const uint32_t* qw, const _Float16* qs, uint32_t* qwf, _Float16* qsf, int N, int K,
                         int geglu_F, int rope_hd, hipStream_t st);

// q4f16_1 helpers
int q4_quantize_launch(const _Float16* w, uint32_t* qw, _Float16* qs, int N, int K, hipStream_t st);
int q4_dequant_launch(const uint32_t* qw, const _Float16* qs, _Float16* out, int N, int K, hipStream_t st);

// ---------------------------------------------------------------------------
// joint attention (suffix-over-cached-prefix, MQA/GQA broadcast), split-KV
// ---------------------------------------------------------------------------
struct AttnArgs {
  const _Float16* q;     // raw q [Tq][q_ld], head h at h*hd
  const _Float16* qf;    // or: q roped and scaled, fp16 hi/lo in B-fragment order (attn_qf_index)
  const float* ks32;     // with qf: suffix k roped, fp32 [Ts][ks_ld]
  int q_ld;
  const float* cos;      // [Tq][hd/2] rope for q (and suffix k); null = already roped
  const float* sin;
  float q_scale;         // applied after rope
  int Tq, H, KV, hd;
  const void* kp;        // prefix K [KV][Sp][hd], roped; fp32 (kp_f32) or fp16
  int kp_f32;
  const _Float16* vp;    // prefix V [KV][Sp][hd]
  int Sp;
  const float* mask;     // [Sp] additive, or null
  const _Float16* ks;    // suffix k raw [Ts][ks_ld] (head kvh at kvh*hd), or null
  int ks_ld;
  const _Float16* vs;    // suffix v [Ts][vs_ld]
  int vs_ld;
  int Ts;
  int ks_roped;          // suffix k already roped
  _Float16* out;         // [Tq][out_ld], head h at h*hd
  int out_ld;
  int out_frag;          // out in the fragment-major layout (xf_index, Tq <= 64, K = H*hd)
  const char* kimg;      // prefix chunk images of this layer [KV][img_chunks] (attn_img_prep_launch), or null
  int img_chunks;
  float* part_o;         // [KV][nsplit][Rpad][hd] fp16 O_s / l_s (the buffer is sized in floats)
  float* part_ml;        // [KV][nsplit][Rpad][2]
  int nsplit, kps;       // splits (the last one is the suffix block when Ts > 0), prefix keys per split
  int rows, rpad;        // rows per kv head (Tq*H/KV) and padded
  Prefetch pf;           // prefetch workgroups appended as grid rows y >= nsplit
  // XCD-grouped order (8-wave q-fragment form): grid (8, Y, KV), column x runs on XCD x and
  // takes every row block of the splits x, x + 8, ..., then pf.nblocks / 8 prefetch
  // workgroups, so a split's K/V is read into one XCD's L2 for all its row blocks
  int xgroup;
  int noskip;            // 1: compute key chunks whose keys are all masked too (testing the skip)
};
// nsplit = prefix key splits of kps keys (a multiple of 32) + 1 split for the suffix block (Ts > 0)
// prefix K (split hi/lo), V (transposed) and mask of `layers` consecutive layers (keys /
// values [layers][KV][Sp][hd]) as per-chunk LDS images: attn_img_bytes(KV, Sp, hd) bytes per layer
size_t attn_img_bytes(int KV, int Sp, int hd);
int attn_img_prep_launch(const void* keys, int k_f32, const _Float16* values, const float* mask, int layers, int KV,
                         int Sp, int hd, char* img, hipStream_t st);
int attn_launch(const AttnArgs& a, hipStream_t st);
// the attention and its split combine in one launch (head_dim 256, at most 32 splits, every
// workgroup resident at once: (row blocks rounded up to 8) x nsplit <= CUs); meet: 32 zeroed
// words per row block, kept between calls; a meeting that runs out of `polls` raises *err
// (pinned host memory) and writes NaN rows
int attn_fused_launch(const AttnArgs& a, unsigned* meet, unsigned polls, unsigned* err, hipStream_t st);

// prefill helpers
// tile: the output in the prefill GEMM's tile-major layout [ceil(rows / 16)][dim / 32][16][32]
int rmsnorm_launch(const _Float16* x, const _Float16* w, _Float16* out, int rows, int dim, float eps,
                   hipStream_t st, bool tile = false);
int kv_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin,
                     int P, int KV, int hd, float* keys, _Float16* values, hipStream_t st);
// q of the prefill [P][ld] (heads of hd columns from column 0) roped with cos / sin [P][hd/2],
// scaled by q_scale and split fp16 hi + lo into the attention's fragment order (attn_qf_index,
// rows = P * H/KV padded to rpad, the padding rows zero); hd % 64 == 0.  The attention then
// reads q as the step's attention does (AttnArgs::qf).
int q_frag_launch(const _Float16* q, int ld, const float* cos, const float* sin, int P, int H, int KV, int hd,
                  float q_scale, int rpad, _Float16* qf, hipStream_t st);
inline size_t q_frag_halfs(int KV, int rpad, int hd) { return (size_t)KV * rpad * hd * 2; }
// kv_writer_launch and q_frag_launch in one launch (where both apply; qf null: K/V only)
int kvq_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin, int P,
                      int H, int KV, int hd, float* keys, _Float16* values, float q_scale, int rpad, _Float16* qf,
                      hipStream_t st);

// ---------------------------------------------------------------------------
// The prefill's attention at head_dim 256 (attn_prefill.hip): per-chunk K/V images and q fragments
// from the layer's writer, 128 query rows per workgroup on 32x32x16 MFMAs, key splits balanced
// over the chunks holding a valid key, the splits combined by the last to arrive.
struct PaPlan {
  int nch;            // 32-key chunks
  int nrb;            // 128-row blocks per kv head
  int nsplit;         // key splits
  size_t img_bytes;   // chunk images [KV][nch][48 KB]
  size_t qf_halfs;    // q fragments [KV][nrb * 128 rows][256][hi, lo]
  size_t part_halfs;  // the splits' fp16 O / l
  size_t ml_floats;   // the splits' (m, l)
  size_t counters;    // arrival counters [KV][nrb] (zero between launches)
};
struct PaArgs {
  const _Float16* qf;   // q fragments (pa_writer_launch)
  const char* img;      // chunk images of this layer
  const float* mask;    // [P] additive, or null
  _Float16* out;        // [P][out_ld], head h at h * 256
  int out_ld;
  int P, H, KV, rows;   // rows = P * H / KV per kv head
  int nch, nrb, nsplit;
  _Float16* part;
  float* part_ml;
  unsigned* ctr;
  int noskip;           // 1: compute chunks whose keys are all masked too (same splits)
  int dev_combine;      // 1: the combine reads at device scope even with every split on one XCD
};
bool pa_supported(int hd, int P, int H, int KV);
PaPlan pa_plan(int P, int H, int KV);
// the layer's K/V cache slices (fp32 roped K, fp16 V from the q/k/v rows), the chunk images and q's
// fragments in one launch; from_cache: images from the cache slices keys / values (read, not
// written) and q from the rows [P][ld]
int pa_writer_launch(const _Float16* qkv, int ld, int koff, int voff, const float* cos, const float* sin, int P, int H,
                     int KV, float q_scale, float* keys, _Float16* values, const PaPlan& plan, char* img, _Float16* qf,
                     int from_cache, hipStream_t st);
int pa_attn_launch(const PaArgs& a, hipStream_t st);

// tiled GEMM for prefill: C[M,N] = A[M,K] . B[N,K]^T, MFMA 32x32x16
// ---------------------------------------------------------------------------
enum TgEpi : int {
  TG_STORE = 0,     // C fp16
  TG_RESIDUAL = 1,  // C = fp16(C + fp16(acc))
  TG_GEGLU = 2,     // B rows interleaved gate/up per 32-col block; C = h [M][F]
};
constexpr unsigned TG_MEET_POLLS = 1u << 22;
constexpr unsigned TG_ERR_MEET = 2;
struct TgArgs {
  const _Float16* a; int lda;
  const _Float16* b0; const _Float16* b1; const _Float16* b2;  // up to 3 stacked weight segments
  int n1, n2;            // segment boundaries in N (b1 rows start at n1, b2 at n2)
  int ldb;
  _Float16* c; int ldc;
  int M, N, K;
  int epi;
  int F;                 // TG_GEGLU: up rows offset in b0
  // split-K of the 256-row tile path (narrow N): partials workspace and per-tile meeting
  // counters (32 words per tile, zero at allocation); null = no split-K
  float* ws;
  size_t ws_floats;
  unsigned* sync;
  int sync_tiles;
  int small_tiles;       // 1: the 128 x 128 tile kernel only
  // the split-K meeting's bounded wait: polls before a workgroup gives up; it then writes NaN
  // into its part of the output and stores TG_ERR_MEET into *err (pinned host memory that the
  // entry points read back), when err is set
  unsigned meet_polls = TG_MEET_POLLS;
  unsigned* err = nullptr;
  // optional tile-major copy of b0 for the 32-k tiles: [rows / 16][K / 32][16][32] halfs (one
  // DMA instruction of 16 rows x 64 B then reads one contiguous 1 KB); only with one weight
  // segment or GeGLU; null: b0 row-major
  const _Float16* bt = nullptr;
  // the 32-k tiles' X (a) read / GeGLU output (c) written tile-major [ceil(rows / 16)][K / 32][16][32]
  // (a: its buffer holds whole 16-row blocks; rows past M are never stored to by c)
  int at = 0, ct = 0;
};
// whether tg_launch runs this GEMM on the 256 x 256 tiles of 32 k (the only tiles that read
// TgArgs::at and write TgArgs::ct)
bool tg_plan_k32(const TgArgs& a);
// the tile-major copy of a row-major [rows][K] fp16 matrix (rows % 16 == 0, K % 32 == 0)
int wtile_shuffle_launch(const _Float16* w, _Float16* wt, int rows, int K, hipStream_t st);
// out[t] = fp16(table[ids[t]] * fp16(sqrt(width))) for n tokens (ids clamped into the table)
int embed_language_launch(const int32_t* ids, int n, const _Float16* table, int vocab, int width, _Float16* out,
                          hipStream_t st);

// SigLIP tower + projector of one image (vision.hip); params in named_params order:
// patch_embedding w, b, position_embedding, per layer q w,b k w,b v w,b out w,b fc1 w,b
// fc2 w,b layer_norm1 w,b layer_norm2 w,b, then post_layernorm w,b, projector w,b
struct VisionCfg {
  int image_size, patch_size, num_channels, hidden, inter, layers, heads, proj;
  float eps;
};
size_t vision_ws_bytes(const VisionCfg& v);
int embed_image_enqueue(const VisionCfg& v, const _Float16* const* prm, const _Float16* image, _Float16* out,
                        void* ws, size_t ws_bytes, float* gemm_ws, size_t gemm_ws_floats, unsigned* gemm_sync,
                        int gemm_sync_tiles, unsigned* gemm_err, hipStream_t st);

// compute units of the current device (cached per device; 0 if it cannot be queried)
int device_cus();
// words of meeting counters and floats of partials the 256-row tile path can use
size_t tg_sync_words();
size_t tg_ws_floats();
int tg_launch(const TgArgs& a, hipStream_t st);

int euler_init_launch(const float* x0, float* x32, _Float16* x16, int n, hipStream_t st);

// ---------------------------------------------------------------------------
// Persistent step (step_persistent.hip): one launch of one workgroup per CU runs a whole
// denoise_step_kv after the modulations -- action_in, the decoder layers (q/k/v, joint
// attention, split combine, o_proj, gate_up, down) and the head -- as a sequence of phases.
// Every workgroup owns fixed tasks (weight tiles, attention blocks) of each phase; it loads
// the weights of its next task before it waits for the previous phase, and the phases
// meet through per-workgroup progress words instead of kernel boundaries.
// ---------------------------------------------------------------------------
// The float32 model (model_f32.hip): generic fp32 kernels for prefill / step / loop / chunk.
struct F32Model;
int f32_create(const ::mlcv_config& cfg, F32Model** out);
void f32_destroy(F32Model* m);
int f32_bind(F32Model& m, const void* const* ptrs, int count);
int f32_prefill(F32Model& m, const void* prefix_embs, const float* prefix_mask, float* keys, void* values,
                hipStream_t st);
int f32_step(F32Model& m, const float* keys, const void* values, const void* x_t, const void* time_emb,
             const float* cos, const float* sin, const float* prefix_mask, float* v_out, hipStream_t st);
int f32_loop(F32Model& m, const float* keys, const void* values, const float* x0, const void* time_embs,
             const float* cos, const float* sin, const float* prefix_mask, float* x_out, hipStream_t st);
int f32_chunk(F32Model& m, const void* prefix_embs, const float* prefix_mask, const float* x0, const void* time_embs,
              const float* cos, const float* sin, float* x_out, hipStream_t st);

struct PkLin {
  const _Float16* w;     // fragment-major 16-row slabs (wf_shuffle_launch), fp16, or
  const uint32_t* qw;    // q4f16_1 blocks (wf_shuffle_q4_launch)
  const _Float16* qs;
  const _Float16* bias;  // [N] or null
};
enum : int { PK_Q = 0, PK_K, PK_V, PK_O, PK_GU, PK_DN, PK_NLIN };

struct PkArgs {
  const PkLin* lw;        // [D][PK_NLIN] weights of the decoder layers
  PkLin aout;             // action_out, fragment-major [A][W1]
  const _Float16* ain_w;  // action_in, row-major [W1][A]
  const _Float16* ain_b;  // [W1]
  const _Float16* modp;   // [2D+1][3 W1] adaRMS (scale | shift | gate) of this step
  const float* nscale;    // [2D+1] power of two per norm with max |(1 + scale) * nscale| <= 1
  const float* keys;      // prefix K [D][KV][P][HD] f32 (roped)
  const _Float16* values; // prefix V [D][KV][P][HD]
  const float* mask;      // [P] additive
  const float* cos;       // suffix RoPE [T][HD/2]
  const float* sin;
  const _Float16* xin;    // x_t [T][A] fp16
  float* vout;            // head: v [T][A] f32, or (euler) x32 += dt v and x16 = fp16(x32)
  float* x32;
  _Float16* x16;
  float dt;
  int euler;
  // activations, each written once per launch (element strides per layer below)
  _Float16* xres;         // [D+1][T][W1] residual stream entering layer L (D: final)
  float* rres;            // [D+1][T][W1/16] its row sums of squares per 16 columns
  _Float16* ures;         // [D+1][64][W1] fragment-major fp16(x (1 + scale) nscale), shift in row T
  _Float16* xmid;         // [D][T][W1] after the attention residual
  float* rmid;
  _Float16* umid;
  _Float16* qf;           // [D] q fragments (attn_qf_index)
  float* k32;             // [D][T][nkv]
  _Float16* vs;           // [D][T][nkv]
  float* part;            // [D] attention split partials
  _Float16* attn;         // [D][64][nq] fragment-major
  _Float16* h;            // [D][64][F1] fragment-major
  float* sko;             // [D] o_proj / down split-K partials
  float* skd;
  unsigned* cnto;         // [D][W1/16] split-K arrival counters (monotonic)
  unsigned* cntd;
  size_t s_x, s_r, s_u, s_qf, s_k, s_part, s_attn, s_h, s_sko, s_skd;
  int D, T, A, W1, F1, H, KV, HD, P, nq, nkv;
  float eps;
  int G;                  // workgroups: one per CU, all resident
  int so, sd;             // K slices of o_proj and down (powers of two)
  int gu_sw;              // 16-row slabs per gate_up task (1 or 2)
  int nsplit, kps, rows, rpad;  // attention plan
  unsigned* prog;         // [G] progress words
  unsigned* err;          // device error word (non-zero: a wait gave up)
  unsigned spin;          // polls before a wait gives up
  int merge_comb;         // the attention's key splits combine their row block after meeting
  unsigned* cntm;         // [D][KV][row blocks] arrival counters of those meetings (monotonic)
  int prefetch;           // workgroups idle in the attention phase prefetch the layer's later weights
  unsigned* sink;         // null (keeps the prefetch loads)
  int noskip;             // 1: compute key chunks whose keys are all masked too (testing the skip)
};
// device-scope error codes of the persistent step
constexpr unsigned PK_ERR_TIMEOUT = 1;
int pk_launch(const PkArgs& p, bool q4, hipStream_t st);
// head dims the persistent step is built for
bool pk_head_dim_ok(int hd);

// ---------------------------------------------------------------------------
// XCD tensor-parallel step (step_xtp.hip): the decoder layers of one denoise_step_kv as two
// launches per layer of one workgroup per CU, tensor-parallel over the 8 XCDs.  XCD x owns
// query head x (its q rows, its attention, its 256 columns of o_proj's K) and MLP columns
// [512 x, 512 x + 512) (gate_up rows, down's K); each XCD computes the shared k / v itself.
// Inside a launch the 32 workgroups of an XCD meet at barriers in that XCD's L2; the two
// cross-XCD sums per layer (o_proj's and down's partials) happen at the launch boundaries,
// where every XCD adds the 8 partials of its own 32-column slice of the residual stream.
// Shape it is built for: width 1024, MLP 4096, 8 query heads / 1 kv head of 256 dims,
// T < 64 tokens, P + T <= 1024 keys, fp16 weights, 8 XCDs x 32 CUs.
// ---------------------------------------------------------------------------
struct XtArgs {
  const PkLin* lw;         // [D][PK_NLIN] fragment-major weights (wf_shuffle_launch copies)
  const _Float16* ain_w;   // action_in, row-major [W1][A]
  const _Float16* ain_b;   // [W1] or null
  const _Float16* modp;    // [2D+1][3 W1] adaRMS (scale | shift | gate) of this step
  const float* nscale;     // [2D+1] power-of-two prescale of each norm's pre-scaled input
  const float* keys;       // prefix K [D][P][HD] f32 (roped)
  const _Float16* values;  // prefix V [D][P][HD]
  const float* mask;       // [P] additive
  const float* cos;        // suffix RoPE [T][HD/2]
  const float* sin;
  const _Float16* xin;     // x_t [T][A] fp16
  // per layer and XCD (XCD 0's copies are probed); with ls == 0 every layer reuses layer 0's set
  // (its pages and lines stay warm: 0.7 us per launch faster), with ls == 1 each keeps its own
  _Float16* x;      // [D][8][T][W1]  residual stream entering layer L
  _Float16* xm;     // [D][8][T][W1]  after the attention's gated residual
  _Float16* qf;     // [D][8][XT_QF]  q roped, scaled, fp16 hi/lo in the attention's fragment order
  float* k32;       // [D][8][T][HD]  suffix k roped
  _Float16* v;      // [D][8][T][HD]  suffix v
  _Float16* attn;   // [D][8][64][HD] attention output of head x, fragment-major
  _Float16* h;      // [D][8][64][512] GeGLU output of the XCD's MLP columns, fragment-major
  // reused by every launch
  _Float16* u;      // [8][64][W1] fragment-major pre-scaled adaRMS input, shift in row T
  float* rss;       // [8][T][W1/16] row sums of squares of the residual stream per 16 columns
  _Float16* ap;     // [8][32][64][HD] attention split partials O_s / l_s
  float* aml;       // [8][32][64][2]  their (m, l)
  float* opart;     // [8][32][T][32]  o_proj partials (stored as fp16): [XCD][residual column slice][row][column]
  float* dpart;     // [8][32][T][32]  down partials
  unsigned* flags;  // [8][32] monotonic barrier words (all equal between launches)
  unsigned* err;    // non-zero: a barrier wait gave up
  unsigned spin;    // polls before a wait gives up
  int D, T, P, A, L;
  int ls;           // layer stride of the per-layer buffers (0 or 1)
  int noskip;       // 1: compute key chunks whose keys are all masked too (testing the skip)
  int q4;           // the weight table holds q4f16_1 blocks (qw / qs) instead of fp16 slabs
  float eps;
  // the residual stream after the last layer in the launch chain's layout (the head writes it)
  _Float16* x16;    // [T][W1]
  // the head after the last layer (xt_head_launch): final adaRMS + action_out_proj
  const _Float16* aout_w;  // action_out, row-major [A][W1] fp16 (q4 models: dequantized at bind)
  const _Float16* aout_b;  // [A] or null
  float* vout;             // [T][A] velocity (euler == 0)
  float* vout_user;        // a second copy of the velocity (the caller's output) or null
  float* x32;              // [T][A] Euler state, updated in place (euler == 1)
  _Float16* xnext;         // [T][A] fp16 copy of the updated state: the next step's action input
  float dt;                // Euler step
  int euler;
};
constexpr int XT_QF = 4 * 8 * 2 * 512;  // halfs of one head's q fragments (64 rows, 256 dims)
// the shape the XCD tensor-parallel step is built for
bool xt_shape_ok(int W1, int F1, int H, int KV, int HD, int T, int P, int A);
// layer L's attention half (reduce or action_in, q/k/v, attention, combine, o_proj) and MLP
// half (reduce, gate_up, down)
int xt_attn_launch(const XtArgs& a, hipStream_t st);
int xt_mlp_launch(const XtArgs& a, hipStream_t st);
// the last layer's down partials -> residual stream (into x16) -> final adaRMS -> action_out_proj
// -> velocity (vout) or Euler update (x32, xnext): one launch after the last layer
int xt_head_launch(const XtArgs& a, hipStream_t st);

// a batch of device-to-device copies in one launch (the entry points stage their inputs
// into the context's buffers with one kernel instead of one copy launch per buffer)
struct CopyJob {
  const void* src;
  void* dst;
  size_t bytes;
};
constexpr int COPY_MAX = 8;
int copy_list_launch(const CopyJob* jobs, int n, hipStream_t st);

}  // namespace mlcv
