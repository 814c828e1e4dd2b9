/*
 * qdec.h -- C ABI of the MI355X (gfx950) Qwen3 greedy-decode kernel library.
 *
 * Every decode-step operation of a Qwen3 model (the reference engine's
 * engine/kernels/{ops,fused}.py and notes/v10/spec.py, all Triton) is one
 * hand-written HIP kernel behind one entry point here.  Conventions:
 *
 *   - All device pointers are owned by the caller (the Python host allocates
 *     them as PyTorch-ROCm tensors).  The library never allocates, frees or
 *     synchronises inside an entry point, so every call may be recorded into
 *     a hipGraph.  Scratch buffers (split partials, arrival counters) are
 *     caller-provided; their sizes come from the *_workspace queries.
 *   - Arrival counters must be zero before the first call that uses them;
 *     every kernel leaves the counters it used at zero again, so one zeroed
 *     buffer serves any number of calls on one stream.  Two calls that share
 *     a counter or partial buffer must not run concurrently.
 *   - Per-step scalars (token ids, cache lengths) are device pointers, never
 *     host ints, so a captured graph stays valid across replays.
 *   - Entry points return QDEC_OK (0) or a negative QDEC_E* code; the text of
 *     the last error on the calling thread is qdec_last_error().  Argument
 *     validation happens before any HIP call, so it also works on a host
 *     without a GPU.
 *   - bf16 tensors are passed as void* holding IEEE bfloat16 bit patterns.
 *   - `stream` is a hipStream_t (NULL = the default stream).
 *
 * Data layouts (all row-major unless stated):
 *   tiled weight  : a [N, K] bf16 matrix (N % 16 == 0, K % 32 == 0) stored as
 *                   1 KiB blocks, block (nt, ks) at element ((nt*(K/32))+ks)*512;
 *                   inside a block lane l (0..63) owns elements [8l, 8l+8) =
 *                   W[16*nt + (l & 15)][32*ks + 8*(l >> 4) + e], e = 0..7.
 *                   One wavefront reads one block with one 16-byte load per
 *                   lane; the block is the A operand of one
 *                   v_mfma_f32_16x16x32_bf16.
 *   K cache slab  : [batch][n_kv_heads][cap][head_dim] bf16, per layer.
 *   V cache slab  : [batch][n_kv_heads][cap/8][head_dim][8] bf16, per layer:
 *                   8 consecutive slots of one channel are 16 contiguous bytes
 *                   (the A operand of the P.V product).
 *   cap is a multiple of 32.
 */
#ifndef QDEC_H
#define QDEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QDEC_ABI_VERSION 1

#define QDEC_OK 0
#define QDEC_EINVAL (-1)       /* bad shape or argument */
#define QDEC_EALIGN (-2)       /* pointer not 16-byte aligned */
#define QDEC_EUNSUPPORTED (-3) /* configuration the kernels do not implement */
#define QDEC_ELAUNCH (-4)      /* hipGetLastError after the launch */
#define QDEC_ENODEV (-5)       /* no usable HIP device */

/* Greedy pick of a row whose logits are all NaN.  Invalid inputs are never
 * silently replaced: an out-of-range token id (qdec_embed) or cache length
 * (qdec_attn, and the merge of x_attn) makes the affected rows NaN, which
 * reaches the argmax as this out-of-vocabulary id; the host checks for it. */
#define QDEC_NAN_ID 2147483647

/* qdec_gemm flags */
#define QDEC_NORM_IN 1u  /* x is the residual stream; RMSNorm(x) * norm_w feeds the product */
#define QDEC_GLU 2u      /* w holds gate tiles then up tiles; out = silu(gate) * up */
#define QDEC_RES_OUT 4u  /* res += x @ W^T, rounded as the reference rounds */
#define QDEC_ARGMAX 8u   /* greedy argmax of the bf16 logits of every row into ids_out */

typedef void *qdec_stream_t;

/* Library ABI version (QDEC_ABI_VERSION). */
int qdec_version(void);

/* Text of the last error returned on this thread ("" if none). */
const char *qdec_last_error(void);

/* Number of visible HIP devices (0 on a host without a GPU; never fails). */
int qdec_device_count(void);

/* ------------------------------------------------------------------ layout */

/* Element offset of W[n][k] inside the tiled layout of a [*, K] matrix.
 * Host-only helper; returns -1 for an invalid K or index. */
int64_t qdec_tiled_offset(int64_t n, int64_t k, int64_t K);

/* Repack a row-major [n, k] bf16 matrix into the tiled layout.
 * Replaces the load-time packing of engine/engine.py:271-287 (which only
 * concatenates q|k|v and gate|up; the tiling is this library's own). */
int qdec_pack_tiles(const void *src, void *dst, int64_t n, int64_t k,
                    qdec_stream_t stream);

/* Measurement only, no counterpart in the reference: reads `bytes` of `buf`
 * once, in 16-byte non-temporal loads as the decode kernels stream their
 * weights, over `blocks` workgroups; `sink` ([blocks] uint32) is written only
 * when the data hash takes one specific value.  Timing it over a buffer well
 * beyond the 256 MB memory-side cache gives the streaming-read ceiling the
 * decode roofline is compared with, beside the 8 TB/s HBM peak. */
int qdec_read_probe(const void *buf, int64_t bytes, uint32_t *sink, int32_t blocks, qdec_stream_t stream);

/* ------------------------------------------------------------- embedding */

/* h[m, :] = E[ids[m], :] for m < rows.  E is the tiled [vocab, hidden]
 * embedding (the same buffer feeds the tied lm_head).  An id outside
 * [0, vocab) reads nothing and makes row m NaN (QDEC_NAN_ID below).
 * Replaces fused.embed_ssq, engine/kernels/fused.py:341-357 (the sum of
 * squares it also produced is recomputed by each NORM_IN consumer). */
typedef struct {
  const int64_t *ids; /* [rows] */
  const void *emb;    /* tiled [vocab, hidden] bf16 */
  void *h;            /* [rows, hidden] bf16 out */
  int32_t rows;
  int32_t hidden;
  int32_t vocab;
} qdec_embed_args;
int qdec_embed(const qdec_embed_args *a, qdec_stream_t stream);

/* ------------------------------------------------------------ skinny GEMM */

struct qdec_attn_args;  /* below: the attention call a GEMM may take its x from */

/* y[m, n] = sum_k x'[m, k] * W[n, k] over the tiled weight, for m < rows
 * (1 <= rows <= 64), fp32 accumulation, one rounding to bf16, then:
 *   plain   : out = bf16(y)
 *   NORM_IN : x' = bf16(norm_w * bf16(x * rsqrt(mean(x^2) + eps))) per row
 *   GLU     : out = bf16(bf16(silu(bf16(y_gate))) * bf16(y_up)), n = #act cols
 *   RES_OUT : res = bf16(res + bf16(y))   (in place; out unused)
 *   ARGMAX  : ids_out[m] = lowest index of max_n bf16(y[m, n]) (QDEC_NAN_ID
 *             when every logit of the row is NaN);
 *             out (optional, may be NULL) receives the bf16 logits;
 *             lens_inc (optional) gets lens_inc[m] += 1 after the pick.
 * flags: 0, NORM_IN, NORM_IN|GLU, RES_OUT, NORM_IN|ARGMAX; GLU and ARGMAX
 * also without NORM_IN when x_frag = 1 (the input of a norm hand-over).
 * The summation order of every output element depends only on k, ksplit and
 * waves -- never on rows -- so a row's result is bit-identical whether it is
 * computed alone or inside a larger batch.
 * Replaces fused.gemv (engine/kernels/fused.py:33-338: NORM_IN / GLU /
 * RES_OUT / split-K) and the lm_head + torch.argmax pair of
 * engine/engine.py:492-498, 542-545. */
typedef struct {
  const void *x;        /* [rows, k] bf16 */
  const void *w;        /* tiled weight: [n, k], or [2n, k] with QDEC_GLU */
  void *out;            /* [rows, n] bf16 (plain, GLU, optional with ARGMAX) */
  void *res;            /* [rows, n] bf16 residual (RES_OUT) */
  const void *norm_w;   /* [k] bf16 (NORM_IN) */
  float *partial;       /* split-K / pre-pass scratch (qdec_gemm_workspace) */
  uint32_t *counters;   /* zeroed arrival counters and argmax keys (qdec_gemm_workspace;
                           8-byte aligned with ARGMAX); zero again on return */
  int64_t *ids_out;     /* [rows] (ARGMAX) */
  int32_t *lens_inc;    /* [rows] or NULL (ARGMAX) */
  float eps;
  int32_t rows;
  int32_t n;
  int32_t k;
  uint32_t flags;
  int32_t ksplit;       /* workgroups sharing one output tile along k (>= 1) */
  int32_t waves;        /* wavefronts per workgroup, splitting its k range (1..8) */
  int32_t tiles_per_wg; /* output tiles per workgroup (>= 1, divides n/16) */
  /* NULL, or an attention call made with out_partials = 1: then x is not
   * read; activation row m = b*t_rows + t is the merge of that call's chunk
   * partials for sequence b, query row t (k = nq*head_dim, rows =
   * batch*t_rows), bit-identical to what the attention would have written to
   * its out.  Needs activations staged from registers (rows <= 4 and the
   * workgroup's k range within 2 vectors per thread); QDEC_EUNSUPPORTED
   * otherwise. */
  const struct qdec_attn_args *x_attn;
  /* Activation layouts for batched calls (0 = row-major [rows, k] / [rows, n]).
   * Fragment order, nmt = ceil(rows / 16) M tiles: element (m, c) of a matrix
   * with C columns sits at ((c/32 * nmt + m/16) * 64 + m%16 + 16*(c%32/8)) * 8
   * + c%8 -- the operand order of the kernels' 16x16x32 MFMA, so a direct
   * call loads each fragment as one contiguous KiB; rows past `rows` in the
   * last M tile are ignored.
   * x_frag = 1: x is in fragment order (as a call with out_frag = 1 or an
   * attention call with out_frag = 1 over the same rows wrote it).  Not with
   * NORM_IN or x_attn (the call takes the direct path).
   * out_frag = 1: out is written in fragment order (plain or GLU only). */
  int32_t x_frag;
  int32_t out_frag;
  /* Residual update left to the next NORM_IN call (RES_OUT with ksplit > 1):
   * each k split writes its fp32 partial sum of y to
   * parts_out[split][rows][n]; res is not touched and no counters are used.
   * The consumer passes the same buffer as x_parts. */
  float *parts_out;
  /* NORM_IN (with or without GLU): the residual x still owes a RES_OUT
   * update held in k-split partials x_parts[j][rows][k], j < x_nparts
   * (1..8).  The call first forms x = bf16(x + bf16(((p0 + p1) + p2) + ...))
   * per element -- the rounding a RES_OUT call applies -- uses it as its
   * input and writes it to x_merged ([rows, k] bf16, not x itself: other
   * workgroups of the call still read x).  Needs ksplit 1 and a plan that
   * stages x from registers (one row, without GLU) or through the
   * normalisation pre-pass (QDEC_EUNSUPPORTED otherwise). */
  const float *x_parts;
  int32_t x_nparts;
  void *x_merged;
  /* Norm hand-over (RES_OUT on the direct path, i.e. x_frag = 1 or 17+
   * rows): this call also produces the input of the NORM_IN call that
   * follows it, so that call runs as a plain x_frag = 1 call on next_xn
   * (same flags without QDEC_NORM_IN, no x_parts) and launches no
   * normalisation pre-pass.  Let r be the updated residual row: res after
   * this call's update, or -- with parts_out -- bf16(res + bf16(((p0 + p1)
   * + p2) + ...)), which is then also written to next_merged ([rows, n]
   * bf16; res is still not touched).  Row m of next_xn (fragment order,
   * ceil(rows / 16) M tiles, n columns; rows past `rows` zero) is
   * bf16(next_norm_w * bf16(r * rsqrt(mean(r^2) + eps))), its statistic
   * summed in the order a pre-pass of the consumer would use: pass
   * next_threads = that call's workgroup size (qdec_gemm_prepass).  The
   * result is bit-identical to the consumer's own pre-pass.  The last
   * ceil(rows / 16) * 16 workgroups of this call to finish each take one
   * row, after every workgroup has arrived (three words of the counters
   * workspace; a wait longer than about 2^22 polls writes NaN rows and sets
   * the third word, after which every hand-over row of every later call is
   * NaN until the caller zeroes the counters).
   * Needs next_threads a multiple of 64 and at most twice this call's
   * workgroup size, n / 8 at most 2 * next_threads (at most next_threads
   * when that exceeds this call's workgroup size), and at least
   * ceil(rows / 16) * 16 workgroups (QDEC_EUNSUPPORTED otherwise).
   * next_norm_w = NULL: off.
   * No counterpart in the reference, whose fused.gemv epilogue leaves the
   * statistic to the consumer's own pass (engine/kernels/fused.py:33-338). */
  const void *next_norm_w; /* [n] bf16 */
  void *next_xn;
  void *next_merged;
  int32_t next_threads;
  /* 1: gate/up with its rows resident in LDS.  For NORM_IN | GLU with
   * ksplit 1, 4 waves, one tile per workgroup, row-major x (no x_frag,
   * x_attn, x_parts or next_norm_w), 1..8 or 17..32 rows, k <= 2560 and
   * k / 128 a multiple of 10: one workgroup per compute unit takes a
   * contiguous run of (gate, up) tile pairs and reads its MFMA operands
   * from one copy of the normalised rows in LDS, so no workgroup re-reads
   * the activations from L2.  At 1..8 rows the workgroup normalises the
   * rows itself (no normalisation pre-pass is launched, no workspace); at
   * 17..32 rows the pre-pass still normalises them into the workspace and
   * each workgroup copies them in.  The output is bit-identical to the same
   * call with resident = 0 (the statistic, the k split over 4 waves and the
   * epilogue are the same).
   * NORM_IN alone (QKV), under the same bounds at 1..8 or 17..32 rows with
   * k / 128 a multiple of 20: the same plan with single output tiles in
   * place of the pairs (one or two per workgroup); the same bits as
   * resident = 0.
   * For RES_OUT with ksplit 1, one tile per workgroup, row-major x (no
   * x_frag, x_attn, parts_out or next_norm_w), 1..8 rows and k / 32 a
   * multiple of 16 and at most 304: every workgroup first copies the rows
   * into LDS (LDS DMA, up to 8 rows x 64 bytes per k step) and its weight
   * ring then holds
   * weights only, where the direct path loads each k step's rows beside
   * its weight block; the same bits as resident = 0.
   * For RES_OUT with parts_out (ksplit > 1, 4 waves, x_frag = 1, 17..32
   * rows, at most 76 k steps per split): the workgroups of each k split
   * share its slice of the rows -- workgroup w takes split w % ksplit and
   * 2 or 3 output tiles, copies that slice into LDS once (LDS DMA) and
   * streams weights only; parts_out receives the same bits as with
   * resident = 0.
   * QDEC_EUNSUPPORTED outside those bounds.  0: off.
   * No counterpart in the reference: its fused.gemv launches one program
   * per output block, each normalising the rows itself
   * (engine/kernels/fused.py:33-172). */
  int32_t resident;
} qdec_gemm_args;
int qdec_gemm(const qdec_gemm_args *a, qdec_stream_t stream);
/* Scratch sizes (bytes) a qdec_gemm call with these arguments needs. */
int qdec_gemm_workspace(const qdec_gemm_args *a, size_t *partial_bytes,
                        size_t *counter_bytes);
/* Whether a qdec_gemm call with these arguments normalises its rows in a
 * pre-pass of its own (1) or not (0); *threads receives its workgroup size
 * (the statistic order a norm hand-over to it must follow).  Negative: the
 * arguments are invalid (the error of qdec_gemm). */
int qdec_gemm_prepass(const qdec_gemm_args *a, int32_t *threads);

/* --------------------------------------------------- GQA decode attention */

/* For every sequence b and query row t < t_rows (absolute position
 * lens[b] + t), from the raw projection row qkv[b*t_rows + t]:
 *   q, k = per-head RMSNorm (q_norm_w / k_norm_w, rounded as Qwen3RMSNorm),
 *          then RoPE  bf16(bf16(y*cos) + bf16(rotate_half(y)*sin));
 *   the new k and the raw v are written into cache slot lens[b] + t;
 *   out  = softmax(q . K^T / sqrt(D)) . V over slots 0 .. lens[b] + t,
 *          fp32 scores and accumulation, probabilities rounded to bf16
 *          before the P.V product (flash-decoding), output rounded once.
 * A length with lens[b] < 0 or lens[b] + t_rows > cap touches no cache
 * memory; the rows of sequence b become NaN (QDEC_NAN_ID).
 * Slots are processed in chunks of `chunk` slots keyed to absolute slot
 * numbers, one workgroup per (chunk, kv head, sequence); the last workgroup
 * of a (sequence, kv head) to finish merges the chunk partials in chunk
 * order (or, with out_partials, the consuming GEMM merges them in the same
 * order and arithmetic).  A row's result therefore does not depend on t_rows (for a fixed
 * chunk and waves).
 * Replaces fused.attention_fused (engine/kernels/fused.py:360-479),
 * ops.qkv_post + ops.DecodeAttention (engine/kernels/ops.py:84-431) and the
 * multi-row verify attention of notes/v10/spec.py:111-182. */
typedef struct qdec_attn_args {
  const void *qkv;      /* [batch*t_rows, (nq + 2*nkv)*head_dim] bf16 */
  const void *q_norm_w; /* [head_dim] bf16 */
  const void *k_norm_w; /* [head_dim] bf16 */
  const void *cos_tab;  /* [cap, head_dim] bf16 */
  const void *sin_tab;  /* [cap, head_dim] bf16 */
  const int32_t *lens;  /* [batch] slots already in the cache per sequence */
  void *k_cache;        /* K slab of this layer */
  void *v_cache;        /* V slab of this layer */
  void *out;            /* [batch*t_rows, nq*head_dim] bf16 */
  float *partial;       /* chunk partials (qdec_attn_workspace) */
  uint32_t *counters;   /* zeroed arrival counters (qdec_attn_workspace) */
  float eps;
  float sm_scale;       /* 1/sqrt(head_dim) */
  int32_t batch;
  int32_t t_rows;       /* query rows per sequence (1 = plain decode) */
  int32_t nq;           /* a multiple of nkv (G = nq / nkv query heads per */
  int32_t nkv;          /* kv head); t_rows * G <= 64, <= 32 with 8 waves  */
  int32_t head_dim;     /* 128, or 64 with waves = 4 */
  int32_t cap;          /* slots per sequence, multiple of 32 */
  int32_t chunk;        /* slots per workgroup, multiple of 32 */
  int32_t waves;        /* wavefronts per workgroup: 4, or 8 for t_rows <= 8;
                           blocks of 32 slots are dealt to them round robin.
                           A row's result depends on chunk and waves, never
                           on t_rows */
  int32_t out_partials; /* 0: merged rows to out.  1: every chunk leaves its
                           unnormalised (acc, max, sum) in partial, out is not
                           written, and a qdec_gemm with x_attn = these
                           arguments merges them (no arrival pass) */
  int32_t out_frag;     /* 1: out in the fragment order of qdec_gemm_args
                           (rows = batch*t_rows, columns nq*head_dim) */
  int32_t strided;      /* 0: chunk c holds slots [c*chunk, (c+1)*chunk).
                           1: with C = ceil(cap / chunk) chunks, chunk c
                           holds the 32-slot blocks c, c + C, c + 2C, ...,
                           so a partly filled cache spreads evenly over the
                           chunks.  Either way the dealing is keyed to
                           absolute slots: a row's result depends on chunk,
                           waves and strided, never on t_rows.  No
                           counterpart in the reference, whose split
                           attention takes contiguous ranges
                           (engine/kernels/ops.py:219-431). */
} qdec_attn_args;
int qdec_attn(const qdec_attn_args *a, qdec_stream_t stream);
int qdec_attn_workspace(const qdec_attn_args *a, size_t *partial_bytes,
                        size_t *counter_bytes);

/* qdec_attn with no workspace arguments: a->partial and a->counters are
 * ignored; the chunk partials and arrival counters live in a device array
 * the library owns (QDEC_NOALLOC_PARTIAL_BYTES + QDEC_NOALLOC_COUNTER_BYTES
 * per GPU, held until the process ends).  Nothing is allocated or freed.
 * A call whose qdec_attn_workspace exceeds either size, or that asks for
 * out_partials, fails with an error.  All calls on one GPU share the array:
 * calls that overlap in time on one GPU race.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under hipGraph
 * capture, serving loops or harnesses that forbid hipMalloc). */
#define QDEC_NOALLOC_PARTIAL_BYTES (8u << 20)
#define QDEC_NOALLOC_COUNTER_BYTES (64u << 10)
int qdec_attn_noalloc(const qdec_attn_args *a, qdec_stream_t stream);

/* -------------------------------------------- one decode layer per launch */

/* A whole decoder layer of plain decode in one launch: the qkv, attn, o,
 * gate_up and down calls above as the stages of one kernel whose workgroups
 * all stay resident and meet at a grid barrier between stages.  Each stage
 * runs the per-block code of its own launch under a 4-wave plan, so the
 * layer computes what those five calls would (the engine's own plans use 8
 * waves for O and down at batch 1, which sums their k ranges in another
 * order).  Accepted plans: batch <= 4 rows, t_rows 1; every GEMM waves 4,
 * ksplit 1, no fragment order, no split residual; qkv NORM_IN, o RES_OUT
 * with x_attn == attn, gate_up NORM_IN | GLU with tiles_per_wg 2, down
 * RES_OUT; attn waves 4, out_partials 1; at most `workgroups` blocks per
 * stage.  Anything else fails with QDEC_EUNSUPPORTED.
 *
 * plan: device memory for the launch parameters, written by
 *   qdec_layer_prepare (synchronous; not under stream capture) and read by
 *   every qdec_layer call with the same arguments (a call whose arguments
 *   differ from the prepared ones runs nothing and sets the error word to 2).
 * ctl: barrier state, zeroed before the first call, then left to the
 *   library (tickets that only grow, an error word, uint32 at ctl + 8, and
 *   the workgroup count of the first launch on it, uint32 at ctl + 12).  A
 *   workgroup that waits longer than spin_limit polls sets the word to 1 and
 *   every later wait gives up, so a launch whose workgroups cannot all be
 *   resident ends with wrong numbers and the flag, never with a hang; zero
 *   ctl again before reusing it.  Calls sharing ctl must use one workgroup
 *   count (a launch of another count runs nothing and sets the word to 3)
 *   and must not overlap in time.
 * Replaces the reference's one-launch layer (engine/kernels/layer.py:46-285:
 * _arrive_and_wait with SPIN_LIMIT, _layer_kernel) and its engine hook
 * (engine/engine.py:834-884; MEGA_ENABLED = False there, :81). */
#define QDEC_LAYER_PLAN_BYTES 4096u
#define QDEC_LAYER_CTL_BYTES 1152u
typedef struct {
  const qdec_gemm_args *qkv;
  const qdec_attn_args *attn;
  const qdec_gemm_args *o;
  const qdec_gemm_args *gate_up;
  const qdec_gemm_args *down;
  void *plan;          /* QDEC_LAYER_PLAN_BYTES, 16-byte aligned */
  void *ctl;           /* QDEC_LAYER_CTL_BYTES, 8-byte aligned */
  uint32_t spin_limit; /* polls before a barrier wait gives up; 0 = 1 << 22 */
  int32_t workgroups;  /* a multiple of 8; 0: as many as fit the GPU at once
                          (the most allowed) */
} qdec_layer_args;
int qdec_layer_prepare(const qdec_layer_args *a);
int qdec_layer(const qdec_layer_args *a, qdec_stream_t stream);

/* ------------------------------------------------ n-gram speculation */

/* Suffix-match drafter over each sequence's own history hist[b, 0..lens[b]]
 * (hist[b, lens[b]] is the token not yet fed).  Pattern = the last `primary`
 * tokens; the most recent earlier occurrence whose k-token continuation lies
 * inside the history wins; otherwise the same with `backoff` tokens;
 * otherwise the draft is all zeros.  Writes ids[b*(k+1)] = hist[b, lens[b]],
 * ids[b*(k+1) + 1 + t] = draft[b*k + t].  k = 0 only feeds the current token
 * (a plain step that keeps the history: what the acceptance gate falls back
 * to); draft must still be a valid pointer.
 * Replaces notes/v10/spec.py:36-108 (_ngram_draft_kernel / ngram_draft). */
typedef struct {
  const int64_t *hist; /* [batch, cap] */
  const int32_t *lens; /* [batch] */
  int64_t *ids;        /* [batch*(k+1)] out */
  int64_t *draft;      /* [batch*k] out */
  int32_t batch;
  int32_t cap;
  int32_t primary;
  int32_t backoff;
  int32_t k;
} qdec_draft_args;
int qdec_ngram_draft(const qdec_draft_args *a, qdec_stream_t stream);

/* Longest-prefix greedy acceptance: a = number of leading drafts equal to the
 * model's argmax at the same row; rows 0..a are appended to the history at
 * lens[b]+1 ..; lens[b] += a+1.  A sequence with lens[b] >= stop_len is
 * frozen (a = 0, nothing written).  naccept[b] = a.
 * Replaces notes/v10/spec.py:185-224 (_accept_kernel / accept). */
typedef struct {
  const int64_t *out_tok; /* [batch*(k+1)] argmax per verify row */
  const int64_t *draft;   /* [batch*k] */
  int64_t *hist;          /* [batch, cap] */
  int32_t *lens;          /* [batch] */
  int32_t *naccept;       /* [batch] out */
  int32_t batch;
  int32_t cap;
  int32_t k;
  int32_t stop_len;
} qdec_accept_args;
int qdec_spec_accept(const qdec_accept_args *a, qdec_stream_t stream);

/* ------------------------------------------------------------ prefill */

/* Prompt processing: every prompt position of every sequence in one forward
 * (or a few position chunks), so each weight matrix is read once per call
 * and the products run on the matrix cores.  Row m = b*t_rows + t of a call
 * is sequence b at position pos0 + t (equal-length prompts).  Activations
 * that feed a product are in the fragment order of qdec_gemm_args with
 * `tiles` M tiles (16 rows each); rows past the last real one are zero. */

/* RMSNorm of every row into fragment order: out = bf16(w * bf16(x * rsqrt(
 * mean(x^2) + eps))), or a plain re-layout when norm_w is NULL.  Rows
 * rows .. 16*tiles-1 of out are written with zeros.
 * Replaces ops.add_rms_norm (engine/kernels/ops.py:27-76) as the prefill
 * forward uses it (engine/engine.py:448-461). */
typedef struct {
  const void *x;      /* [rows, k] bf16 */
  const void *norm_w; /* [k] bf16, or NULL */
  void *out;          /* fragment order, `tiles` M tiles */
  float eps;
  int32_t rows;
  int32_t k;          /* multiple of 32 */
  int32_t tiles;      /* >= ceil(rows / 16) */
} qdec_rownorm_args;
int qdec_rownorm(const qdec_rownorm_args *a, qdec_stream_t stream);

/* out = x @ W^T on the matrix cores for x in fragment order (`tiles` M
 * tiles, a multiple of 16), W tiled [n, k].  A workgroup computes tile_rows
 * x tile_cols of it: 256 x 128, 256 x 256 or 64 x 64 (0 x 0 picks by launch
 * size: 256 x 256 while it keeps 600 workgroups, 256 x 128 while 512, else
 * 64 x 64); n must be a multiple of tile_cols, k of 64.  flags:
 *   0            out = bf16(x @ W^T): [rows, n] row-major, or fragment order
 *                with out_frag;
 *   QDEC_RES_OUT out = bf16(res + bf16(x @ W^T)), row-major; res may be out;
 *   QDEC_GLU     W holds n/2 gate rows then n/2 up rows; out = bf16(bf16(
 *                silu(bf16 gate)) * bf16 up), n/2 columns, row-major or
 *                fragment order.
 * fp32 accumulation in k order, rounded as qdec_gemm rounds.
 * Replaces F.linear and ops.silu_mul (engine/kernels/ops.py:242-267) and the
 * residual adds of the prefill forward (engine/engine.py:448-461). */
typedef struct {
  const void *x;    /* fragment order, `tiles` M tiles */
  const void *w;    /* tiled [n, k] bf16 */
  void *out;
  const void *res;  /* QDEC_RES_OUT: [rows, n] bf16 */
  uint32_t flags;   /* 0, QDEC_RES_OUT or QDEC_GLU */
  int32_t rows;
  int32_t n;
  int32_t k;
  int32_t tiles;
  int32_t out_frag; /* 1: out in fragment order with `tiles` M tiles */
  int32_t tile_rows; /* 0, 256 or 64 */
  int32_t tile_cols; /* 0, 128 or 256 (with 256 rows), 64 (with 64 rows) */
} qdec_pgemm_args;
int qdec_prefill_gemm(const qdec_pgemm_args *a, qdec_stream_t stream);

/* Per-head RMSNorm (q_norm / k_norm) and RoPE of every row's query and key
 * heads, with the arithmetic of qdec_attn; the rotated keys and the raw
 * values go to cache slot pos0 + t of sequence b, the rotated queries back
 * over the query columns of qkv.  head_dim 128, nq + nkv <= 80.
 * Replaces ops.qkv_post_rows (engine/kernels/ops.py:149-205). */
typedef struct {
  void *qkv;            /* [batch*t_rows, (nq + 2*nkv)*head_dim] bf16; queries rewritten */
  const void *q_norm_w; /* [head_dim] bf16 */
  const void *k_norm_w; /* [head_dim] bf16 */
  const void *cos_tab;  /* [cap, head_dim] bf16 */
  const void *sin_tab;  /* [cap, head_dim] bf16 */
  void *k_cache;        /* K slab of this layer */
  void *v_cache;        /* V slab of this layer */
  float eps;
  int32_t batch;
  int32_t t_rows;
  int32_t pos0;         /* position of row t = 0 */
  int32_t nq;
  int32_t nkv;
  int32_t head_dim;     /* 128 */
  int32_t cap;          /* multiple of 32; pos0 + t_rows <= cap */
} qdec_prefill_qk_args;
int qdec_prefill_qk(const qdec_prefill_qk_args *a, qdec_stream_t stream);

/* Causal GQA attention of the rows at positions pos0 .. pos0 + t_rows - 1
 * (queries as qdec_prefill_qk leaves them) over cache slots 0 .. position,
 * written in fragment order (`tiles` M tiles) for the O projection.  A
 * workgroup takes 64 positions of the G = nq / nkv query heads of one kv
 * head (G = 2, 4 or 8; QDEC_EUNSUPPORTED otherwise); same
 * arithmetic as qdec_attn (base-2 online softmax in fp32, probabilities
 * rounded to bf16 before P.V, fp32 accumulation, one rounding).
 * Replaces Engine._attend_prefill (engine/engine.py:464-478: SDPA flash
 * attention, causal, GQA). */
typedef struct {
  const void *qkv;     /* [batch*t_rows, (nq + 2*nkv)*head_dim] bf16 */
  const void *k_cache;
  const void *v_cache;
  void *out;           /* fragment order, rows batch*t_rows, columns nq*head_dim */
  float sm_scale;      /* 1/sqrt(head_dim) */
  int32_t batch;
  int32_t t_rows;
  int32_t pos0;
  int32_t nq;
  int32_t nkv;
  int32_t head_dim;    /* 128 */
  int32_t cap;         /* multiple of 32; pos0 + t_rows <= cap */
  int32_t tiles;       /* >= ceil(batch*t_rows / 16) */
} qdec_prefill_attn_args;
int qdec_prefill_attn(const qdec_prefill_attn_args *a, qdec_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QDEC_H */
