/*
 * mi355moe -- C ABI of the MI355X (gfx950) codebook-dequant MoE expert path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream (as void*), validates its arguments on the
 * host before launching anything, and returns MI_OK or an MI_ERR_* code.  The library allocates nothing: the caller
 * owns every buffer, including the workspace.  Work is launched only on the given stream; calls that share a
 * workspace must be ordered on one stream.  Nothing here is internally threaded.
 *
 * Reference interfaces (shallmall/kaggle-llm-endpoint, paths relative to launcher/glm53-flash/engine/glm53/):
 *   ResidentFetch.apply(p, x, idx, w, layer, limit)        resident.py:100-108   -> mi_moe_decode / mi_moe_prefill
 *   moe_matvec(planes, qtype, nblk, idx, X)                pallas_moe.py:238-307 -> mi_matvec
 *   ragged_plan(idx, w, E, tm)                             pallas_moe.py:564-592 -> mi_ragged_plan
 *   moe_route(p, x, cfg)                                   model.py:798-808      -> mi_moe_route
 *   pack_layer_from_gguf / pack_planes                     resident.py:29-60, planes.py:136-170 -> mi_pack_planes
 *   moe_ragged_gateup / moe_ragged_down                    pallas_moe.py:622-755 -> mi_moe_prefill
 *   moe_sweep_gateup / moe_sweep_down, _apply_sweep_kernel  pallas_moe.py:382-555, resident.py:169-187
 *                                                                                 -> mi_moe_prefill_form (SWEEP)
 *   _apply_gather / _apply_sweep_xla (use_pallas=False)    resident.py:122-135,189-210 -> mi_moe_prefill_form
 *   dequant_planes (XLA dequant of the planar tables)      planes.py:196-206     -> mi_dequant
 *   quant8.dequant_tree + x @ W (int8 projections)         quant8.py:91-99       -> mi_int8_project(_many)
 *   Engine._logits_local, int8 lm_head (scale after dot)   engine.py:345-351     -> mi_int8_project (MI_I8_COL_AFTER)
 *   mlp_partial over int8 leaves (shared expert, dense MLP) model.py:125-127,855  -> mi_int8_mlp
 *   mlp_partial / x @ W over bf16 leaves (int8_nonexpert off) model.py:125-127,855, engine.py:281 -> mi_bf16_mlp,
 *                                                                                   mi_bf16_project
 */
#ifndef MI355MOE_H
#define MI355MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------------------------------ */
#define MI_OK              0
#define MI_ERR_NULL        1  /* a required pointer is NULL                                                      */
#define MI_ERR_QTYPE       2  /* unsupported qtype (the reference raises ValueError, planes.py:70,206)           */
#define MI_ERR_SHAPE       3  /* rows/cols/experts outside what the kernels tile (pallas_moe.py:252-255 asserts) */
#define MI_ERR_TOKENS      4  /* N, k or N*k outside the entry point's limits                                    */
#define MI_ERR_WORKSPACE   5  /* workspace NULL or smaller than the *_workspace() size                           */
#define MI_ERR_MISMATCH    6  /* gate/up/down tables do not chain (up != gate shape, down.cols != gate.rows)     */
#define MI_ERR_LAUNCH      7  /* the HIP runtime reported an error at launch                                     */
#define MI_ERR_ARG         8  /* any other invalid scalar argument                                               */

/* ---- formats ----------------------------------------------------------------------------------------------- */
#define MI_QT_CB3    1   /* 3-bit codes (10 per u32) + 8 bf16 centroids per (row, 128-column group)              */
#define MI_QT_IQ3_S  2   /* llama.cpp IQ3_S in the reference's planar tables (planes.py:22-25)                   */
#define MI_QT_IQ4_XS 3   /* llama.cpp IQ4_XS in the reference's planar tables (planes.py:26-28)                  */
#define MI_QT_IQ2_S  4   /* llama.cpp IQ2_S in the reference's planar tables (planes.py:17-21)                   */
#define MI_QT_Q2_K   5   /* ggml Q2_K (the MTP layer's experts) in the reference's planar tables (planes.py:34-41) */
#define MI_QT_Q3_K   6   /* ggml Q3_K, likewise                                                                  */

/*
 * One expert table: E experts of one matrix kind (gate, up or down), every expert R rows x K inputs.  plane[] order:
 *   MI_QT_IQ3_S : {qs, sg, qh, sc, d}   -- the reference's planes, unchanged: u32 [E * rows_p, R], the matrix row
 *                                          on the minor axis (planes.py:5-14,45).  R % 64 == 0, K % 256 == 0.
 *   MI_QT_IQ4_XS: {qs, sl, sh, d}       -- likewise (planes.py:26-28,46).  R % 64 == 0, K % 256 == 0.
 *   MI_QT_IQ2_S : {qs, sg, qh, sc, d}   -- likewise (planes.py:17-21,45).  R % 64 == 0, K % 256 == 0.
 *   MI_QT_Q2_K  : {qs, sc, d}           -- likewise (planes.py:34-41,46).  R % 64 == 0, K % 256 == 0.
 *   MI_QT_Q3_K  : {qs, hm, sc, d}       -- likewise (sc: the 16 six-bit scales unpacked to bytes).
 *   MI_QT_CB3   : {qs, cb}              -- qs: u32 [E][ceil(K/160)][R/16][64][4] code tiles (16 rows x 160 columns,
 *                                          1 KB each, in the lane order of the matrix-core decoder; formats.py
 *                                          cb3_tile_words gives the bit map); cb: u32 [E][K/128][R][4] = bytes
 *                                          lo[0..3], lo[4..7], hi[0..3], hi[4..7] of the 8 bf16 centroids of each
 *                                          (group, row).  R % 64 == 0, K % 128 == 0.  The codes hold the canonical
 *                                          10-per-u32 bytes per row plus the zero padding of the last tile.
 */
typedef struct mi_table {
    int32_t qtype;
    int32_t rows;        /* R */
    int32_t cols;        /* K */
    int32_t n_experts;   /* E */
    const uint32_t *plane[5];
} mi_table;

/* x dtypes for mi_matvec */
#define MI_X_BF16  0     /* bf16 activations: dot products on bf16 pairs, exact products, f32 accumulation        */
#define MI_X_F32   1     /* f32 activations: split into bf16 hi + lo, two exact bf16 dots per pair (~2^-17 rel)   */

/*
 * Fused routed-expert matvec, one output row vector per slot (moe_matvec, pallas_moe.py:238-307):
 *   out[i, r] = sum_n W_{idx[i]}[r, n] * x_i[n]       for i < n_slots, r < R     (f32 accumulation, f32 out)
 * x: n_slots rows of K values (bf16 bits or f32 per x_dtype), row stride x_stride elements.
 * Slots that share an expert are grouped so each expert's codes are read once.  Rows of slots whose idx is outside
 * [0, E) are not written.  n_slots <= MI_MAX_SLOTS.  The workspace needs no initialisation.
 */
#define MI_MAX_SLOTS 128
int mi_matvec(const mi_table *t, const int32_t *idx, int32_t n_slots, const void *x, int32_t x_dtype,
              int32_t x_stride, float *out, void *workspace, size_t workspace_bytes, void *stream);
size_t mi_matvec_workspace(const mi_table *t, int32_t n_slots);

/*
 * Fused MoE decode layer (ResidentFetch._apply_kernel composition, resident.py:110-120), tokens grouped by expert:
 *   for each token n < N and slot j < k with e = idx[n, j]:
 *     g = Wgate_e x_n, u = Wup_e x_n, h = silu(min(g, limit)) * clip(u, -limit, limit)   (model.py:119-122)
 *     y = Wdown_e h
 *   out[n] = sum_j w[n, j] y_{n,j}  (+ the shared expert's y for every token, weight 1, if shared_expert >= 0)
 * x: bf16 [N, D] (D = gate.cols), idx int32 [N, k], w f32 [N, k].  Every product is exact and every accumulation
 * f32 (resident.py:114-120); x enters the matrix cores exactly, h (f32) as its bf16 high part plus a bf16 remainder,
 * i.e. 16 mantissa bits (~2^-17 relative per element).  out_f32 [N, D] and/or out_bf16 [N, D] (either may be NULL,
 * not both).  shared_expert: an expert index of the same tables applied to every token with weight 1, or -1.
 * Limits: N <= 16, N*k <= MI_MAX_SLOTS, E <= 1024.  Deterministic (fixed-order reductions, no float atomics).
 * Launches on the stream: gate/up partials, down partials and the routing-weighted combine, with a SwiGLU launch
 * between gate/up and down (four launches, as mi_moe_decode_phases with phases = 3), except for CB3 tables at one
 * token: two launches, gate/up, then down, which forms h from the gate/up partials while staging and does the
 * combine itself (the last workgroup to finish each 16-row tile sums it in the combine launch's order; no waits).
 * The workspace (mi_moe_decode_workspace bytes) holds a counter region of max(1 MiB, the layer's counter block)
 * bytes (the block: info[15] of mi_moe_decode_plan), then the partials and h; the counter region must be zero before
 * the workspace's first call (a zero-filled allocation), and every call leaves it zero.  The data never enters the
 * first MiB, so layers of different shapes (whose counters sit at different offsets) may share one workspace when
 * their counter blocks fit in it.
 * Calls that share a workspace must be ordered on one stream.
 */
int mi_moe_decode(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                  int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                  float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream);
size_t mi_moe_decode_workspace(const mi_table *gate, const mi_table *down, int32_t N, int32_t k,
                               int32_t shared_expert);

/*
 * mi_moe_decode with the activations in the layer dtype (the reference's apply takes x as the layer stores it:
 * bf16 in production, f32 in its CPU tests, test_resident_cpu.py:81; resident.py:114 upcasts it to f32):
 * x_dtype MI_X_BF16 (x bf16 [N, D], exactly mi_moe_decode) or MI_X_F32 (x f32 [N, D], staged as bf16 high part +
 * remainder: 16 mantissa bits, ~2^-17 relative, one workgroup per task).  Same workspace size, limits and results.
 */
int mi_moe_decode_x(const mi_table *gate, const mi_table *up, const mi_table *down, const void *x, int32_t x_dtype,
                    int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                    float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream);

/*
 * mi_moe_decode as ONE persistent launch (CB3 tables, N <= 8): gate/up, SwiGLU, down and the combine run as ordered
 * tasks that hand their results over through completion counters kept in the workspace; each workgroup streams its
 * gate/up tasks and then its down tasks with the next task's weights in flight.  Same arguments, workspace size and
 * results as mi_moe_decode (up to the f32 summation order of the column splits).  A small fill kernel zeroes the
 * workspace's counter block first (so the workspace needs no initialisation): two launches on the stream.  A
 * bounded wait that gives up (workgroups of the launch not resident together) ends the launch with invalid results
 * and a nonzero error word, u32 index info[14] of mi_moe_decode_plan in the workspace, until the next call on that
 * workspace.  MI_ERR_QTYPE for tables other than CB3, MI_ERR_TOKENS for N > 8.
 */
int mi_moe_decode_fused(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                        int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                        float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream);

/*
 * mi_moe_decode as separate launches (the reference runs gate/up and down as separate kernels too,
 * resident.py:116-119), any qtype: phases = 1: the gate/up launch only (its partials stay in the workspace);
 * 2: SwiGLU + down + combine only (consumes what a previous phase-1 call left in the same workspace, same arguments);
 * 3: both -- the launches of mi_moe_decode (gate/up partials, SwiGLU unless the down launch forms h, down partials,
 * routing-weighted combine).  CB3 with N > 8: the
 * gate/up and down launches are persistent (resident workgroups working through contiguous task ranges with the next
 * task's weights in flight); otherwise one workgroup per (expert group, row range, column split).  It never touches
 * the counter block of mi_moe_decode_fused.
 */
int mi_moe_decode_phases(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                         int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert,
                         float limit, float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes,
                         int32_t phases, void *stream);

/*
 * mi_moe_decode without a workspace argument, for callers that cannot allocate (code under HIP graph capture, serving
 * loops and harnesses that forbid hipMalloc).  No counterpart in the reference: its operator allocates through XLA.
 * The partials and h live in a static device array of MI_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends);
 * the call allocates nothing and returns MI_ERR_WORKSPACE when the layer's data region (the partials and h,
 * mi_moe_decode_workspace minus its counter region) exceeds the array less its first 256 KB -- the benchmark layer
 * (D 6144, I 2048) fits at every N <= 16, k = 8.  Same arguments (minus the workspace), launches and results as
 * mi_moe_decode (the first call on a GPU adds one fill launch).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, or two threads) race and
 * give wrong results; order them on one stream.  The array's first 256 KB hold the down launch's row-tile counters
 * (CB3 at one token), cleared by a fill kernel on the first call on each GPU and left zero by every call; nothing
 * else in it needs to start at zero.
 */
#define MI_NOALLOC_SCRATCH_BYTES (64u << 20)
int mi_moe_decode_noalloc(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                          int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert,
                          float limit, float *out_f32, uint16_t *out_bf16, void *stream);

/*
 * The launch plans of mi_moe_decode_fused and mi_moe_decode (no launch; for tests and tuning).  info[0..n_info):
 *   [0] 1 if mi_moe_decode_fused applies; [1] its workgroups; [2] 0 (reserved);
 *   [3..6] gate/up column splits, split alignment (column tiles), row tiles per wavefront, row ranges;
 *   [7..10] the same for down; [11] dynamic LDS bytes; [12] groups bound; [13] token class (entries 1-13: the one
 *   launch);
 *   [14] u32 index of the error word in the workspace (nonzero after a call whose wait gave up: results invalid);
 *   [15] bytes of the counter block at the start of the workspace (zero between calls);
 *   [16..23] mi_moe_decode's launches: gate/up splits, row tiles per wavefront, workgroups (0: one per task), down
 *   splits, row tiles per wavefront, workgroups (0: one per task), gate/up and down dynamic LDS bytes (persistent).
 *   [24] mi_moe_decode's gate/up and down kernels: 0 grouped (one workgroup per task), 1 persistent streams,
 *   2 CU-balanced streams (one workgroup per CU, CB3 at one token), 3 CU-balanced multi-token streams (CB3, 2-16
 *   tokens);
 *   [25] 1 if the CU-balanced down launch (CB3 at one token) does the combine itself (no combine launch); [26] 0
 *   (reserved).
 * Returns MI_OK or MI_ERR_ARG.
 */
int mi_moe_decode_plan(const mi_table *gate, const mi_table *down, int32_t N, int32_t k, int32_t shared_expert,
                       int32_t *info, int32_t n_info);

/*
 * GGUF blocks -> the reference's planar tables, on the device (planes.py:136-170 as resident.py:29-60 applies it
 * when loading a layer): blocks = one expert tensor as stored in the file, u8 [E][R][K/256][block bytes] (2-byte
 * aligned); planes = the table's plane pointers in mi_table order, u32 [E * rows_p, R] each (IQ2_S / IQ3_S: 5
 * planes, IQ4_XS: 4).  Bit-exact byte movement, one launch.  E <= 65535, K % 256 == 0.
 */
int mi_pack_planes(int32_t qtype, const uint8_t *blocks, int32_t E, int32_t R, int32_t K, void *const *planes,
                   void *stream);

/*
 * The MoE block's router (moe_route, model.py:798-808), the step before ResidentFetch.apply (model.py:843-848):
 *   logits = f32(x) @ router_w, scores = sigmoid(logits), idx = top_k(scores + bias, k) (largest first, equal values
 *   lower expert id first, as lax.top_k), w = scores[idx], w /= (sum_j w + 1e-20) if norm_topk, w *= scaling.
 * x bf16 [N, D] (4-byte aligned), router_w f32 [D, E] (the reference's layout), bias f32 [E] or NULL (zero);
 * idx_out int32 [N, k], w_out f32 [N, k].  N <= 2^19, D even, E <= 1024, 1 <= k <= min(E, 32), norm_topk 0 or 1.
 * f32 dot products (the reference's f32 matmul on its own hardware may round the logits differently: choices
 * within a few ulps of each other can order differently).  Two launches; the workspace (mi_moe_route_workspace
 * bytes) holds the partial logits and needs no initialisation.
 */
int mi_moe_route(const uint16_t *x_bf16, const float *router_w, const float *bias, int32_t N, int32_t D, int32_t E,
                 int32_t k, int32_t norm_topk, float scaling, int32_t *idx_out, float *w_out, void *workspace,
                 size_t workspace_bytes, void *stream);
size_t mi_moe_route_workspace(int32_t N, int32_t D, int32_t E);

/*
 * The reference's prefill slot layout (ragged_plan, pallas_moe.py:564-592), built on the device:
 *   S = T*k slots (token t, column j) sorted stably by expert idx[t, j]; every expert's rows padded to whole blocks
 *   of tm rows; G = ceil(S / tm) + E blocks, Rp = G * tm rows.
 *   blk_expert int32 [G]: expert of block g (blocks >= n_blocks repeat the last used expert; E - 1 if none)
 *   n_blocks   int32 [1]
 *   tok_row    int32 [Rp]: token of every sorted row, -1 = padding
 *   w_row      f32   [Rp]: routing weight w[t, j] of every sorted row, 0 = padding
 *   row_slot   int32 [T, k]: sorted row of every slot (-1 for an expert id outside [0, E), which the reference
 *                            does not define)
 * 1 <= E <= 1024, 1 <= tm <= 65536, T*k <= 2^22.  One workgroup; no workspace.
 */
int mi_ragged_plan(const int32_t *idx, const float *w, int32_t T, int32_t k, int32_t E, int32_t tm,
                   int32_t *blk_expert, int32_t *n_blocks, int32_t *tok_row, float *w_row, int32_t *row_slot,
                   void *stream);

/*
 * Fused MoE prefill layer (ResidentFetch._apply_ragged_kernel, resident.py:144-165) for CB3, IQ2_S, IQ3_S, IQ4_XS,
 * Q2_K or Q3_K tables (gate and up in one format, down in the same or another), grouped GEMMs on the matrix cores:
 *   plan   = ragged_plan over the T*k slots (+ one shared-expert column of weight 1 if shared_expert >= 0), tm = 80
 *   W      = bf16(dequantized weight): CB3 centroids as stored; IQ2_S bf16(level * f16(d) * (0.5 + sc) * 0.25);
 *            IQ3_S bf16(level * f16(d) * (1 + 2 sc)); IQ4_XS bf16(kvalue * f16(d) * (s - 32)); Q2_K / Q3_K
 *            bf16 of the f32 dequantized weight; rounded once to nearest even as the reference's tiles are
 *            (pallas_moe.py:341-350)
 *   h[row] = bf16(silu(min(g, L)) * clip(u, -L, L)),  g, u = Wgate_e x_t, Wup_e x_t in f32   (pallas_moe.py:622-690)
 *   y[row] = bf16(Wdown_e h[row]), f32 accumulation                                           (pallas_moe.py:693-755)
 *   out[t] = sum_j wt(t, j) y[row_slot(t, j)] in f32, wt = bf16(w[t, j]) for MI_COMBINE_MATMUL (resident.py:161-163)
 *            or w[t, j] for MI_COMBINE_GATHER (resident.py:164-165); the shared column has weight 1.
 * x bf16 [T, D], idx int32 [T, k], w f32 [T, k]; out_f32 and/or out_bf16 [T, D] (16-byte aligned, as the workspace).
 * Every expert's weights are read once per block of 80 rows. T*(k+1) <= 2^22, E <= 1024, gate.rows % 128 == 0,
 * down.rows % 256 == 0; the IQ formats also need cols % 256 == 0. MI_ERR_MISMATCH when gate and up differ in format
 * or shape. Four launches: plan, gate/up, down, combine. The workspace (mi_moe_prefill_workspace bytes) holds the
 * plan, h and y; it needs no initialisation.
 */
#define MI_COMBINE_MATMUL 0
#define MI_COMBINE_GATHER 1
int mi_moe_prefill(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                   int32_t T, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                   int32_t combine, float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes,
                   void *stream);
size_t mi_moe_prefill_workspace(const mi_table *gate, const mi_table *down, int32_t T, int32_t k,
                                int32_t shared_expert);

/*
 * The same grouped GEMMs with the rounding points of the reference's other bf16 branches of ResidentFetch.apply
 * (combine selects the branch; MI_COMBINE_MATMUL / MI_COMBINE_GATHER are mi_moe_prefill's):
 *   MI_COMBINE_SWEEP      the dense sweep, sweep_mode="dense" (_apply_sweep_kernel, resident.py:169-187, with
 *                         moe_sweep_gateup / moe_sweep_down, pallas_moe.py:382-555):
 *                           rw(t, e) = sum of w[t, j] over the token's columns j with idx[t, j] = e, in column order
 *                           hk = bf16(f32(bf16(swiglu(g, u))) * rw),  y = Wdown_e hk in f32 (not rounded)
 *                           out[t] = f32 sum of y over the token's experts
 *   MI_COMBINE_XLA_GATHER the XLA decode path, use_pallas=False (_apply_gather, resident.py:122-135):
 *                           g, u rounded to bf16 (the einsums' bf16 outputs), h = bf16(swiglu(g, u)),
 *                           y = bf16(Wdown_e h), out[t] = sum_j w[t, j] y in f32
 *   MI_COMBINE_XLA_SWEEP  the XLA prefill path, use_pallas=False (_apply_sweep_xla, resident.py:189-210):
 *                           g, u rounded to bf16, hk = bf16(f32(bf16(swiglu(g, u))) * rw), y = Wdown_e hk in f32;
 *                           per group of `chunk` consecutive expert ids, the group's y summed in f32, rounded to
 *                           bf16 once, added to out[t] in f32 in ascending group order
 * The shared column (shared_expert >= 0) is one more expert of weight 1 in every form. A token's second column of an
 * expert it names already gets weight 0 in the sweeps (its weight is in the first column's rw) and adds exactly 0.
 * chunk > 0 for MI_COMBINE_XLA_SWEEP, ignored otherwise. The sweeps keep y in f32: their workspace
 * (mi_moe_prefill_form_workspace) is larger than mi_moe_prefill_workspace.
 */
#define MI_COMBINE_SWEEP 2
#define MI_COMBINE_XLA_GATHER 3
#define MI_COMBINE_XLA_SWEEP 4
int mi_moe_prefill_form(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                        int32_t T, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                        int32_t combine, int32_t chunk, float *out_f32, uint16_t *out_bf16, void *workspace,
                        size_t workspace_bytes, void *stream);
size_t mi_moe_prefill_form_workspace(const mi_table *gate, const mi_table *down, int32_t T, int32_t k,
                                     int32_t shared_expert, int32_t combine);

/*
 * Exact dequantized weights of expert e (natural input order): out f32 [R, K].  Restates dequant_planes
 * (planes.py:196-206) / the codebook closed form; used to check the kernels' decode bit for bit.
 */
int mi_dequant(const mi_table *t, int32_t expert, float *out, void *stream);

/*
 * int8 projection (quant8.py:91-99 + x @ W) with the reference's scale layouts (quantize_array, quant8.py:26-32;
 * scale_axis, quant8.py:59-60) and the lm_head form (engine.py:345-351):
 *   MI_I8_ROW_SCALES (0): s f32 [n_in] (the reference's [in, 1], row-sharded leaves):
 *                         y[b, o] = sum_i x[b, i] * bf16(f32(q[o, i]) * s[i])
 *   MI_I8_COL_SCALES (1): s f32 [n_out] (the reference's [1, out]):  y[b, o] = sum_i x[b, i] * bf16(f32(q[o, i]) * s[o])
 *   MI_I8_COL_AFTER  (2): s f32 [n_out], the scale after the dot:      y[b, o] = (sum_i x[b, i] * q[o, i]) * s[o]
 * f32 accumulation; bf16 out (one rounding of the f32 result) and/or f32 out.
 * x bf16 [B, n_in]; qT int8 [n_out, n_in] (the reference's q [in, out] transposed once at load).
 * 1 <= B <= 32, n_in % 256 == 0, n_out % 16 == 0.  The weights are dequantized to bf16 in registers and contracted
 * on the matrix cores (bf16 x bf16 products are exact, f32 accumulation).
 * The workspace (mi_int8_project_workspace bytes, 16-byte aligned) starts with 256 KB of completion counters, then
 * the split-K partials.  The counters must be zero before a workspace's first int8 call (allocate it zero-filled);
 * every int8 call leaves them zero, so mi_int8_project, mi_int8_project_many and mi_int8_mlp may share one
 * workspace, ordered on one stream.  One launch: the workgroup that completes a row group's splits last adds the
 * partials in split order (a second, summing launch when a launch has more than 1024 row groups of 64 outputs).
 * scale_axis | MI_I8_TILED: qT is in the tiled layout that mi_int8_tile writes (same values, another byte order).
 */
#define MI_I8_ROW_SCALES 0
#define MI_I8_COL_SCALES 1
#define MI_I8_COL_AFTER  2
#define MI_I8_TILED      0x100
int mi_int8_project(const uint16_t *x_bf16, int32_t B, const int8_t *qT, const float *s, int32_t scale_axis,
                    int32_t n_in, int32_t n_out, uint16_t *y_bf16, float *y_f32, void *workspace,
                    size_t workspace_bytes, void *stream);
size_t mi_int8_project_workspace(int32_t B, int32_t n_in, int32_t n_out, int32_t scale_axis);

/*
 * The tiled layout of an int8 weight (no counterpart in the reference: a load-time repack, as the planar IQ tables
 * are): qT [n_out, n_in] -> tiled, n_out * n_in bytes, per 128-column block b and 16-row tile t one 2 KB piece at
 * (b * n_out / 16 + t) * 2048 in the order the projection kernels load it (1 KB contiguous per wavefront load
 * instead of 16 rows x 64 bytes at a stride of n_in).  n_out % 16 == 0, n_in % 256 == 0, both pointers 16-byte aligned.  Pass MI_I8_TILED in
 * scale_axis (mi_int8_project, mi_int8_project_many; gu_scale_axis / down_scale_axis of mi_int8_mlp) with it.
 */
int mi_int8_tile(const int8_t *qT, int32_t n_out, int32_t n_in, int8_t *tiled, void *stream);

/*
 * Several int8 projections of the same activations in one launch (Q, K, V of x; the shared expert's gate and up),
 * all with the same scale layout: projs[j] = {qT [n_out_j, n_in], s (as scale_axis), n_out_j, y_bf16 and/or y_f32
 * [B, n_out_j]}, 1 <= n_proj <= 8.  Each output equals what mi_int8_project gives for that projection alone.
 */
typedef struct mi_i8_proj {
    const int8_t *qT;
    const float *s;
    int32_t n_out;
    uint16_t *y_bf16;
    float *y_f32;
} mi_i8_proj;
int mi_int8_project_many(const uint16_t *x_bf16, int32_t B, int32_t n_in, const mi_i8_proj *projs, int32_t n_proj,
                         int32_t scale_axis, void *workspace, size_t workspace_bytes, void *stream);
size_t mi_int8_project_many_workspace(int32_t B, int32_t n_in, const int32_t *n_out, int32_t n_proj,
                                      int32_t scale_axis);

/*
 * int8 MLP (mlp_partial, model.py:125-127, over quant8.dequant_tree's bf16(f32(q) * s) weights, quant8.py:91-99):
 * the shared expert of the MoE block (moe_dense, model.py:855) and the dense MLP layers.
 *   g = bf16(x Wg), u = bf16(x Wu)                  (bf16 matmuls with f32 accumulation)
 *   h = bf16(silu(min(g, L)) * clip(u, -L, L))      (swiglu_clamped, model.py:119-122, evaluated in f32 once)
 *   y = h Wd in f32; y_bf16 = bf16(y)               (the reference's output is the bf16 one)
 * x bf16 [B, D]; gate/up qT int8 [I, D] with s per gu_scale_axis ([I] MI_I8_COL_SCALES or [D] MI_I8_ROW_SCALES);
 * down qT int8 [D, I] with s per down_scale_axis ([D] or [I]).  1 <= B <= 32, D % 256 == 0, I % 256 == 0.  Two
 * launches: gate and up together (their last workgroups form h), then down with its split sums.  Workspace:
 * mi_int8_mlp_workspace bytes, 256-byte aligned, its counters as for mi_int8_project (zero before the first call).
 */
int mi_int8_mlp(const uint16_t *x_bf16, int32_t B, int32_t D, int32_t I, const int8_t *gate_qT, const float *gate_s,
                const int8_t *up_qT, const float *up_s, int32_t gu_scale_axis, const int8_t *down_qT,
                const float *down_s, int32_t down_scale_axis, float limit, uint16_t *y_bf16, float *y_f32,
                void *workspace, size_t workspace_bytes, void *stream);
size_t mi_int8_mlp_workspace(int32_t B, int32_t D, int32_t I, int32_t gu_scale_axis, int32_t down_scale_axis);

/*
 * bf16 projection and MLP: the same contractions over the reference's non-int8 leaves, a bf16 W [in, out] used as
 * x @ W (model.py:125-127; the shared expert of moe_dense, model.py:855, and the dense MLP layers, model.py:131, when
 * the engine keeps its non-expert weights in bf16, int8_nonexpert=False, engine.py:281,305).
 *   mi_bf16_project: y = x W, f32 accumulation; bf16 out (one rounding of the f32 result) and/or f32 out.
 *   mi_bf16_mlp:     g = bf16(x Wg), u = bf16(x Wu), h = bf16(swiglu_clamped(g, u)) evaluated in f32 once,
 *                    y = h Wd in f32, y_bf16 = bf16(y) -- mi_int8_mlp's steps with W the bf16 leaf itself.
 * Weights are wT bf16 [n_out, n_in] (gate/up [I, D], down [D, I]): the reference's leaf transposed once at load,
 * 16-byte aligned.  Shapes, token limit, workspace layout and counter rule as for the int8 entry points (the
 * workspace's first 256 KB are counters that must be zero before its first call; every call leaves them zero, so
 * one workspace may serve the int8 and bf16 calls ordered on one stream).  No tiled form.
 */
int mi_bf16_project(const uint16_t *x_bf16, int32_t B, const uint16_t *wT, int32_t n_in, int32_t n_out,
                    uint16_t *y_bf16, float *y_f32, void *workspace, size_t workspace_bytes, void *stream);
size_t mi_bf16_project_workspace(int32_t B, int32_t n_in, int32_t n_out);
int mi_bf16_mlp(const uint16_t *x_bf16, int32_t B, int32_t D, int32_t I, const uint16_t *gate_wT,
                const uint16_t *up_wT, const uint16_t *down_wT, float limit, uint16_t *y_bf16, float *y_f32,
                void *workspace, size_t workspace_bytes, void *stream);
size_t mi_bf16_mlp_workspace(int32_t B, int32_t D, int32_t I);

/*
 * Launch-plan overrides, for tests and measurement runs only (no counterpart in the reference).  The library reads
 * no environment variables: every call plans its launches from built-in defaults, except for the names set here,
 * which replace those defaults process-wide until mi_tuning_reset.  Names (an unknown one gives MI_ERR_ARG):
 * split counts and row tiles of the decode launch families (S1, S2, FS1, FS2, SMV, each with _RTW and _AL; MS1, MS2,
 * CS1, CS2 with _RTW; MGMAX), launch-family switches (CUSTREAM, CUMULTI, PERSIST_ABOVE, FUSE_SWIGLU, CU_FORM_H), the
 * one-launch decode's poll limit (SPIN_LIMIT) and the int8 split plan (I8S, I8_WAVES, I8_FUSE).  Overrides change
 * launch shapes and summation orders, never the result beyond f32 rounding; workspace sizes follow them, so set them
 * before sizing a workspace.  Not synchronised with calls running on other host threads.
 */
int mi_tuning_set(const char *name, int32_t value);
void mi_tuning_reset(void);

const char *mi_strerror(int status);
int mi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MI355MOE_H */
