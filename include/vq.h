/* vq.h -- C ABI of the MI355X quantized-weight matvec library (libvq_hip.so).
 *
 * Plain pointers and sizes only. Every device pointer is a HIP device allocation on the current device;
 * `stream` is a hipStream_t (NULL = the null stream). All launches are asynchronous on `stream`.
 * Weights, fp32 activations and packed activations passed to the matvec entry points must be 16-byte
 * aligned (VQ_ERR_ARG otherwise): weights are streamed with 16-byte global-to-LDS loads.
 * Every entry point returns an int status: 0 on success, a negative VQ_ERR_* code for an invalid
 * argument (checked on the host before anything is launched), or a positive hipError_t value.
 *
 * Layouts (the reference's, see /root/reference/engine/csrc/megakernel/qwen_runtime.cu:616,626 and
 * csrc/cpu/qwen_cpu.c:603,635):
 *   w    raw GGUF blocks, row-major: row r occupies bytes [r*row_bytes, (r+1)*row_bytes) with
 *        row_bytes = cols/block_size*type_size, and at least VQ_TAIL_PAD (16) readable bytes follow the
 *        last row (the reference pads uploads the same way, qwen_runtime.cu:1366-1367)
 *   x    fp32 activations [ntok][cols]
 *   y    fp32 outputs     [ntok][rows]
 *   xq   int8 [ntok][cols], xd/xs fp32 [ntok][cols/32]: per 32-group scale d and d*sum(q)
 *   xpack  packed quantized activations, one record per token, vq_xpack_bytes(cols,1) bytes apart
 *        (16-byte multiple): xq[cols] int8 | xd[cols/32] fp32 | xh[cols/32] u32, where xh holds the
 *        sums of q over elements 0..15 (low 16 bits, signed) and 16..31 (high 16 bits, signed) of each
 *        group. The matvec copies a record verbatim into LDS.
 */
#ifndef VQ_H_
#define VQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (positive values are hipError_t). */
#define VQ_OK 0
#define VQ_ERR_TYPE (-1)      /* unsupported GGUF type id                                   */
#define VQ_ERR_SHAPE (-2)     /* rows/cols/ntok invalid, cols not a multiple of 32 / block  */
#define VQ_ERR_WORKSPACE (-3) /* workspace NULL or smaller than the matching *_bytes query  */
#define VQ_ERR_ARG (-4)       /* NULL pointer or other invalid argument                     */
#define VQ_ERR_NOT_INIT (-5)  /* vq_init() has not run on this device                        */
#define VQ_ERR_TOO_LARGE (-6) /* the call needs more than VQ_NOALLOC_SCRATCH_BYTES of scratch   */

/* GGUF type ids accepted by every entry point (qwen_quant.cuh:17-33, parser.py:33-63). */
#define VQ_TYPE_F32 0
#define VQ_TYPE_F16 1
#define VQ_TYPE_Q8_0 8
#define VQ_TYPE_Q2_K 10
#define VQ_TYPE_Q3_K 11
#define VQ_TYPE_Q4_K 12
#define VQ_TYPE_Q5_K 13
#define VQ_TYPE_Q6_K 14
#define VQ_TYPE_IQ2_XXS 16
#define VQ_TYPE_IQ2_XS 17
#define VQ_TYPE_IQ3_XXS 18
#define VQ_TYPE_IQ4_NL 20
#define VQ_TYPE_IQ3_S 21
#define VQ_TYPE_IQ2_S 22
#define VQ_TYPE_IQ4_XS 23

/* Replaces: type_traits() (qwen_quant.cuh:40-58) / GGUF_TYPE_TRAITS (parser.py:65-94). */
int vq_type_traits(int type, int *block_size, int *type_size);

/* Bytes of one weight row, or -1 for an unsupported type / cols not a multiple of the block size.
 * Replaces: row_bytes computation in Runtime_upload (qwen_runtime.cu:1352). */
long long vq_row_bytes(int type, int cols);

/* Human-readable text for a status code (for RuntimeError messages, qwen_runtime.cu:1100-1103). */
const char *vq_status_string(int status);

/* Prepare the library on the current device. Replaces: Runtime_init (qwen_runtime.cu:1272-1297). */
int vq_init(void);

/* Replace the IQ3_S codebook (512 entries x 4 magnitudes, 2048 bytes, host memory) on the current device.
 * Replaces: the iq3s_grid argument of Runtime(iq3s_grid) (qwen_runtime.cu:1272-1286, cuda/qwen_runtime.py:41-44). */
int vq_set_iq3s_grid(const uint8_t *grid);

/* Bytes of the packed activations (xpack) of `ntok` tokens of `cols` columns; 0 if cols % 32 != 0. */
size_t vq_xpack_bytes(int cols, int ntok);

/* Workspace bytes vq_qmv needs: 0 for cols <= 24576 (the activations are quantized inside the matvec),
 * else vq_xpack_bytes(cols, ntok) (they are packed into the workspace by vq_pack_x first). */
size_t vq_qmv_workspace_bytes(int cols, int ntok);

/* Workspace bytes with which vq_qmv takes its fastest path for this matrix and ntok: for 5..16 tokens of
 * Q3_K/Q4_K/Q5_K/Q6_K and the IQ types except IQ4_NL (cols a multiple of 256) the f16-MFMA small-batch matvec
 * (its split-K partial sums; 0 when cols <= 512), for 6..16 tokens of Q2_K, Q8_0 and IQ4_NL the int8-MFMA
 * small-batch matvec (its split-K partial sums; 0 when the columns are not split), else
 * vq_qmv_workspace_bytes. A smaller (but sufficient) workspace still works and selects the streaming matvec. */
size_t vq_qmv_workspace_bytes_for(int type, int rows, int cols, int ntok);

/* Paths of vq_qmv (the values vq_qmv_path returns). */
#define VQ_PATH_STREAM 0   /* streaming matvec (float weights: their own matvec)                */
#define VQ_PATH_MFMA_I8 1  /* int8-MFMA small-batch matvec                                      */
#define VQ_PATH_MFMA_F16 2 /* f16-MFMA small-batch matvec (Q3_K..Q6_K, IQ types but IQ4_NL)     */

/* The path vq_qmv takes for this matrix and ntok with a 16-byte aligned workspace of workspace_bytes (0: no
 * workspace), or the negative VQ_ERR_* status of a shape vq_qmv rejects. No counterpart in the reference
 * (its qmv has one path): for callers that choose between the grouped launches (streaming only) and
 * per-matrix vq_qmv calls. */
int vq_qmv_path(int type, int rows, int cols, int ntok, size_t workspace_bytes);

/* Quantize activations to int8 per 32-group: d = amax/127, id = 1/d, q = rint(x*id), xs = d*sum(q).
 * xs may be NULL. Replaces: the activation quantizer of Cpu_qmv (qwen_cpu.c:607-627). */
int vq_quantize_x(const float *x, int ntok, int cols, int8_t *xq, float *xd, float *xs, void *stream);

/* The same quantizer writing the packed layout `xpack` (vq_xpack_bytes(cols, ntok) bytes) that
 * vq_qmv_packed and vq_int_partials read. Replaces: the same quantizer (qwen_cpu.c:607-627). */
int vq_pack_x(const float *x, int ntok, int cols, void *xpack, void *stream);

/* y[t][r] = W[r] . x[t] for t < ntok (any ntok >= 1; weights are read once per launch of up to 8 tokens).
 * Quantized types quantize x per 32-group with the vq_pack_x quantizer: inside the matvec, or into
 * `workspace` (>= vq_qmv_workspace_bytes, else VQ_ERR_WORKSPACE) when that is non-zero; F32/F16 weights use
 * x directly. Replaces: Runtime_qmv (qwen_runtime.cu:1860-1912) on its matvec branch,
 * whose numerics contract is Cpu_qmv (qwen_cpu.c:581-641). */
int vq_qmv(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, void *workspace,
           size_t workspace_bytes, void *stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). vq_qmv with no workspace argument: the
 * small-batch paths' scratch (split-K partial sums, packed activations) lives in one static device array of
 * VQ_NOALLOC_SCRATCH_BYTES per GPU, set up by vq_init (VQ_ERR_NOT_INIT before it). Same kernels, routing and
 * results as vq_qmv with vq_qmv_workspace_bytes_for bytes of workspace; calls that would need more scratch
 * than the array holds return VQ_ERR_TOO_LARGE (e.g. 5 or more tokens of a 248320-row LM head). It allocates
 * nothing. Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU (different
 * streams, or several host threads) race and must be serialised by the caller. */
#define VQ_NOALLOC_SCRATCH_BYTES (32u << 20)
int vq_qmv_noalloc(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, float *y, void *stream);

/* Group g of x (n floats each): y = x * rsqrt(mean(x^2) + eps) * w, times silu(z) elementwise when z is not
 * NULL; in-place (y == x) allowed. Replaces: Runtime.rmsnorm / Runtime.gated_rmsnorm (qwen_runtime.cu:36-52,
 * 1914-1939). */
int vq_rmsnorm(const float *x, const float *w, const float *z, float *y, int n, int groups, float eps, void *stream);

/* out[i] = a[i] + b[i] (op 0), silu(a[i]) * b[i] (op 1), a[i] * sigmoid(b[i]) (op 2), i < n. Replaces:
 * Runtime.add / silu_mul / sigmoid_mul (binary_op, qwen_runtime.cu:54-67, 1941-1958; same op codes). */
int vq_binary(int op, const float *a, const float *b, float *out, long n, void *stream);

/* q[h][d] = raw[h][d], gate[h][d] = raw[h][hd + d] for heads x hd (raw rows are [query, gate]). Replaces:
 * Runtime.split_gated_q (qwen_runtime.cu:70-76). */
int vq_split_gated_q(const float *raw, float *q, float *gate, int heads, int hd, void *stream);

/* dst[r] = [a[r] | b[r]] for rows of `width` floats (dst holds rows x 2*width). Replaces: Runtime.concat_rows
 * (qwen_runtime.cu:2567-2587). */
int vq_concat_rows(float *dst, const float *a, const float *b, int rows, int width, void *stream);

/* Clear nbytes bytes at p with a fill kernel (no hipMemsetAsync, so the call can be captured in a graph).
 * Replaces: Runtime.zero_range (qwen_runtime.cu:2589-2600) and Runtime.zero. */
int vq_zero(void *p, size_t nbytes, void *stream);

/* ---- sequence ops -------------------------------------------------------------------------------------
 * The multi-sequence (_seg) forms take the pass's segment table as a HOST array segs[nseg][4] of int32
 * (slot, pos0, rows, row0): segment i is `rows` consecutive positions pos0.. of sequence slot `slot`, stored
 * in buffer rows row0 .. row0 + rows - 1 (the layout set_segments defines, qwen_runtime.cu:2352-2385).
 * nseg <= VQ_MAX_SEGMENTS; the table is copied into the launch arguments, so each op is one launch for the
 * whole pass. Paged KV caches are page pools [page][kv_head][page_size][hd] (fp32 or fp16) with the int32
 * DEVICE page table page_table[slot * pages_per_seq + pos / page_size] (set_paging, qwen_runtime.cu:100-110,
 * 2333-2350); every pos0 + rows must fit in page_size * pages_per_seq. */
#define VQ_MAX_SEGMENTS 64
#define VQ_CONV_MAX_K 8
/* Attention of a pass whose longest segment has more rows than this (a prompt pass) runs on the tiled MFMA
 * kernel (K/V read once per 16 query rows), else on the per-row decode kernel; results agree within fp32
 * rounding. The reference switches at the same row count (kMaxTokens, qwen_runtime.cu:572,2003). */
#define VQ_ATTN_ROW_MAX 8

/* NeoX RoPE in place on x [ntok][heads][hd], dims [0, rot) of each head, token t at position pos0 + t:
 * (x[j], x[j + rot/2]) turns by (pos0 + t) * base^(-2j/rot). Replaces: Runtime.rope (qwen_runtime.cu:81-92,
 * 1966-1977). */
int vq_rope(float *x, int ntok, int heads, int hd, int rot, int pos0, double base, void *stream);

/* vq_rope with each segment's positions (row row0 + t at position pos0 + t). Replaces: Runtime.rope_seg
 * (qwen_runtime.cu:2400-2417). */
int vq_rope_seg(float *x, const int32_t *segs, int nseg, int heads, int hd, int rot, double base, void *stream);

/* k, v [ntok][kv_heads][hd] fp32 into contiguous caches kc, vc [kv_heads][max_seq][hd] of `elem` bytes per
 * value (4: fp32, 2: fp16 rounded to nearest) at positions pos0 .. pos0 + ntok - 1. Replaces:
 * Runtime.kv_append (qwen_runtime.cu:115-128, 1979-2000, contiguous caches). */
int vq_kv_append(const float *k, const float *v, void *kc, void *vc, int elem, int ntok, int kv_heads, int max_seq,
                 int hd, int pos0, void *stream);

/* Each segment's k, v rows into its sequence's pages of the paged caches kc, vc. Replaces: Runtime.kv_append_seg
 * (qwen_runtime.cu:2419-2447). */
int vq_kv_append_seg(const float *k, const float *v, void *kc, void *vc, int elem, const int32_t *segs, int nseg,
                     int kv_heads, int hd, const int32_t *page_table, int page_size, int pages_per_seq, void *stream);

/* GQA attention: out[t][h] = softmax(q[t][h] . K / sqrt(hd)) V over the positions query token t sees, with K,
 * V the rows of kv head h / (heads / kv_heads) in caches [kv_heads][max_seq][hd] (`elem` 4: fp32, 2: fp16).
 * Token t sees [start, seq_len + t) (causal) or [start, seq_len + ntok - 1) (bidirectional != 0); start =
 * seq_len + t - window when window > 0 and that is positive, else 0. hd <= 256. Replaces: Runtime.attention
 * (qwen_runtime.cu:128-162, 2043-2067, contiguous caches). */
int vq_attention(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads, int hd,
                 int max_seq, int seq_len, int ntok, int bidirectional, int window, void *stream);

/* Causal attention of each segment's rows over its own pages: row t of a segment sees positions
 * [0, pos0 + t + 1). Replaces: Runtime.attention_seg (qwen_runtime.cu:2449-2478). */
int vq_attention_seg(const float *q, const void *kc, const void *vc, float *out, int elem, const int32_t *segs,
                     int nseg, int heads, int kv_heads, int hd, const int32_t *page_table, int page_size,
                     int pages_per_seq, void *stream);

/* Workspace bytes of vq_attention_ws for these shapes (0: the call takes the per-row kernel, ntok > VQ_ATTN_ROW_MAX
 * or invalid arguments). */
size_t vq_attention_workspace_bytes(int heads, int kv_heads, int hd, int seq_len, int ntok, int window);

/* vq_attention for decode and verify passes (ntok <= VQ_ATTN_ROW_MAX) with a workspace (>=
 * vq_attention_workspace_bytes, 16-byte aligned): the context is cut into chunks over about 512 workgroups, each
 * running every query head of a kv head on fp32 MFMA against its chunk, and the chunks' partial softmax
 * results are merged in chunk order (flash decoding; deterministic). Longer passes run as vq_attention.
 * Replaces: Runtime.attention on its decode path (qwen_runtime.cu:128-162, 2003-2050), which runs one block per
 * (head, token) over the whole context. */
int vq_attention_ws(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads,
                    int hd, int max_seq, int seq_len, int ntok, int bidirectional, int window, void *workspace,
                    size_t workspace_bytes, void *stream);

/* Workspace bytes of vq_attention_seg_ws for this segment table (0 when a segment has more than VQ_ATTN_ROW_MAX rows:
 * the call then takes the prompt kernel and needs none). */
size_t vq_attention_seg_workspace_bytes(const int32_t *segs, int nseg, int heads, int kv_heads, int hd);

/* vq_attention_seg with the workspace of the split-context decode kernel (as vq_attention_ws). Replaces:
 * Runtime.attention_seg (qwen_runtime.cu:2449-2478). */
int vq_attention_seg_ws(const float *q, const void *kc, const void *vc, float *out, int elem, const int32_t *segs,
                        int nseg, int heads, int kv_heads, int hd, const int32_t *page_table, int page_size,
                        int pages_per_seq, void *workspace, size_t workspace_bytes, void *stream);

/* vq_attention / vq_attention_seg on the tiled MFMA kernel whatever the row count: each row's result then depends
 * only on its own sequence (the same key tiles in the same order whatever else runs in the pass), the
 * attention half of the batch-invariant mode (the reference runs its tensor-core prompt kernel for every
 * pass then, qwen_runtime.cu:2003-2050, qwen_gpu.py:738-744). */
int vq_attention_tiled(const float *q, const void *kc, const void *vc, float *out, int elem, int heads, int kv_heads,
                       int hd, int max_seq, int seq_len, int ntok, int bidirectional, int window, void *stream);
int vq_attention_seg_tiled(const float *q, const void *kc, const void *vc, float *out, int elem, const int32_t *segs,
                           int nseg, int heads, int kv_heads, int hd, const int32_t *page_table, int page_size,
                           int pages_per_seq, void *stream);

/* Causal depthwise conv + SiLU over ntok tokens: per channel the state [channels][K] (K <= VQ_CONV_MAX_K) holds
 * the last K inputs; per token it shifts, appends x[t][c], and out[t][c] = silu(state . w[c]). snap (may be
 * NULL): [ntok - 1][channels][K] states after each token but the last. write_state = 0 leaves the state
 * untouched (a speculative verification pass). Replaces: Runtime.conv_update (qwen_runtime.cu:397-426,
 * 2081-2100). */
int vq_conv_update(const float *x, float *state, const float *w, float *out, int channels, int K, int ntok, float *snap,
                   int write_state, void *stream);

/* vq_conv_update per segment over the slot's state (state [slot][channels][K]); snap needs a single segment.
 * Replaces: Runtime.conv_update_seg (qwen_runtime.cu:2480-2511). */
int vq_conv_update_seg(const float *x, float *state, const float *w, float *out, int channels, int K,
                       const int32_t *segs, int nseg, float *snap, int write_state, void *stream);

/* Gated delta rule over ntok tokens, state [value_heads][kd][vd] of state_elem bytes per value (4: fp32, 2: fp16,
 * widened to fp32 for the pass and rounded once at its end), kd <= 256: conv rows [q (key_heads*kd) |
 * k (key_heads*kd) | v (value_heads*vd)], b / a [ntok][value_heads] raw beta / alpha, ssm_a / dt [value_heads];
 * head_order 0: key head h / (vh / kh), 1: h % kh. out [ntok][value_heads][vd]; snap (fp32 state only, may be
 * NULL) [ntok - 1][vh][kd][vd]; write_state = 0 leaves the state untouched. Replaces: Runtime.gated_delta
 * (qwen_runtime.cu:433-567, 2102-2165; fp16 state as its launch_gated_delta_h). */
int vq_gated_delta(const float *conv, const float *b, const float *a, const float *ssm_a, const float *dt, void *state,
                   int state_elem, float *out, int key_heads, int value_heads, int kd, int vd, float eps,
                   int head_order, int ntok, float *snap, int write_state, void *stream);

/* vq_gated_delta per segment over the slot's state ([slot][vh][kd][vd]); snap needs a single segment and fp32
 * state. Replaces: Runtime.gated_delta_seg (qwen_runtime.cu:2513-2565). */
int vq_gated_delta_seg(const float *conv, const float *b, const float *a, const float *ssm_a, const float *dt,
                       void *state, int state_elem, float *out, int key_heads, int value_heads, int kd, int vd,
                       float eps, int head_order, const int32_t *segs, int nseg, float *snap, int write_state,
                       void *stream);

/* Activation staging flags of vq_qmv_staged: the bits of the reference megakernel's QMV flags
 * (runtime/instructions.py:179-182; QMV_FLAG_ARGMAX = 4 is vq_lmhead_argmax here). */
#define VQ_QMV_ADD 1      /* y[t][r] += (W v)[r] instead of =                                      */
#define VQ_QMV_NORM 2     /* v = rmsnorm(v) * norm_w: v * norm_w[i] / sqrt(mean(v^2) + eps), per token */
#define VQ_QMV_SILU_MUL 8 /* v = silu(x) * x2 (applied before NORM), silu(z) = z / (1 + exp(-z))  */

/* y = W v with v staged from fp32 activations inside the matvec (flags VQ_QMV_*, 0 = plain x): x, x2
 * [ntok][cols], norm_w [cols], all 16-byte aligned; quantized types, cols <= 24576, no workspace.
 * Replaces: the megakernel's op_qmv staging (qwen_megakernel.cu:468-551), which removes the separate
 * silu_mul / rmsnorm / add passes around a projection. */
int vq_qmv_staged(int type, const uint8_t *w, int rows, int cols, const float *x, const float *x2,
                  const float *norm_w, float eps, int flags, int ntok, float *y, void *stream);

/* Workspace bytes with which vq_qmv_staged_ws runs 5-16 tokens (3-4 over inputs wider than the streaming kernel's
 * activation image holds twice) of Q3_K..Q6_K and the IQ types but IQ4_NL on the f16-MFMA small-batch matvec: the
 * per-token RMS scales (256 B) and the K ranges' partial sums. 0 for every other call (it then streams). */
size_t vq_qmv_staged_workspace_bytes(int type, int rows, int cols, int ntok);

/* vq_qmv_staged with a workspace: with >= vq_qmv_staged_workspace_bytes (16-byte aligned) the staging runs inside
 * the f16-MFMA small-batch matvec, which stages each K range's activations before quantizing them (SILU_MUL;
 * NORM with per-token scales rsqrt(mean(v^2) + eps) from one prepass launch) and adds y's previous value in its
 * K-range sum (ADD); any cols multiple of 256. Otherwise it is vq_qmv_staged. Replaces: the megakernel's op_qmv
 * staging at every batch size (qwen_megakernel.cu:468-551), for speculative-verify passes of 5-16 tokens. */
int vq_qmv_staged_ws(int type, const uint8_t *w, int rows, int cols, const float *x, const float *x2,
                     const float *norm_w, float eps, int flags, int ntok, float *y, void *workspace,
                     size_t workspace_bytes, void *stream);

/* Same as vq_qmv with activations already packed by vq_pack_x (quantized types only), so several
 * matrices that share one input (gate/up, q/k/v) quantize it once. Replaces: dot_row_q's caller loop
 * (qwen_cpu.c:628-637). */
int vq_qmv_packed(int type, const uint8_t *w, int rows, int cols, const void *xpack, int ntok, float *y,
                  void *stream);

/* Grouped matvec: y[k][t][r] = W_k[r] . x[t] for k < n <= VQ_MAX_GROUP matrices of one quantized type and
 * width sharing packed activations (a layer's gate/up or q/k/v): one launch streams all of them. w, rows, y
 * are host arrays of n entries. No counterpart in the reference's per-matrix qmv (qwen_runtime.cu:1860);
 * its effect equals n vq_qmv_packed calls. */
#define VQ_MAX_GROUP 4
int vq_qmv_group(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                 const void *xpack, int ntok, void *stream);

/* vq_qmv_group on fp32 activations, quantized inside the matvec by every workgroup (no separate quantizer
 * launch; best up to cols = 24576, which covers a qwen35 FFN down input). Same numerics as vq_pack_x +
 * vq_qmv_group. */
int vq_qmv_group_f32(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                     const float *x, int ntok, void *stream);

/* vq_qmv_group_f32 with vq_qmv's batch routing, for callers that pass a workspace: 5-16 tokens of Q3_K, Q4_K,
 * Q5_K or Q6_K run all n matrices in one f16-MFMA launch (plus one launch adding the K ranges' partial sums);
 * other MFMA batches run matrix by matrix as vq_qmv; everything else as vq_qmv_group_f32. The workspace size
 * is vq_qmv_group_workspace_bytes (rows: the n row counts); with less, the call routes as if it had none. No
 * counterpart in the reference's per-matrix qmv (qwen_runtime.cu:1860); its effect equals n vq_qmv calls with
 * that workspace. */
size_t vq_qmv_group_workspace_bytes(int type, int n, const int *rows, int cols, int ntok);
int vq_qmv_group_ws(int type, int n, const uint8_t *const *w, const int *rows, float *const *y, int cols,
                    const float *x, int ntok, void *workspace, size_t workspace_bytes, void *stream);

/* vq_qmv_group_f32 over matrices of up to two quantized types (types[k] per matrix): a main type and Q8_0,
 * the type GGUF mixes give a layer's small tensors (e.g. the gated-delta beta/alpha projections next to its
 * Q5_K qkv/gate), or Q5_K and Q6_K (a full-attention layer's q next to its k and v). One launch per token chunk
 * of at most 4; other type mixes run as one launch per type. No
 * counterpart in the reference's per-matrix qmv (qwen_runtime.cu:1860); its effect equals n vq_qmv calls. */
int vq_qmv_group_mixed_f32(int n, const int *types, const uint8_t *const *w, const int *rows, float *const *y,
                           int cols, const float *x, int ntok, void *stream);

/* Prefill contraction: y[t][r] = W[r] . x[t] for t < M (any M >= 1; meant for M >= 64) on int8 MFMA
 * (v_mfma_i32_16x16x32_i8), activations packed by vq_pack_x. Same quantized numerics as the matvec (rel-L2
 * <= 1e-5 against the reference CPU path), weights read once per 128 tokens. Replaces: the prefill branch of
 * Runtime_qmv for ntok >= gemm_min_rows, vinf_qgemm_kernel (qwen_runtime.cu:1886-1902,663-739), which rounds
 * x to fp16 instead of using the CPU path's int8 activations. */
int vq_qgemm(int type, const uint8_t *w, int rows, int cols, const void *xpack, int M, float *y, void *stream);

/* Workspace bytes of vq_qgemm_ws for this matrix and M tokens: non-zero for Q2_K..Q6_K, IQ2_XXS/XS/S and IQ3_XXS
 * (the f16-MFMA path, M * cols < 2^30), 0 otherwise (vq_qgemm_ws then runs vq_qgemm and ignores the workspace). */
size_t vq_qgemm_workspace_bytes(int type, int rows, int cols, int M);

/* vq_qgemm with a workspace: for Q2_K..Q6_K, IQ2_XXS/XS/S and IQ3_XXS the contraction runs on f16 MFMA
 * (v_mfma_f32_16x16x32_f16) with each weight element as the exact f16 integer code * sub-block scale (IQ2 and
 * IQ3_XXS: grid magnitude * sign * (2s + 1); Q6_K: its f16 rounding plus the exact remainder, whose b_lo product,
 * under ~1e-7 of it, is left out) and each
 * activation element as xq * xd split into two f16 (22 significant bits); d and dmin apply once per super-block. Same bar against
 * the reference CPU path (rel-L2 <= 1e-5), deterministic (split-K partials add in a fixed order). Workspace
 * below vq_qgemm_workspace_bytes -> VQ_ERR_WORKSPACE. Replaces: as vq_qgemm (qwen_runtime.cu:1886-1902). */
int vq_qgemm_ws(int type, const uint8_t *w, int rows, int cols, const void *xpack, int M, float *y, void *workspace,
                size_t workspace_bytes, void *stream);

/* vq_qgemm_ws with flags. VQ_GEMM_BATCH_INVARIANT: the f16 path cuts every tile's K range at boundaries that
 * depend only on the matrix (not on M), so each token's outputs are bit-identical whatever batch it runs in
 * (the int8 path, every other type, takes the whole K range per tile and is so already). This is the contract
 * of the reference's prompt kernels (K order independent of tiling, qwen_runtime.cu:650-654,1883-1885) and of
 * its --batch-invariant mode (qwen_cli.py:47-49); it costs 10-20 % at 512 tokens. */
#define VQ_GEMM_BATCH_INVARIANT 1
size_t vq_qgemm_workspace_bytes_ex(int type, int rows, int cols, int M, int flags);
int vq_qgemm_ws_ex(int type, const uint8_t *w, int rows, int cols, const void *xpack, int M, float *y, void *workspace,
                   size_t workspace_bytes, int flags, void *stream);

/* The prefill contraction with the reference's tensor-core numerics: fp32 activations x [M][cols] rounded to f16
 * (each token first scaled by a power of two that puts its largest |x| just below 2^15, undone on the outputs, so
 * no token overflows or flushes to zero where the reference's plain conversion would), weights exact, fp32
 * accumulation: y = sum_k deq(w) f16(x). One MFMA per product instead of the b_hi/b_lo pair of vq_qgemm_ws, for the
 * types of vq_qgemm_ws's f16 path (Q2_K-Q6_K, IQ2_XXS/XS/S, IQ3_XXS; other types -> VQ_ERR_TYPE). Weights are exact
 * but for Q6_K, whose integer product (q - 32) sc is rounded to f16 once (within 2^-11, as the reference rounds
 * every dequantized weight to fp16). Workspace and flags as vq_qgemm_ws_ex (same byte count).
 * Against the int8 activations of vq_qgemm_ws the outputs move by the f16 rounding of x (rel-L2 ~1e-4); against
 * those operands evaluated exactly, rel-L2 <= 1e-5. Replaces: f32_to_f16_rows_kernel + vinf_qgemm_kernel
 * (qwen_runtime.cu:657-661,663-739, launched :1898). */
int vq_qgemm_f16x_ws(int type, const uint8_t *w, int rows, int cols, const float *x, int M, float *y, void *workspace,
                     size_t workspace_bytes, int flags, void *stream);

/* Workspace bytes vq_lmhead_argmax needs for this matrix and ntok (0 for invalid arguments). */
size_t vq_lmhead_argmax_workspace_bytes(int type, int rows, int cols, int ntok);

/* Fused LM head: out_idx[t] = argmax_r (W[r] . x[t]) for t < ntok (ties -> lowest row; NaN and -inf never
 * win; INT32_MAX when no row qualifies), without re-reading the logits: each wave keeps the best of its
 * rows and a one-block kernel reduces the per-wave bests. logits may be NULL; if not, y[t][r] is written
 * too. Replaces: the QMV_FLAG_ARGMAX path + op_argmax (qwen_megakernel.cu:552-606,800-829) and
 * Runtime_qmv + Runtime_argmax_rows (qwen_runtime.cu:1860-1912,2181-2197). */
int vq_lmhead_argmax(int type, const uint8_t *w, int rows, int cols, const float *x, int ntok, int32_t *out_idx,
                     float *logits, void *workspace, size_t workspace_bytes, void *stream);

/* Test hook: part[((t*rows + r)*(cols/32) + g)*2 + h] = exact int32 sum over the 16 elements of half h
 * of group g of (weight code * xq), computed by the matvec's own decoders from packed activations.
 * Replaces: the integer stage of dot_row_q (qwen_cpu.c:125-342). */
int vq_int_partials(int type, const uint8_t *w, int rows, int cols, const void *xpack, int ntok, int32_t *part,
                    void *stream);

/* Test hook: out[r*cols + c] = fp32 value of W[r][c]. Replaces: deq8 (qwen_quant.cuh:151-279) and
 * dequantize_tensor (dequant.py:17-57). */
int vq_dequant_rows(int type, const uint8_t *w, int rows, int cols, float *out, void *stream);

/* out[t] = argmax_i x[t*n + i] (ties -> lowest index; NaN never wins; an all -inf/NaN row gives INT32_MAX).
 * Replaces: argmax_kernel + Runtime_argmax / Runtime_argmax_rows (qwen_runtime.cu:850-876, 2167-2197). */
int vq_argmax_rows(const float *x, int n, int ntok, int32_t *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VQ_H_ */
