/* librfill -- MI355X (gfx950) kernels for the RidgeFill late-layer fill.
 *
 * A flat C ABI: plain device pointers, element counts and strides, and the HIP stream every call is
 * ordered on. Nothing here allocates device memory, and nothing keeps state between calls except the
 * thread-local error text, the side stream and events rf_gdn_fill creates once per device, and
 * rf_gdn_fill_noalloc's static device array. Every call returns RF_OK or a negative status and leaves a
 * message for rf_last_error(). Tensors are row-major; "bf16" buffers hold IEEE bfloat16 bit patterns (uint16_t).
 *
 * Each entry point names the reference code it replaces (paths in the reference repository,
 * Approximate-Science/ridgefill-data).
 */
#ifndef RFILL_H
#define RFILL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RF_OK 0
#define RF_EINVAL_SHAPE (-1)   /* a size, stride or alignment the kernels do not take */
#define RF_EINVAL_ARG (-2)     /* a null pointer or an out-of-range scalar argument */
#define RF_EUNSUPPORTED (-3)   /* a model feature these kernels do not implement (never approximated) */
#define RF_EHIP (-4)           /* the HIP runtime reported an error (launch or device) */

/* Columns per row sum-of-squares partial: RMSNorm statistics travel as fp32 [rows, H / 256]. */
#define RF_SSQ_COLS 256

const char* rf_last_error(void);
int rf_version(void);

/* Ridge-map apply, x = b W^T + c in bf16 (one rounding after the fp32 sum and the bias), for P rows.
 * Replaces Projector.__call__ (code/kva/kva.py:150-156, F.linear in bf16).
 * b [P, h_in] (row stride ldb), w [h_out, h_in] (F.linear layout), c [h_out] or NULL,
 * x [P, h_out] (row stride ldx). Also writes ssq [P, h_out / 256]: each row's sum of squares of the
 * rounded x over consecutive 256-column groups (the next layer's RMSNorm statistics).
 * Needs h_in % 64 == 0, h_out % 256 == 0, ldb / ldx multiples of 8, 16-byte aligned pointers.
 * workspace / ws_bytes (optional, NULL / 0): see rf_gemm_workspace_bytes. */
int rf_map_apply(const uint16_t* b, int64_t ldb, const uint16_t* w, const uint16_t* c,
                 uint16_t* x, int64_t ldx, float* ssq, int64_t P, int64_t h_in, int64_t h_out,
                 void* workspace, size_t ws_bytes, hipStream_t stream);

/* Bytes of the optional workspace of the GEMM entry points (rf_map_apply, rf_norm_kv_write, rf_norm_q,
 * rf_norm_linear) for an M x N x K product (M rows, N outputs, K inputs): nonzero for products of at most
 * 512 rows (the exact rows' projections: a kernel that takes all of a row block's rows against 256 weight
 * rows, K split up to 16 ways), when the output tiles (256 x 256) are too few to give every CU one, e.g.
 * the tail's projections, or when the last wave of whole tile rows is at most half full (then only those
 * rows split; the rest run as usual), e.g. the 32K-row K/V product of an 8B model (896 tiles: 768 + 128
 * split two ways). Given a workspace at least this large (caller-owned device memory, 16-byte aligned),
 * the entry point keeps the fp32 partial sums of its K ranges there and adds them in a fixed order before
 * the epilogue (the same bits every run; with one range, the unsplit kernels' bits; otherwise the sum
 * order differs within fp32 rounding). With a smaller or NULL workspace it runs unsplit. Host only. */
int rf_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes);

/* Bytes of the workspace rf_norm_kv_rows and rf_norm_qkv_rows require for `rows` scattered rows of an
 * N-output, K-input product (N = 2 hkv d, or hq d + 2 hkv d; K = H). They run the rows in chunks of 512,
 * each chunk planned on its own, and a shorter last chunk can take more K splits than a full one: this is
 * the largest of the chunks' rf_gemm_workspace_bytes. Host only. The few-rows sizing of the exact rows'
 * cache writes (code/kva/model.py:259-276 runs them as ordinary layer products). */
int rf_rows_workspace_bytes(int64_t rows, int64_t N, int64_t K, size_t* bytes);

/* Row sum-of-squares partials of given layer inputs x [P, H] -> ssq [P, H / 256], the statistics the
 * fused input RMSNorm of rf_norm_kv_write reads (the mean of x^2 in code/kva/ops.py:14-25).
 * Bitwise the partials rf_map_apply writes for the same x. */
int rf_row_ssq(const uint16_t* x, int64_t ldx, float* ssq, int64_t P, int64_t H, hipStream_t stream);

/* Exact-row scatter x[rows[j]] = hr[j] for j < nrows, bit-exact, and those rows' ssq partials.
 * Replaces x.index_copy(0, rows, hr) (code/kva/kva.py:428-431). rows: int64 on the device; the caller
 * checks they are sorted, unique and < P (as kva.py:357-362 does); a row outside [0, P) is skipped. */
int rf_row_scatter(uint16_t* x, int64_t ldx, float* ssq, int64_t P, int64_t H, const int64_t* rows,
                   int64_t nrows, const uint16_t* hr, int64_t ldhr, hipStream_t stream);

/* Fold an RMSNorm gain into projection weights: w_out[n, k] = bf16(w[n, k] * g(k)), with
 * g = gain (Llama / Qwen3 rms_norm, kind 0) or 1 + gain (Qwen3.5 rms_norm_zc, kind 1).
 * Run once per layer when weights are packed; feeds rf_norm_kv_write. w, w_out [N, K]; gain [K]. */
int rf_fold_norm(const uint16_t* w, const uint16_t* gain, int kind, uint16_t* w_out, int64_t N,
                 int64_t K, hipStream_t stream);

/* RoPE table for P rows: cs [P, rot] bf16 with cs[j, 0 : rot/2] = bf16(cos(float(pos[j]) * inv_freq))
 * and cs[j, rot/2 : rot] = bf16(sin(...)), fp32 angles (code/kva/ops.py:59-63; the reference's cos /
 * sin tables repeat the half table twice, so the half table is all that is kept). One table serves
 * every late layer of a prompt: the positions and frequencies do not change between layers. */
int rf_rope_table(const int64_t* pos, int64_t P, const float* inv_freq, int rot, uint16_t* cs,
                  hipStream_t stream);

/* Fused attention-layer fill from layer inputs: input RMSNorm, K / V projections, optional per-head
 * k_norm, RoPE on K and the write of P rows into the K / V cache.
 * Replaces Model.fill (code/kva/model.py:278-280) = in_norm (ops.py:14-25) + Llama._kv /
 * Qwen3._kv / Qwen35._attn_kv (model.py:234-239, 340-345, 415-421) + _append_kv (model.py:139-159).
 *   x [P, H] layer inputs (row stride ldx), ssq [P, H / 256] their partials, eps the norm epsilon;
 *   wkv [2 hkv d, H]: rows [0, hkv d) the K projection, then the V projection, both with the input
 *       norm gain folded in (rf_fold_norm);
 *   knorm [d] bf16 or NULL, knorm_kind 0 = Llama rms_norm, 1 = Qwen3.5 rms_norm_zc (ignored if NULL);
 *   cs [P, rot] the RoPE table of the rows' positions (rf_rope_table), rot the rotated dims (partial
 *       RoPE when rot < d, half-split rotation as ops.py:66-77);
 *   kbuf / vbuf: cache [hkv, cap, d] with element strides head_stride / row_stride; row j goes to
 *       slot slot_begin + j.
 * Needs H % 64 == 0, 2 hkv d % 256 == 0, 256 % d == 0, d % 8 == 0, rot even, rot <= d, rot / 2 a
 * multiple of 8 or equal to 4, slot_begin + P <= cap. workspace / ws_bytes (optional, NULL / 0): see
 * rf_gemm_workspace_bytes (M = P, N = 2 hkv d, K = H). */
int rf_norm_kv_write(const uint16_t* x, int64_t ldx, const float* ssq, int64_t P, int64_t H, float eps,
                     const uint16_t* wkv, int hkv, int d, const uint16_t* knorm, int knorm_kind,
                     const uint16_t* cs, int rot,
                     uint16_t* kbuf, uint16_t* vbuf, int64_t head_stride, int64_t row_stride,
                     int64_t slot_begin, int64_t cap, void* workspace, size_t ws_bytes,
                     hipStream_t stream);

/* ---- several late layers per launch (finish()'s fill loop, code/kva/kva.py:413-452, over a group of
 * consecutive late layers: the maps of every layer read the same rows h_split[:P]) ---- */

/* rf_map_apply for nl (1 .. 32) layers in one launch: x[l] = b w[l]^T + c[l] and ssq[l], each layer
 * bit-identical to rf_map_apply of it alone without a workspace. w, c, x, ssq: host arrays of nl device
 * pointers (c may be NULL, or hold NULL entries: no bias); one output row stride ldx for every layer.
 * Needs h_in >= 128 besides rf_map_apply's conditions. Replaces kva.py:413-415 for each layer. */
int rf_map_apply_batch(int nl, const uint16_t* b, int64_t ldb, const uint16_t* const* w, const uint16_t* const* c,
                       uint16_t* const* x, int64_t ldx, float* const* ssq, int64_t P, int64_t h_in, int64_t h_out,
                       hipStream_t stream);

/* rf_norm_kv_write for nl (1 .. 32) attention layers in one launch over the same P rows: layer l's inputs
 * x[l] (one row stride ldx) with statistics ssq[l], its weights wkv[l], k_norm gains knorm[l] (knorm NULL:
 * none for any layer) and caches kbuf[l] / vbuf[l] (one shape and stride for every layer); eps, heads, the
 * RoPE table cs and the slots [slot_begin, slot_begin + P) shared. Each layer's K / V are bit-identical to
 * rf_norm_kv_write of it alone without a workspace. H a multiple of 1024 up to 4096 with a power-of-two
 * rot <= 128 runs every layer's tiles on one persistent grid; other shapes launch per layer.
 * Replaces Model.fill (code/kva/model.py:278-280) of each layer. */
int rf_norm_kv_write_batch(int nl, const uint16_t* const* x, int64_t ldx, const float* const* ssq, int64_t P,
                           int64_t H, float eps, const uint16_t* const* wkv, int hkv, int d,
                           const uint16_t* const* knorm, int knorm_kind, const uint16_t* cs, int rot,
                           uint16_t* const* kbuf, uint16_t* const* vbuf, int64_t head_stride, int64_t row_stride,
                           int64_t slot_begin, int64_t cap, hipStream_t stream);

/* rf_norm_linear for nl (1 .. 32) entries in one launch (the in-projections of a group of Gated DeltaNet
 * layers, code/kva/model.py:448-450 per layer): entry l is rows[l] rows of x[l] (statistics ssq[l]) against the
 * n[l] weight rows of w[l] (a multiple of 256) into out[l], out[l] = bf16(rms-normed x[l] w[l]^T), each
 * bit-identical to rf_norm_linear of it alone without a workspace. A GDN fill passes two entries per layer:
 * every row against the k | v | b | a rows, and the last 3 rows (the conv state's) against the q rows. x, ssq,
 * w, out: host arrays of nl device pointers; rows, n: host arrays of nl counts; one input row stride ldx and
 * one output row stride ldo (>= every n[l]). H a multiple of 1024 up to 4096 runs every entry's tiles on one
 * persistent grid; other widths launch per entry. Entries of 0 rows are skipped. */
int rf_norm_linear_batch(int nl, const uint16_t* const* x, int64_t ldx, const float* const* ssq, const int64_t* rows,
                         int64_t H, float eps, const uint16_t* const* w, const int64_t* n, uint16_t* const* out,
                         int64_t ldo, hipStream_t stream);

/* RoPE on given pre-RoPE K and the K / V cache write of m rows.
 * Replaces Model.fill_kv (code/kva/model.py:161-165): ops.apply_rope (ops.py:66-77) + _append_kv.
 * k / v: [m, hkv, d] with token strides ld_k / ld_v (a head's d values contiguous, heads d apart);
 * cs, rot and the cache arguments as rf_norm_kv_write. */
int rf_rope_kv_write(const uint16_t* k, int64_t ld_k, const uint16_t* v, int64_t ld_v, int64_t m, int hkv,
                     int d, const uint16_t* cs, int rot,
                     uint16_t* kbuf, uint16_t* vbuf, int64_t head_stride, int64_t row_stride,
                     int64_t slot_begin, int64_t cap, hipStream_t stream);

/* ---- the exact rows' full layer (Model.layer_rows, code/kva/model.py:259-276) ---- */

/* K / V of scattered rows into their own cache slots: for j < rows, input row j (x [rows, H], statistics
 * ssq) at position pos[j] (int64, device) is normed, projected by wkv, k_normed and rotated with table row
 * pos[j] of cs exactly as rf_norm_kv_write does it, and written to cache slot pos[j]. The exact rows of a
 * filled layer (code/kva/kva.py:392-454 scatters the rows' inputs into the layer's fill): once the layer
 * is filled from every prefix row, this overwrites the rows' slots with the K / V of their exact inputs.
 * Arguments and limits as rf_norm_kv_write. pos_limit (> 0): the smaller of the cache's capacity and the
 * table's rows; a row whose pos[j] lies outside [0, pos_limit) is skipped on the device (no table read, no
 * cache write), since the positions live on the device and are not read back. The rows run through the
 * few-rows partials (M <= 512 per launch) and the reduce epilogue: a workspace of
 * rf_rows_workspace_bytes(rows, 2 hkv d, H) bytes is required. */
int rf_norm_kv_rows(const uint16_t* x, int64_t ldx, const float* ssq, int64_t rows, int64_t H, float eps,
                    const uint16_t* wkv, int hkv, int d, const uint16_t* knorm, int knorm_kind, const uint16_t* cs,
                    int rot, const int64_t* pos, int64_t pos_limit, uint16_t* kbuf, uint16_t* vbuf,
                    int64_t head_stride, int64_t row_stride, void* workspace, size_t ws_bytes, hipStream_t stream);

/* The queries and the K / V of scattered rows in one product: wqkv [hq d + 2 hkv d, H] holds the query
 * projection's rows then the K and V projections' (each with the input norm gain folded in). Row j of
 * x [rows, H] (statistics ssq) at position pos[j]: its queries, with qnorm (or none) and RoPE table row
 * pos[j], to q row j (row stride ldq), as rf_norm_q writes them; its K / V, with knorm, to cache slot pos[j],
 * as rf_norm_kv_rows writes them (norm_kind is the kind of both norms). One few-rows product per 512 rows,
 * then the two epilogues over its column ranges. Limits and pos_limit as rf_norm_kv_rows (a row skipped for
 * its position leaves its q row unwritten too); a workspace of rf_rows_workspace_bytes(rows, hq d + 2 hkv d,
 * H) bytes is required. The exact rows' layer input side (code/kva/model.py:234-245, :340-352 on the rows of
 * a filled layer). */
int rf_norm_qkv_rows(const uint16_t* x, int64_t ldx, const float* ssq, int64_t rows, int64_t H, float eps,
                     const uint16_t* wqkv, int hq, int hkv, int d, const uint16_t* qnorm, const uint16_t* knorm,
                     int norm_kind, const uint16_t* cs, int rot, const int64_t* pos, int64_t pos_limit, uint16_t* q,
                     int64_t ldq, uint16_t* kbuf, uint16_t* vbuf, int64_t head_stride, int64_t row_stride,
                     void* workspace, size_t ws_bytes, hipStream_t stream);

/* out[j] = x[rows[j]] for j < nrows, bit-exact, and out's row sum-of-squares partials ssq [nrows, H / 256]
 * (the rows' input RMSNorm statistics). The gather of h[rows] in layer_rows (code/kva/model.py:270); a row
 * outside [0, P) gives a zero row. rows: int64 on the device. */
int rf_row_gather(const uint16_t* x, int64_t ldx, int64_t P, int64_t H, const int64_t* rows, int64_t nrows,
                  uint16_t* out, int64_t ldo, float* ssq, hipStream_t stream);

/* Query projection of rows x [rows, H] at positions pos [rows] (int64, device): input RMSNorm (gain folded
 * into wq, rf_fold_norm; row statistics ssq), q = xn wq^T [hq d], optional per-head q_norm (qnorm [d],
 * kind 0 rms_norm, 1 rms_norm_zc), RoPE with table row pos[j] of cs (rf_rope_table of positions 0..).
 * Writes q [rows, hq d] (row stride ldq). Replaces Llama.queries / Qwen3 q_norm (code/kva/model.py:241-245,
 * :347-352) on the normed rows. Needs H % 256 == 0, hq d % 256 == 0, and the rotary limits of
 * rf_norm_kv_write. workspace / ws_bytes (optional): see rf_gemm_workspace_bytes (M = rows, N = hq d). */
int rf_norm_q(const uint16_t* x, int64_t ldx, const float* ssq, int64_t rows, int64_t H, float eps,
              const uint16_t* wq, int hq, int d, const uint16_t* qnorm, int qnorm_kind, const uint16_t* cs, int rot,
              const int64_t* pos, uint16_t* q, int64_t ldq, void* workspace, size_t ws_bytes,
              hipStream_t stream);

/* Causal attention of nq query rows q [nq, hq d] at sorted positions qpos [nq] (int64, device; each
 * < cache_rows) over the cache kbuf / vbuf [hkv, cap, d] (element strides head_stride / row_stride): query
 * j sees keys 0 .. qpos[j]; scores in fp32 scaled by `scale`, softmax in fp32, probabilities as bf16 into
 * the second product. Writes out [nq, hq d] (row stride ldo). Replaces ops.attend_at / attend_rows
 * (code/kva/ops.py:131-170) in layer_rows. Needs d 64, 128 or 256 and hq / hkv dividing 64. With a workspace
 * (caller-owned device memory, 16-byte aligned) the key range is split over more blocks and the splits are
 * merged in a fixed order (rf_attend_rows_workspace_bytes gives the size for the full split; a smaller one
 * gives fewer splits, NULL none). */
int rf_attend_rows(const uint16_t* q, int64_t ldq, const int64_t* qpos, int64_t nq, int hq, int d,
                   const uint16_t* kbuf, const uint16_t* vbuf, int hkv, int64_t head_stride, int64_t row_stride,
                   int64_t cache_rows, float scale, uint16_t* out, int64_t ldo, void* workspace, size_t ws_bytes,
                   hipStream_t stream);

/* Workspace bytes rf_attend_rows uses to split the key range fully for these sizes (0: no split). Host only. */
int rf_attend_rows_workspace_bytes(int64_t nq, int hq, int hkv, int d, int64_t cache_rows, size_t* bytes);

/* Causal attention of nq queries q [nq, hq d] over the first n_keys rows of kbuf / vbuf [hkv, cap, d]:
 * query j sees keys 0 .. qpos[j] (qpos: sorted int64 positions on the device; one past n_keys - 1 sees
 * every key), or, with qpos NULL,
 * consecutive queries at slots slot0 .. slot0 + nq - 1 (slot0 + nq <= n_keys). Scores in fp32 scaled by
 * `scale`, softmax in fp32, probabilities as bf16 into the second product; writes out [nq, hq d] (row
 * stride ldo, 8-byte aligned). With slot0 = n_keys - nq this is the exact tail's attention in
 * Model.layer, ops.attend (code/kva/ops.py:107-128, code/kva/model.py:247-257); with qpos the exact
 * rows' attention in layer_rows, ops.attend_at / attend_rows (code/kva/ops.py:131-170), Qwen3.5's gated
 * attention included (code/kva/model.py:436-446; the gate multiplies the output afterwards). Needs d 64 or
 * 128 with hq / hkv in {1, 2, 4, 8}, or d 256 with hq / hkv in {1, 2, 4, 8, 16}. The workspace
 * (caller-owned device memory, 16-byte aligned; may be NULL) receives, when the query blocks are too few for the GPU, the partial results of a key-range split,
 * merged in a fixed order: rf_attend_causal_workspace_bytes gives the size for the full split (a smaller
 * one gives fewer splits, NULL none). */
int rf_attend_causal(const uint16_t* q, int64_t ldq, int64_t nq, const int64_t* qpos, int64_t slot0, int hq, int d,
                     const uint16_t* kbuf, const uint16_t* vbuf, int hkv, int64_t head_stride, int64_t row_stride,
                     int64_t n_keys, float scale, uint16_t* out, int64_t ldo, void* workspace, size_t ws_bytes,
                     hipStream_t stream);

/* Workspace bytes rf_attend_causal uses for nq queries over n_keys keys (the full key-range split; 0 when the
 * query blocks alone fill the GPU). Host only. */
int rf_attend_causal_workspace_bytes(int64_t nq, int hq, int hkv, int d, int64_t n_keys, size_t* bytes);

/* out = bf16(x + y) row by row (rows x H) and out's row sum-of-squares partials ssq [rows, H / 256]: the
 * residual adds of layer_rows (code/kva/model.py:274, Model.mlp :114). out may alias x. */
int rf_residual_add(const uint16_t* x, int64_t ldx, const uint16_t* y, int64_t ldy, uint16_t* out, int64_t ldo,
                    float* ssq, int64_t rows, int64_t H, hipStream_t stream);

/* out = bf16(res + bf16(x w^T)) for x [M, K] (row stride ldx), w [N, K], res [M, N] (row stride ldr), and
 * out's row sum-of-squares partials ssq [M, N / 256]: rf_map_apply without a bias followed by
 * rf_residual_add(res, out), bit-identical to that pair, in one pass: the residual is added in the
 * product's tile epilogue (K >= 128), or in the split sums' epilogue for rows that run through the
 * split-K sums (a few rows with the workspace of rf_gemm_workspace_bytes(M, N, K)). K = 64 runs the pair.
 * o_proj and down with their residuals (code/kva/model.py:112-118). */
int rf_map_apply_residual(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* res, int64_t ldr,
                          uint16_t* out, int64_t ldo, float* ssq, int64_t M, int64_t K, int64_t N, void* workspace,
                          size_t ws_bytes, hipStream_t stream);

/* SwiGLU of a normed [gate; up] product: act [P, I] = rf_silu_mul of rf_norm_linear(x, ssq, eps, w) with
 * w [2 I, H] (gate rows then up rows, the norm gain folded in), bit-identical to that pair. With a few rows
 * and the workspace of rf_gemm_workspace_bytes(P, 2 I, H) SwiGLU runs in the split sums' epilogue and gu
 * is not touched (may be NULL); otherwise gu [P, 2 I] (row stride ldg) receives the product first. Needs
 * H and I multiples of 256. The MLP's first half (code/kva/model.py:112-118). */
int rf_norm_linear_swiglu(const uint16_t* x, int64_t ldx, const float* ssq, int64_t P, int64_t H, float eps,
                          const uint16_t* w, int64_t I, uint16_t* act, int64_t lda, uint16_t* gu, int64_t ldg,
                          void* workspace, size_t ws_bytes, hipStream_t stream);

/* SwiGLU: act[j, c] = bf16(bf16(silu(gu[j, c])) * gu[j, I + c]) for c < I (gate columns then up columns of
 * one in-projection). Model.mlp's F.silu(gate) * up (code/kva/model.py:112-119). */
int rf_silu_mul(const uint16_t* gu, int64_t ldg, int64_t rows, int64_t I, uint16_t* act, int64_t lda,
                hipStream_t stream);

/* Fused RMSNorm + linear: out[P, N] = bf16(r_row * (x w^T)) with r_row = 1 / sqrt(mean(x^2) + eps) from
 * the row partials ssq [P, H / 256] and the norm gain folded into w [N, H] (rf_fold_norm). The Gated
 * DeltaNet in-projections of a fill (code/kva/model.py:448-450 after in_norm, :513). Needs
 * H % 256 == 0, N % 256 == 0 (pad w with zero rows), 16-byte aligned pointers. workspace / ws_bytes
 * (optional): see rf_gemm_workspace_bytes (M = P, K = H). */
int rf_norm_linear(const uint16_t* x, int64_t ldx, const float* ssq, int64_t P, int64_t H, float eps,
                   const uint16_t* w, int64_t N, uint16_t* out, int64_t ldo, void* workspace, size_t ws_bytes,
                   hipStream_t stream);

/* Gated DeltaNet fill of one layer from its in-projection rows pre [P, ld] bf16 (columns: q [nk dk] |
 * k [nk dk] | v [nv dv] | b [nv] | a [nv]): causal conv + SiLU (conv_w [C, 4], C = 2 nk dk + nv dv,
 * continuing conv_in [3, C] or zeros), k l2-norm, beta = sigmoid(b), g = -exp(a_log) softplus(a +
 * dt_bias) (a_log, dt_bias [nv] fp32), and the chunked (64-row) gated delta rule updating state
 * [nv, dk, dv] fp32 in place. Writes conv_out [3, C] (the last 3 pre-conv rows; must not alias conv_in).
 * Replaces Qwen35._gdn_core with need_out = False (code/kva/model.py:452-484, ops.py:173-262) inside
 * Qwen35.fill (model.py:510-523). Needs dk = dv = 128, nv % nk == 0, ld % 8 == 0 and 16-byte aligned
 * pre, conv_w, conv_in and workspace. The workspace (caller-owned device memory) holds the per-chunk
 * products between the two kernels; a workspace of rf_gdn_workspace_bytes(P, ...) does the fill in one
 * pass, a smaller one (at least one chunk's worth) in several passes with the same result. A workspace of
 * two or more chunks is used as two halves: the prep of the next pass runs on a second stream the library
 * keeps per device (default priority) beside the scan of the current pass on `stream`, ordered by events;
 * `stream` waits for all of it, so work queued after the call on `stream` sees the finished fill. Results
 * are bit-identical to the one-stream schedule. That stream and its events are created on the first such
 * call on a device (under a mutex) and kept until the process ends: the library's one piece of global
 * state besides the thread-local error text and rf_gdn_fill_noalloc's array. No device memory is
 * allocated for it. */
int rf_gdn_fill(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv, const uint16_t* conv_w,
                const uint16_t* conv_in, uint16_t* conv_out, const float* a_log, const float* dt_bias, float* state,
                void* workspace, size_t ws_bytes, hipStream_t stream);

/* One layer's operands of rf_gdn_fill_batch: as the arguments of rf_gdn_fill of the same names. */
typedef struct rf_gdn_layer {
  const uint16_t* pre;
  int64_t ld;
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out;
  const float* a_log;
  const float* dt_bias;
  float* state;
} rf_gdn_layer;

#define RF_GDN_BATCH_MAX 2

/* rf_gdn_fill of n_layers (1 .. RF_GDN_BATCH_MAX) independent layers over the same P rows and head shapes, in
 * one prep and one scan launch per pass for all of them: the late GDN layers of a fill each start from
 * their own cache (code/kva/model.py:510-523 per layer inside code/kva/kva.py:396-449), so their sequential
 * chunk scans run side by side on the GPU. Each layer's result is bit-identical to its rf_gdn_fill. The
 * workspace is split evenly between the layers (rf_gdn_workspace_bytes(rows, ...) each for one pass of
 * `rows` rows); states and conv_out buffers must be distinct. */
int rf_gdn_fill_batch(const rf_gdn_layer* layers, int n_layers, int64_t P, int nk, int nv, int dk, int dv,
                      void* workspace, size_t ws_bytes, hipStream_t stream);

/* Workspace bytes rf_gdn_fill needs to fill `rows` rows in one pass (rows = 0: the one-chunk minimum).
 * Host-only; no device work. */
int rf_gdn_workspace_bytes(int64_t rows, int nk, int nv, int dk, int dv, size_t* bytes);

/* Size in MiB of the device array rf_gdn_fill_noalloc uses as its workspace (one per GPU, for the life of
 * the process). */
#define RF_GDN_SCRATCH_MAX 56

/* rf_gdn_fill without a workspace argument and without any allocation: the per-chunk products go to a
 * file-scope device array of RF_GDN_SCRATCH_MAX MiB inside the library (its address on each GPU is taken
 * once, on the first call with that GPU current), which holds as many 64-row chunks as fit per pass
 * (39 at 16 key / 32 value heads), so any P runs, in as many passes as it needs; results are
 * bit-identical to rf_gdn_fill's. Heads whose one chunk exceeds the array are refused (RF_EINVAL_SHAPE).
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). Every call on one GPU shares its
 * array, so calls that overlap on one GPU (different streams or threads) race: order them. The stream must
 * belong to the current device. */
int rf_gdn_fill_noalloc(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv,
                        const uint16_t* conv_w, const uint16_t* conv_in, uint16_t* conv_out, const float* a_log,
                        const float* dt_bias, float* state, hipStream_t stream);

/* The exact GDN layer's mixing (Qwen35._gdn_core with need_out = True, code/kva/model.py:452-484 and
 * ops.py:199-262): as rf_gdn_fill (state and conv state continued over the P rows), and also the
 * delta-rule outputs out [P, nv dv] bf16 (row stride ldo): per chunk o = Qd S + P v_new, Qd = q_n e^gamma,
 * P = tril(q_n k_n^T e^{gamma_i - gamma_j}), q_n = l2norm(conv q) dk^-1/2, with S the state before the chunk
 * (stored by the scan) -- fp32 throughout, rounded once to bf16. Workspace: rf_gdn_forward_workspace_bytes
 * (a smaller one of at least one chunk's worth gives several passes with the same result). */
int rf_gdn_forward(const uint16_t* pre, int64_t ld, int64_t P, int nk, int nv, int dk, int dv,
                   const uint16_t* conv_w, const uint16_t* conv_in, uint16_t* conv_out, const float* a_log,
                   const float* dt_bias, float* state, uint16_t* out, int64_t ldo, void* workspace, size_t ws_bytes,
                   hipStream_t stream);

/* Workspace bytes rf_gdn_forward needs for `rows` rows in one pass (rows = 0: one chunk). Host-only. */
int rf_gdn_forward_workspace_bytes(int64_t rows, int nk, int nv, int dk, int dv, size_t* bytes);

/* Qwen3.5's attention output gate (code/kva/model.py:444-445, o * torch.sigmoid(gate) in bf16):
 * out = bf16(o * bf16(sigmoid(g))) over rows x n values (n % 8 == 0; strides % 8 == 0; out may alias o). */
int rf_sigmoid_mul(const uint16_t* o, int64_t ldo, const uint16_t* g, int64_t ldg, int64_t rows, int64_t n,
                   uint16_t* out, int64_t ld_out, hipStream_t stream);

/* The GDN output norm (ops.rms_norm_gated, code/kva/ops.py:28-33; code/kva/model.py:494-499) over rows x
 * heads vectors of dv values: y = bf16(bf16(weight * bf16(x / sqrt(mean(x^2) + eps))) * silu(z)), silu in
 * fp32. weight [dv] bf16; dv 64, 128 or 256; strides % 8 == 0. */
int rf_gated_rms_norm(const uint16_t* x, int64_t ldx, const uint16_t* z, int64_t ldz, const uint16_t* weight,
                      int64_t rows, int heads, int dv, float eps, uint16_t* y, int64_t ldy, hipStream_t stream);

/* ---- closed-form fit (code/kva/ridge.py:19-105, code/scripts/fit_sweep.py:87-144) ---- */

/* Transpose row-major samples src [rows, cols] into dst [cols, >= round_up(rows, 64)] (row stride
 * ld_dst), zero-filling the columns past `rows`: the K-contiguous operand of rf_gram_accumulate. If
 * partial is not NULL it receives the column sums of every 64-row tile, fp32 [round_up(rows, 64)/64, cols]
 * (fold them with rf_colsum_fold). Needs cols % 64 == 0, 16-byte aligned pointers, strides % 8 == 0. */
int rf_transpose(const uint16_t* src, int64_t ld_src, int64_t rows, int64_t cols, uint16_t* dst, int64_t ld_dst,
                 float* partial, hipStream_t stream);

/* rf_transpose with centring, for channels whose mean dwarfs their spread: column c's values become
 * d = x - shift[c] (fp32), written to dst as hi = bf16(d) (round to nearest even) and, when lo_row[c] >= 0,
 * mid = bf16(d - hi) to row lo_row[c] of dst_lo and lo = bf16(d - hi - mid) to row n_centred + lo_row[c]
 * (row stride ld_dst). hi + mid + lo == d exactly, so one rf_gram_accumulate over [dst rows; dst_lo rows]
 * yields the products of the centred values -- the reference subtracts its shifts before its per-block
 * fp32 GEMM (code/kva/ridge.py:44-47, :58-61; code/scripts/fit_sweep.py:100-105) -- on bf16 MFMA. Columns
 * with shift 0 and lo_row -1 are copied as rf_transpose copies them. partial / partial_sq (each optional):
 * fp32 column sums / sums of squares of d per 64-row tile, [round_up(rows, 64) / 64, cols] (fold with
 * rf_colsum_fold). shift, lo_row (int32 [cols], distinct rows < n_centred for the centred columns) and
 * dst_lo ([2 n_centred, ld_dst] at least) are all given or all NULL (then this is rf_transpose plus the
 * squares). A shifted column needs a lo row (without one its values are rounded to bf16). Limits as
 * rf_transpose; dst_lo 16-byte aligned. */
int rf_transpose_centred(const uint16_t* src, int64_t ld_src, int64_t rows, int64_t cols, const float* shift,
                         const int32_t* lo_row, int64_t n_centred, uint16_t* dst, int64_t ld_dst, uint16_t* dst_lo,
                         float* partial, float* partial_sq, hipStream_t stream);

/* sums[c] += sum_j partial[j, c] in fp64 and a fixed order (16 interleaved runs over j, then a pairwise
 * fold; the same bits every run): the sum(0) of a sample block (RidgeStats' sx / sy, code/kva/ridge.py:46, :61). */
int rf_colsum_fold(const float* partial, int64_t ntiles, int64_t cols, double* sums, hipStream_t stream);

/* A measurement, with no counterpart in the reference: `blocks` workgroups of 256 threads each run 4 x iters
 * back-to-back v_mfma_f32_32x32x16_bf16 per wave on register operands (pseudo-random bf16), then store one
 * float per thread to out [blocks * 256]. 32768 flop per MFMA: timed, it gives the MFMA throughput the
 * GPU's power limit allows with no memory traffic, the ceiling the fill's GEMMs are compared with beside
 * the nominal peak. */
int rf_mfma_ceiling(int blocks, int iters, float* out, hipStream_t stream);

/* Gram / cross accumulation C[M, N] += A[M, K] B[N, K]^T: bf16 products summed in fp32 on MFMA over runs
 * of at most fold_rows of K (0: the whole K; else a multiple of 64), each run's sums added into the fp64
 * accumulator C (row stride ldc) as it ends. With A = X^T and B = X^T or Y^T of sample rows and fold_rows
 * the block, this is RidgeStats' per-block fp32 GEMM into fp64 (code/kva/ridge.py:47, :62) over many
 * blocks in one launch (runs start at K offsets 0, fold_rows, 2 fold_rows, ...). Needs N % 256 == 0,
 * K % 64 == 0 (pad samples with zero rows), lda / ldb % 8 == 0, ldc even.
 * The 256 x 256 output tiles run one per workgroup. When they are slightly more than one round of the
 * GPU's 256 CUs (centred channels add a tile row or column to a 4096-wide product), a workspace of
 * rf_gram_workspace_bytes lets the launch cut the tiles past the first 256 into their runs, which take
 * one short extra round instead of a second round of whole tiles; their fp32 run sums go to the
 * workspace and a second kernel adds them into C in run order. The result is bit-identical either way;
 * workspace NULL or smaller than needed: every tile whole. */
int rf_gram_accumulate(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t M, int64_t N,
                       int64_t K, int64_t fold_rows, double* c, int64_t ldc, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes of rf_gram_accumulate's run-split schedule for this shape (0: it uses none). */
int rf_gram_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t fold_rows, size_t* bytes);

/* The symmetric X^T X of RidgeStats.begin (code/kva/ridge.py:47, `sxx += xw.T @ xc`): rf_gram_accumulate with
 * both operands taken from one K-contiguous buffer a [N rows, K] (A = its first M rows, B = all N, M <= N),
 * on C's block-upper 256 x 256 tiles only (tile column >= tile row): C[i, j] += sum_k a[i, k] a[j, k]. The
 * block-lower tiles are not written; C's leading M x M part is symmetric, so the caller copies them from
 * the block-upper ones (C[i, j] = C[j, i]) before reading. Each tile written is bit-identical to
 * rf_gram_accumulate(a, lda, a, lda, M, N, ...)'s. With a workspace of rf_gram_upper_workspace_bytes (at
 * most one round of tiles), every tile is split into its fold runs, one workgroup per (tile, run), and
 * the run sums are added into C in run order by a second kernel, so about half the product's work
 * spreads over every CU; workspace NULL or smaller: every tile whole, same bits. Limits as
 * rf_gram_accumulate. */
int rf_gram_accumulate_upper(const uint16_t* a, int64_t lda, int64_t M, int64_t N, int64_t K, int64_t fold_rows,
                             double* c, int64_t ldc, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes of rf_gram_accumulate_upper's run-split schedule for this shape (0: it uses none). */
int rf_gram_upper_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t fold_rows, size_t* bytes);

/* Held-out read cosine of one late layer for one document (code/scripts/fit_sweep.py:307-313): pred and
 * truth are [rows, >= (na + nb) d] bf16 reads, each row na vectors of group a then nb vectors of group b,
 * each d wide. An attention layer's reads are its pre-RoPE K and V (code/kva/model.py:282-287, one
 * norm_linear of [W_k; W_v]): na = nb = hkv. A GDN layer's reads are its in-projection outputs
 * (code/kva/model.py:566-571, one norm_linear of [W_qkv; W_b; W_a]): q | k (na = nb = nk, d = dk), v
 * (na = nv, nb = 0, d = dv) and [b | a] (na = 1, nb = 0, d = 2 nv), one call each on their column range. Per
 * row and vector, cos = a . b / (max(|a|, 1e-8) max(|b|, 1e-8)) in fp32 (F.cosine_similarity over the
 * vector); group a's vectors are first scaled elementwise by the k_norm gain kgain [d] bf16 (gain_kind 1:
 * 1 + gain; NULL: no k norm), which is the cosine of the k-normed reads (code/kva/model.py:353-359) since
 * the per-head RMS factor cancels. out[0] += weight * (sum of group a's cosines) and, when nb > 0,
 * out[1] += weight * (sum of group b's), in fp64 and a fixed order (weight = 1 / (rows na) gives a group's
 * document mean). workspace: at least 8 * ceil(rows / 16) bytes. d a power of two from 8 to 256;
 * ld_pred / ld_true multiples of 8, pointers 16-byte aligned. */
int rf_read_cosine(const uint16_t* pred, int64_t ld_pred, const uint16_t* truth, int64_t ld_true, int64_t rows,
                   int na, int nb, int d, const uint16_t* kgain, int gain_kind, double weight, double* out,
                   void* workspace, size_t ws_bytes, hipStream_t stream);

/* The ridge solve of RidgeFit (code/kva/ridge.py:80-105) in fp64: for each of the nlam values lam (host array
 * lams, each > 0), W_lam = (C + lam scale I)^-1 Cxy with C = cxx [d, d] (row stride ldc; symmetric positive
 * semi-definite, the centred scatter) and Cxy = cxy [d, R] (row stride ldb; the cross statistics of every
 * target side by side), written to w + l w_stride as [d, R] (row stride ldw); and, if bias is not NULL,
 * bias + l bias_stride = mean_y - mean_x W_lam ([R]; mean_x [d], mean_y [R] on the device): the unpenalised
 * bias of the centred fit. The inverse of C + lam scale I comes from a block recursion on its Schur
 * complements over a 64 x 64 Gauss-Jordan base (the matrix padded with an identity block to a multiple of 64)
 * and every product runs on fp64 MFMA; the reference's eigendecomposition gives the same closed form.
 * Needs d, R, ldb, ldw even; cxy, w, mean_x and the workspace 16-byte aligned; a workspace of
 * rf_ridge_solve_workspace_bytes(d, nlam) bytes. */
int rf_ridge_solve(const double* cxx, int64_t ldc, int64_t d, const double* cxy, int64_t ldb, int64_t R,
                   const double* mean_x, const double* mean_y, const double* lams, int nlam, double scale, double* w,
                   int64_t ldw, int64_t w_stride, double* bias, int64_t bias_stride, void* workspace, size_t ws_bytes,
                   hipStream_t stream);

/* Bytes of rf_ridge_solve's workspace for dimension d and nlam lambdas (up to 8 are inverted together).
 * Host only. */
int rf_ridge_solve_workspace_bytes(int64_t d, int nlam, size_t* bytes);

/* ---- exact-row selection (the qattn selector) ---- */

/* Bytes of rf_window_mass's workspace: w window rows, hq query / hkv K-V heads of head_dim d, keys
 * 0 .. n_end - 1 (n_end = the window's end). */
int rf_window_mass_workspace_bytes(int w, int hq, int hkv, int d, int64_t n_end, size_t* bytes);

/* Window attention mass of one exact lower attention layer (code/kva/select.py:223-245 window_mass):
 * mass[j] += sum over the w window query rows (positions pos0 .. pos0 + w - 1) and all hq query heads of
 * softmax_j(scale q . k_j), keys j <= the query's position (dense causal softmax over every key), for
 * j < pos0 + w; later keys get nothing. q [w, >= hq d] post-RoPE queries of the window rows (rf_norm_q),
 * kbuf the layer's post-RoPE K cache [hkv, cap, d] (head_stride, row_stride); mass fp64 [>= pos0 + w], the
 * caller's accumulator over layers (zero it per prompt). Each K / V head group's sum is fp32 (rows, then
 * heads, in a fixed order), added into mass as fp64 in group order. d 64, 128 or 256; (hq / hkv) * w a
 * multiple of 32, at most 1024. */
int rf_window_mass(const uint16_t* q, int64_t ldq, int w, int64_t pos0, int hq, int d, const uint16_t* kbuf,
                   int hkv, int64_t head_stride, int64_t row_stride, float scale, double* mass, void* workspace,
                   size_t ws_bytes, hipStream_t stream);

/* ---- map formats ---- */

/* int8 map rows with per-row group scales -> bf16 maps: out[i][j] = bf16(codes[i][j] * scale[i][j / group]),
 * the product exact in fp32 and one round-to-nearest-even cast. The i8_row128 release layout (group 128:
 * codes int8 [d_out, d_in], scale bf16 [d_out, d_in / 128]) expands to the Projector's bf16 maps exactly
 * as the reference's conversion does (code/c5/convert.py:91-97 dequant, :100-109 maps; the bias column
 * stays bf16). Needs group % 16 == 0, width % group == 0, ld_codes >= width and a multiple of 16,
 * ld_out >= width and a multiple of 8, ld_scale >= width / group, 16-byte aligned codes and out. */
int rf_dequant_i8_rows(const int8_t* codes, int64_t ld_codes, const uint16_t* scale, int64_t ld_scale,
                       int64_t rows, int64_t width, int group, uint16_t* out, int64_t ld_out, hipStream_t stream);

/* llama.cpp GGUF map tensors as bf16 maps (the adapter's blk.L.ridgefill.weight / .bias tensors the
 * reference writes and checks, code/qwen38-27b-kit/identity_projector.py:26-43, :64-80): src holds `rows`
 * rows of `width` values of ggml type ggml_type, row stride ld_src BYTES -- F32 (0), F16 (1), Q8_0 (8:
 * blocks of 32 values, an fp16 scale d and 32 int8 codes q, value d * q) or BF16 (30). out[i, j] =
 * bf16(value) (round to nearest even; the values are exact in fp32). Q8_0: width % 32 == 0, src and
 * ld_src 2-byte aligned; the others: width % 8 == 0, src and ld_src 16-byte aligned. ld_out % 8 == 0.
 * Other ggml types: RF_EUNSUPPORTED. */
int rf_dequant_gguf_rows(int ggml_type, const void* src, int64_t ld_src, int64_t rows, int64_t width, uint16_t* out,
                         int64_t ld_out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RFILL_H */
