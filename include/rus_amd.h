/*
 * rus_amd.h — C ABI of the MI355X (gfx950) kernels for the fused QLoRA training hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, element counts/strides (in ELEMENTS, not bytes) and a HIP stream
 *     (hipStream_t passed as void*; NULL = the legacy default stream);
 *   - never allocates device memory and never synchronises; it only enqueues work on `stream`;
 *   - returns RUS_OK (0) on success, or a non-zero RUS_ERR_* code with a message available from
 *     rus_last_error() (thread-local, valid until the next failing call on that thread).
 *
 * Floating-point tensors are fp16 (RUS_DTYPE_F16) or fp32 (RUS_DTYPE_F32), row-major, with a
 * contiguous innermost dimension. Kernels compute in fp32 and round to the storage type with
 * round-to-nearest-even.
 *
 * Reference interfaces (fokyso82002-rgb/rus) that each entry point replaces are cited per function.
 */
#ifndef RUS_AMD_H
#define RUS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RUS_ABI_VERSION 17

#define RUS_DTYPE_F16 0
#define RUS_DTYPE_F32 1

#define RUS_OK 0
#define RUS_ERR_INVALID 1     /* bad pointer, size, stride, alignment or dtype */
#define RUS_ERR_UNSUPPORTED 2 /* valid but outside what the kernels implement (e.g. row too wide) */
#define RUS_ERR_LAUNCH 3      /* the HIP runtime rejected the launch */

/* Message of the last failing call on this thread ("" if none). */
const char* rus_last_error(void);

/* RUS_ABI_VERSION of the loaded library. */
int rus_abi_version(void);

/*
 * Copies n_bytes (a multiple of 16; 16-byte aligned pointers) from page-locked, device-mapped
 * host memory into device memory with a kernel on `stream` (no copy-engine transfer), so that a
 * captured step graph can start by reading its batch from a host staging image. Replaces: the
 * per-step transfer of the packed batch to the device (the reference packs device tensors,
 * solution/ops.py:1103-1127). RUS_ERR_INVALID when host_src is not pinned and mapped.
 */
int rus_copy_from_host(void* dst, const void* host_src, int64_t n_bytes, void* stream);

/*
 * Row gather from page-locked, device-mapped host memory: dst[i, :] = host_src[ids[i], :] for
 * i < n_ids, rows of row_bytes bytes (a multiple of 16; 16-byte aligned pointers), ids an int64
 * DEVICE array. A kernel on `stream` reads each selected row over the bus, so nothing waits on the
 * host. An id outside [0, n_src_rows) gives a zero row and sets *err_flag (device int32, optional).
 * Replaces: HostHead.embed's host index_select + pinned staging + H2D copy
 * (solution/hostload.py:381-386), which needs the ids on the host (a device synchronisation).
 */
int rus_gather_rows_from_host(const void* host_src, int64_t n_src_rows, int64_t row_bytes,
                              const int64_t* ids, int64_t n_ids, void* dst, int32_t* err_flag,
                              void* stream);

/*
 * Diagnostic (no counterpart in the reference): node census of a captured hipGraph_t.
 * counts[t] = number of nodes of hipGraphNodeType t (0 kernel, 1 memcpy, 2 memset, 3 host,
 * 4 child graph, 5 empty, 6 wait event, 7 event record, ...) for t < n_counts; later types are
 * added to counts[n_counts - 1]. Used to check that a captured training step holds no memset.
 */
int rus_graph_node_counts(void* graph, int64_t* counts, int32_t n_counts);

/*
 * NF4 double-quant dequantisation over 1..3 concatenated segments.
 * Replaces: solution/kernels.py:27-118 (nf4_dequant_turing_kernel) and its launcher
 *           solution/kernels.py:572-619 (dequant_nf4_tensor); called by
 *           solution/hostload.py:325-342 (WeightStream.dequant).
 *
 * For output element e (byte b = e/2; the HIGH nibble of packed[b] is element 2b, the LOW nibble
 * element 2b+1), in segment s = (b >= split_byte_1) + (b >= split_byte_2) starting at byte
 * start_s (0, split_byte_1, split_byte_2):
 *     blk    = b / (blocksize/2)                       (index into absmax, global)
 *     sup    = absmax2_base_s + (blk - start_s/(blocksize/2)) / super_blocksize
 *     scale  = fp32( fp32(code2[absmax[blk]] * absmax2[sup]) + off_s )      (no FMA)
 *     out[e] = fp16_rne( fp32(NF4[nibble] * scale) )
 * absmax2_base_0 is 0. The reference indexes absmax2 with the global block (kernels.py:53-57); that
 * equals this rule whenever every segment holds a multiple of super_blocksize blocks, which the
 * per-segment bases generalise. Segment starts must be multiples of blocksize/2 bytes; blocksize
 * and super_blocksize must be powers of two with blocksize >= 8; code2 holds 256 floats.
 * out_u32 receives n_bytes words (fp16 pairs, even element in the low half); it must be 16-byte
 * aligned and packed 4-byte aligned. n_bytes < 2^31. n_absmax / n_absmax2 are the lengths of
 * absmax / absmax2; the call is rejected unless every index the rule above produces is in range.
 */
int rus_nf4_dequant(const uint8_t* packed, const uint8_t* absmax, const float* code2,
                    const float* absmax2, float off0, float off1, float off2,
                    int64_t split_byte_1, int64_t split_byte_2, int64_t absmax2_base_1,
                    int64_t absmax2_base_2, int64_t n_bytes, int64_t n_absmax,
                    int64_t n_absmax2, int32_t blocksize, int32_t super_blocksize,
                    uint32_t* out_u32, void* stream);

/* One segment job of rus_nf4_dequant_multi: the per-segment arguments of rus_nf4_dequant. */
typedef struct rus_nf4_job {
  const uint8_t* packed;
  const uint8_t* absmax;
  const float* absmax2;
  float off0, off1, off2;
  int64_t split_byte_1, split_byte_2;
  int64_t absmax2_base_1, absmax2_base_2;
  int64_t n_bytes, n_absmax, n_absmax2;
  uint32_t* out_u32;
} rus_nf4_job;

/*
 * rus_nf4_dequant over 1..4 independent segment jobs (e.g. the four fused segments
 * [q|k|v], o, [gate|up], down of one layer) in a single launch, sharing one code2 table and one
 * (blocksize, super_blocksize). Each job is validated as rus_nf4_dequant validates its arguments.
 * Replaces: the per-segment WeightStream.dequant calls of solution/hostload.py:325-342 (one launch
 *           per segment there); no single reference counterpart.
 */
int rus_nf4_dequant_multi(const rus_nf4_job* jobs, int32_t n_jobs, const float* code2,
                          int32_t blocksize, int32_t super_blocksize, void* stream);

#define RUS_NORM_FWD 1
#define RUS_NORM_BWD 2

/*
 * One RMSNorm (fp16 activations, weight fp16 or fp32) for rus_nf4_dequant_multi_norm:
 *   RUS_NORM_FWD: as rus_rmsnorm_fwd with x, residual (or NULL), weight, sum_out, y = out, rstd;
 *   RUS_NORM_BWD: as rus_rmsnorm_bwd with dy = x, h, weight, rstd, dresidual = residual (or
 *                 NULL), dx = out.
 */
typedef struct rus_norm_side {
  int32_t kind;
  int32_t w_dtype;
  int64_t n_rows, n_cols, stride_row;
  float eps;
  const void* x;
  const void* residual;
  const void* h;
  const void* weight;
  float* rstd;
  void* sum_out;
  void* out;
} rus_norm_side;

/*
 * LoRA-down of rank r over token rows, by blocks of four tokens:
 *   mid_q = fp16(drop_q(x) A_q^T), mid_v = fp16(drop_v(x) A_v^T)
 * x [n_tokens, stride_x] fp16 (d a multiple of 64, stride_x a multiple of 8, 16-byte aligned),
 * A_q, A_v [r, d] fp16 (16-byte aligned), r in {4, 8, 16}, mid_q / mid_v [n_tokens, r] fp16.
 * Dropout: keep bits of both branches ([n_tokens, ceil(d / 32)] words, bit c % 32 of word c / 32
 * keeps element c) with scale 1 / (1 - p), or both NULL (no dropout). fp32 sums: each of the
 * block's four waves reduces a quarter of d on MFMA, the quarters added in order, one fp16
 * rounding; the same bits as the product carried by rus_nf4_dequant_multi_norm.
 * Replaces: mid_q = F.linear(lora_dropout(norm1), A_q) (and v) in solution/ops.py:775-778.
 */
typedef struct rus_lora_rows {
  const void* x;
  int64_t stride_x, n_tokens, d;
  int32_t r;
  const void* a_q;
  const void* a_v;
  const uint32_t* bits_q;
  const uint32_t* bits_v;
  float p_q, p_v;
  void* mid_q;
  void* mid_v;
} rus_lora_rows;

int rus_lora_down_rows(const rus_lora_rows* args, void* stream);

/*
 * rus_nf4_dequant_multi and one independent RMSNorm in a single launch (the norm's rows run in
 * blocks of their own beside the decode): a layer's weight dequant with that layer's input norm
 * (solution/ops.py:760-766 before 768-771) or with the norm backward of the layer above
 * (ops.py:994-996, then the next layer's dequant, ops.py:855-860). Same results as the two
 * separate calls. The norm must satisfy n_cols <= 2048, n_cols and stride_row multiples of 8,
 * 16-byte aligned rows; otherwise RUS_ERR_UNSUPPORTED (nothing launched).
 * down (forward norm only, or NULL): the LoRA-down of the norm's output, formed by the same
 * blocks right after their rows (down->x is the norm's out, with its rows, width and stride):
 * the bits of rus_lora_down_rows on that output.
 */
int rus_nf4_dequant_multi_norm(const rus_nf4_job* jobs, int32_t n_jobs, const float* code2,
                               int32_t blocksize, int32_t super_blocksize,
                               const rus_norm_side* side, const rus_lora_rows* down,
                               void* stream);

/*
 * Product with an NF4 double-quant weight W [w_rows, w_cols] (one job of up to three row
 * segments, blocksize 64) decoded inside the GEMM main loop; fp16 activations, fp32 sums rounded
 * once:
 *   trans = 0: y[m, n] = fp16(sum_k x[m, k] W[n, k] + bias[n])   x [m, w_cols], y [m, w_rows]
 *   trans = 1: y[m, k] = fp16(sum_n x[m, n] W[n, k])             x [m, w_rows], y [m, w_cols]
 * W[n, k] is exactly the fp16 value rus_nf4_dequant writes for the job (out_u32 is unused);
 * segment starts must be whole rows and w_rows, w_cols multiples of 64. Row strides: stride_x
 * (multiple of 8, x 16-byte aligned), stride_y (multiple of 4, y 8-byte aligned). bias: fp16
 * [w_rows] or NULL (trans = 0 only).
 * split: reduction splits (0: the library chooses). rus_nf4_gemm_plan returns the split it will
 * use and the fp32 workspace elements and int32 counters that split needs (0 when unsplit);
 * counters must be zero before the first call and are left zero; calls sharing counters must not
 * run concurrently.
 * Replaces: dequant_nf4_tensor (solution/kernels.py:572-619) into the shared workspace followed
 *           by F.linear / torch.mm on it: solution/ops.py:771, 810, 710/720, 714/724 (forward),
 *           873, 921, 932 (recompute), 934, 939, 949, 993 (backward).
 */
int rus_nf4_gemm_plan(int64_t m, int64_t w_rows, int64_t w_cols, int32_t trans, int32_t* split,
                      int64_t* workspace_floats, int64_t* n_counters);
int rus_nf4_gemm(const void* x, int64_t m, int64_t stride_x, const rus_nf4_job* w,
                 const float* code2, int64_t w_rows, int64_t w_cols, int32_t blocksize,
                 int32_t super_blocksize, int32_t trans, const void* bias, void* y,
                 int64_t stride_y, int32_t split, float* workspace, int64_t workspace_floats,
                 int32_t* counters, int64_t n_counters, void* stream);

/*
 * Split-K fp16 product into fp32 partials: parts[s] = A[:, Ks] . op(B)[Ks, :] for s = 0..n_split-1,
 * parts = [n_split][m][n] fp32 (contiguous), Ks the s-th of the n_split pieces of round_up(
 * ceil(k / n_split), 64) columns (n_split must equal the number of such pieces). A is [m, lda]
 * fp16 (K-contiguous); B is [n, ldb] (b_kn = 0: op(B) = B^T, K-contiguous) or [k, ldb] (b_kn = 1:
 * op(B) = B, N-contiguous, the weight as dequantised). k > 0 a multiple of 64, n a multiple of 8,
 * strides multiples of 8, operands 16-byte aligned, each operand under 4 GiB. The partials feed
 * rus_rmsnorm_bwd_parts, which sums them in part order.
 * Replaces: d_norm2 = torch.mm(d_gu_c, w_gu) (solution/ops.py:939), an fp16 product there.
 */
int rus_gemm_parts(const void* a, int64_t lda, const void* b, int64_t ldb, int32_t b_kn,
                   int64_t m, int64_t n, int64_t k, float* parts, int32_t n_split, void* stream);

/*
 * Fused residual add + RMSNorm forward, one row per wavefront.
 * Replaces: solution/kernels.py:125-163 (rms_norm_residual_fwd_kernel), launcher
 *           solution/kernels.py:622-668 (rms_norm_fwd).
 *   h    = residual ? T(x + residual) : x          (stored to sum_out when residual != NULL)
 *   rstd = 1 / sqrt(sum(h^2)/n_cols + eps)         (fp32, stored)
 *   y    = T( fp32(T(h * rstd)) * fp32(weight) )
 * x, residual, sum_out and y share dtype and stride_row; weight has w_dtype and n_cols entries.
 */
int rus_rmsnorm_fwd(const void* x, const void* residual, const void* weight, int32_t w_dtype,
                    void* sum_out, void* y, float* rstd, int64_t n_rows, int64_t n_cols,
                    int64_t stride_row, float eps, int32_t dtype, void* stream);

/*
 * RMSNorm backward with the residual gradient folded in (norm weights are frozen: no dweight).
 * Replaces: solution/kernels.py:166-199 (rms_norm_bwd_kernel), launcher kernels.py:671-714.
 *   xhat = h * rstd;  g = weight * dy;  c = sum(xhat * g) / n_cols
 *   dx   = T( (g - xhat * c) * rstd + (dresidual ? dresidual : 0) )
 * dy, h, dresidual and dx share dtype and stride_row.
 */
int rus_rmsnorm_bwd(const void* dy, const void* h, const void* weight, int32_t w_dtype,
                    const float* rstd, const void* dresidual, void* dx, int64_t n_rows,
                    int64_t n_cols, int64_t stride_row, int32_t dtype, void* stream);

/*
 * rus_rmsnorm_bwd (fp16 activations) whose dy is the fp16 rounding of the sum, in part order, of
 * n_parts fp32 partial products dy_parts [n_parts, n_rows, n_cols] (contiguous): the split-K
 * MLP-backward product d_norm2 = gu W_gu (solution/ops.py:939) consumed by the following
 * norm backward (ops.py:941-943) with exactly the values a separate reduce would write.
 * n_cols and stride_row multiples of 8, operands 16-byte aligned.
 */
int rus_rmsnorm_bwd_parts(const float* dy_parts, int32_t n_parts, const void* h,
                          const void* weight, int32_t w_dtype, const float* rstd,
                          const void* dresidual, void* dx, int64_t n_rows, int64_t n_cols,
                          int64_t stride_row, void* stream);

/*
 * LoRA-delta add + NeoX rotary embedding on packed tokens.
 * Replaces: solution/kernels.py:206-283 (qkv_lora_rope_fwd_kernel), launcher
 *           solution/kernels.py:717-761 (qkv_rope_fwd).
 * qkv is [n_tokens, (h_q + 2 h_kv) * head_dim] = [Q | K | V]; q_lora [n_tokens, h_q*head_dim] and
 * v_lora [n_tokens, h_kv*head_dim] are both given or both NULL. With half = head_dim/2, p = pos[t]:
 *   a = q[j] + scale_q*ql[j], b = q[j+half] + scale_q*ql[j+half]    (fp32, no FMA)
 *   q_out[j]      = T(a*cos[p][j]      - b*sin[p][j])
 *   q_out[j+half] = T(b*cos[p][j+half] + a*sin[p][j+half])
 * K is rotated the same way without LoRA; v_out = T(v + scale_v*vl). Outputs are contiguous
 * [n_tokens, h, head_dim]. cos/sin are [n_pos, stride_cos] of dtype; a position outside
 * [0, n_pos) is clamped into range (never read out of bounds) and, when err_flag != NULL, sets
 * *err_flag = 1. head_dim must be a multiple of 16.
 */
int rus_qkv_lora_rope_fwd(const void* qkv, const void* q_lora, const void* v_lora, const void* cos,
                          const void* sin, const int64_t* pos_ids, void* q_out, void* k_out,
                          void* v_out, int64_t n_tokens, int64_t stride_qkv, int64_t stride_ql,
                          int64_t stride_vl, int64_t stride_cos, int64_t n_pos, float scale_q,
                          float scale_v, int32_t h_q, int32_t h_kv, int32_t head_dim,
                          int32_t* err_flag, int32_t dtype, void* stream);

/*
 * Adjoint NeoX rotation and [dQ | dK | dV] packing.
 * Replaces: solution/kernels.py:286-348 (qkv_lora_rope_bwd_kernel), launcher kernels.py:764-798,
 *           plus the LoRA-gradient scaling of solution/ops.py:144-147 (and ops.py:970-973).
 *   dx[j]      = T(dy[j]*cos[p][j]           + dy[j+half]*sin[p][j+half])
 *   dx[j+half] = T(dy[j+half]*cos[p][j+half] - dy[j]*sin[p][j])
 * for the h_q Q heads and h_kv K heads; dV is copied. dq_rot/dk_rot/dv are contiguous
 * [n_tokens, h, head_dim]; dqkv is [n_tokens, stride_dqkv]. When dq_lora/dv_lora are non-NULL
 * (both or neither) they receive T(fp32(dQ_T) * scale_q) and T(fp32(dV_T) * scale_v), computed
 * from the already-rounded packed values, as contiguous [n_tokens, h*head_dim].
 */
int rus_qkv_rope_bwd(const void* dq_rot, const void* dk_rot, const void* dv, const void* cos,
                     const void* sin, const int64_t* pos_ids, void* dqkv, void* dq_lora,
                     void* dv_lora, int64_t n_tokens, int64_t stride_dqkv, int64_t stride_cos,
                     int64_t n_pos, float scale_q, float scale_v, int32_t h_q, int32_t h_kv,
                     int32_t head_dim, int32_t* err_flag, int32_t dtype, void* stream);

/*
 * rus_qkv_rope_bwd (fp16, dq_lora / dv_lora required) that also forms the LoRA products of the
 * scaled gradients in the same launch: d_mid_q = fp16(dq_lora B_q), d_mid_v = fp16(dv_lora B_v)
 * [n_tokens, r] (solution/ops.py:975-992: d_mid = dq @ B). bt_q / bt_v are B^T [r, h*head_dim]
 * (contiguous, 16-byte aligned). r must be 16, and a token's (h_q + 2 h_kv) * head_dim / 16
 * thread slots must divide 256 with each head kind's slots a multiple of 16 (12 / 2 heads of
 * 128: yes); otherwise RUS_ERR_UNSUPPORTED.
 */
int rus_qkv_rope_bwd_mid(const void* dq_rot, const void* dk_rot, const void* dv, const void* cos,
                         const void* sin, const int64_t* pos_ids, void* dqkv, void* dq_lora,
                         void* dv_lora, const void* bt_q, const void* bt_v, int32_t r,
                         void* d_mid_q, void* d_mid_v, int64_t n_tokens, int64_t stride_dqkv,
                         int64_t stride_cos, int64_t n_pos, float scale_q, float scale_v,
                         int32_t h_q, int32_t h_kv, int32_t head_dim, int32_t* err_flag,
                         void* stream);

/*
 * rus_qkv_rope_bwd_mid with dK and dV given as the per-query-head fp32 partials that
 * rus_attn_varlen_bwd_parts leaves ([h_q, n_tokens, head_dim] each, dK already scaled): each KV
 * head's values are the sum of its h_q / h_kv query heads' partials in head order, rounded to
 * fp16 once -- the dk / dv rus_attn_varlen_bwd writes -- so the packed outputs are the same.
 * At most 8 query heads per KV head.
 * Replaces: as rus_qkv_rope_bwd_mid, fed by the attention backward's sum over the expanded K/V
 * heads (solution/ops.py:669-696, 903-928).
 */
int rus_qkv_rope_bwd_mid_parts(const void* dq_rot, const float* dk_part, const float* dv_part,
                               const void* cos, const void* sin, const int64_t* pos_ids,
                               void* dqkv, void* dq_lora, void* dv_lora, const void* bt_q,
                               const void* bt_v, int32_t r, void* d_mid_q, void* d_mid_v,
                               int64_t n_tokens, int64_t stride_dqkv, int64_t stride_cos,
                               int64_t n_pos, float scale_q, float scale_v, int32_t h_q,
                               int32_t h_kv, int32_t head_dim, int32_t* err_flag, void* stream);

/*
 * LoRA-input dropout, both branches in one pass: out_a = dropout(x; stream_a, p_a),
 * out_b = dropout(x; stream_b, p_b), out = keep ? T(x * (1/(1-p))) : 0.
 * Replaces: the two F.dropout calls on the attention-norm output, solution/ops.py:775-777 (and
 * their RNG-replayed recompute, ops.py:868-869, 882-886).
 * The mask is a pure function of (*seed, stream, row * n_cols + col): element e is kept when the
 * 32-bit word e % 8 of Philox4x64-10(counter = (e / 8, 0, 0, 0), key = (*seed, stream)) is
 * >= round(p * 2^32) (words in order w0.lo, w0.hi, w1.lo, ..., w3.hi). *seed is read on the
 * device. 0 <= p < 1.
 */
int rus_lora_dropout_fwd(const void* x, void* out_a, void* out_b, int64_t n_rows, int64_t n_cols,
                         int64_t stride_x, int64_t stride_a, int64_t stride_b,
                         const uint64_t* seed, uint64_t stream_a, uint64_t stream_b, float p_a,
                         float p_b, int32_t dtype, void* stream);

/*
 * Backward of both dropouts plus the two adds into the input gradient, in place:
 *   acc = T( T(acc + T(dropout(grad_a; stream_a, p_a))) + T(dropout(grad_b; stream_b, p_b)) )
 * with the masks of rus_lora_dropout_fwd.
 * Replaces: solution/ops.py:986-992 (RNG replay, two F.dropout, d_norm1.add_(dx_q).add_(dx_v)).
 */
int rus_lora_dropout_bwd_add(void* acc, const void* grad_a, const void* grad_b, int64_t n_rows,
                             int64_t n_cols, int64_t stride_acc, int64_t stride_a,
                             int64_t stride_b, const uint64_t* seed, uint64_t stream_a,
                             uint64_t stream_b, float p_a, float p_b, int32_t dtype, void* stream);

/*
 * Packed dropout keep bits of n_streams masks [n_rows, n_cols] (n_cols % 8 == 0), the masks of
 * rus_lora_dropout_fwd for streams stream0 .. stream0 + n_streams - 1: bits is uint32
 * [n_streams, n_rows, ceil(n_cols / 32)], bit i of word w of row t of stream s set when element
 * (t, 32 w + i) is kept (0 past the row's end); stream s uses p_even when s is even, else p_odd
 * (so streams 2l / 2l + 1 are the q / v branch of layer l). *seed is read on the device.
 * Replaces: the generator state the reference saves and replays for the LoRA dropouts
 * (solution/ops.py:775-777, 868-869, 882-886, 986-992): all layers' masks of a step in one launch.
 */
int rus_dropout_keep_bits(const uint64_t* seed, uint64_t stream0, int32_t n_streams,
                          int64_t n_rows, int64_t n_cols, float p_even, float p_odd,
                          uint32_t* bits, void* stream);

/*
 * Scratch of the rank-r LoRA entry points below: which = RUS_LORA_DOWN (rus_lora_down_fwd),
 * RUS_LORA_BWD_X (rus_lora_bwd_x) or RUS_LORA_BWD_W (rus_lora_bwd_w). Sets *workspace_floats, the
 * fp32 elements of the caller's workspace (per-block partial sums, 16-byte aligned), and
 * *n_counters, the int32 arrival counters that entry point uses. Counters must be zero before
 * the entry point's first call and are left zero by every call; calls that share counters must
 * not run concurrently (a buffer per entry point and stream). d_q and d_v are ignored for
 * RUS_LORA_DOWN. No counterpart in the reference (its products are torch.mm calls that allocate
 * their own scratch); the sizes follow from the block decomposition of the kernels.
 */
enum { RUS_LORA_DOWN = 0, RUS_LORA_BWD_X = 1, RUS_LORA_BWD_W = 2 };
int rus_lora_workspace_size(int32_t which, int64_t n_tokens, int64_t d, int64_t d_q, int64_t d_v,
                            int32_t r, int64_t* workspace_floats, int64_t* n_counters);

/*
 * Rank-r LoRA down projections of both branches, fp16 (r in {4, 8, 16, 32}):
 *   mid_q = fp16(x_q A_q^T), mid_v = fp16(x_v A_v^T)   x [n_tokens, d] (row stride stride_x),
 *   A [r, d] row-major, mid [n_tokens, r] contiguous,
 * x_q = keep_q ? fp16(x / (1 - p_q)) : 0 with the keep bits bits_q [n_tokens, ceil(d / 32)] of
 * rus_dropout_keep_bits (NULL: x_q = x), x_v likewise.
 * Replaces: the dropouts and the first F.linear of each branch, solution/ops.py:775-778 and the
 * recompute ops.py:882-888. d % 16 == 0, stride_x % 8 == 0, x and A 16-byte aligned.
 * workspace / counters: see rus_lora_workspace_size.
 */
int rus_lora_down_fwd(const void* x, int64_t n_tokens, int64_t d, int64_t stride_x,
                      const void* a_q, const void* a_v, int32_t r, void* mid_q, void* mid_v,
                      const uint32_t* bits_q, const uint32_t* bits_v, float p_q, float p_v,
                      float* workspace, int64_t workspace_floats, int32_t* counters,
                      int64_t n_counters, void* stream);

/*
 * rus_lora_down_fwd without the workspace and counters arguments, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The scratch is a file-scope device array of this
 * library: 4,194,304 fp32 partials (16 MiB) and 4,096 int32 counters per device, held until the
 * process ends; its address is taken with hipGetSymbolAddress on the first call on each device,
 * which also clears the counters on `stream` (every launch leaves them zero). Shapes whose scratch
 * (rus_lora_workspace_size(RUS_LORA_DOWN, ...)) exceeds that are rejected with RUS_ERR_UNSUPPORTED
 * (d = 1536: up to 10,912 tokens at r <= 16, 5,440 at r = 32). The call itself allocates nothing.
 * All calls on one device share the array: calls that overlap in time on one device race.
 */
int rus_lora_down_fwd_noalloc(const void* x, int64_t n_tokens, int64_t d, int64_t stride_x,
                              const void* a_q, const void* a_v, int32_t r, void* mid_q,
                              void* mid_v, const uint32_t* bits_q, const uint32_t* bits_v,
                              float p_q, float p_v, void* stream);

/*
 * rus_qkv_lora_rope_fwd with the LoRA deltas formed in-kernel from the rank-r factors (fp16):
 *   q_lora[t, c] = fp16(mid_q[t, :] . b_q[c, :]), v_lora likewise (b_q [h_q*head_dim, r],
 *   b_v [h_kv*head_dim, r], mid [n_tokens, r], all contiguous), then exactly the RoPE forward.
 * Replaces: the second F.linear of each branch (solution/ops.py:776, 778) plus
 *           kernels.py:206-283 (qkv_lora_rope_fwd_kernel). r in {4, 8, 16, 32}.
 */
int rus_qkv_lora_rope_fwd_mid(const void* qkv, const void* mid_q, const void* mid_v,
                              const void* b_q, const void* b_v, int32_t r, const void* cos,
                              const void* sin, const int64_t* pos_ids, void* q_out, void* k_out,
                              void* v_out, int64_t n_tokens, int64_t stride_qkv,
                              int64_t stride_cos, int64_t n_pos, float scale_q, float scale_v,
                              int32_t h_q, int32_t h_kv, int32_t head_dim, int32_t* err_flag,
                              void* stream);

/*
 * LoRA backward into the input gradient, fp16, in place on dx [n_tokens, d] (row stride
 * stride_dx):
 *   d_mid_q = fp16(dq_lora B_q)  [n_tokens, r]    (dq_lora [n_tokens, d_q] contiguous)
 *   d_mid_v = fp16(dv_lora B_v)
 *   dx = fp16(fp16(dx + fp16 drop_q(fp16(d_mid_q A_q))) + fp16 drop_v(fp16(d_mid_v A_v)))
 * with the forward's keep bits (NULL: no dropout on that branch). The factors come rank-major:
 * a_t_q = A_q^T [d, r], b_t_q = B_q^T [r, d_q] (v alike). d_mid_q / d_mid_v are written for
 * rus_lora_bwd_w. Replaces: solution/ops.py:976-978, 980-982 (d_mid and dx_drop products) and
 * 986-992 (mask replay, two F.dropout, d_norm1.add_(dx_q).add_(dx_v)).
 * d % 32 == 0, d_q % 16 == 0, d_v % 16 == 0, stride_dx % 4 == 0; workspace / counters: see
 * rus_lora_workspace_size.
 */
int rus_lora_bwd_x(const void* dq_lora, const void* dv_lora, int64_t n_tokens, int64_t d_q,
                   int64_t d_v, const void* a_t_q, const void* a_t_v, const void* b_t_q,
                   const void* b_t_v, int32_t r, int64_t d, void* d_mid_q, void* d_mid_v,
                   void* dx, int64_t stride_dx, const uint32_t* bits_q, const uint32_t* bits_v,
                   float p_q, float p_v, float* workspace, int64_t workspace_floats,
                   int32_t* counters, int64_t n_counters, void* stream);

/*
 * LoRA weight gradients, fp16 (each an fp32 sum over tokens in a fixed order, rounded once):
 *   g_a_q [r, d]   = d_mid_q^T x_q      g_b_q [d_q, r] = dq_lora^T mid_q
 *   g_a_v [r, d]   = d_mid_v^T x_v      g_b_v [d_v, r] = dv_lora^T mid_v
 * x_q / x_v: the dropped LoRA inputs, formed from x [n_tokens, d] (row stride stride_x) and the
 * forward's keep bits as in rus_lora_down_fwd; the [n_tokens, r] operands contiguous and 8-byte
 * aligned. Replaces: solution/ops.py:975, 977, 979, 981 (d_qB, d_qA, d_vB, d_vA as torch.mm in
 * fp16). workspace / counters: see rus_lora_workspace_size.
 */
int rus_lora_bwd_w(const void* x, int64_t stride_x, const uint32_t* bits_q,
                   const uint32_t* bits_v, float p_q, float p_v, const void* dq_lora,
                   const void* dv_lora, const void* mid_q, const void* mid_v,
                   const void* d_mid_q, const void* d_mid_v, int64_t n_tokens, int64_t d,
                   int64_t d_q, int64_t d_v, int32_t r, void* g_a_q, void* g_b_q, void* g_a_v,
                   void* g_b_v, float* workspace, int64_t workspace_floats, int32_t* counters,
                   int64_t n_counters, void* stream);

/*
 * rus_lora_bwd_w plus the input-gradient expansion of rus_lora_bwd_x in the same launch, for a
 * caller that already holds d_mid_q / d_mid_v (e.g. from rus_qkv_rope_bwd_mid):
 *   dx = fp16(fp16(dx + fp16 drop_q(fp16(d_mid_q A_q))) + fp16 drop_v(fp16(d_mid_v A_v)))
 * in place on dx [n_tokens, d] (row stride stride_dx), a_t_q = A_q^T [d, r] (v alike), with the
 * weight gradients as rus_lora_bwd_w. Replaces: solution/ops.py:975-992 after d_mid (the dx_drop
 * products, the masked adds and the four weight-gradient products). d % 32 == 0; workspace /
 * counters: those of RUS_LORA_BWD_W.
 */
int rus_lora_bwd_xw(const void* x, int64_t stride_x, const uint32_t* bits_q,
                    const uint32_t* bits_v, float p_q, float p_v, const void* dq_lora,
                    const void* dv_lora, const void* mid_q, const void* mid_v,
                    const void* d_mid_q, const void* d_mid_v, int64_t n_tokens, int64_t d,
                    int64_t d_q, int64_t d_v, int32_t r, void* g_a_q, void* g_b_q, void* g_a_v,
                    void* g_b_v, const void* a_t_q, const void* a_t_v, void* dx,
                    int64_t stride_dx, float* workspace, int64_t workspace_floats,
                    int32_t* counters, int64_t n_counters, void* stream);

/*
 * SwiGLU forward: out = T( g*sigmoid(g) * u ), sigmoid(g) = 1/(1+exp(-g)).
 * Replaces: solution/kernels.py:355-392 (tiled_mlp_glu_fwd_kernel), launcher kernels.py:801-847.
 * For the fused [gate | up] layout pass up = gate + n_cols and stride_u = stride_g.
 */
int rus_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n_rows, int64_t n_cols,
                   int64_t stride_g, int64_t stride_u, int64_t stride_o, int32_t dtype,
                   void* stream);

/*
 * SwiGLU backward: s = sigmoid(g), silu = g*s,
 *   dup   = T(dout * silu)
 *   dgate = T((dout * u) * (s + silu*(1 - s)))
 * Replaces: solution/kernels.py:395-446 (tiled_mlp_glu_bwd_kernel), launcher kernels.py:850-912.
 * In place is allowed (dgate == gate, dup == up with equal strides): every element is read before
 * the same thread overwrites it.
 */
int rus_swiglu_bwd(const void* dout, const void* gate, const void* up, void* dgate, void* dup,
                   int64_t n_rows, int64_t n_cols, int64_t stride_do, int64_t stride_g,
                   int64_t stride_u, int64_t stride_dg, int64_t stride_du, int32_t dtype,
                   void* stream);

/*
 * lm_head cross-entropy, forward statistics over vocabulary rows [vocab_start, vocab_start+n_vocab)
 * of W (weight points at row vocab_start; [n_vocab, ld_w] fp16) against hidden [n_tok, ld_h] fp16.
 * Replaces: the forward chunk loop of solution/ops.py:217-251 (torch.mm into an fp16 logits chunk +
 *           lm_head_piece_kernel MODE 0, solution/kernels.py:480-516). No logits are stored: for
 * every token and every 256 vocabulary rows this writes one partial (m = max z, s = sum e^{z-m},
 * w = sum e^{z-m} z, idx = first global index of the max) at partial row part_base + r/256 of the
 * [*, part_stride] arrays, with z = fp16(H.W^T) (fp32 accumulation), and stores target[t] = z at
 * the token's label when the label falls in the range. d must be a multiple of 64; rows 16-byte
 * aligned; each operand < 4 GiB.
 */
int rus_lmhead_ce_fwd(const void* hidden, const void* weight, const int64_t* labels, int64_t n_tok,
                      int64_t d, int64_t ld_h, int64_t ld_w, int64_t n_vocab, int64_t vocab_start,
                      float* part_m, float* part_s, float* part_w, int32_t* part_idx,
                      int64_t part_base, int64_t part_stride, float* target, void* stream);

/*
 * rus_lmhead_ce_fwd plus the logits it rounds: logits[t][v - vocab_start] = z (fp16) for columns up
 * to round_up(n_vocab, 64) (zeros past n_vocab), ld_z >= that, 16-byte aligned. The buffer is the
 * one rus_lmhead_ce_grad_from_logits later turns into the logit gradient, so a single-pass head
 * forms the gradient without a second GEMM.
 * Replaces: lm_head_piece_kernel MODE 0 (solution/kernels.py:480-516) together with the logit
 *           recompute GEMM of the gradient pass (solution/ops.py:287-319), whose product it keeps.
 */
int rus_lmhead_ce_fwd_keep(const void* hidden, const void* weight, const int64_t* labels,
                           int64_t n_tok, int64_t d, int64_t ld_h, int64_t ld_w, int64_t n_vocab,
                           int64_t vocab_start, float* part_m, float* part_s, float* part_w,
                           int32_t* part_idx, int64_t part_base, int64_t part_stride, float* target,
                           void* logits, int64_t ld_z, void* stream);

/*
 * Logits only: logits[t][v] = fp16(hidden[t] . weight[v]) (fp32 accumulation) for t < n_tok,
 * v < n_vocab, 0 in the columns n_vocab .. round_up(n_vocab, 64) (ld_z >= that). The statistics
 * GEMM without its statistics epilogue; rus_lmhead_ce_rows forms them from the stored rows.
 * Replaces: the chunk GEMM of solution/ops.py:231-237 (the logits of lm_head_piece_kernel's input).
 */
int rus_lmhead_ce_logits(const void* hidden, const void* weight, int64_t n_tok, int64_t d,
                         int64_t ld_h, int64_t ld_w, int64_t n_vocab, void* logits, int64_t ld_z,
                         void* stream);

/*
 * Per-token statistics of kept logit rows [n_tok, n_vocab] (row stride ld_z): lse, entropy,
 * nll (lse - logits[t][labels[t]], 0 for label -100; lse where the label is outside the
 * vocabulary), argmax (first index of the maximum); then, when denom (device scalar) is not NULL,
 * each row becomes its fp16 logit gradient in place: G = fp16((e^{z - lse} - 1[v = label]) *
 * 2^16 / max(denom, 1)) (0 for label -100 and in the padding columns up to round_up(n_vocab, 64)).
 * Replaces: lm_head_piece_kernel MODE 0 and MODE 1 plus lm_head_finish_kernel over one whole row
 * (solution/kernels.py:453-565), for a row the caller holds whole.
 */
int rus_lmhead_ce_rows(void* logits, int64_t ld_z, int64_t n_tok, int64_t n_vocab,
                       const int64_t* labels, const float* denom, float* lse, float* nll,
                       float* entropy, int64_t* argmax, void* stream);

/*
 * Merges n_parts partial rows per token and finishes the statistics.
 * Replaces: solution/kernels.py:534-565 (lm_head_finish_kernel) plus the cross-chunk argmax of
 *           kernels.py:494-498. lse = M + ln S, entropy = lse - W/S, nll = lse - target (0 where the
 * label is -100), argmax = smallest vocabulary index attaining the maximum.
 */
int rus_lmhead_ce_combine(const float* part_m, const float* part_s, const float* part_w,
                          const int32_t* part_idx, int64_t n_parts, int64_t part_stride,
                          const float* target, const int64_t* labels, int64_t n_tok, float* lse,
                          float* nll, float* entropy, int64_t* argmax, void* stream);

/*
 * Loss reduction: denom = max(*num_items, 1) when num_items is not NULL, else
 * max(#(labels != -100), 1); loss = sum(nll) / denom. One workgroup; both outputs on the device.
 * With nll NULL only denom is written (loss may then be NULL too): the denominator the gradient
 * needs before the per-token losses exist. Replaces: solution/ops.py:268-277 (loss = nll.sum() /
 * denominator, with its host .item()).
 */
int rus_lmhead_ce_loss(const float* nll, const int64_t* labels, int64_t n_tok,
                       const float* num_items, float* loss, float* denom, void* stream);

/*
 * Logit gradient for vocabulary rows [vocab_start, vocab_start+n_vocab):
 *   grad_logits[t][v - vocab_start] = fp16((e^{z - lse[t]} - 1[v = label[t]]) * 2^16 / max(*denom, 1))
 * and 0 for tokens whose label is -100; columns up to round_up(n_vocab, 64) are written (zeros past
 * n_vocab). denom is a device scalar (float32).
 * Replaces: lm_head_piece_kernel MODE 1 (solution/kernels.py:517-531) and its recompute GEMM
 *           (solution/ops.py:287-319).
 */
int rus_lmhead_ce_grad_logits(const void* hidden, const void* weight, const int64_t* labels,
                              const float* lse, const float* denom, int64_t n_tok, int64_t d,
                              int64_t ld_h, int64_t ld_w, int64_t n_vocab, int64_t vocab_start,
                              void* grad_logits, int64_t ld_g, void* stream);

/*
 * In place: logits_grad[t][c] = fp16((e^{z - lse[t]} - 1[c = label[t] - vocab_start]) * 2^16 /
 * max(*denom, 1)) with z = logits_grad[t][c] as written by rus_lmhead_ce_fwd_keep, 0 for labels
 * -100 and for columns n_vocab .. round_up(n_vocab, 64). Element for element the formula of
 * rus_lmhead_ce_grad_logits on the same fp16 logits, so both give the same bits.
 * Replaces: lm_head_piece_kernel MODE 1 (solution/kernels.py:517-531) without its recompute GEMM.
 */
int rus_lmhead_ce_grad_from_logits(void* logits_grad, int64_t ld_g, const int64_t* labels,
                                   const float* lse, const float* denom, int64_t n_tok,
                                   int64_t n_vocab, int64_t vocab_start, void* stream);

/*
 * Hidden-state gradient partials: parts[s] (+)= grad_logits[:, Ks] . (W^T[:, Ks])^T over split s of
 * the round_up(n_vocab, 64) columns, parts = [n_split][n_tok][d] fp32 (accumulate != 0 adds to the
 * existing contents). weight_t is W^T ([d, ld_wt] fp16, K-contiguous) positioned at the same first
 * vocabulary column as grad_logits, with zero columns up to round_up(n_vocab, 64). n_split must be
 * ceil(K / round_up(ceil(K / n_split), 64)) for K = round_up(n_vocab, 64).
 * Replaces: d_h_prescaled.addmm_(G, W_chunk) of solution/ops.py:320 (fp16 accumulator there).
 */
int rus_lmhead_ce_grad_hidden(const void* grad_logits, int64_t ld_g, const void* weight_t,
                              int64_t ld_wt, int64_t n_tok, int64_t d, int64_t n_vocab,
                              float* parts, int32_t n_split, int32_t accumulate, void* stream);

/*
 * The hidden-gradient GEMM of the single-pass head: as rus_lmhead_ce_grad_hidden with the
 * chunk's probabilities P (rus_lmhead_ce_chunk_scale) as the first operand, except that with
 * accumulate != 0 each partial row is rescaled before the sum: parts[s][t][:] =
 * parts[s][t][:] * alpha[t] + (P . W_chunk)[t][:] over split s. alpha (device, n_tok floats) is
 * the factor e^{M_old - M_new} that chunk_scale wrote. n_split may exceed the number of 64-wide
 * K pieces: the splits past them have an empty K range and only rescale their partials (so a
 * shorter last chunk keeps every split's rows on the same maximum). Replaces: the per-chunk
 * backward GEMM of
 * solution/ops.py:300-322 (dH += G . W_chunk), without its logit recompute.
 */
int rus_lmhead_ce_grad_hidden_scaled(const void* probs, int64_t ld_p, const void* weight_t,
                                     int64_t ld_wt, int64_t n_tok, int64_t d, int64_t n_vocab,
                                     float* parts, int32_t n_split, int32_t accumulate,
                                     const float* alpha, void* stream);

/*
 * One vocabulary chunk of the single-pass head, between its statistics GEMM (which kept the
 * chunk's fp16 logits in `logits`, rus_lmhead_ce_fwd_keep, partial rows from part_base) and its
 * hidden-gradient GEMM: with the running maximum M_run[t] (ignored when first != 0) and the
 * chunk's maximum (from its partials), M = max(M_run[t], chunk max); the logits become
 * P = fp16(e^{z - M}) in place (0 in the padding columns up to round_up(n_vocab, 64)),
 * M_run[t] = M and alpha[t] = e^{M_run_old - M} (0 when first). Replaces: the logit recompute
 * and lm_head_piece_kernel MODE 1 of solution/ops.py:287-319 / kernels.py:517-531 (the gradient
 * is formed from P once lse is known, in rus_lmhead_ce_dh_finish).
 */
int rus_lmhead_ce_chunk_scale(void* logits, int64_t ld_z, int64_t n_tok, int64_t n_vocab,
                              const float* part_m, int64_t part_stride, int64_t part_base,
                              float* m_run, float* alpha, int32_t first, void* stream);

/*
 * Hidden gradient of the single-pass head from its accumulated partials:
 *   out[t][c] = (sum_s parts[s][t][c] * e^{M_run[t] - lse[t]} - W[y_t][c]) * 2^16 / denom * scale
 *               (* *scale_dev when given)
 * for tokens with y_t != -100 (the W row only when 0 <= y_t < n_vocab), 0 otherwise; since
 * sum_s parts = sum_v e^{z_v - M_run} W_v, this is sum_v (softmax - onehot) W_v with the
 * reference's 2^16 / denom prescale. w_rows [n_vocab, ld_w] fp16 is device memory, or pinned
 * host memory when w_on_host != 0 (label rows read over the bus). d % 4 == 0; out fp16 or fp32.
 * Replaces: the backward's fp16 dH accumulation and rescale, solution/ops.py:283, 320, 332-339.
 */
int rus_lmhead_ce_dh_finish(const float* parts, int32_t n_parts, int64_t n_tok, int64_t d,
                            const float* m_run, const float* lse, const int64_t* labels,
                            const void* w_rows, int64_t ld_w, int64_t n_vocab, int32_t w_on_host,
                            const float* denom, float scale, const float* scale_dev, void* out,
                            int32_t out_dtype, void* stream);

/*
 * out[i] = T(scale * (*scale_dev) * sum_p parts[p * n_elem + i]), T = out_dtype (fp16 or fp32);
 * scale_dev is an optional device scalar (NULL = 1), e.g. the incoming loss gradient, so the
 * caller never has to read it back to the host.
 * Replaces: the prescale undo of solution/ops.py:337-338 (and the split-K sum).
 */
int rus_lmhead_dh_reduce(const float* parts, int32_t n_parts, int64_t n_elem, float scale,
                         const float* scale_dev, void* out, int32_t out_dtype, void* stream);

/*
 * dst[c][r] = src[r][c] for r < rows, c < cols and dst[c][r] = 0 for rows <= r < rows_pad (fp16,
 * row strides ld_src >= cols, ld_dst >= rows_pad). Builds the K-contiguous W^T operand of the
 * hidden-gradient GEMM from W rows on the device (once for a resident head; per chunk for a head
 * streamed from the host). Replaces: the weight transpose inside the reference's backward GEMM
 * call (solution/ops.py:320, torch addmm on W^T views).
 */
int rus_transpose_f16(const void* src, int64_t rows, int64_t cols, int64_t ld_src, void* dst,
                      int64_t ld_dst, int64_t rows_pad, void* stream);

/*
 * Varlen causal GQA attention forward over packed tokens (fp16, head_dim 128 only):
 *   out[t, h, :] = softmax_j( scale * q[t, h, :] . k[j, g, :] ) v[j, g, :],  g = h / (h_q / h_kv),
 * j over the tokens of t's row with j <= t; rows are [cu[i], cu[i+1]) of the device int32
 * cu_seqlens [n_seq + 1], which must cover all n_tokens tokens. q [n_tokens, h_q, 128],
 * k/v [n_tokens, h_kv, 128], out like q (all contiguous, 16-byte aligned); lse [h_q, n_tokens]
 * fp32 natural-log sum-exp of the scaled scores. max_blocks >= sum_i ceil(len_i / 32)
 * (n_tokens / 32 + n_seq always suffices); extra blocks exit. P is rounded to fp16 for the PV
 * product, accumulation is fp32.
 * Replaces: solution/ops.py:669-696 (_run_packed_sdpa: torch SDPA per row with K/V expanded
 * to the query heads, is_causal=True).
 */
int rus_attn_varlen_fwd(const void* q, const void* k, const void* v, const int32_t* cu_seqlens,
                        int32_t n_seq, int64_t n_tokens, int32_t max_blocks, int32_t h_q,
                        int32_t h_kv, int32_t head_dim, float scale, void* out, float* lse,
                        void* stream);

/*
 * Backward of rus_attn_varlen_fwd: dq like q, dk / dv like k / v (fp16; dk and dv sum the h_q /
 * h_kv query heads of each group in fp32 and are rounded once). out and lse are the forward's.
 * workspace: fp32, at least 2 * h_q * n_tokens * 128 elements (per-query-head dK and dV
 * partials [h_q, n_tokens, 128] each, dK scaled). Both passes (dQ, and dK / dV with the sum over
 * each group's heads) run as one launch, each block forming D = rowsum(dO o O) of the query rows
 * it visits; max_blocks at most 32767.
 * counters: int32, at least max_blocks * h_kv, zero before the first call and left zero (calls
 * sharing them must not run concurrently).
 * Replaces: the autograd backward of solution/ops.py:669-696 (torch SDPA backward plus the
 * sum over the expanded K/V heads), run by solution/ops.py:903-928.
 */
int rus_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* out,
                        const void* dout, const float* lse, const int32_t* cu_seqlens,
                        int32_t n_seq, int64_t n_tokens, int32_t max_blocks, int32_t h_q,
                        int32_t h_kv, int32_t head_dim, float scale, void* dq, void* dk,
                        void* dv, float* workspace, int32_t* counters, int64_t n_counters,
                        void* stream);

/*
 * rus_attn_varlen_bwd without the sum over each KV group's query heads: dq as there; dK and dV
 * stay in the workspace as the per-query-head fp32 partials (layout above), for
 * rus_qkv_rope_bwd_mid_parts to sum while it packs them (no counters, no dk / dv outputs).
 * Replaces: as rus_attn_varlen_bwd.
 */
int rus_attn_varlen_bwd_parts(const void* q, const void* k, const void* v, const void* out,
                              const void* dout, const float* lse, const int32_t* cu_seqlens,
                              int32_t n_seq, int64_t n_tokens, int32_t max_blocks, int32_t h_q,
                              int32_t h_kv, int32_t head_dim, float scale, void* dq,
                              float* workspace, void* stream);

/*
 * A step's fp16 LoRA factors in both layouts, one launch. flat: fp32, n_layers x [segment 0 |
 * ... | segment n_seg-1] (n_seg <= 4), segment j row-major [seg_rows[j], seg_cols[j]]
 * (host arrays). out: fp16, the same layout (each value rounded to nearest even once); out_t
 * (optional): fp16, region j = [n_layers, seg_cols[j], seg_rows[j]], each layer's segment
 * transposed, regions back to back in segment order (region j starts at n_layers times the
 * per-layer offset of segment j).
 * Replaces: the per-layer fp16 casts of the LoRA factors (solution/ops.py:776, 778, and the
 * backward's q_B_fp16 / q_A_fp16 operands, ops.py:979-987); out_t is the rank-major layout the
 * fused LoRA backward kernels read.
 */
int rus_lora_cast_t(const float* flat, int64_t n_layers, int32_t n_seg, const int64_t* seg_rows,
                    const int64_t* seg_cols, void* out, void* out_t, void* stream);

/*
 * One AdamW step (step number step >= 1) over n fp32 values: param, exp_avg and exp_avg_sq
 * updated in place from grad with torch.optim.AdamW's update (amsgrad and maximize off), in the
 * order of torch's single- and multi-tensor paths: param *= 1 - lr weight_decay; exp_avg =
 * lerp(exp_avg, grad, 1 - beta1); exp_avg_sq = exp_avg_sq beta2 + (1 - beta2) grad grad;
 * param += -(lr / bc1) exp_avg / (sqrt(exp_avg_sq) / sqrt(bc2) + eps), bc1 = 1 - beta1^step,
 * bc2 = 1 - beta2^step. The scalars are formed in double and rounded once to fp32. Buffers
 * 16-byte aligned, not overlapping. One launch.
 * Replaces: the trainer's torch.optim.AdamW step over the LoRA factors (HF "adamw_torch";
 * reference harness/_train.py:30 forwards the trainer's optim settings).
 */
int rus_adamw_step(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, int64_t n,
                   double lr, double beta1, double beta2, double eps, double weight_decay,
                   int64_t step, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RUS_AMD_H */
