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

#define RUS_ABI_VERSION 1

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

#ifdef __cplusplus
}
#endif

#endif /* RUS_AMD_H */
