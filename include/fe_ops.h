/*
 * fe_ops.h - the per-token operators around the attention path: the rest of
 * the reference's native op boundary (include/fe/native_cuda.hpp:11,12,15)
 * and the fused q/k RMSNorm + RoPE + paged-KV append.
 *
 * Same conventions as fe_attn.h: 16-bit tensors are bf16 when bf16 != 0,
 * fp16 otherwise; device pointers; every call is ordered on `stream` (a
 * hipStream_t) and does no allocation or host synchronisation; FE_OK or a
 * negative FE_E* code with the message in fe_attn_last_error().
 */
#ifndef FE_OPS_H
#define FE_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces fe::cuda::norm (native_cuda.hpp:11; cuda_kernels.cu:11-17,28-31):
 * per row of x [rows][width], v = x (+ residual when residual != NULL),
 * new_residual = v (when != NULL), output = v * rsqrt(mean(v^2) + eps) *
 * weight.  The sum of squares is taken in the reference kernel's order (a
 * 256-way strided FMA accumulation, then a pairwise tree); rsqrt is
 * 1 / sqrt in double precision rounded once to float.  output may alias x. */
int fe_norm(const void* x, const void* residual, const void* weight, void* output, void* new_residual, int rows,
            int width, float eps, int bf16, void* stream);

/* Replaces fe::cuda::silu_mul (native_cuda.hpp:12; cuda_kernels.cu:18,32):
 * gate_up [rows][2*width] -> output [rows][width] = silu(gate) * up in fp32,
 * rounded once to bf16/fp16. */
int fe_silu_mul(const void* gate_up, void* output, int rows, int width, int bf16, void* stream);

/* Replaces fe::cuda::accept (native_cuda.hpp:15; cuda_kernels.cu:25,35;
 * portable_gpu_ops.cpp:56-58): draft [batch][k], verify [batch][k+1] ->
 * out [batch][k+2]: out[b][0..k] = verify[b][0..k], out[b][k+1] = m + 1 where
 * m is the length of the longest prefix on which draft and verify agree
 * (out[b][0..m] is the accepted tokens plus the bonus token, as
 * accept_greedy in scheduler.cpp:110).  Writes nothing outside out. */
int fe_accept(const int64_t* draft, const int64_t* verify, int64_t* out, int batch, int k, void* stream);

/* No single reference counterpart: the per-layer sequence of
 * src/cuda_model.cpp:91-95 (q = norm(q, q_weight), k = norm(k, k_weight),
 * rope(q, k), store(k, v)) in one pass, bit-identical to fe_norm +
 * fe_rope + fe_store on the same inputs.  Row r of qkv holds hq query heads,
 * hkv key heads and hkv value heads of dim 128 (in that order) starting at
 * qkv + r*row_stride elements.  q_out [rows][hq][128] receives the normalized
 * rotated queries; the caches receive the normalized rotated keys and the
 * values at slots[r] (rows with slot < 0 or >= cache_slots write no cache
 * entry).  hq = 0 is the draft context projection of cuda_model.cpp:104-107
 * (keys and values only; q_out and q_weight unused). */
int fe_norm_rope_append(const void* qkv, int64_t row_stride, const void* q_weight, const void* k_weight,
                        float eps, void* q_out, void* k_cache, void* v_cache, const int64_t* pos,
                        const int64_t* slots, const float* cache, int rows, int hq, int hkv, int dim, int bf16,
                        int max_positions, int cache_slots, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FE_OPS_H */
