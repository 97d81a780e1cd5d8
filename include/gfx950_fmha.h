/*
 * gfx950_fmha.h -- C ABI of the MI355X (gfx950) flash-attention forward pass,
 * built into the same library as gfx950_gemm.h (whose status codes and
 * element types it uses).
 *
 * O = softmax(Q K^T * sm_scale) V for every (batch, query head), non-causal,
 * with grouped K/V heads: query head h reads K/V head h * HK / HQ (HQ a
 * multiple of HK; HK == HQ is plain multi-head, HK == 1 multi-query).  Q, K, V
 * and O hold 16-bit elements (`dtype` G9_F16 or G9_BF16) with head dim 128
 * or 64; scores, softmax and the output accumulator are fp32.
 */
#ifndef GFX950_FMHA_H
#define GFX950_FMHA_H

#include <stdint.h>

#include "gfx950_gemm.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Replaces the launch in run_gluon_attention
 * (kernels/attention/fmha_v4.py:761-790; same interface as
 * kernels/attention/fmha_v3.py:522-549), including its kernel arguments
 * (q, k, v, sm_scale, L, o, the four stride tuples, HQ, HK, N_CTX, SCALE_ON_Q).
 *
 * q, o: B x HQ x S x D; k, v: B x HK x S x D, addressed through strides in
 * ELEMENTS given as (batch, head, seq, dim) -- the order of
 * get_strides_from_layout (kernels/attention/common.py:84-92), so both the
 * bhsd and the bshd layouts (and any other with a unit dim stride) are
 * accepted.  Requirements: D == 128 or D == 64 (the reference's powers of
 * two; its layouts are written for 128), S a multiple of 64, unit dim stride,
 * 16-byte aligned base pointers and batch / head / seq strides, and
 * (S + 256) * seq_stride * 2 < 2^31 bytes for each tensor.
 *
 * lse: optional (NULL to skip) fp32 B x HQ x S, contiguous: the natural-log
 * log-sum-exp of each query's scaled scores (the reference's L / M buffer).
 * scale_on_q != 0 multiplies Q by sm_scale * log2(e) and rounds it to the
 * input type before the loop (SCALE_ON_Q=True, the reference default); 0
 * applies the scale to the fp32 scores.  sm_scale must be positive.
 * variant selects the softmax rescale of the reference kernel of that number:
 * 3 rescales the output accumulator whenever a row's running max grows
 * (kernels/attention/fmha_v3.py:96-152), 4 advances a row's max only when a
 * tile exceeds it by more than 8 (log2 units) and skips the rescale when no
 * row of a wave moved (kernels/attention/fmha_v4.py:143-210, 247-270).  Both
 * give the same softmax up to fp32 rounding; another value -> G9_ERR_SCHEDULE.
 *
 * Launches one kernel on `stream`; allocates nothing.
 */
int g9_fmha_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t HQ,
                int64_t HK, int64_t S, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                const int64_t* v_strides, const int64_t* o_strides, float sm_scale, int dtype, int scale_on_q,
                int variant, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GFX950_FMHA_H */
