/*
 * Runner ops of libvasc_hip.so: kernels of the VGGT/Pi3-shaped benchmark
 * models around the sparse global-attention operator. They have no
 * counterpart in the reference's sparse-attention interface (the reference
 * runs these steps as separate torch kernels of the upstream models); the
 * library's runners (vasc_amd/aggregator.py) call them.
 *
 * Conventions as in vasc_hip.h: raw device pointers, int64 sizes and row
 * strides in elements, the HIP stream as void*, an int status (0 ok) with
 * the message in vasc_last_error().
 */
#ifndef VASC_RUNNER_H
#define VASC_RUNNER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Residual update and LayerNorm between the sub-layers of a pre-norm block
 * (upstream block: x = x + ls(branch(norm(x))), then the next norm):
 *   s = bf16(x + bf16(y * gamma))       (torch's bf16 LayerScale and add)
 *   x_out = s                           (may be x itself; NULL: not written)
 *   norm_out = bf16((s - mean) * rstd * norm_w + norm_b)  (NULL: not written)
 * with mean, variance and rstd = 1/sqrt(var + eps) of the row in fp32.
 * x, y, x_out, norm_out: [rows, dim] bf16, row strides ldx, ldy, ldo, ldn;
 * gamma, norm_w, norm_b: [dim] bf16, each may be NULL (no scale, weight 1,
 * bias 0). Built variants: dim 512, 1024, 1536, 2048.
 */
int vasc_residual_norm(const uint16_t *x, int64_t ldx, const uint16_t *y, int64_t ldy, const uint16_t *gamma,
                       const uint16_t *norm_w, const uint16_t *norm_b, float eps, uint16_t *x_out, int64_t ldo,
                       uint16_t *norm_out, int64_t ldn, int64_t rows, int64_t dim, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VASC_RUNNER_H */
