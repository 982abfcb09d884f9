/*
 * vx_oracle_internal.h -- helpers of vx_oracle.c shared with
 * vx_oracle_codec.c.  TEST INFRASTRUCTURE ONLY (see vx_oracle.h).
 */
#ifndef VX_ORACLE_INTERNAL_H
#define VX_ORACLE_INTERNAL_H

#include <stdint.h>

/* f16 -> f32 table (all 65536 halves) */
const float *vxo_i_h2f_table(void);
/* shared-memory tree of the 256-thread reduction shaders over sd[256] */
float vxo_i_tree_sum(float *sd);
/* matvecF16 rows (src/shaders.ts:21-71) for nb <= 8 vectors sharing A:
 * ys[b][m] = A[m,:] . xs[b] in the 256-lane order */
void vxo_i_matvec_multi(const uint16_t *A, const float *const *xs, float *const *ys, int nb,
                        int M, int K);

#endif
