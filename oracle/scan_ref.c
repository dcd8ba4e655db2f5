/*
 * C restatement of selective_scan_ref (external/mamba/mamba_ssm/ops/
 * selective_scan_interface.py:115-181 of the reference) for real A, variable
 * B / C, fp32 state and fp32 silu(z). TEST INFRASTRUCTURE ONLY: used by
 * tests/ to check the GPU scan at full Mamba sizes in seconds; never part of
 * the product.
 *
 * Layouts (all float32, contiguous):
 *   u, delta, z, out : [batch, dim, seqlen]
 *   A                : [dim, dstate]
 *   B, C             : [batch, ngroups, dstate, seqlen]
 *   D, delta_bias    : [dim]            (may be NULL)
 *   last_state       : [batch, dim, dstate] (may be NULL)
 *   initial_state    : [batch, dim, dstate] (may be NULL = zeros)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

static float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

void ak_oracle_selective_scan(const float* u, const float* delta, const float* A, const float* B,
                              const float* C, const float* D, const float* z,
                              const float* delta_bias, const float* initial_state, float* out,
                              float* last_state, int64_t batch, int64_t dim, int64_t seqlen,
                              int64_t dstate, int64_t ngroups, int delta_softplus) {
  const int64_t per_group = dim / ngroups;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t d = 0; d < dim; ++d) {
      float x[256];
      const int64_t g = d / per_group;
      const float* Bg = B + (b * ngroups + g) * dstate * seqlen;
      const float* Cg = C + (b * ngroups + g) * dstate * seqlen;
      const int64_t row = (b * dim + d) * seqlen;
      for (int64_t n = 0; n < dstate; ++n)
        x[n] = initial_state ? initial_state[(b * dim + d) * dstate + n] : 0.0f;
      for (int64_t l = 0; l < seqlen; ++l) {
        float dl = delta[row + l] + (delta_bias ? delta_bias[d] : 0.0f);
        if (delta_softplus) dl = softplus_f(dl);
        const float ul = u[row + l];
        float y = 0.0f;
        for (int64_t n = 0; n < dstate; ++n) {
          const float da = expf(dl * A[d * dstate + n]);
          x[n] = da * x[n] + dl * Bg[n * seqlen + l] * ul;
          y += x[n] * Cg[n * seqlen + l];
        }
        float o = D ? y + ul * D[d] : y;
        if (z) {
          const float zl = z[row + l];
          o *= zl / (1.0f + expf(-zl));
        }
        out[row + l] = o;
      }
      if (last_state)
        for (int64_t n = 0; n < dstate; ++n) last_state[(b * dim + d) * dstate + n] = x[n];
    }
  }
}
