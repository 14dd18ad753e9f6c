/* C restatement of the causal prefix mean (TEST INFRASTRUCTURE ONLY).
 *
 * h[b][t][d] = fp32( sum_{s<=t} x[b][s][d] accumulated in fp64 ) / fp32(t+1)
 *
 * Follows mom_kernels/reference.py:32-36 and model.py:169-176
 * (torch.cumsum(x.float(), 1) / arange(1, T+1)): CPU torch accumulates an
 * fp32 cumsum in double and rounds each prefix once; the divide is IEEE
 * fp32.  Used by the tests to pin oracle.prefix_mean independently of torch.
 */
#include <stddef.h>

void naylis_oracle_prefix_mean_f32(const float* x, float* h, long B, long T, long D) {
  for (long b = 0; b < B; ++b)
    for (long d = 0; d < D; ++d) {
      double run = 0.0;
      for (long t = 0; t < T; ++t) {
        run += (double)x[(b * T + t) * D + d];
        const float cs = (float)run;
        const float denom = (float)(t + 1);
        h[(b * T + t) * D + d] = cs / denom;
      }
    }
}
