/* CPU oracle helpers in C (test infrastructure only: tests/ and bench.py's
 * cpu_baseline leg load this through oracle/cref.py; the product never does).
 *
 * vq_assign_direct: the nearest-centroid rule of the reference's assignment
 * kernel's statement (triton_kernels.py:703-725), uncontracted: for each row,
 * the squared distance to centroid k is summed over dims 0..d-1 in order as
 * fp32 (difference, square, add: three roundings, no fused multiply-add), and
 * the first centroid with the strictly smallest distance wins.  Leaving the
 * multiply-add unfused is this project's choice: Triton's default fp fusion
 * may compile the kernel's `dist += diff * diff` to an FMA, which can pick
 * another centroid on exact near-ties; that form is not restated here.
 * It restates oracle/ref.py's numpy vq_assign_direct row by row; built with
 * -ffp-contract=off so the compiler keeps the three roundings.  Rows are independent, so the OpenMP split over
 * rows does not change any result.
 */
#include <math.h>
#include <stdint.h>

void vq_assign_direct(const float* x, int64_t n, int d, const float* c, int k, int64_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float* xi = x + i * d;
    float best = INFINITY;
    int64_t arg = 0;
    for (int j = 0; j < k; ++j) {
      const float* cj = c + (int64_t)j * d;
      float dist = 0.0f;
      for (int e = 0; e < d; ++e) {
        const float df = xi[e] - cj[e];
        const float sq = df * df;
        dist = dist + sq;
      }
      if (dist < best) {
        best = dist;
        arg = j;
      }
    }
    out[i] = arg;
  }
}
