/*
 * oracle/fmaf.c — CPU restatement of the arithmetic on the eas hot path.
 *
 * TEST INFRASTRUCTURE ONLY: called by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never part of the product.
 *
 * Reference semantics restated:
 *   - f32 add of the SPMD add kernel (examples/add.py:23-31, MSL `a + b`,
 *     eas/codegen/msl.py:224-237): IEEE-754 binary32 round-to-nearest-even;
 *   - fused multiply-add produced by the IR pass _fuse_fma
 *     (eas/compiler.py:1019-1096) and lowered to MSL `fma(x, y, z)`
 *     (eas/codegen/msl.py:296): one rounding of the exact x*y+z, i.e. C99 fmaf
 *     (glibc's fmaf is correctly rounded in every rounding mode);
 *   - the f16 fma `half(fma((float)x, (float)y, (float)z))` (msl.py:291-294)
 *     is this f32 fmaf followed by an f32->f16 RNE conversion (done in Python).
 */
#include <math.h>
#include <stddef.h>

void eas_oracle_add_f32(const float* a, const float* b, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void eas_oracle_fmaf(const float* a, const float* b, const float* c, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = fmaf(a[i], b[i], c[i]);
}

/* One fma per k, k ascending from 0, accumulator starting at +0.0f: the
 * per-thread `dot` (eas/codegen/msl.py:920-952) for one output. */
float eas_oracle_dot_f32(const float* a, size_t a_stride, const float* b, size_t b_stride, size_t k) {
  float acc = 0.0f;
  for (size_t i = 0; i < k; ++i) acc = fmaf(a[i * a_stride], b[i * b_stride], acc);
  return acc;
}
