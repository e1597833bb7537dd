/*
 * CPU oracle for the selective-scan inference path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker / CPU baseline.  The product package
 * (mamba_metal_amd) never links, imports or calls it.
 *
 * This is a plain sequential restatement of the reference's selective-scan
 * semantics:
 *   - recurrence and D / SiLU(z) placement: experiments/09-features/test_features.py:23-43
 *     (h = exp(delta*A)*h + delta*u*B ; y_t = <h, C_t> ; y += D*u ; y *= silu(z))
 *   - softplus with the "> 20 passes through" cutoff:
 *     mamba_metal/kernels/selective_scan_chunked.metal:60-65 and
 *     experiments/09-features/test_features.py:13-16 (log1p(exp(x)) form)
 *   - fp16 inputs are upcast before any arithmetic: experiments/10-fp16/test_fp16.py:147-156
 *     (callers convert to float before calling in here)
 *   - final state = h at position seqlen-1: experiments/18-prefill/verify_state_out.py:13-26,
 *     mamba_metal/kernels/selective_scan_chunked.metal:151-155
 *   - b = (delta*u)*B grouping: selective_scan_chunked.metal:79
 *
 * Layouts are the reference's row-major contiguous ones
 * (mamba_metal/selective_scan.py:36-44): u, delta, z, y: (batch, dim, seqlen);
 * A: (dim, dstate); B, C: (batch, dstate, seqlen); D: (dim,); state: (batch, dim, dstate).
 *
 * h0 (nullable) is an initial state, an oracle-only extension used by the
 * composition tests (scan(x1 ++ x2) == scan(x2, h0 = state(x1))).
 *
 * Two precisions: *_f64 accumulates everything in double (the reference point
 * for tolerance checks), *_f32 mirrors the reference's float arithmetic.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static double softplus_d(double x) { return x <= 20.0 ? log1p(exp(x)) : x; }
static float softplus_f(float x) { return x <= 20.0f ? log1pf(expf(x)) : x; }
static double silu_d(double x) { return x / (1.0 + exp(-x)); }
static float silu_f(float x) { return x / (1.0f + expf(-x)); }

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/*
 * Channel range [c_begin, c_end) over the flattened (batch, dim) index lets the
 * CPU baseline time a bounded sample of a large workload.
 */
void oracle_selective_scan_f64(const float* u, const float* delta, const float* A,
                               const float* B, const float* C, const float* D,
                               const float* z, const float* h0, float* y, float* state_out,
                               int64_t batch, int64_t dim, int64_t dstate, int64_t seqlen,
                               int delta_softplus, int64_t c_begin, int64_t c_end) {
  (void)batch;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t ch = c_begin; ch < c_end; ++ch) {
    const int64_t bi = ch / dim, di = ch % dim;
    double h[64 * 4];
    double* hp = dstate <= 256 ? h : (double*)malloc(sizeof(double) * (size_t)dstate);
    for (int64_t n = 0; n < dstate; ++n) hp[n] = h0 ? (double)h0[ch * dstate + n] : 0.0;
    const float* ur = u + ch * seqlen;
    const float* dr = delta + ch * seqlen;
    const float* Br = B + bi * dstate * seqlen;
    const float* Cr = C + bi * dstate * seqlen;
    for (int64_t t = 0; t < seqlen; ++t) {
      double dt = (double)dr[t];
      if (delta_softplus) dt = softplus_d(dt);
      const double ut = (double)ur[t];
      const double du = dt * ut;
      double acc = 0.0;
      for (int64_t n = 0; n < dstate; ++n) {
        const double a = exp(dt * (double)A[di * dstate + n]);
        hp[n] = a * hp[n] + du * (double)Br[n * seqlen + t];
        acc += hp[n] * (double)Cr[n * seqlen + t];
      }
      if (D) acc += (double)D[di] * ut;
      if (z) acc *= silu_d((double)z[ch * seqlen + t]);
      if (y) y[ch * seqlen + t] = (float)acc;
    }
    if (state_out)
      for (int64_t n = 0; n < dstate; ++n) state_out[ch * dstate + n] = (float)hp[n];
    if (hp != h) free(hp);
  }
}

void oracle_selective_scan_f32(const float* u, const float* delta, const float* A,
                               const float* B, const float* C, const float* D,
                               const float* z, const float* h0, float* y, float* state_out,
                               int64_t batch, int64_t dim, int64_t dstate, int64_t seqlen,
                               int delta_softplus, int64_t c_begin, int64_t c_end) {
  (void)batch;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t ch = c_begin; ch < c_end; ++ch) {
    const int64_t bi = ch / dim, di = ch % dim;
    float h[256];
    float* hp = dstate <= 256 ? h : (float*)malloc(sizeof(float) * (size_t)dstate);
    for (int64_t n = 0; n < dstate; ++n) hp[n] = h0 ? h0[ch * dstate + n] : 0.0f;
    const float* ur = u + ch * seqlen;
    const float* dr = delta + ch * seqlen;
    const float* Br = B + bi * dstate * seqlen;
    const float* Cr = C + bi * dstate * seqlen;
    const float* Ar = A + di * dstate;
    for (int64_t t = 0; t < seqlen; ++t) {
      float dt = dr[t];
      if (delta_softplus) dt = softplus_f(dt);
      const float ut = ur[t];
      const float du = dt * ut;
      float acc = 0.0f;
      for (int64_t n = 0; n < dstate; ++n) {
        const float a = expf(dt * Ar[n]);
        hp[n] = a * hp[n] + du * Br[n * seqlen + t];
        acc += hp[n] * Cr[n * seqlen + t];
      }
      if (D) acc += D[di] * ut;
      if (z) acc *= silu_f(z[ch * seqlen + t]);
      if (y) y[ch * seqlen + t] = acc;
    }
    if (state_out)
      for (int64_t n = 0; n < dstate; ++n) state_out[ch * dstate + n] = hp[n];
    if (hp != h) free(hp);
  }
}

/*
 * Inclusive (a, b) pair scan: h_i = a_i * h_{i-1} + b_i, h_{-1} = 0;
 * a_out_i = prod_{k<=i} a_k.  Restates mamba_metal/kernels/pair_scan.metal:1-76
 * (combine (a2,b2)o(a1,b1) = (a2*a1, a2*b1 + b2), identity (1, 0)) sequentially,
 * as experiments/05-pair-scan/pair_scan.py:36-42 does.
 */
void oracle_pair_scan_f64(const float* a, const float* b, float* a_out, float* h_out, int64_t n) {
  double ha = 1.0, hb = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    hb = (double)a[i] * hb + (double)b[i];
    ha = (double)a[i] * ha;
    if (a_out) a_out[i] = (float)ha;
    if (h_out) h_out[i] = (float)hb;
  }
}
