/*
 * TEST INFRASTRUCTURE ONLY -- C99 restatement of TensorPlay's CPU softmax /
 * log_softmax composite, the autograd formulas for their gradients, and the
 * CPU nll_loss / nll_loss_backward kernels.  It is the checker for the HIP
 * path and never part of the product.
 *
 * Arrays are dense float32 in the logical layout [outer, n, inner] (the
 * softmax dim is n); the Python front-end makes them so.  Built with
 * -ffp-contract=off: every float operation rounds as the reference's does.
 */
#include <math.h>
#include <stdint.h>

#include "tp_cpu_reduce.h"

/* softmax_kernel / log_softmax_kernel
 * (/root/reference/p10/src/backend/cpu/PointwiseKernels.cpp:519-545):
 *   max_val = input.max({dim}, true)   max_dim_kernel: -inf start, strict >
 *                                       (ReductionKernels.cpp:256-315)
 *   shifted = input - max_val          fp32 subtract
 *   exp_val = shifted.exp()            std::exp on float (PointwiseKernels.cpp:227)
 *   sum_exp = exp_val.sum({dim}, true) fp32 accumulation in input order
 *                                       (ReductionKernels.cpp:157-178)
 *   softmax = exp_val / sum_exp        fp32 divide (ArithmeticKernels.cpp:1373-1379)
 *   log_softmax = shifted - log(sum_exp)  std::log on float (PointwiseKernels.cpp:228) */
void or_softmax(const float* x, int64_t outer, int64_t n, int64_t inner, int32_t log_mode, float* y) {
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t i = 0; i < inner; ++i) {
            const float* xs = x + o * n * inner + i;
            float* ys = y + o * n * inner + i;
            float m = -INFINITY;
            for (int64_t r = 0; r < n; ++r)
                if (xs[r * inner] > m) m = xs[r * inner];
            float s = 0.0f;
            for (int64_t r = 0; r < n; ++r) {
                const float sh = xs[r * inner] - m;
                const float e = expf(sh);
                s += e;
                ys[r * inner] = log_mode ? sh : e; /* shifted or exp_val */
            }
            if (log_mode) {
                const float ls = logf(s);
                for (int64_t r = 0; r < n; ++r) ys[r * inner] = ys[r * inner] - ls;
            } else {
                for (int64_t r = 0; r < n; ++r) ys[r * inner] = ys[r * inner] / s;
            }
        }
    }
}

/* Gradients, /root/reference/config/derivatives.yaml:91-95, composed op by op
 * as TensorPlay's autograd evaluates them (fp32 each step):
 *   softmax:     (grad - (grad * result).sum({dim}, true)) * result
 *   log_softmax: grad - self.log_softmax(dim).exp() * grad.sum({dim}, true)
 * with y = the forward output (result, or log_softmax(self)). */
void or_softmax_bwd(const float* g, const float* y, int64_t outer, int64_t n, int64_t inner, int32_t log_mode,
                    float* gx) {
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t i = 0; i < inner; ++i) {
            const int64_t b = o * n * inner + i;
            float s = 0.0f;
            for (int64_t r = 0; r < n; ++r) {
                const int64_t k = b + r * inner;
                if (log_mode) {
                    s += g[k];
                } else {
                    const float p = g[k] * y[k];
                    s += p;
                }
            }
            for (int64_t r = 0; r < n; ++r) {
                const int64_t k = b + r * inner;
                if (log_mode) {
                    const float e = expf(y[k]);
                    const float t = e * s;
                    gx[k] = g[k] - t;
                } else {
                    const float d = g[k] - s;
                    gx[k] = d * y[k];
                }
            }
        }
    }
}

/* nll_loss_kernel (/root/reference/p10/src/backend/cpu/LossKernels.cpp:12-55).
 * x dense [N, C]; w NULL or [C].  out: [N] (reduction 0) or one value.
 * Returns 1 for a target outside [0, C) that is not ignore_index (the
 * reference raises "Target out of bounds"), else 0. */
int32_t or_nll_loss(const float* x, int64_t N, int64_t C, const int64_t* t, const float* w, int64_t reduction,
                    int64_t ignore_index, float* out, float* total_weight) {
    float tw = 0.0f;
    for (int64_t i = 0; i < N; ++i) {
        const int64_t ti = t[i];
        if (ti == ignore_index) {
            if (reduction == 0) out[i] = 0.0f;
            continue;
        }
        if (ti < 0 || ti >= C) return 1;
        const float wi = w ? w[ti] : 1.0f;
        const float li = -x[i * C + ti] * wi;
        if (reduction == 0) out[i] = li;
        tw += wi;
    }
    *total_weight = tw;
    if (reduction != 0) {
        double sum = 0.0;
        for (int64_t i = 0; i < N; ++i) {
            const int64_t ti = t[i];
            if (ti == ignore_index) continue;
            const float wi = w ? w[ti] : 1.0f;
            sum += (double)(-x[i * C + ti] * wi);
        }
        if (reduction == 1 && tw > 0) sum /= tw;
        out[0] = (float)sum;
    }
    return 0;
}

/* nll_loss_backward_kernel (LossKernels.cpp:57-101).  has_tw: total_weight is
 * defined (value tw); otherwise reduction 1 recomputes it in double.  Targets
 * outside [0, C) are skipped (the reference leaves them undefined). */
void or_nll_loss_backward(const float* g, const int64_t* t, const float* w, int64_t reduction,
                          int64_t ignore_index, int32_t has_tw, float tw_in, int64_t N, int64_t C, float* gi) {
    for (int64_t k = 0; k < N * C; ++k) gi[k] = 0.0f;
    double tw = 0.0;
    if (has_tw) {
        tw = tw_in;
    } else if (reduction == 1) {
        for (int64_t i = 0; i < N; ++i)
            if (t[i] != ignore_index) tw += w ? w[t[i]] : 1.0f;
    }
    float gv = g[0];
    if (reduction == 1 && tw > 0) gv = (float)((double)gv / tw);
    for (int64_t i = 0; i < N; ++i) {
        const int64_t ti = t[i];
        if (ti == ignore_index || ti < 0 || ti >= C) continue;
        const float wi = w ? w[ti] : 1.0f;
        gi[i * C + ti] = -wi * (reduction == 0 ? g[i] : gv);
    }
}
