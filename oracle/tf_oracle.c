/*
 * tf_oracle.c — CPU restatement of tensorforge's training hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or the timed CPU baseline), never as part of the product path.
 *
 * Every function restates one reference function in the reference's own
 * scalar loop order and float32 arithmetic (compile with -O2
 * -ffp-contract=off, no FMA), so that on the same inputs it reproduces the
 * reference bit for bit.  Citations are relative to the reference repository
 * root.  Functions for which the reference has no implementation say so and
 * state the rule they follow; their pinning is described in oracle/README.md.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Tensor::matmul (tensor/Tensor.cpp:354-362): single accumulator, k ascending. */
void orc_matmul(const float* a, const float* b, float* c, int64_t M, int64_t K, int64_t N) {
    for (int64_t i = 0; i < M; ++i) {
        for (int64_t j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int64_t k = 0; k < K; ++k) acc += a[i * K + k] * b[k * N + j];
            c[i * N + j] = acc;
        }
    }
}

/* Tensor::transpose for 2-D (tensor/Tensor.cpp:579-612): out[j][i] = in[i][j]. */
void orc_transpose2d(const float* in, float* out, int64_t R, int64_t C) {
    for (int64_t i = 0; i < R; ++i)
        for (int64_t j = 0; j < C; ++j) out[j * R + i] = in[i * C + j];
}

/* elementwise_cpu AddOp / MulOp (tensor/Tensor.cpp:33-69). */
void orc_add(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
void orc_mul(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

/* Tensor::relu / sigmoid / tanh forward (tensor/Tensor.cpp:227-301). */
void orc_relu_fwd(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}
/* Tensor::leaky_relu, CPU loop (tensor/Tensor.cpp:306-311): x > 0 ? x : alpha * x. */
void orc_leaky_relu_fwd(const float* x, float* y, int64_t n, float alpha) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : alpha * x[i];
}
void orc_sigmoid_fwd(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = 1.0f / (1.0f + expf(-x[i]));
}
void orc_tanh_fwd(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = tanhf(x[i]);
}

/* ReluBackward::apply (autograd/ops/ReluBackward.hpp:22-32): mask = (x > 0 ? 1 : 0),
 * then grads[0] * mask through operator* (dy * mask). */
void orc_relu_bwd(const float* dy, const float* x, float* dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float mask = x[i] > 0.0f ? 1.0f : 0.0f;
        dx[i] = dy[i] * mask;
    }
}

/* Sigmoid / Tanh backward.  NOT IMPLEMENTED in the reference: its wirers are
 * no-ops (autograd/TensorAutograd.cpp:152-164); the rule is the derivative
 * stated there, sigma' = y (1 - y), and tanh' = 1 - y^2, on the saved output. */
void orc_sigmoid_bwd(const float* dy, const float* y, float* dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = dy[i] * (y[i] * (1.0f - y[i]));
}
void orc_tanh_bwd(const float* dy, const float* y, float* dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = dy[i] * (1.0f - y[i] * y[i]);
}

/* Tensor::softmax (tensor/Tensor.cpp:370-409). */
void orc_softmax_fwd(const float* x, float* y, int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r) {
        const float* row = x + r * C;
        float* yr = y + r * C;
        float maxv = row[0];
        for (int64_t j = 1; j < C; ++j)
            if (row[j] > maxv) maxv = row[j];
        float sumv = 0.0f;
        for (int64_t j = 0; j < C; ++j) {
            yr[j] = expf(row[j] - maxv);
            sumv += yr[j];
        }
        float inv = 1.0f / sumv;
        for (int64_t j = 0; j < C; ++j) yr[j] *= inv;
    }
}

/* Tensor::log_softmax (tensor/Tensor.cpp:411-447). */
void orc_log_softmax_fwd(const float* x, float* y, int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r) {
        const float* row = x + r * C;
        float* yr = y + r * C;
        float maxv = row[0];
        for (int64_t j = 1; j < C; ++j)
            if (row[j] > maxv) maxv = row[j];
        float sum_exp = 0.0f;
        for (int64_t j = 0; j < C; ++j) sum_exp += expf(row[j] - maxv);
        float log_z = logf(sum_exp) + maxv;
        for (int64_t j = 0; j < C; ++j) yr[j] = row[j] - log_z;
    }
}

/* LogSoftmaxBackward::apply (autograd/ops/LogSoftmaxBackward.hpp:26-58):
 * sp = exp(y); s_r = sum_j gy (sequential); gx = gy - sp * s_r. */
void orc_log_softmax_bwd(const float* y, const float* gy, float* gx, int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < C; ++j) s += gy[r * C + j];
        for (int64_t j = 0; j < C; ++j) {
            int64_t idx = r * C + j;
            float sp = expf(y[idx]);
            gx[idx] = gy[idx] - sp * s;
        }
    }
}

/* SoftmaxBackward::apply (autograd/ops/SoftmaxBackward.hpp:27-55):
 * gyy = gy * y; s = sum(gyy, -1); diff = gy - s; gx = y * diff. */
void orc_softmax_bwd(const float* y, const float* gy, float* gx, int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < C; ++j) s += gy[r * C + j] * y[r * C + j];
        for (int64_t j = 0; j < C; ++j) {
            int64_t idx = r * C + j;
            float diff = gy[idx] - s;
            gx[idx] = y[idx] * diff;
        }
    }
}

/* The cross-entropy chain of examples/train_mlp.cpp:54-76 and its backward as
 * the reference engine runs it:
 *   y = log_softmax(logits); mask = onehot(labels) (labels outside [0,C) give
 *   an all-zero row); picked = y * mask; row_sum = sum(picked, 1) (sequential
 *   over j, Tensor.cpp:547-558); total = sum(row_sum, 0) (sequential over r);
 *   total_nll = (-1) * total; loss = total_nll * float(1/N).
 * Backward (seed 1): MulBackward gives d total_nll = 1 * n_inv; MulBackward
 * gives d total = (-1) * that; SumBackward broadcasts up[0]
 * (autograd/ops/SumBackward.hpp:35-37) twice, so d picked = that everywhere;
 * MulBackward gives d y = d picked * mask; LogSoftmaxBackward gives dlogits.
 * Writes loss[0] and dlogits[R*C]; y_out (may be NULL) receives y. */
void orc_ce_chain(const float* logits, const int64_t* labels, int64_t R, int64_t C, float* loss,
                  float* dlogits, float* y_out) {
    float* y = y_out ? y_out : (float*)malloc(sizeof(float) * (size_t)(R * C));
    float* mask = (float*)calloc((size_t)(R * C), sizeof(float));
    float* gy = (float*)malloc(sizeof(float) * (size_t)(R * C));
    orc_log_softmax_fwd(logits, y, R, C);
    for (int64_t i = 0; i < R; ++i) {
        int64_t t = labels[i];
        if (t >= 0 && t < C) mask[i * C + t] = 1.0f;
    }
    float total = 0.0f;
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < C; ++j) s += y[r * C + j] * mask[r * C + j];
        total += s;
    }
    const float neg_one = -1.0f;
    const float n_inv = (float)(1.0 / (double)R);
    float total_nll = neg_one * total;
    loss[0] = total_nll * n_inv;

    const float seed = 1.0f;
    float d_total_nll = seed * n_inv;         /* MulBackward: grads[0] * b */
    float d_total = neg_one * d_total_nll;    /* MulBackward: a * grads[0] */
    float d_row = d_total;                    /* SumBackward broadcast */
    float d_picked = d_row;                   /* SumBackward broadcast */
    for (int64_t i = 0; i < R * C; ++i) gy[i] = d_picked * mask[i];
    orc_log_softmax_bwd(y, gy, dlogits, R, C);
    free(gy);
    free(mask);
    if (!y_out) free(y);
}

/* Column sum db[c] = sum_r dy[r][c], rows ascending (the order of
 * Tensor::sum(0), tensor/Tensor.cpp:547-558).  The reference Linear has no
 * bias gradient (nn/Linear.cpp:60-63); this is the rule of the bias add. */
void orc_colsum(const float* dy, float* db, int64_t R, int64_t C) {
    for (int64_t c = 0; c < C; ++c) {
        float s = 0.0f;
        for (int64_t r = 0; r < R; ++r) s += dy[r * C + c];
        db[c] = s;
    }
}

/* Conv bias grad, loop order of nn/conv2d_backward_test.cpp:94-105. */
void orc_chansum_nchw(const float* dy, float* db, int64_t N, int64_t Cc, int64_t HW) {
    for (int64_t c = 0; c < Cc; ++c) db[c] = 0.0f;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < Cc; ++c)
            for (int64_t p = 0; p < HW; ++p) db[c] += dy[(n * Cc + c) * HW + p];
}

/* SGD with momentum.  The rule is nn/optim/SGD.hpp:3-6 and the operation order
 * nn/optim/SGD.cpp:50-56 (velocity * momentum + g; p - velocity * lr;
 * mu == 0: p - g * lr).  SGD::step itself throws for any non-scalar parameter
 * (its lr/momentum are Shape{1} tensors and operator* does not broadcast,
 * tensor/Tensor.cpp:131-133), so the runnable reference is the manual loop
 * p -= lr * g of examples/train_mlp.cpp:145-159, which mu == 0 reproduces. */
void orc_sgd_momentum(float* p, const float* g, float* v, int64_t n, float lr, float mu) {
    for (int64_t i = 0; i < n; ++i) {
        if (mu != 0.0f) {
            float vm = v[i] * mu;
            v[i] = vm + g[i];
            float step = v[i] * lr;
            p[i] = p[i] - step;
        } else {
            float step = g[i] * lr;
            p[i] = p[i] - step;
        }
    }
}

/* Tensor::layer_norm (tensor/Tensor.cpp:449-494): two-pass mean / variance. */
void orc_layernorm_fwd(const float* x, const float* gamma, const float* beta, float* y, float* mean,
                       float* rstd, int64_t R, int64_t C, float eps) {
    for (int64_t r = 0; r < R; ++r) {
        const float* row = x + r * C;
        float sum = 0.0f;
        for (int64_t j = 0; j < C; ++j) sum += row[j];
        float m = sum / (float)C;
        float var_sum = 0.0f;
        for (int64_t j = 0; j < C; ++j) {
            float d = row[j] - m;
            var_sum += d * d;
        }
        float v = var_sum / (float)C;
        float rs = 1.0f / sqrtf(v + eps);
        mean[r] = m;
        rstd[r] = rs;
        for (int64_t j = 0; j < C; ++j) y[r * C + j] = (row[j] - m) * rs * gamma[j] + beta[j];
    }
}

/* LayerNormBackward::apply as shipped (autograd/ops/LayerNormBackward.hpp:39-59):
 * dx = dy * gamma[col]; dgamma = dbeta = 0.  A known reference defect kept
 * for the reference-compatible mode. */
void orc_layernorm_bwd_stub(const float* dy, const float* gamma, float* dx, float* dgamma, float* dbeta,
                            int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r)
        for (int64_t j = 0; j < C; ++j) dx[r * C + j] = dy[r * C + j] * gamma[j];
    for (int64_t j = 0; j < C; ++j) {
        dgamma[j] = 0.0f;
        dbeta[j] = 0.0f;
    }
}

/* True LayerNorm gradient of the forward above, evaluated in double (the
 * reference ships only the stub).  xhat = (x - mean) * rstd, g = dy * gamma,
 * dx = rstd * (g - mean_j(g) - xhat * mean_j(g * xhat)),
 * dgamma = sum_r dy * xhat, dbeta = sum_r dy. */
void orc_layernorm_bwd(const float* x, const float* dy, const float* gamma, const float* mean,
                       const float* rstd, float* dx, float* dgamma, float* dbeta, int64_t R, int64_t C) {
    double* dg = (double*)calloc((size_t)C, sizeof(double));
    double* db = (double*)calloc((size_t)C, sizeof(double));
    for (int64_t r = 0; r < R; ++r) {
        double m = mean[r], rs = rstd[r];
        double s1 = 0.0, s2 = 0.0;
        for (int64_t j = 0; j < C; ++j) {
            double xh = ((double)x[r * C + j] - m) * rs;
            double g = (double)dy[r * C + j] * gamma[j];
            s1 += g;
            s2 += g * xh;
            dg[j] += (double)dy[r * C + j] * xh;
            db[j] += dy[r * C + j];
        }
        s1 /= (double)C;
        s2 /= (double)C;
        for (int64_t j = 0; j < C; ++j) {
            double xh = ((double)x[r * C + j] - m) * rs;
            double g = (double)dy[r * C + j] * gamma[j];
            dx[r * C + j] = (float)(rs * (g - s1 - xh * s2));
        }
    }
    for (int64_t j = 0; j < C; ++j) {
        dgamma[j] = (float)dg[j];
        dbeta[j] = (float)db[j];
    }
    free(dg);
    free(db);
}

/* im2col index map (cuda/kernels/im2col.cu:57-99):
 * col[n][c*kH*kW + ki*kW + kj][oh*outW + ow] = x[n][c][ih][iw] or 0,
 * ih = oh*sh + ki*dh - ph, iw = ow*sw + kj*dw - pw. */
void orc_im2col(const float* x, float* col, int64_t N, int64_t Cc, int64_t H, int64_t W, int64_t kH,
                int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
    int64_t outH = (H + 2 * ph - dh * (kH - 1) - 1) / sh + 1;
    int64_t outW = (W + 2 * pw - dw * (kW - 1) - 1) / sw + 1;
    int64_t rows = Cc * kH * kW, sp = outH * outW;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t row = 0; row < rows; ++row) {
            int64_t c = row / (kH * kW), rk = row % (kH * kW), ki = rk / kW, kj = rk % kW;
            for (int64_t o = 0; o < sp; ++o) {
                int64_t oh = o / outW, ow = o % outW;
                int64_t ih = oh * sh + ki * dh - ph, iw = ow * sw + kj * dw - pw;
                float v = 0.0f;
                if (ih >= 0 && ih < H && iw >= 0 && iw < W) v = x[((n * Cc + c) * H + ih) * W + iw];
                col[(n * rows + row) * sp + o] = v;
            }
        }
}

/* col2im scatter-add (cuda/kernels/col2im.cu:50-80), the adjoint of im2col:
 * dx[n][c][ih][iw] += col[...] for every in-bounds tap, in flat col order. */
void orc_col2im(const float* col, float* dx, int64_t N, int64_t Cc, int64_t H, int64_t W, int64_t kH,
                int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
    int64_t outH = (H + 2 * ph - dh * (kH - 1) - 1) / sh + 1;
    int64_t outW = (W + 2 * pw - dw * (kW - 1) - 1) / sw + 1;
    int64_t rows = Cc * kH * kW, sp = outH * outW;
    memset(dx, 0, sizeof(float) * (size_t)(N * Cc * H * W));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t row = 0; row < rows; ++row) {
            int64_t c = row / (kH * kW), rk = row % (kH * kW), ki = rk / kW, kj = rk % kW;
            for (int64_t o = 0; o < sp; ++o) {
                int64_t oh = o / outW, ow = o % outW;
                int64_t ih = oh * sh + ki * dh - ph, iw = ow * sw + kj * dw - pw;
                if (ih >= 0 && ih < H && iw >= 0 && iw < W)
                    dx[((n * Cc + c) * H + ih) * W + iw] += col[(n * rows + row) * sp + o];
            }
        }
}

/* cpu_conv2d (nn/Conv2dModule.cpp:26-70), square kernel generalised to kH, kW. */
void orc_conv2d_fwd(const float* in, const float* w, const float* bias, float* out, int64_t N, int64_t Cin,
                    int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t stride, int64_t pad,
                    int64_t dil) {
    int64_t outH = (H + 2 * pad - (dil * (kH - 1) + 1)) / stride + 1;
    int64_t outW = (W + 2 * pad - (dil * (kW - 1) + 1)) / stride + 1;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t co = 0; co < Cout; ++co)
            for (int64_t oh = 0; oh < outH; ++oh)
                for (int64_t ow = 0; ow < outW; ++ow) {
                    float acc = 0.0f;
                    for (int64_t ci = 0; ci < Cin; ++ci)
                        for (int64_t kh = 0; kh < kH; ++kh)
                            for (int64_t kw = 0; kw < kW; ++kw) {
                                int64_t ih = oh * stride - pad + kh * dil;
                                int64_t iw = ow * stride - pad + kw * dil;
                                if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                                acc += in[((n * Cin + ci) * H + ih) * W + iw] *
                                       w[((co * Cin + ci) * kH + kh) * kW + kw];
                            }
                    if (bias) acc += bias[co];
                    out[((n * Cout + co) * outH + oh) * outW + ow] = acc;
                }
}

/* ref_conv2d_backward (nn/conv2d_backward_test.cpp:50-106), the reference's
 * host loop for Conv2d::backward: scatter-add over (n, co, oh, ow, ci, ki, kj). */
void orc_conv2d_bwd(const float* in, const float* w, int has_bias, const float* gout, float* gin, float* gw,
                    float* gb, int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kH,
                    int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
    int64_t outH = (H + 2 * ph - dh * (kH - 1) - 1) / sh + 1;
    int64_t outW = (W + 2 * pw - dw * (kW - 1) - 1) / sw + 1;
    memset(gin, 0, sizeof(float) * (size_t)(N * Cin * H * W));
    memset(gw, 0, sizeof(float) * (size_t)(Cout * Cin * kH * kW));
    memset(gb, 0, sizeof(float) * (size_t)Cout);
    for (int64_t n = 0; n < N; ++n)
        for (int64_t co = 0; co < Cout; ++co)
            for (int64_t oh = 0; oh < outH; ++oh)
                for (int64_t ow = 0; ow < outW; ++ow) {
                    float go = gout[((n * Cout + co) * outH + oh) * outW + ow];
                    for (int64_t ci = 0; ci < Cin; ++ci)
                        for (int64_t ki = 0; ki < kH; ++ki)
                            for (int64_t kj = 0; kj < kW; ++kj) {
                                int64_t ih = oh * sh + ki * dh - ph;
                                int64_t iw = ow * sw + kj * dw - pw;
                                if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                                float kv = w[((co * Cin + ci) * kH + ki) * kW + kj];
                                gin[((n * Cin + ci) * H + ih) * W + iw] += go * kv;
                                gw[((co * Cin + ci) * kH + ki) * kW + kj] += go * in[((n * Cin + ci) * H + ih) * W + iw];
                            }
                }
    if (has_bias)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t co = 0; co < Cout; ++co)
                for (int64_t oh = 0; oh < outH; ++oh)
                    for (int64_t ow = 0; ow < outW; ++ow) gb[co] += gout[((n * Cout + co) * outH + oh) * outW + ow];
}

/* Tensor::sum along one dim (tensor/Tensor.cpp:513-561) on data viewed as
 * [outer][reduce][inner]: out[o][i] = sum_d x[o][d][i], d ascending from 0.0f. */
void orc_sum_dim(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner) {
    for (int64_t oi = 0; oi < outer * inner; ++oi) {
        const int64_t o = oi / inner, i = oi % inner;
        float s = 0.0f;
        for (int64_t d = 0; d < reduce; ++d) s += x[(o * reduce + d) * inner + i];
        out[oi] = s;
    }
}

/* nn::CrossEntropyLoss::forward (nn/CrossEntropyLoss.cpp:36-62): softmax
 * rows, p = probs[r][t_r] clamped below at 1e-9f, loss_r = -log(p), then
 * Tensor::mean (tensor/Tensor.cpp:562-576: sequential sum / n).  Returns -1
 * when a target lies outside [0, C) (the reference throws), else 0. */
int orc_ce_module(const float* logits, const int64_t* t, int64_t R, int64_t C, float* loss, float* probs) {
    orc_softmax_fwd(logits, probs, R, C);
    float s = 0.0f;
    for (int64_t r = 0; r < R; ++r) {
        if (t[r] < 0 || t[r] >= C) return -1;
        const float p = probs[r * C + t[r]];
        const float clamped = p < 1e-9f ? 1e-9f : p;
        s += -logf(clamped);
    }
    loss[0] = s / (float)R;
    return 0;
}

/* First-max argmax with strict '>' (examples/train_mlp.cpp:95-100). */
void orc_argmax_rows(const float* x, int64_t* out, int64_t R, int64_t C) {
    for (int64_t r = 0; r < R; ++r) {
        int64_t pred = 0;
        float maxv = -1e30f;
        for (int64_t c = 0; c < C; ++c) {
            float v = x[r * C + c];
            if (v > maxv) {
                maxv = v;
                pred = c;
            }
        }
        out[r] = pred;
    }
}

/* IEEE 754 binary16 <-> binary32.  The reference has no host function for
 * this: its 16-bit device paths convert with __half2float (exact) and
 * __float2half (round to nearest, ties to even), cuda/kernels/elementwise.cu
 * :42-64, col2im.cu:44, im2col.cu:133-150.  Written from the format's
 * definition (1 sign, 5 exponent bits biased by 15, 10 fraction bits;
 * subnormals k * 2^-24).  A NaN stays a NaN (made quiet, top fraction bits
 * kept); its payload is not part of any check. */
static uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xFFu;
    const uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0u));
    if (exp == 0u) return (uint16_t)sign; /* f32 subnormal or zero: below half of the smallest f16 subnormal */
    const int32_t e = (int32_t)exp - 127 + 15; /* biased f16 exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t q, rem, half;
    if (e >= 1) {
        /* normal: keep 10 of the 23 fraction bits; a carry out of the
         * fraction moves into the exponent (and to infinity at the top) */
        q = ((uint32_t)e << 10) | (man >> 13);
        rem = man & 0x1FFFu;
        half = 0x1000u;
    } else {
        /* subnormal result: value = M * 2^(exp - 150) = k * 2^-24 with
         * k = M >> (126 - exp), M the 24-bit significand */
        const uint32_t M = man | 0x800000u;
        const int s = 14 - e; /* 126 - exp, >= 14 */
        if (s > 25) return (uint16_t)sign;
        q = M >> s;
        rem = M & ((1u << s) - 1u);
        half = 1u << (s - 1);
    }
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

static float f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t man = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (exp == 0u) {
        const float v = ldexpf((float)man, -24); /* exact: at most 10 significant bits */
        memcpy(&x, &v, sizeof x);
        x |= sign;
    } else if (exp == 31u) {
        x = sign | 0x7F800000u | (man << 13);
    } else {
        x = sign | ((exp - 15u + 127u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, sizeof f);
    return f;
}

void orc_f32_to_f16(const float* x, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = f32_to_f16_rne(x[i]);
}
void orc_f16_to_f32(const uint16_t* h, float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = f16_to_f32(h[i]);
}
