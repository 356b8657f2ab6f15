/*
 * vdttfs_oracle.c -- CPU restatement of the reference VD-TTFS kernels.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); see the
 * header for the citation legend and what pins each function.  Compiled with
 * -ffp-contract=off: every fused multiply-add below is an explicit fmaf().
 */
#include "vdttfs_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define MAX_DELTA 1024

static int nthr(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

int orc_num_chunks(const orc_consts* c) { return (c->T + c->delta - 1) / c->delta; }

/* T1V:208-216 / T2V:236-243 */
void orc_build_luts(int T, float vth, float tc_i, float td_i, float tc_f, float td_f,
                    float* alpha, float* theta) {
    for (int t = 0; t <= T; ++t) alpha[t] = expf(-((float)t - td_i) / tc_i);
    for (int t = 0; t < T; ++t) theta[t] = vth * expf(-((float)t - td_f) / tc_f);
}

/* T1V:32-42 (nvcc contracts td - tc*logf(x) to one fma). */
void orc_encode_log(const float* img, float* out, int64_t n, float tc, float td, int T) {
    for (int64_t i = 0; i < n; ++i) {
        float pixel = img[i];
        if (pixel < 1e-5) { out[i] = ORC_INF; continue; }
        float tf = fmaf(-tc, logf(pixel), td);
        if (tf < 0.0f) tf = 0.0f;
        float ts = ceilf(tf);
        out[i] = (ts > (float)T) ? ORC_INF : ts;
    }
}

/* Configs' rule t = floor(T*(1-x)), with T1V:36's x<1e-5 -> no spike. */
void orc_encode_linear(const float* img, float* out, int64_t n, int T) {
    for (int64_t i = 0; i < n; ++i) {
        float x = img[i];
        if (x < 1e-5) { out[i] = ORC_INF; continue; }
        out[i] = floorf((float)T * (1.0f - x));
    }
}

/* tb rule shared by T1V:58-59 / T2V:59-60 and the integrators. */
static inline int bin_of(float t_in, float tfs) {
    int tb = (int)floorf(t_in - tfs);
    if (tb < 0) tb = 0;
    return tb;
}

/* T1V:45-80 / T2V:45-81 */
void orc_bucketize(const orc_consts* c, const float* in, int64_t n_cols, int c_in,
                   int32_t* out_cin, float* out_tin, int32_t* out_off, int nthreads) {
    const int T = c->T, D = c->delta, NC = orc_num_chunks(c), OS = NC + 1;
    const float tfs = c->tfs;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t col = 0; col < n_cols; ++col) {
        const float* src = in + col * (int64_t)c_in;
        int cnt[MAX_DELTA];
        for (int k = 0; k < NC; ++k) cnt[k] = 0;
        for (int i = 0; i < c_in; ++i) {
            float t_in = src[i];
            if (t_in < ORC_INF) {
                int tb = bin_of(t_in, tfs);
                if (tb < T) cnt[tb / D]++;
            }
        }
        int cursor[MAX_DELTA];
        int run = 0;
        for (int k = 0; k < NC; ++k) {
            out_off[col * OS + k] = run;
            cursor[k] = run;
            run += cnt[k];
        }
        out_off[col * OS + NC] = run;
        int32_t* dc = out_cin + col * (int64_t)c_in;
        float* dt = out_tin + col * (int64_t)c_in;
        for (int i = 0; i < c_in; ++i) {
            float t_in = src[i];
            if (t_in < ORC_INF) {
                int tb = bin_of(t_in, tfs);
                if (tb < T) {
                    int pos = cursor[tb / D]++;
                    dc[pos] = i;
                    dt[pos] = t_in;
                }
            }
        }
    }
}

static inline int alpha_index(const orc_consts* c, float t_in, int tb) {
    if (!c->alpha_by_time) return tb;          /* T1V:128,144 */
    int ti = (int)t_in;                         /* T2V:132,150 */
    if (ti < 0) ti = 0;
    else if (ti > c->T) ti = c->T;
    return ti;
}

/* neuron index decode, c_out fastest (T1V:98-109) */
static inline void decode(int64_t nid, int is_fc, int H_out, int W_out, int C_out, int* c_out,
                          int* img, int* h_out, int* w_out) {
    *c_out = (int)(nid % C_out);
    if (is_fc) {
        *img = (int)(nid / C_out);
        *h_out = 0;
        *w_out = 0;
    } else {
        int64_t t1 = nid / C_out;
        *w_out = (int)(t1 % W_out);
        int64_t t2 = t1 / W_out;
        *h_out = (int)(t2 % H_out);
        *img = (int)(t2 / H_out);
    }
}

/* T1V:83-162 / T2V:84-170, E_proc as T2M:99,136,155,170-176 */
void orc_integrate(const orc_consts* c, float* out,
                   const int32_t* bcin, const float* btin, const int32_t* boff,
                   const float* W, const float* bias, const float* alpha, const float* theta,
                   int t_min, int B, int H_in, int W_in, int C_in,
                   int H_out, int W_out, int C_out, int K_h, int K_w, int pad_h, int pad_w, int is_fc,
                   int no_early_exit, uint64_t* eproc, uint64_t* ebin, int nthreads) {
    const int T = c->T, D = c->delta, NC = orc_num_chunks(c), OS = NC + 1;
    const float tfs = c->tfs;
    const int64_t total = (int64_t)B * H_out * W_out * C_out;
    uint64_t sum_proc = 0, sum_bin = 0;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static) reduction(+ : sum_proc, sum_bin)
    for (int64_t nid = 0; nid < total; ++nid) {
        int c_out, img, h_out, w_out;
        decode(nid, is_fc, H_out, W_out, C_out, &c_out, &img, &h_out, &w_out);
        float carry = bias[c_out];
        float result = ORC_INF;
        int first_cross = -1;          /* bin of the first threshold crossing */
        uint64_t my_proc = 0;
        uint64_t bins_cnt[MAX_DELTA];  /* per-bin event count within the current chunk */
        uint64_t my_bin = 0;
        float delta[MAX_DELTA];
        for (int tau = 0; tau < NC; ++tau) {
            for (int i = 0; i < D; ++i) { delta[i] = 0.0f; bins_cnt[i] = 0; }
            int base_t = tau * D;
            if (is_fc) {
                int64_t col = img;
                int s = boff[col * OS + tau], e = boff[col * OS + tau + 1];
                const int32_t* bc = bcin + col * (int64_t)C_in;
                const float* bt = btin + col * (int64_t)C_in;
                for (int idx = s; idx < e; ++idx) {
                    int cin = bc[idx];
                    float t_in = bt[idx];
                    int tb = bin_of(t_in, tfs);
                    float a = alpha[alpha_index(c, t_in, tb)];
                    delta[tb - base_t] = fmaf(W[(int64_t)cin * C_out + c_out], a, delta[tb - base_t]);
                    ++my_proc;
                    bins_cnt[tb - base_t]++;
                }
            } else {
                for (int kh = 0; kh < K_h; ++kh) {
                    int h_in = h_out - pad_h + kh;
                    if (h_in < 0 || h_in >= H_in) continue;
                    for (int kw = 0; kw < K_w; ++kw) {
                        int w_in = w_out - pad_w + kw;
                        if (w_in < 0 || w_in >= W_in) continue;
                        int64_t col = ((int64_t)img * H_in + h_in) * W_in + w_in;
                        int s = boff[col * OS + tau], e = boff[col * OS + tau + 1];
                        const int32_t* bc = bcin + col * (int64_t)C_in;
                        const float* bt = btin + col * (int64_t)C_in;
                        int64_t wbase = (int64_t)(kh * K_w + kw) * C_in;
                        for (int idx = s; idx < e; ++idx) {
                            int cin = bc[idx];
                            float t_in = bt[idx];
                            int tb = bin_of(t_in, tfs);
                            float a = alpha[alpha_index(c, t_in, tb)];
                            delta[tb - base_t] =
                                fmaf(W[(wbase + cin) * C_out + c_out], a, delta[tb - base_t]);
                            ++my_proc;
                            bins_cnt[tb - base_t]++;
                        }
                    }
                }
            }
            /* T1V:150-157 / T2V:158-165 */
            int crossed_i = -1;
            for (int i = 0; i < D; ++i) {
                int t = base_t + i;
                if (t >= T) break;
                carry = carry + delta[i];
                float th = theta[t];
                if (t >= t_min && carry >= th && th >= 1e-5f) {
                    result = (float)t;
                    crossed_i = i;
                    break;
                }
            }
            if (first_cross < 0) {
                int last = crossed_i >= 0 ? crossed_i : D - 1;
                for (int i = 0; i <= last; ++i) my_bin += bins_cnt[i];
                if (crossed_i >= 0) first_cross = base_t + crossed_i;
            }
            /* T1V:158 / T2V:166.  Under T2M's NOEARLYEXIT (T2M:170-172) the
             * chunk loop runs on and a crossing in a later chunk overwrites
             * result, exactly as the reference does. */
            if (!no_early_exit && result < ORC_INF) break;
        }
        out[nid] = result;
        sum_proc += my_proc;
        sum_bin += my_bin;
    }
    if (eproc) *eproc = sum_proc;
    if (ebin) *ebin = sum_bin;
}

/* Brute force, time-driven: the step-by-step view of T1S:47-102 applied to
 * the VD-TTFS neuron (per-bin fma order (kh,kw) outer, cin ascending). */
void orc_integrate_timedriven(const orc_consts* c, float* out, const float* spikes,
                              const float* W, const float* bias, const float* alpha,
                              const float* theta, int t_min, int B, int H_in, int W_in,
                              int C_in, int H_out, int W_out, int C_out, int K_h, int K_w,
                              int pad_h, int pad_w, int is_fc, int nthreads) {
    const int T = c->T;
    const float tfs = c->tfs;
    const int64_t total = (int64_t)B * H_out * W_out * C_out;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t nid = 0; nid < total; ++nid) {
        int c_out, img, h_out, w_out;
        decode(nid, is_fc, H_out, W_out, C_out, &c_out, &img, &h_out, &w_out);
        float carry = bias[c_out];
        float result = ORC_INF;
        for (int t = 0; t < T && result == ORC_INF; ++t) {
            float acc = 0.0f;
            int kh_n = is_fc ? 1 : K_h, kw_n = is_fc ? 1 : K_w;
            for (int kh = 0; kh < kh_n; ++kh) {
                int h_in = is_fc ? 0 : h_out - pad_h + kh;
                if (h_in < 0 || h_in >= (is_fc ? 1 : H_in)) continue;
                for (int kw = 0; kw < kw_n; ++kw) {
                    int w_in = is_fc ? 0 : w_out - pad_w + kw;
                    if (w_in < 0 || w_in >= (is_fc ? 1 : W_in)) continue;
                    int64_t col = is_fc ? img : ((int64_t)img * H_in + h_in) * W_in + w_in;
                    const float* src = spikes + col * (int64_t)C_in;
                    int64_t wbase = is_fc ? 0 : (int64_t)(kh * K_w + kw) * C_in;
                    for (int cin = 0; cin < C_in; ++cin) {
                        float t_in = src[cin];
                        if (!(t_in < ORC_INF)) continue;
                        int tb = bin_of(t_in, tfs);
                        if (tb != t) continue;
                        float a = alpha[alpha_index(c, t_in, tb)];
                        acc = fmaf(W[(wbase + cin) * C_out + c_out], a, acc);
                    }
                }
            }
            carry = carry + acc;
            float th = theta[t];
            if (t >= t_min && carry >= th && th >= 1e-5f) result = (float)t;
        }
        out[nid] = result;
    }
}

void orc_integrate_margin(const orc_consts* c, double* margin, const float* spikes,
                          const float* W, const float* bias, const float* alpha,
                          const float* theta, int t_min, int B, int H_in, int W_in,
                          int C_in, int H_out, int W_out, int C_out, int K_h, int K_w,
                          int pad_h, int pad_w, int is_fc, int nthreads) {
    const int T = c->T;
    const float tfs = c->tfs;
    const int64_t total = (int64_t)B * H_out * W_out * C_out;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t nid = 0; nid < total; ++nid) {
        int c_out, img, h_out, w_out;
        decode(nid, is_fc, H_out, W_out, C_out, &c_out, &img, &h_out, &w_out);
        float carry = bias[c_out];
        double carry_d = (double)bias[c_out];
        double scale = fabs((double)bias[c_out]);
        double m = INFINITY;
        int fired = 0;
        /* scale first: sum |w*alpha| over the whole receptive field */
        int kh_n = is_fc ? 1 : K_h, kw_n = is_fc ? 1 : K_w;
        for (int kh = 0; kh < kh_n; ++kh) {
            int h_in = is_fc ? 0 : h_out - pad_h + kh;
            if (h_in < 0 || h_in >= (is_fc ? 1 : H_in)) continue;
            for (int kw = 0; kw < kw_n; ++kw) {
                int w_in = is_fc ? 0 : w_out - pad_w + kw;
                if (w_in < 0 || w_in >= (is_fc ? 1 : W_in)) continue;
                int64_t col = is_fc ? img : ((int64_t)img * H_in + h_in) * W_in + w_in;
                const float* src = spikes + col * (int64_t)C_in;
                int64_t wbase = is_fc ? 0 : (int64_t)(kh * K_w + kw) * C_in;
                for (int cin = 0; cin < C_in; ++cin) {
                    float t_in = src[cin];
                    if (!(t_in < ORC_INF)) continue;
                    int tb = bin_of(t_in, tfs);
                    if (tb >= T) continue;
                    scale += fabs((double)W[(wbase + cin) * C_out + c_out] *
                                  (double)alpha[alpha_index(c, t_in, tb)]);
                }
            }
        }
        if (scale == 0.0) scale = 1.0;
        for (int t = 0; t < T && !fired; ++t) {
            float acc = 0.0f;
            double acc_d = 0.0;
            for (int kh = 0; kh < kh_n; ++kh) {
                int h_in = is_fc ? 0 : h_out - pad_h + kh;
                if (h_in < 0 || h_in >= (is_fc ? 1 : H_in)) continue;
                for (int kw = 0; kw < kw_n; ++kw) {
                    int w_in = is_fc ? 0 : w_out - pad_w + kw;
                    if (w_in < 0 || w_in >= (is_fc ? 1 : W_in)) continue;
                    int64_t col = is_fc ? img : ((int64_t)img * H_in + h_in) * W_in + w_in;
                    const float* src = spikes + col * (int64_t)C_in;
                    int64_t wbase = is_fc ? 0 : (int64_t)(kh * K_w + kw) * C_in;
                    for (int cin = 0; cin < C_in; ++cin) {
                        float t_in = src[cin];
                        if (!(t_in < ORC_INF)) continue;
                        int tb = bin_of(t_in, tfs);
                        if (tb != t) continue;
                        float w = W[(wbase + cin) * C_out + c_out];
                        float a = alpha[alpha_index(c, t_in, tb)];
                        acc = fmaf(w, a, acc);
                        acc_d += (double)w * (double)a;
                    }
                }
            }
            carry = carry + acc;
            carry_d += acc_d;
            float th = theta[t];
            if (t >= t_min && th >= 1e-5f) {
                double d = fabs(carry_d - (double)th) / scale;
                if (d < m) m = d;
                if (carry >= th) fired = 1;
            }
        }
        margin[nid] = m;
    }
}

/* T1V:164-181 / T2V:192-209 */
void orc_pool_min(const float* in, float* out, int B, int H_in, int W_in, int C, int nthreads) {
    const int H_out = H_in / 2, W_out = W_in / 2;
    const int64_t total = (int64_t)B * H_out * W_out * C;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int64_t per = (int64_t)H_out * W_out * C;
        int64_t b = idx / per;
        int64_t local = idx % per;
        int ch_ = (int)(local % C);
        int w = (int)((local / C) % W_out);
        int h = (int)(local / C / W_out);
        float min_t = ORC_INF;
        for (int i = 0; i < 2; ++i)
            for (int j = 0; j < 2; ++j) {
                int hh = h * 2 + i, ww = w * 2 + j;
                if (hh < H_in && ww < W_in) {
                    float t = in[b * ((int64_t)H_in * W_in * C) + ((int64_t)hh * W_in + ww) * C + ch_];
                    if (t < min_t) min_t = t;
                }
            }
        out[idx] = min_t;
    }
}

/* T2V:172-190 */
void orc_fc_vmem(const orc_consts* c, const float* in, float* out, const float* W,
                 const float* bias, const float* alpha, int B, int C_in, int C_out) {
    const int T = c->T;
    for (int64_t id = 0; id < (int64_t)B * C_out; ++id) {
        int img = (int)(id / C_out), c_out = (int)(id % C_out);
        float acc = 0.0f;
        for (int i = 0; i < C_in; ++i) {
            float t_in = in[(int64_t)img * C_in + i];
            if (t_in < ORC_INF && (t_in - c->tfs) <= (float)T) {
                int ti = (int)t_in;
                if (ti < 0) ti = 0;
                else if (ti > T) ti = T;
                acc = fmaf(W[(int64_t)i * C_out + c_out], alpha[ti], acc);
            }
        }
        out[id] = acc + bias[c_out];
    }
}

void orc_readout_argmin(const float* out, int B, int C, int32_t* pred) {
    for (int b = 0; b < B; ++b) {
        float m = ORC_INF;
        int p = -1;
        for (int i = 0; i < C; ++i) {
            float t = out[(int64_t)b * C + i];
            if (t < m) { m = t; p = i; }
        }
        pred[b] = p;
    }
}

void orc_readout_argmax(const float* out, int B, int C, int32_t* pred) {
    for (int b = 0; b < B; ++b) {
        float m = -1e9f;
        int p = -1;
        for (int i = 0; i < C; ++i) {
            float v = out[(int64_t)b * C + i];
            if (v > m) { m = v; p = i; }
        }
        pred[b] = p;
    }
}

void orc_readout_t3(const float* out, int B, int C, int32_t* pred) {
    for (int b = 0; b < B; ++b) {
        int p = 0;
        float m = out[(int64_t)b * C];
        for (int i = 1; i < C; ++i)
            if (out[(int64_t)b * C + i] < m) { m = out[(int64_t)b * C + i]; p = i; }
        pred[b] = p;
    }
}

static int64_t layer_out_elems(const orc_layer* L, int B) {
    return (int64_t)B * L->H_out * L->W_out * L->C_out;
}

/* Driver sequencing: T1V:286-319 / T2V:337-396.  LUT for layer l uses the
 * previous integrating layer's fire constants (T2V:343-384). */
int orc_net_forward(const orc_consts* c, const orc_layer* layers, int n_layers, int B,
                    const float* img, int64_t img_elems_per_image, int encode_mode,
                    float tc_in, float td_in, int readout,
                    float** layer_outs, float* final_out, int32_t* pred,
                    uint64_t* eproc, uint64_t* ebin, int nthreads) {
    if (n_layers <= 0) return -1;
    const int NC = orc_num_chunks(c), OS = NC + 1;
    int64_t max_elems = (int64_t)B * img_elems_per_image, max_cols = 0, max_bkt = 0;
    for (int l = 0; l < n_layers; ++l) {
        const orc_layer* L = &layers[l];
        int64_t in_e = (int64_t)B * L->H_in * L->W_in * L->C_in;
        int64_t oe = layer_out_elems(L, B);
        if (in_e > max_elems) max_elems = in_e;
        if (oe > max_elems) max_elems = oe;
        int64_t cols = (L->kind == ORC_CONV) ? (int64_t)B * L->H_in * L->W_in : B;
        if (cols > max_cols) max_cols = cols;
        if (in_e > max_bkt) max_bkt = in_e;
    }
    float* cur = (float*)malloc(sizeof(float) * max_elems);
    float* nxt = (float*)malloc(sizeof(float) * max_elems);
    int32_t* bcin = (int32_t*)malloc(sizeof(int32_t) * max_bkt);
    float* btin = (float*)malloc(sizeof(float) * max_bkt);
    int32_t* boff = (int32_t*)malloc(sizeof(int32_t) * max_cols * OS);
    float* alpha = (float*)malloc(sizeof(float) * (c->T + 1));
    float* theta = (float*)malloc(sizeof(float) * (c->T > 0 ? c->T : 1));
    if (!cur || !nxt || !bcin || !btin || !boff || !alpha || !theta) {
        free(cur); free(nxt); free(bcin); free(btin); free(boff); free(alpha); free(theta);
        return -2;
    }
    int64_t n_img = (int64_t)B * img_elems_per_image;
    if (encode_mode == ORC_ENC_LOG) orc_encode_log(img, cur, n_img, tc_in, td_in, c->T);
    else if (encode_mode == ORC_ENC_TIMES) memcpy(cur, img, sizeof(float) * (size_t)n_img);
    else orc_encode_linear(img, cur, n_img, c->T);

    float tc_i = tc_in, td_i = td_in;
    int rc = 0;
    for (int l = 0; l < n_layers && rc == 0; ++l) {
        const orc_layer* L = &layers[l];
        if (L->kind == ORC_POOL) {
            orc_pool_min(cur, nxt, B, L->H_in, L->W_in, L->C_in, nthreads);
        } else {
            orc_build_luts(c->T, c->vth, tc_i, td_i, L->tc_fire, L->td, alpha, theta);
            int t_min = (int)ceilf(L->td);
            if (t_min < 0) t_min = 0;
            if (L->kind == ORC_VMEM) {
                orc_fc_vmem(c, cur, nxt, L->W, L->bias, alpha, B, L->C_in, L->C_out);
            } else {
                int is_fc = (L->kind == ORC_FC);
                int64_t cols = is_fc ? B : (int64_t)B * L->H_in * L->W_in;
                int cin = is_fc ? L->H_in * L->W_in * L->C_in : L->C_in;
                orc_bucketize(c, cur, cols, cin, bcin, btin, boff, nthreads);
                uint64_t ep = 0, eb = 0;
                orc_integrate(c, nxt, bcin, btin, boff, L->W, L->bias, alpha, theta, t_min, B,
                              is_fc ? 1 : L->H_in, is_fc ? 1 : L->W_in, cin,
                              is_fc ? 1 : L->H_out, is_fc ? 1 : L->W_out, L->C_out,
                              is_fc ? 1 : L->K_h, is_fc ? 1 : L->K_w, L->pad_h, L->pad_w, is_fc, 0, &ep, &eb,
                              nthreads);
                if (eproc) eproc[l] = ep;
                if (ebin) ebin[l] = eb;
            }
            tc_i = L->tc_fire;
            td_i = L->td;
        }
        if (layer_outs && layer_outs[l])
            memcpy(layer_outs[l], nxt, sizeof(float) * layer_out_elems(L, B));
        float* tmp = cur; cur = nxt; nxt = tmp;
    }
    const orc_layer* last = &layers[n_layers - 1];
    int C_last = last->H_out * last->W_out * last->C_out;
    if (final_out) memcpy(final_out, cur, sizeof(float) * layer_out_elems(last, B));
    if (pred) {
        if (readout == ORC_READ_ARGMAX) orc_readout_argmax(cur, B, C_last, pred);
        else if (readout == ORC_READ_T3) orc_readout_t3(cur, B, C_last, pred);
        else orc_readout_argmin(cur, B, C_last, pred);
    }
    free(cur); free(nxt); free(bcin); free(btin); free(boff); free(alpha); free(theta);
    return rc;
}

/* ----------------------- step-by-step baselines (T1S, T2S) ------------------ */

/* Number of global steps: T (T1S:229) or, for T2S, until the last weighted
 * layer's integration window [ (D-1)*tfs, (D-1)*tfs + T ) has passed
 * (TIME_STEPS = 680 for 16 weighted layers, tfs 40, T 80; T2S:13). */
static int step_count(const orc_consts* c, const orc_layer* layers, int n_layers, int mode) {
    if (mode == 1) return c->T;
    int D = 0;
    for (int l = 0; l < n_layers; ++l)
        if (layers[l].kind != ORC_POOL) ++D;
    return (int)ceilf((float)(D - 1) * c->tfs + (float)c->T);
}

int orc_stepnet_forward(const orc_consts* c, const orc_layer* layers, int n_layers, int B,
                        const float* img, int64_t img_elems_per_image, int encode_mode,
                        float tc_in, float td_in, int mode, float* final_out, int32_t* pred,
                        int* steps_out, int nthreads) {
    if (n_layers <= 0 || (mode != 1 && mode != 2)) return -1;
    const int T = c->T;
    const int64_t n_img = (int64_t)B * img_elems_per_image;
    float* tin = (float*)malloc(sizeof(float) * n_img);
    unsigned char* s0 = (unsigned char*)calloc(n_img, 1);
    unsigned char** spk = (unsigned char**)calloc(n_layers, sizeof(void*));
    unsigned char** fired = (unsigned char**)calloc(n_layers, sizeof(void*));
    float** vmem = (float**)calloc(n_layers, sizeof(void*));
    int* depth = (int*)calloc(n_layers, sizeof(int));
    float *tci = (float*)calloc(n_layers, sizeof(float)), *tdi = (float*)calloc(n_layers, sizeof(float));
    int last_w = -1;
    int rc = 0;
    if (!tin || !s0 || !spk || !fired || !vmem || !depth || !tci || !tdi) rc = -2;
    if (encode_mode == ORC_ENC_LOG) orc_encode_log(img, tin, n_img, tc_in, td_in, T);
    else orc_encode_linear(img, tin, n_img, T);
    {
        int d = 0;
        float tc = tc_in, td = td_in;
        for (int l = 0; l < n_layers && rc == 0; ++l) {
            const orc_layer* L = &layers[l];
            int64_t n = layer_out_elems(L, B);
            spk[l] = (unsigned char*)calloc(n, 1);
            fired[l] = (unsigned char*)calloc(n, 1);
            if (!spk[l] || !fired[l]) rc = -2;
            if (L->kind != ORC_POOL) {
                vmem[l] = (float*)calloc(n, sizeof(float));
                if (!vmem[l]) rc = -2;
                depth[l] = ++d;
                tci[l] = tc;
                tdi[l] = td;
                tc = L->tc_fire;
                td = L->td;
                last_w = l;
            }
        }
    }
    const int steps = step_count(c, layers, n_layers, mode);
    if (steps_out) *steps_out = steps;
    const orc_layer* LL = &layers[n_layers - 1];
    const int64_t n_out = layer_out_elems(LL, B);
    for (int64_t i = 0; i < n_out && rc == 0; ++i) final_out[i] = (mode == 1) ? ORC_INF : -1e9f;
    if (rc == 0 && last_w != n_layers - 1) rc = -3; /* the readout layer must be a weighted layer */

    for (int t = 0; t < steps && rc == 0; ++t) {
        for (int64_t i = 0; i < n_img; ++i) s0[i] = (tin[i] == (float)t);
        const unsigned char* s_in = s0;
        for (int l = 0; l < n_layers; ++l) {
            const orc_layer* L = &layers[l];
            const int64_t n = layer_out_elems(L, B);
            unsigned char* so = spk[l];
            unsigned char* fr = fired[l];
            if (L->kind == ORC_POOL) {
                const int Ho = L->H_in / 2, Wo = L->W_in / 2, C = L->C_in;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
                for (int64_t idx = 0; idx < n; ++idx) {
                    if (fr[idx]) { so[idx] = 0; continue; }
                    int ch = (int)(idx % C), w = (int)((idx / C) % Wo), h = (int)((idx / C / Wo) % Ho);
                    int64_t b = idx / ((int64_t)C * Wo * Ho);
                    so[idx] = 0;
                    for (int i = 0; i < 2 && !so[idx]; ++i)
                        for (int j = 0; j < 2; ++j) {
                            int hi = h * 2 + i, wi = w * 2 + j;
                            if (hi < L->H_in && wi < L->W_in &&
                                s_in[((b * L->H_in + hi) * L->W_in + wi) * C + ch]) {
                                so[idx] = 1;
                                fr[idx] = 1;
                                break;
                            }
                        }
                }
            } else {
                const int is_fc = (L->kind != ORC_CONV);
                const int out_layer = (l == n_layers - 1);
                const int d = depth[l];
                int int_ok, fire_ok;
                float kv, th;
                if (mode == 1) {
                    int t_min = (int)ceilf(L->td);
                    if (t_min < 0) t_min = 0;
                    kv = expf(-((float)t - tdi[l]) / tci[l]);
                    th = c->vth * expf(-((float)t - L->td) / L->tc_fire);
                    int_ok = 1;
                    fire_ok = t >= t_min;
                } else {
                    float t_integ = (float)t - (float)(d - 1) * c->tfs;
                    float t_fire = (float)t - (float)d * c->tfs;
                    float start = L->td > 0.0f ? ceilf(L->td) : 0.0f;
                    kv = expf(-(t_integ - tdi[l]) / tci[l]);
                    th = c->vth * expf(-(t_fire - L->td) / L->tc_fire);
                    int_ok = t_integ >= 0.0f && t_integ < (float)T;
                    fire_ok = t_fire >= start && t_fire < (float)T;
                }
                const int cin_tot = is_fc ? L->H_in * L->W_in * L->C_in : L->C_in;
                float* V = vmem[l];
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
                for (int64_t nid = 0; nid < n; ++nid) {
                    const int keep_max = (mode == 2 && out_layer);
                    if (!keep_max && fr[nid]) { so[nid] = 0; continue; }
                    int co, im, ho, wo;
                    decode(nid, is_fc, is_fc ? 1 : L->H_out, is_fc ? 1 : L->W_out, L->C_out, &co, &im, &ho, &wo);
                    if (int_ok) {
                        float psp = 0.0f;
                        if (is_fc) {
                            const unsigned char* src = s_in + (int64_t)im * cin_tot;
                            for (int ci = 0; ci < cin_tot; ++ci)
                                if (src[ci]) {
                                    float w = L->W[(int64_t)ci * L->C_out + co];
                                    psp = (mode == 1) ? psp + w : fmaf(w, kv, psp);
                                }
                        } else {
                            for (int kh = 0; kh < L->K_h; ++kh) {
                                int hi = ho - L->pad_h + kh;
                                if (hi < 0 || hi >= L->H_in) continue;
                                for (int kw = 0; kw < L->K_w; ++kw) {
                                    int wi = wo - L->pad_w + kw;
                                    if (wi < 0 || wi >= L->W_in) continue;
                                    const unsigned char* src =
                                        s_in + (((int64_t)im * L->H_in + hi) * L->W_in + wi) * L->C_in;
                                    int64_t wb = (int64_t)(kh * L->K_w + kw) * L->C_in;
                                    for (int ci = 0; ci < L->C_in; ++ci)
                                        if (src[ci]) {
                                            float w = L->W[(wb + ci) * L->C_out + co];
                                            psp = (mode == 1) ? psp + w : fmaf(w, kv, psp);
                                        }
                                }
                            }
                        }
                        V[nid] = (mode == 1) ? fmaf(psp, kv, V[nid]) : V[nid] + psp;
                    }
                    so[nid] = 0;
                    if (keep_max) {
                        if (int_ok) {
                            float v = V[nid] + L->bias[co];
                            if (v > final_out[nid]) final_out[nid] = v;
                        }
                    } else if (fire_ok) {
                        if (V[nid] + L->bias[co] >= th && th >= 1e-5f) {
                            so[nid] = 1;
                            fr[nid] = 1;
                            if (mode == 1 && out_layer && final_out[nid] >= ORC_INF) final_out[nid] = (float)t;
                        }
                    }
                }
            }
            s_in = so;
        }
    }
    if (rc == 0 && pred) {
        int C_last = LL->H_out * LL->W_out * LL->C_out;
        if (mode == 1) orc_readout_argmin(final_out, B, C_last, pred);
        else orc_readout_argmax(final_out, B, C_last, pred);
    }
    for (int l = 0; l < n_layers; ++l) {
        if (spk) free(spk[l]);
        if (fired) free(fired[l]);
        if (vmem) free(vmem[l]);
    }
    free(tin); free(s0); free(spk); free(fired); free(vmem); free(depth); free(tci); free(tdi);
    return rc;
}

/* ------------------------------- CuLIF (T3V) ------------------------------ */

/* One chunk of the CuLIF neuron: T3V:58-62 (I = I*decay + in, V += I). */
static inline int lif_chunk(float* I, float* V, const float* in_val, int D, float decay,
                            float th) {
    for (int t = 0; t < D; ++t) {
        *I = fmaf(*I, decay, in_val[t]);
        *V = *V + *I;
        if (*V >= th) return t;
    }
    return -1;
}

/* T3V:30-65 */
void orc_culif_conv1_raw(const float* data, float* out, const float* weight, int N, int C_in,
                         int C_out, int H, int W, int T, int delta, float decay, float th,
                         int nthreads) {
    const int64_t total = (int64_t)N * C_out * H * W;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int64_t n = idx / ((int64_t)C_out * H * W), rem = idx % ((int64_t)C_out * H * W);
        int c_out = (int)(rem / (H * W)), y = (int)((rem / W) % H), x = (int)(rem % W);
        float I = 0.0f, V = 0.0f, res = ORC_INF;
        for (int chunk = 0; chunk < T && res == ORC_INF; chunk += delta) {
            float in_val[MAX_DELTA];
            for (int t = 0; t < delta; ++t) in_val[t] = 0.0f;
            for (int ci = 0; ci < C_in; ++ci)
                for (int ky = 0; ky < 3; ++ky) {
                    int iy = y + ky - 1;
                    if (iy < 0 || iy >= H) continue;
                    for (int kx = 0; kx < 3; ++kx) {
                        int ix = x + kx - 1;
                        if (ix < 0 || ix >= W) continue;
                        float w = weight[(((int64_t)c_out * C_in + ci) * 3 + ky) * 3 + kx];
                        const float* dv = data + ((((n * C_in + ci) * H + iy) * W + ix) * (int64_t)T) + chunk;
                        for (int t = 0; t < delta; ++t) in_val[t] = fmaf(w, dv[t], in_val[t]);
                    }
                }
            int f = lif_chunk(&I, &V, in_val, delta, decay, th);
            if (f >= 0) res = (float)(chunk + f);
        }
        out[idx] = res;
    }
}

/* T3V:70-90 */
void orc_culif_bucketize_nchw(const float* in, int N, int C, int H, int W, int T, int delta,
                              int32_t* out_cin, float* out_tin, int32_t* out_off, int nthreads) {
    const int NC = (T + delta - 1) / delta, OS = NC + 1;
    const int64_t sites = (int64_t)N * H * W;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t site = 0; site < sites; ++site) {
        int64_t n = site / (H * W), hw = site % (H * W);
        int64_t base = n * C * H * W + hw;
        int cnt[MAX_DELTA], cur[MAX_DELTA];
        for (int k = 0; k < NC; ++k) cnt[k] = 0;
        for (int ch = 0; ch < C; ++ch) {
            float tf = in[base + (int64_t)ch * H * W];
            if (tf < ORC_INF) { int tb = (int)tf; if (tb >= 0 && tb < T) cnt[tb / delta]++; }
        }
        int run = 0;
        for (int k = 0; k < NC; ++k) { out_off[site * OS + k] = run; cur[k] = run; run += cnt[k]; }
        out_off[site * OS + NC] = run;
        int32_t* dc = out_cin + site * C;
        float* dt = out_tin + site * C;
        for (int ch = 0; ch < C; ++ch) {
            float tf = in[base + (int64_t)ch * H * W];
            if (tf < ORC_INF) {
                int tb = (int)tf;
                if (tb >= 0 && tb < T) { int p = cur[tb / delta]++; dc[p] = ch; dt[p] = tf; }
            }
        }
    }
}

/* T3V:93-106 */
void orc_culif_bucketize_fc(const float* in, int N, int F, int T, int delta,
                            int32_t* out_cin, float* out_tin, int32_t* out_off, int nthreads) {
    const int NC = (T + delta - 1) / delta, OS = NC + 1;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int n = 0; n < N; ++n) {
        const float* src = in + (int64_t)n * F;
        int cnt[MAX_DELTA], cur[MAX_DELTA];
        for (int k = 0; k < NC; ++k) cnt[k] = 0;
        for (int j = 0; j < F; ++j) {
            float tf = src[j];
            if (tf < ORC_INF) { int tb = (int)tf; if (tb >= 0 && tb < T) cnt[tb / delta]++; }
        }
        int run = 0;
        for (int k = 0; k < NC; ++k) { out_off[(int64_t)n * OS + k] = run; cur[k] = run; run += cnt[k]; }
        out_off[(int64_t)n * OS + NC] = run;
        int32_t* dc = out_cin + (int64_t)n * F;
        float* dt = out_tin + (int64_t)n * F;
        for (int j = 0; j < F; ++j) {
            float tf = src[j];
            if (tf < ORC_INF) {
                int tb = (int)tf;
                if (tb >= 0 && tb < T) { int p = cur[tb / delta]++; dc[p] = j; dt[p] = tf; }
            }
        }
    }
}

/* T3V:109-143 */
void orc_culif_conv(const int32_t* bcin, const float* btin, const int32_t* boff, float* out,
                    const float* weight, int N, int C_in, int C_out, int H, int W, int T,
                    int delta, float decay, float th, int nthreads) {
    const int NC = (T + delta - 1) / delta, OS = NC + 1;
    const int64_t total = (int64_t)N * C_out * H * W;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int64_t n = idx / ((int64_t)C_out * H * W), rem = idx % ((int64_t)C_out * H * W);
        int c_out = (int)(rem / (H * W)), y = (int)((rem / W) % H), x = (int)(rem % W);
        float I = 0.0f, V = 0.0f, res = ORC_INF;
        int64_t w_out_base = (int64_t)c_out * C_in * 9;
        for (int ch = 0; ch < NC && res == ORC_INF; ++ch) {
            int base_t = ch * delta;
            float in_val[MAX_DELTA];
            for (int t = 0; t < delta; ++t) in_val[t] = 0.0f;
            for (int ky = 0; ky < 3; ++ky) {
                int iy = y + ky - 1;
                if (iy < 0 || iy >= H) continue;
                for (int kx = 0; kx < 3; ++kx) {
                    int ix = x + kx - 1;
                    if (ix < 0 || ix >= W) continue;
                    int64_t site = (n * H + iy) * W + ix;
                    int s = boff[site * OS + ch], e = boff[site * OS + ch + 1];
                    const int32_t* sc = bcin + site * C_in;
                    const float* st = btin + site * C_in;
                    int64_t wk = w_out_base + ky * 3 + kx;
                    for (int p = s; p < e; ++p) {
                        int cin = sc[p];
                        int tt = (int)st[p];
                        in_val[tt - base_t] = in_val[tt - base_t] + weight[wk + (int64_t)cin * 9];
                    }
                }
            }
            int f = lif_chunk(&I, &V, in_val, delta, decay, th);
            if (f >= 0) res = (float)(base_t + f);
        }
        out[idx] = res;
    }
}

/* T3V:146-168 */
void orc_culif_pool(const float* in, float* out, int N, int C, int H_in, int W_in, int T,
                    int delta, float decay, float th, int nthreads) {
    const int H_out = H_in / 2, W_out = W_in / 2;
    const int64_t total = (int64_t)N * C * H_out * W_out;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int64_t n = idx / ((int64_t)C * H_out * W_out), rem = idx % ((int64_t)C * H_out * W_out);
        int ch = (int)(rem / (H_out * W_out)), yo = (int)((rem / W_out) % H_out), xo = (int)(rem % W_out);
        float I = 0.0f, V = 0.0f, res = ORC_INF;
        int64_t base = (n * C + ch) * (int64_t)H_in * W_in;
        for (int chunk = 0; chunk < T && res == ORC_INF; chunk += delta) {
            float in_val[MAX_DELTA];
            for (int t = 0; t < delta; ++t) in_val[t] = 0.0f;
            for (int dy = 0; dy < 2; ++dy)
                for (int dx = 0; dx < 2; ++dx) {
                    float tf = in[base + (int64_t)(yo * 2 + dy) * W_in + (xo * 2 + dx)];
                    if (tf >= chunk && tf < chunk + delta) in_val[(int)tf - chunk] = 1.0f;
                }
            int f = lif_chunk(&I, &V, in_val, delta, decay, th);
            if (f >= 0) res = (float)(chunk + f);
        }
        out[idx] = res;
    }
}

/* T3V:171-200 */
void orc_culif_fc_recurrent(const int32_t* bcin, const float* btin, const int32_t* boff,
                            float* out, const float* w, const float* w_rec, int N, int in_f,
                            int out_f, int T, int delta, float decay, float th, int nthreads) {
    const int NC = (T + delta - 1) / delta, OS = NC + 1;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int n = 0; n < N; ++n) {
        float* I = (float*)calloc((size_t)out_f, sizeof(float));
        float* V = (float*)calloc((size_t)out_f, sizeof(float));
        float* my_fire = (float*)malloc(sizeof(float) * out_f);
        unsigned char* has_fired = (unsigned char*)calloc((size_t)out_f, 1);
        unsigned char* fired_prev = (unsigned char*)calloc((size_t)out_f, 1);
        unsigned char* fire_now = (unsigned char*)calloc((size_t)out_f, 1);
        float* in_ff = (float*)malloc(sizeof(float) * (size_t)out_f * delta);
        for (int i = 0; i < out_f; ++i) my_fire[i] = ORC_INF;
        const int32_t* sc = bcin + (int64_t)n * in_f;
        const float* st = btin + (int64_t)n * in_f;
        for (int ch = 0; ch < NC; ++ch) {
            int base_t = ch * delta;
            int s = boff[(int64_t)n * OS + ch], e = boff[(int64_t)n * OS + ch + 1];
            for (int i = 0; i < out_f; ++i) {
                float* f = in_ff + (int64_t)i * delta;
                for (int t = 0; t < delta; ++t) f[t] = 0.0f;
                for (int p = s; p < e; ++p) {
                    int j = sc[p];
                    int tt = (int)st[p];
                    f[tt - base_t] = f[tt - base_t] + w[(int64_t)i * in_f + j];
                }
            }
            for (int t = 0; t < delta; ++t) {
                /* between the two barriers every neuron reads fired_prev */
                for (int i = 0; i < out_f; ++i) {
                    float in_rec = 0.0f;
                    for (int j = 0; j < out_f; ++j)
                        if (fired_prev[j]) in_rec = in_rec + w_rec[(int64_t)i * out_f + j];
                    I[i] = fmaf(I[i], decay, in_ff[(int64_t)i * delta + t]) + in_rec;
                    V[i] = V[i] + I[i];
                    fire_now[i] = 0;
                    if (V[i] >= th && !has_fired[i]) {
                        fire_now[i] = 1;
                        has_fired[i] = 1;
                        my_fire[i] = (float)(base_t + t);
                        V[i] = -10000.0f;
                    }
                }
                for (int i = 0; i < out_f; ++i) fired_prev[i] = fire_now[i];
            }
        }
        for (int i = 0; i < out_f; ++i) out[(int64_t)n * out_f + i] = my_fire[i];
        free(I); free(V); free(my_fire); free(has_fired); free(fired_prev); free(fire_now); free(in_ff);
    }
}

/* T3V:203-225 */
void orc_culif_fc(const int32_t* bcin, const float* btin, const int32_t* boff, float* out,
                  const float* w, int N, int in_f, int out_f, int T, int delta, float decay,
                  float th, int nthreads) {
    const int NC = (T + delta - 1) / delta, OS = NC + 1;
    const int64_t total = (int64_t)N * out_f;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int n = (int)(idx / out_f), i = (int)(idx % out_f);
        float I = 0.0f, V = 0.0f, res = ORC_INF;
        const int32_t* sc = bcin + (int64_t)n * in_f;
        const float* st = btin + (int64_t)n * in_f;
        for (int ch = 0; ch < NC && res == ORC_INF; ++ch) {
            int base_t = ch * delta;
            float in_val[MAX_DELTA];
            for (int t = 0; t < delta; ++t) in_val[t] = 0.0f;
            int s = boff[(int64_t)n * OS + ch], e = boff[(int64_t)n * OS + ch + 1];
            for (int p = s; p < e; ++p) {
                int j = sc[p];
                int tt = (int)st[p];
                in_val[tt - base_t] = in_val[tt - base_t] + w[(int64_t)i * in_f + j];
            }
            int f = lif_chunk(&I, &V, in_val, delta, decay, th);
            if (f >= 0) res = (float)(base_t + f);
        }
        out[idx] = res;
    }
}

float orc_culif_neuron_steps(const float* in, int T, float decay, float th) {
    float I = 0.0f, V = 0.0f;
    for (int t = 0; t < T; ++t) {
        I = fmaf(I, decay, in[t]);
        V = V + I;
        if (V >= th) return (float)t;
    }
    return ORC_INF;
}

/* ---- T3S: step-by-step CuLIF baseline ---------------------------------- */
static int64_t culif_out_elems(const orc_culif_layer* L, int N) {
    if (L->kind == ORC_CULIF_FC || L->kind == ORC_CULIF_FC_REC) return (int64_t)N * L->C_out;
    if (L->kind == ORC_CULIF_POOL) return (int64_t)N * L->C_in * (L->H_in / 2) * (L->W_in / 2);
    return (int64_t)N * L->C_out * L->H_in * L->W_in;
}

/* conv2d_kernel (T3S:41-68) at step t; raw: the input is data[site*T + t]. */
static void s3_conv(const orc_culif_layer* L, int N, const float* in, int raw, int T, int t, float* cur,
                    int nthreads) {
    const int C_in = L->C_in, C_out = L->C_out, H = L->H_in, W = L->W_in;
    const int64_t total = (int64_t)N * C_out * H * W;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        const int x = (int)(idx % W), y = (int)((idx / W) % H);
        const int co = (int)((idx / ((int64_t)W * H)) % C_out);
        const int64_t n = idx / ((int64_t)C_out * H * W);
        float sum = 0.0f;
        for (int c = 0; c < C_in; ++c)
            for (int ky = 0; ky < 3; ++ky)
                for (int kx = 0; kx < 3; ++kx) {
                    const int iy = y + ky - 1, ix = x + kx - 1;
                    if (iy < 0 || iy >= H || ix < 0 || ix >= W) continue;
                    const int64_t site = ((n * C_in + c) * H + iy) * (int64_t)W + ix;
                    const float v = raw ? in[site * T + t] : in[site];
                    sum = fmaf(v, L->w[(((int64_t)co * C_in + c) * 3 + ky) * 3 + kx], sum);
                }
        cur[idx] = sum;
    }
}

/* maxpool2d_kernel (T3S:70-94) */
static void s3_pool(const orc_culif_layer* L, int N, const float* in, float* cur, int nthreads) {
    const int C = L->C_in, H_in = L->H_in, W_in = L->W_in, H_out = H_in / 2, W_out = W_in / 2;
    const int64_t total = (int64_t)N * C * H_out * W_out;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        const int xo = (int)(idx % W_out), yo = (int)((idx / W_out) % H_out);
        const int c = (int)((idx / ((int64_t)W_out * H_out)) % C);
        const int64_t n = idx / ((int64_t)C * H_out * W_out);
        float m = -1e9f;
        for (int dy = 0; dy < 2; ++dy)
            for (int dx = 0; dx < 2; ++dx)
                m = fmaxf(m, in[((n * C + c) * H_in + (yo * 2 + dy)) * (int64_t)W_in + (xo * 2 + dx)]);
        cur[idx] = m;
    }
}

/* fc_kernel (T3S:96-109): cur[row][col] = sum_i in[row][i] * w[col][i]; with
 * add = 1 the sum is added to cur afterwards (add_tensors_kernel, T3S:111-114). */
static void s3_fc(const float* in, const float* w, float* cur, int N, int in_f, int out_f, int add,
                  int nthreads) {
    const int64_t total = (int64_t)N * out_f;
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t row = idx / out_f;
        const int col = (int)(idx % out_f);
        float sum = 0.0f;
        for (int i = 0; i < in_f; ++i) sum = fmaf(in[row * in_f + i], w[(int64_t)col * in_f + i], sum);
        cur[idx] = add ? cur[idx] + sum : sum;
    }
}

/* cuif_step_kernel (T3S:119-140) */
static void s3_neuron(const float* cur, float* I, float* V, float* spk, unsigned char* fired, float* ft,
                      int64_t n, float decay, float th, int t) {
    for (int64_t i = 0; i < n; ++i) {
        const float ci = fmaf(I[i], decay, cur[i]);
        const float cv = V[i] + ci;
        I[i] = ci;
        V[i] = cv;
        if (!fired[i] && cv >= th) {
            spk[i] = 1.0f;
            fired[i] = 1;
            ft[i] = (float)t;
        } else {
            spk[i] = 0.0f;
        }
    }
}

int orc_culif_stepnet_forward(const orc_culif_layer* layers, int n_layers, int N, const float* data,
                              int T, float** layer_outs, float* final_out, int32_t* pred, int nthreads) {
    if (n_layers <= 0 || N <= 0 || T <= 0 || layers[0].kind != ORC_CULIF_RAW_CONV) return -1;
    for (int l = 0; l < n_layers; ++l) {
        const orc_culif_layer* L = &layers[l];
        if (L->kind < ORC_CULIF_RAW_CONV || L->kind > ORC_CULIF_FC || (l > 0 && L->kind == ORC_CULIF_RAW_CONV))
            return -1;
        if (L->kind != ORC_CULIF_POOL && !L->w) return -1;
        if (L->kind == ORC_CULIF_FC_REC && !L->w_rec) return -1;
        if (l > 0) {
            const int64_t prev = culif_out_elems(&layers[l - 1], N) / N;
            const int64_t need = (int64_t)L->C_in * L->H_in * L->W_in;
            if (prev != need) return -1;
        }
    }
    float** cur = (float**)calloc(n_layers, sizeof(float*));
    float** I = (float**)calloc(n_layers, sizeof(float*));
    float** V = (float**)calloc(n_layers, sizeof(float*));
    float** spk = (float**)calloc(n_layers, sizeof(float*));
    float** ft = (float**)calloc(n_layers, sizeof(float*));
    unsigned char** fired = (unsigned char**)calloc(n_layers, sizeof(void*));
    int rc = (!cur || !I || !V || !spk || !ft || !fired) ? -2 : 0;
    for (int l = 0; l < n_layers && rc == 0; ++l) {
        const int64_t n = culif_out_elems(&layers[l], N);
        cur[l] = (float*)calloc(n, sizeof(float));
        I[l] = (float*)calloc(n, sizeof(float));
        V[l] = (float*)calloc(n, sizeof(float));
        spk[l] = (float*)calloc(n, sizeof(float));
        ft[l] = (float*)malloc(sizeof(float) * n);
        fired[l] = (unsigned char*)calloc(n, 1);
        if (!cur[l] || !I[l] || !V[l] || !spk[l] || !ft[l] || !fired[l]) rc = -2;
        else
            for (int64_t i = 0; i < n; ++i) ft[l][i] = ORC_INF;
    }
    for (int t = 0; t < T && rc == 0; ++t) {
        const float* in = NULL;
        for (int l = 0; l < n_layers; ++l) {
            const orc_culif_layer* L = &layers[l];
            const int64_t n = culif_out_elems(L, N);
            switch (L->kind) {
                case ORC_CULIF_RAW_CONV: s3_conv(L, N, data, 1, T, t, cur[l], nthreads); break;
                case ORC_CULIF_CONV: s3_conv(L, N, in, 0, T, t, cur[l], nthreads); break;
                case ORC_CULIF_POOL: s3_pool(L, N, in, cur[l], nthreads); break;
                case ORC_CULIF_FC: s3_fc(in, L->w, cur[l], N, L->C_in, L->C_out, 0, nthreads); break;
                default: /* FC_REC: spk[l] still holds step t-1 */
                    s3_fc(in, L->w, cur[l], N, L->C_in, L->C_out, 0, nthreads);
                    s3_fc(spk[l], L->w_rec, cur[l], N, L->C_out, L->C_out, 1, nthreads);
                    break;
            }
            s3_neuron(cur[l], I[l], V[l], spk[l], fired[l], ft[l], n, L->decay, L->th, t);
            in = spk[l];
        }
    }
    if (rc == 0) {
        const orc_culif_layer* last = &layers[n_layers - 1];
        const int64_t n = culif_out_elems(last, N);
        for (int l = 0; l < n_layers; ++l)
            if (layer_outs && layer_outs[l])
                memcpy(layer_outs[l], ft[l], sizeof(float) * (size_t)culif_out_elems(&layers[l], N));
        if (final_out) memcpy(final_out, ft[n_layers - 1], sizeof(float) * (size_t)n);
        if (pred) orc_readout_t3(ft[n_layers - 1], N, (int)(n / N), pred);
    }
    for (int l = 0; l < n_layers; ++l) {
        if (cur) free(cur[l]);
        if (I) free(I[l]);
        if (V) free(V[l]);
        if (spk) free(spk[l]);
        if (ft) free(ft[l]);
        if (fired) free(fired[l]);
    }
    free(cur); free(I); free(V); free(spk); free(ft); free(fired);
    return rc;
}
