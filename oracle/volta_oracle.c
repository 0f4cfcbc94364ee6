/*
 * volta_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A single-threaded CPU restatement of the algorithms that Volta (rlarson20/Volta,
 * Rust) runs on its CPU path for Conv2d (Direct / Im2col / iGEMM + auto-select),
 * ConvTranspose2d, the matmul behind Linear, and PixelShuffle.  Each function cites
 * the reference file:line it follows (paths relative to the reference root).
 *
 * It exists to CHECK the HIP library, never to be shipped or measured as the
 * product: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.  The product path (volta_amd / libvolta_hip.so) never calls it.
 *
 * Arithmetic is f32 with the reference's accumulation order wherever the reference
 * fixes one (scalar loops).  Where the reference delegates to a third-party crate
 * (`matrixmultiply` 0.3.10 sgemm, src/ops/matmul.rs:100-123) the order is not
 * pinned by the reference; or_matmul uses a plain i-k-j loop with one f32
 * accumulator per output element in ascending k (documented stand-in).
 *
 * Every function is pinned by tests/test_oracle.py against the reference's own
 * known-answer tests, closed forms (all-ones convs), adjointness identities,
 * cross-algorithm equalities and float64 library routines on small inputs.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef ptrdiff_t isz;

/* ---------------------------------------------------------------------------
 * ConvAlgo::auto_select -- src/nn/layers/conv.rs:29-69.
 * Returns 0 = Direct, 1 = Im2col, 2 = IGEMM; -1 if height/width < kernel_size
 * (the reference subtracts usize values there, conv.rs:42-43, which panics in a
 * debug build).
 * ------------------------------------------------------------------------- */
int or_auto_select(size_t batch, size_t channels, size_t height, size_t width,
                   size_t kernel_size, int has_gpu) {
    const size_t max_im2col = 5000000; /* conv.rs:38 */
    if (height < kernel_size || width < kernel_size) return -1;
    size_t h_out = (height - kernel_size) + 1;
    size_t w_out = (width - kernel_size) + 1;
    size_t e = batch * h_out * w_out * channels * kernel_size * kernel_size;
    if (has_gpu) return e > 1000000 ? 2 : 1;           /* conv.rs:46-54 */
    if (e > max_im2col) return 0;                       /* conv.rs:55-57 */
    if (kernel_size <= 3 && batch <= 4) return 0;       /* conv.rs:58-60 */
    if (e > 1000000) return 2;                          /* conv.rs:61-64 */
    return 1;                                           /* conv.rs:65-67 */
}

/* ---------------------------------------------------------------------------
 * Direct convolution forward -- conv.rs:1305-1436 (hot loop 1359-1419).
 * One f32 accumulator per output, order ic -> kh -> kw, padding skipped.
 * ------------------------------------------------------------------------- */
void or_direct_conv(const float *x, const float *w, float *y, size_t B, size_t C,
                    size_t O, size_t H, size_t W, size_t KH, size_t KW, size_t SH,
                    size_t SW, size_t PH, size_t PW) {
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    for (size_t b = 0; b < B; ++b)
        for (size_t oc = 0; oc < O; ++oc)
            for (size_t oh = 0; oh < HO; ++oh)
                for (size_t ow = 0; ow < WO; ++ow) {
                    float sum = 0.0f;
                    for (size_t ic = 0; ic < C; ++ic)
                        for (size_t kh = 0; kh < KH; ++kh)
                            for (size_t kw = 0; kw < KW; ++kw) {
                                isz ih = (isz)(oh * SH + kh) - (isz)PH;
                                isz iw = (isz)(ow * SW + kw) - (isz)PW;
                                if (ih >= 0 && ih < (isz)H && iw >= 0 && iw < (isz)W)
                                    sum += x[((b * C + ic) * H + (size_t)ih) * W + (size_t)iw] *
                                           w[((oc * C + ic) * KH + kh) * KW + kw];
                            }
                    y[((b * O + oc) * HO + oh) * WO + ow] = sum;
                }
}

/* Smallest oh with oh*S > t - K (i.e. t - oh*S < K), clamped at 0. */
static size_t first_out(isz t, size_t K, size_t S) {
    isz lo = t - (isz)K + 1; /* need oh*S >= lo */
    if (lo <= 0) return 0;
    return (size_t)((lo + (isz)S - 1) / (isz)S);
}

/* ---------------------------------------------------------------------------
 * Direct conv input gradient -- DirectConvGradFn::compute_input_gradient_cpu,
 * conv.rs:427-518 (hot loop 450-515).  The reference scans every (oc, oh, ow)
 * and adds only the in-receptive-field terms, in ascending oc -> oh -> ow order.
 * This restatement visits exactly those terms in the same order (it skips the
 * out-of-field ones arithmetically instead of testing them), so the f32 sum is
 * bit-identical while the cost drops from O(B*C*H*W*O*HO*WO) to
 * O(B*C*H*W*O*KH*KW/(SH*SW)).
 * ------------------------------------------------------------------------- */
void or_direct_conv_backward_input(const float *dy, const float *w, float *dx,
                                   size_t B, size_t C, size_t O, size_t H, size_t W,
                                   size_t KH, size_t KW, size_t SH, size_t SW,
                                   size_t PH, size_t PW) {
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    for (size_t b = 0; b < B; ++b)
        for (size_t ic = 0; ic < C; ++ic)
            for (size_t ih = 0; ih < H; ++ih)
                for (size_t iw = 0; iw < W; ++iw) {
                    float sum = 0.0f;
                    isz th = (isz)ih + (isz)PH, tw = (isz)iw + (isz)PW;
                    size_t oh0 = first_out(th, KH, SH), ow0 = first_out(tw, KW, SW);
                    for (size_t oc = 0; oc < O; ++oc)
                        for (size_t oh = oh0; oh < HO && (isz)(oh * SH) <= th; ++oh)
                            for (size_t ow = ow0; ow < WO && (isz)(ow * SW) <= tw; ++ow) {
                                size_t kh = (size_t)(th - (isz)(oh * SH));
                                size_t kw = (size_t)(tw - (isz)(ow * SW));
                                sum += dy[((b * O + oc) * HO + oh) * WO + ow] *
                                       w[((oc * C + ic) * KH + kh) * KW + kw];
                            }
                    dx[((b * C + ic) * H + ih) * W + iw] = sum;
                }
}

/* Literal O(B*C*H*W*O*HO*WO) form of conv.rs:450-515, for tiny shapes only; the
 * tests use it to show or_direct_conv_backward_input is bit-identical. */
void or_direct_conv_backward_input_literal(const float *dy, const float *w, float *dx,
                                           size_t B, size_t C, size_t O, size_t H,
                                           size_t W, size_t KH, size_t KW, size_t SH,
                                           size_t SW, size_t PH, size_t PW) {
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    for (size_t b = 0; b < B; ++b)
        for (size_t ic = 0; ic < C; ++ic)
            for (size_t ih = 0; ih < H; ++ih)
                for (size_t iw = 0; iw < W; ++iw) {
                    float sum = 0.0f;
                    for (size_t oc = 0; oc < O; ++oc)
                        for (size_t oh = 0; oh < HO; ++oh)
                            for (size_t ow = 0; ow < WO; ++ow) {
                                isz ho = (isz)ih - (isz)(oh * SH) + (isz)PH;
                                isz wo = (isz)iw - (isz)(ow * SW) + (isz)PW;
                                if (ho >= 0 && wo >= 0 && ho < (isz)KH && wo < (isz)KW)
                                    sum += dy[((b * O + oc) * HO + oh) * WO + ow] *
                                           w[((oc * C + ic) * KH + (size_t)ho) * KW + (size_t)wo];
                            }
                    dx[((b * C + ic) * H + ih) * W + iw] = sum;
                }
}

/* ---------------------------------------------------------------------------
 * Direct conv weight gradient -- compute_weight_gradient_cpu, conv.rs:522-609
 * (hot loop 544-606): order b -> oc -> oh -> ow -> ic -> kh -> kw, so each dW
 * element accumulates over (b, oh, ow) ascending.
 * ------------------------------------------------------------------------- */
void or_direct_conv_backward_weight(const float *dy, const float *x, float *dw,
                                    size_t B, size_t C, size_t O, size_t H, size_t W,
                                    size_t KH, size_t KW, size_t SH, size_t SW,
                                    size_t PH, size_t PW) {
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    memset(dw, 0, sizeof(float) * O * C * KH * KW);
    for (size_t b = 0; b < B; ++b)
        for (size_t oc = 0; oc < O; ++oc)
            for (size_t oh = 0; oh < HO; ++oh)
                for (size_t ow = 0; ow < WO; ++ow) {
                    float dout = dy[((b * O + oc) * HO + oh) * WO + ow];
                    for (size_t ic = 0; ic < C; ++ic)
                        for (size_t kh = 0; kh < KH; ++kh)
                            for (size_t kw = 0; kw < KW; ++kw) {
                                isz ih = (isz)(oh * SH + kh) - (isz)PH;
                                isz iw = (isz)(ow * SW + kw) - (isz)PW;
                                if (ih >= 0 && ih < (isz)H && iw >= 0 && iw < (isz)W)
                                    dw[((oc * C + ic) * KH + kh) * KW + kw] +=
                                        x[((b * C + ic) * H + (size_t)ih) * W + (size_t)iw] * dout;
                            }
                }
}

/* Bias gradient of Conv2d: bias is reshaped to [1,O,1,1] and expanded to
 * [B,O,HO,WO] (conv.rs:1915-1926); the expand backward sums dY in linear index
 * order into db[o] (movement.rs:441-485). */
void or_conv_bias_grad(const float *dy, float *db, size_t B, size_t O, size_t HO,
                       size_t WO) {
    memset(db, 0, sizeof(float) * O);
    for (size_t b = 0; b < B; ++b)
        for (size_t o = 0; o < O; ++o)
            for (size_t i = 0; i < HO * WO; ++i) db[o] += dy[(b * O + o) * HO * WO + i];
}

/* ---------------------------------------------------------------------------
 * Zero padding -- RawTensor::pad with [(0,0),(0,0),(PH,PH),(PW,PW)],
 * src/ops/movement.rs:848-990, as called from conv.rs:1862-1866.
 * ------------------------------------------------------------------------- */
void or_pad(const float *x, float *xp, size_t B, size_t C, size_t H, size_t W,
            size_t PH, size_t PW) {
    size_t HP = H + 2 * PH, WP = W + 2 * PW;
    memset(xp, 0, sizeof(float) * B * C * HP * WP);
    for (size_t bc = 0; bc < B * C; ++bc)
        for (size_t h = 0; h < H; ++h)
            memcpy(xp + (bc * HP + h + PH) * WP + PW, x + (bc * H + h) * W, sizeof(float) * W);
}

/* Pad backward: crop (movement.rs:486-530 restated as the adjoint of or_pad). */
void or_pad_backward(const float *gp, float *g, size_t B, size_t C, size_t H,
                     size_t W, size_t PH, size_t PW) {
    size_t HP = H + 2 * PH, WP = W + 2 * PW;
    for (size_t bc = 0; bc < B * C; ++bc)
        for (size_t h = 0; h < H; ++h)
            memcpy(g + (bc * H + h) * W, gp + (bc * HP + h + PH) * WP + PW, sizeof(float) * W);
}

/* ---------------------------------------------------------------------------
 * im2col on an already padded input -- Conv2d::im2col, conv.rs:1119-1239
 * (hot loop 1190-1224): row = (b, oh, ow), col = (c, kh, kw).
 * ------------------------------------------------------------------------- */
void or_im2col(const float *x, float *col, size_t B, size_t C, size_t H, size_t W,
               size_t KH, size_t KW, size_t SH, size_t SW) {
    size_t HO = (H - KH) / SH + 1, WO = (W - KW) / SW + 1, cols = C * KH * KW;
    for (size_t b = 0; b < B; ++b)
        for (size_t oh = 0; oh < HO; ++oh)
            for (size_t ow = 0; ow < WO; ++ow) {
                size_t row = (b * HO + oh) * WO + ow;
                for (size_t c = 0; c < C; ++c)
                    for (size_t kh = 0; kh < KH; ++kh)
                        for (size_t kw = 0; kw < KW; ++kw)
                            col[row * cols + (c * KH + kh) * KW + kw] =
                                x[((b * C + c) * H + oh * SH + kh) * W + ow * SW + kw];
            }
}

/* col2im -- Conv2d::col2im, conv.rs:1242-1298: scatter-add in the same loop order. */
void or_col2im(const float *col, float *x, size_t B, size_t C, size_t H, size_t W,
               size_t KH, size_t KW, size_t SH, size_t SW) {
    size_t HO = (H - KH) / SH + 1, WO = (W - KW) / SW + 1, cols = C * KH * KW;
    memset(x, 0, sizeof(float) * B * C * H * W);
    for (size_t b = 0; b < B; ++b)
        for (size_t oh = 0; oh < HO; ++oh)
            for (size_t ow = 0; ow < WO; ++ow) {
                size_t row = (b * HO + oh) * WO + ow;
                for (size_t c = 0; c < C; ++c)
                    for (size_t kh = 0; kh < KH; ++kh)
                        for (size_t kw = 0; kw < KW; ++kw)
                            x[((b * C + c) * H + oh * SH + kh) * W + ow * SW + kw] +=
                                col[row * cols + (c * KH + kh) * KW + kw];
            }
}

/* ---------------------------------------------------------------------------
 * matmul_raw -- src/ops/matmul.rs:56-124: C[m,n] = A[m,k] B[k,n], row-major,
 * alpha 1 beta 0.  The reference calls matrixmultiply::sgemm (third-party,
 * 0.3.10, not vendored); its blocking/FMA order is not pinned by the reference,
 * so this stand-in keeps one f32 accumulator per C element over ascending k.
 * ------------------------------------------------------------------------- */
void or_matmul(const float *a, const float *b, float *c, size_t m, size_t k, size_t n) {
    float *acc = (float *)calloc(n, sizeof(float));
    for (size_t i = 0; i < m; ++i) {
        memset(acc, 0, sizeof(float) * n);
        for (size_t p = 0; p < k; ++p) {
            float av = a[i * k + p];
            const float *brow = b + p * n;
            for (size_t j = 0; j < n; ++j) acc[j] += av * brow[j];
        }
        memcpy(c + i * n, acc, sizeof(float) * n);
    }
    free(acc);
}

/* transpose_2d -- matmul.rs:34-49. */
void or_transpose(const float *a, float *at, size_t m, size_t n) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) at[j * m + i] = a[i * n + j];
}

/* MatMulGradFn 2-D CPU branch, matmul.rs:450-460: dA[m,k] = G[m,n] . B[k,n]^T
 * (the reference materialises B^T, then sgemm). */
void or_matmul_backward_a(const float *g, const float *b, float *da, size_t m,
                          size_t k, size_t n) {
    float *bt = (float *)malloc(sizeof(float) * k * n);
    or_transpose(b, bt, k, n);
    or_matmul(g, bt, da, m, n, k);
    free(bt);
}

/* MatMulGradFn 2-D CPU branch, matmul.rs:563-574: dB[k,n] = A[m,k]^T . G[m,n]. */
void or_matmul_backward_b(const float *a, const float *g, float *db, size_t m,
                          size_t k, size_t n) {
    float *at = (float *)malloc(sizeof(float) * m * k);
    or_transpose(a, at, m, k);
    or_matmul(at, g, db, k, m, n);
    free(at);
}

/* ---------------------------------------------------------------------------
 * Im2col convolution forward -- Conv2d::forward Im2col arm, conv.rs:1858-1908:
 * pad -> im2col -> col[M, CKK] . (W reshaped [O, CKK], permuted to [CKK, O])
 * -> reshape [B,HO,WO,O] -> permute [0,3,1,2].
 * ------------------------------------------------------------------------- */
void or_im2col_conv_forward(const float *x, const float *w, float *y, size_t B,
                            size_t C, size_t O, size_t H, size_t W, size_t KH,
                            size_t KW, size_t SH, size_t SW, size_t PH, size_t PW) {
    size_t HP = H + 2 * PH, WP = W + 2 * PW;
    size_t HO = (HP - KH) / SH + 1, WO = (WP - KW) / SW + 1;
    size_t M = B * HO * WO, K = C * KH * KW;
    float *xp = (float *)malloc(sizeof(float) * B * C * HP * WP);
    float *col = (float *)malloc(sizeof(float) * M * K);
    float *wt = (float *)malloc(sizeof(float) * K * O);
    float *out = (float *)malloc(sizeof(float) * M * O);
    or_pad(x, xp, B, C, H, W, PH, PW);
    or_im2col(xp, col, B, C, HP, WP, KH, KW, SH, SW);
    or_transpose(w, wt, O, K);
    or_matmul(col, wt, out, M, K, O);
    for (size_t b = 0; b < B; ++b)
        for (size_t o = 0; o < O; ++o)
            for (size_t s = 0; s < HO * WO; ++s)
                y[(b * O + o) * HO * WO + s] = out[(b * HO * WO + s) * O + o];
    free(xp); free(col); free(wt); free(out);
}

/* Im2col convolution backward: permute/reshape backward (movement.rs:394-440),
 * MatMulGradFn (matmul.rs:450-460, 563-574), Im2colGradFn -> col2im
 * (conv.rs:145-208, 1242-1298), pad backward; dW flows back through the weight
 * permute [1,0] and reshape.  dx/dw may be NULL to skip. */
void or_im2col_conv_backward(const float *dy, const float *x, const float *w, float *dx,
                             float *dw, size_t B, size_t C, size_t O, size_t H, size_t W,
                             size_t KH, size_t KW, size_t SH, size_t SW, size_t PH,
                             size_t PW) {
    size_t HP = H + 2 * PH, WP = W + 2 * PW;
    size_t HO = (HP - KH) / SH + 1, WO = (WP - KW) / SW + 1;
    size_t M = B * HO * WO, K = C * KH * KW;
    float *g = (float *)malloc(sizeof(float) * M * O); /* dOut_2d [M, O] */
    for (size_t b = 0; b < B; ++b)
        for (size_t o = 0; o < O; ++o)
            for (size_t s = 0; s < HO * WO; ++s)
                g[(b * HO * WO + s) * O + o] = dy[(b * O + o) * HO * WO + s];
    if (dx) {
        float *wt = (float *)malloc(sizeof(float) * K * O);
        float *dcol = (float *)malloc(sizeof(float) * M * K);
        float *dxp = (float *)malloc(sizeof(float) * B * C * HP * WP);
        or_transpose(w, wt, O, K);                       /* weight_t [K, O] */
        or_matmul_backward_a(g, wt, dcol, M, K, O);      /* dcol = g . wt^T */
        or_col2im(dcol, dxp, B, C, HP, WP, KH, KW, SH, SW);
        or_pad_backward(dxp, dx, B, C, H, W, PH, PW);
        free(wt); free(dcol); free(dxp);
    }
    if (dw) {
        float *xp = (float *)malloc(sizeof(float) * B * C * HP * WP);
        float *col = (float *)malloc(sizeof(float) * M * K);
        float *dwt = (float *)malloc(sizeof(float) * K * O);
        or_pad(x, xp, B, C, H, W, PH, PW);
        or_im2col(xp, col, B, C, HP, WP, KH, KW, SH, SW);
        or_matmul_backward_b(col, g, dwt, M, K, O);      /* dwt = col^T . g  [K, O] */
        or_transpose(dwt, dw, K, O);                     /* permute backward -> [O, K] */
        free(xp); free(col); free(dwt);
    }
    free(g);
}

/* ---------------------------------------------------------------------------
 * Tiled iGEMM forward -- Conv2d::igemm_tiled, conv.rs:1679-1782, tiles
 * oc 32 / spatial 64 / ic 16 (TileConfig::default, conv.rs:117-127).
 * For each ic tile a partial sum is formed and added to the output (1776).
 * bug_compat != 0 reproduces the output index of conv.rs:1773,
 *   out_idx = b*O*HO*WO + oc*HO*WO + s_idx,
 * where s_idx already contains b*HO*WO, so batches b >= 1 land in shifted slots
 * and writes past the end are dropped (`get_mut` -> None).  bug_compat == 0 uses
 * the intended index b*O*HO*WO + oc*HO*WO + (oh*WO + ow).
 * ------------------------------------------------------------------------- */
void or_igemm_forward(const float *x, const float *w, float *y, size_t B, size_t C,
                      size_t O, size_t H, size_t W, size_t KH, size_t KW, size_t SH,
                      size_t SW, size_t PH, size_t PW, int bug_compat) {
    const size_t TO = 32, TC = 16, TS = 64;
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    size_t SP = HO * WO, total = B * O * SP;
    memset(y, 0, sizeof(float) * total);
    for (size_t o0 = 0; o0 < O; o0 += TO) {
        size_t o1 = o0 + TO < O ? o0 + TO : O;
        for (size_t s0 = 0; s0 < B * SP; s0 += TS) {
            size_t s1 = s0 + TS < B * SP ? s0 + TS : B * SP;
            for (size_t c0 = 0; c0 < C; c0 += TC) {
                size_t c1 = c0 + TC < C ? c0 + TC : C;
                for (size_t s = s0; s < s1; ++s) {
                    size_t b = s / SP, rem = s % SP, oh = rem / WO, ow = rem % WO;
                    for (size_t oc = o0; oc < o1; ++oc) {
                        float sum = 0.0f;
                        for (size_t ic = c0; ic < c1; ++ic)
                            for (size_t kh = 0; kh < KH; ++kh)
                                for (size_t kw = 0; kw < KW; ++kw) {
                                    isz ih = (isz)(oh * SH + kh) - (isz)PH;
                                    isz iw = (isz)(ow * SW + kw) - (isz)PW;
                                    if (ih >= 0 && ih < (isz)H && iw >= 0 && iw < (isz)W)
                                        sum += x[((b * C + ic) * H + (size_t)ih) * W + (size_t)iw] *
                                               w[((oc * C + ic) * KH + kh) * KW + kw];
                                }
                        size_t idx = bug_compat ? b * O * SP + oc * SP + s
                                                : b * O * SP + oc * SP + rem;
                        if (idx < total) y[idx] += sum;
                    }
                }
            }
        }
    }
}

/* iGEMM input gradient -- IGEMMGradFn::igemm_backward_input, conv.rs:822-912.
 * Order per dX element: oc -> oh -> ow over the in-field terms (same pruning as
 * or_direct_conv_backward_input).  bug_compat != 0 reproduces the write index of
 * conv.rs:904, in_idx = b*C*H*W + ic*H*W + s_idx (s_idx includes b*H*W). */
void or_igemm_backward_input(const float *dy, const float *w, float *dx, size_t B,
                             size_t C, size_t O, size_t H, size_t W, size_t KH,
                             size_t KW, size_t SH, size_t SW, size_t PH, size_t PW,
                             int bug_compat) {
    const size_t TC = 16, TS = 64;
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    size_t HW = H * W, total = B * C * HW;
    memset(dx, 0, sizeof(float) * total);
    for (size_t c0 = 0; c0 < C; c0 += TC) {
        size_t c1 = c0 + TC < C ? c0 + TC : C;
        for (size_t s0 = 0; s0 < B * HW; s0 += TS) {
            size_t s1 = s0 + TS < B * HW ? s0 + TS : B * HW;
            for (size_t s = s0; s < s1; ++s) {
                size_t b = s / HW, rem = s % HW, ih = rem / W, iw = rem % W;
                isz th = (isz)ih + (isz)PH, tw = (isz)iw + (isz)PW;
                size_t oh0 = first_out(th, KH, SH), ow0 = first_out(tw, KW, SW);
                for (size_t ic = c0; ic < c1; ++ic) {
                    float sum = 0.0f;
                    for (size_t oc = 0; oc < O; ++oc)
                        for (size_t oh = oh0; oh < HO && (isz)(oh * SH) <= th; ++oh)
                            for (size_t ow = ow0; ow < WO && (isz)(ow * SW) <= tw; ++ow) {
                                size_t kh = (size_t)(th - (isz)(oh * SH));
                                size_t kw = (size_t)(tw - (isz)(ow * SW));
                                sum += dy[((b * O + oc) * HO + oh) * WO + ow] *
                                       w[((oc * C + ic) * KH + kh) * KW + kw];
                            }
                    size_t idx = bug_compat ? b * C * HW + ic * HW + s : b * C * HW + ic * HW + rem;
                    if (idx < total) dx[idx] = sum;
                }
            }
        }
    }
}

/* iGEMM weight gradient -- IGEMMGradFn::igemm_backward_weight, conv.rs:916-1012.
 * Loop order oc-tile -> s-tile -> ic-tile -> s -> oc -> ic -> kh -> kw.
 * bug_compat != 0 reproduces the dY read index of conv.rs:961,
 * out_idx = b*O*HO*WO + s_idx + oc*HO*WO (s_idx includes b*HO*WO); reads past the
 * end contribute 0 (`unwrap_or(&0.0)`). */
void or_igemm_backward_weight(const float *x, const float *dy, float *dw, size_t B,
                              size_t C, size_t O, size_t H, size_t W, size_t KH,
                              size_t KW, size_t SH, size_t SW, size_t PH, size_t PW,
                              int bug_compat) {
    const size_t TO = 32, TC = 16, TS = 64;
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    size_t SP = HO * WO, total_dy = B * O * SP;
    memset(dw, 0, sizeof(float) * O * C * KH * KW);
    for (size_t o0 = 0; o0 < O; o0 += TO) {
        size_t o1 = o0 + TO < O ? o0 + TO : O;
        for (size_t s0 = 0; s0 < B * SP; s0 += TS) {
            size_t s1 = s0 + TS < B * SP ? s0 + TS : B * SP;
            for (size_t c0 = 0; c0 < C; c0 += TC) {
                size_t c1 = c0 + TC < C ? c0 + TC : C;
                for (size_t s = s0; s < s1; ++s) {
                    size_t b = s / SP, rem = s % SP, oh = rem / WO, ow = rem % WO;
                    size_t base = bug_compat ? b * O * SP + s : b * O * SP + rem;
                    for (size_t oc = o0; oc < o1; ++oc) {
                        size_t oi = base + oc * SP;
                        float dout = oi < total_dy ? dy[oi] : 0.0f;
                        for (size_t ic = c0; ic < c1; ++ic)
                            for (size_t kh = 0; kh < KH; ++kh)
                                for (size_t kw = 0; kw < KW; ++kw) {
                                    isz ih = (isz)(oh * SH + kh) - (isz)PH;
                                    isz iw = (isz)(ow * SW + kw) - (isz)PW;
                                    if (ih >= 0 && ih < (isz)H && iw >= 0 && iw < (isz)W)
                                        dw[((oc * C + ic) * KH + kh) * KW + kw] +=
                                            x[((b * C + ic) * H + (size_t)ih) * W + (size_t)iw] * dout;
                                }
                    }
                }
            }
        }
    }
}

/* ---------------------------------------------------------------------------
 * ConvTranspose2d forward -- src/nn/layers/conv_transpose.rs:356-435:
 * x permute [0,2,3,1] + reshape [B*H*W, Cin] (385-386), W reshape [Cin, Cout*K*K]
 * (389), matmul (392), col2im_transpose (74-143) which skips taps in the p border,
 * then bias [1,Cout,1,1] broadcast add (411-414).  bias may be NULL.
 * Output HO = (H-1)*SH + KH - 2*PH.
 * ------------------------------------------------------------------------- */
void or_conv_transpose_forward(const float *x, const float *w, const float *bias,
                               float *y, size_t B, size_t CI, size_t CO, size_t H,
                               size_t W, size_t KH, size_t KW, size_t SH, size_t SW,
                               size_t PH, size_t PW) {
    size_t HO = (H - 1) * SH + KH - 2 * PH, WO = (W - 1) * SW + KW - 2 * PW;
    size_t M = B * H * W, N = CO * KH * KW;
    float *xin = (float *)malloc(sizeof(float) * M * CI);
    float *col = (float *)malloc(sizeof(float) * M * N);
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < CI; ++c)
            for (size_t s = 0; s < H * W; ++s) xin[(b * H * W + s) * CI + c] = x[(b * CI + c) * H * W + s];
    or_matmul(xin, w, col, M, CI, N);
    memset(y, 0, sizeof(float) * B * CO * HO * WO);
    for (size_t b = 0; b < B; ++b)
        for (size_t ih = 0; ih < H; ++ih)
            for (size_t iw = 0; iw < W; ++iw) {
                size_t row = (b * H + ih) * W + iw;
                for (size_t c = 0; c < CO; ++c)
                    for (size_t kh = 0; kh < KH; ++kh)
                        for (size_t kw = 0; kw < KW; ++kw) {
                            size_t hp = ih * SH + kh, wp = iw * SW + kw;
                            if (hp < PH || hp >= HO + PH) continue;
                            if (wp < PW || wp >= WO + PW) continue;
                            y[((b * CO + c) * HO + hp - PH) * WO + wp - PW] +=
                                col[row * N + (c * KH + kh) * KW + kw];
                        }
            }
    if (bias)
        for (size_t b = 0; b < B; ++b)
            for (size_t c = 0; c < CO; ++c)
                for (size_t s = 0; s < HO * WO; ++s) y[(b * CO + c) * HO * WO + s] += bias[c];
    free(xin); free(col);
}

/* ConvTranspose2dGradFn::backward -- conv_transpose.rs:161-341.
 * dX loop 200-251 (order c_out -> kh -> kw per dX element), dW loop 262-315
 * (order b -> ih -> iw per dW element), db = sum_dim(3), sum_dim(2), sum_dim(0)
 * (329-335; per channel: for each b, sum of row sums).  Any output may be NULL. */
void or_conv_transpose_backward(const float *dy, const float *x, const float *w,
                                float *dx, float *dw, float *db, size_t B, size_t CI,
                                size_t CO, size_t H, size_t W, size_t KH, size_t KW,
                                size_t SH, size_t SW, size_t PH, size_t PW) {
    isz HO = (isz)((H - 1) * SH + KH - 2 * PH), WO = (isz)((W - 1) * SW + KW - 2 * PW);
    if (dx)
        for (size_t b = 0; b < B; ++b)
            for (size_t ci = 0; ci < CI; ++ci)
                for (size_t ih = 0; ih < H; ++ih)
                    for (size_t iw = 0; iw < W; ++iw) {
                        float s = 0.0f;
                        for (size_t co = 0; co < CO; ++co)
                            for (size_t kh = 0; kh < KH; ++kh)
                                for (size_t kw = 0; kw < KW; ++kw) {
                                    isz ho = (isz)(ih * SH + kh) - (isz)PH;
                                    isz wo = (isz)(iw * SW + kw) - (isz)PW;
                                    if (ho >= 0 && ho < HO && wo >= 0 && wo < WO)
                                        s += dy[((b * CO + co) * (size_t)HO + (size_t)ho) * (size_t)WO + (size_t)wo] *
                                             w[((ci * CO + co) * KH + kh) * KW + kw];
                                }
                        dx[((b * CI + ci) * H + ih) * W + iw] = s;
                    }
    if (dw)
        for (size_t ci = 0; ci < CI; ++ci)
            for (size_t co = 0; co < CO; ++co)
                for (size_t kh = 0; kh < KH; ++kh)
                    for (size_t kw = 0; kw < KW; ++kw) {
                        float s = 0.0f;
                        for (size_t b = 0; b < B; ++b)
                            for (size_t ih = 0; ih < H; ++ih)
                                for (size_t iw = 0; iw < W; ++iw) {
                                    isz ho = (isz)(ih * SH + kh) - (isz)PH;
                                    isz wo = (isz)(iw * SW + kw) - (isz)PW;
                                    if (ho >= 0 && ho < HO && wo >= 0 && wo < WO)
                                        s += x[((b * CI + ci) * H + ih) * W + iw] *
                                             dy[((b * CO + co) * (size_t)HO + (size_t)ho) * (size_t)WO + (size_t)wo];
                                }
                        dw[((ci * CO + co) * KH + kh) * KW + kw] = s;
                    }
    if (db) {
        size_t hw = (size_t)HO * (size_t)WO;
        for (size_t co = 0; co < CO; ++co) {
            float total = 0.0f;
            for (size_t b = 0; b < B; ++b) {
                float sb = 0.0f;
                for (isz ho = 0; ho < HO; ++ho) {
                    float sr = 0.0f;
                    for (isz wo = 0; wo < WO; ++wo) sr += dy[(b * CO + co) * hw + (size_t)ho * (size_t)WO + (size_t)wo];
                    sb += sr;
                }
                total += sb;
            }
            db[co] = total;
        }
    }
}

/* ---------------------------------------------------------------------------
 * Linear -- src/nn/layers/linear.rs:110-117: y = x . W + b, W stored [in, out];
 * the broadcast add runs on the CPU (binary.rs:57-62, 644-690).  bias may be NULL.
 * ------------------------------------------------------------------------- */
void or_linear_forward(const float *x, const float *w, const float *bias, float *y,
                       size_t m, size_t in, size_t out) {
    or_matmul(x, w, y, m, in, out);
    if (bias)
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < out; ++j) y[i * out + j] += bias[j];
}

/* Linear backward: MatMulGradFn (matmul.rs:450-460, 563-574) for dX and dW and
 * BinaryGradFn -> sum_over_broadcast_dims (binary.rs:533-598) for db, which
 * adds dY rows into db in linear index order. */
void or_linear_backward(const float *dy, const float *x, const float *w, float *dx,
                        float *dw, float *db, size_t m, size_t in, size_t out) {
    if (dx) or_matmul_backward_a(dy, w, dx, m, in, out);
    if (dw) or_matmul_backward_b(x, dy, dw, m, in, out);
    if (db) {
        memset(db, 0, sizeof(float) * out);
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < out; ++j) db[j] += dy[i * out + j];
    }
}

/* ---------------------------------------------------------------------------
 * PixelShuffle -- src/nn/layers/pixelshuffle.rs:50-85: reshape
 * [B, C, r, r, H, W] -> permute [0,1,4,2,5,3] -> reshape [B, C, H*r, W*r], i.e.
 * out[b, c, h*r+i, w*r+j] = in[b, c*r*r + i*r + j, h, w].  Backward is the
 * inverse permutation (movement.rs:407-440).
 * ------------------------------------------------------------------------- */
void or_pixel_shuffle(const float *x, float *y, size_t B, size_t C, size_t H, size_t W,
                      size_t r) {
    size_t HO = H * r, WO = W * r;
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c)
            for (size_t i = 0; i < r; ++i)
                for (size_t j = 0; j < r; ++j)
                    for (size_t h = 0; h < H; ++h)
                        for (size_t w = 0; w < W; ++w)
                            y[((b * C + c) * HO + h * r + i) * WO + w * r + j] =
                                x[(((b * C + c) * r + i) * r + j) * H * W + h * W + w];
}

void or_pixel_shuffle_backward(const float *dy, float *dx, size_t B, size_t C,
                               size_t H, size_t W, size_t r) {
    size_t HO = H * r, WO = W * r;
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c)
            for (size_t i = 0; i < r; ++i)
                for (size_t j = 0; j < r; ++j)
                    for (size_t h = 0; h < H; ++h)
                        for (size_t w = 0; w < W; ++w)
                            dx[(((b * C + c) * r + i) * r + j) * H * W + h * W + w] =
                                dy[((b * C + c) * HO + h * r + i) * WO + w * r + j];
}

/* ---------------------------------------------------------------------------
 * Glue of the config graphs (not contractions).
 * ReLU forward, unary.rs:272: y = x.max(0.0) -- Rust's f32::max returns the
 * other operand for a NaN, so NaN -> 0; for x = -0.0 either zero is allowed
 * (the doc of f32::max), this restatement returns +0.
 * ReLU backward, unary.rs:150-155: dx = x > 0 ? g : 0 (x is the forward input).
 * Sum, reduce.rs:160-180 (ReduceOp::Sum on the CPU): data.iter().sum(), one f32
 * accumulator in index order.  SumGradFn, reduce.rs:22-45: every element of
 * the input gradient is the upstream scalar (the autograd seed is 1.0,
 * autograd.rs:49-62).
 * ------------------------------------------------------------------------- */
void or_relu(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

void or_relu_backward(const float *g, const float *x, float *dx, size_t n) {
    for (size_t i = 0; i < n; ++i) dx[i] = x[i] > 0.0f ? g[i] : 0.0f;
}

float or_sum(const float *x, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i];
    return s;
}

void or_sum_backward(float grad, float *dx, size_t n) {
    for (size_t i = 0; i < n; ++i) dx[i] = grad;
}

/* ---------------------------------------------------------------------------
 * The step after the weight gradient.
 * Gradient accumulation, autograd.rs:158-184: existing += new (gpu_add).
 * Optimizer step, optimizer_step.wgsl (the GPU path of SGD::step, sgd.rs:94-180;
 * op 0 SGD, 1 SGD + momentum, 2 Adam), per element, f32, unfused:
 *   g = grad (+ weight_decay * param when weight_decay != 0)
 *   0: param -= lr * g
 *   1: v = beta1 * v - lr * g; param += v
 *   2: m = beta1*m + (1-beta1)*g; v = beta2*v + (1-beta2)*g*g;
 *      param -= lr * (m / (1 - beta1^t)) / (sqrt(v / (1 - beta2^t)) + eps)
 * ------------------------------------------------------------------------- */
void or_add_inplace(float *a, const float *b, size_t n) {
    for (size_t i = 0; i < n; ++i) a[i] += b[i];
}

void or_optimizer_step(int op, float lr, float beta1, float beta2, float t, float eps, float wd,
                       float *param, const float *grad, float *s1, float *s2, size_t n) {
    const float mh = 1.0f / (1.0f - powf(beta1, t)), vh = 1.0f / (1.0f - powf(beta2, t));
    for (size_t i = 0; i < n; ++i) {
        float g = grad[i];
        if (wd != 0.0f) g = g + wd * param[i];
        if (op == 0) {
            param[i] = param[i] - lr * g;
        } else if (op == 1) {
            s1[i] = beta1 * s1[i] - lr * g;
            param[i] = param[i] + s1[i];
        } else {
            s1[i] = beta1 * s1[i] + (1.0f - beta1) * g;
            s2[i] = beta2 * s2[i] + (1.0f - beta2) * g * g;
            const float m_hat = s1[i] * mh, v_hat = s2[i] * vh;
            param[i] = param[i] - lr * m_hat / (sqrtf(v_hat) + eps);
        }
    }
}

/* ---------------------------------------------------------------------------
 * bf16 storage conversion: Storage::to_dtype(BF16) goes through
 * half::bf16::from_f32 (storage.rs:503-505, half 2.7.1), round-to-nearest-even
 * with NaN kept quiet.  The bf16 oracle is f32 math on inputs rounded this way.
 * ------------------------------------------------------------------------- */
static uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

void or_round_bf16(const float *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t u = (uint32_t)f32_to_bf16_rne(in[i]) << 16;
        memcpy(&out[i], &u, 4);
    }
}

void or_f32_to_bf16_bits(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f32_to_bf16_rne(in[i]);
}

/* ---------------------------------------------------------------------------
 * Independent float64 reference (not a restatement): the textbook convolution
 * sum with double accumulation, used to bound the f32 rounding of both sides.
 * ------------------------------------------------------------------------- */
void or_conv_forward_f64(const float *x, const float *w, double *y, size_t B, size_t C,
                         size_t O, size_t H, size_t W, size_t KH, size_t KW, size_t SH,
                         size_t SW, size_t PH, size_t PW) {
    size_t HO = (H + 2 * PH - KH) / SH + 1, WO = (W + 2 * PW - KW) / SW + 1;
    for (size_t b = 0; b < B; ++b)
        for (size_t oc = 0; oc < O; ++oc)
            for (size_t oh = 0; oh < HO; ++oh)
                for (size_t ow = 0; ow < WO; ++ow) {
                    double s = 0.0;
                    for (size_t ic = 0; ic < C; ++ic)
                        for (size_t kh = 0; kh < KH; ++kh) {
                            isz ih = (isz)(oh * SH + kh) - (isz)PH;
                            if (ih < 0 || ih >= (isz)H) continue;
                            for (size_t kw = 0; kw < KW; ++kw) {
                                isz iw = (isz)(ow * SW + kw) - (isz)PW;
                                if (iw < 0 || iw >= (isz)W) continue;
                                s += (double)x[((b * C + ic) * H + (size_t)ih) * W + (size_t)iw] *
                                     (double)w[((oc * C + ic) * KH + kh) * KW + kw];
                            }
                        }
                    y[((b * O + oc) * HO + oh) * WO + ow] = s;
                }
}
