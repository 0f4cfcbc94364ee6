/* Host memory-safety check of the CPU oracle (test infrastructure only).
 *
 * Built with AddressSanitizer and UndefinedBehaviorSanitizer together with
 * volta_oracle.c (`make -C oracle asan-check`), it calls every exported or_*
 * function over a grid of small shapes that includes the edges: 1x1 images,
 * kernels larger than the padded image is rejected, stride larger than the
 * kernel, padding as large as the kernel, batch and channel counts of one, and
 * the bug-compatible index forms whose out-of-range writes must be dropped.
 * Every buffer is allocated at exactly the size the function's contract names,
 * so a read or write one element past it is reported by the sanitizer.
 * Direct, im2col and implicit-GEMM forward results are also compared with one
 * another (they sum the same products in different orders).
 *
 * Exit status 0 and one summary line on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef size_t sz;
#define CONV_DIMS sz, sz, sz, sz, sz, sz, sz, sz, sz, sz, sz
void or_direct_conv(const float *, const float *, float *, CONV_DIMS);
void or_direct_conv_backward_input(const float *, const float *, float *, CONV_DIMS);
void or_direct_conv_backward_input_literal(const float *, const float *, float *, CONV_DIMS);
void or_direct_conv_backward_weight(const float *, const float *, float *, CONV_DIMS);
void or_conv_bias_grad(const float *, float *, sz, sz, sz, sz);
void or_pad(const float *, float *, sz, sz, sz, sz, sz, sz);
void or_pad_backward(const float *, float *, sz, sz, sz, sz, sz, sz);
void or_im2col(const float *, float *, sz, sz, sz, sz, sz, sz, sz, sz);
void or_col2im(const float *, float *, sz, sz, sz, sz, sz, sz, sz, sz);
void or_matmul(const float *, const float *, float *, sz, sz, sz);
void or_matmul_backward_a(const float *, const float *, float *, sz, sz, sz);
void or_matmul_backward_b(const float *, const float *, float *, sz, sz, sz);
void or_transpose(const float *, float *, sz, sz);
void or_im2col_conv_forward(const float *, const float *, float *, CONV_DIMS);
void or_im2col_conv_backward(const float *, const float *, const float *, float *, float *,
                             CONV_DIMS);
void or_igemm_forward(const float *, const float *, float *, CONV_DIMS, int);
void or_igemm_backward_input(const float *, const float *, float *, CONV_DIMS, int);
void or_igemm_backward_weight(const float *, const float *, float *, CONV_DIMS, int);
void or_conv_transpose_forward(const float *, const float *, const float *, float *, sz, sz, sz,
                               sz, sz, sz, sz, sz, sz, sz, sz);
void or_conv_transpose_backward(const float *, const float *, const float *, float *, float *,
                                float *, sz, sz, sz, sz, sz, sz, sz, sz, sz, sz, sz);
void or_linear_forward(const float *, const float *, const float *, float *, sz, sz, sz);
void or_linear_backward(const float *, const float *, const float *, float *, float *, float *,
                        sz, sz, sz);
void or_pixel_shuffle(const float *, float *, sz, sz, sz, sz, sz);
void or_pixel_shuffle_backward(const float *, float *, sz, sz, sz, sz, sz);
void or_relu(const float *, float *, sz);
void or_relu_backward(const float *, const float *, float *, sz);
float or_sum(const float *, sz);
void or_sum_backward(float, float *, sz);
void or_add_inplace(float *, const float *, sz);
void or_optimizer_step(int, float, float, float, float, float, float, float *, const float *,
                       float *, float *, sz);
void or_round_bf16(const float *, float *, sz);
void or_f32_to_bf16_bits(const float *, uint16_t *, sz);
void or_conv_forward_f64(const float *, const float *, double *, CONV_DIMS);

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static float urand(void) {
    rng ^= rng << 13, rng ^= rng >> 7, rng ^= rng << 17;
    return (float)((rng >> 40) & 0xffff) / 32768.0f - 1.0f;
}

/* exact-size buffers; malloc(0) may return NULL, which no oracle function
 * dereferences for a zero-element operand */
static float *buf(sz n) {
    float *p = (float *)malloc(n ? n * sizeof(float) : 1);
    for (sz i = 0; i < n; ++i) p[i] = urand();
    return p;
}

static long failures = 0, calls = 0;

static void agree(const float *a, const float *b, sz n, const char *what, const sz *dims) {
    for (sz i = 0; i < n; ++i) {
        float d = fabsf(a[i] - b[i]), s = fabsf(a[i]) + fabsf(b[i]) + 1.0f;
        if (!(d <= 1e-4f * s)) {
            if (failures++ < 10)
                fprintf(stderr, "%s differs at %zu (B%zu C%zu O%zu H%zu W%zu K%zu S%zu P%zu): %g vs %g\n",
                        what, i, dims[0], dims[1], dims[2], dims[3], dims[4], dims[5], dims[6],
                        dims[7], a[i], b[i]);
            return;
        }
    }
}

static void conv_case(sz B, sz C, sz O, sz H, sz W, sz K, sz S, sz P) {
    const sz dims[8] = {B, C, O, H, W, K, S, P};
    if (H + 2 * P < K || W + 2 * P < K) return;
    const sz HO = (H + 2 * P - K) / S + 1, WO = (W + 2 * P - K) / S + 1;
    const sz nx = B * C * H * W, nw = O * C * K * K, ny = B * O * HO * WO;
    float *x = buf(nx), *w = buf(nw), *dy = buf(ny);
    float *y0 = buf(ny), *y1 = buf(ny), *y2 = buf(ny), *y3 = buf(ny);
    float *dx = buf(nx), *dx2 = buf(nx), *dw = buf(nw), *dw2 = buf(nw), *db = buf(O);
    double *yd = (double *)malloc(ny ? ny * sizeof(double) : 1);

    or_direct_conv(x, w, y0, B, C, O, H, W, K, K, S, S, P, P);
    or_im2col_conv_forward(x, w, y1, B, C, O, H, W, K, K, S, S, P, P);
    or_igemm_forward(x, w, y2, B, C, O, H, W, K, K, S, S, P, P, 0);
    or_igemm_forward(x, w, y3, B, C, O, H, W, K, K, S, S, P, P, 1);
    or_conv_forward_f64(x, w, yd, B, C, O, H, W, K, K, S, S, P, P);
    agree(y0, y1, ny, "im2col forward", dims);
    agree(y0, y2, ny, "igemm forward", dims);
    for (sz i = 0; i < ny; ++i) y1[i] = (float)yd[i];
    agree(y0, y1, ny, "f64 forward", dims);

    or_direct_conv_backward_input(dy, w, dx, B, C, O, H, W, K, K, S, S, P, P);
    or_direct_conv_backward_input_literal(dy, w, dx2, B, C, O, H, W, K, K, S, S, P, P);
    agree(dx, dx2, nx, "backward input (literal loop)", dims);
    or_igemm_backward_input(dy, w, dx2, B, C, O, H, W, K, K, S, S, P, P, 0);
    agree(dx, dx2, nx, "igemm backward input", dims);
    or_igemm_backward_input(dy, w, dx2, B, C, O, H, W, K, K, S, S, P, P, 1);
    or_direct_conv_backward_weight(dy, x, dw, B, C, O, H, W, K, K, S, S, P, P);
    or_igemm_backward_weight(x, dy, dw2, B, C, O, H, W, K, K, S, S, P, P, 0);
    agree(dw, dw2, nw, "igemm backward weight", dims);
    or_igemm_backward_weight(x, dy, dw2, B, C, O, H, W, K, K, S, S, P, P, 1);
    or_im2col_conv_backward(dy, x, w, dx2, dw2, B, C, O, H, W, K, K, S, S, P, P);
    agree(dx, dx2, nx, "im2col backward input", dims);
    agree(dw, dw2, nw, "im2col backward weight", dims);
    or_conv_bias_grad(dy, db, B, O, HO, WO);

    /* padding and the unpadded im2col pair */
    const sz HP = H + 2 * P, WP = W + 2 * P;
    float *xp = buf(B * C * HP * WP), *gx = buf(nx);
    or_pad(x, xp, B, C, H, W, P, P);
    or_pad_backward(xp, gx, B, C, H, W, P, P);
    agree(x, gx, nx, "pad round trip", dims);
    const sz HOp = (HP - K) / S + 1, WOp = (WP - K) / S + 1;
    float *col = buf(B * HOp * WOp * C * K * K), *xb = buf(B * C * HP * WP);
    or_im2col(xp, col, B, C, HP, WP, K, K, S, S);
    or_col2im(col, xb, B, C, HP, WP, K, K, S, S);

    /* ConvTranspose2d with the same dimensions read as (CI=C, CO=O) */
    if ((H - 1) * S + K > 2 * P && (W - 1) * S + K > 2 * P) {
        const sz TH = (H - 1) * S + K - 2 * P, TW = (W - 1) * S + K - 2 * P;
        float *tw = buf(C * O * K * K), *tb = buf(O), *ty = buf(B * O * TH * TW);
        float *tdy = buf(B * O * TH * TW), *tdx = buf(nx), *tdw = buf(C * O * K * K), *tdb = buf(O);
        or_conv_transpose_forward(x, tw, tb, ty, B, C, O, H, W, K, K, S, S, P, P);
        or_conv_transpose_forward(x, tw, NULL, ty, B, C, O, H, W, K, K, S, S, P, P);
        or_conv_transpose_backward(tdy, x, tw, tdx, tdw, tdb, B, C, O, H, W, K, K, S, S, P, P);
        free(tw), free(tb), free(ty), free(tdy), free(tdx), free(tdw), free(tdb);
    }
    free(x), free(w), free(dy), free(y0), free(y1), free(y2), free(y3), free(dx), free(dx2);
    free(dw), free(dw2), free(db), free(yd), free(xp), free(gx), free(col), free(xb);
    ++calls;
}

static void dense_case(sz m, sz k, sz n) {
    float *a = buf(m * k), *b = buf(k * n), *c = buf(m * n), *g = buf(m * n);
    float *da = buf(m * k), *dbm = buf(k * n), *at = buf(m * k), *bias = buf(n), *db = buf(n);
    or_matmul(a, b, c, m, k, n);
    or_matmul_backward_a(g, b, da, m, k, n);
    or_matmul_backward_b(a, g, dbm, m, k, n);
    or_transpose(a, at, m, k);
    or_linear_forward(a, b, bias, c, m, k, n);
    or_linear_forward(a, b, NULL, c, m, k, n);
    or_linear_backward(g, a, b, da, dbm, db, m, k, n);
    or_linear_backward(g, a, b, NULL, NULL, db, m, k, n);
    free(a), free(b), free(c), free(g), free(da), free(dbm), free(at), free(bias), free(db);
    ++calls;
}

static void elementwise_case(sz n) {
    float *x = buf(n), *y = buf(n), *g = buf(n), *p = buf(n), *s1 = buf(n), *s2 = buf(n);
    uint16_t *h = (uint16_t *)malloc(n ? n * sizeof(uint16_t) : 1);
    if (n) x[0] = NAN, x[n - 1] = INFINITY;
    or_relu(x, y, n);
    or_relu_backward(g, x, y, n);
    (void)or_sum(g, n);
    or_sum_backward(1.0f, y, n);
    or_add_inplace(y, g, n);
    for (int op = 0; op < 3; ++op) {
        for (sz i = 0; i < n; ++i) s2[i] = fabsf(s2[i]);
        or_optimizer_step(op, 1e-2f, 0.9f, 0.999f, 3.0f, 1e-8f, op == 2 ? 0.0f : 1e-4f, p, g, s1,
                          s2, n);
    }
    or_round_bf16(x, y, n);
    or_f32_to_bf16_bits(x, h, n);
    free(x), free(y), free(g), free(p), free(s1), free(s2), free(h);
    ++calls;
}

static void shuffle_case(sz B, sz C, sz H, sz W, sz r) {
    const sz n = B * C * r * r * H * W;
    float *x = buf(n), *y = buf(n), *dx = buf(n);
    or_pixel_shuffle(x, y, B, C, H, W, r);
    or_pixel_shuffle_backward(y, dx, B, C, H, W, r);
    agree(x, dx, n, "pixel shuffle round trip", (const sz[8]){B, C, 0, H, W, r, 0, 0});
    free(x), free(y), free(dx);
    ++calls;
}

int main(void) {
    const sz Bs[] = {1, 2}, Cs[] = {1, 3}, Os[] = {1, 4}, Hs[] = {1, 2, 5, 8}, Ws[] = {1, 4, 7};
    const sz Ks[] = {1, 2, 3, 5}, Ss[] = {1, 2, 3, 5}, Ps[] = {0, 1, 2, 3};
    for (sz a = 0; a < 2; ++a)
        for (sz c = 0; c < 2; ++c)
            for (sz o = 0; o < 2; ++o)
                for (sz h = 0; h < 4; ++h)
                    for (sz w = 0; w < 3; ++w)
                        for (sz k = 0; k < 4; ++k)
                            for (sz s = 0; s < 4; ++s)
                                for (sz p = 0; p < 4; ++p)
                                    conv_case(Bs[a], Cs[c], Os[o], Hs[h], Ws[w], Ks[k], Ss[s], Ps[p]);
    const sz Ms[] = {0, 1, 3, 17}, Kd[] = {1, 2, 9}, Nd[] = {1, 5, 16};
    for (sz i = 0; i < 4; ++i)
        for (sz j = 0; j < 3; ++j)
            for (sz l = 0; l < 3; ++l) dense_case(Ms[i], Kd[j], Nd[l]);
    for (sz n = 0; n < 70; n += 7) elementwise_case(n);
    for (sz r = 1; r <= 3; ++r) shuffle_case(2, 3, 2, 5, r);
    printf("oracle asan_check: %ld cases, %ld failures\n", calls, failures);
    return failures ? 1 : 0;
}
