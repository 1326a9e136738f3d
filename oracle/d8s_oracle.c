/* d8s_oracle.c -- CPU restatement of the INT8 DenseNet encoder's arithmetic, in plain C.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker of the HIP kernels: only tests/, the smoke
 * check of __graft_entry__.py and the CPU-baseline leg of bench.py may load it.  The product never
 * calls it and has no CPU fallback.
 *
 * Every function recomputes, one pixel at a time, what a kernel writes, with the same fp32 / fp16
 * roundings, so the HIP results are compared BIT FOR BIT.  Rows are selected by index, so full-size
 * problems can be checked on a sample of pixels.  Sources followed:
 *   prologue      src/knee/dense8s_kernels.cu:122-139 (pro4h), src/knee/dense8s.py:584-587 (emulation)
 *   conv1         src/knee/dense8s_kernels.cu:479-627 (conv1w_body), epilogue :595-611
 *   conv2         src/knee/dense8s_kernels.cu:2664-2824 (conv2t_body), epilogue :2797-2809
 *   transition    src/knee/dense8s_kernels.cu:3041-3262 (trans_w_body), integer form
 *                 src/knee/dense8s.py:605-617
 *   final         src/knee/dense8s_kernels.cu:2304-2323 (final_q)
 *   stem          src/knee/dense8s.py:574-578 (fp formula), src/knee/dense8s_kernels.cu:2365-2412
 *                 (quant_seg with the 3x3/2 max-pool)
 * Build: oracle/Makefile (gcc, -ffp-contract=off: no fused operation except the explicit fmaf).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- fp16 ---------------------------------------------------------------------------------- */

double orc_f16_value(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexp((double)m, -24);
    else v = ldexp((double)(m | 1024), e - 25);
    return s ? -v : v;
}

/* Round a double to the nearest fp16 value (ties to even, subnormals kept, overflow to inf).
 * Returns the fp16 bits. */
uint16_t orc_f16_bits(double x) {
    if (isnan(x)) return 0x7e00;
    uint16_t sign = signbit(x) ? 0x8000 : 0;
    double a = fabs(x);
    if (a == 0.0) return sign;
    int E;
    frexp(a, &E);                           /* a = f 2^E, f in [0.5, 1): exponent e = E - 1 */
    int e = E - 1;
    if (e < -14) e = -14;                   /* subnormal quantum 2^-24 */
    const double quantum = ldexp(1.0, e - 10);
    double r = nearbyint(a / quantum) * quantum;    /* exact scaling, one rounding (ties to even) */
    if (r >= 65520.0 || r > 65504.0) return sign | 0x7c00;
    if (r < ldexp(1.0, -14)) return sign | (uint16_t)(r / ldexp(1.0, -24));   /* subnormal or 0 */
    int E2;
    frexp(r, &E2);
    const int be = E2 - 1 + 15;
    const uint16_t mant = (uint16_t)(r / ldexp(1.0, E2 - 1 - 10)) - 1024;
    return sign | (uint16_t)(be << 10) | mant;
}

double orc_f16_round(double x) { return orc_f16_value(orc_f16_bits(x)); }

/* ---- prologue ------------------------------------------------------------------------------ */

/* u = RNE(255 sat(fp16(A q + B))): A q + B is exact in double (fp16 operands, |q| <= 128), so the
 * conversion to fp16 is the single rounding of the fused fp16 fma; sat maps NaN to 0. */
uint8_t orc_prologue(int8_t q, uint16_t A16, uint16_t B16) {
    const double t = orc_f16_value(A16) * (double)q + orc_f16_value(B16);
    double v = orc_f16_round(t);
    if (!(v > 0.0)) v = 0.0;                /* NaN and negatives */
    if (v > 1.0) v = 1.0;
    return (uint8_t)nearbyint(255.0 * v);   /* 255 v exact in double */
}

/* The prologue of every channel of a table abh [C/2][4] (A_2p, A_2p+1, B_2p, B_2p+1), as a lookup
 * table lut[c][q + 128]. */
static void prologue_lut(const uint16_t* abh, int C, uint8_t* lut) {
    for (int c = 0; c < C; ++c) {
        const uint16_t A = abh[(c >> 1) * 4 + (c & 1)], B = abh[(c >> 1) * 4 + 2 + (c & 1)];
        for (int q = -128; q < 128; ++q) lut[c * 256 + q + 128] = orc_prologue((int8_t)q, A, B);
    }
}

/* Store byte of channel c (group g = c / 32) of pixel p of image n. */
static int8_t store_at(const int8_t* in0, const int8_t* seg, int G0, int N, int64_t HW, int64_t n,
                       int64_t p, int c) {
    const int g = c >> 5, i = c & 31;
    if (g < G0) return in0[((n * G0 + g) * HW + p) * 32 + i];
    return seg[(((int64_t)(g - G0) * N + n) * HW + p) * 32 + i];
}

/* ---- conv1 --------------------------------------------------------------------------------- */

/* Rows sel[0..nsel): acc[r][128] = sum_k w[o][k] u[k] (int32), out[r][128] = low byte of
 * fma(sat(fma(g_o, float(acc), d_o)), 255, 2^23).  w is [G][128][32], gd [128][2].  lut_buf holds
 * G * 32 * 256 bytes of scratch. */
void orc_conv1(const int8_t* in0, const int8_t* seg, int G0, int G, int N, int HW,
               const uint16_t* abh, const int8_t* w, const float* gd, const int64_t* sel,
               int64_t nsel, int32_t* acc, uint8_t* out, uint8_t* lut_buf) {
    const int C = G * 32;
    prologue_lut(abh, C, lut_buf);
    uint8_t u[1216 * 32];
    for (int64_t r = 0; r < nsel; ++r) {
        const int64_t m = sel[r], n = m / HW, p = m - n * HW;
        for (int c = 0; c < C; ++c)
            u[c] = lut_buf[c * 256 + store_at(in0, seg, G0, N, HW, n, p, c) + 128];
        for (int o = 0; o < 128; ++o) {
            int32_t s = 0;
            for (int c = 0; c < C; ++c) s += (int32_t)w[((int64_t)(c >> 5) * 128 + o) * 32 + (c & 31)] * u[c];
            if (acc) acc[r * 128 + o] = s;
            if (out) {
                float y = fmaf(gd[2 * o], (float)s, gd[2 * o + 1]);
                y = fminf(fmaxf(y, 0.0f), 1.0f);
                const float f = fmaf(y, 255.0f, 8388608.0f);
                uint32_t bits;
                memcpy(&bits, &f, 4);
                out[r * 128 + o] = (uint8_t)(bits & 0xff);
            }
        }
    }
}

/* ---- conv2 --------------------------------------------------------------------------------- */

/* Pixels sel[0..nsel) of the N x H x W map: acc[r][32] = sum over taps and the 128 channels of the
 * planar bottleneck x [4][N*H*W][32] (zero padding) of w2k[b][tap][o][i] v, q = RNE(clamp(float(acc)
 * sc_o, -127, 127)). */
void orc_conv2(const uint8_t* x, int N, int H, int W, const int8_t* w2k, const float* sc,
               const int64_t* sel, int64_t nsel, int32_t* acc, int8_t* out) {
    const int64_t M = (int64_t)N * H * W;
    for (int64_t r = 0; r < nsel; ++r) {
        const int64_t m = sel[r], n = m / ((int64_t)H * W), p = m - n * H * W;
        const int y = (int)(p / W), xx = (int)(p % W);
        for (int o = 0; o < 32; ++o) {
            int32_t s = 0;
            for (int tap = 0; tap < 9; ++tap) {
                const int yy = y + tap / 3 - 1, xs = xx + tap % 3 - 1;
                if (yy < 0 || yy >= H || xs < 0 || xs >= W) continue;
                const int64_t pix = (n * H + yy) * W + xs;
                for (int b = 0; b < 4; ++b)
                    for (int i = 0; i < 32; ++i)
                        s += (int32_t)w2k[((b * 9 + tap) * 32 + o) * 32 + i] * x[(b * M + pix) * 32 + i];
            }
            if (acc) acc[r * 32 + o] = s;
            if (out) {
                const float t = fminf(fmaxf((float)s * sc[o], -127.0f), 127.0f);
                out[r * 32 + o] = (int8_t)nearbyintf(t);
            }
        }
    }
}

/* ---- transition ---------------------------------------------------------------------------- */

/* Output pixels sel[0..nsel) (index n * HW/4 + oy * W/2 + ox): s[k] = sum of the prologue of the 2x2
 * square, S[r][o] = sum_k w[o][k] s[k] (exact int32), q = RNE(clamp(kq_o * (float(S) / 4), +-127)),
 * kq_o = gdf[o][0].  w is [G][cout][32]. */
void orc_trans(const int8_t* in0, const int8_t* seg, int G0, int G, int N, int HW, int W,
               const uint16_t* abh, const int8_t* w, const float* gdf, int cout, const int64_t* sel,
               int64_t nsel, int32_t* Sout, int8_t* out, uint8_t* lut_buf) {
    const int C = G * 32, W2 = W / 2, HW4 = HW / 4;
    prologue_lut(abh, C, lut_buf);
    int32_t s[1216 * 32];
    for (int64_t r = 0; r < nsel; ++r) {
        const int64_t op = sel[r], n = op / HW4, p4 = op - n * HW4;
        const int64_t oy = p4 / W2, ox = p4 - oy * W2;
        for (int c = 0; c < C; ++c) {
            int32_t t = 0;
            for (int k = 0; k < 4; ++k) {
                const int64_t p = (2 * oy + (k >> 1)) * W + 2 * ox + (k & 1);
                t += lut_buf[c * 256 + store_at(in0, seg, G0, N, HW, n, p, c) + 128];
            }
            s[c] = t;
        }
        for (int o = 0; o < cout; ++o) {
            int64_t S = 0;
            for (int c = 0; c < C; ++c) S += (int64_t)w[((int64_t)(c >> 5) * cout + o) * 32 + (c & 31)] * s[c];
            if (Sout) Sout[r * cout + o] = (int32_t)S;
            if (out) {
                const float xq = gdf[2 * o] * ((float)(int32_t)S * 0.25f);
                out[r * cout + o] = (int8_t)nearbyintf(fminf(fmaxf(xq, -127.0f), 127.0f));
            }
        }
    }
}

/* ---- epilogues alone (accumulators computed elsewhere, e.g. by an exact float64 matmul) ----- */

void orc_prologue_lut(const uint16_t* abh, int C, uint8_t* lut) { prologue_lut(abh, C, lut); }

/* conv1: acc [n][cout] -> bytes [n][cout], gd [cout][2]. */
void orc_conv1_epilogue(const int32_t* acc, int64_t n, int cout, const float* gd, uint8_t* out) {
    for (int64_t r = 0; r < n; ++r)
        for (int o = 0; o < cout; ++o) {
            float y = fmaf(gd[2 * o], (float)acc[r * cout + o], gd[2 * o + 1]);
            y = fminf(fmaxf(y, 0.0f), 1.0f);
            const float f = fmaf(y, 255.0f, 8388608.0f);
            uint32_t bits;
            memcpy(&bits, &f, 4);
            out[r * cout + o] = (uint8_t)(bits & 0xff);
        }
}

/* conv2: acc [n][32] -> int8 [n][32]. */
void orc_conv2_epilogue(const int32_t* acc, int64_t n, const float* sc, int8_t* out) {
    for (int64_t r = 0; r < n; ++r)
        for (int o = 0; o < 32; ++o)
            out[r * 32 + o] = (int8_t)nearbyintf(fminf(fmaxf((float)acc[r * 32 + o] * sc[o], -127.0f), 127.0f));
}

/* transition: S [n][cout] -> int8 [n][cout], gdf [cout][2]. */
void orc_trans_epilogue(const int32_t* S, int64_t n, int cout, const float* gdf, int8_t* out) {
    for (int64_t r = 0; r < n; ++r)
        for (int o = 0; o < cout; ++o) {
            const float xq = gdf[2 * o] * ((float)S[r * cout + o] * 0.25f);
            out[r * cout + o] = (int8_t)nearbyintf(fminf(fmaxf(xq, -127.0f), 127.0f));
        }
}

/* ---- final features ------------------------------------------------------------------------ */

/* out[n][c] = (((P0 + P1) + P2) + P3) / HW, P_q = sum (in order) over s = q, q + 4, ... of
 * relu(fmaf(a_c, q_s, b_c)): the reference's final_q summation order. */
void orc_final(const int8_t* in0, int G0, const int8_t* seg, int N, int HW, const float* ab,
               float* out, int ctot) {
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < ctot; ++c) {
            float P[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int q = 0; q < 4; ++q)
                for (int s = q; s < HW; s += 4) {
                    const float v = fmaf(ab[2 * c], (float)store_at(in0, seg, G0, N, HW, n, s, c), ab[2 * c + 1]);
                    P[q] += fmaxf(v, 0.0f);
                }
            out[(int64_t)n * ctot + c] = (((P[0] + P[1]) + P[2]) + P[3]) / (float)HW;
        }
}

/* ---- stem ---------------------------------------------------------------------------------- */

/* Pooled pixels sel[0..nsel) (index n * Hp*Wp + py * Wp + px): the 64 int8 channels of
 * maxpool3x3/2(q), q = RNE(min(relu(y) inv_o, 127)), y = bias_o + sum_{c,ky,kx} w16 x16 (7x7/2, pad 3)
 * summed in double and rounded once to fp32.  x16 = lut[c][u] (kind 1, uint8 x) or the fp16 input
 * (kind 0); flip mirrors the columns.  w16 is [64][3][7][8] with kx' = kx + 1 (kx' = 0 unused).  conv_out, if not NULL,
 * receives the 9 x 64 fp32 values y of each pooled pixel's window (-1 outside the image). */
void orc_stem(const void* x, int kind, const uint16_t* lut, int flip, int N, int H, int W,
              const uint16_t* w16, const float* bias, const float* inv, const int64_t* sel,
              int64_t nsel, int8_t* out, float* conv_out) {
    const int Hc = H / 2, Wc = W / 2, Hp = H / 4, Wp = W / 4;
    for (int64_t r = 0; r < nsel; ++r) {
        const int64_t idx = sel[r], n = idx / ((int64_t)Hp * Wp);
        const int p = (int)(idx - n * Hp * Wp), py = p / Wp, px = p % Wp;
        int best[64];
        for (int o = 0; o < 64; ++o) best[o] = 0;
        for (int d = 0; d < 9; ++d) {
            const int cy = 2 * py - 1 + d / 3, cx = 2 * px - 1 + d % 3;
            const int valid = cy >= 0 && cy < Hc && cx >= 0 && cx < Wc;
            for (int o = 0; o < 64; ++o) {
                if (!valid) {
                    if (conv_out) conv_out[(r * 9 + d) * 64 + o] = -1.0f;
                    continue;
                }
                double y = 0.0;
                for (int c = 0; c < 3; ++c)
                    for (int ky = 0; ky < 7; ++ky) {
                        const int iy = 2 * cy + ky - 3;
                        if (iy < 0 || iy >= H) continue;
                        for (int kx = 0; kx < 7; ++kx) {
                            const int ix = 2 * cx + kx - 3;
                            if (ix < 0 || ix >= W) continue;
                            const int xs = flip ? W - 1 - ix : ix;
                            const int64_t e = ((n * 3 + c) * H + iy) * W + xs;
                            const double xv = kind == 1
                                ? orc_f16_value(lut[c * 256 + ((const uint8_t*)x)[e]])
                                : orc_f16_value(((const uint16_t*)x)[e]);
                            y += orc_f16_value(w16[((o * 3 + c) * 7 + ky) * 8 + kx + 1]) * xv;
                        }
                    }
                const float yf = (float)((double)bias[o] + y);
                if (conv_out) conv_out[(r * 9 + d) * 64 + o] = yf;
                const float t = fmaxf(yf, 0.0f) * inv[o];
                const int q = (int)nearbyintf(fminf(t, 127.0f));
                if (q > best[o]) best[o] = q;
            }
        }
        for (int o = 0; o < 64; ++o) out[r * 64 + o] = (int8_t)best[o];
    }
}
