/* prep_oracle.c -- CPU restatement of the raw-crop resize that precedes the uint8 normalisation.
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the HIP preprocessing kernels (loaded by tests/ and the
 * CPU-baseline leg of bench.py), never part of the product.
 *
 * One stack = the slices [k0, k1) of a series region (K slices of hr x wr stored uint16 values),
 * each cropped to the box (y0, y1, x0, x1) and resized to img x img in float32, exactly as the
 * reference's GPU path computes it (src/knee/data/raw_crop.py:492-549, payloads_to_uint8_torch):
 *   rescale   v = (float)u * slope + intercept, product then sum in float32, when a [K][2] table is
 *             given (raw_crop.py:520-522; the reference rounds its float64 table to float32 first);
 *   identity  box already img x img: the values themselves (raw_crop.py:426-427);
 *   area      box taller than img: cv2 INTER_AREA tables (raw_crop.py:347-381, `_area_taps`), columns
 *             first then rows, every product and sum rounded separately, in table order, including
 *             the zero-weight padding taps (raw_crop.py:396-416, `area_resize_torch`); an axis already
 *             at img passes through;
 *   bilinear  otherwise: torch.nn.functional.interpolate(mode="bilinear", align_corners=False,
 *             antialias=False) (raw_crop.py:431-432) as PyTorch's GPU kernel computes it
 *             (aten/src/ATen/native/cuda/UpSampleBilinear2d.cu `upsample_bilinear2d_out_frame`,
 *             UpSample.h `area_pixel_compute_source_index`): scale = (float)in / out, source index
 *             fma(scale, d + 0.5, -0.5) clamped at 0, lambdas in float32, and
 *             val = fma(h0, fma(w0, a, w1 * b), h1 * fma(w0, c, w1 * d)) -- the contraction the
 *             compiler makes of the kernel's `h0 * (w0 * a + w1 * b) + h1 * (w0 * c + w1 * d)`.
 * Build: oracle/Makefile (gcc, -ffp-contract=off: only the explicit fmaf are fused).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

/* cv2's INTER_AREA table for one axis (src/knee/data/raw_crop.py:347-381): for each output index d,
 * up to maxT (source index, float32 weight) pairs, zero-padded to the longest row.  Python float
 * arithmetic is IEEE double, so every step below is the same operation on the same values.
 * Returns the number of taps T (or -1 if a row needs more than maxT). */
int orc_area_taps(int ssize, int dsize, int maxT, int32_t* idx, float* w) {
    const double scale = 1.0 / ((double)dsize / (double)ssize);
    int T = 0;
    int32_t ti[64];
    float tw[64];
    for (int pass = 0; pass < 2; ++pass) {
        for (int dx = 0; dx < dsize; ++dx) {
            const double fsx1 = (double)dx * scale;
            const double fsx2 = fsx1 + scale;
            const double rem = (double)ssize - fsx1;
            const double cw = rem < scale ? rem : scale;
            long sx1 = (long)ceil(fsx1), sx2 = (long)floor(fsx2);
            if (sx2 > ssize - 1) sx2 = ssize - 1;
            if (sx1 > sx2) sx1 = sx2;
            int n = 0;
            if ((double)sx1 - fsx1 > 1e-3) {
                if (n < 64) { ti[n] = (int32_t)(sx1 - 1); tw[n] = (float)(((double)sx1 - fsx1) / cw); }
                ++n;
            }
            for (long sx = sx1; sx < sx2; ++sx) {
                if (n < 64) { ti[n] = (int32_t)sx; tw[n] = (float)(1.0 / cw); }
                ++n;
            }
            if (fsx2 - (double)sx2 > 1e-3) {
                double a = fsx2 - (double)sx2;
                if (1.0 < a) a = 1.0;
                if (cw < a) a = cw;
                if (n < 64) { ti[n] = (int32_t)sx2; tw[n] = (float)(a / cw); }
                ++n;
            }
            if (pass == 0) {
                if (n > T) T = n;
                continue;
            }
            for (int j = 0; j < T; ++j) {
                idx[dx * T + j] = j < n ? ti[j] : 0;
                w[dx * T + j] = j < n ? tw[j] : 0.0f;
            }
        }
        if (pass == 0 && (T > maxT || T > 64)) return -1;
    }
    return T;
}

static float src_value(const uint16_t* region, const float* resc, int hr, int wr, int k, int y,
                       int x) {
    const float u = (float)region[((int64_t)k * hr + y) * wr + x];
    if (!resc) return u;
    const float p = u * resc[2 * k];
    return p + resc[2 * k + 1];
}

/* torch's source index for output index d (align_corners=False, not cubic). */
static float src_index(float scale, int d) {
    const float s = fmaf(scale, (float)d + 0.5f, -0.5f);
    return s < 0.0f ? 0.0f : s;
}

/* Slices [k0, k1) of the stack into out [K][img][img] (the other slices are not written).
 * Returns 0, or -1 if an area table is longer than 16 taps. */
int orc_resize_stack(const uint16_t* region, int K, int hr, int wr, const float* resc, int y0, int y1,
                     int x0, int x1, int img, int k0, int k1, float* out) {
    const int h = y1 - y0, w = x1 - x0;
    (void)K;
    if (h == img && w == img) {
        for (int k = k0; k < k1; ++k)
            for (int y = 0; y < img; ++y)
                for (int x = 0; x < img; ++x)
                    out[((int64_t)k * img + y) * img + x] =
                        src_value(region, resc, hr, wr, k, y0 + y, x0 + x);
        return 0;
    }
    if (h > img) {
        enum { MT = 16 };
        static int32_t ix[4096 * MT], iy[4096 * MT];
        static float wx[4096 * MT], wy[4096 * MT];
        if (img > 4096) return -1;
        int Tx = 0;
        if (w != img && (Tx = orc_area_taps(w, img, MT, ix, wx)) < 0) return -1;
        const int Ty = orc_area_taps(h, img, MT, iy, wy);
        if (Ty < 0) return -1;
        const int wi = w != img ? img : w;
        float* inter = (float*)malloc(sizeof(float) * (size_t)h * (size_t)wi);
        if (!inter) return -1;
        for (int k = k0; k < k1; ++k) {
            for (int y = 0; y < h; ++y)
                for (int dx = 0; dx < wi; ++dx) {
                    float acc;
                    if (w == img) {
                        acc = src_value(region, resc, hr, wr, k, y0 + y, x0 + dx);
                    } else {
                        acc = 0.0f;
                        for (int j = 0; j < Tx; ++j) {
                            const float p = src_value(region, resc, hr, wr, k, y0 + y,
                                                      x0 + ix[dx * Tx + j]) * wx[dx * Tx + j];
                            acc = acc + p;
                        }
                    }
                    inter[(int64_t)y * wi + dx] = acc;
                }
            for (int dy = 0; dy < img; ++dy)
                for (int dx = 0; dx < wi; ++dx) {
                    float acc = 0.0f;
                    for (int j = 0; j < Ty; ++j) {
                        const float p = inter[(int64_t)iy[dy * Ty + j] * wi + dx] * wy[dy * Ty + j];
                        acc = acc + p;
                    }
                    out[((int64_t)k * img + dy) * img + dx] = acc;
                }
        }
        free(inter);
        return 0;
    }
    const float rh = (float)h / (float)img, rw = (float)w / (float)img;
    for (int k = k0; k < k1; ++k)
        for (int dy = 0; dy < img; ++dy) {
            const float hr1 = src_index(rh, dy);
            const int h1 = (int)hr1, h1p = h1 < h - 1 ? 1 : 0;
            const float l1 = hr1 - (float)h1, l0 = 1.0f - l1;
            for (int dx = 0; dx < img; ++dx) {
                const float wr1 = src_index(rw, dx);
                const int w1 = (int)wr1, w1p = w1 < w - 1 ? 1 : 0;
                const float m1 = wr1 - (float)w1, m0 = 1.0f - m1;
                const float a = src_value(region, resc, hr, wr, k, y0 + h1, x0 + w1);
                const float b = src_value(region, resc, hr, wr, k, y0 + h1, x0 + w1 + w1p);
                const float c = src_value(region, resc, hr, wr, k, y0 + h1 + h1p, x0 + w1);
                const float d = src_value(region, resc, hr, wr, k, y0 + h1 + h1p, x0 + w1 + w1p);
                const float top = fmaf(m0, a, m1 * b), bot = fmaf(m0, c, m1 * d);
                out[((int64_t)k * img + dy) * img + dx] = fmaf(l0, top, l1 * bot);
            }
        }
    return 0;
}
