// gfx950 kernels of the upstream preprocessing (raw uint16 crops -> resize -> exact 1/99 percentiles
// -> uint8 -> side flip) and their C ABI, d8s_prep / d8s_prep_resize (include/d8s_hip.h).
//
// The work is byte and float bookkeeping bound by memory, not matrix work.  Design:
//   - uint16 regions (kind 0): the first pass evaluates the resize from the region and writes the
//     float32 stacks once to the workspace's scratch while it counts the first radix level; the
//     later passes read the stored stacks (k_prep_hist<1, 1, true>, then float_view).  Evaluating
//     the resize again in every pass instead was VALU-bound at about 40 instructions per pixel and
//     2-3x slower.  Float32 stacks (kind 1) are read as given by every pass;
//   - the order statistics k1, k1+1, k2, k2+1 are selected exactly by a three-level radix histogram
//     of the float's order key (11 + 11 + 10 bits).  Each level is one pass over the stack that
//     counts in LDS and adds the nonzero bins to a global histogram, then one workgroup per stack
//     finds the bins holding the four ranks;  equal ranks share a histogram (at most four per level);
//   - the last pass writes the uint8 value of every pixel (float64 arithmetic, the reference's exact
//     operations) at its flipped position.
// A pass works on blocks of output rows of one slice: the source rows a block needs are resized along x
// once into LDS, then every output pixel combines them along y (the bilinear formula is separable as
// written: fma(h0, top, h1 * bottom) with top and bottom the x interpolations of two source rows).  A
// histogram workgroup runs several blocks of one stack before it adds its LDS counts to the global
// histogram; the final pass runs one block per workgroup.
//
// Numerics (the file is compiled with -ffp-contract=off: only the explicit fmaf are fused):
//   rescale   (float)u * slope, then + intercept (raw_crop.py:520-522);
//   bilinear  torch's upsample_bilinear2d kernel with the fused multiply-adds its compiler forms
//             (src index fma(scale, d + 0.5, -0.5) clamped at 0; fma(h0, fma(w0, a, w1 b), h1 fma(w0, c,
//             w1 d))), raw_crop.py:431-432;
//   area      cv2's INTER_AREA tables (raw_crop.py:347-381) in float64 on the device, columns then rows,
//             each product and sum rounded, in table order with the zero padding taps
//             (raw_crop.py:396-416);
//   uint8     numpy's _lerp on the order statistics (float32 difference, float64 product and sum, the
//             t >= 0.5 form), scale = 255 / (hi - lo) (correctly rounded float64 division), then
//             ((double)x - lo) * scale clipped to [0, 255] and truncated (cache.py:319-340).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <string>
#include <type_traits>

#include "d8s_hip.h"
#include "d8s_host.h"

#define DEV __device__ __forceinline__

namespace {

constexpr int NT = 256;                          // threads per workgroup
constexpr int NB1 = 2048, NB2 = 2048, NB3 = 1024;  // radix levels: key bits 31..21, 20..10, 9..0
constexpr int MAX_S = D8S_PREP_MAX_STACKS;
constexpr int MAX_T = D8S_PREP_MAX_TAPS;
constexpr int UP = 4;                            // output pixels per thread step (one 16-byte LDS read)
constexpr int STAGE = 10240;                     // LDS of the block kernels: 40 KB (resized rows + raw rows)

// per-stack workspace block, in 32-bit words
constexpr int W_H1 = 0;
constexpr int W_H2 = W_H1 + NB1;                 // 4 histograms of level 2
constexpr int W_H3 = W_H2 + 4 * NB2;             // 4 histograms of level 3
constexpr int W_NAN = W_H3 + 4 * NB3;            // nonzero if the stack holds a NaN
constexpr int W_SEL1 = W_NAN + 4;                // selection after level 1 (Sel, 16 words)
constexpr int W_SEL2 = W_SEL1 + 16;              // selection after level 2
constexpr int W_CLEAR = W_SEL2 + 16;             // words cleared at the start of d8s_prep
constexpr int W_TAPS = (W_CLEAR + 63) / 64 * 64; // area tables: ix, wx [img][Tx], iy, wy [img][Ty]
constexpr uint64_t WS_HEAD = 1024;               // D8sPrepStat[16] (512 bytes), then the stacks

static_assert(sizeof(D8sPrepStat) * MAX_S <= WS_HEAD, "stat header");

uint64_t stack_words(int img) { return ((uint64_t)W_TAPS + 4ull * img * MAX_T + 63) / 64 * 64; }

enum Mode { M_IDENT = 0, M_BILIN = 1, M_AREA = 2, M_FLOAT = 3 };

// The selection a level leaves for the next: `nslot` distinct key prefixes (one histogram each at the
// next level), and for each of the 4 ranks its slot and its rank among the keys of that prefix.
struct Sel {
    uint32_t nslot;
    uint32_t pre[4];
    uint32_t slot[4];
    uint32_t res[4];
    uint32_t pad_[3];
};
static_assert(sizeof(Sel) == 64, "Sel is 16 words");

struct PStack {
    const void* src;
    const float* resc;
    void* out;
    uint32_t* ws;
    float* sc;           // kind 0 in d8s_prep: the resized stack (slice kk at sc + kk img img)
    int K, hr, wr, y0, x0, h, w, k0, k1, flip, mode, Tx, Ty, r1, r2;
    float rh, rw;
    double g1, g2;
    int rb, bps, nblk;   // output rows per block, blocks per slice, blocks of the slices [k0, k1)
    int ns_max, rp, dpl; // source rows a block may read; LDS dwords per staged raw row; per lane
    int dbuf;            // 1: two raw buffers (block b+1 copied during block b's x pass); 0: one
    float inv_rp;
    int hb, hb2, nb;     // blocks per workgroup: histogram level 1, levels 2-3, final pass
    int wg_hist, wg_hist2, wg_norm;  // first workgroup of this stack in each grid
};

struct PArgs {
    PStack s[MAX_S];
    D8sPrepStat* stat;
    int n, img, upr;     // stacks, output side, UP-pixel units per output row (img / UP)
    float inv_img, inv_upr;
};

// ---- float order keys -------------------------------------------------------------------------
// unsigned key with the order of the floats: sign bit set for positives, all bits flipped for
// negatives.
DEV uint32_t order_key(float v) {
    const uint32_t b = __float_as_uint(v);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
DEV float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// ---- cv2 INTER_AREA table, one output index (raw_crop.py:347-381) --------------------------------
// Python float arithmetic is IEEE double: the same operations in the same order.  Writes up to
// `cap` taps (when idx != nullptr) and returns the row's number of taps.
__host__ __device__ inline int area_row(int ssize, int dsize, int d, int cap, int32_t* idx, float* w) {
    const double scale = 1.0 / ((double)dsize / (double)ssize);
    const double fsx1 = (double)d * scale;
    const double fsx2 = fsx1 + scale;
    const double rem = (double)ssize - fsx1;
    const double cw = rem < scale ? rem : scale;
    long sx1 = (long)ceil(fsx1), sx2 = (long)floor(fsx2);
    if (sx2 > ssize - 1) sx2 = ssize - 1;
    if (sx1 > sx2) sx1 = sx2;
    int n = 0;
    if ((double)sx1 - fsx1 > 1e-3) {
        if (idx && n < cap) { idx[n] = (int32_t)(sx1 - 1); w[n] = (float)(((double)sx1 - fsx1) / cw); }
        ++n;
    }
    for (long sx = sx1; sx < sx2; ++sx) {
        if (idx && n < cap) { idx[n] = (int32_t)sx; w[n] = (float)(1.0 / cw); }
        ++n;
    }
    if (fsx2 - (double)sx2 > 1e-3) {
        double a = fsx2 - (double)sx2;
        if (1.0 < a) a = 1.0;
        if (cw < a) a = cw;
        if (idx && n < cap) { idx[n] = (int32_t)sx2; w[n] = (float)(a / cw); }
        ++n;
    }
    return n;
}

int area_taps_max(int ssize, int dsize) {
    int T = 0;
    for (int d = 0; d < dsize; ++d) {
        const int n = area_row(ssize, dsize, d, 0, nullptr, nullptr);
        if (n > T) T = n;
    }
    return T;
}

// ---- evaluation of 8 output pixels -------------------------------------------------------------
DEV float src_index(float scale, int d) {
    const float s = __builtin_fmaf(scale, (float)d + 0.5f, -0.5f);
    return s < 0.0f ? 0.0f : s;
}

// n / d for 0 <= n < 2^22 and 1 <= d <= 4096 (inv = 1 / d): a float estimate, corrected.
DEV int fdiv(int n, int d, float inv) {
    int q = (int)((float)n * inv);
    q -= q * d > n ? 1 : 0;
    q += (q + 1) * d <= n ? 1 : 0;
    return q;
}

// A block: output rows [r0, r0 + rb) of slice kk, reading source rows [s0, s0 + ns) of the crop.
struct Geo {
    int kk, r0, rb, s0, ns;
};

template <int MODE>
DEV Geo block_geo(const PStack& st, const PArgs& a, int b) {
    Geo g;
    const int q = b / st.bps;
    g.kk = st.k0 + q;
    g.r0 = (b - q * st.bps) * st.rb;
    g.rb = min(st.rb, a.img - g.r0);
    if constexpr (MODE == M_FLOAT) {
        g.s0 = 0;
        g.ns = 0;
        return g;
    } else {
        int s1;
        if constexpr (MODE == M_IDENT) {
            g.s0 = g.r0;
            s1 = g.r0 + g.rb;
        } else if constexpr (MODE == M_BILIN) {
            g.s0 = (int)src_index(st.rh, g.r0);
            const int h1 = (int)src_index(st.rh, g.r0 + g.rb - 1);
            s1 = h1 + (h1 < st.h - 1 ? 1 : 0) + 1;
        } else {
            const int32_t* iy = (const int32_t*)st.ws + W_TAPS + 2 * a.img * st.Tx;
            const float* wy = (const float*)(iy + a.img * st.Ty);
            const int last = g.r0 + g.rb - 1;
            int t = st.Ty - 1;
            while (t > 0 && !(wy[last * st.Ty + t] > 0.0f)) --t;   // the padding taps have weight 0
            g.s0 = iy[g.r0 * st.Ty];
            s1 = iy[last * st.Ty] + t + 1;
        }
        g.ns = min(s1 - g.s0, st.ns_max);
        return g;
    }
}

constexpr int NW = NT / 64;  // waves per workgroup

// Copies source rows [s0, s0 + ns) of a block, crop columns [0, w), to LDS with gfx950's
// global_load_lds (memory to LDS without registers).  Wave v copies rows v, v + NW, ...; row r starts
// at element e_r = e0 + r wr of the dword-aligned series base, and its dwords [0, nd) from element
// e_r & ~1 (the first and last may hold 2 bytes of the neighbouring rows, nothing outside the dwords
// that hold the row) go to s_raw[r][0 .. nd); lanes past nd repeat the last dword, inside the row's
// 64-dword-padded slot.  The caller waits for the copies (vmcnt) and synchronises.
DEV void raw_stage(const PStack& st, const Geo& g, uint32_t* s_raw) {
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = (int)threadIdx.x & 63;
    const uint32_t* base = (const uint32_t*)((uintptr_t)st.src & ~(uintptr_t)3);
    const int e0 = (int)(((uintptr_t)st.src >> 1) & 1u) + (g.kk * st.hr + st.y0 + g.s0) * st.wr + st.x0;
    const int pitch = st.dpl * 64;
    for (int r = wv; r < g.ns; r += NW) {
        const int er = e0 + r * st.wr;
        const int nd = ((er & 1) + st.w + 1) >> 1;
        const uint32_t* row = base + (er >> 1);
        for (int m = 0; m < st.dpl; ++m) {
            const int d = min(lane + 64 * m, nd - 1);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(row + d),
                                             (__attribute__((address_space(3))) void*)(s_raw + r * pitch + 64 * m),
                                             4, 0, 0);
        }
    }
}

template <bool HAS>
DEV float rescale(uint32_t u, float sl, float ic) {
    const float f = (float)u;
    if constexpr (!HAS) {
        return f;
    } else {
        const float p = f * sl;
        return p + ic;
    }
}

// The values of every block b0 .. b1-1 of stack st, UP consecutive pixels of a row at a time, handed to
// f(kk, dy, dx0, v).  Region modes: a block's raw rows are copied to LDS (two buffers: the copy of block
// b+1 runs while block b is computed), resized along x into
// s_st [ns][img] (bilinear `top`/`bottom` values fma(w0, a, w1 b), area column sums, identity values),
// and every pixel combines them along y.  A thread keeps the same output columns in the x pass, so
// their interpolation positions are computed once.  The workgroup calls this uniformly (it holds
// barriers).
//
// The area taps of an output index are consecutive source indices (raw_crop.py:361-369), so a tap's
// source is the first index + t; a zero-weight padding tap then reads a neighbour instead of index 0,
// which changes nothing for finite values (x * 0 = +-0 added to a sum that is never -0).
template <int MODE, bool HAS, bool WROW, class F>
DEV void run_blocks(const PStack& st, const PArgs& a, int b0, int b1, float* s_st, F&& f) {
    const int img = a.img;
    if constexpr (MODE == M_FLOAT) {
        // a thread's units u = tid + NT i of a block in batches of FB: the batch's loads are issued
        // before any of its values is used (the histogram passes' LDS atomics would otherwise keep
        // each load behind the previous unit's counting); units past the block load its last unit
        // again and are not used
        constexpr int FB = 4;
        for (int b = b0; b < b1; ++b) {
            const Geo g = block_geo<MODE>(st, a, b);
            const int n = g.rb * a.upr;
            const float* base = (const float*)st.src + (int64_t)g.kk * img * img;
            for (int u0 = threadIdx.x; u0 < n; u0 += FB * NT) {
                float4 x[FB];
                int dy[FB], dx0[FB];
#pragma unroll
                for (int i = 0; i < FB; ++i) {
                    const int u = min(u0 + i * NT, n - 1);
                    const int row = fdiv(u, a.upr, a.inv_upr);
                    dx0[i] = (u - row * a.upr) * UP;
                    dy[i] = g.r0 + row;
                    x[i] = *(const float4*)(base + (int64_t)dy[i] * img + dx0[i]);
                }
#pragma unroll
                for (int i = 0; i < FB; ++i) {
                    if (u0 + i * NT < n) {
                        float v[UP] = {x[i].x, x[i].y, x[i].z, x[i].w};
                        f(g.kk, dy[i], dx0[i], v);
                    }
                }
            }
        }
        return;
    } else {
        constexpr int CMAX = 4;                      // output columns per thread in the x pass (img <= 1024)
        const int32_t* ix = (const int32_t*)st.ws + W_TAPS;
        const float* wx = (const float*)(ix + img * st.Tx);
        const int32_t* iy = (const int32_t*)(wx + img * st.Tx);
        const float* wy = (const float*)(iy + img * st.Ty);
        const int pitch = st.dpl * 64;               // dwords per staged raw row
        // raw buffers: with two, block b+1 is copied during block b's x pass; with one, during its
        // y pass
        uint32_t* s_raw0 = (uint32_t*)(s_st + st.ns_max * img);
        uint32_t* s_raw1 = st.dbuf ? s_raw0 + st.ns_max * pitch : s_raw0;
        // x-pass mapping: img >= NT: columns tid + c NT, every row; img < NT: column tid % img, rows
        // tid / img + P j (threads beyond P img rest)
        const int P = img >= NT ? 1 : NT / img;
        const int ph = img >= NT ? 0 : (int)threadIdx.x / img;
        const int col0 = (int)threadIdx.x - ph * img;
        const bool xact = ph < P;
        int ca[CMAX], cb[CMAX];          // uint16 index of the two taps (bilinear) / first tap (area)
        float cm0[CMAX], cm1[CMAX];      // bilinear weights / area: first and middle tap weights
        float cwl[CMAX];                 // area: last tap weight; cb = number of real taps
#pragma unroll
        for (int c = 0; c < CMAX; ++c) {
            const int dx = min(col0 + c * NT, img - 1);
            ca[c] = cb[c] = dx;
            cm0[c] = cm1[c] = 0.0f;
            if constexpr (MODE == M_BILIN) {
                const float sx = src_index(st.rw, dx);
                const int w1 = (int)sx;
                ca[c] = w1;
                cb[c] = w1 + (w1 < st.w - 1 ? 1 : 0);
                cm1[c] = sx - (float)w1;
                cm0[c] = 1.0f - cm1[c];
            } else if constexpr (MODE == M_AREA) {
                // a table row is [first, middle ..., last] with equal middle weights
                // (raw_crop.py:361-369), then zero padding: keep first / middle / last and the count
                cwl[c] = 0.0f;
                if (st.w != img) {
                    const float* tw = wx + dx * st.Tx;
                    ca[c] = ix[dx * st.Tx];
                    int n = 0;
                    for (int t = 0; t < st.Tx; ++t) n += tw[t] > 0.0f ? 1 : 0;
                    cb[c] = n;
                    cm0[c] = tw[0];
                    cm1[c] = n > 2 ? tw[1] : 0.0f;
                    cwl[c] = tw[n > 0 ? n - 1 : 0];
                }
            }
        }
        // uint16 parity of the crop rows: row index q starts at element (src / 2) + q wr + x0
        const int par0 = (int)((((uintptr_t)st.src >> 1) + (uintptr_t)st.x0) & 1u);
        const int last = st.ns_max - 1;
        // y-pass mapping: RS rows at a time, thread (tr, tc); with WROW (a row is a multiple of 64
        // units) every wave works on one row, so the row quantities are wave-uniform
        const int RS = NT / a.upr;
        int tr = (int)threadIdx.x / a.upr;
        if constexpr (WROW) tr = __builtin_amdgcn_readfirstlane(tr);
        const int dx0 = ((int)threadIdx.x - ((int)threadIdx.x / a.upr) * a.upr) * UP;
        const bool yact = tr < RS;
        // bilinear: the taps and weights of the thread's UP output columns dx0 .. dx0 + UP - 1
        int ba[UP], bb[UP];
        float bw0[UP], bw1[UP];
        if constexpr (MODE == M_BILIN) {
#pragma unroll
            for (int i = 0; i < UP; ++i) {
                const float sx = src_index(st.rw, dx0 + i);
                const int w1 = (int)sx;
                ba[i] = w1;
                bb[i] = w1 + (w1 < st.w - 1 ? 1 : 0);
                bw1[i] = sx - (float)w1;
                bw0[i] = 1.0f - bw1[i];
            }
        }
        Geo nxt = block_geo<MODE>(st, a, b0);
        raw_stage(st, nxt, s_raw0);
        for (int b = b0; b < b1; ++b) {
            const Geo g = nxt;
            const uint16_t* raw16 = (const uint16_t*)((b - b0) & 1 ? s_raw1 : s_raw0);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (st.dbuf && b + 1 < b1) {
                nxt = block_geo<MODE>(st, a, b + 1);
                raw_stage(st, nxt, (b - b0) & 1 ? s_raw0 : s_raw1);
            }
            const float sl = HAS ? st.resc[2 * g.kk] : 1.0f, ic = HAS ? st.resc[2 * g.kk + 1] : 0.0f;
            const int e0 = par0 + (g.kk * st.hr + st.y0 + g.s0) * st.wr;
            if constexpr (MODE == M_BILIN) {
                // one pass: thread (tr, tc) walks the contiguous rows tr rpg .. (tr + 1) rpg - 1 of the
                // block down its UP columns and keeps the horizontal interpolations of the two source
                // rows it combines in registers (consecutive output rows mostly share them when
                // upsampling); the same operations as the x and y passes below, in the same order
                if (yact) {
                    const int rpg = (g.rb + RS - 1) / RS;
                    const int rr1 = min(g.rb, (tr + 1) * rpg);
                    int cq0 = -1, cq1 = -1;
                    float X0[UP], X1[UP];
                    auto xrow = [&](int q, float* X) {
                        const uint16_t* row = raw16 + q * 2 * pitch + ((e0 + q * st.wr) & 1);
#pragma unroll
                        for (int i = 0; i < UP; ++i)
                            X[i] = __builtin_fmaf(bw0[i], rescale<HAS>(row[ba[i]], sl, ic),
                                                  bw1[i] * rescale<HAS>(row[bb[i]], sl, ic));
                    };
                    for (int rr = tr * rpg; rr < rr1; ++rr) {
                        const int dy = g.r0 + rr;
                        const float sy = src_index(st.rh, dy);
                        const int h1 = (int)sy;
                        const int h1p = h1 < st.h - 1 ? 1 : 0;
                        const float l1 = sy - (float)h1, l0 = 1.0f - l1;
                        const int q0 = min(h1 - g.s0, last), q1 = min(h1 + h1p - g.s0, last);
                        if (q0 != cq0) {
                            if (q0 == cq1) {
#pragma unroll
                                for (int i = 0; i < UP; ++i) X0[i] = X1[i];
                            } else {
                                xrow(q0, X0);
                            }
                            cq0 = q0;
                            cq1 = -1;
                        }
                        if (q1 != cq1) {
                            if (q1 == q0) {
#pragma unroll
                                for (int i = 0; i < UP; ++i) X1[i] = X0[i];
                            } else {
                                xrow(q1, X1);
                            }
                            cq1 = q1;
                        }
                        float v[UP];
#pragma unroll
                        for (int i = 0; i < UP; ++i) v[i] = __builtin_fmaf(l0, X0[i], l1 * X1[i]);
                        f(g.kk, dy, dx0, v);
                    }
                }
                if (!st.dbuf && b + 1 < b1) {
                    __syncthreads();                      // every thread is done with this block's rows
                    nxt = block_geo<MODE>(st, a, b + 1);
                    raw_stage(st, nxt, s_raw0);
                }
                continue;
            }
            if (xact) {
                for (int r = ph; r < g.ns; r += P) {
                    const uint16_t* row = raw16 + r * 2 * pitch + ((e0 + r * st.wr) & 1);
                    float* dst = s_st + r * img;
#pragma unroll
                    for (int c = 0; c < CMAX; ++c) {
                        const int dx = col0 + c * NT;
                        if (c * NT < img && dx < img) {
                            float v;
                            if constexpr (MODE == M_IDENT) {
                                v = rescale<HAS>(row[dx], sl, ic);
                            } else if constexpr (MODE == M_BILIN) {
                                const float xa = rescale<HAS>(row[ca[c]], sl, ic);
                                const float xb = rescale<HAS>(row[cb[c]], sl, ic);
                                v = __builtin_fmaf(cm0[c], xa, cm1[c] * xb);
                            } else if (st.w == img) {
                                v = rescale<HAS>(row[dx], sl, ic);
                            } else {
                                // every tap of the table in order; the padding taps (weight 0) read
                                // a neighbour (x * 0 adds nothing to a finite sum)
                                v = 0.0f;
                                const uint16_t* tp = row + ca[c];
                                const int lim = st.w - 1 - ca[c];
                                for (int t = 0; t < st.Tx; ++t) {
                                    const float wt = t == 0 ? cm0[c]
                                                   : t >= cb[c] ? 0.0f
                                                   : t == cb[c] - 1 ? cwl[c] : cm1[c];
                                    const float p = rescale<HAS>(tp[min(t, lim)], sl, ic) * wt;
                                    v = v + p;
                                }
                            }
                            dst[dx] = v;
                        }
                    }
                }
            }
            __syncthreads();
            if (!st.dbuf && b + 1 < b1) {
                nxt = block_geo<MODE>(st, a, b + 1);
                raw_stage(st, nxt, s_raw0);
            }
            // combine along y: thread (row phase tr, unit column tc) runs rows tr, tr + RS, ...
            if (yact) {
                for (int rr = tr; rr < g.rb; rr += RS) {
                    const int dy = g.r0 + rr;
                    float v[UP];
                    if constexpr (MODE == M_IDENT) {
                        const float* p = s_st + min(dy - g.s0, last) * img + dx0;
#pragma unroll
                        for (int i = 0; i < UP; ++i) v[i] = p[i];
                    } else if constexpr (MODE == M_BILIN) {
                        const float sy = src_index(st.rh, dy);
                        const int h1 = (int)sy;
                        const int h1p = h1 < st.h - 1 ? 1 : 0;
                        const float l1 = sy - (float)h1, l0 = 1.0f - l1;
                        const float* p0 = s_st + min(h1 - g.s0, last) * img + dx0;
                        const float* p1 = s_st + min(h1 + h1p - g.s0, last) * img + dx0;
#pragma unroll
                        for (int i = 0; i < UP; ++i) v[i] = __builtin_fmaf(l0, p0[i], l1 * p1[i]);
                    } else {
                        // the row's real taps in table order (its zero-weight padding taps add +0 to
                        // a finite sum and are skipped: their source row need not be staged)
                        const int y0t = iy[dy * st.Ty] - g.s0;
                        const float* tw = wy + dy * st.Ty;
#pragma unroll
                        for (int i = 0; i < UP; ++i) v[i] = 0.0f;
                        for (int j = 0; j < st.Ty; ++j) {
                            const float wyj = tw[j];
                            if (!(wyj > 0.0f)) break;
                            const float* p = s_st + min(y0t + j, last) * img + dx0;
#pragma unroll
                            for (int i = 0; i < UP; ++i) {
                                const float q = p[i] * wyj;
                                v[i] = v[i] + q;
                            }
                        }
                    }
                    f(g.kk, dy, dx0, v);
                }
            }
            __syncthreads();
        }
    }
}

// REGION: the kernel instance for uint16 regions (kind 0) or for float32 stacks (kind 1).  Runs
// body(mode, rescale, wave-uniform rows) with the stack's mode, whether it has a Rescale and whether
// an output row is a multiple of 64 units as constants.
template <int REGION, class B>
DEV void with_mode(const PStack& st, const PArgs& a, B&& body) {
    using T = std::true_type;
    using N = std::false_type;
    if constexpr (REGION) {
        const bool h = st.resc != nullptr;
        auto go = [&](auto m) {
            if (a.upr % 64 == 0)
                h ? body(m, T{}, T{}) : body(m, N{}, T{});
            else
                h ? body(m, T{}, N{}) : body(m, N{}, N{});
        };
        switch (st.mode) {
            case M_IDENT: go(std::integral_constant<int, M_IDENT>{}); break;
            case M_BILIN: go(std::integral_constant<int, M_BILIN>{}); break;
            default: go(std::integral_constant<int, M_AREA>{}); break;
        }
    } else {
        body(std::integral_constant<int, M_FLOAT>{}, N{}, N{});
    }
}

// grid 0: histogram level 1; 1: levels 2 and 3; 2: final pass and resize
DEV int first_wg(const PStack& p, int grid) { return grid == 0 ? p.wg_hist : grid == 1 ? p.wg_hist2 : p.wg_norm; }

DEV int stack_of(const PArgs& a, int grid) {
    int s = 0;
    for (int i = 1; i < a.n; ++i)
        if ((int)blockIdx.x >= first_wg(a.s[i], grid)) s = i;
    return s;
}

// ---- kernels ------------------------------------------------------------------------------------

// Clears the histograms and selections of every stack, writes the zeros of the output slices outside
// [k0, k1) (d8s_prep: clear = 1) and builds the area tables.
__global__ void __launch_bounds__(NT) k_prep_setup(PArgs a, int clear) {
    const PStack& st = a.s[blockIdx.y];
    const int gid = blockIdx.x * NT + threadIdx.x, gsz = gridDim.x * NT;
    if (clear) {
        for (int i = gid; i < W_CLEAR; i += gsz) st.ws[i] = 0u;
        const int per = a.img * a.img / 8;            // 8-byte words per slice
        const int outside = (st.K - (st.k1 - st.k0)) * per;
        for (int i = gid; i < outside; i += gsz) {
            int kk = i / per;
            kk = kk < st.k0 ? kk : kk + (st.k1 - st.k0);
            const int ko = st.flip == D8S_FLIP_SLICES ? st.K - 1 - kk : kk;
            ((uint2*)st.out)[(int64_t)ko * per + (i % per)] = make_uint2(0u, 0u);
        }
    }
    if (st.mode != M_AREA) return;
    int32_t* ix = (int32_t*)st.ws + W_TAPS;
    float* wx = (float*)(ix + a.img * st.Tx);
    int32_t* iy = (int32_t*)(wx + a.img * st.Tx);
    float* wy = (float*)(iy + a.img * st.Ty);
    for (int d = gid; d < a.img; d += gsz) {
        int32_t ti[MAX_T];
        float tw[MAX_T];
        if (st.w != a.img) {
            const int n = area_row(st.w, a.img, d, MAX_T, ti, tw);
            for (int j = 0; j < st.Tx; ++j) {
                ix[d * st.Tx + j] = j < n ? ti[j] : 0;
                wx[d * st.Tx + j] = j < n ? tw[j] : 0.0f;
            }
        }
        const int n = area_row(st.h, a.img, d, MAX_T, ti, tw);
        for (int j = 0; j < st.Ty; ++j) {
            iy[d * st.Ty + j] = j < n ? ti[j] : 0;
            wy[d * st.Ty + j] = j < n ? tw[j] : 0.0f;
        }
    }
}

// One radix level over the blocks [b0, b0 + hb) of one stack.
template <int LEVEL, int REGION, bool STORE = false>
__global__ void __launch_bounds__(NT) k_prep_hist(PArgs a) {
    constexpr int NB = LEVEL == 1 ? NB1 : LEVEL == 2 ? NB2 : NB3;
    constexpr int NH = LEVEL == 1 ? 1 : 2;    // LDS histograms; slots 2 and 3 (rare) count in memory
    __shared__ uint32_t s_h[NH * NB];
    __shared__ float s_st[REGION ? STAGE : 1];
    const int s = stack_of(a, LEVEL == 1 ? 0 : 1);
    const PStack& st = a.s[s];
    for (int i = threadIdx.x; i < NH * NB; i += NT) s_h[i] = 0u;
    uint32_t nslot = 0, pre[4] = {0u, 0u, 0u, 0u};
    if constexpr (LEVEL > 1) {
        const Sel* sel = (const Sel*)(st.ws + (LEVEL == 2 ? W_SEL1 : W_SEL2));
        nslot = sel->nslot;
#pragma unroll
        for (int t = 0; t < 4; ++t) pre[t] = sel->pre[t];
    }
    __syncthreads();
    const int hb = LEVEL == 1 ? st.hb : st.hb2;
    const int b0 = ((int)blockIdx.x - (LEVEL == 1 ? st.wg_hist : st.wg_hist2)) * hb;
    const int b1 = min(b0 + hb, st.nblk);
    bool nan = false;
    uint32_t run_bin = 0xffffffffu, run_n = 0u;   // the thread's current run of one histogram index
    uint32_t* gh = st.ws + (LEVEL == 1 ? W_H1 : LEVEL == 2 ? W_H2 : W_H3);
    auto run_flush = [&]() {
        if (LEVEL == 1 || run_bin < (uint32_t)(NH * NB))
            atomicAdd(&s_h[run_bin], run_n);
        else
            atomicAdd(gh + run_bin, run_n);
    };
    auto count = [&](int kk, int dy, int dx0, const float* v) {
        if constexpr (STORE)
            *(float4*)(st.sc + ((int64_t)kk * a.img + dy) * a.img + dx0) = make_float4(v[0], v[1], v[2], v[3]);
        // The UP values of a unit are counted in one step when every counted one continues the
        // thread's run (the common case: no branch taken); otherwise value by value.
        if constexpr (LEVEL == 1) {
            // a thread's values are neighbours (UP along x, then the next row of its column), so they
            // mostly share a (coarse) level-1 bin: the thread counts a run in a register and adds it
            // to LDS when the bin changes
            uint32_t b[UP];
            bool same = true;
#pragma unroll
            for (int i = 0; i < UP; ++i) {
                nan |= v[i] != v[i];
                b[i] = order_key(v[i]) >> 21;
                same &= b[i] == run_bin;
            }
            if (same) {
                run_n += UP;
                return;
            }
#pragma unroll
            for (int i = 0; i < UP; ++i) {
                if (b[i] != run_bin) {
                    if (run_n) run_flush();
                    run_bin = b[i];
                    run_n = 0u;
                }
                ++run_n;
            }
            return;
        }
        // the keys under one of the slots' prefixes (unused slots hold 0xffffffff, which no key has at
        // these levels), counted in runs as at level 1 (runs of equal values, e.g. a zero background,
        // are common); index = slot * NB + bin, slots from NH on count in memory
        uint32_t idx[UP];
        bool ok[UP], same = true;
        uint32_t add = 0u;
#pragma unroll
        for (int i = 0; i < UP; ++i) {
            const uint32_t k = order_key(v[i]);
            const uint32_t p = LEVEL == 2 ? k >> 21 : k >> 10;
            const uint32_t bin = LEVEL == 2 ? (k >> 10) & (NB2 - 1) : k & (NB3 - 1);
            ok[i] = p == pre[0] || p == pre[1] || p == pre[2] || p == pre[3];
            const uint32_t t = p == pre[0] ? 0u : p == pre[1] ? 1u : p == pre[2] ? 2u : 3u;
            idx[i] = t * NB + bin;
            same &= !ok[i] || idx[i] == run_bin;
            add += ok[i] ? 1u : 0u;
        }
        if (same) {
            run_n += add;
            return;
        }
#pragma unroll
        for (int i = 0; i < UP; ++i) {
            if (ok[i]) {
                if (idx[i] != run_bin) {
                    if (run_n) run_flush();
                    run_bin = idx[i];
                    run_n = 0u;
                }
                ++run_n;
            }
        }
    };
    with_mode<REGION>(st, a, [&](auto m, auto h, auto w) {
        run_blocks<decltype(m)::value, decltype(h)::value, decltype(w)::value>(st, a, b0, b1, s_st, count);
    });
    if (run_n) run_flush();
    if constexpr (LEVEL == 1) {
        if (__ballot(nan) != 0ull && (int)__lane_id() == 0) atomicOr(st.ws + W_NAN, 1u);
    }
    __syncthreads();
    const int nh = LEVEL == 1 ? 1 : min((int)nslot, NH);
    for (int i = threadIdx.x; i < nh * NB; i += NT) {
        const uint32_t c = s_h[i];
        if (c) atomicAdd(gh + i, c);
    }
}

// Exclusive prefix sum over the workgroup (one value per thread) and the total.
DEV uint32_t block_excl_scan(uint32_t x, uint32_t* s_w, uint32_t& total) {
    const int lane = __lane_id(), wv = threadIdx.x >> 6;
    uint32_t incl = x;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
    }
    if (lane == 63) s_w[wv] = incl;
    __syncthreads();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
        const uint32_t c = s_w[i];
        base += i < wv ? c : 0u;
        tot += c;
    }
    __syncthreads();
    total = tot;
    return base + incl - x;
}

// The bins holding the 4 ranks at one level (one workgroup per stack); the last level also derives
// the percentiles, the scale and the bad flag.
template <int LEVEL>
__global__ void __launch_bounds__(NT) k_prep_select(PArgs a) {
    constexpr int NB = LEVEL == 1 ? NB1 : LEVEL == 2 ? NB2 : NB3;
    constexpr int PER = NB / NT;
    __shared__ uint32_t s_w[NT / 64];
    __shared__ uint32_t s_bin[4], s_res[4];
    const PStack& st = a.s[blockIdx.x];
    uint32_t rank[4], slot[4] = {0u, 0u, 0u, 0u}, pre[4] = {0u, 0u, 0u, 0u};
    if constexpr (LEVEL == 1) {
        rank[0] = (uint32_t)st.r1; rank[1] = (uint32_t)st.r1 + 1u;
        rank[2] = (uint32_t)st.r2; rank[3] = (uint32_t)st.r2 + 1u;
    } else {
        const Sel* sel = (const Sel*)(st.ws + (LEVEL == 2 ? W_SEL1 : W_SEL2));
#pragma unroll
        for (int t = 0; t < 4; ++t) { rank[t] = sel->res[t]; slot[t] = sel->slot[t] & 3u; pre[t] = sel->pre[t]; }
    }
    const uint32_t* gh = st.ws + (LEVEL == 1 ? W_H1 : LEVEL == 2 ? W_H2 : W_H3);
    if (threadIdx.x < 4) { s_bin[threadIdx.x] = 0u; s_res[threadIdx.x] = 0u; }
    for (int t = 0; t < 4; ++t) {
        const uint32_t* h = gh + slot[t] * NB + threadIdx.x * PER;
        uint32_t c[PER], sum = 0;
#pragma unroll
        for (int i = 0; i < PER; ++i) { c[i] = h[i]; sum += c[i]; }
        uint32_t total;
        const uint32_t excl = block_excl_scan(sum, s_w, total);
        if (excl <= rank[t] && rank[t] < excl + sum) {
            uint32_t acc = excl;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                if (rank[t] >= acc && rank[t] < acc + c[i]) {
                    s_bin[t] = threadIdx.x * PER + i;
                    s_res[t] = rank[t] - acc;
                }
                acc += c[i];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    uint32_t key[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t b = s_bin[t];
        key[t] = LEVEL == 1 ? b : LEVEL == 2 ? ((pre[slot[t]] << 11) | b) : ((pre[slot[t]] << 10) | b);
    }
    if constexpr (LEVEL < 3) {
        Sel out;
        out.nslot = 0;
        for (int t = 0; t < 4; ++t) {
            uint32_t j = 0;
            while (j < out.nslot && out.pre[j] != key[t]) ++j;
            if (j == out.nslot) out.pre[out.nslot++] = key[t];
            out.slot[t] = j;
            out.res[t] = s_res[t];
        }
        for (uint32_t j = out.nslot; j < 4; ++j) out.pre[j] = 0xffffffffu;
        out.pad_[0] = out.pad_[1] = out.pad_[2] = 0u;
        Sel* dst = (Sel*)(st.ws + (LEVEL == 1 ? W_SEL1 : W_SEL2));
        *dst = out;
    } else {
        // numpy's _lerp: difference in float32, product and sum in float64, the t >= 0.5 form
        const float pv[2] = {key_float(key[0]), key_float(key[2])};
        const float nx[2] = {key_float(key[1]), key_float(key[3])};
        const double g[2] = {st.g1, st.g2};
        double q[2];
        for (int i = 0; i < 2; ++i) {
            const float diff = nx[i] - pv[i];
            double lerp = (double)pv[i] + (double)diff * g[i];
            if (g[i] >= 0.5) lerp = (double)nx[i] - (double)diff * (1.0 - g[i]);
            q[i] = lerp;
        }
        const double lo = q[0], hi = q[1];
        const bool nan = st.ws[W_NAN] != 0u;
        const bool bad = nan || !isfinite(lo) || !isfinite(hi) || hi <= lo;
        D8sPrepStat r;
        r.lo = lo;
        r.hi = hi;
        r.scale = 255.0 / (hi - lo);
        r.bad = bad ? 1 : 0;
        r.pad_ = 0;
        a.stat[blockIdx.x] = r;
    }
}

// Final pass: uint8 of every pixel, written at its flipped position.
template <int REGION>
__global__ void __launch_bounds__(NT) k_prep_norm(PArgs a) {
    const int s = stack_of(a, 2);
    const PStack& st = a.s[s];
    const D8sPrepStat r = a.stat[s];
    const double nlo = -r.lo;
    __shared__ float s_st[REGION ? STAGE : 1];
    const int b0 = ((int)blockIdx.x - st.wg_norm) * st.nb;
    const int b1 = min(b0 + st.nb, st.nblk);
    uint8_t* out = (uint8_t*)st.out;
    auto write = [&](int kk, int dy, int dx0, const float* v) {
        uint32_t b[UP];
#pragma unroll
        for (int i = 0; i < UP; ++i) {
            // (x - lo) * scale clipped to [0, 255] and truncated; x + (-lo) is x - lo exactly
            double y = (double)v[i] + nlo;
            y = y * r.scale;
            y = __builtin_fmax(y, 0.0);
            y = __builtin_fmin(y, 255.0);
            b[i] = (uint32_t)y;
        }
        const int ko = st.flip == D8S_FLIP_SLICES ? st.K - 1 - kk : kk;
        uint32_t word;
        int xo = dx0;
        if (st.flip == D8S_FLIP_X) {
            xo = a.img - UP - dx0;
            word = b[3] | (b[2] << 8) | (b[1] << 16) | (b[0] << 24);
        } else {
            word = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        }
        *(uint32_t*)(out + ((int64_t)ko * a.img + dy) * a.img + xo) = word;
    };
    if (r.bad) {
        // a stack with non-finite or equal percentiles (or a NaN) is all zeros: its rows of the blocks
        const int per = a.img / 4;
        for (int b = b0; b < b1; ++b) {
            const int q = b / st.bps, kk = st.k0 + q, r0 = (b - q * st.bps) * st.rb;
            const int rb = min(st.rb, a.img - r0);
            const int ko = st.flip == D8S_FLIP_SLICES ? st.K - 1 - kk : kk;
            uint32_t* o = (uint32_t*)(out + ((int64_t)ko * a.img + r0) * a.img);
            for (int i = threadIdx.x; i < rb * per; i += NT) o[i] = 0u;
        }
        return;
    }
    with_mode<REGION>(st, a, [&](auto m, auto h, auto w) {
        run_blocks<decltype(m)::value, decltype(h)::value, decltype(w)::value>(st, a, b0, b1, s_st, write);
    });
}

// The resized float32 values themselves.
__global__ void __launch_bounds__(NT) k_prep_resize(PArgs a) {
    const int s = stack_of(a, 2);
    const PStack& st = a.s[s];
    __shared__ float s_st[STAGE];
    const int b0 = ((int)blockIdx.x - st.wg_norm) * st.nb;
    const int b1 = min(b0 + st.nb, st.nblk);
    float* out = (float*)st.out;
    auto write = [&](int kk, int dy, int dx0, const float* v) {
        *(float4*)(out + ((int64_t)kk * a.img + dy) * a.img + dx0) = make_float4(v[0], v[1], v[2], v[3]);
    };
    with_mode<1>(st, a, [&](auto m, auto h, auto w) {
        run_blocks<decltype(m)::value, decltype(h)::value, decltype(w)::value>(st, a, b0, b1, s_st, write);
    });
}

// ---- grid sampling (geometric TTA view) -------------------------------------------------------
// A thread owns one output pixel for a group of GIMG images: the grid is shared by all images, so the
// source taps and weights are computed once and applied to each image (torch's grid_sampler_2d
// arithmetic in float32, as its compiler contracts it, rounded once to fp16).  KIND 1 gathers the
// images from the uint8 volume through the u / 255 fp16 table; KIND 2 is that gather alone.
constexpr int GIMG = 8;

template <int KIND>
__global__ void __launch_bounds__(NT) k_grid_sample(D8sGridArgs a) {
    __shared__ uint16_t s_lut[256];
    if constexpr (KIND >= 1) {
        if (threadIdx.x < 256) s_lut[threadIdx.x] = ((const uint16_t*)a.lut)[threadIdx.x];
        __syncthreads();
    }
    const int HW = a.H * a.W;
    const int p = blockIdx.x * NT + threadIdx.x;
    const int n0 = blockIdx.y * GIMG, n1 = min(n0 + GIMG, a.N);
    if (p >= HW) return;
    // the image n: its source plane
    // (a slice index outside 0 .. SK-1 is clamped into it, so every read stays inside the volume)
    auto plane = [&](int n) -> int64_t {
        if constexpr (KIND >= 1) {
            const int b = n / a.M, m = n - b * a.M;
            int64_t si = ((const int64_t*)a.slice_idx)[m];
            si = si < 0 ? 0 : si >= a.SK ? (int64_t)a.SK - 1 : si;
            return ((int64_t)b * a.SK + si) * HW;
        } else {
            return (int64_t)n * HW;
        }
    };
    // the GIMG images' planes first (their slice indices are loads), then every gather of every image
    // (loads clamped to the last image, stores predicated), so they are all in flight together
    int64_t pl[GIMG];
#pragma unroll
    for (int i = 0; i < GIMG; ++i) pl[i] = plane(min(n0 + i, n1 - 1));
    if constexpr (KIND == 2) {
        uint8_t v[GIMG];
#pragma unroll
        for (int i = 0; i < GIMG; ++i) v[i] = ((const uint8_t*)a.src)[pl[i] + p];
#pragma unroll
        for (int i = 0; i < GIMG; ++i)
            if (n0 + i < n1) ((uint16_t*)a.out)[(int64_t)(n0 + i) * HW + p] = s_lut[v[i]];
        return;
    } else {
        const __half2 g = ((const __half2*)a.grid)[p];
        const float gx = __low2float(g), gy = __high2float(g);
        const float ix = __builtin_fmaf(gx + 1.0f, (float)a.W, -1.0f) * 0.5f;
        const float iy = __builtin_fmaf(gy + 1.0f, (float)a.H, -1.0f) * 0.5f;
        const int x0 = (int)floorf(ix), y0 = (int)floorf(iy);
        const int x1 = x0 + 1, y1 = y0 + 1;
        const float w[4] = {((float)x1 - ix) * ((float)y1 - iy), (ix - (float)x0) * ((float)y1 - iy),
                            ((float)x1 - ix) * (iy - (float)y0), (ix - (float)x0) * (iy - (float)y0)};
        const bool vx0 = x0 >= 0 && x0 < a.W, vx1 = x1 >= 0 && x1 < a.W;
        const bool vy0 = y0 >= 0 && y0 < a.H, vy1 = y1 >= 0 && y1 < a.H;
        const bool ok[4] = {vy0 && vx0, vy0 && vx1, vy1 && vx0, vy1 && vx1};
        // taps outside the image read the plane's first pixel and are not added
        const int off[4] = {ok[0] ? y0 * a.W + x0 : 0, ok[1] ? y0 * a.W + x1 : 0,
                            ok[2] ? y1 * a.W + x0 : 0, ok[3] ? y1 * a.W + x1 : 0};
        float v[GIMG][4];
#pragma unroll
        for (int i = 0; i < GIMG; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if constexpr (KIND == 1)
                    v[i][t] = (float)((const uint8_t*)a.src)[pl[i] + off[t]];
                else
                    v[i][t] = __half2float(((const __half*)a.src)[pl[i] + off[t]]);
            }
#pragma unroll
        for (int i = 0; i < GIMG; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (ok[t]) {
                    float x = v[i][t];
                    if constexpr (KIND == 1) x = __half2float(__ushort_as_half(s_lut[(int)x]));
                    acc = __builtin_fmaf(x, w[t], acc);
                }
            }
            if (n0 + i < n1) ((__half*)a.out)[(int64_t)(n0 + i) * HW + p] = __float2half_rn(acc);
        }
    }
}

// The uint8 gather + table + bilinear view (KIND 1 above) with four consecutive output pixels of a row
// per thread (W a multiple of 4, the grid 16-byte aligned).  Where the four pixels share their source
// rows and all their taps lie in one 8-byte aligned window of those rows inside the image (a zoom or
// shift of at most about 1.75 source pixels per output pixel), each image's taps come from two dword
// loads per row instead of sixteen byte loads; elsewhere each pixel takes KIND 1's taps.  Per pixel the
// arithmetic is KIND 1's (the same values, weights and fma order), so the outputs are identical.
// GIMG4 images per thread (16 measured 8 % faster than 8 and than 4 at the submission's shape).
constexpr int GIMG4 = 16;
__global__ void __launch_bounds__(NT) k_grid_sample4(D8sGridArgs a) {
    __shared__ uint16_t s_lut[256];
    if (threadIdx.x < 256) s_lut[threadIdx.x] = ((const uint16_t*)a.lut)[threadIdx.x];
    __syncthreads();
    const int HW = a.H * a.W;
    const int p0 = 4 * (blockIdx.x * NT + threadIdx.x);
    const int n0 = blockIdx.y * GIMG4, n1 = min(n0 + GIMG4, a.N);
    if (p0 >= HW) return;
    int64_t pl[GIMG4];
#pragma unroll
    for (int i = 0; i < GIMG4; ++i) {
        const int n = min(n0 + i, n1 - 1), b = n / a.M, m = n - b * a.M;
        int64_t si = ((const int64_t*)a.slice_idx)[m];
        si = si < 0 ? 0 : si >= a.SK ? (int64_t)a.SK - 1 : si;
        pl[i] = ((int64_t)b * a.SK + si) * HW;
    }
    const uint4 gq = ((const uint4*)a.grid)[p0 >> 2];         // 4 pixels x (gx, gy) fp16
    const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
    float w[4][4];
    int x0[4], y0[4];
    bool ok[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const __half2 g = __builtin_bit_cast(__half2, gw[k]);
        const float gx = __low2float(g), gy = __high2float(g);
        const float ix = __builtin_fmaf(gx + 1.0f, (float)a.W, -1.0f) * 0.5f;
        const float iy = __builtin_fmaf(gy + 1.0f, (float)a.H, -1.0f) * 0.5f;
        x0[k] = (int)floorf(ix);
        y0[k] = (int)floorf(iy);
        const int x1 = x0[k] + 1, y1 = y0[k] + 1;
        w[k][0] = ((float)x1 - ix) * ((float)y1 - iy);
        w[k][1] = (ix - (float)x0[k]) * ((float)y1 - iy);
        w[k][2] = ((float)x1 - ix) * (iy - (float)y0[k]);
        w[k][3] = (ix - (float)x0[k]) * (iy - (float)y0[k]);
        const bool vx0 = x0[k] >= 0 && x0[k] < a.W, vx1 = x1 >= 0 && x1 < a.W;
        const bool vy0 = y0[k] >= 0 && y0[k] < a.H, vy1 = y1 >= 0 && y1 < a.H;
        ok[k][0] = vy0 && vx0;
        ok[k][1] = vy0 && vx1;
        ok[k][2] = vy1 && vx0;
        ok[k][3] = vy1 && vx1;
    }
    const int xmin = min(min(x0[0], x0[1]), min(x0[2], x0[3])), xmax = max(max(x0[0], x0[1]), max(x0[2], x0[3]));
    const int base = xmin & ~3;
    const bool fast = y0[0] == y0[1] && y0[0] == y0[2] && y0[0] == y0[3] && y0[0] >= 0 && y0[0] + 1 < a.H &&
                      xmin >= 0 && xmax + 1 - base <= 7 && base + 8 <= a.W;
    float acc[GIMG4][4];
    if (fast) {
        // rows y0, y0 + 1 of each image: bytes base .. base + 7 as two dwords per row
        const int r0 = y0[0] * a.W + base;
        uint32_t d[GIMG4][4];
#pragma unroll
        for (int i = 0; i < GIMG4; ++i) {
            const uint32_t* q0 = (const uint32_t*)((const uint8_t*)a.src + pl[i] + r0);
            const uint32_t* q1 = (const uint32_t*)((const uint8_t*)a.src + pl[i] + r0 + a.W);
            d[i][0] = q0[0];
            d[i][1] = q0[1];
            d[i][2] = q1[0];
            d[i][3] = q1[1];
        }
#pragma unroll
        for (int i = 0; i < GIMG4; ++i) {
            const uint64_t row0 = (uint64_t)d[i][0] | ((uint64_t)d[i][1] << 32);
            const uint64_t row1 = (uint64_t)d[i][2] | ((uint64_t)d[i][3] << 32);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int o = 8 * (x0[k] - base);
                const uint32_t t0 = (uint32_t)(row0 >> o), t1 = (uint32_t)(row1 >> o);
                const float v[4] = {__half2float(__ushort_as_half(s_lut[t0 & 0xffu])),
                                    __half2float(__ushort_as_half(s_lut[(t0 >> 8) & 0xffu])),
                                    __half2float(__ushort_as_half(s_lut[t1 & 0xffu])),
                                    __half2float(__ushort_as_half(s_lut[(t1 >> 8) & 0xffu]))};
                float s = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) s = __builtin_fmaf(v[t], w[k][t], s);
                acc[i][k] = s;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int off[4] = {ok[k][0] ? y0[k] * a.W + x0[k] : 0, ok[k][1] ? y0[k] * a.W + x0[k] + 1 : 0,
                                ok[k][2] ? (y0[k] + 1) * a.W + x0[k] : 0, ok[k][3] ? (y0[k] + 1) * a.W + x0[k] + 1 : 0};
            float v[GIMG4][4];
#pragma unroll
            for (int i = 0; i < GIMG4; ++i)
#pragma unroll
                for (int t = 0; t < 4; ++t) v[i][t] = (float)((const uint8_t*)a.src)[pl[i] + off[t]];
#pragma unroll
            for (int i = 0; i < GIMG4; ++i) {
                float s = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (ok[k][t]) s = __builtin_fmaf(__half2float(__ushort_as_half(s_lut[(int)v[i][t]])), w[k][t], s);
                acc[i][k] = s;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < GIMG4; ++i)
        if (n0 + i < n1) {
            const uint32_t lo = (uint32_t)__half_as_ushort(__float2half_rn(acc[i][0])) |
                                ((uint32_t)__half_as_ushort(__float2half_rn(acc[i][1])) << 16);
            const uint32_t hi = (uint32_t)__half_as_ushort(__float2half_rn(acc[i][2])) |
                                ((uint32_t)__half_as_ushort(__float2half_rn(acc[i][3])) << 16);
            *(uint2*)((uint16_t*)a.out + (int64_t)(n0 + i) * HW + p0) = make_uint2(lo, hi);
        }
}

// ---- host side ----------------------------------------------------------------------------------
#define PREQ(cond, msg) \
    do { if (!(cond)) return d8s_host_fail((int)hipErrorInvalidValue, std::string(what) + ": " + (msg)); } while (0)

// The workgroup ranges of every stack in the three grids (4 blocks per workgroup); returns the size of
// the per-block grid.
int assign_grids(PArgs& a) {
    int wh = 0, wh2 = 0, wn = 0;
    for (int i = 0; i < a.n; ++i) {
        PStack& p = a.s[i];
        p.hb = p.hb2 = p.nb = 4;
        p.wg_hist = wh;
        p.wg_hist2 = wh2;
        p.wg_norm = wn;
        wh += (p.nblk + p.hb - 1) / p.hb;
        wh2 += (p.nblk + p.hb2 - 1) / p.hb2;
        wn += (p.nblk + p.nb - 1) / p.nb;
    }
    return wn;
}

// The float32 view of a kind-0 call after the first pass: every stack reads its resized slices from
// the scratch buffer (M_FLOAT), in blocks of about 4096 pixels.
PArgs float_view(const PArgs& a) {
    PArgs f = a;
    const int rb = a.img >= 4096 ? 1 : 4096 / a.img;
    for (int i = 0; i < f.n; ++i) {
        PStack& p = f.s[i];
        p.src = p.sc;
        p.resc = nullptr;
        p.mode = M_FLOAT;
        p.rb = rb;
        p.bps = (a.img + rb - 1) / rb;
        p.nblk = (p.k1 - p.k0) * p.bps;
    }
    assign_grids(f);
    return f;
}

int prepare(const D8sPrepArgs* in, const char* what, bool resize_only, PArgs& a, int& setup_blocks) {
    PREQ(in != nullptr, "null arguments");
    PREQ(in->kind == 0 || in->kind == 1, "kind must be 0 (uint16 regions) or 1 (float32 stacks)");
    PREQ(!resize_only || in->kind == 0, "kind 1 has nothing to resize");
    PREQ(in->n_stacks >= 1 && in->n_stacks <= MAX_S, "n_stacks must be 1 .. 16");
    PREQ(in->img >= 8 && in->img <= 4096 && in->img % 8 == 0, "img must be a multiple of 8 in 8 .. 4096");
    PREQ(in->workspace != 0 && in->workspace % 256 == 0, "workspace null or not 256-byte aligned");
    uint64_t need = 0;
    d8s_prep_workspace(in->n_stacks, in->img, &need);
    PREQ(in->ws_bytes >= need, "workspace smaller than d8s_prep_workspace()");
    const int img = in->img;
    if (in->kind == 0 && !resize_only) {
        uint64_t sc = 0;
        for (int i = 0; i < in->n_stacks; ++i) {
            const int64_t sl = (int64_t)in->s[i].k1 - in->s[i].k0;
            sc += 4ull * (uint64_t)(sl > 0 ? sl : 0) * img * img;
        }
        PREQ(in->scratch != 0 && in->scratch % 16 == 0, "scratch null or not 16-byte aligned");
        PREQ(in->scratch_bytes >= sc, "scratch smaller than 4 * sum(k1 - k0) * img * img bytes");
    }
    a = PArgs{};
    a.n = in->n_stacks;
    a.img = img;
    a.upr = img / UP;
    a.stat = (D8sPrepStat*)in->workspace;
    a.inv_img = 1.0f / (float)img;
    a.inv_upr = 1.0f / (float)a.upr;
    PREQ(in->kind == 1 || img <= 1024, "img above 1024 is supported for float32 stacks (kind 1) only");
    const int rb_want = 4096 / img > 1 ? 4096 / img : 1;     // about 4096 output pixels per block
    int64_t sc_off = 0;
    for (int i = 0; i < a.n; ++i) {
        const D8sPrepStack& s = in->s[i];
        PStack& p = a.s[i];
        const std::string at = "stack " + std::to_string(i) + ": ";
        PREQ(s.src != 0 && s.out != 0, at + "null src or out");
        PREQ(s.K >= 1 && s.k0 >= 0 && s.k0 < s.k1 && s.k1 <= s.K, at + "slice range outside 0 .. K");
        const int64_t n = (int64_t)(s.k1 - s.k0) * img * img;
        PREQ((int64_t)s.K * img * img < (1ll << 31), at + "more than 2^31 - 1 pixels");
        if (!resize_only) {
            PREQ(n >= 4, at + "fewer than 4 pixels");
            PREQ(s.r1 >= 0 && (int64_t)s.r1 + 1 < n && s.r2 >= 0 && (int64_t)s.r2 + 1 < n,
                 at + "ranks outside the stack");
            PREQ(s.g1 >= 0.0 && s.g1 < 1.0 && s.g2 >= 0.0 && s.g2 < 1.0, at + "gamma outside [0, 1)");
            PREQ(s.flip >= 0 && s.flip <= 2, at + "flip must be 0, 1 or 2");
            PREQ(s.out % 8 == 0, at + "uint8 output not 8-byte aligned");
        } else {
            PREQ(s.out % 16 == 0, at + "float32 output not 16-byte aligned");
        }
        p.src = (const void*)s.src;
        p.out = (void*)s.out;
        p.resc = in->kind == 0 ? (const float*)s.resc : nullptr;
        p.ws = (uint32_t*)(in->workspace + WS_HEAD) + (uint64_t)i * stack_words(img);
        if (in->kind == 0 && !resize_only) {
            // compact: the slices [k0, k1) of the stacks back to back; sc is offset so that slice kk
            // is at sc + kk img img
            p.sc = (float*)in->scratch + (int64_t)sc_off - (int64_t)s.k0 * img * img;
            sc_off += (int64_t)(s.k1 - s.k0) * img * img;
        }
        p.K = s.K;
        p.k0 = s.k0;
        p.k1 = s.k1;
        p.flip = resize_only ? 0 : s.flip;
        p.r1 = s.r1;
        p.r2 = s.r2;
        p.g1 = s.g1;
        p.g2 = s.g2;
        if (in->kind == 1) {
            PREQ(s.src % 16 == 0, at + "float32 input not 16-byte aligned");
            p.mode = M_FLOAT;
            p.rb = rb_want;
        } else {
            PREQ(s.hr >= 1 && s.wr >= 1, at + "empty region");
            PREQ(s.y0 >= 0 && s.y0 < s.y1 && s.y1 <= s.hr && s.x0 >= 0 && s.x0 < s.x1 && s.x1 <= s.wr,
                 at + "box outside the region");
            PREQ((int64_t)s.K * s.hr * s.wr < (1ll << 31) - 2, at + "region of 2^31 or more values");
            p.hr = s.hr;
            p.wr = s.wr;
            p.y0 = s.y0;
            p.x0 = s.x0;
            p.h = s.y1 - s.y0;
            p.w = s.x1 - s.x0;
            // LDS per block: ns_max resized rows of img floats + ns_max raw rows of rp dwords
            p.rp = (p.w + 2) / 2;
            p.inv_rp = 1.0f / (float)p.rp;
            p.dpl = (p.rp + 63) / 64;
            // the LDS holds ns_max rows of img floats and one or two buffers of ns_max rows of
            // dpl * 64 raw dwords: two when that still gives blocks of rb_want rows
            const double sc_h = p.h > img ? (double)p.h / img : 1.0;
            const int need = (int)ceil(rb_want * sc_h) + 2;
            p.dbuf = need * (img + 128 * p.dpl) <= STAGE ? 1 : 0;
            const int cap = STAGE / (img + (p.dbuf ? 128 : 64) * p.dpl);
            if (p.h == img && p.w == img) {
                p.mode = M_IDENT;
                PREQ(cap >= 1, at + "crop too wide for this img");
                p.rb = rb_want < cap ? rb_want : cap;
                p.ns_max = p.rb;
            } else if (p.h > img) {
                p.mode = M_AREA;
                p.Tx = p.w != img ? area_taps_max(p.w, img) : 0;
                p.Ty = area_taps_max(p.h, img);
                PREQ(p.Tx <= MAX_T && p.Ty <= MAX_T, at + "area table longer than 16 taps");
                // rb output rows read at most rb * h / img + 2 source rows
                const double scale = (double)p.h / img;
                PREQ(scale + 2.0 <= cap, at + "area downscale factor too large for this img and width");
                const int fit = (int)((cap - 2) / scale);
                p.rb = rb_want < fit ? rb_want : fit;
                p.ns_max = (int)ceil(p.rb * scale) + 2;
            } else {
                p.mode = M_BILIN;
                p.rh = (float)p.h / (float)img;
                p.rw = (float)p.w / (float)img;
                PREQ(cap >= 2, at + "crop too wide for this img");
                p.rb = rb_want < cap - 1 ? rb_want : cap - 1;   // rb + 1 source rows
                p.ns_max = p.rb + 1;
            }
        }
        p.bps = (img + p.rb - 1) / p.rb;
        p.nblk = (s.k1 - s.k0) * p.bps;
    }
    int outside = 0;
    for (int i = 0; i < a.n; ++i) {
        const PStack& p = a.s[i];
        const int o = (p.K - (p.k1 - p.k0)) * (img * img / 8);
        outside = o > outside ? o : outside;
    }
    const int wn = assign_grids(a);
    PREQ(wn < (1 << 30), "too many workgroups");
    int sb = (img + NT - 1) / NT;
    const int sc = (W_CLEAR + NT * 4 - 1) / (NT * 4), so = (outside + NT * 4 - 1) / (NT * 4);
    sb = sb > sc ? sb : sc;
    sb = sb > so ? sb : so;
    setup_blocks = sb < 1024 ? sb : 1024;
    return 0;
}

int grid_of(const PArgs& a, int grid) {
    const PStack& l = a.s[a.n - 1];
    return grid == 0 ? l.wg_hist + (l.nblk + l.hb - 1) / l.hb
         : grid == 1 ? l.wg_hist2 + (l.nblk + l.hb2 - 1) / l.hb2
                     : l.wg_norm + (l.nblk + l.nb - 1) / l.nb;
}

}  // namespace

extern "C" int d8s_prep_workspace(int32_t n_stacks, int32_t img, uint64_t* bytes) {
    const char* what = "d8s_prep_workspace";
    PREQ(bytes != nullptr, "null output");
    PREQ(n_stacks >= 1 && n_stacks <= MAX_S, "n_stacks must be 1 .. 16");
    PREQ(img >= 8 && img <= 4096 && img % 8 == 0, "img must be a multiple of 8 in 8 .. 4096");
    *bytes = WS_HEAD + 4ull * stack_words(img) * (uint64_t)n_stacks;
    return 0;
}

extern "C" int d8s_prep(const D8sPrepArgs* in, void* stream) {
    PArgs a;
    int sb = 0;
    if (const int rc = prepare(in, "d8s_prep", false, a, sb)) return rc;
    hipStream_t st = (hipStream_t)stream;
    const dim3 gs(sb, a.n);
    k_prep_setup<<<gs, NT, 0, st>>>(a, 1);
    const int gh = grid_of(a, 0), gh2 = grid_of(a, 1), gn = grid_of(a, 2);
    if (in->kind == 0) {
        // resize once (with the level-1 count) into the scratch stacks, then the float32 passes
        k_prep_hist<1, 1, true><<<gh, NT, 0, st>>>(a);
        k_prep_select<1><<<a.n, NT, 0, st>>>(a);
        const PArgs f = float_view(a);
        const int fh2 = grid_of(f, 1), fn = grid_of(f, 2);
        k_prep_hist<2, 0><<<fh2, NT, 0, st>>>(f);
        k_prep_select<2><<<f.n, NT, 0, st>>>(f);
        k_prep_hist<3, 0><<<fh2, NT, 0, st>>>(f);
        k_prep_select<3><<<f.n, NT, 0, st>>>(f);
        k_prep_norm<0><<<fn, NT, 0, st>>>(f);
        (void)gh2;
        (void)gn;
    } else {
        k_prep_hist<1, 0><<<gh, NT, 0, st>>>(a);
        k_prep_select<1><<<a.n, NT, 0, st>>>(a);
        k_prep_hist<2, 0><<<gh2, NT, 0, st>>>(a);
        k_prep_select<2><<<a.n, NT, 0, st>>>(a);
        k_prep_hist<3, 0><<<gh2, NT, 0, st>>>(a);
        k_prep_select<3><<<a.n, NT, 0, st>>>(a);
        k_prep_norm<0><<<gn, NT, 0, st>>>(a);
    }
    return d8s_host_launched("d8s_prep");
}

extern "C" int d8s_prep_resize(const D8sPrepArgs* in, void* stream) {
    PArgs a;
    int sb = 0;
    if (const int rc = prepare(in, "d8s_prep_resize", true, a, sb)) return rc;
    hipStream_t st = (hipStream_t)stream;
    k_prep_setup<<<dim3(sb, a.n), NT, 0, st>>>(a, 0);
    k_prep_resize<<<grid_of(a, 2), NT, 0, st>>>(a);
    return d8s_host_launched("d8s_prep_resize");
}

extern "C" int d8s_grid_sample(const D8sGridArgs* a, void* stream) {
    const char* what = "d8s_grid_sample";
    PREQ(a != nullptr, "null arguments");
    PREQ(a->kind == 0 || a->kind == 1, "kind must be 0 (fp16 images) or 1 (uint8 volume gather)");
    PREQ(a->src && a->out && (a->grid || a->kind == 1), "null pointer");
    PREQ(a->H >= 1 && a->W >= 1 && (int64_t)a->H * a->W < (1ll << 31), "bad image size");
    PREQ(a->grid % 4 == 0, "grid not 4-byte aligned");
    if (a->kind == 1) {
        PREQ(a->slice_idx && a->lut, "null slice_idx or lut");
        PREQ(a->B >= 1 && a->M >= 1 && a->SK >= 1, "bad B, M or SK");
        PREQ((int64_t)a->B * a->M == a->N, "N must be B * M");
    }
    PREQ(a->N >= 1 && a->N < 65536 * GIMG, "N must be 1 .. 524287");
    const dim3 grid((unsigned)(((int64_t)a->H * a->W + NT - 1) / NT), (unsigned)((a->N + GIMG - 1) / GIMG));
    hipStream_t st = (hipStream_t)stream;
    if (a->kind == 1 && a->grid != 0 && a->W % 4 == 0 && a->grid % 16 == 0 && a->out % 8 == 0 && a->src % 4 == 0) {
        const dim3 grid4((unsigned)(((int64_t)a->H * a->W / 4 + NT - 1) / NT), (unsigned)((a->N + GIMG4 - 1) / GIMG4));
        k_grid_sample4<<<grid4, NT, 0, st>>>(*a);
    } else if (a->kind == 1 && a->grid == 0)
        k_grid_sample<2><<<grid, NT, 0, st>>>(*a);
    else if (a->kind == 1)
        k_grid_sample<1><<<grid, NT, 0, st>>>(*a);
    else
        k_grid_sample<0><<<grid, NT, 0, st>>>(*a);
    return d8s_host_launched("d8s_grid_sample");
}
