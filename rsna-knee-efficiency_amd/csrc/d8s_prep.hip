// gfx950 kernels of the upstream preprocessing (raw uint16 crops -> resize -> exact 1/99 percentiles
// -> uint8 -> side flip) and their C ABI, d8s_prep / d8s_prep_resize (include/d8s_hip.h).
//
// The work is byte and float bookkeeping bound by memory, not matrix work.  Design:
//   - the resized float32 stacks are never stored: every pass evaluates the resize again from the
//     uint16 region (2 bytes per source pixel, a region of a study is ~50 MB and stays in the
//     256 MB last-level cache between passes) instead of reading 4 bytes per output pixel of a
//     materialised stack;
//   - the order statistics k1, k1+1, k2, k2+1 are selected exactly by a three-level radix histogram
//     of the float's order key (11 + 11 + 10 bits).  Each level is one pass over the stack that
//     counts in LDS and adds the nonzero bins to a global histogram, then one workgroup per stack
//     finds the bins holding the four ranks;  equal ranks share a histogram (at most four per level);
//   - the last pass evaluates the pixel again and writes the uint8 value (float64 arithmetic, the
//     reference's exact operations) at its flipped position.
// A pass handles units of 8 consecutive output pixels of one row; a workgroup owns a contiguous run of
// units of one stack, so neighbouring source rows are read from cache.
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
    int K, hr, wr, y0, x0, h, w, k0, k1, flip, mode, Tx, Ty, r1, r2;
    float rh, rw;
    double g1, g2;
    int units;       // (k1 - k0) * img * img / 8
    int wg_hist, wg_norm;
};

struct PArgs {
    PStack s[MAX_S];
    D8sPrepStat* stat;
    int n, img, upr;          // stacks, output side, units per output row (img / 8)
    int hist_units, norm_units;
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
DEV float rescaled(uint16_t u, bool has, float sl, float ic) {
    const float f = (float)u;
    if (!has) return f;
    const float p = f * sl;
    return p + ic;
}

DEV float src_index(float scale, int d) {
    const float s = __builtin_fmaf(scale, (float)d + 0.5f, -0.5f);
    return s < 0.0f ? 0.0f : s;
}

// Values of output pixels (kk, dy, dx0 .. dx0 + 7) of stack `st` (mode MODE) into v.
template <int MODE>
DEV void eval8(const PStack& st, int img, int kk, int dy, int dx0, float v[8]) {
    if constexpr (MODE == M_FLOAT) {
        const float4* p = (const float4*)((const float*)st.src + ((int64_t)kk * img + dy) * img + dx0);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        return;
    } else {
        const uint16_t* reg = (const uint16_t*)st.src + (int64_t)kk * st.hr * st.wr;
        const bool has = st.resc != nullptr;
        const float sl = has ? st.resc[2 * kk] : 1.0f, ic = has ? st.resc[2 * kk + 1] : 0.0f;
        if constexpr (MODE == M_IDENT) {
            const uint16_t* row = reg + (int64_t)(st.y0 + dy) * st.wr + st.x0 + dx0;
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = rescaled(row[i], has, sl, ic);
        } else if constexpr (MODE == M_BILIN) {
            const float sy = src_index(st.rh, dy);
            const int h1 = (int)sy;
            const int h1p = h1 < st.h - 1 ? 1 : 0;
            const float l1 = sy - (float)h1, l0 = 1.0f - l1;
            const uint16_t* r0 = reg + (int64_t)(st.y0 + h1) * st.wr + st.x0;
            const uint16_t* r1 = r0 + (int64_t)h1p * st.wr;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float sx = src_index(st.rw, dx0 + i);
                const int w1 = (int)sx;
                const int w1p = w1 < st.w - 1 ? 1 : 0;
                const float m1 = sx - (float)w1, m0 = 1.0f - m1;
                const float a = rescaled(r0[w1], has, sl, ic), b = rescaled(r0[w1 + w1p], has, sl, ic);
                const float c = rescaled(r1[w1], has, sl, ic), d = rescaled(r1[w1 + w1p], has, sl, ic);
                const float top = __builtin_fmaf(m0, a, m1 * b);
                const float bot = __builtin_fmaf(m0, c, m1 * d);
                v[i] = __builtin_fmaf(l0, top, l1 * bot);
            }
        } else {  // M_AREA: rows of the column-resized intermediate, weighted, in table order
            const int32_t* ix = (const int32_t*)st.ws + W_TAPS;
            const float* wx = (const float*)(ix + img * st.Tx);
            const int32_t* iy = (const int32_t*)(wx + img * st.Tx);
            const float* wy = (const float*)(iy + img * st.Ty);
            float acc[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
            for (int j = 0; j < st.Ty; ++j) {
                const int sy = iy[dy * st.Ty + j];
                const float wyj = wy[dy * st.Ty + j];
                const uint16_t* row = reg + (int64_t)(st.y0 + sy) * st.wr + st.x0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int dx = dx0 + i;
                    float c;
                    if (st.w == img) {
                        c = rescaled(row[dx], has, sl, ic);
                    } else {
                        c = 0.0f;
                        for (int t = 0; t < st.Tx; ++t) {
                            const float p = rescaled(row[ix[dx * st.Tx + t]], has, sl, ic) * wx[dx * st.Tx + t];
                            c = c + p;
                        }
                    }
                    const float p = c * wyj;
                    acc[i] = acc[i] + p;
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = acc[i];
        }
    }
}

// Runs f(kk, dy, dx0, v) over units [ub, ue) of stack st, thread-strided, with the mode fixed.
template <class F>
DEV void for_units(const PStack& st, const PArgs& a, int ub, int ue, F&& f) {
    auto run = [&](auto mode_tag) {
        constexpr int MODE = decltype(mode_tag)::value;
        for (int u = ub + (int)threadIdx.x; u < ue; u += NT) {
            const int row = u / a.upr;
            const int dx0 = (u - row * a.upr) * 8;
            const int kk = st.k0 + row / a.img;
            const int dy = row - (row / a.img) * a.img;
            float v[8];
            eval8<MODE>(st, a.img, kk, dy, dx0, v);
            f(kk, dy, dx0, v);
        }
    };
    switch (st.mode) {
        case M_IDENT: run(std::integral_constant<int, M_IDENT>{}); break;
        case M_BILIN: run(std::integral_constant<int, M_BILIN>{}); break;
        case M_AREA: run(std::integral_constant<int, M_AREA>{}); break;
        default: run(std::integral_constant<int, M_FLOAT>{}); break;
    }
}

DEV int stack_of(const PArgs& a, bool norm) {
    int s = 0;
    for (int i = 1; i < a.n; ++i)
        if ((int)blockIdx.x >= (norm ? a.s[i].wg_norm : a.s[i].wg_hist)) s = i;
    return s;
}

// LDS histogram increment; when every active lane of the wave hits the same bin (runs of equal
// values, e.g. a zero background) one lane adds the count instead of 64 conflicting atomics.
DEV void hist_inc(uint32_t* h, uint32_t bin) {
    const uint32_t first = __builtin_amdgcn_readfirstlane(bin);
    const uint64_t act = __ballot(1);
    const uint64_t same = __ballot(bin == first);
    if (same == act) {
        if ((int)__lane_id() == __builtin_ctzll(act)) atomicAdd(&h[first], (uint32_t)__popcll(act));
    } else {
        atomicAdd(&h[bin], 1u);
    }
}

// ---- kernels ------------------------------------------------------------------------------------

// Clears the histograms and selections of every stack and builds the area tables.
__global__ void __launch_bounds__(NT) k_prep_setup(PArgs a, int clear) {
    const PStack& st = a.s[blockIdx.y];
    const int gid = blockIdx.x * NT + threadIdx.x, gsz = gridDim.x * NT;
    if (clear)
        for (int i = gid; i < W_CLEAR; i += gsz) st.ws[i] = 0u;
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

// One radix level over the units of a run of one stack.
template <int LEVEL>
__global__ void __launch_bounds__(NT) k_prep_hist(PArgs a) {
    constexpr int NB = LEVEL == 1 ? NB1 : LEVEL == 2 ? NB2 : NB3;
    constexpr int NH = LEVEL == 1 ? 1 : 4;
    __shared__ uint32_t s_h[NH * NB];
    const int s = stack_of(a, false);
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
    const int ub = ((int)blockIdx.x - st.wg_hist) * a.hist_units;
    const int ue = min(ub + a.hist_units, st.units);
    bool nan = false;
    for_units(st, a, ub, ue, [&](int, int, int, const float* v) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t k = order_key(v[i]);
            if constexpr (LEVEL == 1) {
                nan |= v[i] != v[i];
                hist_inc(s_h, k >> 21);
            } else if constexpr (LEVEL == 2) {
                const uint32_t p = k >> 21;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (t < (int)nslot && p == pre[t]) hist_inc(s_h + t * NB, (k >> 10) & (NB2 - 1));
            } else {
                const uint32_t p = k >> 10;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (t < (int)nslot && p == pre[t]) hist_inc(s_h + t * NB, k & (NB3 - 1));
            }
        }
    });
    if constexpr (LEVEL == 1) {
        if (__ballot(nan) != 0ull && (int)__lane_id() == 0) atomicOr(st.ws + W_NAN, 1u);
    }
    __syncthreads();
    uint32_t* gh = st.ws + (LEVEL == 1 ? W_H1 : LEVEL == 2 ? W_H2 : W_H3);
    const int nh = LEVEL == 1 ? 1 : (int)nslot;
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
__global__ void __launch_bounds__(NT) k_prep_norm(PArgs a) {
    const int s = stack_of(a, true);
    const PStack& st = a.s[s];
    const D8sPrepStat r = a.stat[s];
    const int ub = ((int)blockIdx.x - st.wg_norm) * a.norm_units;
    const int ue = min(ub + a.norm_units, st.units);
    uint8_t* out = (uint8_t*)st.out;
    for_units(st, a, ub, ue, [&](int kk, int dy, int dx0, const float* v) {
        uint32_t b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            double y = (double)v[i] - r.lo;
            y = y * r.scale;
            y = y < 0.0 ? 0.0 : y;
            y = y > 255.0 ? 255.0 : y;
            b[i] = r.bad ? 0u : (uint32_t)y;
        }
        const int ko = st.flip == D8S_FLIP_SLICES ? st.K - 1 - kk : kk;
        uint32_t lo, hi;
        int xo = dx0;
        if (st.flip == D8S_FLIP_X) {
            xo = a.img - 8 - dx0;
            lo = b[7] | (b[6] << 8) | (b[5] << 16) | (b[4] << 24);
            hi = b[3] | (b[2] << 8) | (b[1] << 16) | (b[0] << 24);
        } else {
            lo = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
            hi = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
        }
        uint2* p = (uint2*)(out + ((int64_t)ko * a.img + dy) * a.img + xo);
        *p = make_uint2(lo, hi);
    });
}

// The resized float32 values themselves.
__global__ void __launch_bounds__(NT) k_prep_resize(PArgs a) {
    const int s = stack_of(a, true);
    const PStack& st = a.s[s];
    const int ub = ((int)blockIdx.x - st.wg_norm) * a.norm_units;
    const int ue = min(ub + a.norm_units, st.units);
    float* out = (float*)st.out;
    for_units(st, a, ub, ue, [&](int kk, int dy, int dx0, const float* v) {
        float4* p = (float4*)(out + ((int64_t)kk * a.img + dy) * a.img + dx0);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    });
}

// ---- host side ----------------------------------------------------------------------------------
#define PREQ(cond, msg) \
    do { if (!(cond)) return d8s_host_fail((int)hipErrorInvalidValue, std::string(what) + ": " + (msg)); } while (0)

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
    a = PArgs{};
    a.n = in->n_stacks;
    a.img = img;
    a.upr = img / 8;
    a.stat = (D8sPrepStat*)in->workspace;
    int64_t total_units = 0;
    for (int i = 0; i < a.n; ++i) {
        const D8sPrepStack& s = in->s[i];
        PStack& p = a.s[i];
        const std::string at = "stack " + std::to_string(i) + ": ";
        PREQ(s.src != 0 && s.out != 0, at + "null src or out");
        PREQ(s.K >= 1 && s.k0 >= 0 && s.k0 < s.k1 && s.k1 <= s.K, at + "slice range outside 0 .. K");
        const int64_t n = (int64_t)(s.k1 - s.k0) * img * img;
        PREQ(n < (1ll << 31), at + "more than 2^31 - 1 pixels");
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
        p.K = s.K;
        p.k0 = s.k0;
        p.k1 = s.k1;
        p.flip = resize_only ? 0 : s.flip;
        p.r1 = s.r1;
        p.r2 = s.r2;
        p.g1 = s.g1;
        p.g2 = s.g2;
        p.units = (int)(n / 8);
        total_units += p.units;
        if (in->kind == 1) {
            PREQ(s.src % 16 == 0, at + "float32 input not 16-byte aligned");
            p.mode = M_FLOAT;
            continue;
        }
        PREQ(s.hr >= 1 && s.wr >= 1, at + "empty region");
        PREQ(s.y0 >= 0 && s.y0 < s.y1 && s.y1 <= s.hr && s.x0 >= 0 && s.x0 < s.x1 && s.x1 <= s.wr,
             at + "box outside the region");
        PREQ((int64_t)s.K * s.hr * s.wr < (1ll << 40), at + "region too large");
        p.hr = s.hr;
        p.wr = s.wr;
        p.y0 = s.y0;
        p.x0 = s.x0;
        p.h = s.y1 - s.y0;
        p.w = s.x1 - s.x0;
        if (p.h == img && p.w == img) {
            p.mode = M_IDENT;
        } else if (p.h > img) {
            p.mode = M_AREA;
            p.Tx = p.w != img ? area_taps_max(p.w, img) : 0;
            p.Ty = area_taps_max(p.h, img);
            PREQ(p.Tx <= MAX_T && p.Ty <= MAX_T, at + "area table longer than 16 taps");
        } else {
            p.mode = M_BILIN;
            p.rh = (float)p.h / (float)img;
            p.rw = (float)p.w / (float)img;
        }
    }
    // histogram passes: about 3 workgroups per CU over all stacks (each flushes its LDS histogram
    // with global atomics, so a workgroup should see many pixels); normalisation: 4 units per thread
    const int64_t want = 3ll * d8s_host_cu_count();
    int64_t hu = (total_units + want - 1) / want;
    hu = (hu + NT - 1) / NT * NT;
    if (hu < 8 * NT) hu = 8 * NT;
    a.hist_units = (int)hu;
    a.norm_units = 4 * NT;
    int wh = 0, wn = 0;
    for (int i = 0; i < a.n; ++i) {
        a.s[i].wg_hist = wh;
        a.s[i].wg_norm = wn;
        wh += (a.s[i].units + a.hist_units - 1) / a.hist_units;
        wn += (a.s[i].units + a.norm_units - 1) / a.norm_units;
    }
    PREQ(wn < (1 << 30), "too many workgroups");
    setup_blocks = (img + NT - 1) / NT;
    if (setup_blocks < (W_CLEAR + NT * 4 - 1) / (NT * 4)) setup_blocks = (W_CLEAR + NT * 4 - 1) / (NT * 4);
    return 0;
}

int grid_of(const PArgs& a, bool norm) {
    const PStack& l = a.s[a.n - 1];
    return (norm ? l.wg_norm : l.wg_hist) +
           (l.units + (norm ? a.norm_units : a.hist_units) - 1) / (norm ? a.norm_units : a.hist_units);
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
    const int gh = grid_of(a, false), gn = grid_of(a, true);
    k_prep_hist<1><<<gh, NT, 0, st>>>(a);
    k_prep_select<1><<<a.n, NT, 0, st>>>(a);
    k_prep_hist<2><<<gh, NT, 0, st>>>(a);
    k_prep_select<2><<<a.n, NT, 0, st>>>(a);
    k_prep_hist<3><<<gh, NT, 0, st>>>(a);
    k_prep_select<3><<<a.n, NT, 0, st>>>(a);
    k_prep_norm<<<gn, NT, 0, st>>>(a);
    return d8s_host_launched("d8s_prep");
}

extern "C" int d8s_prep_resize(const D8sPrepArgs* in, void* stream) {
    PArgs a;
    int sb = 0;
    if (const int rc = prepare(in, "d8s_prep_resize", true, a, sb)) return rc;
    hipStream_t st = (hipStream_t)stream;
    k_prep_setup<<<dim3(sb, a.n), NT, 0, st>>>(a, 0);
    k_prep_resize<<<grid_of(a, true), NT, 0, st>>>(a);
    return d8s_host_launched("d8s_prep_resize");
}
