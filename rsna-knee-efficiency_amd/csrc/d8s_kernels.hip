// gfx950 kernels of the INT8 DenseNet encoder and their C ABI (include/d8s_hip.h).
//
// Matrix products run on the CDNA4 int8 MFMA v_mfma_i32_32x32x32_i8 (wave64, 32 x 32 int32 tile,
// K = 32 = one store group per instruction) and, in the stem, on v_mfma_f32_32x32x16_f16.  The
// weights are the MFMA's A operand (rows = output channels) and the activations its B operand
// (columns = pixels): after the MFMA every lane holds 16 output channels of ONE pixel, so one lane
// exchange (lanes l <-> l ^ 32) gives each lane 16 consecutive channel bytes and the epilogues store
// whole 16-byte chunks of the [pixel][32] rows.
//
// Lane layouts relied on (checked by d8s_probe_mfma_i8 / d8s_probe_mfma_f16 on the GPU):
//   operands: lane l holds row (A) / column (B) l & 31 and the K-chunk (l >> 5) of the instruction's K;
//   result:   lane l, element v: column j = l & 31, row i = 8 (v >> 2) + 4 (l >> 5) + (v & 3).
//
// Unsigned activations: the MFMA multiplies signed bytes.  The u8 values u are fed as u - 128
// (= u ^ 0x80 read as int8) and every accumulator starts at 128 * sum_k w[o][k], so it ends at
// sum_k w[o][k] u[k] exactly (int32).  Zero padding of the 3x3 conv is u = 0, i.e. byte 0x80.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <type_traits>

#include "d8s_hip.h"
#include "d8s_host.h"

#ifndef D8S_SRC_HASH
#define D8S_SRC_HASH "unknown"
#endif

#define DEV __device__ __forceinline__
#define INLINE __attribute__((always_inline))   // lambdas: slot indices must fold to constants

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef int16_t i16x2 __attribute__((ext_vector_type(2)));

static constexpr uint32_t SIGN4 = 0x80808080u;

DEV f16x2 as_h2(uint32_t x) { return __builtin_bit_cast(f16x2, x); }
DEV uint32_t h2_bits(f16x2 x) { return __builtin_bit_cast(uint32_t, x); }

DEV i32x16 mfma_i8(u32x4 a, u32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                                 __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// v_perm_b32: byte i of the result is byte sel.i of the pair (s0:s1), bytes 0-3 from s1, 4-7 from s0.
DEV uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) { return __builtin_amdgcn_perm(s0, s1, sel); }

// The four low bytes of the 16-bit halves of (lo, hi) as one dword: byte order lo.0, lo.1, hi.0, hi.1.
DEV uint32_t pack_low_bytes(uint32_t lo, uint32_t hi) { return perm(hi, lo, 0x06040200u); }

// fp16 prologue of 4 store bytes (4 consecutive channels): q -> u = RNE(255 sat(fp16(A q + B))).
// The byte q + 128 goes into the mantissa of fp16 1024 (exact 1024 + 128 + q), -1152 leaves q exactly,
// one fused fp16 fma with saturation gives v, and fma(v, 255, 1152) = 1152 + RNE(255 v) (ulp 1 in
// [1024, 2048); a tie goes to the even sum, i.e. to the even u, 1152 being even): the low byte of each
// half is u + 128 mod 256 = u ^ 0x80, the MFMA operand u - 128 as a signed byte.  (a01, b01) are the
// fp16 pairs (A, B) of channels 0-1, (a23, b23) of channels 2-3.  Returns the halves 1152 + u for
// channels (0, 1) and (2, 3).
// Same roundings as the reference's `pro4h` (src/knee/dense8s_kernels.cu:122-139) and its emulation
// `emulate(f16_layers)` (src/knee/dense8s.py:584-587).
DEV void pro4_halves(uint32_t x, uint32_t a01, uint32_t b01, uint32_t a23, uint32_t b23,
                     uint32_t& rl, uint32_t& rh) {
    const uint32_t w = x ^ SIGN4;
    const uint32_t lo = perm(0x64646464u, w, 0x04010400u);    // halves 0x64 b0, 0x64 b1
    const uint32_t hi = perm(0x64646464u, w, 0x04030402u);    // halves 0x64 b2, 0x64 b3
    const f16x2 m1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const f16x2 zero = {(_Float16)0.0f, (_Float16)0.0f};
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    const f16x2 k255 = {(_Float16)255.0f, (_Float16)255.0f};
    const f16x2 k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    f16x2 vl = __builtin_elementwise_fma(as_h2(lo) + m1152, as_h2(a01), as_h2(b01));
    f16x2 vh = __builtin_elementwise_fma(as_h2(hi) + m1152, as_h2(a23), as_h2(b23));
    vl = __builtin_elementwise_min(__builtin_elementwise_max(vl, zero), one);
    vh = __builtin_elementwise_min(__builtin_elementwise_max(vh, zero), one);
    rl = h2_bits(__builtin_elementwise_fma(vl, k255, k1152));
    rh = h2_bits(__builtin_elementwise_fma(vh, k255, k1152));
}

// The prologue of 4 store bytes as the MFMA operand: 4 bytes u - 128.
DEV uint32_t pro4(uint32_t x, uint32_t a01, uint32_t b01, uint32_t a23, uint32_t b23) {
    uint32_t rl, rh;
    pro4_halves(x, a01, b01, a23, b23, rl, rh);
    return pack_low_bytes(rl, rh);
}

// 16 channels: x = 4 store dwords, p = 16 parameter dwords (A01, B01, A23, B23 per store dword).
DEV u32x4 pro16(u32x4 x, u32x4 p0, u32x4 p1, u32x4 p2, u32x4 p3) {
    return u32x4{pro4(x.x, p0.x, p0.y, p0.z, p0.w), pro4(x.y, p1.x, p1.y, p1.z, p1.w),
                 pro4(x.z, p2.x, p2.y, p2.z, p2.w), pro4(x.w, p3.x, p3.y, p3.z, p3.w)};
}

// Lanes l and l ^ 32 hold the same pixel: lane half h = l >> 5 has channel dwords 2k + h (channels
// 8k + 4h .. 8k + 4h + 3, k = 0..3) of a 32-channel row.  After the exchange lane half h holds the row's
// bytes 16h .. 16h + 15 (dwords 4h .. 4h + 3).
// (v_permlane32_swap exchanges the upper 32 lanes of its first operand with the lower 32 of its
// second: (e0, e2) and (e1, e3) give both halves their dwords in order.)
DEV u32x4 xchg_rows(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, int h) {
    (void)h;
    const auto s02 = __builtin_amdgcn_permlane32_swap(e0, e2, false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(e1, e3, false, false);
    return u32x4{s02[0], s02[1], s13[0], s13[1]};
}

// Byte 0 of each of four dwords, as one dword (a0 in byte 0).
DEV uint32_t pack_b0(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
    return perm(a1, a0, 0x0c0c0400u) | perm(a3, a2, 0x04000c0cu);
}

// Bottleneck bytes of 4 conv1 results (rows 4q .. 4q + 3 of a lane, consecutive channels, tables
// gd = (g, d) of those channels): low byte of fma(sat(fma(g, acc, d)), 255, 2^23 + 128), i.e.
// u ^ 0x80 with u = RNE(255 sat(g acc + d)), the conv2 operand.
DEV uint32_t epi1_x80(i32x16 acc, int q, float4 gd01, float4 gd23) {
    const float g[4] = {gd01.x, gd01.z, gd23.x, gd23.z}, d[4] = {gd01.y, gd01.w, gd23.y, gd23.w};
    uint32_t b[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float y = __builtin_amdgcn_fmed3f(__builtin_fmaf(g[r], (float)acc[4 * q + r], d[r]), 0.0f, 1.0f);
        b[r] = __float_as_uint(__builtin_fmaf(y, 255.0f, 8388736.0f));
    }
    return pack_b0(b[0], b[1], b[2], b[3]);
}

// Store bytes of 4 conv2 results (scales sc of those channels): q = RNE(clamp(float(acc) sc, -127,
// 127)), as the low byte of q + 1.5 * 2^23 (exact: |q| <= 127).
DEV uint32_t epi2_q(i32x16 acc, int q, float4 sc) {
    const float s[4] = {sc.x, sc.y, sc.z, sc.w};
    uint32_t b[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float t = __builtin_amdgcn_fmed3f((float)acc[4 * q + r] * s[r], -127.0f, 127.0f);
        b[r] = __float_as_uint(t + 12582912.0f);
    }
    return pack_b0(b[0], b[1], b[2], b[3]);
}

// LDS position of 16-byte chunk i of a [G][128][32] conv1 weight table (chunk 64 c + 2 j + h within a
// group: output tile c, row j, half h): 64 c + 32 h + j, so the 16 lanes one LDS cycle serves (same
// h, consecutive j) read consecutive chunks.
DEV int wperm(int i) { return (i & ~63) | ((i & 1) << 5) | ((i >> 1) & 31); }

// Row i (output channel) of element v of a 32x32 MFMA result, for lane half h.
DEV int res_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

// Swizzled 16-byte half `half` of 32-byte row r in LDS: the halves swap on every other group of 8
// rows, so the 16-byte reads of 16 consecutive rows (the lanes one LDS cycle serves) hit distinct
// banks.  (Swapping every 4 rows leaves 2-way conflicts: measured 1.7x slower on gfx950.)
DEV int swz(int r, int half) { return r * 2 + (half ^ ((r >> 3) & 1)); }

// A launch may carry two problems of one shape (the same layer of two encoders' passes): workgroups
// below `split` run the first arguments, the rest the second, the workgroup index and count rebased.
// A single problem passes its arguments twice and split = the grid.
struct PairSlot {
    int bid, nblk;
    bool second;
};
DEV PairSlot pair_slot(int split) {
    const int b = (int)blockIdx.x;
    const bool s = b >= split;
    return {s ? b - split : b, s ? (int)gridDim.x - split : split, s};
}

// ------------------------------------------------------------------------------------------------
// conv1: 1x1 GEMM, M = N*HW pixels, K = G*32 store channels, 128 outputs.
// A wave computes 64 pixels x 128 outputs (2 x 4 MFMA tiles per K group) over the K groups of its
// k-slice: with KS slices a workgroup of 4 waves covers 64 * 4 / KS pixels, slice s taking groups
// s, s + KS, ... and the partial sums are added through LDS at the end (KS > 1 fills the chip when
// there are few pixels: the 16 x 16 and 32 x 32 blocks).  The main loop has no barrier: the store
// bytes go global -> registers (4 groups ahead) -> prologue -> MFMA operand, the weights global ->
// registers (1 group ahead, L1/L2 hits: every wave reads the same layer); only the fp16 prologue
// table of the layer sits in LDS.
// ------------------------------------------------------------------------------------------------
static constexpr int C1_RED = 20;                        // dwords per lane row of the k-slice sums
static constexpr size_t C1_RED_BYTES = 2 * 8 * 64 * C1_RED * 4;   // two regions: 80 KB

template <int KS, bool ACC32>
__global__ __launch_bounds__(256, 2) void k_conv1(D8sGemmArgs a, int32_t* __restrict__ acc_out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int PX = 64 * 4 / KS;                       // pixels per workgroup
    const int G = a.G, G0 = a.G0;
    uint32_t* s_abh = (uint32_t*)smem;                    // [G * 32] dwords
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);    // uniform: scalar branches
    const int h = lane >> 5, j = lane & 31;
    const int slice = wave % KS, pg = wave / KS;

    const uint32_t* abh32 = (const uint32_t*)a.abh;
    for (int i = tid; i < G * 32; i += 256) s_abh[i] = abh32[i];

    // the lane's two pixels (columns of the two MFMA tiles) and their store rows
    const int64_t rows = a.rows, HW = a.HW;
    const int64_t in_gs = HW * 32, seg_gs = (int64_t)a.N * HW * 32;
    const int64_t mbase = (int64_t)blockIdx.x * PX + pg * 64 + j;
    const int8_t* pin[2];
    const int8_t* pseg[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        int64_t m = mbase + 32 * t;
        if (m >= rows) m = rows - 1;
        const int64_t n = m / HW, p = m - n * HW;
        pin[t] = a.in0 + (n * G0 * HW + p) * 32 + 16 * h;
        pseg[t] = a.seg + (n * HW + p) * 32 + 16 * h;
    }
    auto src = [&](int t, int g) -> const u32x4* {
        return (const u32x4*)(g < G0 ? pin[t] + g * in_gs : pseg[t] + (g - G0) * seg_gs);
    };
    // weights: output tile c, row 32 c + j, half h of group g at wl + g * 256 + 64 c
    const u32x4* wl = (const u32x4*)a.w + j * 2 + h;

    i32x16 acc[2][4];
    const int32_t wmul = slice == 0 ? 128 : 0;            // the offset is added by slice 0 only
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        i32x16 init;
#pragma unroll
        for (int v = 0; v < 16; ++v) init[v] = wmul * a.wsum[32 * c + res_row(v, h)];
        acc[0][c] = init;
        acc[1][c] = init;
    }

    // this slice's groups: g_k = slice + k KS, k < nk
    // Vector loads retire in issue order (s_waitcnt vmcnt), so each step issues the weights it will
    // need next BEFORE the activations four steps ahead: waiting for this step's weights then leaves
    // the later activation loads in flight.
    const int nk = (G - slice + KS - 1) / KS;
    u32x4 ra[4][2];
    u32x4 rb[2][4];
    auto load_a = [&](int slot, int k) {
        const int g = slice + k * KS;
        ra[slot][0] = *src(0, g);
        ra[slot][1] = *src(1, g);
    };
    auto load_b = [&](int bslot, int k) {
        const u32x4* p = wl + (int64_t)(slice + k * KS) * 256;
#pragma unroll
        for (int c = 0; c < 4; ++c) rb[bslot][c] = p[64 * c];
    };
    // The prefetches are unconditional (past the last group they reload it): conditional loads would
    // leave the compiler unable to count the loads in flight, and it would wait for all of them.
    const int klast = nk - 1;
    if (nk > 0) {
        load_b(0, 0);
#pragma unroll
        for (int k = 0; k < 4; ++k) load_a(k, k < klast ? k : klast);
    }
    __syncthreads();                                      // s_abh

    auto step = [&](const int slot, const int k) {
        const int g = slice + k * KS;
        load_b((slot + 1) & 1, k + 1 < klast ? k + 1 : klast);
        asm volatile("" ::: "memory");                   // keep the weight loads ahead in issue order
        const u32x4* pp = (const u32x4*)(s_abh + g * 32 + h * 16);
        const u32x4 p0 = pp[0], p1 = pp[1], p2 = pp[2], p3 = pp[3];
        const u32x4 b0 = pro16(ra[slot][0], p0, p1, p2, p3);
        const u32x4 b1 = pro16(ra[slot][1], p0, p1, p2, p3);
        load_a(slot, k + 4 < klast ? k + 4 : klast);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            acc[0][c] = mfma_i8(rb[slot & 1][c], b0, acc[0][c]);
            acc[1][c] = mfma_i8(rb[slot & 1][c], b1, acc[1][c]);
        }
    };
    for (int k = 0; k < nk; k += 4) {
        step(0, k);
        if (k + 1 < nk) step(1, k + 1);
        if (k + 2 < nk) step(2, k + 2);
        if (k + 3 < nk) step(3, k + 3);
    }

    if (KS > 1) {
        // partial sums of the slices into slice 0 through LDS: [region][t][c][lane] rows of 16 int32,
        // rows C1_RED dwords apart (the padding spreads 8 consecutive lanes over distinct banks)
        auto row = [&](int region, int t, int c) {
            return (i32x16*)((int32_t*)smem + ((region * 8 + t * 4 + c) * 64 + lane) * C1_RED);
        };
        auto put = [&](int region) {
            __syncthreads();
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c) *row(region, t, c) = acc[t][c];
        };
        auto take = [&](int region) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[t][c] += *row(region, t, c);
        };
        if (KS == 2) {
            if (slice == 1) put(pg);
            else __syncthreads();
            __syncthreads();
            if (slice == 0) take(pg);
        } else {
            if (slice >= 2) put(slice - 2);
            else __syncthreads();
            __syncthreads();
            if (slice < 2) take(slice);
            if (slice == 1) put(0);
            else __syncthreads();
            __syncthreads();
            if (slice == 0) take(0);
        }
        if (slice != 0) return;
    }

    // epilogue: v = low byte of fma(sat(fma(g, acc, d)), 255, 2^23) (conv1w_body epilogue,
    // src/knee/dense8s_kernels.cu:595-611), planar bottleneck [4][rows][32]
    const float2* gd = (const float2*)a.gd;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float2 prm[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) prm[v] = gd[32 * c + res_row(v, h)];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t m = mbase + 32 * t;
            if (ACC32) {
                if (m < rows) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const i32x4 q = {acc[t][c][4 * k], acc[t][c][4 * k + 1],
                                         acc[t][c][4 * k + 2], acc[t][c][4 * k + 3]};
                        *(i32x4*)(acc_out + m * 128 + 32 * c + 8 * k + 4 * h) = q;
                    }
                }
                if (a.out == nullptr) continue;
            }
            uint32_t e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t d = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int v = 4 * k + r;
                    float y = __builtin_fmaf(prm[v].x, (float)acc[t][c][v], prm[v].y);
                    y = __builtin_fminf(__builtin_fmaxf(y, 0.0f), 1.0f);
                    const uint32_t b = __float_as_uint(__builtin_fmaf(y, 255.0f, 8388608.0f)) & 0xffu;
                    d |= b << (8 * r);
                }
                e[k] = d;
            }
            const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
            if (m < rows) *(u32x4*)((uint8_t*)a.out + ((int64_t)c * rows + m) * 32 + 16 * h) = row;
        }
        asm volatile("" ::: "memory");                  // one output tile's parameters live at a time
    }
}

// ------------------------------------------------------------------------------------------------
// conv1, persistent: every wave streams 64-pixel tiles t = wave id, + waves in the grid, ... (no
// workgroup-level sharing besides the layer's tables in LDS, no barrier after the start).  Per tile the
// K loop is the one of k_conv1 over G rounded up to a multiple of 4 (padded steps multiply zero
// operands), and the activation prefetch, 4 groups ahead, runs on into the next tile's first groups:
// the first loads of a tile are in flight during the previous tile's last steps and epilogue, so the
// pipeline fills once per wave instead of once per tile.  Used for the large maps (many tiles per
// wave); the pixel offsets are 32-bit (in0 and each store slot < 4 GiB, checked on the host).
// ------------------------------------------------------------------------------------------------
// Activation bytes of step t of a persistent conv1 tile (see k_conv1p): t < Gp this tile's group t
// (past G - 1 a repeat of it, unused), t >= Gp the next tile's group t - Gp (clamped).  Plain values
// in and out: the pixel offsets of the two tiles must stay in registers (selected, never addressed).
template <int U>
DEV void c1p_act(u32x4& r0, u32x4& r1, const uint8_t* in0, const uint8_t* seg, int64_t in_gs,
                 int64_t seg_gs, int G0, int G, int Gp, int t, uint32_t ci0, uint32_t ci1, uint32_t cs0,
                 uint32_t cs1, uint32_t ni0, uint32_t ni1, uint32_t ns0, uint32_t ns1) {
    const bool cur = t < Gp;
    int g = cur ? t : t - Gp;
    g = g < G ? g : G - 1;
    const bool in = g < G0;
    const uint8_t* base = in ? in0 + g * in_gs : seg + (int64_t)(g - G0) * seg_gs;
    const uint32_t o0 = cur ? (in ? ci0 : cs0) : (in ? ni0 : ns0);
    const uint32_t o1 = cur ? (in ? ci1 : cs1) : (in ? ni1 : ns1);
    r0 = *(const u32x4*)(base + o0);
    if (U > 1) r1 = *(const u32x4*)(base + o1);
}

// Byte offsets of the lane's pixels (j, j + 32) of (32 U)-pixel tile t in an in0 group (i0, i1) and
// in a store slot (s0, s1); pixels past the last row repeat it.
template <int U>
DEV void c1p_pixels(int t, int j, int h, int64_t rows, int64_t HW, int G0, uint32_t& i0, uint32_t& i1,
                    uint32_t& s0, uint32_t& s1) {
    int64_t m0 = (int64_t)t * (32 * U) + j, m1 = m0 + 32;
    if (m0 >= rows) m0 = rows - 1;
    if (m1 >= rows) m1 = rows - 1;
    const int64_t n0 = m0 / HW, p0 = m0 - n0 * HW, n1 = m1 / HW, p1 = m1 - n1 * HW;
    i0 = (uint32_t)((n0 * G0 * HW + p0) * 32 + 16 * h);
    i1 = (uint32_t)((n1 * G0 * HW + p1) * 32 + 16 * h);
    s0 = (uint32_t)((n0 * HW + p0) * 32 + 16 * h);
    s1 = (uint32_t)((n1 * HW + p1) * 32 + 16 * h);
}

// LDS of k_conv1p: tables, prologue table, the layer's weights (WM 1) or two 4-group chunks (WM 2)
static size_t c1p_lds(int G, int wm) {
    return 128 * 4 + 128 * 8 + (size_t)G * 128 + (wm == 1 ? (size_t)G * 4096 : 2 * 4 * 4096);
}

// WM: where the conv1 weights are read from.  1: all of the layer's in LDS, loaded once; 2: 4-group
// chunks staged through LDS (double-buffered, one barrier per 4 steps; the waves of a workgroup run
// in step).  From L2 one step ahead they would stall the steps once the layer no longer fits L1.
// U: 32-pixel column blocks per wave (a tile is 32 U pixels).  U = 1 halves the registers, so more
// waves per SIMD hide the latency of layers with few tiles.  PF: activation groups in flight (4, or 8
// where the registers allow); the K loop runs over G rounded up to a multiple of PF.
template <bool ACC32, int WM, int U, int PF>
__global__ __launch_bounds__(256, U == 2 ? 2 : 3) void k_conv1p(D8sGemmArgs a0, int32_t* __restrict__ acc_out,
                                                               D8sGemmArgs a1, int split) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const PairSlot ps = pair_slot(split);
    const D8sGemmArgs a = ps.second ? a1 : a0;
    int32_t* s_wsum = (int32_t*)smem;                     // [128]
    float2* s_gd = (float2*)(s_wsum + 128);               // [128]
    uint32_t* s_abh = (uint32_t*)(s_gd + 128);            // [G * 32]
    const int G = a.G, G0 = a.G0;
    u32x4* s_w = (u32x4*)(s_abh + G * 32);                // WM 1: [G * 256]; WM 2: [2][4 * 256]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int64_t rows = a.rows, HW = a.HW;
    const int ntiles = (int)((rows + 32 * U - 1) / (32 * U));
    const int stride = ps.nblk * 4;
    // the workgroup's tiles are first, first + 1, ..., first + 3 (then + stride ...): it runs while its
    // first tile exists, so its waves run in step (a wave past the last tile works on a repeat of the
    // last pixel and stores nothing)
    int first = ps.bid * 4;
    if (first >= ntiles) return;                         // (uniform per workgroup)
    int tile = first + wave;

    const uint8_t* in0 = (const uint8_t*)a.in0;
    const uint8_t* seg = (const uint8_t*)a.seg;
    uint8_t* out = (uint8_t*)a.out;
    const int64_t in_gs = HW * 32, seg_gs = (int64_t)a.N * HW * 32;
    uint32_t ci0, ci1, cs0, cs1, ni0, ni1, ns0, ns1;      // this tile's and the next tile's offsets
    c1p_pixels<U>(tile, j, h, rows, HW, G0, ci0, ci1, cs0, cs1);
    int next = tile + stride;
    c1p_pixels<U>(next, j, h, rows, HW, G0, ni0, ni1, ns0, ns1);

    const int Gp = (G + PF - 1) & ~(PF - 1);
    u32x4 ra[PF][2];                                      // [slot][block] (block 1 unused for U = 1)
    u32x4 rb[4];
    u32x4 stg[4];                                         // WM 2: the next chunk on its way
    int cc = 0;                                           // WM 2: chunks done (buffer cc & 1)
    const u32x4* wg = (const u32x4*)a.w;
    // weights of step k for the MFMA: output tile c, row 32 c + j, half h of group g (chunk
    // g * 256 + 64 c + 2 j + h of the layer; of the chunk buffer for WM 2)
#define C1P_LOAD_B(k)                                                                             \
    do {                                                                                          \
        const int g_ = (k) < G ? (k) : G - 1;                                                     \
        const u32x4* p_ = WM == 1 ? s_w + g_ * 256 : s_w + (cc & 1) * 1024 + ((k) & 3) * 256;     \
        p_ += j + 32 * h;                                                                         \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) rb[c_] = p_[64 * c_];                    \
    } while (0)
#define C1P_LOAD_A(slot, t)                                                                       \
    c1p_act<U>(ra[slot][0], ra[slot][1], in0, seg, in_gs, seg_gs, G0, G, Gp, (t), ci0, ci1, cs0, cs1, \
            ni0, ni1, ns0, ns1)

    // the first activation groups are requested before the layer's tables are staged, so the two
    // latencies overlap
#pragma unroll
    for (int s0 = 0; s0 < PF; ++s0) C1P_LOAD_A(s0, s0);
    // the tables and the weights (WM 2: chunk 0): the first NW weight and NAB table items per thread
    // requested at once (clamped addresses), then stored; loops stage what is left (a load-and-store
    // loop waits one L2 round trip per iteration)
    {
        constexpr int NW = WM == 1 ? 16 : 4, NAB = 2;     // 16 (4) groups of weights, 16 of tables
        const uint32_t* abh32 = (const uint32_t*)a.abh;
        const u32x4* w = (const u32x4*)a.w;
        const int nw = WM == 1 ? G * 256 : min(G, 4) * 256;
        u32x4 v[NW];
        uint32_t vab[NAB];
#pragma unroll
        for (int k = 0; k < NW; ++k) v[k] = w[min(tid + 256 * k, G * 256 - 1)];
#pragma unroll
        for (int k = 0; k < NAB; ++k) vab[k] = abh32[min(tid + 256 * k, G * 32 - 1)];
        const int32_t t_ws = a.wsum[min(tid, 127)];
        const float2 t_gd = ((const float2*)a.gd)[min(tid, 127)];
#pragma unroll
        for (int k = 0; k < NW; ++k)
            if (tid + 256 * k < nw) s_w[wperm(tid + 256 * k)] = v[k];
#pragma unroll
        for (int k = 0; k < NAB; ++k)
            if (tid + 256 * k < G * 32) s_abh[tid + 256 * k] = vab[k];
        if (tid < 128) {
            s_wsum[tid] = t_ws;
            s_gd[tid] = t_gd;
        }
        for (int i = tid + 256 * NAB; i < G * 32; i += 256) s_abh[i] = abh32[i];
        for (int i = tid + 256 * NW; i < nw; i += 4 * 256) {
            u32x4 x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = w[min(i + u * 256, G * 256 - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i + u * 256 < nw) s_w[wperm(i + u * 256)] = x[u];
        }
    }
    __syncthreads();

    for (;;) {
        i32x16 acc[U][4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            i32x16 init;
#pragma unroll
            for (int v = 0; v < 16; ++v) init[v] = 128 * s_wsum[32 * c + res_row(v, h)];
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u][c] = init;
        }
        // one K step: weights of the next step first (issue order), the prologue of this step's bytes
        // (zero operands on padded steps), the activations 4 steps ahead, the 8 MFMAs
#define C1P_STEP(slot, k, PAD)                                                                    \
    do {                                                                                          \
        const int k_ = (k);                                                                       \
        C1P_LOAD_B(k_);                                                                           \
        u32x4 b0_, b1_;                                                                           \
        if (!PAD || k_ < G) {                                                                     \
            const u32x4* pp_ = (const u32x4*)(s_abh + k_ * 32 + h * 16);                          \
            const u32x4 p0_ = pp_[0], p1_ = pp_[1], p2_ = pp_[2], p3_ = pp_[3];                   \
            b0_ = pro16(ra[slot][0], p0_, p1_, p2_, p3_);                                         \
            if (U > 1) b1_ = pro16(ra[slot][1], p0_, p1_, p2_, p3_);                              \
        } else {                                                                                  \
            b0_ = u32x4{0, 0, 0, 0};                                                              \
            b1_ = u32x4{0, 0, 0, 0};                                                              \
        }                                                                                         \
        C1P_LOAD_A(slot, k_ + PF);                                                                \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) {                                        \
            acc[0][c_] = mfma_i8(rb[c_], b0_, acc[0][c_]);                                        \
            if (U > 1) acc[U - 1][c_] = mfma_i8(rb[c_], b1_, acc[U - 1][c_]);                     \
        }                                                                                         \
    } while (0)
        // four steps = one weight chunk; PAD: the last chunk of a tile, whose steps past G - 1 multiply
        // zero operands (the others need no test)
#define C1P_CHUNK(PAD, SB)                                                                        \
    do {                                                                                          \
        if (WM == 2) {                             /* the next chunk (the next tile's first) */   \
            const int nc_ = k + 4 < Gp ? (k >> 2) + 1 : 0;                                        \
            _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_)                                      \
                stg[u_] = wg[min(nc_ * 1024 + tid + 256 * u_, G * 256 - 1)];                      \
        }                                                                                         \
        C1P_STEP((SB) + 0, k, PAD);                                                               \
        C1P_STEP((SB) + 1, k + 1, PAD);                                                           \
        C1P_STEP((SB) + 2, k + 2, PAD);                                                           \
        C1P_STEP((SB) + 3, k + 3, PAD);                                                           \
        if (WM == 2) {                             /* its buffer was last read in chunk cc - 1 */ \
            _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_)                                      \
                s_w[((cc + 1) & 1) * 1024 + wperm(tid + 256 * u_)] = stg[u_];                     \
            __syncthreads();                                                                      \
            ++cc;                                                                                 \
        }                                                                                         \
        k += 4;                                                                                   \
    } while (0)
        // chunks of 4 steps; with PF = 8 in pairs, so that step k uses activation slot k % 8
        int k = 0;
        for (; k < (G & ~(PF - 1));) {
            C1P_CHUNK(false, 0);
            if (PF == 8) C1P_CHUNK(false, 4);
        }
        if (k < Gp) {
            C1P_CHUNK(true, 0);
            if (PF == 8) C1P_CHUNK(true, 4);
        }
#undef C1P_CHUNK
#undef C1P_STEP

        // epilogue as k_conv1 (conv1w_body epilogue, src/knee/dense8s_kernels.cu:595-611)
        const int64_t mbase = (int64_t)tile * (32 * U) + j;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t m = mbase + 32 * u;
                if (ACC32) {
                    if (m < rows) {
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const i32x4 q = {acc[u][c][4 * kk], acc[u][c][4 * kk + 1],
                                             acc[u][c][4 * kk + 2], acc[u][c][4 * kk + 3]};
                            *(i32x4*)(acc_out + m * 128 + 32 * c + 8 * kk + 4 * h) = q;
                        }
                    }
                    if (out == nullptr) continue;
                }
                uint32_t e[4];
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    uint32_t d = 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int v = 4 * kk + r;
                        const float2 prm = s_gd[32 * c + res_row(v, h)];
                        float y = __builtin_fmaf(prm.x, (float)acc[u][c][v], prm.y);
                        y = __builtin_fminf(__builtin_fmaxf(y, 0.0f), 1.0f);
                        const uint32_t b = __float_as_uint(__builtin_fmaf(y, 255.0f, 8388608.0f)) & 0xffu;
                        d |= b << (8 * r);
                    }
                    e[kk] = d;
                }
                const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
                if (m < rows) *(u32x4*)(out + ((int64_t)c * rows + m) * 32 + 16 * h) = row;
            }
            __builtin_amdgcn_sched_barrier(0);         // one output tile's values live at a time
        }
        first += stride;
        if (first >= ntiles) break;
        tile = next;
        ci0 = ni0;
        ci1 = ni1;
        cs0 = ns0;
        cs1 = ns1;
        next = tile + stride;
        c1p_pixels<U>(next, j, h, rows, HW, G0, ni0, ni1, ns0, ns1);
    }
#undef C1P_LOAD_A
#undef C1P_LOAD_B
}

// ------------------------------------------------------------------------------------------------
// conv2: 3x3 pad 1, 128 -> 32.  Persistent workgroups with the 36 KB of weights resident in LDS, one
// spatial tile of TH x TW output pixels at a time with the halo of its 4 bottleneck planes in LDS.
// The next tile's halo is loaded into registers while the current one is computed.
//   KSPL = 1: the 4 waves take PT MFMA pixel tiles (32 pixels) each over all 4 planes (36 MFMA
//             K-steps of 32), TH x TW = 4 * 32 * PT;
//   KSPL = 4: wave w takes plane w (9 K-steps) of the same PT pixel tiles, TH x TW = 32 * PT, and the
//             four partial sums are added through LDS (narrow maps: 4x the tiles).
// Tile shapes are compile-time so the halo's 16-byte chunks decompose without runtime divisions.
// ------------------------------------------------------------------------------------------------
static constexpr int C2_RED = 20;                         // dwords per lane row of the partial sums

template <int TW, int TH, int KSPL, int PT>
struct C2Shape {
    static constexpr int HWd = TW + 2, HP = (TH + 2) * HWd;
    static constexpr int NCHUNK = 8 * HP;                 // 16-byte halo chunks (4 planes x 2 halves)
    static constexpr int NCH = (NCHUNK + 255) / 256;      // per thread
    static constexpr size_t HALO_BYTES = (size_t)NCHUNK * 16;
    static constexpr size_t RED_BYTES = KSPL > 1 ? (size_t)3 * PT * 64 * C2_RED * 4 : 0;
    static_assert(TW * TH == (KSPL == 1 ? 4 : 1) * 32 * PT, "tile = the waves' pixel tiles");
};

template <int TW, int TH, int KSPL, int PT>
__global__ __launch_bounds__(256, 2) void k_conv2(D8sConv2Args a0, int tiles_x, int tiles_y, D8sConv2Args a1,
                                                  int split) {
    using S = C2Shape<TW, TH, KSPL, PT>;
    const PairSlot ps = pair_slot(split);
    const D8sConv2Args a = ps.second ? a1 : a0;
    constexpr int HWd = S::HWd, HP = S::HP, NCH = S::NCH;
    __shared__ __attribute__((aligned(16))) u32x4 s_w[4 * 9 * 32 * 2];
    extern __shared__ __attribute__((aligned(16))) u32x4 s_x[];       // [4][HP][2], then partial sums
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int H = a.H, W = a.W;
    const int64_t M = (int64_t)a.N * H * W;

    {
        u32x4 wv[9];                                      // 2304 chunks = 9 per thread, all in flight
#pragma unroll
        for (int k = 0; k < 9; ++k) wv[k] = ((const u32x4*)a.w)[tid + 256 * k];
#pragma unroll
        for (int k = 0; k < 9; ++k) s_w[swz((tid + 256 * k) >> 1, tid & 1)] = wv[k];
    }

    const int32_t wmul = (KSPL == 1 || wave == 0) ? 128 : 0;
    i32x16 init;
    float sc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        init[v] = wmul * a.wsum[res_row(v, h)];
        sc[v] = a.sc[res_row(v, h)];
    }
    int q0[PT], ty[PT], tx[PT];
#pragma unroll
    for (int t = 0; t < PT; ++t) {
        const int p = (KSPL == 1 ? wave * PT * 32 : 0) + 32 * t + j;
        ty[t] = p / TW;
        tx[t] = p - ty[t] * TW;
        q0[t] = ty[t] * HWd + tx[t];
    }

    // halo chunks of this thread: chunk i = tid + 256 k -> plane c, halo pixel hp, half hh.  Every
    // chunk is loaded (chunks outside the image from the tile's first pixel) with no use of the data
    // until the LDS store, so all NCH loads are in flight together; the store applies the padding
    // (u = 0, i.e. byte 0x80) and the u - 128 offset.
    u32x4 hreg[NCH];
    uint32_t hvalid = 0;
    auto hload = [&](int tile) {
        const int per_img = tiles_x * tiles_y;
        const int n = tile / per_img, r = tile - n * per_img;
        const int y0 = (r / tiles_x) * TH, x0 = (r % tiles_x) * TW;
        const uint8_t* base = a.x + (((int64_t)n * H + y0) * W + x0) * 32;
        hvalid = 0;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int i = tid + 256 * k;
            const int c = i / (2 * HP), rr = i - c * (2 * HP);
            const int hp = rr >> 1, hh = rr & 1;
            const int hy = hp / HWd, hx = hp - hy * HWd;
            const int y = y0 - 1 + hy, x = x0 - 1 + hx;
            const bool ok = i < S::NCHUNK && (unsigned)y < (unsigned)H && (unsigned)x < (unsigned)W;
            const int64_t off = ok ? (c * M + (int64_t)(hy - 1) * W + (hx - 1)) * 32 + 16 * hh : 0;
            hreg[k] = *(const u32x4*)(base + off);
            hvalid |= (uint32_t)ok << k;
        }
    };
    auto hstore = [&]() {
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int i = tid + 256 * k;
            const int c = i / (2 * HP), rr = i - c * (2 * HP);
            const u32x4 pad = {SIGN4, SIGN4, SIGN4, SIGN4};
            if (i < S::NCHUNK) s_x[c * HP * 2 + swz(rr >> 1, rr & 1)] = ((hvalid >> k) & 1) ? hreg[k] ^ SIGN4 : pad;
        }
    };

    // tile order: workgroups are dispatched to the 8 XCDs round robin (workgroup b on XCD b % 8), so
    // a persistent grid gives XCD x one contiguous eighth of the tiles, walked by its workgroups
    // together: tiles in flight on one XCD are neighbours, and their shared halo rows hit its L2
    const int total = a.N * tiles_x * tiles_y;
    // (a pair's split is a multiple of 8, so the rebased index keeps the XCD)
    int tile = ps.bid, tend = total, tstep = ps.nblk;
    if (total > ps.nblk && (ps.nblk & 7) == 0) {
        const int chunk = (total + 7) / 8, xcd = ps.bid & 7;
        tstep = ps.nblk >> 3;
        tile = xcd * chunk + (ps.bid >> 3);
        tend = min(total, (xcd + 1) * chunk);
    }
    if (tile >= tend) return;
    hload(tile);
    __syncthreads();                                      // weights
    hstore();
    __syncthreads();
    for (; tile < tend; tile += tstep) {
        const int next = tile + tstep;
        if (next < tend) hload(next);                     // in flight during this tile's MFMAs
        i32x16 acc[PT];
#pragma unroll
        for (int t = 0; t < PT; ++t) acc[t] = init;
        // K steps (plane, tap); the operands of step s + FD are read from LDS before step s's MFMAs (an
        // LDS read takes longer than a step's MFMAs: FD 3 for one pixel tile, 2 for two)
        constexpr int NS = KSPL == 1 ? 36 : 9;
        constexpr int FD = PT == 1 ? 3 : PT == 2 ? 2 : 1;
        u32x4 aw[4], bx[4][PT];
        auto fetch = [&](int s, int slot) INLINE {
            const int c = KSPL == 1 ? s / 9 : wave, tap = s % 9;
            const int off = (tap / 3) * HWd + (tap % 3);
            aw[slot] = s_w[swz((c * 9 + tap) * 32 + j, h)];
#pragma unroll
            for (int t = 0; t < PT; ++t) bx[slot][t] = s_x[c * HP * 2 + swz(q0[t] + off, h)];
        };
#pragma unroll
        for (int f = 0; f < FD; ++f) fetch(f, f);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if (s + FD < NS) fetch(s + FD, (s + FD) & 3);
#pragma unroll
            for (int t = 0; t < PT; ++t) acc[t] = mfma_i8(aw[s & 3], bx[s & 3][t], acc[t]);
            if constexpr (FD > 1) __builtin_amdgcn_sched_barrier(0);
        }
        if (KSPL > 1) {
            // waves 1..3 hand their partial sums to wave 0 (rows of 16 int32 per lane, padded)
            int32_t* red = (int32_t*)((uint8_t*)s_x + S::HALO_BYTES);
            if (wave > 0) {
#pragma unroll
                for (int t = 0; t < PT; ++t)
                    *(i32x16*)(red + (((wave - 1) * PT + t) * 64 + lane) * C2_RED) = acc[t];
            }
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (int w = 0; w < 3; ++w)
#pragma unroll
                    for (int t = 0; t < PT; ++t)
                        acc[t] += *(const i32x16*)(red + ((w * PT + t) * 64 + lane) * C2_RED);
            }
        }
        // epilogue: q = RNE(clamp(float(acc) * sc, -127, 127)) (conv2t_body,
        // src/knee/dense8s_kernels.cu:2797-2809)
        if (KSPL == 1 || wave == 0) {
            const int per_img = tiles_x * tiles_y;
            const int n = tile / per_img, r = tile - n * per_img;
            const int y0 = (r / tiles_x) * TH, x0 = (r % tiles_x) * TW;
#pragma unroll
            for (int t = 0; t < PT; ++t) {
                uint32_t e[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t d = 0;
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const int v = 4 * k + rr;
                        const float q = __builtin_rintf(
                            __builtin_fminf(__builtin_fmaxf((float)acc[t][v] * sc[v], -127.0f), 127.0f));
                        d |= ((uint32_t)(int)q & 0xffu) << (8 * rr);
                    }
                    e[k] = d;
                }
                const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
                const int y = y0 + ty[t], x = x0 + tx[t];
                if (y < H && x < W)
                    *(u32x4*)(a.out + (((int64_t)n * H + y) * W + x) * 32 + 16 * h) = row;
            }
        }
        __syncthreads();                                  // this tile's halo and partial sums read
        if (next < tend) {
            hstore();
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------------------------------------
// conv2 of layer l, then conv1 of layer l + 1, in one launch.  conv1 is pixel-local, so the 32
// channels conv2 gives a pixel are the last K group of the next layer's conv1 on the same pixel: a
// lane's conv2 epilogue leaves exactly the 16 bytes the conv1 B operand of that lane needs (pixel j,
// bytes 16 h .. 16 h + 15), which stay in registers while the bytes go to the layer's store slot.
// Only the bottleneck crosses the launch boundary, in two buffers: conv2 reads layer l's while
// conv1 writes layer l + 1's.
// Persistent workgroups of 4 waves over tiles of 128 pixels of one image (R = 128 / W rows, W = 16,
// 32 or 64); wave w owns pixels 32 w .. 32 w + 31 of the tile in both phases.  One LDS region serves
// the two phases in turn (a workgroup runs them one after the other; the workgroups sharing a CU
// overlap each other's):
//   conv2 (as k_conv2 with one pixel tile per wave): the tile's (R + 2) x (W + 2) halo of the 4
//         bottleneck planes and the weights one input plane (9 KB) at a time, double-buffered;
//   conv1 (as k_conv1p, one 32-pixel column block): activations from the store 4 groups ahead, the
//         prefetch running on into the next tile's first groups (in flight during its conv2), the
//         weights in 4-group chunks double-buffered.
// Group G - 1 (the new one) is never read from memory: its step takes the conv2 result (the load of
// that slot is clamped to G - 2 and its value unused).  At most 53 KB of LDS per workgroup (W = 64:
// one plane buffer, two barriers per plane) and 168 VGPRs: three workgroups share a CU.  Offsets are
// 32-bit where the host checked the sizes.
// ------------------------------------------------------------------------------------------------
template <int W_>
struct CcShape {
    static constexpr int R = 128 / W_;                    // rows of a tile
    static constexpr int HWd = W_ + 2, HP = (R + 2) * HWd;
    static constexpr int NCHUNK = 8 * HP;                 // 16-byte halo chunks (4 planes x 2 halves)
    static constexpr int NCH = (NCHUNK + 255) / 256;      // per thread
    static constexpr size_t HALO = (size_t)NCHUNK * 16;
    static constexpr size_t W2BUF = 9 * 32 * 32;          // one input plane of the conv2 weights
    static constexpr int NW2 = W_ <= 32 ? 2 : 1;          // plane buffers (one where the halo is large)
    static constexpr size_t A_BYTES = HALO + NW2 * W2BUF, B_BYTES = 2 * 4 * 4096;
    static constexpr size_t UNION = A_BYTES > B_BYTES ? A_BYTES : B_BYTES;
    static constexpr int OCC = 3;                         // workgroups per CU
    static_assert(128 % W_ == 0 && R >= 2, "tile = whole rows of 128 pixels");
};

static constexpr size_t CC_TABLES = 128 * 4 + 128 * 8 + 32 * 4 + 32 * 4;

template <int W_>
static size_t cc_lds(int G) {
    return CcShape<W_>::UNION + CC_TABLES + (size_t)G * 128;
}

// activation bytes of conv1 step t (t < Gp: this tile's group t, else the next tile's group t - Gp),
// groups past G - 2 clamped to G - 2 (G - 1 comes from registers, padded steps are unused).  Without a
// next tile (nx false) the loads past Gp are unused too and read group G - 2 again, which the last
// steps just read (an L2 hit, not the tile's first groups again from HBM).
DEV u32x4 cc_act(const uint8_t* in0, const uint8_t* seg, int64_t in_gs, int64_t seg_gs, int G0, int G, int Gp,
                 int t, uint32_t ci, uint32_t cs, uint32_t ni, uint32_t ns, bool nx) {
    const bool cur = t < Gp;
    int g = cur ? t : (nx ? t - Gp : G - 2);
    g = g < G - 1 ? g : G - 2;
    const bool in = g < G0;
    const uint8_t* base = in ? in0 + g * in_gs : seg + (int64_t)(g - G0) * seg_gs;
    const uint32_t o = cur ? (in ? ci : cs) : (in ? ni : ns);
    return *(const u32x4*)(base + o);
}

template <int W_>
__global__ __launch_bounds__(256, CcShape<W_>::OCC) void k_c21(D8sConv2Args c2, D8sGemmArgs c1) {
    using S = CcShape<W_>;
    constexpr int R = S::R, HWd = S::HWd, HP = S::HP, NCH = S::NCH, PF = 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    u32x4* s_u = (u32x4*)smem;                                      // halo [4][HP][2] | chunks [2][1024]
    u32x4* s_w2 = (u32x4*)(smem + S::HALO);                         // [2][9 * 32 * 2] swizzled planes
    int32_t* s_wsum = (int32_t*)(smem + S::UNION);                  // [128]
    float2* s_gd = (float2*)(s_wsum + 128);                         // [128]
    float* s_sc2 = (float*)(s_gd + 128);                            // [32]
    int32_t* s_ini2 = (int32_t*)(s_sc2 + 32);                       // [32] 128 sum(w2)
    uint32_t* s_abh = (uint32_t*)(s_ini2 + 32);                     // [G * 32]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int G = c1.G, G0 = c1.G0, HW = c1.HW, H = c2.H;
    const int per_img = HW / 128, total = c1.N * per_img;
    const int64_t M = c1.rows;
    const int p = 32 * wave + j, ty = p / W_, tx = p - ty * W_, q0 = ty * HWd + tx;

    // tile order as k_conv2: XCD x walks one contiguous eighth of the tiles (also with one tile per
    // workgroup: neighbouring tiles share halo rows in that XCD's L2)
    int tile = blockIdx.x, tend = total, tstep = gridDim.x;
    if (total >= (int)gridDim.x && (gridDim.x & 7) == 0) {
        const int chunk = (total + 7) / 8, xcd = blockIdx.x & 7;
        tstep = gridDim.x >> 3;
        tile = xcd * chunk + (blockIdx.x >> 3);
        tend = min(total, (xcd + 1) * chunk);
    }
    if (tile >= tend) return;                               // (uniform per workgroup)

    const uint8_t* in0 = (const uint8_t*)c1.in0;
    const uint8_t* seg = (const uint8_t*)c1.seg;
    const int64_t in_gs = (int64_t)HW * 32, seg_gs = M * 32;
    // conv1 pixel offsets of a tile's pixel for this lane: in0 group 0 and store slot 0
    // (the lane's pixel and half recomputed from an opaque copy of the thread index: kept across the
    // tile loop they were spilled, and their reload at each tile's start waited for every load in
    // flight)
    auto offs = [&](int t, uint32_t& oi, uint32_t& os) INLINE {
        int t0 = tid;
        asm volatile("" : "+v"(t0));
        const int lp = 32 * (t0 >> 6) + (t0 & 31), lh = 16 * ((t0 >> 5) & 1);
        const int n = t / per_img, pi = (t - n * per_img) * 128 + lp;
        oi = (uint32_t)(((int64_t)n * G0 * HW + pi) * 32 + lh);
        os = (uint32_t)(((int64_t)n * HW + pi) * 32 + lh);
    };
    uint32_t ci, cs, ni, ns;
    offs(tile, ci, cs);
    offs(tile + tstep < tend ? tile + tstep : tile, ni, ns);

    // halo chunks of this thread: chunk i = tid + 256 k -> plane c, halo pixel (hy, hx), half hh, at
    // byte (c M + hy W + hx) 32 + 16 hh from the pixel above-left of the tile (a buffer resource based
    // there, uniform per tile).  Chunks outside the image (or past the halo) take an offset past the
    // resource's range, which reads zero: u = 0 after the XOR, the padding.  The chunk geometry is
    // recomputed per tile from an opaque copy of the thread index (kept out of registers across the
    // phases).
    constexpr uint32_t CC_OOB = 0xffffff00u;
    u32x4 hreg[NCH];
    auto hload = [&](int t) INLINE {
        const int n = t / per_img, y0 = (t - n * per_img) * R;
        const bool top = y0 == 0, bot = y0 + R == H;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(c2.x + ((int64_t)n * HW + (int64_t)y0 * W_ - W_ - 1) * 32), 0, 0x7fffffff, 0x00020000);
        int t0 = tid;
        asm volatile("" : "+v"(t0));
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int i = t0 + 256 * k;
            const int c = i / (2 * HP), rr = i - c * (2 * HP);
            const int hp = rr >> 1, hh = rr & 1;
            const int hy = hp / HWd, hx = hp - hy * HWd;
            const bool ok = i < S::NCHUNK && hx >= 1 && hx <= W_ && !(top && hy == 0) && !(bot && hy == R + 1);
            const uint32_t off = (uint32_t)((c * M + hy * W_ + hx) * 32 + 16 * hh);
            hreg[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, ok ? off : CC_OOB, 0, 0));
        }
    };
    auto hstore = [&]() INLINE {
        int t0 = tid;
        asm volatile("" : "+v"(t0));
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int i = t0 + 256 * k;
            const int c = i / (2 * HP), rr = i - c * (2 * HP);
            if (i < S::NCHUNK) s_u[c * HP * 2 + swz(rr >> 1, rr & 1)] = hreg[k] ^ SIGN4;
        }
    };
    // conv2 weights of input plane c: 576 chunks ([tap][out][half]), at most 3 per thread (buffer loads:
    // one lane offset, the plane and part in the scalar offset; every read inside the table: the third
    // part's chunks 512-575 are read by lanes tid & 63, the other lanes' copies unused)
    const __amdgpu_buffer_rsrc_t rw2 = __builtin_amdgcn_make_buffer_rsrc((void*)c2.w, 0, 36864, 0x00020000);
    u32x4 wst[3];
    auto w2load = [&](int c) INLINE {
#pragma unroll
        for (int u = 0; u < 3; ++u)
            wst[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                rw2, (uint32_t)((u < 2 ? tid : tid & 63) * 16), (uint32_t)(c * 9216 + u * 4096), 0));
    };
    auto w2store = [&](int buf) INLINE {
        int t0 = tid;
        asm volatile("" : "+v"(t0));
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int i = t0 + 256 * u;
            if (i < 576) s_w2[buf * 576 + swz(i >> 1, i & 1)] = wst[u];
        }
    };

    const int Gp = (G + PF - 1) & ~(PF - 1), nchunk = Gp >> 2;
    // conv1 weights: 4-group chunks of 16 KB, 4 loads per thread (one group each), as buffer loads with
    // the group in the scalar offset, clamped to group G - 1 past the table (read only by padded steps,
    // whose activation operand is zero): every read inside the table
    const __amdgpu_buffer_rsrc_t rw1 = __builtin_amdgcn_make_buffer_rsrc((void*)c1.w, 0, G * 4096, 0x00020000);
    auto w1load = [&](u32x4* dst, int chunk) INLINE {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            dst[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                rw1, (uint32_t)tid * 16, (uint32_t)(min(4 * chunk + u, G - 1) * 4096), 0));
    };
    auto w1store = [&](const u32x4* src, int buf) INLINE {
        int t0 = tid;
        asm volatile("" : "+v"(t0));
#pragma unroll
        for (int u = 0; u < 4; ++u) s_u[buf * 1024 + wperm(t0 + 256 * u)] = src[u];
    };
    // the two outputs through buffer stores: the lane's byte offset p 32 + 16 h, the tile (and plane)
    // in the scalar offset (the host checked 4 M 32 < 2^31)
    const __amdgpu_buffer_rsrc_t ro2 = __builtin_amdgcn_make_buffer_rsrc((void*)c2.out, 0, (int)(M * 32), 0x00020000);
    const __amdgpu_buffer_rsrc_t ro1 = __builtin_amdgcn_make_buffer_rsrc(c1.out, 0, (int)(M * 128), 0x00020000);
    const uint32_t lo_off = (uint32_t)(p * 32 + 16 * h);
    u32x4 ra[PF], rb[4], stg[4];
    // the tables first (all their loads at once, from clamped addresses: a load per loop iteration,
    // each waited for before its store, made the start wait for every load in flight and then one L2
    // round trip per iteration), then the first tile's halo, activations, conv2 plane 0 and conv1
    // chunk 0, in flight while the tables are stored
    constexpr int NAB = (D8S_C21_MAX_GROUPS * 32 + 255) / 256;
    uint32_t tab[NAB], t_ws;
    float2 t_gd;
    float t_sc2;
    int32_t t_w2;
    {
        const uint32_t* abh32 = (const uint32_t*)c1.abh;
#pragma unroll
        for (int k = 0; k < NAB; ++k) tab[k] = abh32[min(tid + 256 * k, G * 32 - 1)];
        t_ws = (uint32_t)c1.wsum[min(tid, 127)];
        t_gd = ((const float2*)c1.gd)[min(tid, 127)];
        t_sc2 = c2.sc[min(tid, 31)];
        t_w2 = c2.wsum[min(tid, 31)];
    }
    hload(tile);
    w2load(0);
#pragma unroll
    for (int s = 0; s < PF; ++s)
        ra[s] = cc_act(in0, seg, in_gs, seg_gs, G0, G, Gp, s, ci, cs, ni, ns, true);
    w1load(stg, 0);
    {
#pragma unroll
        for (int k = 0; k < NAB; ++k)
            if (tid + 256 * k < G * 32) s_abh[tid + 256 * k] = tab[k];
        if (tid < 128) {
            s_wsum[tid] = (int32_t)t_ws;
            s_gd[tid] = t_gd;
        }
        if (tid < 32) {
            s_sc2[tid] = t_sc2;
            s_ini2[tid] = 128 * t_w2;
        }
    }
    hstore();
    w2store(0);
    __syncthreads();

    for (;;) {
        const int next = tile + tstep;
        const bool more = next < tend;
        const uint32_t tb = (uint32_t)tile * 4096;           // the tile's first byte in a plane / slot

        // ---- conv2 of layer l: per input plane c, 9 taps; plane c + 1's weights staged meanwhile ----
        i32x16 acc2;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc2[v] = s_ini2[res_row(v, h)];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (S::NW2 == 1 && c > 0) {                      // one buffer: plane c replaces c - 1
                __syncthreads();
                w2store(0);
                __syncthreads();
            }
            if (c < 3) w2load(c + 1);
            __builtin_amdgcn_sched_barrier(0);               // (issued before the plane's MFMAs)
            const u32x4* pw = s_w2 + (S::NW2 == 1 ? 0 : (c & 1) * 576);
            const u32x4* px = s_u + c * HP * 2;
            u32x4 aw[2], bx[2];
            auto fetch = [&](int tap, int slot) INLINE {
                const int off = (tap / 3) * HWd + (tap % 3);
                aw[slot] = pw[swz(tap * 32 + j, h)];
                bx[slot] = px[swz(q0 + off, h)];
            };
            fetch(0, 0);
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) {
                if (tap + 1 < 9) fetch(tap + 1, (tap + 1) & 1);
                acc2 = mfma_i8(aw[tap & 1], bx[tap & 1], acc2);
            }
            if (S::NW2 == 2 && c < 3) {
                w2store((c + 1) & 1);                        // buffer last read in plane c - 1
                __syncthreads();
            }
        }
        // epilogue (conv2t_body, src/knee/dense8s_kernels.cu:2797-2809): the layer's store bytes,
        // kept as conv1's last group
        u32x4 row;
        {
            uint32_t e[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) e[q] = epi2_q(acc2, q, *(const float4*)(s_sc2 + 8 * q + 4 * h));
            row = xchg_rows(e[0], e[1], e[2], e[3], h);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, row), ro2, lo_off, tb, 0);
        }
        __syncthreads();                                     // the halo and plane 3 are read
        w1store(stg, 0);
        __syncthreads();

        // ---- conv1 of layer l + 1 ----
        i32x16 acc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[c][v] = 128 * s_wsum[32 * c + res_row(v, h)];
        int k = 0, cc = 0;
#define CC_STEP(slot, PAD)                                                                        \
    do {                                                                                          \
        const int k_ = k + (slot);                                                                \
        const u32x4* pw_ = s_u + (cc & 1) * 1024 + (slot) * 256 + j + 32 * h;                     \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) rb[c_] = pw_[64 * c_];                   \
        u32x4 b_;                                                                                 \
        if (!PAD || k_ < G) {                                                                     \
            const u32x4* pp_ = (const u32x4*)(s_abh + k_ * 32 + h * 16);                          \
            const u32x4 x_ = (PAD && k_ == G - 1) ? row : ra[slot];                               \
            b_ = pro16(x_, pp_[0], pp_[1], pp_[2], pp_[3]);                                       \
        } else {                                                                                  \
            b_ = u32x4{0, 0, 0, 0};                                                               \
        }                                                                                         \
        ra[slot] = cc_act(in0, seg, in_gs, seg_gs, G0, G, Gp, k_ + PF, ci, cs, ni, ns, more);     \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) acc[c_] = mfma_i8(rb[c_], b_, acc[c_]);  \
    } while (0)
        // the last chunk holds group G - 1 (G - 1 >= Gp - 4) and the padded steps
        for (; cc + 1 < nchunk; ++cc, k += 4) {
            w1load(stg, cc + 1);
            CC_STEP(0, false);
            CC_STEP(1, false);
            CC_STEP(2, false);
            CC_STEP(3, false);
            w1store(stg, (cc + 1) & 1);
            __syncthreads();
        }
        w1load(stg, 0);                                      // the next tile's chunk 0
        CC_STEP(0, true);
        CC_STEP(1, true);
        CC_STEP(2, true);
        CC_STEP(3, true);
#undef CC_STEP

        // epilogue as k_conv1p: the planar u8 bottleneck of layer l + 1
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint32_t e[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                uint32_t d = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int v = 4 * kk + r;
                    const float2 prm = s_gd[32 * c + res_row(v, h)];
                    float y = __builtin_fmaf(prm.x, (float)acc[c][v], prm.y);
                    y = __builtin_fminf(__builtin_fmaxf(y, 0.0f), 1.0f);
                    const uint32_t b = __float_as_uint(__builtin_fmaf(y, 255.0f, 8388608.0f)) & 0xffu;
                    d |= b << (8 * r);
                }
                e[kk] = d;
            }
            const u32x4 orow = xchg_rows(e[0], e[1], e[2], e[3], h);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, orow), ro1, lo_off,
                                                   (uint32_t)(c * M * 32) + tb, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (!more) break;
        hload(next);                                         // the next tile's halo and plane 0
        w2load(0);
        __syncthreads();                                     // the weight chunks are read
        hstore();
        w2store(0);
        __syncthreads();
        tile = next;
        ci = ni;
        cs = ns;
        offs(tile + tstep < tend ? tile + tstep : tile, ni, ns);
    }
}

// ------------------------------------------------------------------------------------------------
// Dense layer with conv1 and conv2 fused: the bottleneck of a spatial tile never leaves LDS.
// A workgroup of NW waves (two per SIMD) loops over TH x TW output tiles.  For a tile it computes the
// bottleneck of the (TH + 2) x (TW + 2) window around it (its in-image pixels, numbered row by row and
// packed 32 to an MFMA column block: wave w takes blocks w, w + NW, ...; the halo is recomputed by the
// neighbouring tiles), writes it to LDS as conv2 operands (u - 128, out-of-image pixels = zero
// padding), then runs the 3x3 conv from LDS (wave w: output pixel blocks w, w + NW, ..., all 36
// K-steps).  The K loop of conv1 runs over G rounded up to a multiple of 4 (padded steps multiply zero
// operands) so that the activation prefetch, 4 groups ahead, runs on into the next tile's first
// groups: they are in flight while the bottleneck epilogue and the 3x3 conv of this tile run.  Every
// global load of the steady state is an activation or weight load and the layer's small tables sit
// in LDS, so no wait drains the prefetch.  (No lambdas and no arrays selected at run time in the hot
// code: either puts locals in scratch memory, whose loads wait for every load in flight.)
// ------------------------------------------------------------------------------------------------
template <int TW, int TH, int CPW, int NW, bool WL>
struct DnShape {
    static constexpr int NT = 64 * NW;                              // threads
    static constexpr int BW = TW + 2, BH = TH + 2, WIN = BW * BH;    // bottleneck window
    static constexpr int NB2 = TW * TH / 32;                        // output pixel blocks
    static constexpr int PT = (NB2 + NW - 1) / NW;                  // per wave (the last may be short)
    static constexpr size_t BOT_BYTES = (size_t)WIN * 128;          // [4][WIN][2] 16-byte chunks
    static constexpr size_t PRM_BYTES = 128 * 4 + 128 * 8 + 32 * 4 + 32 * 4;
    static_assert(TW * TH % 32 == 0, "output tile = whole pixel blocks");
    static_assert(CPW == 1 || CPW == 2, "one or two conv1 column blocks per wave");
    // bottleneck window, tables, prologue table [G][32] dwords, (WL) conv1 weights [G][256] chunks
    static constexpr size_t lds(int G) { return BOT_BYTES + PRM_BYTES + (size_t)G * (WL ? 128 + 4096 : 128); }
};

// Tile geometry (uniform): image n, output origin (y0, x0), in-image window [ya, ya + npx / ww) x
// [xa, xa + ww).
struct DnGeo { int n, y0, x0, ya, xa, ww, npx; };

template <int TW, int TH>
DEV DnGeo dn_geo(int t, int tiles_x, int tiles_y, int H, int W) {
    DnGeo g;
    const int per = tiles_x * tiles_y;
    g.n = t / per;
    const int r = t - g.n * per;
    g.y0 = (r / tiles_x) * TH;
    g.x0 = (r % tiles_x) * TW;
    g.ya = g.y0 > 0 ? g.y0 - 1 : 0;
    g.xa = g.x0 > 0 ? g.x0 - 1 : 0;
    const int yb = g.y0 + TH + 1 < H ? g.y0 + TH + 1 : H;
    const int xb = g.x0 + TW + 1 < W ? g.x0 + TW + 1 : W;
    g.ww = xb - g.xa;
    g.npx = (yb - g.ya) * g.ww;
    return g;
}

// Byte offset in a store group of window pixel q (clamped to the window's last pixel), lane half h.
DEV uint32_t dn_pixel(const DnGeo& g, int q, int W, int h) {
    q = q < g.npx ? q : g.npx - 1;
    const int wy = q / g.ww, wx = q - wy * g.ww;
    return (uint32_t)((g.ya + wy) * W + g.xa + wx) * 32u + 16u * h;
}

template <int TW, int TH, int CPW, int NW, bool WL>
__global__ __launch_bounds__(64 * NW, 1) void k_dense(D8sDenseArgs a, int tiles_x, int tiles_y) {
    using S = DnShape<TW, TH, CPW, NW, WL>;
    constexpr int BW = S::BW, WIN = S::WIN, NT = S::NT, NB2 = S::NB2, PT = S::PT;
    __shared__ __attribute__((aligned(16))) u32x4 s_w[4 * 9 * 32 * 2];    // conv2 weights, 36 KB
    extern __shared__ __attribute__((aligned(16))) u32x4 s_dyn[];
    u32x4* s_b = s_dyn;                                                    // [4][WIN][2]
    int32_t* s_w1sum = (int32_t*)((uint8_t*)s_dyn + S::BOT_BYTES);        // [128]
    float2* s_gd = (float2*)(s_w1sum + 128);                              // [128]
    float* s_sc = (float*)(s_gd + 128);                                   // [32]
    int32_t* s_w2sum = (int32_t*)(s_sc + 32);                             // [32]
    uint32_t* s_abh = (uint32_t*)(s_w2sum + 32);                          // [G * 32]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int G = a.G, G0 = a.G0, H = a.H, W = a.W, N = a.N;
    u32x4* s_w1 = (u32x4*)(s_abh + G * 32);                               // [G * 256]
    const int64_t HW = (int64_t)H * W;
    const int total = N * tiles_x * tiles_y;
    int tile = blockIdx.x;
    if (tile >= total) return;

    // the weights and tables: the first items of each per thread requested at once (clamped
    // addresses), then stored; loops stage what is left (a load-and-store loop waits one L2 round
    // trip per iteration)
    {
        constexpr int NCH = (2304 + NT - 1) / NT, NW1 = WL ? 8 : 1, NAB = 2;
        u32x4 wv[NCH], v1[NW1];
        uint32_t vab[NAB];
        const u32x4* w2 = (const u32x4*)a.w2;
        const u32x4* w1 = (const u32x4*)a.w1;
        const uint32_t* abh32 = (const uint32_t*)a.abh;
        const int ti = min(tid, 127), ts = min(max(tid - 128, 0), 31);
        const int32_t t_w1sum = a.w1sum[ti], t_w2sum = a.w2sum[ts];
        const float2 t_gd = ((const float2*)a.gd)[ti];
        const float t_sc = a.sc[ts];
#pragma unroll
        for (int k = 0; k < NCH; ++k) wv[k] = w2[min(tid + NT * k, 2303)];
#pragma unroll
        for (int k = 0; k < NAB; ++k) vab[k] = abh32[min(tid + NT * k, G * 32 - 1)];
#pragma unroll
        for (int k = 0; WL && k < NW1; ++k) v1[k] = w1[min(tid + NT * k, G * 256 - 1)];
#pragma unroll
        for (int k = 0; k < NCH; ++k)
            if (tid + NT * k < 2304) s_w[swz((tid + NT * k) >> 1, tid & 1)] = wv[k];
        if (tid < 128) {
            s_w1sum[tid] = t_w1sum;
            s_gd[tid] = t_gd;
        } else if (tid < 160) {
            s_sc[tid - 128] = t_sc;
            s_w2sum[tid - 128] = t_w2sum;
        }
#pragma unroll
        for (int k = 0; k < NAB; ++k)
            if (tid + NT * k < G * 32) s_abh[tid + NT * k] = vab[k];
#pragma unroll
        for (int k = 0; WL && k < NW1; ++k)
            if (tid + NT * k < G * 256) s_w1[wperm(tid + NT * k)] = v1[k];
        for (int i = tid + NT * NAB; i < G * 32; i += NT) s_abh[i] = abh32[i];
        // the layer's conv1 weights (WL): every wave reads all of them for every tile
        for (int i = tid + NT * NW1; WL && i < G * 256; i += 4 * NT) {
            u32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = w1[min(i + u * NT, G * 256 - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i + u * NT < G * 256) s_w1[wperm(i + u * NT)] = v[u];
        }
    }

    const uint8_t* in0 = (const uint8_t*)a.in0;
    const uint8_t* seg = (const uint8_t*)a.seg;
    const int64_t in_img = (int64_t)G0 * HW * 32, grp = HW * 32, seg_slot = (int64_t)N * HW * 32;
    // this tile's and the next tile's geometry and the lane's pixel offsets (column blocks 0, 1)
    DnGeo cg = dn_geo<TW, TH>(tile, tiles_x, tiles_y, H, W);
    int next = tile + (int)gridDim.x;
    DnGeo ng = dn_geo<TW, TH>(next < total ? next : tile, tiles_x, tiles_y, H, W);
    uint32_t co0 = dn_pixel(cg, 32 * wave + j, W, h), co1 = 0;
    uint32_t no0 = dn_pixel(ng, 32 * wave + j, W, h), no1 = 0;
    if (CPW > 1) {
        co1 = dn_pixel(cg, 32 * (wave + NW) + j, W, h);
        no1 = dn_pixel(ng, 32 * (wave + NW) + j, W, h);
    }

    const int Gp = (G + 3) & ~3;                       // K steps per tile
    u32x4 ra[4][CPW];
    u32x4 rb[WL ? 1 : 2][4];
    // conv1 weights: output tile c, row 32 c + j, half h of group g in chunk g * 256 + 64 c + 2 j + h;
    // from LDS for the step itself (WL), else from global memory one step ahead (double-buffered)
    const u32x4* wl = (const u32x4*)a.w1 + j * 2 + h;
#define DN_LOAD_B(bslot, g)                                                                       \
    do {                                                                                          \
        const u32x4* p_ = (WL ? (const u32x4*)s_w1 + j + 32 * h : wl) + (int64_t)(g) * 256;       \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) rb[WL ? 0 : (bslot)][c_] = p_[64 * c_];  \
    } while (0)
    // activations of step t: t < Gp this tile's group t (repeats of G - 1 past it, unused), t >= Gp
    // the next tile's group t - Gp (clamped; this tile's again when there is none).  Unconditional:
    // the compiler can count the loads in flight instead of waiting for all of them.
#define DN_LOAD_A(slot, t)                                                                        \
    do {                                                                                          \
        const int t_ = (t);                                                                       \
        const bool cur_ = t_ < Gp;                                                                \
        int g_ = cur_ ? t_ : t_ - Gp;                                                             \
        g_ = g_ < G ? g_ : G - 1;                                                                 \
        const int n_ = cur_ ? cg.n : ng.n;                                                        \
        const uint8_t* b_ = g_ < G0 ? in0 + n_ * in_img + g_ * grp                                \
                                    : seg + (int64_t)(g_ - G0) * seg_slot + n_ * grp;             \
        ra[slot][0] = *(const u32x4*)(b_ + (cur_ ? co0 : no0));                                   \
        if (CPW > 1) ra[slot][CPW - 1] = *(const u32x4*)(b_ + (cur_ ? co1 : no1));                \
    } while (0)

    if (!WL) DN_LOAD_B(0, 0);
    DN_LOAD_A(0, 0);
    DN_LOAD_A(1, 1);
    DN_LOAD_A(2, 2);
    DN_LOAD_A(3, 3);
    __syncthreads();                                   // LDS tables and conv2 weights

    for (;;) {
        // ---- conv1 of the window: acc = 128 sum_k w + sum_k w (u - 128) ----
        i32x16 acc[CPW][4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            i32x16 init;
#pragma unroll
            for (int v = 0; v < 16; ++v) init[v] = 128 * s_w1sum[32 * c + res_row(v, h)];
#pragma unroll
            for (int i = 0; i < CPW; ++i) acc[i][c] = init;
        }
#define DN_STEP(slot, k)                                                                          \
    do {                                                                                          \
        const int k_ = (k);                                                                       \
        if (WL) {                                                                                 \
            DN_LOAD_B(0, k_ < G ? k_ : G - 1);                                                    \
        } else {                                                                                  \
            DN_LOAD_B(((slot) + 1) & 1, k_ + 1 < G ? k_ + 1 : (k_ + 1 < Gp ? G - 1 : 0));         \
            asm volatile("" ::: "memory");                                                        \
        }                                                                                         \
        u32x4 bx_[CPW];                                                                           \
        _Pragma("unroll") for (int i_ = 0; i_ < CPW; ++i_) bx_[i_] = u32x4{0, 0, 0, 0};           \
        if (k_ < G) {                                                                             \
            const u32x4* pp_ = (const u32x4*)(s_abh + k_ * 32 + h * 16);                          \
            const u32x4 p0_ = pp_[0], p1_ = pp_[1], p2_ = pp_[2], p3_ = pp_[3];                   \
            _Pragma("unroll") for (int i_ = 0; i_ < CPW; ++i_)                                    \
                bx_[i_] = pro16(ra[slot][i_], p0_, p1_, p2_, p3_);                                \
        }                                                                                         \
        DN_LOAD_A(slot, k_ + 4);                                                                  \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_)                                          \
            _Pragma("unroll") for (int i_ = 0; i_ < CPW; ++i_)                                    \
                acc[i_][c_] = mfma_i8(rb[WL ? 0 : (slot) & 1][c_], bx_[i_], acc[i_][c_]);          \
    } while (0)
        int k = 0;
        do {                                           // Gp >= 4: no path around the loop
            DN_STEP(0, k);
            DN_STEP(1, k + 1);
            DN_STEP(2, k + 2);
            DN_STEP(3, k + 3);
            k += 4;
        } while (k < Gp);
#undef DN_STEP

        // ---- bottleneck into LDS: v = low byte of fma(sat(fma(g, acc, d)), 255, 2^23), stored as
        // v ^ 0x80 (the conv2 operand); out-of-image window pixels get 0x80 (zero padding) ----
        const bool interior = cg.y0 >= 1 && cg.x0 >= 1 && cg.y0 + TH + 1 <= H && cg.x0 + TW + 1 <= W;
        if (!interior) {
            const u32x4 pad = {SIGN4, SIGN4, SIGN4, SIGN4};
            for (int idx = tid; idx < WIN * 8; idx += NT) {
                const int wp = idx >> 3, c = (idx >> 1) & 3, hh = idx & 1;
                const int wy = wp / BW, wx = wp - wy * BW;
                const int y = cg.y0 - 1 + wy, x = cg.x0 - 1 + wx;
                if ((unsigned)y >= (unsigned)H || (unsigned)x >= (unsigned)W)
                    s_b[c * WIN * 2 + swz(wp, hh)] = pad;
            }
        }
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            // the lane's window slot (-1 past the window's end)
            const int q = 32 * (wave + NW * i) + j;
            int dst = -1;
            if (q < cg.npx) {
                const int wy = q / cg.ww, wx = q - wy * cg.ww;
                dst = (cg.ya + wy - cg.y0 + 1) * BW + (cg.xa + wx - cg.x0 + 1);
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint32_t e[4];
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    uint32_t d = 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int v = 4 * kk + r;
                        const float2 prm = s_gd[32 * c + res_row(v, h)];
                        float y = __builtin_fmaf(prm.x, (float)acc[i][c][v], prm.y);
                        y = __builtin_fminf(__builtin_fmaxf(y, 0.0f), 1.0f);
                        // low byte of 2^23 + 128 + RNE(255 y): u ^ 0x80, the conv2 operand
                        const uint32_t b = __float_as_uint(__builtin_fmaf(y, 255.0f, 8388736.0f)) & 0xffu;
                        d |= b << (8 * r);
                    }
                    e[kk] = d;
                }
                const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
                if (dst >= 0) s_b[c * WIN * 2 + swz(dst, h)] = row;
                // one accumulator tile at a time: read all of them ahead and the registers run out
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();                               // the window's bottleneck is in LDS

        // ---- conv2 (3x3, pad 1) from LDS: wave w, output pixel blocks w + NW t (t < np: PT, or PT - 1
        // for the last waves when NW does not divide NB2) ----
        const int np = (NB2 - wave + NW - 1) / NW;
        if (np > 0) {
            i32x16 acc2[PT];
            int q0[PT];
#pragma unroll
            for (int t = 0; t < PT; ++t) {
                const int p = (wave + NW * t) * 32 + j;
                q0[t] = t < np ? (p / TW) * BW + (p % TW) : 0;
            }
            {
                i32x16 init2;
#pragma unroll
                for (int v = 0; v < 16; ++v) init2[v] = 128 * s_w2sum[res_row(v, h)];
#pragma unroll
                for (int t = 0; t < PT; ++t) acc2[t] = init2;
            }
            u32x4 aw[2], bq[2][PT];
#define DN_FETCH(s, sl)                                                                           \
    do {                                                                                          \
        const int c_ = (s) / 9, tap_ = (s) % 9;                                                   \
        const int o_ = (tap_ / 3) * BW + (tap_ % 3);                                              \
        aw[sl] = s_w[swz((c_ * 9 + tap_) * 32 + j, h)];                                           \
        _Pragma("unroll") for (int t_ = 0; t_ < PT; ++t_)                                         \
            bq[sl][t_] = s_b[c_ * WIN * 2 + swz(q0[t_] + o_, h)];                                 \
    } while (0)
            DN_FETCH(0, 0);
#pragma unroll
            for (int s = 0; s < 36; ++s) {
                if (s + 1 < 36) DN_FETCH(s + 1, (s + 1) & 1);
                acc2[0] = mfma_i8(aw[s & 1], bq[s & 1][0], acc2[0]);
#pragma unroll
                for (int t = 1; t < PT; ++t)
                    if (t < np) acc2[t] = mfma_i8(aw[s & 1], bq[s & 1][t], acc2[t]);
                __builtin_amdgcn_sched_barrier(0);     // operands one step ahead, no further
            }
#undef DN_FETCH
            // q = RNE(clamp(float(acc) * sc, -127, 127)) into the layer's store slot
#pragma unroll
            for (int t = 0; t < PT; ++t) {
                if (t >= np) break;
                uint32_t e[4];
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    uint32_t d = 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int v = 4 * kk + r;
                        const float q = __builtin_rintf(__builtin_fminf(
                            __builtin_fmaxf((float)acc2[t][v] * s_sc[res_row(v, h)], -127.0f), 127.0f));
                        d |= ((uint32_t)(int)q & 0xffu) << (8 * r);
                    }
                    e[kk] = d;
                }
                const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
                const int p = (wave + NW * t) * 32 + j;
                const int y = cg.y0 + p / TW, x = cg.x0 + p % TW;
                if (y < H && x < W)
                    *(u32x4*)(a.out + (((int64_t)cg.n * H + y) * W + x) * 32 + 16 * h) = row;
            }
        }

        if (next >= total) break;
        __syncthreads();                               // this tile's window is read: LDS free again
        tile = next;
        cg = ng;
        co0 = no0;
        co1 = no1;
        next = tile + (int)gridDim.x;
        ng = dn_geo<TW, TH>(next < total ? next : tile, tiles_x, tiles_y, H, W);
        no0 = dn_pixel(ng, 32 * wave + j, W, h);
        if (CPW > 1) no1 = dn_pixel(ng, 32 * (wave + NW) + j, W, h);
    }
#undef DN_LOAD_A
#undef DN_LOAD_B
}

// ------------------------------------------------------------------------------------------------
// Dense layer fused over a band of rows (W = 64 or 128): conv1 and conv2 of a layer, the bottleneck
// kept in a ring of rows in LDS.  A workgroup of 8 waves owns band_rows output rows of one image
// across the whole width and walks down them; each step, wave w (tile row rw = w / TPR, column
// block cb = w % TPR) computes conv1 of one 32-pixel tile of RS new bottleneck rows (all 128
// outputs, the store read from global memory 4 groups ahead, the prefetch running on into the next
// step), writes it to the ring (u ^ 0x80, the conv2 operand; rows outside the image: 0x80, the
// zero padding), then conv2 of one 32-pixel tile of RS output rows from the ring.  The first step
// of a band computes the two bottleneck rows above it; after that no pixel is computed twice.  The
// bytes equal those of d8s_conv1 + d8s_conv2 (the same integer sums and epilogues).
// Ring: SL = RS + 2 slots of [4 planes][PS pixels][2 halves], PS a multiple of 16 so a lane's
// swizzled column offset does not depend on the slot or plane; columns 0 and W + 1.. hold the
// padding.
// ------------------------------------------------------------------------------------------------
template <int W_>
struct BnShape {
    static constexpr int TPR = W_ / 32;                            // pixel tiles per row
    static constexpr int RS = 8 / TPR;                             // rows per step (8 waves)
    static constexpr int SL = RS + 2;                              // ring slots
    static constexpr int PS = (W_ + 2 + 15) / 16 * 16;             // ring row stride (pixels)
    static constexpr size_t RING = (size_t)SL * 4 * PS * 32;
    static constexpr size_t PRM = 128 * 4 + 128 * 8 + 32 * 4 + 32 * 4;
    static constexpr size_t lds(int G) { return RING + PRM + (size_t)G * (128 + 4096); }
    static_assert(W_ == 64 || W_ == 128, "band widths");
};

// conv1 row of step s of a band starting at y0 (step 0: the two rows above the band)
DEV int bn_row(int s, int y0, int rw, int RS) { return s == 0 ? y0 - 1 + rw : y0 + 1 + (s - 1) * RS + rw; }

// byte offset in a store group of pixel (ry clamped to the image, x), lane half h
DEV uint32_t bn_off(int ry, int H, int W, int x, int h) {
    ry = ry < 0 ? 0 : (ry >= H ? H - 1 : ry);
    return (uint32_t)((ry * W + x) * 32 + 16 * h);
}

// (LDS allows one workgroup, i.e. two waves per SIMD: the register budget is 256, and the scheduler
// is told so, or it sinks the prefetched LDS operands next to their MFMAs to save registers)
template <int W_, int GM>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_band(D8sDenseArgs a0, int bands, int band_rows, D8sDenseArgs a1, int split) {
    using S = BnShape<W_>;
    const PairSlot ps = pair_slot(split);
    const D8sDenseArgs a = ps.second ? a1 : a0;
    constexpr int TPR = S::TPR, RS = S::RS, SL = S::SL, PS = S::PS, NT = 512;
    __shared__ __attribute__((aligned(16))) u32x4 s_w[4 * 9 * 32 * 2];    // conv2 weights, 36 KB
    extern __shared__ __attribute__((aligned(16))) u32x4 s_dyn[];
    u32x4* s_r = s_dyn;                                                    // [SL][4][PS][2]
    int32_t* s_w1sum = (int32_t*)((uint8_t*)s_dyn + S::RING);             // [128]
    float2* s_gd = (float2*)(s_w1sum + 128);                              // [128]
    float* s_sc = (float*)(s_gd + 128);                                   // [32]
    int32_t* s_w2sum = (int32_t*)(s_sc + 32);                             // [32]
    uint32_t* s_abh = (uint32_t*)(s_w2sum + 32);                          // [G * 32]
    const int G = a.G, G0 = a.G0, H = a.H, N = a.N;
    u32x4* s_w1 = (u32x4*)(s_abh + G * 32);                               // [G * 256]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int rw = wave / TPR, cb = wave - rw * TPR;
    const int x = 32 * cb + j;
    const int n = ps.bid / bands, band = ps.bid - n * bands;
    const int y0 = band * band_rows, nr = min(band_rows, H - y0);
    const int M = (nr + RS - 1) / RS;                                     // conv2 steps
    const int64_t HW = (int64_t)H * W_;

    // the layer's weights and tables: every load first (clamped addresses, all in flight together),
    // then the stores (a load-and-store loop waits one L2 round trip per iteration)
    {
        constexpr int NCH = (2304 + NT - 1) / NT;
        constexpr int NW1 = (GM * 256 + NT - 1) / NT, NAB = (GM * 32 + NT - 1) / NT;
        u32x4 wv[NCH], v1[NW1];
        uint32_t vab[NAB];
        const u32x4* w2 = (const u32x4*)a.w2;
        const u32x4* w1 = (const u32x4*)a.w1;
        const uint32_t* abh32 = (const uint32_t*)a.abh;
        const int ti = min(tid, 127), ts = min(max(tid - 128, 0), 31);
        const int32_t t_w1sum = a.w1sum[ti], t_w2sum = a.w2sum[ts];
        const float2 t_gd = ((const float2*)a.gd)[ti];
        const float t_sc = a.sc[ts];
#pragma unroll
        for (int k = 0; k < NCH; ++k) wv[k] = w2[min(tid + NT * k, 2303)];
#pragma unroll
        for (int k = 0; k < NAB; ++k) vab[k] = abh32[min(tid + NT * k, G * 32 - 1)];
#pragma unroll
        for (int k = 0; k < NW1; ++k) v1[k] = w1[min(tid + NT * k, G * 256 - 1)];
#pragma unroll
        for (int k = 0; k < NCH; ++k)
            if (tid + NT * k < 2304) s_w[swz((tid + NT * k) >> 1, tid & 1)] = wv[k];
        if (tid < 128) {                               // the sums times 128: the accumulators' start
            s_w1sum[tid] = 128 * t_w1sum;
            s_gd[tid] = t_gd;
        } else if (tid < 160) {
            s_sc[tid - 128] = t_sc;
            s_w2sum[tid - 128] = 128 * t_w2sum;
        }
#pragma unroll
        for (int k = 0; k < NAB; ++k)
            if (tid + NT * k < G * 32) s_abh[tid + NT * k] = vab[k];
#pragma unroll
        for (int k = 0; k < NW1; ++k)
            if (tid + NT * k < G * 256) s_w1[wperm(tid + NT * k)] = v1[k];
    }
    {
        // padding columns of every ring row: 0 and W + 1 .. PS - 1
        constexpr int NPAD = PS - W_;
        const u32x4 pad = {SIGN4, SIGN4, SIGN4, SIGN4};
        for (int i = tid; i < SL * 4 * NPAD * 2; i += NT) {
            const int row = i / (NPAD * 2), rem = i - row * (NPAD * 2), p = rem >> 1, hh = rem & 1;
            const int xx = p == 0 ? 0 : W_ + p;
            s_r[row * PS * 2 + swz(xx, hh)] = pad;
        }
    }

    const uint8_t* in0n = (const uint8_t*)a.in0 + (int64_t)n * G0 * HW * 32;
    const uint8_t* segn = (const uint8_t*)a.seg + (int64_t)n * HW * 32;
    const int64_t grp = HW * 32, seg_slot = (int64_t)N * HW * 32;
    // ra: the step's G groups (GM >= G registers; past G, group G - 1 again, unused), each reloaded
    // with the next step's group right after its prologue
    u32x4 ra[GM], rb[4], pk[4];
    // conv2 operands read C2D steps ahead (fewer where the activation registers leave no room)
    constexpr int C2D = GM <= 10 ? 3 : 1;
#define BN_LOAD_B(g)                                                                              \
    do {                                                                                          \
        const u32x4* p_ = (const u32x4*)s_w1 + j + 32 * h + (g) * 256;                           \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) rb[c_] = p_[64 * c_];                    \
    } while (0)
    // group k (clamped to G - 1) at pixel offset o; unconditional, so the compiler counts the loads
    // in flight instead of draining them
#define BN_LOAD_A(k, o)                                                                           \
    do {                                                                                          \
        const int g_ = (k) < G ? (k) : G - 1;                                                     \
        const uint8_t* b_ = g_ < G0 ? in0n + g_ * grp : segn + (int64_t)(g_ - G0) * seg_slot;     \
        ra[k] = *(const u32x4*)(b_ + (o));                                                        \
    } while (0)
    // conv1 K step k of this step (a step past G multiplies a zero operand: no branch in the loop,
    // whose loads would then all be drained), the register reloaded with the next step's group
// (split in two: the LDS operands of a K step are read well before the step runs)
#define BN_K_FETCH(k)                                                                             \
    do {                                                                                          \
        const int kc_ = (k) < GM - 1 ? (k) : G - 1;      /* G is GM or GM - 1 */                  \
        BN_LOAD_B(kc_);                                                                           \
        const u32x4* pp_ = (const u32x4*)(s_abh + kc_ * 32 + h * 16);                             \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) pk[c_] = pp_[c_];                        \
    } while (0)
#define BN_K_RUN(k)                                                                               \
    do {                                                                                          \
        u32x4 bx_ = pro16(ra[k], pk[0], pk[1], pk[2], pk[3]);                                     \
        if ((k) == GM - 1) bx_ &= kmask;                  /* bitwise: keeps the code branch-free */ \
        BN_LOAD_A(k, no);                                                                         \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) acc[c_] = mfma_i8(rb[c_], bx_, acc[c_]); \
    } while (0)
#define BN_K(k)                                                                                   \
    do {                                                                                          \
        BN_K_FETCH(k);                                                                            \
        BN_K_RUN(k);                                                                              \
    } while (0)
#define BN_INIT1()                                                                                \
    _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_)                                              \
        _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) acc[c_][v_] = s_w1sum[32 * c_ + res_row(v_, h)]
    // conv1 results -> bottleneck bytes (u ^ 0x80; 0x80 for rows outside the image), before the
    // barrier; written to the ring after it
#define BN_EPI1_C(c)                                                                              \
    do {                                                                                          \
        const uint32_t pm_ = (unsigned)ry >= (unsigned)H ? ~0u : 0u;                              \
        uint32_t e_[4];                                                                           \
        _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_) {                                        \
            const float4* pg_ = (const float4*)(s_gd + 32 * (c) + 8 * q_ + 4 * h);                \
            e_[q_] = (epi1_x80(acc[c], q_, pg_[0], pg_[1]) & ~pm_) | (SIGN4 & pm_);               \
        }                                                                                         \
        brow[c] = xchg_rows(e_[0], e_[1], e_[2], e_[3], h);                                       \
    } while (0)
#define BN_EPI1()                                                                                 \
    do {                                                                                          \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) BN_EPI1_C(c_);                           \
    } while (0)
#define BN_RING_WRITE()                                                                           \
    do {                                                                                          \
        const int dst_ = (((ry + 1) % SL) * 4) * PS * 2 + swz(x + 1, h);                          \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) s_r[dst_ + c_ * PS * 2] = brow[c_];      \
    } while (0)
    // conv2 of output row yo: ring rows yo - 1 .. yo + 1; step st = (plane, tap).  Operand addresses
    // are per-lane pointers plus immediates (weights: swz(K * 32 + j, h) = 64 K + swz(j, h)); two
    // accumulators (even and odd steps) make two independent MFMA chains.
#define BN_C2_FETCH(st, sl)                                                                       \
    do {                                                                                          \
        const int c_ = (st) / 9, tap_ = (st) % 9, dy_ = tap_ / 3, dx_ = tap_ % 3;                 \
        const u32x4* pr_ = dy_ == 0 ? (dx_ == 0 ? p00 : dx_ == 1 ? p01 : p02)                     \
                         : dy_ == 1 ? (dx_ == 0 ? p10 : dx_ == 1 ? p11 : p12)                     \
                                    : (dx_ == 0 ? p20 : dx_ == 1 ? p21 : p22);                    \
        aw[sl] = pw2[64 * (c_ * 9 + tap_)];                                                       \
        bq[sl] = pr_[c_ * PS * 2];                                                                \
    } while (0)
#define BN_C2_SETUP(yo_)                                                                          \
    const int yo = (yo_);                                                                         \
    const u32x4* q0_ = s_r + ((yo + 0) % SL) * 4 * PS * 2;                                        \
    const u32x4* q1_ = s_r + ((yo + 1) % SL) * 4 * PS * 2;                                        \
    const u32x4* q2_ = s_r + ((yo + 2) % SL) * 4 * PS * 2;                                        \
    const u32x4 *p00 = q0_ + sx0, *p01 = q0_ + sx1, *p02 = q0_ + sx2;                             \
    const u32x4 *p10 = q1_ + sx0, *p11 = q1_ + sx1, *p12 = q1_ + sx2;                             \
    const u32x4 *p20 = q2_ + sx0, *p21 = q2_ + sx1, *p22 = q2_ + sx2;                             \
    i32x16 acc2, acc2b;                                                                           \
    _Pragma("unroll") for (int v_ = 0; v_ < 16; ++v_) {                                           \
        acc2[v_] = s_w2sum[res_row(v_, h)];                                                       \
        acc2b[v_] = 0;                                                                            \
    }                                                                                             \
    u32x4 aw[4], bq[4];                                /* operands C2D steps ahead */             \
    _Pragma("unroll") for (int f_ = 0; f_ < C2D; ++f_) BN_C2_FETCH(f_, f_)
#define BN_C2_STEP(st)                                                                            \
    do {                                                                                          \
        if ((st) + C2D < 36) BN_C2_FETCH((st) + C2D, ((st) + C2D) & 3);                           \
        __builtin_amdgcn_sched_barrier(0);             /* the reads stay C2D steps ahead */       \
        if (((st) & 1) == 0) acc2 = mfma_i8(aw[(st) & 3], bq[(st) & 3], acc2);                    \
        else acc2b = mfma_i8(aw[(st) & 3], bq[(st) & 3], acc2b);                                  \
    } while (0)
#define BN_C2_STORE()                                                                             \
    do {                                                                                          \
        acc2 += acc2b;                                                                            \
        uint32_t e_[4];                                                                           \
        _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_)                                          \
            e_[q_] = epi2_q(acc2, q_, *(const float4*)(s_sc + 8 * q_ + 4 * h));                   \
        const u32x4 row_ = xchg_rows(e_[0], e_[1], e_[2], e_[3], h);                              \
        if (yo < y0 + nr) *(u32x4*)(a.out + (((int64_t)n * H + yo) * W_ + x) * 32 + 16 * h) = row_; \
    } while (0)

    if (G < GM - 1 || G > GM) __builtin_unreachable();
    const uint32_t km = G == GM ? ~0u : 0u;            // K step GM - 1: real, or a zero operand
    const u32x4 kmask = {km, km, km, km};
    int ry = bn_row(0, y0, rw, RS);
    uint32_t no = bn_off(bn_row(1, y0, rw, RS), H, W_, x, h);
    {
        const uint32_t co = bn_off(ry, H, W_, x, h);
#pragma unroll
        for (int k = 0; k < GM; ++k) BN_LOAD_A(k, co);
    }
    // conv2: the lane's swizzled offsets of ring columns x + dx (dx = 0, 1, 2), its weight rows
    const int sx0 = swz(x, h), sx1 = swz(x + 1, h), sx2 = swz(x + 2, h);
    const u32x4* pw2 = s_w + swz(j, h);
    i32x16 acc[4];
    u32x4 brow[4];
    __syncthreads();                                   // tables, weights, padding

    // steps 0 and 1: conv1 only (step 0: the two rows above the band, waves of tile rows 0-1)
    for (int s = 0; s < 2; ++s) {
        BN_INIT1();
#pragma unroll
        for (int k = 0; k < GM; ++k) BN_K(k);
        BN_EPI1();
        __syncthreads();
        if (s > 0 || rw < 2) BN_RING_WRITE();
        __syncthreads();
        ry = bn_row(s + 1, y0, rw, RS);
        no = bn_off(bn_row(s + 2, y0, rw, RS), H, W_, x, h);
    }
    // steps 2 .. M: conv1 of step s with conv2 of step s - 2 (rows of conv1 steps s - 2 and s - 1)
    // interleaved: the prologue's VALU work and the 3x3's LDS reads next to each other's MFMAs
    for (int s = 2; s <= M; ++s) {
        BN_INIT1();
        {
            BN_C2_SETUP(y0 + (s - 2) * RS + rw);
            // conv1's K steps beside the first 18 conv2 steps, its epilogue (one output tile every 4
            // steps) beside the last 16: the VALU work of both next to conv2's MFMAs
            BN_K_FETCH(0);
#pragma unroll
            for (int st = 0; st < 36; ++st) {
                BN_C2_STEP(st);
#pragma unroll
                for (int k = 0; k < GM; ++k)
                    if (st == (18 * (k + 1)) / GM - 1) {
                        BN_K_RUN(k);
                        if (k + 1 < GM) BN_K_FETCH(k + 1);
                        __builtin_amdgcn_sched_barrier(0);     // read a K step ahead
                    }
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (st == 20 + 4 * c) {
                        BN_EPI1_C(c);
                        __builtin_amdgcn_sched_barrier(0);
                    }
            }
            BN_C2_STORE();
        }
        __syncthreads();                               // the ring rows of step s - 2 are read
        BN_RING_WRITE();
        __syncthreads();
        ry = bn_row(s + 1, y0, rw, RS);
        no = bn_off(bn_row(s + 2, y0, rw, RS), H, W_, x, h);
    }
    // conv2 of step M - 1
    {
        BN_C2_SETUP(y0 + (M - 1) * RS + rw);
#pragma unroll
        for (int st = 0; st < 36; ++st) BN_C2_STEP(st);
        BN_C2_STORE();
    }
#undef BN_C2_STORE
#undef BN_C2_STEP
#undef BN_C2_SETUP
#undef BN_C2_FETCH
#undef BN_RING_WRITE
#undef BN_EPI1
#undef BN_EPI1_C
#undef BN_INIT1
#undef BN_K
#undef BN_K_RUN
#undef BN_K_FETCH
#undef BN_LOAD_A
#undef BN_LOAD_B
}

// Raw buffer loads: a uniform base and size (a buffer resource in scalar registers), a 32-bit lane
// offset and a uniform scalar offset; bytes past the size read as zero.
DEV __amdgpu_buffer_rsrc_t brsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
DEV uint32_t bload32(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, 0);
}
DEV u32x4 bload128(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0));
}

// Loads through pointers read from memory (the layer tables): the compiler cannot tell their address
// space and would use flat loads, which also count as LDS operations, so every wait for an LDS read
// would wait for them too.  These say "global".
typedef __attribute__((address_space(1))) const u32x4 gu32x4;
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const int32_t gi32;
typedef __attribute__((address_space(1))) const u32x2 gu32x2;
DEV u32x4 ldg_u32x4(const void* p) { return *(gu32x4*)p; }
DEV uint32_t ldg_u32(const void* p) { return *(gu32*)p; }
DEV int32_t ldg_i32(const void* p) { return *(gi32*)p; }
DEV float2 ldg_f2(const void* p) {
    const u32x2 v = *(gu32x2*)p;
    return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
}
DEV float ldg_f(const void* p) { return __uint_as_float(*(gu32*)p); }

// ------------------------------------------------------------------------------------------------
// A whole dense block per image (small maps, H W <= 256): one workgroup of 8 waves per image runs every
// layer of the block: conv1 of the image's 256 pixels (wave w: pixels 32 w .. 32 w + 31, all 128
// outputs, the image's store read from global memory, where it stays in L2), the bottleneck into LDS
// (with a zero-padding ring), conv2 from LDS into the layer's store slot, a barrier, the next layer.
// No per-layer launches and no bottleneck in memory; the layers of one image depend only on that
// image, so workgroups never wait for each other.  The layer tables come from a device array of
// D8sLayerP.  Per layer the first activation groups (the block input, unchanged by the layers) and
// weights are requested before the layer's tables are staged.
// ------------------------------------------------------------------------------------------------
static constexpr int DB_NT = 512;                          // 8 waves: 8 x 32 pixels

DEV const uint8_t* db_sel(bool c, const uint8_t* a, const uint8_t* b) {
    const uint64_t ua = (uint64_t)a, ub = (uint64_t)b, m = c ? ~0ull : 0ull;
    return (const uint8_t*)((ua & m) | (ub & ~m));
}
static constexpr size_t DB_PRM = 128 * 4 + 128 * 8 + 32 * 4 + 32 * 4;

static size_t dblock_lds(int H, int W, int Gmax) {
    return (size_t)(H + 2) * (W + 2) * 128 + DB_PRM + (size_t)Gmax * 128 + 2 * 8 * 4096;
}

__global__ __launch_bounds__(DB_NT, 1) void k_dblock(D8sBlockArgs a0, D8sBlockArgs a1, int split) {
    const PairSlot ps = pair_slot(split);
    const D8sBlockArgs a = ps.second ? a1 : a0;
    __shared__ __attribute__((aligned(16))) u32x4 s_w[2304];              // conv2 weights, 36 KB
    extern __shared__ __attribute__((aligned(16))) u32x4 s_dyn[];
    const int H = a.H, W = a.W, HW = H * W, BW = W + 2, WIN = (H + 2) * (W + 2);
    const int G0 = a.G0, L = a.L, N = a.N;
    u32x4* s_b = s_dyn;                                                    // [4][WIN][2]
    int32_t* s_w1sum = (int32_t*)(s_dyn + 8 * WIN);                       // [128]
    float2* s_gd = (float2*)(s_w1sum + 128);                              // [128]
    float* s_sc = (float*)(s_gd + 128);                                   // [32]
    int32_t* s_w2sum = (int32_t*)(s_sc + 32);                             // [32]
    uint32_t* s_abh = (uint32_t*)(s_w2sum + 32);                          // [Gmax * 32]
    u32x4* s_wc = (u32x4*)(s_abh + (G0 + L - 1) * 32);                   // [2][8 * 256] weight chunks

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int n = ps.bid;

    // the layers' descriptors in LDS (L <= 64: the launch checks G0 + L - 1 <= 64), so that a layer's
    // table and weight pointers are an LDS read away, not a global load whose pending count the
    // conv1 loop's first wait would have to include
    __shared__ uint64_t s_lp[64 * 7];
    static_assert(sizeof(D8sLayerP) == 7 * sizeof(uint64_t), "descriptor layout");
    for (int q = tid; q < min(L, 64) * 7; q += DB_NT) s_lp[q] = ((const uint64_t*)a.layers)[q];
#define DB_LP(l_) (*(const D8sLayerP*)(s_lp + 7 * (l_)))
    // zero-padding ring of the window (the layers write only its interior)
    {
        const u32x4 pad = {SIGN4, SIGN4, SIGN4, SIGN4};
        for (int idx = tid; idx < WIN * 8; idx += DB_NT) {
            const int wp = idx >> 3, c = (idx >> 1) & 3, hh = idx & 1;
            const int wy = wp / BW, wx = wp - wy * BW;
            if (wy == 0 || wy == H + 1 || wx == 0 || wx == W + 1) s_b[c * WIN * 2 + swz(wp, hh)] = pad;
        }
    }
    // the lane's pixel (a repeat of the last one past the image)
    const int p = 32 * wave + j;
    const bool live = p < HW;
    const int pc = live ? p : HW - 1;
    const int py = pc / W, px = pc - py * W;
    const uint32_t off = (uint32_t)pc * 32u + 16u * h;
    const int dst = (py + 1) * BW + px + 1;
    const int q0 = py * BW + px;                          // the 3 x 3 window's corner
    const uint8_t* in0 = (const uint8_t*)a.in0 + (int64_t)n * G0 * HW * 32;
    const uint8_t* segn = (const uint8_t*)a.seg + (int64_t)n * HW * 32;
    const int64_t slot = (int64_t)N * HW * 32;
    // group g's byte at the lane's pixel: a uniform base (scalar registers) plus the lane's 32-bit offset
// (both candidate bases computed and one selected: a branch here would make the loop's waits wait for
// every load in flight)
#define DB_SRC(g) (db_sel((g) < G0, in0 + (int64_t)min((g), G0 - 1) * HW * 32, \
                          segn + (int64_t)max((g) - G0, 0) * slot) + offl)

    // A layer's tables, its first conv1 weight chunk and its first 4 activation groups are requested
    // during the previous layer's conv2 (layer 0: before the loop) and stored to LDS after that
    // layer's last barrier.  (Activation groups of the previous layer's own output are requested
    // after the barrier: when G0 + l < 4.)
    u32x4 wv[5], stg[4], ra[4];                          // conv2 weights, chunk, activations 4 ahead
    int32_t t_w1sum = 0, t_w2sum = 0;
    float2 t_gd = {0.f, 0.f};
    float t_sc = 0.f;
    uint32_t t_abh[4];
#define DB_TABLES(lp_, G_)                                                                        \
    do {                                                                                          \
        int t_ = tid;                                    /* recomputed indices, not kept live */  \
        asm volatile("" : "+v"(t_));                                                              \
        _Pragma("unroll") for (int k_ = 0; k_ < 5; ++k_)                                          \
            wv[k_] = ldg_u32x4((const u32x4*)(lp_).w2 + min(t_ + DB_NT * k_, 2303));             \
        const int ti_ = min(t_, 127), ts_ = min(max(t_ - 128, 0), 31);                             \
        t_w1sum = ldg_i32((lp_).w1sum + ti_);                                                     \
        t_gd = ldg_f2((const float2*)(lp_).gd + ti_);                                             \
        t_sc = ldg_f((lp_).sc + ts_);                                                             \
        t_w2sum = ldg_i32((lp_).w2sum + ts_);                                                     \
        _Pragma("unroll") for (int k_ = 0; k_ < 4; ++k_)                                          \
            t_abh[k_] = ldg_u32((const uint32_t*)(lp_).abh + min(t_ + DB_NT * k_, (G_) * 32 - 1)); \
        const u32x4* w1_ = (const u32x4*)(lp_).w1;                                                \
        _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_)                                          \
            stg[u_] = ldg_u32x4(w1_ + min(t_ + DB_NT * u_, (G_) * 256 - 1));                      \
    } while (0)
#define DB_RA(G_)                                                                                 \
    _Pragma("unroll") for (int s_ = 0; s_ < 4; ++s_)                                              \
        ra[s_] = *(const u32x4*)DB_SRC(s_ < (G_) - 1 ? s_ : (G_) - 1)
    uint32_t offl = off;                                 // (opaque per layer: no address hoisted out
    {                                                    // of the layer loop to live in registers)
        __syncthreads();                                 // the descriptors
        const D8sLayerP lp0 = DB_LP(0);
        DB_TABLES(lp0, G0);
        DB_RA(G0);
    }
    bool ra_ready = true;

    for (int l = 0; l < L; ++l) {
        asm volatile("" : "+v"(offl));
        const D8sLayerP lp = DB_LP(l);
        const int G = G0 + l;
        const int nk = G;
        if (!ra_ready) {                                 // groups of the layer before: now complete
            DB_RA(G);
        }
#pragma unroll
        for (int k = 0; k < 5; ++k)
            if (tid + DB_NT * k < 2304) s_w[swz((tid + DB_NT * k) >> 1, tid & 1)] = wv[k];
        if (tid < 128) {
            s_w1sum[tid] = t_w1sum;
            s_gd[tid] = t_gd;
        } else if (tid < 160) {
            s_sc[tid - 128] = t_sc;
            s_w2sum[tid - 128] = t_w2sum;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (tid + DB_NT * k < G * 32) s_abh[tid + DB_NT * k] = t_abh[k];

        // conv1 weights go through LDS in chunks of 8 groups (32 KB, double-buffered): every wave
        // reads all of them, and from L2 one step ahead they would stall every step
        const u32x4* w1 = (const u32x4*)lp.w1;
        const int nch = (G + 7) / 8;
#define DB_STAGE_LOAD(c)                                                                          \
    _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_)                                              \
        stg[u_] = ldg_u32x4(w1 + min((c) * 2048 + tid + DB_NT * u_, G * 256 - 1))
#define DB_STAGE_STORE(c)                                                                         \
    _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) s_wc[((c) & 1) * 2048 + wperm(tid + DB_NT * u_)] = stg[u_]
        const int klast = nk - 1;
        DB_STAGE_STORE(0);
        __syncthreads();                                 // this layer's tables, weight chunk 0

        // ---- conv1 of the image: acc = 128 sum_k w + sum_k w (u - 128) ----
        i32x16 acc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[c][v] = 128 * s_w1sum[32 * c + res_row(v, h)];
        }
        // step k (group k, the (k % 8)-th of chunk k / 8 in buffer (k / 8) & 1)
    // a step's prologue tables were read from LDS by the step before (so the prologue starts at once),
    // its weights at its start (needed only by the MFMAs, after the prologue)
#define DB_PQ(dst, k)                                                                             \
    do {                                                                                          \
        const u32x4* pn_ = (const u32x4*)(s_abh + (k) * 32 + h * 16);                             \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) dst[c_] = pn_[c_];                       \
    } while (0)
#define DB_STEP(slot, k)                                                                          \
    do {                                                                                          \
        const int k_ = (k);                                                                       \
        const u32x4* wq_ = s_wc + ((k_ >> 3) & 1) * 2048 + (k_ & 7) * 256 + j + 32 * h;           \
        u32x4 rb_[4];                                                                             \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) rb_[c_] = wq_[64 * c_];                  \
        DB_PQ(pq[((slot) + 1) & 1], min(k_ + 1, klast));                                          \
        const u32x4* pp_ = pq[(slot) & 1];                                                        \
        const u32x4 bx_ = pro16(ra[(slot) & 3], pp_[0], pp_[1], pp_[2], pp_[3]);                  \
        ra[(slot) & 3] = *(const u32x4*)DB_SRC(k_ + 4 < klast ? k_ + 4 : klast);                  \
        _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) acc[c_] = mfma_i8(rb_[c_], bx_, acc[c_]); \
    } while (0)
        u32x4 pq[2][4];
        DB_PQ(pq[0], 0);
        // the whole chunks without a branch, so every wait counts exactly the loads before it (a step
        // under a branch makes the next wait wait for every load in flight); the next chunk's weights
        // staged unconditionally (past the last chunk: a clamped read into the idle buffer); then the
        // last, partial chunk step by step
        const int nfull = nk >> 3;
        for (int ch = 0; ch < nfull; ++ch) {
            const int k0 = ch * 8;
            DB_STAGE_LOAD(ch + 1);
            DB_STEP(0, k0);
            DB_STEP(1, k0 + 1);
            DB_STEP(2, k0 + 2);
            DB_STEP(3, k0 + 3);
            DB_STEP(4, k0 + 4);
            DB_STEP(5, k0 + 5);
            DB_STEP(6, k0 + 6);
            DB_STEP(7, k0 + 7);
            DB_STAGE_STORE(ch + 1);                      // its buffer was last read in chunk ch - 1
            __syncthreads();
        }
        if (nfull < nch) {
            const int k0 = nfull * 8;
            DB_STEP(0, k0);
            if (k0 + 1 < nk) DB_STEP(1, k0 + 1);
            if (k0 + 2 < nk) DB_STEP(2, k0 + 2);
            if (k0 + 3 < nk) DB_STEP(3, k0 + 3);
            if (k0 + 4 < nk) DB_STEP(4, k0 + 4);
            if (k0 + 5 < nk) DB_STEP(5, k0 + 5);
            if (k0 + 6 < nk) DB_STEP(6, k0 + 6);
        }
#undef DB_STEP
#undef DB_PQ
#undef DB_STAGE_STORE
#undef DB_STAGE_LOAD

        // ---- bottleneck into LDS (v ^ 0x80, the conv2 operand) ----
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint32_t e[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const float4* pg = (const float4*)(s_gd + 32 * c + 8 * kk + 4 * h);
                e[kk] = epi1_x80(acc[c], kk, pg[0], pg[1]);
            }
            const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
            if (live) s_b[c * WIN * 2 + swz(dst, h)] = row;
            __builtin_amdgcn_sched_barrier(0);           // one accumulator tile at a time
        }
        __syncthreads();                                 // the image's bottleneck is in LDS

        // the next layer's tables and chunk 0 (its first activation groups after the 3x3's MFMAs)
        if (l + 1 < L) {
            const D8sLayerP ln = DB_LP(l + 1);
            DB_TABLES(ln, G + 1);
        }

        // ---- conv2 (3x3, pad 1) from LDS into store slot l ----
        {
            i32x16 acc2;
#pragma unroll
            for (int v = 0; v < 16; ++v) acc2[v] = 128 * s_w2sum[res_row(v, h)];
            // operands read C2D steps ahead (an LDS read takes longer than one MFMA step)
            constexpr int C2D = 3;
            u32x4 aw[4], bq[4];
#define DB_FETCH(s, sl)                                                                           \
    do {                                                                                          \
        const int c_ = (s) / 9, tap_ = (s) % 9;                                                   \
        aw[sl] = s_w[swz((c_ * 9 + tap_) * 32 + j, h)];                                           \
        bq[sl] = s_b[c_ * WIN * 2 + swz(q0 + (tap_ / 3) * BW + (tap_ % 3), h)];                   \
    } while (0)
#pragma unroll
            for (int f = 0; f < C2D; ++f) DB_FETCH(f, f);
#pragma unroll
            for (int s = 0; s < 36; ++s) {
                if (s + C2D < 36) DB_FETCH(s + C2D, (s + C2D) & 3);
                acc2 = mfma_i8(aw[s & 3], bq[s & 3], acc2);
                __builtin_amdgcn_sched_barrier(0);
            }
#undef DB_FETCH
            ra_ready = l + 1 < L && G0 + l >= 4;         // the next layer's groups 0..3 exist already
            if (ra_ready) {
                DB_RA(G + 1);
            }
            uint32_t e[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) e[kk] = epi2_q(acc2, kk, *(const float4*)(s_sc + 8 * kk + 4 * h));
            const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
            if (live) *(u32x4*)((uint8_t*)segn + (int64_t)l * slot + off) = row;
        }
        // slot l is complete (every wave's stores retired) before any wave's next conv1 reads it,
        // and LDS is free for the next layer's tables
        __syncthreads();
    }
#undef DB_RA
#undef DB_TABLES
#undef DB_LP
#undef DB_SRC
}

// ------------------------------------------------------------------------------------------------
// A whole dense block with every image split into row bands ("parts"): K = parts bands of R = H / K
// rows (P = R W pixels, PT = P / 32 pixel tiles), one workgroup of 8 waves per (image, band), every
// layer in one launch.  For batches too small to fill the chip with one workgroup per image: the
// configuration-4 study (24 images) runs its 32 x 32 and 16 x 16 blocks on ~200 CUs instead of 24 or
// 88 latency-bound launches.  Per layer:
//   prologue  the groups' store bytes of the band's pixels go through the fp16 prologue once, chunk by
//          chunk (CG groups x PT pixel tiles, one 1 KB MFMA operand each), into a double-buffered LDS
//          chunk shared by all waves: the next chunk's prologue is computed beside the current chunk's
//          MFMAs, one barrier per chunk;
//   conv1  wave w computes output tile c = w % 4 (32 of the 128 bottleneck channels) for its pixel
//          tiles (the band's half w / 4 of them; for a 32-pixel band, half of the groups, the two
//          halves added through LDS): it reads only its tile's weights, streamed from L2 four groups
//          ahead in registers;
//   bottleneck  the bytes of the band's rows into an LDS window of R + 2 rows (zero padding around);
//          the band's first and last rows also go to `xchg` as (4-byte value, 4-byte tag) pairs, one
//          64-bit store each, the tag naming the launch and the layer; the neighbours' rows come back
//          into the window's halo rows by polling those pairs until every tag is current;
//   conv2  split over the waves of a pixel tile by K step (36 = 4 planes x 9 taps), added through LDS,
//          stored into the layer's slot.
// conv1 is pixel-local: a band's next layer reads only its own pixels, so the halo rows are the only
// data that crosses workgroups, and only conv2 waits for them.  A layer's conv1 over every group but
// the newest (the previous layer's conv2 output) runs before that conv2, while the previous layer's
// rows are on their way between the bands: pass i is conv1 of layer i over its older groups, then the
// neighbours' rows of layer i - 1 and its conv2, whose output bytes (the newest group of layer i, this
// band's own pixels) go through layer i's prologue straight into LDS, then that group's MFMAs and
// layer i's epilogue and rows out.  The exchange pairs are written and read with relaxed agent-scope
// atomics (performed at the device's coherence point, visible across the XCDs' L2s); a 64-bit pair is
// written in one access, so a current tag comes with its value.  A band sends layer i's rows only
// after it has read its neighbours' rows of layer i - 1, which they sent after reading its rows of
// layer i - 2: two buffers (by layer parity) are never overwritten before they are read.  Workgroups
// take their (image, band) from a ticket counter in the order they start, so a band only ever waits
// for bands whose tickets are adjacent to its own, taken by workgroups already running or next to
// start: the waits cannot form a cycle whatever the dispatch order, and every wait is bounded (a wait
// that runs out counts in sync[2] and the kernel carries on, so every workgroup reaches its end).  The
// last workgroup to end resets the ticket and the end count and advances the launch count (sync[3])
// the tags are made of, so the next launch needs no clearing.  Tables, weights and the next pass's
// first chunk of store bytes are requested a phase ahead of their use.
// ------------------------------------------------------------------------------------------------
static constexpr int DP_NT = 512;
static constexpr int DP_SPIN = 1 << 20;                   // polls before a wait gives up

DEV uint64_t ld_agent64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV void st_agent64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV void st_agent(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Shape constants of k_dparts<PT>, shared by the kernel's static LDS arrays and the host's LDS check.
template <int PT>
struct DpShape {
    static_assert(PT == 1 || PT == 2 || PT == 4 || PT == 8, "pixel tiles per band");
    // groups per prologue chunk: 4 for 128- and 256-pixel bands (for 128: a 24-image study's 32 x 32
    // block 0.76-0.77 against 0.79-0.82 ms with 8, 0.78-0.80 with 2), 8 for the narrower ones (a
    // 32-pixel band needs 8 for one operand per wave; 16 was slower)
    static constexpr int CG = PT == 4 || PT == 8 ? 4 : 8;
    static constexpr int ITEMS = CG * PT;                  // (group, pixel tile) operands per chunk
    static constexpr int S2 = PT == 8 ? 1 : (PT == 4 ? 2 : 4);   // conv2 K slices per pixel tile
    static constexpr int NRED = PT == 1 ? 4 * 1024 : ((S2 - 1) * PT * 1024 > 0 ? (S2 - 1) * PT * 1024 : 1);
    static constexpr int NLP = 64 * 7;                     // layer descriptors (at most 64 layers)
    // static LDS bytes: conv2 weights, two prologue chunks, partial sums, the ticket words and the
    // descriptors (the arrays of k_dparts, in that order), plus 64 bytes for their alignment
    static constexpr size_t STATIC = 2304 * 16 + 2 * ITEMS * 64 * 16 + NRED * 4 + 2 * 4 + NLP * 8 + 64;
};

template <int PT>
__global__ __launch_bounds__(DP_NT, 1) void k_dparts(D8sPartsArgs a) {
    using SH = DpShape<PT>;
    constexpr int CG = SH::CG;
    constexpr int ITEMS = SH::ITEMS;                       // (group, pixel tile) operands per chunk
    constexpr int IPW = ITEMS / 8;                         // of them per wave
    constexpr int NPT = PT == 1 ? 1 : PT / 2;              // conv1 pixel tiles per wave
    constexpr int KH = PT == 1 ? 2 : 1;                    // conv1 K halves (32-pixel bands)
    constexpr int QC = CG / KH;                            // a wave's groups per chunk
    constexpr int DW = 4;                                  // weight groups in flight per wave
    constexpr int S2 = SH::S2;                             // conv2 K slices per pixel tile
    constexpr int NRED = SH::NRED;
    static_assert(QC % DW == 0 && IPW >= 1, "chunk shape");
    __shared__ __attribute__((aligned(16))) u32x4 s_w[2304];              // conv2 weights, 36 KB
    __shared__ __attribute__((aligned(16))) u32x4 s_pro[2 * ITEMS * 64];  // prologue chunks
    __shared__ __attribute__((aligned(16))) int32_t s_red[NRED];          // partial sums
    __shared__ uint32_t s_tk[2];
    // the layers' descriptors (L <= 64: the launch checks G0 + L - 1 <= 64), so that a layer's table
    // and weight pointers are an LDS read away, not a global load the table loads depend on
    __shared__ uint64_t s_lp[SH::NLP];
    static_assert(sizeof(D8sLayerP) == 7 * sizeof(uint64_t), "descriptor layout");
    extern __shared__ __attribute__((aligned(16))) u32x4 s_dyn[];
    const int H = a.H, W = a.W, HW = H * W, K = a.parts, R = H / K, BW = W + 2, WIN = (R + 2) * BW;
    const int G0 = a.G0, L = a.L, N = a.N;
    u32x4* s_b = s_dyn;                                                    // [4][WIN][2]
    int32_t* s_w1sum = (int32_t*)(s_dyn + 8 * WIN);                       // [128]
    float2* s_gd = (float2*)(s_w1sum + 128);                              // [128]
    float* s_sc = (float*)(s_gd + 128);                                   // [32]
    int32_t* s_w2sum = (int32_t*)(s_sc + 32);                             // [32]
    uint32_t* s_abh = (uint32_t*)(s_w2sum + 32);                          // [Gmax * 32]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    const int c = wave & 3, hv = wave >> 2;                // conv1: output tile, half
    uint32_t* sync = a.sync;
    const int nparts = N * K;

    if (tid == 0) {
        s_tk[0] = __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_tk[1] = ld_agent(sync + 3);                      // the launch count, stable during a launch
    }
    for (int q = tid; q < min(a.L, 64) * 7; q += DP_NT) s_lp[q] = ((const uint64_t*)a.layers)[q];
    __syncthreads();
#define DP_LP(l_) (*(const D8sLayerP*)(s_lp + 7 * (l_)))
    // a ticket past the last band means the sync words were not zero at the launch: nothing to do
    // but count it (the bands left without a workgroup make their neighbours' waits run out)
    const bool valid = (int)s_tk[0] < nparts;
    const int ticket = valid ? (int)s_tk[0] : 0;
    const uint32_t epoch = s_tk[1];
    const int n = ticket / K, part = ticket - n * K;
    if (!valid && tid == 0) atomicAdd(sync + 2, 1u);
    {
        const u32x4 pad = {SIGN4, SIGN4, SIGN4, SIGN4};
        for (int idx = tid; idx < WIN * 8; idx += DP_NT) {
            const int wp = idx >> 3, cc = (idx >> 1) & 3, hh = idx & 1;
            const int wy = wp / BW, wx = wp - wy * BW;
            if ((wy == 0 && part == 0) || (wy == R + 1 && part == K - 1) || wx == 0 || wx == W + 1)
                s_b[cc * WIN * 2 + swz(wp, hh)] = pad;
        }
    }
    const int bandp = part * R * W;                        // the band's first pixel in the image
    const uint8_t* img0 = (const uint8_t*)a.in0 + (int64_t)n * G0 * HW * 32;
    uint8_t* segn = (uint8_t*)a.seg + (int64_t)n * HW * 32;
    const int64_t slot = (int64_t)N * HW * 32;
    uint64_t* xpair = (uint64_t*)a.xchg;                  // [nparts][parity][top, bottom][4][W][8]
    bool broken = false;                                   // a wait ran out: skip the later ones
    // store bytes of group g at band pixel 32 t + j (a uniform base plus the lane's 32-bit offset)
#define DP_SRC(g, t) (((g) < G0 ? img0 + (int64_t)(g) * HW * 32 : segn + (int64_t)((g) - G0) * slot) + \
                      (uint32_t)((bandp + 32 * (t) + j) * 32 + 16 * h))
#define DP_XP(tk, par, which, cc) (xpair + ((((int64_t)(tk) * 2 + (par)) * 2 + (which)) * 4 + (cc)) * W * 8)
    // a wave's conv1 groups: q -> g = q (PT >= 2) or 2 q + hv (32-pixel bands)
#define DP_G(q) (KH == 1 ? (q) : 2 * (q) + hv)

    // prefetched state: conv1 tables of the next conv1 pass (t_abh, t_w1sum, t_gd), conv2 tables of the
    // next conv2 (t_w2, t_sc, t_w2sum), the weights of a layer's newest group (t_wn)
    u32x4 t_w2[5];
    uint32_t t_abh[4];
    int32_t t_w1sum = 0, t_w2sum = 0;
    float2 t_gd = {0.f, 0.f};
    float t_sc = 0.f;
    u32x4 t_wn = {0u, 0u, 0u, 0u};
    u32x4 rw[DW], ra[IPW];
#define DP_TAB1(lp_, G_)                                                                          \
    do {                                                                                          \
        const int ti_ = min(tid, 127);                                                            \
        t_w1sum = ldg_i32((lp_).w1sum + ti_);                                                     \
        t_gd = ldg_f2((const float2*)(lp_).gd + ti_);                                             \
        _Pragma("unroll") for (int k_ = 0; k_ < 4; ++k_)                                          \
            t_abh[k_] = ldg_u32((const uint32_t*)(lp_).abh + min(tid + DP_NT * k_, (G_) * 32 - 1)); \
    } while (0)
#define DP_TAB2(lp_)                                                                              \
    do {                                                                                          \
        _Pragma("unroll") for (int k_ = 0; k_ < 5; ++k_)                                          \
            t_w2[k_] = ldg_u32x4((const u32x4*)(lp_).w2 + min(tid + DP_NT * k_, 2303));          \
        const int ts_ = min(max(tid - 128, 0), 31);                                               \
        t_sc = ldg_f((lp_).sc + ts_);                                                             \
        t_w2sum = ldg_i32((lp_).w2sum + ts_);                                                     \
    } while (0)
    // weights of output tile c of group g (the MFMA A operand: rows 32 c + j, bytes 16 h ..)
#define DP_W(lp_, g) ldg_u32x4((const uint8_t*)(lp_).w1 + ((int64_t)(g) * 128 + 32 * c + j) * 32 + 16 * h)
#define DP_RW(lp_, G_)                                                                            \
    _Pragma("unroll") for (int q_ = 0; q_ < DW; ++q_) rw[q_] = DP_W(lp_, min(DP_G(q_), (G_) - 1))
    // store bytes of the items of chunk ch a wave prologues (item i = wave + 8 q: group i / PT, tile
    // i % PT); `ready_` = groups that exist already
#define DP_RA(ch_, G_, ready_)                                                                    \
    _Pragma("unroll") for (int q_ = 0; q_ < IPW; ++q_) {                                          \
        const int i_ = wave + 8 * q_, g_ = min((ch_) * CG + i_ / PT, (ready_) - 1);                \
        ra[q_] = *(const u32x4*)DP_SRC(g_, i_ % PT);                                              \
    }
#define DP_XCH_TAG(l_) ((uint64_t)(epoch * 64u + (uint32_t)(l_) + 1u) << 32)

    if (valid) {
        const D8sLayerP lp0 = DP_LP(0);
        DP_TAB1(lp0, G0);
        DP_TAB2(lp0);
        DP_RA(0, G0, G0);
    }
    // Pass i: (A) conv1 of layer i over the groups that exist before layer i - 1's conv2 (all but the
    // newest), (B) layer i - 1's halo rows and its conv2, whose output (the newest group) goes
    // through layer i's prologue straight into LDS, (C) that group's MFMAs, layer i's epilogue into
    // the window and its first / last rows out to the neighbours.  The neighbours' rows of layer i are
    // waited for only in pass i + 1, after its conv1: the exchange runs beside that conv1.
    i32x16 acc[NPT];
    for (int i = 0; i <= (valid ? L : -1); ++i) {
        // ==== (A) conv1 of layer i over its groups 0 .. G - 1 ====
        if (i < L) {
            const D8sLayerP lp = DP_LP(i);
            const int G = i == 0 ? G0 : G0 + i - 1;
            const int nch = (G + CG - 1) / CG;
            if (i > 0) __syncthreads();                    // layer i - 1's epilogue has read its tables
            if (i == 0) {
#pragma unroll
                for (int k = 0; k < 5; ++k)
                    if (tid + DP_NT * k < 2304) s_w[swz((tid + DP_NT * k) >> 1, tid & 1)] = t_w2[k];
                if (tid >= 128 && tid < 160) {
                    s_sc[tid - 128] = t_sc;
                    s_w2sum[tid - 128] = t_w2sum;
                }
            }
            if (tid < 128) {
                s_w1sum[tid] = t_w1sum;
                s_gd[tid] = t_gd;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (tid + DP_NT * k < (G0 + i) * 32) s_abh[tid + DP_NT * k] = t_abh[k];
            // group G - 1 (layer i - 2's output), if it is in chunk 0, was not ready when chunk 0 was
            // requested: its bytes from the copy conv2 left in LDS (a global load here would make the
            // prologue below wait for every store in flight)
            if (i > 1 && G - 1 < CG) {
#pragma unroll
                for (int q_ = 0; q_ < IPW; ++q_) {
                    const int i_ = wave + 8 * q_;
                    if (i_ / PT == G - 1) ra[q_] = s_pro[(ITEMS + i_ % PT) * 64 + lane];
                }
            }
            __syncthreads();                               // tables in LDS

            // ---- prologue of chunk ch into LDS buffer ch & 1 ----
#define DP_PRO(ch_)                                                                               \
    _Pragma("unroll") for (int q_ = 0; q_ < IPW; ++q_) {                                          \
        const int i_ = wave + 8 * q_, g_ = min((ch_) * CG + i_ / PT, G - 1);                      \
        const u32x4* pp_ = (const u32x4*)(s_abh + g_ * 32 + h * 16);                              \
        s_pro[(((ch_) & 1) * ITEMS + i_) * 64 + lane] = pro16(ra[q_], pp_[0], pp_[1], pp_[2], pp_[3]); \
    }
            DP_PRO(0);
            // the next layer's conv1 tables and this layer's newest-group weights (unconditional, a
            // clamped layer: a load under a branch makes later waits wait for every load), then the
            // loads in the loop's order (activations two chunks ahead, then the weight ring), so the
            // wait counts at the loop's head are the same from both of its entries
            {
                const int ln_ = min(i + 1, L - 1);
                const D8sLayerP ln = DP_LP(ln_);
                DP_TAB1(ln, G0 + ln_);
                t_wn = DP_W(lp, G0 + i - 1);                 // (i = 0: group G0 - 1, unused)
            }
            DP_RA(1, G, G);
            DP_RW(lp, G);
            __syncthreads();
            const int32_t m128 = hv == 0 || KH == 1 ? 128 : 0;      // one K half starts at 128 sum w
#pragma unroll
            for (int tt = 0; tt < NPT; ++tt) {
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[tt][v] = m128 * s_w1sum[32 * c + res_row(v, h)];
            }
            for (int ch = 0; ch < nch; ++ch) {
                // straight-line steps (no load under a branch: the wait counts stay exact and the
                // prefetched loads stay in flight); a step past the last group multiplies zero weights.
                // The next chunk's prologue items are spread between the steps, so their VALU work runs
                // beside the MFMAs already issued (an item past the last chunk is never read).
                const u32x4* bsrc = s_pro + (ch & 1) * ITEMS * 64 + lane;
                constexpr int EVERY = QC / IPW;            // steps per prologue item
                // the chunk's operands read from LDS together, so the steps wait for one latency (where
                // the registers allow: up to 8 operands)
                constexpr bool BX = QC * NPT <= 8;
                u32x4 bx[BX ? QC : 1][BX ? NPT : 1];
                if constexpr (BX) {
#pragma unroll
                    for (int u = 0; u < QC; ++u) {
                        const int gi = (KH == 2 ? 2 * u + hv : u);
#pragma unroll
                        for (int tt = 0; tt < NPT; ++tt)
                            bx[u][tt] = bsrc[(gi * PT + (KH == 2 ? 0 : hv * NPT + tt)) * 64];
                    }
                }
#pragma unroll
                for (int u = 0; u < QC; ++u) {
                    const int q = ch * QC + u, g = DP_G(q);
                    const uint32_t live = g < G ? ~0u : 0u;
                    const u32x4 wa = rw[u % DW] & u32x4{live, live, live, live};
                    rw[u % DW] = DP_W(lp, min(DP_G(q + DW), G - 1));
                    const int gi = (KH == 2 ? 2 * u + hv : u);
#pragma unroll
                    for (int tt = 0; tt < NPT; ++tt) {
                        const int t = KH == 2 ? 0 : hv * NPT + tt;
                        acc[tt] = mfma_i8(wa, BX ? bx[BX ? u : 0][BX ? tt : 0] : bsrc[(gi * PT + t) * 64], acc[tt]);
                    }
                    if ((u + 1) % EVERY == 0) {
                        const int qi = (u + 1) / EVERY - 1;    // item wave + 8 qi of chunk ch + 1
                        const int i_ = wave + 8 * qi, g_ = min((ch + 1) * CG + i_ / PT, G - 1);
                        const u32x4* pp_ = (const u32x4*)(s_abh + g_ * 32 + h * 16);
                        s_pro[(((ch + 1) & 1) * ITEMS + i_) * 64 + lane] =
                            pro16(ra[qi], pp_[0], pp_[1], pp_[2], pp_[3]);
                        const int g2 = min((ch + 2) * CG + i_ / PT, G - 1);
                        ra[qi] = *(const u32x4*)DP_SRC(g2, i_ % PT);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                __syncthreads();                           // chunk ch read, chunk ch + 1 written
            }
            // the next pass's first chunk: its groups but the newest exist (that one: see above)
            DP_RA(0, G0 + i, G);
        }

        // ==== (B) layer i - 1's halo rows and conv2 ====
        if (i > 0) {
            const int lc = i - 1, par = lc & 1;
            const uint64_t tag = DP_XCH_TAG(lc);
            // the last pass has no (A): its barriers ordered the window rows (C) wrote before this
            if (i == L) __syncthreads();
            // conv2's pixel tile t2 and K steps st = s2, s2 + S2, ... of 36 for this wave; a tile whose
            // rows all lie inside the band (rows 1 .. R - 2) reads no halo row, so its MFMAs run while
            // the neighbours' rows are read
            const bool active = PT == 1 ? wave < 4 : true;
            const int t2 = PT == 1 ? 0 : wave / S2, s2 = PT == 1 ? wave : wave % S2;
            const int pl = 32 * t2 + j, yl = pl / W, x = pl - yl * W;
            const int q0 = yl * BW + x;
            const bool inner = (32 * t2) / W >= 1 && (32 * t2 + 31) / W <= R - 2;
            i32x16 acc2;
#pragma unroll
            for (int v = 0; v < 16; ++v) acc2[v] = s2 == 0 ? 128 * s_w2sum[res_row(v, h)] : 0;
            constexpr int NS = (36 + S2 - 1) / S2;
            // the steps' operands read C2D steps ahead (an LDS read takes longer than one MFMA step;
            // the compiler on its own waits for each pair of reads), where the registers allow
            constexpr int C2D = PT <= 4 ? 3 : 1;
#define DP_C2F(k_, sl_)                                                                           \
    do {                                                                                          \
        const int st_ = min(s2 + (k_) * S2, 35);                                                  \
        const int cc_ = st_ / 9, tap_ = st_ - 9 * cc_, ty_ = tap_ / 3, tx_ = tap_ - 3 * ty_;       \
        c2w[sl_] = s_w[swz(st_ * 32 + j, h)];                                                     \
        c2b[sl_] = s_b[cc_ * WIN * 2 + swz(q0 + ty_ * BW + tx_, h)];                              \
    } while (0)
#define DP_CONV2()                                                                                \
    do {                                                                                          \
        u32x4 c2w[4], c2b[4];                                                                     \
        _Pragma("unroll") for (int f_ = 0; f_ < C2D; ++f_) DP_C2F(f_, f_);                        \
        _Pragma("unroll") for (int k_ = 0; k_ < NS; ++k_) {                                       \
            if (k_ + C2D < NS) DP_C2F(k_ + C2D, (k_ + C2D) & 3);                                  \
            if (s2 + k_ * S2 < 36) acc2 = mfma_i8(c2w[k_ & 3], c2b[k_ & 3], acc2);                \
            __builtin_amdgcn_sched_barrier(0);                                                    \
        }                                                                                         \
    } while (0)
            // the neighbours' rows into the halo rows (window row 0 = the band above's last row, row
            // R + 1 = the band below's first row), polling each pair until its tag is current; a
            // thread's first pair is read before the inner tiles' MFMAs (an edge band reads its own
            // pairs there, unused)
            uint64_t f[4];
            {
                const int idx = min(tid, 16 * W - 1);
                const int hh = idx & 1, xx = (idx >> 1) % W, cc = ((idx >> 1) / W) & 3, below = idx / (8 * W);
                const bool has = below ? part < K - 1 : part > 0;
                const int tk = has ? (below ? ticket + 1 : ticket - 1) : ticket;
                const uint64_t* xp = DP_XP(tk, par, below ? 0 : 1, cc) + xx * 8 + 4 * hh;
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4) f[e4] = ld_agent64(xp + e4);
            }
            if (active && inner) {
                DP_CONV2();
            }
            for (int idx = tid; idx < 2 * 4 * W * 2; idx += DP_NT) {
                const int hh = idx & 1, xx = (idx >> 1) % W, cc = ((idx >> 1) / W) & 3, below = idx / (8 * W);
                if (below ? part < K - 1 : part > 0) {
                    const uint64_t* xp = DP_XP(below ? ticket + 1 : ticket - 1, par, below ? 0 : 1, cc) + xx * 8 + 4 * hh;
                    uint64_t v0 = f[0], v1 = f[1], v2 = f[2], v3 = f[3];
                    bool ok = idx == tid && ((v0 & v1 & v2 & v3) >> 32) == (tag >> 32) &&
                              ((v0 | v1 | v2 | v3) >> 32) == (tag >> 32);
                    for (int it = 0; it < DP_SPIN && !ok && !broken; ++it) {
                        __builtin_amdgcn_s_sleep(1);
                        v0 = ld_agent64(xp); v1 = ld_agent64(xp + 1); v2 = ld_agent64(xp + 2); v3 = ld_agent64(xp + 3);
                        if (((v0 & v1 & v2 & v3) >> 32) == (tag >> 32) && ((v0 | v1 | v2 | v3) >> 32) == (tag >> 32)) {
                            ok = true;
                            break;
                        }
                    }
                    if (!ok && !broken) {
                        broken = true;
                        atomicAdd(sync + 2, 1u);
                    }
                    s_b[cc * WIN * 2 + swz((below ? R + 1 : 0) * BW + xx + 1, hh)] =
                        u32x4{(uint32_t)v0, (uint32_t)v1, (uint32_t)v2, (uint32_t)v3};
                }
            }
            __syncthreads();

            // ---- conv2 (3x3, pad 1) of the tiles next to the halo rows ----
            if (active && !inner) {
                DP_CONV2();
            }
#undef DP_CONV2
#undef DP_C2F
            // layer i's conv2 tables (stored at the start of (C))
            {
                const D8sLayerP ln = DP_LP(min(i, L - 1));
                DP_TAB2(ln);
            }
            if constexpr (S2 > 1) {
                if (active && s2 > 0) {
                    int32_t* r = s_red + ((s2 - 1) * PT + t2) * 1024 + lane;
#pragma unroll
                    for (int v = 0; v < 16; ++v) r[v * 64] = acc2[v];
                }
                __syncthreads();
                if (active && s2 == 0) {
#pragma unroll
                    for (int qq = 1; qq < S2; ++qq) {
                        const int32_t* r = s_red + ((qq - 1) * PT + t2) * 1024 + lane;
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc2[v] += r[v * 64];
                    }
                }
            }
            if (active && s2 == 0) {
                uint32_t e[4];
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) e[kk] = epi2_q(acc2, kk, *(const float4*)(s_sc + 8 * kk + 4 * h));
                const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
                *(u32x4*)(segn + (int64_t)lc * slot + (uint32_t)((bandp + pl) * 32 + 16 * h)) = row;
                // the new group's bytes of pixel tile t2 through layer i's prologue: exactly the MFMA B
                // operand of that tile (pixel j, bytes 16 h ..)
                if (i < L) {
                    const u32x4* pp_ = (const u32x4*)(s_abh + (G0 + i - 1) * 32 + h * 16);
                    s_pro[t2 * 64 + lane] = pro16(row, pp_[0], pp_[1], pp_[2], pp_[3]);
                    s_pro[(ITEMS + t2) * 64 + lane] = row;   // the raw bytes, for the next pass's chunk 0
                }
            }
            // slot i - 1 stored and the new group's operands written; the conv2 weights read
            __syncthreads();
        }

        // ==== (C) layer i's newest group, epilogue, rows out ====
        if (i < L) {
            if (i > 0) {
                // layer i's conv2 tables (before the rows go out: a wait after those stores would
                // wait for them)
#pragma unroll
                for (int k = 0; k < 5; ++k)
                    if (tid + DP_NT * k < 2304) s_w[swz((tid + DP_NT * k) >> 1, tid & 1)] = t_w2[k];
                if (tid >= 128 && tid < 160) {
                    s_sc[tid - 128] = t_sc;
                    s_w2sum[tid - 128] = t_w2sum;
                }
                // 32-pixel bands: the group belongs to the K half of its parity
                const uint32_t live = KH == 1 || ((G0 + i - 1) & 1) == hv ? ~0u : 0u;
                const u32x4 wa = t_wn & u32x4{live, live, live, live};
#pragma unroll
                for (int tt = 0; tt < NPT; ++tt) {
                    const int t = KH == 2 ? 0 : hv * NPT + tt;
                    acc[tt] = mfma_i8(wa, s_pro[t * 64 + lane], acc[tt]);
                }
            }
            // 32-pixel bands: the two K halves of each output tile added through LDS
            if constexpr (KH == 2) {
                if (hv == 1) {
                    int32_t* r = s_red + c * 1024 + lane;
#pragma unroll
                    for (int v = 0; v < 16; ++v) r[v * 64] = acc[0][v];
                }
                __syncthreads();
                if (hv == 0) {
                    const int32_t* r = s_red + c * 1024 + lane;
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[0][v] += r[v * 64];
                }
            }
            // ---- bottleneck bytes (v ^ 0x80) into the window; the band's first / last row out ----
            const int par = i & 1;
            const uint64_t tag = DP_XCH_TAG(i);
            if (KH == 1 || hv == 0) {
                uint32_t e[4];
#pragma unroll
                for (int tt = 0; tt < NPT; ++tt) {
                    const int t = KH == 2 ? 0 : hv * NPT + tt;
                    const int pl = 32 * t + j, yl = pl / W, x = pl - yl * W;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const float4* pg = (const float4*)(s_gd + 32 * c + 8 * kk + 4 * h);
                        e[kk] = epi1_x80(acc[tt], kk, pg[0], pg[1]);
                    }
                    const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
                    s_b[c * WIN * 2 + swz((yl + 1) * BW + x + 1, h)] = row;
                    if (yl == 0 && part > 0) {
                        uint64_t* xp = DP_XP(ticket, par, 0, c) + x * 8 + 4 * h;
#pragma unroll
                        for (int e4 = 0; e4 < 4; ++e4) st_agent64(xp + e4, tag | row[e4]);
                    }
                    if (yl == R - 1 && part < K - 1) {
                        uint64_t* xp = DP_XP(ticket, par, 1, c) + x * 8 + 4 * h;
#pragma unroll
                        for (int e4 = 0; e4 < 4; ++e4) st_agent64(xp + e4, tag | row[e4]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
#undef DP_PRO
#undef DP_RA
#undef DP_RW
#undef DP_W
#undef DP_TAB1
#undef DP_TAB2
#undef DP_XCH_TAG
#undef DP_LP
#undef DP_G
#undef DP_XP
#undef DP_SRC
    // the last workgroup to end resets the ticket and the end count, and counts the launch
    if (tid == 0) {
        const uint32_t done = __hip_atomic_fetch_add(sync + 1, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (uint32_t)nparts - 1) {
            st_agent(sync, 0u);
            st_agent(sync + 1, 0u);
            st_agent(sync + 3, epoch + 1u);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Transition, pool first: conv and 2x2 mean commute, so S = sum_k w[o][k] s[k] with s[k] = the sum of the
// prologue outputs u of channel k over the four pixels of the square (0 <= s <= 1020).  s = 256 h + l
// (h <= 3, l <= 255) goes to the MFMAs as two int8 operands, h and l - 128, into two accumulators:
// S = 256 acc_h + acc_l with acc_l starting at 128 sum_k w (exact int32).  Two MFMAs per output tile and
// K group instead of one per pixel of the square.
// A workgroup takes PT pixel tiles (32 output pixels each) and ALL output channels: the prologue runs
// once per input byte.  Staging item = (output pixel, channel quad): four dword loads (the square's
// pixels), the prologue's fp16 halves 0x6480 + u summed as plain integers (four halves of at most
// 0x657f carry exactly one bit out of the low half, so the total less 4 * 0x64806480 mod 2^32 is
// s0 | s1 << 16), the two operand bytes of the quad's channels written to LDS (double-buffered, one
// barrier per group).  The four waves split the output tiles (wave w: tiles w, w + 4, ..., NT of them).
// Activations are loaded D groups ahead (registers, D | G); a group's weights are loaded after its
// predecessor's MFMAs and before the next activation loads, so waiting for them never waits for the
// activations still in flight.  Loads take a uniform base plus a 32-bit lane offset.
// ------------------------------------------------------------------------------------------------
template <int NT, int PT, int D, int WB>
__global__ __launch_bounds__(256, NT <= 5 && WB < 4 ? 2 : 1) void k_trans(D8sGemmArgs a0, D8sGemmArgs a1, int split) {
    const PairSlot ps = pair_slot(split);
    const D8sGemmArgs a = ps.second ? a1 : a0;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int PX = 32 * PT;                            // output pixels per workgroup
    constexpr int PLANE = PX * 2;                          // 16-byte chunks of one operand plane
    const int G = a.G, G0 = a.G0;
    u32x4* s_b = (u32x4*)smem;                             // [2 buf][2 plane (l, h)][PX][2]
    uint32_t* s_abh = (uint32_t*)(smem + 4 * PLANE * 16);  // [G * 32]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31;
    // the prologue tables: the first NAB dwords per thread requested now and stored after the first
    // groups' loads are on their way (a load-and-store loop waits one L2 round trip per iteration);
    // NAB covers 40 groups, the widest transition input of DenseNet169 (none for the widest outputs,
    // whose registers are full: they stage the tables here)
    constexpr int NAB = NT >= 8 ? 0 : 5;
    const uint32_t* abh32 = (const uint32_t*)a.abh;
    uint32_t vab[NAB > 0 ? NAB : 1];
#pragma unroll
    for (int k = 0; k < NAB; ++k) vab[k] = abh32[min(tid + 256 * k, G * 32 - 1)];
    if constexpr (NAB == 0)
        for (int i = tid; i < G * 32; i += 256) s_abh[i] = abh32[i];

    // pixel counts fit 32 bits (the launcher checks N * HW)
    const uint32_t HW = (uint32_t)a.HW, W = (uint32_t)a.W;
    const uint32_t W2 = W >> 1, HW4 = HW >> 2;
    const uint32_t NO = (uint32_t)a.N * HW4;
    const uint32_t op0 = (uint32_t)ps.bid * (uint32_t)PX;
    const int OT = a.cout >> 5;

    // staging items of this thread.  Narrow (PT < 4): item = tid + 256 k -> channel quad cq = item & 7,
    // output pixel px = item >> 3, four dword loads.  Wide (PT = 4, the 128 pixels of a workgroup): item
    // = tid -> channel half hh = tid & 1, output pixel tid >> 1, four 16-byte loads (a quarter of the
    // load instructions per byte: the data return path is paced by instructions, not bytes).
    constexpr bool WIDE = PT == 4;
    constexpr int IT = WIDE ? 1 : PT, RW = WIDE ? 4 : 1;   // items per thread, registers per item
    const int cq = tid & 7, hh = tid & 1;
    uint32_t oin[IT], oseg[IT];                            // byte offsets of the square's top-left pixel
    int sdst[IT];
#pragma unroll
    for (int k = 0; k < IT; ++k) {
        const uint32_t px = WIDE ? (uint32_t)(tid >> 1) : (uint32_t)(tid >> 3) + 32u * k;
        uint32_t op = op0 + px;
        if (op >= NO) op = NO - 1;
        const uint32_t n = op / HW4, p4 = op - n * HW4;
        const uint32_t oy = p4 / W2, ox = p4 - oy * W2;
        const uint32_t p = 2 * oy * W + 2 * ox;
        const uint32_t cb = WIDE ? 16 * hh : 4 * cq;
        oin[k] = (n * (uint32_t)G0 * HW + p) * 32 + cb;
        oseg[k] = (n * HW + p) * 32 + cb;
        sdst[k] = WIDE ? swz((int)px, hh) * 16 : swz((int)px, cq >> 2) * 16 + 4 * (cq & 3);  // plane bytes
    }
    const uint32_t row = W * 32;
    const int64_t in_gs = (int64_t)HW * 32, seg_gs = (int64_t)a.N * HW * 32;
    const uint32_t in_bytes = (uint32_t)a.N * (uint32_t)G0 * HW * 32;
    // the square's data of item k, group g: buffer loads (uniform base and size, the row step as the
    // scalar offset)
    auto ld = [&](int k, int g, u32x4* x) {
        const bool lo = g < G0;
        const auto r = lo ? brsrc(a.in0 + g * in_gs, in_bytes - (uint32_t)(g * in_gs))
                          : brsrc(a.seg + (g - G0) * seg_gs, (uint32_t)seg_gs);
        const uint32_t o = lo ? oin[k] : oseg[k];
        if constexpr (WIDE) {
            x[0] = bload128(r, o, 0);
            x[1] = bload128(r, o + 32, 0);
            x[2] = bload128(r, o, row);
            x[3] = bload128(r, o + 32, row);
        } else {
            x[0].x = bload32(r, o, 0);
            x[0].y = bload32(r, o + 32, 0);
            x[0].z = bload32(r, o, row);
            x[0].w = bload32(r, o + 32, row);
        }
    };

    uint32_t wof[NT];                                      // weight row offsets (clamped past OT)
    i32x16 accl[NT][PT], acch[NT][PT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int ot = wave + 4 * i < OT ? wave + 4 * i : OT - 1;
        wof[i] = (uint32_t)((32 * ot + j) * 32 + 16 * h);
        i32x16 init;
#pragma unroll
        for (int v = 0; v < 16; ++v) init[v] = 128 * a.wsum[32 * ot + res_row(v, h)];
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            accl[i][t] = init;
            acch[i][t] = i32x16{};
        }
    }
    auto wload = [&](int g, u32x4* aw) {
        const auto r = brsrc(a.w + (int64_t)g * a.cout * 32, (uint32_t)a.cout * 32);
#pragma unroll
        for (int i = 0; i < NT; ++i) aw[i] = bload128(r, wof[i], 0);
    };
    // one staging item: prologue of the square's bytes, the sums, both operand planes to LDS (sums of
    // channel pairs of one dword: sl = channels 0, 1, sh = 2, 3)
    auto sum4 = [&](uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3, const u32x4& p, uint32_t& lb,
                    uint32_t& hb) {
        const uint32_t xs[4] = {x0, x1, x2, x3};
        uint32_t sl = 0, sh = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint32_t rl, rh;
            pro4_halves(xs[c], p.x, p.y, p.z, p.w, rl, rh);
            sl += rl;
            sh += rh;
        }
        sl -= 0x92019200u;                                 // 4 * 0x64806480 mod 2^32
        sh -= 0x92019200u;
        lb = perm(sh, sl, 0x06040200u) ^ SIGN4;            // l - 128
        hb = perm(sh, sl, 0x07050301u);                    // h
    };
    auto stage = [&](const u32x4* x, uint8_t* dst, const u32x4* prm) {
        if constexpr (WIDE) {
            uint32_t lb[4], hb[4];
            sum4(x[0].x, x[1].x, x[2].x, x[3].x, prm[0], lb[0], hb[0]);
            sum4(x[0].y, x[1].y, x[2].y, x[3].y, prm[1], lb[1], hb[1]);
            sum4(x[0].z, x[1].z, x[2].z, x[3].z, prm[2], lb[2], hb[2]);
            sum4(x[0].w, x[1].w, x[2].w, x[3].w, prm[3], lb[3], hb[3]);
            *(u32x4*)dst = u32x4{lb[0], lb[1], lb[2], lb[3]};
            *(u32x4*)(dst + PLANE * 16) = u32x4{hb[0], hb[1], hb[2], hb[3]};
        } else {
            uint32_t lb, hb;
            sum4(x[0].x, x[0].y, x[0].z, x[0].w, prm[0], lb, hb);
            *(uint32_t*)dst = lb;
            *(uint32_t*)(dst + PLANE * 16) = hb;
        }
    };

    // weights: WB register sets (WB | D): group g's in set g % WB, loaded WB - 1 groups ahead before
    // a group's prologue (WB = 4 for the wide outputs, whose weights are most of the bytes and come
    // from L2: one workgroup per CU then, the registers of four sets); one set when D is odd (loaded
    // after the MFMAs)
    static_assert(D % WB == 0, "weight sets divide the activation depth");
    u32x4 raw[D][IT][RW], aw[WB][NT];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int k = 0; k < IT; ++k) ld(k, d < G ? d : G - 1, raw[d][k]);
#pragma unroll
    for (int w = 0; w < (WB > 1 ? WB - 1 : 1); ++w) wload(w < G ? w : G - 1, aw[w]);
#pragma unroll
    for (int k = 0; k < NAB; ++k)
        if (tid + 256 * k < G * 32) s_abh[tid + 256 * k] = vab[k];
    if constexpr (NAB > 0)
        for (int i = tid + 256 * NAB; i < G * 32; i += 256) s_abh[i] = abh32[i];
    __syncthreads();                                       // s_abh
    // D groups per step; the first step is peeled so that the loop's waits see only the steady state
    // (the preamble's load order would otherwise make them wait for every load)
    auto step = [&](int g0) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int g = g0 + d;
            u32x4* awc = aw[d % WB];
            if constexpr (WB > 1) {
                const int gw = g + WB - 1 < G ? g + WB - 1 : G - 1;
                wload(gw, aw[(d + WB - 1) % WB]);
                __builtin_amdgcn_sched_barrier(0);         // issued ahead of the prologue
            }
            uint8_t* sb = (uint8_t*)(s_b + (g & 1) * 2 * PLANE);
            u32x4 prm[RW];
#pragma unroll
            for (int c = 0; c < RW; ++c)
                prm[c] = *(const u32x4*)(s_abh + g * 32 + (WIDE ? hh * 16 + 4 * c : cq * 4));
#pragma unroll
            for (int k = 0; k < IT; ++k) stage(raw[d][k], sb + sdst[k], prm);
            __syncthreads();
            const u32x4* bl = (const u32x4*)sb;
#pragma unroll
            for (int t = 0; t < PT; ++t) {
                const u32x4 vl = bl[swz(32 * t + j, h)], vh = bl[PLANE + swz(32 * t + j, h)];
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    accl[i][t] = mfma_i8(awc[i], vl, accl[i][t]);
                    acch[i][t] = mfma_i8(awc[i], vh, acch[i][t]);
                }
            }
            // (one set: the next group's weights now, before the activations), then this slot's
            // activations D groups on (the last groups reload the last one: the loads stay
            // unconditional and countable)
            if constexpr (WB == 1) {
                wload(g + 1 < G ? g + 1 : g, aw[0]);
                __builtin_amdgcn_sched_barrier(0);
            }
            const int gn = g + D < G ? g + D : G - 1;
#pragma unroll
            for (int k = 0; k < IT; ++k) ld(k, gn, raw[d][k]);
            // keep the next slot's prologue below this point: hoisted, it would wait for loads still
            // in flight
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    step(0);
    for (int g0 = D; g0 < G; g0 += D) step(g0);
    // epilogue: q = RNE(clamp(S * (float(k) / 4), -127, 127)) (trans_w_body with the exact mean,
    // src/knee/dense8s_kernels.cu:3226-3245), as the low byte of q + 1.5 * 2^23
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int ot = wave + 4 * i;
        if (ot >= OT) break;
        float kq[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) kq[v] = a.gd[2 * (32 * ot + res_row(v, h))];
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            uint32_t e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t b[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int v = 4 * k + rr;
                    const int32_t S = acch[i][t][v] * 256 + accl[i][t][v];
                    const float x = kq[v] * ((float)S * 0.25f);
                    b[rr] = __float_as_uint(__builtin_amdgcn_fmed3f(x, -127.0f, 127.0f) + 12582912.0f);
                }
                e[k] = pack_b0(b[0], b[1], b[2], b[3]);
            }
            const u32x4 rowv = xchg_rows(e[0], e[1], e[2], e[3], h);
            const uint32_t op = op0 + 32 * t + j;
            if (op < NO) {
                const uint32_t n = op / HW4, p4 = op - n * HW4;
                *(u32x4*)((int8_t*)a.out + ((int64_t)(n * (uint32_t)a.G0n + ot) * HW4 + p4) * 32 + 16 * h) = rowv;
            }
        }
        asm volatile("" ::: "memory");
    }
}

// ------------------------------------------------------------------------------------------------
// Linear head on the final features (configuration 4's 1664 -> 8 logits): out[n][k] = b[k] + the
// float32 dot product of x[n][.] and w[k][.].  Workgroup = one image, wave = output k (k, k + 4, ...):
// lane l sums c = l, l + 64, ... with fma in that order, then the 64 lane sums are added by a butterfly
// (xor 32, 16, ..., 1), and b[k] last.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_linear(const float* __restrict__ x, int C, const float* __restrict__ w,
                                                const float* __restrict__ b, int K, float* __restrict__ out) {
    const int n = blockIdx.x, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const float* xn = x + (int64_t)n * C;
    for (int k = wave; k < K; k += 4) {
        const float* wk = w + (int64_t)k * C;
        float s = 0.0f;
        for (int c = lane; c < C; c += 64) s = __builtin_fmaf(xn[c], wk[c], s);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) out[(int64_t)n * K + k] = s + b[k];
    }
}

// ------------------------------------------------------------------------------------------------
// Final features: out[n][c] = (((P0 + P1) + P2) + P3) / HW with P_q = sum over pixels s = q, q + 4, ...
// (in order) of relu(fma(a_c, q_s, b_c)): the summation order of the reference's `final_q`
// (src/knee/dense8s_kernels.cu:2304-2323), so the fp32 result is the same.  Workgroup = one image x 2
// groups: 64 channels x 4 partials.
// `status` (may be null): the pass's error word (the banded whole-block launches' count of bounded waits
// that ran out).  When it is not zero the features of the pass are NaN instead, so that features built
// from stale halo rows cannot pass for valid ones; `report` (may be null, host-mapped memory) receives
// the word from one thread, for the host to read without a synchronisation.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_final(const int8_t* __restrict__ in0, int G0,
                                               const int8_t* __restrict__ seg, int N, int HW, int G,
                                               const float* __restrict__ ab, float* __restrict__ out,
                                               int ctot, const uint32_t* __restrict__ status,
                                               uint32_t* __restrict__ report) {
    __shared__ float part[4][64];
    const uint32_t err = status ? status[0] : 0u;
    if (report && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)   // to host memory, past the caches
        __hip_atomic_store(report, err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int n = blockIdx.x;
    const int c64 = threadIdx.x & 63, qp = threadIdx.x >> 6;
    const int g = blockIdx.y * 2 + (c64 >> 5), cc = c64 & 31;
    float acc = 0.0f;
    if (g < G) {
        const int8_t* base = g < G0 ? in0 + ((int64_t)n * G0 + g) * HW * 32
                                    : seg + ((int64_t)(g - G0) * N + n) * HW * 32;
        const float2 p = ((const float2*)ab)[g * 32 + cc];
        // 8 pixels' bytes loaded before they are added (in order), so 8 loads are in flight
        int s = qp;
        for (; s + 28 < HW; s += 32) {
            int8_t q[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) q[k] = base[(int64_t)(s + 4 * k) * 32 + cc];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc += __builtin_fmaxf(__builtin_fmaf(p.x, (float)q[k], p.y), 0.0f);
        }
        for (; s < HW; s += 4)
            acc += __builtin_fmaxf(__builtin_fmaf(p.x, (float)base[(int64_t)s * 32 + cc], p.y), 0.0f);
    }
    part[qp][c64] = acc;
    __syncthreads();
    if (qp == 0 && g < G)
        out[(int64_t)n * ctot + g * 32 + cc] =
            err ? __builtin_nanf("") : (((part[0][c64] + part[1][c64]) + part[2][c64]) + part[3][c64]) / (float)HW;
}

// ------------------------------------------------------------------------------------------------
// Stem: 7x7/2 conv (pad 3) on fp16 MFMA 32x32x16 (fp32 accumulation, bias as the initial value),
// ReLU, int8 quantisation q = RNE(min(relu(y) / sigma0, 127)), 3x3/2 max-pool (pad 1) on the bytes
// (quantisation is monotonic, so pooling after it gives the same bytes), into in0 of block 0.
// Workgroup = 8 x 16 pooled pixels = 17 x 33 conv pixels (18 MFMA pixel tiles) x 64 channels.
// K = (channel, ky, kx') with kx' = kx + 1 in 1..7 and kx' = 0 a zero weight (the reference's `S_w16`
// layout, src/knee/dense8s.py:522-530): 168 -> 11 steps of 16.  A lane's 8 K values are 8 consecutive
// input columns 2 cx - 4 .. 2 cx + 3, whose start is even: 4-byte aligned fp16 pairs in LDS.
// The input tile (39 x 72 per channel) is built in LDS as fp16: x16 = lut[c][u] (uint8 input) or the
// fp16 input itself, zero outside the image, mirrored when flip = 1 (every image) or, with flip = 2
// (flip-TTA pairs), for the second half of the batch: output image n >= N/2 is source image n - N/2
// mirrored, so N/2 input images give N encoded images without a mirrored copy in memory.
// ------------------------------------------------------------------------------------------------
static constexpr int ST_PY = 8, ST_PX = 16;
static constexpr int ST_CY = 2 * ST_PY + 1, ST_CX = 2 * ST_PX + 1, ST_NCP = ST_CY * ST_CX;   // 17 x 33
static constexpr int ST_IY = 4 * ST_PY + 7, ST_IX = 4 * ST_PX + 8;                        // 39 x 72
static constexpr int ST_WROW = 184;                      // fp16 per weight row in LDS (168 + pad)
static constexpr int ST_PT = (ST_NCP + 31) / 32;         // 18 pixel tiles

__global__ __launch_bounds__(256) void k_stem(D8sStemArgs a, int tiles_x, int tiles_y) {
    __shared__ __attribute__((aligned(16))) _Float16 s_in[3 * ST_IY * ST_IX];
    __shared__ __attribute__((aligned(16))) _Float16 s_wt[64 * ST_WROW];
    __shared__ __attribute__((aligned(16))) uint8_t s_c[ST_PT * 32 * 64];
    __shared__ _Float16 s_lut[3 * 256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, j = lane & 31;
    const int H = a.H, W = a.W, Hc = H / 2, Wc = W / 2, Hp = H / 4, Wp = W / 4;
    const int per_img = tiles_x * tiles_y;
    const int n = blockIdx.x / per_img, r = blockIdx.x - n * per_img;
    const int py0 = (r / tiles_x) * ST_PY, px0 = (r % tiles_x) * ST_PX;
    const int cy0 = 2 * py0 - 1, cx0 = 2 * px0 - 1;
    const int iy0 = 2 * cy0 - 3, ix0 = 2 * cx0 - 4;
    const int half = a.N >> 1;
    const int ns = (a.flip == 2 && n >= half) ? n - half : n;          // source image
    const bool mirror = a.flip == 1 || (a.flip == 2 && n >= half);

    // Loads are issued all together and their data used only afterwards (a use right after a load
    // would make every load wait for the previous one).
    // weights [64][168] (21 chunks of 16 bytes per row) -> LDS rows of 184 fp16, zero tail
    {
        constexpr int NWC = 64 * 21, KW = (NWC + 255) / 256;
        u32x4 wv[KW];
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            const int i = tid + 256 * k;
            wv[k] = ((const u32x4*)a.w16)[i < NWC ? i : 0];
        }
        if (tid < 128) {                                  // rows' chunks 21 and 22: K 168..183
            const u32x4 z = {0u, 0u, 0u, 0u};
            *(u32x4*)(s_wt + (tid >> 1) * ST_WROW + 168 + 8 * (tid & 1)) = z;
        }
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            const int i = tid + 256 * k;
            if (i < NWC) *(u32x4*)(s_wt + (i / 21) * ST_WROW + 8 * (i % 21)) = wv[k];
        }
    }
    if (a.kind == D8S_IN_U8) {
        for (int i = tid; i < 3 * 256; i += 256) s_lut[i] = __builtin_bit_cast(_Float16, a.lut[i]);
        // uint8 input: every row of the tile (3 x 39 rows of 72 bytes, starting at x = ix0 = 4 px0 - 6,
        // or mirrored) is fetched as 19 aligned dwords (W is a multiple of 4, so a dword is wholly in
        // or out of the image), then each pair of bytes becomes two fp16 LUT values written as one
        // dword: bytes (0, 1) of dword d land at lx = 4 d - 2 (mirrored: 72 - 4 d, swapped), bytes
        // (2, 3) at lx = 4 d (mirrored: 70 - 4 d, swapped); the first pair of d = 0 and the second of
        // d = 18 fall outside the tile.
        constexpr int ND = 19, NROW = 3 * ST_IY, NI = NROW * ND, KD = (NI + 255) / 256;
        const int a0 = mirror ? W - 4 * px0 - 68 : 4 * px0 - 8;          // first aligned source x
        const uint8_t* x8 = (const uint8_t*)a.x;
        uint32_t raw[KD];
        uint32_t okm = 0;
#pragma unroll
        for (int k = 0; k < KD; ++k) {
            const int i = tid + 256 * k;
            const int r = i / ND, d = i - r * ND;
            const int c = r / ST_IY, ly = r - c * ST_IY;
            const int y = iy0 + ly, xd = a0 + 4 * d;
            const bool ok = i < NI && (unsigned)y < (unsigned)H && (unsigned)xd < (unsigned)W;
            const int64_t off = ok ? (((int64_t)ns * 3 + c) * H + y) * W + xd : 0;
            raw[k] = *(const uint32_t*)(x8 + off);
            okm |= (uint32_t)ok << k;
        }
        __syncthreads();                                  // s_lut
#pragma unroll
        for (int k = 0; k < KD; ++k) {
            const int i = tid + 256 * k;
            if (i >= NI) break;
            const int r = i / ND, d = i - r * ND;
            const int c = r / ST_IY;
            const uint32_t v = ((okm >> k) & 1) ? raw[k] : 0u;
            const _Float16* lt = s_lut + c * 256;
            const uint32_t zero = 0u;
            const uint32_t h0 = (okm >> k) & 1 ? __builtin_bit_cast(uint16_t, lt[v & 0xff]) : zero;
            const uint32_t h1 = (okm >> k) & 1 ? __builtin_bit_cast(uint16_t, lt[(v >> 8) & 0xff]) : zero;
            const uint32_t h2 = (okm >> k) & 1 ? __builtin_bit_cast(uint16_t, lt[(v >> 16) & 0xff]) : zero;
            const uint32_t h3 = (okm >> k) & 1 ? __builtin_bit_cast(uint16_t, lt[v >> 24]) : zero;
            uint32_t* row = (uint32_t*)(s_in + r * ST_IX);
            if (d >= 1) row[mirror ? (72 - 4 * d) / 2 : (4 * d - 2) / 2] = mirror ? h1 | (h0 << 16) : h0 | (h1 << 16);
            if (d <= 17) row[mirror ? (70 - 4 * d) / 2 : (4 * d) / 2] = mirror ? h3 | (h2 << 16) : h2 | (h3 << 16);
        }
    } else {
        constexpr int NIN = 3 * ST_IY * ST_IX, KIN = (NIN + 255) / 256;
        uint32_t raw[KIN];
        uint64_t okm = 0;
        int64_t idx[KIN];
#pragma unroll
        for (int k = 0; k < KIN; ++k) {
            const int i = tid + 256 * k;
            const int c = i / (ST_IY * ST_IX), rr = i - c * (ST_IY * ST_IX);
            const int ly = rr / ST_IX, lx = rr - ly * ST_IX;
            const int y = iy0 + ly, x = ix0 + lx;
            const bool ok = i < NIN && (unsigned)y < (unsigned)H && (unsigned)x < (unsigned)W;
            const int xs = mirror ? W - 1 - x : x;
            idx[k] = ok ? (((int64_t)ns * 3 + c) * H + y) * W + xs : 0;
            okm |= (uint64_t)ok << k;
        }
        const uint16_t* x16 = (const uint16_t*)a.x;
#pragma unroll
        for (int k = 0; k < KIN; ++k) raw[k] = x16[idx[k]];
#pragma unroll
        for (int k = 0; k < KIN; ++k) {
            const int i = tid + 256 * k;
            if (i >= NIN) break;
            s_in[i] = ((okm >> k) & 1) ? __builtin_bit_cast(_Float16, (uint16_t)raw[k]) : (_Float16)0.0f;
        }
    }
    __syncthreads();

    float bias[2][16], inv[2][16];
#pragma unroll
    for (int ot = 0; ot < 2; ++ot)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            bias[ot][v] = a.bias[32 * ot + res_row(v, h)];
            inv[ot][v] = a.inv[32 * ot + res_row(v, h)];
        }
    for (int pt = wave; pt < ST_PT; pt += 4) {
        int cp = pt * 32 + j;
        const bool cp_ok = cp < ST_NCP;
        if (!cp_ok) cp = ST_NCP - 1;
        const int ly = cp / ST_CX, lx = cp - ly * ST_CX;
        f32x16 acc[2];
#pragma unroll
        for (int ot = 0; ot < 2; ++ot)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[ot][v] = bias[ot][v];
#pragma unroll
        for (int s = 0; s < 11; ++s) {
            int rk = 2 * s + h;                           // (channel, ky) row of K
            if (rk > 20) rk = 20;                         // its weights are zero
            const int c = rk / 7, ky = rk - 7 * (rk / 7);
            const uint32_t* pin = (const uint32_t*)(s_in + (c * ST_IY + 2 * ly + ky) * ST_IX + 2 * lx);
            const u32x4 bx = {pin[0], pin[1], pin[2], pin[3]};
            const f16x8 b = __builtin_bit_cast(f16x8, bx);
#pragma unroll
            for (int ot = 0; ot < 2; ++ot) {
                const f16x8 w = *(const f16x8*)(s_wt + (32 * ot + j) * ST_WROW + 16 * s + 8 * h);
                acc[ot] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w, b, acc[ot], 0, 0, 0);
            }
        }
        const int cy = cy0 + ly, cx = cx0 + lx;
        const bool in_img = cp_ok && (unsigned)cy < (unsigned)Hc && (unsigned)cx < (unsigned)Wc;
#pragma unroll
        for (int ot = 0; ot < 2; ++ot) {
            uint32_t e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t d = 0;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int v = 4 * k + rr;
                    const float t = __builtin_fmaxf(acc[ot][v], 0.0f) * inv[ot][v];
                    const float q = __builtin_rintf(__builtin_fminf(t, 127.0f));
                    d |= ((uint32_t)(int)q & 0xffu) << (8 * rr);
                }
                e[k] = in_img ? d : 0u;
            }
            const u32x4 row = xchg_rows(e[0], e[1], e[2], e[3], h);
            if (cp_ok) *(u32x4*)(s_c + cp * 64 + 32 * ot + 16 * h) = row;
        }
    }
    __syncthreads();
    // 3x3/2 max-pool of the bytes (all in [0, 127]: byte-wise max by the borrow-free difference)
    for (int i = tid; i < ST_PY * ST_PX * 4; i += 256) {
        const int k = i & 3, pix = i >> 2;
        const int py = pix / ST_PX, px = pix - py * ST_PX;
        u32x4 m = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int dy = 0; dy < 3; ++dy)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) {
                const u32x4 v = *(const u32x4*)(s_c + ((2 * py + dy) * ST_CX + 2 * px + dx) * 64 + 16 * k);
                const u32x4 ge = (((m | SIGN4) - v) & SIGN4) >> 7;     // 1 per byte where m >= v
                const u32x4 mask = ge * 255u;
                m = (m & mask) | (v & ~mask);
            }
        const int gy = py0 + py, gx = px0 + px;
        if (gy < Hp && gx < Wp)
            *(u32x4*)(a.out + ((((int64_t)n * 2 + (k >> 1)) * Hp + gy) * Wp + gx) * 32 + 16 * (k & 1)) = m;
    }
}

// ------------------------------------------------------------------------------------------------
// Stem, row-band form (W <= 512): the same conv, quantisation and pool as k_stem, for a workgroup
// that owns SR rows of pooled output of one image across the whole width.  Wave w computes conv
// columns 32 w .. 32 w + 31; B-operand column n holds conv column 32 w + 2 n (n < 16) or
// 32 w + 2 (n - 16) + 1 (n >= 16), even columns in the first 16 lanes of each half, odd columns in
// the last 16.  Per pooled row py a wave computes conv rows 2 py and 2 py + 1 (row 2 py - 1 is the
// previous pooled row's second row) and pools in registers:
//   * the max over the three conv rows, per lane;
//   * v_permlane16_swap pairs each even column (the window's centre) with the odd column to its
//     right in one lane (lanes 0-15 of each half for output tile 1, lanes 16-31 for tile 0), and a
//     DPP row shift brings the odd column to its left; lane 0 of a row takes the previous wave's
//     last column through LDS (zero at the image's edge).
// Quantisation q = RNE(min(max(y, 0) inv, 127)) with inv > 0 is monotonic, so it commutes with the
// max: only the pooled values are quantised, giving the same bytes as quantising every conv pixel
// and pooling the bytes; 0 stands for the padding (q(0) = 0 is the least byte).
// K order and weights in LDS as in k_stem (identical fp32 sums, so identical bytes); a lane's row
// offset per K step is one of four per-lane bases plus an immediate.
// Input rows: a ring of 16 rows per channel in LDS, each row stored twice (slots r & 15 and
// (r & 15) + 16) so that the 13 rows a pooled row reads are consecutive slots.  The rows a pooled
// row adds (4 per channel) are fetched into registers two pooled rows ahead (uint8 through the LUT
// into fp16, mirrored on the way when the image is flipped).
// ------------------------------------------------------------------------------------------------
static constexpr int SR_NWV = 8;                           // waves at most: 256 conv columns
static constexpr int SR_RS = 288;                          // ring row stride (dwords, = 32 mod 64)
static constexpr int SR_CH = 32 * SR_RS + 32;              // ring channel stride (dwords, = 32 mod 64)
static constexpr int SR_WROW = 184;                        // fp16 per weight row (176 used)
static constexpr size_t SR_LDS = (size_t)3 * SR_CH * 4 + 64 * SR_WROW * 2 + (2 * SR_NWV * 64 + 16 + 128) * 4
                                 + 3 * 256 * 2;

// One unit of an input row: 4 fp16 values of channel c, row y, landing at columns 4 D .. 4 D + 3
// (mirrored: source columns W - 4 D - 4 .. W - 4 D - 1 reversed).  Rows outside the image: 0.
struct SrUnit {
    u32x2 raw;
    bool ok;
};

// (valid = false: an unused unit of the thread; it loads element 0 and is never stored.)  e0: the
// element offset of the unit in row 0; the input has fewer than 2^31 elements.
template <bool U8>
DEV SrUnit sr_fetch(const void* x, int H, int W, int e0, int y, bool valid) {
    SrUnit u;
    u.ok = valid && (unsigned)y < (unsigned)H;
    const int e = u.ok ? e0 + y * W : 0;
    if (U8) u.raw = u32x2{*(const uint32_t*)((const uint8_t*)x + e), 0u};
    else u.raw = *(const u32x2*)((const uint16_t*)x + e);
    return u;
}

// element offset of unit D of row 0 of channel c of source image ns
DEV int sr_e0(int ns, int c, int H, int W, int D, bool mirror) {
    return ((ns * 3 + c) * H) * W + 4 * (mirror ? (W >> 2) - 1 - D : D);
}

DEV uint32_t lut2(const _Float16* lt, uint32_t b0, uint32_t b1) {
    return (uint32_t)__builtin_bit_cast(uint16_t, lt[b0]) | ((uint32_t)__builtin_bit_cast(uint16_t, lt[b1]) << 16);
}

// q0: the unit's dword offset in ring slot 0 (channel c, column unit D: c SR_CH + 2 + 2 D)
template <bool U8>
DEV void sr_put(uint32_t* s_ring, const _Float16* s_lut, bool mirror, SrUnit u, int c, int q0, int y) {
    uint32_t lo, hi;
    if (U8) {
        const _Float16* lt = s_lut + 256 * c;
        const uint32_t v = u.raw.x;
        const uint32_t b0 = v & 255u, b1 = (v >> 8) & 255u, b2 = (v >> 16) & 255u, b3 = v >> 24;
        lo = mirror ? lut2(lt, b3, b2) : lut2(lt, b0, b1);
        hi = mirror ? lut2(lt, b1, b0) : lut2(lt, b2, b3);
    } else {
        lo = mirror ? __builtin_amdgcn_alignbit(u.raw.y, u.raw.y, 16) : u.raw.x;
        hi = mirror ? __builtin_amdgcn_alignbit(u.raw.x, u.raw.x, 16) : u.raw.y;
    }
    lo = u.ok ? lo : 0u;
    hi = u.ok ? hi : 0u;
    uint32_t* p = s_ring + q0 + (y & 15) * SR_RS;
    *(u32x2*)p = u32x2{lo, hi};
    *(u32x2*)(p + 16 * SR_RS) = u32x2{lo, hi};
}

// B operand: 8 fp16 at a 4-byte aligned LDS byte address.
DEV f16x8 sr_b(const uint8_t* p) {
    const uint32_t* q = (const uint32_t*)p;
    return __builtin_bit_cast(f16x8, u32x4{q[0], q[1], q[2], q[3]});
}

// Conv rows whose input windows start at ring slot sb (and sb + 2 for the second row): accumulators
// (r0t0, r0t1) and (r1t0, r1t1) for output tiles 0 and 1, started from the bias.  K step s, lane half
// h covers row rk = 2 s + h of the (channel, ky) rows (the order of k_stem, so the sums are the same):
// h = 1 reads the next ky of the same channel except at s = 3 (channel 0 ky 6 / channel 1 ky 0) and
// s = 10 (rk 21 is a zero weight row: it reads rk 20 again).  pA: channels 0-1, + h rows; pB: + h
// (channel - 6 rows); pC: channel 2, + h rows; pD: channel 2.
DEV f32x16 ld16(const float* p) {                         // 16 result rows of a lane (4 x 4 channels)
    f32x16 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 v = *(const float4*)(p + 8 * q);
        r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
    }
    return r;
}

template <bool TWO>
DEV void sr_rows(const uint8_t* pA, const uint8_t* pB, const uint8_t* pC, const uint8_t* pD, const _Float16* wl,
                 const float* bl, f32x16& r0t0, f32x16& r0t1, f32x16& r1t0, f32x16& r1t1) {
    const f32x16 bias0 = ld16(bl), bias1 = ld16(bl + 32);
#pragma unroll
    for (int s = 0; s < 11; ++s) {
        const uint8_t* rp = s < 3    ? pA + 2 * s * SR_RS * 4
                            : s == 3 ? pB + 6 * SR_RS * 4
                            : s < 7  ? pA + SR_CH * 4 + (2 * s - 7) * SR_RS * 4
                            : s < 10 ? pC + (2 * s - 14) * SR_RS * 4
                                     : pD + 6 * SR_RS * 4;
        const f16x8 w0 = *(const f16x8*)(wl + 16 * s);
        const f16x8 w1 = *(const f16x8*)(wl + 32 * SR_WROW + 16 * s);
        const f16x8 b0 = sr_b(rp);
        r0t0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w0, b0, s == 0 ? bias0 : r0t0, 0, 0, 0);
        r0t1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1, b0, s == 0 ? bias1 : r0t1, 0, 0, 0);
        if (TWO) {
            const f16x8 b1 = sr_b(rp + 2 * SR_RS * 4);
            r1t0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w0, b1, s == 0 ? bias0 : r1t0, 0, 0, 0);
            r1t1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w1, b1, s == 0 ? bias1 : r1t1, 0, 0, 0);
        }
    }
}

DEV float f32_of(uint32_t x) { return __builtin_bit_cast(float, x); }
DEV uint32_t bits_of(float x) { return __builtin_bit_cast(uint32_t, x); }

// One pooled row py = py0 + T: conv rows 2 py, 2 py + 1 (into O0, O1), the ring rows of the next
// pooled row from BUF, BUF refetched with the rows of pooled row py + 3, the pool with conv row
// 2 py - 1 (P0, P1), quantisation and the store.  Two calls per loop iteration swap BUF and (P, O), so
// the loop carries no register copies.
#define SR_STEP(T, BUF, P0, P1, O0, O1)                                                                \
    do {                                                                                             \
        const int py_ = py0 + (T), sb_ = (4 * py_ - 3) & 15;                                         \
        f32x16 e0_, e1_;                                                                             \
        {                                                                                            \
            const uint8_t* r_ = ringb + sb_ * SR_RS * 4;                                             \
            sr_rows<true>(r_ + offA, r_ + offB, r_ + offC, r_ + offD, wl, bl, e0_, e1_, O0, O1);  \
        }                                                                                            \
        if ((T) + 1 < npy) {                                                                         \
            _Pragma("unroll") for (int k = 0; k < 3; ++k) if (uv[k])                                 \
                sr_put<U8>(s_ring, s_lut, mirror, BUF[k], uc[k], uq[k], 4 * (py_ + 1) + 2 + um[k]);  \
        }                                                                                            \
        _Pragma("unroll") for (int k = 0; k < 3; ++k)                                                \
            BUF[k] = sr_fetch<U8>(a.x, a.H, a.W, ue[k], 4 * (py_ + 3) + 2 + um[k],                  \
                                  uv[k] && (T) + 3 < npy);                                           \
        f32x16 c_, r_;                                                                               \
        _Pragma("unroll") for (int v = 0; v < 16; ++v) {                                             \
            const float m0_ = __builtin_fmaxf(__builtin_fmaxf(P0[v], e0_[v]), O0[v]);               \
            const float m1_ = __builtin_fmaxf(__builtin_fmaxf(P1[v], e1_[v]), O1[v]);               \
            const auto sw_ = __builtin_amdgcn_permlane16_swap(bits_of(m1_), bits_of(m0_), false, false); \
            c_[v] = f32_of(sw_[0]);                                                                  \
            r_[v] = f32_of(sw_[1]);                                                                  \
        }                                                                                            \
        float* hb_ = s_halo + ((T) & 1) * SR_NWV * 64;                                               \
        if (i == 15) {                                                                               \
            float* hp_ = hb_ + (wave * 4 + rr + 2 * h) * 16;                                         \
            _Pragma("unroll") for (int q = 0; q < 4; ++q)                                            \
                *(float4*)(hp_ + 4 * q) = float4{r_[4 * q], r_[4 * q + 1], r_[4 * q + 2], r_[4 * q + 3]}; \
        }                                                                                            \
        __syncthreads();                                                                             \
        const float* hl_ = (i == 0 && wave > 0) ? hb_ + ((wave - 1) * 4 + rr + 2 * h) * 16           \
                                                : s_halo + 2 * SR_NWV * 64;                          \
        const f32x16 invq = ld16(il);                                                                \
        uint32_t dw_[4];                                                                             \
        _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                              \
            const float4 hv_ = *(const float4*)(hl_ + 4 * q);                                        \
            const float hq_[4] = {hv_.x, hv_.y, hv_.z, hv_.w};                                       \
            uint32_t d_ = 0u;                                                                        \
            _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                          \
                const int v = 4 * q + e;                                                             \
                const float p_ = __builtin_fmaxf(__builtin_fmaxf(c_[v], r_[v]), hq_[e]);            \
                const float l_ = f32_of((uint32_t)__builtin_amdgcn_update_dpp(                       \
                    (int)bits_of(p_), (int)bits_of(r_[v]), 0x111, 0xf, 0xf, false));                 \
                const float m_ = __builtin_amdgcn_fmed3f(p_, l_, 3.0e38f);    /* max of finite */    \
                const float qv_ = __builtin_rintf(__builtin_amdgcn_fmed3f(m_ * invq[v], 0.0f, 127.0f)); \
                d_ = __builtin_amdgcn_cvt_pk_u8_f32(qv_, e, d_);                                     \
            }                                                                                        \
            dw_[q] = d_;                                                                             \
        }                                                                                            \
        const auto s02_ = __builtin_amdgcn_permlane32_swap(dw_[0], dw_[2], false, false);            \
        const auto s13_ = __builtin_amdgcn_permlane32_swap(dw_[1], dw_[3], false, false);            \
        if (px < Wp)                                                                                 \
            *(u32x4*)(a.out + ((((int64_t)n * 2 + (1 - rr)) * Hp + py_) * Wp + px) * 32 + 16 * h) =  \
                u32x4{s02_[0], s02_[1], s13_[0], s13_[1]};                                           \
    } while (0)

template <bool U8>
__global__ __launch_bounds__(512, 1) void k_stem_rows(D8sStemArgs a0, int bands, int band_rows, D8sStemArgs a1,
                                                      int split) {
    const PairSlot ps = pair_slot(split);
    const D8sStemArgs a = ps.second ? a1 : a0;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint32_t* s_ring = (uint32_t*)smem;                                 // [3][SR_CH]
    _Float16* s_wt = (_Float16*)(s_ring + 3 * SR_CH);                   // [64][SR_WROW]
    float* s_halo = (float*)(s_wt + 64 * SR_WROW);                      // [2][SR_NWV][4][16], 16 zeros
    float* s_bias = s_halo + 2 * SR_NWV * 64 + 16;                      // [64]
    float* s_inv = s_bias + 64;                                         // [64]
    _Float16* s_lut = (_Float16*)(s_inv + 64);                          // [3][256]
    const int nt = blockDim.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, j = lane & 31, rr = j >> 4, i = j & 15;
    const int Hp = a.H >> 2, Wp = a.W >> 2, W4 = a.W >> 2;
    const int n = ps.bid / bands, band = ps.bid - n * bands;
    const int py0 = band * band_rows, npy = min(band_rows, Hp - py0);
    const int half = a.N >> 1;
    const int ns = (a.flip == 2 && n >= half) ? n - half : n;          // source image
    const bool mirror = a.flip == 1 || (a.flip == 2 && n >= half);

    // The set-up's loads first, all in flight together (clamped addresses): the weights ([64][168]
    // fp16 + zero K 168..175: rows of 21 16-byte chunks and a zero one), bias, inv, the LUT, and rows
    // 4 py0 - 5 .. 4 py0 + 5 (the first pooled row's window and the conv row above it); then the LDS
    // stores (a load-and-store loop waits one memory round trip per iteration), the ring zeros first
    // (the column padding is never written again).  The first batches cover 512 threads; narrower
    // workgroups stage the rest in the loops after them.
    constexpr int NWB = (64 * 22 + 511) / 512, NLB = (3 * 256 + 511) / 512;
    constexpr int KI = 9;                                               // 33 W/4 units over >= W threads
    u32x4 wv[NWB];
    uint16_t lv[NLB];
#pragma unroll
    for (int k = 0; k < NWB; ++k) {
        const int q = min(tid + k * nt, 64 * 22 - 1), o = q / 22, rk = q - o * 22;
        wv[k] = ((const u32x4*)a.w16)[o * 21 + min(rk, 20)];
    }
#pragma unroll
    for (int k = 0; k < NLB; ++k) lv[k] = U8 ? a.lut[min(tid + k * nt, 3 * 256 - 1)] : (uint16_t)0;
    const float t_bias = a.bias[min(tid, 63)], t_inv = a.inv[min(tid, 63)];
    SrUnit u[KI];
#pragma unroll
    for (int k = 0; k < KI; ++k) {
        const int q = tid + k * nt, rb = q / W4, D = q - rb * W4, c = rb / 11;
        u[k] = sr_fetch<U8>(a.x, a.H, a.W, sr_e0(ns, c, a.H, a.W, D, mirror), 4 * py0 - 5 + (rb - 11 * c),
                            q < 33 * W4);
    }
    for (int k = tid; k < 3 * SR_CH / 4; k += nt) ((u32x4*)s_ring)[k] = u32x4{0u, 0u, 0u, 0u};
    if (tid < 16) s_halo[2 * SR_NWV * 64 + tid] = 0.0f;
#pragma unroll
    for (int k = 0; k < NWB; ++k) {
        const int q = tid + k * nt, o = q / 22, rk = q - o * 22;
        uint32_t m = rk < 21 ? ~0u : 0u;                                // chunk 21: the zero K rows
        asm volatile("" : "+v"(m));                                     // (an AND, not a branch)
        if (q < 64 * 22) *(u32x4*)(s_wt + o * SR_WROW + 8 * rk) = wv[k] & u32x4{m, m, m, m};
    }
    for (int k = tid + NWB * nt; k < 64 * 22; k += nt) {
        const int o = k / 22, rk = k - o * 22;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (rk < 21) v = ((const u32x4*)a.w16)[o * 21 + rk];
        *(u32x4*)(s_wt + o * SR_WROW + 8 * rk) = v;
    }
    if (tid < 64) {
        s_bias[tid] = t_bias;
        s_inv[tid] = t_inv;
    }
    if (U8) {
#pragma unroll
        for (int k = 0; k < NLB; ++k)
            if (tid + k * nt < 3 * 256) s_lut[tid + k * nt] = __builtin_bit_cast(_Float16, lv[k]);
        for (int k = tid + NLB * nt; k < 3 * 256; k += nt) s_lut[k] = __builtin_bit_cast(_Float16, a.lut[k]);
    }
    __syncthreads();

    {
#pragma unroll
        for (int k = 0; k < KI; ++k) {
            const int q = tid + k * nt, rb = q / W4, D = q - rb * W4, c = rb / 11;
            if (q < 33 * W4)
                sr_put<U8>(s_ring, s_lut, mirror, u[k], c, c * SR_CH + 2 + 2 * D, 4 * py0 - 5 + (rb - 11 * c));
        }
    }
    // this thread's units of the 4 rows per channel a pooled row adds: (channel, row m, column unit)
    int uc[3], um[3], ue[3], uq[3];
    bool uv[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int q = tid + k * nt, rb = q / W4, D = q - rb * W4;
        uv[k] = q < 12 * W4;
        uc[k] = rb >> 2;
        um[k] = rb & 3;
        ue[k] = sr_e0(ns, rb >> 2, a.H, a.W, D, mirror);
        uq[k] = (rb >> 2) * SR_CH + 2 + 2 * D;
    }
    // rows added by pooled row py0 + t: 4 (py0 + t) + 2 + m; na holds those of odd t, nb of even t
    SrUnit na[3], nb[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        na[k] = sr_fetch<U8>(a.x, a.H, a.W, ue[k], 4 * (py0 + 1) + 2 + um[k], uv[k] && npy > 1);
        nb[k] = sr_fetch<U8>(a.x, a.H, a.W, ue[k], 4 * (py0 + 2) + 2 + um[k], uv[k] && npy > 2);
    }

    // per-lane constants
    const int cx = 32 * wave + (rr ? 2 * i + 1 : 2 * i);                // this B column's conv column
    const int px = 16 * wave + i;                                       // this lane's pooled column
    const uint8_t* ringb = (const uint8_t*)s_ring;
    const int offA = 4 * cx + h * SR_RS * 4;
    const int offB = 4 * cx + h * (SR_CH - 6 * SR_RS) * 4;
    const int offC = 4 * cx + 2 * SR_CH * 4 + h * SR_RS * 4;
    const int offD = 4 * cx + 2 * SR_CH * 4;
    const _Float16* wl = s_wt + j * SR_WROW + 8 * h;
    const float* bl = s_bias + 4 * h;                                   // this lane's result rows
    const float* il = s_inv + 32 * (1 - rr) + 4 * h;                    // lanes 0-15: tile 1, 16-31: tile 0
    __syncthreads();

    f32x16 pa0, pa1, pb0, pb1;                                          // conv rows 2 py - 1 / 2 py + 1
    if (py0 > 0) {
        const int sb = (4 * py0 - 5) & 15;
        const uint8_t* r = ringb + sb * SR_RS * 4;
        sr_rows<false>(r + offA, r + offB, r + offC, r + offD, wl, bl, pa0, pa1, pb0, pb1);
    } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) pa0[v] = pa1[v] = 0.0f;
    }
    int t = 0;
    for (; t + 1 < npy; t += 2) {                     // (no branch inside: exact wait counts across steps)
        SR_STEP(t, na, pa0, pa1, pb0, pb1);
        SR_STEP(t + 1, nb, pb0, pb1, pa0, pa1);
    }
    if (t < npy) SR_STEP(t, na, pa0, pa1, pb0, pb1);
}
#undef SR_STEP

// ------------------------------------------------------------------------------------------------
// Diagnostics
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                              int64_t n) {
    // tiles of 1024 chunks: four coalesced loads in flight per thread, then the four stores
    for (int64_t t = (int64_t)blockIdx.x * 1024; t < n; t += (int64_t)gridDim.x * 1024) {
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t i = t + 256 * k + threadIdx.x;
            if (i < n) v[k] = __builtin_nontemporal_load(src + i);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t i = t + 256 * k + threadIdx.x;
            if (i < n) __builtin_nontemporal_store(v[k], dst + i);
        }
    }
}

__global__ __launch_bounds__(256) void k_mfma_loop(int iters, int32_t* sink) {
    const int lane = threadIdx.x & 63;
    u32x4 a = {(uint32_t)lane, 1u, 2u, 3u}, b = {3u, (uint32_t)lane, 1u, 2u};
    i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; ++i) {
        c0 = mfma_i8(a, b, c0);
        c1 = mfma_i8(a, b, c1);
        c2 = mfma_i8(a, b, c2);
        c3 = mfma_i8(a, b, c3);
    }
    int32_t s = 0;
#pragma unroll
    for (int v = 0; v < 16; ++v) s += c0[v] ^ c1[v] ^ c2[v] ^ c3[v];
    if (threadIdx.x == 0) sink[blockIdx.x] = s;
}

__global__ void k_probe_i8(const int8_t* A, const int8_t* B, int32_t* D) {
    const int l = threadIdx.x, h = l >> 5, j = l & 31;
    u32x4 av, bv;
    uint8_t* pa = (uint8_t*)&av;
    uint8_t* pb = (uint8_t*)&bv;
    for (int k = 0; k < 16; ++k) {
        pa[k] = (uint8_t)A[j * 32 + 16 * h + k];          // A[i = j][k]
        pb[k] = (uint8_t)B[(16 * h + k) * 32 + j];        // B[k][j]
    }
    const i32x16 d = mfma_i8(av, bv, i32x16{});
    for (int v = 0; v < 16; ++v) D[res_row(v, h) * 32 + j] = d[v];
}

__global__ void k_probe_f16(const uint16_t* A, const uint16_t* B, float* D) {
    const int l = threadIdx.x, h = l >> 5, j = l & 31;
    f16x8 av, bv;
    for (int k = 0; k < 8; ++k) {
        av[k] = __builtin_bit_cast(_Float16, A[j * 16 + 8 * h + k]);
        bv[k] = __builtin_bit_cast(_Float16, B[(8 * h + k) * 32 + j]);
    }
    const f32x16 d = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, f32x16{}, 0, 0, 0);
    for (int v = 0; v < 16; ++v) D[res_row(v, h) * 32 + j] = d[v];
}

// ------------------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------------------
static thread_local std::string g_err;

static int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

static int launched(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string(what) + ": " + hipGetErrorString(e));
    return 0;
}

static int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cached[dev] = v;
    }
    return cached[dev];
}

int d8s_host_fail(int code, const std::string& msg) { return fail(code, msg); }
int d8s_host_launched(const char* what) { return launched(what); }
int d8s_host_cu_count() { return cu_count(); }

#define REQUIRE(cond, msg) \
    do { if (!(cond)) return fail((int)hipErrorInvalidValue, msg); } while (0)

static int check_gemm(const D8sGemmArgs* a, const char* what) {
    REQUIRE(a != nullptr, std::string(what) + ": null arguments");
    REQUIRE(a->in0 && a->w && a->abh && a->gd && a->wsum, std::string(what) + ": null pointer");
    REQUIRE(a->G0 >= 1 && a->G >= 1 && a->N >= 1 && a->HW >= 1 && a->W >= 1,
            std::string(what) + ": G0, G, N, HW, W must be >= 1");
    REQUIRE(a->G <= a->G0 || a->seg != nullptr, std::string(what) + ": seg is null with G > G0");
    REQUIRE(a->HW % a->W == 0, std::string(what) + ": HW is not a multiple of W");
    REQUIRE((int64_t)a->rows == (int64_t)a->N * a->HW, std::string(what) + ": rows != N * HW");
    REQUIRE(a->G <= 1200, std::string(what) + ": more than 1200 groups");
    return 0;
}

// Pairs (`b` not null): two problems of one shape in one launch (PairSlot); sizes and the variant
// are chosen for the two problems' pixels together, persistent grids split evenly between them.
static bool same_gemm(const D8sGemmArgs* a, const D8sGemmArgs* b) {
    return a->G0 == b->G0 && a->G == b->G && a->N == b->N && a->HW == b->HW && a->W == b->W &&
           a->rows == b->rows && a->cout == b->cout && a->G0n == b->G0n;
}

// conv1 kernel variants (d8s_conv1_as): 1, 2 the persistent form with 32- / 64-pixel tiles (three /
// two workgroups per CU), 3, 4, 5 the one-pass form with 1, 2, 4 k-slices; 0 the choice below.
enum { C1V_P32 = 1, C1V_P64 = 2, C1V_K1 = 3, C1V_K2 = 4, C1V_K4 = 5, C1V_MAX = 5 };

// The variant a launch of conv1 with `variant` runs (the choice for 0), or -1 where the shape does
// not take it (the persistent form keeps 32-bit byte offsets: in0 and a slot below 4 GiB).
static int conv1_variant(const D8sGemmArgs* a, const D8sGemmArgs* b, int variant) {
    const int np = b ? 2 : 1;                              // problems in the launch
    const int64_t rows = (int64_t)a->rows * np;
    const int64_t in0_bytes = (int64_t)a->N * a->G0 * a->HW * 32, slot_bytes = (int64_t)a->rows * 32;
    const bool p_ok = in0_bytes < (1ll << 32) && slot_bytes < (1ll << 32);
    if (variant != 0) {
        if (variant < 1 || variant > C1V_MAX) return -1;
        return variant <= C1V_P64 && !p_ok ? -1 : variant;
    }
    // k-slices: the fewest that give at least 1.5 workgroups per CU
    const int64_t want = 3 * (int64_t)cu_count() / 2;
    int ks = 1;
    while (ks < 4 && (rows + 64 * 4 / ks - 1) / (64 * 4 / ks) < want) ks *= 2;
    // one k-slice: the persistent form (the weights through LDS); 64-pixel tiles when every wave of
    // two per SIMD gets at least two, else 32-pixel tiles and three waves per SIMD
    if (ks == 1 && p_ok) return (rows + 63) / 64 >= 2 * 8 * (int64_t)cu_count() ? C1V_P64 : C1V_P32;
    return ks == 1 ? C1V_K1 : ks == 2 ? C1V_K2 : C1V_K4;
}

static int conv1_launch(const D8sGemmArgs* a, const D8sGemmArgs* b, int32_t* acc, hipStream_t st,
                        int variant = 0) {
    if (int rc = check_gemm(a, "d8s_conv1")) return rc;
    REQUIRE(a->cout == 128, "d8s_conv1: cout must be 128");
    REQUIRE(acc != nullptr || a->out != nullptr, "d8s_conv1: null output");
    const int v = conv1_variant(a, b, variant);
    REQUIRE(v >= 1, "d8s_conv1: variant " + std::to_string(variant) + " is not taken for this shape");
    const int np = b ? 2 : 1;                              // problems in the launch
    const int64_t rows = (int64_t)a->rows * np;
    if (v == C1V_P32 || v == C1V_P64) {
        const int u = v == C1V_P64 ? 2 : 1;
        const int64_t ntiles = (rows + 32 * u - 1) / (32 * u);
        const int per_cu = u == 2 ? 2 : 3;                        // workgroups per CU
        const int64_t want_blocks = (ntiles + 3) / 4;
        const int64_t all = want_blocks < per_cu * cu_count() ? want_blocks : per_cu * cu_count();
        const unsigned split = (unsigned)((all + np - 1) / np), grid = split * np;
        const int wm = c1p_lds(a->G, 1) <= (size_t)(160 / per_cu) * 1024 ? 1 : 2;   // still per_cu per CU
        const size_t shm1 = c1p_lds(a->G, wm);
#define C1P_LAUNCH(ACC_, WM_, U_)                                                                 \
    hipLaunchKernelGGL((k_conv1p<ACC_, WM_, U_, U_ == 1 && WM_ == 1 ? 8 : 4>), dim3(grid), dim3(256), shm1,  \
                       st, *a, ACC_ ? acc : nullptr, b ? *b : *a, (int)split)
        if (u == 2) {
            if (acc && wm == 1) C1P_LAUNCH(true, 1, 2);
            else if (acc) C1P_LAUNCH(true, 2, 2);
            else if (wm == 1) C1P_LAUNCH(false, 1, 2);
            else C1P_LAUNCH(false, 2, 2);
        } else {
            if (acc && wm == 1) C1P_LAUNCH(true, 1, 1);
            else if (acc) C1P_LAUNCH(true, 2, 1);
            else if (wm == 1) C1P_LAUNCH(false, 1, 1);
            else C1P_LAUNCH(false, 2, 1);
        }
#undef C1P_LAUNCH
        return launched("d8s_conv1");
    }
    if (b) {                                               // the split-K form: two launches
        if (int rc = conv1_launch(a, nullptr, acc, st, variant)) return rc;
        return conv1_launch(b, nullptr, acc, st, variant);
    }
    const int ks = v == C1V_K1 ? 1 : v == C1V_K2 ? 2 : 4;
    const int px = 64 * 4 / ks;
    const unsigned blocks = (unsigned)((a->rows + px - 1) / px);
    size_t shm = (size_t)a->G * 128;
    if (ks > 1 && shm < C1_RED_BYTES) shm = C1_RED_BYTES;
#define C1_LAUNCH(KS_)                                                                        \
    do {                                                                                      \
        if (acc)                                                                              \
            hipLaunchKernelGGL((k_conv1<KS_, true>), dim3(blocks), dim3(256), shm, st, *a, acc); \
        else                                                                                  \
            hipLaunchKernelGGL((k_conv1<KS_, false>), dim3(blocks), dim3(256), shm, st, *a,     \
                               nullptr);                                                      \
    } while (0)
    if (ks == 1) C1_LAUNCH(1);
    else if (ks == 2) C1_LAUNCH(2);
    else C1_LAUNCH(4);
#undef C1_LAUNCH
    return launched("d8s_conv1");
}

extern "C" int d8s_conv1(const D8sGemmArgs* a, void* stream) {
    if (a != nullptr && a->out == nullptr) return fail((int)hipErrorInvalidValue, "d8s_conv1: null output");
    return conv1_launch(a, nullptr, nullptr, (hipStream_t)stream);
}

extern "C" int d8s_conv1_variant(const D8sGemmArgs* a, int32_t variant) {
    if (a == nullptr || check_gemm(a, "d8s_conv1_variant") != 0 || a->cout != 128) return -1;
    return conv1_variant(a, nullptr, variant);
}

extern "C" int d8s_conv1_as(const D8sGemmArgs* a, int32_t variant, void* stream) {
    if (a != nullptr && a->out == nullptr) return fail((int)hipErrorInvalidValue, "d8s_conv1_as: null output");
    return conv1_launch(a, nullptr, nullptr, (hipStream_t)stream, variant);
}

extern "C" int d8s_conv1_acc32(const D8sGemmArgs* a, int32_t* acc, void* stream) {
    REQUIRE(acc != nullptr, "d8s_conv1_acc32: null accumulator buffer");
    return conv1_launch(a, nullptr, acc, (hipStream_t)stream);
}

extern "C" int d8s_conv1_pair(const D8sGemmArgs* a, const D8sGemmArgs* b, void* stream) {
    REQUIRE(a != nullptr && b != nullptr, "d8s_conv1_pair: null arguments");
    REQUIRE(a->out != nullptr, "d8s_conv1_pair: null output");
    if (int rc = check_gemm(b, "d8s_conv1_pair")) return rc;
    REQUIRE(b->out != nullptr, "d8s_conv1_pair: null output");
    REQUIRE(same_gemm(a, b), "d8s_conv1_pair: the two problems differ in shape");
    return conv1_launch(a, b, nullptr, (hipStream_t)stream);
}

template <int TW, int TH, int KSPL, int PT>
static int conv2_launch(const D8sConv2Args* a, const D8sConv2Args* b, hipStream_t st, int64_t min_tiles) {
    using S = C2Shape<TW, TH, KSPL, PT>;
    const int np = b ? 2 : 1;
    const int tiles_x = (a->W + TW - 1) / TW, tiles_y = (a->H + TH - 1) / TH;
    const int64_t total = (int64_t)a->N * tiles_x * tiles_y;            // per problem
    if (total * np < min_tiles) return -1;
    REQUIRE(total * np < (1ll << 31), "d8s_conv2: too many tiles");
    const int64_t all = total * np < 2 * cu_count() ? total * np : 2 * cu_count();
    int64_t split = (all + np - 1) / np;
    if (np == 2 && split > 8) split = (split + 7) / 8 * 8;   // a rebased workgroup keeps its XCD
    hipLaunchKernelGGL((k_conv2<TW, TH, KSPL, PT>), dim3((unsigned)(split * np)), dim3(256),
                       S::HALO_BYTES + S::RED_BYTES, st, *a, tiles_x, tiles_y, b ? *b : *a, (int)split);
    return launched("d8s_conv2");
}

static int check_conv2(const D8sConv2Args* a, const char* what) {
    REQUIRE(a != nullptr, std::string(what) + ": null arguments");
    REQUIRE(a->x && a->w && a->sc && a->wsum && a->out, std::string(what) + ": null pointer");
    REQUIRE(a->N >= 1 && a->H >= 1 && a->W >= 1, std::string(what) + ": N, H, W must be >= 1");
    return 0;
}

// conv2 kernel variants (d8s_conv2_as), the tile shapes TW x TH: 1 32 x 8, 2 32 x 4, 3 32 x 2 (K split
// in 4), 4 16 x 4, 5 8 x 8, 6 4 x 16, 7 2 x 32, 8 1 x 64 (K split in 4 from 3 on), each taken for maps
// at least TW wide; 0 the choice below (the widest tile that fits, and for 32-wide tiles the tallest
// that still gives three tiles per CU).
static const int C2V_TW[9] = {0, 32, 32, 32, 16, 8, 4, 2, 1};

static int conv2_variant(const D8sConv2Args* a, int variant) {
    if (variant < 0 || variant > 8) return -1;
    if (variant != 0) return C2V_TW[variant] <= a->W ? variant : -1;
    if (a->W >= 32) {
        const int64_t enough = 3 * (int64_t)cu_count();
        if ((int64_t)a->N * ((a->W + 31) / 32) * ((a->H + 7) / 8) >= enough) return 1;
        if ((int64_t)a->N * ((a->W + 31) / 32) * ((a->H + 3) / 4) >= enough) return 2;
        return 3;
    }
    return a->W >= 16 ? 4 : a->W >= 8 ? 5 : a->W >= 4 ? 6 : a->W >= 2 ? 7 : 8;
}

static int conv2_dispatch(const D8sConv2Args* a, const D8sConv2Args* b, hipStream_t st, int variant) {
    if (variant != 0) {
        REQUIRE(conv2_variant(a, variant) >= 1,
                "d8s_conv2: variant " + std::to_string(variant) + " is not taken for this shape");
        switch (variant) {
            case 1: return conv2_launch<32, 8, 1, 2>(a, b, st, 0);
            case 2: return conv2_launch<32, 4, 1, 1>(a, b, st, 0);
            case 3: return conv2_launch<32, 2, 4, 2>(a, b, st, 0);
            case 4: return conv2_launch<16, 4, 4, 2>(a, b, st, 0);
            case 5: return conv2_launch<8, 8, 4, 2>(a, b, st, 0);
            case 6: return conv2_launch<4, 16, 4, 2>(a, b, st, 0);
            case 7: return conv2_launch<2, 32, 4, 2>(a, b, st, 0);
            default: return conv2_launch<1, 64, 4, 2>(a, b, st, 0);
        }
    }
    const int64_t enough = 3 * (int64_t)cu_count();        // tiles for a persistent grid to pipeline
    if (a->W >= 32) {
        int rc = conv2_launch<32, 8, 1, 2>(a, b, st, enough);
        if (rc >= 0) return rc;
        rc = conv2_launch<32, 4, 1, 1>(a, b, st, enough);
        if (rc >= 0) return rc;
        return conv2_launch<32, 2, 4, 2>(a, b, st, 0);
    }
    if (a->W >= 16) return conv2_launch<16, 4, 4, 2>(a, b, st, 0);
    if (a->W >= 8) return conv2_launch<8, 8, 4, 2>(a, b, st, 0);
    if (a->W >= 4) return conv2_launch<4, 16, 4, 2>(a, b, st, 0);
    if (a->W >= 2) return conv2_launch<2, 32, 4, 2>(a, b, st, 0);
    return conv2_launch<1, 64, 4, 2>(a, b, st, 0);
}

extern "C" int d8s_conv2(const D8sConv2Args* a, void* stream) {
    if (int rc = check_conv2(a, "d8s_conv2")) return rc;
    return conv2_dispatch(a, nullptr, (hipStream_t)stream, 0);
}

extern "C" int d8s_conv2_variant(const D8sConv2Args* a, int32_t variant) {
    if (a == nullptr || check_conv2(a, "d8s_conv2_variant") != 0) return -1;
    return conv2_variant(a, variant);
}

extern "C" int d8s_conv2_as(const D8sConv2Args* a, int32_t variant, void* stream) {
    if (int rc = check_conv2(a, "d8s_conv2_as")) return rc;
    return conv2_dispatch(a, nullptr, (hipStream_t)stream, variant);
}

extern "C" int d8s_conv2_pair(const D8sConv2Args* a, const D8sConv2Args* b, void* stream) {
    if (int rc = check_conv2(a, "d8s_conv2_pair")) return rc;
    if (int rc = check_conv2(b, "d8s_conv2_pair")) return rc;
    REQUIRE(a->N == b->N && a->H == b->H && a->W == b->W, "d8s_conv2_pair: the two problems differ in shape");
    return conv2_dispatch(a, b, (hipStream_t)stream, 0);
}

// Whether d8s_conv2_conv1 takes maps of this shape and a conv1 reading G groups.
static bool c21_shape_ok(int H, int W, int G) {
    return (W == 16 || W == 32 || W == 64) && (H * W) % 128 == 0 && G >= 2 && G <= D8S_C21_MAX_GROUPS;
}

extern "C" int d8s_c21_supported(int H, int W, int G) { return c21_shape_ok(H, W, G) ? 1 : 0; }

extern "C" int d8s_conv2_conv1(const D8sConv2Args* c2, const D8sGemmArgs* c1, void* stream) {
    if (int rc = check_conv2(c2, "d8s_conv2_conv1")) return rc;
    if (int rc = check_gemm(c1, "d8s_conv2_conv1")) return rc;
    REQUIRE(c1->cout == 128, "d8s_conv2_conv1: cout must be 128");
    REQUIRE(c1->out != nullptr, "d8s_conv2_conv1: null output");
    REQUIRE(c2->N == c1->N && (int64_t)c2->H * c2->W == c1->HW && c2->W == c1->W,
            "d8s_conv2_conv1: conv2 and conv1 differ in shape");
    REQUIRE(c21_shape_ok(c2->H, c2->W, c1->G),
            "d8s_conv2_conv1: needs W in {16, 32, 64}, H * W a multiple of 128 and 2 <= G <= " +
                std::to_string(D8S_C21_MAX_GROUPS));
    REQUIRE(c1->G > c1->G0, "d8s_conv2_conv1: conv1's last group must be a store slot (G > G0)");
    const int64_t slot = (int64_t)c1->rows * 32;
    REQUIRE((const int8_t*)c2->out == c1->seg + (int64_t)(c1->G - 1 - c1->G0) * slot,
            "d8s_conv2_conv1: conv2's output must be conv1's last group (store slot G - 1 - G0)");
    const uint8_t* xb = c2->x;
    const uint8_t* ob = (const uint8_t*)c1->out;
    REQUIRE(xb + 4 * slot <= ob || ob + 4 * slot <= xb,
            "d8s_conv2_conv1: conv2's bottleneck and conv1's output overlap");
    const int64_t in0_bytes = (int64_t)c1->N * c1->G0 * c1->HW * 32;
    REQUIRE(in0_bytes < (1ll << 32) && 4 * slot + (1ll << 20) < (1ll << 31),
            "d8s_conv2_conv1: in0 of 4 GiB or more, or a bottleneck of 2 GiB or more");
    const int64_t total = (int64_t)c1->N * (c1->HW / 128);
    const int occ = CcShape<32>::OCC;                      // workgroups per CU (3 for every width)
    const int64_t grid = total < occ * cu_count() ? total : occ * cu_count();
    hipStream_t st = (hipStream_t)stream;
#define C21_LAUNCH(W_)                                                                              \
    hipLaunchKernelGGL((k_c21<W_>), dim3((unsigned)grid), dim3(256), cc_lds<W_>(c1->G), st, *c2, *c1)
    if (c2->W == 16) C21_LAUNCH(16);
    else if (c2->W == 32) C21_LAUNCH(32);
    else C21_LAUNCH(64);
#undef C21_LAUNCH
    return launched("d8s_conv2_conv1");
}

template <int TW, int TH, int CPW, int NW>
static int dense_launch(const D8sDenseArgs* a, hipStream_t st) {
    using SL = DnShape<TW, TH, CPW, NW, true>;
    using S = DnShape<TW, TH, CPW, NW, false>;
    const int wh = a->H < TH + 2 ? a->H : TH + 2, ww = a->W < TW + 2 ? a->W : TW + 2;
    REQUIRE(wh * ww <= 32 * NW * CPW, "d8s_dense: window larger than the workgroup's column blocks");
    REQUIRE(S::lds(a->G) + 36864 <= 160 * 1024, "d8s_dense: too many groups for LDS");
    const bool wl = SL::lds(a->G) + 36864 <= 160 * 1024;   // conv1 weights fit in LDS too
    const int tiles_x = (a->W + TW - 1) / TW, tiles_y = (a->H + TH - 1) / TH;
    const int64_t total = (int64_t)a->N * tiles_x * tiles_y;
    REQUIRE(total < (1ll << 31), "d8s_dense: too many tiles");
    const unsigned grid = (unsigned)(total < cu_count() ? total : cu_count());
    if (wl)
        hipLaunchKernelGGL((k_dense<TW, TH, CPW, NW, true>), dim3(grid), dim3(S::NT), SL::lds(a->G), st,
                           *a, tiles_x, tiles_y);
    else
        hipLaunchKernelGGL((k_dense<TW, TH, CPW, NW, false>), dim3(grid), dim3(S::NT), S::lds(a->G), st,
                           *a, tiles_x, tiles_y);
    return launched("d8s_dense");
}

// Band form for W = 64 / 128 while the layer's conv1 weights fit in LDS: bands of 32, 16, 8 .. rows
// (a multiple of the rows per step), the largest that still gives 3 workgroups per CU.
template <int W_>
static int band_launch(const D8sDenseArgs* a, const D8sDenseArgs* b, hipStream_t st) {
    using S = BnShape<W_>;
    const size_t shm = S::lds(a->G);
    if (shm + 36864 > 160 * 1024 || a->G > 16) return -1;
    const int np = b ? 2 : 1;
    // band height: the least of rounds x (rows + 2) over the multiples of RS up to 32 (one workgroup
    // per CU; each band also computes the two bottleneck rows above it; ties go to the taller band):
    // 16 rows at 96 images (768 bands, three rounds); 14 at 24 (240 bands in one round: 16 row-steps
    // of work instead of 18 with 16-row bands, which took the study from 1.489-1.493 to 1.454-1.459
    // ms against 4-row bands in three rounds)
    int rows = 32;
    {
        int64_t best = -1;
        for (int r = 32; r >= S::RS; r -= S::RS) {
            const int64_t nb = (int64_t)a->N * np * ((a->H + r - 1) / r);
            const int64_t cost = (nb + cu_count() - 1) / cu_count() * (r + 2);
            if (best < 0 || cost < best) { best = cost; rows = r; }
        }
    }
    const int bands = (a->H + rows - 1) / rows;
    const int64_t blocks = (int64_t)a->N * bands;          // per problem
    REQUIRE(blocks * np < (1ll << 31), "d8s_dense: too many bands");
    // activation registers (K steps per step): G itself up to 8, then G rounded up to even
    const int gm = a->G <= 8 ? a->G : (a->G + 1) & ~1;
#define BN_LAUNCH(GM_)                                                                             \
    hipLaunchKernelGGL((k_band<W_, GM_>), dim3((unsigned)(blocks * np)), dim3(512), shm, st, *a, bands, rows, \
                       b ? *b : *a, (int)blocks)
    switch (gm) {
        case 1: BN_LAUNCH(1); break;
        case 2: BN_LAUNCH(2); break;
        case 3: BN_LAUNCH(3); break;
        case 4: BN_LAUNCH(4); break;
        case 5: BN_LAUNCH(5); break;
        case 6: BN_LAUNCH(6); break;
        case 7: BN_LAUNCH(7); break;
        case 8: BN_LAUNCH(8); break;
        case 10: BN_LAUNCH(10); break;
        case 12: BN_LAUNCH(12); break;
        case 14: BN_LAUNCH(14); break;
        default: BN_LAUNCH(16); break;
    }
#undef BN_LAUNCH
    return launched("d8s_dense");
}

static int check_dense(const D8sDenseArgs* a, const char* what) {
    REQUIRE(a != nullptr, std::string(what) + ": null arguments");
    REQUIRE(a->in0 && a->w1 && a->abh && a->gd && a->w1sum && a->w2 && a->sc && a->w2sum && a->out,
            std::string(what) + ": null pointer");
    REQUIRE(a->G0 >= 1 && a->G >= 1 && a->N >= 1 && a->H >= 1 && a->W >= 1,
            std::string(what) + ": G0, G, N, H, W must be >= 1");
    REQUIRE(a->G <= a->G0 || a->seg != nullptr, std::string(what) + ": seg is null with G > G0");
    REQUIRE(a->G <= 512, std::string(what) + ": more than 512 groups");
    REQUIRE((int64_t)a->H * a->W <= (1 << 26), std::string(what) + ": more than 2^26 pixels per image");
    return 0;
}

// (the 2-D tile form has no pair launch: a pair runs as two launches)
static int dense_dispatch(const D8sDenseArgs* a, const D8sDenseArgs* b, hipStream_t st) {
    if (a->W == 128 || a->W == 64) {
        const int rc = a->W == 128 ? band_launch<128>(a, b, st) : band_launch<64>(a, b, st);
        if (rc >= 0) return rc;
    }
    if (b) {
        if (int rc = dense_dispatch(a, nullptr, st)) return rc;
        return dense_dispatch(b, nullptr, st);
    }
    if (a->W >= 32) return dense_launch<32, 12, 2, 8>(a, st);
    if (a->W <= 16 && a->H <= 16) return dense_launch<16, 16, 1, 8>(a, st);
    return dense_launch<16, 12, 1, 8>(a, st);
}

extern "C" int d8s_dense(const D8sDenseArgs* a, void* stream) {
    if (int rc = check_dense(a, "d8s_dense")) return rc;
    return dense_dispatch(a, nullptr, (hipStream_t)stream);
}

extern "C" int d8s_dense_pair(const D8sDenseArgs* a, const D8sDenseArgs* b, void* stream) {
    if (int rc = check_dense(a, "d8s_dense_pair")) return rc;
    if (int rc = check_dense(b, "d8s_dense_pair")) return rc;
    REQUIRE(a->G0 == b->G0 && a->G == b->G && a->N == b->N && a->H == b->H && a->W == b->W,
            "d8s_dense_pair: the two problems differ in shape");
    return dense_dispatch(a, b, (hipStream_t)stream);
}

static int dblock_launch(const D8sBlockArgs* a, const D8sBlockArgs* b, hipStream_t st) {
    REQUIRE(a != nullptr, "d8s_dense_block: null arguments");
    REQUIRE(a->in0 && a->layers && (a->L <= 0 || a->seg), "d8s_dense_block: null pointer");
    REQUIRE(a->G0 >= 1 && a->L >= 1 && a->N >= 1 && a->H >= 1 && a->W >= 1,
            "d8s_dense_block: G0, L, N, H, W must be >= 1");
    REQUIRE(a->H * a->W <= DB_NT / 2, "d8s_dense_block: more than 256 pixels per image");
    REQUIRE(a->G0 + a->L - 1 <= 4 * DB_NT / 32, "d8s_dense_block: more than 64 groups");
    const size_t shm = dblock_lds(a->H, a->W, a->G0 + a->L - 1);
    REQUIRE(shm + 36864 + 64 * 7 * 8 <= 160 * 1024, "d8s_dense_block: block too large for LDS");
    const int np = b ? 2 : 1;
    hipLaunchKernelGGL(k_dblock, dim3((unsigned)(a->N * np)), dim3(DB_NT), shm, st, *a, b ? *b : *a, a->N);
    return launched("d8s_dense_block");
}

extern "C" int d8s_dense_block(const D8sBlockArgs* a, void* stream) {
    return dblock_launch(a, nullptr, (hipStream_t)stream);
}

extern "C" int d8s_dense_block_pair(const D8sBlockArgs* a, const D8sBlockArgs* b, void* stream) {
    REQUIRE(a != nullptr && b != nullptr, "d8s_dense_block_pair: null arguments");
    REQUIRE(b->in0 && b->layers && (b->L <= 0 || b->seg), "d8s_dense_block_pair: null pointer");
    REQUIRE(a->N == b->N && a->H == b->H && a->W == b->W && a->G0 == b->G0 && a->L == b->L,
            "d8s_dense_block_pair: the two problems differ in shape");
    return dblock_launch(a, b, (hipStream_t)stream);
}

// The shape checks of d8s_dense_block_parts (H, W, groups read by the last layer, bands per image):
// nullptr if it runs, else the reason; *shm = its dynamic LDS bytes.
static const char* parts_shape(int H, int W, int G, int parts, size_t* shm) {
    if (H < 1 || W < 1 || G < 1 || parts < 1) return "H, W, groups and parts must be >= 1";
    if (H % parts) return "H must be a multiple of parts";
    const int R = H / parts, P = R * W;
    if (P != 32 && P != 64 && P != 128 && P != 256) return "(H / parts) * W must be 32, 64, 128 or 256 pixels";
    if (G > 64) return "more than 64 groups";
    // the band's window (R + 2 rows of W + 2 pixels, 4 planes), the layer tables, the prologue tables
    const size_t dyn = (size_t)(R + 2) * (W + 2) * 128 + DB_PRM + (size_t)G * 128;
    const size_t stat = P == 32 ? DpShape<1>::STATIC : P == 64 ? DpShape<2>::STATIC
                      : P == 128 ? DpShape<4>::STATIC : DpShape<8>::STATIC;
    if (dyn + stat > 160 * 1024) return "band too large for LDS";
    if (shm) *shm = dyn;
    return nullptr;
}

extern "C" int d8s_parts_supported(int32_t H, int32_t W, int32_t G, int32_t parts) {
    return parts_shape(H, W, G, parts, nullptr) == nullptr ? 1 : 0;
}

extern "C" int d8s_dense_block_parts(const D8sPartsArgs* a, void* stream) {
    REQUIRE(a != nullptr, "d8s_dense_block_parts: null arguments");
    REQUIRE(a->in0 && a->seg && a->layers && a->sync && a->xchg, "d8s_dense_block_parts: null pointer");
    REQUIRE(a->G0 >= 1 && a->L >= 1 && a->N >= 1 && a->H >= 1 && a->W >= 1 && a->parts >= 1,
            "d8s_dense_block_parts: G0, L, N, H, W, parts must be >= 1");
    size_t shm = 0;
    const char* why = parts_shape(a->H, a->W, a->G0 + a->L - 1, a->parts, &shm);
    REQUIRE(why == nullptr, std::string("d8s_dense_block_parts: ") + (why ? why : ""));
    REQUIRE((int64_t)a->N * a->parts < (1 << 24), "d8s_dense_block_parts: too many parts");
    REQUIRE((int64_t)a->N * a->H * a->W * 32 < (1ll << 31), "d8s_dense_block_parts: store slot over 2 GiB");
    REQUIRE(a->parts <= cu_count(), "d8s_dense_block_parts: more bands per image than compute units");
    const int P = (a->H / a->parts) * a->W;
    // the LDS check above counts DpShape<PT>::STATIC bytes of static LDS: make sure the compiled kernel
    // uses no more (checked once per band size)
    {
        static int checked[9] = {0};
        const int PT = P / 32;
        if (!checked[PT]) {
            hipFuncAttributes at{};
            const void* fn = PT == 1 ? (const void*)k_dparts<1> : PT == 2 ? (const void*)k_dparts<2>
                           : PT == 4 ? (const void*)k_dparts<4> : (const void*)k_dparts<8>;
            const size_t want = PT == 1 ? DpShape<1>::STATIC : PT == 2 ? DpShape<2>::STATIC
                              : PT == 4 ? DpShape<4>::STATIC : DpShape<8>::STATIC;
            const hipError_t e = hipFuncGetAttributes(&at, fn);
            if (e != hipSuccess) return fail((int)e, std::string("d8s_dense_block_parts: ") + hipGetErrorString(e));
            REQUIRE(at.sharedSizeBytes <= want, "d8s_dense_block_parts: the kernel's static LDS exceeds its estimate");
            checked[PT] = 1;
        }
    }
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(a->N * a->parts));
    switch (P / 32) {
        case 1: hipLaunchKernelGGL(k_dparts<1>, grid, dim3(DP_NT), shm, st, *a); break;
        case 2: hipLaunchKernelGGL(k_dparts<2>, grid, dim3(DP_NT), shm, st, *a); break;
        case 4: hipLaunchKernelGGL(k_dparts<4>, grid, dim3(DP_NT), shm, st, *a); break;
        default: hipLaunchKernelGGL(k_dparts<8>, grid, dim3(DP_NT), shm, st, *a); break;
    }
    return launched("d8s_dense_block_parts");
}

template <int NT, int PT, int D, int WB>
static int trans_launch_d(const D8sGemmArgs* a, const D8sGemmArgs* b, hipStream_t st) {
    REQUIRE((int64_t)a->N * a->HW < (1ll << 31) && (int64_t)a->N * a->G0 * a->HW * 32 < (1ll << 32) &&
            (int64_t)a->N * a->HW * 32 < (1ll << 32), "d8s_transition: too many pixels");
    const int64_t NO = (int64_t)a->N * (a->HW / 4);
    const int64_t blocks = (NO + 32 * PT - 1) / (32 * PT);
    const size_t shm = (size_t)2 * 2 * 32 * PT * 32 + (size_t)a->G * 128;
    const int np = b ? 2 : 1;
    hipLaunchKernelGGL((k_trans<NT, PT, D, WB>), dim3((unsigned)(blocks * np)), dim3(256), shm, st, *a,
                       b ? *b : *a, (int)blocks);
    return launched("d8s_transition");
}

// Transition variants (d8s_transition_as), activation prefetch depth D (groups ahead; D divides the
// group count) and weight register sets WB (groups of weights ahead): 1 D 4 WB 2 (G a multiple of 4),
// 2 D 4 WB 4 (G a multiple of 4, 4 or 5 output tiles per wave), 3 D 2 WB 2 (G even), 4 D 1 WB 1.  0
// (the launches' own choice): D 2 WB 2 where G is even, else D 1.  Measured per transition of the
// 512-px encoder (each variant's launches replayed back to back, three rounds on one box): 128 x 128
// (G 8) 89-91 against 95-103 us with D 4 at 96 images, 22.7-23.1 against 25.4-26.7 us at 24; 64 x 64
// (G 16) 47.6-48.0 against 50.1-51.0 and 16.2 against 17.3-17.4 us; 32 x 32 (G 40) 51.6-51.9 against
// 51.3-52.2 us at 96 and 23.8-23.9 against 23.8 us at 24 images, where four weight sets took 25.0 us.
static int trans_variant(const D8sGemmArgs* a, const D8sGemmArgs* b, int variant) {
    (void)b;
    const int nt = (a->cout / 32 + 3) / 4;                 // output tiles per wave
    switch (variant) {
        case 0: return a->G % 2 == 0 ? 3 : 4;
        case 1: return a->G % 4 == 0 ? 1 : -1;
        case 2: return a->G % 4 == 0 && (nt == 4 || nt == 5) ? 2 : -1;
        case 3: return a->G % 2 == 0 ? 3 : -1;
        case 4: return 4;
        default: return -1;
    }
}

template <int NT, int PT>
static int trans_launch(const D8sGemmArgs* a, const D8sGemmArgs* b, hipStream_t st, int variant) {
    const int v = trans_variant(a, b, variant);
    REQUIRE(v >= 1, "d8s_transition: variant " + std::to_string(variant) + " is not taken for this shape");
    if constexpr (NT == 4 || NT == 5)
        if (v == 2) return trans_launch_d<NT, PT, 4, 4>(a, b, st);
    if (v == 1) return trans_launch_d<NT, PT, 4, 2>(a, b, st);
    if (v == 3) return trans_launch_d<NT, PT, 2, 2>(a, b, st);
    return trans_launch_d<NT, PT, 1, 1>(a, b, st);
}

static int check_trans(const D8sGemmArgs* a, const char* what) {
    if (int rc = check_gemm(a, what)) return rc;
    REQUIRE(a->out != nullptr, std::string(what) + ": null output");
    REQUIRE(a->cout >= 32 && a->cout % 32 == 0 && a->cout <= 1024,
            std::string(what) + ": cout must be a multiple of 32 in [32, 1024]");
    REQUIRE(a->G0n == a->cout / 32, std::string(what) + ": G0n != cout / 32");
    REQUIRE(a->W % 2 == 0 && (a->HW / a->W) % 2 == 0, std::string(what) + ": H and W must be even");
    return 0;
}

static int trans_dispatch(const D8sGemmArgs* a, const D8sGemmArgs* b, hipStream_t st, int variant) {
    switch ((a->cout / 32 + 3) / 4) {                      // output tiles per wave
        case 1: return trans_launch<1, 4>(a, b, st, variant);
        case 2: return trans_launch<2, 2>(a, b, st, variant);
        case 3: return trans_launch<3, 1>(a, b, st, variant);
        case 4: return trans_launch<4, 1>(a, b, st, variant);
        case 5: return trans_launch<5, 1>(a, b, st, variant);
        case 6: return trans_launch<6, 1>(a, b, st, variant);
        default: return trans_launch<8, 1>(a, b, st, variant);
    }
}

extern "C" int d8s_transition(const D8sGemmArgs* a, void* stream) {
    if (int rc = check_trans(a, "d8s_transition")) return rc;
    return trans_dispatch(a, nullptr, (hipStream_t)stream, 0);
}

extern "C" int d8s_transition_variant(const D8sGemmArgs* a, int32_t variant) {
    if (a == nullptr || check_trans(a, "d8s_transition_variant") != 0) return -1;
    return trans_variant(a, nullptr, variant);
}

extern "C" int d8s_transition_as(const D8sGemmArgs* a, int32_t variant, void* stream) {
    if (int rc = check_trans(a, "d8s_transition_as")) return rc;
    return trans_dispatch(a, nullptr, (hipStream_t)stream, variant);
}

extern "C" int d8s_transition_pair(const D8sGemmArgs* a, const D8sGemmArgs* b, void* stream) {
    if (int rc = check_trans(a, "d8s_transition_pair")) return rc;
    if (int rc = check_trans(b, "d8s_transition_pair")) return rc;
    REQUIRE(same_gemm(a, b), "d8s_transition_pair: the two problems differ in shape");
    return trans_dispatch(a, b, (hipStream_t)stream, 0);
}

static int final_launch(const int8_t* in0, int32_t G0, const int8_t* seg, int32_t N, int32_t HW,
                        const float* ab, float* out, int32_t ctot, const uint32_t* status, uint32_t* report,
                        void* stream, const char* what) {
    REQUIRE(in0 && ab && out, std::string(what) + ": null pointer");
    REQUIRE(G0 >= 1 && N >= 1 && HW >= 1 && ctot >= 32 * G0 && ctot % 32 == 0,
            std::string(what) + ": bad sizes (G0, N, HW >= 1, ctot a multiple of 32 and >= 32 G0)");
    REQUIRE(ctot == 32 * G0 || seg != nullptr, std::string(what) + ": seg is null with ctot > 32 G0");
    const int G = ctot / 32;
    hipLaunchKernelGGL(k_final, dim3((unsigned)N, (unsigned)((G + 1) / 2)), dim3(256), 0,
                       (hipStream_t)stream, in0, G0, seg, N, HW, G, ab, out, ctot, status, report);
    return launched(what);
}

extern "C" int d8s_final(const int8_t* in0, int32_t G0, const int8_t* seg, int32_t N, int32_t HW,
                         const float* ab, float* out, int32_t ctot, void* stream) {
    return final_launch(in0, G0, seg, N, HW, ab, out, ctot, nullptr, nullptr, stream, "d8s_final");
}

extern "C" int d8s_final_checked(const int8_t* in0, int32_t G0, const int8_t* seg, int32_t N, int32_t HW,
                                 const float* ab, float* out, int32_t ctot, const uint32_t* status,
                                 uint32_t* report, void* stream) {
    REQUIRE(status != nullptr, "d8s_final_checked: null status word");
    return final_launch(in0, G0, seg, N, HW, ab, out, ctot, status, report, stream, "d8s_final_checked");
}

extern "C" int d8s_host_mapped(void* host, void** dev) {
    REQUIRE(host && dev, "d8s_host_mapped: null pointer");
    const hipError_t e = hipHostGetDevicePointer(dev, host, 0);
    if (e != hipSuccess) return fail((int)e, std::string("d8s_host_mapped: ") + hipGetErrorString(e));
    return 0;
}

extern "C" int d8s_linear(const float* x, int32_t N, int32_t C, const float* w, const float* b, int32_t K,
                          float* out, void* stream) {
    REQUIRE(x && w && b && out, "d8s_linear: null pointer");
    REQUIRE(N >= 1 && C >= 1 && K >= 1 && K <= 4096, "d8s_linear: N, C >= 1 and 1 <= K <= 4096");
    REQUIRE(N < (1 << 30), "d8s_linear: N too large");
    hipLaunchKernelGGL(k_linear, dim3((unsigned)N), dim3(256), 0, (hipStream_t)stream, x, C, w, b, K, out);
    return launched("d8s_linear");
}

static int check_stem(const D8sStemArgs* a, const char* what) {
    const std::string w(what);
    REQUIRE(a != nullptr, w + ": null arguments");
    REQUIRE(a->x && a->w16 && a->bias && a->inv && a->out, w + ": null pointer");
    REQUIRE(a->kind == D8S_IN_F16 || (a->kind == D8S_IN_U8 && a->lut != nullptr),
            w + ": kind must be D8S_IN_F16, or D8S_IN_U8 with a lut");
    REQUIRE(a->N >= 1 && a->H >= 4 && a->W >= 4 && a->H % 4 == 0 && a->W % 4 == 0,
            w + ": H and W must be positive multiples of 4");
    REQUIRE(a->kind != D8S_IN_U8 || ((uintptr_t)a->x & 3) == 0, w + ": uint8 input not 4-byte aligned");
    REQUIRE(a->flip >= 0 && a->flip <= 2 && (a->flip != 2 || a->N % 2 == 0),
            w + ": flip must be 0, 1, or 2 (TTA pairs, N even)");
    REQUIRE(a->kind != D8S_IN_F16 || a->W > 64 * SR_NWV || ((uintptr_t)a->x & 7) == 0,
            w + ": fp16 input not 8-byte aligned");
    return 0;
}

// (the tile form, for widths past the row-band form's, has no pair launch: a pair runs as two)
static int stem_dispatch(const D8sStemArgs* a, const D8sStemArgs* b, hipStream_t st) {
    const int Hp = a->H / 4, Wp = a->W / 4;
    if (a->W <= 64 * SR_NWV && (int64_t)(a->flip == 2 ? a->N / 2 : a->N) * 3 * a->H * a->W < (1ll << 31)) {
        // row bands: one wave per 32 conv columns, one workgroup per CU; the band height is the least
        // of rounds x (rows + 1) over 2 .. 16 pooled rows (a band's first pooled row also needs the
        // conv row above it; ties go to the taller band): 16 rows at 96 images of 512 px (768 bands,
        // three rounds), 13 at 24 (240 bands in one round instead of 192 of 16 rows)
        const int np = b ? 2 : 1;
        const int nwv = (a->W / 2 + 31) / 32;
        int rows = 16;
        {
            int64_t best = -1;
            for (int r = 16; r >= 2; --r) {
                const int64_t nb = (int64_t)a->N * np * ((Hp + r - 1) / r);
                const int64_t cost = (nb + cu_count() - 1) / cu_count() * (r + 1);
                if (best < 0 || cost < best) { best = cost; rows = r; }
            }
        }
        const int bands = (Hp + rows - 1) / rows;
        const int64_t blocks = (int64_t)a->N * bands;      // per problem
        REQUIRE(blocks * np < (1ll << 31), "d8s_stem: too many bands");
        if (a->kind == D8S_IN_U8)
            hipLaunchKernelGGL(k_stem_rows<true>, dim3((unsigned)(blocks * np)), dim3(64 * nwv), SR_LDS, st,
                               *a, bands, rows, b ? *b : *a, (int)blocks);
        else
            hipLaunchKernelGGL(k_stem_rows<false>, dim3((unsigned)(blocks * np)), dim3(64 * nwv), SR_LDS, st,
                               *a, bands, rows, b ? *b : *a, (int)blocks);
        return launched("d8s_stem");
    }
    if (b) {
        if (int rc = stem_dispatch(a, nullptr, st)) return rc;
        return stem_dispatch(b, nullptr, st);
    }
    const int tiles_x = (Wp + ST_PX - 1) / ST_PX, tiles_y = (Hp + ST_PY - 1) / ST_PY;
    const int64_t blocks = (int64_t)a->N * tiles_x * tiles_y;
    REQUIRE(blocks < (1ll << 31), "d8s_stem: too many tiles");
    hipLaunchKernelGGL(k_stem, dim3((unsigned)blocks), dim3(256), 0, st, *a, tiles_x, tiles_y);
    return launched("d8s_stem");
}

extern "C" int d8s_stem(const D8sStemArgs* a, void* stream) {
    if (int rc = check_stem(a, "d8s_stem")) return rc;
    return stem_dispatch(a, nullptr, (hipStream_t)stream);
}

extern "C" int d8s_stem_pair(const D8sStemArgs* a, const D8sStemArgs* b, void* stream) {
    if (int rc = check_stem(a, "d8s_stem_pair")) return rc;
    if (int rc = check_stem(b, "d8s_stem_pair")) return rc;
    REQUIRE(a->N == b->N && a->H == b->H && a->W == b->W && a->kind == b->kind && a->flip == b->flip,
            "d8s_stem_pair: the two problems differ in shape, input kind or flip");
    return stem_dispatch(a, b, (hipStream_t)stream);
}

extern "C" const char* d8s_version(void) {
    static const std::string v = std::string("d8s-hip ") + std::to_string(D8S_ABI_VERSION) + " " +
                                 D8S_SRC_HASH + " gfx950";
    return v.c_str();
}

extern "C" const char* d8s_last_error(void) { return g_err.c_str(); }

extern "C" int d8s_micro_copy(const void* src, void* dst, size_t bytes, void* stream) {
    REQUIRE(src && dst && bytes % 16 == 0, "d8s_micro_copy: null pointer or size not a multiple of 16");
    const int64_t n = (int64_t)(bytes / 16);
    const int64_t want = (n + 1023) / 1024;
    const unsigned grid = (unsigned)(want < 8 * cu_count() ? (want > 0 ? want : 1) : 8 * cu_count());
    hipLaunchKernelGGL(k_copy, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)src,
                       (u32x4*)dst, n);
    return launched("d8s_micro_copy");
}

extern "C" int d8s_micro_mfma(int32_t blocks, int32_t iters, int32_t* sink, void* stream) {
    REQUIRE(sink && blocks >= 1 && iters >= 1, "d8s_micro_mfma: bad arguments");
    hipLaunchKernelGGL(k_mfma_loop, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, iters,
                       sink);
    return launched("d8s_micro_mfma");
}

extern "C" int d8s_probe_mfma_i8(const int8_t* A, const int8_t* B, int32_t* D, void* stream) {
    REQUIRE(A && B && D, "d8s_probe_mfma_i8: null pointer");
    hipLaunchKernelGGL(k_probe_i8, dim3(1), dim3(64), 0, (hipStream_t)stream, A, B, D);
    return launched("d8s_probe_mfma_i8");
}

extern "C" int d8s_probe_mfma_f16(const uint16_t* A, const uint16_t* B, float* D, void* stream) {
    REQUIRE(A && B && D, "d8s_probe_mfma_f16: null pointer");
    hipLaunchKernelGGL(k_probe_f16, dim3(1), dim3(64), 0, (hipStream_t)stream, A, B, D);
    return launched("d8s_probe_mfma_f16");
}
