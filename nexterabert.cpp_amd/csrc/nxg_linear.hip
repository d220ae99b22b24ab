// nxg_linear.hip -- gfx950 kernels of the int8 linear path and their C ABI.
//
//   quantize_kernel  f32 rows -> int8 fragment tiles + per-(token, 256-block) scales
//                    (the reference's quantize_row, src/nexterabert.cpp:378-403)
//   gemm_kernel      v_mfma_i32_16x16x64_i8 GEMM; per 256-input block the int32 tile is
//                    folded into fp32 accumulators with the reference's epilogue
//                    f = fma((float) s * sx, sw, f) (src/nexterabert.cpp:909-916,957-958)
//   export_kernel    int8 tiles -> the reference's u8 row layout
//
// Data layouts are described in include/nxg_linear.h. Weights are re-laid out once,
// at upload, into the same fragment tiles as the activations, so that every copy
// into LDS is a straight 1 KiB run and every LDS read is one conflict-free
// ds_read_b128 per lane.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "nxg_linear.h"
#include "nxg_internal.h"
#include "nxg_gemm_plan.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define NXG_ATTN_MAX_KEYS 16384          // keys per query the attention's LDS holds (64 KiB)

namespace {

// tiles, fragments, the tile walk, the operand and output addresses, the launch plan
using namespace nxg_gemm;

// ---------------------------------------------------------------------------
// quantize
// ---------------------------------------------------------------------------

// The reference folds |x| with MAXPS (dst = a > b ? a : b, so a NaN operand
// yields the second operand) over 8 lanes, lane j seeing elements j, j+8, ...
// The result of such a fold over a sequence S is described by (nan, tail):
//   nan   S contains a NaN
//   tail  the fold's result from any start value: max(S) without NaN, else the
//         max of the elements after the last NaN (NaN if the NaN is last).
// Folding A then B gives  B.nan ? B.tail : (A.tail is NaN ? B.tail : max(A.tail, B.tail)),
// an associative combination, so lanes can be reduced in a tree as long as the
// earlier part stays on the left.
struct fold {
    float tail;
    int   flags;   // bit 0: contains NaN, bit 1: empty
};

__device__ __forceinline__ float maxps1(float a, float b) { return a > b ? a : b; }

__device__ __forceinline__ fold fold_elem(float a) {
    fold r;
    r.tail = a;
    r.flags = __builtin_isnan(a) ? 1 : 0;
    return r;
}

__device__ __forceinline__ fold fold_join(fold a, fold b) {
    if (b.flags & 2) return a;
    if (a.flags & 2) return b;
    fold r;
    r.flags = (a.flags | b.flags) & 1;
    r.tail = ((b.flags & 1) || __builtin_isnan(a.tail)) ? b.tail : fmaxf(a.tail, b.tail);
    return r;
}

__device__ __forceinline__ float abs_bits(float x) {
    return __uint_as_float(__float_as_uint(x) & 0x7fffffffu);
}

// CVTPS2DQ (round to nearest even; NaN or out of int32 range -> 0x80000000),
// + ACT_OFF with 32-bit wrap-around, then signed-16 and unsigned-8 saturation
// (PACKSSDW, PACKUSWB), minus ACT_OFF: the reference's u8 as a signed value.
template <int ACT_MAX>
__device__ __forceinline__ int quant1(float x, float inv) {
    const float y = x * inv;
    int c;
    if (__builtin_isnan(y) || !(fabsf(y) < 2147483648.0f)) {
        c = INT32_MIN;
    } else {
        c = (int) __builtin_rintf(y);
    }
    const int cw = (int) ((unsigned) c + (unsigned) (ACT_MAX + 1));
    const int u = min(max(cw, 0), 255);
    return u - (ACT_MAX + 1);
}

// Row sources of quantize_row: what a producer hands to for_rows' quantize branch
// (src/nexterabert.cpp:414-438). A source has a per-row state row(t) (computed once per
// row and lane) and load(rs, t, col, v): the 4 f32 values of row t at inputs col..col+3
// (t < T, col + 3 < n_in), computed with the producer's own operations in its order.

struct no_row {};

// op_copy (:453-461) and any f32 rows handed over as they are.
struct src_rows {
    const float * x;
    int n;
    __device__ no_row row(int) const { return {}; }
    __device__ void load(no_row, int t, int col, float (&v)[4]) const {
        const v4f f = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(x + (size_t) t * n + col));
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    }
};

// op_relu_sqr (:484-505): r = x > 0 ? x : 0 (MAXPS with zero second: a NaN gives 0), r * r.
struct src_relu2 {
    src_rows in;
    __device__ no_row row(int) const { return {}; }
    __device__ void load(no_row, int t, int col, float (&v)[4]) const {
        in.load({}, t, col, v);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = v[e] > 0.0f ? v[e] : 0.0f;
            v[e] = r * r;
        }
    }
};

// op_rms_norm (:463-482) once the row's inv = 1 / sqrt(mean(x^2) + eps) is known:
// (x * inv) * gain.
struct src_rms {
    src_rows in;
    const float * gain;
    float inv;
    __device__ no_row row(int) const { return {}; }
    __device__ void load(no_row, int t, int col, float (&v)[4]) const {
        in.load({}, t, col, v);
        const v4f gv = *reinterpret_cast<const v4f *>(gain + col);
        const float gr[4] = { gv.x, gv.y, gv.z, gv.w };
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (v[e] * inv) * gr[e];
    }
};

// quantize_row (src/nexterabert.cpp:378-403) of one row's 256-input block on a 16-lane group,
// lane c = lane % 16 holding inputs 64i + 4c + e (i, e = 0..3) in xv[i][e] (0 where
// !present[i]; a padding row, row_ok false, is all 0). Returns the block's amax; packed[i]
// gets input 64i + 4c + e at byte e: the reference's u8 minus ACT_OFF, as a signed byte (0
// where !present[i]). amax reproduces MAXPS: a plain maximum when the wave holds no NaN,
// otherwise the ordered fold (nan, tail) over the 8 AVX lanes and the reference's horizontal
// tree. The conversion is CVTPS2DQ (RNE; NaN or out of int32 range -> 0x80000000), + ACT_OFF
// with 32-bit wrap, then the two saturating packs (quant1); when the wave holds no NaN and
// every amax and inv = ACT_MAX / amax of it is finite, |x * inv| <= ACT_MAX + 1/2 and that
// reduces to rint(x * inv) + ACT_OFF packed by v_cvt_pk_u8_f32, which this path uses.
template <int ACT_MAX>
__device__ __forceinline__ float quantize_group16(const float (&xv)[4][4], const bool (&present)[4], bool row_ok,
                                                  int c, int (&packed)[4]) {
    bool any_nan = false;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) any_nan |= __builtin_isnan(xv[i][e]);
    const bool wave_nan = __any(any_nan);

    float amax;
    if (!wave_nan) {
        // No NaN in this wave: the fold is the plain maximum.
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) m = fmaxf(m, abs_bits(xv[i][e]));
#pragma unroll
        for (int sft = 1; sft < 16; sft <<= 1) m = fmaxf(m, __shfl_xor(m, sft));
        amax = m;
    } else {
        // Exact MAXPS semantics. Input k of the block is AVX lane k % 8 at position k / 8; for
        // this lane k = 64i + 4c + e: AVX lane 4(c%2) + e, position 8i + c/2. Fold the
        // 8 lanes of one parity for each i (ordered by c/2), then the four i in order.
        fold acc[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) { acc[e].tail = 0.0f; acc[e].flags = 2; }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                fold fi;
                if (present[i]) {
                    fi = fold_elem(abs_bits(xv[i][e]));
                } else {
                    fi.tail = 0.0f;
                    fi.flags = 2;
                }
#pragma unroll
                for (int sft = 2; sft < 16; sft <<= 1) {
                    fold o;
                    o.tail = __shfl_xor(fi.tail, sft);
                    o.flags = __shfl_xor(fi.flags, sft);
                    fi = (c & sft) ? fold_join(o, fi) : fold_join(fi, o);
                }
                acc[e] = fold_join(acc[e], fi);
            }
        }
        // acc[e] is AVX lane 4(c%2) + e. The reference's horizontal tree: lanes
        // (j, j+4), then (0,2), (1,3), then (0,1).
        float m[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float other = __shfl_xor(acc[e].tail, 1);
            m[e] = (c & 1) ? maxps1(other, acc[e].tail) : maxps1(acc[e].tail, other);
        }
        amax = maxps1(maxps1(m[0], m[2]), maxps1(m[1], m[3]));
        if (!row_ok) amax = 0.0f;
    }

    const float inv = amax > 0.0f ? (float) ACT_MAX / amax : 0.0f;
    const bool fast = __builtin_amdgcn_ballot_w64(wave_nan || !(amax < INFINITY) || !(inv < INFINITY)) == 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int v = 0;
        if (present[i]) {
            if (fast) {
                unsigned u = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_rintf(xv[i][0] * inv) + (float) (ACT_MAX + 1), 0, 0u);
                u = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_rintf(xv[i][1] * inv) + (float) (ACT_MAX + 1), 1, u);
                u = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_rintf(xv[i][2] * inv) + (float) (ACT_MAX + 1), 2, u);
                u = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_rintf(xv[i][3] * inv) + (float) (ACT_MAX + 1), 3, u);
                // u8 - ACT_OFF per byte: ACT_OFF = ACT_MAX + 1 is 128 or 64
                v = ACT_MAX == 127 ? (int) (u ^ 0x80808080u) : (int) (((u | 0x80808080u) - 0x40404040u) ^ 0x80808080u);
            } else {
                v = (quant1<ACT_MAX>(xv[i][0], inv) & 0xff) | ((quant1<ACT_MAX>(xv[i][1], inv) & 0xff) << 8)
                  | ((quant1<ACT_MAX>(xv[i][2], inv) & 0xff) << 16) | ((quant1<ACT_MAX>(xv[i][3], inv) & 0xff) << 24);
            }
        }
        packed[i] = v;
    }
    return amax;
}

// quantize_row of one (16-row group g, 256-input block B) by a workgroup of 4 waves.
// Wave w quantizes rows 4w..4w+3; the 16 lanes of a row read its 256 inputs as 4
// contiguous 256-byte pieces, so lane c holds inputs 64i + 4c + e (i, e = 0..3). The
// int8 results are gathered in LDS in fragment order and each wave stores one 1 KiB
// fragment. Ends with the stage buffer still being read by the stores: callers looping
// over blocks sync before reuse.
template <int ACT_MAX, typename Src>
__device__ __forceinline__ void quantize_block(const Src & src, int T, int n_in, int KS, int n_blk,
                                               int8_t * __restrict__ q, float * __restrict__ sx, int g, int B,
                                               int * stage) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rl = wave * 4 + (lane >> 4);     // row within the 16-row group
    const int t = g * 16 + rl;
    const int c = lane & 15;
    const int kb = B * BLK;                    // first input of the block

    float xv[4][4];                            // [i][e]: input kb + 64i + 4c + e
    bool present[4];
    const auto rs = src.row(min(t, T - 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        present[i] = t < T && kb + 64 * i + 4 * c < n_in;
        if (present[i]) {
            src.load(rs, t, kb + 64 * i + 4 * c, xv[i]);
        } else {
            xv[i][0] = xv[i][1] = xv[i][2] = xv[i][3] = 0.0f;
        }
    }
    int packed[4];
    const float amax = quantize_group16<ACT_MAX>(xv, present, t < T, c, packed);
    const float scale = amax / (float) ACT_MAX;

    // Place in LDS: input kb + 64i + 4c + e goes to fragment i, lane rl + 16 (c/4), byte
    // 4 (c%4) + e. Padding (absent inputs, rows >= T) is 0.
#pragma unroll
    for (int i = 0; i < 4; ++i) stage[(i * FRAG + (rl + 16 * (c >> 2)) * 16) / 4 + (c & 3)] = packed[i];
    if (c == 0) {
        sx[((size_t) (t >> 2) * n_blk + B) * 4 + (t & 3)] = t < T ? scale : 0.0f;
    }
    __syncthreads();
    // wave w stores fragment w of the block (k-step 4B + w), if it exists
    const int ks = 4 * B + wave;
    if (ks < KS) {
        const int4 v = reinterpret_cast<const int4 *>(stage)[wave * 64 + lane];
        *reinterpret_cast<int4 *>(q + ((size_t) g * KS + ks) * FRAG + lane * 16) = v;
    }
}

// One workgroup per (16-row group, 256-input block), the block index fastest, so that
// consecutive workgroups read consecutive 1 KiB pieces of the same rows.
enum qmode { Q_PLAIN = 0, Q_RELU2 = 1 };
template <int ACT_MAX, int MODE>
__global__ __launch_bounds__(256) void quantize_kernel(const float * __restrict__ x, int T, int n_in, int KS,
                                                       int n_blk, int8_t * __restrict__ q, float * __restrict__ sx) {
    __shared__ __attribute__((aligned(16))) int stage[4 * FRAG / 4];
    const int g = (int) (blockIdx.x / (unsigned) n_blk), B = (int) (blockIdx.x % (unsigned) n_blk);
    const src_rows in{x, n_in};
    if (MODE == Q_RELU2) quantize_block<ACT_MAX>(src_relu2{in}, T, n_in, KS, n_blk, q, sx, g, B, stage);
    else                 quantize_block<ACT_MAX>(in, T, n_in, KS, n_blk, q, sx, g, B, stage);
}

// The end of dot_f32 (src/nexterabert.cpp:124-149) on the 16 lanes c = 0..15 of a lane
// group, lane c holding the sums of chains 2c (a0) and 2c + 1 (a1): (s0 + s1) + (s2 + s3)
// lane-wise (chains 8k + j are accumulator s_k, lane j), then hsum256: lanes j and j+4, then
// 0+2 and 1+3, then those two. fp32 addition is commutative, so both lanes of a shuffle pair
// get the same bits and every lane of the group returns the dot.
__device__ __forceinline__ float dot_tree16(float a0, float a1) {
    // lane c holds s_k[j], s_k[j+1] with k = c/4, j = 2(c%4)
    a0 = a0 + __shfl_xor(a0, 4);               // s0 + s1, s2 + s3
    a1 = a1 + __shfl_xor(a1, 4);
    a0 = a0 + __shfl_xor(a0, 8);               // v[j] = (s0 + s1) + (s2 + s3)
    a1 = a1 + __shfl_xor(a1, 8);
    a0 = a0 + __shfl_xor(a0, 2);               // v[j] + v[j+4]: lanes q and q^2 (q = c%4)
    a1 = a1 + __shfl_xor(a1, 2);
    a0 = a0 + __shfl_xor(a0, 1);               // (v0+v4) + (v2+v6), (v1+v5) + (v3+v7)
    a1 = a1 + __shfl_xor(a1, 1);
    return a0 + a1;
}

// dot_f32(x, x) over a row of n floats (n % 32 == 0) in the reference's AVX2 order
// (src/nexterabert.cpp:124-149), on the 16 lanes c = 0..15 of a lane group (xr null: the
// row does not exist, the lanes still join the shuffles). 32 FMA chains, chain a taking
// elements 32m + a (lane c runs chains 2c and 2c+1), then dot_tree16.
__device__ __forceinline__ float dot_sq_ref16(const float * xr, int n, int c) {
    float a0 = 0.0f, a1 = 0.0f;                // chains 2c and 2c + 1
    if (xr) {
        xr += 2 * c;
        for (int m = 0; m < n / 32; ++m) {
            const float2 v = *reinterpret_cast<const float2 *>(xr + 32 * m);
            a0 = __builtin_fmaf(v.x, v.x, a0);
            a1 = __builtin_fmaf(v.y, v.y, a1);
        }
    }
    return dot_tree16(a0, a1);
}

// op_rms_norm feeding an int8 linear (src/nexterabert.cpp:463-482 through for_rows'
// quantize_row, :414-438): one workgroup per (16-row group, block), 16 lanes per row. Each row's
// dot_f32(x, x) in the reference's order (dot_sq_ref16), inv = 1 / sqrt(dot / C + eps)
// correctly rounded, then every block re-read and quantized as (x * inv) * gain. C % 32
// == 0, so the reference's remainder loops never run.
template <int ACT_MAX>
__global__ __launch_bounds__(256) void rmsnorm_quantize_kernel(const float * __restrict__ x, const float * __restrict__ gain,
                                                               float eps, int T, int n_in, int KS, int n_blk,
                                                               int8_t * __restrict__ q, float * __restrict__ sx) {
    __shared__ __attribute__((aligned(16))) int stage[4 * FRAG / 4];
    // workgroup b runs on XCD b % 8: the n_blk workgroups of one row group share an XCD
    // (and its L2, which serves their repeated reads of the rows for the dot)
    const int xcd = (int) (blockIdx.x & 7u), slot = (int) (blockIdx.x >> 3);
    const int g = (slot / n_blk) * 8 + xcd, B = slot % n_blk;
    if (g * 16 >= T) return;                   // the padding of the grid to whole XCD rounds
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = g * 16 + wave * 4 + (lane >> 4);
    const int c = lane & 15;
    const float dot = dot_sq_ref16(t < T ? x + (size_t) t * n_in : nullptr, n_in, c);
    const float inv = 1.0f / __builtin_sqrtf(dot / (float) n_in + eps);
    quantize_block<ACT_MAX>(src_rms{src_rows{x, n_in}, gain, inv}, T, n_in, KS, n_blk, q, sx, g, B, stage);
}

// The same op for n_in = 256 NB with the whole row group in registers: one workgroup per
// 16-row group, 16 lanes per row; lane c holds inputs 32m + 2c and 32m + 2c + 1 for every m,
// exactly what the reference's dot chains 2c and 2c + 1 consume (dot_sq_ref16's order), so
// each input is read from HBM once. Every block is then quantized from those registers:
// amax over the row's 16 lanes, quant1, and the int8 pairs gathered in LDS in fragment
// order (input kb + 32m' + 2c + e goes to k-step 4B + m'/2, piece row + 16 (kq / 16), byte
// kq % 16, kq = 32 (m' % 2) + 2c + e), then each wave stores whole 1 KiB fragments. A
// NaN anywhere in the group's normalized values sends the group through quantize_block,
// whose fold gives the reference's MAXPS result; without NaN that fold is the plain max.
// SPLIT (few rows): one workgroup per (row group, block), the dot still over the whole row
// from registers, only one block quantized and stored -- NB times the workgroups for
// launches too small to fill the device. Workgroup b runs on XCD b % 8, so the NB
// workgroups of a row group are given the same b % 8 and share that XCD's L2 for the rows
// they all read (the grid is padded to whole rounds of 8 row groups).
template <int ACT_MAX, int NB, bool SPLIT>
__global__ __launch_bounds__(256) void rmsnorm_q8_kernel(const float * __restrict__ x, const float * __restrict__ gain,
                                                         float eps, int T, int8_t * __restrict__ q,
                                                         float * __restrict__ sx) {
    constexpr int n_in = NB * BLK, M = n_in / 32, KS = 4 * NB;
    __shared__ __attribute__((aligned(16))) int stage[KS * FRAG / 4];
    const int xcd = (int) (blockIdx.x & 7u), slot = (int) (blockIdx.x >> 3);
    const int g = SPLIT ? (slot / NB) * 8 + xcd : (int) blockIdx.x;
    const int Bs = SPLIT ? slot % NB : 0;                      // SPLIT: the block of this workgroup
    if (SPLIT && g * 16 >= T) return;                          // padding of the grid to whole rounds
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rl = wave * 4 + (lane >> 4), t = g * 16 + rl, c = lane & 15;
    float2 v[M];
    if (t < T) {
        const float * xr = x + (size_t) t * n_in + 2 * c;
#pragma unroll
        for (int m = 0; m < M; ++m) v[m] = *reinterpret_cast<const float2 *>(xr + 32 * m);
    } else {
#pragma unroll
        for (int m = 0; m < M; ++m) v[m] = float2{ 0.0f, 0.0f };
    }
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        a0 = __builtin_fmaf(v[m].x, v[m].x, a0);
        a1 = __builtin_fmaf(v[m].y, v[m].y, a1);
    }
    const float dot = dot_tree16(a0, a1);
    const float inv = 1.0f / __builtin_sqrtf(dot / (float) n_in + eps);
    bool nan = false;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float2 gv = *reinterpret_cast<const float2 *>(gain + 32 * m + 2 * c);
        v[m].x = (v[m].x * inv) * gv.x;
        v[m].y = (v[m].y * inv) * gv.y;
        nan |= __builtin_isnan(v[m].x) || __builtin_isnan(v[m].y);
    }
    if (__syncthreads_or(nan)) {
        const src_rms src{src_rows{x, n_in}, gain, inv};
        for (int B = 0; B < NB; ++B) {
            if (SPLIT && B != Bs) continue;
            quantize_block<ACT_MAX>(src, T, n_in, KS, NB, q, sx, g, B, stage);
            __syncthreads();
        }
        return;
    }
    unsigned short * st16 = reinterpret_cast<unsigned short *>(stage);
#pragma unroll
    for (int B = 0; B < NB; ++B) {
        if (SPLIT && B != Bs) continue;
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fmaxf(abs_bits(v[8 * B + i].x), abs_bits(v[8 * B + i].y)));
#pragma unroll
        for (int sft = 1; sft < 16; sft <<= 1) amax = fmaxf(amax, __shfl_xor(amax, sft));
        const float scale = amax / (float) ACT_MAX;
        const float qinv = amax > 0.0f ? (float) ACT_MAX / amax : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kq = 32 * (i & 1) + 2 * c;
            const int pair = (quant1<ACT_MAX>(v[8 * B + i].x, qinv) & 0xff) | ((quant1<ACT_MAX>(v[8 * B + i].y, qinv) & 0xff) << 8);
            st16[((4 * B + (i >> 1)) * FRAG + (rl + 16 * (kq >> 4)) * 16 + (kq & 15)) / 2] = (unsigned short) pair;
        }
        if (c == 0) sx[((size_t) (t >> 2) * NB + B) * 4 + (t & 3)] = t < T ? scale : 0.0f;
    }
    __syncthreads();
    if (SPLIT) {
        const int f = 4 * Bs + wave;                       // wave w stores fragment w of the block
        const int4 w = reinterpret_cast<const int4 *>(stage)[f * 64 + lane];
        *reinterpret_cast<int4 *>(q + ((size_t) g * KS + f) * FRAG + lane * 16) = w;
        return;
    }
#pragma unroll
    for (int f = wave; f < KS; f += 4) {
        const int4 w = reinterpret_cast<const int4 *>(stage)[f * 64 + lane];
        *reinterpret_cast<int4 *>(q + ((size_t) g * KS + f) * FRAG + lane * 16) = w;
    }
}

// ---------------------------------------------------------------------------
// Mixer producers quantizing for an int8 consumer (row_op(..., int8_only(...)))
// ---------------------------------------------------------------------------

__device__ __forceinline__ float minps1(float a, float b) { return a < b ? a : b; }

// exp(x) as the reference's exp256 computes it (src/nexterabert.cpp:81-100), lane by
// lane: clamp to [-87.3, 88.3762626647949] with MINPS/MAXPS semantics (a NaN becomes the
// upper bound); n = x * log2(e) rounded to the nearest integer (ties to even); the
// argument reduced in two fused steps, r = x - n * 0.693359375 - n * (-2.12194440e-4);
// the degree-5 Cephes polynomial in r by fused Horner steps, completed as p * r^2 + (r + 1);
// scaled by 2^n built in the exponent field ((n + 127) << 23).
__device__ __forceinline__ float exp_cephes(float x) {
    constexpr float P[6] = { 1.9875691500e-4f, 1.3981999507e-3f, 8.3334519073e-3f,
                             4.1665795894e-2f, 1.6666665459e-1f, 5.0000001201e-1f };
    x = minps1(x, 88.3762626647949f);
    x = maxps1(x, -87.3f);
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693359375f, x);
    r = __builtin_fmaf(-n, -2.12194440e-4f, r);
    const float r2 = r * r;
    float p = P[0];
#pragma unroll
    for (int i = 1; i < 6; ++i) p = __builtin_fmaf(p, r, P[i]);
    p = __builtin_fmaf(p, r2, r + 1.0f);
    const uint32_t e = (uint32_t) ((int) n + 127) << 23;
    return p * __uint_as_float(e);
}

// op_gate (src/nexterabert.cpp:507-522, AVX2 path; C % 8 == 0): sigmoid(g) * y with
// sigmoid(g) = 1 / (1 + exp(0 - g)), the division correctly rounded.
struct src_gate {
    const float * g;
    const float * y;
    int C;
    __device__ no_row row(int) const { return {}; }
    __device__ void load(no_row, int t, int col, float (&v)[4]) const {
        const size_t o = (size_t) t * C + col;
        const v4f gv = *reinterpret_cast<const v4f *>(g + o);
        const v4f yv = *reinterpret_cast<const v4f *>(y + o);
        const float gr[4] = { gv.x, gv.y, gv.z, gv.w }, yr[4] = { yv.x, yv.y, yv.z, yv.w };
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (1.0f / (1.0f + exp_cephes(0.0f - gr[e]))) * yr[e];
    }
};

// The document of row t in a packed layout given by its cumulative offsets cu[0..n]
// (device): the largest d with cu[d] <= t, and its rows [lo, hi) clamped to [0, T)
// so that any offsets give in-bounds rows.
struct doc_rows {
    int lo, hi, d;
};
__device__ __forceinline__ doc_rows doc_of(const int32_t * cu, int n, int t, int T) {
    int a = 0, b = n - 1;                      // search d in [0, n)
    while (a < b) {
        const int m = (a + b + 1) >> 1;
        if (cu[m] <= t) a = m; else b = m - 1;
    }
    doc_rows r;
    r.d = a;
    r.lo = min(max(cu[a], 0), T);
    r.hi = min(max(cu[a + 1], r.lo), T);
    return r;
}

// op_dwconv (src/nexterabert.cpp:524-543): out = r (or 0), then for every tap j whose
// row t + j - k/2 lies in t's document, out = fma(taps[j], x[t + j - k/2], out) in order
// of j (addmul_f32, :166-176). taps [k][C].
// taps whose rows a convolution source loads before any of its fmas (the models' kernels: 3, 5)
constexpr int TAPS_HOIST = 5;

struct src_dwconv {
    const float * x;
    const float * r;                           // may be null
    const float * taps;
    const int32_t * cu;
    int n_seqs, T, C, k;
    __device__ doc_rows row(int t) const { return doc_of(cu, n_seqs, t, T); }
    __device__ void load(const doc_rows & dr, int t, int col, float (&v)[4]) const {
        if (r) {
            const v4f rv = *reinterpret_cast<const v4f *>(r + (size_t) t * C + col);
            v[0] = rv.x; v[1] = rv.y; v[2] = rv.z; v[3] = rv.w;
        } else {
            v[0] = v[1] = v[2] = v[3] = 0.0f;
        }
        if (k <= TAPS_HOIST) {
            // every tap's row loaded first (rows clamped into the batch, so always in bounds),
            // then the fmas of the taps inside the document in tap order
            v4f w[TAPS_HOIST], xv[TAPS_HOIST];
#pragma unroll
            for (int j = 0; j < TAPS_HOIST; ++j) {
                if (j >= k) break;
                const int tt = min(max(t + j - k / 2, 0), T - 1);
                w[j] = *reinterpret_cast<const v4f *>(taps + (size_t) j * C + col);
                xv[j] = *reinterpret_cast<const v4f *>(x + (size_t) tt * C + col);
            }
#pragma unroll
            for (int j = 0; j < TAPS_HOIST; ++j) {
                const int tt = t + j - k / 2;
                if (j >= k || tt < dr.lo || tt >= dr.hi) continue;
                v[0] = __builtin_fmaf(w[j].x, xv[j].x, v[0]);
                v[1] = __builtin_fmaf(w[j].y, xv[j].y, v[1]);
                v[2] = __builtin_fmaf(w[j].z, xv[j].z, v[2]);
                v[3] = __builtin_fmaf(w[j].w, xv[j].w, v[3]);
            }
            return;
        }
        for (int j = 0; j < k; ++j) {
            const int tt = t + j - k / 2;
            if (tt < dr.lo || tt >= dr.hi) continue;
            const v4f w = *reinterpret_cast<const v4f *>(taps + (size_t) j * C + col);
            const v4f xv = *reinterpret_cast<const v4f *>(x + (size_t) tt * C + col);
            v[0] = __builtin_fmaf(w.x, xv.x, v[0]);
            v[1] = __builtin_fmaf(w.y, xv.y, v[1]);
            v[2] = __builtin_fmaf(w.z, xv.z, v[2]);
            v[3] = __builtin_fmaf(w.w, xv.w, v[3]);
        }
    }
};

// op_lily_state (src/nexterabert.cpp:545-578, AVX2 path): acc = 0; for the taps j whose
// row t + j - k/2 lies in t's document, acc = fma(taps[j], a[tt] * x[tt], acc); out =
// acc * b[t].
struct src_lily_state {
    const float * a;
    const float * x;
    const float * b;
    const float * taps;
    const int32_t * cu;
    int n_seqs, T, C, k;
    __device__ doc_rows row(int t) const { return doc_of(cu, n_seqs, t, T); }
    __device__ void load(const doc_rows & dr, int t, int col, float (&v)[4]) const {
        const int j0 = max(0, dr.lo - (t - k / 2)), j1 = min(k, dr.hi - (t - k / 2));
        float acc[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
        if (k <= TAPS_HOIST) {
            // every tap's rows loaded first (clamped into the batch), then the fmas of taps j0..j1-1
            v4f w[TAPS_HOIST], av[TAPS_HOIST], xv[TAPS_HOIST];
#pragma unroll
            for (int j = 0; j < TAPS_HOIST; ++j) {
                if (j >= k) break;
                const size_t o = (size_t) min(max(t + j - k / 2, 0), T - 1) * C + col;
                w[j] = *reinterpret_cast<const v4f *>(taps + (size_t) j * C + col);
                av[j] = *reinterpret_cast<const v4f *>(a + o);
                xv[j] = *reinterpret_cast<const v4f *>(x + o);
            }
#pragma unroll
            for (int j = 0; j < TAPS_HOIST; ++j) {
                if (j >= k || j < j0 || j >= j1) continue;
                acc[0] = __builtin_fmaf(w[j].x, av[j].x * xv[j].x, acc[0]);
                acc[1] = __builtin_fmaf(w[j].y, av[j].y * xv[j].y, acc[1]);
                acc[2] = __builtin_fmaf(w[j].z, av[j].z * xv[j].z, acc[2]);
                acc[3] = __builtin_fmaf(w[j].w, av[j].w * xv[j].w, acc[3]);
            }
            const v4f bv = *reinterpret_cast<const v4f *>(b + (size_t) t * C + col);
            v[0] = acc[0] * bv.x; v[1] = acc[1] * bv.y; v[2] = acc[2] * bv.z; v[3] = acc[3] * bv.w;
            return;
        }
        for (int j = j0; j < j1; ++j) {
            const size_t o = (size_t) (t + j - k / 2) * C + col;
            const v4f w = *reinterpret_cast<const v4f *>(taps + (size_t) j * C + col);
            const v4f av = *reinterpret_cast<const v4f *>(a + o);
            const v4f xv = *reinterpret_cast<const v4f *>(x + o);
            acc[0] = __builtin_fmaf(w.x, av.x * xv.x, acc[0]);
            acc[1] = __builtin_fmaf(w.y, av.y * xv.y, acc[1]);
            acc[2] = __builtin_fmaf(w.z, av.z * xv.z, acc[2]);
            acc[3] = __builtin_fmaf(w.w, av.w * xv.w, acc[3]);
        }
        const v4f bv = *reinterpret_cast<const v4f *>(b + (size_t) t * C + col);
        v[0] = acc[0] * bv.x; v[1] = acc[1] * bv.y; v[2] = acc[2] * bv.z; v[3] = acc[3] * bv.w;
    }
};

// op_block_mean (src/nexterabert.cpp:638-659): block row b of document d covers tokens
// ts .. ts + n - 1 (ts = cu[d] + block * (b - cub[d]), n = min(block, len_d - that));
// out = 0, then out = fma(h, g, out) per token in order (addmul_f32; with no g,
// axpy_f32 with weight 1: out + h), then out * (1 / n).
struct block_rows {
    int ts, n;
    float inv;
};
struct src_block_mean {
    const float * h;
    const float * g;                           // may be null
    const int32_t * cu;                        // token offsets, n_seqs + 1
    const int32_t * cub;                       // block-row offsets, n_seqs + 1
    int n_seqs, T_tok, n_rows, C, block;
    __device__ block_rows row(int b) const {
        const doc_rows d = doc_of(cub, n_seqs, b, n_rows);
        const int tok_lo = min(max(cu[d.d], 0), T_tok), tok_hi = min(max(cu[d.d + 1], tok_lo), T_tok);
        block_rows r;
        r.ts = min(max(tok_lo + block * (b - d.lo), tok_lo), tok_hi);
        r.n = max(0, min(block, tok_hi - r.ts));
        r.inv = 1.0f / (float) r.n;
        return r;
    }
    __device__ void load(const block_rows & br, int, int col, float (&v)[4]) const {
        v[0] = v[1] = v[2] = v[3] = 0.0f;
        for (int i = 0; i < br.n; ++i) {
            const size_t o = (size_t) (br.ts + i) * C + col;
            const v4f hv = *reinterpret_cast<const v4f *>(h + o);
            if (g) {
                const v4f gv = *reinterpret_cast<const v4f *>(g + o);
                v[0] = __builtin_fmaf(hv.x, gv.x, v[0]);
                v[1] = __builtin_fmaf(hv.y, gv.y, v[1]);
                v[2] = __builtin_fmaf(hv.z, gv.z, v[2]);
                v[3] = __builtin_fmaf(hv.w, gv.w, v[3]);
            } else {
                v[0] = v[0] + hv.x; v[1] = v[1] + hv.y; v[2] = v[2] + hv.z; v[3] = v[3] + hv.w;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v[e] * br.inv;
    }
};

// quantize_row over the rows a source produces: one workgroup per (16-row group,
// 256-input block), as quantize_kernel.
template <int ACT_MAX, typename Src>
__global__ __launch_bounds__(256) void produce_quantize_kernel(Src src, int T, int n_in, int KS, int n_blk,
                                                               int8_t * __restrict__ q, float * __restrict__ sx) {
    __shared__ __attribute__((aligned(16))) int stage[4 * FRAG / 4];
    const int g = (int) (blockIdx.x / (unsigned) n_blk), B = (int) (blockIdx.x % (unsigned) n_blk);
    quantize_block<ACT_MAX>(src, T, n_in, KS, n_blk, q, sx, g, B, stage);
}

// ---------------------------------------------------------------------------
// Attention (head_dim 64) inside each document of a packed layout
// ---------------------------------------------------------------------------

// expf as the reference's C library computes it (glibc 2.35 on x86-64 with FMA; the
// published ARM optimized-routines method): x / ln2 * 32 rounded to an integer k by the
// 1.5 * 2^52 shift, r = x * 32/ln2 - k (both fused), 2^(k/32) from a 32-entry table with
// k's high part added to the exponent bits, a degree-3 polynomial in r, all in double,
// then rounded to float once; |x| >= 88 handled as the library's special cases. Equal to
// the host library's expf for every float input (checked exhaustively on the host).
__device__ __forceinline__ float expf_libm(float x) {
    constexpr uint64_t TAB[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull };
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                                       // |x| >= 88, or NaN / Inf
        if (ux == 0xff800000u) return 0.0f;                      // -Inf
        if (abstop >= 0x7f8) return x + x;                       // NaN, +Inf
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double xd = (double) x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = (uint64_t) __double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = TAB[ki % 32] + (ki << 47);
    const double s = __longlong_as_double((long long) t);
    const double z = __builtin_fma(0x1.c6af84b912394p-5 / 32 / 32 / 32, r, 0x1.ebfce50fac4f3p-3 / 32 / 32);
    const double r2 = r * r;
    double y = __builtin_fma(0x1.62e42ff0c52d6p-1 / 32, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float) (y * s);
}

// One wave per (query t, head h), the head outermost so that neighbouring workgroups read
// one head's keys. Keys [lo, hi) of t's document (the band |t - j| <= half when half >= 0);
// their scores and exponentials live in this workgroup's LDS (max_keys floats).
//  - scores (scores_d64, src/nexterabert.cpp:704-731): 8 keys at a time, lane 8 kk + l
//    holding key kk's lane-l partial of the 64-term chain (l-th elements of the 8 chunks:
//    one multiply, then 7 fused steps); the keys of whole groups of 8 summed as HADDPS and
//    VPERM2F128 order them ((l0+l1)+(l2+l3)) + ((l4+l5)+(l6+l7)) (shuffles xor 1, 2, 4), the
//    remaining keys as hsum256 does ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) (xor 4, 2, 1);
//  - softmax_exp (:177-197): m the running maximum from the first score (a NaN first
//    score makes it NaN; later NaNs never replace it); exp256 for the whole groups of 8,
//    summed into 8 lane sums in order and reduced by hsum256; the library's expf for
//    the rest, added one by one;
//  - values (values_d64, :733-756): lane e accumulates fma(w_j * inv, v_j[e], acc) in key
//    order, inv = 1 / sum correctly rounded.
// A document with more keys than max_keys gets NaN outputs (the caller's bound was wrong).
struct attn_params {
    const float * q;       // [T][H * 64]
    const float * k;       // [G][T][64]
    const float * v;       // [G][T][64]
    const int32_t * cu;    // n_seqs + 1 offsets (device)
    const float * scale;   // [n_seqs] (device)
    float * out;           // [T][H * 64]
    int n_seqs, T, H, G, half, max_keys;
};

__global__ __launch_bounds__(64) void attention_kernel(attn_params p) {
    extern __shared__ float sc[];
    const int lane = threadIdx.x;
    const int h = blockIdx.x / p.T, t = blockIdx.x - h * p.T;
    const int g = h / (p.H / p.G);
    const doc_rows dr = doc_of(p.cu, p.n_seqs, t, p.T);
    int lo = dr.lo, hi = dr.hi;
    if (p.half >= 0) {
        lo = max(lo, t - p.half);
        hi = min(hi, t + p.half + 1);
    }
    const int n = hi - lo;
    float * o = p.out + (size_t) t * p.H * 64 + (size_t) h * 64;
    if (n <= 0 || n > p.max_keys) {
        o[lane] = __uint_as_float(0x7fc00000u);
        return;
    }
    const float scale = p.scale[dr.d];
    const float * qr = p.q + (size_t) t * p.H * 64 + (size_t) h * 64;
    const float * kh = p.k + ((size_t) g * p.T + lo) * 64;
    const float * vh = p.v + ((size_t) g * p.T + lo) * 64;

    // scores
    const int kk = lane >> 3, l = lane & 7;
    float qv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) qv[c] = qr[8 * c + l];
    auto partial = [&](int j) {
        const float * kp = kh + (size_t) j * 64 + l;
        float a = qv[0] * kp[0];
#pragma unroll
        for (int c = 1; c < 8; ++c) a = __builtin_fmaf(qv[c], kp[8 * c], a);
        return a;
    };
    const int ng = n & ~7;
    for (int j0 = 0; j0 < ng; j0 += 8) {
        float a = partial(j0 + kk);
        a = a + __shfl_xor(a, 1);
        a = a + __shfl_xor(a, 2);
        a = a + __shfl_xor(a, 4);
        if (l == 0) sc[j0 + kk] = a * scale;
    }
    if (ng < n) {
        const int j = min(ng + kk, n - 1);                      // lanes past the last key repeat it
        float a = partial(j);
        a = a + __shfl_xor(a, 4);
        a = a + __shfl_xor(a, 2);
        a = a + __shfl_xor(a, 1);
        if (l == 0 && ng + kk < n) sc[j] = scale * a;
    }
    __syncthreads();

    // m: NaN if the first score is NaN, else the largest score that is not NaN
    float mx = -__builtin_inff();
    for (int j = lane; j < n; j += 64) mx = fmaxf(mx, sc[j]);
#pragma unroll
    for (int sft = 32; sft >= 1; sft >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sft));
    const float m = __builtin_isnan(sc[0]) ? sc[0] : mx;
    __syncthreads();
    for (int j = lane; j < ng; j += 64) sc[j] = exp_cephes(sc[j] - m);
    for (int j = ng + lane; j < n; j += 64) sc[j] = expf_libm(sc[j] - m);
    __syncthreads();
    // lane sums of the whole groups (lane l < 8 takes elements 8i + l in order), hsum256
    float ls = 0.0f;
    if (lane < 8) {
        for (int j = lane; j < ng; j += 8) ls = ls + sc[j];
    }
    ls = ls + __shfl_xor(ls, 4);
    ls = ls + __shfl_xor(ls, 2);
    ls = ls + __shfl_xor(ls, 1);
    float sum = __shfl(ls, 0);
    for (int j = ng; j < n; ++j) sum = sum + sc[j];
    const float inv = 1.0f / sum;

    // values, key by key
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) acc = __builtin_fmaf(sc[j] * inv, vh[(size_t) j * 64 + lane], acc);
    o[lane] = acc;
}

// softmax_exp (src/nexterabert.cpp:177-200) for one (query, head) pair whose n scores sit in
// LDS at Sp, by the 16 lanes sk of the pair (one wave's 16-lane group), in three steps with a
// workgroup barrier between them (the callers hold it):
//   softmax_max_exp   m (a NaN first score wins, else the largest score), then exp256(s - m)
//                     in place for the n & ~7 grouped keys and the C library's expf for the rest
//   softmax_inv       lanes l < 8 add keys 8i + l in order of i, hsum256 over the 8 lanes, the
//                     tail keys added after in order; returns 1 / sum (on lane 0 of the group)
//   softmax_weights   w = e * (1 / sum) in place
// Loads are issued 16 at a time ahead of the adds that consume them in order.
__device__ __forceinline__ void softmax_max_exp(float * Sp, int n, int sk) {
    const int ng = n & ~7;
    const float s0 = Sp[0];
    float mx = -__builtin_inff();
#pragma unroll 8
    for (int j = sk; j < n; j += 16) mx = fmaxf(mx, Sp[j]);
#pragma unroll
    for (int sft = 8; sft >= 1; sft >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sft));
    const float m = __builtin_isnan(s0) ? s0 : mx;
#pragma unroll 8
    for (int j = sk; j < ng; j += 16) Sp[j] = exp_cephes(Sp[j] - m);
    for (int j = ng + sk; j < n; j += 16) Sp[j] = expf_libm(Sp[j] - m);
}

__device__ __forceinline__ float softmax_inv(const float * Sp, int n, int sk, bool active) {
    const int ng = n & ~7;
    float ls = 0.0f;
    if (active && sk < 8) {
        int j = sk;
        for (; j + 8 * 15 < ng; j += 8 * 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = Sp[j + 8 * u];
#pragma unroll
            for (int u = 0; u < 16; ++u) ls = ls + v[u];
        }
        for (; j < ng; j += 8) ls = ls + Sp[j];
    }
    ls = ls + __shfl_xor(ls, 4);                           // lanes 8..15 hold 0 and stay among themselves
    ls = ls + __shfl_xor(ls, 2);
    ls = ls + __shfl_xor(ls, 1);
    float sum = ls;
    if (active && sk == 0) {
        for (int j = ng; j < n; ++j) sum = sum + Sp[j];
    }
    return 1.0f / sum;
}

__device__ __forceinline__ void softmax_weights(float * Sp, int n, int sk, float inv) {
#pragma unroll 8
    for (int j = sk; j < n; j += 16) Sp[j] = Sp[j] * inv;
}

// acc[i] = fma(w_i[lane L of this lane's 16-lane row], v_L, acc[i]) for i < 4 and the 16 keys
// L of a half tile in order: v_fmac_f32 (one rounding, as fmaf) with its first operand
// broadcast by DPP row_newbcast. With w_i holding key k of a 16-key group in lanes k, k + 16,
// k + 32, k + 48, every lane gets key L's weight; key L's value is vt[L]. One asm block, so that
// the 16 values are in registers before the first FMA (their LDS reads issued together, one
// wait; the compiler otherwise spread them among the FMAs, one wait per two keys), and one
// s_nop gives the DPP reads their two wait states after the VALU writes of w: full attention
// over 1,024 keys 170.5 -> 164.5 us, banded attention over 8 x 1,024 tokens 295 -> 282 us.
#define NXG_FB4(k, vo) \
    "v_fmac_f32_dpp %0, %4, %" #vo " row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %1, %5, %" #vo " row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %2, %6, %" #vo " row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %3, %7, %" #vo " row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n\t"
__device__ __forceinline__ void fmac_bcast4_16(float (&acc)[4], const float (&w)[4], const float * vt) {
    asm("s_nop 1\n\t"
        NXG_FB4(0, 8) NXG_FB4(1, 9) NXG_FB4(2, 10) NXG_FB4(3, 11) NXG_FB4(4, 12) NXG_FB4(5, 13)
        NXG_FB4(6, 14) NXG_FB4(7, 15) NXG_FB4(8, 16) NXG_FB4(9, 17) NXG_FB4(10, 18) NXG_FB4(11, 19)
        NXG_FB4(12, 20) NXG_FB4(13, 21) NXG_FB4(14, 22) NXG_FB4(15, 23)
        : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
        : "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]),
          "v"(vt[0]), "v"(vt[1]), "v"(vt[2]), "v"(vt[3]), "v"(vt[4]), "v"(vt[5]), "v"(vt[6]), "v"(vt[7]),
          "v"(vt[8]), "v"(vt[9]), "v"(vt[10]), "v"(vt[11]), "v"(vt[12]), "v"(vt[13]), "v"(vt[14]), "v"(vt[15]));
}
#undef NXG_FB4

// The same attention for a tile of (query, head) pairs: the ATT_P pairs of one workgroup are
// ATT_P / rep consecutive query rows times the rep query heads of one KV head, so that every
// key and value row read into LDS serves all of them. Per pair the operations and their
// order are attention_kernel's (the reference's scores_d64, softmax_exp, values_d64):
//   scores    the 8 FMA chains (a_l = q[l] k[l], then fma(q[8c+l], k[8c+l], a_l) for
//             c = 1..7) and the HADD tree (keys of whole groups of 8) or hsum256's (the last
//             n % 8 keys) in registers, times the scale; kept in LDS, [pair][key - the pair's
//             first key]. Chain-parallel: 8 lanes per key, each one chain of 16 pairs
//             (WIDE, 128 query registers, chosen when the scores' LDS already limits a CU to
//             two workgroups) or of 8 pairs (64 registers), so that a staged key row is read
//             from LDS once for 16 or 8 pairs (att_chain_tree)
//   softmax   16 threads per pair: the maximum (a NaN first score wins), exp256 / the C
//             library's expf in place, then threads l < 8 add the keys 8i + l in order of i
//             (the 8 lanes of softmax_exp's accumulator) and hsum256 over them, the tail keys
//             added after; each weight becomes w * (1 / sum)
//   values    thread (dim d, 4 pairs): acc = fma(w_j, v_j[d], acc) over the keys in order;
//             a tile's weights of a pair are read once, key j0 + 16h + k in lane k of every
//             16-lane row of register h, and each fma takes its weight through DPP row_newbcast
//             (keys outside a pair's range with weight 0, adding fma(0, v, acc) = acc; readlane
//             and a per-key range test on tiles whose staged values hold an Inf or NaN), so the
//             key loop reads only v_j[d] from LDS.
// Keys are staged ATT_KT at a time ([key][ATT_KS] floats; the padding puts the 16 rows one
// wave reads on different banks). Pairs whose keys exceed smax get NaN, as attention_kernel.
// One key's score for a query held in registers, before the scale (scores_d64,
// src/nexterabert.cpp:704-731): the 8 chains a_l = q_l k_l, fma(q[8c+l], k[8c+l], a_l) for
// c = 1..7, then the HADD tree for a key of a whole group of 8, hsum256's for a tail key.
__device__ __forceinline__ float score_d64(const float (&qv)[64], const float * kp, bool grouped) {
    float a[8];
    {
        const v4f k0 = *reinterpret_cast<const v4f *>(kp), k1 = *reinterpret_cast<const v4f *>(kp + 4);
        a[0] = qv[0] * k0.x; a[1] = qv[1] * k0.y; a[2] = qv[2] * k0.z; a[3] = qv[3] * k0.w;
        a[4] = qv[4] * k1.x; a[5] = qv[5] * k1.y; a[6] = qv[6] * k1.z; a[7] = qv[7] * k1.w;
    }
#pragma unroll
    for (int c = 1; c < 8; ++c) {
        const v4f k0 = *reinterpret_cast<const v4f *>(kp + 8 * c);
        const v4f k1 = *reinterpret_cast<const v4f *>(kp + 8 * c + 4);
        a[0] = __builtin_fmaf(qv[8 * c + 0], k0.x, a[0]);
        a[1] = __builtin_fmaf(qv[8 * c + 1], k0.y, a[1]);
        a[2] = __builtin_fmaf(qv[8 * c + 2], k0.z, a[2]);
        a[3] = __builtin_fmaf(qv[8 * c + 3], k0.w, a[3]);
        a[4] = __builtin_fmaf(qv[8 * c + 4], k1.x, a[4]);
        a[5] = __builtin_fmaf(qv[8 * c + 5], k1.y, a[5]);
        a[6] = __builtin_fmaf(qv[8 * c + 6], k1.z, a[6]);
        a[7] = __builtin_fmaf(qv[8 * c + 7], k1.w, a[7]);
    }
    return grouped ? ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))
                   : ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
}

// Chain-parallel scores: lane L of an 8-lane group computes chain L of one
// key's dot products with all 16 pairs of the workgroup, a_L = q[L] k[L], then fma(q[8c+L],
// k[8c+L], a_L) for c = 1..7, and the group adds the 8 chains in the tree
// ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)) by three exchange steps: DPP quad_perm
// with lane L ^ 1, quad_perm with lane L ^ 2, row_half_mirror with lane 7 - L (the other
// half of the group). Register i of lane L holds pair i ^ att_chain_g(L): with that
// assignment every exchange adds the same pair's partial sums from registers of one index
// (step 1: register i + 8 of the partner to register i, i < 8; step 2: i + 4 to i, i < 4;
// step 3: i + 2 to i, i < 2), and lane L ends with the scores of pairs att_chain_g(L) and
// att_chain_g(L) + 1. Each addition is commutative, so the lane order inside a step does not
// change the bits.
__device__ __forceinline__ int att_chain_g(int L) { return ((L & 1) ? 8 : 0) ^ ((L & 2) ? 4 : 0) ^ ((L & 4) ? 14 : 0); }

// The tree of the 16 pairs' chain-L values a[i] (pair i ^ att_chain_g(L)) into the two
// scores of this lane's pairs. The s_nop gives each step's DPP reads their two wait states
// after the VALU writes of their sources.
__device__ __forceinline__ void att_chain_tree(const float (&a)[16], float (&s)[2]) {
    float b[8], c[4];
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %16, %8 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %1, %17, %9 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %2, %18, %10 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %3, %19, %11 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %4, %20, %12 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %5, %21, %13 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %6, %22, %14 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %7, %23, %15 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
        : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]), "=&v"(b[6]), "=&v"(b[7])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
          "v"(a[8]), "v"(a[9]), "v"(a[10]), "v"(a[11]), "v"(a[12]), "v"(a[13]), "v"(a[14]), "v"(a[15]));
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %8, %4 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %1, %9, %5 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %2, %10, %6 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %3, %11, %7 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf"
        : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3])
        : "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(b[4]), "v"(b[5]), "v"(b[6]), "v"(b[7]));
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %4, %2 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %1, %5, %3 row_half_mirror row_mask:0xf bank_mask:0xf"
        : "=&v"(s[0]), "=&v"(s[1])
        : "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]));
}

// The same for 8 pairs (register i: pair i ^ att_chain_g8(L)): steps of 4, 2 and 1 registers,
// lane L ending with the score of pair att_chain_g8(L) (0..7, one per lane of the group).
__device__ __forceinline__ int att_chain_g8(int L) { return ((L & 1) ? 4 : 0) ^ ((L & 2) ? 2 : 0) ^ ((L & 4) ? 7 : 0); }
__device__ __forceinline__ void att_chain_tree(const float (&a)[8], float (&s)[1]) {
    float b[4], c[2];
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %8, %4 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %1, %9, %5 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %2, %10, %6 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %3, %11, %7 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
        : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %4, %2 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %1, %5, %3 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf"
        : "=&v"(c[0]), "=&v"(c[1])
        : "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]));
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %2, %1 row_half_mirror row_mask:0xf bank_mask:0xf"
        : "=&v"(s[0])
        : "v"(c[0]), "v"(c[1]));
}

__device__ __forceinline__ bool finite4(const v4f & x) {
    return __builtin_isfinite(x.x) && __builtin_isfinite(x.y) && __builtin_isfinite(x.z) && __builtin_isfinite(x.w);
}
#ifndef NXG_ATT_WIDE
#define NXG_ATT_WIDE 1         // 16 pairs per lane group where LDS allows two workgroups per CU (0: always 8)
#endif
constexpr int ATT_P = 16;      // (query, head) pairs per workgroup
constexpr int ATT_KT = 32;     // keys per staged tile
constexpr int ATT_KS = 68;     // floats per staged row

template <bool WIDE>
__global__ __launch_bounds__(256) void attention_tile_kernel(attn_params p, int smax) {
    extern __shared__ __attribute__((aligned(16))) float att_lds[];
    float * S = att_lds;                                   // [ATT_P][smax]
    float * tile = att_lds + (size_t) ATT_P * smax;        // [ATT_KT][ATT_KS]
    __shared__ int lo_s[ATT_P], hi_s[ATT_P];
    __shared__ float scale_s[ATT_P], inv_s[ATT_P];
    const int tid = (int) threadIdx.x;
    const int rep = p.H / p.G, nq = ATT_P / rep;
    const int n_qblk = (p.T + nq - 1) / nq;
    const int g = (int) blockIdx.x / n_qblk, t0 = ((int) blockIdx.x - g * n_qblk) * nq;

    if (tid < ATT_P) {
        const int t = t0 + tid / rep;
        int lo = 0, hi = 0;
        float sc = 0.0f;
        if (t < p.T) {
            const doc_rows dr = doc_of(p.cu, p.n_seqs, t, p.T);
            lo = dr.lo;
            hi = dr.hi;
            if (p.half >= 0) {
                lo = max(lo, t - p.half);
                hi = min(hi, t + p.half + 1);
            }
            sc = p.scale[dr.d];
        }
        lo_s[tid] = lo;
        hi_s[tid] = hi;
        scale_s[tid] = sc;
    }
    __syncthreads();
    // keys any pair reads: [kl, kh)
    int kl = INT_MAX, kh = INT_MIN;
#pragma unroll
    for (int i = 0; i < ATT_P; ++i) {
        if (hi_s[i] > lo_s[i] && hi_s[i] - lo_s[i] <= smax) {
            kl = min(kl, lo_s[i]);
            kh = max(kh, hi_s[i]);
        }
    }
    const float * kg = p.k + (size_t) g * p.T * 64;
    const float * vg = p.v + (size_t) g * p.T * 64;

    // softmax threads: 16 per pair, pair sp
    const int sp = tid >> 4, sk = tid & 15;
    const int n_p = hi_s[sp] - lo_s[sp];
    const bool valid = n_p > 0 && n_p <= smax;
    float * Sp = S + (size_t) sp * smax;
    // staged rows: thread tid moves row (tid >> 4) + 16 r, floats 4 (tid & 15) .. + 3, r < 2;
    // the next tile's rows are fetched into registers while the current one is used
    const int st_r = tid >> 4, st_c = 4 * (tid & 15);
    v4f pre[2];
    auto fetch = [&](const float * src, int j0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int j = j0 + st_r + 16 * r;
            pre[r] = j < kh ? *reinterpret_cast<const v4f *>(src + (size_t) j * 64 + st_c) : v4f{ 0.0f, 0.0f, 0.0f, 0.0f };
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int r = 0; r < 2; ++r) *reinterpret_cast<v4f *>(tile + (st_r + 16 * r) * ATT_KS + st_c) = pre[r];
    };

    // scores, chain-parallel (att_chain_tree): lane L of an 8-lane group holds element 8c + L
    // of NPG pairs' queries and computes chain L of one key's dot products with them, so that
    // each key's 8 values read from LDS serve NPG pairs' FMAs. WIDE: one group per key for all
    // 16 pairs (128 query registers; for launches whose LDS admits at most two workgroups per
    // CU); else two groups per key, 8 pairs each (64 registers), each group taking two keys per
    // tile. Keys are staged chain-major (row j: [L][c], element 8c + L at 8L + c), the queries
    // likewise through the tile before the first key tile. The scores of keys of whole groups
    // of 8 come out of the tree; a pair's last n % 8 keys take hsum256's tree, one thread per
    // (pair, key) afterwards.
    {
        constexpr int NPG = WIDE ? ATT_P : ATT_P / 2;          // pairs per 8-lane group
        constexpr int NO = WIDE ? 2 : 1;                       // scores per lane out of the tree
        constexpr int NK = WIDE ? 1 : 2;                       // keys per group per tile
        const int L = tid & 7, gi = tid >> 3;
        const int gL = WIDE ? att_chain_g(L) : att_chain_g8(L);
        const int pbase = WIDE ? 0 : NPG * (gi & 1);
        const int js0 = WIDE ? gi : gi >> 1;
        {
            const int pp = tid >> 4, m = tid & 15;
            const int t = t0 + pp / rep, h = g * rep + pp % rep;
            const v4f f = *reinterpret_cast<const v4f *>(p.q + (size_t) min(t, p.T - 1) * p.H * 64 + (size_t) h * 64 + 4 * m);
            const float fe[4] = { f.x, f.y, f.z, f.w };
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int d = 4 * m + u;
                tile[pp * ATT_KS + (d & 7) * 8 + (d >> 3)] = fe[u];
            }
        }
        __syncthreads();
        float qr[NPG][8];
#pragma unroll
        for (int i = 0; i < NPG; ++i) {
            const float * src = tile + (pbase + (i ^ gL)) * ATT_KS + L * 8;
            const v4f a0 = *reinterpret_cast<const v4f *>(src), a1 = *reinterpret_cast<const v4f *>(src + 4);
            qr[i][0] = a0.x; qr[i][1] = a0.y; qr[i][2] = a0.z; qr[i][3] = a0.w;
            qr[i][4] = a1.x; qr[i][5] = a1.y; qr[i][6] = a1.z; qr[i][7] = a1.w;
        }
        int lo2[NO], ng2[NO], pp2[NO];
        bool ok2[NO];
        float sc2[NO];
#pragma unroll
        for (int u = 0; u < NO; ++u) {
            const int pp = pbase + gL + u, n = hi_s[pp] - lo_s[pp];
            pp2[u] = pp;
            lo2[u] = lo_s[pp];
            ok2[u] = n > 0 && n <= smax;
            ng2[u] = n & ~7;
            sc2[u] = scale_s[pp];
        }
        auto stage_chain = [&]() {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float * row = tile + (st_r + 16 * r) * ATT_KS;
                const float e[4] = { pre[r].x, pre[r].y, pre[r].z, pre[r].w };
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int d = st_c + u;
                    row[(d & 7) * 8 + (d >> 3)] = e[u];
                }
            }
        };
        if (kl < kh) fetch(kg, kl);
        for (int j0 = kl; j0 < kh; j0 += ATT_KT) {
            __syncthreads();                               // the previous tile (or the queries) read
            stage_chain();
            __syncthreads();
            if (j0 + ATT_KT < kh) fetch(kg, j0 + ATT_KT);
#pragma unroll
            for (int r = 0; r < NK; ++r) {
                const int js = js0 + 16 * r;
                const float * kp = tile + js * ATT_KS + L * 8;
                const v4f k0 = *reinterpret_cast<const v4f *>(kp), k1 = *reinterpret_cast<const v4f *>(kp + 4);
                const float kk[8] = { k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w };
                float a[NPG];
#pragma unroll
                for (int i = 0; i < NPG; ++i) a[i] = qr[i][0] * kk[0];
#pragma unroll
                for (int c = 1; c < 8; ++c)
#pragma unroll
                    for (int i = 0; i < NPG; ++i) a[i] = __builtin_fmaf(qr[i][c], kk[c], a[i]);
                float s2[NO];
                att_chain_tree(a, s2);
#pragma unroll
                for (int u = 0; u < NO; ++u) {
                    const int jr = j0 + js - lo2[u];
                    if (ok2[u] && jr >= 0 && jr < ng2[u]) S[(size_t) pp2[u] * smax + jr] = s2[u] * sc2[u];
                }
            }
        }
        if (valid && sk < n_p - (n_p & ~7)) {
            const int jr = (n_p & ~7) + sk;
            float qv[64];
            const int t = t0 + sp / rep, h = g * rep + sp % rep;
            const float * qrow = p.q + (size_t) min(t, p.T - 1) * p.H * 64 + (size_t) h * 64;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const v4f f = *reinterpret_cast<const v4f *>(qrow + 4 * i);
                qv[4 * i] = f.x; qv[4 * i + 1] = f.y; qv[4 * i + 2] = f.z; qv[4 * i + 3] = f.w;
            }
            Sp[jr] = score_d64(qv, kg + (size_t) (lo_s[sp] + jr) * 64, false) * scale_s[sp];
        }
    }
    __syncthreads();

    // softmax: 16 threads per pair
    if (valid) softmax_max_exp(Sp, n_p, sk);
    __syncthreads();
    {
        const float inv = softmax_inv(Sp, n_p, sk, valid);
        if (valid && sk == 0) inv_s[sp] = inv;
    }
    __syncthreads();
    if (valid) softmax_weights(Sp, n_p, sk, inv_s[sp]);

    // values: thread (dim d, pairs 4 pg .. 4 pg + 3); pg is the wave's, so the pairs' key
    // ranges are scalars and a key outside a pair's range costs a scalar branch
    const int d = tid & 63, pg = __builtin_amdgcn_readfirstlane(tid >> 6);
    int vlo[4], vn[4];
    float acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pp = 4 * pg + i;
        vlo[i] = __builtin_amdgcn_readfirstlane(lo_s[pp]);
        vn[i] = __builtin_amdgcn_readfirstlane(hi_s[pp] - lo_s[pp]);
        if (vn[i] > smax) vn[i] = 0;
        acc[i] = 0.0f;
    }
    // a staged value tile holding a non-finite value (by tile parity): without one, every tile,
    // also one only partly in a pair's keys, takes the broadcast path, its keys outside the pair's
    // range adding fma(0, v, acc) = acc (acc is never -0: it starts at +0): banded attention
    // over 8 x 1,024 tokens 343 -> 291 us, documents of 300 / 45 / 700 tokens 217 -> 144 us
    __shared__ int vbad_s[2];
    if (tid < 2) vbad_s[tid] = 0;
    int par = 0;
    if (kl < kh) fetch(vg, kl);
    for (int j0 = kl; j0 < kh; j0 += ATT_KT, par ^= 1) {
        __syncthreads();                                   // weights written / previous tile read
        if (tid == 0) vbad_s[par ^ 1] = 0;                 // the previous tile's flag, read by all
        stage();
        if (!(finite4(pre[0]) && finite4(pre[1]))) vbad_s[par] = 1;
        __syncthreads();
        if (j0 + ATT_KT < kh) fetch(vg, j0 + ATT_KT);
        const int jn = min(ATT_KT, kh - j0);
        int a[4], b[4];
        const bool full = vbad_s[par] == 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {                      // keys [a, b) of the tile are pair i's
            a[i] = min(max(vlo[i] - j0, 0), jn);
            b[i] = max(min(vlo[i] + vn[i] - j0, jn), a[i]);
        }
        // the tile's weights: pair i's weight of key j0 + l in lane l (l < 32), read once and
        // broadcast per key (readlane), so the key loop reads only the value row from LDS
        // weights of keys j0 + k (w0) and j0 + 16 + k (w1) of pair i in lane k of every 16-lane row
        float w0[4], w1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int jr = j0 + (d & 15) - vlo[i];
            w0[i] = (jr >= 0 && jr < vn[i]) ? S[(size_t) (4 * pg + i) * smax + jr] : 0.0f;
            w1[i] = (jr + 16 >= 0 && jr + 16 < vn[i]) ? S[(size_t) (4 * pg + i) * smax + jr + 16] : 0.0f;
        }
        auto wk = [&](int i, int jj) {
            return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(jj < 16 ? w0[i] : w1[i]), jj & 15));
        };
        if (full) {
            float vt[ATT_KT];                              // the tile's values of dimension d, read up front
#pragma unroll
            for (int jj = 0; jj < ATT_KT; ++jj) vt[jj] = tile[jj * ATT_KS + d];
            fmac_bcast4_16(acc, w0, vt);
            fmac_bcast4_16(acc, w1, vt + 16);
        } else {
            for (int jj = 0; jj < jn; ++jj) {
                const float v = tile[jj * ATT_KS + d];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (jj >= a[i] && jj < b[i]) acc[i] = __builtin_fmaf(wk(i, jj), v, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pp = 4 * pg + i, t = t0 + pp / rep, h = g * rep + pp % rep;
        if (t >= p.T) continue;
        const int n = hi_s[pp] - lo_s[pp];
        p.out[(size_t) t * p.H * 64 + (size_t) h * 64 + d] = (n > 0 && n <= smax) ? acc[i] : __uint_as_float(0x7fc00000u);
    }
}


// attention_tile_kernel's pairs, thread mapping and per-pair order for documents whose
// scores do not fit in LDS: nothing is kept per key; the scores are computed three times,
// bit-identically.
//   pass 1  the maximum (a NaN first score wins, else the largest score that is not NaN)
//   pass 2  e = exp256(s - m) (grouped keys) or the C library's expf (the n % 8 tail keys);
//           each tile's e go through LDS so that lanes l < 8 of a pair add keys 8i + l in
//           order of i, as softmax_exp's 8 accumulator lanes do; the tail e are kept apart and
//           added after hsum256, in order
//   pass 3  w = e * (1 / sum) per key through LDS, then thread (dim d, 4 pairs) acc = fma(w,
//           v[d], acc) over the keys in order, as attention_tile_kernel (the tile's weights
//           read once per lane and broadcast per key by DPP row_newbcast, or by readlane with a
//           per-key range test on partial tiles (ZW: only on tiles with an Inf or NaN value))
// Keys and values are staged ATT_KT at a time ([key][ATT_KS]).
// STORED: pass 1 also writes each score to the workgroup's slot of the workspace sc
// ([gridDim.x][ATT_P][max_keys] floats, pair-relative key index), and passes 2 and 3 read the
// scores back instead of recomputing them, the same bits; pass 2 then needs no staged keys
// (lane l < 8 of a pair adds keys 16b + l and 16b + 8 + l, the second taken from lane l + 8),
// pass 3 stages only the values. ESTORE: pass 2 also writes each e = exp(s - m) over
// its score and pass 3 takes w = e * (1 / sum) from it (the same bits as recomputing e).
// One call is the tile bt = (KV head, query block).
#ifndef NXG_ATT_STORED_WIDE
#define NXG_ATT_STORED_WIDE 0  // attention_stored_kernel's scores: 16 pairs per lane group (0: 8)
#endif
#ifndef NXG_ATT_E_STORE_MIB
#define NXG_ATT_E_STORE_MIB 192   // the largest workspace in use (all slots) for which pass 2 stores e
#endif
template <bool STORED, bool ESTORE, bool ZW>
__device__ __forceinline__ void attention_long_tile(const attn_params & p, float * __restrict__ sc, int bt) {
    __shared__ __attribute__((aligned(16))) float tile[ATT_KT * ATT_KS];
    __shared__ float E[ATT_P][ATT_KT + 1];                 // one tile's e (pass 2) or w (pass 3)
    __shared__ float tail_e[ATT_P][8];
    __shared__ int lo_s[ATT_P], hi_s[ATT_P];
    __shared__ float scale_s[ATT_P], m_s[ATT_P], s0_s[ATT_P], inv_s[ATT_P];
    const int tid = (int) threadIdx.x;
    const int rep = p.H / p.G, nq = ATT_P / rep;
    const int n_qblk = (p.T + nq - 1) / nq;
    const int g = bt / n_qblk, t0 = (bt - g * n_qblk) * nq;

    if (tid < ATT_P) {
        const int t = t0 + tid / rep;
        int lo = 0, hi = 0;
        float sc = 0.0f;
        if (t < p.T) {
            const doc_rows dr = doc_of(p.cu, p.n_seqs, t, p.T);
            lo = dr.lo;
            hi = dr.hi;
            if (p.half >= 0) {
                lo = max(lo, t - p.half);
                hi = min(hi, t + p.half + 1);
            }
            sc = p.scale[dr.d];
        }
        lo_s[tid] = lo;
        hi_s[tid] = hi;
        scale_s[tid] = sc;
    }
    __syncthreads();
    int kl = INT_MAX, kh = INT_MIN;
#pragma unroll
    for (int i = 0; i < ATT_P; ++i) {
        if (hi_s[i] > lo_s[i] && hi_s[i] - lo_s[i] <= p.max_keys) {
            kl = min(kl, lo_s[i]);
            kh = max(kh, hi_s[i]);
        }
    }
    const float * kg = p.k + (size_t) g * p.T * 64;
    const float * vg = p.v + (size_t) g * p.T * 64;

    const int sp = tid >> 4, sk = tid & 15;
    const int plo = lo_s[sp], n_p = hi_s[sp] - plo, ng_p = n_p & ~7;
    const bool valid = n_p > 0 && n_p <= p.max_keys;     // more keys than max_keys: NaN, as the other kernels
    float * const scp = STORED ? sc + ((size_t) blockIdx.x * ATT_P + sp) * (size_t) p.max_keys : nullptr;
    // this thread's pair's query (STORED: only for its tail keys, loaded there)
    float qv[64];
    const float * const qrow = p.q + (size_t) min(t0 + sp / rep, p.T - 1) * p.H * 64 + (size_t) (g * rep + sp % rep) * 64;
    if constexpr (!STORED) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const v4f f = *reinterpret_cast<const v4f *>(qrow + 4 * i);
            qv[4 * i] = f.x; qv[4 * i + 1] = f.y; qv[4 * i + 2] = f.z; qv[4 * i + 3] = f.w;
        }
    }
    const float scale = scale_s[sp];
    const int st_r = tid >> 4, st_c = 4 * (tid & 15);
    v4f pre[2];
    auto fetch = [&](const float * src, int j0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int j = j0 + st_r + 16 * r;
            pre[r] = j < kh ? *reinterpret_cast<const v4f *>(src + (size_t) j * 64 + st_c) : v4f{ 0.0f, 0.0f, 0.0f, 0.0f };
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int r = 0; r < 2; ++r) *reinterpret_cast<v4f *>(tile + (st_r + 16 * r) * ATT_KS + st_c) = pre[r];
    };

    // pass 1: the maximum
    if constexpr (STORED) {
        // the scores chain-parallel, as attention_tile_kernel (att_chain_tree; SW: 16 pairs
        // per lane group, else 8 pairs and two keys per group and tile), each written to the
        // workspace; the maxima of a pair's key slots meet in E, then its 16 lanes; a pair's
        // last n % 8 keys by hsum256's tree, one thread per key
        constexpr bool SW = NXG_ATT_STORED_WIDE;
        constexpr int NPG = SW ? ATT_P : ATT_P / 2;            // pairs per 8-lane group
        constexpr int NO = SW ? 2 : 1;                         // scores per lane out of the tree
        constexpr int NK = SW ? 1 : 2;                         // keys per group per tile
        const int L = tid & 7, gi = tid >> 3;
        const int gL = SW ? att_chain_g(L) : att_chain_g8(L);
        const int pbase = SW ? 0 : NPG * (gi & 1);
        const int js0 = SW ? gi : gi >> 1;
        {
            const int pp = tid >> 4, m = tid & 15;
            const int t = t0 + pp / rep, h = g * rep + pp % rep;
            const v4f f = *reinterpret_cast<const v4f *>(p.q + (size_t) min(t, p.T - 1) * p.H * 64 + (size_t) h * 64 + 4 * m);
            const float fe[4] = { f.x, f.y, f.z, f.w };
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int d = 4 * m + u;
                tile[pp * ATT_KS + (d & 7) * 8 + (d >> 3)] = fe[u];
            }
        }
        __syncthreads();
        float qr[NPG][8];
#pragma unroll
        for (int i = 0; i < NPG; ++i) {
            const float * src = tile + (pbase + (i ^ gL)) * ATT_KS + L * 8;
            const v4f a0 = *reinterpret_cast<const v4f *>(src), a1 = *reinterpret_cast<const v4f *>(src + 4);
            qr[i][0] = a0.x; qr[i][1] = a0.y; qr[i][2] = a0.z; qr[i][3] = a0.w;
            qr[i][4] = a1.x; qr[i][5] = a1.y; qr[i][6] = a1.z; qr[i][7] = a1.w;
        }
        int lo2[NO], ng2[NO];
        bool ok2[NO];
        float sc2[NO], mx2[NO];
        float * sp2[NO];
#pragma unroll
        for (int u = 0; u < NO; ++u) {
            const int pp = pbase + gL + u, n = hi_s[pp] - lo_s[pp];
            lo2[u] = lo_s[pp];
            ok2[u] = n > 0 && n <= p.max_keys;
            ng2[u] = n & ~7;
            sc2[u] = scale_s[pp];
            mx2[u] = -__builtin_inff();
            sp2[u] = sc + ((size_t) blockIdx.x * ATT_P + pp) * (size_t) p.max_keys;
        }
        auto stage_chain = [&]() {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float * row = tile + (st_r + 16 * r) * ATT_KS;
                const float e[4] = { pre[r].x, pre[r].y, pre[r].z, pre[r].w };
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int d = st_c + u;
                    row[(d & 7) * 8 + (d >> 3)] = e[u];
                }
            }
        };
        if (kl < kh) fetch(kg, kl);
        for (int j0 = kl; j0 < kh; j0 += ATT_KT) {
            __syncthreads();                               // the previous tile (or the queries) read
            stage_chain();
            __syncthreads();
            if (j0 + ATT_KT < kh) fetch(kg, j0 + ATT_KT);
#pragma unroll
            for (int r = 0; r < NK; ++r) {
                const int js = js0 + 16 * r;
                const float * kp = tile + js * ATT_KS + L * 8;
                const v4f k0 = *reinterpret_cast<const v4f *>(kp), k1 = *reinterpret_cast<const v4f *>(kp + 4);
                const float kk[8] = { k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w };
                float a[NPG];
#pragma unroll
                for (int i = 0; i < NPG; ++i) a[i] = qr[i][0] * kk[0];
#pragma unroll
                for (int c = 1; c < 8; ++c)
#pragma unroll
                    for (int i = 0; i < NPG; ++i) a[i] = __builtin_fmaf(qr[i][c], kk[c], a[i]);
                float s2[NO];
                att_chain_tree(a, s2);
#pragma unroll
                for (int u = 0; u < NO; ++u) {
                    const int jr = j0 + js - lo2[u];
                    if (ok2[u] && jr >= 0 && jr < ng2[u]) {
                        const float s = s2[u] * sc2[u];
                        mx2[u] = fmaxf(mx2[u], s);
                        sp2[u][jr] = s;
                        if (jr == 0) s0_s[pbase + gL + u] = s;
                    }
                }
            }
        }
        // SW: pair gL + u's maxima over key slots js0 (0..31); else pair pbase + gL's over
        // key slots js0 and js0 + 16 in slot js0 (0..15)
#pragma unroll
        for (int u = 0; u < NO; ++u) E[pbase + gL + u][js0] = mx2[u];
        __syncthreads();
        float mx = SW ? fmaxf(E[sp][sk], E[sp][sk + 16]) : E[sp][sk];
        if (valid && sk < n_p - ng_p) {
            const int jr = ng_p + sk;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const v4f f = *reinterpret_cast<const v4f *>(qrow + 4 * i);
                qv[4 * i] = f.x; qv[4 * i + 1] = f.y; qv[4 * i + 2] = f.z; qv[4 * i + 3] = f.w;
            }
            const float s = score_d64(qv, kg + (size_t) (plo + jr) * 64, false) * scale;
            mx = fmaxf(mx, s);
            scp[jr] = s;
            if (jr == 0) s0_s[sp] = s;
        }
#pragma unroll
        for (int sft = 8; sft >= 1; sft >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sft));
        __syncthreads();                                   // s0_s written
        if (valid && sk == 0) m_s[sp] = __builtin_isnan(s0_s[sp]) ? s0_s[sp] : mx;
        __syncthreads();
    } else {
        float mx = -__builtin_inff();
        if (kl < kh) fetch(kg, kl);
        for (int j0 = kl; j0 < kh; j0 += ATT_KT) {
            __syncthreads();
            stage();
            __syncthreads();
            if (j0 + ATT_KT < kh) fetch(kg, j0 + ATT_KT);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int jr = j0 + sk + 16 * r - plo;
                if (!valid || jr < 0 || jr >= n_p) continue;
                const float s = score_d64(qv, tile + (sk + 16 * r) * ATT_KS, jr < ng_p) * scale;
                mx = fmaxf(mx, s);
                if (jr == 0) s0_s[sp] = s;
                if constexpr (STORED) scp[jr] = s;
            }
        }
#pragma unroll
        for (int sft = 8; sft >= 1; sft >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sft));
        __syncthreads();                                   // s0_s written
        if (valid && sk == 0) m_s[sp] = __builtin_isnan(s0_s[sp]) ? s0_s[sp] : mx;
        __syncthreads();
    }
    const float m = m_s[sp];

    // pass 2: the ordered sum of the exponentials
    if constexpr (STORED) {
        float ls = 0.0f;
        const int ng = valid ? ng_p : 0;                   // the same for the 16 lanes of a pair
        constexpr int U = 16;                              // 16-key steps per batch of loads
        float cur[U], nxt[U];
        auto load = [&](float (&dst)[U], int b) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int jr = b + 16 * u + sk;
                dst[u] = jr < ng ? scp[jr] : 0.0f;
            }
        };
        if (ng > 0) load(cur, 0);
        for (int b = 0; b < ng; b += 16 * U) {
            if (b + 16 * U < ng) load(nxt, b + 16 * U);    // the next batch in flight meanwhile
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (b + 16 * u >= ng) break;               // uniform over the pair's 16 lanes
                const int jr = b + 16 * u + sk;
                const float e = jr < ng ? exp_cephes(cur[u] - m) : 0.0f;
                if (ESTORE && jr < ng) scp[jr] = e;        // pass 3 reads e in place of the score
                const float e8 = __shfl_down(e, 8, 16);    // key jr + 8, from lane sk + 8
                if (sk < 8) {
                    ls = ls + e;
                    if (jr + 8 < ng) ls = ls + e8;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) cur[u] = nxt[u];
        }
        ls = ls + __shfl_xor(ls, 4);                       // lanes 8..15 hold 0 and stay among themselves
        ls = ls + __shfl_xor(ls, 2);
        ls = ls + __shfl_xor(ls, 1);
        if (valid && sk == 0) {
            float sum = ls;
            for (int jr = ng_p; jr < n_p; ++jr) {
                const float e = expf_libm(scp[jr] - m);
                if (ESTORE) scp[jr] = e;
                sum = sum + e;
            }
            inv_s[sp] = 1.0f / sum;
        }
        __syncthreads();
    } else {
        float ls = 0.0f;
        if (kl < kh) fetch(kg, kl);
        for (int j0 = kl; j0 < kh; j0 += ATT_KT) {
            __syncthreads();                               // E and the tile are free
            stage();
            __syncthreads();
            if (j0 + ATT_KT < kh) fetch(kg, j0 + ATT_KT);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int kt = sk + 16 * r, jr = j0 + kt - plo;
                if (!valid || jr < 0 || jr >= n_p) continue;
                const float s = score_d64(qv, tile + kt * ATT_KS, jr < ng_p) * scale;
                if (jr < ng_p) E[sp][kt] = exp_cephes(s - m);
                else tail_e[sp][jr - ng_p] = expf_libm(s - m);
            }
            __syncthreads();
            if (valid && sk < 8) {
                // the tile's keys jr = 8 i + sk (jr < ng) in order
                const int jt = j0 - plo;                   // jr of the tile's first key
                int kt0 = ((sk - jt) % 8 + 8) % 8;
                for (int kt = kt0; kt < ATT_KT; kt += 8) {
                    const int jr = jt + kt;
                    if (jr >= 0 && jr < ng_p) ls = ls + E[sp][kt];
                }
            }
        }
        ls = ls + __shfl_xor(ls, 4);                       // lanes 8..15 hold 0 and stay among themselves
        ls = ls + __shfl_xor(ls, 2);
        ls = ls + __shfl_xor(ls, 1);
        __syncthreads();                                   // tail_e written
        if (valid && sk == 0) {
            float sum = ls;
            for (int j = 0; j < n_p - ng_p; ++j) sum = sum + tail_e[sp][j];
            inv_s[sp] = 1.0f / sum;
        }
        __syncthreads();
    }
    const float inv = inv_s[sp];

    // pass 3: the weights, then the values
    const int d = tid & 63, pg = __builtin_amdgcn_readfirstlane(tid >> 6);
    int vlo[4], vn[4];
    float acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = hi_s[4 * pg + i] - lo_s[4 * pg + i];
        vlo[i] = __builtin_amdgcn_readfirstlane(lo_s[4 * pg + i]);
        vn[i] = __builtin_amdgcn_readfirstlane(n <= p.max_keys ? n : 0);
        acc[i] = 0.0f;
    }
    float snx[2] = { 0.0f, 0.0f };                          // STORED: the next tile's scores of this thread
    auto sfetch = [&](int j0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int jr = j0 + sk + 16 * r - plo;
            snx[r] = valid && jr >= 0 && jr < n_p ? scp[jr] : 0.0f;
        }
    };
    // ZW: a staged value tile holding a non-finite value (by tile parity), as attention_tile_kernel:
    // without one, a partial tile takes the broadcast path with zero weights outside a pair's keys
    __shared__ int vbad_s[2];
    if (tid < 2) vbad_s[tid] = 0;
    int par = 0;
    if (kl < kh) {
        fetch(STORED ? vg : kg, kl);
        if constexpr (STORED) sfetch(kl);
    }
    for (int j0 = kl; j0 < kh; j0 += ATT_KT, par ^= 1) {
        __syncthreads();                                   // E and the tile are free
        if (ZW && tid == 0) vbad_s[par ^ 1] = 0;           // the previous tile's flag, read by all
        stage();
        if constexpr (STORED) {
            if (ZW && !(finite4(pre[0]) && finite4(pre[1]))) vbad_s[par] = 1;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int kt = sk + 16 * r, jr = j0 + kt - plo;
                if (!valid || jr < 0 || jr >= n_p) {
                    if (ZW) E[sp][kt] = 0.0f;
                    continue;
                }
                const float s = snx[r];
                if (ESTORE) E[sp][kt] = s * inv;          // s holds e = exp(score - m), written by pass 2
                else E[sp][kt] = (jr < ng_p ? exp_cephes(s - m) : expf_libm(s - m)) * inv;
            }
            __syncthreads();                               // the values and the weights are in LDS
            if (j0 + ATT_KT < kh) {
                fetch(vg, j0 + ATT_KT);
                sfetch(j0 + ATT_KT);
            }
        } else {
            __syncthreads();
            fetch(vg, j0);                                 // this tile's values, staged after the weights
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int kt = sk + 16 * r, jr = j0 + kt - plo;
                if (!valid || jr < 0 || jr >= n_p) {
                    if (ZW) E[sp][kt] = 0.0f;
                    continue;
                }
                const float s = score_d64(qv, tile + kt * ATT_KS, jr < ng_p) * scale;
                E[sp][kt] = (jr < ng_p ? exp_cephes(s - m) : expf_libm(s - m)) * inv;
            }
            __syncthreads();                               // the keys have been read
            stage();
            if (ZW && !(finite4(pre[0]) && finite4(pre[1]))) vbad_s[par] = 1;
            __syncthreads();
            if (j0 + ATT_KT < kh) fetch(kg, j0 + ATT_KT);
        }
        const int jn = min(ATT_KT, kh - j0);
        // pair i's weights of the tile: lane l holds key j0 + l (l < 32), broadcast per key
        int a[4], b[4];
        bool full = ZW ? vbad_s[par] == 0 : jn == ATT_KT;
        float w0[4], w1[4];                                // keys j0 + k, j0 + 16 + k in lane k of each row
#pragma unroll
        for (int i = 0; i < 4; ++i) {                      // keys [a, b) of the tile are pair i's
            a[i] = min(max(vlo[i] - j0, 0), jn);
            b[i] = max(min(vlo[i] + vn[i] - j0, jn), a[i]);
            if (!ZW) full = full && a[i] == 0 && b[i] == jn;
            w0[i] = E[4 * pg + i][d & 15];
            w1[i] = E[4 * pg + i][16 + (d & 15)];
        }
        auto wk = [&](int i, int jj) {
            return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(jj < 16 ? w0[i] : w1[i]), jj & 15));
        };
        if (full) {
            float vt[ATT_KT];
#pragma unroll
            for (int jj = 0; jj < ATT_KT; ++jj) vt[jj] = tile[jj * ATT_KS + d];
            fmac_bcast4_16(acc, w0, vt);
            fmac_bcast4_16(acc, w1, vt + 16);
        } else {
            for (int jj = 0; jj < jn; ++jj) {
                const float v = tile[jj * ATT_KS + d];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (jj >= a[i] && jj < b[i]) acc[i] = __builtin_fmaf(wk(i, jj), v, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pp = 4 * pg + i, t = t0 + pp / rep, h = g * rep + pp % rep;
        if (t >= p.T) continue;
        const int n = hi_s[pp] - lo_s[pp];
        p.out[(size_t) t * p.H * 64 + (size_t) h * 64 + d] = (n > 0 && n <= p.max_keys) ? acc[i] : __uint_as_float(0x7fc00000u);
    }
}

__global__ __launch_bounds__(256) void attention_long_kernel(attn_params p) {
    attention_long_tile<false, false, true>(p, nullptr, (int) blockIdx.x);
}

// The scores kept in the workspace: a persistent grid, one slot of sc per workgroup, which
// takes tiles blockIdx.x, blockIdx.x + gridDim.x, ... ESTORE: pass 2 stores the exponentials.
// ZW (banded launches, where most value tiles are partial for some pair): partial tiles on the
// broadcast path (16,384 keys in bands of 2,601 5.27 -> 5.18 ms); without a band only a pair's
// last tile is partial, and the flags cost 1-2% (8,192 keys 8.31 -> 8.46 ms).
// Three workgroups per CU (at most 168 registers; 8 pairs per lane group in pass 1, as 16 would
// spill): 16,384 keys 40.9 -> 34.7 ms, 8,192 keys 10.2 -> 8.4 ms against two workgroups per CU with
// 16 pairs per group (256 registers); four per CU (128 registers) spill and lose 1-10%.
#ifndef NXG_ATT_STORED_MINB
#define NXG_ATT_STORED_MINB 3
#endif
template <bool ESTORE, bool ZW>
__global__ __launch_bounds__(256, NXG_ATT_STORED_MINB) void attention_stored_kernel(attn_params p, float * __restrict__ sc) {
    const int nq = ATT_P / (p.H / p.G);
    const int n_tiles = p.G * ((p.T + nq - 1) / nq);
    for (int bt = (int) blockIdx.x; bt < n_tiles; bt += (int) gridDim.x) {
        __syncthreads();                                   // the previous tile's shared reads are done
        attention_long_tile<true, ESTORE, ZW>(p, sc, bt);
    }
}

// tanh256 (src/nexterabert.cpp:103-117) lane by lane: big = (1 - t) / (1 + t) with t =
// exp256(|x| * -2) and x's sign bit ORed in, small = the fused odd polynomial * x, small
// where |x| < 0.1 (ordered: a NaN takes big).
__device__ __forceinline__ float tanh_ref(float x) {
    const uint32_t ux = __float_as_uint(x);
    const float ax = __uint_as_float(ux & 0x7fffffffu);
    const float t = exp_cephes(ax * -2.0f);
    const float big = __uint_as_float(__float_as_uint((1.0f - t) / (1.0f + t)) | (ux & 0x80000000u));
    const float x2 = x * x;
    float p = -17.0f / 315.0f;
    p = __builtin_fmaf(p, x2, 2.0f / 15.0f);
    p = __builtin_fmaf(p, x2, -1.0f / 3.0f);
    p = __builtin_fmaf(p, x2, 1.0f);
    const float small = p * x;
    return ax < 0.1f ? small : big;
}

// op_qk_prep (src/nexterabert.cpp:590-632): separable DyT then RoPE, one thread per (row,
// head, i < D/2): a = beta[i] tanh(alpha[i] x1[i]), b = beta[D/2+i] tanh(alpha[D/2+i] x2[i]),
// y1 = fma(a, cos, b sin), y2 = fma(-a, sin, b cos) at the row's position in its document.
// Output row-major [T][H*D] or head-major [H][T][D].
__device__ __forceinline__ void qk_prep_elem(const float * __restrict__ x, const float * __restrict__ alpha,
                                             const float * __restrict__ beta, const float * __restrict__ cos_t,
                                             const float * __restrict__ sin_t, const int32_t * __restrict__ cu,
                                             int n_seqs, int T, int H, int D, int n_pos, int head_major,
                                             float * __restrict__ out, int t, int h, int i) {
    const int half = D / 2;
    const doc_rows dr = doc_of(cu, n_seqs, t, T);
    const int pos = min(max(t - dr.lo, 0), n_pos - 1);
    const float c = cos_t[(size_t) pos * half + i], s = sin_t[(size_t) pos * half + i];
    const float * x1 = x + (size_t) t * H * D + (size_t) h * D;
    const float a = beta[i] * tanh_ref(alpha[i] * x1[i]);
    const float b = beta[half + i] * tanh_ref(alpha[half + i] * x1[half + i]);
    float * y = head_major ? out + ((size_t) h * T + t) * D : out + (size_t) t * H * D + (size_t) h * D;
    y[i] = __builtin_fmaf(a, c, b * s);
    y[half + i] = __builtin_fmaf(-a, s, b * c);
}

__global__ __launch_bounds__(256) void qk_prep_kernel(const float * __restrict__ x, const float * __restrict__ alpha,
                                                      const float * __restrict__ beta, const float * __restrict__ cos_t,
                                                      const float * __restrict__ sin_t, const int32_t * __restrict__ cu,
                                                      int n_seqs, int T, int H, int D, int n_pos, int head_major,
                                                      float * __restrict__ out) {
    // workgroup (row t, piece y) of a [T][H * D / 2] index space: no 64-bit divisions
    const int t = (int) blockIdx.x, half = D / 2;
    const int r = (int) blockIdx.y * 256 + (int) threadIdx.x;
    if (r >= H * half) return;
    qk_prep_elem(x, alpha, beta, cos_t, sin_t, cu, n_seqs, T, H, D, n_pos, head_major, out, t, r / half, r % half);
}

// op_head_major (src/nexterabert.cpp:620-632): [T][H*D] -> [H][T][D].
__device__ __forceinline__ void head_major_elem(const float * __restrict__ x, int T, int H, int D,
                                                float * __restrict__ out, int t, int h, int e) {
    out[((size_t) h * T + t) * D + e] = x[((size_t) t * H + h) * D + e];
}

__global__ __launch_bounds__(256) void head_major_kernel(const float * __restrict__ x, int T, int H, int D,
                                                         float * __restrict__ out) {
    const int t = (int) blockIdx.x;
    const int r = (int) blockIdx.y * 256 + (int) threadIdx.x;
    if (r >= H * D) return;
    head_major_elem(x, T, H, D, out, t, r / D, r % D);
}

// builder::attention's three ops on one layer's projections (src/nexterabert.cpp:1186-1188) in
// one launch: qk_prep of the queries (row-major), qk_prep of the keys (head-major) and the
// values' head-major copy. Workgroup (row t, piece y): thread r of the row's
// H * D / 2 + G * D / 2 + G * D elements takes one of them by index range.
struct qkv_prep_params {
    const float * q;
    const float * k;
    const float * v;
    const float * q_alpha;
    const float * q_beta;
    const float * k_alpha;
    const float * k_beta;
    const float * cos_t;
    const float * sin_t;
    const int32_t * cu;
    int n_seqs, T, H, G, D, n_pos;
    float * q_out;
    float * k_out;
    float * v_out;
};
__global__ __launch_bounds__(256) void qkv_prep_kernel(qkv_prep_params p) {
    const int t = (int) blockIdx.x, half = p.D / 2;
    const int r = (int) blockIdx.y * 256 + (int) threadIdx.x;
    const int nq = p.H * half, nk = p.G * half, nv = p.G * p.D;
    if (r < nq) {
        qk_prep_elem(p.q, p.q_alpha, p.q_beta, p.cos_t, p.sin_t, p.cu, p.n_seqs, p.T, p.H, p.D, p.n_pos, 0, p.q_out,
                     t, r / half, r % half);
    } else if (r < nq + nk) {
        qk_prep_elem(p.k, p.k_alpha, p.k_beta, p.cos_t, p.sin_t, p.cu, p.n_seqs, p.T, p.G, p.D, p.n_pos, 1, p.k_out,
                     t, (r - nq) / half, (r - nq) % half);
    } else if (r < nq + nk + nv) {
        head_major_elem(p.v, p.T, p.G, p.D, p.v_out, t, (r - nq - nk) / p.D, (r - nq - nk) % p.D);
    }
}

// ---------------------------------------------------------------------------
// Row ops writing fp32 rows (consumers that are not int8 linears, and the output)
// ---------------------------------------------------------------------------

// The rows a source produces as fp32 [T][C] (C % 4 == 0): 2^lg lanes per row, 4 columns
// per lane per step, 256 >> lg rows per workgroup.
template <typename Src>
__global__ __launch_bounds__(256) void produce_rows_kernel(Src src, int T, int C, int lg, float * __restrict__ out) {
    const int t = (int) blockIdx.x * (256 >> lg) + (int) (threadIdx.x >> lg);
    const int lane = (int) threadIdx.x & ((1 << lg) - 1);
    if (t >= T) return;
    const auto r = src.row(t);
    for (int col = 4 * lane; col < C; col += 4 << lg) {
        float v[4];
        src.load(r, t, col, v);
        *reinterpret_cast<v4f *>(out + (size_t) t * C + col) = v4f{ v[0], v[1], v[2], v[3] };
    }
}

// op_upsample_add (src/nexterabert.cpp:675-690): out[t] = yb[b] + r[t] with b = cub[d] +
// (t - cu[d]) / block the block row of t in its document d (clamped into the block rows).
struct src_upsample_add {
    const float * yb;
    const float * r;
    const int32_t * cu;
    const int32_t * cub;
    int n_seqs, T, n_blocks, C, block;
    __device__ int row(int t) const {
        const doc_rows d = doc_of(cu, n_seqs, t, T);
        return min(max(cub[d.d] + (t - d.lo) / block, 0), n_blocks - 1);
    }
    __device__ void load(int b, int t, int col, float (&v)[4]) const {
        const v4f y = *reinterpret_cast<const v4f *>(yb + (size_t) b * C + col);
        const v4f rv = *reinterpret_cast<const v4f *>(r + (size_t) t * C + col);
        v[0] = y.x + rv.x; v[1] = y.y + rv.y; v[2] = y.z + rv.z; v[3] = y.w + rv.w;
    }
};

// ggml_get_rows of the embedding (src/nexterabert.cpp:1271-1272) from a table held in
// fp32 (a block-quantized table is decoded once at load, the values to_float gives), plus
// the segment embedding's row where given (ggml_add: one fp32 addition). Ids are clamped
// into the tables so that any ids read in bounds; the host rejects bad ids first.
__global__ __launch_bounds__(256) void embed_rows_kernel(const float * __restrict__ table, int n_vocab,
                                                         const int32_t * __restrict__ ids,
                                                         const float * __restrict__ type_table, int n_types,
                                                         const int32_t * __restrict__ types, int T, int C, int lg,
                                                         float * __restrict__ out) {
    const int t = (int) blockIdx.x * (256 >> lg) + (int) (threadIdx.x >> lg);
    const int lane = (int) threadIdx.x & ((1 << lg) - 1);
    if (t >= T) return;
    const float * er = table + (size_t) min(max(ids[t], 0), n_vocab - 1) * C;
    const float * tr = type_table ? type_table + (size_t) min(max(types[t], 0), n_types - 1) * C : nullptr;
    for (int col = 4 * lane; col < C; col += 4 << lg) {
        v4f e = *reinterpret_cast<const v4f *>(er + col);
        if (tr) e = e + *reinterpret_cast<const v4f *>(tr + col);
        *reinterpret_cast<v4f *>(out + (size_t) t * C + col) = e;
    }
}

// ggml_norm (ggml v0.9.9's CPU op; ggml is not in the reference's tree) then ggml_mul by w
// and ggml_add of b (src/nexterabert.cpp:1290-1291, :1296-1297): mean = (float) sum(x) /
// C; v = x - mean; variance = (float) (sum((double) (v * v)) / C); y = v * (1 / sqrtf(
// variance + eps)); out = y * w + b, each operation rounded on its own. The sums are taken
// in double by one wave per row: lane l adds elements l + 64 j in order of j, then a
// butterfly over the 64 lanes (the same order in the oracle).
__global__ __launch_bounds__(256) void layer_norm_kernel(const float * __restrict__ x, const float * __restrict__ w,
                                                         const float * __restrict__ b, float eps, int T, int C,
                                                         float * __restrict__ out) {
    const int t = (int) blockIdx.x * 4 + (int) (threadIdx.x >> 6), lane = (int) threadIdx.x & 63;
    if (t >= T) return;                        // uniform across the wave
    const float * xr = x + (size_t) t * C;
    double s = 0.0;
    for (int i = lane; i < C; i += 64) s += (double) xr[i];
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    const float mean = (float) s / (float) C;
    double s2 = 0.0;
    for (int i = lane; i < C; i += 64) {
        const float v = xr[i] - mean;
        s2 += (double) (v * v);
    }
    for (int m = 32; m >= 1; m >>= 1) s2 += __shfl_xor(s2, m);
    const float variance = (float) (s2 / (double) C);
    const float scale = 1.0f / __builtin_sqrtf(variance + eps);
    float * o = out + (size_t) t * C;
    for (int i = lane; i < C; i += 64) {
        float y = (xr[i] - mean) * scale;
        if (w) y = y * w[i];
        if (b) y = y + b[i];
        o[i] = y;
    }
}

// The pooled vector of nextera_encode (src/nexterabert.cpp:1913-1925) and op_doc_mean
// (:659-672): the sum of the document's rows in row order (axpy_f32 with weight 1, one
// rounding per row) times 1 / n -- or, with normalize, times 1 / sqrt(dot_f32(p, p)) (0
// for a zero vector; dot in the reference's order, C % 32 == 0).
//
// doc_sum_kernel: one workgroup per (document, 32-column slice). The row order fixes one
// dependent chain of adds per column, so the slice's 32 columns are summed by 32 lanes of
// wave 0 out of LDS, while all 256 threads stream the next 256-row chunk of the slice
// (128-byte row pieces, one float4 per thread and row group) into registers. mean != 0
// applies 1 / n; otherwise the raw sums are written for doc_norm_kernel.
constexpr int DS_COLS = 32, DS_ROWS = 256;
__global__ __launch_bounds__(256) void doc_sum_kernel(const float * __restrict__ x, const int32_t * __restrict__ cu,
                                                      int T, int C, int n_slices, int mean, float * __restrict__ out) {
    __shared__ __attribute__((aligned(16))) float tile[DS_ROWS * DS_COLS];
    const int d = (int) blockIdx.x / n_slices, c0 = ((int) blockIdx.x % n_slices) * DS_COLS;
    const int lo = min(max(cu[d], 0), T), hi = min(max(cu[d + 1], lo), T);
    const int tid = (int) threadIdx.x;
    const int lr = tid >> 3, lc = (tid & 7) * 4;              // row in a 32-row group, column in the slice
    const bool col_ok = c0 + lc < C;                          // C % 4 == 0: a float4 is all in or all out
    const float * xs = x + c0 + lc;
    v4f buf[DS_ROWS / 32];
    auto load = [&](int base) {
#pragma unroll
        for (int j = 0; j < DS_ROWS / 32; ++j) {
            const int r = base + lr + 32 * j;
            buf[j] = (col_ok && r < hi) ? *reinterpret_cast<const v4f *>(xs + (size_t) r * C) : v4f{ 0.0f, 0.0f, 0.0f, 0.0f };
        }
    };
    float acc = 0.0f;
    load(lo);
    for (int base = lo; base < hi; base += DS_ROWS) {
#pragma unroll
        for (int j = 0; j < DS_ROWS / 32; ++j) *reinterpret_cast<v4f *>(tile + (lr + 32 * j) * DS_COLS + lc) = buf[j];
        __syncthreads();
        if (base + DS_ROWS < hi) load(base + DS_ROWS);
        if (tid < DS_COLS) {
            const int n = min(DS_ROWS, hi - base);
            if (n == DS_ROWS) {
#pragma unroll 32
                for (int r = 0; r < DS_ROWS; ++r) acc = acc + tile[r * DS_COLS + tid];
            } else {
                for (int r = 0; r < n; ++r) acc = acc + tile[r * DS_COLS + tid];
            }
        }
        __syncthreads();
    }
    if (tid < DS_COLS && c0 + tid < C) out[(size_t) d * C + c0 + tid] = mean ? acc * (1.0f / (float) (hi - lo)) : acc;
}

// doc_norm_kernel: one workgroup per document scales its column sums by 1 / sqrt(dot_f32(p, p))
// (0 for a zero vector), the dot on 16 lanes in the reference's order.
__global__ __launch_bounds__(256) void doc_norm_kernel(int C, float * __restrict__ out) {
    __shared__ float scale_s;
    float * p = out + (size_t) blockIdx.x * C;
    if (threadIdx.x < 16) {
        const float dot = dot_sq_ref16(p, C, (int) threadIdx.x);
        if (threadIdx.x == 0) {
            const float nrm = __builtin_sqrtf(dot);
            scale_s = nrm > 0.0f ? 1.0f / nrm : 0.0f;
        }
    }
    __syncthreads();
    const float scale = scale_s;
    for (int col = 4 * (int) threadIdx.x; col < C; col += 1024) {
        const v4f a = *reinterpret_cast<const v4f *>(p + col);
        *reinterpret_cast<v4f *>(p + col) = v4f{ a.x * scale, a.y * scale, a.z * scale, a.w * scale };
    }
}

// int8 tiles -> the reference's u8 rows (q + act_off); one thread per 16 bytes.
__global__ void export_kernel(const int8_t * __restrict__ q, int T, int n_in, int KS, int act_off,
                              uint8_t * __restrict__ u8) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int chunks = n_in / 16;
    if (i >= (size_t) T * chunks) return;
    const int t = (int) (i / chunks), k = (int) (i % chunks) * 16;
    const size_t src = ((size_t) (t >> 4) * KS + (k >> 6)) * FRAG + (size_t) ((t & 15) + 16 * ((k & 63) >> 4)) * 16;
    const int4 v = *reinterpret_cast<const int4 *>(q + src);
    const int w[4] = { v.x, v.y, v.z, v.w };
    int o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int r = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int s = (int) (int8_t) (w[j] >> (8 * b));
            r |= ((s + act_off) & 0xff) << (8 * b);
        }
        o[j] = r;
    }
    *reinterpret_cast<int4 *>(u8 + (size_t) t * n_in + k) = make_int4(o[0], o[1], o[2], o[3]);
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------

struct gemm_params {
    const int8_t * a;     // qact tiles
    const float *  sx;    // [MP/4][n_blk][4]
    const int8_t * w;     // weight tiles, NP rows
    const float *  sw;    // [n_blk][NP]
    const float *  res;   // [T][N] or null
    float *        out;   // [T][N]
    int32_t *      sums;  // [n_blk][T][N] (block-sum variant)
    int T, N, NP, KS, n_blk, MF, n_mt, n_nt;
    int G;                // tiles: n_mt * n_nt
    // relu^2 -> int8 output (gemm_wide): the next linear's activation tiles, N channels
    int8_t *       qo;    // MF x KSo fragments
    float *        sxo;   // [MP/4][n_nt][4]
    int KSo;              // ceil(N / 64)
    // fp32 input rows [T][n_in] quantized inside the relu^2 row-tile kernel (instead of a, sx)
    const float *  xf;
    // split output (0: none): columns [seg_end[k-1], seg_end[k]) go to seg_out[k], a dense
    // [T][seg_end[k] - seg_end[k-1]] array; every boundary is a multiple of 64
    int n_seg;
    int seg_end[4];
    float * seg_out[4];
};

// Where output column n of row t goes: base + t * ld + col.
typedef out_col<float *> out_map;
__device__ __forceinline__ out_map out_of(const gemm_params & p, int n) {
    return out_col_of<float *>(n, p.N, p.n_seg, p.seg_end, p.out, p.seg_out);
}

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at
// LDS address lds + 16 l (global_load_lds_dwordx4; M0 holds the wave's LDS base).
// Issued from inline asm so that the compiler's wait-count pass does not track it
// (it would drain every prefetch at the loop back-edge); each use is synchronized
// explicitly with wait_vm before the barrier that precedes its readers.
__device__ __forceinline__ void dma16l(const void * gptr, uint32_t la) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(gptr), "s"(la) : "memory", "m0");
}
__device__ __forceinline__ void dma16(const void * gptr, const void * lds) {
    dma16l(gptr, (uint32_t) (uintptr_t) (lds_void *) lds);
}

// Waits until at most n of this wave's vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Workgroup barrier for the LDS ring. __syncthreads() (and any fence on LDS) makes
// every wave wait for all of its outstanding loads, since LDS-DMA writes count as
// pending LDS stores -- including the prefetches of later k-steps that must stay in
// flight. Here the LDS-DMA of the k-step about to be read is waited for explicitly
// (wait_vm) before the barrier, and the barrier itself only drains this wave's own
// LDS reads and writes. The "memory" clobber keeps the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One workgroup: 4 waves (2 x 2), each computing a 64 x 64 piece of a 128 x 128
// output tile with v_mfma_i32_16x16x64_i8, the weight fragment as the MFMA's A
// operand and the activation fragment as its B operand. A lane then holds, for
// each 16 x 16 piece, 4 consecutive output features of one token: out[t][n..n+3].
// Per 256-input block the int32 sums are folded into fp32 with the reference's
// step f = fma((float) s * sx[t], sw[n], f); the block's scales come through LDS.
// With K256 (n_in a multiple of 256) a workgroup walks several tiles and its LDS
// ring runs on across them; otherwise it computes one tile.
template <bool RES, bool SUMS, bool K256>
__global__ __launch_bounds__(NTHREADS, 2) void gemm_kernel(gemm_params p) {
    __shared__ __attribute__((aligned(1024))) int8_t s0[SLOT];
    __shared__ __attribute__((aligned(1024))) int8_t s1[SLOT];
    __shared__ __attribute__((aligned(1024))) int8_t s2[SLOT];
    __shared__ __attribute__((aligned(1024))) int8_t s3[SLOT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const tile_walk walk(blockIdx.x, gridDim.x, p.G);
    if (walk.count == 0) return;
    const int n_steps = walk.count * p.KS;   // k-steps of all this workgroup's tiles

    // Scales of block B of tile (mt, nt) for lane l of wave 0: l < 32 sx of row group
    // l of the tile, l >= 32 sw of columns 4(l-32)..+3.
    auto scale_src = [&](int mt, int nt, int B) -> const float * {
        if (lane < 32) return p.sx + sx_group_index(mt, lane, p.MF, p.n_blk, B);
        return p.sw + sw_index(B, p.NP, nt * BN + 4 * (lane - 32));
    };

    // The load stream: k-steps in order, across this workgroup's tiles. Wave w moves
    // fragments w and w+4 of A and of B, 1 KiB each. A fragment rows past the last
    // row of A re-read its last fragment row (those output rows are never stored),
    // so that every wave issues exactly 4 loads per k-step: the waits count on it.
    // Wave 0 also loads a block's scales with the block's last k-step (slot 3).
    int iss_it = 0, iss_ks = 0;          // next k-step to load
    int iss_mt = 0, iss_nt = 0;
    const int8_t * ia0 = nullptr;
    const int8_t * ia1 = nullptr;
    const int8_t * ib0 = nullptr;
    const int8_t * ib1 = nullptr;
    auto issue_tile = [&]() {            // per-lane sources of k-step 0 of tile iss_it
        const int tile = walk.tile(iss_it);
        iss_mt = tile / p.n_nt;
        iss_nt = tile - iss_mt * p.n_nt;
        ia0 = p.a + frag_byte(a_frag(iss_mt, wave, p.MF), p.KS, 0, lane);
        ia1 = p.a + frag_byte(a_frag(iss_mt, wave + 4, p.MF), p.KS, 0, lane);
        ib0 = p.w + frag_byte(w_frag(iss_nt, BN, wave), p.KS, 0, lane);
        ib1 = p.w + frag_byte(w_frag(iss_nt, BN, wave + 4), p.KS, 0, lane);
    };
    issue_tile();
    auto issue = [&](int8_t * slot) {
        if (iss_it >= walk.count) return;
        const size_t o = (size_t) iss_ks * FRAG;
        dma16(ia0 + o, slot + wave * FRAG);
        dma16(ia1 + o, slot + (wave + 4) * FRAG);
        dma16(ib0 + o, slot + (8 + wave) * FRAG);
        dma16(ib1 + o, slot + (12 + wave) * FRAG);
        if (!SUMS && wave == 0 && (iss_ks & 3) == 3) dma16(scale_src(iss_mt, iss_nt, iss_ks >> 2), s3 + SLOT_AB);
        if (++iss_ks == p.KS) {
            iss_ks = 0;
            if (++iss_it < walk.count) issue_tile();
        }
    };

    // Wait for k-step g's slot: the loads of later k-steps (up to two, 4 per wave each,
    // plus one scale load on wave 0) may stay in flight.
    auto arrive = [&](int g) {
        const int later = min(2, n_steps - 1 - g);
        if (later >= 2) wait_vm<8>();
        else if (later == 1) wait_vm<4>();
        else wait_vm<0>();
        lds_barrier();
    };

    v4i acc[4][4];
    float f[4][4][4];

    auto mma = [&](const int8_t * slot, bool first) {
        v4i a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = *reinterpret_cast<const v4i *>(slot + (wm * 4 + i) * FRAG + lane * 16);
            b[i] = *reinterpret_cast<const v4i *>(slot + (8 + wn * 4 + i) * FRAG + lane * 16);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                acc[mi][ni] = first
                    ? __builtin_amdgcn_mfma_i32_16x16x64_i8(b[ni], a[mi], v4i{0, 0, 0, 0}, 0, 0, 0)
                    : __builtin_amdgcn_mfma_i32_16x16x64_i8(b[ni], a[mi], acc[mi][ni], 0, 0, 0);
    };

    issue(s0);
    issue(s1);
    issue(s2);
    for (int it = 0; it < walk.count; ++it) {
        const int tile = walk.tile(it);
        const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
        // this lane's outputs: token t0 + mi*16, features n0 + ni*16 + 0..3
        const int t0 = mt * BM + wm * 64 + (lane & 15);
        const int n0 = nt * BN + wn * 64 + 4 * (lane >> 4);

        const int g0 = it * p.KS;
        for (int B = 0; B < p.n_blk; ++B) {
            const int g = g0 + 4 * B;
            const int nks = K256 ? 4 : min(4, p.KS - 4 * B);
            arrive(g);
            issue(s3);
            mma(s0, true);
            if (K256 || nks > 1) {
                arrive(g + 1);
                issue(s0);
                mma(s1, false);
            }
            if (K256 || nks > 2) {
                arrive(g + 2);
                issue(s1);
                mma(s2, false);
            }
            if (K256 || nks > 3) {
                arrive(g + 3);
                issue(s2);
                mma(s3, false);
            } else if (!SUMS) {
                // Partial last block (one tile per workgroup here): there is no k-step
                // 4B+3 to bring its scales, so fetch them now. s3's scale area is free:
                // its last readers (block B-1's epilogue) have all passed arrive(4B).
                if (wave == 0) dma16(scale_src(mt, nt, B), s3 + SLOT_AB);
                wait_vm<0>();
                lds_barrier();
            }

            if (SUMS) {
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int t = t0 + mi * 16, n = n0 + ni * 16 + r;
                            if (t < p.T && n < p.N) p.sums[((size_t) B * p.T + t) * p.N + n] = acc[mi][ni][r];
                        }
            } else {
                // f = fma((float) s * sx[t, B], sw[B, n], f): the reference's per-block step.
                const float * scl = reinterpret_cast<const float *>(s3 + SLOT_AB);
                float sxv[4];
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) sxv[mi] = scl[wm * 64 + mi * 16 + (lane & 15)];
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const float4 sw4 = *reinterpret_cast<const float4 *>(scl + 128 + wn * 64 + ni * 16 + 4 * (lane >> 4));
                    const float swr[4] = { sw4.x, sw4.y, sw4.z, sw4.w };
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float prod = (float) acc[mi][ni][r] * sxv[mi];
                            // block 0 starts from f = 0: fma(prod, sw, +0.0)
                            f[mi][ni][r] = __builtin_fmaf(prod, swr[r], B == 0 ? 0.0f : f[mi][ni][r]);
                        }
                }
            }
        }

        if (!SUMS) {
            if ((p.N & 3) == 0) {
                // Full-line stores through LDS. After the tile's last epilogue slot 3 is
                // free (the next tile's k-step 3 is loaded only after the next barrier):
                // each wave owns 4352 bytes of it, 16 rows of 64 floats at a 272-byte
                // pitch. Per 16-token piece mi: write it in MFMA order (lane: token
                // lane%16, features 16ni + 4(lane/16) + 0..3), read it back as 4 rows of
                // 256 bytes per instruction, and store whole 128-byte lines.
                lds_barrier();
                float * stg = reinterpret_cast<float *>(s3 + wave * STAGE_BYTES);
                const int trow = lane & 15, tcol = 4 * (lane >> 4);
                const int rrow = lane >> 4, rcol = 4 * (lane & 15);
                const int tbase = mt * BM + wm * 64, nb = nt * BN + wn * 64 + rcol;
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni) {
                        const v4f y = { f[mi][ni][0], f[mi][ni][1], f[mi][ni][2], f[mi][ni][3] };
                        *reinterpret_cast<v4f *>(stg + trow * STAGE_PITCH + 16 * ni + tcol) = y;
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int row = 4 * q + rrow;
                        v4f y = *reinterpret_cast<const v4f *>(stg + row * STAGE_PITCH + rcol);
                        const int t = tbase + mi * 16 + row;
                        if (t < p.T && nb < p.N) {
                            const size_t o = (size_t) t * p.N + nb;
                            if (RES) y = *reinterpret_cast<const v4f *>(p.res + o) + y;
                            __builtin_nontemporal_store(y, reinterpret_cast<v4f *>(p.out + o));
                        }
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                }
            } else {
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) {
                    const int t = t0 + mi * 16;
                    if (t >= p.T) continue;
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni) {
                        const int n = n0 + ni * 16;
                        const size_t o = (size_t) t * p.N + n;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (n + r < p.N) {
                                const float y = RES ? p.res[o + r] + f[mi][ni][r] : f[mi][ni][r];
                                __builtin_nontemporal_store(y, p.out + o + r);
                            }
                        }
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMM for n_in % 256 == 0 and N % 4 == 0: the projections of the encoder
// ---------------------------------------------------------------------------

// A 64-bit pointer that the compiler can see is the same in every lane, so that it
// lives in an SGPR pair.
__device__ __forceinline__ const int8_t * uniform_ptr(const int8_t * ptr) {
    const uint64_t v = (uint64_t) (uintptr_t) ptr;
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (v >> 32));
    return reinterpret_cast<const int8_t *>((uintptr_t) (((uint64_t) hi << 32) | lo));
}

// This lane's number, computed where it is used: an asm the compiler cannot hoist, so
// that values derived from it are not kept live across a loop (register pressure).
__device__ __forceinline__ int lane_here() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// A raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3): buffer
// loads take a scalar base, a scalar offset and one vector offset, so that a wave's
// address arithmetic stays on the scalar unit, and they count in vmcnt only.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void * base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short) 0, (int) bytes, 0x00020000);
}
// 16 bytes per lane at byte soff (wave-uniform) + voff (per lane) of the buffer.
__device__ __forceinline__ v4i bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int) voff, (int) soff, 0);
}

// dma16 from a scalar base: lane l copies the 16 bytes at base + voff_l to LDS
// address lds + 16 l. The address arithmetic stays on the scalar unit.
__device__ __forceinline__ void dma16s(const int8_t * base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(voff), "s"(base), "s"(lds) : "memory", "m0");
}

// The same tiles, warps and per-block epilogue as gemm_kernel, with a load
// schedule that has no data-dependent branches inside a tile:
//  - k-step g of the walk lives in ring slot g % 4; because a tile has a multiple
//    of 4 k-steps, the slot of each k-step of a block is a compile-time constant;
//  - a k-step is read from LDS one step ahead, into the second of two operand sets:
//    the barrier of step g publishes k-step g + 1 and certifies that every wave has
//    read k-step g, so each wave then loads its 4 fragments of k-step g + 4 into slot
//    g % 4 and reads k-step g + 1 among k-step g's MFMAs; the last block loads the
//    next tile's k-steps 0..2 (past the last tile, the last tile again: harmless
//    re-reads that keep the counts constant); wave 0 adds block B's scales at k-step 4B;
//  - the wait at each k-step is therefore a constant vmcnt: 8, or 9 on wave 0 for
//    the two k-steps whose later loads include its scale load;
//  - the output phase issues its stores at once (they write slot 3, which the last
//    block leaves unloaded); vmcnt counts the stores too, so the next tile starts by
//    waiting for every outstanding operation (its k-steps 0..2 and the stores), then
//    loads its k-step 3 into slot 3, and the constant counts resume.
// The residual rows are loaded after the tile's last MFMAs, under the last epilogue.
template <bool RES>
__global__ __launch_bounds__(NTHREADS, 2) void gemm_k256(gemm_params p) {
    __shared__ __attribute__((aligned(1024))) int8_t ring[4 * SLOT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const tile_walk walk(blockIdx.x, gridDim.x, p.G);
    if (walk.count == 0) return;
    const int nb = p.KS >> 2;                        // 256-input blocks per tile
    const size_t frow = (size_t) p.KS * FRAG;        // bytes of one fragment row
    const uint32_t ring_lds = (uint32_t) (uintptr_t) (lds_void *) ring;
    const uint32_t lane16 = (uint32_t) lane * 16;

    struct frag_rows {                               // this wave's 4 fragment rows of a tile
        const int8_t * a0;
        const int8_t * a1;
        const int8_t * w0;
        const int8_t * w1;
    };
    // Tile i of the walk (clamped to the last one). A fragment rows past the last
    // row of A re-read its last fragment row; those output rows are never stored.
    auto rows_of = [&](int i) {
        const int tile = walk.tile_clamped(i);
        const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
        frag_rows r;
        r.a0 = uniform_ptr(p.a + (size_t) a_frag(mt, wave, p.MF) * frow);
        r.a1 = uniform_ptr(p.a + (size_t) a_frag(mt, wave + 4, p.MF) * frow);
        r.w0 = uniform_ptr(p.w + (size_t) w_frag(nt, BN, wave) * frow);
        r.w1 = uniform_ptr(p.w + (size_t) w_frag(nt, BN, wave + 4) * frow);
        return r;
    };
    // k-step ks of a tile into ring slot j: A fragments w and w + 4 of the slot,
    // then B fragments w and w + 4.
    auto issue = [&](const frag_rows & r, int ks, int j) {
        const uint32_t vo = lane16 + (uint32_t) ks * FRAG;
        const uint32_t m = ring_lds + (uint32_t) (j * SLOT + wave * FRAG);
        dma16s(r.a0, vo, m);
        dma16s(r.a1, vo, m + 4 * FRAG);
        dma16s(r.w0, vo, m + 8 * FRAG);
        dma16s(r.w1, vo, m + 12 * FRAG);
    };

    v4i acc[4][4];
    float f[4][4][4];
    v4i oa[2][4], ob[2][4];                          // operand sets: k-step g in set g % 2
    auto rd = [&](int j, int set) {
        const int8_t * slot = ring + j * SLOT;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            oa[set][i] = *reinterpret_cast<const v4i *>(slot + (wm * 4 + i) * FRAG + lane * 16);
            ob[set][i] = *reinterpret_cast<const v4i *>(slot + (8 + wn * 4 + i) * FRAG + lane * 16);
        }
    };
    auto mm = [&](int set, bool first, int m0, int m1) {
#pragma unroll
        for (int mi = m0; mi < m1; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                acc[mi][ni] = first
                    ? __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[set][ni], oa[set][mi], v4i{0, 0, 0, 0}, 0, 0, 0)
                    : __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[set][ni], oa[set][mi], acc[mi][ni], 0, 0, 0);
    };

    {
        const frag_rows r0 = rows_of(0);
        issue(r0, 0, 0);
        issue(r0, 1, 1);
        issue(r0, 2, 2);
        wait_vm<0>();
    }
    // The tile walk, instantiated for one 256-input block per tile and for several, so that
    // whether a block's fold starts from +0 is static in every block.
    auto walk_tiles = [&](auto one_tag) {
        constexpr bool one = decltype(one_tag)::value;
        for (int it = 0; it < walk.count; ++it) {
            const int tile = walk.tile(it);
            const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
            const frag_rows cur = rows_of(it), nxt = rows_of(it + 1);
            // wave 0's scale loads: lane l < 32 the sx of row group l of the tile, lane
            // l >= 32 the sw of columns 4(l-32)..+3; block B adds B * sstep bytes.
            const float * ssrc;
            size_t sstep;
            if (lane < 32) {
                ssrc = p.sx + sx_group_index(mt, lane, p.MF, p.n_blk, 0);
                sstep = 4 * sizeof(float);
            } else {
                ssrc = p.sw + sw_index(0, p.NP, nt * BN + 4 * (lane - 32));
                sstep = (size_t) p.NP * sizeof(float);
            }
            v4f rv[4][4];                                // residual rows (RES)
            const int rrow = lane >> 4, rcol = 4 * (lane & 15);
            const int tbase = mt * BM + wm * 64, ncol = nt * BN + wn * 64 + rcol;
            const bool col_ok = ncol < p.N;
            // Tile start: every outstanding operation (the tile's k-steps 0..2, loaded under the
            // previous tile, and that tile's output stores) done, slot 3 free of the staged
            // output, then k-step 3 into slot 3 and k-step 0 into operand set 0.
            wait_vm<0>();
            lds_barrier();
            issue(cur, 3, 3);
            rd(0, 0);
            // Residual rows of pieces m0 and m0 + 1 (half before the last epilogue, half
            // after it, to stay within the register budget), read once: nontemporal loads, which
            // leave L2 to the operand tiles. Full row tiles: a scalar row
            // base plus one 32-bit lane offset; the last row tile clamps rows to T - 1
            // (never stored). Columns past N read the last 4 columns (never stored).
            auto load_res = [&](int m0) {
                const int row0 = mt * BM + wm * 64;
                const uint32_t col = (uint32_t) clamp_col4(ncol, p.N);
                if (row0 + 64 <= p.T) {
                    const uint32_t lo = (uint32_t) rrow * (uint32_t) p.N + col;
#pragma unroll
                    for (int mi = m0; mi < m0 + 2; ++mi)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            rv[mi][q] = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p.res + (size_t) (row0 + mi * 16 + 4 * q) * p.N + lo));
                } else {
#pragma unroll
                    for (int mi = m0; mi < m0 + 2; ++mi)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int t = clamp_row(row0 + mi * 16 + 4 * q + rrow, p.T);
                            rv[mi][q] = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p.res + (size_t) t * p.N + col));
                        }
                }
            };

            // One 256-input block: its 4 k-steps, then the epilogue. LAST: the tile's last
            // block, whose k-steps 1..3 load the next tile's first three.
            auto run_block = [&](int B, auto last_tag, auto first_tag) {
                constexpr bool last = decltype(last_tag)::value, first = decltype(first_tag)::value;
                // Step s (k-step g = 4B + s, in registers since step s - 1): publish k-step g + 1
                // and certify that every wave has read k-step g, load k-step g + 4 into slot s
                // (in the last block the next tile's k-step s; its k-step 3 waits for the tile
                // start, slot 3 staging the output), read k-step g + 1 among k-step g's MFMAs.
                auto step = [&](auto s_tag) {
                    constexpr int s = decltype(s_tag)::value;
                    if ((s == 1 || s == 2) && wave == 0) wait_vm<9>();
                    else wait_vm<8>();
                    lds_barrier();
                    const ring_load l = ring_prefetch(it, B, s, last, true);
                    if (l.pos >= 0) issue(l.pos == it ? cur : nxt, l.ks, l.slot);
                    if (s == 0 && wave == 0) dma16(reinterpret_cast<const char *>(ssrc) + (size_t) B * sstep, ring + 3 * SLOT + SLOT_AB);
                    mm(s & 1, s == 0, 0, 3);
                    if (!(last && s == 3)) rd((s + 1) & 3, (s + 1) & 1);
                    mm(s & 1, s == 0, 3, 4);
                };
                // Wave priority: k-steps 2, fold 1, output 0 (s_setprio). A SIMD holds one wave
                // of each of the CU's two workgroups; when both have an instruction ready, the
                // one feeding the matrix core issues first, and a workgroup writing its output
                // yields to the other's k-loop.
                __builtin_amdgcn_s_setprio(2);
                step(std::integral_constant<int, 0>{});
                step(std::integral_constant<int, 1>{});
                step(std::integral_constant<int, 2>{});
                step(std::integral_constant<int, 3>{});
                if (RES && last) load_res(0);
                __builtin_amdgcn_s_setprio(1);

                // f = fma((float) s * sx[t, B], sw[B, n], f): the reference's per-block step.
                const float * scl = reinterpret_cast<const float *>(ring + 3 * SLOT + SLOT_AB);
                float sxv[4];
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) sxv[mi] = scl[wm * 64 + mi * 16 + (lane & 15)];
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const float4 sw4 = *reinterpret_cast<const float4 *>(scl + 128 + wn * 64 + ni * 16 + 4 * (lane >> 4));
                    const float swr[4] = { sw4.x, sw4.y, sw4.z, sw4.w };
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float prod = (float) acc[mi][ni][r] * sxv[mi];
                            // block 0 starts from f = 0: fma(prod, sw, +0.0)
                            f[mi][ni][r] = __builtin_fmaf(prod, swr[r], first ? 0.0f : f[mi][ni][r]);
                        }
                }
                if (RES && last) load_res(2);
            };
            if constexpr (one) {
                run_block(0, std::true_type{}, std::true_type{});
            } else {
                run_block(0, std::false_type{}, std::true_type{});
                for (int B = 1; B < nb - 1; ++B) run_block(B, std::false_type{}, std::false_type{});
                run_block(nb - 1, std::true_type{}, std::false_type{});
            }
            __builtin_amdgcn_s_setprio(0);

            // Output through LDS, whole 128-byte lines per store. Slot 3 is free once
            // every wave has passed this barrier (the next tile's k-step 3 is loaded only
            // after its first barrier); each wave owns 4352 bytes of it, 16 rows of 64
            // floats at a 272-byte pitch. Per 16-token piece mi: write it in MFMA order
            // (lane: token lane%16, features 16ni + 4(lane/16) + 0..3), read it back as 4
            // rows of 256 bytes per instruction and store whole lines.
            lds_barrier();
            const out_map om = out_of(p, ncol);
            float * stg = reinterpret_cast<float *>(ring + 3 * SLOT + wave * STAGE_BYTES);
            const int trow = lane & 15, tcol = 4 * (lane >> 4);
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const v4f y = { f[mi][ni][0], f[mi][ni][1], f[mi][ni][2], f[mi][ni][3] };
                    *reinterpret_cast<v4f *>(stg + trow * STAGE_PITCH + 16 * ni + tcol) = y;
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                // the piece's 4 reads first, then its stores: one LDS round trip per piece
                // (the empty asm keeps the compiler from sinking each read into its store's branch)
                v4f y[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) y[q] = *reinterpret_cast<const v4f *>(stg + (4 * q + rrow) * STAGE_PITCH + rcol);
                asm volatile("s_waitcnt lgkmcnt(0)" :: "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]) : "memory");
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int t = tbase + mi * 16 + 4 * q + rrow;
                    if (t < p.T && col_ok) {
                        const v4f o = RES ? rv[mi][q] + y[q] : y[q];
                        __builtin_nontemporal_store(o, reinterpret_cast<v4f *>(om.base + (size_t) t * om.ld + om.col));
                    }
                }
                // The residual rows count as used on every path: where no lane of a store is
                // active, the compiler would otherwise wait for their loads (vmcnt(0), draining
                // the prefetched k-steps) only where the next tile first writes those registers.
                if (RES) asm volatile("" :: "v"(rv[mi][0]), "v"(rv[mi][1]), "v"(rv[mi][2]), "v"(rv[mi][3]));
            }
        }
    };
    if (nb == 1) walk_tiles(std::true_type{});
    else         walk_tiles(std::false_type{});
    wait_vm<0>();
}

// ---------------------------------------------------------------------------
// GEMMs for few rows: latency-bound, so operands go straight to registers
// ---------------------------------------------------------------------------

// sw of blocks 0 .. n_blk - 1 for the nw features n0 .. n0 + nw - 1 into LDS, sl[B * nw + c].
// nw divides 256 and n0 is a multiple of nw, so the rows exist (NP is a multiple of 256).
template <int NW>
__device__ __forceinline__ void small_sw_fill(const gemm_params & p, int n0, float * sl) {
    for (int i = threadIdx.x; i < p.n_blk * (NW / 4); i += blockDim.x) {
        const int B = i / (NW / 4), c = (i - B * (NW / 4)) * 4;
        *reinterpret_cast<v4f *>(sl + B * NW + c) = *reinterpret_cast<const v4f *>(p.sw + sw_index(B, p.NP, n0 + c));
    }
}

// One wave's 32 x 16FN piece: tokens of fragment rows 2mt, 2mt + 1, features of weight
// fragment rows nr0 .. nr0 + FN - 1. Per k-step the wave loads its 2 + FN fragments
// (1 KiB each, one dwordx4 per lane, already in MFMA operand order) from global memory
// straight into registers, D k-steps ahead, so that it keeps that many k-steps of
// loads in flight however little it computes per k-step. The MFMA operands, the lane
// layout of the accumulators and the per-block epilogue f = fma((float) s * sx[t], sw[n], f)
// are those of gemm_kernel: f[j][i][r] is token 16(2mt + j) + lane % 16, feature
// 16(nr0 + i) + 4(lane / 16) + r. sx is loaded one block ahead; sw comes from LDS,
// swl[B * PITCH + 16 i + 4(lane / 16)], written by fill() once the first k-steps' loads
// are in flight (so that its wait for its own loads costs no extra round trip) and
// published by the workgroup barrier that follows it here. last() runs at the start of
// the last block (the caller's residual loads then overlap its MFMAs). With K256
// (n_in % 256 == 0) no k-step is loaded twice; otherwise the last block has fewer than
// 4 k-steps and refills past the last k-step re-read it.
template <int FN, bool K256, int PITCH, typename Fill, typename Last>
__device__ __forceinline__ void small_piece(const gemm_params & p, int mt, int nr0, const float * swl,
                                            float (&f)[SDT][FN][4], Fill fill, Last last) {
    constexpr int NF = SDT + FN;           // fragments per k-step
    constexpr int D = small_depth(FN);
    static_assert(D == 4 || D == 8, "k-steps in flight: one or two blocks");
    const int lane = threadIdx.x & 63;
    const int nb = p.n_blk;
    const size_t frow = (size_t) p.KS * FRAG;

    // Fragment rows past the activation's last re-read its last one (their outputs are
    // not stored). Weight rows are padded to a multiple of 256: rows nr0 .. nr0 + FN - 1
    // exist when 16 nr0 < N and nr0 is a multiple of FN.
    int fr[SDT];
    const int8_t * base[NF];               // fragment rows, uniform
#pragma unroll
    for (int j = 0; j < SDT; ++j) {
        fr[j] = small_a_frag(mt, j, p.MF);
        base[j] = p.a + fr[j] * frow;
    }
#pragma unroll
    for (int i = 0; i < FN; ++i) base[SDT + i] = p.w + (nr0 + i) * frow;
    const uint32_t lane16 = (uint32_t) lane * 16;

    v4i buf[D][NF];
    // k-step ks (< KS) into d. The scheduling barrier keeps each k-step's loads where
    // they are issued: the compiler would otherwise sink them towards their first use
    // and shorten the prefetch.
    auto load = [&](v4i (&d)[NF], int ks) {
        const size_t ko = (size_t) ks * FRAG;
#pragma unroll
        for (int u = 0; u < NF; ++u) d[u] = *reinterpret_cast<const v4i *>(base[u] + ko + lane16);
        __builtin_amdgcn_sched_barrier(0);
    };
    float sxs[2][SDT];
    auto load_sx = [&](float (&d)[SDT], int B) {
#pragma unroll
        for (int j = 0; j < SDT; ++j) {
            const int t = fr[j] * 16 + (lane & 15);
            d[j] = p.sx[sx_index(t, nb, B)];
        }
    };

    load_sx(sxs[0], 0);
#pragma unroll
    for (int s = 0; s < D; ++s) {
        if (s < p.KS) load(buf[s], s);
    }
    fill();
    lds_barrier();

    v4i acc[SDT][FN];
#pragma unroll
    for (int j = 0; j < SDT; ++j)
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) f[j][i][r] = 0.0f;   // the reference's f = 0 before block 0

    // Block b (H = b % 2): k-step 4b + ks lives in buf[(4H + ks) % D]; each slot, once
    // multiplied, is refilled with the k-step D later: always (R_FULL), clamped to the
    // last k-step (R_CLAMP, n_in % 256 != 0 only), or not at all (R_NONE, R_LAST). The
    // block's sx are in set H; the last block (R_LAST) runs last() instead of loading
    // the next block's sx. The refill mode is static: a run-time test around the loads
    // would make the compiler keep both versions of every buffer register.
    enum { R_FULL, R_CLAMP, R_NONE, R_LAST };
    auto block = [&](int b, auto h_tag, auto mode_tag) {
        constexpr int H = decltype(h_tag)::value;
        constexpr int MODE = decltype(mode_tag)::value;
        if (MODE == R_LAST) last();
        else load_sx(sxs[H ^ 1], b + 1);
        const int nks = K256 ? 4 : min(4, p.KS - 4 * b);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (K256 || ks < nks) {
#pragma unroll
                for (int j = 0; j < SDT; ++j)
#pragma unroll
                    for (int i = 0; i < FN; ++i)
                        acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            buf[(4 * H + ks) % D][SDT + i], buf[(4 * H + ks) % D][j], ks == 0 ? v4i{0, 0, 0, 0} : acc[j][i], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (MODE == R_FULL) load(buf[(4 * H + ks) % D], 4 * b + ks + D);
                if (MODE == R_CLAMP) load(buf[(4 * H + ks) % D], min(4 * b + ks + D, p.KS - 1));
            }
        }
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const v4f sw4 = *reinterpret_cast<const v4f *>(swl + b * PITCH + 16 * i + 4 * (lane >> 4));
            const float swr[4] = { sw4.x, sw4.y, sw4.z, sw4.w };
#pragma unroll
            for (int j = 0; j < SDT; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float prod = (float) acc[j][i][r] * sxs[H][j];
                    f[j][i][r] = __builtin_fmaf(prod, swr[r], f[j][i][r]);
                }
        }
    };
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    using FULL = std::integral_constant<int, R_FULL>;
    using CLAMP = std::integral_constant<int, R_CLAMP>;
    using NONE = std::integral_constant<int, R_NONE>;
    using LAST = std::integral_constant<int, R_LAST>;
    int b = 0;
    if (K256) {
        // The last D/4 blocks have no k-step left to load; the others refill every slot.
        const int nfull = nb - D / 4;
        for (; b + 1 < nfull; b += 2) {
            block(b, H0{}, FULL{});
            block(b + 1, H1{}, FULL{});
        }
        if (b < nfull) {
            block(b, H0{}, FULL{});
            ++b;
        }
        // blocks b .. nb - 1 remain: one, or (D == 8) two
        if (D == 8 && b + 2 == nb) {
            if (b & 1) { block(b, H1{}, NONE{}); block(b + 1, H0{}, LAST{}); }
            else       { block(b, H0{}, NONE{}); block(b + 1, H1{}, LAST{}); }
        } else {
            if (b & 1) block(b, H1{}, LAST{});
            else       block(b, H0{}, LAST{});
        }
    } else {
        for (; b + 2 < nb; b += 2) {
            block(b, H0{}, CLAMP{});
            block(b + 1, H1{}, CLAMP{});
        }
        if (b + 2 == nb) {
            block(b, H0{}, CLAMP{});
            block(b + 1, H1{}, LAST{});
        } else {
            block(b, H0{}, LAST{});
        }
    }
}

// fp32 rows out of a few-row GEMM: one wave per workgroup and piece (32 tokens x 16FN
// features), pieces numbered with the feature piece fastest. One-wave workgroups let the
// dispatcher spread a launch of few pieces over as many CUs as there are pieces; the
// limit then is the bytes a CU takes in per cycle. Needs N % 4 == 0 (16-byte stores)
// and n_blk <= SNB_MAX.
template <int FN, bool RES, bool K256>
__global__ __launch_bounds__(64) void gemm_small(gemm_params p) {
    __shared__ __attribute__((aligned(16))) float swl[SNB_MAX * 16 * FN];
    const int lane = threadIdx.x;
    const int mt = blockIdx.x / p.n_nt, nt = blockIdx.x - mt * p.n_nt;
    const int fr0 = mt * SDT, nr0 = w_frag(nt, 16 * FN, 0);
    float f[SDT][FN][4];
    // The residual of this lane's outputs, loaded at the start of the last block; rows
    // and features past the output read row T - 1 / feature N - 4 (never stored).
    v4f rv[SDT][FN];
    auto load_res = [&] {
        if (RES) {
#pragma unroll
            for (int j = 0; j < SDT; ++j)
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    const int t = clamp_row((fr0 + j) * 16 + (lane & 15), p.T);
                    const int n = clamp_col4((nr0 + i) * 16 + 4 * (lane >> 4), p.N);
                    rv[j][i] = *reinterpret_cast<const v4f *>(p.res + (size_t) t * p.N + n);
                }
        }
    };
    small_piece<FN, K256, 16 * FN>(p, mt, nr0, swl, f, [&] { small_sw_fill<16 * FN>(p, nr0 * 16, swl); }, load_res);

    // out[t][n .. n + 3] = (res +) f: 16 bytes per lane and fragment pair.
#pragma unroll
    for (int j = 0; j < SDT; ++j) {
        const int t = (fr0 + j) * 16 + (lane & 15);
        if (t >= p.T) continue;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int n = (nr0 + i) * 16 + 4 * (lane >> 4);
            if (n >= p.N) continue;
            v4f y = { f[j][i][0], f[j][i][1], f[j][i][2], f[j][i][3] };
            if (RES) y = rv[j][i] + y;
            const out_map om = out_of(p, n);
            *reinterpret_cast<v4f *>(om.base + (size_t) t * om.ld + om.col) = y;
        }
    }
}

// fp32 rows out of a few-row GEMM with its 256-input blocks split over the waves of a
// workgroup: one workgroup per 64 x TN output tile (TN = 64, or 32 for n_blk = 9), wave b
// computes block b alone. Its 4 k-steps of the tile's 4 activation and TN / 16 weight
// fragments are loaded straight into registers at once, so a launch spends one memory round
// trip on its operands however long the input is, and a CU takes each operand byte once per
// 64 x TN tile. The block's exact int32 sums go to LDS with the block's scales; after one
// barrier, wave w (< 4) folds row group w of the tile over the blocks in order with the
// reference's step f = fma((float) s * sx[t, b], sw[b, n], f) from +0, which gives the same
// bits whatever wave computed a block (the int32 sums are exact), then adds the residual and
// stores 16 bytes per lane and fragment. Workgroups of max(n_blk, 4) waves; n_in % 256 == 0,
// n_blk <= NBM, N % 4 == 0. Instances: TN 64 for up to 4 blocks (64 KiB of LDS: two
// workgroups per CU), TN 32 for up to 9 (9 waves, at most 168 registers each).
template <int TN, int NBM, bool RES>
__global__ __launch_bounds__(64 * (NBM > 4 ? NBM : 4)) void gemm_fsk(gemm_params p) {
    constexpr int NJ = TN / 16;                      // weight fragments (16 columns each)
    __shared__ __attribute__((aligned(16))) int32_t sums[NBM * 64 * TN];         // [b][(i NJ + j) 64 + lane][4]
    __shared__ __attribute__((aligned(16))) float sxl[NBM * 64];                  // [b][row of the tile]
    __shared__ __attribute__((aligned(16))) float swl[NBM * TN];                  // [b][column of the tile]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int) threadIdx.x >> 6);
    const int mt = blockIdx.x / p.n_nt, nt = blockIdx.x - mt * p.n_nt;
    const int nb = p.n_blk;
    const size_t frow = (size_t) p.KS * FRAG;
    if (wave < nb) {
        const int b = wave;
        // activation fragment rows 4 mt + i (past the last one: the last one, never stored),
        // weight fragment rows nt NJ + j (NP is a multiple of 256: they exist)
        const int8_t * abase[4];
        const int8_t * wbase[NJ];
#pragma unroll
        for (int i = 0; i < 4; ++i) abase[i] = p.a + (size_t) fsk_a_frag(mt, i, p.MF) * frow + (size_t) lane * 16;
#pragma unroll
        for (int j = 0; j < NJ; ++j) wbase[j] = p.w + (size_t) (nt * NJ + j) * frow + (size_t) lane * 16;
        v4i oa[4][4], ob[4][NJ];                     // [k-step][fragment]
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const size_t ko = (size_t) (4 * b + s) * FRAG;
#pragma unroll
            for (int i = 0; i < 4; ++i) oa[s][i] = *reinterpret_cast<const v4i *>(abase[i] + ko);
#pragma unroll
            for (int j = 0; j < NJ; ++j) ob[s][j] = *reinterpret_cast<const v4i *>(wbase[j] + ko);
        }
        // the block's scales: sx of the tile's 16 row groups of 4 (lanes 0..15; groups past the
        // last one re-read it), sw of its TN columns (lanes 16..16 + TN / 4)
        if (lane < 16) {
            const v4f sx4 = *reinterpret_cast<const v4f *>(p.sx + fsk_sx_group(mt, lane, p.MF, nb, b));
            *reinterpret_cast<v4f *>(sxl + b * 64 + 4 * lane) = sx4;
        } else if (lane < 16 + TN / 4) {
            const int c = 4 * (lane - 16);
            *reinterpret_cast<v4f *>(swl + b * TN + c) = *reinterpret_cast<const v4f *>(p.sw + sw_index(b, p.NP, nt * TN + c));
        }
        v4i acc[4][NJ];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[s][j], oa[s][i], s == 0 ? v4i{0, 0, 0, 0} : acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                *reinterpret_cast<v4i *>(sums + ((size_t) b * 64 * TN) + ((i * NJ + j) * 64 + lane) * 4) = acc[i][j];
    }
    __syncthreads();
    if (wave >= 4) return;
    // wave w: row group w, lane: token 64 mt + 16 w + lane % 16, columns 16 j + 4 (lane / 16) + r
    const int t = mt * 64 + wave * 16 + (lane & 15);
    const int c0 = 4 * (lane >> 4);
    v4f rv[NJ];
    if (RES) {
        const int tr = clamp_row(t, p.T);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            rv[j] = *reinterpret_cast<const v4f *>(p.res + (size_t) tr * p.N + clamp_col4(nt * TN + 16 * j + c0, p.N));
    }
    float f[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) f[j][r] = 0.0f;                  // the reference's f = 0 before block 0
    for (int b = 0; b < nb; ++b) {
        const float sxv = sxl[b * 64 + wave * 16 + (lane & 15)];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const v4i s4 = *reinterpret_cast<const v4i *>(sums + ((size_t) b * 64 * TN) + ((wave * NJ + j) * 64 + lane) * 4);
            const v4f sw4 = *reinterpret_cast<const v4f *>(swl + b * TN + 16 * j + c0);
            const float swr[4] = { sw4.x, sw4.y, sw4.z, sw4.w };
#pragma unroll
            for (int r = 0; r < 4; ++r) f[j][r] = __builtin_fmaf((float) s4[r] * sxv, swr[r], f[j][r]);
        }
    }
    if (t >= p.T) return;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = nt * TN + 16 * j + c0;
        if (n >= p.N) continue;
        v4f y = { f[j][0], f[j][1], f[j][2], f[j][3] };
        if (RES) y = rv[j] + y;
        const out_map om = out_of(p, n);
        *reinterpret_cast<v4f *>(om.base + (size_t) t * om.ld + om.col) = y;
    }
}

// ---------------------------------------------------------------------------
// Wide GEMM with the relu^2 -> int8 output: 128 x 256 tiles, n_in % 256 == 0
// ---------------------------------------------------------------------------

// Across the four 16-lane rows of a wave: lane l gets the maximum of lanes
// l % 16 + 16 r, r = 0..3 (values without NaN).
__device__ __forceinline__ float rows_max(float m) {
    // ([lo, lo], [hi, hi]): row r now holds max(row r % 2, row r % 2 + 2)
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_int(m), __float_as_int(m), false, false);
    m = fmaxf(__int_as_float(h[0]), __int_as_float(h[1]));
    // ([r0, r0, r2, r2], [r1, r1, r3, r3]): every row the maximum of the four
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_int(m), __float_as_int(m), false, false);
    return fmaxf(__int_as_float(q[0]), __int_as_float(q[1]));
}

// 4 x 4 transpose of (16-lane row, register): on entry row g of d[j] holds item (g, j),
// on exit row j of d[g] holds it. permlane32_swap(a, b) gives ([a.lo, b.lo], [a.hi, b.hi])
// in 32-lane halves, permlane16_swap(a, b) gives ([a.r0, b.r0, a.r2, b.r2],
// [a.r1, b.r1, a.r3, b.r3]) in 16-lane rows.
__device__ __forceinline__ void rows_transpose(int (&d)[4]) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
    const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    d[0] = s01[0]; d[1] = s01[1]; d[2] = s23[0]; d[3] = s23[1];
}

// relu(linear(x))^2 quantized for the next linear, the reference's op_relu_sqr feeding
// an int8 linear (src/nexterabert.cpp:484-505 through for_rows' quantize_row, :414-438;
// the MLP's c_fc -> c_proj, :1284-1289). One workgroup per CU: 8 waves (2 x 4), each
// computing the same 64 x 64 piece as in gemm_k256, over a 128 x 256 tile -- exactly one
// 256-input block of the next linear, so a row's block amax is reduced here (over the
// lanes of a wave, then over the 4 waves through LDS) and each wave stores whole 1 KiB
// activation fragments; the fp32 rows are never written. The k-step schedule: k-step g
// lives in ring slot g % 4 and is read into registers one step ahead (two operand sets).
// Step g's barrier publishes k-step g + 1 and certifies that every wave has read k-step g,
// so each wave then loads its A fragment and its 2 B fragments of k-step g + 4 into slot
// g % 4 (the last four k-steps of a tile load the first four of the next), reads k-step
// g + 1 from LDS among k-step g's MFMAs, and runs them; constant waits (6 later loads; 7
// on waves 0 and 1 at the two k-steps whose later loads include their scale loads). The
// block scales have an LDS area of their own.
template <int ACT_MAX>
__global__ __launch_bounds__(WTHREADS, 1) void gemm_relu2_q8(gemm_params p) {
    __shared__ __attribute__((aligned(1024))) int8_t ring[4 * WSLOT];
    __shared__ __attribute__((aligned(16))) float scl[WSCALE / 4];
    __shared__ __attribute__((aligned(16))) float am[2 * 64 * 4];   // row maxima [wm][row][wn]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const tile_walk walk(blockIdx.x, gridDim.x, p.G);
    if (walk.count == 0) return;
    const int nb = p.KS >> 2;                        // 256-input blocks per tile
    const size_t frow = (size_t) p.KS * FRAG;        // bytes of one fragment row
    const uint32_t ring_lds = (uint32_t) (uintptr_t) (lds_void *) ring;
    const uint32_t lane16 = (uint32_t) lane * 16;
    // LDS address of the scale area as an integer, so that no generic pointer to it is
    // merged across the waves' branches below
    const uint32_t scl_lds = (uint32_t) (uintptr_t) (lds_void *) scl;

    struct frag_rows {                               // this wave's 3 fragment rows of a tile
        const int8_t * a;
        const int8_t * w0;
        const int8_t * w1;
    };
    auto rows_of = [&](int i) {                      // tile i of the walk (clamped)
        const int tile = walk.tile_clamped(i);
        const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
        frag_rows r;
        r.a = uniform_ptr(p.a + (size_t) a_frag(mt, wave, p.MF) * frow);
        r.w0 = uniform_ptr(p.w + (size_t) w_frag(nt, WBN, wave) * frow);
        r.w1 = uniform_ptr(p.w + (size_t) w_frag(nt, WBN, wave + 8) * frow);
        return r;
    };
    // k-step ks of a tile into ring slot j: A fragment w, B fragments w and w + 8.
    auto issue = [&](const frag_rows & r, int ks, int j) {
        const uint32_t vo = lane16 + (uint32_t) ks * FRAG;
        const uint32_t m = ring_lds + (uint32_t) (j * WSLOT + wave * FRAG);
        dma16s(r.a, vo, m);
        dma16s(r.w0, vo, m + 8 * FRAG);
        dma16s(r.w1, vo, m + 16 * FRAG);
    };

    v4i acc[4][4];
    float f[4][4][4];
    v4i oa[2][4], ob[2][4];                          // operand sets: k-step g in set g % 2
    auto rd = [&](int j, int set) {
        const int8_t * slot = ring + j * WSLOT;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            oa[set][i] = *reinterpret_cast<const v4i *>(slot + (wm * 4 + i) * FRAG + lane * 16);
            ob[set][i] = *reinterpret_cast<const v4i *>(slot + (8 + wn * 4 + i) * FRAG + lane * 16);
        }
    };
    auto mm = [&](int set, bool first, int m0, int m1) {
#pragma unroll
        for (int mi = m0; mi < m1; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                acc[mi][ni] = first
                    ? __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[set][ni], oa[set][mi], v4i{0, 0, 0, 0}, 0, 0, 0)
                    : __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[set][ni], oa[set][mi], acc[mi][ni], 0, 0, 0);
    };

    {
        const frag_rows r0 = rows_of(0);
        issue(r0, 0, 0);
        issue(r0, 1, 1);
        issue(r0, 2, 2);
        issue(r0, 3, 3);
        wait_vm<0>();
        lds_barrier();
    }
    // The tile walk, instantiated for one 256-input block per tile and for several, so that
    // whether a block's fold starts from +0 is static in every block.
    auto walk_tiles = [&](auto one_tag) {
        constexpr bool one = decltype(one_tag)::value;
        for (int it = 0; it < walk.count; ++it) {
            const int tile = walk.tile(it);
            const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
            const frag_rows cur = rows_of(it), nxt = rows_of(it + 1);
            // Scale loads of block B (B * sstep bytes on): wave 0 lane l < 32 the sx of row
            // group l, wave 0 lane l >= 32 the sw of columns 4(l-32)..+3, wave 1 lane l < 32
            // the sw of columns 128 + 4l..+3; lane l lands at scl + 16 l (+ 1024 on wave 1).
            const float * ssrc;
            size_t sstep;
            if (wave == 0 && lane < 32) {
                ssrc = p.sx + sx_group_index(mt, lane, p.MF, p.n_blk, 0);
                sstep = 4 * sizeof(float);
            } else {
                ssrc = p.sw + sw_index(0, p.NP, nt * WBN + (wave == 0 ? 4 * (lane - 32) : 128 + 4 * lane));
                sstep = (size_t) p.NP * sizeof(float);
            }
            const int tbase = mt * BM + wm * 64;
            rd(0, 0);                                // the tile's k-step 0 (slots 0..3 published)

            auto run_block = [&](int B, auto last_tag, auto first_tag) {
                constexpr bool last = decltype(last_tag)::value, first = decltype(first_tag)::value;
                // Step s (k-step g = 4B + s, in registers since step s - 1): publish k-step g + 1
                // (its DMA, issued 3 steps ago, waited; every wave done reading k-step g), load
                // k-step g + 4 into slot s, read k-step g + 1 into the other operand set, then
                // k-step g's MFMAs. The tile's last step reads nothing ahead.
                auto step = [&](auto s_tag) {
                    constexpr int s = decltype(s_tag)::value;
                    if ((s == 1 || s == 2) && wave < 2) wait_vm<7>();
                    else wait_vm<6>();
                    lds_barrier();
                    const ring_load l = ring_prefetch(it, B, s, last, false);
                    issue(l.pos == it ? cur : nxt, l.ks, l.slot);
                    if (s == 0) {
                        if (wave == 0) {
                            dma16l(reinterpret_cast<const char *>(ssrc) + (size_t) B * sstep, scl_lds);
                        } else if (wave == 1 && lane < 32) {
                            dma16l(reinterpret_cast<const char *>(ssrc) + (size_t) B * sstep, scl_lds + 1024);
                        }
                    }
                    // three quarters of the MFMAs first: their A operands are then free for the next
                    // set (earlier, the two sets do not fit in the register budget)
                    mm(s & 1, s == 0, 0, 3);
                    if (!(last && s == 3)) rd((s + 1) & 3, (s + 1) & 1);
                    mm(s & 1, s == 0, 3, 4);
                };
                step(std::integral_constant<int, 0>{});
                step(std::integral_constant<int, 1>{});
                step(std::integral_constant<int, 2>{});
                step(std::integral_constant<int, 3>{});

                // f = fma((float) s * sx[t, B], sw[B, n], f): the reference's per-block step.
                float sxv[4];
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) sxv[mi] = scl[wm * 64 + mi * 16 + (lane & 15)];
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const float4 sw4 = *reinterpret_cast<const float4 *>(scl + BM + wn * 64 + ni * 16 + 4 * (lane >> 4));
                    const float swr[4] = { sw4.x, sw4.y, sw4.z, sw4.w };
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float prod = (float) acc[mi][ni][r] * sxv[mi];
                            // block 0 starts from f = 0: fma(prod, sw, +0.0)
                            f[mi][ni][r] = __builtin_fmaf(prod, swr[r], first ? 0.0f : f[mi][ni][r]);
                        }
                }
            };
            if constexpr (one) {
                run_block(0, std::true_type{}, std::true_type{});
            } else {
                run_block(0, std::false_type{}, std::true_type{});
                for (int B = 1; B < nb - 1; ++B) run_block(B, std::false_type{}, std::false_type{});
                run_block(nb - 1, std::true_type{}, std::false_type{});
            }

            // Every load of this wave first: the next tile's first three k-steps (its block
            // 0 then waits only at k-step 3, and the stores below stand behind no load it
            // waits for).
            wait_vm<0>();
            {
                // Row maxima of relu(f) = max(f, 0) (maxNum: a NaN counts as 0; f is never a
                // signalling NaN, being an fma result): over this lane's 16 values, the wave's 4
                // lanes of the row, then the 4 waves of the row through LDS, am[wm][row][wn]. The
                // block amax of relu(f)^2 (values >= 0, no NaN: the reference's MAXPS fold is the
                // plain maximum) is the square of that maximum, r * r being monotonic in r >= 0.
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) {
                    float m = 0.0f;
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
                        for (int r = 0; r < 4; ++r) m = fmaxf(m, f[mi][ni][r]);
                    m = rows_max(m);
                    if (lane < 16) am[(wm * 64 + mi * 16 + lane) * 4 + wn] = m;
                }
                lds_barrier();
                // Lane l takes row l of the wave's 64 (row group l / 16, row l % 16): the row's
                // maximum over the 4 waves, its scale amax / ACT_MAX and inv = ACT_MAX / amax, each
                // computed once per row; a transpose then gives every lane the inv of its 4 row
                // groups. With every maximum of the wave finite (the usual case) each value f * inv
                // lies in [0, ACT_MAX + 1/2), so CVTPS2DQ and the saturating packs reduce to
                // round-to-nearest-even, which v_cvt_pk_u8_f32 does while packing the byte. An
                // infinite maximum, or one so small (below ACT_MAX / FLT_MAX, denormals
                // included) that inv overflows to +Inf, takes quant1: there x * inv is Inf or
                // NaN, which CVTPS2DQ turns into 0x80000000 (u8 0) for every value of the row.
                const int tl = tbase + lane;
                const v4f a4 = *reinterpret_cast<const v4f *>(am + (wm * 64 + lane) * 4);
                const float rmax = tl < p.T ? fmaxf(fmaxf(a4.x, a4.y), fmaxf(a4.z, a4.w)) : 0.0f;
                const float amax_l = rmax * rmax;
                const float inv_l = amax_l > 0.0f ? (float) ACT_MAX / amax_l : 0.0f;
                const bool fast = __builtin_amdgcn_ballot_w64(!(amax_l < INFINITY) || !(inv_l < INFINITY)) == 0;
                int invs[4] = { __float_as_int(inv_l), __float_as_int(inv_l), __float_as_int(inv_l), __float_as_int(inv_l) };
                rows_transpose(invs);                        // invs[mi]: row group mi, row lane % 16
                if (wn == 0 && mt * (BM / 16) + wm * 4 + (lane >> 4) < p.MF)
                    p.sxo[sxo_index(tl, p.n_nt, nt)] = amax_l / (float) ACT_MAX;
                // Row group mi: its int8 values, zero past row T - 1 and column N - 1 (GUARD; a
                // tile inside both bounds skips the tests).
                auto quantize_store = [&](int mi, auto guard_tag) {
                    constexpr bool guard = decltype(guard_tag)::value;
                    const float inv = __int_as_float(invs[mi]);
                    const bool row_ok = tbase + mi * 16 + (lane & 15) < p.T;
                    // column 16ni + 4(lane/16) + r of the wave's 64: byte r of d[ni]
                    int d[4];
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni) {
                        int packed;
                        if (fast) {
                            // f * |f| is relu(f)^2 for f >= +0 and <= 0 (or NaN) otherwise, which
                            // v_cvt_pk_u8_f32 turns into 0 like the reference's relu
                            unsigned u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][0] * fabsf(f[mi][ni][0]) * inv, 0, 0u);
                            u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][1] * fabsf(f[mi][ni][1]) * inv, 1, u);
                            u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][2] * fabsf(f[mi][ni][2]) * inv, 2, u);
                            u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][3] * fabsf(f[mi][ni][3]) * inv, 3, u);
                            packed = (int) u;
                        } else {
                            float r2[4];
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float x = fmaxf(f[mi][ni][r], 0.0f);
                                r2[r] = x * x;
                            }
                            packed = (quant1<ACT_MAX>(r2[0], inv) & 0xff) | ((quant1<ACT_MAX>(r2[1], inv) & 0xff) << 8)
                                   | ((quant1<ACT_MAX>(r2[2], inv) & 0xff) << 16) | ((quant1<ACT_MAX>(r2[3], inv) & 0xff) << 24);
                        }
                        if (guard) {
                            const int n = nt * WBN + wn * 64 + ni * 16 + 4 * (lane >> 4);
                            packed = row_ok && n < p.N ? packed : 0;
                        }
                        d[ni] = packed;
                    }
                    // lane c + 16 j now gets columns 16 j + 0..15 of row c: one fragment lane
                    rows_transpose(d);
                    const int rf = mt * (BM / 16) + wm * 4 + mi, kf = nt * (WBN / 64) + wn;
                    if (rf < p.MF && kf < p.KSo) {
                        // device scope (sc1): the int8 rows go past L2, where they would evict the
                        // activation row tile that this row's other column tiles re-read, yet
                        // (unlike a nontemporal store) into the last-level cache, from which the next
                        // GEMM reads them. The s_nop gives the store its wait states before the
                        // data registers are written again (the compiler does not see into asm).
                        asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1"
                                     :: "v"(p.qo + qo_byte(rf, p.KSo, kf, lane)), "v"(v4i{d[0], d[1], d[2], d[3]})
                                     : "memory");
                    }
                };
                if (mt * BM + BM <= p.T && nt * WBN + WBN <= p.N) {
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi) quantize_store(mi, std::false_type{});
                } else {
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi) quantize_store(mi, std::true_type{});
                }
            }
        }
    };
    if (nb == 1) walk_tiles(std::true_type{});
    else         walk_tiles(std::false_type{});
    wait_vm<0>();
}

// relu(linear(x))^2 quantized for the next linear (the same output as gemm_relu2_q8), for
// n_in <= 1024. Tiles of 64 rows x 256 columns (one 256-input block of the next linear),
// two workgroups of 4 waves per CU, each wave the 64 x 64 piece of gemm_k256 at columns
// 64 w. A workgroup walks a contiguous range of tiles (tile_span), so it loads each
// activation row tile (64 rows x n_in, at most 64 KiB) into LDS once and walks its column
// tiles; every wave loads its 4 weight fragments per k-step straight into registers,
// RDEPTH k-steps ahead. So the k-loop has no barrier: each wave runs its k-steps and
// per-block folds in its own phase, and a fold overlaps the MFMAs of the waves of the other
// workgroup and of its own. The tile's one barrier publishes the row maxima (each row's
// 256 columns span the 4 waves) and the next tile's scales, which were loaded under this
// tile; the next tile's first weight k-steps are loaded before this tile's stores, so that
// their waits do not wait for the stores. A new row tile is loaded after that barrier,
// under the tile's quantization and stores, and published by a second barrier.
// With FQ the input is fp32 rows (p.xf): each row tile is quantized into LDS as quantize_row
// does it (quantize_group16: the same int8 values and scales as nxg_quantize_rows), its row
// scales kept in LDS for the tile's column tiles, so the activations never go to memory as
// int8; a new row tile is quantized after the previous tile's stores.
template <int ACT_MAX, int NB, bool FQ>
__global__ __launch_bounds__(RTHREADS, 2) void gemm_relu2_rt(gemm_params p) {
    constexpr int KS = 4 * NB;                       // k-steps of a tile (p.KS)
    constexpr int D = RDEPTH;
    static_assert(NB >= 1 && NB <= RNB_MAX, "row tile of 1..4 blocks");
    __shared__ __attribute__((aligned(1024))) int8_t arow[KS * (RM / 16) * FRAG];   // [ks][row group] fragments
    __shared__ __attribute__((aligned(16))) float scl[2][RSCALE / 4];             // two tiles' scales
    __shared__ __attribute__((aligned(16))) float am[2][RM * 4];                  // row maxima [row][wave]
    __shared__ __attribute__((aligned(16))) float sxr[FQ ? RM * NB : 4];         // FQ: the row tile's sx [row/4][B][row%4]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const tile_span span(blockIdx.x, gridDim.x, p.G);
    if (span.count == 0) return;
    const size_t frow = (size_t) KS * FRAG;          // bytes of one fragment row
    const uint32_t lane16 = (uint32_t) lane * 16;
    const uint32_t arow_lds = (uint32_t) (uintptr_t) (lds_void *) arow;
    const uint32_t scl_lds = (uint32_t) (uintptr_t) (lds_void *) &scl[0][0];

    // Row tile mt into LDS: wave w loads row group w of every k-step.
    auto load_rows = [&](int mt) {
        const int8_t * src = p.a + (size_t) a_frag_rt(mt, wave, p.MF) * frow;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            dma16s(uniform_ptr(src + (size_t) ks * FRAG), lane16, arow_lds + (uint32_t) ((ks * 4 + wave) * FRAG));
    };
    // FQ: row tile mt quantized into LDS. Wave w takes row group w (rows 16w .. 16w + 15 of
    // the tile) in 4 NB stages of (4 rows, one block): lane row 4 (s / NB) + lane / 16, c =
    // lane % 16 reading inputs 256 B + 64i + 4c .. + 3 of block B = s % NB; four stages of
    // loads in flight. Input 256B + 64i + 4c + e goes to k-step 4B + i, fragment lane
    // (row % 16) + 16 (c / 4), byte 4 (c % 4) + e. Rows past T are zeros with scale 0.
    const float * const xf = p.xf;
    const int T = p.T;
    auto quantize_rows = [&](int mt) __attribute__((always_inline)) {
        constexpr int NS = 4 * NB, DQ = 4;
        const int ln = lane_here();
        const int c = ln & 15, rl = ln >> 4;
        float xs[DQ][4][4];                          // stage s in xs[s % DQ]: [i][e]
        auto load_stage = [&](int st, float (&d)[4][4]) {
            const float * xr = xf + (size_t) rt_x_row(mt, wave * 16 + 4 * (st / NB) + rl, T) * (size_t) (256 * NB)
                             + 256 * (st % NB) + 4 * c;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(xr + 64 * i));
                d[i][0] = v.x; d[i][1] = v.y; d[i][2] = v.z; d[i][3] = v.w;
            }
        };
#pragma unroll
        for (int st = 0; st < DQ && st < NS; ++st) load_stage(st, xs[st]);
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const int B = st % NB;
            const int r = wave * 16 + 4 * (st / NB) + rl;    // row within the tile
            const bool row_ok = mt * RM + r < T;
            const bool present[4] = { row_ok, row_ok, row_ok, row_ok };
            float x4[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) x4[i][e] = row_ok ? xs[st % DQ][i][e] : 0.0f;
            if (st + DQ < NS) load_stage(st + DQ, xs[st % DQ]);
            int packed[4];
            const float amax = quantize_group16<ACT_MAX>(x4, present, row_ok, c, packed);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<int *>(arow + ((4 * B + i) * 4 + wave) * FRAG + ((r & 15) + 16 * (c >> 2)) * 16 + 4 * (c & 3)) = packed[i];
            if (c == 0) sxr[((r >> 2) * NB + B) * 4 + (r & 3)] = row_ok ? amax / (float) ACT_MAX : 0.0f;
        }
    };
    // A tile's scales into buffer b: wave w < NB the sw of block w (1 KiB: lane l columns
    // 4l..4l+3); wave 0 lanes l < 16 NB the sx of row group l / NB, block l % NB.
    // Scalar bases and 32-bit lane offsets (computed here, not kept across the tile loop).
    auto load_scales = [&](int tile, int b) {
        const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
        const uint32_t base = scl_lds + (uint32_t) (b * RSCALE);
        const int ln = lane_here();
        if (wave < NB) {
            const int8_t * sw_row = uniform_ptr(reinterpret_cast<const int8_t *>(p.sw + sw_index(wave, p.NP, nt * WBN)));
            dma16s(sw_row, (uint32_t) ln * 16, base + RSX_BYTES + wave * (WBN * 4));
        }
        if (!FQ && wave == 0 && ln < 16 * NB) {
            dma16s(uniform_ptr(reinterpret_cast<const int8_t *>(p.sx)),
                   (uint32_t) (sx_group_index_rt(mt, ln / NB, p.MF, NB, ln % NB) * sizeof(float)), base);
        }
    };

    v4i acc[4][4];
    float f[4][4][4];
    v4i oa[4];                                       // activation operands (row groups) of one k-step
    v4i ob[D][4];                                    // weight operands: k-step ks in ob[ks % D]
    auto rd = [&](int ks, int i) {
        oa[i] = *reinterpret_cast<const v4i *>(arow + (ks * 4 + i) * FRAG + lane * 16);
    };
    // The weight fragments 4w .. 4w + 3 of column tile nt, k-step ks, into ob[j]. The
    // scheduling barrier keeps the loads where they are issued.
    const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(p.w, (uint32_t) ((size_t) p.NP * KS * 64));
    auto ldw = [&](int nt, int ks, int j) {
        const uint32_t so = (uint32_t) __builtin_amdgcn_readfirstlane(w_frag(nt, WBN, 4 * wave) * (int) frow + ks * FRAG);
#pragma unroll
        for (int i = 0; i < 4; ++i) ob[j][i] = bload16(wrsrc, lane16, so + (uint32_t) (i * frow));
        __builtin_amdgcn_sched_barrier(0);
    };
    // One k-step's 16 MFMAs (weights in ob[j]); as soon as the 4 that use row group mi are
    // issued, oa[mi] is refilled with row group mi of k-step nk (none if nk < 0), so that
    // every LDS read has 12 MFMAs to land before its use. The group barriers keep that order.
    auto kstep = [&](int j, bool first, int nk) {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                acc[mi][ni] = first
                    ? __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[j][ni], oa[mi], v4i{0, 0, 0, 0}, 0, 0, 0)
                    : __builtin_amdgcn_mfma_i32_16x16x64_i8(ob[j][ni], oa[mi], acc[mi][ni], 0, 0, 0);
            if (nk >= 0) rd(nk, mi);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);       // 4 MFMAs
            if (nk >= 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // 1 LDS read
        }
    };

    int tile = span.first;
    int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
    if (FQ) quantize_rows(mt);
    else    load_rows(mt);
    load_scales(tile, 0);
    wait_vm<0>();
    lds_barrier();
#pragma unroll
    for (int j = 0; j < D; ++j) ldw(nt, j, j);

    for (int it = 0; it < span.count; ++it) {
        const int cur = it & 1;
        const bool more = it + 1 < span.count;
        // the next tile's scales into the other buffer (its last readers, the previous
        // tile's folds, are all behind the previous tile's barrier)
        if (more) load_scales(tile + 1, cur ^ 1);
        const float * sc = &scl[cur][0];
        const int nt_next = more ? (tile + 1) % p.n_nt : 0;

        // Block B: k-steps 4B .. 4B + 3 (k-step ks's weights in ob[ks % 4], RDEPTH == 4), each
        // slot refilled with the k-step 4 later (REFILL: every block but the tile's last),
        // then the block's fold. Blocks past the first run in a loop that is not unrolled,
        // so that the compiler keeps one block's load addresses at a time. Wave priority as
        // in gemm_k256: k-steps 2, fold 1, row maxima, quantization and stores 0.
        static_assert(D == 4, "one block of weight k-steps in flight");
        auto block = [&](int B, auto first_tag, auto refill_tag) {
            constexpr bool first = decltype(first_tag)::value, refill = decltype(refill_tag)::value;
            __builtin_amdgcn_s_setprio(2);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                kstep(s, s == 0, s < 3 || refill ? 4 * B + s + 1 : -1);
                __builtin_amdgcn_sched_barrier(0);
                if (refill) ldw(nt, 4 * B + 4 + s, s);
                else if (s == 0 && more) ldw(nt_next, 0, 0);  // the tile's last block: the next tile's k-step 0
            }
            __builtin_amdgcn_s_setprio(1);
            // f = fma((float) s * sx[t, B], sw[B, n], f): the reference's per-block step.
            const int ln = lane_here();
            float sxv[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const int r = mi * 16 + (ln & 15);
                sxv[mi] = FQ ? sxr[((r >> 2) * NB + B) * 4 + (r & 3)] : sc[((r >> 2) * NB + B) * 4 + (r & 3)];
            }
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const float4 sw4 = *reinterpret_cast<const float4 *>(sc + RSX_BYTES / 4 + B * WBN + wave * 64 + ni * 16 + 4 * (ln >> 4));
                const float swr[4] = { sw4.x, sw4.y, sw4.z, sw4.w };
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float prod = (float) acc[mi][ni][r] * sxv[mi];
                        // block 0 starts from f = 0: fma(prod, sw, +0.0)
                        f[mi][ni][r] = __builtin_fmaf(prod, swr[r], first ? 0.0f : f[mi][ni][r]);
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) rd(0, i);
        if (NB == 1) {
            block(0, std::true_type{}, std::false_type{});
        } else {
            block(0, std::true_type{}, std::true_type{});
#pragma unroll 1
            for (int B = 1; B < NB - 1; ++B) block(B, std::false_type{}, std::true_type{});
            block(NB - 1, std::false_type{}, std::false_type{});
        }

        __builtin_amdgcn_s_setprio(0);
        // Row maxima of relu(f) = max(f, 0) (maxNum: a NaN counts as 0): over this lane's 16
        // values, the wave's 4 lanes of the row, then the 4 waves through LDS, am[cur][row][w].
        // The block amax of relu(f)^2 (values >= 0, no NaN: the reference's MAXPS fold is the
        // plain maximum) is the square of that maximum, r * r being monotonic in r >= 0.
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            float m = 0.0f;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
#pragma unroll
                for (int r = 0; r < 4; ++r) m = fmaxf(m, f[mi][ni][r]);
            m = rows_max(m);
            const int ln = lane_here();
            if (ln < 16) am[cur][(mi * 16 + ln) * 4 + wave] = m;
        }
        // This wave's loads done but the next tile's first weight k-step (4 loads, issued
        // after the scale loads), then the barrier: the row maxima and the next tile's scales
        // published, and every wave past its last read of this row tile.
        if (more) wait_vm<4>();
        else      wait_vm<0>();
        lds_barrier();
        const int tbase = mt * RM;
        const int mt_t = mt, nt_t = nt;
        const bool reload = more && (tile + 1) / p.n_nt != mt;
        if (more) {
            ++tile;
            mt = tile / p.n_nt;
            nt = tile - mt * p.n_nt;
            if (reload && !FQ) load_rows(mt);
        }

        // Lane l takes row l of the tile: the row's maximum over the 4 waves, its scale
        // amax / ACT_MAX and inv = ACT_MAX / amax, each computed once per row; a transpose
        // then gives every lane the inv of its 4 row groups. With every maximum of the wave
        // finite and inv finite (the usual case) each value f * inv lies in [0, ACT_MAX + 1/2),
        // so CVTPS2DQ and the saturating packs reduce to round-to-nearest-even, which
        // v_cvt_pk_u8_f32 does while packing the byte. An infinite maximum, or one so small
        // that inv overflows to +Inf, takes quant1 (NaN and Inf -> 0x80000000, u8 0).
        {
            const int lane = lane_here();               // (shadows the outer one: see lane_here)
            const int tl = tbase + lane;
            const v4f a4 = *reinterpret_cast<const v4f *>(&am[cur][lane * 4]);
            const float rmax = tl < p.T ? fmaxf(fmaxf(a4.x, a4.y), fmaxf(a4.z, a4.w)) : 0.0f;
            const float amax_l = rmax * rmax;
            const float inv_l = amax_l > 0.0f ? (float) ACT_MAX / amax_l : 0.0f;
            const bool fast = __builtin_amdgcn_ballot_w64(!(amax_l < INFINITY) || !(inv_l < INFINITY)) == 0;
            int invs[4] = { __float_as_int(inv_l), __float_as_int(inv_l), __float_as_int(inv_l), __float_as_int(inv_l) };
            rows_transpose(invs);                        // invs[mi]: row group mi, row lane % 16
            if (wave == 0 && mt_t * (RM / 16) + (lane >> 4) < p.MF)
                p.sxo[sxo_index(tl, p.n_nt, nt_t)] = amax_l / (float) ACT_MAX;
            // Row group mi: its int8 values, zero past row T - 1 and column N - 1 (GUARD; a
            // tile inside both bounds skips the tests).
            auto quantize_store = [&](int mi, auto guard_tag) {
                constexpr bool guard = decltype(guard_tag)::value;
                const float inv = __int_as_float(invs[mi]);
                const bool row_ok = tbase + mi * 16 + (lane & 15) < p.T;
                // column 16ni + 4(lane/16) + r of the wave's 64: byte r of d[ni]
                int d[4];
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    int packed;
                    if (fast) {
                        // f * |f| is relu(f)^2 for f >= +0 and <= 0 (or NaN) otherwise, which
                        // v_cvt_pk_u8_f32 turns into 0 like the reference's relu
                        unsigned u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][0] * fabsf(f[mi][ni][0]) * inv, 0, 0u);
                        u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][1] * fabsf(f[mi][ni][1]) * inv, 1, u);
                        u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][2] * fabsf(f[mi][ni][2]) * inv, 2, u);
                        u = __builtin_amdgcn_cvt_pk_u8_f32(f[mi][ni][3] * fabsf(f[mi][ni][3]) * inv, 3, u);
                        packed = (int) u;
                    } else {
                        float r2[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float x = fmaxf(f[mi][ni][r], 0.0f);
                            r2[r] = x * x;
                        }
                        packed = (quant1<ACT_MAX>(r2[0], inv) & 0xff) | ((quant1<ACT_MAX>(r2[1], inv) & 0xff) << 8)
                               | ((quant1<ACT_MAX>(r2[2], inv) & 0xff) << 16) | ((quant1<ACT_MAX>(r2[3], inv) & 0xff) << 24);
                    }
                    if (guard) {
                        const int n = nt_t * WBN + wave * 64 + ni * 16 + 4 * (lane >> 4);
                        packed = row_ok && n < p.N ? packed : 0;
                    }
                    d[ni] = packed;
                }
                // lane c + 16 j now gets columns 16 j + 0..15 of row c: one fragment lane
                rows_transpose(d);
                const int rf = mt_t * (RM / 16) + mi, kf = nt_t * (WBN / 64) + wave;
                if (rf < p.MF && kf < p.KSo) {
                    // device scope (sc1): past L2, into the last-level cache, from which the next
                    // GEMM reads them. The s_nop gives the store its wait states before the data
                    // registers are written again (the compiler does not see into asm).
                    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1"
                                 :: "v"(p.qo + qo_byte(rf, p.KSo, kf, lane)), "v"(v4i{d[0], d[1], d[2], d[3]})
                                 : "memory");
                }
            };
            if (tbase + RM <= p.T && nt_t * WBN + WBN <= p.N) {
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) quantize_store(mi, std::false_type{});
            } else {
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) quantize_store(mi, std::true_type{});
            }
        }
        if (more) {
            // the next tile's weight k-steps 1..3 (0 is in flight since this tile's last block)
            ldw(nt, 1, 1);
            ldw(nt, 2, 2);
            ldw(nt, 3, 3);
        }
        if (reload) {
            // the new row tile (and the weight loads and stores before it) landed, then
            // published to every wave
            if (FQ) quantize_rows(mt);
            wait_vm<0>();
            lds_barrier();
        }
    }
    wait_vm<0>();
}

// relu(linear(x))^2 quantized for the next linear, for few rows (the same output as
// gemm_relu2_q8): workgroups of 4 waves over 32 tokens x 256 features -- one 256-input
// block of the next linear -- each wave a 32 x 64 piece computed by small_piece. The row
// amax is reduced over the lanes of a wave (rows_max) and the 4 waves (LDS); relu^2, the
// quantization, the fragment stores and the scale layout are gemm_relu2_q8's. Needs
// n_in % 256 == 0 and n_blk <= SNB_MAX.
template <int ACT_MAX>
__global__ __launch_bounds__(256) void gemm_relu2_small(gemm_params p) {
    __shared__ __attribute__((aligned(16))) float swl[SNB_MAX * WBN];
    __shared__ __attribute__((aligned(16))) float am[SDT * 16 * 4];   // row maxima [row][wave]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int mt = blockIdx.x / p.n_nt, nt = blockIdx.x - mt * p.n_nt;
    const int fr0 = mt * SDT, nr0 = w_frag(nt, WBN, 4 * wave);
    float f[SDT][4][4];
    small_piece<4, true, WBN>(p, mt, nr0, swl + wave * 64, f, [&] { small_sw_fill<WBN>(p, nt * WBN, swl); }, [] {});

    // relu(f)^2 in place: f > 0 ? f : 0 (a NaN gives 0), then r * r.
#pragma unroll
    for (int j = 0; j < SDT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = f[j][i][r] > 0.0f ? f[j][i][r] : 0.0f;
                f[j][i][r] = x * x;
            }
    // Row maxima (values >= 0, no NaN: the reference's MAXPS fold is the plain maximum
    // here): this lane's 16 values, the wave's 4 lanes of the row, then the 4 waves.
#pragma unroll
    for (int j = 0; j < SDT; ++j) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) m = fmaxf(m, f[j][i][r]);
        m = rows_max(m);
        if (lane < 16) am[(j * 16 + lane) * 4 + wave] = m;
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < SDT; ++j) {
        const int t = (fr0 + j) * 16 + (lane & 15);
        const v4f a4 = *reinterpret_cast<const v4f *>(am + (j * 16 + (lane & 15)) * 4);
        const bool row_ok = t < p.T;
        const float amax = row_ok ? fmaxf(fmaxf(a4.x, a4.y), fmaxf(a4.z, a4.w)) : 0.0f;
        const float scale = amax / (float) ACT_MAX;
        const float inv = amax > 0.0f ? (float) ACT_MAX / amax : 0.0f;
        // column 16i + 4(lane/16) + r of the wave's 64: byte r of d[i]
        int d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = (nr0 + i) * 16 + 4 * (lane >> 4);
            int packed = 0;
            if (row_ok && n < p.N) {
                packed = (quant1<ACT_MAX>(f[j][i][0], inv) & 0xff) | ((quant1<ACT_MAX>(f[j][i][1], inv) & 0xff) << 8)
                       | ((quant1<ACT_MAX>(f[j][i][2], inv) & 0xff) << 16) | ((quant1<ACT_MAX>(f[j][i][3], inv) & 0xff) << 24);
            }
            d[i] = packed;
        }
        // lane c + 16 i now gets columns 16 i + 0..15 of row c: one fragment lane
        rows_transpose(d);
        const int rf = fr0 + j, kf = nt * (WBN / 64) + wave;
        if (rf < p.MF) {
            if (kf < p.KSo) {
                *reinterpret_cast<v4i *>(p.qo + qo_byte(rf, p.KSo, kf, lane)) = v4i{d[0], d[1], d[2], d[3]};
            }
            if (wave == 0 && lane < 16) p.sxo[sxo_index(t, p.n_nt, nt)] = scale;
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int fail(int code, const char * fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    nxg_set_error(buf);
    return code;
}

int hip_fail(hipError_t e, const char * what) {
    return fail(NXG_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

thread_local int g_cus = 0;   // compute units of the checked device

int check_device() {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    static thread_local int checked_dev = -1;
    if (checked_dev == dev) return NXG_OK;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return fail(NXG_EDEVICE, "device %d is %s; this engine is built for gfx950 (MI355X)", dev, prop.gcnArchName);
    }
    checked_dev = dev;
    g_cus = prop.multiProcessorCount;
    return NXG_OK;
}

int device_cus() { return g_cus > 0 ? g_cus : 256; }

int launch_check(const char * what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? NXG_OK : hip_fail(e, what);
}

struct qact_dims {
    int T, n_in, KS, n_blk, MP;
};

bool qact_dims_of(int T, int n_in, qact_dims & d) {
    if (T < 0 || n_in <= 0 || n_in % 32 != 0) return false;
    d.T = T;
    d.n_in = n_in;
    d.KS = ceil_div(n_in, 64);
    d.n_blk = ceil_div(n_in, BLK);
    d.MP = ceil_div(T, 16) * 16;
    return true;
}

} // namespace

struct nxg_weight {
    int32_t n_in = 0, n_out = 0, n_blk = 0, KS = 0, NP = 0;
    int8_t * w = nullptr;    // NP x KS*64 bytes in fragment tiles
    float *  sw = nullptr;   // [n_blk][NP]
    size_t   bytes = 0;
};

// Device buffers are read and written 16 bytes per lane (and by LDS DMA): null or 16-byte aligned.
static bool aligned16(const void * p) { return ((uintptr_t) p & 15u) == 0; }

// A producer's rows quantized for an int8 consumer: shared checks and launch.
template <typename Src>
static int32_t launch_produce(const char * what, const Src & src, int32_t T, int32_t n_in, int32_t act_max,
                              int8_t * q, float * sx, void * stream) {
    qact_dims d;
    if (!qact_dims_of(T, n_in, d)) return fail(NXG_EINVAL, "%s: T=%d n_in=%d (n_in must be a positive multiple of 32)", what, T, n_in);
    if (act_max != 127 && act_max != 63) return fail(NXG_EINVAL, "%s: act_max must be 127 or 63, got %d", what, act_max);
    if (T == 0) return NXG_OK;
    if (!q || !sx) return fail(NXG_EINVAL, "%s: null output", what);
    if (!aligned16(q) || !aligned16(sx)) return fail(NXG_EINVAL, "%s: q and sx must be 16-byte aligned", what);
    int rc = check_device();
    if (rc) return rc;
    const long long n_wg = (long long) (d.MP / 16) * d.n_blk;
    if (n_wg > INT32_MAX) return fail(NXG_EINVAL, "%s: T=%d n_in=%d too large", what, T, n_in);
    const dim3 grid((unsigned) n_wg);
    hipStream_t s = (hipStream_t) stream;
    if (act_max == 127) produce_quantize_kernel<127, Src><<<grid, 256, 0, s>>>(src, T, n_in, d.KS, d.n_blk, q, sx);
    else                produce_quantize_kernel<63, Src><<<grid, 256, 0, s>>>(src, T, n_in, d.KS, d.n_blk, q, sx);
    return launch_check(what);
}

// Dynamic LDS the tiled attention kernel may take on the current device: the device's
// shared memory per workgroup less the kernel's static arrays, with the attribute that
// allows more than the default raised to it, once per thread and device (as check_device).
static size_t attention_tile_lds_limit() {
    static thread_local size_t limit = 0;
    static thread_local int limit_dev = -1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void) hipGetLastError();
        dev = -1;
    }
    if (dev < 0 || dev != limit_dev) {
        int v = 0;
        limit = 0;
        if (dev >= 0 &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 1024) {
            const size_t want = (size_t) v - 1024;           // static arrays of the kernel: 4 x ATT_P words
            if (hipFuncSetAttribute((const void *) attention_tile_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int) want) == hipSuccess &&
                hipFuncSetAttribute((const void *) attention_tile_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int) want) == hipSuccess) {
                limit = want;
            } else {
                (void) hipGetLastError();
                limit = 65536 - 1024;
            }
        }
        limit_dev = dev;
    }
    return limit;
}

// Lanes per row of the fp32 row kernels: the largest power of two <= min(64, C / 4).
static int row_lanes_log2(int C) {
    int lg = 0;
    while (lg < 6 && (4 << (lg + 1)) <= C) ++lg;
    return lg;
}


// A producer's rows written as fp32: shared checks and launch.
template <typename Src>
static int32_t launch_rows(const char * what, const Src & src, int32_t T, int32_t C, float * out, void * stream) {
    if (T < 0 || C < 4 || C % 4 != 0) return fail(NXG_EINVAL, "%s: T=%d C=%d (C must be a positive multiple of 4)", what, T, C);
    if (T == 0) return NXG_OK;
    if (!out || !aligned16(out)) return fail(NXG_EINVAL, "%s: output null or not 16-byte aligned", what);
    int rc = check_device();
    if (rc) return rc;
    const int lg = row_lanes_log2(C);
    const int rows_per_wg = 256 >> lg;
    const unsigned grid = (unsigned) ((T + rows_per_wg - 1) / rows_per_wg);
    produce_rows_kernel<Src><<<grid, 256, 0, (hipStream_t) stream>>>(src, T, C, lg, out);
    return launch_check(what);
}

extern "C" {

int32_t nxg_init(void) { return check_device(); }

size_t nxg_qact_q_bytes(int32_t T, int32_t n_in) {
    qact_dims d;
    return qact_dims_of(T, n_in, d) ? (size_t) d.MP * d.KS * 64 : 0;
}

size_t nxg_qact_sx_bytes(int32_t T, int32_t n_in) {
    qact_dims d;
    return qact_dims_of(T, n_in, d) ? (size_t) d.MP * d.n_blk * sizeof(float) : 0;
}

static int32_t launch_quantize(const float * x, int32_t T, int32_t n_in, int32_t act_max,
                               int8_t * q, float * sx, void * stream, bool relu2) {
    qact_dims d;
    if (!qact_dims_of(T, n_in, d)) return fail(NXG_EINVAL, "quantize: T=%d n_in=%d (n_in must be a positive multiple of 32)", T, n_in);
    if (act_max != 127 && act_max != 63) return fail(NXG_EINVAL, "quantize: act_max must be 127 or 63, got %d", act_max);
    if (T == 0) return NXG_OK;
    if (!x || !q || !sx) return fail(NXG_EINVAL, "quantize: null buffer");
    if (!aligned16(x) || !aligned16(q) || !aligned16(sx)) return fail(NXG_EINVAL, "quantize: x, q and sx must be 16-byte aligned");
    int rc = check_device();
    if (rc) return rc;
    const long long n_wg = (long long) (d.MP / 16) * d.n_blk;
    if (n_wg > INT32_MAX) return fail(NXG_EINVAL, "quantize: T=%d n_in=%d too large", T, n_in);
    const dim3 grid((unsigned) n_wg);
    hipStream_t s = (hipStream_t) stream;
    if (act_max == 127) {
        if (relu2) quantize_kernel<127, Q_RELU2><<<grid, 256, 0, s>>>(x, T, n_in, d.KS, d.n_blk, q, sx);
        else       quantize_kernel<127, Q_PLAIN><<<grid, 256, 0, s>>>(x, T, n_in, d.KS, d.n_blk, q, sx);
    } else {
        if (relu2) quantize_kernel<63, Q_RELU2><<<grid, 256, 0, s>>>(x, T, n_in, d.KS, d.n_blk, q, sx);
        else       quantize_kernel<63, Q_PLAIN><<<grid, 256, 0, s>>>(x, T, n_in, d.KS, d.n_blk, q, sx);
    }
    return launch_check("quantize_kernel");
}

int32_t nxg_quantize_rows(const float * x, int32_t T, int32_t n_in, int32_t act_max,
                          int8_t * q, float * sx, void * stream) {
    return launch_quantize(x, T, n_in, act_max, q, sx, stream, false);
}

int32_t nxg_quantize_rows_relu2(const float * x, int32_t T, int32_t n_in, int32_t act_max,
                                int8_t * q, float * sx, void * stream) {
    return launch_quantize(x, T, n_in, act_max, q, sx, stream, true);
}

int32_t nxg_rmsnorm_quantize_rows(const float * x, const float * gain, float eps, int32_t T, int32_t n_in,
                                  int32_t act_max, int8_t * q, float * sx, void * stream) {
    qact_dims d;
    if (!qact_dims_of(T, n_in, d)) return fail(NXG_EINVAL, "rmsnorm_quantize: T=%d n_in=%d (n_in must be a positive multiple of 32)", T, n_in);
    if (act_max != 127 && act_max != 63) return fail(NXG_EINVAL, "rmsnorm_quantize: act_max must be 127 or 63, got %d", act_max);
    if (T == 0) return NXG_OK;
    if (!x || !gain || !q || !sx) return fail(NXG_EINVAL, "rmsnorm_quantize: null buffer");
    if (!aligned16(x) || !aligned16(gain) || !aligned16(q) || !aligned16(sx)) {
        return fail(NXG_EINVAL, "rmsnorm_quantize: x, gain, q and sx must be 16-byte aligned");
    }
    int rc = check_device();
    if (rc) return rc;
    hipStream_t s = (hipStream_t) stream;
    if (n_in % BLK == 0) {
        // the whole row group in registers: n_in = 256, 512, 1024 or 2048
        // fewer row groups than twice the CUs: one workgroup per (row group, block)
        const bool split = (long long) (d.MP / 16) < 2LL * device_cus();
        const dim3 grid((unsigned) (d.MP / 16)), grid_s((unsigned) ((d.MP / 16 + 7) / 8 * 8 * d.n_blk));
#define NXG_RMS_Q8(NB)                                                                                        \
        case NB:                                                                                              \
            if (split) {                                                                                      \
                if (act_max == 127) rmsnorm_q8_kernel<127, NB, true><<<grid_s, 256, 0, s>>>(x, gain, eps, T, q, sx); \
                else                rmsnorm_q8_kernel<63, NB, true><<<grid_s, 256, 0, s>>>(x, gain, eps, T, q, sx);  \
            } else {                                                                                          \
                if (act_max == 127) rmsnorm_q8_kernel<127, NB, false><<<grid, 256, 0, s>>>(x, gain, eps, T, q, sx); \
                else                rmsnorm_q8_kernel<63, NB, false><<<grid, 256, 0, s>>>(x, gain, eps, T, q, sx);  \
            }                                                                                                 \
            return launch_check("rmsnorm_q8_kernel");
        switch (d.n_blk) {
            NXG_RMS_Q8(1)
            NXG_RMS_Q8(2)
            NXG_RMS_Q8(4)
            NXG_RMS_Q8(8)
            default: break;
        }
#undef NXG_RMS_Q8
    }
    const long long n_wg = (long long) ((d.MP / 16 + 7) / 8) * 8 * d.n_blk;   // (row group, block), whole XCD rounds
    if (n_wg > INT32_MAX) return fail(NXG_EINVAL, "rmsnorm_quantize: T=%d n_in=%d too large", T, n_in);
    const dim3 grid((unsigned) n_wg);
    if (act_max == 127) rmsnorm_quantize_kernel<127><<<grid, 256, 0, s>>>(x, gain, eps, T, n_in, d.KS, d.n_blk, q, sx);
    else                rmsnorm_quantize_kernel<63><<<grid, 256, 0, s>>>(x, gain, eps, T, n_in, d.KS, d.n_blk, q, sx);
    return launch_check("rmsnorm_quantize_kernel");
}

int32_t nxg_gate_quantize_rows(const float * g, const float * y, int32_t T, int32_t n_in, int32_t act_max,
                               int8_t * q, float * sx, void * stream) {
    if (T > 0 && (!g || !y)) return fail(NXG_EINVAL, "gate_quantize: null input");
    if (!aligned16(g) || !aligned16(y)) return fail(NXG_EINVAL, "gate_quantize: inputs must be 16-byte aligned");
    return launch_produce("gate_quantize", src_gate{g, y, n_in}, T, n_in, act_max, q, sx, stream);
}

int32_t nxg_dwconv_quantize_rows(const float * x, const float * r, const float * taps, int32_t k,
                                 const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t n_in,
                                 int32_t act_max, int8_t * q, float * sx, void * stream) {
    if (T > 0 && (!x || !taps || !cu_offsets)) return fail(NXG_EINVAL, "dwconv_quantize: null input");
    if (k < 1 || n_seqs < 1) return fail(NXG_EINVAL, "dwconv_quantize: k=%d n_seqs=%d (both must be >= 1)", k, n_seqs);
    if (!aligned16(x) || !aligned16(r) || !aligned16(taps)) return fail(NXG_EINVAL, "dwconv_quantize: inputs must be 16-byte aligned");
    return launch_produce("dwconv_quantize", src_dwconv{x, r, taps, cu_offsets, n_seqs, T, n_in, k},
                          T, n_in, act_max, q, sx, stream);
}

int32_t nxg_lily_state_quantize_rows(const float * a, const float * x, const float * b, const float * taps, int32_t k,
                                     const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t n_in,
                                     int32_t act_max, int8_t * q, float * sx, void * stream) {
    if (T > 0 && (!a || !x || !b || !taps || !cu_offsets)) return fail(NXG_EINVAL, "lily_state_quantize: null input");
    if (k < 1 || n_seqs < 1) return fail(NXG_EINVAL, "lily_state_quantize: k=%d n_seqs=%d (both must be >= 1)", k, n_seqs);
    if (!aligned16(a) || !aligned16(x) || !aligned16(b) || !aligned16(taps)) {
        return fail(NXG_EINVAL, "lily_state_quantize: inputs must be 16-byte aligned");
    }
    return launch_produce("lily_state_quantize", src_lily_state{a, x, b, taps, cu_offsets, n_seqs, T, n_in, k},
                          T, n_in, act_max, q, sx, stream);
}

int32_t nxg_block_mean_quantize_rows(const float * h, const float * g, const int32_t * cu_offsets,
                                     const int32_t * cu_blocks, int32_t n_seqs, int32_t T, int32_t n_blocks,
                                     int32_t block, int32_t n_in, int32_t act_max, int8_t * q, float * sx,
                                     void * stream) {
    if (n_blocks > 0 && (!h || !cu_offsets || !cu_blocks)) return fail(NXG_EINVAL, "block_mean_quantize: null input");
    if (block < 1 || n_seqs < 1 || T < 0) {
        return fail(NXG_EINVAL, "block_mean_quantize: block=%d n_seqs=%d T=%d (block, n_seqs >= 1)", block, n_seqs, T);
    }
    if (!aligned16(h) || !aligned16(g)) return fail(NXG_EINVAL, "block_mean_quantize: inputs must be 16-byte aligned");
    return launch_produce("block_mean_quantize", src_block_mean{h, g, cu_offsets, cu_blocks, n_seqs, T, n_blocks, n_in, block},
                          n_blocks, n_in, act_max, q, sx, stream);
}

// Resident workgroups of attention_stored_kernel on the device (its persistent grid and
// the workspace slots), queried once.
// The scratch of nxg_attention_noalloc: a device array of the code object, so the entry point
// allocates nothing. Each GPU the library runs on holds its own copy at its own address (until
// the process ends); host code uses that address, found once per device by
// hipGetSymbolAddress, never the array's name (a host-side stand-in). Every call on a GPU
// shares the array: the scores a workgroup writes to its slot are read back by the same
// workgroup within the call, so nothing needs clearing, and calls that overlap on one GPU race.
static __device__ __align__(256) float scratch[NXG_NOALLOC_SCRATCH_BYTES / sizeof(float)];

static constexpr int MAX_DEVICES = 64;
static std::mutex scratch_mutex;
static void * scratch_ptr[MAX_DEVICES] = {};

static int scratch_of_device(void ** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= MAX_DEVICES) return fail(NXG_EDEVICE, "attention_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void * p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return NXG_OK;
}

// Workgroups of the long attention kernel resident at once on the current device (its
// compute units x occupancy), each needing one workspace slot. Cached per thread for the
// device it was computed on, like check_device's device check.
static long long attention_long_slots() {
    static thread_local long long slots = 0;
    static thread_local int slots_dev = -1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void) hipGetLastError();
        dev = -1;
    }
    if (dev < 0 || dev != slots_dev) {
        int cus = 0, per_cu = 0;
        if (dev >= 0 &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attention_stored_kernel<false, false>, 256, 0) == hipSuccess &&
            cus > 0 && per_cu > 0) {
            slots = (long long) cus * per_cu;
        } else {
            (void) hipGetLastError();
            slots = 256;
        }
        slots_dev = dev;
    }
    return slots;
}

// The launch nxg_attention_ws makes for (T, heads, max_keys): 0 tile kernel, 1 stored kernel
// given a workspace slot (else the tile kernel where its LDS fits, else the recomputing long
// kernel), 2 row kernel; the tiles, the workspace bytes of one slot, and whether the tile
// kernel's LDS fits.
struct attn_plan {
    int kind;
    long long n_tiles;
    long long slot_bytes;
    bool tile_fits;
};

// The tile kernel keeps its scores in LDS: ATT_P * smax floats beside one staged tile. Where
// that leaves room for one workgroup per CU, or for two while the launch has more than two
// rounds of them, attention_stored_kernel (the scores in a workspace slot, three workgroups
// per CU) is faster: 2,048 keys 970 -> 560 us, 1,536 keys 560 -> 320 us, 2 x 1,024 keys
// 314 -> 279 us, 8 x 1,024 keys 1,098 -> 1,015 us; one 1,024-key document (1,024 tiles, two
// rounds) stays 3% faster on the tile kernel.
static bool attention_tile_first(size_t tile_lds, size_t lds_max, long long n_tiles) {
    if (tile_lds > lds_max) return false;
    const size_t per_cu = (lds_max + 1024) / (tile_lds + 1024);   // the static 1 KiB included
    return per_cu >= 3 || (per_cu == 2 && n_tiles <= 4LL * device_cus());
}

static attn_plan plan_attention(int32_t T, int32_t n_head, int32_t n_kv_head, int32_t max_keys) {
    const int rep = n_head / n_kv_head;
    if (ATT_P % rep != 0) return {2, 0, 0, false};
    const long long n_tiles = (long long) n_kv_head * ((T + ATT_P / rep - 1) / (ATT_P / rep));
    const int smax = (max_keys + 3) & ~3;
    const size_t tile_lds = ((size_t) ATT_P * smax + (size_t) ATT_KT * ATT_KS) * sizeof(float);
    const size_t lds_max = attention_tile_lds_limit();
    if (attention_tile_first(tile_lds, lds_max, n_tiles)) return {0, n_tiles, 0, true};
    return {1, n_tiles, (long long) ATT_P * max_keys * (long long) sizeof(float), tile_lds <= lds_max};
}

int64_t nxg_attention_workspace_bytes(int32_t T, int32_t n_head, int32_t n_kv_head, int32_t max_keys) {
    if (T < 0 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head != 0 || max_keys < 1) {
        return fail(NXG_EINVAL, "attention_workspace_bytes: T=%d n_head=%d n_kv_head=%d max_keys=%d", T, n_head,
                    n_kv_head, max_keys);
    }
    if (T == 0) return 0;
    int rc = check_device();
    if (rc) return rc;
    const attn_plan pl = plan_attention(T, n_head, n_kv_head, max_keys);
    if (pl.kind != 1) return 0;
    return std::min(pl.n_tiles, attention_long_slots()) * pl.slot_bytes;
}

int32_t nxg_attention_noalloc(const float * q, const float * k, const float * v, const int32_t * cu_offsets,
                              int32_t n_seqs, const float * scale, int32_t T, int32_t n_head, int32_t n_kv_head,
                              int32_t half, int32_t max_keys, float * out, void * stream) {
    if (T < 0 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head != 0 || max_keys < 1) {
        return fail(NXG_EINVAL, "attention_noalloc: T=%d n_head=%d n_kv_head=%d max_keys=%d", T, n_head, n_kv_head,
                    max_keys);
    }
    if (T == 0) return NXG_OK;
    int rc = check_device();
    if (rc) return rc;
    const attn_plan pl = plan_attention(T, n_head, n_kv_head, max_keys);
    const bool use_scratch = pl.kind == 1 && pl.slot_bytes <= (long long) NXG_NOALLOC_SCRATCH_BYTES;
    if (pl.kind == 1 && !use_scratch && !pl.tile_fits) {
        return fail(NXG_EINVAL,
                    "attention_noalloc: max_keys=%d needs %lld bytes per workgroup's scores; the static scratch "
                    "holds %lld (at most %lld keys)", max_keys, pl.slot_bytes, (long long) NXG_NOALLOC_SCRATCH_BYTES,
                    (long long) NXG_NOALLOC_SCRATCH_BYTES / (ATT_P * (long long) sizeof(float)));
    }
    void * ws = nullptr;                       // none: the tile kernel, its scores in LDS
    if (use_scratch) {
        rc = scratch_of_device(&ws);
        if (rc) return rc;
    }
    return nxg_attention_ws(q, k, v, cu_offsets, n_seqs, scale, T, n_head, n_kv_head, half, max_keys, out, ws,
                            ws ? (int64_t) NXG_NOALLOC_SCRATCH_BYTES : 0, stream);
}

int32_t nxg_attention(const float * q, const float * k, const float * v, const int32_t * cu_offsets,
                      int32_t n_seqs, const float * scale, int32_t T, int32_t n_head, int32_t n_kv_head,
                      int32_t half, int32_t max_keys, float * out, void * stream) {
    return nxg_attention_ws(q, k, v, cu_offsets, n_seqs, scale, T, n_head, n_kv_head, half, max_keys, out, nullptr,
                            0, stream);
}

int32_t nxg_attention_ws(const float * q, const float * k, const float * v, const int32_t * cu_offsets,
                         int32_t n_seqs, const float * scale, int32_t T, int32_t n_head, int32_t n_kv_head,
                         int32_t half, int32_t max_keys, float * out, void * workspace, int64_t workspace_bytes,
                         void * stream) {
    if (T < 0 || n_seqs < 1 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head != 0) {
        return fail(NXG_EINVAL, "attention: T=%d n_seqs=%d n_head=%d n_kv_head=%d", T, n_seqs, n_head, n_kv_head);
    }
    if (max_keys < 1) return fail(NXG_EINVAL, "attention: max_keys=%d (must be >= 1)", max_keys);
    if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) || ((uintptr_t) workspace & 3)) {
        return fail(NXG_EINVAL, "attention: workspace %p of %lld bytes", workspace, (long long) workspace_bytes);
    }
    if (T == 0) return NXG_OK;
    if (!q || !k || !v || !cu_offsets || !scale || !out) return fail(NXG_EINVAL, "attention: null buffer");
    const long long n_wg = (long long) T * n_head;
    if (n_wg > INT32_MAX) return fail(NXG_EINVAL, "attention: T=%d n_head=%d too large", T, n_head);
    int rc = check_device();
    if (rc) return rc;
    attn_params p{q, k, v, cu_offsets, scale, out, n_seqs, T, n_head, n_kv_head, half < 0 ? -1 : half, max_keys};
    // the tiled kernel when its LDS (scores of ATT_P pairs + one staged tile) fits a workgroup
    // and attention_tile_first prefers it, or no workspace slot is given
    const int rep = n_head / n_kv_head;
    const int smax = (max_keys + 3) & ~3;
    const size_t tile_lds = ((size_t) ATT_P * smax + (size_t) ATT_KT * ATT_KS) * sizeof(float);
    if (ATT_P % rep == 0) {
        const attn_plan pl = plan_attention(T, n_head, n_kv_head, max_keys);
        const long long n_tiles = pl.n_tiles;
        const size_t lds_max = attention_tile_lds_limit();
        // scores written once into the workspace: as many slots as it holds, up to the resident workgroups
        const long long n_slots =
            pl.kind == 1 ? std::min({n_tiles, attention_long_slots(), (long long) (workspace_bytes / pl.slot_bytes)}) : 0;
        if (tile_lds <= lds_max && n_slots < 1) {
            // fewer than 3 workgroups per CU by LDS (the static 1 KiB included): 16 pairs per lane group
            if (NXG_ATT_WIDE && 3 * (tile_lds + 1024) > lds_max + 1024) {
                attention_tile_kernel<true><<<dim3((unsigned) n_tiles), dim3(256), tile_lds, (hipStream_t) stream>>>(p, smax);
            } else {
                attention_tile_kernel<false><<<dim3((unsigned) n_tiles), dim3(256), tile_lds, (hipStream_t) stream>>>(p, smax);
            }
            return launch_check("attention_tile_kernel");
        }
        if (n_slots >= 1) {
            // e stored by pass 2 (4 more bytes per (pair, key)) pays while the slots in use stay
            // in the last-level cache: 4,096 keys 1.97 -> 1.94 ms, 16,384 keys in bands of 2,601
            // 5.39 -> 5.32 ms; beyond it even or slower (at two workgroups per CU: 8,192 keys even,
            // 16,384 keys 40.8 -> 44.6 ms)
            const bool e_store = (double) n_slots * (double) pl.slot_bytes <= (double) NXG_ATT_E_STORE_MIB * 1048576.0;
            const dim3 grid((unsigned) n_slots), block(256);
            float * const ws = (float *) workspace;
            hipStream_t s = (hipStream_t) stream;
            if (e_store && p.half >= 0) attention_stored_kernel<true, true><<<grid, block, 0, s>>>(p, ws);
            else if (e_store)           attention_stored_kernel<true, false><<<grid, block, 0, s>>>(p, ws);
            else if (p.half >= 0)       attention_stored_kernel<false, true><<<grid, block, 0, s>>>(p, ws);
            else                        attention_stored_kernel<false, false><<<grid, block, 0, s>>>(p, ws);
            return launch_check("attention_stored_kernel");
        }
        attention_long_kernel<<<dim3((unsigned) n_tiles), dim3(256), 0, (hipStream_t) stream>>>(p);
        return launch_check("attention_long_kernel");
    }
    if (max_keys > NXG_ATTN_MAX_KEYS) {
        return fail(NXG_EINVAL, "attention: max_keys=%d: with n_head / n_kv_head = %d (not a divisor of %d) at most %d",
                    max_keys, rep, ATT_P, NXG_ATTN_MAX_KEYS);
    }
    attention_kernel<<<dim3((unsigned) n_wg), dim3(64), (size_t) max_keys * sizeof(float), (hipStream_t) stream>>>(p);
    return launch_check("attention_kernel");
}

int32_t nxg_qk_prep(const float * x, const float * alpha, const float * beta, const float * cos_t, const float * sin_t,
                    int32_t n_pos, const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t n_head,
                    int32_t head_dim, int32_t head_major, float * out, void * stream) {
    if (T < 0 || n_head < 1 || head_dim < 2 || head_dim % 2 != 0 || n_pos < 1 || n_seqs < 1) {
        return fail(NXG_EINVAL, "qk_prep: T=%d n_head=%d head_dim=%d n_pos=%d n_seqs=%d", T, n_head, head_dim, n_pos, n_seqs);
    }
    if (T == 0) return NXG_OK;
    if (!x || !alpha || !beta || !cos_t || !sin_t || !cu_offsets || !out) return fail(NXG_EINVAL, "qk_prep: null buffer");
    const long long per_row = (long long) n_head * (head_dim / 2);
    if (per_row > INT32_MAX / 2) return fail(NXG_EINVAL, "qk_prep: too large");
    int rc = check_device();
    if (rc) return rc;
    qk_prep_kernel<<<dim3((unsigned) T, (unsigned) ((per_row + 255) / 256)), 256, 0, (hipStream_t) stream>>>(
        x, alpha, beta, cos_t, sin_t, cu_offsets, n_seqs, T, n_head, head_dim, n_pos, head_major ? 1 : 0, out);
    return launch_check("qk_prep_kernel");
}

int32_t nxg_head_major(const float * x, int32_t T, int32_t n_head, int32_t head_dim, float * out, void * stream) {
    if (T < 0 || n_head < 1 || head_dim < 1) return fail(NXG_EINVAL, "head_major: T=%d n_head=%d head_dim=%d", T, n_head, head_dim);
    if (T == 0) return NXG_OK;
    if (!x || !out) return fail(NXG_EINVAL, "head_major: null buffer");
    const long long per_row = (long long) n_head * head_dim;
    if (per_row > INT32_MAX / 2) return fail(NXG_EINVAL, "head_major: too large");
    int rc = check_device();
    if (rc) return rc;
    head_major_kernel<<<dim3((unsigned) T, (unsigned) ((per_row + 255) / 256)), 256, 0, (hipStream_t) stream>>>(
        x, T, n_head, head_dim, out);
    return launch_check("head_major_kernel");
}

int32_t nxg_qkv_prep(const float * q, const float * k, const float * v, const float * q_alpha, const float * q_beta,
                     const float * k_alpha, const float * k_beta, const float * cos_t, const float * sin_t, int32_t n_pos,
                     const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t n_head, int32_t n_kv_head,
                     int32_t head_dim, float * q_out, float * k_out, float * v_out, void * stream) {
    if (T < 0 || n_head < 1 || n_kv_head < 1 || head_dim < 2 || head_dim % 2 != 0 || n_pos < 1 || n_seqs < 1) {
        return fail(NXG_EINVAL, "qkv_prep: T=%d n_head=%d n_kv_head=%d head_dim=%d n_pos=%d n_seqs=%d", T, n_head,
                    n_kv_head, head_dim, n_pos, n_seqs);
    }
    if (T == 0) return NXG_OK;
    if (!q || !k || !v || !q_alpha || !q_beta || !k_alpha || !k_beta || !cos_t || !sin_t || !cu_offsets || !q_out ||
        !k_out || !v_out) {
        return fail(NXG_EINVAL, "qkv_prep: null buffer");
    }
    const long long per_row = (long long) (n_head + n_kv_head) * (head_dim / 2) + (long long) n_kv_head * head_dim;
    if (per_row > INT32_MAX / 2) return fail(NXG_EINVAL, "qkv_prep: too large");
    int rc = check_device();
    if (rc) return rc;
    const qkv_prep_params p{ q, k, v, q_alpha, q_beta, k_alpha, k_beta, cos_t, sin_t, cu_offsets, n_seqs, T,
                             n_head, n_kv_head, head_dim, n_pos, q_out, k_out, v_out };
    qkv_prep_kernel<<<dim3((unsigned) T, (unsigned) ((per_row + 255) / 256)), 256, 0, (hipStream_t) stream>>>(p);
    return launch_check("qkv_prep_kernel");
}

int32_t nxg_dwconv_rows(const float * x, const float * r, const float * taps, int32_t k, const int32_t * cu_offsets,
                        int32_t n_seqs, int32_t T, int32_t C, float * out, void * stream) {
    if (T > 0 && (!x || !taps || !cu_offsets)) return fail(NXG_EINVAL, "dwconv_rows: null input");
    if (k < 1 || n_seqs < 1) return fail(NXG_EINVAL, "dwconv_rows: k=%d n_seqs=%d (both must be >= 1)", k, n_seqs);
    if (T > 0 && (!aligned16(x) || !aligned16(taps) || (r && !aligned16(r)))) {
        return fail(NXG_EINVAL, "dwconv_rows: inputs must be 16-byte aligned");
    }
    return launch_rows("dwconv_rows", src_dwconv{x, r, taps, cu_offsets, n_seqs, T, C, k}, T, C, out, stream);
}

int32_t nxg_upsample_add(const float * yb, const float * r, const int32_t * cu_offsets, const int32_t * cu_blocks,
                         int32_t n_seqs, int32_t T, int32_t n_blocks, int32_t block, int32_t C, float * out,
                         void * stream) {
    if (block < 1 || n_seqs < 1 || (T > 0 && n_blocks < 1)) {
        return fail(NXG_EINVAL, "upsample_add: block=%d n_seqs=%d n_blocks=%d", block, n_seqs, n_blocks);
    }
    if (T > 0 && (!yb || !r || !cu_offsets || !cu_blocks)) return fail(NXG_EINVAL, "upsample_add: null input");
    if (T > 0 && (!aligned16(yb) || !aligned16(r))) return fail(NXG_EINVAL, "upsample_add: inputs must be 16-byte aligned");
    return launch_rows("upsample_add", src_upsample_add{yb, r, cu_offsets, cu_blocks, n_seqs, T, n_blocks, C, block},
                       T, C, out, stream);
}

int32_t nxg_embed_rows(const float * table, int32_t n_vocab, const int32_t * ids, const float * type_table,
                       int32_t n_types, const int32_t * types, int32_t T, int32_t C, float * out, void * stream) {
    if (T < 0 || C < 4 || C % 4 != 0 || n_vocab < 1 || (type_table && n_types < 1)) {
        return fail(NXG_EINVAL, "embed_rows: T=%d C=%d n_vocab=%d n_types=%d", T, C, n_vocab, n_types);
    }
    if (T == 0) return NXG_OK;
    if (!table || !ids || !out || (type_table && !types)) return fail(NXG_EINVAL, "embed_rows: null buffer");
    if (!aligned16(table) || !aligned16(out) || (type_table && !aligned16(type_table))) {
        return fail(NXG_EINVAL, "embed_rows: tables and output must be 16-byte aligned");
    }
    int rc = check_device();
    if (rc) return rc;
    const int lg = row_lanes_log2(C);
    const int rows_per_wg = 256 >> lg;
    embed_rows_kernel<<<(unsigned) ((T + rows_per_wg - 1) / rows_per_wg), 256, 0, (hipStream_t) stream>>>(
        table, n_vocab, ids, type_table, n_types, types, T, C, lg, out);
    return launch_check("embed_rows_kernel");
}

int32_t nxg_layer_norm(const float * x, const float * w, const float * b, float eps, int32_t T, int32_t C, float * out,
                       void * stream) {
    if (T < 0 || C < 1) return fail(NXG_EINVAL, "layer_norm: T=%d C=%d", T, C);
    if (T == 0) return NXG_OK;
    if (!x || !out) return fail(NXG_EINVAL, "layer_norm: null buffer");
    int rc = check_device();
    if (rc) return rc;
    layer_norm_kernel<<<(unsigned) ((T + 3) / 4), 256, 0, (hipStream_t) stream>>>(x, w, b, eps, T, C, out);
    return launch_check("layer_norm_kernel");
}

int32_t nxg_doc_mean(const float * x, const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t C, int32_t normalize,
                     float * out, void * stream) {
    if (n_seqs < 0 || T < 0 || C < 4 || C % 4 != 0) return fail(NXG_EINVAL, "doc_mean: n_seqs=%d T=%d C=%d", n_seqs, T, C);
    if (normalize && C % 32 != 0) return fail(NXG_EINVAL, "doc_mean: normalize needs C a multiple of 32, got %d", C);
    if (n_seqs == 0) return NXG_OK;
    if (!x || !cu_offsets || !out || !aligned16(x) || !aligned16(out)) {
        return fail(NXG_EINVAL, "doc_mean: null or unaligned buffer");
    }
    int rc = check_device();
    if (rc) return rc;
    const int n_slices = (C + DS_COLS - 1) / DS_COLS;
    if ((int64_t) n_seqs * n_slices > INT32_MAX) return fail(NXG_EINVAL, "doc_mean: %d documents of %d columns", n_seqs, C);
    doc_sum_kernel<<<(unsigned) (n_seqs * n_slices), 256, 0, (hipStream_t) stream>>>(x, cu_offsets, T, C, n_slices,
                                                                                     normalize ? 0 : 1, out);
    rc = launch_check("doc_sum_kernel");
    if (rc || !normalize) return rc;
    doc_norm_kernel<<<(unsigned) n_seqs, 256, 0, (hipStream_t) stream>>>(C, out);
    return launch_check("doc_norm_kernel");
}

int32_t nxg_qact_export(const int8_t * q, const float * sx, int32_t T, int32_t n_in, int32_t act_max,
                        uint8_t * u8, float * sx_ref, void * stream) {
    qact_dims d;
    if (!qact_dims_of(T, n_in, d)) return fail(NXG_EINVAL, "export: T=%d n_in=%d", T, n_in);
    if (act_max != 127 && act_max != 63) return fail(NXG_EINVAL, "export: act_max must be 127 or 63");
    if (T == 0) return NXG_OK;
    if (!q || !sx || !u8 || !sx_ref) return fail(NXG_EINVAL, "export: null buffer");
    int rc = check_device();
    if (rc) return rc;
    hipStream_t s = (hipStream_t) stream;
    const size_t n = (size_t) T * (n_in / 16);
    export_kernel<<<(unsigned) ((n + 255) / 256), 256, 0, s>>>(q, T, n_in, d.KS, act_max + 1, u8);
    rc = launch_check("export_kernel");
    if (rc) return rc;
    const size_t sx_n = (size_t) ((T + 3) / 4) * d.n_blk * 4;
    const hipError_t e = hipMemcpyAsync(sx_ref, sx, sx_n * sizeof(float), hipMemcpyDeviceToDevice, s);
    return e == hipSuccess ? NXG_OK : hip_fail(e, "export: hipMemcpyAsync");
}

int32_t nxg_weight_create(const int8_t * w, const float * scale, int32_t n_in, int32_t n_out, nxg_weight ** out) {
    if (!out) return fail(NXG_EINVAL, "weight_create: null out");
    *out = nullptr;
    if (!w || !scale) return fail(NXG_EINVAL, "weight_create: null input");
    if (n_in <= 0 || n_in % 32 != 0 || n_out <= 0) {
        return fail(NXG_EINVAL, "weight_create: n_in=%d n_out=%d (n_in must be a positive multiple of 32)", n_in, n_out);
    }
    int rc = check_device();
    if (rc) return rc;
    nxg_weight * W = new nxg_weight();
    W->n_in = n_in;
    W->n_out = n_out;
    W->n_blk = ceil_div(n_in, BLK);
    W->KS = ceil_div(n_in, 64);
    W->NP = ceil_div(n_out, WBN) * WBN;   // whole tiles of the widest kernel
    const size_t wbytes = (size_t) W->NP * W->KS * 64;
    const size_t sbytes = (size_t) W->n_blk * W->NP * sizeof(float);
    // Re-layout on the host into fragment tiles (zero padding), then one copy.
    std::vector<int8_t> tiled(wbytes, 0);
    nxg_tile_rows(w, n_out, n_in, W->KS, tiled.data());
    std::vector<float> sw((size_t) W->n_blk * W->NP, 0.0f);
    for (int B = 0; B < W->n_blk; ++B) {
        std::memcpy(&sw[(size_t) B * W->NP], scale + (size_t) B * n_out, sizeof(float) * n_out);
    }
    hipError_t e = hipMalloc((void **) &W->w, wbytes);
    if (e != hipSuccess) { delete W; return fail(NXG_ENOMEM, "weight_create: hipMalloc(%zu): %s", wbytes, hipGetErrorString(e)); }
    e = hipMalloc((void **) &W->sw, sbytes);
    if (e != hipSuccess) { (void) hipFree(W->w); delete W; return fail(NXG_ENOMEM, "weight_create: hipMalloc(%zu): %s", sbytes, hipGetErrorString(e)); }
    e = hipMemcpy(W->w, tiled.data(), wbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(W->sw, sw.data(), sbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) { nxg_weight_destroy(W); return hip_fail(e, "weight_create: hipMemcpy"); }
    W->bytes = wbytes + sbytes;
    *out = W;
    return NXG_OK;
}

void nxg_weight_destroy(nxg_weight * W) {
    if (!W) return;
    if (W->w) (void) hipFree(W->w);
    if (W->sw) (void) hipFree(W->sw);
    delete W;
}

int32_t nxg_weight_n_in(const nxg_weight * W) { return W ? W->n_in : 0; }
int32_t nxg_weight_n_out(const nxg_weight * W) { return W ? W->n_out : 0; }
size_t nxg_weight_device_bytes(const nxg_weight * W) { return W ? W->bytes : 0; }

// Where a GEMM writes: fp32 rows (+ residual), per-block int32 sums, or relu^2
// quantized for the next linear.
struct gemm_out {
    const float * residual = nullptr;
    float *       out = nullptr;
    int32_t *     sums = nullptr;
    int8_t *      qo = nullptr;
    float *       sxo = nullptr;
    int           act_max = 127;
    int           n_seg = 0;                 // split output: column counts and buffers
    const int32_t * seg_cols = nullptr;
    float * const * seg_out = nullptr;
    const float * xf = nullptr;              // relu^2 output only: fp32 input rows quantized in the GEMM
};

static int32_t launch_gemm(const nxg_weight * W, const int8_t * q, const float * sx, int32_t T,
                           const gemm_out & o, void * stream) {
    if (!W) return fail(NXG_EINVAL, "linear: null weight");
    if (T < 0) return fail(NXG_EINVAL, "linear: T=%d", T);
    if (T == 0) return NXG_OK;
    const bool k256 = W->KS % 4 == 0;
    if (o.n_seg) {
        // split output: n_in % 256 == 0 (gemm_k256 / gemm_small / gemm_fsk), boundaries at multiples of 64
        if (o.n_seg < 1 || o.n_seg > 4 || !o.seg_cols || !o.seg_out || o.residual || o.sums || o.qo) {
            return fail(NXG_EINVAL, "linear_split: n_seg=%d (1..4, no residual)", o.n_seg);
        }
        if (!k256 || W->n_out % 4 != 0 || NXG_WG_PER_CU <= 0) {
            return fail(NXG_EINVAL, "linear_split: needs n_in %% 256 == 0 and n_out %% 4 == 0 (n_in=%d n_out=%d)",
                        W->n_in, W->n_out);
        }
        int end = 0;
        for (int k = 0; k < o.n_seg; ++k) {
            if (o.seg_cols[k] <= 0 || (k + 1 < o.n_seg && (end + o.seg_cols[k]) % 64 != 0) || o.seg_cols[k] % 4 != 0) {
                return fail(NXG_EINVAL, "linear_split: segment %d has %d columns (boundaries at multiples of 64)", k,
                            o.seg_cols[k]);
            }
            if (!o.seg_out[k] || ((uintptr_t) o.seg_out[k] & 15)) {
                return fail(NXG_EINVAL, "linear_split: segment %d: null or unaligned buffer", k);
            }
            end += o.seg_cols[k];
        }
        if (end != W->n_out) return fail(NXG_EINVAL, "linear_split: segments cover %d columns, the weight has %d", end, W->n_out);
    } else if ((!o.xf && (!q || (!o.sums && !sx))) || (!o.sums && !o.qo && !o.out) || (o.qo && !o.sxo)) {
        return fail(NXG_EINVAL, "linear: null buffer");
    }
    if (!o.xf && (!q || (!o.sums && !sx))) return fail(NXG_EINVAL, "linear: null buffer");
    if (!aligned16(q) || !aligned16(sx) || !aligned16(o.out) || !aligned16(o.residual) || !aligned16(o.qo) ||
        !aligned16(o.sxo) || !aligned16(o.sums)) {
        return fail(NXG_EINVAL, "linear: device buffers must be 16-byte aligned");
    }
    if (o.xf && (!o.qo || !aligned16(o.xf))) return fail(NXG_EINVAL, "linear_f32: fp32 rows need the relu^2 output and 16-byte alignment");
    if (o.qo) {
        if (!k256 || W->n_out % 32 != 0) {
            return fail(NXG_EINVAL, "linear_relu2_q8: needs n_in %% 256 == 0 and n_out %% 32 == 0 (n_in=%d n_out=%d)",
                        W->n_in, W->n_out);
        }
        if (o.act_max != 127 && o.act_max != 63) return fail(NXG_EINVAL, "linear_relu2_q8: act_max must be 127 or 63, got %d", o.act_max);
    }
    int rc = check_device();
    if (rc) return rc;
    gemm_plan pl;
    if (!plan_gemm(T, W->n_in, W->n_out, o.sums != nullptr, o.qo != nullptr, device_cus(), pl)) {
        return fail(NXG_EINVAL, "linear: T=%d too large", T);
    }
    gemm_params p;
    p.a = q;
    p.sx = sx;
    p.w = W->w;
    p.sw = W->sw;
    p.res = o.residual;
    p.out = o.out;
    p.sums = o.sums;
    p.qo = o.qo;
    p.sxo = o.sxo;
    p.T = pl.T;
    p.N = pl.N;
    p.NP = pl.NP;
    p.KS = pl.KS;
    p.KSo = pl.KSo;
    p.n_blk = pl.n_blk;
    p.MF = pl.MF;
    p.n_mt = pl.n_mt;
    p.n_nt = pl.n_nt;
    p.G = pl.G;
    p.xf = o.xf;
    p.n_seg = o.n_seg;
    for (int k = 0, end = 0; k < 4; ++k) {
        if (k < o.n_seg) end += o.seg_cols[k];
        p.seg_end[k] = end;
        p.seg_out[k] = k < o.n_seg ? o.seg_out[k] : nullptr;
    }
    if (p.NP != W->NP || p.KS != W->KS || p.n_blk != W->n_blk) return fail(NXG_EINVAL, "linear: weight layout mismatch");
    hipStream_t s = (hipStream_t) stream;
    const dim3 grid((unsigned) pl.grid), block((unsigned) pl.block);
    const bool res = o.residual != nullptr;
    if (o.xf && pl.kind != GEMM_RELU2_RT) return fail(NXG_EINVAL, "linear_f32: no fused kernel for this shape");
    switch (pl.kind) {
    case GEMM_RELU2_SMALL:
        if (o.act_max == 127) gemm_relu2_small<127><<<grid, block, 0, s>>>(p);
        else                  gemm_relu2_small<63><<<grid, block, 0, s>>>(p);
        return launch_check("gemm_relu2_small");
    case GEMM_RELU2_Q8:
        if (o.act_max == 127) gemm_relu2_q8<127><<<grid, block, 0, s>>>(p);
        else                  gemm_relu2_q8<63><<<grid, block, 0, s>>>(p);
        return launch_check("gemm_relu2_q8");
    case GEMM_RELU2_RT:
        if ((p.n_blk != 1 && p.n_blk != RNB_MAX) || p.KS != 4 * p.n_blk) return fail(NXG_EINVAL, "linear_relu2_q8: plan/shape mismatch");
        if (o.xf) {
            if (o.act_max == 127) {
                if (p.n_blk == 1) gemm_relu2_rt<127, 1, true><<<grid, block, 0, s>>>(p);
                else              gemm_relu2_rt<127, 4, true><<<grid, block, 0, s>>>(p);
            } else {
                if (p.n_blk == 1) gemm_relu2_rt<63, 1, true><<<grid, block, 0, s>>>(p);
                else              gemm_relu2_rt<63, 4, true><<<grid, block, 0, s>>>(p);
            }
        } else if (o.act_max == 127) {
            if (p.n_blk == 1) gemm_relu2_rt<127, 1, false><<<grid, block, 0, s>>>(p);
            else              gemm_relu2_rt<127, 4, false><<<grid, block, 0, s>>>(p);
        } else {
            if (p.n_blk == 1) gemm_relu2_rt<63, 1, false><<<grid, block, 0, s>>>(p);
            else              gemm_relu2_rt<63, 4, false><<<grid, block, 0, s>>>(p);
        }
        return launch_check("gemm_relu2_rt");
    case GEMM_SMALL:
        if (pl.fn == 2) {
            if (res) { if (pl.k256) gemm_small<2, true, true><<<grid, block, 0, s>>>(p); else gemm_small<2, true, false><<<grid, block, 0, s>>>(p); }
            else     { if (pl.k256) gemm_small<2, false, true><<<grid, block, 0, s>>>(p); else gemm_small<2, false, false><<<grid, block, 0, s>>>(p); }
        } else {
            if (res) { if (pl.k256) gemm_small<4, true, true><<<grid, block, 0, s>>>(p); else gemm_small<4, true, false><<<grid, block, 0, s>>>(p); }
            else     { if (pl.k256) gemm_small<4, false, true><<<grid, block, 0, s>>>(p); else gemm_small<4, false, false><<<grid, block, 0, s>>>(p); }
        }
        return launch_check("gemm_small");
    case GEMM_FSK:
        if (!pl.k256 || p.n_blk > FSK_NB || p.n_nt * pl.fn < p.N || p.n_nt * pl.fn > p.NP)
            return fail(NXG_EINVAL, "linear: plan/shape mismatch (split-block few-row GEMM)");
        if (pl.fn == 64) { if (res) gemm_fsk<64, 4, true><<<grid, block, 0, s>>>(p); else gemm_fsk<64, 4, false><<<grid, block, 0, s>>>(p); }
        else             { if (res) gemm_fsk<32, FSK_NB, true><<<grid, block, 0, s>>>(p); else gemm_fsk<32, FSK_NB, false><<<grid, block, 0, s>>>(p); }
        return launch_check("gemm_fsk");
    case GEMM_SUMS:
        if (pl.k256) gemm_kernel<false, true, true><<<grid, block, 0, s>>>(p);
        else         gemm_kernel<false, true, false><<<grid, block, 0, s>>>(p);
        return launch_check("gemm_kernel");
    case GEMM_K256:
        if (res) gemm_k256<true><<<grid, block, 0, s>>>(p);
        else     gemm_k256<false><<<grid, block, 0, s>>>(p);
        return launch_check("gemm_k256");
    case GEMM_GENERAL:
        break;
    }
    if (res) {
        if (pl.k256) gemm_kernel<true, false, true><<<grid, block, 0, s>>>(p);
        else         gemm_kernel<true, false, false><<<grid, block, 0, s>>>(p);
    } else {
        if (pl.k256) gemm_kernel<false, false, true><<<grid, block, 0, s>>>(p);
        else         gemm_kernel<false, false, false><<<grid, block, 0, s>>>(p);
    }
    return launch_check("gemm_kernel");
}

// Rows of a packed batch: the total of cu_offsets, after checking it.
static int32_t packed_rows(const int32_t * cu_offsets, int32_t n_seqs, int32_t & T) {
    if (!cu_offsets || n_seqs <= 0) return fail(NXG_EINVAL, "linear: need cu_offsets and n_seqs >= 1");
    if (cu_offsets[0] != 0) return fail(NXG_EINVAL, "linear: cu_offsets[0] = %d, expected 0", cu_offsets[0]);
    for (int i = 0; i < n_seqs; ++i) {
        if (cu_offsets[i + 1] <= cu_offsets[i]) {
            return fail(NXG_EINVAL, "linear: empty or negative sequence %d (cu_offsets %d -> %d)", i,
                        cu_offsets[i], cu_offsets[i + 1]);
        }
    }
    T = cu_offsets[n_seqs];
    return NXG_OK;
}

int32_t nxg_linear_i8_rows(const nxg_weight * W, const int8_t * q, const float * sx, int32_t T,
                           const float * residual, float * out, void * stream) {
    gemm_out o;
    o.residual = residual;
    o.out = out;
    return launch_gemm(W, q, sx, T, o, stream);
}

int32_t nxg_linear_i8_rows_split(const nxg_weight * W, const int8_t * q, const float * sx, int32_t T,
                                 int32_t n_seg, const int32_t * cols, float * const * outs, void * stream) {
    gemm_out o;
    if (n_seg < 1) return fail(NXG_EINVAL, "linear_split: n_seg=%d", n_seg);
    o.n_seg = n_seg;
    o.seg_cols = cols;
    o.seg_out = outs;
    return launch_gemm(W, q, sx, T, o, stream);
}

int32_t nxg_linear_i8(const nxg_weight * W, const int8_t * q, const float * sx,
                      const int32_t * cu_offsets, int32_t n_seqs,
                      const float * residual, float * out, void * stream) {
    int32_t T = 0;
    const int32_t rc = packed_rows(cu_offsets, n_seqs, T);
    return rc ? rc : nxg_linear_i8_rows(W, q, sx, T, residual, out, stream);
}

int32_t nxg_linear_i8_relu2_q8_rows(const nxg_weight * W, const int8_t * q, const float * sx, int32_t T,
                                    int32_t act_max, int8_t * q_out, float * sx_out, void * stream) {
    gemm_out o;
    o.qo = q_out;
    o.sxo = sx_out;
    o.act_max = act_max;
    if (!q_out || !sx_out) return fail(NXG_EINVAL, "linear_relu2_q8: null output");
    return launch_gemm(W, q, sx, T, o, stream);
}

int32_t nxg_linear_f32_relu2_q8_rows(const nxg_weight * W, const float * x, int32_t T, int32_t act_max,
                                     int8_t * q_ws, float * sx_ws, int8_t * q_out, float * sx_out, void * stream) {
    if (!W) return fail(NXG_EINVAL, "linear_f32_relu2_q8: null weight");
    if (T < 0) return fail(NXG_EINVAL, "linear_f32_relu2_q8: T=%d", T);
    if (T == 0) return NXG_OK;
    if (!x || !q_out || !sx_out || !q_ws || !sx_ws) return fail(NXG_EINVAL, "linear_f32_relu2_q8: null buffer");
    if (W->n_in % 256 != 0 || W->n_out % 32 != 0) {
        return fail(NXG_EINVAL, "linear_f32_relu2_q8: needs n_in %% 256 == 0 and n_out %% 32 == 0 (n_in=%d n_out=%d)",
                    W->n_in, W->n_out);
    }
    if (act_max != 127 && act_max != 63) return fail(NXG_EINVAL, "linear_f32_relu2_q8: act_max must be 127 or 63, got %d", act_max);
    int rc = check_device();
    if (rc) return rc;
    gemm_plan pl;
    if (!plan_gemm(T, W->n_in, W->n_out, false, true, device_cus(), pl)) return fail(NXG_EINVAL, "linear: T=%d too large", T);
    if (relu2_fuses_quant(pl)) {
        gemm_out o;
        o.qo = q_out;
        o.sxo = sx_out;
        o.act_max = act_max;
        o.xf = x;
        return launch_gemm(W, nullptr, nullptr, T, o, stream);
    }
    // quantize_row into the workspace, then the GEMM: shapes without the row-tile kernel,
    // or too few row tiles per workgroup to hide reading the fp32 rows
    rc = nxg_quantize_rows(x, T, W->n_in, act_max, q_ws, sx_ws, stream);
    return rc ? rc : nxg_linear_i8_relu2_q8_rows(W, q_ws, sx_ws, T, act_max, q_out, sx_out, stream);
}

int32_t nxg_linear_f32_relu2_q8(const nxg_weight * W, const float * x, const int32_t * cu_offsets, int32_t n_seqs,
                                int32_t act_max, int8_t * q_ws, float * sx_ws, int8_t * q_out, float * sx_out,
                                void * stream) {
    int32_t T = 0;
    const int32_t rc = packed_rows(cu_offsets, n_seqs, T);
    return rc ? rc : nxg_linear_f32_relu2_q8_rows(W, x, T, act_max, q_ws, sx_ws, q_out, sx_out, stream);
}

int32_t nxg_linear_i8_relu2_q8(const nxg_weight * W, const int8_t * q, const float * sx,
                               const int32_t * cu_offsets, int32_t n_seqs, int32_t act_max,
                               int8_t * q_out, float * sx_out, void * stream) {
    int32_t T = 0;
    const int32_t rc = packed_rows(cu_offsets, n_seqs, T);
    return rc ? rc : nxg_linear_i8_relu2_q8_rows(W, q, sx, T, act_max, q_out, sx_out, stream);
}

const char * nxg_gemm_kernel_name(int32_t T, int32_t n_in, int32_t n_out, int32_t flags, int32_t cus) {
    const bool res = flags & NXG_GEMM_RESIDUAL, relu2 = flags & NXG_GEMM_RELU2, sums = flags & NXG_GEMM_SUMS;
    const bool f32_in = flags & NXG_GEMM_F32_IN;
    if (T <= 0 || n_in <= 0 || n_in % 32 != 0 || n_out <= 0 || (relu2 && (res || sums)) || (res && sums)) return nullptr;
    if (f32_in && !relu2) return nullptr;
    if (relu2 && (n_in % 256 != 0 || n_out % 32 != 0)) return nullptr;
    if (cus <= 0) {
        if (check_device() != NXG_OK) return nullptr;
        cus = device_cus();
    }
    gemm_plan pl;
    if (!plan_gemm(T, n_in, n_out, sums, relu2, cus, pl)) return nullptr;
    const bool a63 = flags & NXG_GEMM_ACT63;
    switch (pl.kind) {
    case GEMM_RELU2_SMALL: return a63 ? "gemm_relu2_small<63>" : "gemm_relu2_small<127>";
    case GEMM_RELU2_Q8:    return a63 ? "gemm_relu2_q8<63>" : "gemm_relu2_q8<127>";
    case GEMM_RELU2_RT: {
        static const char * const names[2][2][2] = {       // [f32 input][n_blk == 4][act_max 63]
            { { "gemm_relu2_rt<127, 1, false>", "gemm_relu2_rt<63, 1, false>" },
              { "gemm_relu2_rt<127, 4, false>", "gemm_relu2_rt<63, 4, false>" } },
            { { "gemm_relu2_rt<127, 1, true>", "gemm_relu2_rt<63, 1, true>" },
              { "gemm_relu2_rt<127, 4, true>", "gemm_relu2_rt<63, 4, true>" } } };
        return names[f32_in && relu2_fuses_quant(pl)][pl.n_blk != 1][a63];
    }
    case GEMM_SMALL: {
        static const char * const names[2][2][2] = {
            { { "gemm_small<2, false, false>", "gemm_small<2, false, true>" },
              { "gemm_small<2, true, false>", "gemm_small<2, true, true>" } },
            { { "gemm_small<4, false, false>", "gemm_small<4, false, true>" },
              { "gemm_small<4, true, false>", "gemm_small<4, true, true>" } } };
        return names[pl.fn == 4][res][pl.k256];
    }
    case GEMM_FSK:
        if (pl.fn == 64) return res ? "gemm_fsk<64, 4, true>" : "gemm_fsk<64, 4, false>";
        return res ? "gemm_fsk<32, 9, true>" : "gemm_fsk<32, 9, false>";
    case GEMM_SUMS:  return pl.k256 ? "gemm_kernel<false, true, true>" : "gemm_kernel<false, true, false>";
    case GEMM_K256:  return res ? "gemm_k256<true>" : "gemm_k256<false>";
    case GEMM_GENERAL: break;
    }
    if (res) return pl.k256 ? "gemm_kernel<true, false, true>" : "gemm_kernel<true, false, false>";
    return pl.k256 ? "gemm_kernel<false, false, true>" : "gemm_kernel<false, false, false>";
}

int32_t nxg_linear_i8_block_sums(const nxg_weight * W, const int8_t * q, int32_t T, int32_t * sums, void * stream) {
    if (!sums) return fail(NXG_EINVAL, "block_sums: null output");
    gemm_out o;
    o.sums = sums;
    return launch_gemm(W, q, nullptr, T, o, stream);
}

} // extern "C"
