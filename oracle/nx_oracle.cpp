// nx_oracle.cpp -- CPU oracle for NexteraBERT.cpp's int8 linear-layer path.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP engine is
// compared against: only the test suite, the smoke check and the CPU-baseline
// leg of the benchmark load it. Nothing in the product library links to it.
//
// It restates, from the reference source, the three steps of the path:
//
//   quantize   per (token, 256-input block): amax -> u8 = sat(RNE(x * ACT_MAX/amax) + ACT_OFF),
//              scale amax / ACT_MAX, scales laid out [token/4][block][token%4]
//              (src/nexterabert.cpp:368-403)
//   expand     per (weight row, 256-input block): s8 = lround(w * 127/amax), scale amax/127,
//              off = -ACT_OFF * sum(s8)                     (src/nexterabert.cpp:1009-1049)
//   linear     y[t,r] = res[t,r] + f,  f = fma((float) s_B * sx[t,B], sw[B,r], f) over B ascending,
//              s_B = sum_i w8[r,i] * u8[t,i] + off[B,r]     (src/nexterabert.cpp:854-1007)
//
// Two versions of each step are given:
//   * scalar: plain C++ that states each instruction's semantics explicitly
//     (MAXPS operand order, CVTPS2DQ's integer-indefinite result, the saturating
//     packs). This is the statement the tests pin with closed forms.
//   * simd:   the same arithmetic on the x86 instructions the reference uses
//     (AVX2 max/cvt/pack for the quantizer, 256-bit VPDPBUSD for the GEMM), built
//     with function-level target attributes and dispatched at run time. It is the
//     CPU baseline timed beside the GPU and a cross-check of the scalar statement.
//
// ACT_MAX is 127 on VNNI builds of the reference and 63 on AVX2-only builds
// (src/nexterabert.cpp:53-70); every function takes it as an argument.
//
// The producers that hand rows to quantize_row are restated too (their AVX2 paths, the
// ones every row of 32k inputs takes): relu^2 (in oracle.py), op_rms_norm with dot_f32's
// accumulation order, exp256 / op_gate (with an AVX2 + FMA version of exp256 to check the
// scalar statement against), op_dwconv, op_lily_state and op_block_mean.

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include <immintrin.h>

namespace {

const int BLK = 256;   // I8_BLOCK, src/nexterabert.cpp:254

inline int n_blocks(int n_in) { return (n_in + BLK - 1) / BLK; }

// Position of the scale of (token t, block B): [t/4][B][t%4], src/nexterabert.cpp:372,392.
inline size_t sx_index(int t, int B, int n_blk) {
    return ((size_t) (t / 4) * n_blk + B) * 4 + (t % 4);
}

// MAXPS / MAXSS: dst = (a > b) ? a : b. Any NaN operand selects b.
inline float maxps1(float a, float b) { return a > b ? a : b; }

// ANDNOT with the sign mask: clears bit 31, NaN payloads untouched.
inline float absbits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u &= 0x7fffffffu;
    std::memcpy(&x, &u, 4);
    return x;
}

// CVTPS2DQ under the default MXCSR (round to nearest even). NaN and values
// outside int32 give the integer-indefinite value 0x80000000.
inline int32_t cvtps_epi32(float y) {
    if (std::isnan(y) || y >= 2147483648.0f || y < -2147483648.0f) return INT32_MIN;
    return (int32_t) std::nearbyint(y);
}

inline int32_t sat_i16(int32_t v) { return v < -32768 ? -32768 : v > 32767 ? 32767 : v; }
inline uint8_t sat_u8(int32_t v) { return (uint8_t) (v < 0 ? 0 : v > 255 ? 255 : v); }

// amax of one block with the reference's reduction tree: an 8-lane MAXPS fold
// (lane j sees elements j, j+8, ...), then lanes (j, j+4), then (0,2) and
// (1,3), then (0,1). Elements [i0, i1) of xr; i1 - i0 is a multiple of 8.
float block_amax_scalar(const float * xr, int i0, int i1) {
    float v[8] = { 0, 0, 0, 0, 0, 0, 0, 0 };
    for (int i = i0; i < i1; i += 8) {
        for (int j = 0; j < 8; ++j) v[j] = maxps1(v[j], absbits(xr[i + j]));
    }
    float m[4];
    for (int j = 0; j < 4; ++j) m[j] = maxps1(v[j], v[j + 4]);
    const float m0 = maxps1(m[0], m[2]);
    const float m1 = maxps1(m[1], m[3]);
    return maxps1(m0, m1);
}

} // namespace

extern "C" {

int orc_n_blocks(int n_in) { return n_blocks(n_in); }

// Bytes of a quantized activation buffer, src/nexterabert.cpp:372-375.
size_t orc_qact_bytes(int T, int n_in) {
    return (size_t) T * n_in + (size_t) ((T + 3) / 4) * n_blocks(n_in) * 4 * sizeof(float);
}

// quantize_row over T rows, scalar statement. q: T*n_in u8; sx: ((T+3)/4)*n_blk*4 floats.
// src/nexterabert.cpp:378-403 (and op_copy, :453-461, which applies it to every row).
void orc_quantize_rows_scalar(const float * x, int T, int n_in, int act_max, uint8_t * q, float * sx) {
    const int n_blk = n_blocks(n_in);
    const int act_off = act_max + 1;
    for (int t = 0; t < T; ++t) {
        const float * xr = x + (size_t) t * n_in;
        uint8_t * qr = q + (size_t) t * n_in;
        for (int B = 0; B < n_blk; ++B) {
            const int i0 = B * BLK, i1 = std::min(n_in, i0 + BLK);
            const float amax = block_amax_scalar(xr, i0, i1);
            sx[sx_index(t, B, n_blk)] = amax / (float) act_max;
            const float inv = amax > 0.0f ? (float) act_max / amax : 0.0f;
            for (int i = i0; i < i1; ++i) {
                const float y = xr[i] * inv;
                // 32-bit wrap-around add, then the two saturating packs.
                const int32_t c = (int32_t) ((uint32_t) cvtps_epi32(y) + (uint32_t) act_off);
                qr[i] = sat_u8(sat_i16(c));
            }
        }
    }
}

// The same, on AVX2 instructions: MAXPS fold and horizontal tree, CVTPS2DQ,
// PACKSSDW, PACKUSWB. Returns -1 if the CPU has no AVX2.
__attribute__((target("avx2,fma")))
static void quantize_rows_avx2(const float * x, int T, int n_in, int act_max, uint8_t * q, float * sx) {
    const int n_blk = n_blocks(n_in);
    const __m256 sign = _mm256_set1_ps(-0.0f);
    const __m256i off = _mm256_set1_epi32(act_max + 1);
    for (int t = 0; t < T; ++t) {
        const float * xr = x + (size_t) t * n_in;
        uint8_t * qr = q + (size_t) t * n_in;
        for (int B = 0; B < n_blk; ++B) {
            const int i0 = B * BLK, i1 = std::min(n_in, i0 + BLK);
            __m256 acc = _mm256_setzero_ps();
            for (int i = i0; i < i1; i += 8) {
                acc = _mm256_max_ps(acc, _mm256_andnot_ps(sign, _mm256_loadu_ps(xr + i)));
            }
            __m128 h = _mm_max_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
            h = _mm_max_ps(h, _mm_movehl_ps(h, h));
            h = _mm_max_ss(h, _mm_movehdup_ps(h));
            const float amax = _mm_cvtss_f32(h);
            sx[sx_index(t, B, n_blk)] = amax / (float) act_max;
            const __m256 inv = _mm256_set1_ps(amax > 0.0f ? (float) act_max / amax : 0.0f);
            for (int i = i0; i < i1; i += 8) {
                const __m256i c = _mm256_add_epi32(_mm256_cvtps_epi32(_mm256_mul_ps(_mm256_loadu_ps(xr + i), inv)), off);
                // i32 -> i16 (signed saturation) -> u8 (unsigned saturation); the
                // low 128-bit half of each pack holds the 8 values in order after
                // the lane-crossing extract.
                const __m128i w16 = _mm_packs_epi32(_mm256_castsi256_si128(c), _mm256_extracti128_si256(c, 1));
                const __m128i b8 = _mm_packus_epi16(w16, w16);
                _mm_storel_epi64((__m128i *) (qr + i), b8);
            }
        }
    }
}

int orc_quantize_rows_simd(const float * x, int T, int n_in, int act_max, uint8_t * q, float * sx) {
    if (!__builtin_cpu_supports("avx2")) return -1;
    quantize_rows_avx2(x, T, n_in, act_max, q, sx);
    return 0;
}

// The same over n_threads threads, rows in groups of 16 (a multiple of 4) so that threads write
// disjoint scale groups (the reference quantizes rows inside its multi-threaded
// row ops, src/nexterabert.cpp:414-439).
int orc_quantize_rows_simd_mt(const float * x, int T, int n_in, int act_max, uint8_t * q, float * sx, int n_threads) {
    if (!__builtin_cpu_supports("avx2")) return -1;
    const int n_blk = n_blocks(n_in);
    std::atomic<int> next(0);
    auto work = [&]() {
        for (;;) {
            const int t0 = next.fetch_add(16);
            if (t0 >= T) break;
            const int n = std::min(16, T - t0);
            quantize_rows_avx2(x + (size_t) t0 * n_in, n, n_in, act_max, q + (size_t) t0 * n_in,
                               sx + (size_t) (t0 / 4) * n_blk * 4);
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < n_threads; ++i) pool.emplace_back(work);
    work();
    for (std::thread & th : pool) th.join();
    return 0;
}

// dot_f32 (src/nexterabert.cpp:133-149) in the AVX2 build's order: four 8-lane FMA
// accumulators s0..s3 over 32-element chunks (s_k lane j takes element 32m + 8k + j), the
// 8-element remaining chunks into s0, then hsum256 (src/nexterabert.cpp:124-129) of
// (s0 + s1) + (s2 + s3): lanes j and j+4, then 0+2 and 1+3, then those two. n % 8 == 0
// (the scalar tail after the vector part is not used: every qact row has n % 32 == 0).
static float dot_avx2_order(const float * a, const float * b, int n) {
    float s[4][8] = {};
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        for (int k = 0; k < 4; ++k) {
            for (int j = 0; j < 8; ++j) s[k][j] = std::fma(a[i + 8 * k + j], b[i + 8 * k + j], s[k][j]);
        }
    }
    for (; i + 8 <= n; i += 8) {
        for (int j = 0; j < 8; ++j) s[0][j] = std::fma(a[i + j], b[i + j], s[0][j]);
    }
    float v[8];
    for (int j = 0; j < 8; ++j) v[j] = (s[0][j] + s[1][j]) + (s[2][j] + s[3][j]);
    float h[4];
    for (int j = 0; j < 4; ++j) h[j] = v[j] + v[j + 4];
    const float h0 = h[0] + h[2], h1 = h[1] + h[3];
    return h0 + h1;
}


// src/nexterabert.cpp:1030-1042. scale/off are [n_blk][n_out].
void orc_expand_rows(const float * rows, int n_in, int n_out, int act_off,
                     int8_t * w, float * scale, int32_t * off) {
    const int n_blk = n_blocks(n_in);
    for (int r = 0; r < n_out; ++r) {
        const float * row = rows + (size_t) r * n_in;
        int8_t * qr = w + (size_t) r * n_in;
        for (int B = 0; B < n_blk; ++B) {
            const int i0 = B * BLK, i1 = std::min(n_in, i0 + BLK);
            float amax = 0.0f;
            for (int i = i0; i < i1; ++i) amax = std::max(amax, std::fabs(row[i]));
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            int32_t sum = 0;
            for (int i = i0; i < i1; ++i) {
                qr[i] = (int8_t) std::lround(row[i] * inv);   // ties away from zero
                sum += qr[i];
            }
            scale[(size_t) B * n_out + r] = amax / 127.0f;
            off[(size_t) B * n_out + r] = -act_off * sum;
        }
    }
}

// GGUF Q8_0 rows (34-byte blocks: fp16 d, 32 x s8) to f32. d * q is exact in fp32.
static float fp16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    float v;
    if (e == 0) {
        v = std::ldexp((float) m, -24);
    } else if (e == 31) {
        v = m ? NAN : INFINITY;
    } else {
        v = std::ldexp((float) (m | 0x400), (int) e - 25);
    }
    uint32_t u;
    std::memcpy(&u, &v, 4);
    u |= sign;
    std::memcpy(&v, &u, 4);
    return v;
}

// op_rms_norm's row (src/nexterabert.cpp:463-482): inv = 1 / sqrt(dot(x, x) / C + eps),
// out = (x * inv) * gain, with dot in the AVX2 order above. C % 8 == 0.
void orc_rms_norm_rows(const float * x, const float * gain, float eps, int T, int C, float * out) {
    for (int t = 0; t < T; ++t) {
        const float * xr = x + (size_t) t * C;
        float * o = out + (size_t) t * C;
        const float inv = 1.0f / std::sqrt(dot_avx2_order(xr, xr, C) / (float) C + eps);
        for (int i = 0; i < C; ++i) o[i] = (xr[i] * inv) * gain[i];
    }
}

// exp256 (src/nexterabert.cpp:81-100) for one lane: clamp with MINPS/MAXPS semantics
// (the second operand when either is NaN, so a NaN becomes the upper bound), n = x * log2 e
// rounded to an integer with ties to even (ROUNDPS, nearest), r = x - n c1 - n c2 as two
// fused steps (FNMADD), the degree-5 polynomial by fused Horner steps, p r^2 + (r + 1)
// fused, times 2^n assembled in the exponent field (CVTPS2DQ, + 127, << 23).
static const float EXP_P[6] = { 1.9875691500e-4f, 1.3981999507e-3f, 8.3334519073e-3f,
                                4.1665795894e-2f, 1.6666665459e-1f, 5.0000001201e-1f };

float orc_exp_cephes(float x) {
    x = x < 88.3762626647949f ? x : 88.3762626647949f;
    x = x > -87.3f ? x : -87.3f;
    const float n = std::nearbyint(x * 1.44269504088896341f);
    float r = std::fma(-n, 0.693359375f, x);
    r = std::fma(-n, -2.12194440e-4f, r);
    const float r2 = r * r;
    float p = EXP_P[0];
    for (int i = 1; i < 6; ++i) p = std::fma(p, r, EXP_P[i]);
    p = std::fma(p, r2, r + 1.0f);
    const uint32_t bits = (uint32_t) ((int32_t) n + 127) << 23;
    float scale;
    std::memcpy(&scale, &bits, 4);
    return p * scale;
}

void orc_exp_cephes_rows(const float * x, int64_t n, float * out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_exp_cephes(x[i]);
}

// op_gate's row (src/nexterabert.cpp:507-522, AVX2 path): sigmoid(g) * y with
// sigmoid256 (:119-122) = 1 / (1 + exp256(0 - g)).
void orc_gate_rows(const float * g, const float * y, int T, int C, float * out) {
    for (size_t i = 0; i < (size_t) T * C; ++i) out[i] = (1.0f / (1.0f + orc_exp_cephes(0.0f - g[i]))) * y[i];
}

// op_dwconv (src/nexterabert.cpp:524-543) over a packed batch: out = r (or 0), then
// out = fma(taps[j], x[t + j - k/2], out) for j ascending, skipping rows outside t's
// document. taps [k][C], cu: n_seqs + 1 offsets.
void orc_dwconv_rows(const float * x, const float * r, const float * taps, int k, const int32_t * cu, int n_seqs,
                     int C, float * out) {
    for (int d = 0; d < n_seqs; ++d) {
        const int lo = cu[d], hi = cu[d + 1];
        for (int t = lo; t < hi; ++t) {
            float * o = out + (size_t) t * C;
            for (int i = 0; i < C; ++i) o[i] = r ? r[(size_t) t * C + i] : 0.0f;
            for (int j = 0; j < k; ++j) {
                const int tt = t + j - k / 2;
                if (tt < lo || tt >= hi) continue;
                for (int i = 0; i < C; ++i) o[i] = std::fma(taps[(size_t) j * C + i], x[(size_t) tt * C + i], o[i]);
            }
        }
    }
}

// op_lily_state (src/nexterabert.cpp:545-578, AVX2 path): acc = 0, acc = fma(taps[j],
// a[tt] * x[tt], acc) for the taps j whose row tt = t + j - k/2 is in t's document,
// out = acc * b[t].
void orc_lily_state_rows(const float * a, const float * x, const float * b, const float * taps, int k,
                         const int32_t * cu, int n_seqs, int C, float * out) {
    for (int d = 0; d < n_seqs; ++d) {
        const int lo = cu[d], hi = cu[d + 1];
        for (int t = lo; t < hi; ++t) {
            const int j0 = std::max(0, lo - (t - k / 2)), j1 = std::min(k, hi - (t - k / 2));
            for (int i = 0; i < C; ++i) {
                float acc = 0.0f;
                for (int j = j0; j < j1; ++j) {
                    const size_t o = (size_t) (t + j - k / 2) * C + i;
                    acc = std::fma(taps[(size_t) j * C + i], a[o] * x[o], acc);
                }
                out[(size_t) t * C + i] = acc * b[(size_t) t * C + i];
            }
        }
    }
}

// op_block_mean (src/nexterabert.cpp:638-659): per document, runs of `block` tokens
// (the last one shorter), out = 0, out = fma(h, g, out) per token (out + h without g),
// then out * (1 / n). Output rows: ceil(len / block) per document, in order.
void orc_block_mean_rows(const float * h, const float * g, const int32_t * cu, int n_seqs, int block, int C,
                         float * out) {
    size_t row = 0;
    for (int d = 0; d < n_seqs; ++d) {
        const int lo = cu[d], len = cu[d + 1] - cu[d];
        for (int bi = 0; bi * block < len; ++bi, ++row) {
            const int ts = lo + bi * block, n = std::min(block, len - bi * block);
            float * o = out + row * C;
            for (int i = 0; i < C; ++i) o[i] = 0.0f;
            for (int u = 0; u < n; ++u) {
                const float * hr = h + (size_t) (ts + u) * C;
                if (g) {
                    const float * gr = g + (size_t) (ts + u) * C;
                    for (int i = 0; i < C; ++i) o[i] = std::fma(hr[i], gr[i], o[i]);
                } else {
                    for (int i = 0; i < C; ++i) o[i] = o[i] + hr[i];
                }
            }
            const float inv = 1.0f / (float) n;
            for (int i = 0; i < C; ++i) o[i] *= inv;
        }
    }
}

void orc_dequant_q8_0(const uint8_t * data, int64_t n, float * out) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t * blk = data + b * 34;
        const float d = fp16_to_f32((uint16_t) (blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float) (int8_t) blk[2 + i];
    }
}

// Per-block integer sums s_B = sum_i w8[r,i] * u8[t,i] + off[B,r], as int32
// [n_blk][T][n_out] (the quantity the VPDPBUSD loop and the offset produce,
// src/nexterabert.cpp:892-916).
void orc_block_sums(const int8_t * w, const int32_t * off, int n_in, int n_out,
                    const uint8_t * q, int T, int32_t * sums) {
    const int n_blk = n_blocks(n_in);
    for (int B = 0; B < n_blk; ++B) {
        const int i0 = B * BLK, i1 = std::min(n_in, i0 + BLK);
        for (int t = 0; t < T; ++t) {
            const uint8_t * qt = q + (size_t) t * n_in;
            for (int r = 0; r < n_out; ++r) {
                const int8_t * wr = w + (size_t) r * n_in;
                int32_t s = 0;
                for (int i = i0; i < i1; ++i) s += (int32_t) wr[i] * (int32_t) qt[i];
                sums[((size_t) B * T + t) * n_out + r] = s + off[(size_t) B * n_out + r];
            }
        }
    }
}

// op_linear_i8, scalar statement: out[t*n_out + r]. res may be NULL.
void orc_linear_scalar(const int8_t * w, const float * scale, const int32_t * off, int n_in, int n_out,
                       const uint8_t * q, const float * sx, int T, const float * res, float * out) {
    const int n_blk = n_blocks(n_in);
    for (int t = 0; t < T; ++t) {
        const uint8_t * qt = q + (size_t) t * n_in;
        for (int r = 0; r < n_out; ++r) {
            const int8_t * wr = w + (size_t) r * n_in;
            float f = 0.0f;
            for (int B = 0; B < n_blk; ++B) {
                const int i0 = B * BLK, i1 = std::min(n_in, i0 + BLK);
                int32_t s = 0;
                for (int i = i0; i < i1; ++i) s += (int32_t) wr[i] * (int32_t) qt[i];
                s += off[(size_t) B * n_out + r];
                const float p = (float) s * sx[sx_index(t, B, n_blk)];
                f = std::fma(p, scale[(size_t) B * n_out + r], f);
            }
            out[(size_t) t * n_out + r] = res ? res[(size_t) t * n_out + r] + f : f;
        }
    }
}

} // extern "C"

// ---------------------------------------------------------------------------
// VPDPBUSD GEMM (the CPU baseline). A tile of NR weight rows x NT tokens keeps
// NR*NT 8-lane int32 accumulators; per 32 inputs it does NR*NT VPDPBUSD. The
// per-(token, row) arithmetic is the scalar statement's, so any tile shape
// gives the same bits.
// ---------------------------------------------------------------------------

namespace {

struct gemm_args {
    const int8_t * w; const float * scale; const int32_t * off;
    int n_in, n_out, n_blk;
    const uint8_t * q; const float * sx; int T;
    const float * res; float * out;
};

#define ORC_VNNI_TILE(TARGET, DPBUSD, NAME)                                                        \
template <int NR, int NT>                                                                          \
__attribute__((target(TARGET))) inline void NAME(const gemm_args & a, int r, int t) {              \
    float f[NR][NT];                                                                               \
    for (int i = 0; i < NR; ++i) for (int j = 0; j < NT; ++j) f[i][j] = 0.0f;                      \
    for (int B = 0; B < a.n_blk; ++B) {                                                            \
        const int i0 = B * BLK, i1 = std::min(a.n_in, i0 + BLK);                                   \
        __m256i acc[NR][NT];                                                                       \
        for (int i = 0; i < NR; ++i) for (int j = 0; j < NT; ++j) acc[i][j] = _mm256_setzero_si256(); \
        for (int k = i0; k < i1; k += 32) {                                                        \
            __m256i xv[NT];                                                                        \
            for (int j = 0; j < NT; ++j)                                                           \
                xv[j] = _mm256_loadu_si256((const __m256i *) (a.q + (size_t) (t + j) * a.n_in + k)); \
            for (int i = 0; i < NR; ++i) {                                                         \
                const __m256i wv = _mm256_loadu_si256((const __m256i *) (a.w + (size_t) (r + i) * a.n_in + k)); \
                for (int j = 0; j < NT; ++j) acc[i][j] = DPBUSD(acc[i][j], xv[j], wv);             \
            }                                                                                      \
        }                                                                                          \
        for (int i = 0; i < NR; ++i) {                                                             \
            const float sw = a.scale[(size_t) B * a.n_out + r + i];                                \
            const int32_t of = a.off[(size_t) B * a.n_out + r + i];                                \
            for (int j = 0; j < NT; ++j) {                                                         \
                __m128i h = _mm_add_epi32(_mm256_castsi256_si128(acc[i][j]),                       \
                                          _mm256_extracti128_si256(acc[i][j], 1));                 \
                h = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0x4e));                                  \
                h = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0xb1));                                  \
                const int32_t s = _mm_cvtsi128_si32(h) + of;                                       \
                const float p = (float) s * a.sx[sx_index(t + j, B, a.n_blk)];                     \
                f[i][j] = std::fma(p, sw, f[i][j]);                                                \
            }                                                                                      \
        }                                                                                          \
    }                                                                                              \
    for (int j = 0; j < NT; ++j) {                                                                 \
        float * o = a.out + (size_t) (t + j) * a.n_out + r;                                        \
        const float * rr = a.res ? a.res + (size_t) (t + j) * a.n_out + r : nullptr;               \
        for (int i = 0; i < NR; ++i) o[i] = rr ? rr[i] + f[i][j] : f[i][j];                        \
    }                                                                                              \
}

#define ORC_DPBUSD_AVXVNNI(acc, x, w) _mm256_dpbusd_avx_epi32(acc, x, w)
#define ORC_DPBUSD_AVX512VNNI(acc, x, w) _mm256_dpbusd_epi32(acc, x, w)
ORC_VNNI_TILE("avx2,fma,avxvnni", ORC_DPBUSD_AVXVNNI, tile_avxvnni)
ORC_VNNI_TILE("avx2,fma,avx512f,avx512vl,avx512vnni", ORC_DPBUSD_AVX512VNNI, tile_avx512vnni)

// One work item: tokens [t0, t1) x rows [r0, r1). Main tiles are 3 rows x 4
// tokens; edges fall back to 1 x 4, 3 x 1 and 1 x 1 tiles.
template <void (*T34)(const gemm_args &, int, int), void (*T14)(const gemm_args &, int, int),
          void (*T31)(const gemm_args &, int, int), void (*T11)(const gemm_args &, int, int)>
void run_item(const gemm_args & a, int t0, int t1, int r0, int r1) {
    const int tq = t0 + ((t1 - t0) & ~3), rq = r0 + (r1 - r0) / 3 * 3;
    for (int t = t0; t < tq; t += 4) {
        int r = r0;
        for (; r < rq; r += 3) T34(a, r, t);
        for (; r < r1; ++r) T14(a, r, t);
    }
    for (int t = tq; t < t1; ++t) {
        int r = r0;
        for (; r < rq; r += 3) T31(a, r, t);
        for (; r < r1; ++r) T11(a, r, t);
    }
}

template <void (*ITEM)(const gemm_args &, int, int, int, int)>
void run_threads(const gemm_args & a, int n_threads) {
    // (token block x row chunk) items from a shared cursor, so that threads
    // that finish early take more work.
    const int tok_blk = std::max(4, std::min(64, (32 * 1024 / a.n_in) & ~3));
    const int row_chk = 24;
    const int n_tb = (a.T + tok_blk - 1) / tok_blk, n_rc = (a.n_out + row_chk - 1) / row_chk;
    std::atomic<int> next(0);
    auto work = [&]() {
        for (;;) {
            const int it = next.fetch_add(1, std::memory_order_relaxed);
            if (it >= n_tb * n_rc) break;
            const int t0 = (it / n_rc) * tok_blk, r0 = (it % n_rc) * row_chk;
            ITEM(a, t0, std::min(a.T, t0 + tok_blk), r0, std::min(a.n_out, r0 + row_chk));
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < n_threads; ++i) pool.emplace_back(work);
    work();
    for (std::thread & th : pool) th.join();
}

void item_avxvnni(const gemm_args & a, int t0, int t1, int r0, int r1) {
    run_item<tile_avxvnni<3, 4>, tile_avxvnni<1, 4>, tile_avxvnni<3, 1>, tile_avxvnni<1, 1>>(a, t0, t1, r0, r1);
}
void item_avx512vnni(const gemm_args & a, int t0, int t1, int r0, int r1) {
    run_item<tile_avx512vnni<3, 4>, tile_avx512vnni<1, 4>, tile_avx512vnni<3, 1>, tile_avx512vnni<1, 1>>(a, t0, t1, r0, r1);
}

int vnni_kind() {
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl")) return 2;
    if (__builtin_cpu_supports("avxvnni")) return 1;
    return 0;
}

} // namespace

extern "C" {

// "AVX512-VNNI", "AVX-VNNI" or "" (no VNNI on this CPU).
const char * orc_vnni_flavour(void) {
    switch (vnni_kind()) {
        case 2: return "AVX512-VNNI";
        case 1: return "AVX-VNNI";
        default: return "";
    }
}

// op_linear_i8 on VPDPBUSD with n_threads threads. n_in must be a multiple of
// 32 (the load-time rule, src/nexterabert.cpp:1667). Returns -1 without VNNI.
int orc_linear_simd(const int8_t * w, const float * scale, const int32_t * off, int n_in, int n_out,
                    const uint8_t * q, const float * sx, int T, const float * res, float * out, int n_threads) {
    if (n_in % 32 != 0) return -2;
    const gemm_args a = { w, scale, off, n_in, n_out, n_blocks(n_in), q, sx, T, res, out };
    switch (vnni_kind()) {
        case 2: run_threads<item_avx512vnni>(a, std::max(1, n_threads)); return 0;
        case 1: run_threads<item_avxvnni>(a, std::max(1, n_threads)); return 0;
        default: return -1;
    }
}

} // extern "C"

namespace {

// exp256 on the instructions the reference uses (AVX2 + FMA), to check the scalar
// statement orc_exp_cephes against the hardware semantics of ROUNDPS, FNMADD, CVTPS2DQ.
__attribute__((target("avx2,fma")))
void exp_cephes_avx2(const float * x, int64_t n, float * out) {
    for (int64_t i = 0; i + 8 <= n; i += 8) {
        __m256 v = _mm256_loadu_ps(x + i);
        v = _mm256_min_ps(v, _mm256_set1_ps(88.3762626647949f));
        v = _mm256_max_ps(v, _mm256_set1_ps(-87.3f));
        const __m256 fn = _mm256_round_ps(_mm256_mul_ps(v, _mm256_set1_ps(1.44269504088896341f)),
                                          _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        v = _mm256_fnmadd_ps(fn, _mm256_set1_ps(0.693359375f), v);
        v = _mm256_fnmadd_ps(fn, _mm256_set1_ps(-2.12194440e-4f), v);
        const __m256 v2 = _mm256_mul_ps(v, v);
        __m256 p = _mm256_set1_ps(EXP_P[0]);
        for (int k = 1; k < 6; ++k) p = _mm256_fmadd_ps(p, v, _mm256_set1_ps(EXP_P[k]));
        p = _mm256_fmadd_ps(p, v2, _mm256_add_ps(v, _mm256_set1_ps(1.0f)));
        const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(fn), _mm256_set1_epi32(127)), 23);
        _mm256_storeu_ps(out + i, _mm256_mul_ps(p, _mm256_castsi256_ps(e)));
    }
}

} // namespace

extern "C" int orc_exp_cephes_simd(const float * x, int64_t n, float * out) {
    if (n % 8 != 0 || !__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma")) return -1;
    exp_cephes_avx2(x, n, out);
    return 0;
}
