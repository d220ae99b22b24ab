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

// op_upsample_add (src/nexterabert.cpp:675-690): row t of document d gets yb[cub[d] + (t -
// cu[d]) / block] + r[t].
void orc_upsample_add(const float * yb, const float * r, const int32_t * cu, const int32_t * cub, int n_seqs,
                      int block, int C, float * out) {
    for (int d = 0; d < n_seqs; ++d) {
        for (int t = cu[d]; t < cu[d + 1]; ++t) {
            const float * y = yb + (size_t) (cub[d] + (t - cu[d]) / block) * C;
            const float * rr = r + (size_t) t * C;
            float * o = out + (size_t) t * C;
            for (int c = 0; c < C; ++c) o[c] = y[c] + rr[c];
        }
    }
}

// ggml_norm (ggml v0.9.9's CPU op, published as: mean = (float) sum / n with the sum in
// double; v = x - mean; variance = (float) (sum of (double) (v * v) / n); y = v * (1 /
// sqrtf(variance + eps))) then ggml_mul by w and ggml_add of b (src/nexterabert.cpp:
// 1290-1291), each rounded on its own. ggml is not in the reference's tree, so the order
// of the double sums is this build's: 64 partial sums, partial l taking elements l + 64 j
// in order of j, then combined pairwise l + (l ^ m) for m = 32, 16, ..., 1.
static double lane_sum64(const double (&p)[64]) {
    double s[64];
    for (int l = 0; l < 64; ++l) s[l] = p[l];
    for (int m = 32; m >= 1; m >>= 1) {
        double n[64];
        for (int l = 0; l < 64; ++l) n[l] = s[l] + s[l ^ m];
        for (int l = 0; l < 64; ++l) s[l] = n[l];
    }
    return s[0];
}

void orc_layer_norm(const float * x, const float * w, const float * b, float eps, int T, int C, float * out) {
    for (int t = 0; t < T; ++t) {
        const float * xr = x + (size_t) t * C;
        double p[64] = {};
        for (int i = 0; i < C; ++i) p[i % 64] += (double) xr[i];
        const float mean = (float) lane_sum64(p) / (float) C;
        double p2[64] = {};
        for (int i = 0; i < C; ++i) {
            const float v = xr[i] - mean;
            p2[i % 64] += (double) (v * v);
        }
        const float variance = (float) (lane_sum64(p2) / (double) C);
        const float scale = 1.0f / std::sqrt(variance + eps);
        float * o = out + (size_t) t * C;
        for (int i = 0; i < C; ++i) {
            float y = (xr[i] - mean) * scale;
            if (w) y = y * w[i];
            if (b) y = y + b[i];
            o[i] = y;
        }
    }
}

// nextera_encode's pooled vectors (src/nexterabert.cpp:1913-1925), op_doc_mean (:659-672):
// per document the sum of its rows in order, then times 1 / n, or (normalize) times 1 /
// sqrt(dot_f32(p, p)), 0 for a zero vector.
void orc_doc_mean(const float * x, const int32_t * cu, int n_seqs, int C, int normalize, float * out) {
    for (int d = 0; d < n_seqs; ++d) {
        float * o = out + (size_t) d * C;
        for (int c = 0; c < C; ++c) o[c] = 0.0f;
        for (int t = cu[d]; t < cu[d + 1]; ++t) {
            const float * xr = x + (size_t) t * C;
            for (int c = 0; c < C; ++c) o[c] = std::fma(1.0f, xr[c], o[c]);
        }
        float scale = 1.0f / (float) (cu[d + 1] - cu[d]);
        if (normalize) {
            const float nrm = std::sqrt(dot_avx2_order(o, o, C));
            scale = nrm > 0.0f ? 1.0f / nrm : 0.0f;
        }
        for (int c = 0; c < C; ++c) o[c] *= scale;
    }
}

// The scale op_attention applies to one document of n keys (src/nexterabert.cpp:1196-1201):
// 1 / sqrt(head_dim) times builder::ssmax_scale (:1172-1181) -- 1 (mode 0: "none", or an
// swa layer), s * ln n (mode 1), s * ln n + ssmax_base + max(b, 0) (mode 2), ln n =
// logf(max(n, 1)). GCC's default contraction (the reference's -O3 -march=native build)
// makes s * ln n + ssmax_base one fma.
float orc_attention_scale(int n, int head_dim, int mode, float s, float b, float ssmax_base) {
    const float base = 1.0f / std::sqrt((float) head_dim);
    if (mode == 0) return base * 1.0f;
    const float ln = std::log((float) std::max(n, 1));
    const float f = mode == 1 ? s * ln : std::fma(s, ln, ssmax_base) + std::max(b, 0.0f);
    return base * f;
}

// build_rope (src/nexterabert.cpp:1322-1338): cos / sin of t * (1 / base^(2i / head_dim)),
// each step a float C library call or operation. out [n_pos][head_dim / 2].
void orc_rope_table(int n_pos, float base, int head_dim, float * cos_out, float * sin_out) {
    const int half = head_dim / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = 1.0f / std::pow(base, (float) (2 * i) / (float) head_dim);
    for (int t = 0; t < n_pos; ++t) {
        for (int i = 0; i < half; ++i) {
            const float a = (float) t * inv[i];
            cos_out[(size_t) t * half + i] = std::cos(a);
            sin_out[(size_t) t * half + i] = std::sin(a);
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

// ---------------------------------------------------------------------------
// op_attention, head_dim 64 (src/nexterabert.cpp:704-852), lane by lane.
// ---------------------------------------------------------------------------

// One key's 8 lane partials of the NEXTERA_DOT64 chain: lane l = q[l] * k[l], then
// fma(q[8c + l], k[8c + l], .) for c = 1..7.
static void dot64_lanes(const float * q, const float * k, float p[8]) {
    for (int l = 0; l < 8; ++l) {
        float a = q[l] * k[l];
        for (int c = 1; c < 8; ++c) a = std::fma(q[8 * c + l], k[8 * c + l], a);
        p[l] = a;
    }
}

// scores_d64 (:704-731): keys in groups of 8 from the first, each total reduced by the
// HADDPS / VPERM2F128 tree ((l0+l1)+(l2+l3)) + ((l4+l5)+(l6+l7)); the remaining keys by
// hsum256 ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)); then * scale.
static void scores_d64_lanes(const float * q, const float * k, int n, float scale, float * sc) {
    float p[8];
    const int n_groups = n & ~7;
    int j = 0;
    for (; j < n_groups; ++j) {
        dot64_lanes(q, k + (size_t) j * 64, p);
        sc[j] = (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]))) * scale;
    }
    for (; j < n; ++j) {
        dot64_lanes(q, k + (size_t) j * 64, p);
        sc[j] = scale * (((p[0] + p[4]) + (p[2] + p[6])) + ((p[1] + p[5]) + (p[3] + p[7])));
    }
}

// softmax_exp (:177-197): m = the running std::max from s[0]; for the whole 8-groups
// e = exp256(s - m) added into 8 lane sums, reduced by hsum256; then the remaining
// elements with the C library's expf, added one by one. Returns the sum.
static float softmax_exp_lanes(float * s, int n) {
    float m = s[0];
    for (int i = 1; i < n; ++i) m = m < s[i] ? s[i] : m;
    float v[8] = { 0, 0, 0, 0, 0, 0, 0, 0 };
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int l = 0; l < 8; ++l) {
            s[i + l] = orc_exp_cephes(s[i + l] - m);
            v[l] = v[l] + s[i + l];
        }
    }
    float sum = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
    for (; i < n; ++i) {
        s[i] = std::exp(s[i] - m);
        sum += s[i];
    }
    return sum;
}

// Grouped-query attention inside each document (optionally the band |i - j| <= half):
// q [T][H*64] row-major, k / v [G][T][64] head-major, out [T][H*64]; scale per document.
// attend (:758-774): scores, inv = 1 / sum, out = fma(w_j * inv, v_j, out) over j in order.
void orc_attention(const float * q, const float * k, const float * v, const int32_t * cu, int n_seqs,
                   const float * scale, int T, int H, int G, int half, float * out) {
    std::vector<float> sc;
    const int rep = H / G;
    for (int d = 0; d < n_seqs; ++d) {
        for (int t = cu[d]; t < cu[d + 1]; ++t) {
            int lo = cu[d], hi = cu[d + 1];
            if (half >= 0) {
                lo = std::max(lo, t - half);
                hi = std::min(hi, t + half + 1);
            }
            const int n = hi - lo;
            sc.resize(n);
            for (int h = 0; h < H; ++h) {
                const size_t go = (size_t) (h / rep) * T * 64;
                const float * kh = k + go + (size_t) lo * 64, * vh = v + go + (size_t) lo * 64;
                scores_d64_lanes(q + (size_t) t * H * 64 + (size_t) h * 64, kh, n, scale[d], sc.data());
                const float inv = 1.0f / softmax_exp_lanes(sc.data(), n);
                float * o = out + (size_t) t * H * 64 + (size_t) h * 64;
                for (int e = 0; e < 64; ++e) o[e] = 0.0f;
                for (int j = 0; j < n; ++j) {
                    const float c = sc[j] * inv;
                    for (int e = 0; e < 64; ++e) o[e] = std::fma(c, vh[(size_t) j * 64 + e], o[e]);
                }
            }
        }
    }
}

// The C library's expf restated (glibc 2.35's FMA path, the published ARM optimized-routines
// method): the statement the GPU computes for softmax_exp's tail, checked here against
// the host's expf.
static const uint64_t EXPF_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull };

float orc_expf_restated(float x) {
    uint32_t ux;
    std::memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double xd = (double) x;
    double kd = std::fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    std::memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = std::fma(inv_ln2_n, xd, -kd);
    const uint64_t t = EXPF_TAB[ki % 32] + (ki << 47);
    double s;
    std::memcpy(&s, &t, 8);
    const double z = std::fma(0x1.c6af84b912394p-5 / 32 / 32 / 32, r, 0x1.ebfce50fac4f3p-3 / 32 / 32);
    const double r2 = r * r;
    double y = std::fma(0x1.62e42ff0c52d6p-1 / 32, r, 1.0);
    y = std::fma(z, r2, y);
    return (float) (y * s);
}

// Floats u = first, first + stride, ... (as bit patterns) where the restatement differs from
// the host's expf (NaN results compared as NaN); returns the count, the first few in bad.
int64_t orc_expf_restated_check(uint32_t first, uint32_t stride, uint64_t count, uint32_t * bad, int n_bad) {
    int64_t n = 0;
    uint64_t u = first;
    for (uint64_t i = 0; i < count && u <= 0xffffffffull; ++i, u += stride) {
        const uint32_t v = (uint32_t) u;
        float x;
        std::memcpy(&x, &v, 4);
        const float a = std::exp(x), b = orc_expf_restated(x);
        uint32_t ua, ub;
        std::memcpy(&ua, &a, 4);
        std::memcpy(&ub, &b, 4);
        if (ua != ub && !(std::isnan(a) && std::isnan(b))) {
            if (n < n_bad) bad[n] = v;
            ++n;
        }
    }
    return n;
}

// tanh256 (src/nexterabert.cpp:103-117) for one lane: big = (1 - t) / (1 + t) with
// t = exp256(|x| * -2) and x's sign bit ORed in; small = (((-17/315 x^2 + 2/15) x^2 - 1/3)
// x^2 + 1) * x by fused steps; small where |x| < 0.1 (an ordered compare: NaN takes big).
float orc_tanh_ref(float x) {
    uint32_t ux;
    std::memcpy(&ux, &x, 4);
    const uint32_t sign = ux & 0x80000000u;
    float ax;
    const uint32_t uax = ux & 0x7fffffffu;
    std::memcpy(&ax, &uax, 4);
    const float t = orc_exp_cephes(ax * -2.0f);
    float big = (1.0f - t) / (1.0f + t);
    uint32_t ub;
    std::memcpy(&ub, &big, 4);
    ub |= sign;
    std::memcpy(&big, &ub, 4);
    const float x2 = x * x;
    float p = -17.0f / 315.0f;
    p = std::fma(p, x2, 2.0f / 15.0f);
    p = std::fma(p, x2, -1.0f / 3.0f);
    p = std::fma(p, x2, 1.0f);
    const float small = p * x;
    return ax < 0.1f ? small : big;
}

// op_qk_prep (src/nexterabert.cpp:590-632): per row t (position pos = t - its document's
// start) and head h, with half = D/2: a = beta[i] * tanh(alpha[i] * x1[i]), b = beta[half+i] *
// tanh(alpha[half+i] * x2[i]); y1 = fma(a, cos, b * sin), y2 = fma(-a, sin, b * cos).
// x [T][H*D]; alpha, beta [D]; cos, sin [n_pos][half]; out [T][H*D] (head_major 0) or
// [H][T][D] (head_major 1).
void orc_qk_prep(const float * x, const float * alpha, const float * beta, const float * cos_t, const float * sin_t,
                 const int32_t * cu, int n_seqs, int T, int H, int D, int head_major, float * out) {
    const int half = D / 2;
    for (int d = 0; d < n_seqs; ++d) {
        for (int t = cu[d]; t < cu[d + 1]; ++t) {
            const int pos = t - cu[d];
            const float * c = cos_t + (size_t) pos * half, * s = sin_t + (size_t) pos * half;
            for (int h = 0; h < H; ++h) {
                const float * x1 = x + (size_t) t * H * D + (size_t) h * D, * x2 = x1 + half;
                float * y1 = head_major ? out + ((size_t) h * T + t) * D : out + (size_t) t * H * D + (size_t) h * D;
                float * y2 = y1 + half;
                for (int i = 0; i < half; ++i) {
                    const float a = beta[i] * orc_tanh_ref(alpha[i] * x1[i]);
                    const float b = beta[half + i] * orc_tanh_ref(alpha[half + i] * x2[i]);
                    y1[i] = std::fma(a, c[i], b * s[i]);
                    y2[i] = std::fma(-a, s[i], b * c[i]);
                }
            }
        }
    }
}

void orc_tanh_rows(const float * x, int64_t n, float * out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_tanh_ref(x[i]);
}

void orc_expf_rows(const float * x, int64_t n, float * out) {
    for (int64_t i = 0; i < n; ++i) out[i] = std::exp(x[i]);
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

namespace {

// scores_d64's reduction of 8 keys on the instructions the reference uses (HADDPS,
// VPERM2F128), to check the scalar statement's summation trees against them.
__attribute__((target("avx2,fma")))
void scores8_avx2(const float * q, const float * k, float scale, float * sc) {
    __m256 qv[8], a[8];
    for (int c = 0; c < 8; ++c) qv[c] = _mm256_loadu_ps(q + 8 * c);
    for (int key = 0; key < 8; ++key) {
        const float * kp = k + (size_t) key * 64;
        __m256 acc = _mm256_mul_ps(qv[0], _mm256_loadu_ps(kp));
        for (int c = 1; c < 8; ++c) acc = _mm256_fmadd_ps(qv[c], _mm256_loadu_ps(kp + 8 * c), acc);
        a[key] = acc;
    }
    const __m256 h0 = _mm256_hadd_ps(_mm256_hadd_ps(a[0], a[1]), _mm256_hadd_ps(a[2], a[3]));
    const __m256 h1 = _mm256_hadd_ps(_mm256_hadd_ps(a[4], a[5]), _mm256_hadd_ps(a[6], a[7]));
    const __m256 t = _mm256_add_ps(_mm256_permute2f128_ps(h0, h1, 0x20), _mm256_permute2f128_ps(h0, h1, 0x31));
    _mm256_storeu_ps(sc, _mm256_mul_ps(t, _mm256_set1_ps(scale)));
}

__attribute__((target("avx2,fma")))
float hsum_key_avx2(const float * q, const float * k, float scale) {
    __m256 acc = _mm256_mul_ps(_mm256_loadu_ps(q), _mm256_loadu_ps(k));
    for (int c = 1; c < 8; ++c) acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + 8 * c), _mm256_loadu_ps(k + 8 * c), acc);
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return scale * _mm_cvtss_f32(s);
}

} // namespace

// The scores of n keys (n % 8 == 0 taken as groups, the rest one by one) on AVX2.
extern "C" int orc_scores_d64_simd(const float * q, const float * k, int n, float scale, float * sc) {
    if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma")) return -1;
    int j = 0;
    for (; j + 8 <= n; j += 8) scores8_avx2(q, k + (size_t) j * 64, scale, sc + j);
    for (; j < n; ++j) sc[j] = hsum_key_avx2(q, k + (size_t) j * 64, scale);
    return 0;
}

extern "C" void orc_scores_d64(const float * q, const float * k, int n, float scale, float * sc) {
    scores_d64_lanes(q, k, n, scale, sc);
}

namespace {

// tanh256 on AVX2 + FMA, to check orc_tanh_ref's reading of ANDNOT / OR / BLENDV / CMP_LT_OQ.
__attribute__((target("avx2,fma")))
__m256 exp256_avx2(__m256 x) {
    x = _mm256_min_ps(x, _mm256_set1_ps(88.3762626647949f));
    x = _mm256_max_ps(x, _mm256_set1_ps(-87.3f));
    const __m256 fn = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896341f)),
                                      _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    x = _mm256_fnmadd_ps(fn, _mm256_set1_ps(0.693359375f), x);
    x = _mm256_fnmadd_ps(fn, _mm256_set1_ps(-2.12194440e-4f), x);
    const __m256 x2 = _mm256_mul_ps(x, x);
    __m256 p = _mm256_set1_ps(EXP_P[0]);
    for (int k = 1; k < 6; ++k) p = _mm256_fmadd_ps(p, x, _mm256_set1_ps(EXP_P[k]));
    p = _mm256_fmadd_ps(p, x2, _mm256_add_ps(x, _mm256_set1_ps(1.0f)));
    const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(fn), _mm256_set1_epi32(127)), 23);
    return _mm256_mul_ps(p, _mm256_castsi256_ps(e));
}

__attribute__((target("avx2,fma")))
void tanh_avx2(const float * x, int64_t n, float * out) {
    const __m256 sign = _mm256_set1_ps(-0.0f), one = _mm256_set1_ps(1.0f);
    for (int64_t i = 0; i + 8 <= n; i += 8) {
        const __m256 v = _mm256_loadu_ps(x + i);
        const __m256 ax = _mm256_andnot_ps(sign, v);
        const __m256 t = exp256_avx2(_mm256_mul_ps(ax, _mm256_set1_ps(-2.0f)));
        __m256 big = _mm256_div_ps(_mm256_sub_ps(one, t), _mm256_add_ps(one, t));
        big = _mm256_or_ps(big, _mm256_and_ps(sign, v));
        const __m256 v2 = _mm256_mul_ps(v, v);
        __m256 p = _mm256_set1_ps(-17.0f / 315.0f);
        p = _mm256_fmadd_ps(p, v2, _mm256_set1_ps(2.0f / 15.0f));
        p = _mm256_fmadd_ps(p, v2, _mm256_set1_ps(-1.0f / 3.0f));
        p = _mm256_fmadd_ps(p, v2, one);
        const __m256 small = _mm256_mul_ps(p, v);
        _mm256_storeu_ps(out + i, _mm256_blendv_ps(big, small, _mm256_cmp_ps(ax, _mm256_set1_ps(0.1f), _CMP_LT_OQ)));
    }
}

} // namespace

namespace {

// softmax_exp (src/nexterabert.cpp:177-197) on the instructions the reference uses: the
// running std::max, exp256 of each whole 8-group added into one 256-bit lane sum, hsum256
// (VEXTRACTF128 / ADDPS / MOVHLPS / ADDPS / MOVSHDUP / ADDSS), then the tail with the C
// library's expf added one by one. The scalar statement softmax_exp_lanes is checked
// against it.
__attribute__((target("avx2,fma")))
float softmax_exp_avx2(float * s, int n) {
    float m = s[0];
    for (int i = 1; i < n; ++i) m = std::max(m, s[i]);
    int i = 0;
    float sum = 0.0f;
    const __m256 vm = _mm256_set1_ps(m);
    __m256 vs = _mm256_setzero_ps();
    for (; i + 8 <= n; i += 8) {
        const __m256 e = exp256_avx2(_mm256_sub_ps(_mm256_loadu_ps(s + i), vm));
        _mm256_storeu_ps(s + i, e);
        vs = _mm256_add_ps(vs, e);
    }
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(vs), _mm256_extractf128_ps(vs, 1));
    h = _mm_add_ps(h, _mm_movehl_ps(h, h));
    h = _mm_add_ss(h, _mm_movehdup_ps(h));
    sum = _mm_cvtss_f32(h);
    for (; i < n; ++i) {
        s[i] = std::exp(s[i] - m);
        sum += s[i];
    }
    return sum;
}

} // namespace

// softmax_exp on s[0..n): the weights in place, the sum in *sum; simd != 0: on AVX2 + FMA
// (returns -1 without them), else the scalar statement the attention oracle uses.
extern "C" int orc_softmax_exp(float * s, int n, int simd, float * sum) {
    if (simd) {
        if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma")) return -1;
        *sum = softmax_exp_avx2(s, n);
        return 0;
    }
    *sum = softmax_exp_lanes(s, n);
    return 0;
}

extern "C" int orc_tanh_simd(const float * x, int64_t n, float * out) {
    if (n % 8 != 0 || !__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma")) return -1;
    tanh_avx2(x, n, out);
    return 0;
}
