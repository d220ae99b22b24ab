// nxg_host.cpp -- host half of libnxg: the load-time weight expansion of the
// int8 path, the GGUF block decoders it needs, and the placement rule.
//
//   nxg_weight_is_int8   src/nexterabert.cpp:1658-1667
//   nxg_expand_weight    src/nexterabert.cpp:1010-1049 (build_i8_weight)
//   nxg_dequantize_rows  ggml's to_float for the block types a NexteraBERT GGUF
//                        uses (ggml v0.9.9 is not vendored by the reference; the
//                        decoders here follow the published GGUF block formats)
//   nxg_quantize_weight  Q8_0 / Q4_K / Q6_K encoders for synthetic weight files
//
// Everything here is plain C++ on the CPU: it runs once per weight at load time.

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "nxg_linear.h"
#include "nxg_internal.h"

namespace {

thread_local std::string g_err;

int host_fail(int code, const char * msg) {
    g_err = msg;
    return code;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                       // subnormal half: normalise into an f32 normal
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 0x400u)) { mm <<= 1; ++sh; }
            bits = sign | ((uint32_t) (127 - 15 + 1 - sh) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Round-to-nearest-even f32 -> half (for the synthetic-file encoders).
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);          // overflows to inf
    if (ax < 0x38800000u) {                                              // half subnormal or zero
        const float v = std::fabs(f) * 16777216.0f;                     // / 2^-24
        return (uint16_t) (sign | (uint32_t) std::nearbyint(v));
    }
    const uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t r = (e << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) ++r;
    return (uint16_t) (sign | r);
}

inline uint16_t rd16(const uint8_t * p) { return (uint16_t) (p[0] | (p[1] << 8)); }

struct type_info { int blck; int bytes; };

bool info_of(int type, type_info & ti) {
    switch (type) {
        case NXG_TYPE_F32:  ti = { 1, 4 }; return true;
        case NXG_TYPE_F16:  ti = { 1, 2 }; return true;
        case NXG_TYPE_BF16: ti = { 1, 2 }; return true;
        case NXG_TYPE_Q4_0: ti = { 32, 18 }; return true;
        case NXG_TYPE_Q4_1: ti = { 32, 20 }; return true;
        case NXG_TYPE_Q5_0: ti = { 32, 22 }; return true;
        case NXG_TYPE_Q5_1: ti = { 32, 24 }; return true;
        case NXG_TYPE_Q8_0: ti = { 32, 34 }; return true;
        case NXG_TYPE_Q2_K: ti = { 256, 84 }; return true;
        case NXG_TYPE_Q3_K: ti = { 256, 110 }; return true;
        case NXG_TYPE_Q4_K: ti = { 256, 144 }; return true;
        case NXG_TYPE_Q5_K: ti = { 256, 176 }; return true;
        case NXG_TYPE_Q6_K: ti = { 256, 210 }; return true;
        default: return false;
    }
}

// --- block decoders (one block of `blck` values each) ----------------------

// Q4_0: half d, 16 bytes of nibbles; low nibbles are values 0..15, high 16..31.
void dec_q4_0(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b));
    const uint8_t * qs = b + 2;
    for (int j = 0; j < 16; ++j) {
        y[j]      = (float) ((qs[j] & 0x0f) - 8) * d;
        y[j + 16] = (float) ((qs[j] >> 4) - 8) * d;
    }
}

// Q4_1: half d, half m, 16 bytes of nibbles; y = q * d + m.
void dec_q4_1(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b)), m = half_to_float(rd16(b + 2));
    const uint8_t * qs = b + 4;
    for (int j = 0; j < 16; ++j) {
        y[j]      = (float) (qs[j] & 0x0f) * d + m;
        y[j + 16] = (float) (qs[j] >> 4) * d + m;
    }
}

// Q5_0: half d, 32 high bits, 16 bytes of low nibbles; q = (nibble | high << 4) - 16.
void dec_q5_0(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b));
    uint32_t qh;
    std::memcpy(&qh, b + 2, 4);
    const uint8_t * qs = b + 6;
    for (int j = 0; j < 16; ++j) {
        const int h0 = (qh >> j) & 1, h1 = (qh >> (j + 16)) & 1;
        y[j]      = (float) (((qs[j] & 0x0f) | (h0 << 4)) - 16) * d;
        y[j + 16] = (float) (((qs[j] >> 4) | (h1 << 4)) - 16) * d;
    }
}

// Q5_1: half d, half m, 32 high bits, 16 bytes of low nibbles; y = q * d + m.
void dec_q5_1(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b)), m = half_to_float(rd16(b + 2));
    uint32_t qh;
    std::memcpy(&qh, b + 4, 4);
    const uint8_t * qs = b + 8;
    for (int j = 0; j < 16; ++j) {
        const int h0 = (qh >> j) & 1, h1 = (qh >> (j + 16)) & 1;
        y[j]      = (float) ((qs[j] & 0x0f) | (h0 << 4)) * d + m;
        y[j + 16] = (float) ((qs[j] >> 4) | (h1 << 4)) * d + m;
    }
}

// Q8_0: half d, 32 x s8; y = q * d (exact in f32).
void dec_q8_0(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b));
    for (int j = 0; j < 32; ++j) y[j] = (float) (int8_t) b[2 + j] * d;
}

// The 6-bit (scale, min) pair j of a K-quant super-block's 12 scale bytes.
void scale_min_k4(int j, const uint8_t * s, int & sc, int & mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Q2_K: 16 bytes of (4-bit scale | 4-bit min) per 16 values, 64 bytes of 2-bit
// values, half d, half dmin. Values of 128 are packed 4 per byte in 32-byte runs.
void dec_q2_k(const uint8_t * b, float * y) {
    const uint8_t * sc = b;
    const uint8_t * q = b + 16;
    const float d = half_to_float(rd16(b + 80)), dmin = half_to_float(rd16(b + 82));
    int is = 0;
    for (int half = 0; half < 2; ++half) {
        for (int shift = 0; shift < 8; shift += 2) {
            for (int part = 0; part < 2; ++part) {
                const int s = sc[is++];
                const float dl = d * (float) (s & 0x0f), ml = dmin * (float) (s >> 4);
                for (int l = 0; l < 16; ++l) *y++ = dl * (float) ((q[l + 16 * part] >> shift) & 3) - ml;
            }
        }
        q += 32;
    }
}

// Q3_K: 32 bytes of high bits, 64 bytes of 2-bit values, 12 bytes holding 16
// 6-bit scales (biased by 32), half d.
void dec_q3_k(const uint8_t * b, float * y) {
    const uint8_t * hm = b;
    const uint8_t * q = b + 32;
    const uint8_t * s12 = b + 96;
    const float d = half_to_float(rd16(b + 108));
    int8_t scales[16];
    for (int j = 0; j < 16; ++j) {
        const int low = j < 8 ? (s12[j] & 0x0f) : (s12[j - 8] >> 4);
        const int high = (s12[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
        scales[j] = (int8_t) ((low | (high << 4)) - 32);
    }
    int is = 0;
    uint8_t m = 1;
    for (int half = 0; half < 2; ++half) {
        for (int shift = 0; shift < 8; shift += 2) {
            for (int part = 0; part < 2; ++part) {
                const float dl = d * (float) scales[is++];
                for (int l = 0; l < 16; ++l) {
                    const int i = l + 16 * part;
                    const int v = ((q[i] >> shift) & 3) - ((hm[i] & m) ? 0 : 4);
                    *y++ = dl * (float) v;
                }
            }
            m <<= 1;
        }
        q += 32;
    }
}

// Q4_K: half d, half dmin, 12 scale bytes (8 x 6-bit scale and min), 128 bytes
// of nibbles; each 32-byte run holds 64 values (low nibbles first).
void dec_q4_k(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b)), dmin = half_to_float(rd16(b + 2));
    const uint8_t * s = b + 4;
    const uint8_t * q = b + 16;
    for (int j = 0; j < 4; ++j) {
        int sc, mn;
        scale_min_k4(2 * j, s, sc, mn);
        const float d1 = d * (float) sc, m1 = dmin * (float) mn;
        scale_min_k4(2 * j + 1, s, sc, mn);
        const float d2 = d * (float) sc, m2 = dmin * (float) mn;
        for (int l = 0; l < 32; ++l) *y++ = d1 * (float) (q[l] & 0x0f) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * (float) (q[l] >> 4) - m2;
        q += 32;
    }
}

// Q5_K: as Q4_K plus 32 bytes of fifth bits (bit 2j / 2j+1 of byte l for run j).
void dec_q5_k(const uint8_t * b, float * y) {
    const float d = half_to_float(rd16(b)), dmin = half_to_float(rd16(b + 2));
    const uint8_t * s = b + 4;
    const uint8_t * qh = b + 16;
    const uint8_t * ql = b + 48;
    for (int j = 0; j < 4; ++j) {
        int sc, mn;
        scale_min_k4(2 * j, s, sc, mn);
        const float d1 = d * (float) sc, m1 = dmin * (float) mn;
        scale_min_k4(2 * j + 1, s, sc, mn);
        const float d2 = d * (float) sc, m2 = dmin * (float) mn;
        const uint8_t u1 = (uint8_t) (1u << (2 * j)), u2 = (uint8_t) (2u << (2 * j));
        for (int l = 0; l < 32; ++l) *y++ = d1 * (float) ((ql[l] & 0x0f) + ((qh[l] & u1) ? 16 : 0)) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * (float) ((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - m2;
        ql += 32;
    }
}

// Q6_K: 128 bytes of low nibbles, 64 bytes of high 2-bit pairs, 16 s8 scales,
// half d; q = (low | high << 4) - 32, y = d * scale * q.
void dec_q6_k(const uint8_t * b, float * y) {
    const uint8_t * ql = b;
    const uint8_t * qh = b + 128;
    const int8_t * sc = (const int8_t *) (b + 192);
    const float d = half_to_float(rd16(b + 208));
    for (int half = 0; half < 2; ++half) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l]      = d * (float) sc[is + 0] * (float) q1;
            y[l + 32] = d * (float) sc[is + 2] * (float) q2;
            y[l + 64] = d * (float) sc[is + 4] * (float) q3;
            y[l + 96] = d * (float) sc[is + 6] * (float) q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

bool decode_row(int type, const uint8_t * src, int64_t n, float * y) {
    switch (type) {
        case NXG_TYPE_F32: std::memcpy(y, src, sizeof(float) * (size_t) n); return true;
        case NXG_TYPE_F16:
            for (int64_t i = 0; i < n; ++i) y[i] = half_to_float(rd16(src + 2 * i));
            return true;
        case NXG_TYPE_BF16:
            for (int64_t i = 0; i < n; ++i) {
                const uint32_t bits = (uint32_t) rd16(src + 2 * i) << 16;
                std::memcpy(&y[i], &bits, 4);
            }
            return true;
        default: break;
    }
    type_info ti;
    if (!info_of(type, ti) || n % ti.blck) return false;
    void (*dec)(const uint8_t *, float *) = nullptr;
    switch (type) {
        case NXG_TYPE_Q4_0: dec = dec_q4_0; break;
        case NXG_TYPE_Q4_1: dec = dec_q4_1; break;
        case NXG_TYPE_Q5_0: dec = dec_q5_0; break;
        case NXG_TYPE_Q5_1: dec = dec_q5_1; break;
        case NXG_TYPE_Q8_0: dec = dec_q8_0; break;
        case NXG_TYPE_Q2_K: dec = dec_q2_k; break;
        case NXG_TYPE_Q3_K: dec = dec_q3_k; break;
        case NXG_TYPE_Q4_K: dec = dec_q4_k; break;
        case NXG_TYPE_Q5_K: dec = dec_q5_k; break;
        case NXG_TYPE_Q6_K: dec = dec_q6_k; break;
        default: return false;
    }
    for (int64_t b = 0; b < n / ti.blck; ++b) dec(src + b * ti.bytes, y + b * ti.blck);
    return true;
}

// --- encoders for synthetic files -----------------------------------------

// Q8_0: d = amax / 127 (stored as half), q = round(x / d).
void enc_q8_0(const float * x, uint8_t * b) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
    const uint16_t h = float_to_half(d);
    b[0] = (uint8_t) h;
    b[1] = (uint8_t) (h >> 8);
    for (int j = 0; j < 32; ++j) b[2 + j] = (uint8_t) (int8_t) std::lround(std::min(127.0f, std::max(-127.0f, x[j] * id)));
}

// Q5_0 from the published block format: d = m / -16 with m the element of largest
// magnitude (its sign kept), q = min(31, trunc(x / d + 16.5)) split into a low nibble and
// a high bit; decodes as (q - 16) * d.
void enc_q5_0(const float * x, uint8_t * b) {
    float amax = 0.0f, m = 0.0f;
    for (int j = 0; j < 32; ++j) {
        if (std::fabs(x[j]) > amax) {
            amax = std::fabs(x[j]);
            m = x[j];
        }
    }
    const float d = m / -16.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t h = float_to_half(d);
    b[0] = (uint8_t) h;
    b[1] = (uint8_t) (h >> 8);
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
        const int q0 = std::min(31, (int) (int8_t) (x[j] * id + 16.5f));
        const int q1 = std::min(31, (int) (int8_t) (x[j + 16] * id + 16.5f));
        b[6 + j] = (uint8_t) ((q0 & 0x0f) | ((q1 & 0x0f) << 4));
        qh |= (uint32_t) ((q0 >> 4) & 1) << j;
        qh |= (uint32_t) ((q1 >> 4) & 1) << (j + 16);
    }
    std::memcpy(b + 2, &qh, 4);
}

void put_scale_min_k4(int j, int sc, int mn, uint8_t * s) {
    if (j < 4) {
        s[j] = (uint8_t) ((s[j] & 0xc0) | sc);
        s[j + 4] = (uint8_t) ((s[j + 4] & 0xc0) | mn);
    } else {
        s[j + 4] = (uint8_t) ((sc & 0x0f) | ((mn & 0x0f) << 4));
        s[j - 4] = (uint8_t) ((s[j - 4] & 0x3f) | ((sc >> 4) << 6));
        s[j] = (uint8_t) ((s[j] & 0x3f) | ((mn >> 4) << 6));
    }
}

// Q4_K: per 32 values an affine grid x ~ d*sc*q - dmin*mn with q in 0..15,
// 6-bit sc and mn. One pass: range per sub-block, then the two super scales.
void enc_q4_k(const float * x, uint8_t * b) {
    float scl[8], mnv[8];
    for (int j = 0; j < 8; ++j) {
        float lo = 0.0f, hi = 0.0f;
        for (int l = 0; l < 32; ++l) {
            lo = std::min(lo, x[32 * j + l]);
            hi = std::max(hi, x[32 * j + l]);
        }
        scl[j] = (hi - lo) / 15.0f;
        mnv[j] = -lo;
    }
    float smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; ++j) { smax = std::max(smax, scl[j]); mmax = std::max(mmax, mnv[j]); }
    const float d = smax / 63.0f, dmin = mmax / 63.0f;
    const uint16_t hd = float_to_half(d), hm = float_to_half(dmin);
    b[0] = (uint8_t) hd; b[1] = (uint8_t) (hd >> 8);
    b[2] = (uint8_t) hm; b[3] = (uint8_t) (hm >> 8);
    const float dq = half_to_float(hd), mq = half_to_float(hm);
    uint8_t * s = b + 4;
    std::memset(s, 0, 12);
    int sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = dq > 0.0f ? std::min(63, (int) std::lround(scl[j] / dq)) : 0;
        mn[j] = mq > 0.0f ? std::min(63, (int) std::lround(mnv[j] / mq)) : 0;
        put_scale_min_k4(j, sc[j], mn[j], s);
    }
    uint8_t * q = b + 16;
    for (int j = 0; j < 4; ++j) {
        for (int h = 0; h < 2; ++h) {
            const int sb = 2 * j + h;
            const float dl = dq * (float) sc[sb], ml = mq * (float) mn[sb];
            for (int l = 0; l < 32; ++l) {
                int v = dl > 0.0f ? (int) std::lround((x[32 * sb + l] + ml) / dl) : 0;
                v = std::min(15, std::max(0, v));
                if (h == 0) q[32 * j + l] = (uint8_t) v;
                else        q[32 * j + l] |= (uint8_t) (v << 4);
            }
        }
    }
}

// Q6_K: per 16 values a symmetric grid x ~ d*sc*q with q in -32..31 and s8 sc.
void enc_q6_k(const float * x, uint8_t * b) {
    float scl[16];
    float smax = 0.0f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.0f;
        for (int l = 0; l < 16; ++l) amax = std::max(amax, std::fabs(x[16 * j + l]));
        scl[j] = amax / 31.0f;
        smax = std::max(smax, scl[j]);
    }
    const float d = smax / 127.0f;
    const uint16_t hd = float_to_half(d);
    const float dq = half_to_float(hd);
    uint8_t * ql = b;
    uint8_t * qh = b + 128;
    int8_t * sc = (int8_t *) (b + 192);
    b[208] = (uint8_t) hd;
    b[209] = (uint8_t) (hd >> 8);
    std::memset(ql, 0, 128);
    std::memset(qh, 0, 64);
    int q[256];
    for (int j = 0; j < 16; ++j) {
        sc[j] = (int8_t) (dq > 0.0f ? std::min(127, (int) std::lround(scl[j] / dq)) : 0);
        const float dl = dq * (float) sc[j];
        for (int l = 0; l < 16; ++l) {
            int v = dl > 0.0f ? (int) std::lround(x[16 * j + l] / dl) : 0;
            q[16 * j + l] = std::min(31, std::max(-32, v)) + 32;
        }
    }
    // inverse of dec_q6_k's unpacking
    for (int half = 0; half < 2; ++half) {
        for (int l = 0; l < 32; ++l) {
            const int * qq = q + 128 * half;
            uint8_t * L = ql + 64 * half;
            uint8_t * H = qh + 32 * half;
            L[l]      = (uint8_t) ((qq[l] & 0x0f) | ((qq[l + 64] & 0x0f) << 4));
            L[l + 32] = (uint8_t) ((qq[l + 32] & 0x0f) | ((qq[l + 96] & 0x0f) << 4));
            H[l] = (uint8_t) ((qq[l] >> 4) | ((qq[l + 32] >> 4) << 2) | ((qq[l + 64] >> 4) << 4) | ((qq[l + 96] >> 4) << 6));
        }
    }
}

} // namespace

void nxg_set_error(const char * msg) { g_err = msg; }

void nxg_tile_rows(const int8_t * rows, int n_rows, int n_in, int KS, int8_t * tiled) {
    for (int r = 0; r < n_rows; ++r) {
        for (int k = 0; k < n_in; k += 16) {
            const size_t dst = ((size_t) (r / 16) * KS + k / 64) * 1024 + (size_t) ((r % 16) + 16 * ((k % 64) / 16)) * 16;
            std::memcpy(tiled + dst, rows + (size_t) r * n_in + k, 16);
        }
    }
}

extern "C" {

const char * nxg_last_error(void) { return g_err.c_str(); }

int32_t nxg_weight_is_int8(const char * name, int32_t n_dims, int32_t type, int64_t ne0, int64_t ne1, int32_t use_int8) {
    if (!name || !use_int8) return 0;
    const std::string n = name;
    if (n == "embedding.weight" || n == "mlm.decoder.weight" || n == "token_type_embeddings.weight") return 0;
    type_info ti;
    const bool quantized = info_of(type, ti) && type != NXG_TYPE_F32 && type != NXG_TYPE_F16 && type != NXG_TYPE_BF16;
    return (n_dims == 2 && quantized && ne0 % 32 == 0 && ne1 % 4 == 0) ? 1 : 0;
}

size_t nxg_row_bytes(int32_t type, int64_t n_in) {
    type_info ti;
    if (!info_of(type, ti) || n_in < 0 || n_in % ti.blck) return 0;
    return (size_t) (n_in / ti.blck) * ti.bytes;
}

int32_t nxg_dequantize_rows(int32_t type, const void * data, int64_t n_in, int64_t n_rows, float * out) {
    const size_t rb = nxg_row_bytes(type, n_in);
    if (!data || !out || rb == 0 || n_rows < 0) return host_fail(NXG_EINVAL, "dequantize: unsupported type or size");
    for (int64_t r = 0; r < n_rows; ++r) {
        if (!decode_row(type, (const uint8_t *) data + r * rb, n_in, out + r * n_in)) {
            return host_fail(NXG_EINVAL, "dequantize: decode failed");
        }
    }
    return NXG_OK;
}

int32_t nxg_expand_weight(int32_t type, const void * data, int32_t n_in, int32_t n_out, int32_t act_off,
                          int32_t n_threads, int8_t * w, float * scale, int32_t * off) {
    const size_t rb = nxg_row_bytes(type, n_in);
    if (!data || !w || !scale || rb == 0 || n_in <= 0 || n_out <= 0) {
        return host_fail(NXG_EINVAL, "expand_weight: unsupported type or size");
    }
    const int n_blk = (n_in + NXG_BLOCK - 1) / NXG_BLOCK;
    if (n_threads <= 0) n_threads = (int) std::max(1u, std::thread::hardware_concurrency());
    n_threads = std::min(n_threads, n_out);
    std::atomic<int> next(0);
    std::atomic<bool> bad(false);
    auto work = [&]() {
        std::vector<float> row((size_t) n_in);
        for (;;) {
            const int r = next.fetch_add(1);
            if (r >= n_out) break;
            if (!decode_row(type, (const uint8_t *) data + (size_t) r * rb, n_in, row.data())) {
                bad = true;
                break;
            }
            int8_t * q = w + (size_t) r * n_in;
            for (int B = 0; B < n_blk; ++B) {
                const int i0 = B * NXG_BLOCK, i1 = std::min(n_in, i0 + NXG_BLOCK);
                float amax = 0.0f;
                for (int i = i0; i < i1; ++i) amax = std::max(amax, std::fabs(row[i]));
                const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
                int32_t sum = 0;
                for (int i = i0; i < i1; ++i) {
                    q[i] = (int8_t) std::lround(row[i] * inv);
                    sum += q[i];
                }
                scale[(size_t) B * n_out + r] = amax / 127.0f;
                if (off) off[(size_t) B * n_out + r] = -act_off * sum;
            }
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < n_threads; ++i) pool.emplace_back(work);
    work();
    for (std::thread & th : pool) th.join();
    return bad ? host_fail(NXG_EINVAL, "expand_weight: decode failed") : NXG_OK;
}

int32_t nxg_quantize_weight(int32_t type, const float * x, int64_t n_in, int64_t n_rows, void * out) {
    const size_t rb = nxg_row_bytes(type, n_in);
    if (!x || !out || rb == 0) return host_fail(NXG_EINVAL, "quantize_weight: unsupported type or size");
    void (*enc)(const float *, uint8_t *) = nullptr;
    int blck = 0, bytes = 0;
    switch (type) {
        case NXG_TYPE_Q8_0: enc = enc_q8_0; blck = 32; bytes = 34; break;
        case NXG_TYPE_Q5_0: enc = enc_q5_0; blck = 32; bytes = 22; break;
        case NXG_TYPE_Q4_K: enc = enc_q4_k; blck = 256; bytes = 144; break;
        case NXG_TYPE_Q6_K: enc = enc_q6_k; blck = 256; bytes = 210; break;
        default: return host_fail(NXG_EINVAL, "quantize_weight: only Q8_0, Q5_0, Q4_K and Q6_K are encoded");
    }
    uint8_t * o = (uint8_t *) out;
    for (int64_t r = 0; r < n_rows; ++r) {
        for (int64_t b = 0; b < n_in / blck; ++b) enc(x + r * n_in + b * blck, o + r * rb + b * bytes);
    }
    return NXG_OK;
}

int32_t nxg_attention_scales(const int32_t * cu_offsets, int32_t n_seqs, int32_t head_dim, int32_t mode,
                             float s, float b, float ssmax_base, float * out) {
    if (!cu_offsets || !out || n_seqs < 1 || head_dim < 1 || mode < 0 || mode > 2) {
        return host_fail(NXG_EINVAL, "attention_scales: bad arguments");
    }
    // src/nexterabert.cpp:1196-1201 with ssmax_scale, :1174-1181 (std::log on a float: logf).
    // The reference is built with -O3 -march=native and GCC's default floating-point
    // contraction, which fuses s * ln + ssmax_base into one fma (CMakeLists.txt:6-7,77-78).
    const float base = 1.0f / std::sqrt((float) head_dim);
    for (int32_t d = 0; d < n_seqs; ++d) {
        const int n = cu_offsets[d + 1] - cu_offsets[d];
        float f = 1.0f;
        if (mode != 0) {
            const float ln = std::log((float) std::max(n, 1));
            f = mode == 1 ? s * ln : std::fma(s, ln, ssmax_base) + std::max(b, 0.0f);
        }
        out[d] = base * f;
    }
    return NXG_OK;
}

int32_t nxg_rope_table(int32_t n_pos, float base, int32_t head_dim, float * cos_out, float * sin_out) {
    if (n_pos < 1 || head_dim < 2 || head_dim % 2 != 0 || !cos_out || !sin_out) {
        return host_fail(NXG_EINVAL, "rope_table: bad arguments");
    }
    // build_rope, src/nexterabert.cpp:1322-1338, with the same C library calls on floats
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
    return NXG_OK;
}

} // extern "C"
