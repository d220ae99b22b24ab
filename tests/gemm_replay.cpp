// gemm_replay.cpp -- host replay of every global load and store of the int8 GEMM kernels.
//
// For one GEMM shape, plan_gemm picks the kernel and grid exactly as the launcher does
// (nexterabert.cpp_amd/csrc/nxg_linear.hip, launch_gemm), and this file walks that
// kernel's workgroups, waves and lanes through the same tile walk and the same address
// functions (csrc/nxg_gemm_plan.h) that the kernel calls. The loop structure of each
// kernel -- which k-step is loaded when, which lanes load scales, which rows are staged
// -- is restated here from the kernel's source; each replay function names its kernel.
// Every access is checked against the bytes its buffer holds as the C ABI sizes it
// (nxg_qact_q_bytes / nxg_qact_sx_bytes for activations, NP rows for weights, T x N
// floats for rows), every LDS access against the kernel's LDS arrays, and every output
// element is counted: written exactly once, padding of the int8 outputs included.
//
// Built by the CPU tests with g++ and called through ctypes:
//   gemm_replay(T, n_in, n_out, mode, n_seg, seg_cols, cus, &kind, &accesses, err, err_len)
//   mode 0 fp32 rows, 1 fp32 rows + residual, 2 per-block int32 sums, 3 relu^2 -> int8,
//   4 relu^2 -> int8 from fp32 input rows (nxg_linear_f32_relu2_q8_rows)
//   returns 0 (all in bounds and covered), 1 (an access out of bounds), 2 (an output
//   written zero or several times), 3 (no plan for the shape)
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "nxg_gemm_plan.h"

using namespace nxg_gemm;

namespace {

enum buf_id { A, SX, W, SW, RES, OUT, SEG0, SEG1, SEG2, SEG3, SUMS, QO, SXO, XF, N_BUF };
const char * const BUF_NAME[N_BUF] = { "a", "sx", "w", "sw", "res", "out", "seg0", "seg1", "seg2", "seg3",
                                       "sums", "qo", "sxo", "xf" };

struct replay {
    gemm_plan pl{};
    bool xf = false;                         // relu^2 row-tile kernel quantizing fp32 rows itself
    size_t bytes[N_BUF] = {};
    int n_seg = 0;
    int seg_end[4] = {};
    long long accesses = 0;
    int status = 0;
    char * err = nullptr;
    int err_len = 0;
    std::vector<uint8_t> written[N_BUF];   // per 4-byte word of the outputs

    void failf(int code, const char * fmt, ...) __attribute__((format(printf, 3, 4))) {
        if (status) return;
        status = code;
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, (size_t) err_len, fmt, ap);
        va_end(ap);
    }
    // A global access of len bytes at byte offset off of buffer b, by workgroup wg,
    // wave, lane.
    bool load(int b, size_t off, size_t len, int wg, int wave, int lane, const char * what) {
        ++accesses;
        if (off + len > bytes[b]) {
            failf(1, "%s: %s bytes [%zu, %zu) past its %zu (workgroup %d wave %d lane %d)", what, BUF_NAME[b], off,
                  off + len, bytes[b], wg, wave, lane);
            return false;
        }
        return true;
    }
    bool store(int b, size_t off, size_t len, int wg, int wave, int lane, const char * what) {
        if (!load(b, off, len, wg, wave, lane, what)) return false;
        for (size_t i = off / 4; i < (off + len) / 4; ++i) {
            if (written[b][i] < 255) ++written[b][i];
        }
        return true;
    }
    bool lds(size_t off, size_t len, size_t size, int wg, int wave, int lane, const char * what) {
        ++accesses;
        if (off + len > size) {
            failf(1, "%s: LDS bytes [%zu, %zu) past the %zu of the array (workgroup %d wave %d lane %d)", what, off,
                  off + len, size, wg, wave, lane);
            return false;
        }
        return true;
    }
    void track(int b) { written[b].assign(bytes[b] / 4, 0); }
    // Every word of [0, words) of b written exactly once; `row` / `cols` name a word in
    // messages (row-major [rows][cols] words).
    void covered(int b, size_t words, size_t cols) {
        for (size_t i = 0; i < words && !status; ++i) {
            if (written[b][i] != 1) {
                failf(2, "%s: word %zu (row %zu, column %zu) written %d times", BUF_NAME[b], i, i / cols, i % cols,
                      (int) written[b][i]);
            }
        }
    }
};

// --- gemm_k256 ------------------------------------------------------------------------

void replay_k256(replay & r, bool res) {
    const gemm_plan & p = r.pl;
    const size_t frow = (size_t) p.KS * FRAG;
    const int nb = p.KS / 4;
    const size_t ring = 4 * SLOT;
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const tile_walk walk(wg, p.grid, p.G);
        if (walk.count == 0) continue;
        for (int wave = 0; wave < NTHREADS / 64; ++wave) {
            const int wm = wave >> 1, wn = wave & 1;
            struct rows { size_t a0, a1, w0, w1; };
            auto rows_of = [&](int i) {
                const int tile = walk.tile_clamped(i);
                const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
                return rows{ (size_t) a_frag(mt, wave, p.MF) * frow, (size_t) a_frag(mt, wave + 4, p.MF) * frow,
                             (size_t) w_frag(nt, BN, wave) * frow, (size_t) w_frag(nt, BN, wave + 4) * frow };
            };
            auto issue = [&](const rows & rw, int ks, int j) {
                for (int lane = 0; lane < 64; ++lane) {
                    const size_t vo = (size_t) lane * 16 + (size_t) ks * FRAG;
                    const size_t m = (size_t) j * SLOT + (size_t) wave * FRAG + (size_t) lane * 16;
                    r.load(A, rw.a0 + vo, 16, wg, wave, lane, "gemm_k256 A fragment");
                    r.load(A, rw.a1 + vo, 16, wg, wave, lane, "gemm_k256 A fragment");
                    r.load(W, rw.w0 + vo, 16, wg, wave, lane, "gemm_k256 B fragment");
                    r.load(W, rw.w1 + vo, 16, wg, wave, lane, "gemm_k256 B fragment");
                    for (int q = 0; q < 4; ++q) r.lds(m + (size_t) q * 4 * FRAG, 16, ring, wg, wave, lane, "gemm_k256 ring");
                }
            };
            {
                const rows r0 = rows_of(0);
                issue(r0, 0, 0);
                issue(r0, 1, 1);
                issue(r0, 2, 2);
            }
            for (int it = 0; it < walk.count && !r.status; ++it) {
                const int tile = walk.tile(it);
                const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
                if (tile >= p.G) r.failf(1, "gemm_k256: workgroup %d walks tile %d of %d", wg, tile, p.G);
                issue(rows_of(it), 3, 3);        // the tile start: its k-step 3 into slot 3
                for (int B = 0; B < nb; ++B) {
                    const bool last = B == nb - 1;
                    for (int j = 0; j < 4; ++j) {
                        const ring_load l = ring_prefetch(it, B, j, last, true);
                        if (l.pos >= 0) issue(rows_of(l.pos), l.ks, l.slot);
                        if (j == 0 && wave == 0) {
                            // the block's scales, lane l at ring + 3 SLOT + SLOT_AB + 16 l
                            for (int lane = 0; lane < 64; ++lane) {
                                if (lane < 32) {
                                    const size_t o = sx_group_index(mt, lane, p.MF, p.n_blk, 0) * 4 + (size_t) B * 16;
                                    if (o != sx_group_index(mt, lane, p.MF, p.n_blk, B) * 4) r.failf(1, "gemm_k256: sx step");
                                    r.load(SX, o, 16, wg, wave, lane, "gemm_k256 sx");
                                } else {
                                    const size_t o = sw_index(0, p.NP, nt * BN + 4 * (lane - 32)) * 4 + (size_t) B * p.NP * 4;
                                    r.load(SW, o, 16, wg, wave, lane, "gemm_k256 sw");
                                }
                                r.lds(3 * SLOT + SLOT_AB + (size_t) lane * 16, 16, ring, wg, wave, lane, "gemm_k256 scales");
                            }
                        }
                    }
                }
                for (int lane = 0; lane < 64; ++lane) {
                    const int rrow = lane >> 4, rcol = 4 * (lane & 15);
                    const int tbase = mt * BM + wm * 64, ncol = nt * BN + wn * 64 + rcol;
                    if (res) {
                        // load_res(0) and load_res(2): pieces 0..3
                        const int row0 = mt * BM + wm * 64;
                        const size_t col = (size_t) clamp_col4(ncol, p.N);
                        for (int mi = 0; mi < 4; ++mi)
                            for (int q = 0; q < 4; ++q) {
                                size_t o;
                                if (row0 + 64 <= p.T) {
                                    o = (size_t) (row0 + mi * 16 + 4 * q) * p.N + ((size_t) rrow * p.N + col);
                                } else {
                                    o = (size_t) clamp_row(row0 + mi * 16 + 4 * q + rrow, p.T) * p.N + col;
                                }
                                r.load(RES, o * 4, 16, wg, wave, lane, "gemm_k256 residual");
                            }
                    }
                    // staging: written in MFMA order, read back as rows
                    const size_t stg = 3 * SLOT + (size_t) wave * STAGE_BYTES;
                    const int trow = lane & 15, tcol = 4 * (lane >> 4);
                    for (int ni = 0; ni < 4; ++ni)
                        r.lds(stg + (size_t) (trow * STAGE_PITCH + 16 * ni + tcol) * 4, 16, ring, wg, wave, lane, "gemm_k256 staging");
                    const int seg_ids[4] = { SEG0, SEG1, SEG2, SEG3 };
                    const out_col<int> om = out_col_of<int>(ncol, p.N, r.n_seg, r.seg_end, (int) OUT, seg_ids);
                    for (int mi = 0; mi < 4; ++mi)
                        for (int q = 0; q < 4; ++q) {
                            const int row = 4 * q + rrow;
                            r.lds(stg + (size_t) (row * STAGE_PITCH + rcol) * 4, 16, ring, wg, wave, lane, "gemm_k256 staging");
                            const int t = tbase + mi * 16 + row;
                            if (t < p.T && ncol < p.N) {
                                r.store(om.base, ((size_t) t * om.ld + om.col) * 4, 16, wg, wave, lane, "gemm_k256 output");
                            }
                        }
                }
            }
        }
    }
}

// --- gemm_kernel (fp32 rows, or per-block sums) ----------------------------------------

void replay_general(replay & r, bool res, bool sums) {
    const gemm_plan & p = r.pl;
    const bool k256 = p.k256;
    const size_t slot_bytes = SLOT;
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const tile_walk walk(wg, p.grid, p.G);
        if (walk.count == 0) continue;
        if (!k256 && walk.count > 1) r.failf(1, "gemm_kernel: workgroup %d has %d tiles without K256", wg, walk.count);
        for (int wave = 0; wave < NTHREADS / 64; ++wave) {
            const int wm = wave >> 1, wn = wave & 1;
            // the load stream: every k-step of every tile of the walk, in order (the issues
            // past the last k-step return without loading)
            for (int it = 0; it < walk.count; ++it) {
                const int tile = walk.tile(it);
                const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
                for (int ks = 0; ks < p.KS; ++ks) {
                    for (int lane = 0; lane < 64; ++lane) {
                        const size_t o = (size_t) ks * FRAG;
                        r.load(A, frag_byte(a_frag(mt, wave, p.MF), p.KS, 0, lane) + o, 16, wg, wave, lane, "gemm_kernel A");
                        r.load(A, frag_byte(a_frag(mt, wave + 4, p.MF), p.KS, 0, lane) + o, 16, wg, wave, lane, "gemm_kernel A");
                        r.load(W, frag_byte(w_frag(nt, BN, wave), p.KS, 0, lane) + o, 16, wg, wave, lane, "gemm_kernel B");
                        r.load(W, frag_byte(w_frag(nt, BN, wave + 4), p.KS, 0, lane) + o, 16, wg, wave, lane, "gemm_kernel B");
                        for (int q = 0; q < 4; ++q) {
                            r.lds((size_t) (wave + 4 * q) * FRAG + (size_t) lane * 16, 16, slot_bytes, wg, wave, lane, "gemm_kernel slot");
                        }
                    }
                    // the block's scales: with its last k-step, or after a partial last block
                    const bool scale_now = (ks & 3) == 3 || (!k256 && ks == p.KS - 1 && (p.KS & 3) != 0);
                    if (!sums && wave == 0 && scale_now) {
                        const int B = ks >> 2;
                        for (int lane = 0; lane < 64; ++lane) {
                            if (lane < 32) r.load(SX, sx_group_index(mt, lane, p.MF, p.n_blk, B) * 4, 16, wg, wave, lane, "gemm_kernel sx");
                            else r.load(SW, sw_index(B, p.NP, nt * BN + 4 * (lane - 32)) * 4, 16, wg, wave, lane, "gemm_kernel sw");
                            r.lds(SLOT_AB + (size_t) lane * 16, 16, slot_bytes, wg, wave, lane, "gemm_kernel scales");
                        }
                    }
                }
                for (int lane = 0; lane < 64; ++lane) {
                    const int t0 = mt * BM + wm * 64 + (lane & 15);
                    const int n0 = nt * BN + wn * 64 + 4 * (lane >> 4);
                    if (sums) {
                        for (int B = 0; B < p.n_blk; ++B)
                            for (int mi = 0; mi < 4; ++mi)
                                for (int ni = 0; ni < 4; ++ni)
                                    for (int e = 0; e < 4; ++e) {
                                        const int t = t0 + mi * 16, n = n0 + ni * 16 + e;
                                        if (t < p.T && n < p.N) {
                                            r.store(SUMS, (((size_t) B * p.T + t) * p.N + n) * 4, 4, wg, wave, lane, "gemm_kernel sums");
                                        }
                                    }
                    } else if ((p.N & 3) == 0) {
                        const int trow = lane & 15, tcol = 4 * (lane >> 4);
                        const int rrow = lane >> 4, rcol = 4 * (lane & 15);
                        const int tbase = mt * BM + wm * 64, nb = nt * BN + wn * 64 + rcol;
                        const size_t stg = (size_t) wave * STAGE_BYTES;
                        for (int ni = 0; ni < 4; ++ni)
                            r.lds(stg + (size_t) (trow * STAGE_PITCH + 16 * ni + tcol) * 4, 16, slot_bytes, wg, wave, lane, "gemm_kernel staging");
                        for (int mi = 0; mi < 4; ++mi)
                            for (int q = 0; q < 4; ++q) {
                                const int row = 4 * q + rrow;
                                r.lds(stg + (size_t) (row * STAGE_PITCH + rcol) * 4, 16, slot_bytes, wg, wave, lane, "gemm_kernel staging");
                                const int t = tbase + mi * 16 + row;
                                if (t < p.T && nb < p.N) {
                                    const size_t o = (size_t) t * p.N + nb;
                                    if (res) r.load(RES, o * 4, 16, wg, wave, lane, "gemm_kernel residual");
                                    r.store(OUT, o * 4, 16, wg, wave, lane, "gemm_kernel output");
                                }
                            }
                    } else {
                        for (int mi = 0; mi < 4; ++mi) {
                            const int t = t0 + mi * 16;
                            if (t >= p.T) continue;
                            for (int ni = 0; ni < 4; ++ni) {
                                const int n = n0 + ni * 16;
                                const size_t o = (size_t) t * p.N + n;
                                for (int e = 0; e < 4; ++e) {
                                    if (n + e < p.N) {
                                        if (res) r.load(RES, (o + e) * 4, 4, wg, wave, lane, "gemm_kernel residual");
                                        r.store(OUT, (o + e) * 4, 4, wg, wave, lane, "gemm_kernel output");
                                    }
                                }
                            }
                        }
                    }
                }
            }
        }
    }
}

// --- small_piece (gemm_small, gemm_relu2_small) -----------------------------------------

// The loads of one wave's piece: fragment rows of piece row mt and weight rows nr0 ..
// nr0 + fn - 1, the k-steps small_piece loads (its prologue, then per block the refills
// of each mode), and the sx of each block.
void replay_small_piece(replay & r, int wg, int wave, int mt, int nr0, int fn, bool k256) {
    const gemm_plan & p = r.pl;
    const size_t frow = (size_t) p.KS * FRAG;
    const int D = small_depth(fn);
    const int nb = p.n_blk;
    int fr[SDT];
    for (int j = 0; j < SDT; ++j) fr[j] = small_a_frag(mt, j, p.MF);
    auto load = [&](int ks) {
        if (ks < 0 || ks >= p.KS) r.failf(1, "small_piece: workgroup %d loads k-step %d of %d", wg, ks, p.KS);
        for (int lane = 0; lane < 64; ++lane) {
            for (int j = 0; j < SDT; ++j) r.load(A, (size_t) fr[j] * frow + (size_t) ks * FRAG + (size_t) lane * 16, 16, wg, wave, lane, "small_piece A");
            for (int i = 0; i < fn; ++i) r.load(W, (size_t) (nr0 + i) * frow + (size_t) ks * FRAG + (size_t) lane * 16, 16, wg, wave, lane, "small_piece B");
        }
    };
    auto load_sx = [&](int B) {
        for (int lane = 0; lane < 64; ++lane)
            for (int j = 0; j < SDT; ++j) r.load(SX, sx_index(fr[j] * 16 + (lane & 15), nb, B) * 4, 4, wg, wave, lane, "small_piece sx");
    };
    enum { R_FULL, R_CLAMP, R_NONE, R_LAST };
    auto block = [&](int b, int mode) {
        if (mode != R_LAST) load_sx(b + 1);
        const int nks = k256 ? 4 : imin(4, p.KS - 4 * b);
        for (int ks = 0; ks < 4; ++ks) {
            if (!(k256 || ks < nks)) continue;
            if (mode == R_FULL) load(4 * b + ks + D);
            if (mode == R_CLAMP) load(imin(4 * b + ks + D, p.KS - 1));
        }
    };
    load_sx(0);
    for (int s = 0; s < D; ++s)
        if (s < p.KS) load(s);
    int b = 0;
    if (k256) {
        const int nfull = nb - D / 4;
        for (; b + 1 < nfull; b += 2) { block(b, R_FULL); block(b + 1, R_FULL); }
        if (b < nfull) { block(b, R_FULL); ++b; }
        if (D == 8 && b + 2 == nb) { block(b, R_NONE); block(b + 1, R_LAST); }
        else block(b, R_LAST);
    } else {
        for (; b + 2 < nb; b += 2) { block(b, R_CLAMP); block(b + 1, R_CLAMP); }
        if (b + 2 == nb) { block(b, R_CLAMP); block(b + 1, R_LAST); }
        else block(b, R_LAST);
    }
}

// small_sw_fill: threads of the workgroup copy sw of blocks 0 .. n_blk - 1, features n0 ..
// n0 + nw - 1, into an LDS array of lds_floats.
void replay_sw_fill(replay & r, int wg, int threads, int n0, int nw, size_t lds_floats) {
    const gemm_plan & p = r.pl;
    for (int th = 0; th < threads; ++th)
        for (int i = th; i < p.n_blk * (nw / 4); i += threads) {
            const int B = i / (nw / 4), c = (i - B * (nw / 4)) * 4;
            r.load(SW, sw_index(B, p.NP, n0 + c) * 4, 16, wg, th >> 6, th & 63, "small_sw_fill");
            r.lds((size_t) (B * nw + c) * 4, 16, lds_floats * 4, wg, th >> 6, th & 63, "small_sw_fill LDS");
        }
}

void replay_small(replay & r, bool res) {
    const gemm_plan & p = r.pl;
    const int fn = p.fn;
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const int mt = wg / p.n_nt, nt = wg - mt * p.n_nt;
        const int fr0 = mt * SDT, nr0 = w_frag(nt, 16 * fn, 0);
        replay_small_piece(r, wg, 0, mt, nr0, fn, p.k256);
        replay_sw_fill(r, wg, 64, nr0 * 16, 16 * fn, (size_t) SNB_MAX * 16 * fn);
        const int seg_ids[4] = { SEG0, SEG1, SEG2, SEG3 };
        for (int lane = 0; lane < 64; ++lane)
            for (int j = 0; j < SDT; ++j)
                for (int i = 0; i < fn; ++i) {
                    if (res) {
                        const int t = clamp_row((fr0 + j) * 16 + (lane & 15), p.T);
                        const int n = clamp_col4((nr0 + i) * 16 + 4 * (lane >> 4), p.N);
                        r.load(RES, ((size_t) t * p.N + n) * 4, 16, wg, 0, lane, "gemm_small residual");
                    }
                    const int t = (fr0 + j) * 16 + (lane & 15);
                    const int n = (nr0 + i) * 16 + 4 * (lane >> 4);
                    if (t >= p.T || n >= p.N) continue;
                    const out_col<int> om = out_col_of<int>(n, p.N, r.n_seg, r.seg_end, (int) OUT, seg_ids);
                    r.store(om.base, ((size_t) t * om.ld + om.col) * 4, 16, wg, 0, lane, "gemm_small output");
                }
    }
}

// gemm_fsk: one workgroup per 64 x TN tile (TN = p.fn), wave b < n_blk loads block b's 4
// k-steps of the tile's 4 activation and TN / 16 weight fragments and the block's scales into
// LDS; waves 0..3 fold one row group each and store.
void replay_fsk(replay & r, bool res) {
    const gemm_plan & p = r.pl;
    const int TN = p.fn, NJ = TN / 16, nb = p.n_blk;
    if (!p.k256 || nb > FSK_NB || (TN != 64 && TN != 32) || (TN == 64 && nb > 4)) {
        r.failf(1, "gemm_fsk: n_blk %d, TN %d", nb, TN);
        return;
    }
    const int NBM = TN == 64 ? 4 : FSK_NB;
    const size_t frow = (size_t) p.KS * FRAG;
    const size_t sums = (size_t) NBM * 64 * TN * 4, sxl = (size_t) NBM * 64 * 4, swl = (size_t) NBM * TN * 4;
    const int seg_ids[4] = { SEG0, SEG1, SEG2, SEG3 };
    if (p.block != 64 * (nb > 4 ? nb : 4)) r.failf(1, "gemm_fsk: %d threads for %d blocks", p.block, nb);
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const int mt = wg / p.n_nt, nt = wg - mt * p.n_nt;
        for (int b = 0; b < nb; ++b)
            for (int lane = 0; lane < 64; ++lane) {
                for (int s = 0; s < 4; ++s) {
                    const size_t ko = (size_t) (4 * b + s) * FRAG + (size_t) lane * 16;
                    for (int i = 0; i < 4; ++i)
                        r.load(A, (size_t) fsk_a_frag(mt, i, p.MF) * frow + ko, 16, wg, b, lane, "gemm_fsk A fragment");
                    for (int j = 0; j < NJ; ++j)
                        r.load(W, (size_t) (nt * NJ + j) * frow + ko, 16, wg, b, lane, "gemm_fsk B fragment");
                }
                if (lane < 16) {
                    r.load(SX, fsk_sx_group(mt, lane, p.MF, nb, b) * 4, 16, wg, b, lane, "gemm_fsk sx");
                    r.lds(((size_t) b * 64 + 4 * lane) * 4, 16, sxl, wg, b, lane, "gemm_fsk sx");
                } else if (lane < 16 + TN / 4) {
                    const int c = 4 * (lane - 16);
                    r.load(SW, sw_index(b, p.NP, nt * TN + c) * 4, 16, wg, b, lane, "gemm_fsk sw");
                    r.lds(((size_t) b * TN + c) * 4, 16, swl, wg, b, lane, "gemm_fsk sw");
                }
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < NJ; ++j)
                        r.lds(((size_t) b * 64 * TN + (size_t) ((i * NJ + j) * 64 + lane) * 4) * 4, 16, sums, wg, b, lane,
                              "gemm_fsk sums");
            }
        for (int w = 0; w < 4; ++w)
            for (int lane = 0; lane < 64; ++lane) {
                const int t = mt * 64 + w * 16 + (lane & 15), c0 = 4 * (lane >> 4);
                for (int j = 0; j < NJ; ++j) {
                    if (res)
                        r.load(RES, ((size_t) clamp_row(t, p.T) * p.N + clamp_col4(nt * TN + 16 * j + c0, p.N)) * 4, 16, wg, w,
                               lane, "gemm_fsk residual");
                    for (int b = 0; b < nb; ++b) {
                        r.lds(((size_t) b * 64 * TN + (size_t) ((w * NJ + j) * 64 + lane) * 4) * 4, 16, sums, wg, w, lane,
                              "gemm_fsk fold");
                        r.lds(((size_t) b * TN + 16 * j + c0) * 4, 16, swl, wg, w, lane, "gemm_fsk fold sw");
                        r.lds(((size_t) b * 64 + w * 16 + (lane & 15)) * 4, 4, sxl, wg, w, lane, "gemm_fsk fold sx");
                    }
                    const int n = nt * TN + 16 * j + c0;
                    if (t >= p.T || n >= p.N) continue;
                    const out_col<int> om = out_col_of<int>(n, p.N, r.n_seg, r.seg_end, (int) OUT, seg_ids);
                    r.store(om.base, ((size_t) t * om.ld + om.col) * 4, 16, wg, w, lane, "gemm_fsk output");
                }
            }
    }
}

// --- relu^2 -> int8 outputs -----------------------------------------------------------

// The stores of fragment row rf, fragment column kf (one wave's 64 lanes), and with
// `scales` the sxo of its 16 rows (lanes 0..15).
void relu2_store(replay & r, int wg, int wave, int rf, int kf, int nt, bool scales, const char * what) {
    const gemm_plan & p = r.pl;
    if (rf >= p.MF) return;
    for (int lane = 0; lane < 64; ++lane) {
        if (kf < p.KSo) r.store(QO, qo_byte(rf, p.KSo, kf, lane), 16, wg, wave, lane, what);
        if (scales && lane < 16) {
            const int t = rf * 16 + lane;
            r.store(SXO, sxo_index(t, p.n_nt, nt) * 4, 4, wg, wave, lane, what);
        }
    }
}

void replay_relu2_q8(replay & r) {
    const gemm_plan & p = r.pl;
    const size_t frow = (size_t) p.KS * FRAG;
    const int nb = p.KS / 4;
    const size_t ring = 4 * WSLOT;
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const tile_walk walk(wg, p.grid, p.G);
        if (walk.count == 0) continue;
        for (int wave = 0; wave < WTHREADS / 64; ++wave) {
            const int wm = wave >> 2, wn = wave & 3;
            struct rows { size_t a, w0, w1; };
            auto rows_of = [&](int i) {
                const int tile = walk.tile_clamped(i);
                const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
                return rows{ (size_t) a_frag(mt, wave, p.MF) * frow, (size_t) w_frag(nt, WBN, wave) * frow,
                             (size_t) w_frag(nt, WBN, wave + 8) * frow };
            };
            auto issue = [&](const rows & rw, int ks, int j) {
                for (int lane = 0; lane < 64; ++lane) {
                    const size_t vo = (size_t) lane * 16 + (size_t) ks * FRAG;
                    const size_t m = (size_t) j * WSLOT + (size_t) wave * FRAG + (size_t) lane * 16;
                    r.load(A, rw.a + vo, 16, wg, wave, lane, "gemm_relu2_q8 A fragment");
                    r.load(W, rw.w0 + vo, 16, wg, wave, lane, "gemm_relu2_q8 B fragment");
                    r.load(W, rw.w1 + vo, 16, wg, wave, lane, "gemm_relu2_q8 B fragment");
                    r.lds(m, 16, ring, wg, wave, lane, "gemm_relu2_q8 ring");
                    r.lds(m + 8 * FRAG, 16, ring, wg, wave, lane, "gemm_relu2_q8 ring");
                    r.lds(m + 16 * FRAG, 16, ring, wg, wave, lane, "gemm_relu2_q8 ring");
                }
            };
            {
                const rows r0 = rows_of(0);
                issue(r0, 0, 0);
                issue(r0, 1, 1);
                issue(r0, 2, 2);
                issue(r0, 3, 3);
            }
            for (int it = 0; it < walk.count && !r.status; ++it) {
                const int tile = walk.tile(it);
                const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
                if (tile >= p.G) r.failf(1, "gemm_relu2_q8: workgroup %d walks tile %d of %d", wg, tile, p.G);
                for (int B = 0; B < nb; ++B) {
                    const bool last = B == nb - 1;
                    for (int j = 0; j < 4; ++j) {
                        const ring_load l = ring_prefetch(it, B, j, last, false);
                        issue(rows_of(l.pos), l.ks, l.slot);
                        if (j == 0 && (wave == 0 || wave == 1)) {
                            for (int lane = 0; lane < (wave == 0 ? 64 : 32); ++lane) {
                                if (wave == 0 && lane < 32) {
                                    r.load(SX, sx_group_index(mt, lane, p.MF, p.n_blk, 0) * 4 + (size_t) B * 16, 16, wg, wave, lane, "gemm_relu2_q8 sx");
                                } else {
                                    const int n = nt * WBN + (wave == 0 ? 4 * (lane - 32) : 128 + 4 * lane);
                                    r.load(SW, sw_index(0, p.NP, n) * 4 + (size_t) B * p.NP * 4, 16, wg, wave, lane, "gemm_relu2_q8 sw");
                                }
                                r.lds((size_t) lane * 16 + (wave == 1 ? 1024 : 0), 16, WSCALE, wg, wave, lane, "gemm_relu2_q8 scales");
                            }
                        }
                    }
                }
                for (int mi = 0; mi < 4; ++mi) {
                    const int rf = mt * (BM / 16) + wm * 4 + mi, kf = nt * (WBN / 64) + wn;
                    relu2_store(r, wg, wave, rf, kf, nt, false, "gemm_relu2_q8 output");
                }
                // the row scales: lane l of a wn == 0 wave stores row l of the wave's 64 (row
                // group l / 16) when that fragment row exists
                for (int lane = 0; lane < 64 && wn == 0; ++lane)
                    if (mt * (BM / 16) + wm * 4 + (lane >> 4) < p.MF)
                        r.store(SXO, sxo_index(mt * BM + wm * 64 + lane, p.n_nt, nt) * 4, 4, wg, wave, lane,
                                "gemm_relu2_q8 row scales");
            }
        }
    }
}

// gemm_relu2_rt: a contiguous span of 64 x 256 tiles per workgroup, the row tile in LDS
// (loaded at the span's start and whenever the row tile changes), each wave's 4 weight
// fragments per k-step into registers 4 k-steps ahead, a tile's scales loaded under the
// previous tile into the other of two buffers.
void replay_relu2_rt(replay & r) {
    const gemm_plan & p = r.pl;
    const int NB = p.n_blk, KS = p.KS;
    if (KS != 4 * NB || (NB != 1 && NB != RNB_MAX)) {
        r.failf(1, "gemm_relu2_rt: n_blk %d, KS %d", NB, KS);
        return;
    }
    const size_t frow = (size_t) KS * FRAG;
    const size_t arow = (size_t) KS * (RM / 16) * FRAG, scl = 2 * (size_t) RSCALE, am = 2 * RM * 4 * sizeof(float);
    const size_t sxr = (size_t) RM * NB * sizeof(float);
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const tile_span span(wg, p.grid, p.G);
        if (span.count < 0 || (span.count > 0 && (span.first < 0 || span.first + span.count > p.G))) {
            r.failf(1, "gemm_relu2_rt: workgroup %d spans tiles [%d, %d) of %d", wg, span.first, span.first + span.count, p.G);
            return;
        }
        if (span.count == 0) continue;
        for (int wave = 0; wave < RTHREADS / 64; ++wave) {
            auto load_rows = [&](int mt) {
                if (r.xf) {
                    // fp32 rows quantized into LDS: stage st = (4 rows, block st % NB), lane row
                    // 16 wave + 4 (st / NB) + lane / 16, c = lane % 16
                    for (int st = 0; st < 4 * NB; ++st)
                        for (int lane = 0; lane < 64; ++lane) {
                            const int c = lane & 15, rr = wave * 16 + 4 * (st / NB) + (lane >> 4), B = st % NB;
                            const int t = rt_x_row(mt, rr, p.T);
                            for (int i = 0; i < 4; ++i) {
                                r.load(XF, ((size_t) t * 256 * NB + 256 * B + 64 * i + 4 * c) * 4, 16, wg, wave, lane,
                                       "gemm_relu2_rt fp32 rows");
                                r.lds((size_t) ((4 * B + i) * 4 + wave) * FRAG + (size_t) ((rr & 15) + 16 * (c >> 2)) * 16 + 4 * (c & 3),
                                      4, arow, wg, wave, lane, "gemm_relu2_rt quantized row tile");
                            }
                            if (c == 0)
                                r.lds((((size_t) (rr >> 2) * NB + B) * 4 + (rr & 3)) * 4, 4, sxr, wg, wave, lane,
                                      "gemm_relu2_rt row scales");
                        }
                    return;
                }
                for (int ks = 0; ks < KS; ++ks)
                    for (int lane = 0; lane < 64; ++lane) {
                        r.load(A, (size_t) a_frag_rt(mt, wave, p.MF) * frow + (size_t) ks * FRAG + (size_t) lane * 16, 16,
                               wg, wave, lane, "gemm_relu2_rt row tile");
                        r.lds((size_t) (ks * 4 + wave) * FRAG + (size_t) lane * 16, 16, arow, wg, wave, lane,
                              "gemm_relu2_rt row tile");
                    }
            };
            auto load_scales = [&](int tile, int b) {
                const int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
                for (int lane = 0; lane < 64; ++lane) {
                    if (wave < NB) {
                        r.load(SW, sw_index(wave, p.NP, nt * WBN + 4 * lane) * 4, 16, wg, wave, lane, "gemm_relu2_rt sw");
                        r.lds((size_t) b * RSCALE + RSX_BYTES + (size_t) wave * WBN * 4 + (size_t) lane * 16, 16, scl, wg,
                              wave, lane, "gemm_relu2_rt sw");
                    }
                    if (!r.xf && wave == 0 && lane < 16 * NB) {
                        r.load(SX, sx_group_index_rt(mt, lane / NB, p.MF, NB, lane % NB) * 4, 16, wg, wave, lane,
                               "gemm_relu2_rt sx");
                        r.lds((size_t) b * RSCALE + (size_t) lane * 16, 16, scl, wg, wave, lane, "gemm_relu2_rt sx");
                    }
                }
            };
            auto ldw = [&](int nt, int ks) {
                for (int i = 0; i < 4; ++i)
                    for (int lane = 0; lane < 64; ++lane)
                        r.load(W, (size_t) w_frag(nt, WBN, 4 * wave) * frow + (size_t) ks * FRAG + (size_t) i * frow +
                                      (size_t) lane * 16, 16, wg, wave, lane, "gemm_relu2_rt weights");
            };
            int tile = span.first;
            int mt = tile / p.n_nt, nt = tile - mt * p.n_nt;
            load_rows(mt);
            load_scales(tile, 0);
            for (int j = 0; j < RDEPTH; ++j) ldw(nt, j);
            for (int it = 0; it < span.count && !r.status; ++it) {
                const int cur = it & 1;
                const bool more = it + 1 < span.count;
                if (more) load_scales(tile + 1, cur ^ 1);
                for (int B = 0; B < NB; ++B) {
                    for (int s4 = 0; s4 < 4; ++s4) {
                        for (int lane = 0; lane < 64; ++lane)
                            for (int i = 0; i < 4; ++i)
                                r.lds((size_t) ((4 * B + s4) * 4 + i) * FRAG + (size_t) lane * 16, 16, arow, wg, wave, lane,
                                      "gemm_relu2_rt operand read");
                        if (B < NB - 1) ldw(nt, 4 * B + 4 + s4);
                        else if (s4 == 0 && more) ldw((tile + 1) % p.n_nt, 0);   // the next tile's k-step 0
                    }
                    for (int lane = 0; lane < 64; ++lane) {
                        for (int mi = 0; mi < 4; ++mi) {
                            const int rr = mi * 16 + (lane & 15);
                            if (r.xf)
                                r.lds((((size_t) (rr >> 2) * NB + B) * 4 + (rr & 3)) * 4, 4, sxr, wg, wave, lane,
                                      "gemm_relu2_rt row scale read");
                            else
                                r.lds((size_t) cur * RSCALE + (((size_t) (rr >> 2) * NB + B) * 4 + (rr & 3)) * 4, 4, scl, wg,
                                      wave, lane, "gemm_relu2_rt sx read");
                        }
                        for (int ni = 0; ni < 4; ++ni)
                            r.lds((size_t) cur * RSCALE + RSX_BYTES + ((size_t) B * WBN + wave * 64 + ni * 16 + 4 * (lane >> 4)) * 4,
                                  16, scl, wg, wave, lane, "gemm_relu2_rt sw read");
                    }
                }
                for (int lane = 0; lane < 64; ++lane) {
                    for (int mi = 0; mi < 4 && lane < 16; ++mi)
                        r.lds(((size_t) cur * RM * 4 + (size_t) (mi * 16 + lane) * 4 + wave) * 4, 4, am, wg, wave, lane,
                              "gemm_relu2_rt row maxima");
                    r.lds(((size_t) cur * RM * 4 + (size_t) lane * 4) * 4, 16, am, wg, wave, lane, "gemm_relu2_rt row maxima");
                }
                const int mt_t = mt, nt_t = nt;
                if (more) {
                    const bool reload = (tile + 1) / p.n_nt != mt;
                    ++tile;
                    mt = tile / p.n_nt;
                    nt = tile - mt * p.n_nt;
                    if (reload) load_rows(mt);
                }
                for (int mi = 0; mi < 4; ++mi)
                    relu2_store(r, wg, wave, mt_t * (RM / 16) + mi, nt_t * (WBN / 64) + wave, nt_t, false, "gemm_relu2_rt output");
                for (int lane = 0; lane < 64 && wave == 0; ++lane)
                    if (mt_t * (RM / 16) + (lane >> 4) < p.MF)
                        r.store(SXO, sxo_index(mt_t * RM + lane, p.n_nt, nt_t) * 4, 4, wg, wave, lane, "gemm_relu2_rt row scales");
                if (more)
                    for (int j = 1; j < RDEPTH; ++j) ldw(nt, j);   // the next tile's k-steps 1..3
            }
        }
    }
}

void replay_relu2_small(replay & r) {
    const gemm_plan & p = r.pl;
    for (int wg = 0; wg < p.grid && !r.status; ++wg) {
        const int mt = wg / p.n_nt, nt = wg - mt * p.n_nt;
        const int fr0 = mt * SDT;
        replay_sw_fill(r, wg, 256, nt * WBN, WBN, (size_t) SNB_MAX * WBN);
        for (int wave = 0; wave < 4; ++wave) {
            const int nr0 = w_frag(nt, WBN, 4 * wave);
            replay_small_piece(r, wg, wave, mt, nr0, 4, true);
            for (int j = 0; j < SDT; ++j) {
                const int kf = nt * (WBN / 64) + wave;
                relu2_store(r, wg, wave, fr0 + j, kf, nt, wave == 0, "gemm_relu2_small output");
            }
        }
    }
}

} // namespace

extern "C" int gemm_replay(int T, int n_in, int n_out, int mode, int n_seg, const int * seg_cols, int cus, int * kind,
                           long long * accesses, char * err, int err_len) {
    replay r;
    r.err = err;
    r.err_len = err_len;
    if (err_len > 0) err[0] = 0;
    const bool sums = mode == 2, relu2 = mode == 3 || mode == 4, res = mode == 1;
    if (T <= 0 || n_in <= 0 || n_in % 32 != 0 || n_out <= 0 || !plan_gemm(T, n_in, n_out, sums, relu2, cus, r.pl)) {
        snprintf(err, (size_t) err_len, "no plan for T=%d n_in=%d n_out=%d", T, n_in, n_out);
        return 3;
    }
    const gemm_plan & p = r.pl;
    *kind = (int) p.kind;
    if (n_seg > 0 && (p.kind != GEMM_K256 && p.kind != GEMM_SMALL && p.kind != GEMM_FSK)) {
        snprintf(err, (size_t) err_len, "split output on kernel %d", (int) p.kind);
        return 3;
    }
    const size_t MP = (size_t) p.MF * 16;
    r.bytes[A] = MP * p.KS * 64;                       // nxg_qact_q_bytes(T, n_in)
    r.bytes[SX] = MP * p.n_blk * sizeof(float);        // nxg_qact_sx_bytes(T, n_in)
    r.bytes[W] = (size_t) p.NP * p.KS * 64;            // the weight's fragment rows
    r.bytes[SW] = (size_t) p.n_blk * p.NP * sizeof(float);
    r.bytes[RES] = res ? (size_t) T * n_out * sizeof(float) : 0;
    r.bytes[OUT] = (!sums && !relu2 && n_seg == 0) ? (size_t) T * n_out * sizeof(float) : 0;
    r.bytes[SUMS] = sums ? (size_t) p.n_blk * T * n_out * sizeof(int32_t) : 0;
    r.bytes[QO] = relu2 ? MP * p.KSo * 64 : 0;         // nxg_qact_q_bytes(T, n_out)
    r.bytes[SXO] = relu2 ? MP * (size_t) ceil_div(n_out, BLK) * sizeof(float) : 0;   // nxg_qact_sx_bytes(T, n_out)
    // mode 4: the row-tile kernel of nxg_linear_f32_relu2_q8_rows reading the fp32 rows [T][n_in]
    // itself, replayed at every shape that plans it (the library launches it only from
    // NXG_RELU2_FQ_MIN_TILES_PER_WG tiles per workgroup); other kernels run on a qact
    r.xf = mode == 4 && p.kind == GEMM_RELU2_RT;
    r.bytes[XF] = r.xf ? (size_t) T * n_in * sizeof(float) : 0;
    if (r.xf) r.bytes[A] = r.bytes[SX] = 0;
    r.n_seg = n_seg;
    for (int k = 0, end = 0; k < 4; ++k) {
        if (k < n_seg) {
            end += seg_cols[k];
            r.bytes[SEG0 + k] = (size_t) T * seg_cols[k] * sizeof(float);
        }
        r.seg_end[k] = end;
    }
    for (int b : { (int) OUT, (int) SEG0, (int) SEG1, (int) SEG2, (int) SEG3, (int) SUMS, (int) QO, (int) SXO }) r.track(b);

    switch (p.kind) {
    case GEMM_K256: replay_k256(r, res); break;
    case GEMM_GENERAL: replay_general(r, res, false); break;
    case GEMM_SUMS: replay_general(r, false, true); break;
    case GEMM_SMALL: replay_small(r, res); break;
    case GEMM_FSK: replay_fsk(r, res); break;
    case GEMM_RELU2_Q8: replay_relu2_q8(r); break;
    case GEMM_RELU2_SMALL: replay_relu2_small(r); break;
    case GEMM_RELU2_RT: replay_relu2_rt(r); break;
    }
    if (!r.status) {
        if (sums) r.covered(SUMS, r.bytes[SUMS] / 4, (size_t) n_out);
        else if (relu2) {
            r.covered(QO, r.bytes[QO] / 4, 16);
            r.covered(SXO, r.bytes[SXO] / 4, 4);
        } else if (n_seg == 0) r.covered(OUT, r.bytes[OUT] / 4, (size_t) n_out);
        else
            for (int k = 0; k < n_seg; ++k) r.covered(SEG0 + k, r.bytes[SEG0 + k] / 4, (size_t) seg_cols[k]);
    }
    *accesses = r.accesses;
    return r.status;
}
