// nxg_gemm_plan.h -- launch plan and address arithmetic of the int8 GEMMs.
//
// One definition, two users: the gfx950 kernels and their launcher in nxg_linear.hip,
// and a host replay of every global load and store those kernels issue, which checks
// each one against the bytes its buffer holds (tests/gemm_replay.cpp). Everything here
// is plain integer arithmetic; under hipcc the functions are __host__ __device__.
//
// Buffers, as the C ABI sizes them (include/nxg_linear.h):
//   a    activation fragment tiles, MF x KS fragments of FRAG bytes (MF = ceil(T / 16))
//   sx   activation scales, [MF * 4][n_blk][4] floats ([t / 4][B][t % 4])
//   w    weight fragment tiles, NP / 16 x KS fragments (NP = n_out rounded up to WBN)
//   sw   weight scales, [n_blk][NP] floats
//   res, out  [T][N] floats; a split output writes segment k as a dense [T][cols_k] array
//   qo, sxo   the relu^2 output as the next linear's activation: MF x KSo fragments,
//             [MF * 4][ceil(N / 256)][4] floats
#pragma once

#include <cstddef>
#include <cstdint>

#include "nxg_linear.h"

#if defined(__HIPCC__)
#  define NXG_HD __host__ __device__ __forceinline__
#else
#  define NXG_HD inline
#endif

#ifndef NXG_WG_PER_CU
#define NXG_WG_PER_CU 2                    // persistent GEMM workgroups per CU (0: one workgroup per tile)
#endif
#ifndef NXG_SMALL_MAX_WAVES_PER_CU
#define NXG_SMALL_MAX_WAVES_PER_CU 4       // gemm_small while its waves number at most this many per CU
#endif
#ifndef NXG_RELU2_SMALL_MAX_WAVES_PER_CU
#define NXG_RELU2_SMALL_MAX_WAVES_PER_CU 4 // gemm_relu2_small likewise (its workgroups: one per CU)
#endif
#ifndef NXG_RELU2_RT
#define NXG_RELU2_RT 1                     // relu^2 -> int8 with n_in 256 or 1024 on gemm_relu2_rt (0: gemm_relu2_q8)
#endif
#ifndef NXG_FSK_MAX_TILES_PER_CU
#define NXG_FSK_MAX_TILES_PER_CU 2         // gemm_fsk while its 64-row tiles number at most this many per CU (0: never)
#endif
#ifndef NXG_RELU2_FQ_MIN_TILES_PER_WG
#define NXG_RELU2_FQ_MIN_TILES_PER_WG 4    // fp32 input rows quantized inside gemm_relu2_rt from this many tiles per workgroup
#endif
#ifndef NXG_SMALL_FN
#define NXG_SMALL_FN 0                     // weight fragments per wave of gemm_small (0: chosen per launch)
#endif
#ifndef NXG_SMALL_DEPTH4
#define NXG_SMALL_DEPTH4 4                 // k-steps in flight per wave of the 32 x 64 pieces
#endif

namespace nxg_gemm {

constexpr int BLK = NXG_BLOCK;   // inputs per scale block
constexpr int FRAG = 1024;       // bytes of one 16-row x 64-input fragment
constexpr int BM = 128;          // GEMM workgroup tile: rows (tokens)
constexpr int BN = 128;          //                      columns (output features)
constexpr int NTHREADS = 256;    // 4 waves, 2 x 2, each 64 x 64
constexpr int WBN = 256;         // relu^2 -> int8 GEMM tile columns: one 256-input block of the next linear
constexpr int WTHREADS = 512;    // relu^2 -> int8 GEMM: 8 waves, 2 x 4, each 64 x 64
constexpr int N_XCD = 8;         // MI355X: 8 XCDs, workgroups dispatched round-robin
constexpr int SDT = 2;           // few-row GEMMs: activation fragments (16 tokens each) per wave
constexpr int SNB_MAX = 16;      // few-row GEMMs: 256-input blocks (n_in <= 4096), sw kept in LDS
constexpr int FSK_NB = 9;        // few-row split-block GEMM: 256-input blocks (one wave each, n_in <= 2304)

// LDS ring of gemm_kernel / gemm_k256: four slots of one 64-input k-step each, 8 A
// fragments, 8 B fragments, then 1 KiB for a block's scales (sx of the tile's 128 rows
// as 32 groups of 4, then sw of its 128 columns).
constexpr int SLOT_AB = (BM / 16 + BN / 16) * FRAG;   // 16 KiB
constexpr int SLOT = SLOT_AB + 1024;
constexpr int STAGE_BYTES = 4352;                      // a wave's output staging: 16 rows x 272 bytes
constexpr int STAGE_PITCH = 68;                        // floats per staging row
// gemm_relu2_q8's ring: 8 A + 16 B fragments per slot; its scales have an area of their own.
constexpr int WSLOT = (BM / 16 + WBN / 16) * FRAG;    // 24 KiB
constexpr int WSCALE = 4 * (BM + WBN);                 // bytes: sx of 128 rows, then sw of 256 columns

// gemm_relu2_rt: 64 x 256 tiles, 4 waves of 64 x 64, two workgroups per CU. The activation
// row tile (64 rows x n_in, n_in <= 1024) stays in LDS while the workgroup walks its column
// tiles; weights go straight to registers. LDS per workgroup: the row tile, two tiles'
// scales (sx of 64 rows as 16 groups x n_blk x 4, then sw of 256 columns per block) and
// two tiles' row maxima.
constexpr int RM = 64;                                  // rows per tile
constexpr int RNB_MAX = 4;                              // 256-input blocks the row tile holds
constexpr int RTHREADS = 256;
constexpr int RDEPTH = 4;                               // k-steps of weights in flight per wave
constexpr int RSX_BYTES = 16 * RNB_MAX * 16;            // sx area: 1 KiB
constexpr int RSCALE = RSX_BYTES + RNB_MAX * WBN * 4;   // bytes per tile's scales: 5 KiB

// Few-row GEMMs: k-steps in flight per wave: two 256-input blocks for 32 x 32 pieces (fn
// 2), one for 32 x 64 pieces (whose 6 fragments per k-step would otherwise need more
// than 256 registers).
constexpr int small_depth(int fn) { return fn == 2 ? 8 : NXG_SMALL_DEPTH4; }

NXG_HD int ceil_div(int a, int b) { return (a + b - 1) / b; }
NXG_HD int imin(int a, int b) { return a < b ? a : b; }

// Tiles of one workgroup. Workgroups are dispatched to the 8 XCDs round-robin
// (workgroup w runs on XCD w % 8). Each XCD owns a contiguous range of tile
// numbers, dealt out round-robin to its workgroups; tiles are numbered with the
// column tile fastest, so the workgroups of an XCD work on neighbouring row tiles
// at the same time and share them (and the whole weight) in that XCD's L2.
struct tile_walk {
    int first, stride, count;
    NXG_HD tile_walk(int wg, int n_wg, int G) {
        const int xcd = wg % N_XCD, idx = wg / N_XCD;
        const int per = n_wg / N_XCD + (xcd < n_wg % N_XCD ? 1 : 0);     // workgroups on this XCD
        const int q = G / N_XCD, r = G % N_XCD;
        const int lo = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
        const int n = q + (xcd < r ? 1 : 0);                              // tiles of this XCD
        first = lo + idx;
        stride = per;
        count = idx < n ? (n - idx + per - 1) / per : 0;
    }
    NXG_HD int tile(int i) const { return first + i * stride; }
    // Tile i, or past the walk's end its last tile: the prefetch of the k-steps after the
    // last tile re-reads that tile, so that the loads per k-step stay constant.
    NXG_HD int tile_clamped(int i) const { return tile(imin(i, count - 1)); }
};

// gemm_relu2_rt: each XCD owns a contiguous range of tile numbers (as tile_walk), split
// into near-equal contiguous pieces, one per workgroup of the XCD. Tiles are numbered with
// the column tile fastest, so a workgroup walks the column tiles of a row tile in turn and
// loads each activation row tile into LDS once; an XCD's workgroups share the weight in L2.
struct tile_span {
    int first, count;
    NXG_HD tile_span(int wg, int n_wg, int G) {
        const int xcd = wg % N_XCD, idx = wg / N_XCD;
        const int per = n_wg / N_XCD + (xcd < n_wg % N_XCD ? 1 : 0);     // workgroups on this XCD
        const int q = G / N_XCD, r = G % N_XCD;
        const int lo = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
        const int n = q + (xcd < r ? 1 : 0);                              // tiles of this XCD
        const long long a = (long long) n * idx / per, b = (long long) n * (idx + 1) / per;
        first = lo + (int) a;
        count = (int) (b - a);
    }
};

// --- operand addresses ------------------------------------------------------------

// Activation fragment row i (0 .. BM/16 - 1) of row tile mt. Rows past the last fragment
// row re-read it: their outputs are never stored, and every wave keeps issuing the same
// number of loads per k-step, which the constant wait counts rely on.
NXG_HD int a_frag(int mt, int i, int MF) { return imin(mt * (BM / 16) + i, MF - 1); }
// Weight fragment row i of column tile nt of `width` columns. NP is a multiple of WBN, so
// every fragment row of a tile exists.
NXG_HD int w_frag(int nt, int width, int i) { return nt * (width / 16) + i; }
// gemm_relu2_rt: activation fragment row i (0 .. 3) of 64-row tile mt, clamped likewise.
NXG_HD int a_frag_rt(int mt, int i, int MF) { return imin(mt * (RM / 16) + i, MF - 1); }
// gemm_relu2_rt quantizing fp32 rows: the input row that row r (0 .. 63) of row tile mt reads,
// the last row for rows past T (quantized as zeros, never stored).
NXG_HD int rt_x_row(int mt, int r, int T) { return imin(mt * RM + r, T - 1); }
// gemm_fsk: activation fragment row i (0 .. 3) of 64-row tile mt, clamped likewise; float
// index of the 4 sx of row group g (0 .. 15) of 64-row tile mt, block B, groups past the last
// one re-reading it.
NXG_HD int fsk_a_frag(int mt, int i, int MF) { return imin(mt * 4 + i, MF - 1); }
NXG_HD size_t fsk_sx_group(int mt, int g, int MF, int n_blk, int B) {
    return ((size_t) imin(mt * 16 + g, MF * 4 - 1) * n_blk + B) * 4;
}
// Few-row GEMMs: activation fragment row j (0 .. SDT - 1) of piece row mt, clamped likewise.
NXG_HD int small_a_frag(int mt, int j, int MF) { return imin(mt * SDT + j, MF - 1); }
// Byte offset of lane `lane`'s 16 bytes of k-step ks of fragment row r.
NXG_HD size_t frag_byte(int r, int KS, int ks, int lane) {
    return ((size_t) r * KS + ks) * FRAG + (size_t) lane * 16;
}

// --- scales -----------------------------------------------------------------------

// Float index of sx[t][B] in the [t / 4][B][t % 4] layout.
NXG_HD size_t sx_index(int t, int n_blk, int B) {
    return ((size_t) (t >> 2) * n_blk + B) * 4 + (t & 3);
}
// Float index of the 4 sx of row group g (0 .. BM/4 - 1) of row tile mt, block B; groups
// past the last one re-read it.
NXG_HD size_t sx_group_index(int mt, int g, int MF, int n_blk, int B) {
    return ((size_t) imin(mt * (BM / 4) + g, MF * 4 - 1) * n_blk + B) * 4;
}
// gemm_relu2_rt: float index of the 4 sx of row group g (0 .. 15) of 64-row tile mt, block
// B; groups past the last one re-read it.
NXG_HD size_t sx_group_index_rt(int mt, int g, int MF, int n_blk, int B) {
    return ((size_t) imin(mt * (RM / 4) + g, MF * 4 - 1) * n_blk + B) * 4;
}
// Float index of sw[B][n].
NXG_HD size_t sw_index(int B, int NP, int n) { return (size_t) B * NP + n; }

// --- outputs ----------------------------------------------------------------------

// Residual reads of rows and columns past the output: the last row, the last 4 columns
// (never stored).
NXG_HD int clamp_row(int t, int T) { return imin(t, T - 1); }
NXG_HD int clamp_col4(int n, int N) { return imin(n, N - 4); }

// Where output column n goes: column `col` of rows `ld` floats long at `base`, which is
// `out` without a split and segment k's buffer seg[k] with one. Written for any handle
// type P (a kernel's pointers, a host replay's buffer numbers); the boundaries and
// buffers are selected with constant indices, so that a kernel keeps its arguments in
// registers rather than indexing them.
template <typename P>
struct out_col {
    P base;
    int col, ld;
};
template <typename P>
NXG_HD out_col<P> out_col_of(int n, int N, int n_seg, const int (&seg_end)[4], P out, const P (&seg)[4]) {
    out_col<P> m{ out, n, N };
    if (n_seg > 0) {
        int lo = 0, hi = seg_end[0];
        P b = seg[0];
        if (n_seg > 1 && n >= seg_end[0]) { b = seg[1]; lo = seg_end[0]; hi = seg_end[1]; }
        if (n_seg > 2 && n >= seg_end[1]) { b = seg[2]; lo = seg_end[1]; hi = seg_end[2]; }
        if (n_seg > 3 && n >= seg_end[2]) { b = seg[3]; lo = seg_end[2]; hi = seg_end[3]; }
        m = out_col<P>{ b, n - lo, hi - lo };
    }
    return m;
}

// Byte offset in qo of lane `lane`'s 16 bytes of fragment (rf, kf); float index of the
// scale of row t, block nt, in sxo.
NXG_HD size_t qo_byte(int rf, int KSo, int kf, int lane) { return frag_byte(rf, KSo, kf, lane); }
NXG_HD size_t sxo_index(int t, int n_nt, int nt) { return sx_index(t, n_nt, nt); }

// --- the k-step schedule of gemm_k256 and gemm_relu2_q8 -----------------------------

// k-step g of a workgroup's walk lives in ring slot g % 4 and is read into registers one
// step ahead. At step s (0..3) of block B of walk position it, after that step's barrier,
// each wave loads the k-step four ahead into slot s: k-step 4B + 4 + s of the same tile,
// or, in the tile's last block (last), k-step s of the next walk position (clamped to the
// last tile by the caller). With stage3 (gemm_k256, whose output is staged in slot 3)
// the last step loads nothing (pos < 0): the next tile's start loads its k-step 3.
struct ring_load {
    int pos, ks, slot;
};
NXG_HD ring_load ring_prefetch(int it, int B, int s, bool last, bool stage3) {
    if (!last) return ring_load{ it, 4 * B + 4 + s, s };
    if (stage3 && s == 3) return ring_load{ -1, 0, 3 };
    return ring_load{ it + 1, s, s };
}

// --- the launch plan ----------------------------------------------------------------

enum gemm_kind : int {
    GEMM_GENERAL = 0,    // gemm_kernel: fp32 out, one tile per workgroup unless n_in % 256 == 0
    GEMM_SUMS = 1,       // gemm_kernel: per-block int32 sums
    GEMM_K256 = 2,       // gemm_k256: fp32 out, n_in % 256 == 0, N % 4 == 0, persistent
    GEMM_SMALL = 3,      // gemm_small: few rows, one wave per 32 x 16fn piece
    GEMM_RELU2_Q8 = 4,   // gemm_relu2_q8: relu^2 -> int8, 128 x 256 tiles, one workgroup per CU
    GEMM_RELU2_SMALL = 5,// gemm_relu2_small: relu^2 -> int8 for few rows
    GEMM_RELU2_RT = 6,   // gemm_relu2_rt: relu^2 -> int8, 64 x 256 tiles, row tile in LDS, n_in 256 or 1024
    GEMM_FSK = 7         // gemm_fsk: few rows, one 64 x fn tile per workgroup, one wave per 256-input block
};

struct gemm_plan {
    gemm_kind kind;
    bool k256;           // n_in % 256 == 0
    int fn;              // gemm_small: weight fragments per wave; gemm_fsk: tile columns (64 or 32)
    int grid, block;     // workgroups, threads per workgroup
    int T, N, NP, KS, n_blk, MF, n_mt, n_nt, G, KSo;
};

// Workgroups of a persistent launch: `want`, but at least one per XCD while there are
// tiles for it -- the walk gives each XCD's workgroups a fixed range of tiles, so an XCD
// without a workgroup would leave its range undone.
inline int persistent_grid(long long G, long long want) {
    const long long lo = G < N_XCD ? G : N_XCD;
    const long long g = G < want ? G : want;
    return (int) (g > lo ? g : lo);
}

// The kernel and grid for a GEMM of T rows, n_in inputs and n_out outputs on a device of
// `cus` compute units: per-block sums (sums), relu^2 -> int8 output (relu2), else fp32
// rows. Returns false when the tile count overflows. The callers check the shape rules
// (n_in % 32, and for relu2 and split outputs n_in % 256 and the column rules) first.
inline bool plan_gemm(int T, int n_in, int n_out, bool sums, bool relu2, int cus, gemm_plan & pl) {
    pl = gemm_plan{};
    pl.T = T;
    pl.N = n_out;
    pl.NP = ceil_div(n_out, WBN) * WBN;
    pl.KS = ceil_div(n_in, 64);
    pl.n_blk = ceil_div(n_in, BLK);
    pl.KSo = ceil_div(n_out, 64);
    pl.MF = ceil_div(T, 16);
    pl.n_mt = ceil_div(T, BM);
    pl.k256 = pl.KS % 4 == 0;
    if (relu2) {
        pl.n_nt = ceil_div(pl.N, WBN);
        const long long G = (long long) pl.n_mt * pl.n_nt;
        if (G > INT32_MAX / 2) return false;
        const long long G_small = (long long) ceil_div(pl.MF, SDT) * pl.n_nt;   // 4 waves each
        if (pl.n_blk <= SNB_MAX && 4 * G_small <= (long long) NXG_RELU2_SMALL_MAX_WAVES_PER_CU * cus) {
            pl.kind = GEMM_RELU2_SMALL;
            pl.n_mt = ceil_div(pl.MF, SDT);
            pl.G = (int) G_small;
            pl.grid = pl.G;
            pl.block = 256;
            return true;
        }
        if ((pl.n_blk == 1 || pl.n_blk == RNB_MAX) && NXG_RELU2_RT) {
            const long long G_rt = (long long) ceil_div(T, RM) * pl.n_nt;
            pl.kind = GEMM_RELU2_RT;
            pl.n_mt = ceil_div(T, RM);
            pl.G = (int) G_rt;
            pl.grid = persistent_grid(G_rt, 2LL * cus);
            pl.block = RTHREADS;
            return true;
        }
        pl.kind = GEMM_RELU2_Q8;
        pl.G = (int) G;
        pl.grid = persistent_grid(G, cus);
        pl.block = WTHREADS;
        return true;
    }
    pl.n_nt = ceil_div(pl.N, BN);
    const long long G = (long long) pl.n_mt * pl.n_nt;
    if (G > INT32_MAX / 2) return false;
    pl.G = (int) G;
    // Few rows with n_in % 256 == 0: one 64 x 64 tile per workgroup (64 x 32 from 5 blocks),
    // one wave per 256-input block, while the tiles number at most NXG_FSK_MAX_TILES_PER_CU
    // per CU.
    if (!sums && pl.k256 && pl.N % 4 == 0 && pl.n_blk <= FSK_NB) {
        const int tn = pl.n_blk <= 4 ? 64 : 32;
        const long long G_fsk = (long long) ceil_div(T, 64) * ceil_div(pl.N, tn);
        if (G_fsk <= (long long) NXG_FSK_MAX_TILES_PER_CU * cus) {
            pl.kind = GEMM_FSK;
            pl.fn = tn;
            pl.n_mt = ceil_div(T, 64);
            pl.n_nt = ceil_div(pl.N, tn);
            pl.G = (int) G_fsk;
            pl.grid = pl.G;
            pl.block = 64 * (pl.n_blk > 4 ? pl.n_blk : 4);
            return true;
        }
    }
    // Few rows, one wave per piece: 32 x 32 pieces while they number at most
    // NXG_SMALL_MAX_WAVES_PER_CU per CU, else 32 x 64 pieces (fewer bytes per output
    // through each CU) while those do; beyond that the 128 x 128 tiles, which read each
    // operand fragment once per tile. (Measured on MI355X at 128..4096 rows.)
    const long long W2 = (long long) ceil_div(pl.MF, SDT) * ceil_div(pl.N, 32);
    const long long W4 = (long long) ceil_div(pl.MF, SDT) * ceil_div(pl.N, 64);
    const long long w_max = (long long) NXG_SMALL_MAX_WAVES_PER_CU * cus;
    const int fn = NXG_SMALL_FN ? NXG_SMALL_FN : (W2 <= w_max ? 2 : 4);
    const long long n_waves = fn == 2 ? W2 : W4;
    if (!sums && pl.N % 4 == 0 && pl.n_blk <= SNB_MAX && n_waves <= w_max) {
        pl.kind = GEMM_SMALL;
        pl.fn = fn;
        pl.n_mt = ceil_div(pl.MF, SDT);
        pl.n_nt = ceil_div(pl.N, 16 * fn);
        pl.G = (int) n_waves;
        pl.grid = pl.G;
        pl.block = 64;
        return true;
    }
    // n_in % 256 == 0: persistent workgroups, NXG_WG_PER_CU per CU (the LDS ring needs
    // 68 KiB of the 160); otherwise one workgroup per tile.
    const bool persistent = pl.k256 && NXG_WG_PER_CU > 0;
    pl.grid = persistent ? persistent_grid(G, (long long) NXG_WG_PER_CU * cus) : (int) G;
    pl.block = NTHREADS;
    pl.kind = sums ? GEMM_SUMS : (persistent && pl.N % 4 == 0) ? GEMM_K256 : GEMM_GENERAL;
    return true;
}

// nxg_linear_f32_relu2_q8: whether the row-tile kernel quantizes the fp32 input rows itself.
// Each workgroup then reads its row tiles' fp32 rows (4 bytes per input instead of 1) with
// no other work to hide them under; from about four tiles per workgroup the quantize launch
// this saves outweighs that (measured on MI355X, one encoder forward's linear path with the
// 18 c_fc GEMMs of 1024 -> 2304: 4.5 tiles per workgroup at 16,384 rows 5.51 -> 5.46 ms,
// 18 tiles at 65,536 rows 18.45 -> 18.01 ms; 2.25 tiles at 8,192 rows 3.43 -> 3.49 ms).
// Below it, the rows are quantized into the workspace first.
NXG_HD bool relu2_fuses_quant(const gemm_plan & pl) {
    return pl.kind == GEMM_RELU2_RT && (long long) pl.G >= (long long) NXG_RELU2_FQ_MIN_TILES_PER_WG * pl.grid;
}

} // namespace nxg_gemm
