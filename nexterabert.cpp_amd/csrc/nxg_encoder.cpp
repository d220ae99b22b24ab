// nxg_encoder.cpp -- the NexteraBERT encoder on one GPU: a model context loaded from a GGUF
// file and the forward pass of builder::encoder (src/nexterabert.cpp:1270-1292), launched
// in graph order on one stream over libnxg's kernels. Host code only.
//
// Device memory: the int8 weights in MFMA tiles (nxg_weight), the fp32 tensors the row ops
// read (norm gains, DyT curves, conv taps one row per tap, the embedding tables decoded to
// fp32), the RoPE tables, and one work area sized for the largest batch seen so far: the
// residual stream (two buffers, each c_proj reads one and writes the other), eight [T][C]
// and four [T][KV] fp32 buffers the mixers share, two [T][rank] ones for SnowLily, the
// qacts of the int8 linears, the batch's ids, offsets and per-layer attention scales.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "nxg_encoder.h"
#include "nxg_gguf.h"
#include "nxg_internal.h"

namespace {

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
    return fail(e == hipErrorOutOfMemory ? NXG_ENOMEM : NXG_EDEVICE, "encoder: %s: %s", what, hipGetErrorString(e));
}

#define NXG_TRY(x)                          \
    do {                                    \
        const int32_t rc_ = (x);            \
        if (rc_ != NXG_OK) return rc_;      \
    } while (0)

#define NXG_HIP(x, what)                                  \
    do {                                                  \
        const hipError_t e_ = (x);                        \
        if (e_ != hipSuccess) return hip_fail(e_, what);  \
    } while (0)

// One launch of the forward pass, then the profiler's mark for its kind (nxg_encoder_profile).
#define NXG_OP(kind, x)                     \
    do {                                    \
        NXG_TRY(x);                         \
        NXG_TRY(mark(kind, s));             \
    } while (0)

// Frees device memory where no error can be reported (destructors, replaced buffers).
void release(void * p) {
    if (p) (void) hipFree(p);
}

enum mixer { MIX_LILY, MIX_SWA, MIX_ATTN, MIX_HRA };

// nextera_load's hyperparameters (src/nexterabert.cpp:213-228, read at :1574-1626).
struct hparams {
    int32_t n_vocab = 0, n_embd = 0, n_layer = 0, n_inter = 0;
    int32_t n_head = 0, n_kv_head = 0, head_dim = 0;
    int32_t lily_rank = 0, lily_kernel = 0, hra_block = 0, swa_window = 0, ntk_train_len = 0;
    float rope_base = 100000.0f, swa_rope_base = 10000.0f, ssmax_base = 0.1f, rms_eps = 1e-8f, ln_eps = 1e-5f;
    int32_t ssmax = 2;                         // nxg_attention_scales' modes: 0 none, 1 ssmax, 2 sssmax
    std::vector<mixer> block_types;
    int32_t n_types = 0;                       // rows of the segment embedding, 0: none
};

// Metadata reads with nextera_load's defaults (kv_u32 / kv_f32 / kv_str, :1434-1455).
struct kv_reader {
    const nxg_gguf * g;
    std::string bad;                           // first required or unreadable key
    int64_t u32(const char * key, int64_t def, bool required = false) {
        const int64_t id = nxg_gguf_find_key(g, key);
        int64_t v = def;
        if (id < 0) {
            if (required && bad.empty()) bad = key;
        } else if (nxg_gguf_get_i64(g, id, &v) != NXG_OK && bad.empty()) {
            bad = key;
        }
        return v;
    }
    float f32(const char * key, float def) {
        const int64_t id = nxg_gguf_find_key(g, key);
        double v = def;
        if (id >= 0 && nxg_gguf_get_f64(g, id, &v) != NXG_OK && bad.empty()) bad = key;
        return (float) v;
    }
    std::string str(const char * key, const char * def) {
        const int64_t id = nxg_gguf_find_key(g, key);
        const char * s = nullptr;
        uint64_t n = 0;
        if (id < 0 || nxg_gguf_get_str(g, id, &s, &n) != NXG_OK) return def;
        return std::string(s, (size_t) n);
    }
};

bool ends_with(const std::string & s, const char * suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

struct qact {
    int8_t * q = nullptr;
    float * sx = nullptr;
};

struct f32_tensor {
    float * dev = nullptr;
    int64_t n = 0;            // elements
    int32_t rows = 1, cols = 0;   // as the op reads it ([k][C] for conv taps)
};

struct rope_dev {
    float base = 0.0f;
    int32_t n_pos = 0, cap = 0;
    float * cos = nullptr;
    float * sin = nullptr;
};

} // namespace

struct nxg_encoder {
    hparams hp;
    int32_t act_max = 127;
    int32_t n_layers_run = -1;                 // nextera_debug_set_layers
    std::unordered_map<std::string, nxg_weight *> i8;
    // projections of one input fused along n_out (key: group name), launched as one split GEMM
    struct fused_w {
        nxg_weight * w = nullptr;
        std::vector<int32_t> cols;
    };
    std::unordered_map<std::string, fused_w> fused;
    std::unordered_map<std::string, f32_tensor> f32;
    std::unordered_map<std::string, float> scalar;   // 1-element tensors (scalable_factor.s / .b)
    size_t weight_bytes = 0;
    hipStream_t stream = nullptr;
    double last_ms = 0.0;

    // work area, sized for cap_T rows, cap_TB block rows, cap_seqs sequences and cap_keys tokens
    // in the longest one
    void * work = nullptr;
    size_t work_bytes = 0;
    int64_t work_limit = 0;                    // nxg_encoder_set_work_limit (0: none)
    int64_t cap_T = -1, cap_TB = -1, cap_seqs = -1, cap_keys = -1;
    float * x[2] = {};
    float * F[8] = {};                         // [T][C]
    float * K[4] = {};                         // [T][KV]
    float * Z[2] = {};                         // [T][rank]
    float * U = nullptr;                       // [T][n_inter], only when c_fc cannot quantize its own output
    float * hidden = nullptr;                  // [T][C] output rows (host API)
    float * pooled = nullptr;                  // [n_seqs][C]
    qact qa_h, qa_y, qa_g, qa_I, qa_R, qa_hb;
    int32_t * ids = nullptr, * types = nullptr, * cu = nullptr, * cub = nullptr;
    float * scales = nullptr;                  // [n_layer][n_seqs]
    void * attn_ws = nullptr;                  // nxg_attention_ws's scores of long documents
    int64_t attn_ws_bytes = 0;

    // the batch layout the device buffers hold (prepare_batch, :1341-1371)
    std::vector<int32_t> lengths, cu_h, cub_h;
    std::vector<float> scales_h;
    int32_t T = 0, TB = 0, max_len = 0, max_blocks = 0;
    rope_dev rope[2];                          // [0]: full attention and HRA, [1]: swa
    bool fuse_mlp = true;
    int32_t n_int8 = 0;                        // int8 linears of the file's encoder, before fusing

    // Device time per kind of launch (the reference's per-op-kind profiler, src/nexterabert.cpp:
    // 262-283): an event after every launch of a pass, on the launching stream; the interval
    // that ends at an event is the time of the launch before it (its dispatch gap included).
    struct profiler {
        bool enabled = false;
        std::vector<hipEvent_t> ev;            // reused from pass to pass
        std::vector<int> kind;                 // kind[i]: the launch ending at ev[i]; ev[0] opens the pass
        size_t used = 0;
        double ms[NXG_PROF_COUNT] = {};
        double device_ms = 0.0, wall_ms = 0.0;
        int64_t passes = 0;
    } prof;

    ~nxg_encoder();
    const float * w(const std::string & name) const { return f32.at(name).dev; }
    int32_t ensure_work(int64_t T, int64_t TB, int64_t n_seqs, int64_t n_keys);
    int32_t prepare(const int32_t * lengths, int32_t n_seqs, hipStream_t s);
    int32_t run(const int32_t * ids, const int32_t * types, int32_t n_seqs, float * hidden, float * pooled,
                int32_t normalize, hipStream_t s);
    // the pieces of builder (src/nexterabert.cpp:1080-1268)
    int32_t linear(const std::string & name, const qact & in, int32_t rows, const float * res, float * out, hipStream_t s);
    // the projections `names` of `in` (fused group `key` when it exists) into outs
    int32_t project(const std::string & key, const std::vector<std::string> & names, const qact & in, int32_t rows,
                    std::initializer_list<float *> outs, hipStream_t s);
    int32_t attention(const std::string & pre, const qact & h, int32_t rows, const int32_t * cu_dev, int32_t n_seqs,
                      const rope_dev & rope, int32_t half, const float * scale, int32_t max_keys, float * out,
                      hipStream_t s);
    int32_t gated_out(const std::string & pre, const float * y, const float * z, const float * x_in, float * x_out,
                      int32_t n_seqs, hipStream_t s);
    int32_t mark(int kind, hipStream_t s);
    // waits for the last pass's events and adds their intervals (wall_ms: the caller's clock, or < 0)
    int32_t collect(double wall_ms);
};

nxg_encoder::~nxg_encoder() {
    for (auto & kv : i8) nxg_weight_destroy(kv.second);
    for (auto & kv : fused) nxg_weight_destroy(kv.second.w);
    for (auto & kv : f32) release(kv.second.dev);
    for (rope_dev & r : rope) {
        release(r.cos);
        release(r.sin);
    }
    release(work);
    for (hipEvent_t ev : prof.ev) (void) hipEventDestroy(ev);
    if (stream) (void) hipStreamDestroy(stream);
}

int32_t nxg_encoder::mark(int k, hipStream_t s) {
    if (!prof.enabled) return NXG_OK;
    if (prof.used == prof.ev.size()) {
        hipEvent_t ev = nullptr;
        NXG_HIP(hipEventCreate(&ev), "hipEventCreate(profile)");
        prof.ev.push_back(ev);
        prof.kind.push_back(0);
    }
    NXG_HIP(hipEventRecord(prof.ev[prof.used], s), "hipEventRecord(profile)");
    prof.kind[prof.used++] = k;
    return NXG_OK;
}

int32_t nxg_encoder::collect(double wall_ms) {
    if (!prof.enabled || prof.used < 2) return NXG_OK;
    NXG_HIP(hipEventSynchronize(prof.ev[prof.used - 1]), "hipEventSynchronize(profile)");
    double pass = 0.0;
    for (size_t i = 1; i < prof.used; ++i) {
        float ms = 0.0f;
        NXG_HIP(hipEventElapsedTime(&ms, prof.ev[i - 1], prof.ev[i]), "hipEventElapsedTime(profile)");
        prof.ms[prof.kind[i]] += ms;
        pass += ms;
    }
    prof.device_ms += pass;
    prof.wall_ms += wall_ms >= 0.0 ? wall_ms : pass;
    prof.passes += 1;
    prof.used = 0;
    return NXG_OK;
}

namespace {

size_t align256(size_t n) { return (n + 255) & ~(size_t) 255; }

// Carves the work area: a first pass with base null sizes it, a second assigns pointers.
struct carver {
    char * base;
    size_t off = 0;
    template <typename P>
    void take(P *& p, size_t bytes) {
        p = base ? reinterpret_cast<P *>(base + off) : nullptr;
        off += align256(std::max<size_t>(bytes, 1));
    }
};

} // namespace

int32_t nxg_encoder::ensure_work(int64_t nT, int64_t nTB, int64_t n_seqs, int64_t n_keys) {
    if (work && nT <= cap_T && nTB <= cap_TB && n_seqs <= cap_seqs && n_keys <= cap_keys) return NXG_OK;
    const int64_t T_ = std::max(nT, cap_T), TB_ = std::max(nTB, cap_TB), S_ = std::max(n_seqs, cap_seqs);
    const int64_t K_ = std::max(n_keys, cap_keys);
    // attention over at most K_ keys on T_ rows (HRA's block rows: fewer rows and keys, less space)
    const int64_t ws_full = nxg_attention_workspace_bytes((int32_t) T_, hp.n_head, hp.n_kv_head, (int32_t) K_);
    if (ws_full < 0) return (int32_t) ws_full;
    int64_t ws = ws_full;
    const int C = hp.n_embd, KV = hp.n_kv_head * hp.head_dim, R = std::max(hp.lily_rank, 32), I = hp.n_inter;
    auto layout = [&](char * base) {
        carver c{base};
        const size_t rowsC = (size_t) T_ * C * sizeof(float);
        for (float *& p : x) c.take(p, rowsC);
        for (float *& p : F) c.take(p, rowsC);
        for (float *& p : K) c.take(p, (size_t) T_ * KV * sizeof(float));
        for (float *& p : Z) c.take(p, (size_t) T_ * R * sizeof(float));
        if (!fuse_mlp) c.take(U, (size_t) T_ * I * sizeof(float));
        c.take(hidden, rowsC);
        c.take(pooled, (size_t) S_ * C * sizeof(float));
        auto qa = [&](qact & a, int64_t rows, int n_in) {
            c.take(a.q, nxg_qact_q_bytes((int32_t) rows, n_in));
            c.take(a.sx, nxg_qact_sx_bytes((int32_t) rows, n_in));
        };
        qa(qa_h, T_, C);
        qa(qa_y, T_, C);
        qa(qa_g, T_, C);
        qa(qa_I, T_, I);
        qa(qa_R, T_, R);
        qa(qa_hb, std::max<int64_t>(TB_, 1), C);
        c.take(ids, (size_t) T_ * sizeof(int32_t));
        c.take(types, (size_t) T_ * sizeof(int32_t));
        c.take(cu, (size_t) (S_ + 1) * sizeof(int32_t));
        c.take(cub, (size_t) (S_ + 1) * sizeof(int32_t));
        c.take(scales, (size_t) std::max(hp.n_layer, 1) * S_ * sizeof(float));
        c.take(attn_ws, (size_t) ws);
        return c.off;
    };
    if (work) {
        NXG_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
        release(work);
        work = nullptr;
        work_bytes = 0;
    }
    // nxg_attention_ws runs with any workspace: fewer score slots, or none (the recomputing
    // kernel). Where the work area does not fit (the device's memory, or work_limit), the
    // attention's share is halved until it does, down to nothing.
    void * p = nullptr;
    size_t bytes = layout(nullptr);
    hipError_t e = hipErrorOutOfMemory;
    for (;;) {
        if (work_limit <= 0 || (int64_t) bytes <= work_limit) {
            e = hipMalloc(&p, bytes);
            if (e == hipSuccess) break;
            (void) hipGetLastError();          // the refused allocation is not a later launch's error
        }
        if (ws == 0) break;
        ws = ws > (int64_t) (64 << 20) ? ws / 2 : 0;
        bytes = layout(nullptr);
    }
    if (e != hipSuccess) {
        cap_T = cap_TB = cap_seqs = cap_keys = -1;
        attn_ws_bytes = 0;
        if (work_limit > 0 && (int64_t) bytes > work_limit) {
            return fail(NXG_ENOMEM, "encoder: %zu bytes of work memory for %lld rows exceed the limit of %lld", bytes,
                        (long long) T_, (long long) work_limit);
        }
        return fail(NXG_ENOMEM, "encoder: %zu bytes of work memory for %lld rows: %s", bytes, (long long) T_,
                    hipGetErrorString(e));
    }
    work = p;
    work_bytes = bytes;
    layout((char *) p);
    cap_T = T_;
    cap_TB = TB_;
    cap_seqs = S_;
    cap_keys = K_;
    attn_ws_bytes = ws;
    lengths.clear();                           // device offsets and scales must be uploaded again
    return NXG_OK;
}

// prepare_batch (src/nexterabert.cpp:1341-1371): the layout, the block layout of HRA, the
// RoPE tables (dynamic NTK for a single sequence beyond rope.ntk_train_length) and the
// attention layers' per-document scales (:1196-1201), uploaded when the layout changes.
int32_t nxg_encoder::prepare(const int32_t * lens, int32_t n_seqs, hipStream_t s) {
    if (n_seqs <= 0 || !lens) return fail(NXG_EINVAL, "encoder: no sequences");
    int64_t total = 0, total_b = 0;
    int32_t mx = 0, mxb = 0;
    for (int32_t i = 0; i < n_seqs; ++i) {
        if (lens[i] <= 0) return fail(NXG_EINVAL, "encoder: empty sequence in batch");
        total += lens[i];
        const int32_t nb = (lens[i] + hp.hra_block - 1) / hp.hra_block;
        total_b += nb;
        mx = std::max(mx, lens[i]);
        mxb = std::max(mxb, nb);
    }
    if (total > INT32_MAX / 4) return fail(NXG_EINVAL, "encoder: %lld tokens in one batch", (long long) total);
    float base = hp.rope_base;
    if (hp.ntk_train_len > 0 && mx > hp.ntk_train_len) {
        if (n_seqs > 1) {
            return fail(NXG_EINVAL, "encoder: sequences beyond rope.ntk_train_length must be encoded one at a time");
        }
        const double d = hp.head_dim;
        base = (float) ((double) base * std::pow((double) mx / hp.ntk_train_len, d / (d - 2.0)));
    }
    const float bases[2] = { base, hp.swa_rope_base };
    if (work && (int64_t) lengths.size() == n_seqs && std::equal(lengths.begin(), lengths.end(), lens)
        && rope[0].base == bases[0] && rope[1].base == bases[1]) {
        return NXG_OK;                         // this layout is on the device
    }
    // the previous forward may still read the offsets, scales and tables being replaced
    NXG_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
    NXG_TRY(ensure_work(total, total_b, n_seqs, mx));
    lengths.clear();                           // recorded again once every upload below has succeeded
    T = (int32_t) total;
    TB = (int32_t) total_b;
    max_len = mx;
    max_blocks = mxb;
    cu_h.assign(n_seqs + 1, 0);
    cub_h.assign(n_seqs + 1, 0);
    for (int32_t i = 0; i < n_seqs; ++i) {
        cu_h[i + 1] = cu_h[i] + lens[i];
        cub_h[i + 1] = cub_h[i] + (lens[i] + hp.hra_block - 1) / hp.hra_block;
    }
    for (int k = 0; k < 2; ++k) {
        rope_dev & r = rope[k];
        if (r.n_pos >= mx && r.base == bases[k]) continue;   // build_rope's reuse rule (:1324)
        const int half = hp.head_dim / 2;
        std::vector<float> c((size_t) mx * half), sn((size_t) mx * half);
        NXG_TRY(nxg_rope_table(mx, bases[k], hp.head_dim, c.data(), sn.data()));
        if (r.cap < mx) {
            release(r.cos);
            release(r.sin);
            r.cos = r.sin = nullptr;
            r.cap = r.n_pos = 0;
            NXG_HIP(hipMalloc((void **) &r.cos, c.size() * sizeof(float)), "hipMalloc(rope)");
            NXG_HIP(hipMalloc((void **) &r.sin, sn.size() * sizeof(float)), "hipMalloc(rope)");
            r.cap = mx;
        }
        NXG_HIP(hipMemcpy(r.cos, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy(rope)");
        NXG_HIP(hipMemcpy(r.sin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy(rope)");
        r.n_pos = mx;
        r.base = bases[k];
    }
    scales_h.assign((size_t) hp.n_layer * n_seqs, 0.0f);
    for (int32_t l = 0; l < hp.n_layer; ++l) {
        const mixer m = hp.block_types[l];
        if (m == MIX_LILY) continue;
        const std::string pre = "blocks." + std::to_string(l) + ".attn.";
        // swa layers take no length-dependent factor (ssmax = !swa, :1218-1220); HRA's is over its blocks
        const int32_t mode = m == MIX_SWA ? 0 : hp.ssmax;
        const float sf = mode ? scalar.at(pre + "scalable_factor.s") : 0.0f;
        const float bf = mode == 2 ? scalar.at(pre + "scalable_factor.b") : 0.0f;
        NXG_TRY(nxg_attention_scales(m == MIX_HRA ? cub_h.data() : cu_h.data(), n_seqs, hp.head_dim, mode, sf, bf,
                                     hp.ssmax_base, scales_h.data() + (size_t) l * n_seqs));
    }
    NXG_HIP(hipMemcpy(cu, cu_h.data(), cu_h.size() * sizeof(int32_t), hipMemcpyHostToDevice), "hipMemcpy(cu)");
    NXG_HIP(hipMemcpy(cub, cub_h.data(), cub_h.size() * sizeof(int32_t), hipMemcpyHostToDevice), "hipMemcpy(cu)");
    NXG_HIP(hipMemcpy(scales, scales_h.data(), scales_h.size() * sizeof(float), hipMemcpyHostToDevice),
            "hipMemcpy(scales)");
    lengths.assign(lens, lens + n_seqs);
    return NXG_OK;
}

int32_t nxg_encoder::linear(const std::string & name, const qact & in, int32_t rows, const float * res, float * out,
                            hipStream_t s) {
    return nxg_linear_i8_rows(i8.at(name), in.q, in.sx, rows, res, out, s);
}

int32_t nxg_encoder::project(const std::string & key, const std::vector<std::string> & names, const qact & in,
                             int32_t rows, std::initializer_list<float *> outs, hipStream_t s) {
    const auto f = fused.find(key);
    if (f != fused.end()) {
        float * o[4] = {};
        int n = 0;
        for (float * p : outs) o[n++] = p;
        return nxg_linear_i8_rows_split(f->second.w, in.q, in.sx, rows, n, f->second.cols.data(), o, s);
    }
    auto it = outs.begin();
    for (const std::string & name : names) NXG_TRY(linear(name, in, rows, nullptr, *it++, s));
    return NXG_OK;
}

namespace {

// The projection groups that read one input: fused along n_out at load when the split GEMM
// takes them (n_in % 256 == 0, boundaries at multiples of 64).
struct proj_group {
    std::string key;
    std::vector<std::string> names;
};

std::vector<proj_group> proj_groups(const hparams & hp) {
    std::vector<proj_group> v;
    for (int32_t l = 0; l < hp.n_layer; ++l) {
        const std::string pre = "blocks." + std::to_string(l) + ".attn.";
        const proj_group qkv{ pre + "qkv", { pre + "c_q.weight", pre + "c_k.weight", pre + "c_v.weight" } };
        switch (hp.block_types[l]) {
            case MIX_SWA:
            case MIX_ATTN: v.push_back(qkv); break;
            case MIX_LILY:
                v.push_back({ pre + "lily_in", { pre + "ltc_conv.in_proj.weight", pre + "ltc_conv.A.weight",
                                                 pre + "x_proj.weight", pre + "B_proj.weight" } });
                break;
            case MIX_HRA:
                v.push_back({ pre + "hra_in", { pre + "qkv_in.weight", pre + "qkv_gate.weight", pre + "c_C.weight" } });
                v.push_back(qkv);
                break;
        }
    }
    return v;
}

} // namespace

// builder::attention (src/nexterabert.cpp:1184-1204): q / k / v projections of h, q and k
// through qk_prep (k head-major), v head-major, then op_attention inside each document.
int32_t nxg_encoder::attention(const std::string & pre, const qact & h, int32_t rows, const int32_t * cu_dev,
                               int32_t n_seqs, const rope_dev & r, int32_t half, const float * scale,
                               int32_t max_keys, float * out, hipStream_t s) {
    const int32_t H = hp.n_head, G = hp.n_kv_head, D = hp.head_dim;
    NXG_OP(NXG_PROF_LINEAR, project(pre + "qkv", { pre + "c_q.weight", pre + "c_k.weight", pre + "c_v.weight" }, h, rows,
                    { F[0], K[0], K[2] }, s));
    NXG_OP(NXG_PROF_ROWS, nxg_qkv_prep(F[0], K[0], K[2], w(pre + "q_norm.alpha"), w(pre + "q_norm.beta"), w(pre + "k_norm.alpha"),
                         w(pre + "k_norm.beta"), r.cos, r.sin, r.n_pos, cu_dev, n_seqs, rows, H, G, D, F[1], K[1], K[3],
                         s));
    NXG_OP(NXG_PROF_ATTN, nxg_attention_ws(F[1], K[1], K[3], cu_dev, n_seqs, scale, rows, H, G, half, max_keys, out,
                                           attn_ws_bytes ? attn_ws : nullptr, attn_ws_bytes, s));
    return NXG_OK;
}

// builder::gated_out (:1206-1213): x + c_proj(sigmoid(c_gate(y)) * z), the gate quantized
// for c_proj; F[3] holds c_gate's output.
int32_t nxg_encoder::gated_out(const std::string & pre, const float * y, const float * z, const float * x_in,
                               float * x_out, int32_t n_seqs, hipStream_t s) {
    (void) n_seqs;
    const int32_t C = hp.n_embd;
    NXG_OP(NXG_PROF_ROWS, nxg_quantize_rows(y, T, C, act_max, qa_y.q, qa_y.sx, s));
    NXG_OP(NXG_PROF_LINEAR, linear(pre + "c_gate.weight", qa_y, T, nullptr, F[3], s));
    NXG_OP(NXG_PROF_ROWS, nxg_gate_quantize_rows(F[3], z, T, C, act_max, qa_g.q, qa_g.sx, s));
    NXG_OP(NXG_PROF_LINEAR, linear(pre + "c_proj.weight", qa_g, T, x_in, x_out, s));
    return NXG_OK;
}

// builder::encoder (src/nexterabert.cpp:1270-1292) and run_forward's pooling (:1913-1925).
int32_t nxg_encoder::run(const int32_t * ids_dev, const int32_t * types_dev, int32_t n_seqs, float * hidden_out,
                         float * pooled_out, int32_t normalize, hipStream_t s) {
    const int32_t C = hp.n_embd, R = hp.lily_rank, I = hp.n_inter;
    const f32_tensor & emb = f32.at("embedding.weight");
    const bool seg = hp.n_types > 0 && types_dev;
    prof.used = 0;
    NXG_TRY(mark(NXG_PROF_OTHER, s));          // opens the pass
    NXG_OP(NXG_PROF_OTHER, nxg_embed_rows(emb.dev, emb.rows, ids_dev, seg ? w("token_type_embeddings.weight") : nullptr,
                           hp.n_types, seg ? types_dev : nullptr, T, C, x[0], s));
    int cur = 0;
    const int32_t n_layer = n_layers_run >= 0 ? std::min(n_layers_run, hp.n_layer) : hp.n_layer;
    for (int32_t l = 0; l < n_layer; ++l) {
        const std::string blk = "blocks." + std::to_string(l) + ".";
        const std::string pre = blk + "attn.";
        float * xi = x[cur];
        float * xo = x[cur ^ 1];
        const float * scale = scales + (size_t) l * n_seqs;
        NXG_OP(NXG_PROF_ROWS, nxg_rmsnorm_quantize_rows(xi, w(blk + "attn_norm.weight"), hp.rms_eps, T, C, act_max, qa_h.q, qa_h.sx, s));
        switch (hp.block_types[l]) {
            case MIX_SWA:
            case MIX_ATTN: {                   // mix_attn (:1215-1222)
                const bool swa = hp.block_types[l] == MIX_SWA;
                const int32_t half = swa ? std::max(1, hp.swa_window / 2) : -1;
                const int32_t keys = swa ? std::min(max_len, 2 * half + 1) : max_len;
                NXG_TRY(attention(pre, qa_h, T, cu, n_seqs, rope[swa ? 1 : 0], half, scale, keys, F[2], s));
                NXG_TRY(gated_out(pre, F[2], F[2], xi, xo, n_seqs, s));
                break;
            }
            case MIX_LILY: {                   // mix_lily (:1224-1244)
                NXG_OP(NXG_PROF_LINEAR, project(pre + "lily_in", { pre + "ltc_conv.in_proj.weight", pre + "ltc_conv.A.weight",
                                                   pre + "x_proj.weight", pre + "B_proj.weight" },
                                qa_h, T, { Z[0], Z[1], F[1], F[2] }, s));
                const f32_tensor & ltc = f32.at(pre + "ltc_conv.kernel");
                NXG_OP(NXG_PROF_ROWS, nxg_dwconv_quantize_rows(Z[0], Z[1], ltc.dev, ltc.rows, cu, n_seqs, T, R, act_max, qa_R.q,
                                                 qa_R.sx, s));
                NXG_OP(NXG_PROF_LINEAR, linear(pre + "ltc_conv.out_proj.weight", qa_R, T, nullptr, F[0], s));
                const f32_tensor & st = f32.at(pre + "state_conv.depthwise.weight");
                NXG_OP(NXG_PROF_ROWS, nxg_lily_state_quantize_rows(F[0], F[1], F[2], st.dev, st.rows, cu, n_seqs, T, C, act_max,
                                                     qa_g.q, qa_g.sx, s));
                NXG_OP(NXG_PROF_LINEAR, linear(pre + "c_proj.weight", qa_g, T, xi, xo, s));
                break;
            }
            case MIX_HRA: {                    // mix_hra (:1246-1268)
                NXG_OP(NXG_PROF_LINEAR, project(pre + "hra_in", { pre + "qkv_in.weight", pre + "qkv_gate.weight", pre + "c_C.weight" },
                                qa_h, T, { F[4], F[6], F[7] }, s));
                const f32_tensor & qc = f32.at(pre + "qkv_conv.depthwise.weight");
                NXG_OP(NXG_PROF_ROWS, nxg_dwconv_rows(F[4], nullptr, qc.dev, qc.rows, cu, n_seqs, T, C, F[5], s));
                NXG_OP(NXG_PROF_ROWS, nxg_block_mean_quantize_rows(F[5], F[6], cu, cub, n_seqs, T, TB, hp.hra_block, C, act_max,
                                                     qa_hb.q, qa_hb.sx, s));
                NXG_TRY(attention(pre, qa_hb, TB, cub, n_seqs, rope[0], -1, scale, max_blocks, F[2], s));
                NXG_OP(NXG_PROF_ROWS, nxg_upsample_add(F[2], F[7], cu, cub, n_seqs, T, TB, hp.hra_block, C, F[4], s));
                const f32_tensor & co = f32.at(pre + "c_o.depthwise.weight");
                NXG_OP(NXG_PROF_ROWS, nxg_dwconv_rows(F[4], nullptr, co.dev, co.rows, cu, n_seqs, T, C, F[5], s));
                NXG_TRY(gated_out(pre, F[4], F[5], xi, xo, n_seqs, s));
                break;
            }
        }
        cur ^= 1;
        // x + c_proj(relu(c_fc(norm(x)))^2) (:1284-1289)
        xi = x[cur];
        xo = x[cur ^ 1];
        NXG_OP(NXG_PROF_ROWS, nxg_rmsnorm_quantize_rows(xi, w(blk + "mlp_norm.weight"), hp.rms_eps, T, C, act_max, qa_h.q, qa_h.sx, s));
        if (fuse_mlp) {
            NXG_OP(NXG_PROF_LINEAR, nxg_linear_i8_relu2_q8_rows(i8.at(blk + "mlp.c_fc.weight"), qa_h.q, qa_h.sx, T, act_max, qa_I.q,
                                                qa_I.sx, s));
        } else {
            NXG_OP(NXG_PROF_LINEAR, linear(blk + "mlp.c_fc.weight", qa_h, T, nullptr, U, s));
            NXG_OP(NXG_PROF_ROWS, nxg_quantize_rows_relu2(U, T, I, act_max, qa_I.q, qa_I.sx, s));
        }
        NXG_OP(NXG_PROF_LINEAR, linear(blk + "mlp.c_proj.weight", qa_I, T, xi, xo, s));
        cur ^= 1;
    }
    const float * out = x[cur];
    if (n_layers_run < 0) {                    // out_norm (:1290-1291)
        float * dst = hidden_out ? hidden_out : x[cur ^ 1];
        NXG_OP(NXG_PROF_OTHER, nxg_layer_norm(out, w("out_norm.weight"), w("out_norm.bias"), hp.ln_eps, T, C, dst, s));
        out = dst;
    } else if (hidden_out) {
        NXG_HIP(hipMemcpyAsync(hidden_out, out, (size_t) T * C * sizeof(float), hipMemcpyDeviceToDevice, s),
                "hipMemcpyAsync(hidden)");
        NXG_TRY(mark(NXG_PROF_OTHER, s));
    }
    if (pooled_out) NXG_OP(NXG_PROF_ROWS, nxg_doc_mean(out, cu, n_seqs, T, C, normalize, pooled_out, s));
    return NXG_OK;
}

namespace {

// The tensors builder::encoder reads for each block type, with the shapes the kernels
// assume: [n_in, n_out] for linears, element counts otherwise.
struct need {
    std::string name;
    int64_t n_in, n_out;   // linears; n_out < 0: an fp32 tensor of n_in elements (0: any)
};

std::vector<need> needed(const hparams & hp) {
    const int64_t C = hp.n_embd, KV = (int64_t) hp.n_kv_head * hp.head_dim, R = hp.lily_rank, D = hp.head_dim;
    std::vector<need> v = { { "embedding.weight", 0, -1 }, { "out_norm.weight", C, -1 }, { "out_norm.bias", C, -1 } };
    for (int32_t l = 0; l < hp.n_layer; ++l) {
        const std::string blk = "blocks." + std::to_string(l) + ".", pre = blk + "attn.";
        v.push_back({ blk + "attn_norm.weight", C, -1 });
        auto attn = [&](bool with_scalars) {
            v.push_back({ pre + "c_q.weight", C, C });
            v.push_back({ pre + "c_k.weight", C, KV });
            v.push_back({ pre + "c_v.weight", C, KV });
            for (const char * n : { "q_norm.alpha", "q_norm.beta", "k_norm.alpha", "k_norm.beta" }) v.push_back({ pre + n, D, -1 });
            if (with_scalars && hp.ssmax >= 1) v.push_back({ pre + "scalable_factor.s", 1, -1 });
            if (with_scalars && hp.ssmax == 2) v.push_back({ pre + "scalable_factor.b", 1, -1 });
            v.push_back({ pre + "c_gate.weight", C, C });
            v.push_back({ pre + "c_proj.weight", C, C });
        };
        switch (hp.block_types[l]) {
            case MIX_SWA: attn(false); break;
            case MIX_ATTN: attn(true); break;
            case MIX_LILY:
                v.push_back({ pre + "ltc_conv.in_proj.weight", C, R });
                v.push_back({ pre + "ltc_conv.A.weight", C, R });
                v.push_back({ pre + "ltc_conv.kernel", 0, -1 });
                v.push_back({ pre + "ltc_conv.out_proj.weight", R, C });
                v.push_back({ pre + "x_proj.weight", C, C });
                v.push_back({ pre + "B_proj.weight", C, C });
                v.push_back({ pre + "state_conv.depthwise.weight", 0, -1 });
                v.push_back({ pre + "c_proj.weight", C, C });
                break;
            case MIX_HRA:
                v.push_back({ pre + "qkv_in.weight", C, C });
                v.push_back({ pre + "qkv_conv.depthwise.weight", 0, -1 });
                v.push_back({ pre + "qkv_gate.weight", C, C });
                v.push_back({ pre + "c_C.weight", C, C });
                v.push_back({ pre + "c_o.depthwise.weight", 0, -1 });
                attn(true);
                break;
        }
        v.push_back({ blk + "mlp_norm.weight", C, -1 });
        v.push_back({ blk + "mlp.c_fc.weight", C, hp.n_inter });
        v.push_back({ blk + "mlp.c_proj.weight", hp.n_inter, C });
    }
    return v;
}

// One int8 weight from the linears `names` of the open file, concatenated along n_out: each
// expanded as nxg_gguf_weight_create does (build_i8_weight, src/nexterabert.cpp:1010-1049),
// rows appended, and the per-block scales of block B side by side in the same order.
int32_t fuse_weights(nxg_gguf * g, const std::unordered_map<std::string, int64_t> & index,
                     const std::vector<std::string> & names, int32_t n_threads, nxg_weight ** out) {
    try {
        std::vector<int8_t> W;
        std::vector<std::vector<float>> S;
        std::vector<int32_t> n_outs;
        int64_t n_in = -1, N = 0;
        for (const std::string & name : names) {
            const auto at = index.find(name);
            if (at == index.end()) return fail(NXG_EINVAL, "encoder: '%s' missing", name.c_str());
            int32_t type = 0, nd = 0;
            int64_t ne[4];
            NXG_TRY(nxg_gguf_tensor_info(g, at->second, &type, &nd, ne, nullptr, nullptr));
            if (n_in < 0) n_in = ne[0];
            if (ne[0] != n_in || ne[1] <= 0 || ne[1] > INT32_MAX) return fail(NXG_EINVAL, "encoder: '%s' cannot join its group", name.c_str());
            const int32_t n_o = (int32_t) ne[1];
            const int64_t n_blk = (n_in + NXG_BLOCK - 1) / NXG_BLOCK;
            std::vector<int8_t> w((size_t) (n_in * n_o));
            std::vector<float> sc((size_t) (n_blk * n_o));
            NXG_TRY(nxg_expand_weight(type, nxg_gguf_tensor_data(g, at->second), (int32_t) n_in, n_o, 128, n_threads,
                                      w.data(), sc.data(), nullptr));
            W.insert(W.end(), w.begin(), w.end());
            S.push_back(std::move(sc));
            n_outs.push_back(n_o);
            N += n_o;
        }
        if (N > INT32_MAX) return fail(NXG_EINVAL, "encoder: fused group of %lld rows", (long long) N);
        const int64_t n_blk = (n_in + NXG_BLOCK - 1) / NXG_BLOCK;
        std::vector<float> SC((size_t) (n_blk * N));
        for (int64_t B = 0; B < n_blk; ++B) {
            int64_t o = 0;
            for (size_t k = 0; k < S.size(); ++k) {
                std::copy_n(S[k].begin() + B * n_outs[k], n_outs[k], SC.begin() + B * N + o);
                o += n_outs[k];
            }
        }
        return nxg_weight_create(W.data(), SC.data(), (int32_t) n_in, (int32_t) N, out);
    } catch (const std::bad_alloc &) {
        return fail(NXG_ENOMEM, "encoder: out of host memory fusing '%s'", names.front().c_str());
    }
}

bool encoder_tensor(const std::string & name) {
    return name.rfind("blocks.", 0) == 0 || name == "embedding.weight" || name == "token_type_embeddings.weight"
           || name == "out_norm.weight" || name == "out_norm.bias";
}

int32_t load_into(nxg_encoder & e, const char * path, const nxg_encoder_params & params) {
    nxg_gguf * g = nullptr;
    NXG_TRY(nxg_gguf_open(path, &g));
    struct closer {
        nxg_gguf * g;
        ~closer() { nxg_gguf_close(g); }
    } close_g{ g };
    kv_reader kv{ g };
    const std::string arch = kv.str("general.architecture", "");
    if (arch != "nexterabert") {
        return fail(NXG_EINVAL, "encoder: '%s' is not a nexterabert GGUF (general.architecture = '%s')", path, arch.c_str());
    }
    hparams & hp = e.hp;
    hp.n_vocab = (int32_t) kv.u32("nexterabert.vocab_size", 0, true);
    hp.n_embd = (int32_t) kv.u32("nexterabert.embedding_length", 0, true);
    hp.n_layer = (int32_t) kv.u32("nexterabert.block_count", 0, true);
    hp.n_inter = (int32_t) kv.u32("nexterabert.feed_forward_length", 0, true);
    hp.n_head = (int32_t) kv.u32("nexterabert.attention.head_count", 0, true);
    hp.n_kv_head = (int32_t) kv.u32("nexterabert.attention.head_count_kv", 0, true);
    if (!kv.bad.empty()) return fail(NXG_EINVAL, "encoder: missing key '%s'", kv.bad.c_str());
    if (hp.n_head <= 0 || hp.n_kv_head <= 0 || hp.n_embd <= 0 || hp.n_layer <= 0 || hp.n_vocab <= 0 || hp.n_inter <= 0) {
        return fail(NXG_EINVAL, "encoder: bad dimensions (n_embd %d, n_layer %d, n_head %d, n_kv_head %d, vocab %d, n_inter %d)",
                    hp.n_embd, hp.n_layer, hp.n_head, hp.n_kv_head, hp.n_vocab, hp.n_inter);
    }
    hp.head_dim = hp.n_embd / hp.n_head;
    hp.lily_rank = (int32_t) kv.u32("nexterabert.lily.low_rank", hp.head_dim);
    hp.lily_kernel = (int32_t) kv.u32("nexterabert.lily.kernel_size", 5);
    hp.hra_block = (int32_t) kv.u32("nexterabert.hra.block_size", 4);
    hp.swa_window = (int32_t) kv.u32("nexterabert.swa.window", 256);
    hp.ntk_train_len = (int32_t) kv.u32("nexterabert.rope.ntk_train_length", 0);
    hp.rope_base = kv.f32("nexterabert.rope.freq_base", 100000.0f);
    hp.swa_rope_base = kv.f32("nexterabert.swa.rope.freq_base", 10000.0f);
    hp.ssmax_base = kv.f32("nexterabert.ssmax.base", 0.1f);
    hp.rms_eps = kv.f32("nexterabert.rms_norm_epsilon", 1e-8f);
    hp.ln_eps = kv.f32("nexterabert.layer_norm_epsilon", 1e-5f);
    const std::string mode = kv.str("nexterabert.ssmax.mode", "sssmax");
    hp.ssmax = mode == "none" ? 0 : mode == "ssmax" ? 1 : 2;
    if (!kv.bad.empty()) return fail(NXG_EINVAL, "encoder: unreadable key '%s'", kv.bad.c_str());
    {
        const int64_t id = nxg_gguf_find_key(g, "nexterabert.block_types");
        int32_t et = -1;
        uint64_t n = 0;
        if (id < 0 || nxg_gguf_arr_info(g, id, &et, &n) != NXG_OK) n = 0;
        if ((int64_t) n != hp.n_layer) {
            return fail(NXG_EINVAL, "encoder: block_types has %llu entries, expected %d", (unsigned long long) n, hp.n_layer);
        }
        for (uint64_t i = 0; i < n; ++i) {
            const char * s = nullptr;
            uint64_t len = 0;
            if (nxg_gguf_arr_str(g, id, i, &s, &len) != NXG_OK) return fail(NXG_EINVAL, "encoder: block_types is not a string array");
            const std::string t(s, (size_t) len);
            if (t == "lily") hp.block_types.push_back(MIX_LILY);
            else if (t == "swa") hp.block_types.push_back(MIX_SWA);
            else if (t == "attn") hp.block_types.push_back(MIX_ATTN);
            else if (t == "hra") hp.block_types.push_back(MIX_HRA);
            else return fail(NXG_EINVAL, "encoder: unsupported block type '%s'", t.c_str());
        }
    }
    if (hp.head_dim % 2 != 0 || hp.n_head % hp.n_kv_head != 0) return fail(NXG_EINVAL, "encoder: unsupported head layout");
    // what the GPU kernels need beyond the reference's own checks
    const bool any_attn = std::any_of(hp.block_types.begin(), hp.block_types.end(), [](mixer m) { return m != MIX_LILY; });
    if (any_attn && (hp.head_dim != 64 || hp.n_head * 64 != hp.n_embd)) {
        return fail(NXG_EINVAL, "encoder: attention needs head_dim 64 (n_embd %d, n_head %d)", hp.n_embd, hp.n_head);
    }
    if (hp.n_embd % 32 != 0 || hp.lily_rank % 32 != 0 || hp.n_inter % 32 != 0 || hp.hra_block < 1 || hp.swa_window < 0) {
        return fail(NXG_EINVAL, "encoder: n_embd %d, lily rank %d, n_inter %d must be multiples of 32; hra block %d",
                    hp.n_embd, hp.lily_rank, hp.n_inter, hp.hra_block);
    }

    // Every encoder linear must take the int8 path (the placement rule of
    // src/nexterabert.cpp:1663-1667): the reference would run the others on ggml_mul_mat
    // (:1140-1142), which this engine does not have. Checked on the tensor table, before
    // the GPU is touched, so that an F32 / F16 file is refused with this reason anywhere.
    for (const need & nd : needed(hp)) {
        if (nd.n_out < 0) continue;
        const int64_t ti = nxg_gguf_find_tensor(g, nd.name.c_str());
        if (ti < 0) return fail(NXG_EINVAL, "encoder: missing tensor '%s'", nd.name.c_str());
        int32_t type = 0, ndim = 0;
        int64_t ne[4];
        NXG_TRY(nxg_gguf_tensor_info(g, ti, &type, &ndim, ne, nullptr, nullptr));
        if (!nxg_weight_is_int8(nd.name.c_str(), ndim, type, ne[0], ndim > 1 ? ne[1] : 1, 1)) {
            return fail(NXG_EINVAL, "encoder: '%s' (ggml type %d) is not on the int8 path: this engine runs every encoder "
                        "linear as an int8 GEMM and has no ggml_mul_mat fallback (F32/F16/BF16 linears are refused)",
                        nd.name.c_str(), type);
        }
    }

    // tensors: the int8 linears expanded and uploaded, the rest decoded to fp32 and uploaded
    NXG_TRY(nxg_init());
    const int64_t n_tensors = nxg_gguf_n_tensors(g);
    for (int64_t i = 0; i < n_tensors; ++i) {
        const std::string name = nxg_gguf_tensor_name(g, i);
        if (!encoder_tensor(name)) continue;
        int32_t type = 0, nd = 0;
        int64_t ne[4];
        NXG_TRY(nxg_gguf_tensor_info(g, i, &type, &nd, ne, nullptr, nullptr));
        if (nxg_weight_is_int8(name.c_str(), nd, type, ne[0], ne[1], 1)) {
            nxg_weight * wt = nullptr;
            NXG_TRY(nxg_gguf_weight_create(g, i, params.load_threads, &wt));
            e.i8[name] = wt;
            e.n_int8 += 1;
            e.weight_bytes += nxg_weight_device_bytes(wt);
            continue;
        }
        const int64_t n = ne[0] * ne[1] * ne[2] * ne[3];
        if (n <= 0 || n > ((int64_t) 1 << 34)) return fail(NXG_EINVAL, "encoder: tensor '%s' has %lld elements", name.c_str(), (long long) n);
        std::vector<float> h;
        try {
            h.resize((size_t) n);
        } catch (const std::bad_alloc &) {
            return fail(NXG_ENOMEM, "encoder: tensor '%s': out of host memory", name.c_str());
        }
        NXG_TRY(nxg_dequantize_rows(type, nxg_gguf_tensor_data(g, i), ne[0], n / ne[0], h.data()));
        f32_tensor t;
        t.n = n;
        t.rows = (int32_t) (n / ne[0]);
        t.cols = (int32_t) ne[0];
        if (ends_with(name, ".depthwise.weight") || ends_with(name, ".kernel")) {
            // stored (k, C) per channel; the ops read one row per tap (:1701-1710)
            const int64_t k = ne[0], C = n / ne[0];
            std::vector<float> taps((size_t) n);
            for (int64_t ch = 0; ch < C; ++ch) {
                for (int64_t j = 0; j < k; ++j) taps[(size_t) (j * C + ch)] = h[(size_t) (ch * k + j)];
            }
            h.swap(taps);
            t.rows = (int32_t) k;
            t.cols = (int32_t) C;
        }
        if (n == 1) e.scalar[name] = h[0];
        NXG_HIP(hipMalloc((void **) &t.dev, (size_t) n * sizeof(float)), "hipMalloc(tensor)");
        e.f32[name] = t;
        NXG_HIP(hipMemcpy(t.dev, h.data(), (size_t) n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy(tensor)");
        e.weight_bytes += (size_t) n * sizeof(float);
    }
    if (e.f32.count("token_type_embeddings.weight")) {
        const f32_tensor & t = e.f32["token_type_embeddings.weight"];
        if (t.cols != hp.n_embd) return fail(NXG_EINVAL, "encoder: token_type_embeddings.weight is not [n][%d]", hp.n_embd);
        hp.n_types = t.rows;
    }
    // every tensor the forward reads, with the shape its kernels assume
    for (const need & nd : needed(hp)) {
        if (nd.n_out >= 0) {
            auto it = e.i8.find(nd.name);
            if (it == e.i8.end()) {
                return fail(NXG_EINVAL, "encoder: '%s' is %s", nd.name.c_str(),
                            e.f32.count(nd.name) ? "not on the int8 path (the GPU encoder runs every encoder linear in int8)"
                                                 : "missing");
            }
            if (nxg_weight_n_in(it->second) != nd.n_in || nxg_weight_n_out(it->second) != nd.n_out) {
                return fail(NXG_EINVAL, "encoder: '%s' is %d x %d, expected %lld x %lld", nd.name.c_str(),
                            nxg_weight_n_in(it->second), nxg_weight_n_out(it->second), (long long) nd.n_in,
                            (long long) nd.n_out);
            }
            continue;
        }
        auto it = e.f32.find(nd.name);
        if (it == e.f32.end()) return fail(NXG_EINVAL, "encoder: missing tensor '%s'", nd.name.c_str());
        const f32_tensor & t = it->second;
        bool ok = nd.n_in == 0 || t.n == nd.n_in;
        if (nd.name == "embedding.weight") ok = t.cols == hp.n_embd && t.rows >= hp.n_vocab;
        if (ends_with(nd.name, ".depthwise.weight")) ok = t.cols == hp.n_embd && t.rows >= 1;
        if (ends_with(nd.name, ".kernel")) ok = t.cols == hp.lily_rank && t.rows >= 1;
        if (!ok) return fail(NXG_EINVAL, "encoder: tensor '%s' has an unexpected shape (%d x %d)", nd.name.c_str(), t.rows, t.cols);
    }
    e.fuse_mlp = hp.n_embd % 256 == 0;         // nxg_linear_i8_relu2_q8's shape rule (n_out % 32 checked above)
    // projections of one input fused along n_out, one split GEMM launch each (the separate
    // weights are then freed); the split GEMM needs n_in % 256 == 0 and boundaries at
    // multiples of 64, otherwise the group stays separate
    if (hp.n_embd % 256 == 0) {
        std::unordered_map<std::string, int64_t> index;
        for (int64_t i = 0; i < n_tensors; ++i) index[nxg_gguf_tensor_name(g, i)] = i;
        for (const proj_group & pg : proj_groups(hp)) {
            std::vector<int32_t> cols;
            int64_t end = 0;
            bool ok = pg.names.size() <= 4;
            for (size_t k = 0; k < pg.names.size(); ++k) {
                const int32_t c = nxg_weight_n_out(e.i8.at(pg.names[k]));
                cols.push_back(c);
                end += c;
                if (c % 4 != 0 || (k + 1 < pg.names.size() && end % 64 != 0)) ok = false;
            }
            if (!ok) continue;
            nxg_encoder::fused_w f;
            f.cols = cols;
            NXG_TRY(fuse_weights(g, index, pg.names, params.load_threads, &f.w));
            e.fused[pg.key] = f;
            e.weight_bytes += nxg_weight_device_bytes(f.w);
            for (const std::string & n : pg.names) {
                e.weight_bytes -= nxg_weight_device_bytes(e.i8[n]);
                nxg_weight_destroy(e.i8[n]);
                e.i8.erase(n);
            }
        }
    }
    return NXG_OK;
}

} // namespace

extern "C" {

nxg_encoder_params nxg_encoder_default_params(void) {
    nxg_encoder_params p;
    p.act_max = 127;
    p.load_threads = 0;
    p.verbosity = 0;
    return p;
}

int32_t nxg_encoder_load(const char * path, const nxg_encoder_params * params, nxg_encoder ** out) {
    if (!out) return fail(NXG_EINVAL, "encoder_load: null out");
    *out = nullptr;
    if (!path) return fail(NXG_EINVAL, "encoder_load: null path");
    const nxg_encoder_params p = params ? *params : nxg_encoder_default_params();
    if (p.act_max != 127 && p.act_max != 63) return fail(NXG_EINVAL, "encoder_load: act_max must be 127 or 63");
    const auto t0 = std::chrono::steady_clock::now();
    nxg_encoder * e = new (std::nothrow) nxg_encoder();
    if (!e) return fail(NXG_ENOMEM, "encoder_load: out of host memory");
    e->act_max = p.act_max;
    int32_t rc = load_into(*e, path, p);
    if (rc == NXG_OK) {
        const hipError_t he = hipStreamCreate(&e->stream);
        if (he != hipSuccess) rc = hip_fail(he, "hipStreamCreate");
    }
    if (rc != NXG_OK) {
        delete e;
        return rc;
    }
    if (p.verbosity > 0) {
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        fprintf(stderr, "nxg_encoder: %s: %d layers, n_embd %d, %zu int8 linears, %zu fp32 tensors, %.1f MiB on the GPU, %.0f ms\n",
                path, e->hp.n_layer, e->hp.n_embd, e->i8.size(), e->f32.size(), e->weight_bytes / 1048576.0, ms);
    }
    *out = e;
    return NXG_OK;
}

void nxg_encoder_free(nxg_encoder * e) {
    if (!e) return;
    if (e->stream) (void) hipStreamSynchronize(e->stream);
    delete e;
}

int32_t nxg_encoder_n_embd(const nxg_encoder * e) { return e ? e->hp.n_embd : 0; }
int32_t nxg_encoder_n_vocab(const nxg_encoder * e) { return e ? e->hp.n_vocab : 0; }
int32_t nxg_encoder_n_layer(const nxg_encoder * e) { return e ? e->hp.n_layer : 0; }
int32_t nxg_encoder_n_token_types(const nxg_encoder * e) { return e ? e->hp.n_types : 0; }
size_t nxg_encoder_device_bytes(const nxg_encoder * e) { return e ? e->weight_bytes + e->work_bytes : 0; }
void nxg_encoder_set_layers(nxg_encoder * e, int32_t n_layers) {
    if (e) e->n_layers_run = n_layers;
}
double nxg_encoder_last_ms(const nxg_encoder * e) { return e ? e->last_ms : 0.0; }
int32_t nxg_encoder_n_int8(const nxg_encoder * e) { return e ? e->n_int8 : 0; }

int32_t nxg_encoder_set_work_limit(nxg_encoder * e, int64_t bytes) {
    if (!e) return fail(NXG_EINVAL, "encoder_set_work_limit: null context");
    if (bytes < 0) return fail(NXG_EINVAL, "encoder_set_work_limit: %lld bytes", (long long) bytes);
    e->work_limit = bytes;
    if (e->work) {
        // the next pass sizes the work area again under the new limit
        NXG_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
        release(e->work);
        e->work = nullptr;
        e->work_bytes = 0;
        e->attn_ws_bytes = 0;
        e->cap_T = e->cap_TB = e->cap_seqs = e->cap_keys = -1;
    }
    return NXG_OK;
}

int64_t nxg_encoder_attention_workspace(const nxg_encoder * e) { return e ? e->attn_ws_bytes : 0; }

void nxg_encoder_profile(nxg_encoder * e, int32_t enable) {
    if (!e) return;
    const std::vector<hipEvent_t> ev = std::move(e->prof.ev);   // the events are kept for reuse
    e->prof = nxg_encoder::profiler();
    e->prof.ev = ev;
    e->prof.kind.assign(ev.size(), 0);
    e->prof.enabled = enable != 0;
}

int32_t nxg_encoder_profile_read(const nxg_encoder * e, double * kind_ms, double * device_ms, double * wall_ms,
                                 int64_t * passes) {
    if (!e) return fail(NXG_EINVAL, "encoder_profile_read: null context");
    for (int k = 0; kind_ms && k < NXG_PROF_COUNT; ++k) kind_ms[k] = e->prof.ms[k];
    if (device_ms) *device_ms = e->prof.device_ms;
    if (wall_ms) *wall_ms = e->prof.wall_ms;
    if (passes) *passes = e->prof.passes;
    return NXG_OK;
}

int32_t nxg_encoder_forward(nxg_encoder * e, const int32_t * tokens, const int32_t * token_types,
                            const int32_t * lengths, int32_t n_seqs, float * hidden, float * pooled,
                            int32_t normalize, void * stream) {
    if (!e || !tokens) return fail(NXG_EINVAL, "encoder_forward: null context or tokens");
    hipStream_t s = (hipStream_t) stream;
    if (e->prof.enabled) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        NXG_HIP(hipStreamIsCapturing(s, &st), "hipStreamIsCapturing");
        if (st != hipStreamCaptureStatusNone) return fail(NXG_EINVAL, "encoder_forward: a profiled pass cannot be captured");
    }
    NXG_TRY(e->prepare(lengths, n_seqs, s));
    NXG_TRY(e->run(tokens, token_types, n_seqs, hidden, pooled, normalize, s));
    return e->collect(-1.0);
}

int32_t nxg_encoder_encode(nxg_encoder * e, const int32_t * tokens, const int32_t * token_types,
                           const int32_t * lengths, int32_t n_seqs, float * hidden, float * pooled,
                           int32_t normalize) {
    if (!e || !tokens || !lengths) return fail(NXG_EINVAL, "encoder_encode: null context, tokens or lengths");
    const auto t0 = std::chrono::steady_clock::now();
    hipStream_t s = e->stream;
    NXG_TRY(e->prepare(lengths, n_seqs, s));
    const int32_t N = e->T, C = e->hp.n_embd;
    // check_tokens / check_types (:1843-1862)
    for (int32_t i = 0; i < N; ++i) {
        if (tokens[i] < 0 || tokens[i] >= e->hp.n_vocab) return fail(NXG_EINVAL, "encoder: token id %d out of range", tokens[i]);
    }
    const bool seg = token_types && e->hp.n_types > 0;
    for (int32_t i = 0; seg && i < N; ++i) {
        if (token_types[i] < 0 || token_types[i] >= e->hp.n_types) {
            return fail(NXG_EINVAL, "encoder: token type id %d out of range", token_types[i]);
        }
    }
    NXG_HIP(hipMemcpyAsync(e->ids, tokens, (size_t) N * sizeof(int32_t), hipMemcpyHostToDevice, s), "hipMemcpyAsync(tokens)");
    if (seg) {
        NXG_HIP(hipMemcpyAsync(e->types, token_types, (size_t) N * sizeof(int32_t), hipMemcpyHostToDevice, s),
                "hipMemcpyAsync(types)");
    }
    NXG_TRY(e->run(e->ids, seg ? e->types : nullptr, n_seqs, e->hidden, pooled ? e->pooled : nullptr, normalize, s));
    if (hidden) {
        NXG_HIP(hipMemcpyAsync(hidden, e->hidden, (size_t) N * C * sizeof(float), hipMemcpyDeviceToHost, s),
                "hipMemcpyAsync(hidden)");
    }
    if (pooled) {
        NXG_HIP(hipMemcpyAsync(pooled, e->pooled, (size_t) n_seqs * C * sizeof(float), hipMemcpyDeviceToHost, s),
                "hipMemcpyAsync(pooled)");
    }
    NXG_HIP(hipStreamSynchronize(s), "compute");
    e->last_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return e->collect(e->last_ms);
}

} // extern "C"
