// nxg_cli.cpp -- the int8 linear path of the NexteraBERT encoder driven from C++ through
// the C ABI (include/nxg_linear.h, include/nxg_gguf.h), the way the reference's own host
// calls it from builder::linear (src/nexterabert.cpp:1121-1143). Its --bench follows the
// reference CLI's rule (tools/cli.cpp:177-204): 3 untimed passes, then R timed ones on
// the host clock around a pass that ends in a stream synchronization; median, min and
// tokens/s = 1000 * T * B / median.
//
//   nxg-cli --info [-m model.gguf]
//   nxg-cli --bench T [--batch B] [--reps R] [--graph] [--profile] [-m model.gguf]
//   nxg-cli --bench T --encode -m model.gguf [--batch B] [--reps R] [--profile]
//
// --encode times the whole encoder instead (include/nxg_encoder.h: nxg_encoder_encode on
// host buffers, the counterpart of nextera_encode) with the reference CLI's inputs: ids
// uniform in [1000, min(vocab, 40000)) from mt19937(0), CLS first and SEP last in each
// sequence, L2-normalised pooled vectors as the only output. --profile profiles the timed
// passes (nxg_encoder_profile) and prints the reference's --profile report
// (src/nexterabert.cpp:1828-1841): int8 linear, attention, row ops, everything else, total.
//
// A pass runs every int8 projection of the 18 layers (src/nexterabert.cpp:1185-1289) over B
// packed sequences of T tokens: per layer each distinct activation is quantized once
// (nxg_quantize_rows, the qcache), linears that read the same activation run as one GEMM
// over their weights concatenated along N, the MLP's c_fc writes c_proj's int8 input
// (nxg_linear_i8_relu2_q8), HRA q/k/v run on ceil(len / 4) block rows, and every GEMM gets
// the batch's cu_offsets. The producers of the activations (norms, attention, convolutions,
// SnowLily state) are not on this path: their outputs are synthetic rows. Weights are
// random N(0, 0.02) encoded as Q8_0, or the file's with -m; either way expanded on the host
// as build_i8_weight (nxg_expand_weight) and uploaded once (nxg_weight_create).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "nxg_encoder.h"
#include "nxg_gguf.h"
#include "nxg_linear.h"

namespace {

// Model dimensions of the 213M-parameter checkpoint; the 18 blocks' order (8 lily, 5 swa,
// 3 attn, 2 hra) does not change any linear's shape.
constexpr int N_EMBD = 1024, N_INTER = 2304, KV = 8 * 64, LILY_RANK = 64, HRA_BLOCK = 4;
constexpr int TYPE_Q8_0 = 8;
const char * const BLOCK_TYPES[18] = { "lily", "lily", "lily", "lily", "lily", "lily", "lily", "lily",
                                       "swa", "swa", "swa", "swa", "swa", "attn", "attn", "attn", "hra", "hra" };

struct spec {
    std::string name;
    int n_in, n_out;
    std::string input;         // the activation it reads; linears sharing one share its GEMM
    bool residual = false;
    bool block_rows = false;   // HRA q/k/v
    std::string relu2_into;    // MLP c_fc: the output only feeds relu^2 into this activation
};

// The int8 linears of block l in graph order (src/nexterabert.cpp:1217-1289).
std::vector<spec> layer_linears(int l, const std::string & kind) {
    const std::string blk = "blocks." + std::to_string(l) + ".", pre = blk + "attn.";
    const int C = N_EMBD;
    std::vector<spec> v;
    if (kind == "attn" || kind == "swa") {
        v = { { pre + "c_q.weight", C, C, "h" }, { pre + "c_k.weight", C, KV, "h" }, { pre + "c_v.weight", C, KV, "h" },
              { pre + "c_gate.weight", C, C, "attn_out" }, { pre + "c_proj.weight", C, C, "gate_out", true } };
    } else if (kind == "lily") {
        v = { { pre + "ltc_conv.in_proj.weight", C, LILY_RANK, "h" }, { pre + "ltc_conv.A.weight", C, LILY_RANK, "h" },
              { pre + "ltc_conv.out_proj.weight", LILY_RANK, C, "conv_out" }, { pre + "x_proj.weight", C, C, "h" },
              { pre + "B_proj.weight", C, C, "h" }, { pre + "c_proj.weight", C, C, "state_out", true } };
    } else {   // hra
        v = { { pre + "qkv_in.weight", C, C, "h" }, { pre + "qkv_gate.weight", C, C, "h" },
              { pre + "c_q.weight", C, C, "block_mean", false, true }, { pre + "c_k.weight", C, KV, "block_mean", false, true },
              { pre + "c_v.weight", C, KV, "block_mean", false, true }, { pre + "c_C.weight", C, C, "h" },
              { pre + "c_gate.weight", C, C, "attn_out" }, { pre + "c_proj.weight", C, C, "gate_out", true } };
    }
    v.push_back({ blk + "mlp.c_fc.weight", C, N_INTER, "mlp_in", false, false, "relu_out" });
    v.push_back({ blk + "mlp.c_proj.weight", N_INTER, C, "relu_out", true });
    return v;
}

[[noreturn]] void die(const char * what, const char * detail) {
    fprintf(stderr, "nxg-cli: %s: %s\n", what, detail);
    exit(1);
}

void check(int32_t rc, const char * what) {
    if (rc != NXG_OK) die(what, nxg_last_error());
}

void hip_check(hipError_t e, const char * what) {
    if (e != hipSuccess) die(what, hipGetErrorString(e));
}

// An expanded weight on the host: w [n_out][n_in], scale [n_blk][n_out].
struct host_weight {
    int n_in = 0, n_out = 0;
    std::vector<int8_t> w;
    std::vector<float> scale;
};

host_weight expand(int type, const void * data, int n_in, int n_out) {
    host_weight h;
    h.n_in = n_in;
    h.n_out = n_out;
    h.w.resize((size_t) n_out * n_in);
    h.scale.resize((size_t) ((n_in + 255) / 256) * n_out);
    check(nxg_expand_weight(type, data, n_in, n_out, 128, 0, h.w.data(), h.scale.data(), nullptr), "expand_weight");
    return h;
}

host_weight random_weight(int n_in, int n_out, std::mt19937_64 & rng) {
    std::normal_distribution<float> nd(0.0f, 0.02f);
    std::vector<float> rows((size_t) n_out * n_in);
    for (float & x : rows) x = nd(rng);
    std::vector<uint8_t> q(nxg_row_bytes(TYPE_Q8_0, n_in) * n_out);
    check(nxg_quantize_weight(TYPE_Q8_0, rows.data(), n_in, n_out, q.data()), "quantize_weight");
    return expand(TYPE_Q8_0, q.data(), n_in, n_out);
}

host_weight file_weight(const nxg_gguf * g, const spec & s) {
    const int64_t i = nxg_gguf_find_tensor(g, s.name.c_str());
    if (i < 0) die(s.name.c_str(), "not in the GGUF file");
    int32_t type = 0, n_dims = 0;
    int64_t ne[4];
    uint64_t off = 0, nbytes = 0;
    check(nxg_gguf_tensor_info(g, i, &type, &n_dims, ne, &off, &nbytes), "gguf_tensor_info");
    if (n_dims != 2 || ne[0] != s.n_in || ne[1] != s.n_out) die(s.name.c_str(), "unexpected shape in the GGUF file");
    return expand(type, nxg_gguf_tensor_data(g, i), s.n_in, s.n_out);
}

// Weights concatenated along the output dimension: rows appended, per-block scales side by side.
host_weight concat(const std::vector<host_weight> & parts) {
    host_weight h;
    h.n_in = parts[0].n_in;
    for (const auto & p : parts) h.n_out += p.n_out;
    const int n_blk = (h.n_in + 255) / 256;
    h.scale.resize((size_t) n_blk * h.n_out);
    int col = 0;
    for (const auto & p : parts) {
        h.w.insert(h.w.end(), p.w.begin(), p.w.end());
        for (int B = 0; B < n_blk; ++B) {
            std::copy(p.scale.begin() + (size_t) B * p.n_out, p.scale.begin() + (size_t) (B + 1) * p.n_out,
                      h.scale.begin() + (size_t) B * h.n_out + col);
        }
        col += p.n_out;
    }
    return h;
}

struct qact {
    int8_t * q = nullptr;
    float * sx = nullptr;
};

struct gemm_step {
    std::string key;           // activation (name/n_in/rows)
    bool quantize_first;       // quantize its f32 rows before this GEMM
    nxg_weight * w;
    bool residual, block_rows, relu2;
    std::string out_key;       // the fp32 rows (or, relu2, the qact) it writes
    int n_in, n_out, rows;
    int64_t ops;
};

struct path {
    int T = 0, rows = 0, rows_block = 0;
    std::vector<int32_t> cu, cub;
    std::vector<gemm_step> steps;
    std::map<std::string, float *> inputs;     // synthetic producer outputs
    std::map<std::string, qact> qacts;
    std::map<std::string, float *> outs;
    float * residual = nullptr;
    std::vector<nxg_weight *> weights;
    std::vector<void *> buffers;
    int64_t ops = 0;
    int n_quant = 0, n_relu2 = 0;

    void * alloc(size_t bytes) {
        void * p = nullptr;
        hip_check(hipMalloc(&p, std::max<size_t>(bytes, 16)), "hipMalloc");
        buffers.push_back(p);
        return p;
    }
    ~path() {
        for (void * b : buffers) (void) hipFree(b);
        for (nxg_weight * w : weights) nxg_weight_destroy(w);
    }
};

void fill_random(float * dev, size_t n, std::mt19937_64 & rng) {
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::vector<float> h(n);
    for (float & x : h) x = nd(rng);
    hip_check(hipMemcpy(dev, h.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
}

void build_path(path & P, int T, int B, const nxg_gguf * g) {
    std::mt19937_64 rng(0);
    P.T = T;
    P.rows = T * B;
    const int blk = (T + HRA_BLOCK - 1) / HRA_BLOCK;
    P.rows_block = blk * B;
    for (int b = 0; b <= B; ++b) {
        P.cu.push_back(b * T);
        P.cub.push_back(b * blk);
    }
    P.residual = (float *) P.alloc((size_t) P.rows * N_EMBD * sizeof(float));
    fill_random(P.residual, (size_t) P.rows * N_EMBD, rng);
    for (int l = 0; l < 18; ++l) {
        // group the layer's linears by input, in order of first appearance
        std::vector<std::vector<spec>> groups;
        std::map<std::string, size_t> group_of;
        for (const spec & s : layer_linears(l, BLOCK_TYPES[l])) {
            auto it = group_of.find(s.input);
            if (it == group_of.end()) {
                group_of[s.input] = groups.size();
                groups.push_back({ s });
            } else {
                groups[it->second].push_back(s);
            }
        }
        std::map<std::string, bool> seen, made;
        for (const auto & grp : groups) {
            const spec & s0 = grp[0];
            const int rows = s0.block_rows ? P.rows_block : P.rows;
            int n_out = 0;
            for (const spec & s : grp) n_out += s.n_out;
            const std::string key = s0.input + "/" + std::to_string(s0.n_in) + "/" + std::to_string(rows);
            if (!P.qacts.count(key)) {
                qact a;
                a.q = (int8_t *) P.alloc(nxg_qact_q_bytes(rows, s0.n_in));
                a.sx = (float *) P.alloc(nxg_qact_sx_bytes(rows, s0.n_in));
                P.qacts[key] = a;
            }
            const bool is_made = made.count(key) > 0;
            if (!is_made && !P.inputs.count(key)) {
                float * x = (float *) P.alloc((size_t) rows * s0.n_in * sizeof(float));
                fill_random(x, (size_t) rows * s0.n_in, rng);
                P.inputs[key] = x;
            }
            gemm_step st;
            st.key = key;
            st.quantize_first = !is_made && !seen.count(key);
            seen[key] = true;
            st.relu2 = grp.size() == 1 && !s0.relu2_into.empty();
            st.residual = false;
            for (const spec & s : grp) st.residual = st.residual || s.residual;
            st.block_rows = s0.block_rows;
            st.n_in = s0.n_in;
            st.n_out = n_out;
            st.rows = rows;
            st.ops = 2LL * rows * s0.n_in * n_out;
            if (st.relu2) {
                st.out_key = s0.relu2_into + "/" + std::to_string(n_out) + "/" + std::to_string(rows);
                if (!P.qacts.count(st.out_key)) {
                    qact a;
                    a.q = (int8_t *) P.alloc(nxg_qact_q_bytes(rows, n_out));
                    a.sx = (float *) P.alloc(nxg_qact_sx_bytes(rows, n_out));
                    P.qacts[st.out_key] = a;
                }
                made[st.out_key] = true;
                ++P.n_relu2;
            } else {
                st.out_key = std::to_string(n_out) + "/" + std::to_string(rows);
                if (!P.outs.count(st.out_key)) P.outs[st.out_key] = (float *) P.alloc((size_t) rows * n_out * sizeof(float));
            }
            std::vector<host_weight> parts;
            for (const spec & s : grp) parts.push_back(g ? file_weight(g, s) : random_weight(s.n_in, s.n_out, rng));
            const host_weight hw = parts.size() == 1 ? std::move(parts[0]) : concat(parts);
            nxg_weight * w = nullptr;
            check(nxg_weight_create(hw.w.data(), hw.scale.data(), hw.n_in, hw.n_out, &w), "weight_create");
            P.weights.push_back(w);
            st.w = w;
            if (st.quantize_first) ++P.n_quant;
            P.ops += st.ops;
            P.steps.push_back(st);
        }
    }
}

// One pass on `stream`; with events, each launch is bracketed (kind 0 quantize, 1 GEMM fp32
// out, 2 GEMM relu^2 -> int8).
struct timed {
    hipEvent_t a, b;
    int kind;
};

void run_pass(path & P, hipStream_t stream, std::vector<timed> * ev) {
    const int n_seqs = (int) P.cu.size() - 1;
    auto mark = [&](int kind, auto && fn) {
        if (!ev) {
            fn();
            return;
        }
        timed t;
        t.kind = kind;
        hip_check(hipEventCreate(&t.a), "hipEventCreate");
        hip_check(hipEventCreate(&t.b), "hipEventCreate");
        hip_check(hipEventRecord(t.a, stream), "hipEventRecord");
        fn();
        hip_check(hipEventRecord(t.b, stream), "hipEventRecord");
        ev->push_back(t);
    };
    for (const gemm_step & st : P.steps) {
        const qact & a = P.qacts[st.key];
        const int32_t * cu = st.block_rows ? P.cub.data() : P.cu.data();
        if (st.quantize_first) {
            mark(0, [&] { check(nxg_quantize_rows(P.inputs[st.key], st.rows, st.n_in, 127, a.q, a.sx, stream), "quantize_rows"); });
        }
        if (st.relu2) {
            const qact & o = P.qacts[st.out_key];
            mark(2, [&] { check(nxg_linear_i8_relu2_q8(st.w, a.q, a.sx, cu, n_seqs, 127, o.q, o.sx, stream), "linear_i8_relu2_q8"); });
        } else {
            mark(1, [&] { check(nxg_linear_i8(st.w, a.q, a.sx, cu, n_seqs, st.residual ? P.residual : nullptr,
                                              P.outs[st.out_key], stream), "linear_i8"); });
        }
    }
}

std::string ftype_of(const nxg_gguf * g) {
    static const std::map<int64_t, const char *> names = {   // src/nexterabert.cpp:1390-1410
        { 0, "F32" }, { 1, "F16" }, { 2, "Q4_0" }, { 3, "Q4_1" }, { 7, "Q8_0" }, { 8, "Q5_0" }, { 9, "Q5_1" },
        { 10, "Q2_K" }, { 11, "Q3_K_S" }, { 12, "Q3_K_M" }, { 13, "Q3_K_L" }, { 14, "Q4_K_S" }, { 15, "Q4_K_M" },
        { 16, "Q5_K_S" }, { 17, "Q5_K_M" }, { 18, "Q6_K" } };
    if (!g) return "Q8_0 (random weights)";
    const int64_t i = nxg_gguf_find_key(g, "general.file_type");
    int64_t v = -1;
    if (i >= 0 && nxg_gguf_get_i64(g, i, &v) == NXG_OK && names.count(v)) return names.at(v);
    return "unknown";
}

void usage(const char * argv0) {
    fprintf(stderr,
            "usage: %s [-m model.gguf] [--info] [--bench T [--batch B] [--reps R] [--graph] [--profile]]\n\n"
            "  -m FILE      GGUF file with the encoder's weights (default: random Q8_0)\n"
            "  --info       print device and model info\n"
            "  --bench T    time passes of the int8 linear path over random sequences of T tokens\n"
            "  --batch B    sequences per pass (default 1)\n"
            "  --reps R     timed repetitions (default 20)\n"
            "  --graph      replay each pass from a HIP graph\n"
            "  --encode     with --bench and -m: time the whole encoder (nxg_encoder_encode)\n"
            "  --profile    print the device time per kind of launch\n",
            argv0);
}

} // namespace

int main(int argc, char ** argv) {
    const char * model = nullptr;
    bool info = false, graph = false, profile = false, encode = false;
    int bench_t = 0, batch = 1, reps = 20;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> const char * {
            if (i + 1 >= argc) {
                usage(argv[0]);
                exit(1);
            }
            return argv[++i];
        };
        if (a == "-m" || a == "--model") model = next();
        else if (a == "--info") info = true;
        else if (a == "--bench") bench_t = atoi(next());
        else if (a == "--batch") batch = atoi(next());
        else if (a == "--reps") reps = atoi(next());
        else if (a == "--graph") graph = true;
        else if (a == "--profile") profile = true;
        else if (a == "--encode") encode = true;
        else if (a == "-h" || a == "--help") {
            usage(argv[0]);
            return 0;
        } else {
            usage(argv[0]);
            return 1;
        }
    }
    if (bench_t < 0 || batch < 1 || reps < 1) {
        usage(argv[0]);
        return 1;
    }
    nxg_gguf * g = nullptr;
    if (model) check(nxg_gguf_open(model, &g), "gguf_open");
    if (info || !bench_t) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess) {
            printf("device: %s (%s), %d CUs, %.0f GiB\n", prop.name, prop.gcnArchName, prop.multiProcessorCount,
                   prop.totalGlobalMem / 1073741824.0);
        } else {
            printf("device: none\n");
        }
        if (g) {
            printf("model: GGUF v%u, %s, %lld tensors\n", nxg_gguf_version(g), ftype_of(g).c_str(),
                   (long long) nxg_gguf_n_tensors(g));
        }
    }
    if (bench_t > 0 && encode) {
        if (!model) {
            fprintf(stderr, "nxg-cli: --encode needs -m model.gguf\n");
            return 1;
        }
        auto kv_id = [&](const char * key) -> int32_t {
            const int64_t i = nxg_gguf_find_key(g, key);
            int64_t v = -1;
            return i >= 0 && nxg_gguf_get_i64(g, i, &v) == NXG_OK ? (int32_t) v : -1;
        };
        const int32_t cls = kv_id("tokenizer.ggml.cls_token_id"), sep = kv_id("tokenizer.ggml.seperator_token_id");
        nxg_encoder_params ep = nxg_encoder_default_params();
        nxg_encoder * enc = nullptr;
        check(nxg_encoder_load(model, &ep, &enc), "encoder_load");
        const int32_t n_vocab = nxg_encoder_n_vocab(enc), n_embd = nxg_encoder_n_embd(enc);
        std::mt19937 rng(0);
        const int32_t hi = std::min(n_vocab, 40000);
        std::uniform_int_distribution<int32_t> dist(std::min(1000, hi - 1), hi - 1);   // a tiny vocabulary: from below 1000
        std::vector<int32_t> tokens((size_t) bench_t * batch), lengths(batch, bench_t);
        for (int32_t & t : tokens) t = dist(rng);
        for (int b = 0; b < batch; ++b) {
            if (cls >= 0 && cls < n_vocab) tokens[(size_t) b * bench_t] = cls;
            if (sep >= 0 && sep < n_vocab) tokens[(size_t) (b + 1) * bench_t - 1] = sep;
        }
        std::vector<float> pooled((size_t) batch * n_embd);
        std::vector<double> ms;
        for (int r = 0; r < reps + 3; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            check(nxg_encoder_encode(enc, tokens.data(), nullptr, lengths.data(), batch, nullptr, pooled.data(), 1),
                  "encoder_encode");
            const auto t1 = std::chrono::steady_clock::now();
            if (r >= 3) ms.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
            if (r == 2 && profile) nxg_encoder_profile(enc, 1);   // the timed passes, as tools/cli.cpp:196
        }
        std::sort(ms.begin(), ms.end());
        const double med = ms[ms.size() / 2];
        printf("bench: %s  T=%d  batch=%d  encoder  median %.3f ms  min %.3f ms  (%.0f tokens/s)\n", ftype_of(g).c_str(),
               bench_t, batch, med, ms.front(), 1000.0 * bench_t * batch / med);
        if (profile) {
            double kind[NXG_PROF_COUNT] = {}, dev_ms = 0.0, wall = 0.0;
            int64_t passes = 0;
            check(nxg_encoder_profile_read(enc, kind, &dev_ms, &wall, &passes), "encoder_profile_read");
            const char * names[3] = { "int8 linear", "attention", "norm / conv / gate / quantize" };
            const double n = (double) std::max<int64_t>(passes, 1), total = std::max(wall, 1e-9);
            double sum = 0.0;
            printf("profile over %lld forward passes (ms per pass, GPU time from HIP events):\n", (long long) passes);
            for (int k = 0; k < 3; ++k) {
                sum += kind[k];
                printf("  %-22s %8.3f  %5.1f%%\n", names[k], kind[k] / n, 100.0 * kind[k] / total);
            }
            printf("  %-22s %8.3f  %5.1f%%   (embedding rows, out_norm, copies, launch gaps, host)\n", "everything else",
                   (total - sum) / n, 100.0 * (total - sum) / total);
            printf("  %-22s %8.3f\n", "total", total / n);
        }
        nxg_encoder_free(enc);
        nxg_gguf_close(g);
        return 0;
    }
    if (bench_t > 0) {
        check(nxg_init(), "init");
        hipStream_t stream;
        hip_check(hipStreamCreate(&stream), "hipStreamCreate");
        {
            path P;
            build_path(P, bench_t, batch, g);
            hipGraphExec_t exec = nullptr;
            if (graph) {
                run_pass(P, stream, nullptr);
                hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
                hipGraph_t gr;
                hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
                run_pass(P, stream, nullptr);
                hip_check(hipStreamEndCapture(stream, &gr), "hipStreamEndCapture");
                hip_check(hipGraphInstantiate(&exec, gr, nullptr, nullptr, 0), "hipGraphInstantiate");
                hip_check(hipGraphDestroy(gr), "hipGraphDestroy");
            }
            std::vector<double> ms;
            for (int r = 0; r < reps + 3; ++r) {
                const auto t0 = std::chrono::steady_clock::now();
                if (exec) hip_check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
                else      run_pass(P, stream, nullptr);
                hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
                const auto t1 = std::chrono::steady_clock::now();
                if (r >= 3) ms.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
            }
            std::sort(ms.begin(), ms.end());
            const double med = ms[ms.size() / 2];
            printf("bench: %s  T=%d  batch=%d  %s  median %.3f ms  min %.3f ms  (%.0f tokens/s)\n", ftype_of(g).c_str(),
                   bench_t, batch, exec ? "graph" : "eager", med, ms.front(), 1000.0 * bench_t * batch / med);
            printf("  %zu GEMMs (%d relu^2 -> int8) + %d quantizations, %.1f G int8 ops per pass: %.1f TOPS at the median\n",
                   P.steps.size(), P.n_relu2, P.n_quant, P.ops / 1e9, P.ops / (med * 1e-3) / 1e12);
            if (profile) {
                std::vector<timed> ev;
                run_pass(P, stream, &ev);
                hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
                const char * names[3] = { "quantize", "GEMM fp32 out", "GEMM relu^2 -> int8" };
                double t[3] = { 0, 0, 0 };
                int n[3] = { 0, 0, 0 };
                for (timed & e : ev) {
                    float x = 0;
                    hip_check(hipEventElapsedTime(&x, e.a, e.b), "hipEventElapsedTime");
                    t[e.kind] += x;
                    ++n[e.kind];
                    (void) hipEventDestroy(e.a);
                    (void) hipEventDestroy(e.b);
                }
                const double total = t[0] + t[1] + t[2];
                for (int k = 0; k < 3; ++k) {
                    printf("  %-22s %4d launches  %8.3f ms  %5.1f%%\n", names[k], n[k], t[k], 100.0 * t[k] / total);
                }
            }
            if (exec) hip_check(hipGraphExecDestroy(exec), "hipGraphExecDestroy");
        }
        hip_check(hipStreamDestroy(stream), "hipStreamDestroy");
    }
    if (g) nxg_gguf_close(g);
    return 0;
}
