// nexterabert_api.cpp -- the reference's public C API (include/nexterabert.h; the reference's
// src/nexterabert.h:28-123 and the diagnostics of src/nexterabert.cpp:1815-1841) over the GPU
// encoder (include/nxg_encoder.h). Built into libnexterabert.so, the library name the
// reference's binding looks for (python/nexterabert_cpp.py:31-44), linked to libnxg.so.
//
// nextera_load reads the metadata the encoder does not use (heads, token ids, tokenizer,
// file type) from the same file, with nextera_load's keys and defaults
// (src/nexterabert.cpp:1570-1637), checks the head tensors the reference requires
// (required_tensors, :1462-1496), then loads the encoder onto the current HIP device.
// Errors go to stderr prefixed "nexterabert: ", as the reference prints them.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "nexterabert.h"
#include "nxg_encoder.h"
#include "nxg_gguf.h"

struct nextera_context {
    nxg_encoder * enc = nullptr;
    int32_t n_threads = 1;
    int32_t has_mlm = 0, has_pooler = 0, n_labels = 0;
    int32_t cls_id = -1, sep_id = -1, pad_id = -1, mask_id = -1;
    std::string task, tokenizer_json, ftype, sysinfo;
    std::vector<std::string> labels;
    double last_ms = 0.0;
};

namespace {

// The reference's classifier task names (CLS_NAMES, src/nexterabert.cpp:207-209).
const char * const TASKS[] = { "sequence-classification", "multiple-choice", "token-classification",
                               "question-answering" };

// general.file_type -> name, as ftype_name (src/nexterabert.cpp:1390-1410) names llama.cpp's
// file types.
const char * ftype_name(int64_t ft) {
    switch (ft) {
        case 0: return "F32";
        case 1: return "F16";
        case 2: return "Q4_0";
        case 3: return "Q4_1";
        case 7: return "Q8_0";
        case 8: return "Q5_0";
        case 9: return "Q5_1";
        case 10: return "Q2_K";
        case 11: return "Q3_K_S";
        case 12: return "Q3_K_M";
        case 13: return "Q3_K_L";
        case 14: return "Q4_K_S";
        case 15: return "Q4_K_M";
        case 16: return "Q5_K_S";
        case 17: return "Q5_K_M";
        case 18: return "Q6_K";
        default: return "unknown";
    }
}

int32_t default_threads() {
    const int hw = (int) std::max(1u, std::thread::hardware_concurrency());
    return hw - hw / 10;
}

void report(const char * what) { fprintf(stderr, "nexterabert: %s\n", what); }

struct gguf_file {
    nxg_gguf * g = nullptr;
    ~gguf_file() { nxg_gguf_close(g); }
    std::string str(const char * key, const char * def) const {
        const int64_t id = nxg_gguf_find_key(g, key);
        const char * s = nullptr;
        uint64_t n = 0;
        if (id < 0 || nxg_gguf_get_str(g, id, &s, &n) != NXG_OK) return def;
        return std::string(s, (size_t) n);
    }
    // kv_u32's reading of a token id: (int32_t) of the stored unsigned value, default -1
    int32_t id32(const char * key) const {
        const int64_t id = nxg_gguf_find_key(g, key);
        int64_t v = -1;
        if (id < 0 || nxg_gguf_get_i64(g, id, &v) != NXG_OK) return -1;
        return (int32_t) (uint32_t) v;
    }
    bool has_tensor(const char * name) const { return nxg_gguf_find_tensor(g, name) >= 0; }
};

// Reads everything nextera_load keeps besides the encoder; false (reason printed) for a file
// the reference refuses.
bool read_metadata(const char * path, nextera_context & c) {
    gguf_file f;
    if (nxg_gguf_open(path, &f.g) != NXG_OK) {
        fprintf(stderr, "nexterabert: failed to open '%s' (%s)\n", path, nxg_last_error());
        return false;
    }
    const std::string arch = f.str("general.architecture", "");
    if (arch != "nexterabert") {
        fprintf(stderr, "nexterabert: '%s' is not a nexterabert GGUF (general.architecture = '%s')\n", path, arch.c_str());
        return false;
    }
    c.cls_id = f.id32("tokenizer.ggml.cls_token_id");
    c.sep_id = f.id32("tokenizer.ggml.seperator_token_id");
    c.pad_id = f.id32("tokenizer.ggml.padding_token_id");
    c.mask_id = f.id32("tokenizer.ggml.mask_token_id");
    {
        const int64_t id = nxg_gguf_find_key(f.g, "nexterabert.mlm_head");
        int64_t v = 0;
        c.has_mlm = id >= 0 && nxg_gguf_get_i64(f.g, id, &v) == NXG_OK && v != 0;
    }
    const std::string task = f.str("nexterabert.classifier.task", "");
    for (const char * t : TASKS) {
        if (task == t) c.task = t;
    }
    if (!task.empty() && c.task.empty()) {
        fprintf(stderr, "nexterabert: unsupported classifier task '%s'\n", task.c_str());
        return false;
    }
    {
        const int64_t id = nxg_gguf_find_key(f.g, "nexterabert.classifier.labels");
        int32_t et = -1;
        uint64_t n = 0;
        if (id >= 0 && nxg_gguf_arr_info(f.g, id, &et, &n) == NXG_OK) {
            for (uint64_t i = 0; i < n; ++i) {
                const char * s = nullptr;
                uint64_t len = 0;
                if (nxg_gguf_arr_str(f.g, id, i, &s, &len) != NXG_OK) break;
                c.labels.emplace_back(s, (size_t) len);
            }
        }
    }
    c.tokenizer_json = f.str("tokenizer.huggingface.json", "");
    {
        const int64_t id = nxg_gguf_find_key(f.g, "general.file_type");
        int64_t ft = 0;
        if (id >= 0) (void) nxg_gguf_get_i64(f.g, id, &ft);
        c.ftype = ftype_name(ft);
    }
    c.has_pooler = f.has_tensor("pooler.dense.weight") && f.has_tensor("pooler.norm.weight");
    if (!c.task.empty()) {
        const int64_t b = nxg_gguf_find_tensor(f.g, "classifier.bias");
        int32_t type = 0, nd = 0;
        int64_t ne[4] = { 0, 0, 0, 0 };
        if (b >= 0 && nxg_gguf_tensor_info(f.g, b, &type, &nd, ne, nullptr, nullptr) == NXG_OK) c.n_labels = (int32_t) ne[0];
        if ((int32_t) c.labels.size() != c.n_labels) c.labels.clear();
    }
    // the head tensors required_tensors asks for (the encoder's own are checked by its loader)
    std::vector<std::string> req;
    if (c.has_mlm) req = { "mlm.dense.weight", "mlm.norm.weight", "mlm.bias" };
    if (!c.task.empty()) {
        const bool pooled = c.task == TASKS[0] || c.task == TASKS[1];
        const std::string pre = pooled ? "pooler." : "head.";
        for (const std::string & n : { std::string("classifier.weight"), std::string("classifier.bias"),
                                       pre + "dense.weight", pre + "norm.weight" }) {
            req.push_back(n);
        }
    }
    for (const std::string & n : req) {
        if (f.has_tensor(n.c_str())) continue;
        fprintf(stderr, "nexterabert: '%s' has no tensor '%s': not a complete nexterabert file\n", path, n.c_str());
        return false;
    }
    return true;
}

int32_t failed(int32_t rc) {
    if (rc != NXG_OK) report(nxg_last_error());
    return rc;
}

// The heads are outside the engine: the reference's message when the file lacks the head,
// otherwise this engine's.
int32_t no_head(bool present, const char * absent, const char * what) {
    report(present ? what : absent);
    return 1;
}

} // namespace

extern "C" {

struct nextera_params nextera_default_params(void) {
    nextera_params p;
    p.n_threads = 0;
    p.use_int8 = 1;
    p.use_repack = 1;
    p.verbosity = 0;
    return p;
}

struct nextera_context * nextera_load(const char * path, struct nextera_params params) {
    const auto t0 = std::chrono::steady_clock::now();
    if (!path) {
        report("no model path");
        return nullptr;
    }
    if (!params.use_int8) {
        report("use_int8 = 0 asks for ggml's kernels, which this engine does not have: every encoder linear runs "
               "on the GPU int8 GEMM");
        return nullptr;
    }
    nextera_context * c = new (std::nothrow) nextera_context();
    if (!c) {
        report("out of host memory");
        return nullptr;
    }
    c->n_threads = params.n_threads > 0 ? params.n_threads : default_threads();
    if (!read_metadata(path, *c)) {
        delete c;
        return nullptr;
    }
    nxg_encoder_params ep = nxg_encoder_default_params();
    ep.act_max = 127;
    ep.load_threads = c->n_threads;
    ep.verbosity = 0;
    if (nxg_encoder_load(path, &ep, &c->enc) != NXG_OK) {
        report(nxg_last_error());
        delete c;
        return nullptr;
    }
    int dev = 0;
    hipDeviceProp_t prop;
    char gpu[600] = "unknown";
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess) {
        snprintf(gpu, sizeof(gpu), "%s (%s), %d CUs", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    }
    char info[900];
    snprintf(info, sizeof(info),
             "GPU = %s | linear layers: %d int8 (MFMA v_mfma_i32_16x16x64_i8, ACT_MAX 127), 0 ggml repack | "
             "custom ops: HIP",
             gpu, nxg_encoder_n_int8(c->enc));
    c->sysinfo = info;
    if (params.verbosity > 0) {
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        fprintf(stderr, "nexterabert: %s | %s | %d layers, n_embd %d | device memory %.1f MiB | loaded in %.0f ms\n", path,
                c->ftype.c_str(), nxg_encoder_n_layer(c->enc), nxg_encoder_n_embd(c->enc),
                nxg_encoder_device_bytes(c->enc) / 1048576.0, ms);
        fprintf(stderr, "nexterabert: n_threads = %d | %s\n", c->n_threads, c->sysinfo.c_str());
        if (!c->task.empty()) fprintf(stderr, "nexterabert: classifier: %s, %d labels\n", c->task.c_str(), c->n_labels);
    }
    return c;
}

void nextera_free(struct nextera_context * c) {
    if (!c) return;
    nxg_encoder_free(c->enc);
    delete c;
}

int32_t nextera_n_embd(const struct nextera_context * c) { return nxg_encoder_n_embd(c->enc); }
int32_t nextera_n_vocab(const struct nextera_context * c) { return nxg_encoder_n_vocab(c->enc); }
int32_t nextera_n_layer(const struct nextera_context * c) { return nxg_encoder_n_layer(c->enc); }
int32_t nextera_has_mlm_head(const struct nextera_context * c) { return c->has_mlm; }
int32_t nextera_has_pooler(const struct nextera_context * c) { return c->has_pooler; }
int32_t nextera_n_token_types(const struct nextera_context * c) { return nxg_encoder_n_token_types(c->enc); }
const char * nextera_classifier_task(const struct nextera_context * c) { return c->task.c_str(); }
int32_t nextera_n_labels(const struct nextera_context * c) { return c->n_labels; }
const char * nextera_label(const struct nextera_context * c, int32_t i) {
    return i >= 0 && i < (int32_t) c->labels.size() ? c->labels[(size_t) i].c_str() : "";
}
int32_t nextera_token_cls(const struct nextera_context * c) { return c->cls_id; }
int32_t nextera_token_sep(const struct nextera_context * c) { return c->sep_id; }
int32_t nextera_token_pad(const struct nextera_context * c) { return c->pad_id; }
int32_t nextera_token_mask(const struct nextera_context * c) { return c->mask_id; }
const char * nextera_tokenizer_json(const struct nextera_context * c) { return c->tokenizer_json.c_str(); }
const char * nextera_ftype(const struct nextera_context * c) { return c->ftype.c_str(); }
const char * nextera_system_info(const struct nextera_context * c) { return c->sysinfo.c_str(); }
int32_t nextera_get_n_threads(const struct nextera_context * c) { return c->n_threads; }
double nextera_last_ms(const struct nextera_context * c) { return c->last_ms; }

void nextera_set_n_threads(struct nextera_context * c, int32_t n_threads) {
    c->n_threads = n_threads > 0 ? n_threads : default_threads();
}

int32_t nextera_encode(struct nextera_context * c, const int32_t * tokens, const int32_t * lengths, int32_t n_seqs,
                       float * hidden, float * pooled, int32_t normalize) {
    return nextera_encode_segments(c, tokens, nullptr, lengths, n_seqs, hidden, pooled, normalize);
}

int32_t nextera_encode_segments(struct nextera_context * c, const int32_t * tokens, const int32_t * token_types,
                                const int32_t * lengths, int32_t n_seqs, float * hidden, float * pooled,
                                int32_t normalize) {
    const auto t0 = std::chrono::steady_clock::now();
    const int32_t rc = failed(nxg_encoder_encode(c->enc, tokens, token_types, lengths, n_seqs, hidden, pooled, normalize));
    c->last_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return rc;
}

int32_t nextera_pooler_output(struct nextera_context * c, const int32_t *, const int32_t *, const int32_t *, int32_t,
                              float *) {
    return no_head(c->has_pooler, "this file has no pooler",
                   "pooler_output is a head, which this engine does not run (it runs the encoder: nextera_encode)");
}

int32_t nextera_classify(struct nextera_context * c, const int32_t *, const int32_t *, const int32_t *, int32_t,
                         float *) {
    return no_head(!c->task.empty(), "this file has no classifier head",
                   "the classifier is a head, which this engine does not run (it runs the encoder: nextera_encode)");
}

int32_t nextera_mlm_logits(struct nextera_context * c, const int32_t *, int32_t, const int32_t *, int32_t, float *) {
    return no_head(c->has_mlm != 0, "this file has no MLM head",
                   "the MLM head is a head, which this engine does not run (it runs the encoder: nextera_encode)");
}

void nextera_debug_set_layers(struct nextera_context * c, int32_t n_layers) { nxg_encoder_set_layers(c->enc, n_layers); }

void nextera_debug_profile(struct nextera_context * c, int32_t enable) { nxg_encoder_profile(c->enc, enable); }

// The reference's report (src/nexterabert.cpp:1828-1841): ms per pass and share of the total
// for each kind, then the rest of the wall time, then the total.
void nextera_debug_profile_print(const struct nextera_context * c) {
    double kind[NXG_PROF_COUNT] = {}, device = 0.0, wall = 0.0;
    int64_t passes = 0;
    if (nxg_encoder_profile_read(c->enc, kind, &device, &wall, &passes) != NXG_OK || passes == 0) return;
    static const char * const names[3] = { "int8 linear", "attention", "norm / conv / gate / quantize" };
    const double total = std::max(wall, 1e-9);
    double sum = 0.0;
    fprintf(stderr, "profile over %lld forward passes (ms per pass, GPU time from HIP events):\n", (long long) passes);
    for (int i = 0; i < 3; ++i) {
        sum += kind[i];
        fprintf(stderr, "  %-22s %8.3f  %5.1f%%\n", names[i], kind[i] / passes, 100.0 * kind[i] / total);
    }
    fprintf(stderr, "  %-22s %8.3f  %5.1f%%   (embedding rows, out_norm, copies, launch gaps, host)\n",
            "everything else", (total - sum) / passes, 100.0 * (total - sum) / total);
    fprintf(stderr, "  %-22s %8.3f\n", "total", total / passes);
}

} // extern "C"
