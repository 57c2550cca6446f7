// Checkpoint layouts of the reference, host side: the quantized GPT's TGMT
// file (src/GPT.swift:265-324) and the DiT's TDIT file (src/DiT.swift:
// 396-451). Both are a little-endian header followed by every parameter's
// fp32 master, in the order the model creates its parameters. The functions
// here validate a file image and give each parameter's name, shape, flags and
// byte offset; the caller uploads the masters and re-quantizes (GPT.load
// calls quantizeAll after reading, src/GPT.swift:318-322). No GPU work, no
// context: plain host code over the caller's bytes.
#include <cstdio>
#include <cstring>

#include "common.hpp"

namespace {

uint32_t rd_u32(const uint8_t* p) {
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24);
}

float rd_f32(const uint8_t* p) {
    const uint32_t u = rd_u32(p);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

void set(dgm_param_info* o, const char* name, int64_t rows, int64_t cols, int quantized, int decay,
         int64_t offset) {
    std::snprintf(o->name, sizeof(o->name), "%s", name);
    o->rows = rows;
    o->cols = cols;
    o->quantized = quantized;
    o->decay = decay;
    o->offset = offset;
}

// ---- TGMT: GPT.init's make() order (src/GPT.swift:118-131 and Block.init,
// src/GPT.swift:44-64): wte, wpe, per layer 16 parameters, ln_f.g, ln_f.b.
constexpr int64_t kTgmtHeader = 4 + 4 * 8;
constexpr int kPerLayer = 16;

// One layer's parameters in Block.init's order; rows/cols code -1 = embd,
// -2 = mlp width (4 * embd).
struct LayerParam {
    const char* name;
    int rows, cols, quant, decay;
};
constexpr LayerParam kLayer[kPerLayer] = {
    {"ln1.g", -1, 1, 0, 0}, {"ln1.b", -1, 1, 0, 0}, {"wq", -1, -1, 1, 1}, {"bq", -1, 1, 0, 0},
    {"wk", -1, -1, 1, 1},   {"bk", -1, 1, 0, 0},    {"wv", -1, -1, 1, 1}, {"bv", -1, 1, 0, 0},
    {"wo", -1, -1, 1, 1},   {"bo", -1, 1, 0, 0},    {"ln2.g", -1, 1, 0, 0}, {"ln2.b", -1, 1, 0, 0},
    {"fc", -2, -1, 1, 1},   {"fc.b", -2, 1, 0, 0},  {"proj", -1, -2, 1, 1}, {"proj.b", -1, 1, 0, 0}};

int64_t dim(int code, int64_t C) { return code == -1 ? C : (code == -2 ? 4 * C : code); }

// Fills `o` for parameter i (byte offsets from the file start, the first
// parameter at `base`) and returns the number of floats it holds, or -1 past
// the end.
int64_t tgmt_param(const dgm_tgmt_header& h, int64_t i, dgm_param_info* o, int64_t base) {
    const int64_t C = h.embd, V = h.vocab, Tb = h.block;
    const int q = h.bits != 32;
    const int64_t nparams = 2 + int64_t(h.layers) * kPerLayer + 2;
    if (i < 0 || i >= nparams) return -1;
    int64_t layer_floats = 0;
    for (const LayerParam& p : kLayer) layer_floats += dim(p.rows, C) * dim(p.cols, C);
    if (i == 0) {
        set(o, "wte", V, C, q, 1, base);
        return V * C;
    }
    if (i == 1) {
        set(o, "wpe", Tb, C, 0, 1, base + 4 * V * C);
        return Tb * C;
    }
    const int64_t after_layers = base + 4 * (V * C + Tb * C + int64_t(h.layers) * layer_floats);
    if (i == nparams - 2) {
        set(o, "ln_f.g", C, 1, 0, 0, after_layers);
        return C;
    }
    if (i == nparams - 1) {
        set(o, "ln_f.b", C, 1, 0, 0, after_layers + 4 * C);
        return C;
    }
    const int64_t layer = (i - 2) / kPerLayer, k = (i - 2) % kPerLayer;
    int64_t off = base + 4 * (V * C + Tb * C + layer * layer_floats);
    for (int64_t j = 0; j < k; ++j) off += 4 * dim(kLayer[j].rows, C) * dim(kLayer[j].cols, C);
    char name[32];
    std::snprintf(name, sizeof(name), "b%lld.%s", (long long)layer, kLayer[k].name);
    const int64_t rows = dim(kLayer[k].rows, C), cols = dim(kLayer[k].cols, C);
    set(o, name, rows, cols, kLayer[k].quant && q, kLayer[k].decay, off);
    return rows * cols;
}

bool tgmt_valid(const dgm_tgmt_header& h) {
    // GPTConfig.validate (src/Params.swift:163-173).
    if (h.block == 0 || h.layers == 0 || h.heads == 0 || h.embd == 0 || h.vocab < 2) return false;
    if (h.embd % h.heads != 0) return false;
    if (h.bits != 4 && h.bits != 8 && h.bits != 32) return false;
    if (h.bits != 32) {
        if (h.qGroup == 0 || h.embd % h.qGroup != 0 || (4 * uint64_t(h.embd)) % h.qGroup != 0 || h.qGroup % 2 != 0)
            return false;
    }
    return h.layers <= 4096 && h.embd <= (1u << 20) && h.vocab <= (1u << 24) && h.block <= (1u << 24);
}

// ---- TDIT: DiT.init's make() order (src/DiT.swift:233-250).
constexpr int kTditParams = 17;

int64_t tdit_param(const dgm_tdit_header& h, int64_t i, dgm_param_info* o, int64_t base) {
    const int64_t C = h.embd, F = h.intermediate, P = int64_t(h.patch) * h.patch * 3;
    const int64_t KV = int64_t(h.kvHeads) * (h.embd / h.heads);
    struct Pm {
        const char* name;
        int64_t rows, cols;
        int decay;
    };
    const Pm table[kTditParams] = {
        {"wpatch", C, P, 0}, {"whead", P, C, 0},  {"wname", int64_t(h.names), C, 1}, {"wtime1", C, int64_t(h.freqDim), 0},
        {"wtime2", C, C, 0}, {"wq", C, C, 0},     {"wk", KV, C, 0},                  {"wv", KV, C, 0},
        {"wo", C, C, 0},     {"wgate", F, C, 0},  {"wup", F, C, 0},                  {"wdown", C, F, 0},
        {"n1", C, 1, 0},     {"n1b", C, 1, 0},    {"n2", C, 1, 0},                   {"n2b", C, 1, 0},
        {"nf", C, 1, 0}};
    if (i < 0 || i >= kTditParams) return -1;
    int64_t off = base;
    for (int64_t j = 0; j < i; ++j) off += 4 * table[j].rows * table[j].cols;
    set(o, table[i].name, table[i].rows, table[i].cols, 0, table[i].decay, off);
    return table[i].rows * table[i].cols;
}

bool tdit_valid(const dgm_tdit_header& h) {
    // DiTConfig.validate (src/DiT.swift:34-40): patch divides side, one KV
    // head, even head dim, even frequency dim of at least 2.
    if (h.side == 0 || h.patch == 0 || h.side % h.patch != 0) return false;
    if (h.names == 0 || h.loops == 0 || h.diffusionSteps < 2) return false;
    if (h.heads == 0 || h.kvHeads != 1 || h.embd == 0 || h.embd % h.heads != 0 || (h.embd / h.heads) % 2 != 0)
        return false;
    if (h.freqDim < 2 || h.freqDim % 2 != 0 || h.intermediate == 0) return false;
    return h.embd <= (1u << 16) && h.intermediate <= (1u << 20) && h.names <= (1u << 20) &&
           h.freqDim <= (1u << 20) && h.patch <= 1024;
}

}  // namespace

extern "C" {

int dgm_tgmt_parse(const void* data, int64_t len, dgm_tgmt_header* hdr, int64_t* itos_offset, int64_t* nparams) {
    if (!data || !hdr || len < 0) return DGM_ERR_ARG;
    const uint8_t* b = static_cast<const uint8_t*>(data);
    if (len < kTgmtHeader || std::memcmp(b, "TGMT", 4) != 0) return DGM_ERR_SHAPE;   // "not a transformer-metal checkpoint"
    dgm_tgmt_header h;
    h.version = rd_u32(b + 4);
    h.bits = rd_u32(b + 8);
    h.vocab = rd_u32(b + 12);
    h.block = rd_u32(b + 16);
    h.layers = rd_u32(b + 20);
    h.heads = rd_u32(b + 24);
    h.embd = rd_u32(b + 28);
    h.qGroup = rd_u32(b + 32);
    if (h.version != 1) return DGM_ERR_SHAPE;   // "unsupported checkpoint version"
    if (!tgmt_valid(h)) return DGM_ERR_SHAPE;
    const int64_t itos = kTgmtHeader;
    const int64_t base = itos + h.vocab;
    const int64_t np = 2 + int64_t(h.layers) * kPerLayer + 2;
    dgm_param_info last;
    const int64_t n = tgmt_param(h, np - 1, &last, base);
    if (n < 0 || last.offset + 4 * n != len) return DGM_ERR_SHAPE;   // "checkpoint length does not match the model"
    *hdr = h;
    if (itos_offset) *itos_offset = itos;
    if (nparams) *nparams = np;
    return DGM_OK;
}

int dgm_tgmt_param(const dgm_tgmt_header* hdr, int64_t i, dgm_param_info* out) {
    if (!hdr || !out) return DGM_ERR_ARG;
    if (!tgmt_valid(*hdr)) return DGM_ERR_SHAPE;
    return tgmt_param(*hdr, i, out, kTgmtHeader + hdr->vocab) < 0 ? DGM_ERR_ARG : DGM_OK;
}

int dgm_tdit_parse(const void* data, int64_t len, dgm_tdit_header* hdr, int64_t* nparams) {
    if (!data || !hdr || len < 0) return DGM_ERR_ARG;
    const uint8_t* b = static_cast<const uint8_t*>(data);
    if (len < 8 + 40 + 4 || std::memcmp(b, "TDIT", 4) != 0) return DGM_ERR_SHAPE;   // "not a diffusion checkpoint"
    dgm_tdit_header h;
    h.version = rd_u32(b + 4);
    if (h.version != 1 && h.version != 2) return DGM_ERR_SHAPE;
    uint32_t f[10];
    for (int i = 0; i < 10; ++i) f[i] = rd_u32(b + 8 + 4 * i);
    h.side = f[0]; h.patch = f[1]; h.names = f[2]; h.loops = f[3]; h.heads = f[4]; h.kvHeads = f[5];
    h.embd = f[6]; h.intermediate = f[7]; h.freqDim = f[8]; h.diffusionSteps = f[9];
    int64_t off = 48;
    // Version 1 has no lastAlpha field (DiT.load defaults it to 0.01).
    if (h.version >= 2) {
        if (len < off + 8) return DGM_ERR_SHAPE;
        h.lastAlpha = rd_f32(b + off);
        off += 4;
    } else {
        h.lastAlpha = 0.01f;
    }
    h.valueMix = rd_f32(b + off);
    off += 4;
    if (!tdit_valid(h)) return DGM_ERR_SHAPE;
    h.header_bytes = uint32_t(off);
    dgm_param_info last;
    const int64_t n = tdit_param(h, kTditParams - 1, &last, off);
    if (n < 0 || last.offset + 4 * n != len) return DGM_ERR_SHAPE;   // "length does not match the model"
    *hdr = h;
    if (nparams) *nparams = kTditParams;
    return DGM_OK;
}

int dgm_tdit_param(const dgm_tdit_header* hdr, int64_t i, dgm_param_info* out) {
    if (!hdr || !out) return DGM_ERR_ARG;
    if (!tdit_valid(*hdr)) return DGM_ERR_SHAPE;
    return tdit_param(*hdr, i, out, hdr->header_bytes) < 0 ? DGM_ERR_ARG : DGM_OK;
}

}  // extern "C"
