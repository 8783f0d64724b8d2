// OLMo-2 model on the device: OlmoModel (OlmoModel.h:14-34) with its blocks (OlmoBlock.cpp),
// MLPs (OlmoMlp.cpp), norms (RMSNorm.cpp), LM head (OlmoLmHead.cpp), and ce_loss
// (CrossEntropyLoss.cpp) with main.cpp's gradient.
//
// Layout: each block owns a dt_attn_layer (the attention path of this library), its two norm
// weights, and the MLP as one [gate; up] matrix [2*hidden][d_model] (one N = 2*hidden GEMM
// instead of the reference's two, OlmoMlp.cpp:40-41) plus down [d_model][hidden]. Parameters are
// fp32 masters; the bf16 mode keeps bf16 copies for the GEMMs, refreshed after step. The
// residual stream stays fp32 as in the reference. GEMMs run on rocBLAS (bf16 inputs with fp32
// accumulation in bf16 mode, fp32 in exact mode); the attention core, norms, SwiGLU, embedding
// and loss run on this library's kernels.
//
// Parameters are addressed by the reference's .npy file stems ("model.embed_tokens.weight",
// "model.layers.{i}.mlp.up_proj.weight", ..., "model.norm.weight", "lm_head.weight";
// OlmoModel.cpp:12-22, OlmoBlock.cpp:5-11, OlmoMlp.cpp:9-24, OlmoAttention.cpp:39-53), so one
// setter serves both dt_model_load and callers that bring their own arrays.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <iterator>
#include <map>
#include <string>
#include <vector>

#include "dt_internal.h"

using namespace dt;

namespace {

struct ModelLayer {
    dt_attn_layer* attn = nullptr;
    float* w_pa = nullptr;    // post_attention_layernorm [dm]
    float* w_gu = nullptr;    // [gate_proj; up_proj] [2*hid][dm]
    float* w_down = nullptr;  // down_proj [dm][hid]
    float* w_pf = nullptr;    // post_feedforward_layernorm [dm]
    uint16_t* w_gu16 = nullptr;
    uint16_t* w_down16 = nullptr;
    // forward state (RMSNorm.h:22-23 for both norms; OlmoMlp's saved input, gate/up and activation)
    DeviceBuffer a, y_pa, rms_pa, h, h16, gu, act, m, y_pf, rms_pf;
    float* g_pa = nullptr;
    float* g_gu = nullptr;
    float* g_down = nullptr;
    float* g_pf = nullptr;
};

constexpr float kEps = DT_RMS_EPS;

}  // namespace

struct dt_model {
    dt_ctx* ctx = nullptr;
    int n_layers = 0, dm = 0, H = 0, hid = 0, V = 0;
    float* embed = nullptr;       // [V][dm]
    float* final_norm = nullptr;  // [dm]
    float* lm_head = nullptr;     // [V][dm]
    uint16_t* lm_head16 = nullptr;
    bool w16_stale = true;
    // zero_grad was called and the model-level gradient buffers (all but the embedding's, which zero_grad clears
    // at once, and the attention layers', which keep their own flag) have not been cleared: they read as zero,
    // the next backward writes them instead of adding to them, and anything else that reads them clears them first
    bool grad_zero_pending = false;
    // embedding-gradient rows a backward has written since the last zero_grad (sorted; on the device in
    // embed_rows_dev), or all rows (embed_rows_all): every other row is zero, so step and zero_grad visit only these
    std::vector<int32_t> embed_rows;
    bool embed_rows_all = false;
    DeviceBuffer embed_rows_dev;
    std::vector<ModelLayer> L;
    DeviceBuffer tok, x, x2, yf, yf16, rmsf, logits;
    // saved forward
    int saved_B = 0, saved_T = 0, saved_dtype = -1;
    std::vector<int32_t> saved_tokens;
    // gradients and backward workspaces
    float* g_embed = nullptr;
    float* g_final = nullptr;
    float* g_lm = nullptr;
    // d16: d_logits as bf16; g16a / g16b: the bf16 gradient rows of a block's two norms (bf16 mode)
    DeviceBuffer d16, g16a, g16b, dx, dh, da, dxa, dm_, d_act, d_gu, partial, csr;
};

namespace {

int alloc_f32(float** p, size_t n) {
    DT_HIP_TRY(hipMalloc(p, n * sizeof(float)));
    DT_HIP_TRY(hipMemset(*p, 0, n * sizeof(float)));
    return DT_OK;
}

struct ParamRef {
    float* w = nullptr;
    float** g = nullptr;  // gradient pointer slot (allocated on first backward)
    size_t offset = 0;    // into *g
    size_t count = 0;
};

// name -> parameter (weights and where its gradient lives)
int find_param(dt_model* M, const std::string& name, ParamRef& r, dt_attn_layer** attn_out = nullptr) {
    const size_t dm = M->dm, hid = M->hid, V = M->V;
    if (name == "model.embed_tokens.weight") {
        r = {M->embed, &M->g_embed, 0, V * dm};
        return DT_OK;
    }
    if (name == "model.norm.weight") {
        r = {M->final_norm, &M->g_final, 0, dm};
        return DT_OK;
    }
    if (name == "lm_head.weight") {
        r = {M->lm_head, &M->g_lm, 0, V * dm};
        return DT_OK;
    }
    int li = -1;
    char rest[128];
    if (std::sscanf(name.c_str(), "model.layers.%d.%127s", &li, rest) != 2 || li < 0 || li >= M->n_layers)
        return set_error(DT_ERR_INVALID_ARG, "unknown parameter '%s'", name.c_str());
    ModelLayer& Ly = M->L[li];
    dt_attn_layer* A = Ly.attn;
    const std::string s(rest);
    if (attn_out) *attn_out = nullptr;
    if (s == "self_attn.q_proj.weight" || s == "self_attn.k_proj.weight" || s == "self_attn.v_proj.weight") {
        const size_t k = s[10] == 'q' ? 0 : (s[10] == 'k' ? 1 : 2);
        r = {A->w_qkv + k * dm * dm, &A->g_qkv, k * dm * dm, dm * dm};
        if (attn_out) *attn_out = A;
    } else if (s == "self_attn.o_proj.weight") {
        r = {A->w_o, &A->g_o, 0, dm * dm};
        if (attn_out) *attn_out = A;
    } else if (s == "self_attn.q_norm.weight") {
        r = {A->q_norm, &A->g_qn, 0, dm};
        if (attn_out) *attn_out = A;
    } else if (s == "self_attn.k_norm.weight") {
        r = {A->k_norm, &A->g_kn, 0, dm};
        if (attn_out) *attn_out = A;
    } else if (s == "post_attention_layernorm.weight") {
        r = {Ly.w_pa, &Ly.g_pa, 0, dm};
    } else if (s == "post_feedforward_layernorm.weight") {
        r = {Ly.w_pf, &Ly.g_pf, 0, dm};
    } else if (s == "mlp.gate_proj.weight") {
        r = {Ly.w_gu, &Ly.g_gu, 0, hid * dm};
    } else if (s == "mlp.up_proj.weight") {
        r = {Ly.w_gu + hid * dm, &Ly.g_gu, hid * dm, hid * dm};
    } else if (s == "mlp.down_proj.weight") {
        r = {Ly.w_down, &Ly.g_down, 0, dm * hid};
    } else {
        return set_error(DT_ERR_INVALID_ARG, "unknown parameter '%s'", name.c_str());
    }
    return DT_OK;
}

std::vector<std::string> param_names(int n_layers) {
    static const char* layer_params[11] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                           "self_attn.o_proj", "self_attn.q_norm", "self_attn.k_norm",
                                           "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj",
                                           "mlp.down_proj", "post_feedforward_layernorm"};
    std::vector<std::string> v = {"model.embed_tokens.weight"};
    for (int i = 0; i < n_layers; ++i)
        for (const char* p : layer_params) v.push_back("model.layers." + std::to_string(i) + "." + p + ".weight");
    v.push_back("model.norm.weight");
    v.push_back("lm_head.weight");
    return v;
}

// every gradient slot of the model (its own and its blocks'; the attention layers keep theirs)
std::vector<float**> model_grad_slots(dt_model* M) {
    std::vector<float**> v = {&M->g_embed, &M->g_final, &M->g_lm};
    for (ModelLayer& Ly : M->L)
        for (float** p : {&Ly.g_pa, &Ly.g_pf, &Ly.g_gu, &Ly.g_down}) v.push_back(p);
    return v;
}

// The gradient buffers exist as a whole set or not at all: a failed allocation frees what was allocated and
// leaves every slot null, so no later backward, step or zero_grad sees a half-made set.
int ensure_model_grads(dt_model* M, hipStream_t s) {
    bool complete = true;
    for (float** p : model_grad_slots(M)) complete = complete && *p;
    for (ModelLayer& Ly : M->L) complete = complete && attn_layer_grads_complete(Ly.attn);
    if (complete) return DT_OK;
    const size_t dm = M->dm, hid = M->hid, V = M->V;
    auto alloc_all = [&]() -> int {
        DT_TRY(alloc_f32(&M->g_embed, V * dm));
        DT_TRY(alloc_f32(&M->g_final, dm));
        DT_TRY(alloc_f32(&M->g_lm, V * dm));
        for (ModelLayer& Ly : M->L) {
            DT_TRY(attn_layer_ensure_grads(Ly.attn, s));
            DT_TRY(alloc_f32(&Ly.g_pa, dm));
            DT_TRY(alloc_f32(&Ly.g_pf, dm));
            DT_TRY(alloc_f32(&Ly.g_gu, 2 * hid * dm));
            DT_TRY(alloc_f32(&Ly.g_down, dm * hid));
        }
        DT_HIP_TRY(hipDeviceSynchronize());  // the hipMemsets above are not stream-ordered with s
        return DT_OK;
    };
    for (float** p : model_grad_slots(M))  // a partial set cannot be left from an earlier call, but be sure
        if (*p) {
            (void)hipFree(*p);
            *p = nullptr;
        }
    const int rc = alloc_all();
    if (rc != DT_OK) {
        for (float** p : model_grad_slots(M))
            if (*p) {
                (void)hipFree(*p);
                *p = nullptr;
            }
        for (ModelLayer& Ly : M->L) attn_layer_free_grads(Ly.attn);
    }
    return rc;
}

// clears the gradient buffers of the model and of its attention layers when a zero_grad is pending
int model_settle_grads(dt_model* M, hipStream_t s) {
    for (ModelLayer& Ly : M->L) DT_TRY(attn_layer_settle_grads(Ly.attn, s));
    if (!M->grad_zero_pending || !M->g_embed) return DT_OK;
    const int64_t dm = M->dm, hid = M->hid, V = M->V;
    for (ModelLayer& Ly : M->L) {
        DT_TRY(launch_fill_zero(Ly.g_pa, dm, s));
        DT_TRY(launch_fill_zero(Ly.g_gu, 2 * hid * dm, s));
        DT_TRY(launch_fill_zero(Ly.g_down, dm * hid, s));
        DT_TRY(launch_fill_zero(Ly.g_pf, dm, s));
    }
    DT_TRY(launch_fill_zero(M->g_final, dm, s));
    DT_TRY(launch_fill_zero(M->g_lm, V * dm, s));
    M->grad_zero_pending = false;
    return DT_OK;
}

int refresh_bf16(dt_model* M, hipStream_t s) {
    const int64_t dm = M->dm, hid = M->hid, V = M->V;
    bool complete = M->lm_head16 != nullptr;
    for (const ModelLayer& Ly : M->L) complete = complete && Ly.w_gu16 && Ly.w_down16;
    if (!complete) {  // first bf16 call, or a failed allocation left the set incomplete: allocate what is missing
        if (!M->lm_head16) DT_HIP_TRY(hipMalloc(&M->lm_head16, V * dm * 2));
        for (ModelLayer& Ly : M->L) {
            if (!Ly.w_gu16) DT_HIP_TRY(hipMalloc(&Ly.w_gu16, 2 * hid * dm * 2));
            if (!Ly.w_down16) DT_HIP_TRY(hipMalloc(&Ly.w_down16, dm * hid * 2));
        }
        M->w16_stale = true;
    }
    if (!M->w16_stale) return DT_OK;
    DT_TRY(launch_f32_to_bf16(M->lm_head, M->lm_head16, V * dm, s));
    for (ModelLayer& Ly : M->L) {
        DT_TRY(launch_f32_to_bf16(Ly.w_gu, Ly.w_gu16, 2 * hid * dm, s));
        DT_TRY(launch_f32_to_bf16(Ly.w_down, Ly.w_down16, dm * hid, s));
    }
    M->w16_stale = false;
    return DT_OK;
}

int check_tokens(const dt_model* M, const int32_t* tokens, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= M->V)
            return set_error(DT_ERR_INVALID_ARG, "token %d at position %lld outside [0, %d)", tokens[i], (long long)i,
                             M->V);
    return DT_OK;
}

}  // namespace

extern "C" {

int dt_model_create(dt_ctx* ctx, int n_layers, int d_model, int n_heads, int hidden, int vocab, dt_model** out) {
    clear_error();
    if (!out) return set_error(DT_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (n_layers < 1 || n_layers > 256) return set_error(DT_ERR_INVALID_ARG, "n_layers=%d outside [1, 256]", n_layers);
    if (n_heads < 1 || n_heads > 256 || d_model != n_heads * DT_HEAD_DIM)
        return set_error(DT_ERR_UNSUPPORTED, "d_model=%d must equal n_heads (%d) * %d", d_model, n_heads, DT_HEAD_DIM);
    if (hidden < 4 || hidden % 4) return set_error(DT_ERR_INVALID_ARG, "hidden=%d must be a positive multiple of 4", hidden);
    if (vocab < 1) return set_error(DT_ERR_INVALID_ARG, "vocab=%d must be >= 1", vocab);
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    DT_TRY(check_device_binding(ctx));
    dt_model* M = new dt_model();
    M->ctx = ctx;
    M->n_layers = n_layers;
    M->dm = d_model;
    M->H = n_heads;
    M->hid = hidden;
    M->V = vocab;
    M->L.resize(n_layers);
    auto fail = [&](int rc) {
        dt_model_destroy(M);
        return rc;
    };
    const size_t dm = d_model, hid = hidden, V = vocab;
    int rc = alloc_f32(&M->embed, V * dm);
    if (rc == DT_OK) rc = alloc_f32(&M->final_norm, dm);
    if (rc == DT_OK) rc = alloc_f32(&M->lm_head, V * dm);
    for (int i = 0; i < n_layers && rc == DT_OK; ++i) {
        ModelLayer& Ly = M->L[i];
        rc = attn_layer_alloc(ctx, d_model, n_heads, &Ly.attn);
        if (rc == DT_OK) rc = alloc_f32(&Ly.w_pa, dm);
        if (rc == DT_OK) rc = alloc_f32(&Ly.w_pf, dm);
        if (rc == DT_OK) rc = alloc_f32(&Ly.w_gu, 2 * hid * dm);
        if (rc == DT_OK) rc = alloc_f32(&Ly.w_down, dm * hid);
    }
    if (rc != DT_OK) return fail(rc);
    *out = M;
    return DT_OK;
}

int dt_model_destroy(dt_model* M) {
    clear_error();
    if (!M) return DT_OK;
    if (M->ctx) (void)hipSetDevice(M->ctx->device);
    for (float* p : {M->embed, M->final_norm, M->lm_head, M->g_embed, M->g_final, M->g_lm})
        if (p) (void)hipFree(p);
    if (M->lm_head16) (void)hipFree(M->lm_head16);
    for (ModelLayer& Ly : M->L) {
        if (Ly.attn) dt_attn_layer_destroy(Ly.attn);
        for (float* p : {Ly.w_pa, Ly.w_gu, Ly.w_down, Ly.w_pf, Ly.g_pa, Ly.g_gu, Ly.g_down, Ly.g_pf})
            if (p) (void)hipFree(p);
        if (Ly.w_gu16) (void)hipFree(Ly.w_gu16);
        if (Ly.w_down16) (void)hipFree(Ly.w_down16);
        for (DeviceBuffer* b : {&Ly.a, &Ly.y_pa, &Ly.rms_pa, &Ly.h, &Ly.h16, &Ly.gu, &Ly.act, &Ly.m, &Ly.y_pf, &Ly.rms_pf})
            b->release();
    }
    for (DeviceBuffer* b : {&M->tok, &M->x, &M->x2, &M->yf, &M->yf16, &M->rmsf, &M->logits, &M->d16, &M->g16a, &M->g16b, &M->dx, &M->dh,
                            &M->da, &M->dxa, &M->dm_, &M->d_act, &M->d_gu, &M->partial, &M->csr,
                            &M->embed_rows_dev})
        b->release();
    delete M;
    return DT_OK;
}

int dt_model_set_param(dt_model* M, const char* name, const float* data, int64_t count, int mem) {
    clear_error();
    if (!M || !name || !data) return set_error(DT_ERR_INVALID_ARG, "model, name and data must be non-NULL");
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    ParamRef r;
    dt_attn_layer* A = nullptr;
    DT_TRY(find_param(M, name, r, &A));
    if ((size_t)count != r.count)
        return set_error(DT_ERR_INVALID_ARG, "parameter '%s' has %zu elements, got %lld", name, r.count, (long long)count);
    DT_TRY(check_device_binding(M->ctx));
    DT_HIP_TRY(hipMemcpy(r.w, data, r.count * sizeof(float), mem == DT_MEM_HOST ? hipMemcpyHostToDevice
                                                                                 : hipMemcpyDeviceToDevice));
    M->w16_stale = true;
    if (A) A->w16_stale = true;
    return DT_OK;
}

int dt_model_get_param(dt_model* M, const char* name, float* out, int64_t count, int grad, int mem, void* stream) {
    clear_error();
    if (!M || !name || !out) return set_error(DT_ERR_INVALID_ARG, "model, name and out must be non-NULL");
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    ParamRef r;
    DT_TRY(find_param(M, name, r));
    if ((size_t)count != r.count)
        return set_error(DT_ERR_INVALID_ARG, "parameter '%s' has %zu elements, got %lld", name, r.count, (long long)count);
    DT_TRY(check_device_binding(M->ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (grad) {
        DT_TRY(ensure_model_grads(M, s));
        DT_TRY(model_settle_grads(M, s));
    }
    const float* src = grad ? *r.g + r.offset : r.w;
    DT_HIP_TRY(hipMemcpyAsync(out, src, r.count * sizeof(float),
                              mem == DT_MEM_HOST ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice, s));
    if (mem == DT_MEM_HOST) DT_HIP_TRY(hipStreamSynchronize(s));
    return DT_OK;
}

int dt_model_load(dt_ctx* ctx, const char* folder, int n_layers, dt_model** out) {
    clear_error();
    if (!out) return set_error(DT_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (!folder) return set_error(DT_ERR_INVALID_ARG, "folder is NULL");
    if (n_layers < 1 || n_layers > 256) return set_error(DT_ERR_INVALID_ARG, "n_layers=%d outside [1, 256]", n_layers);
    const std::string dir(folder);
    // shapes from the embedding and the first MLP (OlmoModel.cpp:12-18, OlmoMlp.cpp:9-19)
    std::vector<size_t> shape, up_shape;
    DT_TRY(read_npy_shape(dir + "/model.embed_tokens.weight.npy", shape));
    if (shape.size() != 2 || shape[0] < 1 || shape[1] < 1 || shape[0] > 0x7fffffff || shape[1] > 0x7fffffff)
        return set_error(DT_ERR_IO, "model.embed_tokens.weight: expected a non-empty matrix");
    const int V = (int)shape[0], dm = (int)shape[1];
    DT_TRY(read_npy_shape(dir + "/model.layers.0.mlp.up_proj.weight.npy", up_shape));
    if (up_shape.size() != 2 || (int)up_shape[1] != dm || up_shape[0] < 1 || up_shape[0] > 0x7fffffff)
        return set_error(DT_ERR_IO, "model.layers.0.mlp.up_proj.weight: unexpected shape");
    if (dm % DT_HEAD_DIM) return set_error(DT_ERR_UNSUPPORTED, "d_model=%d is not a multiple of %d", dm, DT_HEAD_DIM);
    const size_t hid = up_shape[0];
    // every file's header and shape are checked before the device is touched (a Git-LFS pointer, a wrong dtype
    // or a truncated file fails here, not after gigabytes have been uploaded)
    const std::vector<std::string> names = param_names(n_layers);
    for (const std::string& name : names) {
        std::vector<size_t> sh;
        DT_TRY(read_npy_shape(dir + "/" + name + ".npy", sh));
        std::vector<size_t> want;
        const bool vec = name.find("norm") != std::string::npos;  // q_norm, k_norm, the post-norms, model.norm
        if (name == "model.embed_tokens.weight" || name == "lm_head.weight") want = {(size_t)V, (size_t)dm};
        else if (vec) want = {(size_t)dm};
        else if (name.find("gate_proj") != std::string::npos || name.find("up_proj") != std::string::npos)
            want = {hid, (size_t)dm};
        else if (name.find("down_proj") != std::string::npos) want = {(size_t)dm, hid};
        else want = {(size_t)dm, (size_t)dm};  // the attention projections
        if (sh != want) {
            std::string got, exp;
            for (size_t v : sh) got += std::to_string(v) + ",";
            for (size_t v : want) exp += std::to_string(v) + ",";
            return set_error(DT_ERR_IO, "%s: shape (%s) where (%s) was expected", name.c_str(), got.c_str(), exp.c_str());
        }
    }
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    dt_model* M = nullptr;
    DT_TRY(dt_model_create(ctx, n_layers, dm, dm / DT_HEAD_DIM, (int)hid, V, &M));
    for (const std::string& name : names) {
        std::vector<float> w;
        std::vector<size_t> sh;
        int rc = read_npy_f32(dir + "/" + name + ".npy", w, sh);
        if (rc == DT_OK) rc = dt_model_set_param(M, name.c_str(), w.data(), (int64_t)w.size(), DT_MEM_HOST);
        if (rc != DT_OK) {
            std::string msg = dt_last_error();
            dt_model_destroy(M);
            return set_error(rc, "%s", msg.c_str());
        }
    }
    *out = M;
    return DT_OK;
}

int dt_model_fwd(dt_model* M, const int32_t* tokens, int B, int T, float* logits, int dtype, int mem,
                 int save_for_backward, void* stream) {
    clear_error();
    if (!M || !tokens || !logits) return set_error(DT_ERR_INVALID_ARG, "model, tokens and logits must be non-NULL");
    if (B < 1 || T < 1) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d must be >= 1", B, T);
    if (T > DT_MAX_SEQ_LEN) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds max_seq_len %d", T, DT_MAX_SEQ_LEN);
    if ((int64_t)B * T * M->V > ((int64_t)1 << 40)) return set_error(DT_ERR_UNSUPPORTED, "logits too large");
    if ((int64_t)B * T > 0x7fffffff / 8) return set_error(DT_ERR_UNSUPPORTED, "B*T too large");
    if (dtype != DT_FP32_EXACT && dtype != DT_BF16) return set_error(DT_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (save_for_backward != 0 && save_for_backward != 1)
        return set_error(DT_ERR_INVALID_ARG, "save_for_backward must be 0 or 1");
    if (mem == DT_MEM_DEVICE && !aligned16(logits)) return set_error(DT_ERR_INVALID_ARG, "logits must be 16-byte aligned");
    const int64_t rows = (int64_t)B * T;
    DT_TRY(check_tokens(M, tokens, rows));  // tokens are a host array, like seq_lens
    dt_ctx* ctx = M->ctx;
    if (T > ctx->rope_len) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds the RoPE table length %d", T, ctx->rope_len);
    DT_TRY(check_device_binding(ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool bf = dtype == DT_BF16;
    const int dm = M->dm, hid = M->hid, V = M->V;
    const size_t act = (size_t)rows * dm;
    M->saved_T = 0;
    if (bf) DT_TRY(refresh_bf16(M, s));

    // embedding (OlmoModel.cpp:29-38)
    DT_TRY(M->tok.ensure(rows * 4));
    DT_HIP_TRY(hipMemcpyAsync(M->tok.ptr, tokens, rows * 4, hipMemcpyHostToDevice, s));
    DT_TRY(M->x.ensure(act * 4));
    DT_TRY(M->x2.ensure(act * 4));
    float* x = static_cast<float*>(M->x.ptr);
    float* xn = static_cast<float*>(M->x2.ptr);
    DT_TRY(launch_embed_gather(static_cast<const int32_t*>(M->tok.ptr), M->embed, x, (int)rows, dm, s));

    // blocks (OlmoBlock.cpp:13-21)
    for (int li = 0; li < M->n_layers; ++li) {
        ModelLayer& Ly = M->L[li];
        ModelLayer& S = save_for_backward ? Ly : M->L[0];  // state buffers (layer 0's serve as scratch)
        DT_TRY(S.a.ensure(act * 4));
        DT_TRY(S.h.ensure(act * 4));
        DT_TRY(S.gu.ensure((size_t)rows * 2 * hid * (bf ? 2 : 4)));
        DT_TRY(S.act.ensure((size_t)rows * hid * (bf ? 2 : 4)));
        DT_TRY(S.m.ensure(act * 4));
        if (bf) DT_TRY(S.h16.ensure(act * 2));
        if (save_for_backward) {
            DT_TRY(S.y_pa.ensure(act * 4));
            DT_TRY(S.y_pf.ensure(act * 4));
            DT_TRY(S.rms_pa.ensure(rows * 4));
            DT_TRY(S.rms_pf.ensure(rows * 4));
        }
        float* a = static_cast<float*>(S.a.ptr);
        float* h = static_cast<float*>(S.h.ptr);
        void* gu = S.gu.ptr;  // fp32, or bf16 in bf16 mode
        float* mo = static_cast<float*>(S.m.ptr);
        uint16_t* h16 = bf ? static_cast<uint16_t*>(S.h16.ptr) : nullptr;
        float* y_pa = save_for_backward ? static_cast<float*>(S.y_pa.ptr) : nullptr;
        float* y_pf = save_for_backward ? static_cast<float*>(S.y_pf.ptr) : nullptr;
        float* rms_pa = save_for_backward ? static_cast<float*>(S.rms_pa.ptr) : nullptr;
        float* rms_pf = save_for_backward ? static_cast<float*>(S.rms_pf.ptr) : nullptr;
        // attention and h = x + N(attn(x)); in bf16 mode from the second block on, the previous block's last norm
        // has already written x rounded to bf16 into this layer's x16
        DT_TRY(attn_layer_fwd(Ly.attn, x, a, B, T, nullptr, dtype, DT_MEM_DEVICE, save_for_backward, stream,
                              bf && li > 0));
        DT_TRY(launch_rmsnorm_rows(a, Ly.w_pa, x, h, h16, y_pa, rms_pa, (int)rows, dm, kEps, s));
        // MLP (OlmoMlp.cpp:26-63): [gate | up] = h [Wgate; Wup]^T, act = silu(gate) * up, m = act Wdown^T
        // (in bf16 mode the N = 16384 gate|up product is written as bf16: it is only read by SwiGLU)
        if (bf) DT_TRY(gemm_rm_bf16(ctx, s, false, true, (int)rows, 2 * hid, dm, h16, dm, Ly.w_gu16, dm, gu, 2 * hid));
        else DT_TRY(gemm_rm(ctx, s, false, true, (int)rows, 2 * hid, dm, h, dm, Ly.w_gu, dm, 0.0f, static_cast<float*>(gu),
                            2 * hid, false));
        DT_TRY(launch_swiglu(gu, S.act.ptr, (int)rows, hid, bf, s));
        DT_TRY(gemm_rm(ctx, s, false, true, (int)rows, dm, hid, S.act.ptr, hid,
                       bf ? static_cast<const void*>(Ly.w_down16) : static_cast<const void*>(Ly.w_down), hid, 0.0f, mo,
                       dm, bf));
        // x_next = h + N(m), in bf16 mode also as bf16 into the next layer's x16 (the input its projections read)
        uint16_t* xn16 = nullptr;
        if (bf && li + 1 < M->n_layers) {
            dt_attn_layer* next = M->L[li + 1].attn;
            DT_TRY(next->x16.ensure(act * 2));
            xn16 = static_cast<uint16_t*>(next->x16.ptr);
        }
        DT_TRY(launch_rmsnorm_rows(mo, Ly.w_pf, h, xn, xn16, y_pf, rms_pf, (int)rows, dm, kEps, s));
        std::swap(x, xn);
    }
    // final norm and LM head (OlmoModel.cpp:44-47, OlmoLmHead.cpp:11-28)
    DT_TRY(M->yf.ensure(act * 4));
    DT_TRY(M->rmsf.ensure(rows * 4));
    if (bf) DT_TRY(M->yf16.ensure(act * 2));
    float* yf = static_cast<float*>(M->yf.ptr);
    uint16_t* yf16 = bf ? static_cast<uint16_t*>(M->yf16.ptr) : nullptr;
    DT_TRY(launch_rmsnorm_rows(x, M->final_norm, nullptr, yf, yf16, nullptr, static_cast<float*>(M->rmsf.ptr),
                               (int)rows, dm, kEps, s));
    float* lo = logits;
    if (mem == DT_MEM_HOST) {
        DT_TRY(M->logits.ensure((size_t)rows * V * 4));
        lo = static_cast<float*>(M->logits.ptr);
    }
    if (bf) DT_TRY(gemm_rm(ctx, s, false, true, (int)rows, V, dm, yf16, dm, M->lm_head16, dm, 0.0f, lo, V, true));
    else DT_TRY(gemm_rm(ctx, s, false, true, (int)rows, V, dm, yf, dm, M->lm_head, dm, 0.0f, lo, V, false));
    if (mem == DT_MEM_HOST) {
        DT_HIP_TRY(hipMemcpyAsync(logits, lo, (size_t)rows * V * 4, hipMemcpyDeviceToHost, s));
        DT_HIP_TRY(hipStreamSynchronize(s));
        DT_TRY(qkv_status_check(ctx));
    }
    if (save_for_backward) {
        // the final residual stream x is in M->x or M->x2; keep it addressable as M->x
        if (x != static_cast<float*>(M->x.ptr)) std::swap(M->x, M->x2);
        M->saved_B = B;
        M->saved_T = T;
        M->saved_dtype = dtype;
        M->saved_tokens.assign(tokens, tokens + rows);
    }
    return DT_OK;
}

// `writing` is set once the first gradient buffer is about to be written
// The weight-gradient GEMMs (dW of the LM head, the MLP's down and gate/up matrices, and inside each attention
// layer dWo and dWqkv) run on the context's side stream when it has one, beside the chain of input gradients on s,
// which never reads them. Each starts after s has formed its input (slot kEvFork). s waits for the side stream only
// before it overwrites a buffer a pending side GEMM reads: the MLP's norm-gradient rows (slot kEvDown), d_gu
// (kEvGu) and the attention layer's d_out rows (kEvO), each one block later; and at the end (kEvJoin).
static int model_bwd(dt_model* M, const float* d_logits, int mem, void* stream, hipStream_t side, bool& writing) {
    clear_error();
    if (!M || !d_logits) return set_error(DT_ERR_INVALID_ARG, "model and d_logits must be non-NULL");
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (M->saved_T == 0)
        return set_error(DT_ERR_INVALID_ARG, "no saved forward: call dt_model_fwd with save_for_backward = 1 first");
    dt_ctx* ctx = M->ctx;
    DT_TRY(check_device_binding(ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool bf = M->saved_dtype == DT_BF16;
    const int B = M->saved_B, T = M->saved_T, dm = M->dm, hid = M->hid, V = M->V;
    const int rows = B * T;
    const size_t act = (size_t)rows * dm;
    DT_TRY(ensure_model_grads(M, s));
    // after zero_grad the gradients are written, not added to (beta = 0: the buffers still hold old values)
    const bool fresh = M->grad_zero_pending;
    const float gb = fresh ? 0.0f : 1.0f;

    const float* gl = d_logits;
    if (mem == DT_MEM_HOST) {
        DT_TRY(M->logits.ensure((size_t)rows * V * 4));
        DT_HIP_TRY(hipMemcpyAsync(M->logits.ptr, d_logits, (size_t)rows * V * 4, hipMemcpyHostToDevice, s));
        gl = static_cast<const float*>(M->logits.ptr);
    }
    DT_TRY(M->dx.ensure(act * 4));
    DT_TRY(M->dh.ensure(act * 4));
    DT_TRY(M->da.ensure(act * 4));
    DT_TRY(M->dxa.ensure(act * 4));
    DT_TRY(M->dm_.ensure(act * 4));
    DT_TRY(M->d_act.ensure((size_t)rows * hid * 4));
    DT_TRY(M->d_gu.ensure((size_t)rows * 2 * hid * (bf ? 2 : 4)));
    const int nblk = rmsnorm_bwd_blocks(rows);
    DT_TRY(M->partial.ensure((size_t)3 * nblk * dm * 4));  // the final norm's, then N_pf's and N_pa's
    if (bf) {
        DT_TRY(M->d16.ensure((size_t)rows * V * 2));
        DT_TRY(M->g16a.ensure(act * 2));
        DT_TRY(M->g16b.ensure(act * 2));
    }
    float* dx = static_cast<float*>(M->dx.ptr);
    float* dh = static_cast<float*>(M->dh.ptr);
    float* da = static_cast<float*>(M->da.ptr);
    float* dxa = static_cast<float*>(M->dxa.ptr);
    float* dmo = static_cast<float*>(M->dm_.ptr);
    float* d_act = static_cast<float*>(M->d_act.ptr);
    float* part_f = static_cast<float*>(M->partial.ptr);
    float* part_pf = part_f + (size_t)nblk * dm;
    float* part_pa = part_pf + (size_t)nblk * dm;
    uint16_t* d16 = static_cast<uint16_t*>(M->d16.ptr);
    uint16_t* g16a = static_cast<uint16_t*>(M->g16a.ptr);
    uint16_t* g16b = static_cast<uint16_t*>(M->g16b.ptr);
    hipStream_t sw = side ? side : s;  // the weight-gradient GEMMs' stream
    auto fork = [&]() { return side ? stream_after(ctx, side, s, kEvFork) : DT_OK; };
    auto wait_side = [&](int ev) { return side ? stream_wait_slot(ctx, s, ev) : DT_OK; };
    // a norm weight's gradient: the column sums of the partial rows its backward kernel wrote (on the side stream
    // when there is one; each norm has its own partial rows, which the side stream has read before the next
    // kEvDown / kEvO mark)
    auto norm_grad_w = [&](float* g) { return side ? nullptr : g; };
    auto norm_colsum = [&](const float* part, float* g) {
        if (!side) return DT_OK;
        DT_TRY(fork());
        return launch_colsum(part, nblk, dm, g, side, !fresh);
    };

    // LM head (OlmoLmHead.cpp:30-62): d_y = d_logits W; dW += d_logits^T y. The side stream starts dW only once d_y
    // is formed, so the chain's largest product runs alone and dW runs beside the first blocks' backward (the
    // other weight gradients start with their blocks' input-gradient products; placed after them they measured
    // slower)
    float* d_yf = da;
    writing = true;
    if (bf) {
        DT_TRY(launch_f32_to_bf16(gl, d16, (int64_t)rows * V, s));
        DT_TRY(gemm_rm(ctx, s, false, false, rows, dm, V, d16, V, M->lm_head16, dm, 0.0f, d_yf, dm, true));
        DT_TRY(fork());
        DT_TRY(gemm_rm(ctx, sw, true, false, V, dm, rows, d16, V, M->yf16.ptr, dm, gb, M->g_lm, dm, true));
    } else {
        DT_TRY(gemm_rm(ctx, s, false, false, rows, dm, V, gl, V, M->lm_head, dm, 0.0f, d_yf, dm, false));
        DT_TRY(fork());
        DT_TRY(gemm_rm(ctx, sw, true, false, V, dm, rows, gl, V, M->yf.ptr, dm, gb, M->g_lm, dm, false));
    }
    // final norm (OlmoModel.cpp:52): RMSNorm::backward from the saved output y and rms
    DT_TRY(launch_rmsnorm_bwd(d_yf, static_cast<const float*>(M->yf.ptr), static_cast<const float*>(M->rmsf.ptr),
                              M->final_norm, nullptr, dx, part_f, norm_grad_w(M->g_final), rows, dm, s, !fresh));
    DT_TRY(norm_colsum(part_f, M->g_final));
    // blocks in reverse (OlmoBlock.cpp:23-30)
    for (int li = M->n_layers - 1; li >= 0; --li) {
        ModelLayer& Ly = M->L[li];
        // d_m = N_pf.backward(d_x) (in bf16 mode only as bf16: the two GEMMs below are its only readers), over the
        // rows the previous block's dWdown GEMM read
        DT_TRY(wait_side(kEvDown));
        DT_TRY(launch_rmsnorm_bwd(dx, static_cast<const float*>(Ly.y_pf.ptr), static_cast<const float*>(Ly.rms_pf.ptr),
                                  Ly.w_pf, nullptr, bf ? nullptr : dmo, part_pf, norm_grad_w(Ly.g_pf), rows, dm, s,
                                  !fresh, bf ? g16a : nullptr));
        // MLP backward: dWdown += d_m^T act; d_act = d_m Wdown; d_gu = swiglu'; dW_gu += d_gu^T h;
        // d_h = d_gu W_gu + d_x (the residual, OlmoBlock.cpp:28; GEMM with beta = 1 into a copy of d_x)
        DT_HIP_TRY(hipMemcpyAsync(dh, dx, act * 4, hipMemcpyDeviceToDevice, s));
        DT_TRY(norm_colsum(part_pf, Ly.g_pf));  // (forks the side stream for the GEMM below as well)
        if (bf) {
            DT_TRY(gemm_rm(ctx, sw, true, false, dm, hid, rows, g16a, dm, Ly.act.ptr, hid, gb, Ly.g_down, hid, true));
            if (side) DT_TRY(stream_mark(ctx, side, kEvDown));
            DT_TRY(gemm_rm(ctx, s, false, false, rows, hid, dm, g16a, dm, Ly.w_down16, hid, 0.0f, d_act, hid, true));
        } else {
            DT_TRY(gemm_rm(ctx, sw, true, false, dm, hid, rows, dmo, dm, Ly.act.ptr, hid, gb, Ly.g_down, hid, false));
            if (side) DT_TRY(stream_mark(ctx, side, kEvDown));
            DT_TRY(gemm_rm(ctx, s, false, false, rows, hid, dm, dmo, dm, Ly.w_down, hid, 0.0f, d_act, hid, false));
        }
        DT_TRY(wait_side(kEvGu));  // the previous block's dW_gu GEMM has read d_gu
        DT_TRY(launch_swiglu_bwd(d_act, Ly.gu.ptr, M->d_gu.ptr, rows, hid, bf, s));
        const void* hin = bf ? Ly.h16.ptr : Ly.h.ptr;
        const void* wgu = bf ? static_cast<const void*>(Ly.w_gu16) : static_cast<const void*>(Ly.w_gu);
        DT_TRY(fork());
        DT_TRY(gemm_rm(ctx, sw, true, false, 2 * hid, dm, rows, M->d_gu.ptr, 2 * hid, hin, dm, gb, Ly.g_gu, dm, bf));
        if (side) DT_TRY(stream_mark(ctx, side, kEvGu));
        DT_TRY(gemm_rm(ctx, s, false, false, rows, dm, 2 * hid, M->d_gu.ptr, 2 * hid, wgu, dm, 1.0f, dh, dm, bf));
        // d_a = N_pa.backward(d_h); d_x = attn.backward(d_a) + d_h (OlmoBlock.cpp:29-32); in bf16 mode d_a also as
        // bf16, the form the layer's output-projection GEMMs read, over the rows the previous block's dWo GEMM read
        DT_TRY(wait_side(kEvO));
        DT_TRY(launch_rmsnorm_bwd(dh, static_cast<const float*>(Ly.y_pa.ptr), static_cast<const float*>(Ly.rms_pa.ptr),
                                  Ly.w_pa, nullptr, da, part_pa, norm_grad_w(Ly.g_pa), rows, dm, s, !fresh,
                                  bf ? g16b : nullptr));
        DT_TRY(norm_colsum(part_pa, Ly.g_pa));
        DT_TRY(attn_layer_bwd_dev(Ly.attn, da, bf ? g16b : nullptr, dxa, B, T, stream, side));
        DT_TRY(launch_add(dxa, dh, dx, (int64_t)act, s));
    }
    if (side) DT_TRY(stream_after(ctx, s, side, kEvJoin));
    M->grad_zero_pending = false;  // every model-level gradient buffer but the embedding's has been written
    // embedding (OlmoModel.cpp:57-66): per distinct token, its positions in order (CSR built here)
    std::vector<int32_t> order(rows);
    for (int i = 0; i < rows; ++i) order[i] = i;
    const std::vector<int32_t>& tk = M->saved_tokens;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return tk[a] < tk[b]; });
    std::vector<int32_t> uniq, start;
    for (int i = 0; i < rows; ++i)
        if (i == 0 || tk[order[i]] != tk[order[i - 1]]) {
            uniq.push_back(tk[order[i]]);
            start.push_back(i);
        }
    start.push_back(rows);
    const size_t nu = uniq.size();
    if (!M->embed_rows_all) {  // (recorded before the scatter: a superset of the written rows is harmless)
        std::vector<int32_t> merged;
        std::set_union(M->embed_rows.begin(), M->embed_rows.end(), uniq.begin(), uniq.end(),
                       std::back_inserter(merged));
        // many rows: the dense passes are as cheap; a failed upload: fall back to them as well
        const bool ok = merged.size() <= (size_t)V / 8 && M->embed_rows_dev.ensure(merged.size() * 4) == DT_OK &&
                        hipMemcpyAsync(M->embed_rows_dev.ptr, merged.data(), merged.size() * 4,
                                       hipMemcpyHostToDevice, s) == hipSuccess;
        if (ok) {  // (the swap keeps the uploaded array alive; the backward ends with a stream synchronisation)
            M->embed_rows.swap(merged);
        } else {
            M->embed_rows_all = true;
            M->embed_rows.clear();
        }
    }
    DT_TRY(M->csr.ensure((nu + nu + 1 + rows) * 4));
    int32_t* dcsr = static_cast<int32_t*>(M->csr.ptr);
    std::vector<int32_t> packed;
    packed.reserve(nu + nu + 1 + rows);
    packed.insert(packed.end(), uniq.begin(), uniq.end());
    packed.insert(packed.end(), start.begin(), start.end());
    packed.insert(packed.end(), order.begin(), order.end());
    DT_HIP_TRY(hipMemcpyAsync(dcsr, packed.data(), packed.size() * 4, hipMemcpyHostToDevice, s));
    DT_TRY(launch_embed_bwd(dx, dcsr, dcsr + nu, dcsr + 2 * nu + 1, (int)nu, M->g_embed, dm, s));
    DT_HIP_TRY(hipStreamSynchronize(s));  // the host arrays staged above are released on return
    return DT_OK;
}

int dt_model_bwd(dt_model* M, const float* d_logits, int mem, void* stream) {
    bool writing = false;
    const bool was_pending = M && M->grad_zero_pending;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStream_t side = (M && check_device_binding(M->ctx) == DT_OK) ? side_stream(M->ctx, s) : nullptr;
    clear_error();
    const int rc = model_bwd(M, d_logits, mem, stream, side, writing);
    // on an error the caller's stream still takes over what the side stream holds of this call
    if (rc != DT_OK && side) (void)stream_after(M->ctx, s, side, kEvJoin);
    // a backward that failed after zero_grad, once it had begun writing gradients, may have written some of them:
    // clear them all (the layers' too), so that they read as the zero_grad left them (the error stays the one
    // reported)
    if (rc != DT_OK && writing && was_pending) {
        for (ModelLayer& Ly : M->L) Ly.attn->grad_zero_pending = true;
        M->grad_zero_pending = true;
        (void)model_settle_grads(M, static_cast<hipStream_t>(stream));
    }
    return rc;
}

int dt_model_step(dt_model* M, float lr, void* stream) {
    clear_error();
    if (!M) return set_error(DT_ERR_INVALID_ARG, "model is NULL");
    if (!std::isfinite(lr)) return set_error(DT_ERR_INVALID_ARG, "lr must be finite");
    DT_TRY(check_device_binding(M->ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    DT_TRY(ensure_model_grads(M, s));
    DT_TRY(model_settle_grads(M, s));
    const int64_t dm = M->dm, hid = M->hid, V = M->V;
    // the bf16 copies (once the bf16 mode has made them all) are rewritten from the updated weights in the
    // same pass, so they are current afterwards
    bool copies = M->lm_head16 != nullptr;
    for (const ModelLayer& Ly : M->L) copies = copies && Ly.w_gu16 && Ly.w_down16;
    // OlmoModel.cpp:69-75. The embedding gradient is +0 outside embed_rows, and for lr >= +0 the product lr * 0
    // is +0 and w - (+0) is w bit for bit (also for w = -0, inf and NaN), so only those rows are updated; a
    // negative lr or -0 would turn w = -0 into +0 there, so it takes the dense pass.
    if (M->embed_rows_all || std::signbit(lr))
        DT_TRY(launch_sgd(M->embed, M->g_embed, lr, V * dm, s));
    else
        DT_TRY(launch_embed_rows(M->embed, M->g_embed, static_cast<const int32_t*>(M->embed_rows_dev.ptr),
                                 (int)M->embed_rows.size(), (int)dm, lr, false, s));
    // the norm weights (q_norm, k_norm and both block norms of every block, the final norm) are gathered into
    // one launch; each is a single workgroup's work
    std::vector<float*> vw;
    std::vector<const float*> vg;
    auto vec = [&](float* w, const float* g) {
        vw.push_back(w);
        vg.push_back(g);
    };
    for (ModelLayer& Ly : M->L) {
        DT_TRY(attn_layer_step_mats(Ly.attn, lr, s));  // OlmoBlock.cpp:32-37
        vec(Ly.attn->q_norm, Ly.attn->g_qn);
        vec(Ly.attn->k_norm, Ly.attn->g_kn);
        vec(Ly.w_pa, Ly.g_pa);
        DT_TRY(launch_sgd(Ly.w_gu, Ly.g_gu, lr, 2 * hid * dm, s, copies ? Ly.w_gu16 : nullptr));
        DT_TRY(launch_sgd(Ly.w_down, Ly.g_down, lr, dm * hid, s, copies ? Ly.w_down16 : nullptr));
        vec(Ly.w_pf, Ly.g_pf);
    }
    vec(M->final_norm, M->g_final);
    const std::vector<int> vn(vw.size(), (int)dm);
    DT_TRY(launch_sgd_vecs(vw.data(), vg.data(), vn.data(), (int)vw.size(), lr, s));
    DT_TRY(launch_sgd(M->lm_head, M->g_lm, lr, V * dm, s, copies ? M->lm_head16 : nullptr));
    M->w16_stale = !copies;
    return DT_OK;
}

int dt_model_zero_grad(dt_model* M, void* stream) {
    clear_error();
    if (!M) return set_error(DT_ERR_INVALID_ARG, "model is NULL");
    DT_TRY(check_device_binding(M->ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!M->g_embed) return ensure_model_grads(M, s);
    const int64_t dm = M->dm, V = M->V;
    // OlmoModel.cpp:77-83. The embedding gradient is accumulated by a scatter over the batch's tokens, so it is
    // cleared here; the others are cleared lazily (the next backward overwrites them, see grad_zero_pending)
    if (M->embed_rows_all)
        DT_TRY(launch_fill_zero(M->g_embed, V * dm, s));
    else  // only the rows a backward wrote can be nonzero
        DT_TRY(launch_embed_rows(M->embed, M->g_embed, static_cast<const int32_t*>(M->embed_rows_dev.ptr),
                                 (int)M->embed_rows.size(), (int)dm, 0.0f, true, s));
    M->embed_rows.clear();
    M->embed_rows_all = false;
    for (ModelLayer& Ly : M->L) DT_TRY(dt_attn_layer_zero_grad(Ly.attn, stream));
    M->grad_zero_pending = true;
    return DT_OK;
}

int dt_ce_loss(dt_ctx* ctx, const float* logits, const int32_t* tokens, int B, int T, int V, int ignore_index,
               float* loss, float* d_logits, int mem, void* stream) {
    clear_error();
    if (!logits || !tokens || !loss) return set_error(DT_ERR_INVALID_ARG, "logits, tokens and loss must be non-NULL");
    if (B < 1 || T < 1 || V < 1) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d, V=%d must be >= 1", B, T, V);
    if ((int64_t)B * T > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "B*T too large");
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    const int64_t rows = (int64_t)B * T;
    // next-token targets (CrossEntropyLoss.cpp:25-33): position s of row b predicts tokens[b][s+1]
    std::vector<int32_t> target(rows, -1);
    int count = 0;
    for (int b = 0; b < B; ++b)
        for (int s = 0; s + 1 < T; ++s) {
            const int32_t t = tokens[(int64_t)b * T + s + 1];
            if (t == ignore_index) continue;
            if (t < 0 || t >= V)
                return set_error(DT_ERR_INVALID_ARG, "token %d at (%d, %d) outside [0, %d)", t, b, s + 1, V);
            target[(int64_t)b * T + s] = t;
            ++count;
        }
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    DT_TRY(check_device_binding(ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    // workspace in the context's staging buffers: targets, per-row terms, the loss
    DT_TRY(ctx->stage[7].ensure(rows * 4));
    DT_TRY(ctx->stage[8].ensure(rows * 4));
    DT_TRY(ctx->stage[9].ensure(256));
    int32_t* dtarget = static_cast<int32_t*>(ctx->stage[7].ptr);
    float* term = static_cast<float*>(ctx->stage[8].ptr);
    float* dloss = static_cast<float*>(ctx->stage[9].ptr);
    DT_HIP_TRY(hipMemcpyAsync(dtarget, target.data(), rows * 4, hipMemcpyHostToDevice, s));
    const float* lg = logits;
    float* gr = d_logits;
    const size_t lbytes = (size_t)rows * V * 4;
    if (mem == DT_MEM_HOST) {
        DT_TRY(ctx->stage[5].ensure(lbytes));
        DT_HIP_TRY(hipMemcpyAsync(ctx->stage[5].ptr, logits, lbytes, hipMemcpyHostToDevice, s));
        lg = static_cast<const float*>(ctx->stage[5].ptr);
        if (d_logits) {
            DT_TRY(ctx->stage[6].ensure(lbytes));
            gr = static_cast<float*>(ctx->stage[6].ptr);
        }
    }
    DT_TRY(launch_ce_loss(lg, dtarget, term, gr, dloss, (int)rows, V, count, s));
    if (mem == DT_MEM_HOST && d_logits) DT_HIP_TRY(hipMemcpyAsync(d_logits, gr, lbytes, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipMemcpyAsync(loss, dloss, 4, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipStreamSynchronize(s));
    return DT_OK;
}

}  // extern "C"
