// model.h — host-side state of a resident model (not part of the ABI).
#pragma once
#include <vector>

#include "internal.h"

namespace ditch {

struct Mat {
    ditch_hip_tensor *t = nullptr;
    float *da = nullptr, *db = nullptr;  // delta A [rank][cols], B [rows][rank]
    int rank = 0;
    void clear_delta() {
        dev_free(da);
        dev_free(db);
        da = db = nullptr;
        rank = 0;
    }
    void release() {
        free_tensor(t);
        t = nullptr;
        clear_delta();
    }
    bool ok() const { return t != nullptr; }
};

struct Vec {
    float *p = nullptr;
    int64_t len = 0;
    void release() {
        dev_free(p);
        p = nullptr;
        len = 0;
    }
};

struct Layer {
    Vec attn_norm, q_bias, k_bias, v_bias, q_norm, k_norm, ffn_norm, corr, q_a_norm, kv_a_norm;
    Mat q, k, v, o, gate, up, down, router, sh_gate, sh_up, sh_down, q_a, q_b, kv_a, kv_b;
    std::vector<Mat> eg, eu, ed;
};

}  // namespace ditch

struct ditch_hip_model {
    ditch_hip *h = nullptr;
    ditch_model_config c{};
    std::vector<uint8_t> moe_layers;
    std::vector<ditch::Layer> layers;
    ditch::Mat embed, lm_head;
    ditch::Vec final_norm;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    // workspace
    ditch::DevBuf x, hbuf, q, k, v, att, o, g, u, kc, vc, rowsb, xa, logit_h, mla_a, mla_b, mla_c;
    ditch::DevBuf r_logits, r_sel, r_selw, r_counts, r_offsets, r_pair_token, r_pair_of, e_gate, e_up, e_out, e_shared,
        segs, segd, e_xa;
    ditch::DevBuf xsplit;  // split activations of the tiled GEMM
    ditch::DevBuf hs, atts, acts;  // A fragments written by the producers (norm, attention, gate/up)
    ~ditch_hip_model();
};
