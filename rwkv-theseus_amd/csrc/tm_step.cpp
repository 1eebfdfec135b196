// theseus_tm_serving_step: one TimeMix serving step (T = 1, no autograd) in one call.
//
// It issues exactly the launches the Python layer (theseus/timemix.py, TimeMix._run on
// the fused kernels with few rows) issues for such a step, in the same order and with the
// same arguments, so its results are bitwise those of that path: shift-lerp, one grouped
// few-row GEMM for r, k, v and the LoRA first halves, one for the LoRA second halves, the
// decay input, the WKV operands, the single-step recurrence (in place when the state
// pointers agree), GroupNorm + bonus + gate, the output projection and, in place, the
// shift state update.  What it saves is host time: the Python path spends ~0.25 ms per
// token issuing these launches and allocating their outputs (C = 5120, B = 64), twice the
// kernels' own 0.13 ms; here every intermediate lives in the caller's workspace.
#include "../../include/theseus_gemm.h"
#include "../../include/theseus_timemix.h"
#include "../../include/theseus_wkv7.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

// the workspace's pieces, 256-byte aligned
struct Layout {
    size_t mix[6], r, k, v, mid[3], up[3], w, kw, aw, bw, y, gn, gws_a, gws_b, gws_o, fws, total;
    size_t ga = 0, gb = 0, go = 0, fw = 0;  // GEMM and out-of-place forward workspace bytes
};

size_t al(size_t x) { return (x + 255) / 256 * 256; }

// The two grouped products, in the Python layer's order (r, k, v and the LoRA first halves
// w, a, g; then the second halves).  ws null: shapes only (for the workspace sizes).
void problems(const theseus_tm_layer* L, uint8_t* ws, const Layout& o, theseus_gemm_problem (&a)[6],
              theseus_gemm_problem (&b)[3]) {
    auto at = [&](size_t off) -> void* { return ws ? ws + off : nullptr; };
    const int C = L->C, rk[3] = {L->rank_w, L->rank_a, L->rank_g};
    const void* wts[3] = {L->w_r, L->w_k, L->w_v};
    const size_t outs[3] = {o.r, o.k, o.v}, src[3] = {o.mix[0], o.mix[2], o.mix[3]};  // mixes r, k, v
    for (int i = 0; i < 3; i++) a[i] = theseus_gemm_problem{C, C, THESEUS_GEMM_NONE, at(src[i]), wts[i], at(outs[i])};
    const void* downs[3] = {L->w1t, L->a1t, L->g1t};
    const int acts[3] = {THESEUS_GEMM_TANH, THESEUS_GEMM_NONE, THESEUS_GEMM_SIGMOID};
    const size_t dmix[3] = {o.mix[1], o.mix[4], o.mix[5]};  // mixes w, a, g
    for (int i = 0; i < 3; i++) a[3 + i] = theseus_gemm_problem{rk[i], C, acts[i], at(dmix[i]), downs[i], at(o.mid[i])};
    const void* ups[3] = {L->w2t, L->a2t, L->g2t};
    for (int i = 0; i < 3; i++) b[i] = theseus_gemm_problem{C, rk[i], THESEUS_GEMM_NONE, at(o.mid[i]), ups[i], at(o.up[i])};
}

bool layout(const theseus_tm_layer* L, int B, Layout& o) {
    if (!L || B < 1 || B > THESEUS_GEMM_MAX_ROWS || L->N != 64 || L->C < 64 || L->C % 64 || L->C != L->H * L->N)
        return false;
    const size_t act = al((size_t)B * L->C * 2);
    size_t p = 0;
    for (int i = 0; i < 6; i++) o.mix[i] = p, p += act;
    o.r = p, p += act;
    o.k = p, p += act;
    o.v = p, p += act;
    const int rk[3] = {L->rank_w, L->rank_a, L->rank_g};
    for (int i = 0; i < 3; i++) o.mid[i] = p, p += al((size_t)B * rk[i] * 2);
    for (int i = 0; i < 3; i++) o.up[i] = p, p += act;
    o.w = p, p += act;
    o.kw = p, p += act;
    o.aw = p, p += act;
    o.bw = p, p += act;
    o.y = p, p += act;
    o.gn = p, p += act;
    theseus_gemm_problem a[6], b[3];
    problems(L, nullptr, o, a, b);
    for (int i = 0; i < 6; i++)
        if (a[i].N < 1 || a[i].K < 1) return false;
    o.ga = theseus_gemm_rows_group_workspace_size(B, 6, a);
    o.gb = theseus_gemm_rows_group_workspace_size(B, 3, b);
    o.go = theseus_gemm_rows_workspace_size(B, L->C, L->C);
    o.fw = theseus_wkv7_forward_workspace_size(B, 1, L->H, L->N, THESEUS_WKV7_BF16);
    o.gws_a = p, p += al(o.ga);
    o.gws_b = p, p += al(o.gb);
    o.gws_o = p, p += al(o.go);
    o.fws = p, p += al(o.fw);
    o.total = p;
    return true;
}

}  // namespace

extern "C" {

size_t theseus_tm_serving_step_workspace(const theseus_tm_layer* layer, int B) {
    Layout o;
    return layout(layer, B, o) ? o.total : 0;
}

int theseus_tm_serving_step(const theseus_tm_layer* L, int B, const void* x, const void* shift_in, void* shift_out,
                            const float* wkv_in, float* wkv_out, void* out, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    Layout o;
    if (!layout(L, B, o)) return THESEUS_WKV7_ERR_SHAPE;
    if (!x || !shift_in || !wkv_in || !wkv_out || !out || !L->coef || !L->w_o || !L->w0 || !L->a0 || !L->k_k ||
        !L->k_a || !L->r_k || !L->ln_w || !L->ln_b)
        return THESEUS_WKV7_ERR_NULL;
    if (!workspace || workspace_bytes < o.total) return THESEUS_WKV7_ERR_WORKSPACE;
    uint8_t* const ws = static_cast<uint8_t*>(workspace);
    const int C = L->C, H = L->H, N = L->N;
    auto at = [&](size_t off) { return static_cast<void*>(ws + off); };
    int st;
    void* mixes[6];
    for (int i = 0; i < 6; i++) mixes[i] = at(o.mix[i]);
    if ((st = theseus_tm_shift_lerp_fwd(B, 1, C, x, shift_in, L->coef, mixes, stream))) return st;
    theseus_gemm_problem a[6], b[3];
    problems(L, ws, o, a, b);
    if ((st = theseus_gemm_rows_group(B, 6, a, at(o.gws_a), o.ga, stream))) return st;
    if ((st = theseus_gemm_rows_group(B, 3, b, at(o.gws_b), o.gb, stream))) return st;
    if ((st = theseus_tm_add_param_fwd(B, 1, C, at(o.up[0]), L->w0, at(o.w), stream))) return st;
    if ((st = theseus_tm_kk_fwd(B, 1, C, at(o.k), at(o.up[1]), L->a0, L->k_k, L->k_a, at(o.kw), at(o.aw), at(o.bw),
                                stream)))
        return st;
    if (wkv_out == wkv_in)
        st = theseus_wkv7_decode_step(B, H, N, THESEUS_WKV7_BF16, at(o.r), at(o.w), at(o.kw), at(o.v), at(o.aw),
                                      at(o.bw), wkv_out, at(o.y), stream);
    else
        st = theseus_wkv7_forward(B, 1, H, N, THESEUS_WKV7_BF16, at(o.r), at(o.w), at(o.kw), at(o.v), at(o.aw),
                                  at(o.bw), wkv_in, at(o.y), wkv_out, nullptr, o.fw ? at(o.fws) : nullptr, o.fw,
                                  stream);
    if (st) return st;
    if ((st = theseus_tm_gn_fwd(B, 1, C, at(o.y), at(o.r), at(o.k), at(o.up[1]), L->a0, L->k_a, at(o.v), at(o.up[2]),
                                L->r_k, L->ln_w, L->ln_b, L->ln_eps, at(o.gn), stream)))
        return st;
    if ((st = theseus_gemm_rows(B, C, C, THESEUS_GEMM_NONE, at(o.gn), L->w_o, out, at(o.gws_o), o.go, stream)))
        return st;
    if (shift_out && hipMemcpyAsync(shift_out, x, (size_t)B * C * 2, hipMemcpyDeviceToDevice, stream) != hipSuccess)
        return THESEUS_WKV7_ERR_LAUNCH;
    return THESEUS_WKV7_OK;
}

}  // extern "C"
