// Decoder-only LM runner: prefill + KV-cache greedy decode on one HIP stream.
//
// The reference's only decode loop, test_transformer_t::predict (transformer_test.hpp:
// 194-242), re-runs the full prefix through the model every step and feeds the last output
// column back.  This runner computes the same last column incrementally: prefill writes
// every layer's K/V into a device-resident cache, each decode step appends one column per
// sequence and attends over the cache.  Per decode step and layer it issues
//   norm -> QKV GEMM (+bias, +RoPE, K/V appended to the cache in the epilogue)
//   -> split-K attention -> O GEMM (+residual) -> norm -> FFN GEMM(s) (+GELU / SwiGLU,
//   +residual)
// with the decode GEMMs streaming the weights straight from HBM into the matrix cores.
//
// HBM layout (fp32, or bf16 weights / KV cache when the config asks): one weight arena, matrices [out][in] row-major (K-contiguous for
// both the weight-streaming decode GEMM and the tiled prefill GEMM); activations
// token-major [token][feature]; KV cache [layer][seq][head][position][head_dim] so a
// (seq, head) key range is one contiguous stream.
#include "lm.hpp"

#include <cstdlib>

namespace jas {



__global__ void prefill_positions_kernel(int32_t *pos, int B, int P)
{
    long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (n < (long)B * P) pos[n] = (int32_t)(n % P);
}

// copy the k and v sections of the prefill QKV rows into the cache:
// qkv[(b*P + t)*3d + sec*d + h*dh + e] -> cache[b][h][t][e]
template <bool KB>
__global__ void kv_scatter_kernel(const float *__restrict__ qkv, void *kc, void *vc, int B, int P, int H, int dh,
                                  int ctx)
{
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int d4 = (H * dh) / 4;
    long total = (long)B * P * d4;
    if (g >= total) return;
    int c4 = (int)(g % d4);
    long n = g / d4;
    int b = (int)(n / P), t = (int)(n % P);
    int e = c4 * 4, h = e / dh, ee = e % dh;
    int d = H * dh;
    const float *row = qkv + n * 3L * d;
    long dst = (((long)b * H + h) * ctx + t) * dh + ee;
    const float4 k = *(const float4 *)(row + d + e), v = *(const float4 *)(row + 2 * d + e);
    if (KB) {  // bf16 cache, round to nearest even
        *(u32x2 *)((uint16_t *)kc + dst) = u32x2{(uint32_t)f32_to_bf16(k.x) | ((uint32_t)f32_to_bf16(k.y) << 16),
                                                 (uint32_t)f32_to_bf16(k.z) | ((uint32_t)f32_to_bf16(k.w) << 16)};
        *(u32x2 *)((uint16_t *)vc + dst) = u32x2{(uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16),
                                                 (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16)};
    } else {
        *(float4 *)((float *)kc + dst) = k;
        *(float4 *)((float *)vc + dst) = v;
    }
}

// rotary (cos, sin) per (position, frequency), the QKV epilogue's formula in double
__global__ void rope_table_kernel(double2 *tab, int ctx, int dh, float theta)
{
    const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int hp = dh / 2;
    if (g >= (long)ctx * hp) return;
    const int i = (int)(g % hp), p = (int)(g / hp);
    const double a = (double)p * pow((double)theta, -2.0 * i / (double)dh);
    tab[g] = make_double2(cos(a), sin(a));
}

__global__ void swiglu_kernel(const float *__restrict__ gate, const float *__restrict__ up, float *out, long n)
{
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_f(gate[i]) * up[i];
}

// token embedding gather from a packed [V][d] table (GPT-2 ties it to the LM head)
template <bool WB>
__global__ void embed_packed_kernel(const void *__restrict__ wte, const float *__restrict__ wpe,
                                    const int32_t *__restrict__ ids, const int32_t *__restrict__ pos,
                                    float *__restrict__ out, int n, int d, int V)
{
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long)n * d) return;
    int t = (int)(g / d), e = (int)(g % d);
    const long off = WB ? weight_pack_offset_b(ids[t], e, d, (V + 15) >> 4) : weight_pack_offset(ids[t], e, d, (V + 15) >> 4);
    float v = WB ? bf16_to_f32(((const uint16_t *)wte)[off]) : ((const float *)wte)[off];
    if (wpe) v = v + wpe[(long)pos[t] * d + e];
    out[g] = v;
}


// The decode step's first kernel: the position (from the host, or from the device state
// under graph replay) into pos / seqlens, and the embedding of every token at it.  PACKED:
// GPT-2's tied, packed wte plus learned positions; else LLaMA's row-major table.
template <bool PACKED, bool WB>
__global__ void embed_step_kernel(const void *__restrict__ wte, const float *__restrict__ wpe,
                                  const int32_t *__restrict__ ids, const int32_t *__restrict__ state, int host_pos,
                                  int32_t *pos, int32_t *seqlens, float *__restrict__ out, int B, int d, int V)
{
    const int p = state ? state[0] : host_pos;
    const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g < B) {
        pos[g] = p;
        seqlens[g] = p + 1;
    }
    if (g >= (long)B * d) return;
    const int t = (int)(g / d), e = (int)(g % d);
    float v;
    if (PACKED) {
        const long off = WB ? weight_pack_offset_b(ids[t], e, d, (V + 15) >> 4) : weight_pack_offset(ids[t], e, d, (V + 15) >> 4);
        v = WB ? bf16_to_f32(((const uint16_t *)wte)[off]) : ((const float *)wte)[off];
    } else {
        v = ((const float *)wte)[(long)ids[t] * d + e];
    }
    if (wpe) v = v + wpe[(long)p * d + e];
    out[g] = v;
}

// The decode step's last kernel, one workgroup per sequence: the first maximum over the LM
// head's per-workgroup picks (ties to the lowest index) into ids; under graph replay also the
// id into the history at step pos - state[1], and (sequence 0) the device position advanced.
__global__ void __launch_bounds__(256) argmax_finish_kernel(const float *__restrict__ pv, const int *__restrict__ pi,
                                                            int nch, int32_t *ids, int32_t *hist, const int32_t *pos,
                                                            int32_t *state, int B, int cap)
{
    const int row = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int c = threadIdx.x; c < nch; c += 256) {
        const float ov = pv[(long)row * nch + c];
        const int oi = pi[(long)row * nch + c];
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {  // within the wave, then the four waves through LDS
        const float ov = __shfl_xor(bv, o, WAVE);
        const int oi = __shfl_xor(bi, o, WAVE);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    if (threadIdx.x % WAVE == 0) { sv[threadIdx.x / WAVE] = bv; si[threadIdx.x / WAVE] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k)
            if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) { bv = sv[k]; bi = si[k]; }
        const int id = bi == 0x7fffffff ? 0 : bi;
        ids[row] = id;
        if (state) {
            const int p = pos[0], step = p - state[1];
            if (step >= 0 && step < cap) hist[(long)step * B + row] = id;
        }
    }
    // no other workgroup of this kernel reads state[0]: sequence 0's advances it
    if (state && row == 0 && threadIdx.x == 0) state[0] = pos[0] + 1;
}


// token-major x [B][K] -> the packed B-operand layout of 16 token slots (slots >= B zero)
__global__ void pack_tokens_kernel(const float *__restrict__ x, float *__restrict__ out, int B, int K)
{
    const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= 16L * K) return;
    const int n = (int)(g / K), k = (int)(g % K);
    out[packed_b_offset(n, k)] = n < B ? x[(long)n * K + k] : 0.f;
}

// y[n][m] = sum over the K splits, in split order, of part[(s * 16 + n) * M + m]
__global__ void sum_splits_kernel(const float *__restrict__ part, int ks, int B, int M, float *__restrict__ y)
{
    const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long)B * M) return;
    const int n = (int)(g / M), m = (int)(g % M);
    float acc = part[(long)n * M + m];
    for (int sp = 1; sp < ks; ++sp) acc += part[((long)sp * 16 + n) * M + m];
    y[g] = acc;
}

__global__ void copy_ids_kernel(const int32_t *src, int32_t *dst, int B)
{
    int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) dst[b] = src[b];
}

} // namespace jas

using namespace jas;

namespace {

void add_tensor(jas_lm *lm, const char *name, int layers, int rows, int cols, bool packed, size_t &cursor)
{
    Tensor t;
    t.off = cursor;
    t.layers = layers;
    t.rows = rows;
    t.cols = cols;
    t.packed = packed;
    t.bf16 = packed && lm->cfg.weight_bf16;
    t.count = (size_t)layers * t.lstride();
    lm->tensors[name] = t;
    cursor += (t.count + 63) & ~size_t(63);  // 256-byte aligned tensors
}

jas_status prof_begin(jas_lm *lm, int cls)
{
    if (!lm->prof) return JAS_OK;
    if (lm->ev_used + 2 > lm->ev.size()) {
        for (int k = 0; k < 256; ++k) {
            hipEvent_t e;
            JAS_HIP(hipEventCreate(&e));
            lm->ev.push_back(e);
            lm->ev_cls.push_back(0);
        }
    }
    lm->ev_cls[lm->ev_used] = cls;
    JAS_HIP(hipEventRecord(lm->ev[lm->ev_used++], lm->stream));
    return JAS_OK;
}

jas_status prof_end(jas_lm *lm)
{
    if (!lm->prof) return JAS_OK;
    lm->ev_cls[lm->ev_used] = -1;
    JAS_HIP(hipEventRecord(lm->ev[lm->ev_used++], lm->stream));
    return JAS_OK;
}

// y rows are dense [n_vec][d]; x rows are vstride apart
jas_status norm_rows(jas_lm *lm, const float *x, float *y, int n_vec, long vstride, int l_or_f /* -1 final */,
                     int which)
{
    const jas_lm_config &c = lm->cfg;
    const int d = c.d_model;
    const float *g, *b = nullptr;
    if (l_or_f < 0) {
        g = lm->W("lnf_g");
        b = lm->W("lnf_b");
    } else {
        g = lm->LW(which == 1 ? "ln1_g" : "ln2_g", l_or_f);
        b = lm->LW(which == 1 ? "ln1_b" : "ln2_b", l_or_f);
    }
    TRY(prof_begin(lm, 2));
    if (c.kind == 0) TRY(jas_layernorm(x, y, n_vec, d, vstride, d, 1, c.eps, g, b, lm->stream));
    else TRY(jas_rmsnorm(x, y, n_vec, d, vstride, d, 1, c.eps, g, lm->stream));
    return prof_end(lm);
}

// weight GEMM for N tokens whose activations are token-major rows of length K (ld = K)
jas_status proj(jas_lm *lm, const float *Wt, const float *X, int N, int M, int K, const SkinnyEpiArgs &e)
{
    TRY(prof_begin(lm, 0));
    TRY(skinny_gemm(Wt, nullptr, X, K, M, N, K, e, lm->stream, true, nullptr, lm->wbf16()));
    return prof_end(lm);
}

jas_status ensure_prefill(jas_lm *lm, long tokens)
{
    if (tokens <= lm->p_tokens) return JAS_OK;
    const jas_lm_config &c = lm->cfg;
    float **bufs[] = {&lm->pX, &lm->pH, &lm->pQKV, &lm->pATT, &lm->pG, &lm->pU, &lm->pFF};
    for (auto b : bufs) {
        if (*b) JAS_HIP(hipFree(*b));
        *b = nullptr;
    }
    if (lm->pIds) JAS_HIP(hipFree(lm->pIds));
    if (lm->pPos) JAS_HIP(hipFree(lm->pPos));
    const long d = c.d_model, F = c.d_ff;
    size_t sz[] = {(size_t)(tokens * d), (size_t)(tokens * d), (size_t)(tokens * 3 * d), (size_t)(tokens * d),
                   (size_t)(tokens * F), (size_t)(c.kind == 1 ? tokens * F : 4), (size_t)(c.kind == 1 ? tokens * F : 4)};
    for (int k = 0; k < 7; ++k) TRY(jas_malloc((void **)bufs[k], sz[k] * sizeof(float)));
    TRY(jas_malloc((void **)&lm->pIds, tokens * sizeof(int32_t)));
    TRY(jas_malloc((void **)&lm->pPos, tokens * sizeof(int32_t)));
    lm->p_tokens = tokens;
    return JAS_OK;
}

jas_status embed(jas_lm *lm, const int32_t *ids, const int32_t *pos, float *out, int n)
{
    const jas_lm_config &c = lm->cfg;
    TRY(prof_begin(lm, 2));
    if (c.kind == 0) {  // GPT-2: the tied, packed wte plus learned positions
        if (lm->wbf16())
            hipLaunchKernelGGL(embed_packed_kernel<true>, dim3(ceil_div((long)n * c.d_model, 256)), dim3(256), 0,
                               lm->stream, lm->W("wte"), lm->W("wpe"), ids, pos, out, n, c.d_model, c.vocab);
        else
            hipLaunchKernelGGL(embed_packed_kernel<false>, dim3(ceil_div((long)n * c.d_model, 256)), dim3(256), 0,
                               lm->stream, lm->W("wte"), lm->W("wpe"), ids, pos, out, n, c.d_model, c.vocab);
        JAS_LAUNCH_CHECK();
    } else {
        TRY(jas_embed(lm->W("wte"), nullptr, ids, pos, out, n, c.d_model, lm->stream));
    }
    return prof_end(lm);
}

// one decode step for lm->B sequences: d_ids in, argmax written back into d_ids
// One decode step for the active batch.  device_pos: take the position from the device
// state (graph capture/replay) instead of the host counter.  Attention is launched for the
// full cache length (max_ctx) either way -- its splits past a sequence's length are empty --
// so the launch shape, and the arithmetic, do not depend on the step.
jas_status decode_step(jas_lm *lm, bool device_pos)
{
    const jas_lm_config &c = lm->cfg;
    const int B = lm->B, d = c.d_model, F = c.d_ff, H = c.n_head, dh = lm->dh(), V = c.vocab;
    JAS_CHECK(device_pos || lm->position < c.max_ctx, JAS_ERR_RANGE,
              "jas_lm_decode: KV cache full (max_ctx reached)");
    hipStream_t s = lm->stream;
    {  // positions and embeddings in one launch
        TRY(prof_begin(lm, 2));
        const dim3 grid(ceil_div((long)B * d, 256));
        const int32_t *st = device_pos ? lm->dstate : nullptr;
        if (c.kind == 0 && lm->wbf16())
            hipLaunchKernelGGL((embed_step_kernel<true, true>), grid, dim3(256), 0, s, lm->W("wte"), lm->W("wpe"),
                               lm->ids, st, lm->position, lm->pos, lm->seqlens, lm->x, B, d, V);
        else if (c.kind == 0)
            hipLaunchKernelGGL((embed_step_kernel<true, false>), grid, dim3(256), 0, s, lm->W("wte"), lm->W("wpe"),
                               lm->ids, st, lm->position, lm->pos, lm->seqlens, lm->x, B, d, V);
        else
            hipLaunchKernelGGL((embed_step_kernel<false, false>), grid, dim3(256), 0, s, lm->W("wte"), nullptr,
                               lm->ids, st, lm->position, lm->pos, lm->seqlens, lm->x, B, d, V);
        JAS_LAUNCH_CHECK();
        TRY(prof_end(lm));
    }
    // The projections that feed the residual stream (O and down/proj) run K-split and leave
    // their partial sums in lm->part; the next norm kernel adds them (plus the bias) to x.
    int pend_ks = 0;
    const float *pend_bias = nullptr;
    for (int l = 0; l < c.n_layer; ++l) {
        TRY(prof_begin(lm, 2));
        TRY(resid_norm(lm->x, lm->part, pend_ks, pend_bias, lm->LW("ln1_g", l), lm->LW("ln1_b", l), lm->h, B, d,
                       c.eps, c.kind == 1, s, true));
        TRY(prof_end(lm));
        SkinnyEpiArgs eq;
        eq.mode = EPI_QKV;
        eq.bias = lm->LW("b_qkv", l);
        eq.q_out = lm->q;
        eq.k_cache = lm->kv_layer_ptr(lm->kc, l);
        eq.v_cache = lm->kv_layer_ptr(lm->vc, l);
        eq.kv_bf16 = c.kv_bf16;
        eq.pos = lm->pos;
        eq.kv_sb = lm->kv_sb;
        eq.kv_sh = lm->kv_sh;
        eq.d = d;
        eq.dh = dh;
        eq.rope = c.kind == 1;
        eq.theta = c.rope_theta;
        eq.rope_tab = lm->rope_tab;
        TRY(proj(lm, lm->LW("w_qkv", l), lm->h, B, 3 * d, d, eq));
        TRY(prof_begin(lm, 1));
        TRY(attn_decode_impl(lm->q, lm->kv_layer_ptr(lm->kc, l), lm->kv_layer_ptr(lm->vc, l), lm->att, lm->seqlens, B, H,
                             dh, c.max_ctx, lm->kv_sb, lm->kv_sh, 1.0f / sqrtf((float)dh), lm->attn_ws, lm->attn_ctr, s, d,
                             c.kv_bf16 != 0, /*wide*/ true));
        TRY(prof_end(lm));
        SkinnyEpiArgs eo;
        eo.mode = EPI_PARTIAL;
        eo.out = lm->part;
        eo.ksplit = lm->ks_o;
        TRY(proj(lm, lm->LW("w_o", l), lm->att, B, d, d, eo));
        TRY(prof_begin(lm, 2));
        TRY(resid_norm(lm->x, lm->part, lm->ks_o, lm->LW("b_o", l), lm->LW("ln2_g", l), lm->LW("ln2_b", l), lm->h, B,
                       d, c.eps, c.kind == 1, s, true));
        TRY(prof_end(lm));
        SkinnyEpiArgs ed;
        ed.mode = EPI_PARTIAL;
        ed.out = lm->part;
        ed.ksplit = lm->ks_d;
        if (c.kind == 0) {
            SkinnyEpiArgs ef;
            ef.mode = EPI_STORE;
            ef.act = JAS_ACT_GELU;
            ef.bias = lm->LW("b_fc", l);
            ef.out = lm->ff;
            ef.ldo = F;
            ef.out_packed = 1;
            TRY(proj(lm, lm->LW("w_fc", l), lm->h, B, F, d, ef));
            TRY(proj(lm, lm->LW("w_proj", l), lm->ff, B, d, F, ed));
            pend_bias = lm->LW("b_proj", l);
        } else {
            SkinnyEpiArgs eg;
            eg.mode = EPI_SWIGLU;
            eg.out = lm->ff;
            eg.ldo = F;
            eg.out_packed = 1;
            TRY(prof_begin(lm, 0));
            TRY(skinny_gemm(lm->LW("w_gate", l), lm->LW("w_up", l), lm->h, d, F, B, d, eg, s, true, nullptr,
                            lm->wbf16()));
            TRY(prof_end(lm));
            TRY(proj(lm, lm->LW("w_down", l), lm->ff, B, d, F, ed));
            pend_bias = nullptr;
        }
        pend_ks = lm->ks_d;
    }
    TRY(prof_begin(lm, 2));
    TRY(resid_norm(lm->x, lm->part, pend_ks, pend_bias, lm->W("lnf_g"), lm->W("lnf_b"), lm->h, B, d, c.eps,
                   c.kind == 1, s, true));
    TRY(prof_end(lm));
    // LM head; its epilogue also leaves each workgroup's greedy pick per sequence, and one
    // small kernel finishes the argmax (and, under graph replay, records the id and advances
    // the device position)
    SkinnyEpiArgs eh;
    eh.mode = EPI_STORE;
    eh.out = lm->logits;
    eh.ldo = V;
    eh.amax_v = lm->amax_v;
    eh.amax_i = lm->amax_i;
    TRY(proj(lm, c.kind == 0 ? lm->W("wte") : lm->W("w_head"), lm->h, B, V, d, eh));
    TRY(prof_begin(lm, 2));
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(B), dim3(256), 0, s, lm->amax_v, lm->amax_i,
                       skinny_row_groups(V, d, false, false, lm->wbf16()), lm->ids, lm->hist, lm->pos,
                       device_pos ? lm->dstate : nullptr, B, lm->hist_cap);
    JAS_LAUNCH_CHECK();
    TRY(prof_end(lm));
    if (!device_pos) lm->position += 1;
    return JAS_OK;
}

} // namespace

namespace {
// the generator index of element (l, r, k) is (l*rows + r)*cols + k, as for a row-major
// [layers*rows][cols] tensor; each packed layer is filled with its own slice of that stream
jas_status fill_normal_packed_layers(jas_lm *lm, const Tensor &t, float *p, uint64_t seed, uint64_t sid, float std)
{
    if (t.layers == 1) return fill_normal_packed(p, t.rows, t.cols, seed, sid, 0.0f, std, lm->stream, t.bf16);
    // per layer: generate row-major into a scratch buffer, then pack
    float *tmp = nullptr;
    TRY(jas_malloc((void **)&tmp, (size_t)t.rows * t.cols * t.layers * sizeof(float)));
    jas_status st = jas_fill_normal(tmp, (size_t)t.rows * t.cols * t.layers, seed, sid, 0.0f, std, lm->stream);
    for (int l = 0; l < t.layers && st == JAS_OK; ++l)
        st = weight_pack(tmp + (long)l * t.rows * t.cols, p + (long)l * t.lstride(), t.rows, t.cols, false, lm->stream,
                         t.bf16);
    (void)hipStreamSynchronize(lm->stream);
    (void)hipFree(tmp);
    return st;
}
} // namespace

extern "C" {

jas_status jas_lm_create(const jas_lm_config *cfg, jas_lm **out)
{
    JAS_CHECK(cfg && out, JAS_ERR_INVALID, "jas_lm_create: null argument");
    const jas_lm_config &c = *cfg;
    JAS_CHECK(c.kind == 0 || c.kind == 1, JAS_ERR_INVALID, "jas_lm_create: kind must be 0 (GPT-2) or 1 (LLaMA)");
    JAS_CHECK(c.n_layer > 0 && c.d_model > 0 && c.n_head > 0 && c.d_ff > 0 && c.vocab > 0 && c.max_ctx > 0 &&
                  c.max_batch > 0,
              JAS_ERR_INVALID, "jas_lm_create: sizes must be positive");
    // mat_mha_t rejects d_model % heads != 0 (mat_mha_t.hpp:239-240)
    JAS_CHECK(c.d_model % c.n_head == 0, JAS_ERR_INVALID, "d_model must be divisible by num_heads");
    const int dh = c.d_model / c.n_head;
    JAS_CHECK(dh == 32 || dh == 64 || dh == 128, JAS_ERR_INVALID, "jas_lm_create: head dim must be 32, 64 or 128");
    JAS_CHECK(c.d_model % 64 == 0 && c.d_ff % 16 == 0, JAS_ERR_INVALID,
              "jas_lm_create: d_model must be a multiple of 64 and d_ff of 16");
    // one 16-row packed tile never mixes two heads or the q/k/v sections
    JAS_CHECK((c.d_model / c.n_head) % 16 == 0, JAS_ERR_INVALID, "jas_lm_create: head dim must be a multiple of 16");
    JAS_CHECK(c.max_batch <= 16, JAS_ERR_INVALID, "jas_lm_create: max_batch above 16 is not supported");
    JAS_CHECK((c.weight_bf16 == 0 || c.weight_bf16 == 1) && (c.kv_bf16 == 0 || c.kv_bf16 == 1), JAS_ERR_INVALID,
              "jas_lm_create: weight_bf16 and kv_bf16 must be 0 or 1");
    TRY(jas_init(-1));
    jas_lm *lm = new jas_lm();
    lm->cfg = c;
    JAS_HIP(hipStreamCreateWithFlags(&lm->stream, hipStreamNonBlocking));
    const size_t d = c.d_model, F = c.d_ff, L = c.n_layer, V = c.vocab;
    size_t cur = 0;
    const int Li = c.n_layer, di = c.d_model, Fi = c.d_ff, Vi = c.vocab;
    add_tensor(lm, "wte", 1, Vi, di, c.kind == 0, cur);  // GPT-2: also the (packed) LM head
    if (c.kind == 0) add_tensor(lm, "wpe", 1, c.max_ctx, di, false, cur);
    add_tensor(lm, "ln1_g", Li, 1, di, false, cur);
    if (c.kind == 0) add_tensor(lm, "ln1_b", Li, 1, di, false, cur);
    add_tensor(lm, "w_qkv", Li, 3 * di, di, true, cur);
    if (c.kind == 0) add_tensor(lm, "b_qkv", Li, 1, 3 * di, false, cur);
    add_tensor(lm, "w_o", Li, di, di, true, cur);
    if (c.kind == 0) add_tensor(lm, "b_o", Li, 1, di, false, cur);
    add_tensor(lm, "ln2_g", Li, 1, di, false, cur);
    if (c.kind == 0) add_tensor(lm, "ln2_b", Li, 1, di, false, cur);
    if (c.kind == 0) {
        add_tensor(lm, "w_fc", Li, Fi, di, true, cur);
        add_tensor(lm, "b_fc", Li, 1, Fi, false, cur);
        add_tensor(lm, "w_proj", Li, di, Fi, true, cur);
        add_tensor(lm, "b_proj", Li, 1, di, false, cur);
    } else {
        add_tensor(lm, "w_gate", Li, Fi, di, true, cur);
        add_tensor(lm, "w_up", Li, Fi, di, true, cur);
        add_tensor(lm, "w_down", Li, di, Fi, true, cur);
    }
    add_tensor(lm, "lnf_g", 1, 1, di, false, cur);
    if (c.kind == 0) add_tensor(lm, "lnf_b", 1, 1, di, false, cur);
    if (c.kind == 1) add_tensor(lm, "w_head", 1, Vi, di, true, cur);
    lm->arena_count = cur;
    jas_status st = jas_malloc((void **)&lm->arena, cur * sizeof(float));
    if (st != JAS_OK) {
        jas_lm_destroy(lm);
        return st;
    }
    const int Bm = c.max_batch;
    lm->kv_sh = (long)c.max_ctx * dh;
    lm->kv_sb = (long)c.n_head * lm->kv_sh;
    lm->kv_layer = (long)Bm * lm->kv_sb;
    size_t kvn = (size_t)L * lm->kv_layer;
    st = jas_malloc((void **)&lm->kc, kvn * lm->kv_es());
    if (st == JAS_OK) st = jas_malloc((void **)&lm->vc, kvn * lm->kv_es());
    // decode activations span all 16 MFMA token columns (the packed B-operand layout)
    struct { float **p; size_t n; } fb[] = {{&lm->x, 16 * d}, {&lm->h, 16 * d}, {&lm->q, 16 * d}, {&lm->att, 16 * d},
                                            {&lm->ff, 16 * F}, {&lm->logits, Bm * V}};
    for (auto &f : fb) {
        if (st == JAS_OK) st = jas_malloc((void **)f.p, f.n * sizeof(float));
        if (st == JAS_OK) st = jas_memset(*f.p, 0, f.n * sizeof(float), lm->stream);
    }
    if (st == JAS_OK) st = jas_malloc((void **)&lm->ids, 64 * sizeof(int32_t));
    if (st == JAS_OK) st = jas_malloc((void **)&lm->pos, 64 * sizeof(int32_t));
    if (st == JAS_OK) st = jas_malloc((void **)&lm->seqlens, 64 * sizeof(int32_t));
    if (st == JAS_OK) st = jas_malloc((void **)&lm->dstate, 2 * sizeof(int32_t));
    // the LM head's per-workgroup greedy picks: [16 tokens][row groups], at most V / 16 groups
    if (st == JAS_OK) st = jas_malloc((void **)&lm->amax_v, sizeof(float) * 16 * (size_t)ceil_div(V, 16));
    if (st == JAS_OK) st = jas_malloc((void **)&lm->amax_i, sizeof(int) * 16 * (size_t)ceil_div(V, 16));
    lm->attn_ws_bytes = jas_attn_decode_workspace(Bm, c.n_head, dh, c.max_ctx);
    for (int b = 1; b < Bm; ++b)  // workspace must cover every batch size actually used
        lm->attn_ws_bytes = std::max(lm->attn_ws_bytes, jas_attn_decode_workspace(b, c.n_head, dh, c.max_ctx));
    if (st == JAS_OK && lm->attn_ws_bytes) st = jas_malloc(&lm->attn_ws, lm->attn_ws_bytes);
    // split-arrival counters of the attention's in-kernel merge: zero here, and every decode
    // step leaves them zero (outside any captured graph)
    if (st == JAS_OK && lm->attn_ws_bytes) st = jas_malloc((void **)&lm->attn_ctr, sizeof(unsigned) * Bm * c.n_head);
    if (st == JAS_OK && lm->attn_ctr) st = jas_memset(lm->attn_ctr, 0, sizeof(unsigned) * Bm * c.n_head, lm->stream);
    if (st == JAS_OK && c.kind == 1) {
        const long n = (long)c.max_ctx * (dh / 2);
        st = jas_malloc((void **)&lm->rope_tab, sizeof(double2) * n);
        if (st == JAS_OK)
            hipLaunchKernelGGL(rope_table_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, lm->stream, lm->rope_tab,
                               c.max_ctx, dh, c.rope_theta);
    }
    // K splits of the d-row residual projections: enough workgroups to cover the chip
    lm->ks_o = skinny_pick_ksplit(c.d_model, c.d_model, lm->wbf16());
    lm->ks_d = skinny_pick_ksplit(c.d_model, c.d_ff, lm->wbf16());
    if (st == JAS_OK)
        st = jas_malloc((void **)&lm->part, sizeof(float) * (size_t)std::max(lm->ks_o, lm->ks_d) * 16 * c.d_model);
    if (st != JAS_OK) {
        jas_lm_destroy(lm);
        return st;
    }
    *out = lm;
    return JAS_OK;
}

jas_status jas_lm_destroy(jas_lm *lm)
{
    if (!lm) return JAS_OK;
    if (lm->stream) (void)hipStreamSynchronize(lm->stream);
    if (lm->graph) (void)hipGraphExecDestroy(lm->graph);
    void *ptrs[] = {lm->amax_v, lm->amax_i, lm->dstate, lm->arena, lm->kc, lm->vc, lm->x, lm->h, lm->q, lm->att, lm->ff, lm->logits, lm->ids, lm->pos,
                    lm->seqlens, lm->hist, lm->attn_ws, lm->attn_ctr, lm->part, lm->pX, lm->pH, lm->pQKV, lm->pATT, lm->pG, lm->pU, lm->pFF,
                    lm->pIds, lm->pPos, lm->rope_tab};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    for (auto e : lm->ev) (void)hipEventDestroy(e);
    if (lm->proj_done) (void)hipEventDestroy(lm->proj_done);
    if (lm->stream) (void)hipStreamDestroy(lm->stream);
    delete lm;
    return JAS_OK;
}

jas_status jas_lm_init_random(jas_lm *lm, uint64_t seed, float std)
{
    JAS_CHECK(lm, JAS_ERR_INVALID, "jas_lm_init_random: null model");
    uint64_t sid = 0;
    for (auto &kv : lm->tensors) {  // std::map: deterministic (name) order
        const std::string &n = kv.first;
        float *p = lm->arena + kv.second.off;
        size_t cnt = kv.second.count;
        ++sid;
        if (n == "ln1_g" || n == "ln2_g" || n == "lnf_g") {
            std::vector<float> ones(cnt, 1.0f);
            TRY(jas_memcpy_h2d(p, ones.data(), cnt * sizeof(float), lm->stream));
        } else if (n[0] == 'b' || n == "ln1_b" || n == "ln2_b" || n == "lnf_b") {
            JAS_HIP(hipMemsetAsync(p, 0, cnt * sizeof(float), lm->stream));
        } else if (kv.second.packed) {  // same values as a row-major fill of [layers*rows][cols]
            TRY(fill_normal_packed_layers(lm, kv.second, p, seed, sid, std));
        } else {
            TRY(jas_fill_normal(p, cnt, seed, sid, 0.0f, std, lm->stream));
        }
    }
    JAS_HIP(hipStreamSynchronize(lm->stream));
    return JAS_OK;
}

jas_status jas_lm_weight_shape(jas_lm *lm, const char *name, int *layers, int *rows, int *cols)
{
    JAS_CHECK(lm && name && layers && rows && cols, JAS_ERR_INVALID, "jas_lm_weight_shape: null argument");
    auto it = lm->tensors.find(name);
    *layers = *rows = *cols = 0;
    if (it == lm->tensors.end()) return JAS_OK;
    *layers = it->second.layers;
    *rows = it->second.rows;
    *cols = it->second.cols;
    return JAS_OK;
}

// host <-> device copy of a tensor in logical row-major [layers][rows][cols] order
static jas_status weight_copy(jas_lm *lm, const char *name, float *h, size_t count, bool to_host)
{
    JAS_CHECK(lm && name && h, JAS_ERR_INVALID, "jas_lm weight copy: null argument");
    auto it = lm->tensors.find(name);
    JAS_CHECK(it != lm->tensors.end(), JAS_ERR_INVALID, std::string("jas_lm: no weight named ") + name);
    const Tensor &t = it->second;
    const size_t n = (size_t)t.layers * t.rows * t.cols;
    JAS_CHECK(count == n, JAS_ERR_INVALID, "jas_lm weight copy: element count mismatch");
    float *dev = lm->arena + t.off;
    if (!t.packed) {
        return to_host ? jas_memcpy_d2h(h, dev, n * sizeof(float), lm->stream)
                       : jas_memcpy_h2d(dev, h, n * sizeof(float), lm->stream);
    }
    float *tmp = nullptr;
    TRY(jas_malloc((void **)&tmp, n * sizeof(float)));
    jas_status st = JAS_OK;
    const long lsz = (long)t.rows * t.cols;
    if (!to_host) st = jas_memcpy_h2d(tmp, h, n * sizeof(float), lm->stream);
    for (int l = 0; l < t.layers && st == JAS_OK; ++l)
        st = to_host ? weight_pack(dev + l * t.lstride(), tmp + l * lsz, t.rows, t.cols, true, lm->stream, t.bf16)
                     : weight_pack(tmp + l * lsz, dev + l * t.lstride(), t.rows, t.cols, false, lm->stream, t.bf16);
    if (to_host && st == JAS_OK) st = jas_memcpy_d2h(h, tmp, n * sizeof(float), lm->stream);
    (void)hipStreamSynchronize(lm->stream);
    (void)hipFree(tmp);
    return st;
}

jas_status jas_lm_get_weight(jas_lm *lm, const char *name, float *h_dst, size_t count)
{
    return weight_copy(lm, name, h_dst, count, true);
}

jas_status jas_lm_set_weight(jas_lm *lm, const char *name, const float *h_src, size_t count)
{
    return weight_copy(lm, name, const_cast<float *>(h_src), count, false);
}

jas_status jas_lm_prefill(jas_lm *lm, int B, int P, const int32_t *h_ids, int32_t *h_next, float *h_logits)
{
    JAS_CHECK(lm && h_ids, JAS_ERR_INVALID, "jas_lm_prefill: null argument");
    const jas_lm_config &c = lm->cfg;
    JAS_CHECK(B >= 1 && B <= c.max_batch && P >= 1, JAS_ERR_INVALID, "jas_lm_prefill: bad batch/prompt size");
    JAS_CHECK(P <= c.max_ctx, JAS_ERR_RANGE, "jas_lm_prefill: prompt longer than max_ctx");
    for (long i = 0; i < (long)B * P; ++i)
        JAS_CHECK(h_ids[i] >= 0 && h_ids[i] < c.vocab, JAS_ERR_INVALID, "jas_lm_prefill: token id out of range");
    const long T = (long)B * P;
    TRY(ensure_prefill(lm, T));
    hipStream_t s = lm->stream;
    const int d = c.d_model, F = c.d_ff, H = c.n_head, dh = lm->dh(), V = c.vocab;
    lm->B = B;
    lm->position = 0;
    TRY(jas_memcpy_h2d(lm->pIds, h_ids, T * sizeof(int32_t), s));
    hipLaunchKernelGGL(prefill_positions_kernel, dim3(ceil_div(T, 256)), dim3(256), 0, s, lm->pPos, B, P);
    TRY(embed(lm, lm->pIds, lm->pPos, lm->pX, (int)T));
    const bool verbose = getenv("JAS_VERBOSE") != nullptr;
    for (int l = 0; l < c.n_layer; ++l) {
        if (verbose && l % 4 == 0) {  // progress for long prefills (synchronises, diagnostics only)
            JAS_HIP(hipStreamSynchronize(s));
            fprintf(stderr, "[jas] prefill layer %d/%d\n", l, c.n_layer);
            fflush(stderr);
        }
        TRY(norm_rows(lm, lm->pX, lm->pH, (int)T, d, l, 1));
        const float *bq = lm->LW("b_qkv", l);
        float *kcl = lm->kv_layer_ptr(lm->kc, l), *vcl = lm->kv_layer_ptr(lm->vc, l);
        // QKV[n][m] = sum_k w_qkv[m][k] H[n][k] (+ b[m]); weights in the packed layout.  On fp32
        // weights the GEMM's epilogue also applies the rotary (LLaMA) and writes k and v into
        // the KV cache; bf16 weights take the GEMM, then the rotary and scatter kernels.
        DmaFused fq;
        fq.mode = FZ_QKV;
        fq.pos = lm->pPos;
        fq.rope_tab = lm->rope_tab;
        fq.rope = c.kind == 1;
        fq.kc = kcl;
        fq.vc = vcl;
        fq.kv_bf16 = c.kv_bf16;
        fq.d = d, fq.dh = dh, fq.H = H, fq.P = P, fq.ctx = c.max_ctx;
        if (lm->wbf16() || !gemm_prefill_fused(3 * d, (int)T, d, lm->LW("w_qkv", l), lm->pH, lm->pQKV, 3L * d, bq, fq, s)) {
            TRY(gemm_general(3 * d, (int)T, d, lm->LW("w_qkv", l), d, 1, lm->pH, 1, d, lm->pQKV, 1, 3L * d, bq,
                             bq ? 1 : 0, JAS_ACT_NONE, 0, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
            if (c.kind == 1)  // q and k sections are 2H consecutive heads of each row
                TRY(jas_rope_llama(lm->pQKV, lm->pPos, (int)T, 2 * H, dh, 3L * d, c.rope_theta, s));
            if (c.kv_bf16)
                hipLaunchKernelGGL(kv_scatter_kernel<true>, dim3(ceil_div(T * (d / 4), 256)), dim3(256), 0, s,
                                   lm->pQKV, kcl, vcl, B, P, H, dh, c.max_ctx);
            else
                hipLaunchKernelGGL(kv_scatter_kernel<false>, dim3(ceil_div(T * (d / 4), 256)), dim3(256), 0, s,
                                   lm->pQKV, kcl, vcl, B, P, H, dh, c.max_ctx);
        }
        // the prompt attends over the keys/values just computed (fp32, in the QKV rows);
        // the cache keeps them for the decode steps (rounded when it is bf16)
        const long qs = (long)P * 3 * d;
        TRY(jas_attn_prefill(lm->pQKV, lm->pQKV + d, lm->pQKV + 2 * d, lm->pATT, B, H, P, P, dh, qs, dh, 3L * d, qs,
                             dh, 3L * d, (long)P * d, dh, d, 1.0f / sqrtf((float)dh), 1, JAS_F32, s));
        const float *bo = lm->LW("b_o", l);
        TRY(gemm_general(d, (int)T, d, lm->LW("w_o", l), d, 1, lm->pATT, 1, d, lm->pX, 1, d, bo, bo ? 1 : 0,
                         JAS_ACT_NONE, 1, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
        TRY(norm_rows(lm, lm->pX, lm->pH, (int)T, d, l, 2));
        if (c.kind == 0) {
            TRY(gemm_general(F, (int)T, d, lm->LW("w_fc", l), d, 1, lm->pH, 1, d, lm->pG, 1, F, lm->LW("b_fc", l), 1,
                             JAS_ACT_GELU, 0, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
            TRY(gemm_general(d, (int)T, F, lm->LW("w_proj", l), F, 1, lm->pG, 1, F, lm->pX, 1, d,
                             lm->LW("b_proj", l), 1, JAS_ACT_NONE, 1, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
        } else {
            // SwiGLU: gate and up in one GEMM whose epilogue writes silu(gate) * up (fp32 weights)
            DmaFused fs;
            fs.mode = FZ_SWIGLU;
            fs.A2 = lm->LW("w_up", l);
            if (lm->wbf16() ||
                !gemm_prefill_fused(2 * F, (int)T, d, lm->LW("w_gate", l), lm->pH, lm->pFF, F, nullptr, fs, s)) {
                TRY(gemm_general(F, (int)T, d, lm->LW("w_gate", l), d, 1, lm->pH, 1, d, lm->pG, 1, F, nullptr, 0,
                                 JAS_ACT_NONE, 0, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
                TRY(gemm_general(F, (int)T, d, lm->LW("w_up", l), d, 1, lm->pH, 1, d, lm->pU, 1, F, nullptr, 0,
                                 JAS_ACT_NONE, 0, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
                hipLaunchKernelGGL(swiglu_kernel, dim3(ceil_div(T * F, 256)), dim3(256), 0, s, lm->pG, lm->pU,
                                   lm->pFF, T * F);
            }
            TRY(gemm_general(d, (int)T, F, lm->LW("w_down", l), F, 1, lm->pFF, 1, F, lm->pX, 1, d, nullptr, 0,
                             JAS_ACT_NONE, 1, 1, 0, 0, 0, 0, s, true, lm->wbf16()));
        }
    }
    // final norm and LM head on the last position of every sequence (packed B operand)
    JAS_HIP(hipMemcpy2DAsync(lm->x, d * sizeof(float), lm->pX + (long)(P - 1) * d, (size_t)P * d * sizeof(float),
                             d * sizeof(float), B, hipMemcpyDeviceToDevice, s));
    TRY(resid_norm(lm->x, nullptr, 0, nullptr, lm->W("lnf_g"), lm->W("lnf_b"), lm->h, B, d, c.eps, c.kind == 1, s,
                   true));
    SkinnyEpiArgs eh;
    eh.mode = EPI_STORE;
    eh.out = lm->logits;
    eh.ldo = V;
    eh.amax_v = lm->amax_v;
    eh.amax_i = lm->amax_i;
    TRY(skinny_gemm(c.kind == 0 ? lm->W("wte") : lm->W("w_head"), nullptr, lm->h, d, V, B, d, eh, s, true, nullptr,
                    lm->wbf16()));
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(B), dim3(256), 0, s, lm->amax_v, lm->amax_i,
                       skinny_row_groups(V, d, false, false, lm->wbf16()), lm->ids, nullptr, nullptr, nullptr, B, 0);
    JAS_LAUNCH_CHECK();
    lm->position = P;
    if (h_next) TRY(jas_memcpy_d2h(h_next, lm->ids, B * sizeof(int32_t), s));
    if (h_logits) TRY(jas_memcpy_d2h(h_logits, lm->logits, (size_t)B * V * sizeof(float), s));
    JAS_HIP(hipStreamSynchronize(s));
    return JAS_OK;
}

jas_status jas_lm_decode(jas_lm *lm, const int32_t *h_ids, int32_t *h_next, float *h_logits)
{
    JAS_CHECK(lm && lm->B > 0, JAS_ERR_RUNTIME, "jas_lm_decode: call jas_lm_prefill first");
    if (h_ids) {
        for (int b = 0; b < lm->B; ++b)
            JAS_CHECK(h_ids[b] >= 0 && h_ids[b] < lm->cfg.vocab, JAS_ERR_INVALID, "jas_lm_decode: token id out of range");
        TRY(jas_memcpy_h2d(lm->ids, h_ids, lm->B * sizeof(int32_t), lm->stream));
    }
    TRY(decode_step(lm, false));
    if (h_next) TRY(jas_memcpy_d2h(h_next, lm->ids, lm->B * sizeof(int32_t), lm->stream));
    if (h_logits) TRY(jas_memcpy_d2h(h_logits, lm->logits, (size_t)lm->B * lm->cfg.vocab * sizeof(float), lm->stream));
    return JAS_OK;
}

namespace {
// (Re)capture the graph-mode decode step plus its id recording when the batch size or the
// id-history buffer changed.  No memset or allocation happens inside the captured region.
jas_status capture_decode_graph(jas_lm *lm)
{
    // (a regrown history buffer can come back at the old address: compare its capacity too)
    if (lm->graph && lm->graph_B == lm->B && lm->graph_hist == lm->hist && lm->graph_cap == lm->hist_cap)
        return JAS_OK;
    if (lm->graph) {
        (void)hipGraphExecDestroy(lm->graph);
        lm->graph = nullptr;
    }
    hipStream_t s = lm->stream;
    JAS_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    // the step's last kernel records the ids and advances the device position
    jas_status st = decode_step(lm, true);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);  // always end the capture, also after a failure
    if (st != JAS_OK) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return fail(JAS_ERR_HIP, std::string("jas_lm_generate: graph capture: ") + hipGetErrorString(e));
    e = hipGraphInstantiate(&lm->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        lm->graph = nullptr;
        return fail(JAS_ERR_HIP, std::string("jas_lm_generate: graph instantiate: ") + hipGetErrorString(e));
    }
    lm->graph_B = lm->B;
    lm->graph_hist = lm->hist;
    lm->graph_cap = lm->hist_cap;
    return JAS_OK;
}
} // namespace

jas_status jas_lm_generate(jas_lm *lm, int steps, int32_t *h_ids)
{
    JAS_CHECK(lm && lm->B > 0, JAS_ERR_RUNTIME, "jas_lm_generate: call jas_lm_prefill first");
    JAS_CHECK(steps >= 0, JAS_ERR_INVALID, "jas_lm_generate: negative steps");
    JAS_CHECK(lm->position + steps <= lm->cfg.max_ctx, JAS_ERR_RANGE, "jas_lm_generate: would overflow max_ctx");
    if (steps > lm->hist_cap) {
        if (lm->hist) JAS_HIP(hipFree(lm->hist));
        lm->hist = nullptr;
        TRY(jas_malloc((void **)&lm->hist, (size_t)steps * 16 * sizeof(int32_t)));
        lm->hist_cap = steps;
    }
    if (lm->prof || !lm->use_graph) {  // per-launch events, or graphs switched off: eager steps
        for (int st = 0; st < steps; ++st) {
            TRY(decode_step(lm, false));
            hipLaunchKernelGGL(copy_ids_kernel, dim3(1), dim3(64), 0, lm->stream, lm->ids, lm->hist + (long)st * lm->B,
                               lm->B);
        }
    } else if (steps > 0) {
        // one decode step as a HIP graph, replayed `steps` times; the position lives on the
        // device and advances inside the step, so the same graph serves every step
        TRY(capture_decode_graph(lm));
        const int32_t st0[2] = {lm->position, lm->position};
        TRY(jas_memcpy_h2d(lm->dstate, st0, sizeof st0, lm->stream));
        for (int st = 0; st < steps; ++st) JAS_HIP(hipGraphLaunch(lm->graph, lm->stream));
        lm->position += steps;
    }
    if (h_ids && steps) TRY(jas_memcpy_d2h(h_ids, lm->hist, (size_t)steps * lm->B * sizeof(int32_t), lm->stream));
    JAS_HIP(hipStreamSynchronize(lm->stream));
    return JAS_OK;
}

int jas_lm_position(jas_lm *lm) { return lm ? lm->position : -1; }

jas_status jas_lm_project(jas_lm *lm, const char *name, int layer, int B, const float *d_x, float *d_y,
                          jas_stream_t stream)
{
    JAS_CHECK(lm && name && d_x && d_y, JAS_ERR_INVALID, "jas_lm_project: null argument");
    const jas_lm_config &c = lm->cfg;
    JAS_CHECK(B >= 1 && B <= 16, JAS_ERR_INVALID, "jas_lm_project: 1 to 16 tokens");
    const std::string n(name);
    const bool head = n == "w_head" || n == "wte";
    JAS_CHECK(head || (layer >= 0 && layer < c.n_layer), JAS_ERR_RANGE, "jas_lm_project: layer out of range");
    const int d = c.d_model, F = c.d_ff, V = c.vocab;
    const float *W = head ? lm->W(name) : lm->LW(n == "w_gate_up" ? "w_gate" : name, layer);
    JAS_CHECK(W, JAS_ERR_INVALID, "jas_lm_project: no such projection for this model kind");
    int M, K, ks = 0;
    bool dual = false;
    if (n == "w_qkv") M = 3 * d, K = d;
    else if (n == "w_o") M = d, K = d, ks = lm->ks_o;
    else if (n == "w_fc") M = F, K = d;
    else if (n == "w_proj" || n == "w_down") M = d, K = F, ks = lm->ks_d;
    else if (n == "w_gate_up") M = F, K = d, dual = true;
    else if (head) M = V, K = d;
    else return fail(JAS_ERR_INVALID, "jas_lm_project: unknown projection name");
    // the library stream when `stream` is NULL, like every jas_* call; the runner's own
    // stream is drained first, since its decode buffers are reused here
    JAS_HIP(hipStreamSynchronize(lm->stream));
    hipStream_t s = stream_or_default(stream);
    float *xp = K == d ? lm->h : lm->ff;  // the runner's packed activation buffers
    hipLaunchKernelGGL(pack_tokens_kernel, dim3(ceil_div(16L * K, 256)), dim3(256), 0, s, d_x, xp, B, K);
    SkinnyEpiArgs e;
    if (ks) {
        e.mode = EPI_PARTIAL;
        e.out = lm->part;
        e.ksplit = ks;
    } else {
        e.mode = dual ? EPI_SWIGLU : EPI_STORE;
        e.out = d_y;
        e.ldo = M;
    }
    TRY(skinny_gemm(W, dual ? lm->LW("w_up", layer) : nullptr, xp, K, M, B, K, e, s, true, nullptr, lm->wbf16()));
    if (ks)
        hipLaunchKernelGGL(sum_splits_kernel, dim3(ceil_div((long)B * M, 256)), dim3(256), 0, s, lm->part, ks, B, M, d_y);
    JAS_LAUNCH_CHECK();
    // the projection used the runner's decode buffers (h / ff / part) on `s`: later runner
    // work waits for it on the device, so a decode queued right after cannot overwrite them
    if (!lm->proj_done) JAS_HIP(hipEventCreateWithFlags(&lm->proj_done, hipEventDisableTiming));
    JAS_HIP(hipEventRecord(lm->proj_done, s));
    JAS_HIP(hipStreamWaitEvent(lm->stream, lm->proj_done, 0));
    return JAS_OK;
}

jas_status jas_lm_proj_geometry(jas_lm *lm, const char *name, int *geo)
{
    JAS_CHECK(lm && name && geo, JAS_ERR_INVALID, "jas_lm_proj_geometry: null argument");
    const jas_lm_config &c = lm->cfg;
    const std::string n(name);
    const int d = c.d_model, F = c.d_ff, V = c.vocab;
    int M, K, ks = 1;
    bool dual = false, split = false;
    if (n == "w_qkv") M = 3 * d, K = d;
    else if (n == "w_o") M = d, K = d, split = true, ks = lm->ks_o;
    else if (n == "w_fc" && c.kind == 0) M = F, K = d;
    else if ((n == "w_proj" && c.kind == 0) || (n == "w_down" && c.kind == 1)) M = d, K = F, split = true, ks = lm->ks_d;
    else if (n == "w_gate_up" && c.kind == 1) M = F, K = d, dual = true;
    else if ((n == "w_head" && c.kind == 1) || (n == "wte" && c.kind == 0)) M = V, K = d;
    else return fail(JAS_ERR_INVALID, "jas_lm_proj_geometry: no such decode projection for this model kind");
    // the same rule skinny_gemm applies when the runner passes no explicit tuning
    const SkinnyTuning t = skinny_default_tuning(M, K, dual, split, lm->wbf16());
    geo[0] = dual && (t.nt < 2 || t.nt % 2) ? 2 : t.nt;
    geo[1] = t.wpb;
    geo[2] = t.depth;
    geo[3] = ks;
    return JAS_OK;
}

int jas_lm_attn_splits(jas_lm *lm, int B)
{
    if (!lm || B <= 0 || B > lm->cfg.max_batch) return 0;
    const jas_lm_config &c = lm->cfg;
    return attn_decode_splits(B, c.n_head, c.d_model / c.n_head, c.max_ctx, c.kv_bf16 != 0, true);
}

jas_status jas_lm_use_graph(jas_lm *lm, int enable)
{
    JAS_CHECK(lm, JAS_ERR_INVALID, "jas_lm_use_graph: null model");
    lm->use_graph = enable != 0;
    return JAS_OK;
}
jas_stream_t jas_lm_stream(jas_lm *lm) { return lm ? (jas_stream_t)lm->stream : nullptr; }

jas_status jas_lm_profile(jas_lm *lm, int enable, double *ms_by_class, long *launches_by_class)
{
    JAS_CHECK(lm, JAS_ERR_INVALID, "jas_lm_profile: null model");
    JAS_HIP(hipStreamSynchronize(lm->stream));
    if (ms_by_class || launches_by_class) {
        double ms[3] = {0, 0, 0};
        long cnt[3] = {0, 0, 0};
        for (size_t i = 0; i + 1 < lm->ev_used; i += 2) {
            float t = 0.f;
            JAS_HIP(hipEventElapsedTime(&t, lm->ev[i], lm->ev[i + 1]));
            int k = lm->ev_cls[i];
            if (k >= 0 && k < 3) {
                ms[k] += t;
                cnt[k] += 1;
            }
        }
        for (int k = 0; k < 3; ++k) {
            if (ms_by_class) ms_by_class[k] = ms[k];
            if (launches_by_class) launches_by_class[k] = cnt[k];
        }
    }
    lm->ev_used = 0;
    lm->prof = enable != 0;
    return JAS_OK;
}

} // extern "C"
