// Fused elementwise evaluation of a jasmine expression tree.
//
// Reference: mat_express_2_param_stable_t / mat_express_1_param_stable_t
// (mat_express_t.hpp:35-117, 360-436) evaluate lazily, element by element, at clone()
// (:96-112, :416-432).  Here the host serialises the tree into a postfix program
// (jas_ew_ins) and ONE kernel evaluates it for every output element: each leaf is read
// once from HBM, the result written once.  No JIT: the program is interpreted, with the
// operand stack held in VGPRs and indexed with wave-uniform s_set_gpr_idx moves.
//
// Numerics follow jasmine's typing: every node carries its C++ ele_type; float nodes are
// computed in float and double nodes in double, and each node's value is rounded to its
// type before its parent uses it (the typed work() parameters do exactly that).  bf16
// nodes (mat_t<jas::bf16>) compute in float and round the result to bf16, nearest even --
// the arithmetic of the host jas::bf16 type.
#include "jas_leaf.hpp"

namespace jas {

struct EwArgs {
    jas_ew_ins ins[JAS_EW_MAX_INS];
    LeafDev leaf[JAS_EW_MAX_LEAVES];
    int n_ins;
    int rows, cols, col_chunks;
    int out_dtype;
    int contig_vec;       // all CONTIG leaves and the output allow float4 access
    void *out;
};

constexpr int VEC = 4;
// The operand stack: 4 slots x VEC doubles = 1024 bits, the widest VGPR tuple LLVM
// indexes in place with s_set_gpr_idx (wider vectors are lowered through scratch).  The
// host emits Sethi-Ullman ordered postfix (the deeper operand first, binary ops flagged
// when their operands arrive swapped), so 4 slots cover every tree of up to 15 leaves.
typedef double regfile_t __attribute__((ext_vector_type(JAS_EW_MAX_STACK * VEC)));
static_assert(JAS_EW_MAX_STACK * VEC == 16, "one 1024-bit register bank");

__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ double round_to(double v, int dt)
{
    if (dt == JAS_F32) return (double)(float)v;
    if (dt == JAS_I32) return (double)(int32_t)v;
    if (dt == JAS_BF16) return (double)round_bf16((float)v);
    return v;
}

__device__ __forceinline__ double binop(int op, int dt, double x, double y)
{
    if (dt == JAS_BF16) {
        float a = (float)x, b = (float)y;
        switch (op) {
        case JAS_OP_ADD: return (double)round_bf16(a + b);
        case JAS_OP_SUB: return (double)round_bf16(a - b);
        case JAS_OP_MUL: return (double)round_bf16(a * b);
        case JAS_OP_DIV: return (double)round_bf16(a / b);
        case JAS_OP_GT: return a > b ? 1.0 : 0.0;
        default: return a < b ? 1.0 : 0.0;
        }
    }
    if (dt == JAS_F32) {
        float a = (float)x, b = (float)y;
        switch (op) {
        case JAS_OP_ADD: return (double)(a + b);
        case JAS_OP_SUB: return (double)(a - b);
        case JAS_OP_MUL: return (double)(a * b);
        case JAS_OP_DIV: return (double)(a / b);
        case JAS_OP_GT: return a > b ? 1.0 : 0.0;
        default: return a < b ? 1.0 : 0.0;
        }
    }
    if (dt == JAS_I32) {
        int32_t a = (int32_t)x, b = (int32_t)y;
        switch (op) {
        case JAS_OP_ADD: return (double)(a + b);
        case JAS_OP_SUB: return (double)(a - b);
        case JAS_OP_MUL: return (double)(a * b);
        case JAS_OP_DIV: return b ? (double)(a / b) : 0.0;
        case JAS_OP_GT: return a > b ? 1.0 : 0.0;
        default: return a < b ? 1.0 : 0.0;
        }
    }
    switch (op) {
    case JAS_OP_ADD: return x + y;
    case JAS_OP_SUB: return x - y;
    case JAS_OP_MUL: return x * y;
    case JAS_OP_DIV: return x / y;
    case JAS_OP_GT: return x > y ? 1.0 : 0.0;
    default: return x < y ? 1.0 : 0.0;
    }
}

__device__ __forceinline__ double unop(int op, int dt, double x, double imm)
{
    if (dt == JAS_F32 || dt == JAS_BF16) {
        float a = (float)x, r;
        switch (op) {
        case JAS_OP_EXP: r = expf(a); break;
        case JAS_OP_SIGMOID: r = (float)(1.0 / (1.0 + (double)expf(-a))); break;
        case JAS_OP_TANH: r = tanhf(a); break;
        case JAS_OP_GELU: r = gelu_f(a); break;
        case JAS_OP_SILU: r = silu_f(a); break;
        case JAS_OP_SQRT: r = sqrtf(a); break;
        case JAS_OP_POW: r = (float)pow((double)a, imm); break;
        default: r = -a; break;
        }
        return dt == JAS_BF16 ? (double)round_bf16(r) : (double)r;
    }
    switch (op) {
    case JAS_OP_EXP: return exp(x);
    case JAS_OP_SIGMOID: return 1.0 / (1.0 + exp(-x));
    case JAS_OP_TANH: return tanh(x);
    case JAS_OP_GELU: return gelu_d(x);
    case JAS_OP_SILU: return x / (1.0 + exp(-x));
    case JAS_OP_SQRT: return sqrt(x);
    case JAS_OP_POW: return round_to(pow(x, imm), dt);
    default: return round_to(-x, dt);
    }
}

__global__ void __launch_bounds__(256) ew_eval_kernel(const EwArgs A)
{
    long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long total = (long)A.rows * A.col_chunks;
    if (gid >= total) return;
    int i = (int)(gid / A.col_chunks);
    int j0 = (int)(gid % A.col_chunks) * VEC;
    int nv = min(VEC, A.cols - j0);
    long lin0 = (long)i * A.cols + j0;

    regfile_t R = 0.0;
    int sp = 0;  // wave-uniform: the program is identical for every lane
    for (int pc = 0; pc < A.n_ins; ++pc) {
        const int op = __builtin_amdgcn_readfirstlane(A.ins[pc].op);
        const int dt = __builtin_amdgcn_readfirstlane(A.ins[pc].dtype);
        const int arg = __builtin_amdgcn_readfirstlane(A.ins[pc].arg);
        const double imm = A.ins[pc].imm;
        double z[VEC];
        if (op == JAS_OP_LEAF) {
            const LeafDev &L = A.leaf[arg];
            if (L.kind == LK_CONTIG && A.contig_vec && L.dtype == JAS_F32) {
                float4 v = *(const float4 *)((const float *)L.p + lin0);
                z[0] = v.x; z[1] = v.y; z[2] = v.z; z[3] = v.w;
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    int ee = e < nv ? e : 0;
                    long idx = L.kind == LK_CONTIG ? lin0 + ee : leaf_index(L, i, j0 + ee);
                    z[e] = load_elem(L.p, idx, L.dtype);
                }
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) z[e] = round_to(z[e], dt);
            int d = __builtin_amdgcn_readfirstlane(sp * VEC);
#pragma unroll
            for (int e = 0; e < VEC; ++e) R[d + e] = z[e];
            ++sp;
        } else if (op == JAS_OP_CONST) {
            double c = round_to(imm, dt);
            int d = __builtin_amdgcn_readfirstlane(sp * VEC);
#pragma unroll
            for (int e = 0; e < VEC; ++e) R[d + e] = c;
            ++sp;
        } else if (op >= JAS_OP_ADD && op <= JAS_OP_LT) {
            // arg bit 0: the right operand was pushed first (Sethi-Ullman order)
            int lo = __builtin_amdgcn_readfirstlane((sp - 2) * VEC);
            int hi = __builtin_amdgcn_readfirstlane((sp - 1) * VEC);
            double x[VEC], y[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) { x[e] = R[lo + e]; y[e] = R[hi + e]; }
            if (arg & 1) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) z[e] = binop(op, dt, y[e], x[e]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) z[e] = binop(op, dt, x[e], y[e]);
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) R[lo + e] = z[e];
            --sp;
        } else {
            int t = __builtin_amdgcn_readfirstlane((sp - 1) * VEC);
            double x[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) x[e] = R[t + e];
#pragma unroll
            for (int e = 0; e < VEC; ++e) z[e] = unop(op, dt, x[e], imm);
#pragma unroll
            for (int e = 0; e < VEC; ++e) R[t + e] = z[e];
        }
    }
    double res[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) res[e] = R[e];
    // store the root (slot 0) as out_dtype
    if (A.out_dtype == JAS_F64) {
        double *o = (double *)A.out + lin0;
        for (int e = 0; e < nv; ++e) o[e] = res[e];
    } else if (A.out_dtype == JAS_I32) {
        int32_t *o = (int32_t *)A.out + lin0;
        for (int e = 0; e < nv; ++e) o[e] = (int32_t)res[e];
    } else if (A.out_dtype == JAS_BF16) {
        uint16_t *o = (uint16_t *)A.out + lin0;
        for (int e = 0; e < nv; ++e) o[e] = f32_to_bf16((float)res[e]);
    } else {
        float *o = (float *)A.out + lin0;
        if (A.contig_vec) {
            *(float4 *)o = make_float4((float)res[0], (float)res[1], (float)res[2], (float)res[3]);
        } else {
            for (int e = 0; e < nv; ++e) o[e] = (float)res[e];
        }
    }
}

__device__ __forceinline__ void store_elem(void *p, long idx, int dtype, double v)
{
    switch (dtype) {
    case JAS_F64: ((double *)p)[idx] = v; break;
    case JAS_I32: ((int32_t *)p)[idx] = (int32_t)v; break;
    case JAS_BF16: ((uint16_t *)p)[idx] = f32_to_bf16((float)v); break;
    default: ((float *)p)[idx] = (float)v; break;
    }
}

__global__ void leaf_assign_kernel(const void *src, int src_dtype, int rows, int cols, LeafDev L)
{
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long)rows * cols) return;
    int i = (int)(g / cols), j = (int)(g % cols);
    store_elem((void *)L.p, leaf_index(L, i, j), L.dtype, load_elem(src, g, src_dtype));
}

} // namespace jas

using namespace jas;

extern "C" jas_status jas_leaf_assign(const void *src, int32_t src_dtype, int rows, int cols, const jas_leaf *dst,
                                      jas_stream_t stream)
{
    JAS_CHECK(src && dst && dst->d_data && rows >= 0 && cols >= 0, JAS_ERR_INVALID, "jas_leaf_assign: bad arguments");
    JAS_CHECK(dst->rows > 0 && dst->cols > 0, JAS_ERR_INVALID, "jas_leaf_assign: empty destination");
    if (!rows || !cols) return JAS_OK;
    LeafDev L = classify(*dst, rows, cols);
    if (L.kind == LK_CONTIG) {
        L.kind = LK_STRIDED;
        L.rs = cols;
        L.cs = 1;
    }
    long n = (long)rows * cols;
    hipLaunchKernelGGL(leaf_assign_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream_or_default(stream), src,
                       src_dtype, rows, cols, L);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

extern "C" jas_status jas_ew_eval(const jas_ew_ins *prog, int n_ins, const jas_leaf *leaves, int n_leaves,
                                  void *d_out, int32_t out_dtype, int rows, int cols, jas_stream_t stream)
{
    JAS_CHECK(prog && n_ins > 0 && n_ins <= JAS_EW_MAX_INS, JAS_ERR_INVALID, "jas_ew_eval: bad program size");
    JAS_CHECK(n_leaves >= 0 && n_leaves <= JAS_EW_MAX_LEAVES, JAS_ERR_INVALID, "jas_ew_eval: too many leaves");
    JAS_CHECK(rows > 0 && cols > 0 && d_out, JAS_ERR_INVALID, "jas_ew_eval: empty output");
    // validate the program on the host: stack depth, leaf indices, op codes
    int sp = 0;
    for (int k = 0; k < n_ins; ++k) {
        const jas_ew_ins &in = prog[k];
        if (in.op == JAS_OP_LEAF) {
            JAS_CHECK(in.arg >= 0 && in.arg < n_leaves, JAS_ERR_INVALID, "jas_ew_eval: leaf index out of range");
            ++sp;
        } else if (in.op == JAS_OP_CONST) {
            ++sp;
        } else if (in.op >= JAS_OP_ADD && in.op <= JAS_OP_LT) {
            JAS_CHECK(sp >= 2, JAS_ERR_INVALID, "jas_ew_eval: stack underflow");
            --sp;
        } else if (in.op >= JAS_OP_EXP && in.op <= JAS_OP_NEG) {
            JAS_CHECK(sp >= 1, JAS_ERR_INVALID, "jas_ew_eval: stack underflow");
        } else {
            return fail(JAS_ERR_INVALID, "jas_ew_eval: unknown op");
        }
        JAS_CHECK(sp <= JAS_EW_MAX_STACK, JAS_ERR_INVALID, "jas_ew_eval: expression too deep");
        JAS_CHECK(in.dtype == JAS_F32 || in.dtype == JAS_F64 || in.dtype == JAS_I32 || in.dtype == JAS_BF16,
                  JAS_ERR_INVALID, "jas_ew_eval: bad node dtype");
    }
    JAS_CHECK(sp == 1, JAS_ERR_INVALID, "jas_ew_eval: program must leave exactly one value");

    EwArgs A{};
    std::memcpy(A.ins, prog, sizeof(jas_ew_ins) * n_ins);
    A.n_ins = n_ins;
    A.rows = rows; A.cols = cols;
    A.col_chunks = (cols + VEC - 1) / VEC;
    A.out = d_out;
    A.out_dtype = out_dtype;
    JAS_CHECK(out_dtype == JAS_F32 || out_dtype == JAS_F64 || out_dtype == JAS_I32 || out_dtype == JAS_BF16,
              JAS_ERR_INVALID, "jas_ew_eval: bad output dtype");
    bool vec = (cols % VEC) == 0 && ((uintptr_t)d_out % 16) == 0 && out_dtype == JAS_F32;
    for (int k = 0; k < n_leaves; ++k) {
        JAS_CHECK(leaves[k].d_data && leaves[k].rows > 0 && leaves[k].cols > 0, JAS_ERR_INVALID,
                  "jas_ew_eval: empty leaf");
        A.leaf[k] = classify(leaves[k], rows, cols);
        if (A.leaf[k].kind == LK_CONTIG && ((uintptr_t)leaves[k].d_data % 16) != 0) vec = false;
    }
    A.contig_vec = vec ? 1 : 0;
    if (ew_jit_wanted((long)rows * cols))
        return ew_jit_launch(prog, n_ins, A.leaf, n_leaves, vec, d_out, out_dtype, rows, cols, stream_or_default(stream));
    long total = (long)rows * A.col_chunks;
    hipLaunchKernelGGL(ew_eval_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, stream_or_default(stream), A);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}
