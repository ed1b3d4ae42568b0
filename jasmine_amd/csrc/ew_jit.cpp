// Specialised fused elementwise kernels for large expression evaluations.
//
// jas_ew_eval interprets the postfix program (ew_eval_kernel); interpretation costs a
// few hundred instructions per element and leaves an 8192x8192 evaluation compute-bound
// at a fraction of HBM bandwidth.  For large outputs the same program is instead turned
// into straight-line HIP source -- one typed local per node, leaves loaded once per
// element (16-byte non-temporal loads and stores for dense row-major operands, the fastest
// streaming form measured on MI355X), constants as exact hex literals -- and
// compiled once per distinct program shape with hipRTC for the current device, then
// cached for the process.  The numerics are the interpreter's exactly: every node is
// computed in its own type, rounded to it, with the same device math functions and no
// contraction across nodes.
#include "jas_leaf.hpp"

#include <hip/hiprtc.h>

#include <cstdlib>
#include <mutex>
#include <sstream>
#include <unordered_map>
#include <vector>

namespace jas {

// kernel argument block; the generated source declares the same layout
struct JitLeaf {
    const void *p;
    long rs, cs;
    int rows, cols, row_first, roff, coff, transposed;
};
struct JitArgs {
    JitLeaf leaf[JAS_EW_MAX_LEAVES];
    void *out;
    int rows, cols, col_chunks;
};

static const char *kPrelude = R"JAS(
typedef float fx4 __attribute__((ext_vector_type(4)));
// bf16 elements: widened exactly; narrowed to nearest even (NaN stays a quiet NaN)
__device__ __forceinline__ float bf2f(unsigned short v) { return __uint_as_float((unsigned)v << 16); }
__device__ __forceinline__ unsigned short f2bf(float f)
{
    const unsigned u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)(((u >> 16) & 0x8000u) | 0x7fc0u);
    return (unsigned short)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
struct JitLeaf { const void *p; long rs, cs; int rows, cols, row_first, roff, coff, transposed; };
struct JitArgs { JitLeaf leaf[8]; void *out; int rows, cols, col_chunks; };
__device__ __forceinline__ long gen_index(const JitLeaf &L, int i, int j)
{
    int a = L.transposed ? j + L.coff : i + L.roff;
    int b = L.transposed ? i + L.roff : j + L.coff;
    a %= L.rows;
    b %= L.cols;
    return L.row_first ? (long)a * L.cols + b : (long)b * L.rows + a;
}
__device__ __forceinline__ float gelu_f(float x)
{
#pragma clang fp contract(fast)
    float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(u));
}
__device__ __forceinline__ double gelu_d(double x)
{
#pragma clang fp contract(fast)
    return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
}
__device__ __forceinline__ float silu_f(float x)
{
#pragma clang fp contract(fast)
    return x / (1.0f + expf(-x));
}
)JAS";

static int g_jit_mode = 2;  // 0 never, 1 always, 2 large outputs only
static constexpr long kAutoMinElems = 1L << 20;

// C type of a node's value (bf16 nodes hold their rounded value in a float)
static const char *ctype(int dt) { return dt == JAS_F64 ? "double" : dt == JAS_I32 ? "int" : "float"; }
// C type of a stored element
static const char *stype(int dt) { return dt == JAS_BF16 ? "unsigned short" : ctype(dt); }

static std::string hexlit(double v)
{
    char buf[64];
    std::snprintf(buf, sizeof buf, "%a", v);
    std::string s(buf);
    if (s == "inf") return "__builtin_inf()";
    if (s == "-inf") return "(-__builtin_inf())";
    if (s == "nan" || s == "-nan") return "__builtin_nan(\"\")";
    return s;
}

struct Gen {
    std::string src;
    std::vector<int> leaf_slot;  // program leaf index -> deduplicated slot
    int n_slots = 0;
};

static bool same_leaf(const LeafDev &a, const LeafDev &b)
{
    return a.p == b.p && a.kind == b.kind && a.dtype == b.dtype && a.rs == b.rs && a.cs == b.cs && a.rows == b.rows &&
           a.cols == b.cols && a.row_first == b.row_first && a.roff == b.roff && a.coff == b.coff &&
           a.transposed == b.transposed;
}

// Straight-line source for one program.  Every value is produced for VEC = 4 consecutive
// columns of one output row (loop over e); node k becomes the local `T vk`.
static Gen generate(const jas_ew_ins *prog, int n_ins, const LeafDev *leaves, int n_leaves, bool vec, int out_dtype,
                    std::vector<int> &slot_src)
{
    Gen g;
    g.leaf_slot.assign(n_leaves, -1);
    slot_src.clear();
    for (int k = 0; k < n_leaves; ++k) {
        for (int s = 0; s < (int)slot_src.size(); ++s)
            if (same_leaf(leaves[slot_src[s]], leaves[k])) g.leaf_slot[k] = s;
        if (g.leaf_slot[k] < 0) {
            g.leaf_slot[k] = (int)slot_src.size();
            slot_src.push_back(k);
        }
    }
    g.n_slots = (int)slot_src.size();
    std::ostringstream o;
    o << kPrelude;
    // no contraction between nodes (each node rounds to its type, as in the interpreter);
    // the math helpers above contract exactly like their twins in the library
    o << "extern \"C\" __global__ void __launch_bounds__(256) jas_ew_jit(const JitArgs A)\n{\n"
         "#pragma clang fp contract(off)\n"
         "    long gid = (long)blockIdx.x * 256 + threadIdx.x;\n"
         "    if (gid >= (long)A.rows * A.col_chunks) return;\n"
         "    const int i = (int)(gid / A.col_chunks);\n"
         "    const int j0 = (int)(gid % A.col_chunks) * 4;\n"
         "    const long lin0 = (long)i * A.cols + j0;\n";
    if (!vec) o << "    const int nv = min(4, A.cols - j0);\n";
    // leaf loads (each distinct operand once)
    for (int s = 0; s < g.n_slots; ++s) {
        const LeafDev &L = leaves[slot_src[s]];
        const char *T = ctype(L.dtype), *ST = stype(L.dtype);
        const bool wb = L.dtype == JAS_BF16;
        o << "    " << T << " l" << s << "[4];\n    {\n        const " << ST << " *p = (const " << ST << " *)A.leaf[" << s
          << "].p;\n";
        if (L.kind == LK_CONTIG && vec && L.dtype == JAS_F32) {
            o << "        const fx4 v = __builtin_nontemporal_load((const fx4 *)(p + lin0));\n"
                 "        l" << s << "[0] = v[0]; l" << s << "[1] = v[1]; l" << s << "[2] = v[2]; l" << s << "[3] = v[3];\n";
        } else {
            o << "#pragma unroll\n        for (int e = 0; e < 4; ++e) {\n";
            o << (vec ? "            const int ee = e;\n" : "            const int ee = e < nv ? e : 0;\n");
            const char *w0 = wb ? "bf2f(" : "", *w1 = wb ? ")" : "";
            if (L.kind == LK_CONTIG)
                o << "            l" << s << "[e] = " << w0 << "p[lin0 + ee]" << w1 << ";\n";
            else if (L.kind == LK_STRIDED)
                o << "            l" << s << "[e] = " << w0 << "p[(long)i * A.leaf[" << s << "].rs + (long)(j0 + ee) * A.leaf["
                  << s << "].cs]" << w1 << ";\n";
            else
                o << "            l" << s << "[e] = " << w0 << "p[gen_index(A.leaf[" << s << "], i, j0 + ee)]" << w1
                  << ";\n";
            o << "        }\n";
        }
        o << "    }\n";
    }
    // nodes
    std::vector<int> stack;  // node ids on the evaluation stack
    if (vec && out_dtype == JAS_F32) o << "    float ov[4];\n";
    o << "#pragma unroll\n    for (int e = 0; e < 4; ++e) {\n";
    for (int k = 0; k < n_ins; ++k) {
        const jas_ew_ins &in = prog[k];
        const int dt = in.dtype;
        int vt = dt;
        std::ostringstream rhs;
        // bf16 nodes: the float value rounded to bf16 (interpreter: round_to / binop / unop)
        const bool nb = dt == JAS_BF16;
        const char *r0 = nb ? "rbf(" : "", *r1 = nb ? ")" : "";
        if (in.op == JAS_OP_LEAF) {
            rhs << r0 << "(" << ctype(dt) << ")l" << g.leaf_slot[in.arg] << "[e]" << r1;
        } else if (in.op == JAS_OP_CONST) {
            rhs << r0 << "(" << ctype(dt) << ")" << hexlit(in.imm) << r1;
        } else if (in.op >= JAS_OP_ADD && in.op <= JAS_OP_LT) {
            int hi = stack.back();
            stack.pop_back();
            int lo = stack.back();
            stack.pop_back();
            int x = (in.arg & 1) ? hi : lo, y = (in.arg & 1) ? lo : hi;
            std::string a = std::string("(") + ctype(dt) + ")v" + std::to_string(x);
            std::string b = std::string("(") + ctype(dt) + ")v" + std::to_string(y);
            static const char *sym[] = {"+", "-", "*", "/", ">", "<"};
            const char *op = sym[in.op - JAS_OP_ADD];
            if (in.op == JAS_OP_GT || in.op == JAS_OP_LT) {
                vt = JAS_F64;  // the comparison result is exactly 1 or 0 in any type
                rhs << "(" << a << " " << op << " " << b << ") ? 1.0 : 0.0";
            } else if (in.op == JAS_OP_DIV && dt == JAS_I32) {
                rhs << "(" << b << ") ? " << a << " / " << b << " : 0";
            } else {
                rhs << r0 << a << " " << op << " " << b << r1;
            }
        } else {
            int x = stack.back();
            stack.pop_back();
            std::string xs = "v" + std::to_string(x);
            if (dt == JAS_F32 || dt == JAS_BF16) {
                std::string a = "(float)" + xs;
                rhs << r0;
                switch (in.op) {
                case JAS_OP_EXP: rhs << "expf(" << a << ")"; break;
                case JAS_OP_SIGMOID: rhs << "(float)(1.0 / (1.0 + (double)expf(-" << a << ")))"; break;
                case JAS_OP_TANH: rhs << "tanhf(" << a << ")"; break;
                case JAS_OP_GELU: rhs << "gelu_f(" << a << ")"; break;
                case JAS_OP_SILU: rhs << "silu_f(" << a << ")"; break;
                case JAS_OP_SQRT: rhs << "sqrtf(" << a << ")"; break;
                case JAS_OP_POW: rhs << "(float)pow((double)" << a << ", " << hexlit(in.imm) << ")"; break;
                default: rhs << "-" << a; break;
                }
                rhs << r1;
            } else {
                // fp64 nodes (and int nodes, whose transcendental results stay unrounded)
                std::string a = "(double)" + xs;
                vt = JAS_F64;
                switch (in.op) {
                case JAS_OP_EXP: rhs << "exp(" << a << ")"; break;
                case JAS_OP_SIGMOID: rhs << "1.0 / (1.0 + exp(-" << a << "))"; break;
                case JAS_OP_TANH: rhs << "tanh(" << a << ")"; break;
                case JAS_OP_GELU: rhs << "gelu_d(" << a << ")"; break;
                case JAS_OP_SILU: rhs << a << " / (1.0 + exp(-" << a << "))"; break;
                case JAS_OP_SQRT: rhs << "sqrt(" << a << ")"; break;
                case JAS_OP_POW:
                    vt = dt;
                    rhs << "(" << ctype(dt) << ")pow(" << a << ", " << hexlit(in.imm) << ")";
                    break;
                default:
                    vt = dt;
                    rhs << "(" << ctype(dt) << ")(-" << a << ")";
                    break;
                }
            }
        }
        o << "        const " << ctype(vt) << " v" << k << " = " << rhs.str() << ";\n";
        stack.push_back(k);
    }
    const char *OT = ctype(out_dtype);
    o << "        const " << OT << " res = (" << OT << ")v" << stack.back() << ";\n";
    if (vec && out_dtype == JAS_F32) {
        o << "        ov[e] = res;\n    }\n"
             "    *(fx4 *)((float *)A.out + lin0) = fx4{ov[0], ov[1], ov[2], ov[3]};\n}\n";
    } else if (out_dtype == JAS_BF16) {
        o << "        if (" << (vec ? "true" : "e < nv") << ") ((unsigned short *)A.out)[lin0 + e] = f2bf(res);\n    }\n}\n";
    } else {
        o << "        if (" << (vec ? "true" : "e < nv") << ") ((" << OT << " *)A.out)[lin0 + e] = res;\n    }\n}\n";
    }
    g.src = o.str();
    return g;
}

struct JitKernel {
    hipModule_t mod = nullptr;
    hipFunction_t fn = nullptr;
};

static std::mutex g_jit_mu;
static std::unordered_map<std::string, JitKernel> g_jit_cache;

static jas_status compile(const std::string &src, JitKernel &out)
{
    int dev = 0;
    JAS_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    JAS_HIP(hipGetDeviceProperties(&prop, dev));
    std::string arch = std::string("--offload-arch=") + prop.gcnArchName;
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, src.c_str(), "jas_ew_jit.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        return fail(JAS_ERR_RUNTIME, "jas_ew_eval: hiprtcCreateProgram failed");
    // packed-FP32 instructions stay disabled, as for every other kernel of the library
    const char *opts[] = {arch.c_str(), "-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
    hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
    if (rc != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return fail(JAS_ERR_RUNTIME, "jas_ew_eval: specialised kernel failed to compile: " + log);
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    std::vector<char> code(n);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    JAS_HIP(hipModuleLoadData(&out.mod, code.data()));
    JAS_HIP(hipModuleGetFunction(&out.fn, out.mod, "jas_ew_jit"));
    return JAS_OK;
}

bool ew_jit_wanted(long n_elems)
{
    if (g_jit_mode == 0) return false;
    if (g_jit_mode == 1) return true;
    return n_elems >= kAutoMinElems;
}

jas_status ew_jit_launch(const jas_ew_ins *prog, int n_ins, const LeafDev *leaves, int n_leaves, bool vec,
                         void *out, int out_dtype, int rows, int cols, hipStream_t s)
{
    std::vector<int> slot_src;
    Gen g = generate(prog, n_ins, leaves, n_leaves, vec, out_dtype, slot_src);
    int dev = 0;
    JAS_HIP(hipGetDevice(&dev));
    const std::string key = std::to_string(dev) + "\n" + g.src;
    hipFunction_t fn = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_jit_mu);
        auto it = g_jit_cache.find(key);
        if (it == g_jit_cache.end()) {
            JitKernel k;
            jas_status st = compile(g.src, k);
            if (st != JAS_OK) return st;
            it = g_jit_cache.emplace(key, k).first;
        }
        fn = it->second.fn;
    }
    JitArgs A{};
    for (int sl = 0; sl < g.n_slots; ++sl) {
        const LeafDev &L = leaves[slot_src[sl]];
        A.leaf[sl] = JitLeaf{L.p, L.rs, L.cs, L.rows, L.cols, L.row_first, L.roff, L.coff, L.transposed};
    }
    A.out = out;
    A.rows = rows;
    A.cols = cols;
    A.col_chunks = (cols + 3) / 4;
    const long total = (long)rows * A.col_chunks;
    void *params[] = {&A};
    JAS_HIP(hipModuleLaunchKernel(fn, ceil_div(total, 256), 1, 1, 256, 1, 1, 0, s, params, nullptr));
    return JAS_OK;
}

} // namespace jas

extern "C" int jas_ew_jit_mode(int mode)
{
    const int prev = jas::g_jit_mode;
    if (mode >= 0 && mode <= 2) jas::g_jit_mode = mode;
    return prev;
}
