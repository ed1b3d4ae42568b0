// Device-side view of a jas_leaf (a jasmine mat_t or mat_view_t operand): element
// addressing with jasmine's view offsets/transposition and modulo broadcasting.
#pragma once
#include "jas_common.hpp"

namespace jas {

enum LeafKind : int { LK_CONTIG = 0, LK_STRIDED = 1, LK_GENERAL = 2 };

struct LeafDev {
    const void *p;
    long rs, cs;          // strided form: addr = i*rs + j*cs
    int kind, dtype;
    int rows, cols, row_first, roff, coff, transposed;
};

__device__ __forceinline__ double load_elem(const void *p, long idx, int dtype)
{
    switch (dtype) {
    case JAS_F64: return ((const double *)p)[idx];
    case JAS_I32: return (double)((const int32_t *)p)[idx];
    case JAS_BF16: return (double)bf16_to_f32(((const uint16_t *)p)[idx]);
    default: return (double)((const float *)p)[idx];
    }
}

__device__ __forceinline__ long leaf_index(const LeafDev &L, int i, int j)
{
    if (L.kind == LK_STRIDED) return (long)i * L.rs + (long)j * L.cs;
    // mat_view_t::operator() (mat_view_t.hpp:28-38) then mat_t::operator() (mat_t.hpp:312-320)
    int a = L.transposed ? j + L.coff : i + L.roff;
    int b = L.transposed ? i + L.roff : j + L.coff;
    a %= L.rows;
    b %= L.cols;
    return L.row_first ? (long)a * L.cols + b : (long)b * L.rows + a;
}

// classify a leaf against the output shape: CONTIG when it is the output-shaped dense
// row-major matrix itself; STRIDED when no modulo wrap can occur (or a dimension of the
// underlying matrix is 1, the broadcast vector case); GENERAL otherwise.
static inline LeafDev classify(const jas_leaf &l, int rows, int cols)
{
    LeafDev d{};
    d.p = l.d_data;
    d.dtype = l.dtype;
    d.rows = l.rows; d.cols = l.cols; d.row_first = l.row_first;
    d.roff = l.roff; d.coff = l.coff; d.transposed = l.transposed;
    bool plain = !l.transposed && l.roff == 0 && l.coff == 0;
    if (plain && l.row_first && l.rows == rows && l.cols == cols) {
        d.kind = LK_CONTIG;
        return d;
    }
    // range of underlying indices (a, b) over i in [0,rows), j in [0,cols)
    long amax = l.transposed ? (long)cols - 1 + l.coff : (long)rows - 1 + l.roff;
    long bmax = l.transposed ? (long)rows - 1 + l.roff : (long)cols - 1 + l.coff;
    bool a_ok = amax < l.rows || l.rows == 1;
    bool b_ok = bmax < l.cols || l.cols == 1;
    if (a_ok && b_ok) {
        // addr = a*sa + b*sb with a = (t ? j : i) + off_a (or 0), b likewise
        long sa = l.row_first ? l.cols : 1, sb = l.row_first ? 1 : l.rows;
        long a_i = 0, a_j = 0, b_i = 0, b_j = 0, a0, b0;
        if (l.transposed) { a_j = 1; b_i = 1; a0 = l.coff; b0 = l.roff; }
        else { a_i = 1; b_j = 1; a0 = l.roff; b0 = l.coff; }
        if (l.rows == 1) { a_i = a_j = 0; a0 = 0; }
        if (l.cols == 1) { b_i = b_j = 0; b0 = 0; }
        d.kind = LK_STRIDED;
        long esz = l.dtype == JAS_F64 ? 8 : l.dtype == JAS_BF16 ? 2 : 4;
        d.p = (const char *)l.d_data + (a0 * sa + b0 * sb) * esz;
        d.rs = a_i * sa + b_i * sb;
        d.cs = a_j * sa + b_j * sb;
        return d;
    }
    d.kind = LK_GENERAL;
    return d;
}

// specialised (hipRTC-compiled) evaluation of a validated program; ew_jit.cpp
bool ew_jit_wanted(long n_elems);
jas_status ew_jit_launch(const jas_ew_ins *prog, int n_ins, const LeafDev *leaves, int n_leaves, bool vec, void *out,
                         int out_dtype, int rows, int cols, hipStream_t s);

} // namespace jas
