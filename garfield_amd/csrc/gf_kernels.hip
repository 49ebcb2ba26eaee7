// HIP kernels of the MI355X Garfield query path (gfx950, wave64).
//
// Layout: every per-point array on the device is stored cell-major -- row r of
// cell c is point global_idx[offset[c] + r_local] -- so a cell-local neighbour
// id l of cell c is row offset[c] + l and no id indirection sits between a
// graph row and the vector gathers.  One wavefront handles one query; its
// candidate list, visited hash and scratch live in LDS and every step is
// wave-synchronous, so the traversal needs no workgroup barriers.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gf_internal.h"

namespace gf {
namespace {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// Timestamps taken by the kernels of a stage themselves, so that a stage needs
// no kernel of its own for them: stamp_entry -- the first workgroup writes
// st[0..n) when it starts; stamp_exit -- the last workgroup of the launch to
// finish writes *st (ticket: a counter at zero, which that workgroup returns
// to zero, so that the next launch or replay starts from zero).  stamp_exit
// costs one device-scope atomic per workgroup, all on one word: only for
// launches of a few hundred workgroups at most.
__device__ __forceinline__ void stamp_entry(uint64_t* st, uint32_t n) {
    if (st && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x < n)
        st[threadIdx.x] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void stamp_exit(uint32_t* ticket, uint64_t* st) {
    if (!st) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        const uint32_t nb = gridDim.x * gridDim.y * gridDim.z;
        if (atomicAdd(ticket, 1u) == nb - 1u) {
            *st = __builtin_amdgcn_s_memrealtime();
            atomicExch(ticket, 0u);
        }
    }
}


__device__ __forceinline__ uint64_t make_cand(float d, uint32_t row, bool pass) {
    return (uint64_t(__float_as_uint(d)) << 32) | (row << 2) | (pass ? 1u : 0u);
}
__device__ __forceinline__ uint64_t ckey(uint64_t c) { return c & ~uint64_t(3); }
__device__ __forceinline__ uint32_t crow(uint64_t c) { return uint32_t(c) >> 2; }
__device__ __forceinline__ bool cvalid(uint64_t c) { return (uint32_t(c) >> 2) != kRowSent; }
__device__ __forceinline__ bool cexpl(uint64_t c) { return (c & 2u) != 0; }
__device__ __forceinline__ bool cpass(uint64_t c) { return (c & 1u) != 0; }
__device__ __forceinline__ float cdist(uint64_t c) { return __uint_as_float(uint32_t(c >> 32)); }

__device__ __forceinline__ uint32_t readlane32(uint32_t v, uint32_t l) {
    return uint32_t(__builtin_amdgcn_readlane(int(v), int(l)));
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, uint32_t l) {
    uint32_t lo = readlane32(uint32_t(v), l), hi = readlane32(uint32_t(v >> 32), l);
    return (uint64_t(hi) << 32) | lo;
}
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0u));
}
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
// v of lane src (any lane, not necessarily active-uniform).
__device__ __forceinline__ uint64_t shfl64(uint64_t v, uint32_t src) {
    const uint32_t lo = uint32_t(__shfl(int(uint32_t(v)), int(src), 64));
    const uint32_t hi = uint32_t(__shfl(int(uint32_t(v >> 32)), int(src), 64));
    return (uint64_t(hi) << 32) | lo;
}

// Lanes of one wave exchange data through LDS between the phases below
// (one-wave workgroups only).  A wave's LDS instructions execute in issue
// order, so the hardware already orders one lane's store before another
// lane's later load; what must not happen is the compiler moving LDS
// accesses across a hand-off (it assumes no communication between lanes
// without synchronisation).  An empty asm with a memory clobber is that
// fence.  A workgroup barrier would do it too, but it also waits for every
// outstanding global load (the workgroup-scope release of the memory
// model), which serialises the gathers with the LDS work around them.
__device__ __forceinline__ void wave_sync() { __asm__ __volatile__("" ::: "memory"); }

// ---------------------------------------------------------------- visited set
// Open addressing with linear probing in LDS over hsize slots (any multiple
// of 64); set semantics identical to the reference's 2048-slot table
// (gpu_graph.cu:677-711) as long as the table does not fill up, which the
// host guarantees by sizing it for a load factor of at most 0.6 of the keys
// that can be live between two resets.  A key's first slot is the high word
// of (key * 2654435761 mod 2^32) * hsize: for hsize = 2^b, the top b bits of
// the multiplicative hash.
__device__ __forceinline__ uint32_t hash_slot(uint32_t key, uint32_t hsize) {
    return __umulhi(key * 2654435761u, hsize);
}
__device__ __forceinline__ uint32_t hash_next(uint32_t h, uint32_t hsize) { return h + 1u == hsize ? 0u : h + 1u; }
__device__ __forceinline__ bool hash_insert(uint32_t* H, uint32_t hsize, uint32_t key) {
    uint32_t h = hash_slot(key, hsize);
    for (uint32_t i = 0; i < hsize; ++i) {
        uint32_t old = atomicCAS(&H[h], kEmpty, key);
        if (old == kEmpty) return true;
        if (old == key) return false;
        h = hash_next(h, hsize);
    }
    return false;
}
__device__ __forceinline__ void hash_clear(uint32_t* H, uint32_t hsize) {
    uint4* h4 = reinterpret_cast<uint4*>(H);
    const uint4 e = make_uint4(kEmpty, kEmpty, kEmpty, kEmpty);
    for (uint32_t i = lane_id(); i < hsize / 4u; i += 64u) h4[i] = e;
    wave_sync();
}

// ----------------------------------------------------------- row distances
// Vector types: VT 0 = fp32, 1 = binary16, 2 = uint8, 3 = int8 quantised
// per dimension (x = s_d (q - z_d)).  A row is read in 16-byte chunks of
// kEpc<VT> elements; queries are fp32 rows for VT 2, rows [c | s] of 2 x
// nch x 16 floats for VT 3 (c_d = fma(s_d, z_d, query_d)), and rows of the
// data's type otherwise.  VT 3's element term is t = fma(-s_d, q, c_d), the
// query minus the dequantised value, squared and summed as the others.
//
// Summation order (the canonical order the oracle restates): LPR "virtual"
// lanes, virtual lane v accumulating chunks v, v + LPR, ... with fp32 fma in
// element order, then an xor butterfly over the LPR partial sums.  The
// virtual lanes are folded onto PL physical lanes per row (RowPlan), each
// holding V = LPR / PL of them: the butterfly levels >= PL run inside a lane,
// the levels < PL across lanes with DPP moves, so a row costs log2(PL)
// cross-lane steps and 64 / PL rows are in flight per pass.  A physical lane
// reads at most 4 chunks of a row (so a pass is a few 16-byte loads per lane)
// and the loads of up to 16 chunks per lane are issued before the first
// wait.
template <int VT>
constexpr int kEpc = VT == 0 ? 4 : ((VT == 1 || VT == 4) ? 8 : 16);

template <int LPR, int CPL>
struct RowPlan {
    static constexpr int want = LPR * CPL / 4;
    static constexpr int PL0 = want <= 8 ? 8 : (want <= 16 ? 16 : (want <= 32 ? 32 : 64));
    static constexpr int PL = PL0 < LPR ? PL0 : LPR;   // physical lanes per row
    static constexpr int V = LPR / PL;                   // virtual lanes per physical lane
    static constexpr int RPP = 64 / PL;                  // rows per pass
    static constexpr int NCH = V * CPL;                  // chunks per lane per row
    static constexpr int NB = 16 / NCH > 0 ? 16 / NCH : 1;   // passes per batch of loads
};

template <int VT, int LPR, int CPL>
struct QReg {
    float v[RowPlan<LPR, CPL>::NCH][kEpc<VT>];
    float w[VT == 3 ? RowPlan<LPR, CPL>::NCH : 1][VT == 3 ? kEpc<VT> : 1];   // VT 3: per-dimension scales
};
// VT 4: binary16 rows with the reference's half arithmetic; the query stays
// in binary16 (its 16-byte chunks as loaded).
template <int LPR, int CPL>
struct QReg<4, LPR, CPL> {
    uint4 h[RowPlan<LPR, CPL>::NCH];
};

// Chunk k = j * CPL + m of physical lane l: virtual lane l + PL * j, its m-th
// chunk l + PL * j + LPR * m.
template <int LPR, int CPL>
__device__ __forceinline__ uint32_t lane_chunk(uint32_t l, int k) {
    using RP = RowPlan<LPR, CPL>;
    return l + uint32_t(RP::PL * (k / CPL) + LPR * (k % CPL));
}

__device__ __forceinline__ uint4 load16(const char* base, uint32_t c) {
    return *reinterpret_cast<const uint4*>(base + size_t(c) * 16u);
}

template <int VT>
__device__ __forceinline__ void decode_chunk(const uint4& u, float (&x)[kEpc<VT>]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    if constexpr (VT == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = __half2float(__ushort_as_half(uint16_t(w[i] & 0xFFFFu)));
            x[2 * i + 1] = __half2float(__ushort_as_half(uint16_t(w[i] >> 16)));
        }
    } else if constexpr (VT == 2) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) x[4 * i + k] = float((w[i] >> (8 * k)) & 0xFFu);
    } else if constexpr (VT == 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) x[4 * i + k] = float(int8_t(uint8_t(w[i] >> (8 * k))));
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(w[i]);
    }
}

template <int VT, int LPR, int CPL>
__device__ __forceinline__ void load_query(QReg<VT, LPR, CPL>& q, const char* qrow, uint32_t nch) {
    using RP = RowPlan<LPR, CPL>;
    const uint32_t l = lane_id() % RP::PL;
    if constexpr (VT == 4) {
#pragma unroll
        for (int k = 0; k < RP::NCH; ++k) {
            const uint32_t c = lane_chunk<LPR, CPL>(l, k);
            q.h[k] = c < nch ? load16(qrow, c) : make_uint4(0u, 0u, 0u, 0u);
        }
    } else {
#pragma unroll
        for (int k = 0; k < RP::NCH; ++k) {
            const uint32_t c = lane_chunk<LPR, CPL>(l, k);
            if (c < nch) {
                if constexpr (VT == 2 || VT == 3) {
                    // fp32 query: one 16-element chunk is four 16-byte loads
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        float x[4];
                        decode_chunk<0>(load16(qrow, 4 * c + t), x);
#pragma unroll
                        for (int e = 0; e < 4; ++e) q.v[k][4 * t + e] = x[e];
                        if constexpr (VT == 3) {
                            decode_chunk<0>(load16(qrow, 4 * (nch + c) + t), x);   // the scales follow the nch chunks
#pragma unroll
                            for (int e = 0; e < 4; ++e) q.w[k][4 * t + e] = x[e];
                        }
                    }
                } else {
                    decode_chunk<VT>(load16(qrow, c), q.v[k]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < kEpc<VT>; ++e) q.v[k][e] = 0.0f;
                if constexpr (VT == 3) {
#pragma unroll
                    for (int e = 0; e < kEpc<VT>; ++e) q.w[k][e] = 0.0f;
                }
            }
        }
    }
}

// v + the value of lane (this lane + m): correct in every lane whose index
// within its aligned group of 2m lanes is below m, which is all the
// reduction below reads.
template <int M>
__device__ __forceinline__ float add_from_above(float v) {
    if constexpr (M == 1) {
        return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    } else if constexpr (M == 4 || M == 8) {
        return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x100 + M, 0xF, 0xF, false));  // row_shl:M
    } else {
        return v + __shfl_down(v, M, 64);
    }
}

// Binary16 arithmetic of the reference's fp16 distance
// (gpu_graph.cu:3394-3403, 3508-3530): lane r of a 32-lane warp takes the
// 4-element chunks r, r + 32, ... of the row and, per chunk, acc =
// hfma2(q.xy - x.xy, q.xy - x.xy, acc) then the same for .zw (so acc.x sums
// elements 4c, 4c + 2 and acc.y elements 4c + 1, 4c + 3, in chunk order),
// every operation rounded once to binary16; then hadd2 steps with shfl_down
// 16, 8, 4, 2, 1 and float(acc.x) + float(acc.y) in fp32 on lane 0.  Here
// (LPR = 16) virtual lane v takes our 16-byte chunks v, v + 16, ...: chunk c
// is the reference's chunks 2c and 2c + 1, so v accumulates reference lanes
// 2v (a0) and 2v + 1 (a1) in their own order.  Steps 16..2 of the tree pair
// reference lanes of the same parity (v ^ 8 .. v ^ 1, a0 and a1 apart: in
// the lane for the virtual lanes a physical lane folds, then across lanes),
// step 1 adds a1 to a0; for the value that ends in lane 0 the xor pairing
// adds the same operands as shfl_down's, and a binary16 sum does not depend
// on operand order.
__device__ __forceinline__ __half2 h2(uint32_t u) { return __builtin_bit_cast(__half2, u); }
__device__ __forceinline__ uint32_t u2(__half2 h) { return __builtin_bit_cast(uint32_t, h); }
template <int M>
__device__ __forceinline__ uint32_t hadd_from_above(uint32_t v) {
    uint32_t o;
    if constexpr (M == 1) o = uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false));
    else if constexpr (M == 2) o = uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false));
    else if constexpr (M == 4 || M == 8) o = uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x100 + M, 0xF, 0xF, false));
    else o = uint32_t(__shfl_down(int(v), M, 64));
    return u2(__hadd2(h2(v), h2(o)));
}
template <int LPR, int CPL>
__device__ __forceinline__ float row_reduce_ref(const QReg<4, LPR, CPL>& q, const uint4 (&raw)[RowPlan<LPR, CPL>::NCH]) {
    using RP = RowPlan<LPR, CPL>;
    static_assert(LPR == 16, "the reference's 32 lanes as 16 virtual lanes of two");
    // virtual lane l + PL j of this physical lane: reference lanes 2 v and 2 v + 1
    __half2 a0[RP::V], a1[RP::V];
#pragma unroll
    for (int j = 0; j < RP::V; ++j) {
        a0[j] = h2(0u);
        a1[j] = h2(0u);
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            const uint4& qc = q.h[j * CPL + m];
            const uint4& xc = raw[j * CPL + m];
            __half2 d = __hsub2(h2(qc.x), h2(xc.x));
            a0[j] = __hfma2(d, d, a0[j]);
            d = __hsub2(h2(qc.y), h2(xc.y));
            a0[j] = __hfma2(d, d, a0[j]);
            d = __hsub2(h2(qc.z), h2(xc.z));
            a1[j] = __hfma2(d, d, a1[j]);
            d = __hsub2(h2(qc.w), h2(xc.w));
            a1[j] = __hfma2(d, d, a1[j]);
        }
    }
    // tree levels on the virtual lane index, highest first: in-lane (the
    // folded virtual lanes), then across lanes
#pragma unroll
    for (int mm = RP::V / 2; mm >= 1; mm >>= 1)
#pragma unroll
        for (int j = 0; j < mm; ++j) {
            a0[j] = __hadd2(a0[j], a0[j + mm]);
            a1[j] = __hadd2(a1[j], a1[j + mm]);
        }
    uint32_t v0 = u2(a0[0]), v1 = u2(a1[0]);
    if constexpr (RP::PL >= 16) { v0 = hadd_from_above<8>(v0); v1 = hadd_from_above<8>(v1); }
    v0 = hadd_from_above<4>(v0); v1 = hadd_from_above<4>(v1);
    v0 = hadd_from_above<2>(v0); v1 = hadd_from_above<2>(v1);
    v0 = hadd_from_above<1>(v0); v1 = hadd_from_above<1>(v1);
    const __half2 r = __hadd2(h2(v0), h2(v1));
    return __half2float(__low2half(r)) + __half2float(__high2half(r));
}

// Distance of one row's chunks raw[0..NCH) (this lane's part) to the query:
// per-virtual-lane fma chains, the in-lane butterfly levels, then the
// cross-lane levels; the row's distance ends in the group's first lane.
template <int VT, int LPR, int CPL>
__device__ __forceinline__ float row_reduce_gen(const QReg<VT, LPR, CPL>& q, const uint4 (&raw)[RowPlan<LPR, CPL>::NCH]) {
    using RP = RowPlan<LPR, CPL>;
    float s[RP::V];
#pragma unroll
    for (int j = 0; j < RP::V; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            float x[kEpc<VT>];
            decode_chunk<VT>(raw[j * CPL + m], x);
#pragma unroll
            for (int e = 0; e < kEpc<VT>; ++e) {
                float d;
                if constexpr (VT == 3) d = __builtin_fmaf(-q.w[j * CPL + m][e], x[e], q.v[j * CPL + m][e]);
                else d = q.v[j * CPL + m][e] - x[e];
                acc = __builtin_fmaf(d, d, acc);
            }
        }
        s[j] = acc;
    }
#pragma unroll
    for (int mm = RP::V / 2; mm >= 1; mm >>= 1) {
        float t[RP::V];
#pragma unroll
        for (int j = 0; j < RP::V; ++j) t[j] = s[j] + s[j ^ mm];
#pragma unroll
        for (int j = 0; j < RP::V; ++j) s[j] = t[j];
    }
    float v = s[0];
    if constexpr (RP::PL >= 64) v = add_from_above<32>(v);
    if constexpr (RP::PL >= 32) v = add_from_above<16>(v);
    if constexpr (RP::PL >= 16) v = add_from_above<8>(v);
    v = add_from_above<4>(v);
    v = add_from_above<2>(v);
    v = add_from_above<1>(v);
    return v;
}

template <int VT, int LPR, int CPL>
__device__ __forceinline__ float row_reduce(const QReg<VT, LPR, CPL>& q, const uint4 (&raw)[RowPlan<LPR, CPL>::NCH]) {
    if constexpr (VT == 4) return row_reduce_ref<LPR, CPL>(q, raw);
    else return row_reduce_gen<VT, LPR, CPL>(q, raw);
}

// Distances of the n rows listed in S[0..n) (LDS).  Lane j with compact
// index ci (< n) receives the distance of row S[ci] in `dist`.
template <int VT, int LPR, int CPL>
__device__ __forceinline__ void eval_rows(const QReg<VT, LPR, CPL>& q, const char* vec, uint32_t rowbytes,
                                          uint32_t nch, const uint32_t* S, uint32_t n, uint32_t ci,
                                          float& dist) {
    using RP = RowPlan<LPR, CPL>;
    const uint32_t g = lane_id() / RP::PL, l = lane_id() % RP::PL;
    const uint32_t npass = (n + RP::RPP - 1) / RP::RPP;
    for (uint32_t k0 = 0; k0 < npass; k0 += RP::NB) {
        uint4 raw[RP::NB][RP::NCH];
#pragma unroll
        for (int b = 0; b < RP::NB; ++b) {
            const uint32_t i = (k0 + b) * RP::RPP + g;
            const char* row = i < n ? vec + size_t(S[i]) * rowbytes : nullptr;
#pragma unroll
            for (int k = 0; k < RP::NCH; ++k) {
                const uint32_t c = lane_chunk<LPR, CPL>(l, k);
                raw[b][k] = make_uint4(0u, 0u, 0u, 0u);
                if (row && c < nch) raw[b][k] = load16(row, c);
            }
        }
#pragma unroll
        for (int b = 0; b < RP::NB; ++b) {
            if (k0 + b >= npass) break;
            const float v = row_reduce<VT, LPR, CPL>(q, raw[b]);
            const float t = __shfl(v, int((ci % RP::RPP) * RP::PL), 64);
            if (ci < n && ci / RP::RPP == k0 + b) dist = t;
        }
    }
}

__device__ __forceinline__ bool row_pass(const float* attrs, uint32_t a, uint32_t row,
                                         const float (&lo)[kMaxAttr], const float (&hi)[kMaxAttr]) {
    bool ok = true;
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        if (d < a) {
            const float v = attrs[size_t(row) * a + d];
            ok = ok && (v >= lo[d]) && (v <= hi[d]);
        }
    }
    return ok;
}

// Evaluate candidate rows held one per lane (lanes with need=false keep dist
// = +inf).  With lo/hi given, lanes with chk also test their row's attributes
// into `pass`, loaded together with the rows (one wait for both).  Returns
// the number of rows gathered.
template <int VT, int LPR, int CPL>
__device__ __forceinline__ uint32_t eval_lanes(const QReg<VT, LPR, CPL>& q, const TravArgs& p, uint32_t* S,
                                               uint32_t row, bool need, float& dist,
                                               const float (*lo)[kMaxAttr] = nullptr,
                                               const float (*hi)[kMaxAttr] = nullptr, bool chk = false,
                                               bool* pass = nullptr) {
    const uint64_t m = ballot(need);
    const uint32_t ci = need ? lanes_below(m) : 0xFFFFFFFFu;
    wave_sync();
    if (need) S[ci] = row;
    wave_sync();
    float av[kMaxAttr];
    if (pass && chk) {
#pragma unroll
        for (uint32_t d = 0; d < kMaxAttr; ++d)
            if (d < p.a) av[d] = p.attrs[size_t(row) * p.a + d];
    }
    const uint32_t n = __popcll(m);
    dist = __int_as_float(0x7F800000);
    if (n) eval_rows<VT, LPR, CPL>(q, p.vec, p.rowbytes, p.nch, S, n, ci, dist);
    if (pass) {
        bool ok = chk;
#pragma unroll
        for (uint32_t d = 0; d < kMaxAttr; ++d)
            if (d < p.a) ok = ok && (av[d] >= (*lo)[d]) && (av[d] <= (*hi)[d]);
        *pass = ok;
    }
    wave_sync();
    return n;
}

// ------------------------------------------------------------ list merges
// Merge the candidates b (lane j < nb holds one) into the sorted list A[0..L):
// A_i moves to i + #{b <= A_i}, b_j to j' + #{A < b_j} with j' its stable rank
// among b (gpu_graph.cu:162-222).  A-origin entries pushed past L go to Bp
// (as themselves if valid and passing, else the sentinel; quirk of
// merge_top_with_recycle_list, gpu_graph.cu:224-315); Bp has nb slots and is
// pre-filled with sentinels.  Returns the first position that received an
// incoming candidate (L if none).  keep_all (merge_top, gpu_graph.cu:162-222,
// whose B region keeps the n largest of both lists): Bp receives every
// evicted A entry as itself and every incoming candidate that did not enter
// A, each at its merged position minus L.
__device__ uint32_t merge_into(uint64_t* A, uint32_t L, uint64_t b, uint32_t nb, uint64_t* Bp,
                               bool keep_all = false) {
    const uint32_t lane = lane_id();
    const bool mine = lane < nb;
    const uint64_t kb = ckey(b);
    uint32_t r = L;
    wave_sync();
    if (mine) {
        if (kb <= ckey(A[L - 1])) {
            uint32_t lo = 0, hi = L - 1;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (ckey(A[mid]) < kb) lo = mid + 1; else hi = mid;
            }
            r = lo;
        }
    }
    if (Bp && mine) Bp[lane] = kCandSent;
    wave_sync();
    if (keep_all && Bp) {
        // a rejected candidate sorts after all of A: merged position L + its
        // stable rank among the incoming candidates
        uint32_t ra = 0;
        for (uint32_t k = 0; k < nb; ++k) {
            const uint64_t kk = ckey(readlane64(b, k));
            ra += (kk < kb) || (kk == kb && k < lane);
        }
        if (mine && r == L) Bp[ra] = b;
    }
    const uint64_t ins = ballot(mine && r < L);
    if (ins == 0) return L;
    uint32_t rb = 0, rmin = L;
    for (uint64_t m = ins; m; m &= m - 1) {
        const uint32_t k = __builtin_ctzll(m);
        const uint64_t kk = readlane64(kb, k);
        const uint32_t rk = readlane32(r, k);
        rb += (kk < kb) || (kk == kb && k < lane);
        rmin = rk < rmin ? rk : rmin;
    }
    // The incoming positions in rank order (non-decreasing: a smaller key
    // never lands after a larger one): lane t < nins holds the t-th.  A_i
    // moves by #{positions <= i}, counted per 64-entry chunk from the
    // positions before it and the few inside it.
    const uint32_t nins = __popcll(ins);
    const bool me_ins = (ins >> lane) & 1u;
    const uint32_t dst = me_ins ? rb : nins + lanes_below(~ins);
    const uint32_t rs = uint32_t(__builtin_amdgcn_ds_permute(int(dst * 4u), int(r)));
    // Blocks of 4 chunks from the end: a block is read, then written; its
    // writes land at or after its own start, which the blocks below never
    // read, so one barrier per block orders it.
    const uint32_t nA = L - rmin;
    const uint32_t nchunk = (nA + 63u) / 64u;
    for (int blk = int((nchunk + 3u) / 4u) - 1; blk >= 0; --blk) {
        uint64_t av[4];
        uint32_t np[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t ch = uint32_t(blk) * 4u + u;
            const uint32_t c0 = rmin + ch * 64u;
            const uint32_t i = c0 + lane;
            av[u] = 0;
            np[u] = kEmpty;
            if (ch < nchunk) {
                uint32_t s = __popcll(ballot(lane < nins && rs < c0));
                for (uint64_t m = ballot(lane < nins && rs >= c0 && rs < c0 + 64u); m; m &= m - 1)
                    s += lane >= readlane32(rs, __builtin_ctzll(m)) - c0;
                if (i < L) {
                    av[u] = A[i];
                    np[u] = i + s;
                }
            }
        }
        wave_sync();
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            if (np[u] == kEmpty) continue;
            if (np[u] < L) A[np[u]] = av[u];
            else if (Bp) Bp[np[u] - L] = (keep_all || (cvalid(av[u]) && cpass(av[u]))) ? av[u] : kCandSent;
        }
    }
    const uint32_t pos = rb + r;
    if (mine && r < L && pos < L) A[pos] = b;
    else if (keep_all && Bp && mine && r < L) Bp[pos - L] = b;
    wave_sync();
    return rmin;
}

// Recycle-list update (gpu_graph.cu:3412-3425, 3536-3546): rc (lane t < rl
// holds entry t, sorted) takes the rl smallest of rc and the valid evictees in
// Bp[0..nb); ties put the evictee first.  bleft receives everything else
// (the reference's B region, re-hashed at the next reset).
__device__ void recycle_update(uint64_t& rc, uint32_t rl, const uint64_t* Bp, uint32_t nb,
                               uint64_t& bleft, uint64_t* T) {
    const uint32_t lane = lane_id();
    wave_sync();
    const uint64_t e = lane < nb ? Bp[lane] : kCandSent;
    const uint64_t ev = ballot(lane < nb && cvalid(e));
    if (ev == 0) { bleft = e; return; }
    wave_sync();
    const uint64_t ke = ckey(e), kr = ckey(rc);
    const bool is_e = (ev >> lane) & 1u;
    const bool is_r = lane < rl;
    uint32_t re = 0, rr = lane;
    for (uint64_t m = ev; m; m &= m - 1) {
        const uint32_t k = __builtin_ctzll(m);
        const uint64_t kk = readlane64(ke, k);
        re += (kk < ke) || (kk == ke && k < lane);
        rr += (kk <= kr);
    }
    for (uint32_t t = 0; t < rl; ++t) re += (readlane64(kr, t) < ke);
    // T[0..rl) new recycle, T[64..) leftovers
    if (is_e) T[re < rl ? re : 64u + re - rl] = e;
    if (is_r) T[rr < rl ? rr : 64u + rr - rl] = rc;
    wave_sync();
    const uint32_t nleft = __popcll(ev);
    rc = lane < rl ? T[lane] : kCandSent;
    bleft = lane < nleft ? T[64u + lane] : kCandSent;
    wave_sync();
}

__device__ __forceinline__ uint32_t first_unexplored(const uint64_t* A, uint32_t L, uint32_t start) {
    for (uint32_t base = start; base < L; base += 64u) {
        const uint32_t i = base + lane_id();
        const bool un = i < L && !cexpl(A[i]);
        const uint64_t m = ballot(un);
        if (m) return base + __builtin_ctzll(m);
    }
    return L;
}

// Cell offsets for the visited-set keys of other cells' rows: with at most
// 16 cells, offset[0..15] in (wave-uniform) registers; with up to kOffLds - 1
// cells, an LDS copy O of offset[0..P]; beyond, none (lrow[] is gathered).
struct CellOffs {
    const uint32_t* O;
    uint32_t P;
    uint32_t o[16];
};

__device__ __forceinline__ void cell_offs_init(CellOffs& co, const TravArgs& p, uint32_t* O) {
    co.O = O;
    co.P = p.P;
#pragma unroll
    for (uint32_t t = 0; t < 16; ++t) co.o[t] = t <= p.P ? p.offset[t] : 0u;
}

// Cell-local key of a candidate row for the visited set: arithmetic inside
// the cell [off, offn); for rows of other cells, row - offset[c] for the
// cell c holding it (rows are cell-major, so this is lrow[row]).
__device__ __forceinline__ uint32_t local_key(const TravArgs& p, const CellOffs& co, uint32_t row, uint32_t off,
                                              uint32_t offn, uint32_t& nlrow) {
    if (row >= off && row < offn) return row - off;
    ++nlrow;
    if (co.P <= 16) {
        // the largest offset <= row (offsets ascend; empty cells repeat one)
        uint32_t base = 0;
#pragma unroll
        for (uint32_t t = 1; t < 16; ++t)
            if (t < co.P && row >= co.o[t]) base = co.o[t];
        return row - base;
    }
    if (!co.O) return p.lrow[row];
    uint32_t lo = 0, hi = co.P;   // O[lo] <= row < O[hi]
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (co.O[mid] <= row) lo = mid; else hi = mid;
    }
    return row - co.O[lo];
}

// Insert the rows of the valid entries of A[0..L), four per lane at a time,
// their first probes issued before any is awaited.
__device__ void hash_add_rows(uint32_t* H, uint32_t hsize, const uint64_t* A, uint32_t L) {
    constexpr uint32_t U = 4;
    for (uint32_t base = 0; base < L; base += 64u * U) {
        uint32_t key[U], h[U], old[U];
        bool todo[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = base + u * 64u + lane_id();
            const uint64_t c = i < L ? A[i] : kCandSent;
            todo[u] = cvalid(c);
            key[u] = crow(c);
            h[u] = hash_slot(key[u], hsize);
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) old[u] = todo[u] ? atomicCAS(&H[h[u]], kEmpty, key[u]) : kEmpty;
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            if (!todo[u] || old[u] == kEmpty || old[u] == key[u]) continue;
            for (uint32_t j = 0; j + 1u < hsize; ++j) {
                h[u] = hash_next(h[u], hsize);
                const uint32_t o2 = atomicCAS(&H[h[u]], kEmpty, key[u]);
                if (o2 == kEmpty || o2 == key[u]) break;
            }
        }
    }
    wave_sync();
}

// Insert the keys of A[0..L), four per lane at a time: their keys are
// computed, then their first probes issued, before any probe's result is
// awaited (a set: the insertion order does not change membership).
__device__ void hash_add_list(const TravArgs& p, const CellOffs& co, uint32_t* H, const uint64_t* A, uint32_t L,
                              uint32_t off, uint32_t offn, uint32_t& nlrow) {
    constexpr uint32_t U = 4;
    const uint32_t hsize = p.hsize;
    for (uint32_t base = 0; base < L; base += 64u * U) {
        uint32_t key[U], h[U], old[U];
        bool todo[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = base + u * 64u + lane_id();
            const uint64_t c = i < L ? A[i] : kCandSent;
            todo[u] = cvalid(c);
            key[u] = todo[u] ? local_key(p, co, crow(c), off, offn, nlrow) : 0u;
            h[u] = hash_slot(key[u], hsize);
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) old[u] = todo[u] ? atomicCAS(&H[h[u]], kEmpty, key[u]) : kEmpty;
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            if (!todo[u] || old[u] == kEmpty || old[u] == key[u]) continue;
            for (uint32_t j = 0; j + 1u < hsize; ++j) {
                h[u] = hash_next(h[u], hsize);
                const uint32_t o2 = atomicCAS(&H[h[u]], kEmpty, key[u]);
                if (o2 == kEmpty || o2 == key[u]) break;
            }
        }
    }
    wave_sync();
}

// In-LDS bitonic sort of 128 candidates (ascending key).
__device__ void sort128(uint64_t* W) {
    const uint32_t lane = lane_id();
    for (uint32_t k = 2; k <= 128; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            const uint32_t idx = 2u * j * (lane / j) + (lane % j);
            const uint32_t par = idx + j;
            const uint64_t x = W[idx], y = W[par];
            const bool asc = (idx & k) == 0;
            wave_sync();
            if ((ckey(x) > ckey(y)) == asc) { W[idx] = y; W[par] = x; }
            wave_sync();
        }
    }
}

// ------------------------------------------------------------- traversal
// One wavefront per query: the reference's fused kernel
// select_path_contain_attr_filter_V2_without_output_with_post_pre_filter
// (gpu_graph.cu:3266-4131), traversal branch.
template <int VT, int LPR, int CPL>
__global__ __launch_bounds__(64) void k_traverse(TravArgs p) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint64_t* A = reinterpret_cast<uint64_t*>(smem);   // Lpad
    uint64_t* W = A + p.Lpad;                           // 128 (slots, evictees, scratch)
    uint32_t* S = reinterpret_cast<uint32_t*>(W + kXSlots);  // 128 row list
    uint32_t* H = S + 128;                              // visited set
    const uint32_t lane = lane_id();
    const uint32_t si = p.srange[0] + blockIdx.x;
    if (si >= p.srange[1]) return;
    const uint32_t q = p.sched[si];
    const uint32_t hsize = p.hsize;
    const uint32_t L = p.L, R = p.R, P = p.P, E = p.E;
    // cell offsets for the visited-set keys of other cells' rows
    uint32_t* O = p.offl ? H + hsize : nullptr;
    if (O)
        for (uint32_t i = lane; i <= P; i += 64u) O[i] = p.offset[i];
    CellOffs co;
    cell_offs_init(co, p, O);

    QReg<VT, LPR, CPL> qv;
    load_query<VT, LPR, CPL>(qv, p.queries + size_t(q) * p.qbytes, p.nch);
    float lo[kMaxAttr], hi[kMaxAttr];
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        lo[d] = d < p.a ? p.lo[size_t(q) * p.a + d] : 0.0f;
        hi[d] = d < p.a ? p.hi[size_t(q) * p.a + d] : 0.0f;
    }
    for (uint32_t i = lane; i < L; i += 64u) A[i] = kCandSent;
    hash_clear(H, hsize);   // ends with a wave_sync
    uint32_t n_expand = 0, n_dist = 0, n_attr = 0, n_cross = 0, n_lrow = 0;
    uint64_t rc = kCandSent, bleft = kCandSent;

    const uint32_t* cl = p.cells + size_t(q) * P;
    const uint32_t cnt = p.counts[q];

    // Entry points of the first cell; their point ids go into the visited set
    // as in the reference (gpu_graph.cu:3347-3351).
    uint64_t b = kCandSent;
    {
        const uint32_t c0 = cl[0];
        const uint32_t off0 = p.offset[c0], sz0 = p.offset[c0 + 1] - off0;
        const bool mine = lane < R;
        uint32_t row = 0;
        bool pass = false;
        if (mine) {
            row = off0 + p.entry[lane] % sz0;
            hash_insert(H, p.hsize, p.gidx[row]);
            pass = row_pass(p.attrs, p.a, row, lo, hi);
        }
        wave_sync();
        float d;
        n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, row, mine, d);
        n_attr += R;
        if (mine) b = make_cand(d, row, pass);
    }

    for (uint32_t pi = 0; pi < cnt; ++pi) {
        const uint32_t cur = cl[pi];
        const uint32_t off = p.offset[cur], offn = p.offset[cur + 1];
        uint32_t scan = merge_into(A, L, b, R, W);
        recycle_update(rc, p.rl, W, R, bleft, W);

        for (uint32_t it = 0; it < kMaxIter; ++it) {
            if ((it + 1) % kHashReset == 0) {          // gpu_graph.cu:3441-3454
                hash_clear(H, hsize);
                hash_add_list(p, co, H, A, L, off, offn, n_lrow);
                if (lane < R && cvalid(bleft))
                    hash_insert(H, p.hsize, local_key(p, co, crow(bleft), off, offn, n_lrow));
                wave_sync();
            }
            const uint32_t sel = first_unexplored(A, L, scan);
            if (sel == L) break;
            const uint64_t sc = A[sel];
            wave_sync();
            if (lane == 0) A[sel] = sc | 2u;
            wave_sync();
            ++n_expand;
            scan = sel + 1;
            const uint32_t srow = crow(sc);
            // Expand: neighbours of the selected row (gpu_graph.cu:3500-3530).
            const bool mine = lane < R;
            uint32_t nrow = 0;
            bool isnew = false, pass = false;
            if (mine) {
                const uint32_t nl = p.graph[size_t(srow) * R + lane];
                nrow = off + nl;
                isnew = hash_insert(H, p.hsize, nl);
            }
            n_attr += R;
            float d;
            // every neighbour's attributes are tested, loaded with the rows
            n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, nrow, isnew, d, &lo, &hi, mine, &pass);
            b = mine ? make_cand(d, nrow, pass) : kCandSent;
            const uint32_t ip = merge_into(A, L, b, R, W);
            recycle_update(rc, p.rl, W, R, bleft, W);
            scan = ip < scan ? ip : scan;
        }
        // End of cell (gpu_graph.cu:3555-3560).
        for (uint32_t i = lane; i < L; i += 64u) A[i] = A[i] | 2u;
        wave_sync();
        hash_clear(H, hsize);
        if (pi + 1 < cnt) {                             // gpu_graph.cu:3564-3642
            const uint32_t nxt = cl[pi + 1];
            const uint32_t offx = p.offset[nxt], offxn = p.offset[nxt + 1], szx = offxn - offx;
            const uint32_t ncand = L < kXStep ? L : kXStep;
            const uint64_t ac = lane < ncand ? A[lane] : kCandSent;
            const bool cv = lane < ncand && cvalid(ac);
            const uint64_t cvm = ballot(cv);
            n_cross += __popcll(cvm);
            uint32_t keys[kMaxE];
#pragma unroll
            for (uint32_t e = 0; e < kMaxE; ++e) {
                keys[e] = kEmpty;
                if (cv && e < E) keys[e] = p.cross[size_t(crow(ac)) * p.xrow + size_t(nxt) * p.xcell + e];
            }
            // Slots filled in order 0..127 (the reference fills them
            // concurrently); slot i follows candidate i % 64 and takes its
            // first cross edge not yet taken, else the first free local id.
            uint32_t tk0 = kEmpty, tk1 = kEmpty;
            for (uint32_t i = 0; i < kXSlots; ++i) {
                const uint32_t c = i & 63u;
                if (!((cvm >> c) & 1u)) continue;
                uint32_t found = kEmpty;
#pragma unroll
                for (uint32_t e = 0; e < kMaxE; ++e) {
                    if (e < E && found == kEmpty) {
                        const uint32_t k = readlane32(keys[e], c);
                        if (ballot(tk0 == k || tk1 == k) == 0) found = k;
                    }
                }
                for (uint32_t rp = 0; found == kEmpty && rp < szx; ++rp)
                    if (ballot(tk0 == rp || tk1 == rp) == 0) found = rp;
                if (found != kEmpty) {
                    if (i < 64u) tk0 = lane == i ? found : tk0;
                    else tk1 = lane == i - 64u ? found : tk1;
                }
            }
            uint64_t w0 = kCandSent, w1 = kCandSent;
            {
                const bool v0 = tk0 != kEmpty, v1 = tk1 != kEmpty;
                const uint32_t r0 = offx + tk0, r1 = offx + tk1;
                const bool p0 = v0 && row_pass(p.attrs, p.a, r0, lo, hi);
                const bool p1 = v1 && row_pass(p.attrs, p.a, r1, lo, hi);
                float d0, d1;
                const uint32_t n0 = eval_lanes<VT, LPR, CPL>(qv, p, S, r0, v0, d0);
                const uint32_t n1 = eval_lanes<VT, LPR, CPL>(qv, p, S, r1, v1, d1);
                n_dist += n0 + n1;
                n_attr += n0 + n1;
                if (v0) w0 = make_cand(d0, r0, p0);
                if (v1) w1 = make_cand(d1, r1, p1);
            }
            wave_sync();
            W[lane] = w0;
            W[64u + lane] = w1;
            wave_sync();
            sort128(W);
            hash_clear(H, hsize);
            b = lane < R ? W[lane] : kCandSent;
            const uint64_t y = W[R + lane];
            for (uint32_t h = 0; h < 2; ++h) {
                const uint64_t c = W[h * 64u + lane];
                if (cvalid(c)) hash_insert(H, p.hsize, crow(c) - offx);
            }
            wave_sync();
            merge_into(A, L, y, 64u, nullptr);
            hash_add_list(p, co, H, A, L, offx, offxn, n_lrow);
        }
    }

    // Post-filter, then merge the recycle list (gpu_graph.cu:4025-4047):
    // failing entries become sentinels, i.e. the passing ones are compacted
    // in order.
    {
        uint32_t wpos = 0;
        for (uint32_t base = 0; base < L; base += 64u) {
            const uint32_t i = base + lane;
            wave_sync();
            const uint64_t c = i < L ? A[i] : kCandSent;
            const bool keep = i < L && cvalid(c) && cpass(c);
            const uint64_t m = ballot(keep);
            wave_sync();
            if (keep) A[wpos + lanes_below(m)] = c;
            wpos += __popcll(m);
        }
        wave_sync();
        for (uint32_t i = wpos + lane; i < L; i += 64u) A[i] = kCandSent;
        wave_sync();
    }
    if (cvalid(readlane64(rc, 0))) merge_into(A, L, rc, p.rl, nullptr);

    // First K distinct ids.  Copies of one row with equal keys are adjacent,
    // but a row can also sit once with its distance and again at +inf (a
    // neighbour met again after the visited set forgot it), so each candidate
    // is checked against the earlier lanes of its chunk and against the rows
    // already output (kept in S, free from here on).
    uint32_t n = 0;
    for (uint32_t base = 0; base < L && n < p.K; base += 64u) {
        const uint32_t i = base + lane;
        const uint64_t c = i < L ? A[i] : kCandSent;
        const uint32_t row = crow(c);
        bool distinct = cvalid(c);
        for (uint32_t l2 = 0; l2 < 64u; ++l2) {
            const uint32_t r2 = readlane32(row, l2);
            if (l2 < lane && r2 == row) distinct = false;
        }
        const uint32_t nout = n < p.K ? n : p.K;
        for (uint32_t t = 0; t < nout; ++t)
            if (S[t] == row) distinct = false;
        const uint64_t m = ballot(distinct);
        const uint32_t idx = n + lanes_below(m);
        wave_sync();
        if (distinct && idx < p.K) {
            p.out_ids[size_t(q) * p.K + idx] = p.gidx[row];
            p.out_dist[size_t(q) * p.K + idx] = cdist(c);
            S[idx] = row;
        }
        wave_sync();
        n += __popcll(m);
        if (!cvalid(readlane64(c, 63))) break;
    }
    for (uint32_t j = n + lane; j < p.K; j += 64u) {
        p.out_ids[size_t(q) * p.K + j] = GF_NO_RESULT;
        p.out_dist[size_t(q) * p.K + j] = __int_as_float(0x7F800000);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) n_lrow += __shfl_xor(n_lrow, m, 64);  // per-lane count
    if (lane == 0) {
        uint32_t* ctr = p.counters + size_t(q) * GF_NCOUNTERS;
        ctr[C_EXPAND] = n_expand;
        ctr[C_DIST] = n_dist;
        ctr[C_ATTR] = n_attr;
        ctr[C_CROSS] = n_cross;
        ctr[C_LROW] = n_lrow;
        ctr[C_SCAN] = 0;
        ctr[C_PASS] = 0;
        ctr[C_ROUTE] = 1;
    }
}

// ------------------------------------------------------ dual-channel search
__device__ __forceinline__ bool hash_contains(const uint32_t* H, uint32_t hsize, uint32_t key) {
    uint32_t h = hash_slot(key, hsize);
    for (uint32_t i = 0; i < hsize; ++i) {
        const uint32_t v = H[h];
        if (v == key) return true;
        if (v == kEmpty) return false;
        h = hash_next(h, hsize);
    }
    return false;
}

// Index of the first entry of A[start..L) that is unexplored and whose row
// lies in [rlo, rhi) (L if none).  The sentinel carries the explored bit.
__device__ __forceinline__ uint32_t first_unexplored_in(const uint64_t* A, uint32_t L, uint32_t start,
                                                        uint32_t rlo, uint32_t rhi) {
    for (uint32_t base = start; base < L; base += 64u) {
        const uint32_t i = base + lane_id();
        bool un = false;
        if (i < L) {
            const uint64_t c = A[i];
            const uint32_t r = crow(c);
            un = !cexpl(c) && r >= rlo && r < rhi;
        }
        const uint64_t m = ballot(un);
        if (m) return base + __builtin_ctzll(m);
    }
    return L;
}

// One wavefront per query: the traversal of the reference's
// select_path_contain_attr_filter_V2_without_output_dual_channel_in_turn_with_prefilter
// (gpu_graph.cu:6249-6640).  Two channels walk two cells of the query's list
// over one candidate list: per epoch the channel `turn` expands its first
// unexplored entry (its R neighbours) and the other channel a partner, the
// first of that entry's cross edges into the other channel's cell whose
// local id, read as a point id, is not in the visited set (R - 1 neighbours
// plus the partner itself); a channel with nothing left takes the next cell
// of the list through 128 cross-edge slots, or, with none left, joins the
// other channel.
//
// The reference marks entries with two explored bits, one per channel, and
// gives a channel's own points the other channel's bit.  Here an entry has
// one explored bit: a channel inserts only rows of its current cell and
// leaves a cell only when none of its entries there is unexplored, so an
// unexplored entry belongs to the channel whose current cell holds its row
// (after a join, to the one channel left).  The visited set holds rows; the
// partner test looks up the row of the point id (prow).  The 2R expansion
// slots and the 128 switch slots are sorted before they are merged, so only
// the set of rows new to the visited set matters, not which slot took one.
template <int VT, int LPR, int CPL>
__global__ __launch_bounds__(64) void k_traverse_dual(TravArgs p) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint64_t* A = reinterpret_cast<uint64_t*>(smem);   // Lpad
    uint64_t* W = A + p.Lpad;                           // 128: switch slots, merge scratch
    uint64_t* X = W + kXSlots;                          // 128: switch evictees
    uint32_t* S = reinterpret_cast<uint32_t*>(X + kXSlots);  // 128 row list
    uint32_t* H = S + 128;                              // visited set (rows)
    const uint32_t lane = lane_id();
    const uint32_t si = p.srange[0] + blockIdx.x;
    if (si >= p.srange[1]) return;
    const uint32_t q = p.sched[si];
    const uint32_t hsize = p.hsize;
    const uint32_t L = p.L, R = p.R, P = p.P, E = p.E, R2 = 2u * p.R;

    QReg<VT, LPR, CPL> qv;
    load_query<VT, LPR, CPL>(qv, p.queries + size_t(q) * p.qbytes, p.nch);
    float lo[kMaxAttr], hi[kMaxAttr];
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        lo[d] = d < p.a ? p.lo[size_t(q) * p.a + d] : 0.0f;
        hi[d] = d < p.a ? p.hi[size_t(q) * p.a + d] : 0.0f;
    }
    for (uint32_t i = lane; i < L; i += 64u) A[i] = kCandSent;
    hash_clear(H, hsize);   // ends with a wave_sync
    uint32_t n_expand = 0, n_dist = 0, n_cross = 0;
    uint64_t rc = kCandSent, bleft = kCandSent;

    const uint32_t* cl = p.cells + size_t(q) * P;
    const uint32_t cnt = p.counts[q];
    // the two channels' cells as row ranges [off, end)
    uint32_t c0 = cl[0], c1 = cnt >= 2 ? cl[1] : cl[0];
    uint32_t off0 = p.offset[c0], end0 = p.offset[c0 + 1];
    uint32_t off1 = p.offset[c1], end1 = p.offset[c1 + 1];
    bool same = c0 == c1;

    // Entries (gpu_graph.cu:6318-6362): entry i < ceil(L / 2) in channel 0's
    // cell, the rest in channel 1's, reduced modulo the cell size; all L
    // evaluated, then sorted.
    {
        const uint32_t L2 = (L + 1u) / 2u;
        for (uint32_t base = 0; base < L; base += 64u) {
            const uint32_t i = base + lane;
            const bool mine = i < L;
            uint32_t row = 0;
            bool pass = false;
            if (mine) {
                const bool ch1 = i >= L2;
                const uint32_t o = ch1 ? off1 : off0, sz = (ch1 ? end1 : end0) - o;
                row = o + p.entry[i] % sz;
                hash_insert(H, p.hsize, row);
                pass = row_pass(p.attrs, p.a, row, lo, hi);
            }
            wave_sync();
            float d;
            n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, row, mine, d);
            const uint64_t b = mine ? make_cand(d, row, pass) : kCandSent;
            const uint32_t nb = L - base < 64u ? L - base : 64u;
            merge_into(A, L, b, nb, nullptr);
        }
    }

    // scan0 / scan1: no entry of channel 0 / 1 before it is unexplored (an
    // insertion at position i moves entries at i and after to the right)
    uint32_t cur = cnt >= 2 ? 2u : 1u, turn = 0, scan0 = 0, scan1 = 0;
    for (uint32_t ep = 0; ep < kMaxIter; ++ep) {
        if ((ep + 1) % kHashReset == 0) {              // gpu_graph.cu:6364-6378
            hash_clear(H, hsize);
            hash_add_rows(H, p.hsize, A, L);
            if (cvalid(bleft)) hash_insert(H, p.hsize, crow(bleft));
            wave_sync();
        }
        // Selection and partner (gpu_graph.cu:6380-6420).
        const uint32_t tlo = same ? 0u : (turn ? off1 : off0);
        const uint32_t thi = same ? 0xFFFFFFFFu : (turn ? end1 : end0);
        const uint32_t sel = first_unexplored_in(A, L, turn ? scan1 : scan0, tlo, thi);
        uint32_t te_row = kEmpty, pt_row = kEmpty;
        if (sel < L) {
            const uint64_t sc = A[sel];
            wave_sync();
            if (lane == 0) A[sel] = sc | 2u;
            wave_sync();
            if (same) scan0 = scan1 = sel + 1;
            else if (turn) scan1 = sel + 1;
            else scan0 = sel + 1;
            te_row = crow(sc);
            const uint32_t oc = turn ? c0 : c1, ooff = turn ? off0 : off1;
            const uint32_t ne = E < 2u ? E : 2u;
            uint32_t v = 0;
            bool free = false;
            if (lane < ne) {
                v = p.cross[size_t(te_row) * p.xrow + size_t(oc) * p.xcell + lane];
                free = !hash_contains(H, p.hsize, p.prow[v]);
            }
            const uint64_t m = ballot(free);
            if (m) pt_row = ooff + readlane32(v, __builtin_ctzll(m));
        }
        if (sel == L) {                                 // gpu_graph.cu:6422-6547
            if (cur == cnt && same) break;
            if (cur == cnt) {                           // join the other channel's cell
                if (turn) { c1 = c0; off1 = off0; end1 = end0; }
                else { c0 = c1; off0 = off1; end0 = end1; }
                same = true;
                scan0 = scan1 = scan0 < scan1 ? scan0 : scan1;
                continue;
            }
            // Move channel `turn` to the next cell: slot h * 64 + j follows
            // entry j through its cross edge h.
            const uint32_t nxt = cl[cur];
            const uint32_t offx = p.offset[nxt];
            uint64_t w[2];
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const uint64_t c = lane < L ? A[lane] : kCandSent;
                const bool v = lane < L && cvalid(c) && h < E;
                uint32_t row = 0;
                if (v) row = offx + p.cross[size_t(crow(c)) * p.xrow + size_t(nxt) * p.xcell + h];
                const bool isnew = v && hash_insert(H, p.hsize, row);
                wave_sync();
                n_cross += __popcll(ballot(isnew));
                float d;
                bool pass = false;
                n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, row, isnew, d, &lo, &hi, isnew, &pass);
                w[h] = isnew ? make_cand(d, row, pass) : kCandSent;
            }
            wave_sync();
            W[lane] = w[0];
            W[64u + lane] = w[1];
            wave_sync();
            sort128(W);
            // merge_top_with_recycle_list of the 128 slots: the k slots that
            // enter push out A's last k entries (slot rows are new to the
            // visited set, which holds every row of A, so no slot equals an
            // entry); those that pass the filter go to the recycle list.
            uint32_t k = 0;
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const uint64_t x = W[h * 64u + lane];
                bool enter = false;
                if (cvalid(x)) {
                    const uint64_t kx = ckey(x);
                    uint32_t a0 = 0, a1 = L;                 // first entry of A not below x
                    while (a0 < a1) {
                        const uint32_t mid = (a0 + a1) >> 1;
                        if (ckey(A[mid]) < kx) a0 = mid + 1; else a1 = mid;
                    }
                    enter = h * 64u + lane + a0 < L;
                }
                k += __popcll(ballot(enter));
            }
            uint32_t nkeep = 0;
            for (uint32_t base = 0; base < k; base += 64u) {
                const uint32_t t = base + lane;
                const uint64_t e = t < k ? A[L - k + t] : kCandSent;
                const bool keep = t < k && cvalid(e) && cpass(e);
                const uint64_t m = ballot(keep);
                const uint32_t pos = nkeep + lanes_below(m);
                wave_sync();
                if (keep && pos < 64u) X[pos] = e;
                nkeep += __popcll(m);
            }
            wave_sync();
            const uint32_t ip0 = merge_into(A, L, W[lane], 64u, nullptr);
            const uint32_t ip1 = merge_into(A, L, W[64u + lane], 64u, nullptr);
            const uint32_t ip = ip0 < ip1 ? ip0 : ip1;
            scan0 = ip < scan0 ? ip : scan0;
            scan1 = ip < scan1 ? ip : scan1;
            if (nkeep) {
                uint64_t dummy;
                recycle_update(rc, p.rl, X, nkeep < 64u ? nkeep : 64u, dummy, X);
            }
            if (turn) { c1 = nxt; off1 = offx; end1 = p.offset[nxt + 1]; }
            else { c0 = nxt; off0 = offx; end0 = p.offset[nxt + 1]; }
            ++cur;
            continue;
        }
        // Expansion (gpu_graph.cu:6549-6616): slot j < R of channel 0, R + j
        // of channel 1; the partner channel's last slot holds the partner.
        uint32_t row = 0;
        bool v = false;
        if (lane < R2) {
            const uint32_t ch = lane < R ? 0u : 1u, j = lane - ch * R;
            const uint32_t erow = ch == turn ? te_row : pt_row;
            if (erow != kEmpty) {
                v = true;
                if (ch != turn && j == R - 1u) row = erow;
                else row = (ch ? off1 : off0) + p.graph[size_t(erow) * R + j];
            }
        }
        const bool isnew = v && hash_insert(H, p.hsize, row);
        n_expand += (te_row != kEmpty) + (pt_row != kEmpty);
        float d;
        bool pass = false;
        n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, row, isnew, d, &lo, &hi, isnew, &pass);
        const uint64_t b = isnew ? make_cand(d, row, pass) : kCandSent;
        turn ^= 1u;
        const uint32_t ip = merge_into(A, L, b, R2, W);
        recycle_update(rc, p.rl, W, R2, bleft, W);
        scan0 = ip < scan0 ? ip : scan0;
        scan1 = ip < scan1 ? ip : scan1;
    }

    // Post-filter, then merge the recycle list (gpu_graph.cu:6618-6639).
    {
        uint32_t wpos = 0;
        for (uint32_t base = 0; base < L; base += 64u) {
            const uint32_t i = base + lane;
            wave_sync();
            const uint64_t c = i < L ? A[i] : kCandSent;
            const bool keep = i < L && cvalid(c) && cpass(c);
            const uint64_t m = ballot(keep);
            wave_sync();
            if (keep) A[wpos + lanes_below(m)] = c;
            wpos += __popcll(m);
        }
        wave_sync();
        for (uint32_t i = wpos + lane; i < L; i += 64u) A[i] = kCandSent;
        wave_sync();
    }
    if (cvalid(readlane64(rc, 0))) merge_into(A, L, rc, p.rl, nullptr);

    // First K distinct ids (copies of one entry point are equal and adjacent).
    uint32_t n = 0;
    for (uint32_t base = 0; base < L && n < p.K; base += 64u) {
        const uint32_t i = base + lane;
        const uint64_t c = i < L ? A[i] : kCandSent;
        const uint32_t row = crow(c);
        bool distinct = cvalid(c);
        for (uint32_t l2 = 0; l2 < 64u; ++l2) {
            const uint32_t r2 = readlane32(row, l2);
            if (l2 < lane && r2 == row) distinct = false;
        }
        const uint32_t nout = n < p.K ? n : p.K;
        for (uint32_t t = 0; t < nout; ++t)
            if (S[t] == row) distinct = false;
        const uint64_t m = ballot(distinct);
        const uint32_t idx = n + lanes_below(m);
        wave_sync();
        if (distinct && idx < p.K) {
            p.out_ids[size_t(q) * p.K + idx] = p.gidx[row];
            p.out_dist[size_t(q) * p.K + idx] = cdist(c);
            S[idx] = row;
        }
        wave_sync();
        n += __popcll(m);
        if (!cvalid(readlane64(c, 63))) break;
    }
    for (uint32_t j = n + lane; j < p.K; j += 64u) {
        p.out_ids[size_t(q) * p.K + j] = GF_NO_RESULT;
        p.out_dist[size_t(q) * p.K + j] = __int_as_float(0x7F800000);
    }
    if (lane == 0) {
        uint32_t* ctr = p.counters + size_t(q) * GF_NCOUNTERS;
        ctr[C_EXPAND] = n_expand;
        ctr[C_DIST] = n_dist;
        ctr[C_ATTR] = n_dist;
        ctr[C_CROSS] = n_cross;
        ctr[C_LROW] = 0;
        ctr[C_SCAN] = 0;
        ctr[C_PASS] = 0;
        ctr[C_ROUTE] = 4;
    }
}

// prow[gidx[r]] = r: the row of each point id.
__global__ void k_invert_rows(const uint32_t* gidx, uint32_t N, uint32_t* prow) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < N) prow[gidx[r]] = r;
}

// -------------------------------------------------------------- full graph
// The full-graph post-filter branch (gpu_graph.cu:3644-3787; the reference
// disables it with `&& false` and sends these queries to a brute force over
// no cell): a graph search over every point's full-graph row (its own cell's
// first edges and its cross edges into every other cell, assembled as
// full_graph_search.cuh:984-997 does), from the FD entry points of the
// reference's second draw (gpu_graph.cu:12527-12539), with the visited set
// keyed by point (row), neighbours already in it dropped, and the plain
// merge_top whose B region (the FD largest of both lists) is re-hashed at
// every reset; no recycle list.  Then the common post-filter (gpu_graph.cu:
// 4025-4047): passing entries in order, first K distinct.
template <int VT, int LPR, int CPL>
__global__ __launch_bounds__(64) void k_fullgraph(TravArgs p) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint64_t* A = reinterpret_cast<uint64_t*>(smem);   // Lpad
    uint64_t* W = A + p.Lpad;                           // the B region (FD <= 64)
    uint32_t* S = reinterpret_cast<uint32_t*>(W + kXSlots);  // 128 row list
    uint32_t* H = S + 128;                              // visited set
    const uint32_t lane = lane_id();
    const uint32_t si = p.frange[0] + blockIdx.x;
    if (si >= p.frange[1]) return;
    const uint32_t q = p.sched[si];
    const uint32_t hsize = p.hsize;
    const uint32_t L = p.L, FD = p.FD;

    QReg<VT, LPR, CPL> qv;
    load_query<VT, LPR, CPL>(qv, p.queries + size_t(q) * p.qbytes, p.nch);
    float lo[kMaxAttr], hi[kMaxAttr];
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        lo[d] = d < p.a ? p.lo[size_t(q) * p.a + d] : 0.0f;
        hi[d] = d < p.a ? p.hi[size_t(q) * p.a + d] : 0.0f;
    }
    for (uint32_t i = lane; i < L; i += 64u) A[i] = kCandSent;
    hash_clear(H, hsize);
    uint32_t n_expand = 0, n_dist = 0, n_attr = 0;
    {
        const bool mine = lane < FD;
        const uint32_t row = mine ? p.fentry[lane] : 0u;
        bool pass = false;
        if (mine) {
            hash_insert(H, p.hsize, row);
            pass = row_pass(p.attrs, p.a, row, lo, hi);
        }
        wave_sync();
        float d;
        n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, row, mine, d);
        n_attr += FD;
        merge_into(A, L, mine ? make_cand(d, row, pass) : kCandSent, FD, W, true);
    }
    uint32_t scan = 0;
    for (uint32_t it = 0; it < kMaxIter; ++it) {
        if ((it + 1) % kHashReset == 0) {           // gpu_graph.cu:3690-3702
            hash_clear(H, hsize);
            for (uint32_t i = lane; i < L + FD; i += 64u) {
                const uint64_t c = i < L ? A[i] : W[i - L];
                if (cvalid(c)) hash_insert(H, p.hsize, crow(c));
            }
            wave_sync();
        }
        const uint32_t sel = first_unexplored(A, L, scan);
        if (sel == L) break;
        const uint64_t sc = A[sel];
        wave_sync();
        if (lane == 0) A[sel] = sc | 2u;
        wave_sync();
        ++n_expand;
        scan = sel + 1;
        const bool mine = lane < FD;
        uint32_t nrow = kEmpty;
        bool isnew = false, pass = false;
        if (mine) {
            nrow = p.fgraph[size_t(crow(sc)) * FD + lane];
            isnew = nrow != kEmpty && hash_insert(H, p.hsize, nrow);
        }
        n_attr += __popcll(ballot(isnew));
        float d;
        n_dist += eval_lanes<VT, LPR, CPL>(qv, p, S, nrow, isnew, d, &lo, &hi, isnew, &pass);
        const uint32_t ip = merge_into(A, L, isnew ? make_cand(d, nrow, pass) : kCandSent, FD, W, true);
        scan = ip < scan ? ip : scan;
    }
    // Post-filter (gpu_graph.cu:4025-4041): the passing entries, in order.
    uint32_t wpos = 0;
    for (uint32_t base = 0; base < L; base += 64u) {
        const uint32_t i = base + lane;
        wave_sync();
        const uint64_t c = i < L ? A[i] : kCandSent;
        const bool keep = i < L && cvalid(c) && cpass(c);
        const uint64_t m = ballot(keep);
        wave_sync();
        if (keep) A[wpos + lanes_below(m)] = c;
        wpos += __popcll(m);
    }
    wave_sync();
    const uint32_t n = wpos < p.K ? wpos : p.K;     // rows of A are distinct
    for (uint32_t j = lane; j < p.K; j += 64u) {
        const uint64_t c = j < n ? A[j] : kCandSent;
        p.out_ids[size_t(q) * p.K + j] = j < n ? p.gidx[crow(c)] : GF_NO_RESULT;
        p.out_dist[size_t(q) * p.K + j] = j < n ? cdist(c) : __int_as_float(0x7F800000);
    }
    if (lane == 0) {
        uint32_t* ctr = p.counters + size_t(q) * GF_NCOUNTERS;
        ctr[C_EXPAND] = n_expand;
        ctr[C_DIST] = n_dist;
        ctr[C_ATTR] = n_attr;
        ctr[C_CROSS] = 0;
        ctr[C_LROW] = 0;
        ctr[C_SCAN] = 0;
        ctr[C_PASS] = 0;
        ctr[C_ROUTE] = 3;
    }
}

__global__ void k_assemble_full(const uint32_t* graph, const uint32_t* cross, const uint32_t* offset,
                                const uint32_t* rowcell, uint32_t N, uint32_t P, uint32_t R, uint32_t E, uint32_t FE,
                                uint32_t* out) {
    const uint32_t FD = FE * P;
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(N) * FD) return;
    const uint32_t r = uint32_t(i / FD), slot = uint32_t(i % FD), c = slot / FE, e = slot % FE;
    const uint32_t own = rowcell[r], sz = offset[c + 1] - offset[c];
    uint32_t v = kEmpty;
    // local ids reduced modulo the cell size, the in-bounds rule of the
    // traversal's cross-edge reads
    if (sz) v = offset[c] + (c == own ? graph[size_t(r) * R + e] : cross[(size_t(r) * P + c) * E + e]) % sz;
    out[i] = v;
}

// ----------------------------------------------------------- brute force
// Filtered brute force over the query's cells (gpu_graph.cu:3788-4022): an
// attribute scan of each cell's contiguous rows, compaction of the passing
// rows, distance evaluation and a wave-held top-K keyed by (distance, row).
// Exact distances of the rows S[0..nrows) to the query, merged into the
// top-K (lane t < K: t-th best by (distance, row)).
template <int VT, int LPR, int CPL>
__device__ void bf_flush(const QReg<VT, LPR, CPL>& qv, const TravArgs& p, const uint32_t* S, uint32_t nrows,
                         uint64_t& top, uint64_t* T) {
    const uint32_t lane = lane_id(), K = p.K;
    {
        for (uint32_t base = 0; base < nrows; base += 64u) {
            const uint32_t nb = nrows - base < 64u ? nrows - base : 64u;
            const bool mine = lane < nb;
            float d = 0.0f;
            eval_rows<VT, LPR, CPL>(qv, p.vec, p.rowbytes, p.nch, S + base, nb,
                                     mine ? lane : 0xFFFFFFFFu, d);
            const uint64_t c = mine ? make_cand(d, S[base + lane], true) : kCandSent;
            const uint64_t thr = ckey(readlane64(top, K - 1));
            const bool surv = mine && ckey(c) < thr;
            const uint64_t sm = ballot(surv);
            if (sm == 0) continue;
            const uint64_t kc = ckey(c), kt = ckey(top);
            uint32_t rs = 0, rt = lane;
            // ranks in the merged order, ties to the top entry, then to the
            // lower lane: a permutation even if a key repeats
            for (uint64_t m = sm; m; m &= m - 1) {
                const uint32_t j = __builtin_ctzll(m);
                const uint64_t kk = readlane64(kc, j);
                rs += kk < kc || (kk == kc && j < lane);
                rt += kk < kt;
            }
            for (uint32_t t = 0; t < K; ++t) rs += readlane64(kt, t) <= kc;
            wave_sync();
            if (surv && rs < K) T[rs] = c;
            if (lane < K && rt < K) T[rt] = top;
            wave_sync();
            top = lane < K ? T[lane] : kCandSent;
        }
    }
}

// Filtered brute force of query q over the first little[q] cells of its
// list: the passing rows are gathered 64 at a time and ranked exactly.
// Results and counters are written for q.
template <int VT, int LPR, int CPL>
__device__ void bf_scan_query(const TravArgs& p, uint32_t q, uint32_t* S, uint64_t* T) {
    constexpr uint32_t U = 4;                 // 64-row chunks scanned per step (S holds 64 U + 64)
    const uint32_t lane = lane_id();
    const uint32_t K = p.K, P = p.P;
    QReg<VT, LPR, CPL> qv;
    load_query<VT, LPR, CPL>(qv, p.queries + size_t(q) * p.qbytes, p.nch);
    float lo[kMaxAttr], hi[kMaxAttr];
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        lo[d] = d < p.a ? p.lo[size_t(q) * p.a + d] : 0.0f;
        hi[d] = d < p.a ? p.hi[size_t(q) * p.a + d] : 0.0f;
    }
    uint64_t top = kCandSent;                 // lane t < K: t-th best
    uint32_t n_scan = 0, n_pass = 0;
    const uint32_t* cl = p.cells + size_t(q) * P;
    const uint32_t lit = p.little[q];
    uint32_t ns = 0;
    auto flush = [&](uint32_t nrows) { bf_flush<VT, LPR, CPL>(qv, p, S, nrows, top, T); };

    for (uint32_t g = 0; g < lit; ++g) {
        const uint32_t cc = cl[g];
        const uint32_t off = p.offset[cc], end = p.offset[cc + 1];
        n_scan += end - off;
        for (uint32_t base = off; base < end; base += 64u * U) {
            bool ps[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t row = base + u * 64u + lane;
                ps[u] = row < end && row_pass(p.attrs, p.a, row, lo, hi);
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint64_t m = ballot(ps[u]);
                if (ps[u]) S[ns + lanes_below(m)] = base + u * 64u + lane;
                ns += __popcll(m);
            }
            wave_sync();
            if (ns >= 64u) {
                const uint32_t full = ns & ~63u;
                flush(full);
                const uint32_t rest = ns - full;
                const uint32_t tail = lane < rest ? S[full + lane] : 0u;
                wave_sync();
                if (lane < rest) S[lane] = tail;
                wave_sync();
                n_pass += full;
                ns = rest;
            }
        }
    }
    if (ns) { flush(ns); n_pass += ns; }
    if (lane < K) {
        p.out_ids[size_t(q) * K + lane] = cvalid(top) ? p.gidx[crow(top)] : GF_NO_RESULT;
        p.out_dist[size_t(q) * K + lane] = cdist(top);
    }
    if (lane == 0) {
        uint32_t* ctr = p.counters + size_t(q) * GF_NCOUNTERS;
        ctr[C_EXPAND] = 0;
        ctr[C_DIST] = n_pass;
        ctr[C_ATTR] = 0;
        ctr[C_CROSS] = 0;
        ctr[C_LROW] = 0;
        ctr[C_SCAN] = n_scan;
        ctr[C_PASS] = n_pass;
        ctr[C_ROUTE] = lit ? 2u : 0u;
    }
}

template <int VT, int LPR, int CPL>
__global__ __launch_bounds__(64) void k_bruteforce(TravArgs p) {
    __shared__ uint32_t S[64 * 4 + 64];
    __shared__ uint64_t T[64];
    const uint32_t si = p.srange[0] + blockIdx.x;
    if (si >= p.srange[1]) return;
    bf_scan_query<VT, LPR, CPL>(p, p.sched[si], S, T);
}

__global__ void k_fill_results(uint32_t* ids, float* dist, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { ids[i] = GF_NO_RESULT; dist[i] = __int_as_float(0x7F800000); }
}

// ---------------------------------------------------------------- prep
// f2h (tools.cuh:308-320): binary16 round-to-nearest-even of the fp32
// product x*alpha.  The empty asm pins the fp32 product in a register so the
// compiler cannot fold multiply and conversion into one mixed-precision fma,
// which would round once (not twice, as the reference does) and turn
// -0 * a + 0 into +0.
__device__ __forceinline__ uint16_t f2h_scaled(float x, float alpha) {
    float v = x * alpha;
    asm volatile("" : "+v"(v));
    return __half_as_ushort(__float2half_rn(v));
}

__global__ void k_f2h(const float* x, uint16_t* out, size_t n, float alpha) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        out[i] = f2h_scaled(x[i], alpha);
}

__global__ void k_f2h_pad(const float* x, uint32_t rows, uint32_t D, uint16_t* out, uint32_t rows_pad,
                          uint32_t Dp, float alpha) {
    const size_t n = size_t(rows_pad) * Dp;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const uint32_t r = uint32_t(i / Dp), c = uint32_t(i % Dp);
        out[i] = (r < rows && c < D) ? f2h_scaled(x[size_t(r) * D + c], alpha) : uint16_t(0);
    }
}

// find_norm (tools.cuh:1561-1586): one wave per row, lane-strided fp32 fma
// partial sums, xor butterfly.
__global__ __launch_bounds__(64) void k_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, uint32_t ld,
                                                  float* out) {
    const uint32_t r = blockIdx.x, lane = lane_id();
    if (r >= n) return;
    float acc = 0.0f;
    for (uint32_t j = lane; j < D; j += 64u) {
        const float v = __half2float(__ushort_as_half(x[size_t(r) * ld + j]));
        acc = __builtin_fmaf(v, v, acc);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if (lane == 0) out[r] = acc;
}

// Cells each range intersects (real_dataset_adapter.cuh:126-216), ascending
// cell id.  Per attribute: lo cell = first c with r_q[c] >= lo, hi cell =
// (first c with l_q[c] > hi) - 1; the product is enumerated with the last
// attribute fastest (gpu_graph.cu:10965-10973).  A range beyond every cell
// (the reference computes cell -1 or g there) selects nothing; an empty interval between two cells selects
// the next cell, as the reference's do-while does.  Cells holding no point
// are never selected (the reference would read past them).
__device__ __forceinline__ uint32_t cells_of_query(uint32_t q, uint32_t a, const float* lo, const float* hi,
                                                   const uint32_t* grid, const uint32_t* doff, const float* l_q,
                                                   const float* r_q, uint32_t P, const uint32_t* offset,
                                                   uint32_t* cells) {
    uint32_t cl[kMaxAttr], ch[kMaxAttr], idx[kMaxAttr], g[kMaxAttr];
    bool empty = false;
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        if (d >= a) break;
        g[d] = grid[d];
        const float* rq = r_q + doff[d];
        const float* lq = l_q + doff[d];
        const float vl = lo[size_t(q) * a + d], vh = hi[size_t(q) * a + d];
        uint32_t i = 0;
        while (i < g[d] && rq[i] < vl) ++i;
        uint32_t j = 0;
        while (j < g[d] && lq[j] <= vh) ++j;
        if (i >= g[d] || j == 0) empty = true;
        cl[d] = i;
        ch[d] = (j == 0) ? i : ((j - 1) > i ? (j - 1) : i);
        idx[d] = i;
    }
    uint32_t n = 0;
    if (!empty) {
        while (true) {
            uint32_t pid = 0, f = 1;
            for (int d = int(a) - 1; d >= 0; --d) { pid += idx[d] * f; f *= g[d]; }
            if (offset[pid + 1] > offset[pid]) cells[size_t(q) * P + n++] = pid;
            int d = int(a) - 1;
            for (; d >= 0; --d) {
                if (++idx[d] <= ch[d]) break;
                idx[d] = cl[d];
            }
            if (d < 0) break;
        }
    }
    return n;
}
__global__ void k_cells(uint32_t Q, uint32_t a, const float* lo, const float* hi, const uint32_t* grid,
                        const uint32_t* doff, const float* l_q, const float* r_q, uint32_t P,
                        const uint32_t* offset, uint32_t* cells, uint32_t* counts, CellsTail tl) {
    stamp_entry(tl.st_entry, 1);
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q < Q) {
        const uint32_t n = cells_of_query(q, a, lo, hi, grid, doff, l_q, r_q, P, offset, cells);
        counts[q] = n;
        if (tl.little) {
            tl.selcount[q] = 0;
            tl.little[q] = n;
        }
    }
    stamp_exit(tl.ticket, tl.st_exit);
}

__global__ void k_cellq_count(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                              uint32_t* ccount) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    for (uint32_t i = 0; i < counts[q]; ++i) atomicAdd(&ccount[cells[size_t(q) * P + i]], 1u);
}

__global__ void k_cellq_fill(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                             const uint32_t* cstart, uint32_t* cfill, uint32_t* cellq) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    for (uint32_t i = 0; i < counts[q]; ++i) {
        const uint32_t c = cells[size_t(q) * P + i];
        cellq[cstart[c] + atomicAdd(&cfill[c], 1u)] = q;
    }
}

// Exclusive scan of a short array by one workgroup.  Up to kScanLds
// elements: staged in LDS with coalesced loads, each thread scans a
// contiguous run of them, one block-wide scan of the run totals (wave
// shuffles, then the 16 wave sums), coalesced stores.  Longer arrays: chunks
// of 1024 elements with a carry.  Every output is written after every input
// was read, so in and out may alias.
constexpr uint32_t kScanLds = 16384;
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    uint32_t x = v;
#pragma unroll
    for (uint32_t o = 1; o < 64u; o <<= 1) {
        const uint32_t y = uint32_t(__shfl_up(int(x), o));
        x += lane >= o ? y : 0u;
    }
    if (lane == 63u) wsum[w] = x;
    __syncthreads();
    if (w == 0) {
        uint32_t z = lane < 16u ? wsum[lane] : 0u;
#pragma unroll
        for (uint32_t o = 1; o < 16u; o <<= 1) {
            const uint32_t y = uint32_t(__shfl_up(int(z), o));
            z += lane >= o ? y : 0u;
        }
        if (lane < 16u) wsum[lane] = z;
    }
    __syncthreads();
    total = wsum[15];
    return (w ? wsum[w - 1] : 0u) + x - v;
}
// tot (optional): tot[0] = the total, tot[1] = whether it fits cap entries
// (and, times mul, cap2 when cap2 != 0) -- k_total's outputs.
__device__ __forceinline__ void scan_total(uint32_t* tot, uint32_t total, uint32_t cap, uint32_t mul, uint64_t cap2) {
    if (tot && threadIdx.x == 0) {
        tot[0] = total;
        tot[1] = (total <= cap && (cap2 == 0 || uint64_t(total) * mul <= cap2)) ? 1u : 0u;
    }
}
__global__ __launch_bounds__(1024) void k_scan_small(const uint32_t* in, uint32_t n, uint32_t* out, uint32_t* tot,
                                                     uint32_t cap, uint32_t mul, uint64_t cap2) {
    __shared__ uint32_t wsum[16];
    __shared__ uint32_t buf[kScanLds];
    const uint32_t t = threadIdx.x;
    if (n <= kScanLds) {
        for (uint32_t i = t; i < n; i += 1024u) buf[i] = in[i];
        __syncthreads();
        const uint32_t per = (n + 1023u) / 1024u, b0 = min(n, t * per), b1 = min(n, b0 + per);
        uint32_t sum = 0;
        for (uint32_t i = b0; i < b1; ++i) sum += buf[i];
        uint32_t total;
        uint32_t run = block_exclusive_scan(sum, wsum, total);
        for (uint32_t i = b0; i < b1; ++i) {
            const uint32_t v = buf[i];
            buf[i] = run;
            run += v;
        }
        __syncthreads();
        for (uint32_t i = t; i < n; i += 1024u) out[i] = buf[i];
        scan_total(tot, total, cap, mul, cap2);
        return;
    }
    uint32_t carry = 0;
    for (uint32_t base = 0; base < n; base += 1024u) {
        const uint32_t i = base + t;
        const uint32_t v = i < n ? in[i] : 0u;
        uint32_t total;
        const uint32_t ex = block_exclusive_scan(v, wsum, total);
        if (i < n) out[i] = carry + ex;
        carry += total;
        __syncthreads();
    }
    scan_total(tot, carry, cap, mul, cap2);
}

// Exact selectivity counts (real_dataset_adapter.cuh:346-383), tiled: a tile
// of one cell's rows is staged in LDS once and tested against every query
// that selects the cell; points outside a query's selected cells cannot pass
// its range, so they need no test.
__global__ __launch_bounds__(256) void k_selcount(const uint32_t* tile_cell, const uint32_t* tile_row0,
                                                  const uint32_t* tile_n, const float* attrs, uint32_t a,
                                                  const uint32_t* cstart, const uint32_t* ccount,
                                                  const uint32_t* cellq, const float* lo, const float* hi,
                                                  uint32_t* selcount) {
    extern __shared__ float sa[];
    const uint32_t t = blockIdx.x;
    const uint32_t c = tile_cell[t], r0 = tile_row0[t], n = tile_n[t];
    for (uint32_t i = threadIdx.x; i < n * a; i += blockDim.x) sa[i] = attrs[size_t(r0) * a + i];
    __syncthreads();
    const uint32_t qs = cstart[c], qn = ccount[c];
    for (uint32_t k = threadIdx.x; k < qn; k += blockDim.x) {
        const uint32_t q = cellq[qs + k];
        float l[kMaxAttr], h[kMaxAttr];
#pragma unroll
        for (uint32_t d = 0; d < kMaxAttr; ++d) {
            l[d] = d < a ? lo[size_t(q) * a + d] : 0.0f;
            h[d] = d < a ? hi[size_t(q) * a + d] : 0.0f;
        }
        uint32_t cnt = 0;
        if (a == 2) {
            for (uint32_t j = 0; j < n; ++j) {
                const float v0 = sa[2 * j], v1 = sa[2 * j + 1];
                cnt += (v0 >= l[0]) & (v0 <= h[0]) & (v1 >= l[1]) & (v1 <= h[1]);
            }
        } else {
            for (uint32_t j = 0; j < n; ++j) {
                bool ok = true;
#pragma unroll
                for (uint32_t d = 0; d < kMaxAttr; ++d)
                    if (d < a) { const float v = sa[j * a + d]; ok = ok && v >= l[d] && v <= h[d]; }
                cnt += ok;
            }
        }
        if (cnt) atomicAdd(&selcount[q], cnt);
    }
}

// Prefilter routing (real_dataset_adapter.cuh:374-381): the selectivity is
// computed in double, stored as float and compared with the threshold.
__global__ void k_route(uint32_t Q, uint32_t N, float thr, const uint32_t* selcount, const uint32_t* counts,
                        uint32_t* little, uint32_t* ticket, uint64_t* st_exit) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q < Q) {
        const float proportion = float((1.0 * selcount[q]) / (1.0 * N));
        little[q] = proportion <= thr ? counts[q] : 0u;
    }
    stamp_exit(ticket, st_exit);
}

// Arithmetic-grid cells (intersection_area_batch_mark_little_seg,
// gpu_graph.cu:11095-11188): cell index of a value v on attribute d is
// trunc((v - min_d) / width_d) (fp32), clamped to [0, g_d - 1] -- the
// reference clamps only the upper index and writes past its flag array for
// a range starting beyond the grid; clamping both ends selects the edge
// cells, where a builder that clamps puts out-of-grid points.  Every
// selected cell is "little" when the product over attributes of its overlap
// with the range, in units of the cell width, is <= thr (fp64, no fused
// operations, as the reference's double expression).  Cells come out in
// ascending id; flags[q * P + c] = 1 (selected) | 2 (little); little[q] =
// number of little cells.  An empty range (lo > hi) selects nothing, and
// cells holding no point are never selected.
__device__ __forceinline__ uint32_t grid_index(float v, float m, float w, uint32_t g) {
    const float x = __fdiv_rn(__fsub_rn(v, m), w);
    if (!(x > 0.0f)) return 0u;
    if (x >= float(g)) return g - 1;
    return uint32_t(x);
}

__global__ void k_cells_grid(uint32_t Q, uint32_t a, const float* lo, const float* hi, const float* amin,
                             const float* width, const uint32_t* grid, uint32_t P, const uint32_t* offset,
                             double thr, uint32_t* cells, uint32_t* counts, uint32_t* little, uint8_t* flags) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    uint8_t* fl = flags + size_t(q) * P;
    for (uint32_t c = 0; c < P; ++c) fl[c] = 0;
    uint32_t cl[kMaxAttr], ch[kMaxAttr], idx[kMaxAttr], g[kMaxAttr];
    bool empty = false;
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        if (d >= a) break;
        g[d] = grid[d];
        const float vl = lo[size_t(q) * a + d], vh = hi[size_t(q) * a + d];
        if (!(vl <= vh)) empty = true;
        cl[d] = grid_index(vl, amin[d], width[d], g[d]);
        ch[d] = grid_index(vh, amin[d], width[d], g[d]);
        idx[d] = cl[d];
    }
    uint32_t n = 0, nl = 0;
    if (!empty) {
        while (true) {
            uint32_t pid = 0, f = 1;
            for (int d = int(a) - 1; d >= 0; --d) { pid += idx[d] * f; f *= g[d]; }
            if (offset[pid + 1] > offset[pid]) {
                double area = 1.0;
                for (uint32_t d = 0; d < a; ++d) {
                    const double step = double(idx[d]), w = double(width[d]), m = double(amin[d]);
                    const double cl0 = __dadd_rn(m, __dmul_rn(step, w));
                    const double ch0 = __dadd_rn(m, __dmul_rn(__dadd_rn(step, 1.0), w));
                    const double lb = fmax(cl0, double(lo[size_t(q) * a + d]));
                    const double rb = fmin(ch0, double(hi[size_t(q) * a + d]));
                    area = __dmul_rn(area, __ddiv_rn(__dsub_rn(rb, lb), w));
                }
                const bool lit = area <= thr;
                cells[size_t(q) * P + n++] = pid;
                nl += lit;
                fl[pid] = uint8_t(1u | (lit ? 2u : 0u));
            }
            int d = int(a) - 1;
            for (; d >= 0; --d) {
                if (++idx[d] <= ch[d]) break;
                idx[d] = cl[d];
            }
            if (d < 0) break;
        }
    }
    counts[q] = n;
    little[q] = nl;
}

// Per-cell flags from ordered cell lists: the first little[q] cells of a
// query's list are little (the cells the brute-force branch scans).
__global__ void k_cell_flags(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                             const uint32_t* little, uint8_t* flags) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    uint8_t* fl = flags + size_t(q) * P;
    for (uint32_t c = 0; c < P; ++c) fl[c] = 0;
    const uint32_t n = counts[q], l = little[q];
    for (uint32_t i = 0; i < n; ++i) fl[cells[size_t(q) * P + i]] = uint8_t(1u | (i < l ? 2u : 0u));
}

// Cell lists of one streamed batch (fill_partition_info03, tools.cuh:1646-1670):
// the query's selected cells among the batch's, in batch order, as batch
// positions; the query takes the brute-force branch on this batch when all
// of them are little (little = count), else it traverses them (little = 0).
__global__ void k_stream_lists(uint32_t Q, uint32_t P, uint32_t B, const uint32_t* bcell, const uint8_t* flags,
                               uint32_t* lists, uint32_t* counts, uint32_t* little) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    const uint8_t* fl = flags + size_t(q) * P;
    uint32_t n = 0;
    bool all = true;
    for (uint32_t i = 0; i < B; ++i) {
        const uint8_t f = fl[bcell[i]];
        if (f & 1u) {
            lists[size_t(q) * B + n++] = i;
            all = all && (f & 2u);
        }
    }
    counts[q] = n;
    little[q] = (n > 0 && all) ? n : 0u;
}

// The device wall clock (constant rate, hipDeviceAttributeWallClockRate).
__global__ void k_stamp(uint64_t* t, uint32_t n) {
    const uint64_t now = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x < n) t[threadIdx.x] = now;
}

__global__ void k_zero_u32(uint32_t* x, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) x[i] = 0;
}

// Per-query state of the MFMA brute-force schedule, reset in one pass:
// pairs and appended keys zeroed, bounds open.
__global__ void k_bf_reset(uint32_t Q, uint32_t* nsub, uint32_t* pcnt, uint32_t* gbound, uint32_t NS, uint32_t* scnt,
                           uint32_t* nseed) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (scnt && q < NS) scnt[q] = 0;
    if (nseed && q == 0) *nseed = 0;
    if (q >= Q) return;
    nsub[q] = 0;
    pcnt[q] = 0;
    gbound[q] = 0xFFFFFFFFu;
}

// Sentinel results and zero counters for a batch's searches.
__global__ void k_reset_results(uint32_t Q, uint32_t K, uint32_t* ids, float* dist, uint32_t* ctr, uint32_t* z,
                                uint32_t nz, uint64_t* st, uint32_t nst, BfReset br) {
    stamp_entry(st, nst);
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < Q * K) { ids[i] = GF_NO_RESULT; dist[i] = __int_as_float(0x7F800000); }
    if (i < Q * GF_NCOUNTERS) ctr[i] = 0;
    if (i < nz) z[i] = 0;
    // k_bf_reset's work when br.nsub is set
    if (br.nsub) {
        if (br.scnt && i < br.NS) br.scnt[i] = 0;
        if (br.nseed && i == 0) *br.nseed = 0;
        if (i < Q) {
            br.nsub[i] = 0;
            br.pcnt[i] = 0;
            br.gbound[i] = 0xFFFFFFFFu;
        }
    }
}

// A search's small host-side outputs in one kernel instead of three copies:
// the statistics sums (optional), the schedule totals and the timestamps,
// written to page-locked host memory.
__global__ void k_gather_meta(const unsigned long long* stats, const uint32_t* tot, const uint64_t* stamps,
                              unsigned long long* h_stats, uint32_t* h_tot, uint64_t* h_stamps) {
    // the search ends here: its timestamp [2] is taken now
    const uint64_t now = __builtin_amdgcn_s_memrealtime();
    const uint32_t t = threadIdx.x;
    if (stats && t < 16u) h_stats[t] = stats[t];
    if (t < 24u) h_tot[t] = tot[t];
    if (t < 12u) h_stamps[t] = t == 2u ? now : stamps[t];   // the search's [0..4], stages A [5..6] and B [7..8]
}

// What each batch of a streamed plan must do for this query batch (one
// workgroup per batch): need[b] bit 0 = some query takes the brute force on
// it (all its selected cells of the batch little), bit 1 = some query
// traverses it; 0 = no query selects any of its cells.  active[b] = queries
// with a selected cell in batch b.
__global__ __launch_bounds__(256) void k_batch_need(uint32_t Q, uint32_t P, const uint32_t* plan_cells,
                                                    const uint32_t* plan_off, const uint8_t* flags, uint32_t* need,
                                                    uint32_t* active) {
    __shared__ uint32_t acc, nact;
    const uint32_t bi = blockIdx.x;
    if (threadIdx.x == 0) { acc = 0; nact = 0; }
    __syncthreads();
    const uint32_t c0 = plan_off[bi], c1 = plan_off[bi + 1];
    uint32_t mine = 0, na = 0;
    for (uint32_t q = blockIdx.y * blockDim.x + threadIdx.x; q < Q; q += gridDim.y * blockDim.x) {
        const uint8_t* fl = flags + size_t(q) * P;
        uint32_t n = 0;
        bool all = true;
        for (uint32_t i = c0; i < c1; ++i) {
            const uint8_t f = fl[plan_cells[i]];
            if (f & 1u) { ++n; all = all && (f & 2u); }
        }
        if (n) { mine |= all ? 1u : 2u; ++na; }
    }
    if (mine) atomicOr(&acc, mine);
    if (na) atomicAdd(&nact, na);
    __syncthreads();
    if (threadIdx.x == 0 && acc) atomicOr(&need[bi], acc);   // need[] and active[] zeroed before
    if (threadIdx.x == 0 && nact) atomicAdd(&active[bi], nact);
}

// Bounding box of each query's listed cells on a grid of a axes (row-major,
// last axis fastest): box[q * 2a + d] = lowest coordinate on axis d,
// box[q * 2a + a + d] = highest; a query with no cell gets lo = grid, hi = 0.
__global__ __launch_bounds__(256) void k_cell_boxes(uint32_t Q, uint32_t P, uint32_t a, const uint32_t* grid,
                                                    const uint32_t* cells, const uint32_t* counts, uint32_t* box) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    uint32_t lo[kMaxAttr], hi[kMaxAttr], g[kMaxAttr];
#pragma unroll
    for (uint32_t d = 0; d < kMaxAttr; ++d) {
        g[d] = d < a ? grid[d] : 1u;
        lo[d] = g[d];
        hi[d] = 0;
    }
    const uint32_t n = counts[q] < P ? counts[q] : P;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t c = cells[size_t(q) * P + i];
        if (c >= P) continue;
#pragma unroll
        for (int d = kMaxAttr - 1; d >= 0; --d) {
            if (uint32_t(d) >= a) continue;
            const uint32_t x = c % g[d];
            c /= g[d];
            lo[d] = x < lo[d] ? x : lo[d];
            hi[d] = x > hi[d] ? x : hi[d];
        }
    }
    for (uint32_t d = 0; d < a; ++d) {
        box[size_t(q) * 2 * a + d] = lo[d];
        box[size_t(q) * 2 * a + a + d] = hi[d];
    }
}

// A streamed batch's image assembled from pinned host memory over PCIe: the
// pieces of GatherDesc in order, every thread striding over each piece in
// chunks of the widest of 16, 8, 4 or 1 bytes that source, image, pitches
// and width allow, four chunks in flight per thread.  Tile metadata pieces
// get their rows rebased on the way (mw != 0).
template <typename V>
__device__ inline void gather_fix(V& v, uint64_t byte, uint32_t add, uint32_t mw) {
    if (uint32_t((byte / 4) % mw) >= 16u) return;
    uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
    for (uint32_t k = 0; k < sizeof(V) / 4; ++k)
        if (w[k] != 0xFFFFFFFFu) w[k] += add;
}

template <typename V>
__device__ inline void gather_piece(const char* src, char* dst, uint64_t spitch, uint64_t dpitch, uint32_t width,
                                    uint32_t nrow, uint32_t add, uint32_t mw, uint32_t tid, uint32_t nt) {
    const uint64_t wc = width / sizeof(V), total = wc * nrow;
    for (uint64_t i = tid; i < total; i += 4ull * nt) {
        V v[4];
        uint64_t so[4], dof[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint64_t j = i + uint64_t(u) * nt;
            if (j >= total) break;
            const uint64_t r = nrow == 1 ? 0 : j / wc, c = j - r * wc;
            so[u] = r * spitch + c * sizeof(V);
            dof[u] = r * dpitch + c * sizeof(V);
            v[u] = *reinterpret_cast<const V*>(src + so[u]);
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint64_t j = i + uint64_t(u) * nt;
            if (j >= total) break;
            if constexpr (sizeof(V) >= 4) {
                if (mw) gather_fix(v[u], so[u], add, mw);
            }
            *reinterpret_cast<V*>(dst + dof[u]) = v[u];
        }
    }
}

__global__ __launch_bounds__(256) void k_stream_gather(const GatherDesc* __restrict__ desc, uint32_t n,
                                                       const char* arena, const char* head, char* img) {
    const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x, nt = gridDim.x * blockDim.x;
    for (uint32_t k = 0; k < n; ++k) {
        const GatherDesc g = desc[k];
        const char* src = (g.base ? head : arena) + g.src;
        char* dst = img + g.dst;
        const uint64_t al = reinterpret_cast<uint64_t>(src) | reinterpret_cast<uint64_t>(dst) | g.width |
                            (g.nrow > 1 ? (g.spitch | g.dpitch) : 0);
        if ((al & 15u) == 0)
            gather_piece<uint4>(src, dst, g.spitch, g.dpitch, g.width, g.nrow, g.add, g.mw, tid, nt);
        else if ((al & 7u) == 0)
            gather_piece<uint2>(src, dst, g.spitch, g.dpitch, g.width, g.nrow, g.add, g.mw, tid, nt);
        else if ((al & 3u) == 0)
            gather_piece<uint32_t>(src, dst, g.spitch, g.dpitch, g.width, g.nrow, g.add, g.mw, tid, nt);
        else
            gather_piece<uint8_t>(src, dst, g.spitch, g.dpitch, g.width, g.nrow, 0u, 0u, tid, nt);
    }
}

// Running top-K of a streamed search: merge the batch's sorted K results
// into the running ones (a batch's entry goes first at equal distance, as
// the reference's host merge, big_dataset_adapterV3.cuh:3785-3795) and add
// its counters.  Batches hold disjoint cells, so ids never repeat.
__global__ void k_merge_stream(uint32_t Q, uint32_t K, uint32_t* run_ids, float* run_dist, const uint32_t* ids,
                               const float* dist, uint32_t* run_ctr, const uint32_t* ctr, uint32_t first) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    uint32_t* ri = run_ids + size_t(q) * K;
    float* rd = run_dist + size_t(q) * K;
    const uint32_t* ni = ids + size_t(q) * K;
    const float* nd = dist + size_t(q) * K;
    // counters add up; the route counter becomes (traversed batches) |
    // (brute-force batches << 16)
    uint32_t* rc = run_ctr + size_t(q) * GF_NCOUNTERS;
    const uint32_t* nc = ctr + size_t(q) * GF_NCOUNTERS;
    const uint32_t route = nc[C_ROUTE] == 1u ? 1u : (nc[C_ROUTE] == 2u ? 0x10000u : 0u);
    if (first) {
        for (uint32_t k = 0; k < K; ++k) { ri[k] = ni[k]; rd[k] = nd[k]; }
        for (uint32_t c = 0; c < GF_NCOUNTERS; ++c) rc[c] = c == C_ROUTE ? route : nc[c];
        return;
    }
    uint32_t oi[kBfKMax * 4];
    float od[kBfKMax * 4];
    for (uint32_t k = 0; k < K; ++k) { oi[k] = ri[k]; od[k] = rd[k]; }
    uint32_t i = 0, j = 0;
    for (uint32_t t = 0; t < K; ++t) {
        if (od[i] < nd[j]) { ri[t] = oi[i]; rd[t] = od[i]; ++i; }
        else { ri[t] = ni[j]; rd[t] = nd[j]; ++j; }
    }
    for (uint32_t c = 0; c < GF_NCOUNTERS; ++c) rc[c] += c == C_ROUTE ? route : nc[c];
}

// Query x centre squared distances |q|^2 + |c|^2 - 2 q.c with the dot
// products on MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation) -- the
// reference's dis_cal_tensor_core<16> (tools.cuh:1493-1559).  A workgroup of
// four waves takes 16 queries x 64 centres; each wave one 16x16 tile.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// |q|^2 + |c|^2 - 2 q.c rounded step by step (no contraction), so the full
// matrix and the fused nearest-centre selection agree bit for bit.
__device__ __forceinline__ float centre_dist(float qn, float cn, float dot) {
    return __fsub_rn(__fadd_rn(qn, cn), __fmul_rn(2.0f, dot));
}

__global__ __launch_bounds__(256) void k_centroid(const uint16_t* qh, const uint16_t* ch, const float* qn,
                                                  const float* cn, uint32_t Q, uint32_t C, uint32_t Dp,
                                                  float* dist, uint64_t* st_entry) {
    stamp_entry(st_entry, 1);
    const uint32_t lane = lane_id(), wave = threadIdx.x >> 6;
    const uint32_t q0 = blockIdx.x * 16u;
    const uint32_t c0 = (blockIdx.y * 4u + wave) * 16u;
    const uint32_t r = lane & 15u, kq = (lane >> 4) * 8u;
    const half8_t* ap = reinterpret_cast<const half8_t*>(qh + size_t(q0 + r) * Dp + kq);
    const half8_t* bp = reinterpret_cast<const half8_t*>(ch + size_t(c0 + r) * Dp + kq);
    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t k = 0; k < Dp; k += 32u) {
        const half8_t av = ap[k / 8u];
        const half8_t bv = bp[k / 8u];
        // centres as A, queries as B: the operand order of k_centroid_top,
        // so both produce the same bits for every (query, centre)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(bv, av, acc, 0, 0, 0);
    }
    const uint32_t row = q0 + (lane & 15u);
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t col = c0 + (lane >> 4) * 4u + i;
        if (row < Q && col < C) dist[size_t(row) * C + col] = centre_dist(qn[row], cn[col], acc[i]);
    }
}

// (distance, centre) order of the nearest-centre choice; NaN counts as +inf.
__device__ __forceinline__ bool ckey_lt(float d, uint32_t c, float e, uint32_t f) {
    return d < e || (d == e && c < f);
}
__device__ __forceinline__ void ckey_ce(float& ad, uint32_t& ai, float& bd, uint32_t& bi) {
    if (ckey_lt(bd, bi, ad, ai)) {
        const float td = ad; ad = bd; bd = td;
        const uint32_t t = ai; ai = bi; bi = t;
    }
}
// a := the 4 smallest of sorted lists a and b: min(a[k], b[3 - k]) is
// bitonic, then a half-cleaner sorts it.
__device__ __forceinline__ void merge4(float (&ad)[4], uint32_t (&ai)[4], const float (&bd)[4],
                                       const uint32_t (&bi)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (ckey_lt(bd[3 - k], bi[3 - k], ad[k], ai[k])) { ad[k] = bd[3 - k]; ai[k] = bi[3 - k]; }
    ckey_ce(ad[0], ai[0], ad[2], ai[2]);
    ckey_ce(ad[1], ai[1], ad[3], ai[3]);
    ckey_ce(ad[0], ai[0], ad[1], ai[1]);
    ckey_ce(ad[2], ai[2], ad[3], ai[3]);
}

// Stage B's nearest centres without the Q x C matrix: a workgroup takes 16
// queries against every centre tile (each of its kCtW waves every kCtW-th
// tile, the MFMA tiles and distances of k_centroid); lane l keeps, for its
// query, the 4 smallest (distance, centre) keys it saw, then the lists merge
// across the four lanes of the query and the waves.  Writes the first topc (<= 4) centres of each query, as the
// sequential arg-min rounds of k_order would pick them from the matrix.
constexpr uint32_t kCtW = 4;
__global__ __launch_bounds__(64 * kCtW) void k_centroid_top(const uint16_t* qh, const uint16_t* ch, const float* qn,
                                                            const float* cn, uint32_t Q, uint32_t C, uint32_t Cp,
                                                            uint32_t Dp, uint32_t topc, uint32_t* topk,
                                                            uint64_t* st_entry) {
    stamp_entry(st_entry, 1);
    __shared__ float sd[kCtW][16][4];
    __shared__ uint32_t si[kCtW][16][4];
    const uint32_t lane = lane_id(), wave = threadIdx.x >> 6;
    const uint32_t q0 = blockIdx.x * 16u;
    const uint32_t r = lane & 15u, g = lane >> 4, kq = g * 8u;
    // Centres are the A operand and queries the B operand: lane l holds the
    // products of query q0 + l % 16 with centres 4 (l / 16) + i of the tile,
    // so it keeps the top 4 of one query and only the four lanes sharing it
    // merge at the end.
    // The query operand stays in registers for up to kCtK k-steps of 32
    // (256 dimensions); a tile's centre operands and norms are loaded
    // together and waited for once.
    constexpr uint32_t kCtK = 8;
    const uint32_t nks = Dp / 32u;
    const half8_t* qp = reinterpret_cast<const half8_t*>(qh + size_t(q0 + r) * Dp + kq);
    half8_t qv[kCtK];
#pragma unroll
    for (uint32_t k = 0; k < kCtK; ++k)
        if (k < nks) qv[k] = qp[k * 4u];
    const float qr = q0 + r < Q ? qn[q0 + r] : 0.0f;
    float td[4];
    uint32_t ti[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) { td[k] = __int_as_float(0x7F800000); ti[k] = 0xFFFFFFFFu; }
    for (uint32_t ct = wave; ct < Cp / 16u; ct += kCtW) {
        const uint32_t c0 = ct * 16u;
        const half8_t* bp = reinterpret_cast<const half8_t*>(ch + size_t(c0 + r) * Dp + kq);
        half8_t cv[kCtK];
#pragma unroll
        for (uint32_t k = 0; k < kCtK; ++k)
            if (k < nks) cv[k] = bp[k * 4u];
        const float4_t cc = *reinterpret_cast<const float4_t*>(cn + c0 + g * 4u);   // cn holds Cp norms
        float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t k = 0; k < kCtK; ++k)
            if (k < nks) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cv[k], qv[k], acc, 0, 0, 0);
        for (uint32_t k = kCtK; k < nks; ++k)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(bp[k * 4u], qp[k * 4u], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t col = c0 + g * 4u + uint32_t(i);
            if (col < C) {
                float d = centre_dist(qr, cc[i], acc[i]);
                if (d != d) d = __int_as_float(0x7F800000);
                // most centres lose to the current 4th: insert only past it
                if (ckey_lt(d, col, td[3], ti[3])) {
                    bool lt[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) lt[k] = ckey_lt(d, col, td[k], ti[k]);
#pragma unroll
                    for (int k = 3; k >= 1; --k) {
                        td[k] = lt[k - 1] ? td[k - 1] : (lt[k] ? d : td[k]);
                        ti[k] = lt[k - 1] ? ti[k - 1] : (lt[k] ? col : ti[k]);
                    }
                    if (lt[0]) { td[0] = d; ti[0] = col; }
                }
            }
        }
    }
#pragma unroll
    for (uint32_t m = 16; m < 64u; m <<= 1) {
        float od[4];
        uint32_t oi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            od[k] = __shfl_xor(td[k], int(m));
            oi[k] = uint32_t(__shfl_xor(int(ti[k]), int(m)));
        }
        merge4(td, ti, od, oi);
    }
    if (g == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            sd[wave][r][k] = td[k];
            si[wave][r][k] = ti[k];
        }
    }
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < 16u && q0 + t < Q) {
        float ad[4];
        uint32_t ai[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) { ad[k] = sd[0][t][k]; ai[k] = si[0][t][k]; }
        for (uint32_t w = 1; w < kCtW; ++w) {
            float bd[4];
            uint32_t bi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) { bd[k] = sd[w][t][k]; bi[k] = si[w][t][k]; }
            merge4(ad, ai, bd, bi);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (uint32_t(k) < topc) topk[size_t(q0 + t) * topc + k] = ai[k] < C ? ai[k] : 0u;
    }
}

// Cluster-guided cell order (tools.cuh:1398-1491 top clusters, then
// gpu_graph.cu:11343-11396): one wave per query picks its topc nearest centres
// by (distance, index) -- NaN (empty cluster) counts as +inf -- scores every
// selected cell by the sum of its histogram entries over those centres and
// sorts the cells by (score descending, cell ascending), or, with ref_ties, by
// the reference's own network, bitonic_sort_id_by_num_int (gpu_graph.cu:123-141)
// over the cells in their stage A order: a descending flip-bitonic network
// whose order of equal scores is fixed by the network, not by the cells.
__device__ __forceinline__ void order_query(uint32_t Q, uint32_t C, uint32_t P, uint32_t topc,
                                            const float* dist, const uint32_t* hist, uint32_t* cells,
                                            const uint32_t* counts, uint32_t* topk, bool chosen, bool ref_ties) {
    extern __shared__ uint32_t so[];
    uint32_t* tk = so;             // topc
    uint32_t* sc = so + 16;        // P scores
    uint32_t* cc = sc + P;         // P cells
    const uint32_t q = blockIdx.x, lane = lane_id();
    const float* dq = dist + size_t(q) * C;
    float pd = -1.0f;
    uint32_t pi = 0xFFFFFFFFu;
    // chosen: the nearest centres are already in topk (k_centroid_top)
    if (chosen && lane < topc) tk[lane] = topk[size_t(q) * topc + lane];
    for (uint32_t t = 0; !chosen && t < topc; ++t) {
        float bd = __int_as_float(0x7F800000);
        uint32_t bi = 0xFFFFFFFFu;
        for (uint32_t c = lane; c < C; c += 64u) {
            float v = dq[c];
            if (v != v) v = __int_as_float(0x7F800000);
            const bool after = (v > pd) || (v == pd && (pi == 0xFFFFFFFFu || c > pi));
            const bool before = (v < bd) || (v == bd && c < bi);
            if (after && before) { bd = v; bi = c; }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float od = __shfl_xor(bd, m, 64);
            const uint32_t oi = __shfl_xor(bi, m, 64);
            if (od < bd || (od == bd && oi < bi)) { bd = od; bi = oi; }
        }
        pd = bd;
        pi = bi;
        if (lane == 0) { tk[t] = bi < C ? bi : 0u; topk[size_t(q) * topc + t] = bi < C ? bi : 0u; }
    }
    __syncthreads();
    const uint32_t n = counts[q];
    uint32_t* cl = cells + size_t(q) * P;
    for (uint32_t i = lane; i < n; i += 64u) {
        const uint32_t cell = cl[i];
        uint32_t s = 0;
        for (uint32_t t = 0; t < topc; ++t) s += hist[size_t(cell) * C + tk[t]];
        sc[i] = s;
        cc[i] = cell;
    }
    __syncthreads();
    if (ref_ties) {
        // The pairs (u, d) of one (stride, step) pass are disjoint.
        for (uint32_t stride = 1; stride < n; stride <<= 1)
            for (uint32_t step = stride; step > 0; step >>= 1) {
                for (uint32_t k = lane; k < n / 2; k += 64u) {
                    const uint32_t a0 = 2 * step * (k / step), b0 = k % step;
                    const uint32_t u = step == stride ? a0 + step - 1 - b0 : a0 + b0;
                    const uint32_t d = a0 + b0 + step;
                    if (d < n && int32_t(sc[u]) < int32_t(sc[d])) {
                        const uint32_t ts = sc[u], tc = cc[u];
                        sc[u] = sc[d]; cc[u] = cc[d];
                        sc[d] = ts; cc[d] = tc;
                    }
                }
                __syncthreads();
            }
        for (uint32_t i = lane; i < n; i += 64u) cl[i] = cc[i];
        return;
    }
    for (uint32_t i = lane; i < n; i += 64u) {
        const uint32_t s = sc[i], cell = cc[i];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < n; ++j) rank += (sc[j] > s) || (sc[j] == s && cc[j] < cell);
        cl[rank] = cell;
    }
}
__global__ __launch_bounds__(64) void k_order(uint32_t Q, uint32_t C, uint32_t P, uint32_t topc,
                                              const float* dist, const uint32_t* hist, uint32_t* cells,
                                              const uint32_t* counts, uint32_t* topk, bool chosen, bool ref_ties) {
    order_query(Q, C, P, topc, dist, hist, cells, counts, topk, chosen, ref_ties);
}

// ------------------------------------------ query-batch brute force (MFMA)
// Filtered brute force for the queries routed to it, when every vector and
// query is an integer in [0, 255] and every attribute an integer whose spread
// inside a cell is below 65534.  With x' = x - 128 and q' = q - 128 (int8),
// |q - x|^2 = |q'|^2 + |x'|^2 - 2 q'.x' holds exactly in int32, so distances
// are bit-identical to the canonical fp32 ones (all sums < 2^24).
//
// A work item is one sub-cell and up to 64 queries whose range reaches it;
// persistent waves take items in turn.  The queries are the stationary B
// operand (four 16-query column tiles); the sub-cell's 16-point tiles stream
// as the A operand of v_mfma_i32_16x16x64_i8; lane l receives points
// 4 (l / 16) + i, i < 4, of query 16 j + l % 16 for each column tile j.  The
// accumulator starts at -floor(|x'|^2 / 2), so "d <= thr" becomes the single
// compare acc >= ceil((|q'|^2 - thr) / 2) (exact up to the parity of |x'|^2,
// which the owner's exact test settles).  The range test runs, where some pair
// of a column tile is within its bound, on that column tile's pairs as a
// packed u16 clamp (not at all in an item whose queries all contain the
// sub-cell): per cell, attributes are stored as value - base in
// [0, 65533] (tile padding 65535) and a query's range becomes [lo', hi'] in the
// same units (an empty range is [65534, 65534]); a point passes iff clamping
// its packed word leaves it unchanged.  Survivors (rare once the threshold has
// settled) go to a per-query LDS buffer; lane q of the wave owns query q of
// the block, keeps its sorted top-K (distance, row) in registers and merges
// its buffer once some query's buffer holds kBfDrainAt entries.  Thresholds
// tighten from the wave's own top-K and from a per-query global bound that
// every item lowers with atomicMin when it ends and reads when it starts: a
// point farther than some item's K-th distance cannot be in the final top-K,
// and only keys within the bound are appended for the final merge.
typedef int v4i32_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
constexpr uint32_t kQB = 64;        // queries per wave
constexpr uint32_t kBfBufQ = 24;    // survivor slots per query
constexpr uint32_t kBfDrainAt = 8;  // drain once a query holds this many (+ <= 16 per tile < 24)
constexpr uint64_t kKeySent = ~uint64_t(0);
// acc threshold while fewer than K are known: every point passes it except
// tile padding, whose accumulator is seeded with INT32_MIN (its int8 vector is
// zero, so its accumulator stays there); padding never survives, with or
// without the range test.
constexpr int32_t kTpOpen = INT32_MIN + 1;
constexpr int32_t kPadSeed = INT32_MIN;

// LDS ordering between the lanes of one wave of a multi-wave workgroup:
// the fences stop the compiler from moving LDS accesses across this point,
// and the wave executes its LDS instructions in order.
// Workgroup barrier ordering LDS only: global loads in flight stay in
// flight (a full __syncthreads waits for them).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t clamp16(uint32_t x, uint32_t lo, uint32_t hi) {
    u16x2_t v = __builtin_bit_cast(u16x2_t, x);
    v = __builtin_elementwise_min(__builtin_elementwise_max(v, __builtin_bit_cast(u16x2_t, lo)),
                                  __builtin_bit_cast(u16x2_t, hi));
    return __builtin_bit_cast(uint32_t, v);
}

// One attribute range [lo, hi] (floats holding integers) in the units of a
// cell whose attribute values are base + [0, 65533].
__device__ __forceinline__ void range16(float lo, float hi, int32_t base, uint32_t& l16, uint32_t& h16) {
    if (!(lo <= hi)) { l16 = h16 = 65534u; return; }   // empty or NaN bound: nothing passes
    const float lc = ceilf(fmaxf(lo, -4.0e9f)), hc = floorf(fminf(hi, 4.0e9f));
    const int64_t l = int64_t(lc) - base, h = int64_t(hc) - base;
    if (!(lc <= hc) || h < 0 || l > 65533) { l16 = h16 = 65534u; return; }
    l16 = uint32_t(l < 0 ? 0 : l);
    h16 = uint32_t(h > 65533 ? 65533 : h);
}

__device__ __forceinline__ int32_t acc_threshold(int32_t nq, uint32_t thr) {
    if (thr == 0xFFFFFFFFu) return kTpOpen;
    return int32_t((int64_t(nq) - int64_t(thr) + 1) >> 1);   // ceil((nq - thr) / 2)
}

// ------------------------------------------------------------ sub-cells
// Attribute box of one sub-cell as floats (attribute values are integers and
// the conversion is monotone, so comparing the float bounds with the box ends
// decides every point's float comparison of the reference).
struct SubBox {
    float mn[4], mx[4];
};
__device__ __forceinline__ SubBox load_box(const SubArgs& sa, uint32_t s) {
    SubBox b;
#pragma unroll
    for (uint32_t d = 0; d < 4; ++d) {
        b.mn[d] = d < sa.a ? float(sa.sbox[size_t(s) * 2 * sa.a + 2 * d]) : 0.0f;
        b.mx[d] = d < sa.a ? float(sa.sbox[size_t(s) * 2 * sa.a + 2 * d + 1]) : 0.0f;
    }
    return b;
}
// A query's range held in registers.
struct QRange {
    float l[4], h[4];
};
__device__ __forceinline__ QRange load_range(uint32_t a, const float* lo, const float* hi, uint32_t q) {
    QRange r;
#pragma unroll
    for (uint32_t d = 0; d < 4; ++d) {
        r.l[d] = d < a ? lo[size_t(q) * a + d] : 0.0f;
        r.h[d] = d < a ? hi[size_t(q) * a + d] : 0.0f;
    }
    return r;
}
// Relation of a range to a (non-empty) sub-cell: 0 no point can pass,
// 1 partially covered, 2 every point passes.
__device__ __forceinline__ uint32_t sub_relation(const SubBox& b, uint32_t a, const QRange& r) {
    bool inside = true, outside = false;
#pragma unroll
    for (uint32_t d = 0; d < 4; ++d) {
        if (d < a) {
            inside = inside && r.l[d] <= b.mn[d] && b.mx[d] <= r.h[d];
            outside = outside || !(r.h[d] >= b.mn[d]) || !(b.mx[d] >= r.l[d]);
        }
    }
    return outside ? 0u : inside ? 2u : 1u;
}

// Stage A exact counts, one workgroup per sub-cell, over all queries in
// chunks of 256: a query covering the whole box adds the sub-cell's size; the
// partially covered ones are compacted in LDS and tested point by point (each
// lane holds 16 points' packed attribute words, 1024 points per pass; lane k
// of a wave loads the packed range of the k-th such query, then the wave
// tests the queries one by one with the range broadcast from lane k).
// Global atomics are collected in LDS and issued once per workgroup (or when
// the list fills): a device-scope atomic takes microseconds, and later loads
// of the same wave would wait for it.
constexpr uint32_t kFlushCap = 2048;

template <int AW>
__global__ __launch_bounds__(256) void k_subsel(SubSelArgs p) {
    __shared__ uint32_t cutl[256];
    __shared__ uint32_t ncut, fn;
    __shared__ uint32_t fq[kFlushCap], fv[kFlushCap];
    const SubArgs& sa = p.sa;
    const uint32_t s = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const uint32_t size = sa.ssize[s];
    if (size == 0) return;
    const SubBox box = load_box(sa, s);
    const uint32_t c = sa.scell[s], t0 = sa.stile[s], t1 = sa.stile[s + 1];
    constexpr uint32_t MW = 16u * (1u + AW);
    if (tid == 0) fn = 0;
    auto flush = [&]() {   // all threads; between barriers
        for (uint32_t i = tid; i < fn; i += 256u) atomicAdd(&p.selcount[fq[i]], fv[i]);
    };
    for (uint32_t tb = t0; tb < t1; tb += 64u) {
        uint32_t w[16][AW];
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const uint32_t t = tb + 4u * g + (lane >> 4);
#pragma unroll
            for (int k = 0; k < AW; ++k)
                w[g][k] = t < t1 ? sa.tmeta[size_t(t) * MW + 16u * (1 + k) + (lane & 15u)] : 65535u;
        }
        // Each sub-cell starts at its own chunk, so the per-query atomics of
        // concurrent workgroups land on different queries.
        const uint32_t nch = (p.Q + 255u) / 256u;
        // ranges of the next chunk are loaded while the current one is scanned
        uint32_t qn = (s % nch) * 256u + tid;
        QRange rn = load_range(sa.a, p.lo, p.hi, qn < p.Q ? qn : 0u);
        for (uint32_t ci = 0; ci < nch; ++ci) {
            const uint32_t q = qn;
            const QRange rq = rn;
            qn = ((ci + 1 + s) % nch) * 256u + tid;
            if (ci + 1 < nch) rn = load_range(sa.a, p.lo, p.hi, qn < p.Q ? qn : 0u);
            __syncthreads();
            if (fn + 512u > kFlushCap) {   // a chunk adds at most 2 x 256 entries
                flush();
                __syncthreads();
                if (tid == 0) fn = 0;
            }
            if (tid == 0) ncut = 0;
            __syncthreads();
            const uint32_t rel = q < p.Q ? sub_relation(box, sa.a, rq) : 0u;
            if (rel == 2 && tb == t0) {
                const uint32_t i = atomicAdd(&fn, 1u);
                fq[i] = q;
                fv[i] = size;
            }
            if (rel == 1) cutl[atomicAdd(&ncut, 1u)] = q;
            __syncthreads();
            // The waves split the partial queries: wave w takes entries w, w + 4, ...
            const uint32_t n = ncut, nw = n > wave ? (n - wave + 3u) / 4u : 0u;
            for (uint32_t base = 0; base < nw; base += 64u) {
                const uint32_t k = base + lane;
                const uint32_t qq = k < nw ? cutl[wave + 4u * k] : cutl[wave];
                uint32_t lo16[AW], hi16[AW];
#pragma unroll
                for (int x = 0; x < AW; ++x) {
                    uint32_t l0, h0, l1 = 0u, h1 = 0u;
                    const uint32_t d0 = 2u * x, d1 = 2u * x + 1u;
                    range16(p.lo[size_t(qq) * sa.a + d0], p.hi[size_t(qq) * sa.a + d0], sa.abase[c * sa.a + d0], l0,
                            h0);
                    if (d1 < sa.a)
                        range16(p.lo[size_t(qq) * sa.a + d1], p.hi[size_t(qq) * sa.a + d1], sa.abase[c * sa.a + d1],
                                l1, h1);
                    lo16[x] = l0 | (l1 << 16);
                    hi16[x] = h0 | (h1 << 16);
                }
                const uint32_t nb = min(64u, nw - base);
                for (uint32_t u = 0; u < nb; ++u) {
                    uint32_t bl[AW], bh[AW];
#pragma unroll
                    for (int x = 0; x < AW; ++x) {
                        bl[x] = readlane32(lo16[x], u);
                        bh[x] = readlane32(hi16[x], u);
                    }
                    uint32_t cnt = 0;
#pragma unroll
                    for (int g = 0; g < 16; ++g) {
                        bool ok = true;
#pragma unroll
                        for (int x = 0; x < AW; ++x) ok &= clamp16(w[g][x], bl[x], bh[x]) == w[g][x];
                        cnt += __builtin_popcountll(__builtin_amdgcn_ballot_w64(ok));
                    }
                    if (cnt && lane == u) {
                        const uint32_t i = atomicAdd(&fn, 1u);
                        fq[i] = qq;
                        fv[i] = cnt;
                    }
                }
            }
            __syncthreads();
        }
    }
    __syncthreads();
    flush();
}

// Stage C schedule, one workgroup per sub-cell over all queries: the
// brute-force queries (not traversed, little > 0) whose range reaches the
// sub-cell, in query order starting at a chunk that depends on the sub-cell
// (spreading the per-query atomics of concurrent workgroups).  With qcap > 0
// the count pass also writes each list into the sub-cell's own region of bq;
// else pass 1 counts per sub-cell and per query and pass 2 writes the lists
// at their scanned offsets in the same order.
// Items per (query, sub-cell) pair: the sub-cell's tiles in chunks of tch
// (0: one item).
__device__ __forceinline__ uint32_t tile_chunks(const uint32_t* stile, uint32_t s, uint32_t tch) {
    const uint32_t nt = stile[s + 1] - stile[s];
    return tch ? (nt + tch - 1) / tch : 1u;
}

// Seed choice, one wave per candidate query (see BfSeedArgs): among the
// sub-cells of the first cell of the query's list that its brute force
// reaches (stage B puts the cell nearest the query's closest centres first),
// the one with the most points in range, whole sub-cells by size and partial
// ones by size x box overlap per attribute; ties go to the lowest sub-cell.
// Also writes the candidate records and counts the seed pair in nsub.
__global__ __launch_bounds__(256) void k_bfseed(BfSeedArgs p) {
    const SubArgs& sa = p.sa;
    const uint32_t lane = lane_id();
    const uint32_t q0 = p.qrange[0], nq = p.qrange[1] - q0;
    const uint32_t ci = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (ci >= nq) return;
    const uint32_t q = p.qlist[q0 + ci];
    const uint32_t cnt = p.counts[q], lit = p.little[q];
    const bool bf = !(cnt < p.postfilter && cnt != lit) && lit > 0;
    const QRange r = load_range(sa.a, p.lo, p.hi, q);
    uint64_t key = 0;   // (score bits << 32) | ~sub-cell: the largest wins
    for (uint32_t i = 0; bf && i < cnt && key == 0; ++i) {
        const uint32_t c = p.cells[size_t(q) * sa.P + i];
        if (p.bfm && !(p.bfm[size_t(q) * p.bP + c] & 2u)) continue;
        for (uint32_t s = sa.sbase[c] + lane; s < sa.sbase[c + 1]; s += 64u) {
            const uint32_t n = sa.ssize[s];
            if (!n) continue;
            const SubBox b = load_box(sa, s);
            const uint32_t rel = sub_relation(b, sa.a, r);
            if (!rel) continue;
            float sc = float(n);
            if (rel == 1u) {
#pragma unroll
                for (uint32_t d = 0; d < 4; ++d)
                    if (d < sa.a) {
                        const float ov = fminf(r.h[d], b.mx[d]) - fmaxf(r.l[d], b.mn[d]) + 1.0f;
                        sc *= fminf(1.0f, fmaxf(ov, 1.0f) / (b.mx[d] - b.mn[d] + 1.0f));
                    }
            }
            const uint64_t k = (uint64_t(__float_as_uint(sc)) << 32) | (0xFFFFFFFFu - s);
            key = k > key ? k : key;
        }
#pragma unroll
        for (uint32_t o = 32; o; o >>= 1) {
            const uint64_t other = (uint64_t(uint32_t(__shfl_xor(int(key >> 32), int(o)))) << 32) |
                                   uint32_t(__shfl_xor(int(uint32_t(key)), int(o)));
            key = other > key ? other : key;
        }
    }
    const uint32_t s = key ? 0xFFFFFFFFu - uint32_t(key) : kEmpty;
    // The query's regular pairs: every other non-empty sub-cell its range
    // reaches in a cell its brute force scans (the pairs k_bfsched_direct
    // lists), each in chunks of itch tiles.
    uint32_t np = 0;
    if (bf) {
        // four sub-cells per lane per round, their loads issued together
        for (uint32_t s0 = 0; s0 < sa.NS; s0 += 256u) {
            uint32_t sz[4], t0[4], t1[4], cl[4];
            SubBox bx[4];
#pragma unroll
            for (uint32_t u = 0; u < 4u; ++u) {
                const uint32_t s2 = min(s0 + 64u * u + lane, sa.NS - 1u);
                sz[u] = s0 + 64u * u + lane < sa.NS ? sa.ssize[s2] : 0u;
                t0[u] = sa.stile[s2];
                t1[u] = sa.stile[s2 + 1];
                cl[u] = p.bfm ? sa.scell[s2] : 0u;
                bx[u] = load_box(sa, s2);
            }
#pragma unroll
            for (uint32_t u = 0; u < 4u; ++u) {
                const uint32_t s2 = s0 + 64u * u + lane;
                if (!sz[u] || s2 == s) continue;
                if (p.bfm && !(p.bfm[size_t(q) * p.bP + cl[u]] & 2u)) continue;
                if (sub_relation(bx[u], sa.a, r))
                    np += p.itch ? (t1[u] - t0[u] + p.itch - 1u) / p.itch : 1u;
            }
        }
#pragma unroll
        for (uint32_t o = 32; o; o >>= 1) np += uint32_t(__shfl_xor(int(np), int(o)));
    }
    if (lane == 0) {
#pragma unroll
        for (uint32_t d = 0; d < 4; ++d)
            if (d < sa.a) {
                p.rlo[size_t(d) * p.Q + ci] = r.l[d];
                p.rhi[size_t(d) * p.Q + ci] = r.h[d];
            }
        p.rq[ci] = bf ? q : kEmpty;
        p.rseed[ci] = s;
        if (s != kEmpty) {
            const uint32_t slot = atomicAdd(&p.scnt[s], 1u);
            p.bq[size_t(s) * p.qcap + slot] = q;
        }
        p.nsub[q] = np + (s != kEmpty ? tile_chunks(sa.stile, s, p.tch) : 0u);
    }
}

// One-pass lists with candidate records (after k_bfseed): each sub-cell's
// region of bq gets its inside queries after the seeds and its partial ones
// from the back.  Waves take candidate chunks in turn and claim positions
// with one LDS atomic per chunk and kind (the order inside a list only
// groups queries into items; the brute force's results do not depend on
// it); the next chunk's records load while the current one is tested.
__global__ __launch_bounds__(256) void k_bfsched_direct(BfSchedArgs p) {
    __shared__ uint32_t cnt[2];   // inside, partial
    const SubArgs& sa = p.sa;
    const uint32_t s = blockIdx.x, tid = threadIdx.x, lane = lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid < 2u) cnt[tid] = 0;
    __syncthreads();
    if (sa.ssize[s] != 0 && *p.nbf != 0) {
        const SubBox box = load_box(sa, s);
        const uint32_t cell = sa.scell[s];
        const size_t base = size_t(s) * p.qcap;
        const uint32_t nseed = p.scnt[s];
        const uint32_t nq = p.qrange[1] - p.qrange[0];
        const uint32_t nch = (nq + 63u) / 64u;
        // Four chunks per wave per round: their records load together.
        for (uint32_t c0 = wave; c0 < nch; c0 += 16u) {
            uint32_t rq4[4], rs4[4];
            QRange rr4[4];
#pragma unroll
            for (uint32_t u = 0; u < 4u; ++u) {
                const uint32_t c = c0 + 4u * u;
                const uint32_t ci = ((c + s) % nch) * 64u + lane;
                rq4[u] = kEmpty;
                rs4[u] = kEmpty;
                if (c < nch && ci < nq) {
                    rq4[u] = p.rq[ci];
                    rs4[u] = p.rseed[ci];
#pragma unroll
                    for (uint32_t d = 0; d < 4; ++d)
                        if (d < sa.a) {
                            rr4[u].l[d] = p.rlo[size_t(d) * p.Q + ci];
                            rr4[u].h[d] = p.rhi[size_t(d) * p.Q + ci];
                        }
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < 4u; ++u) {
                if (c0 + 4u * u >= nch) break;
                const uint32_t q = rq4[u], sd = rs4[u];
                const QRange r = rr4[u];
                uint32_t rel = 0;
                if (q != kEmpty && sd != s && (!p.bfm || (p.bfm[size_t(q) * p.bP + cell] & 2u)))
                    rel = sub_relation(box, sa.a, r);
                const uint64_t mi = __builtin_amdgcn_ballot_w64(rel == 2u);
                const uint64_t mp = __builtin_amdgcn_ballot_w64(rel == 1u);
                uint32_t bi = 0, bp = 0;
                if (lane == 0) {
                    if (mi) bi = atomicAdd(&cnt[0], uint32_t(__builtin_popcountll(mi)));
                    if (mp) bp = atomicAdd(&cnt[1], uint32_t(__builtin_popcountll(mp)));
                }
                bi = __builtin_amdgcn_readfirstlane(bi);
                bp = __builtin_amdgcn_readfirstlane(bp);
                if (rel == 2u) p.bq[base + nseed + bi + lanes_below(mi)] = q;
                if (rel == 1u) p.bq[base + p.qcap - 1u - (bp + lanes_below(mp))] = q;
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        p.bcnt[s] = cnt[0] + cnt[1];
        p.bin[s] = cnt[0];
    }
}

__global__ __launch_bounds__(256) void k_bfsched(BfSchedArgs p, bool fill) {
    __shared__ uint32_t wcnt[2][4];
    __shared__ uint32_t fq[kFlushCap];
    const SubArgs& sa = p.sa;
    const uint32_t s = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    if (fill && !*p.ok) return;
    if (sa.ssize[s] == 0 || *p.nbf == 0) {
        if (!fill && tid == 0) { p.bcnt[s] = 0; p.bin[s] = 0; }
        return;
    }
    const SubBox box = load_box(sa, s);
    // direct (qcap > 0): one pass writes the list into the sub-cell's own
    // region of qcap entries, inside queries from its front, partial ones
    // from its back; else the fill pass writes at the scanned offsets.
    const bool direct = p.qcap != 0u;
    const uint32_t base = direct ? s * p.qcap : (fill ? p.bstart[s] : 0u);
    const uint32_t nseed = direct && p.scnt ? p.scnt[s] : 0u;   // seeds hold the front of the region
    const uint32_t nch_s = tile_chunks(sa.stile, s, p.tch);   // items per (query, sub-cell) pair
    // A sub-cell's list holds the queries whose range contains its whole box
    // first (their items skip the range test), then the partial ones.
    const uint32_t nin = fill ? p.bin[s] : 0u;
    uint32_t run_in = 0, run_p = 0, fn = 0;   // fn: queries listed since the last flush (uniform)
    // candidates: every query, or the brute-force queries of the schedule
    const uint32_t q0 = p.qlist ? p.qrange[0] : 0u;
    const uint32_t nq = p.qlist ? p.qrange[1] - q0 : p.Q;
    const uint32_t nch = (nq + 255u) / 256u;
    // With candidate records the next chunk's record is loaded while the
    // current one is tested (one load level, no query-indexed gathers; the
    // barriers order LDS only, so the loads stay in flight).
    const bool recs = p.rq != nullptr;
    uint32_t nx_q = kEmpty, nx_s = kEmpty;
    QRange nx_r{};
    auto fetch = [&](uint32_t ci) {
        const uint32_t qi = ((ci + s) % nch) * 256u + tid;
        nx_q = kEmpty;
        if (qi < nq) {
            nx_q = p.rq[qi];
            nx_s = p.rseed[qi];
#pragma unroll
            for (uint32_t d = 0; d < 4; ++d)
                if (d < sa.a) {
                    nx_r.l[d] = p.rlo[size_t(d) * p.Q + qi];
                    nx_r.h[d] = p.rhi[size_t(d) * p.Q + qi];
                }
        }
    };
    if (recs && nch) fetch(0);
    for (uint32_t ci = 0; ci < nch; ++ci) {
        if (!fill && fn + 256u > kFlushCap) {
            for (uint32_t i = tid; i < fn; i += 256u) atomicAdd(&p.nsub[fq[i]], nch_s);
            lds_barrier();
            fn = 0;
        }
        uint32_t q, rel = 0;
        if (recs) {
            q = nx_q;
            const uint32_t sd = nx_s;
            const QRange r = nx_r;
            if (ci + 1 < nch) fetch(ci + 1);
            if (q != kEmpty && sd != s && (!p.bfm || (p.bfm[size_t(q) * p.bP + sa.scell[s]] & 2u)))
                rel = sub_relation(box, sa.a, r);
        } else {
            const uint32_t qi = ((ci + s) % nch) * 256u + tid;
            q = qi < nq ? (p.qlist ? p.qlist[q0 + qi] : qi) : 0xFFFFFFFFu;
            if (q < p.Q) {
                const uint32_t cnt = p.counts[q], lit = p.little[q];
                const bool trav = cnt < p.postfilter && cnt != lit;
                if (!trav && lit > 0 && (!p.bfm || (p.bfm[size_t(q) * p.bP + sa.scell[s]] & 2u)))
                    rel = sub_relation(box, sa.a, load_range(sa.a, p.lo, p.hi, q));
            }
        }
        const uint64_t mi = __builtin_amdgcn_ballot_w64(rel == 2u);
        const uint64_t mp = __builtin_amdgcn_ballot_w64(rel == 1u);
        if (lane == 0) {
            wcnt[0][wave] = uint32_t(__builtin_popcountll(mi));
            wcnt[1][wave] = uint32_t(__builtin_popcountll(mp));
        }
        lds_barrier();
        uint32_t oi = 0, op = 0, ti = 0, tp = 0;
#pragma unroll
        for (uint32_t w = 0; w < 4; ++w) {
            oi += w < wave ? wcnt[0][w] : 0u;
            op += w < wave ? wcnt[1][w] : 0u;
            ti += wcnt[0][w];
            tp += wcnt[1][w];
        }
        if (rel) {
            if (!fill) fq[fn + (rel == 2u ? oi + lanes_below(mi) : ti + op + lanes_below(mp))] = q;
            if (direct) {
                const uint32_t pos = rel == 2u ? nseed + run_in + oi + lanes_below(mi)
                                               : p.qcap - 1u - (run_p + op + lanes_below(mp));
                p.bq[base + pos] = q;
            } else if (fill) {
                const uint32_t pos = rel == 2u ? run_in + oi + lanes_below(mi) : nin + run_p + op + lanes_below(mp);
                p.bq[base + pos] = q;
            }
        }
        run_in += ti;
        run_p += tp;
        fn += ti + tp;
        lds_barrier();
    }
    if (!fill) {
        for (uint32_t i = tid; i < fn; i += 256u) atomicAdd(&p.nsub[fq[i]], nch_s);
        if (tid == 0) { p.bcnt[s] = run_in + run_p; p.bin[s] = run_in; }
    }
}

// Query schedule on the device, one workgroup: routes (traversal if
// counts < postfilter and counts != little; brute force if otherwise little >
// 0; else empty), a counting sort of the traversal queries by descending cell
// count (order inside one count is arbitrary: it only affects load balance),
// then the brute-force queries.
__global__ __launch_bounds__(1024) void k_sched(SchedArgs p) {
    extern __shared__ uint32_t bins[];   // P + 1 counters, then P + 1 offsets
    __shared__ uint32_t nbf, nempty, bffill;
    const uint32_t tid = threadIdx.x, nb = p.P + 1;
    uint32_t* off = bins + nb;
    for (uint32_t i = tid; i < nb; i += blockDim.x) bins[i] = 0;
    if (tid == 0) { nbf = 0; nempty = 0; bffill = 0; }
    __syncthreads();
    // gpu_graph.cu:3377, 3644: traversal, the full graph (the reference's
    // branch is disabled by `&& false`; here it runs when the index has a
    // full graph), or the brute force over the first little cells
    auto route = [&](uint32_t q) -> uint32_t {
        const uint32_t c = p.counts[q], l = p.little[q];
        if (c < p.postfilter && c != l) return 1u;
        if (p.full && c != l) return 3u;
        return l > 0 ? 2u : 0u;
    };
    __shared__ uint32_t nfull, ffill;
    if (tid == 0) { nfull = 0; ffill = 0; }
    __syncthreads();
    // routes other than the traversal count with one LDS atomic per wave
    // (ballots), not one per query
    const uint32_t lane = lane_id();
    auto wave_add = [&](uint32_t* ctr, bool x) -> uint32_t {
        const uint64_t m = __builtin_amdgcn_ballot_w64(x);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u));
        uint32_t base = 0;
        if (lane == 0 && m) base = atomicAdd(ctr, uint32_t(__builtin_popcountll(m)));
        return uint32_t(__shfl(int(base), 0, 64)) + below;
    };
    for (uint32_t q0 = tid & ~63u; q0 < p.Q; q0 += blockDim.x) {
        const uint32_t q = q0 + lane;
        const uint32_t r = q < p.Q ? route(q) : 4u;
        if (r == 1) atomicAdd(&bins[min(p.counts[q], p.P)], 1u);
        wave_add(&nbf, r == 2);
        wave_add(&nfull, r == 3);
        wave_add(&nempty, r == 0);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        for (uint32_t i = nb; i-- > 0;) { off[i] = acc; acc += bins[i]; bins[i] = 0; }
        p.tot[0] = acc; p.tot[1] = nbf; p.tot[2] = nempty; p.tot[3] = nfull;
        p.ranges[0] = 0; p.ranges[1] = acc; p.ranges[2] = acc; p.ranges[3] = acc + nbf;
        if (p.franges) { p.franges[0] = acc + nbf; p.franges[1] = acc + nbf + nfull; }
    }
    __syncthreads();
    const uint32_t ntrav = p.ranges[1], nfirstf = ntrav + nbf;
    for (uint32_t q0 = tid & ~63u; q0 < p.Q; q0 += blockDim.x) {
        const uint32_t q = q0 + lane;
        const uint32_t r = q < p.Q ? route(q) : 4u;
        if (r == 1) {
            const uint32_t c = min(p.counts[q], p.P);
            p.sched[off[c] + atomicAdd(&bins[c], 1u)] = q;
        }
        const uint32_t sb = wave_add(&bffill, r == 2);
        const uint32_t sf = wave_add(&ffill, r == 3);
        if (r == 2) p.sched[ntrav + sb] = q;
        if (r == 3) p.sched[nfirstf + sf] = q;
    }
}

// Statistics sums (see StatsArgs), one thread per query and per sub-cell.
__global__ __launch_bounds__(256) void k_stats(StatsArgs p) {
    __shared__ unsigned long long acc[11];
    const uint32_t tid = threadIdx.x, i = blockIdx.x * 256u + tid;
    if (tid < 11) acc[tid] = 0;
    __syncthreads();
    uint64_t v[11] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (i < p.Q) {
        const uint32_t* c = p.counters + size_t(i) * GF_NCOUNTERS;
        const uint32_t map[7] = {C_EXPAND, C_DIST, C_ATTR, C_CROSS, C_LROW, C_SCAN, C_PASS};
#pragma unroll
        for (int k = 0; k < 7; ++k) v[k] = c[map[k]];
        if (c[C_ROUTE] == 1 || c[C_ROUTE] == 3 || c[C_ROUTE] == 4) v[7] = c[C_DIST];
        if (c[C_ROUTE] == 2) v[8] = c[C_DIST];
    }
    if (p.bcnt && i < p.NS) {
        const uint32_t ns = p.sseed ? p.sseed[i] : 0u, n = p.bcnt[i] + ns;
        if (n) {
            v[9] = uint64_t(n) * p.ssize[i];
            const uint32_t ni = p.split ? p.bin[i] : 0u;
            const uint32_t nb = (ns + kBfQB - 1) / kBfQB + (ni + kBfQB - 1) / kBfQB +
                                (n - ns - ni + kBfQB - 1) / kBfQB;
            v[10] = uint64_t(nb) * (p.stile[i + 1] - p.stile[i]);
        }
    }
    // sums over the wave, then one LDS atomic per wave and counter
#pragma unroll
    for (int k = 0; k < 11; ++k) {
        uint64_t x = v[k];
#pragma unroll
        for (uint32_t o = 32; o; o >>= 1) {
            const uint32_t lo = uint32_t(__shfl_xor(int(uint32_t(x)), int(o), 64));
            const uint32_t hi = uint32_t(__shfl_xor(int(uint32_t(x >> 32)), int(o), 64));
            x += (uint64_t(hi) << 32) | lo;
        }
        if ((tid & 63u) == 0 && x) atomicAdd(&acc[k], (unsigned long long)x);
    }
    __syncthreads();
    if (tid < 11 && acc[tid]) atomicAdd(&p.out[tid], acc[tid]);
}

// Work items of the MFMA brute force: per sub-cell, its query list in groups
// of 64, times its tiles in chunks of tch (0: one chunk).  Sub-cells are
// taken in the order sorder (identity if null), so the items of its first
// ns1 sub-cells come first: *nitems_a of them.
__global__ __launch_bounds__(256) void k_bfitems(const uint32_t* bcnt, const uint32_t* bin, const uint32_t* bstart,
                                                 uint32_t qcap, const uint32_t* stile, uint32_t tch, uint32_t NS,
                                                 uint32_t* icnt, const uint32_t* ioff, BfItem* items,
                                                 uint32_t* nitems, const uint32_t* ok, bool fill, const uint32_t* scnt,
                                                 BfItem* sitems, uint32_t* nseed, uint32_t scap,
                                                 const uint32_t* sorder, uint32_t ns1, uint32_t* nitems_a,
                                                 uint32_t stch) {
    // one wave per sub-cell; its lanes write the sub-cell's items in parallel
    const uint32_t ks = blockIdx.x * 4u + (threadIdx.x >> 6), lane = lane_id();
    if (ks >= NS) return;
    const uint32_t s = sorder ? sorder[ks] : ks;
    if (fill && !*ok) {
        if (lane == 0 && ks == NS - 1) *nitems = 0;
        if (lane == 0 && nitems_a && ks == 0) *nitems_a = 0;
        return;
    }
    const uint32_t ns = qcap && scnt ? scnt[s] : 0u;   // seeds: the front of the region
    if (fill && ns) {
        // seed items go to their own list (order is free: each is one
        // sub-cell), in chunks of stch tiles, one wave per item (no padding)
        const uint32_t nc = tile_chunks(stile, s, stch), gs = (ns + kBfQB - 1) / kBfQB;
        const uint32_t t0 = stile[s], t1 = stile[s + 1], step = stch ? stch : (t1 - t0);
        uint32_t k0 = 0;
        if (lane == 0) k0 = atomicAdd(nseed, gs * nc);
        k0 = uint32_t(__shfl(int(k0), 0, 64));
        for (uint32_t j = lane; j < gs * nc; j += 64u) {
            const uint32_t c = j / gs, b = j - c * gs, k = k0 + j;
            const uint32_t tb = t0 + c * step, te = min(t1, tb + step);
            if (k < scap) sitems[k] = BfItem{s, s * qcap + b * kBfQB, min(kBfQB, ns - b * kBfQB), tb, te, 0u};
        }
    }
    const uint32_t n = bcnt[s], ni = bin[s];
    // direct lists (qcap > 0): inside and partial queries are separate runs,
    // grouped by 64 each; else one run whose first ni entries are inside
    const uint32_t gi = qcap ? (ni + kBfQB - 1) / kBfQB : 0u;
    const uint32_t gp = qcap ? (n - ni + kBfQB - 1) / kBfQB : (n + kBfQB - 1) / kBfQB;
    const uint32_t nc = n ? tile_chunks(stile, s, tch) : 0u, g = gi + gp;
    if (!fill) {
        if (lane == 0) icnt[ks] = g * nc;
        return;
    }
    const uint32_t t0 = stile[s], t1 = stile[s + 1], step = tch ? tch : (t1 - t0);
    const uint32_t k0 = ioff[ks];
    if (lane == 0 && nitems_a) {
        if (ks + 1 == ns1) *nitems_a = k0 + g * nc;
        else if (ns1 == 0 && ks == 0) *nitems_a = 0;
    }
    // item k0 + c g + b: chunk c of the tiles, group b (inside groups first)
    for (uint32_t j = lane; j < g * nc; j += 64u) {
        const uint32_t c = j / g, b = j - c * g;
        const uint32_t tb = t0 + c * step, te = min(t1, tb + step);
        BfItem it;
        if (qcap) {
            const uint32_t np = n - ni;
            it = b < gi ? BfItem{s, s * qcap + ns + b * kBfQB, min(kBfQB, ni - b * kBfQB), tb, te, 1u}
                        : BfItem{s, s * qcap + qcap - np + (b - gi) * kBfQB, min(kBfQB, np - (b - gi) * kBfQB), tb,
                                 te, 0u};
        } else {
            const uint32_t m = min(kBfQB, n - b * kBfQB);
            it = BfItem{s, bstart[s] + b * kBfQB, m, tb, te, b * kBfQB + m <= ni ? 1u : 0u};
        }
        items[k0 + j] = it;
    }
    if (lane == 0 && ks == NS - 1) *nitems = k0 + g * nc;
}

// out[0] = start[n-1] + cnt[n-1], the total of an exclusive scan; out[1] =
// whether it fits a buffer of cap entries (and, times mul, one of cap2).
__global__ void k_total(const uint32_t* cnt, const uint32_t* start, uint32_t n, uint32_t cap, uint32_t mul,
                        uint64_t cap2, uint32_t* out) {
    if (threadIdx.x != 0) return;
    const uint32_t t = n ? start[n - 1] + cnt[n - 1] : 0u;
    out[0] = t;
    out[1] = (t <= cap && (cap2 == 0 || uint64_t(t) * mul <= cap2)) ? 1u : 0u;
}

// Keeps a streamed batch's brute-force schedule fit flag and pair total
// (tot[3], tot[2]) past the next batch: note[0] = fits, note[1] = pairs.
__global__ void k_note_bf(const uint32_t* tot, uint32_t* note) {
    if (threadIdx.x == 0) {
        note[0] = tot[3];
        note[1] = tot[2];
    }
}

// Per-wave state of the int8 brute force over one work item (a sub-cell's
// tiles and up to 64 of its queries): lane q owns query q of the item, with
// its sorted top-K of (distance << 32 | row) keys in registers, its survivor
// buffer (BUFQ slots) and its accumulator threshold in LDS; B holds the
// item's queries as four 16-query column tiles (a dead column repeats the
// first query; its threshold INT32_MAX and its empty range keep it from
// producing survivors).  A lane
// reserves the buffer slots of its survivors of a tile with one LDS atomic
// per column tile (at most four per tile, issued together).
template <int KS, int AW, int KT, uint32_t BUFQ>
struct BfWave {
    static constexpr uint32_t DRAIN_AT = BUFQ - 15u;   // one tile adds at most 16 per query
    uint64_t* buf;
    uint32_t* cnt;
    int32_t* stp;
    uint32_t lane, col, grp, K;
    bool own_live;
    uint32_t own_q, own_thr, thr0;   // the item's bound, and the query's bound when the item began
    int32_t own_nq;
    uint64_t tk[KT];
    uint64_t kth;
    v4i32_t B[4][KS];
    uint32_t blo[4][AW], bhi[4][AW];
    int32_t tp[4];

    __device__ __forceinline__ void begin(const BfGemmArgs& p, const BfItem& it, uint32_t cell) {
        const SubArgs& sa = p.sa;
        own_live = lane < it.nq;
        own_q = p.bq[it.qbase + (own_live ? lane : 0u)];
        own_nq = p.nq[own_q];
        own_thr = own_live ? __hip_atomic_load(&p.gbound[own_q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        thr0 = own_thr;
#pragma unroll
        for (int k = 0; k < KT; ++k) tk[k] = kKeySent;
        kth = kKeySent;
        wave_fence();
        cnt[lane] = 0;
        stp[lane] = own_live ? acc_threshold(own_nq, own_thr) : INT32_MAX;
        // the owner's packed range bounds, then each column lane takes
        // those of its four queries (owner lane 16 j + col)
        uint32_t lw[AW], hw[AW];
#pragma unroll
        for (int w = 0; w < AW; ++w) {
            uint32_t l0 = 65534u, h0 = 65534u, l1 = 0u, h1 = 0u;
            if (own_live) {
                const uint32_t d0 = 2u * w, d1 = 2u * w + 1u;
                range16(p.lo[size_t(own_q) * sa.a + d0], p.hi[size_t(own_q) * sa.a + d0],
                        sa.abase[cell * sa.a + d0], l0, h0);
                if (d1 < sa.a)
                    range16(p.lo[size_t(own_q) * sa.a + d1], p.hi[size_t(own_q) * sa.a + d1],
                            sa.abase[cell * sa.a + d1], l1, h1);
            }
            lw[w] = l0 | (l1 << 16);
            hw[w] = h0 | (h1 << 16);
        }
        wave_fence();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t ql = 16u * j + col;
            const uint32_t q = p.bq[it.qbase + (ql < it.nq ? ql : 0u)];
#pragma unroll
            for (int k = 0; k < KS; ++k)
                B[j][k] = *reinterpret_cast<const v4i32_t*>(p.q8 + size_t(q) * p.D + k * 64 + grp * 16);
#pragma unroll
            for (int w = 0; w < AW; ++w) {
                blo[j][w] = uint32_t(__shfl(int(lw[w]), int(ql), 64));
                bhi[j][w] = uint32_t(__shfl(int(hw[w]), int(ql), 64));
            }
            tp[j] = stp[ql];
        }
    }

    __device__ __forceinline__ void reload_tp() {
#pragma unroll
        for (int j = 0; j < 4; ++j) tp[j] = stp[16u * j + col];
    }
    // Owner: merge the buffered survivors of its query, publish the new
    // threshold and lower the query's bound.
    __device__ __forceinline__ void drain() {
        wave_fence();
        const uint32_t n = cnt[lane];
        if (n) {
            uint64_t nxt = buf[lane * BUFQ];
            for (uint32_t e = 0; e < n; ++e) {
                const uint64_t cur = nxt;
                if (e + 1 < n) nxt = buf[lane * BUFQ + e + 1];
                const int32_t d = own_nq + int32_t(uint32_t(cur >> 32));
                uint64_t c = (uint64_t(uint32_t(d)) << 32) | uint32_t(cur);
                if (c < kth) {
#pragma unroll
                    for (int k = 0; k < KT; ++k) {
                        const bool lt = c < tk[k];
                        const uint64_t v = tk[k];
                        tk[k] = lt ? c : v;
                        c = lt ? v : c;
                    }
                    // the K-th key (a move when K is the template's KT)
                    if (K == uint32_t(KT)) {
                        kth = tk[KT - 1];
                    } else {
#pragma unroll
                        for (int k = 0; k < KT; ++k)
                            if (uint32_t(k) == K - 1) kth = tk[k];
                    }
                }
            }
            cnt[lane] = 0;
            if (kth != kKeySent && uint32_t(kth >> 32) < own_thr) {
                own_thr = uint32_t(kth >> 32);
                stp[lane] = acc_threshold(own_nq, own_thr);
            }
        }
        wave_fence();
        reload_tp();
    }
    // One tile: A (KS k-steps) and mh (-floor(|x'|^2 / 2) of the lane's four
    // points) as operands; meta(mn, mr, ma) fetches the tile's |x'|^2, rows
    // and attribute words for the lane's points when some pair is within its
    // threshold (about two of a tile's 1024 pairs once thresholds settle).
    __device__ __forceinline__ void mma(const v4i32_t (&A)[KS], const v4i32_t& mh, v4i32_t (&acc)[4]) const {
        // k-outer: the four column tiles' MFMAs are independent, so a
        // dependent MFMA (same accumulator) issues three MFMAs later
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B[j][0], mh, 0, 0, 0);
#pragma unroll
        for (int k = 1; k < KS; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[k], B[j][k], acc[j], 0, 0, 0);
    }
    // RANGE false: every query of the item contains the sub-cell's box, so
    // every point is in range and only the distance test runs (padding and
    // dead columns still fail it: their accumulator is INT32_MIN, their
    // threshold INT32_MAX).
    template <bool RANGE, class Meta>
    __device__ __forceinline__ void epilogue(const v4i32_t (&acc)[4], const v4i32_t& mh, Meta meta) {
        // Distance first, on the max of each column tile's four rows: jm
        // has bit j when some lane holds a pair of column tile j within its
        // query's threshold (about two of a tile's 1024 pairs once settled,
        // often failing the range test).
        uint32_t jm = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            jm |= __builtin_amdgcn_ballot_w64(max(max(acc[j][0], acc[j][1]), max(acc[j][2], acc[j][3])) >= tp[j])
                      ? 1u << j : 0u;
        if (!jm) return;
        v4i32_t mn, mr, ma[AW];
        meta(mn, mr, ma);
        bool full = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (!(jm & (1u << j))) continue;
            // pairs (j, i) of this lane within the threshold and the range
            uint32_t okm = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                bool ok = acc[j][i] >= tp[j];
                if constexpr (RANGE) {
                    const uint32_t x0 = uint32_t(ma[0][i]);
                    ok &= clamp16(x0, blo[j][0], bhi[j][0]) == x0;
                    if (AW > 1) {
                        const uint32_t x1 = uint32_t(ma[AW - 1][i]);
                        ok &= clamp16(x1, blo[j][AW - 1], bhi[j][AW - 1]) == x1;
                    }
                }
                okm |= ok ? 1u << i : 0u;
            }
            if (!__builtin_amdgcn_ballot_w64(okm != 0u)) continue;
            // one LDS atomic reserves this lane's slots; the lane holding
            // the last reservation sees the query's new count
            const uint32_t ql = 16u * j + col;
            uint32_t slot = okm ? atomicAdd(&cnt[ql], uint32_t(__builtin_popcount(okm))) : 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (okm & (1u << i)) {
                    // the owner adds |q'|^2 to |x'|^2 - 2 q'.x' later
                    const int32_t v = mn[i] - 2 * (acc[j][i] - mh[i]);
                    buf[ql * BUFQ + slot++] = (uint64_t(uint32_t(v)) << 32) | uint32_t(mr[i]);
                }
            full |= okm && slot >= DRAIN_AT;
        }
        if (__builtin_amdgcn_ballot_w64(full)) drain();
    }
    // End of the item: lower the query's global bound (read at the item's
    // start: a store inside the tile loop would make the compiler wait for
    // every load in flight before the next tile's operands) if the item
    // improved on it, and append the keys within it for the final merge.
    __device__ __forceinline__ void finish(const BfGemmArgs& p) {
        drain();
        if (!own_live) return;
        const bool lower = own_thr < thr0;
        if (lower) atomicMin(&p.gbound[own_q], own_thr);
        uint32_t keep = 0;
#pragma unroll
        for (int k = 0; k < KT; ++k)
            keep += (uint32_t(k) < K && tk[k] != kKeySent && uint32_t(tk[k] >> 32) <= own_thr) ? 1u : 0u;
        if (keep) {
            const size_t slot = size_t(p.part_off[own_q]) * K + atomicAdd(&p.pcnt[own_q], keep);
#pragma unroll
            for (int k = 0; k < KT; ++k)
                if (uint32_t(k) < keep) p.part[slot + k] = tk[k];
        }
    }
};

// The MFMA kernel, one wave per item: the seed items (seeds_on), then the
// launch's range of the item list (irange).  Persistent
// waves, XCD-aware: workgroups go round-robin to the 8 XCDs and XCD x works
// through the x-th eighth of the item list (items of one sub-cell are
// adjacent, so its tiles stay in that XCD's L2).  The operands of tile t + 1
// are loaded while tile t is computed: the int8 k-steps after tile t's MFMAs
// have read them, its norms and meta into the other of two register sets.
template <int KS, int AW, int KT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(AW == 1 && KS <= 2 && KT <= 10 ? 3 : 2))) void k_bf_i8(BfGemmArgs p) {
    stamp_entry(p.stamp, 1);
    __shared__ uint64_t s_buf[4][kQB * kBfBufQ];
    __shared__ uint32_t s_cnt[4][kQB];
    __shared__ int32_t s_tp[4][kQB];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    const SubArgs& sa = p.sa;
    const uint32_t RB = bf_rec_bytes(p.D, AW), KB = KS * 1024u;
    BfWave<KS, AW, KT, kBfBufQ> w;
    w.buf = s_buf[wave]; w.cnt = s_cnt[wave]; w.stp = s_tp[wave];
    w.lane = lane; w.col = lane & 15u; w.grp = lane >> 4; w.K = p.K;
    const uint32_t n_seed = p.sitems && *p.ok && p.seeds_on ? min(*p.nseed, p.nseed_cap) : 0u;
    const uint32_t nwg = gridDim.x, xcd = blockIdx.x & 7u, k8 = blockIdx.x >> 3;
    const uint32_t nwg_x = (nwg - xcd + 7u) >> 3;
    uint32_t i_b = 0, i_e = *p.ok && p.irange != 3u ? *p.nitems : 0u;
    if (p.irange == 1u) i_e = min(i_e, *p.nitems_a);
    if (p.irange == 2u) i_b = min(i_e, *p.nitems_a);
    const uint32_t n_items = i_e - i_b;
    const uint32_t i_lo = i_b + uint32_t(uint64_t(n_items) * xcd / 8u);
    const uint32_t i_hi = i_b + uint32_t(uint64_t(n_items) * (xcd + 1u) / 8u);
    uint32_t seed_id = blockIdx.x * 4u + wave, item_id = i_lo + k8 * 4u + wave;
    for (;;) {
        BfItem it;
        if (seed_id < n_seed) {
            it = p.sitems[seed_id];
            seed_id += nwg * 4u;
        } else if (item_id < i_hi) {
            it = p.items[item_id];
            item_id += nwg_x * 4u;
        } else {
            break;
        }
        const uint32_t t0 = it.tb, t1 = it.te, ntile = t1 - t0;
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(p.rec + size_t(t0) * RB), 0, ntile * RB, 0x00020000);
        struct TileMeta {
            v4i32_t mh, mn, mr, ma[AW];
        };
        v4i32_t A[KS];
        auto bload = [&](uint32_t voff, uint32_t soff) __attribute__((always_inline)) {
            return __builtin_bit_cast(v4i32_t, __builtin_amdgcn_raw_buffer_load_b128(rr, int(voff), int(soff), 0));
        };
        auto load_a = [&](uint32_t t) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < KS; ++k) A[k] = bload(lane * 16u, (t - t0) * RB + k * 1024u);
        };
        // the tile loop, with the range test (rg true) or without it (an
        // inside item: its attribute words are not even loaded)
        auto run = [&](auto rg) __attribute__((always_inline)) {
            constexpr bool RANGE = decltype(rg)::value;
            auto load_m = [&](TileMeta& M, uint32_t t) __attribute__((always_inline)) {
                const uint32_t o = (t - t0) * RB + KB;
                M.mh = bload(16u * w.grp, o);
                M.mn = bload(16u * w.grp, o + 64u);
                M.mr = bload(16u * w.grp, o + 128u);
                if constexpr (RANGE) {
#pragma unroll
                    for (int a = 0; a < AW; ++a) M.ma[a] = bload(16u * w.grp, o + 128u + 64u * (1 + a));
                }
            };
            auto step = [&](const TileMeta& M, TileMeta& Mn, uint32_t t) __attribute__((always_inline)) {
                v4i32_t acc[4];
                w.mma(A, M.mh, acc);
                if (t + 1 < t1) {
                    load_a(t + 1);
                    load_m(Mn, t + 1);
                }
                w.template epilogue<RANGE>(
                    acc, M.mh, [&](v4i32_t& mn, v4i32_t& mr, v4i32_t (&ma)[AW]) __attribute__((always_inline)) {
                        mn = M.mn;
                        mr = M.mr;
                        if constexpr (RANGE) {
#pragma unroll
                            for (int a = 0; a < AW; ++a) ma[a] = M.ma[a];
                        }
                    });
            };
            // the first tile's loads fly while the item's queries load
            TileMeta M0, M1;
            load_a(t0);
            load_m(M0, t0);
            w.begin(p, it, sa.scell[it.sub]);
            for (uint32_t t = t0; t < t1; t += 2) {
                step(M0, M1, t);
                if (t + 1 >= t1) break;
                step(M1, M0, t + 1);
            }
        };
        if (__builtin_amdgcn_readfirstlane(it.inside)) run(std::false_type{});
        else run(std::true_type{});
        w.finish(p);
    }
}

// ------------------------------------------- fp16 query-batch brute force
// Brute force of binary16 rows for a batch of queries on fp16 MFMA
// (v_mfma_f32_16x16x32_f16).  Items and sub-cell tiles are k_bf_i8's; a
// workgroup takes an item, each of its four waves 16 of the item's queries
// (queries as the B operand, D / 32 k-steps held in registers), and streams
// the sub-cell's tiles, 16 rows each, through LDS as the A operand of all
// four, gathered once from the cell-major rows.  The MFMA distance
// d' = |q|^2 + |x|^2 - 2 q.x differs from the canonical fp32 distance d by at
// most eps_q (a bound from the fp32 error of both), so every point whose d
// is among the K smallest has d' within the query's smallest K-th d' plus
// 2 eps_q; k_bf_f16_final re-ranks exactly the keys within that limit.  Per
// item a query keeps its 32 smallest keys (in registers, 8 in each of the
// four lanes of its column); if all 32 lie within min(bound, the item's
// K-th) plus 2 eps_q, keys may have been dropped, and the query is flagged
// for an exact scan.
// Operand chunks of the two row types.  Binary16 rows (VT 1): a chunk is
// one v_mfma_f32_16x16x32_f16 k-step, 8 halves per lane (lane group g holds
// dims 32 c + 8 g .. + 8).  fp32 rows (VT 0): a chunk is four
// v_mfma_f32_16x16x4_f32 k-steps, 4 floats per lane; lane group g supplies
// k-slot g, so it holds dims g D/4 + 4 c .. + 4 (a permutation of the dims,
// the same for rows and queries, which the dot product does not see).
template <int VT> struct BfChunk;
template <> struct BfChunk<1> {
    typedef half8_t T;
    typedef uint16_t E;
    static __device__ __forceinline__ const E* at(const E* row, uint32_t D, uint32_t g, int c) {
        return row + c * 32 + g * 8u;
    }
    static __device__ __forceinline__ float4_t mma(const T& a, const T& b, float4_t acc) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
};
template <> struct BfChunk<0> {
    typedef float4_t T;
    typedef float E;
    static __device__ __forceinline__ const E* at(const E* row, uint32_t D, uint32_t g, int c) {
        return row + g * (D / 4u) + c * 4;
    }
    static __device__ __forceinline__ float4_t mma(const T& a, const T& b, float4_t acc) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
        return acc;
    }
};

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(uintptr_t((const __attribute__((address_space(3))) void*)p));
}
// Asynchronous global-to-LDS copies: 16 (4) bytes per active lane from src to
// LDS at lds_base + 16 (4) x lane, lds_base wave-uniform (in m0).  They count
// in vmcnt and the compiler does not see them: the caller waits
// (wait_vmcnt) and synchronises before the data is read.
__device__ __forceinline__ void lds_copy16(const void* src, uint32_t lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}
__device__ __forceinline__ void lds_copy4(const void* src, uint32_t lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}
// s_waitcnt vmcnt(N), the other counters unconstrained (gfx9 encoding).
template <uint32_t N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64u, "vmcnt");
    __builtin_amdgcn_s_waitcnt(int((N & 15u) | ((N >> 4) << 14) | (7u << 4) | (15u << 8)));
}

template <int VT, int KS, int AW>
__device__ void bf_float_items(const BfHArgs& p) {
    typedef BfChunk<VT> CH;
    typedef typename CH::T ChunkT;
    typedef typename CH::E ElemT;
    static_assert(sizeof(ChunkT) == 16, "16-byte operand chunks");
    // A workgroup takes an item; wave w takes its queries 16 w .. 16 w + 15.
    // The sub-cell's tile records (bf_frec_bytes: operand chunks in MFMA
    // operand order, chunk k = 64 lanes x 16 bytes, lane l holding row
    // l % 16's dims of lane group l / 16; then the meta record and the
    // rows' norms) pass through LDS once for all of them, each copied whole
    // by asynchronous global-to-LDS loads a tile ahead into a double buffer
    // (a third buffer, two tiles ahead, measured slower: it leaves room for
    // one workgroup per CU instead of two); each wave reads its A operands
    // and the epilogue's data from there.
    constexpr uint32_t NSLOT = uint32_t(KS) * 64u;
    constexpr uint32_t NL = (NSLOT + 255u) / 256u;    // 16-byte copies per thread per tile
    constexpr uint32_t MW = 16u * (1u + AW);
    constexpr uint32_t NTAIL = (MW + 16u) / 4u;       // 16-byte chunks of meta record and norms
    constexpr uint32_t RB = uint32_t(KS) * 1024u + 64u * (2u + AW);
    static_assert(RB == NSLOT * 16u + NTAIL * 16u, "record layout");
    __shared__ uint4 s_tile[2][NSLOT];
    __shared__ uint32_t s_tail[2][MW + 16u];   // meta words, then the norms
    // Per-owner survivor buffers padded by one key, so that the 16 owners'
    // buffers start on different LDS banks (the drain reads all 16 at once).
    constexpr uint32_t BQ = kBfBufQ + 1u;
    static_assert(kBfHKT == 32u, "kept keys: 8 per lane of the owner's 4 lanes");
    __shared__ uint64_t s_buf[4][16 * BQ];
    __shared__ uint32_t s_cnt[4][16];
    __shared__ float s_tp[4][16];
    __shared__ uint32_t s_bnd[4][2 * AW][16];
    const ElemT* qrows = reinterpret_cast<const ElemT*>(p.q16);
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = lane_id();
    const SubArgs& sa = p.sa;
    const uint32_t nwg = gridDim.x, xcd = blockIdx.x & 7u, k8 = blockIdx.x >> 3;
    const uint32_t nwg_x = (nwg - xcd + 7u) >> 3;
    uint32_t i_b = 0, i_e = *p.ok && p.irange != 3u ? *p.nitems : 0u;
    if (p.irange == 1u) i_e = min(i_e, *p.nitems_a);
    if (p.irange == 2u) i_b = min(i_e, *p.nitems_a);
    const uint32_t i_lo = i_b + uint32_t(uint64_t(i_e - i_b) * xcd / 8u);
    const uint32_t i_hi = i_b + uint32_t(uint64_t(i_e - i_b) * (xcd + 1u) / 8u);
    uint64_t* buf = s_buf[wave];
    uint32_t* cnt = s_cnt[wave];
    float* stp = s_tp[wave];
    const uint32_t K = p.K;
    const uint32_t col = lane & 15u, grp = lane >> 4;
    const float kInf = __int_as_float(0x7F800000);
    const uint32_t n_seed = p.sitems && *p.ok && p.seeds_on ? min(*p.nseed, p.nseed_cap) : 0u;
    uint32_t seed_id = blockIdx.x, item_id = i_lo + k8;
    for (;;) {
        BfItem it;
        if (seed_id < n_seed) {
            it = p.sitems[seed_id];
            seed_id += nwg;
        } else if (item_id < i_hi) {
            it = p.items[item_id];
            item_id += nwg_x;
        } else {
            break;
        }
        const uint32_t cell = sa.scell[it.sub];
        const uint32_t qb = 16u * wave;
        const uint32_t nqb = it.nq > qb ? min(16u, it.nq - qb) : 0u;   // wave-uniform
        // Owner state: lane < nqb owns query qb + lane.  Its kept keys
        // (d' << 32 | row, ascending, kBfHKT of them) are spread over the
        // four lanes of its column: lane col + 16 g holds keys 8 g .. 8 g + 7.
        const bool own_live = lane < nqb;
        const uint32_t own_q = own_live ? p.bq[it.qbase + qb + lane] : 0u;
        const float own_eps2 = own_live ? 2.0f * p.eps[own_q] : 0.0f;
        const uint32_t gb =
            own_live ? __hip_atomic_load(&p.gbound[own_q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0xFFFFFFFFu;
        const float own_bnd = gb == 0xFFFFFFFFu ? kInf : __uint_as_float(gb);
        uint64_t tk[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) tk[k] = kKeySent;
        float kth = kInf;
        if (nqb) {
            wave_fence();
            if (lane < 16u) {
                cnt[lane] = 0;
                stp[lane] = own_live ? own_bnd + own_eps2 : -1.0f;
            }
#pragma unroll
            for (int w = 0; w < AW; ++w) {
                uint32_t l0 = 65534u, h0 = 65534u, l1 = 0u, h1 = 0u;
                if (own_live) {
                    const uint32_t d0 = 2u * w, d1 = 2u * w + 1u;
                    range16(p.lo[size_t(own_q) * sa.a + d0], p.hi[size_t(own_q) * sa.a + d0],
                            sa.abase[cell * sa.a + d0], l0, h0);
                    if (d1 < sa.a)
                        range16(p.lo[size_t(own_q) * sa.a + d1], p.hi[size_t(own_q) * sa.a + d1],
                                sa.abase[cell * sa.a + d1], l1, h1);
                }
                if (lane < 16u) {
                    s_bnd[wave][2 * w][lane] = l0 | (l1 << 16);
                    s_bnd[wave][2 * w + 1][lane] = h0 | (h1 << 16);
                }
            }
            wave_fence();
        }
        // Column data: query qb + col (a dead column repeats the wave's
        // first query, or the item's; its threshold -1 keeps it from
        // producing survivors).
        const uint32_t qc = p.bq[it.qbase + (nqb ? qb + (col < nqb ? col : 0u) : 0u)];
        ChunkT B[KS];
        if (nqb) {
#pragma unroll
            for (int k = 0; k < KS; ++k)
                B[k] = *reinterpret_cast<const ChunkT*>(CH::at(qrows + size_t(qc) * p.D, p.D, grp, k));
        }
        const float qn = p.qnorm[qc];
        uint32_t blo[AW], bhi[AW];
#pragma unroll
        for (int w = 0; w < AW; ++w) {
            blo[w] = nqb ? s_bnd[wave][2 * w][col] : 0u;
            bhi[w] = nqb ? s_bnd[wave][2 * w + 1][col] : 0u;
        }
        float tp = nqb ? stp[col] : -1.0f;
        // Insert the buffered survivors of every column's query into its
        // kept keys, and the owner publishes the new threshold
        // min(bound, K-th) + 2 eps.  A cascade over the column's four
        // lanes: at step s lane col + 16 g inserts into its 8 keys what lane
        // col + 16 (g - 1) pushed out at step s - 1 (lane col: the buffer's
        // entry s), and pushes out its largest; what the last lane pushes
        // out is dropped.  Each segment sees the entries in buffer order, so
        // the result is the sequential insertion's: the kBfHKT smallest.
        auto drain = [&]() {
            wave_fence();
            const uint32_t n = cnt[col];
            uint32_t nm = n;
#pragma unroll
            for (uint32_t o = 1; o < 16u; o <<= 1) nm = max(nm, uint32_t(__shfl_xor(int(nm), int(o), 64)));
            nm = __builtin_amdgcn_readfirstlane(nm);
            uint64_t pass = kKeySent;
            uint64_t nxt = grp == 0u && n ? buf[col * BQ] : kKeySent;
            for (uint32_t st = 0; st < nm + 3u; ++st) {
                uint64_t c = grp == 0u ? nxt : pass;
                if (grp == 0u) nxt = st + 1u < n ? buf[col * BQ + st + 1u] : kKeySent;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const bool lt = c < tk[k];
                    const uint64_t v = tk[k];
                    tk[k] = lt ? c : v;
                    c = lt ? v : c;
                }
                pass = shfl64(c, (lane - 16u) & 63u);
            }
            // the K-th key: key K - 1 of the column, in lane col + 16 ((K - 1) / 8)
            uint64_t kl = tk[0];
#pragma unroll
            for (int k = 1; k < 8; ++k)
                if (uint32_t(k) == ((K - 1u) & 7u)) kl = tk[k];
            const uint64_t kk = shfl64(kl, col + 16u * ((K - 1u) >> 3));
            wave_fence();
            if (lane < 16u) {
                cnt[lane] = 0;
                if (kk != kKeySent) kth = __uint_as_float(uint32_t(kk >> 32));
                if (own_live) stp[lane] = fminf(own_bnd, kth) + own_eps2;
            }
            wave_fence();
            tp = stp[col];
        };
        // Copy tile t's record into LDS buffer b: thread tid its 16-byte
        // chunks j * 256 + tid of the operand (chunk 4 j + wave: a
        // wave-uniform bound), wave 0 the meta record and norms.
        auto stage = [&](uint32_t t, uint32_t b) {
            const uint8_t* src = p.rec + size_t(t) * RB;
#pragma unroll
            for (uint32_t j = 0; j < NL; ++j)
                if (j * 4u + wave < uint32_t(KS))
                    lds_copy16(src + (j * 256u + tid) * 16u,
                               __builtin_amdgcn_readfirstlane(lds_addr(&s_tile[b][j * 256u + wave * 64u])));
            if (wave == 0 && lane < NTAIL) lds_copy16(src + NSLOT * 16u + lane * 16u, lds_addr(&s_tail[b][0]));
        };
        if (it.tb < it.te) stage(it.tb, 0);
        wait_vmcnt<0>();
        __syncthreads();
        for (uint32_t t = it.tb; t < it.te; ++t) {
            const uint32_t cur = (t - it.tb) & 1u;
            if (t + 1 < it.te) stage(t + 1, cur ^ 1u);
            if (nqb) {
                float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k = 0; k < KS; ++k)
                    acc = CH::mma(*reinterpret_cast<const ChunkT*>(&s_tile[cur][uint32_t(k) * 64u + lane]), B[k], acc);
                const uint32_t* meta = s_tail[cur];
                bool full = false;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // point 4 grp + i, query column col
                    const uint32_t mr = meta[4u * grp + i];
                    const float xn = __uint_as_float(meta[MW + 4u * grp + i]);
                    const float d = fmaxf(__fsub_rn(__fadd_rn(qn, xn), __fmul_rn(2.0f, acc[i])), 0.0f);
                    bool ok = d <= tp && mr != kEmpty;
                    if (!__builtin_amdgcn_ballot_w64(ok)) continue;
                    if (!it.inside) {
#pragma unroll
                        for (int w = 0; w < AW; ++w) {
                            const uint32_t x = meta[16u * (1u + w) + 4u * grp + i];
                            ok &= clamp16(x, blo[w], bhi[w]) == x;
                        }
                    }
                    if (ok) {
                        const uint32_t slot = atomicAdd(&cnt[col], 1u);
                        buf[col * BQ + slot] = (uint64_t(__float_as_uint(d)) << 32) | mr;
                        full |= slot + 1u >= kBfDrainAt;
                    }
                }
                if (__builtin_amdgcn_ballot_w64(full)) drain();
            }
            wait_vmcnt<0>();
            __syncthreads();
        }
        if (nqb) {
            drain();
            // Keys within the query's limit (a prefix of the ascending
            // keys: the lane's count is 8 in the segments before the last
            // one that has any); if all kBfHKT are within it, keys beyond
            // may have been dropped.
            const float lim = __shfl(fminf(own_bnd, kth) + own_eps2, int(col), 64);
            uint32_t kseg = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                kseg += tk[k] != kKeySent && __uint_as_float(uint32_t(tk[k] >> 32)) <= lim ? 1u : 0u;
            uint32_t keep = kseg + uint32_t(__shfl_xor(int(kseg), 16, 64));
            keep += uint32_t(__shfl_xor(int(keep), 32, 64));
            uint64_t base = 0;
            if (own_live) {
                if (kth != kInf) atomicMin(&p.gbound[own_q], __float_as_uint(kth));
                if (keep == kBfHKT) p.over[own_q] = 1u;
                if (keep) base = uint64_t(p.part_off[own_q]) * kBfHKT + atomicAdd(&p.pcnt[own_q], keep);
            }
            base = shfl64(base, col);
            if (col < nqb) {
                uint64_t* dst = p.part + base + 8u * grp;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (uint32_t(k) < kseg) dst[k] = tk[k];
            }
            wave_fence();
        }
    }
}

// Float tile records (bf_frec_bytes) for the float MFMA brute force: one
// wave per tile copies its 16 rows' operand chunks into MFMA operand order
// (BfChunk<VT>::at), then the meta record and the rows' norms; an empty slot
// (row kEmpty) gets zero operands and norm.
template <int VT>
__global__ __launch_bounds__(64) void k_tile_frec(const void* vec, uint32_t D, const uint32_t* tmeta,
                                                  const float* xnorm, uint32_t AW, uint8_t* rec) {
    typedef BfChunk<VT> CH;
    typedef typename CH::E ElemT;
    const uint32_t t = blockIdx.x, lane = lane_id();
    const uint32_t KS = VT == 1 ? D / 32u : D / 16u, MW = 16u * (1u + AW);
    uint8_t* dst = rec + size_t(t) * bf_frec_bytes(KS, AW);
    const uint32_t row = tmeta[size_t(t) * MW + (lane & 15u)];
    const ElemT* src = reinterpret_cast<const ElemT*>(vec) + size_t(row == kEmpty ? 0u : row) * D;
    for (uint32_t k = 0; k < KS; ++k) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (row != kEmpty) v = *reinterpret_cast<const uint4*>(CH::at(src, D, lane >> 4, int(k)));
        *reinterpret_cast<uint4*>(dst + k * 1024u + lane * 16u) = v;
    }
    uint32_t* tail = reinterpret_cast<uint32_t*>(dst + KS * 1024u);
    for (uint32_t w = lane; w < MW; w += 64u) tail[w] = tmeta[size_t(t) * MW + w];
    if (lane < 16u) tail[MW + lane] = row != kEmpty ? __float_as_uint(xnorm[row]) : 0u;
}

template <int KS, int AW>
__global__ __launch_bounds__(256) void k_bf_f16(BfHArgs p) {
    bf_float_items<1, KS, AW>(p);
}
template <int KS, int AW>
__global__ __launch_bounds__(256) void k_bf_f32(BfHArgs p) {
    bf_float_items<0, KS, AW>(p);
}

// Per query of the fp16 brute force: the K-th smallest d' of the keys its
// items kept, then the exact (canonical) distances of the keys within that
// plus 2 eps, ranked by (distance, row).  A flagged query is scanned exactly.
template <int VT, int LPR, int CPL>
__global__ __launch_bounds__(64) void k_bf_f16_final(TravArgs p, BfHFinal f) {
    __shared__ uint32_t S[64 * 4 + 64];
    __shared__ uint64_t T[64];
    const uint32_t lane = lane_id();
    if (!*f.ok) return;
    const uint32_t si = p.srange[0] + blockIdx.x;
    if (si >= p.srange[1]) return;
    const uint32_t q = p.sched[si];
    if (f.over[q]) {
        bf_scan_query<VT, LPR, CPL>(p, q, S, T);
        return;
    }
    const uint32_t K = p.K;
    const uint32_t n = f.pcnt[q];
    const uint64_t* part = f.part + size_t(f.part_off[q]) * kBfHKT;
    // K-th smallest key (a running top-K over chunks of 64)
    uint64_t top = kKeySent;
    for (uint32_t s0 = 0; s0 < n; s0 += 64u) {
        const uint64_t c = s0 + lane < n ? part[s0 + lane] : kKeySent;
        const bool surv = c < readlane64(top, K - 1);
        const uint64_t sm = ballot(surv);
        if (!sm) continue;
        uint32_t rs = 0, rt = lane;
        // ranks in the merged order, ties to the top entry, then to the
        // lower lane: a permutation even if a key repeats
        for (uint64_t m = sm; m; m &= m - 1) {
            const uint32_t j = __builtin_ctzll(m);
            const uint64_t kk = readlane64(c, j);
            rs += kk < c || (kk == c && j < lane);
            rt += kk < top;
        }
        for (uint32_t t = 0; t < K; ++t) rs += readlane64(top, t) <= c;
        wave_sync();
        if (surv && rs < K) T[rs] = c;
        if (lane < K && rt < K) T[rt] = top;
        wave_sync();
        top = lane < K ? T[lane] : kKeySent;
        wave_sync();
    }
    const uint64_t kk = readlane64(top, K - 1);
    const float lim = kk == kKeySent ? __int_as_float(0x7F800000)
                                     : __uint_as_float(uint32_t(kk >> 32)) + 2.0f * f.eps[q];
    QReg<VT, LPR, CPL> qv;
    load_query<VT, LPR, CPL>(qv, p.queries + size_t(q) * p.qbytes, p.nch);
    uint64_t best = kCandSent;
    uint32_t ncand = 0;
    for (uint32_t s0 = 0; s0 < n; s0 += 64u) {
        const uint64_t c = s0 + lane < n ? part[s0 + lane] : kKeySent;
        const bool in = c != kKeySent && __uint_as_float(uint32_t(c >> 32)) <= lim;
        const uint64_t m = ballot(in);
        wave_sync();
        if (in) S[lanes_below(m)] = uint32_t(c);
        wave_sync();
        const uint32_t nb = __popcll(m);
        if (nb) bf_flush<VT, LPR, CPL>(qv, p, S, nb, best, T);
        ncand += nb;
    }
    if (lane < K) {
        p.out_ids[size_t(q) * K + lane] = cvalid(best) ? p.gidx[crow(best)] : GF_NO_RESULT;
        p.out_dist[size_t(q) * K + lane] = cdist(best);
    }
    uint32_t scan = 0;
    for (uint32_t i = lane; i < p.little[q]; i += 64u) {
        const uint32_t c = p.cells[size_t(q) * p.P + i];
        scan += p.offset[c + 1] - p.offset[c];
    }
#pragma unroll
    for (uint32_t o = 32; o; o >>= 1) scan += uint32_t(__shfl_xor(int(scan), int(o)));
    if (lane == 0) {
        uint32_t* ctr = p.counters + size_t(q) * GF_NCOUNTERS;
        ctr[C_EXPAND] = 0;
        ctr[C_DIST] = ncand;
        ctr[C_ATTR] = 0;
        ctr[C_CROSS] = 0;
        ctr[C_LROW] = 0;
        ctr[C_SCAN] = scan;
        ctr[C_PASS] = f.selcount[q];
        ctr[C_ROUTE] = 2;
    }
}

// Per-query merge of the keys the brute-force items appended for the query.
__global__ __launch_bounds__(64) void k_bf_final(BfFinalArgs p) {
    stamp_entry(p.stamp, 1);
    __shared__ uint64_t T[64];
    const uint32_t lane = lane_id();
    if (!*p.ok) return;
    const uint32_t si = p.srange[0] + blockIdx.x;
    if (si >= p.srange[1]) return;
    const uint32_t q = p.bfq[si];
    const uint32_t K = p.K;
    const uint32_t n = p.pcnt[q];
    uint64_t* part = p.part + size_t(p.part_off[q]) * K;
    // The query's final bound: some item held K keys within it, so no key
    // beyond it reaches the top K.
    const uint32_t g = p.gbound ? p.gbound[q] : 0xFFFFFFFFu;
    const uint64_t cap = g == 0xFFFFFFFFu ? kKeySent : (uint64_t(g) + 1u) << 32;
    uint64_t top = kKeySent;
    for (uint32_t s0 = 0; s0 < n; s0 += 64u) {
        const uint64_t c = s0 + lane < n ? part[s0 + lane] : kKeySent;
        const uint64_t t_k = readlane64(top, K - 1);
        const uint64_t thr = t_k < cap ? t_k : cap;
        const bool surv = c < thr;
        const uint64_t sm = ballot(surv);
        if (!sm) continue;
        uint32_t rs = 0, rt = lane;
        // ranks in the merged order, ties to the top entry, then to the
        // lower lane: a permutation even if a key repeats
        for (uint64_t m = sm; m; m &= m - 1) {
            const uint32_t j = __builtin_ctzll(m);
            const uint64_t kk = readlane64(c, j);
            rs += kk < c || (kk == c && j < lane);
            rt += kk < top;
        }
        for (uint32_t t = 0; t < K; ++t) rs += readlane64(top, t) <= c;
        __syncthreads();
        if (surv && rs < K) T[rs] = c;
        if (lane < K && rt < K) T[rt] = top;
        __syncthreads();
        top = lane < K ? T[lane] : kKeySent;
        __syncthreads();
    }
    if (p.bound_only) {
        const uint64_t t_k = readlane64(top, K - 1);
        if (lane == 0 && t_k != kKeySent && uint32_t(t_k >> 32) < g) p.gbound[q] = uint32_t(t_k >> 32);
        // The K smallest keys so far stand for every key read here: the next
        // merge reads them and the keys appended after them (the K smallest
        // of the union are the K smallest of all).  Every key read above was
        // consumed before these writes (top depends on all of them).
        const uint32_t nt = uint32_t(__popcll(ballot(lane < K && top != kKeySent)));
        if (nt < n) {
            if (lane < nt) part[lane] = top;
            if (lane == 0) p.pcnt[q] = nt;
        }
        return;
    }
    if (lane < K) {
        const bool v = top != kKeySent;
        p.out_ids[size_t(q) * K + lane] = v ? p.gidx[uint32_t(top)] : GF_NO_RESULT;
        p.out_dist[size_t(q) * K + lane] = v ? float(uint32_t(top >> 32)) : __int_as_float(0x7F800000);
    }
    uint32_t scan = 0;
    for (uint32_t i = lane; i < p.counts[q]; i += 64u) {
        const uint32_t c = p.cells[size_t(q) * p.P + i];
        scan += p.offset[c + 1] - p.offset[c];
    }
#pragma unroll
    for (uint32_t o = 32; o; o >>= 1) scan += uint32_t(__shfl_xor(int(scan), int(o)));
    if (lane == 0) {
        uint32_t* ctr = p.counters + size_t(q) * GF_NCOUNTERS;
        ctr[C_EXPAND] = 0;
        ctr[C_DIST] = scan;
        ctr[C_ATTR] = 0;
        ctr[C_CROSS] = 0;
        ctr[C_LROW] = 0;
        ctr[C_SCAN] = scan;
        ctr[C_PASS] = p.selcount[q];
        ctr[C_ROUTE] = 2;
    }
}

// Index build: int8 tiles (operand layout of BfGemmArgs::vt) of the sub-cell
// tile order and per tile [-floor(|x'|^2 / 2) x 16][|x'|^2 x 16] (padding
// points are all zero).
template <typename T>
__global__ __launch_bounds__(64) void k_tile_i8(const T* vec, uint32_t D, const uint32_t* tmeta, uint32_t AW,
                                               int8_t* vt, size_t vstride, int32_t* tnorm, size_t nstride,
                                               uint32_t* mdst, size_t mstride) {
    // Tile t's k-steps at vt + t vstride, its norms at tnorm + t nstride and,
    // with mdst, a copy of its meta (16 (1 + AW) words) at mdst + t mstride.
    const uint32_t t = blockIdx.x, lane = lane_id();
    const uint32_t col = lane & 15u;
    const uint32_t MW = 16u * (1u + AW);
    const uint32_t row = tmeta[size_t(t) * MW + col];
    const bool valid = row != 0xFFFFFFFFu;
    const uint32_t KS = D / 64u;
    if (mdst && lane < MW) mdst[size_t(t) * mstride + lane] = tmeta[size_t(t) * MW + lane];
    if constexpr (sizeof(T) == 1) {
        // u8 rows: each lane moves its 16 bytes of a k-step with one load and
        // one store (x - 128 as int8 is x ^ 0x80); the norm of a point is the
        // sum over its four lanes (col, col + 16, col + 32, col + 48).
        int32_t n = 0;
        for (uint32_t s = 0; s < KS; ++s) {
            uint4 v = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
            if (valid) v = *reinterpret_cast<const uint4*>(vec + size_t(row) * D + s * 64u + (lane >> 4) * 16u);
            v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
            *reinterpret_cast<uint4*>(vt + size_t(t) * vstride + s * 1024u + lane * 16u) = v;
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int32_t x = int32_t(int8_t(uint8_t(w[i] >> (8 * k))));
                    n += x * x;
                }
        }
        n += __shfl_xor(n, 16, 64);
        n += __shfl_xor(n, 32, 64);
        if (lane < 16) {
            tnorm[size_t(t) * nstride + col] = valid ? -(n >> 1) : kPadSeed;
            tnorm[size_t(t) * nstride + 16u + col] = n;
        }
        return;
    }
    for (uint32_t s = 0; s < KS; ++s) {
        int8_t* dst = vt + size_t(t) * vstride + s * 1024u + lane * 16u;
        for (uint32_t j = 0; j < 16; ++j) {
            const uint32_t k = s * 64u + (lane >> 4) * 16u + j;
            dst[j] = valid ? int8_t(int32_t(vec[size_t(row) * D + k]) - 128) : int8_t(0);
        }
    }
    if (lane < 16) {
        int32_t n = 0;
        if (valid)
            for (uint32_t k = 0; k < D; ++k) {
                const int32_t v = int32_t(vec[size_t(row) * D + k]) - 128;
                n += v * v;
            }
        tnorm[size_t(t) * nstride + col] = valid ? -(n >> 1) : kPadSeed;
        tnorm[size_t(t) * nstride + 16u + col] = n;
    }
}

__global__ __launch_bounds__(64) void k_q_i8(const float* q, uint32_t D, int8_t* q8, int32_t* nq) {
    const uint32_t r = blockIdx.x, lane = lane_id();
    int32_t n = 0;
    for (uint32_t k = lane; k < D; k += 64u) {
        const int32_t v = int32_t(q[size_t(r) * D + k]) - 128;
        q8[size_t(r) * D + k] = int8_t(v);
        n += v * v;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) n += __shfl_xor(n, m, 64);
    if (lane == 0) nq[r] = n;
}

// ------------------------------------------------------------ index build
// Exact nearest neighbours for the index builder: the per-cell graphs (the
// cell's own points, self included here and dropped when written) and the
// cross-cell graph (every point against every cell).  One item is a group of
// four query tiles (64 points, the MFMA B operand held in registers) of one
// cell against every tile of a target cell (the A operand, streamed); the
// tile layout is the brute force's (k_tile_i8).  Candidates pass a
// per-query accumulator threshold, queue in LDS and are merged by the query's
// owner lane into a register top-K of (distance << 32 | cell-local id) keys:
// the result is the K smallest keys, ties broken by the smaller local id.
template <int KS, int KT, int NB, int QT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KT > 40 ? 1 : 2))) void k_knn_i8(KnnArgs p) {
    __shared__ uint64_t s_buf[4][kQB * kBfBufQ];
    __shared__ uint32_t s_cnt[4][kQB];
    __shared__ int32_t s_tp[4][kQB];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    uint64_t* buf = s_buf[wave];
    uint32_t* cnt = s_cnt[wave];
    int32_t* stp = s_tp[wave];
    const uint32_t K = p.K;
    const uint32_t col = lane & 15u, grp = lane >> 4;
    // Persistent waves, XCD-aware: workgroups go round-robin to the 8 XCDs
    // and XCD x works through the x-th eighth of the item list, whose items
    // share few target cells, so that this launch's chunk of their tiles
    // stays in that XCD's L2.
    const uint32_t nwg = gridDim.x, xcd = blockIdx.x & 7u, k8 = blockIdx.x >> 3;
    const uint32_t nwg_x = (nwg - xcd + 7u) >> 3;
    const uint32_t i_lo = uint32_t(uint64_t(p.nitems) * xcd / 8u);
    const uint32_t i_hi = uint32_t(uint64_t(p.nitems) * (xcd + 1u) / 8u);
    for (uint32_t item = i_lo + k8 * 4u + wave; item < i_hi; item += nwg_x * 4u) {
        const KnnItem it = p.items[item];
        const uint32_t qc = it.qcell, tc = it.tcell;
        const uint32_t qt = it.qtile, qt_end = min(qt + uint32_t(QT), p.ctile[qc + 1]);
        // candidates: this launch's chunk of the target cell's tiles
        const uint32_t t0 = p.ctile[tc], tn = p.ctile[tc + 1];
        const uint32_t tb = t0 + p.chunk * p.ctiles;
        if (tb >= tn) continue;
        const uint32_t t1 = min(tn, tb + p.ctiles);
        const bool first = p.chunk == 0, last = t1 == tn;
        const uint32_t q_lid = (qt - p.ctile[qc]) * 16u + lane;   // the owner's query, cell-local
        const bool own_live = lane < 16u * QT && q_lid < p.coff[qc + 1] - p.coff[qc];
        const uint32_t own_t = own_live ? qt + grp : qt;
        const int32_t own_nq = p.tnorm[size_t(own_t) * 32u + 16u + col];
        // the query's keys so far (earlier chunks), cell-major row order
        uint64_t* kst = p.state + ((size_t(p.coff[qc]) + q_lid) * (p.R ? 1u : p.P) + (p.R ? 0u : tc)) * p.K;
        uint64_t tk[KT];
#pragma unroll
        for (int k = 0; k < KT; ++k) tk[k] = own_live && !first && uint32_t(k) < K ? kst[k] : kKeySent;
        uint64_t kth = kKeySent;
#pragma unroll
        for (int k = 0; k < KT; ++k)
            if (uint32_t(k) == K - 1) kth = tk[k];
        uint32_t own_thr = kth != kKeySent ? uint32_t(kth >> 32) : 0xFFFFFFFFu;
        wave_fence();
        cnt[lane] = 0;
        stp[lane] = own_live ? acc_threshold(own_nq, own_thr) : INT32_MAX;
        wave_fence();
        v4i32_t B[QT][KS];
        int32_t tp[QT];
#pragma unroll
        for (int j = 0; j < QT; ++j) {
            const uint32_t t = qt + j < qt_end ? qt + j : qt;
#pragma unroll
            for (int k = 0; k < KS; ++k)
                B[j][k] = *reinterpret_cast<const v4i32_t*>(p.vt + (size_t(t) * KS + k) * 1024u + lane * 16u);
            tp[j] = stp[16u * j + col];
        }
        auto drain = [&]() {
            wave_fence();
            const uint32_t n = cnt[lane];
            if (n) {
                uint64_t nxt = buf[lane * kBfBufQ];
                for (uint32_t e = 0; e < n; ++e) {
                    const uint64_t cur = nxt;
                    if (e + 1 < n) nxt = buf[lane * kBfBufQ + e + 1];
                    const int32_t d = own_nq + int32_t(uint32_t(cur >> 32));
                    uint64_t c = (uint64_t(uint32_t(d)) << 32) | uint32_t(cur);
                    if (c < kth) {
#pragma unroll
                        for (int k = 0; k < KT; ++k) {
                            const bool lt = c < tk[k];
                            const uint64_t v = tk[k];
                            tk[k] = lt ? c : v;
                            c = lt ? v : c;
                        }
#pragma unroll
                        for (int k = 0; k < KT; ++k)
                            if (uint32_t(k) == K - 1) kth = tk[k];
                    }
                }
                cnt[lane] = 0;
                if (kth != kKeySent && uint32_t(kth >> 32) < own_thr) {
                    own_thr = uint32_t(kth >> 32);
                    stp[lane] = acc_threshold(own_nq, own_thr);
                }
            }
            wave_fence();
#pragma unroll
            for (int j = 0; j < QT; ++j) tp[j] = stp[16u * j + col];
        };
        // Operands of the next NB - 1 tiles are in flight while a tile is
        // computed (a ring of NB register stages, indexed statically; a
        // stage is refilled once its tile is done).
        v4i32_t A[NB][KS], mh[NB], mn[NB];
        auto load_tile = [&](int b, uint32_t t) {
            const v4i32_t* vp = reinterpret_cast<const v4i32_t*>(p.vt + size_t(t) * KS * 1024u) + lane;
            const int32_t* nt = p.tnorm + size_t(t) * 32u;
#pragma unroll
            for (int k = 0; k < KS; ++k) A[b][k] = vp[k * 64];
            mh[b] = *reinterpret_cast<const v4i32_t*>(nt + 4u * grp);
            mn[b] = *reinterpret_cast<const v4i32_t*>(nt + 16u + 4u * grp);
        };
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (tb + b < t1) load_tile(b, tb + b);
        for (uint32_t ts = tb; ts < t1; ts += NB) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint32_t t = ts + b;
                if (t >= t1) break;
                v4i32_t acc[QT];
#pragma unroll
                for (int j = 0; j < QT; ++j)
                    acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][0], B[j][0], mh[b], 0, 0, 0);
#pragma unroll
                for (int k = 1; k < KS; ++k)
#pragma unroll
                    for (int j = 0; j < QT; ++j)
                        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][k], B[j][k], acc[j], 0, 0, 0);
                // any pass in the tile: one compare per column on the max of its four rows
                bool anyl = false;
#pragma unroll
                for (int j = 0; j < QT; ++j)
                    anyl |= max(max(acc[j][0], acc[j][1]), max(acc[j][2], acc[j][3])) >= tp[j];
                if (__builtin_amdgcn_ballot_w64(anyl)) {
                    // The owner adds |q'|^2 to |x'|^2 - 2 q'.x' when it merges.
                    const uint32_t lid0 = (t - t0) * 16u + 4u * grp;
                    const v4i32_t cmh = mh[b], cmn = mn[b];
                    bool full = false;
#pragma unroll
                    for (int j = 0; j < QT; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (acc[j][i] >= tp[j]) {
                                const uint32_t ql = 16u * j + col;
                                const int32_t v = cmn[i] - 2 * (acc[j][i] - cmh[i]);
                                const uint32_t slot = atomicAdd(&cnt[ql], 1u);
                                buf[ql * kBfBufQ + slot] = (uint64_t(uint32_t(v)) << 32) | (lid0 + uint32_t(i));
                                full |= slot + 1u >= kBfDrainAt;
                            }
                    if (__builtin_amdgcn_ballot_w64(full)) drain();
                }
                // the stage's registers are free: load the tile NB ahead
                if (t + NB < t1) load_tile(b, t + NB);
            }
        }
        drain();
        if (!own_live) continue;
        if (!last) {
#pragma unroll
            for (int k = 0; k < KT; ++k)
                if (uint32_t(k) < K) kst[k] = tk[k];
            continue;
        }
        if (p.R) {
            // per-cell graph row of the query: its R nearest other points
            uint32_t* row = p.out + (size_t(p.coff[qc]) + q_lid) * p.R;
            uint32_t o = 0, first = q_lid;
#pragma unroll
            for (int k = 0; k < KT; ++k) {
                const uint32_t lid = uint32_t(tk[k]);
                if (uint32_t(k) < K && tk[k] != kKeySent && lid != q_lid && o < p.R) {
                    if (o == 0) first = lid;
                    row[o++] = lid;
                }
            }
            for (; o < p.R; ++o) row[o] = first;   // fewer than R others: repeat the nearest
        } else {
            // cross-cell edges of the query's point into the target cell
            const uint32_t pid = p.trow[size_t(own_t) * 16u + col];
            uint32_t* row = p.out + (size_t(pid) * p.P + tc) * K;
            const uint32_t first = uint32_t(tk[0]);
#pragma unroll
            for (int k = 0; k < KT; ++k)
                if (uint32_t(k) < K) row[k] = tk[k] != kKeySent ? uint32_t(tk[k]) : first;
        }
    }
}

// Exact fp32 re-rank of the candidate lists of float data (the kNN kernel
// ran on a u8 quantisation of it): distances in the canonical summation
// order of the row-distance helpers, candidates ordered by (distance,
// cell-local id), repeats dropped; the first `keep` are written and a list
// with fewer distinct candidates repeats its nearest (a graph row with none:
// the point itself).
template <int LPR, int CPL>
__global__ __launch_bounds__(64) void k_rerank(RerankArgs p) {
    __shared__ uint32_t S[64];
    const uint32_t li = blockIdx.x, lane = lane_id();
    uint32_t qrow, tc, self = kEmpty;
    if (p.graph) {
        qrow = li;
        tc = p.rowcell[li];
        self = li - p.coff[tc];
    } else {
        qrow = p.cmrow[li / p.P];
        tc = li % p.P;
    }
    const uint32_t base = p.coff[tc], size = p.coff[tc + 1] - base;
    if (!size) return;   // lists into empty cells keep their zeros
    QReg<0, LPR, CPL> qv;
    const char* vec = reinterpret_cast<const char*>(p.vec);
    load_query<0, LPR, CPL>(qv, vec + size_t(qrow) * p.rowbytes, p.nch);
    const uint32_t lid = lane < p.nc ? p.cand[size_t(li) * p.nc + lane] : kEmpty;
    bool ok = lid < size && lid != self;
    for (uint32_t k = 0; k < 64u; ++k)
        if (k < lane && readlane32(lid, k) == lid) ok = false;   // a repeat: its first lane keeps it
    const uint64_t m = ballot(ok);
    const uint32_t n = __popcll(m);
    const uint32_t ci = ok ? lanes_below(m) : 0xFFFFFFFFu;
    if (ok) S[ci] = base + lid;
    wave_sync();
    float d = __int_as_float(0x7F800000);
    if (n) eval_rows<0, LPR, CPL>(qv, vec, p.rowbytes, p.nch, S, n, ci, d);
    const uint64_t key = ok ? (uint64_t(__float_as_uint(d)) << 32) | lid : ~uint64_t(0);
    uint32_t rk = 0;
    for (uint32_t k = 0; k < 64u; ++k) rk += readlane64(key, k) < key;
    uint32_t* o = p.out + size_t(li) * p.keep;
    if (ok && rk < p.keep) o[rk] = lid;
    const uint64_t nm = ballot(ok && rk == 0);
    const uint32_t nearest = nm ? readlane32(lid, uint32_t(__builtin_ctzll(nm))) : (p.graph ? self : 0u);
    for (uint32_t j = n + lane; j < p.keep; j += 64u) o[j] = nearest;
}

// k-means update of the index builder (integer Lloyd step): the members of
// each cluster are listed (count, scan, scatter), then one workgroup per
// cluster sums its members' u8 rows, a thread per dimension, and moves the
// centre to the rounded mean floor((2 sum + n) / (2 n)) (an empty cluster
// keeps its centre).  lab2 holds the assignment as (point, 2) pairs, label
// second.
__global__ void k_kmeans_count(const uint32_t* lab2, uint32_t N, uint32_t* cnt) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p < N) atomicAdd(&cnt[lab2[size_t(p) * 2u + 1u]], 1u);
}

__global__ void k_kmeans_scatter(const uint32_t* lab2, uint32_t N, const uint32_t* start, uint32_t* fill,
                                 uint32_t* mem) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= N) return;
    const uint32_t l = lab2[size_t(p) * 2u + 1u];
    mem[start[l] + atomicAdd(&fill[l], 1u)] = p;
}

__global__ __launch_bounds__(256) void k_kmeans_mean(const uint8_t* vec, uint32_t Dp, const uint32_t* cnt,
                                                     const uint32_t* start, const uint32_t* mem, uint8_t* centres) {
    const uint32_t c = blockIdx.x;
    const uint32_t n = cnt[c], s0 = start[c];
    if (n == 0) return;
    for (uint32_t d = threadIdx.x; d < Dp; d += blockDim.x) {
        // eight members' rows in flight at a time
        uint32_t sum8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint32_t k = 0;
        for (; k + 8u <= n; k += 8u) {
            uint32_t m[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) m[i] = mem[s0 + k + i];
#pragma unroll
            for (int i = 0; i < 8; ++i) sum8[i] += vec[size_t(m[i]) * Dp + d];
        }
        uint64_t sum = 0;
        for (; k < n; ++k) sum += vec[size_t(mem[s0 + k]) * Dp + d];
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += sum8[i];
        centres[size_t(c) * Dp + d] = uint8_t((2 * sum + n) / (2 * uint64_t(n)));
    }
}

// Rank-based reordering of a kNN graph, the first step of CAGRA's graph
// optimisation (Ootomo et al., "CAGRA: Highly Parallel Graph Construction and
// Approximate Nearest Neighbor Search for GPUs", ICDE 2024): the edge A -> D
// at rank k of A's list has a detour through every B at a rank below k in A's
// list that lists D at a rank below k; A's edges are written in ascending
// (detours, rank) order.  One wave per row: A's I neighbour lists are staged
// in LDS (I x I ids) and lane k counts the detours of edge k.  Rows are
// cell-major and ids cell-local (row = offset[cell] + id).
__global__ __launch_bounds__(64) void k_prune(const uint32_t* knn, uint32_t N, uint32_t I, const uint32_t* offset,
                                              uint32_t P, uint32_t* out) {
    extern __shared__ uint32_t nl[];   // I x I
    const uint32_t lane = lane_id(), row = blockIdx.x;
    if (row >= N) return;
    uint32_t lo = 0, hi = P;           // the cell: last c with offset[c] <= row
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (offset[mid] <= row) lo = mid; else hi = mid;
    }
    const uint32_t base = offset[lo];
    const uint32_t d = lane < I ? knn[size_t(row) * I + lane] : kEmpty;
    for (uint32_t k = 0; k < I; ++k) {
        const uint32_t b = readlane32(d, k);
        if (lane < I) nl[k * I + lane] = knn[(size_t(base) + b) * I + lane];
    }
    __syncthreads();
    uint32_t cnt = 0;
    if (lane < I) {
        for (uint32_t kb = 0; kb < lane; ++kb) {
            const uint32_t* lb = nl + kb * I;
            bool f = false;
            for (uint32_t j = 0; j < lane; ++j) f = f || lb[j] == d;
            cnt += f ? 1u : 0u;
        }
    }
    uint32_t pos = 0;
    for (uint32_t k = 0; k < I; ++k) {
        const uint32_t ck = readlane32(cnt, k);
        pos += (ck < cnt || (ck == cnt && k < lane)) ? 1u : 0u;
    }
    if (lane < I) out[size_t(row) * I + pos] = d;
}

}  // namespace

hipError_t launch_prune(const uint32_t* knn, uint32_t N, uint32_t I, const uint32_t* offset, uint32_t P,
                        uint32_t* out, hipStream_t st) {
    if (!N) return hipSuccess;
    if (I < 1 || I > 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_prune, dim3(N), dim3(64), size_t(I) * I * sizeof(uint32_t), st, knn, N, I, offset, P, out);
    return hipGetLastError();
}

template <int KS, int KT, int NB = 1, int QT = 4>
static hipError_t launch_knn_i8_t(const KnnArgs& a, uint32_t ncu, hipStream_t st) {
    static int per_cu = 0;
    if (!per_cu) {
        int n = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_knn_i8<KS, KT, NB, QT>, 256, 0);
        if (e != hipSuccess) return e;
        per_cu = n > 0 ? n : 1;
    }
    // every XCD (workgroup id mod 8) needs a workgroup: it owns an eighth of the items
    if (a.nitems == 0) return hipSuccess;
    const uint32_t need = ((a.nitems + 3u) / 4u + 7u) / 8u * 8u;
    const uint32_t grid = max(8u, min(ncu * uint32_t(per_cu), need));
    hipLaunchKernelGGL((k_knn_i8<KS, KT, NB, QT>), dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

// KS (k-steps of 64 dimensions) 1 to 4: four query tiles per wave; 6, 8, 12
// and 16 (dimensions up to 1024): one query tile per wave, so that the query
// operand (QT x KS registers of 16 bytes) stays in registers.
uint32_t knn_ks(uint32_t D) {
    const uint32_t ks = (D + 63) / 64;
    if (ks <= 4) return ks;
    if (ks <= 6) return 6;
    if (ks <= 8) return 8;
    if (ks <= 12) return 12;
    return ks <= 16 ? 16 : 0;
}

uint32_t knn_qt(uint32_t KS) { return KS <= 4 ? 4u : 1u; }

hipError_t launch_knn_i8(const KnnArgs& a, uint32_t KS, uint32_t ncu, hipStream_t st) {
    if (a.K == 0 || a.K > kKnnKMax || ncu == 0 || (a.R && a.K != a.R + 1)) return hipErrorInvalidValue;
#define KNN(KS_)                                                          \
    if (KS == KS_) {                                                      \
        if (a.K <= 4) return launch_knn_i8_t<KS_, 4, 2>(a, ncu, st);     \
        if (a.K <= 16) return launch_knn_i8_t<KS_, 16, 2>(a, ncu, st);   \
        if (a.K <= 40) return launch_knn_i8_t<KS_, 40, 2>(a, ncu, st);   \
        return launch_knn_i8_t<KS_, 72>(a, ncu, st);                     \
    }
#define KNN1(KS_)                                                          \
    if (KS == KS_) {                                                       \
        if (a.K <= 4) return launch_knn_i8_t<KS_, 4, 1, 1>(a, ncu, st);   \
        if (a.K <= 16) return launch_knn_i8_t<KS_, 16, 1, 1>(a, ncu, st); \
        if (a.K <= 40) return launch_knn_i8_t<KS_, 40, 1, 1>(a, ncu, st); \
        return launch_knn_i8_t<KS_, 72, 1, 1>(a, ncu, st);                \
    }
    KNN(1)
    KNN(2)
    KNN(3)
    KNN(4)
    KNN1(6)
    KNN1(8)
    KNN1(12)
    KNN1(16)
#undef KNN
#undef KNN1
    return hipErrorInvalidValue;
}

hipError_t launch_kmeans_update(const uint8_t* vec, uint32_t Dp, const uint32_t* lab2, uint32_t N, uint32_t C,
                                uint32_t* cnt, uint32_t* start, uint32_t* fill, uint32_t* mem, uint8_t* centres,
                                hipStream_t st) {
    if (N == 0 || C == 0 || Dp > 1024) return N == 0 || C == 0 ? hipSuccess : hipErrorInvalidValue;
    const uint32_t g = (N + 255) / 256;
    hipLaunchKernelGGL(k_kmeans_count, dim3(g), dim3(256), 0, st, lab2, N, cnt);
    hipError_t e = launch_scan_small(cnt, C, start, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_kmeans_scatter, dim3(g), dim3(256), 0, st, lab2, N, start, fill, mem);
    hipLaunchKernelGGL(k_kmeans_mean, dim3(C), dim3(256), 0, st, vec, Dp, cnt, start, mem, centres);
    return hipGetLastError();
}

namespace {

template <int VT, int LPR, int CPL>
hipError_t launch_trav_t(const TravArgs& a, uint32_t lds, uint32_t grid, hipStream_t st) {
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL((k_traverse<VT, LPR, CPL>), dim3(grid), dim3(64), lds, st, a);
    return hipGetLastError();
}
template <int VT, int LPR, int CPL>
hipError_t launch_dual_t(const TravArgs& a, uint32_t lds, uint32_t grid, hipStream_t st) {
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL((k_traverse_dual<VT, LPR, CPL>), dim3(grid), dim3(64), lds, st, a);
    return hipGetLastError();
}
template <int VT, int LPR, int CPL>
hipError_t launch_full_t(const TravArgs& a, uint32_t lds, uint32_t grid, hipStream_t st) {
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL((k_fullgraph<VT, LPR, CPL>), dim3(grid), dim3(64), lds, st, a);
    return hipGetLastError();
}
template <int VT, int LPR, int CPL>
hipError_t launch_bf_t(const TravArgs& a, uint32_t grid, hipStream_t st) {
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL((k_bruteforce<VT, LPR, CPL>), dim3(grid), dim3(64), 0, st, a);
    return hipGetLastError();
}

}  // namespace

RowShape row_shape(uint32_t D, int vt) {
    RowShape r;
    r.vt = vt;
    const uint32_t elems = vt == 0 ? 4u : ((vt == 1 || vt == 4) ? 8u : 16u);   // vt 2 and 3: 16 bytes
    r.nch = (D + elems - 1) / elems;
    if (vt == 4) {
        // the reference's 32 lanes: 16 virtual lanes of two (row_reduce_ref),
        // chunks per lane rounded up to an instantiated count
        r.lpr = 16;
        r.cpl = (r.nch + 15) / 16;
        if (r.cpl == 3) r.cpl = 4;
        else if (r.cpl == 5) r.cpl = 6;
        else if (r.cpl == 7) r.cpl = 8;
        return r;
    }
    r.lpr = 8;
    while (r.lpr < r.nch && r.lpr < 64) r.lpr <<= 1;
    r.cpl = (r.nch + r.lpr - 1) / r.lpr;
    return r;
}

uint32_t row_shape_max_cpl(int vt) { return vt == 0 ? 4u : (vt == 4 ? 8u : 2u); }

// Instantiated shapes: LPR 8..64 with one chunk per lane, and 64 lanes with
// up to 4 (fp32) or 2 (fp16, u8) chunks per lane.
#define GF_DISPATCH_VT(VT_, CALL)                                                  \
    do {                                                                           \
        if (rs.lpr == 8 && rs.cpl == 1) return CALL(VT_, 8, 1);                     \
        if (rs.lpr == 16 && rs.cpl == 1) return CALL(VT_, 16, 1);                   \
        if (rs.lpr == 32 && rs.cpl == 1) return CALL(VT_, 32, 1);                   \
        if (rs.lpr == 64 && rs.cpl == 1) return CALL(VT_, 64, 1);                   \
        if (rs.lpr == 64 && rs.cpl == 2) return CALL(VT_, 64, 2);                   \
        if (VT_ == 0 && rs.lpr == 64 && rs.cpl == 3) return CALL(0, 64, 3);         \
        if (VT_ == 0 && rs.lpr == 64 && rs.cpl == 4) return CALL(0, 64, 4);         \
    } while (0)
// VT 4 (binary16, the reference's arithmetic): 16 lanes, 1..8 chunks each.
#define GF_DISPATCH_VT4(CALL)                                  \
    do {                                                       \
        if (rs.lpr == 16 && rs.cpl == 1) return CALL(4, 16, 1); \
        if (rs.lpr == 16 && rs.cpl == 2) return CALL(4, 16, 2); \
        if (rs.lpr == 16 && rs.cpl == 4) return CALL(4, 16, 4); \
        if (rs.lpr == 16 && rs.cpl == 6) return CALL(4, 16, 6); \
        if (rs.lpr == 16 && rs.cpl == 8) return CALL(4, 16, 8); \
    } while (0)
#define GF_DISPATCH(CALL)                          \
    do {                                           \
        if (rs.vt == 0) GF_DISPATCH_VT(0, CALL);   \
        if (rs.vt == 1) GF_DISPATCH_VT(1, CALL);   \
        if (rs.vt == 2) GF_DISPATCH_VT(2, CALL);   \
        if (rs.vt == 3) GF_DISPATCH_VT(3, CALL);   \
        if (rs.vt == 4) GF_DISPATCH_VT4(CALL);     \
    } while (0)

namespace {
template <int VT, int KS, int AW>
hipError_t launch_bf_float_t(const BfHArgs& a, uint32_t ncu, hipStream_t st) {
    static int per_cu = 0;
    const auto kern = VT == 1 ? k_bf_f16<KS, AW> : k_bf_f32<KS, AW>;
    if (!per_cu) {
        int n = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, 256, 0);
        if (e != hipSuccess) return e;
        per_cu = n > 0 ? n : 1;
    }
    hipLaunchKernelGGL(kern, dim3(ncu * uint32_t(per_cu)), dim3(256), 0, st, a);
    return hipGetLastError();
}
template <int VT, int LPR, int CPL>
hipError_t launch_bf_f16_final_t(const TravArgs& a, const BfHFinal& f, uint32_t grid, hipStream_t st) {
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL((k_bf_f16_final<VT, LPR, CPL>), dim3(grid), dim3(64), 0, st, a, f);
    return hipGetLastError();
}
}  // namespace

bool bf_float_supported(int vt, uint32_t D, uint32_t AW, uint32_t K) {
    if (!(AW == 1 || AW == 2) || K < 1 || K > 10) return false;
    if (vt == 1) {
        const uint32_t ks = D / 32;
        return D % 32 == 0 && (ks == 2 || ks == 3 || ks == 4 || ks == 8 || ks == 16 || ks == 24);
    }
    if (vt == 0) {
        const uint32_t ks = D / 16;
        return D % 16 == 0 && (ks == 4 || ks == 6 || ks == 8 || ks == 16);
    }
    return false;
}

hipError_t launch_bf_float(const BfHArgs& a, int vt, uint32_t AW, uint32_t ncu, hipStream_t st) {
    if (!bf_float_supported(vt, a.D, AW, a.K) || ncu == 0) return hipErrorInvalidValue;
#define BFH(VT_, KS_)                                                                        \
    case KS_:                                                                                \
        return AW == 1 ? launch_bf_float_t<VT_, KS_, 1>(a, ncu, st) : launch_bf_float_t<VT_, KS_, 2>(a, ncu, st);
    if (vt == 1) {
        switch (a.D / 32) {
            BFH(1, 2) BFH(1, 3) BFH(1, 4) BFH(1, 8) BFH(1, 16) BFH(1, 24)
            default: return hipErrorInvalidValue;
        }
    }
    switch (a.D / 16) {
        BFH(0, 4) BFH(0, 6) BFH(0, 8) BFH(0, 16)
        default: return hipErrorInvalidValue;
    }
#undef BFH
}

hipError_t launch_bf_f16_final(const RowShape& rs, const TravArgs& a, const BfHFinal& f, uint32_t grid,
                               hipStream_t st) {
#define CALL_H(V, L_, C_) launch_bf_f16_final_t<V, L_, C_>(a, f, grid, st)
    if (rs.vt == 1) GF_DISPATCH_VT(1, CALL_H);
    if (rs.vt == 0) GF_DISPATCH_VT(0, CALL_H);
#undef CALL_H
    return hipErrorInvalidValue;
}

hipError_t launch_traverse(const RowShape& rs, const TravArgs& a, uint32_t lds, uint32_t grid, hipStream_t st) {
#define CALL_T(V, L_, C_) launch_trav_t<V, L_, C_>(a, lds, grid, st)
    GF_DISPATCH(CALL_T);
#undef CALL_T
    return hipErrorInvalidValue;
}

hipError_t launch_traverse_dual(const RowShape& rs, const TravArgs& a, uint32_t lds, uint32_t grid,
                                hipStream_t st) {
    if (a.R < 1 || a.R > 32 || a.E < 1 || !a.prow) return hipErrorInvalidValue;
#define CALL_D(V, L_, C_) launch_dual_t<V, L_, C_>(a, lds, grid, st)
    GF_DISPATCH(CALL_D);
#undef CALL_D
    return hipErrorInvalidValue;
}

hipError_t launch_invert_rows(const uint32_t* gidx, uint32_t N, uint32_t* prow, hipStream_t st) {
    if (N == 0) return hipSuccess;
    hipLaunchKernelGGL(k_invert_rows, dim3((N + 255) / 256), dim3(256), 0, st, gidx, N, prow);
    return hipGetLastError();
}

hipError_t launch_fullgraph(const RowShape& rs, const TravArgs& a, uint32_t lds, uint32_t grid, hipStream_t st) {
    if (a.FD < 1 || a.FD > 64) return hipErrorInvalidValue;
#define CALL_F(V, L_, C_) launch_full_t<V, L_, C_>(a, lds, grid, st)
    GF_DISPATCH(CALL_F);
#undef CALL_F
    return hipErrorInvalidValue;
}

hipError_t launch_assemble_full(const uint32_t* graph, const uint32_t* cross, const uint32_t* offset,
                                const uint32_t* rowcell, uint32_t N, uint32_t P, uint32_t R, uint32_t E, uint32_t FE,
                                uint32_t* out, hipStream_t st) {
    const size_t n = size_t(N) * FE * P;
    if (!n) return hipSuccess;
    if (FE > R || FE > E) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_assemble_full, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, st, graph, cross, offset,
                       rowcell, N, P, R, E, FE, out);
    return hipGetLastError();
}

hipError_t launch_bruteforce(const RowShape& rs, const TravArgs& a, uint32_t grid, hipStream_t st) {
#define CALL_B(V, L_, C_) launch_bf_t<V, L_, C_>(a, grid, st)
    GF_DISPATCH(CALL_B);
#undef CALL_B
    return hipErrorInvalidValue;
}

template <int L_, int C_>
static hipError_t launch_rerank_t(const RerankArgs& a, uint32_t nlists, hipStream_t st) {
    hipLaunchKernelGGL((k_rerank<L_, C_>), dim3(nlists), dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_rerank(const RerankArgs& a, uint32_t D, uint32_t nlists, hipStream_t st) {
    if (!nlists) return hipSuccess;
    if (a.nc == 0 || a.nc > 64 || a.keep == 0) return hipErrorInvalidValue;
    const RowShape rs = row_shape(D, 0);
#define CALL_R(V, L_, C_) launch_rerank_t<L_, C_>(a, nlists, st)
    GF_DISPATCH_VT(0, CALL_R);
#undef CALL_R
    return hipErrorInvalidValue;
}


// The kernel's waves are persistent and split the items evenly, so the grid
// is exactly the workgroups that fit on the device at once (a workgroup that
// started late would run its share after the others finished).
template <int KS, int AW, int KT>
static hipError_t launch_bf_i8_t(const BfGemmArgs& a, uint32_t ncu, hipStream_t st) {
    static int per_cu = 0;
    if (!per_cu) {
        int n = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_bf_i8<KS, AW, KT>, 256, 0);
        if (e != hipSuccess) return e;
        per_cu = n > 0 ? n : 1;
    }
    hipLaunchKernelGGL((k_bf_i8<KS, AW, KT>), dim3(ncu * uint32_t(per_cu)), dim3(256), 0, st, a);
    return hipSuccess;
}

hipError_t launch_bf_i8(const BfGemmArgs& a, uint32_t ncu, hipStream_t st) {
    if (a.K > kBfKMax || a.sa.a < 1 || a.sa.a > 4 || ncu == 0) return hipErrorInvalidValue;
    const uint32_t AW = a.sa.AW;
    hipError_t e = hipSuccess;
#define BF(KS, AW_)                                                        \
    do {                                                                   \
        if (a.K <= 10)                                                     \
            e = launch_bf_i8_t<KS, AW_, 10>(a, ncu, st);                   \
        else                                                               \
            e = launch_bf_i8_t<KS, AW_, 16>(a, ncu, st);                   \
    } while (0)
    switch ((a.D / 64) * 4 + AW) {
        case 1 * 4 + 1: BF(1, 1); break;
        case 2 * 4 + 1: BF(2, 1); break;
        case 3 * 4 + 1: BF(3, 1); break;
        case 4 * 4 + 1: BF(4, 1); break;
        case 1 * 4 + 2: BF(1, 2); break;
        case 2 * 4 + 2: BF(2, 2); break;
        case 3 * 4 + 2: BF(3, 2); break;
        case 4 * 4 + 2: BF(4, 2); break;
        default: return hipErrorInvalidValue;
    }
#undef BF
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

hipError_t launch_bf_final(const BfFinalArgs& a, uint32_t grid, hipStream_t st) {
    if (!grid) return hipSuccess;
    hipLaunchKernelGGL(k_bf_final, dim3(grid), dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_sched(const SchedArgs& a, hipStream_t st) {
    if (!a.Q) return hipSuccess;
    hipLaunchKernelGGL(k_sched, dim3(1), dim3(1024), size_t(a.P + 1) * 2 * sizeof(uint32_t), st, a);
    return hipGetLastError();
}

hipError_t launch_stats(const StatsArgs& a, hipStream_t st) {
    const uint32_t n = a.Q > a.NS ? a.Q : a.NS;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_stats, dim3((n + 255) / 256), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_tile_i8(const void* vec_cm, bool u8, uint32_t D, const uint32_t* tmeta, uint32_t AW, uint32_t ntile,
                          int8_t* vt, int32_t* tnorm, hipStream_t st) {
    if (!ntile) return hipSuccess;
    const size_t vs = size_t(D / 64) * 1024u;
    if (u8)
        hipLaunchKernelGGL(k_tile_i8<uint8_t>, dim3(ntile), dim3(64), 0, st, static_cast<const uint8_t*>(vec_cm), D,
                           tmeta, AW, vt, vs, tnorm, size_t(32), static_cast<uint32_t*>(nullptr), size_t(0));
    else
        hipLaunchKernelGGL(k_tile_i8<float>, dim3(ntile), dim3(64), 0, st, static_cast<const float*>(vec_cm), D,
                           tmeta, AW, vt, vs, tnorm, size_t(32), static_cast<uint32_t*>(nullptr), size_t(0));
    return hipGetLastError();
}

hipError_t launch_tile_frec(const void* vec, int vt, uint32_t D, const uint32_t* tmeta, const float* xnorm,
                            uint32_t AW, uint32_t ntile, uint8_t* rec, hipStream_t st) {
    if (!ntile) return hipSuccess;
    if (vt == 1)
        hipLaunchKernelGGL(k_tile_frec<1>, dim3(ntile), dim3(64), 0, st, vec, D, tmeta, xnorm, AW, rec);
    else
        hipLaunchKernelGGL(k_tile_frec<0>, dim3(ntile), dim3(64), 0, st, vec, D, tmeta, xnorm, AW, rec);
    return hipGetLastError();
}

hipError_t launch_tile_rec(const void* vec_cm, bool u8, uint32_t D, const uint32_t* tmeta, uint32_t AW, uint32_t ntile,
                           uint8_t* rec, hipStream_t st) {
    if (!ntile) return hipSuccess;
    const size_t rb = bf_rec_bytes(D, AW), ks = size_t(D / 64) * 1024u;
    int8_t* vt = reinterpret_cast<int8_t*>(rec);
    int32_t* tn = reinterpret_cast<int32_t*>(rec + ks);
    uint32_t* md = reinterpret_cast<uint32_t*>(rec + ks + 128u);
    if (u8)
        hipLaunchKernelGGL(k_tile_i8<uint8_t>, dim3(ntile), dim3(64), 0, st, static_cast<const uint8_t*>(vec_cm), D,
                           tmeta, AW, vt, rb, tn, rb / 4u, md, rb / 4u);
    else
        hipLaunchKernelGGL(k_tile_i8<float>, dim3(ntile), dim3(64), 0, st, static_cast<const float*>(vec_cm), D,
                           tmeta, AW, vt, rb, tn, rb / 4u, md, rb / 4u);
    return hipGetLastError();
}

hipError_t launch_note_bf(const uint32_t* tot, uint32_t* note, hipStream_t st) {
    hipLaunchKernelGGL(k_note_bf, dim3(1), dim3(64), 0, st, tot, note);
    return hipGetLastError();
}

hipError_t launch_subsel(const SubSelArgs& a, hipStream_t st) {
    if (!a.sa.NS || !a.Q) return hipSuccess;
    if (a.sa.AW == 1) hipLaunchKernelGGL(k_subsel<1>, dim3(a.sa.NS), dim3(256), 0, st, a);
    else if (a.sa.AW == 2) hipLaunchKernelGGL(k_subsel<2>, dim3(a.sa.NS), dim3(256), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_bfsched(const BfSchedArgs& a, bool fill, hipStream_t st) {
    if (!a.sa.NS) return hipSuccess;
    hipLaunchKernelGGL(k_bfsched, dim3(a.sa.NS), dim3(256), 0, st, a, fill);
    return hipGetLastError();
}

hipError_t launch_bfsched_direct(const BfSchedArgs& a, hipStream_t st) {
    if (!a.sa.NS) return hipSuccess;
    if (!a.qcap || !a.rq || !a.qrange || !a.scnt) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_bfsched_direct, dim3(a.sa.NS), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_bfitems(const uint32_t* bcnt, const uint32_t* bin, const uint32_t* bstart, uint32_t qcap,
                          const uint32_t* stile, uint32_t tch, uint32_t NS, uint32_t* icnt, uint32_t* ioff,
                          BfItem* items, uint32_t* nitems, const uint32_t* ok, bool fill, hipStream_t st,
                          const uint32_t* scnt, BfItem* sitems, uint32_t* nseed, uint32_t scap, const uint32_t* sorder,
                          uint32_t ns1, uint32_t* nitems_a, uint32_t stch) {
    if (!NS) return hipSuccess;
    if (scnt && (!sitems || !nseed)) return hipErrorInvalidValue;
    if (sorder && ns1 > NS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_bfitems, dim3((NS + 3) / 4), dim3(256), 0, st, bcnt, bin, bstart, qcap, stile, tch, NS,
                       icnt, ioff, items, nitems, ok, fill, scnt, sitems, nseed, scap, sorder, ns1, nitems_a,
                       scnt ? stch : tch);
    return hipGetLastError();
}

hipError_t launch_total(const uint32_t* cnt, const uint32_t* start, uint32_t n, uint32_t cap, uint32_t mul,
                        uint64_t cap2, uint32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_total, dim3(1), dim3(64), 0, st, cnt, start, n, cap, mul, cap2, out);
    return hipGetLastError();
}

hipError_t launch_q_i8(const float* q, uint32_t Q, uint32_t D, int8_t* q8, int32_t* nq, hipStream_t st) {
    if (!Q) return hipSuccess;
    hipLaunchKernelGGL(k_q_i8, dim3(Q), dim3(64), 0, st, q, D, q8, nq);
    return hipGetLastError();
}

hipError_t launch_fill_results(uint32_t* ids, float* dist, uint32_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_fill_results, dim3((n + 255) / 256), dim3(256), 0, st, ids, dist, n);
    return hipGetLastError();
}

hipError_t launch_f2h(const float* x, uint16_t* out, size_t n, float alpha, hipStream_t st) {
    if (!n) return hipSuccess;
    const uint32_t blocks = uint32_t(std::min<size_t>((n + 255) / 256, 65536));
    hipLaunchKernelGGL(k_f2h, dim3(blocks), dim3(256), 0, st, x, out, n, alpha);
    return hipGetLastError();
}

hipError_t launch_f2h_pad(const float* x, uint32_t rows, uint32_t D, uint16_t* out, uint32_t rows_pad,
                          uint32_t Dp, float alpha, hipStream_t st) {
    const size_t n = size_t(rows_pad) * Dp;
    if (!n) return hipSuccess;
    const uint32_t blocks = uint32_t(std::min<size_t>((n + 255) / 256, 65536));
    hipLaunchKernelGGL(k_f2h_pad, dim3(blocks), dim3(256), 0, st, x, rows, D, out, rows_pad, Dp, alpha);
    return hipGetLastError();
}

hipError_t launch_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, uint32_t ld, float* out,
                            hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_norms_f16, dim3(n), dim3(64), 0, st, x, n, D, ld, out);
    return hipGetLastError();
}

hipError_t launch_cells(uint32_t Q, uint32_t a, const float* lo, const float* hi, const uint32_t* grid,
                        const uint32_t* doff, const float* l_q, const float* r_q, uint32_t P,
                        const uint32_t* offset, uint32_t* cells, uint32_t* counts, hipStream_t st,
                        const CellsTail& tl) {
    if (!Q) return hipSuccess;
    if (tl.little && !tl.selcount) return hipErrorInvalidValue;
    if (tl.st_exit && !tl.ticket) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cells, dim3((Q + 63) / 64), dim3(64), 0, st, Q, a, lo, hi, grid, doff, l_q, r_q,
                       P, offset, cells, counts, tl);
    return hipGetLastError();
}

hipError_t launch_cellq_count(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                              uint32_t* ccount, hipStream_t st) {
    if (!Q) return hipSuccess;
    hipLaunchKernelGGL(k_cellq_count, dim3((Q + 255) / 256), dim3(256), 0, st, Q, P, cells, counts, ccount);
    return hipGetLastError();
}

hipError_t launch_scan_small(const uint32_t* in, uint32_t n, uint32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_scan_small, dim3(1), dim3(1024), 0, st, in, n, out, nullptr, 0u, 0u, uint64_t(0));
    return hipGetLastError();
}

hipError_t launch_scan_total(const uint32_t* in, uint32_t n, uint32_t* out, uint32_t cap, uint32_t mul, uint64_t cap2,
                             uint32_t* tot, hipStream_t st) {
    if (!tot) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_scan_small, dim3(1), dim3(1024), 0, st, in, n, out, tot, cap, mul, cap2);
    return hipGetLastError();
}

hipError_t launch_cellq_fill(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                             const uint32_t* cstart, uint32_t* cfill, uint32_t* cellq, hipStream_t st) {
    if (!Q) return hipSuccess;
    hipLaunchKernelGGL(k_cellq_fill, dim3((Q + 255) / 256), dim3(256), 0, st, Q, P, cells, counts, cstart,
                       cfill, cellq);
    return hipGetLastError();
}

hipError_t launch_selcount(uint32_t ntiles, const uint32_t* tile_cell, const uint32_t* tile_row0,
                           const uint32_t* tile_n, const float* attrs, uint32_t a, const uint32_t* cstart,
                           const uint32_t* ccount, const uint32_t* cellq, const float* lo, const float* hi,
                           uint32_t* selcount, hipStream_t st) {
    if (!ntiles) return hipSuccess;
    const uint32_t lds = kSelTile * a * sizeof(float);
    hipLaunchKernelGGL(k_selcount, dim3(ntiles), dim3(256), lds, st, tile_cell, tile_row0, tile_n, attrs, a,
                       cstart, ccount, cellq, lo, hi, selcount);
    return hipGetLastError();
}

hipError_t launch_route(uint32_t Q, uint32_t N, float thr, const uint32_t* selcount, const uint32_t* counts,
                        uint32_t* little, hipStream_t st, uint32_t* ticket, uint64_t* st_exit) {
    if (st_exit && !ticket) return hipErrorInvalidValue;
    if (!Q) return hipSuccess;
    hipLaunchKernelGGL(k_route, dim3((Q + 255) / 256), dim3(256), 0, st, Q, N, thr, selcount, counts, little, ticket,
                       st_exit);
    return hipGetLastError();
}

hipError_t launch_cells_grid(uint32_t Q, uint32_t a, const float* lo, const float* hi, const float* amin,
                             const float* width, const uint32_t* grid, uint32_t P, const uint32_t* offset,
                             double thr, uint32_t* cells, uint32_t* counts, uint32_t* little, uint8_t* flags,
                             hipStream_t st) {
    hipLaunchKernelGGL(k_cells_grid, dim3((Q + 63) / 64), dim3(64), 0, st, Q, a, lo, hi, amin, width, grid, P,
                       offset, thr, cells, counts, little, flags);
    return hipGetLastError();
}

hipError_t launch_cell_flags(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                             const uint32_t* little, uint8_t* flags, hipStream_t st) {
    hipLaunchKernelGGL(k_cell_flags, dim3((Q + 63) / 64), dim3(64), 0, st, Q, P, cells, counts, little, flags);
    return hipGetLastError();
}

hipError_t launch_stream_lists(uint32_t Q, uint32_t P, uint32_t B, const uint32_t* bcell, const uint8_t* flags,
                               uint32_t* lists, uint32_t* counts, uint32_t* little, hipStream_t st) {
    hipLaunchKernelGGL(k_stream_lists, dim3((Q + 63) / 64), dim3(64), 0, st, Q, P, B, bcell, flags, lists, counts,
                       little);
    return hipGetLastError();
}

hipError_t launch_bf_reset(uint32_t Q, uint32_t* nsub, uint32_t* pcnt, uint32_t* gbound, hipStream_t st, uint32_t NS,
                          uint32_t* scnt, uint32_t* nseed) {
    const uint32_t n = (Q > NS ? Q : NS) > 0u ? (Q > NS ? Q : NS) : 1u;
    hipLaunchKernelGGL(k_bf_reset, dim3((n + 255) / 256), dim3(256), 0, st, Q, nsub, pcnt, gbound, NS, scnt, nseed);
    return hipGetLastError();
}

hipError_t launch_bfseed(const BfSeedArgs& a, uint32_t Q, hipStream_t st) {
    if (!Q || !a.qcap) return hipSuccess;
    hipLaunchKernelGGL(k_bfseed, dim3((Q + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_stamp(uint64_t* t, hipStream_t st, uint32_t n) {
    if (n < 1 || n > 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stamp, dim3(1), dim3(64), 0, st, t, n);
    return hipGetLastError();
}

hipError_t launch_zero_u32(uint32_t* x, uint32_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(256), 0, st, x, n);
    return hipGetLastError();
}

hipError_t launch_reset_results(uint32_t Q, uint32_t K, uint32_t* ids, float* dist, uint32_t* ctr, hipStream_t st,
                                uint32_t* z, uint32_t nz, uint64_t* stp, uint32_t nst, const BfReset& br) {
    if (nst > 64) return hipErrorInvalidValue;
    if (br.nsub && (!br.pcnt || !br.gbound || (br.scnt && !br.nseed))) return hipErrorInvalidValue;
    uint32_t n = Q * (K > GF_NCOUNTERS ? K : GF_NCOUNTERS);
    n = n > nz ? n : nz;
    if (br.nsub) n = n > br.NS ? n : br.NS;
    hipLaunchKernelGGL(k_reset_results, dim3((n + 255) / 256), dim3(256), 0, st, Q, K, ids, dist, ctr, z, nz, stp,
                       stp ? nst : 0u, br);
    return hipGetLastError();
}

hipError_t launch_gather_meta(const unsigned long long* stats, const uint32_t* tot, const uint64_t* stamps,
                              unsigned long long* h_stats, uint32_t* h_tot, uint64_t* h_stamps, hipStream_t st) {
    hipLaunchKernelGGL(k_gather_meta, dim3(1), dim3(64), 0, st, stats, tot, stamps, h_stats, h_tot, h_stamps);
    return hipGetLastError();
}

hipError_t launch_batch_need(uint32_t Q, uint32_t P, uint32_t nbatch, const uint32_t* plan_cells,
                             const uint32_t* plan_off, const uint8_t* flags, uint32_t* need, hipStream_t st) {
    if (!nbatch) return hipSuccess;
    // need[0, nbatch) and the active counts need[nbatch, 2 nbatch)
    hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(256), 0, st, need, 2u * nbatch);
    const uint32_t gy = (Q + 255) / 256 < 64u ? (Q + 255) / 256 : 64u;
    hipLaunchKernelGGL(k_batch_need, dim3(nbatch, gy), dim3(256), 0, st, Q, P, plan_cells, plan_off, flags, need,
                       need + nbatch);
    return hipGetLastError();
}

hipError_t launch_cell_boxes(uint32_t Q, uint32_t P, uint32_t a, const uint32_t* grid, const uint32_t* cells,
                             const uint32_t* counts, uint32_t* box, hipStream_t st) {
    if (!Q) return hipSuccess;
    hipLaunchKernelGGL(k_cell_boxes, dim3((Q + 255) / 256), dim3(256), 0, st, Q, P, a, grid, cells, counts, box);
    return hipGetLastError();
}

hipError_t launch_stream_gather(const GatherDesc* desc, uint32_t n, const char* arena, const char* head, char* img,
                                hipStream_t st) {
    if (!n) return hipSuccess;
    // 16 workgroups keep enough reads in flight for the PCIe link (56 GB/s
    // alone, 52 GB/s beside a latency-bound kernel, measured) and slow the
    // compute stream's kernels by 5-12 %; 64 reach no more and slow them by
    // up to 75 % (their long-latency host reads hold the memory pipelines of
    // the CUs they share).
    hipLaunchKernelGGL(k_stream_gather, dim3(16), dim3(256), 0, st, desc, n, arena, head, img);
    return hipGetLastError();
}

hipError_t launch_merge_stream(uint32_t Q, uint32_t K, uint32_t* run_ids, float* run_dist, const uint32_t* ids,
                               const float* dist, uint32_t* run_ctr, const uint32_t* ctr, bool first,
                               hipStream_t st) {
    if (K > kBfKMax * 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_merge_stream, dim3((Q + 63) / 64), dim3(64), 0, st, Q, K, run_ids, run_dist, ids, dist,
                       run_ctr, ctr, uint32_t(first));
    return hipGetLastError();
}

hipError_t launch_centroid(const uint16_t* qh, const uint16_t* ch, const float* qn, const float* cn,
                           uint32_t Q, uint32_t C, uint32_t Qp, uint32_t Cp, uint32_t Dp, float* dist,
                           hipStream_t st, uint64_t* st_entry) {
    if (!Q || !C) return hipSuccess;
    // Cp is a multiple of 64 and Qp of 16, so every tile read stays inside the
    // zero-padded operands.
    hipLaunchKernelGGL(k_centroid, dim3(Qp / 16, Cp / 64), dim3(256), 0, st, qh, ch, qn, cn, Q, C, Dp, dist,
                       st_entry);
    return hipGetLastError();
}

hipError_t launch_order(uint32_t Q, uint32_t C, uint32_t P, uint32_t topc, const float* dist,
                        const uint32_t* hist, uint32_t* cells, const uint32_t* counts, uint32_t* topk,
                        hipStream_t st, bool chosen, bool ref_ties) {
    if (!Q) return hipSuccess;
    const uint32_t lds = (16 + 2 * P) * sizeof(uint32_t);
    hipLaunchKernelGGL(k_order, dim3(Q), dim3(64), lds, st, Q, C, P, topc, dist, hist, cells, counts, topk, chosen,
                       ref_ties);
    return hipGetLastError();
}

hipError_t launch_centroid_top(const uint16_t* qh, const uint16_t* ch, const float* qn, const float* cn, uint32_t Q,
                               uint32_t C, uint32_t Qp, uint32_t Cp, uint32_t Dp, uint32_t topc, uint32_t* topk,
                               hipStream_t st, uint64_t* st_entry) {
    if (!Q || !C) return hipSuccess;
    if (topc < 1 || topc > 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_centroid_top, dim3(Qp / 16), dim3(64 * kCtW), 0, st, qh, ch, qn, cn, Q, C, Cp, Dp, topc,
                       topk, st_entry);
    return hipGetLastError();
}

}  // namespace gf
