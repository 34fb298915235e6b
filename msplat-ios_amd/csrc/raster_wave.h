// raster_wave.h -- wave-level building blocks shared by the 2DGS and 3DGS
// rasterizers: per-wave slot lists of a staged batch (forward) and the
// 16-value wave reduction of the per-splat gradients (backward).  All of it
// assumes 256-thread workgroups of four wave64, wave w owning pixel block w
// of a 16x16 tile.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msr {

constexpr int kThreads = 256;

// The blend logs of one frame, in 64-entry chunks taken from a pool as the
// waves fill them.  Wave w of tile t (list [start, start + len)) logs at most
// len entries; its k-th chunk (entries 64k .. 64k + 63) is pool chunk
// c = table[log_table_base(start, len, t, w) + k], whose entries are
// ent[64 c ..] and whose checkpoint, each lane's transmittance before entry
// 64 (k + 1), is ckpt[64 c + lane].  wave_cnt[4 t + w] is the wave's entry
// count.  The pool is split into nsub sub-pools of sub_cap chunks, each with
// its own atomic counter (a single counter serialised the claims of every
// wave and tripled the training forward's time), plus a shared spill region
// of spill_cap chunks for sub-pools that run out; a claim past both stops
// that wave's log and sets *overflow, so the log is then incomplete and its
// consumers do nothing (overflowed()).
struct BlendLog {
    uint4 *ent;
    float *ckpt;
    int *table;
    int *wave_cnt;
    int *counters;  // [nsub + 1]: the sub-pools' and the spill region's
    int *overflow;
    int nsub, sub_cap, spill_cap;
};

// Wave (t, w)'s chunk-table range starts here: the ranges of successive
// waves are disjoint, since a wave's ceil(len / 64) chunks fit between
// floor(4 start + w len) / 64 + 4 t + w and the next wave's base.
__host__ __device__ inline size_t log_table_base(int start, int len, int tile, int wave) {
    return (4 * (size_t)start + (size_t)wave * (size_t)len) / 64 + 4 * (size_t)tile + (size_t)wave;
}
inline size_t log_table_ints(int64_t isect, int tiles) { return (size_t)(4 * isect) / 64 + 4 * (size_t)tiles + 1; }
__device__ __forceinline__ bool overflowed(const BlendLog &L) { return *L.overflow != 0; }
__device__ __forceinline__ int log_subpool(const BlendLog &L, int tile, int wave) { return (4 * tile + wave) % L.nsub; }

// n chunks for sub-pool sp after its counter returned c (the base of a claim
// of n): the chunk index of the first, from the spill region if the
// sub-pool is full, or -1 (and *overflow set) if both are.
__device__ __forceinline__ int log_resolve(const BlendLog &L, int sp, int c, int n) {
    if (c + n <= L.sub_cap) return sp * L.sub_cap + c;
    const int x = atomicAdd(&L.counters[L.nsub], n);
    if (x + n <= L.spill_cap) return L.nsub * L.sub_cap + x;
    atomicOr(L.overflow, 1);
    return -1;
}

// A wave's log writer: entries are staged in lane (count mod 64) of lg_ent
// by the caller.  Each chunk is claimed one chunk ahead: start() (before the
// visits) issues the sub-pool claim of the first, full() writes a completed
// chunk and its checkpoint into the claimed chunk and issues the claim of
// the next, and finish() writes the partial last chunk and the count.  A
// claim's result is only waited for when its chunk is written, 64 entries
// later, and the visit loop itself carries no claim code.  A wave whose log
// ends on a chunk boundary (or is empty) leaves its last claim unused: at
// most one chunk per wave, within the worst case of ceil(len / 64) chunks
// per wave.  cid is written and read in lane 0 only.  Wave-uniform control
// flow.
struct LogWriter {
    size_t tb;
    int sp = 0;
    int cid = 0;  // lane 0: the sub-pool counter's value of the pending claim
    bool ok = true;
    __device__ __forceinline__ void claim_next(const BlendLog &L, int lane) {
        if (lane == 0) cid = atomicAdd(&L.counters[sp], 1);
    }
    __device__ __forceinline__ void start(const BlendLog &L, int lane) { claim_next(L, lane); }
    __device__ __forceinline__ int claimed(const BlendLog &L, int lane) {
        int c = 0;
        if (lane == 0) c = log_resolve(L, sp, cid, 1);
        c = __builtin_amdgcn_readfirstlane(c);
        if (c < 0) ok = false;
        return c;
    }
    __device__ __forceinline__ void full(const BlendLog &L, int lane, int nlog, const uint4 &e, float T) {
        if (!ok) return;
        const int c = claimed(L, lane);
        if (!ok) return;
        L.ent[64 * (size_t)c + lane] = e;
        L.ckpt[64 * (size_t)c + lane] = T;
        if (lane == 0) L.table[tb + (size_t)((nlog >> 6) - 1)] = c;
        claim_next(L, lane);
    }
    __device__ __forceinline__ void finish(const BlendLog &L, int lane, int nlog, const uint4 &e, int tile,
                                           int wave) {
        if (ok && (nlog & 63)) {
            const int c = claimed(L, lane);
            if (ok) {
                if (lane < (nlog & 63)) L.ent[64 * (size_t)c + lane] = e;
                if (lane == 0) L.table[tb + (size_t)(nlog >> 6)] = c;
            }
        }
        if (lane == 0) L.wave_cnt[4 * tile + wave] = nlog;
    }
};

// Per-wave slot lists of one batch: s_list[w][0..n_w) holds, in ascending
// order, the slots whose mask m has bit w (this wave's ballot rank after the
// counts of the waves below it).
// Returns n for the calling thread's wave.  Called by all threads of the
// workgroup (two barriers).
__device__ __forceinline__ int build_wave_lists(int m, unsigned char (*s_list)[kThreads], int4 *s_cnt) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const unsigned long long below = (1ull << lane) - 1ull;
    int pos[4], cnt[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const unsigned long long bal = __ballot((m >> w) & 1);
        pos[w] = __popcll(bal & below);
        cnt[w] = __popcll(bal);
    }
    if (lane == 0) s_cnt[wave] = make_int4(cnt[0], cnt[1], cnt[2], cnt[3]);
    __syncthreads();
    // every wave's counts at once (broadcast reads); the slots of block w
    // from waves below this one precede this wave's
    const int4 c0 = s_cnt[0], c1 = s_cnt[1], c2 = s_cnt[2], c3 = s_cnt[3];
    const int4 z = make_int4(0, 0, 0, 0);
    const int4 p1 = wave > 0 ? c0 : z, p2 = wave > 1 ? c1 : z, p3 = wave > 2 ? c2 : z;
    const int base[4] = {p1.x + p2.x + p3.x, p1.y + p2.y + p3.y, p1.z + p2.z + p3.z, p1.w + p2.w + p3.w};
#pragma unroll
    for (int w = 0; w < 4; ++w)
        if ((m >> w) & 1) s_list[w][base[w] + pos[w]] = (unsigned char)threadIdx.x;
    // this wave's list length (wave-uniform: keeps the visit loop's control
    // in scalar registers)
    const int4 tot = make_int4(c0.x + c1.x + c2.x + c3.x, c0.y + c1.y + c2.y + c3.y, c0.z + c1.z + c2.z + c3.z,
                               c0.w + c1.w + c2.w + c3.w);
    const int n = __builtin_amdgcn_readfirstlane(wave == 0 ? tot.x : wave == 1 ? tot.y : wave == 2 ? tot.z : tot.w);
    __syncthreads();
    return n;
}

// DPP lane permutations within a 16-lane row (CDNA3/4 dpp_ctrl codes).
constexpr int kDppQuad1032 = 0xB1;   // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuad2301 = 0x4E;   // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane i of each 8-lane half row <- 7 - i
constexpr int kDppRowMirror = 0x140;   // lane i of each row <- 15 - i

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum of v[0..15] over the 64 lanes of a wave (a transpose reduction):
// v_permlane32_swap / v_permlane16_swap exchange half-waves / half-rows
// between two value registers, so each of those steps halves the value
// count with one swap and one add per pair and no lane select; two mirror
// DPP steps (partners differ in lane bit 3, then bit 2) and two quad_perm
// DPP adds finish.  Lane l ends with the total of value index
// 8*b5 + 4*b4 + 2*b3 + b2 (b = bits of l); every lane of a quad holds it.
// SKIP1: bit i set when v[i] and v[i + 8] are zero in every lane, so their
// first-stage pair is skipped (it would sum to zero).
template <unsigned SKIP1 = 0>
__device__ __forceinline__ float wave_reduce16(float v[16], int lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if ((SKIP1 >> i) & 1u) continue;
        // vdst lanes 32-63 <-> src lanes 0-31: lanes < 32 end with value i,
        // lanes >= 32 with value i + 8
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // odd rows of vdst <-> even rows of src: lane bit 4 selects i + 4
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 4]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b3 = lane & 8, b2 = lane & 4;
    {
        const float x0 = v[0] + dpp<kDppRowMirror>(v[0]);
        const float x2 = v[2] + dpp<kDppRowMirror>(v[2]);
        const float x1 = v[1] + dpp<kDppRowMirror>(v[1]);
        const float x3 = v[3] + dpp<kDppRowMirror>(v[3]);
        v[0] = b3 ? x2 : x0;
        v[1] = b3 ? x3 : x1;
    }
    {
        const float x0 = v[0] + dpp<kDppHalfMirror>(v[0]);
        const float x1 = v[1] + dpp<kDppHalfMirror>(v[1]);
        v[0] = b2 ? x1 : x0;
    }
    v[0] += dpp<kDppQuad1032>(v[0]);
    v[0] += dpp<kDppQuad2301>(v[0]);
    return v[0];
}

// Orders this wave's LDS stores before its later LDS loads (and the loads of
// one chunk before the stores of the next): a wave's LDS operations execute
// in program order, so only the compiler has to be kept from moving them.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// wave_reduce16 with at most one permlane step and the rest through LDS.
// Row i of this wave's 512-float scratch carries either a pair or one raw
// value.  A pair row (bit i of RAW clear) holds, in lane L, value i + 8 b5(L)
// summed over lanes L and L ^ 32 (one permlane32 swap + add).  A raw row (bit
// i set) holds value i itself in every lane; v[i + 8] is then not read.
// Lane L writes row i at column L ^ c(i), c(i) = 4 (i & 1) + 32 ((i >> 1) & 1).
// Quad q = l >> 2 then takes slot s = (q >> 1) + 8 (q & 1) (s = q when no
// row is raw, which measured 2% faster on the 3DGS backward): its four lanes
// sum the entries of row s & 7 held by lanes 32 (s >> 3) + 8 k .. + 7
// (k = l & 3) with two 16-byte reads, and two quad DPP adds finish.  For a
// pair row that is the total of value s.  For a raw row the quads of slots
// i and i + 8 hold the sums over the two half-waves; they are neighbours in
// one 16-lane DPP row (quad q even, q + 1), so one DPP add (row_shl:4,
// masked to those quads) gives slot i the total, and slot i + 8 is not
// used.  Red8::adds marks the lanes that hold a total (one per quad), so the
// caller's atomic never has two lanes on one address: same-address lanes of
// one atomic instruction are serialised, which made an undivided version of
// this scheme twice as slow.  A raw row saves a permlane swap and an add per
// visit; the raw rows must be the rows 2R + j of a set of R times a set of j
// (the DPP row and bank masks), and n values fit in 8 rows with up to
// 16 - n of them raw.  Each row written is 256 bytes of LDS stores per
// visit, so when a visit is short a raw row can cost more in LDS bandwidth
// than its permlane swap.  Under the XOR swizzle the 64-lane row writes and each
// 16-lane group of 16-byte reads touch distinct banks.  (Measured at the
// 3M-splat step: one permlane step was 5.6% faster than two with a 256-float
// LDS tail; no permlane step with 16 rows, 4 KB of LDS traffic per visit,
// was 9% slower.)
constexpr unsigned raw_dpp_rows(unsigned raw) {
    unsigned m = 0;
    for (int R = 0; R < 4; ++R)
        if ((raw >> (2 * R)) & 3u) m |= 1u << R;
    return m;
}
constexpr unsigned raw_dpp_banks(unsigned raw) {
    unsigned m = 0;
    for (int j = 0; j < 2; ++j)
        if (raw & (0x55u << j)) m |= 1u << (2 * j);
    return m;
}
constexpr bool raw_is_product(unsigned raw) {
    unsigned p = 0;
    for (int R = 0; R < 4; ++R)
        for (int j = 0; j < 2; ++j)
            if (((raw_dpp_rows(raw) >> R) & 1u) && ((raw_dpp_banks(raw) >> (2 * j)) & 1u)) p |= 1u << (2 * R + j);
    return p == raw;
}

// SKIP: rows whose values are zero in every lane; they are never written
// (zero_skipped clears them once).
template <unsigned RAW, unsigned SKIP = 0>
struct Red8 {
    static_assert(raw_is_product(RAW), "raw rows must be a row set times a bank set");
    static_assert((RAW & SKIP) == 0, "a row is raw or skipped");
    float *wb[4];        // scratch + (lane ^ c(j)), j = 0..3; register i writes at wb[i & 3] + 64 i
    const float4 *r0, *r1;  // this lane's two 16-byte read addresses
    int slot;            // the reduction slot this lane ends with
    bool adds;           // lane 0 of its quad, and its slot holds a total

    __device__ __forceinline__ void init(float *scratch, int lane) {
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[j] = scratch + (lane ^ (4 * (j & 1) + 32 * ((j >> 1) & 1)));
        const int q = lane >> 2;
        slot = RAW == 0 ? q : (q >> 1) + 8 * (q & 1);
        const int row = slot & 7, c = 4 * (row & 1) + 32 * ((row >> 1) & 1);
        const int L = 32 * (slot >> 3) + 8 * (lane & 3);
        r0 = reinterpret_cast<const float4 *>(scratch + 64 * row + (L ^ c));
        r1 = reinterpret_cast<const float4 *>(scratch + 64 * row + ((L + 4) ^ c));
        adds = (lane & 3) == 0 && !(((RAW >> row) & 1u) && slot >= 8);
    }
    // zeros in the skipped rows (call before the first reduction; the
    // caller's wave_lds_sync orders it)
    __device__ __forceinline__ void zero_skipped() const {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if ((SKIP >> i) & 1u) wb[i & 3][64 * i] = 0.0f;
    }
};

template <unsigned RAW, unsigned SKIP>
__device__ __forceinline__ float wave_reduce16_lds8(float v[16], const Red8<RAW, SKIP> &r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if ((SKIP >> i) & 1u) continue;
        if ((RAW >> i) & 1u) {
            r.wb[i & 3][64 * i] = v[i];
            continue;
        }
        const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]), false,
                                                        false);
        r.wb[i & 3][64 * i] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
    }
    wave_lds_sync();
    const float4 p = *r.r0, q = *r.r1;
    wave_lds_sync();
    float s = ((p.x + p.y) + (p.z + p.w)) + ((q.x + q.y) + (q.z + q.w));
    s += dpp<kDppQuad1032>(s);
    s += dpp<kDppQuad2301>(s);
    // one masked DPP add: lanes outside the row and bank masks are not
    // written (the builtin's form is a mov, a constant and an add, since no
    // float constant is an exact identity of the add); the nop covers the
    // two wait states a DPP read needs after the VALU write of s
    if constexpr (RAW != 0)
        asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_shl:4 row_mask:%1 bank_mask:%2"
            : "+v"(s)
            : "n"(raw_dpp_rows(RAW)), "n"(raw_dpp_banks(RAW)));
    return s;
}

}  // namespace msr
