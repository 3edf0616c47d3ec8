// Attention kernels of the gfx950 backend.
//
// 1. ICL attention, 64-wide heads, FP32 on matrix cores. It serves both the
//    build's train-row self-attention (N queries x N keys) and prediction's
//    cross-attention of a pass's queries against the resident K/V: the role
//    of icl_attention_f32 + icl_attention_merge in the reference's CUDA
//    backend (src/kernels/cuda/kernels.rs:183-213, 1523-1702), with the
//    semantics of softmax(q k^T / 8) v in FP32 (src/kernels/reference.rs:792-1024).
//
//    A wave owns 64 queries (two blocks of 32). It computes the transposed
//    products
//      S^T[key, q] = K Q^T       (v_mfma_f32_32x32x2f32, k = head dim)
//      O^T[d, q]  += V^T P^T     (k = keys)
//    so that in the accumulator layout lane (q = lane % 32, half = lane / 32)
//    holds all of one query's scores for half of each 32-key block, and all of
//    its 64 output dims across the two 32-row output tiles; each K or V
//    fragment read from LDS feeds both query blocks. The softmax state is per
//    lane. Scores live in the exp2 domain (q pre-scaled by log2(e)/8) and are
//    exponentiated against a lazy reference (see the kernel): the subtraction
//    rides in the first MFMA's accumulator and the maximum is only taken when
//    the reference must move. The P^T operand of the second product is the
//    first product's accumulator register as is; each lane fetches the V
//    elements of the key that register holds. The two output tiles take the
//    even and the odd dims, so one 8-byte LDS read serves both. Keys stream
//    through double-buffered 64-key LDS tiles filled by direct global -> LDS
//    loads; only a range's last tile is clamped and masked. One workgroup of
//    four waves per CU: each wave may use 512 registers.
//
//    Key ranges are split over workgroups to fill the chip (prediction
//    passes); the build's many query tiles run whole rounds with every key
//    and split only the tiles left over (plan_icl_fp32). Each split writes
//    its normalized partial output and log2-sum-exp, and a merge kernel
//    combines them. Workgroups sharing a (pair, split) K/V range are placed on
//    the same XCD so the range is read into one L2.
//
// 2. Attention of 16-wide heads on the vector ALUs (column ISAB and row
//    transformer), one thread per (sequence, head, query row), keys staged
//    through LDS in chunks of 64, optional RoPE on queries and keys.
#include "common.hpp"

#include <type_traits>

#include <algorithm>

namespace irx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// This file builds with IEEE mode off (-mno-amdgpu-ieee), which the device
// library's work-item functions were not built with, so they would stay
// out-of-line calls returning ids in VGPRs: ids come from the builtins.
__device__ __forceinline__ int tid_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int bid_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int bdim_x() { return (int)__builtin_amdgcn_workgroup_size_x(); }

constexpr int kKeyTile = 64;

struct IclLaunch {
    int qtiles, splits, keys_per_split, per_xcd, q_padded;
    // FP32 wide kernel only. count: workgroup units of this launch. A tail
    // launch (tail_units > 0) takes units unit0 .. unit0 + tail_units - 1 of
    // the (query tile, pair) units, each split over `splits` key ranges, with
    // its partials compacted to [splits, tail_units * 256] rows.
    int count, unit0, tail_units;
    long long part_rows;  // partial rows per split
};

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kIclWaves = 4;
constexpr int kIclQueries = kIclWaves * 64;  // queries per workgroup, 64 per wave

// One 64-key tile of K and V in LDS, 16 KB each, written by direct global ->
// LDS loads (a wave-wide 16-byte load lands as 1 KB, lane after lane). K is
// kept in 1 KB blocks b = (chunk / 4) * 4 + key / 16, each holding 16 keys x
// 4 chunks of 4 dims at position (chunk % 4) * 16 + key % 16, so that the 16
// lanes of a 16-byte LDS read that fetch one chunk of 16 consecutive keys
// touch every bank once. V is key-major: a half-wave reads one key's 64 dims.
struct IclTile {
    float k[kKeyTile * 64];
    float v[kKeyTile * 64];
};

__device__ __forceinline__ void wait_loads() {
    // vmcnt(0); expcnt and lgkmcnt left at their maxima (no wait).
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

// Maximum / sum of a lane's value and its partner's in the other half-wave
// (lane l and l ^ 32 hold the same query).
__device__ __forceinline__ float halves_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Long key ranges (FLUSH) accumulate in two levels: every kFlushTiles tiles
// the register accumulators (O^T and the row sums) are added into totals the
// lane keeps in LDS and restart from zero. A single FP32 accumulator over
// tens of thousands of keys loses the contributions that arrive after a
// dominant one (each addend below half an ulp of the sum is rounded away);
// with peaked attention over 50,000 keys that cost 3e-4 of the output.
constexpr int kFlushTiles = 64;
constexpr int kFlushFloats = kIclWaves * 2 * 2 * 16 * 64;  // [j][b][r / 4][thread][r % 4]

// SPLIT: the keys are split over workgroups and each writes a partial output
// and its log2-sum-exp, merged afterwards; otherwise the output is final.
template <bool SPLIT, bool FLUSH>
__global__ __launch_bounds__(kIclWaves * 64, 1) void icl_attention_kernel(IclAttention p, IclLaunch g) {
    // One LDS object: the K/V tiles, then (FLUSH) each thread's O^T totals
    // and its row-sum totals [j][thread]. (As a second LDS object the totals
    // made the compiler wait for the in-flight tile loads before every read
    // of the current tile.)
    struct LdsPlain {
        IclTile tiles[2];
    };
    struct LdsFlush {
        IclTile tiles[2];
        float totals[kFlushFloats + kIclWaves * 2 * 64];
    };
    __shared__ __attribute__((aligned(16))) std::conditional_t<FLUSH, LdsFlush, LdsPlain> lds;
    IclTile *tiles = lds.tiles;
    float *totals = nullptr;
    if constexpr (FLUSH) totals = lds.totals;

    const int bid = bid_x();
    const int t_id = (bid % 8) * g.per_xcd + bid / 8;
    if (t_id >= g.count) return;
    // Units (query tile qt of pair `pair`) in order qt + qtiles * pair. A
    // tail launch's workgroups take its units split-major, so the units that
    // share a key range are consecutive (and on one XCD).
    int qt, split, pair, tail_unit = 0;
    if (g.tail_units) {
        tail_unit = t_id % g.tail_units, split = t_id / g.tail_units;
        const int unit = g.unit0 + tail_unit;
        qt = unit % g.qtiles, pair = unit / g.qtiles;
    } else {
        qt = t_id % g.qtiles;
        const int rest = t_id / g.qtiles;
        split = rest % g.splits, pair = rest / g.splits;
    }
    // Workgroup-uniform; read into scalars so the key loop runs on scalar registers.
    const int k_begin = __builtin_amdgcn_readfirstlane(split * g.keys_per_split);
    const int k_end = __builtin_amdgcn_readfirstlane(min(p.kv_rows, k_begin + g.keys_per_split));

    const int tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    // Query block j of this wave holds rows qrow0 + 32 j.
    const int qrow0 = qt * kIclQueries + wave * 64 + r32;

    // The lane's queries: dims 32*half .. 32*half + 31, scaled into the exp2 domain.
    float qreg[2][32];
    {
        const float scale = 0.125f * kLog2e;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int qrow = qrow0 + 32 * j;
            if (qrow < p.q_rows) {
                const float *src = p.q + pair * p.q_pair_stride + (long long)qrow * 64 + 32 * half;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    f32x4 v = *reinterpret_cast<const f32x4 *>(src + 4 * c);
#pragma unroll
                    for (int e = 0; e < 4; ++e) qreg[j][4 * c + e] = v[e] * scale;
                }
            } else {
#pragma unroll
                for (int t = 0; t < 32; ++t) qreg[j][t] = 0.f;
            }
        }
    }

    // Staging: wave w moves K blocks 4w .. 4w + 3 (chunks 4w .. 4w + 3 of key
    // blocks 0..3) and V blocks 4w .. 4w + 3 (keys 16w .. 16w + 15).
    const float *kbase = p.k + pair * p.kv_pair_stride;
    const float *vbase = p.v + pair * p.kv_pair_stride;
    // Lane offsets (floats) within a full tile: K key 16 i + lane % 16, chunk
    // 4w + lane / 16; V key 16w + 4i + lane / 16, chunk lane % 16. The wave
    // index is read into a scalar so that tile bases and LDS destinations are
    // scalar arithmetic.
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int k_lane = (lane & 15) * 64 + 4 * (4 * wv + (lane >> 4));
    const int v_lane = (lane >> 4) * 64 + 4 * (lane & 15);
    auto issue_tile = [&](int k0, int buf) {
        const float *kt = kbase + (long long)k0 * 64, *vt = vbase + (long long)(k0 + 16 * wv) * 64;
        if (k0 + kKeyTile <= k_end) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_global_load_lds(kt + i * 1024 + k_lane, (lds_void *)&tiles[buf].k[(4 * wv + i) * 256],
                                                 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vt + i * 256 + v_lane, (lds_void *)&tiles[buf].v[(4 * wv + i) * 256],
                                                 16, 0, 0);
            }
        } else {
            // A range's last tile: keys past it repeat its last key (masked later).
            const int last = k_end - 1 - k0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kk = min(16 * i + (lane & 15), last);
                const int vk = min(16 * wv + 4 * i + (lane >> 4), last);
                __builtin_amdgcn_global_load_lds(kbase + (long long)(k0 + kk) * 64 + 4 * (4 * wv + (lane >> 4)),
                                                 (lds_void *)&tiles[buf].k[(4 * wv + i) * 256], 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vbase + (long long)(k0 + vk) * 64 + 4 * (lane & 15),
                                                 (lds_void *)&tiles[buf].v[(4 * wv + i) * 256], 16, 0, 0);
            }
        }
    };

    // O^T accumulators of query block j: o[j][0] even dims d = 2i, o[j][1] odd
    // dims d = 2i + 1, where i = half*4 + (r&3) + 8*(r>>2) for register r.
    f32x16 o[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][0][r] = 0.f, o[j][1][r] = 0.f;
    // Softmax reference m_ref[j] per query (shared by the lane pair l, l ^ 32):
    // probabilities are exp2(s - m_ref). The range's first tile sets it to
    // that tile's maxima (its products start from zero); after that it is
    // raised, and the tile redone, only when a tile's probabilities could
    // exceed 2^64, so most tiles skip the maximum reduction; -m_ref is the
    // products' initial accumulator, which folds the subtraction into the
    // MFMA. Relative to the true running maximum a probability is at most
    // 2^64 and anything below 2^-126 of the maximum is lost, as in the exact
    // online softmax.
    float m_ref[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    f32x16 neg_ref[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) neg_ref[j][r] = 0.f;
    bool fresh = true;  // workgroup-uniform: no tile of the range done yet
    constexpr float kLazyLimit = 18446744073709551616.0f;  // 2^64
    // K fragment of chunk 8*half + cc for key r32 of block 0 is at kfrag + (cc >> 2) * 1024 + (cc & 3) * 64;
    // block 1 (keys 32..63) is 512 floats further.
    const int kfrag = (8 * half + (r32 >> 4)) * 256 + (r32 & 15) * 4;

    // FLUSH: the keys run in chunks of kFlushTiles tiles, each chunk's
    // accumulators added into the lane's LDS totals after it (flushed: some
    // chunk was; workgroup-uniform). The totals' addresses are formed where
    // they are used, so nothing extra stays live through the tile loop.
    bool flushed = false;
    // Rescales owed to the totals since the last flush (the reference moved):
    // applied when the totals are next read, so the tile loop touches no LDS
    // besides its tiles.
    float tot_scale[2] = {1.f, 1.f};
    // O^T totals as [j][b][r / 4][thread] groups of four: one 16-byte LDS
    // access per group of a lane's four consecutive registers.
    auto o_tot = [&](int j, int b, int q) -> f32x4 & {
        return *reinterpret_cast<f32x4 *>(&totals[(((j * 2 + b) * 4 + q) * 64 * kIclWaves + tid_x()) * 4]);
    };
    auto l_tot = [&](int j) -> float & { return totals[kFlushFloats + tid_x() + j * 64 * kIclWaves]; };
    const int chunk = FLUSH ? kFlushTiles * kKeyTile : k_end - k_begin;

    issue_tile(k_begin, 0);
    int buf = 0;
    for (int c0 = k_begin; c0 < k_end; c0 = __builtin_amdgcn_readfirstlane(c0 + chunk)) {
    const int c1 = __builtin_amdgcn_readfirstlane(min(k_end, c0 + chunk));
    for (int k0 = c0; k0 < c1; k0 = __builtin_amdgcn_readfirstlane(k0 + kKeyTile)) {
        wait_loads();
        __syncthreads();
        if (k0 + kKeyTile < k_end) issue_tile(k0 + kKeyTile, buf ^ 1);
        const float *kt = tiles[buf].k;
        const float *vt = tiles[buf].v;

        // S^T[key, q] - m_ref for key blocks 0 / 1 and query blocks 0 / 1.
        f32x16 s[2][2];
        // K fragments are read one chunk ahead of their MFMAs (the scheduling
        // groups keep the compiler from sinking the reads to their first use).
        f32x4 ka = *reinterpret_cast<const f32x4 *>(kt + kfrag);
        f32x4 kb = *reinterpret_cast<const f32x4 *>(kt + kfrag + 512);
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            f32x4 na = ka, nb = kb;
            if (cc < 7) {
                const int off = kfrag + ((cc + 1) >> 2) * 1024 + ((cc + 1) & 3) * 64;
                na = *reinterpret_cast<const f32x4 *>(kt + off);
                nb = *reinterpret_cast<const f32x4 *>(kt + off + 512);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const f32x16 &c0 = (cc == 0 && e == 0) ? neg_ref[j] : s[j][0];
                    const f32x16 &c1 = (cc == 0 && e == 0) ? neg_ref[j] : s[j][1];
                    s[j][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[e], qreg[j][4 * cc + e], c0, 0, 0, 0);
                    s[j][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(kb[e], qreg[j][4 * cc + e], c1, 0, 0, 0);
                }
            if (cc < 7) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the two DS reads
                __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // then this chunk's MFMAs
            }
            ka = na, kb = nb;
        }
        // Only the last tile of a range can hold keys past it.
        if (k0 + kKeyTile > k_end) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + half * 4 + (r & 3) + 8 * (r >> 2);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (key >= k_end) s[j][0][r] = -INFINITY;
                    if (key + 32 >= k_end) s[j][1][r] = -INFINITY;
                }
            }
        }
        if (fresh) {
            // The range's first tile: its scores (from a zero accumulator)
            // give the reference.
            fresh = false;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float mt = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(s[j][0][r], s[j][1][r]));
                const float m = halves_max(mt);
                m_ref[j] = m;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    neg_ref[j][r] = -m;
                    s[j][0][r] -= m, s[j][1][r] -= m;
                }
            }
        }
        // Softmax per query block (exp2 domain) against the lazy reference.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[j][0][r] = __builtin_amdgcn_exp2f(s[j][0][r]);
                s[j][1][r] = __builtin_amdgcn_exp2f(s[j][1][r]);
                lsum += s[j][0][r] + s[j][1][r];
            }
            if (__any(!(lsum <= kLazyLimit))) {
                // The reference is too low for this tile: recompute the
                // block's scores from zero and raise it to the running maximum.
                f32x16 t0, t1;
#pragma unroll
                for (int r = 0; r < 16; ++r) t0[r] = 0.f, t1[r] = 0.f;
#pragma unroll
                for (int cc = 0; cc < 8; ++cc) {
                    const int off = kfrag + (cc >> 2) * 1024 + (cc & 3) * 64;
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(kt + off);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(kt + off + 512);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        t0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qreg[j][4 * cc + e], t0, 0, 0, 0);
                        t1 = __builtin_amdgcn_mfma_f32_32x32x2f32(b[e], qreg[j][4 * cc + e], t1, 0, 0, 0);
                    }
                }
                if (k0 + kKeyTile > k_end) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + half * 4 + (r & 3) + 8 * (r >> 2);
                        if (key >= k_end) t0[r] = -INFINITY;
                        if (key + 32 >= k_end) t1[r] = -INFINITY;
                    }
                }
                float mt = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(t0[r], t1[r]));
                const float m_new = fmaxf(m_ref[j], halves_max(mt));
                const float alpha = __builtin_amdgcn_exp2f(m_ref[j] - m_new);
                l_run[j] *= alpha;
                lsum = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    o[j][0][r] *= alpha, o[j][1][r] *= alpha;
                    neg_ref[j][r] = -m_new;
                    s[j][0][r] = __builtin_amdgcn_exp2f(t0[r] - m_new);
                    s[j][1][r] = __builtin_amdgcn_exp2f(t1[r] - m_new);
                    lsum += s[j][0][r] + s[j][1][r];
                }
                if constexpr (FLUSH) tot_scale[j] *= alpha;  // the totals are in the old scale too
                m_ref[j] = m_new;
            }
            l_run[j] += lsum;
        }
        // O^T += V^T P^T: register r of s[j][b] is key b*32 + half*4 + (r&3) + 8*(r>>2);
        // the lane fetches that key's dims 2*r32 and 2*r32 + 1, one key ahead
        // of its products (scheduling fences keep the reads there: left to
        // itself the compiler moves each read next to its first use).
        auto vrow = [&](int r) { return vt + (half * 4 + (r & 3) + 8 * (r >> 2)) * 64 + 2 * r32; };
        f32x2 v0 = *reinterpret_cast<const f32x2 *>(vrow(0));
        f32x2 v1 = *reinterpret_cast<const f32x2 *>(vrow(0) + 32 * 64);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            f32x2 n0 = v0, n1 = v1;
            if (r < 15) {
                n0 = *reinterpret_cast<const f32x2 *>(vrow(r + 1));
                n1 = *reinterpret_cast<const f32x2 *>(vrow(r + 1) + 32 * 64);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                o[j][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[0], s[j][0][r], o[j][0], 0, 0, 0);
                o[j][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[1], s[j][0][r], o[j][1], 0, 0, 0);
                o[j][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[0], s[j][1][r], o[j][0], 0, 0, 0);
                o[j][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[1], s[j][1][r], o[j][1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            v0 = n0, v1 = n1;
        }
        buf ^= 1;
    }
    if constexpr (FLUSH) {
        if (c1 < k_end) {
            // Each lane moves only its own values: no barrier.
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float ts = tot_scale[j];
                l_tot(j) = flushed ? l_tot(j) * ts + l_run[j] : l_run[j];
                l_run[j] = 0.f;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        f32x4 t = flushed ? o_tot(j, b, q) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            t[e] = flushed ? t[e] * ts + o[j][b][4 * q + e] : o[j][b][4 * q + e];
                            o[j][b][4 * q + e] = 0.f;
                        }
                        o_tot(j, b, q) = t;
                    }
                tot_scale[j] = 1.f;
            }
            flushed = true;
        }
    }
    }
    if constexpr (FLUSH) {
        if (flushed) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float ts = tot_scale[j];
                l_run[j] += l_tot(j) * ts;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 t = o_tot(j, b, q);
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[j][b][4 * q + e] += t[e] * ts;
                    }
            }
        }
    }

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int qrow = qrow0 + 32 * j;
        const float l_tot = halves_sum(l_run[j]);
        if (qrow >= p.q_rows) continue;
        const float inv = 1.0f / l_tot;
        float *dst;
        if constexpr (!SPLIT) {
            const int b = pair / kHeads, head = pair - b * kHeads;
            dst = p.o + ((long long)b * p.q_rows + qrow) * p.ldo + head * 64;
        } else {
            const long long row =
                g.tail_units ? split * g.part_rows + (long long)tail_unit * kIclQueries + (qrow - qt * kIclQueries)
                             : split * g.part_rows + (long long)pair * g.q_padded + qrow;
            dst = p.partial + row * 64;
            if (half == 0) p.partial[(long long)g.splits * g.part_rows * 64 + row] = m_ref[j] + log2f(l_tot);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = half * 4 + (r & 3) + 8 * (r >> 2);
            f32x2 v;
            v[0] = o[j][0][r] * inv, v[1] = o[j][1][r] * inv;
            *reinterpret_cast<f32x2 *>(dst + 2 * i) = v;
        }
    }
}

// ---- Split-FP16 products over an FP16 cache (IRX_PRECISION_SPLIT, the
// reference's optimize="auto": cuda/mod.rs:71-105) ----
//
// The cache holds K as FP16 [pairs, Np, 64] (Np = keys rounded up to 64,
// zero past the keys) and V tile-transposed as FP16 [pairs, Np / 64, 64
// dims, 64 keys], the keys of each 16-key group stored in the order 0..3,
// 8..11, 4..7, 12..15. Queries and probabilities, FP32, are split into a high
// FP16 part and the FP16 remainder (x = hi + lo, about 22 significant bits);
// each product is hi.K + lo.K on the 32x32x16 FP16 MFMA, both into one FP32
// accumulator, so only the cache's own FP16 rounding remains. Layouts per
// tile (64 keys, 4 waves x 64 queries as above):
//   S^T (key x query): A = K[key = lane % 32 (+32)][dims 16 m + 8 (lane / 32)
//     .. +7], B = the lane's query, same dims; result register r is key
//     8 (r / 4) + 4 (lane / 32) + r % 4 (+32), query lane % 32 (+32 j);
//   O^T (dim x query), 16-key step t of the tile: A = V^T[dim][the 8 keys the
//     lane's result registers 8 (t % 2) .. +7 of key block t / 2 hold], which
//     the stored key order makes one 16-byte read; B = those probabilities.
// LDS rows are 128 bytes (one key of K, one dim of V^T); the 16-byte chunk c
// of row r is stored at chunk c ^ (r % 8) so that the 8 rows a half-wave
// group reads hit distinct banks. Probabilities stay below 2^15 (the lazy
// reference's limit here), so their high parts fit FP16.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct IclTile16 {
    u32x4 k[kKeyTile * 8];  // 64 rows x 8 chunks of 16 bytes
    u32x4 v[kKeyTile * 8];
};

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

// FP8 tiles (IRX_PRECISION_HALF): K [64 keys x 64 bytes] and V^T [64 dims x
// 64 keys] bytes, 4 KB each; the 16-byte chunk c of row r is stored at chunk
// c ^ ((r / 4) % 4).
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
struct IclTile8 {
    u32x4 k[kKeyTile * 4];
    u32x4 v[kKeyTile * 4];
};

// Eight E4M3 values (OCP, bias 7) as FP16, exactly (v_cvt_scalef32_pk_f16_fp8, scale 1).
__device__ __forceinline__ half8 fp8x8_to_half8(u32x2 w) {
    typedef _Float16 half2 __attribute__((ext_vector_type(2)));
    const half2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.0f, false);
    const half2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.0f, true);
    const half2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.0f, false);
    const half2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.0f, true);
    return half8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Eight FP32 values rounded to FP16 (nearest even).
__device__ __forceinline__ half8 round8(const float *x) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (_Float16)x[e];
    return h;
}

// Eight FP32 values split into high and low FP16 parts, x = hi + lo. The low
// part is not rescaled: both products accumulate into one FP32 accumulator,
// and a low part below FP16's normal range (only for |x| < 2^-3) loses bits
// worth less than 2^-24 |x|.
__device__ __forceinline__ void split8(const float *x, half8 &hi, half8 &lo) {
    u32x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto hp = __builtin_amdgcn_cvt_pkrtz(x[2 * i], x[2 * i + 1]);
        const float r0 = x[2 * i] - (float)hp[0];
        const float r1 = x[2 * i + 1] - (float)hp[1];
        const auto lp = __builtin_amdgcn_cvt_pkrtz(r0, r1);
        h[i] = __builtin_bit_cast(unsigned, hp);
        l[i] = __builtin_bit_cast(unsigned, lp);
    }
    hi = __builtin_bit_cast(half8, h);
    lo = __builtin_bit_cast(half8, l);
}

// FP8 (IRX_PRECISION_HALF, the reference's optimize="fast"): the same
// tiling over an E4M3 cache (K [pairs, Np, 64] bytes, V^T tiles as above in
// bytes) with a scale per (pair, dim): the key scales are folded into the
// queries, which are rounded once to FP16; each fragment is converted to FP16
// after its LDS read; one FP16 product each (no low parts); the value scales
// multiply the output.
template <bool SPLIT, bool FP8 = false>
__global__ __launch_bounds__(kIclWaves * 64, 1) void icl_attention_split_kernel(IclAttention p, IclLaunch g) {
    __shared__ __attribute__((aligned(16))) std::conditional_t<FP8, IclTile8, IclTile16> tiles[2];

    const int total = g.qtiles * p.pairs * g.splits;
    const int bid = bid_x();
    const int t_id = (bid % 8) * g.per_xcd + bid / 8;
    if (t_id >= total) return;
    const int qt = t_id % g.qtiles;
    const int rest = t_id / g.qtiles;
    const int split = rest % g.splits;
    const int pair = rest / g.splits;
    const int k_begin = __builtin_amdgcn_readfirstlane(split * g.keys_per_split);
    const int k_end = __builtin_amdgcn_readfirstlane(min(p.kv_rows, k_begin + g.keys_per_split));
    const int n_pad = (p.kv_rows + kKeyTile - 1) / kKeyTile * kKeyTile;

    const int tid = tid_x(), lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    const int qrow0 = qt * kIclQueries + wave * 64 + r32;

    // The lane's queries, dims 16 m + 8 half .. +7 for m = 0..3, in the exp2
    // domain, split into high and low FP16 parts (FP8: times the key scales,
    // rounded to FP16).
    half8 qh[2][4], ql[2][4];
    {
        const float scale = 0.125f * kLog2e;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int qrow = qrow0 + 32 * j;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                float x[8];
                if (qrow < p.q_rows) {
                    const float *src = p.q + pair * p.q_pair_stride + (long long)qrow * 64 + 16 * m + 8 * half;
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(src);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = a[e] * scale, x[4 + e] = b[e] * scale;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = 0.f;
                }
                if constexpr (FP8) {
                    const float *ks = p.kscale + pair * 64 + 16 * m + 8 * half;
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] *= ks[e];
                    qh[j][m] = round8(x);
                } else {
                    split8(x, qh[j][m], ql[j][m]);
                }
            }
        }
    }

    // Staging: a tile of K (or V^T) is 8 KB contiguous in HBM; instruction t
    // of 8 fills LDS chunks 64 t .. 64 t + 63. Wave w issues K and V
    // instructions 2 w and 2 w + 1. Lane i of instruction t fills LDS row
    // 8 t + i / 8, stored chunk i % 8, i.e. source chunk (i % 8) ^ (row % 8).
    // FP8: a tile of K (or V^T) is 4 KB; wave w's one instruction fills LDS
    // rows 16 w .. 16 w + 15, lane i row 16 w + i / 4, stored chunk i % 4.
    const unsigned short *kbase = p.k16 + (long long)pair * n_pad * 64;
    const unsigned short *vbase = p.v16 + (long long)pair * n_pad * 64;
    const unsigned char *kbase8 = p.k8 + (long long)pair * n_pad * 64;
    const unsigned char *vbase8 = p.v8 + (long long)pair * n_pad * 64;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    int src_off[2];
    if constexpr (FP8) {
        const int row = 16 * wv + (lane >> 2);
        src_off[0] = row * 64 + 16 * ((lane & 3) ^ ((row >> 2) & 3));  // bytes
        src_off[1] = 0;
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int t = 2 * wv + i, row = 8 * t + (lane >> 3);
            src_off[i] = row * 64 + 8 * ((lane & 7) ^ (row & 7));  // halves
        }
    }
    auto issue_tile = [&](int k0, int buf) {
        if constexpr (FP8) {
            const unsigned char *kt = kbase8 + (long long)k0 * 64, *vt = vbase8 + (long long)k0 * 64;
            __builtin_amdgcn_global_load_lds(kt + src_off[0], (lds_void *)&tiles[buf].k[64 * wv], 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vt + src_off[0], (lds_void *)&tiles[buf].v[64 * wv], 16, 0, 0);
        } else {
            const unsigned short *kt = kbase + (long long)k0 * 64, *vt = vbase + (long long)k0 * 64;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int t = 2 * wv + i;
                __builtin_amdgcn_global_load_lds(kt + src_off[i], (lds_void *)&tiles[buf].k[64 * t], 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vt + src_off[i], (lds_void *)&tiles[buf].v[64 * t], 16, 0, 0);
            }
        }
    };
    // The FP16 operand of row `row`, 8-element group c2 (dims or keys 8 c2 .. +7).
    auto frag = [](const u32x4 *tile, int row, int c2) {
        if constexpr (FP8) {
            const int c = c2 >> 1;
            return fp8x8_to_half8(reinterpret_cast<const u32x2 *>(tile)[2 * (row * 4 + (c ^ ((row >> 2) & 3))) + (c2 & 1)]);
        } else {
            return as_half8(tile[row * 8 + (c2 ^ (row & 7))]);
        }
    };

    f32x16 o[2][2];  // [dim block][query block]
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[d][j][r] = 0.f;
    // The lazy reference as in icl_attention_kernel: set from the range's
    // first tile, raised when a tile's probabilities could pass the limit.
    float m_ref[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    f32x16 neg_ref[2], zero;
#pragma unroll
    for (int r = 0; r < 16; ++r) neg_ref[0][r] = 0.f, neg_ref[1][r] = 0.f, zero[r] = 0.f;
    constexpr float kLazyLimit16 = 32768.0f;  // 2^15: probabilities stay FP16-representable
    bool fresh = true;  // workgroup-uniform: no tile of the range done yet

    // One tile at k0 from LDS buffer `buf`. Only a range's last tile can hold
    // keys past it (RAGGED): full tiles carry no masking code at all (left to
    // itself the compiler computes every key's bound check on every tile).
    auto tile = [&](int k0, int buf, auto ragged) {
        constexpr bool RAGGED = decltype(ragged)::value;
        const u32x4 *kt = tiles[buf].k;
        const u32x4 *vt = tiles[buf].v;

        // Scores of this tile against both query blocks, from the FP16 keys.
        auto scores = [&](int j, const f32x16 &init, f32x16 &s0, f32x16 &s1) {
            s0 = init, s1 = init;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const half8 a0 = frag(kt, r32, 2 * m + half);
                const half8 a1 = frag(kt, r32 + 32, 2 * m + half);
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qh[j][m], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qh[j][m], s1, 0, 0, 0);
                if constexpr (!FP8) {
                    s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, ql[j][m], s0, 0, 0, 0);
                    s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, ql[j][m], s1, 0, 0, 0);
                }
            }
            if constexpr (RAGGED) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (key >= k_end) s0[r] = -INFINITY;
                    if (key + 32 >= k_end) s1[r] = -INFINITY;
                }
            }
        };

        f32x16 s[2][2];  // [query block][key block]
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            scores(j, neg_ref[j], s[j][0], s[j][1]);
            if (fresh) {
                // The range's first tile (scores from a zero accumulator).
                float mt = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(s[j][0][r], s[j][1][r]));
                const float m = halves_max(mt);
                m_ref[j] = m;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    neg_ref[j][r] = -m;
                    s[j][0][r] -= m, s[j][1][r] -= m;
                }
            }
            float lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[j][0][r] = __builtin_amdgcn_exp2f(s[j][0][r]);
                s[j][1][r] = __builtin_amdgcn_exp2f(s[j][1][r]);
                lsum += s[j][0][r] + s[j][1][r];
            }
            if (__any(!(lsum <= kLazyLimit16))) {
                f32x16 t0, t1;
                scores(j, zero, t0, t1);
                float mt = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(t0[r], t1[r]));
                const float m_new = fmaxf(m_ref[j], halves_max(mt));
                const float alpha = __builtin_amdgcn_exp2f(m_ref[j] - m_new);
                l_run[j] *= alpha;
                lsum = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    o[0][j][r] *= alpha, o[1][j][r] *= alpha;
                    neg_ref[j][r] = -m_new;
                    s[j][0][r] = __builtin_amdgcn_exp2f(t0[r] - m_new);
                    s[j][1][r] = __builtin_amdgcn_exp2f(t1[r] - m_new);
                    lsum += s[j][0][r] + s[j][1][r];
                }
                m_ref[j] = m_new;
            }
            l_run[j] += lsum;
        }
        fresh = false;
        // O^T += V^T P^T over the tile's four 16-key steps.
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int kb = t >> 1, g = t & 1;
            half8 ph[2], pl[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = s[j][kb][8 * g + e];
                if constexpr (FP8)
                    ph[j] = round8(x);
                else
                    split8(x, ph[j], pl[j]);
            }
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const half8 a = frag(vt, 32 * d + r32, 2 * t + half);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    o[d][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ph[j], o[d][j], 0, 0, 0);
                    if constexpr (!FP8) o[d][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pl[j], o[d][j], 0, 0, 0);
                }
            }
        }
    };

    issue_tile(k_begin, 0);
    int buf = 0;
    // Full tiles, then the range's ragged last tile if it has one.
    const int k_full = __builtin_amdgcn_readfirstlane(k_begin + (k_end - k_begin) / kKeyTile * kKeyTile);
    int k0 = k_begin;
    for (; k0 < k_full; k0 = __builtin_amdgcn_readfirstlane(k0 + kKeyTile)) {
        wait_loads();
        __syncthreads();
        if (k0 + kKeyTile < k_end) issue_tile(k0 + kKeyTile, buf ^ 1);
        tile(k0, buf, std::false_type{});
        buf ^= 1;
    }
    if (k0 < k_end) {
        wait_loads();
        __syncthreads();
        tile(k0, buf, std::true_type{});
    }

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int qrow = qrow0 + 32 * j;
        const float l_tot = halves_sum(l_run[j]);
        if (qrow >= p.q_rows) continue;
        const float inv = 1.0f / l_tot;
        float *dst;
        if constexpr (!SPLIT) {
            const int b = pair / kHeads, head = pair - b * kHeads;
            dst = p.o + ((long long)b * p.q_rows + qrow) * p.ldo + head * 64;
        } else {
            const long long row = ((long long)split * p.pairs + pair) * g.q_padded + qrow;
            dst = p.partial + row * 64;
            if (half == 0) p.partial[(long long)g.splits * p.pairs * g.q_padded * 64 + row] = m_ref[j] + log2f(l_tot);
        }
        // Register r of block d: dims 32 d + 8 (r / 4) + 4 half + r % 4.
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                f32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = o[d][j][4 * a + e] * inv;
                if constexpr (FP8) v *= *reinterpret_cast<const f32x4 *>(p.vscale + pair * 64 + 32 * d + 8 * a + 4 * half);
                *reinterpret_cast<f32x4 *>(dst + 32 * d + 8 * a + 4 * half) = v;
            }
    }
}

// FP32 or FP16 K/V [pairs, rows, 64] into the FP16 cache layout above (K
// padded with zero rows, V tile-transposed with the stored key order). One
// workgroup per (pair, 64-key tile); counts values that are not finite in
// FP16 (beyond +-65504 or NaN) into `bad`.
template <typename T>
__global__ __launch_bounds__(256) void pack_icl16_kernel(const T *k, const T *v, long long rows, int pairs,
                                                         unsigned short *k16, unsigned short *v16, unsigned *bad) {
    __shared__ float tile[64][65];
    const int tiles = (int)((rows + kKeyTile - 1) / kKeyTile);
    const int pair = bid_x() / tiles, tix = bid_x() % tiles;
    const long long n_pad = (long long)tiles * kKeyTile;
    const long long k0 = (long long)tix * kKeyTile;
    const T *ks = k + (long long)pair * rows * 64, *vs = v + (long long)pair * rows * 64;
    unsigned short *kd = k16 + ((long long)pair * n_pad + k0) * 64, *vd = v16 + ((long long)pair * n_pad + k0) * 64;
    unsigned local_bad = 0;
    for (int i = tid_x(); i < 64 * 64; i += 256) {
        const int key = i / 64, d = i % 64;
        const bool in = k0 + key < rows;
        const float kv = in ? (float)ks[(k0 + key) * 64 + d] : 0.f;
        const float vv = in ? (float)vs[(k0 + key) * 64 + d] : 0.f;
        const _Float16 kh = (_Float16)kv;
        local_bad += !(fabsf(kv) <= 65504.f) + !(fabsf(vv) <= 65504.f);
        kd[i] = __builtin_bit_cast(unsigned short, kh);
        tile[key][d] = vv;
    }
    __syncthreads();
    // V^T: row d holds the tile's keys in the stored order (positions 4..7 and
    // 8..11 of each 16-key group swapped).
    for (int i = tid_x(); i < 64 * 64; i += 256) {
        const int d = i / 64, pos = i % 64;
        const int q16 = pos & 15, swap = (q16 >= 4 && q16 < 8) ? 4 : (q16 >= 8 && q16 < 12 ? -4 : 0);
        const int key = (pos & ~15) + q16 + swap;
        vd[i] = __builtin_bit_cast(unsigned short, (_Float16)tile[key][d]);
    }
    if (local_bad) atomicAdd(bad, local_bad);
}

// The FP16 cache back to logical FP16 K and V [pairs, rows, 64].
__global__ __launch_bounds__(256) void unpack_icl16_kernel(const unsigned short *k16, const unsigned short *v16,
                                                           long long rows, int pairs, unsigned short *k,
                                                           unsigned short *v) {
    const int tiles = (int)((rows + kKeyTile - 1) / kKeyTile);
    const int pair = bid_x() / tiles, tix = bid_x() % tiles;
    const long long n_pad = (long long)tiles * kKeyTile, k0 = (long long)tix * kKeyTile;
    const unsigned short *ks = k16 + ((long long)pair * n_pad + k0) * 64;
    const unsigned short *vs = v16 + ((long long)pair * n_pad + k0) * 64;
    for (int i = tid_x(); i < 64 * 64; i += 256) {
        const int key = i / 64, d = i % 64;
        if (k0 + key >= rows) continue;
        const int q16 = key & 15, swap = (q16 >= 4 && q16 < 8) ? 4 : (q16 >= 8 && q16 < 12 ? -4 : 0);
        const int pos = (key & ~15) + q16 + swap;
        k[((long long)pair * rows + k0 + key) * 64 + d] = ks[i];
        v[((long long)pair * rows + k0 + key) * 64 + d] = vs[d * 64 + pos];
    }
}

// Few queries (a pass of at most 32 rows): the attention is bound by reading
// K and V from HBM. A workgroup of kDecodeWaves waves takes one (pair, key
// range); its waves take the range's 16-key blocks in turn, so together they
// stream it front to back. Products run on the 16x16x4 FP32 MFMA over QG
// groups of 16 queries, which pads a pass to 16 or 32 queries rather than 64.
// Operands go straight from global memory into registers in MFMA order:
//   scores S^T (key x query): A = K[key = lane % 16][dim 16 (m / 4) +
//     4 (lane / 16) + m % 4], B = Q[query = lane % 16][same dim], for
//     m = 0..15; lane l's result register r is key 4 (l / 16) + r, query l % 16;
//   output O^T (dim x query), tile t: A = V[key 4 (l / 16) + r][dim 4 (l % 16)
//     + t], B = that lane's own probability r: no data moves between lanes.
// Each K load instruction reads 64 contiguous bytes of each of 16 keys (the
// four lanes of a key take its consecutive 16-byte chunks) and every V load
// four whole 256-byte rows. The next block's loads are issued
// before the current block's products, into the other of two register sets.
// The softmax is the lazy-reference form above; the waves' partial results
// are merged through LDS at the end.
constexpr int kDecodeQueries = 32;
constexpr int kDecodeWaves = 4;
constexpr int kDecodeOStride = 68;  // floats per query row of the LDS merge area

template <int QG, bool SPLIT>
__global__ __launch_bounds__(kDecodeWaves * 64, 2) void icl_decode_kernel(IclAttention p, IclLaunch g) {
    __shared__ float red_o[kDecodeWaves][QG * 16 * kDecodeOStride];
    __shared__ float red_m[kDecodeWaves][QG * 16], red_l[kDecodeWaves][QG * 16];
    const int wave = tid_x() >> 6, lane = tid_x() & 63, grp = lane >> 4, i16 = lane & 15;
    const int split = bid_x() % g.splits, pair = bid_x() / g.splits;
    const int k_begin = split * g.keys_per_split;
    const int k_end = min(p.kv_rows, k_begin + g.keys_per_split);

    float q[QG][16];
    {
        const float scale = 0.125f * kLog2e;
#pragma unroll
        for (int gq = 0; gq < QG; ++gq) {
            const int row = 16 * gq + i16;
            if (row < p.q_rows) {
                const float *src = p.q + pair * p.q_pair_stride + (long long)row * 64 + 4 * grp;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const f32x4 v = *reinterpret_cast<const f32x4 *>(src + 16 * c);
#pragma unroll
                    for (int e = 0; e < 4; ++e) q[gq][4 * c + e] = v[e] * scale;
                }
            } else {
#pragma unroll
                for (int m = 0; m < 16; ++m) q[gq][m] = 0.f;
            }
        }
    }
    const float *kbase = p.k + pair * p.kv_pair_stride;
    const float *vbase = p.v + pair * p.kv_pair_stride;
    // Block at k0: K dims 16 c + 4 grp .. +3 (c = 0..3) of key k0 + i16, and
    // V dims 4 i16 .. +3 of keys k0 + 4 grp + r. Keys past the range repeat
    // its last key (masked below). Addresses are 32-bit byte offsets from the
    // pair's uniform bases (the launcher checks that 256 bytes per key fit).
    const char *kb8 = reinterpret_cast<const char *>(kbase), *vb8 = reinterpret_cast<const char *>(vbase);
    auto load = [&](int k0, f32x4 *kd, f32x4 *vd) {
        const unsigned key = (unsigned)min(k0 + i16, k_end - 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) kd[c] = *reinterpret_cast<const f32x4 *>(kb8 + (key * 256u + 64u * c + 16u * grp));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const unsigned vk = (unsigned)min(k0 + 4 * grp + r, k_end - 1);
            vd[r] = *reinterpret_cast<const f32x4 *>(vb8 + (vk * 256u + 16u * i16));
        }
    };

    f32x4 o[QG][4];
    float neg_ref[QG], m_ref[QG], l_run[QG];
#pragma unroll
    for (int gq = 0; gq < QG; ++gq) {
#pragma unroll
        for (int t = 0; t < 4; ++t) o[gq][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        neg_ref[gq] = 0.f, m_ref[gq] = -INFINITY, l_run[gq] = 0.f;
    }
    constexpr float kLazyLimit = 18446744073709551616.0f;  // 2^64
    constexpr int kStride = 16 * kDecodeWaves;
    // The wave's first block sets the reference from its own maxima (its
    // scores start from zero); later blocks redo theirs only when their
    // probabilities could exceed 2^64.
    bool fresh = true;

    // One 16-key block at kk (kk < k_end): scores, lazy softmax, output.
    auto process = [&](int kk, const f32x4 *kf, const f32x4 *vf) {
        const bool tail = kk + 16 > k_end;
#pragma unroll
        for (int gq = 0; gq < QG; ++gq) {
            f32x4 s = {neg_ref[gq], neg_ref[gq], neg_ref[gq], neg_ref[gq]};
#pragma unroll
            for (int m = 0; m < 16; ++m) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[m >> 2][m & 3], q[gq][m], s, 0, 0, 0);
            if (tail) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (kk + 4 * grp + r >= k_end) s[r] = -INFINITY;
            }
            if (fresh) {
                float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
                mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
                mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
                neg_ref[gq] = -mt;
                m_ref[gq] = mt;
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] -= mt;
            }
            float lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = __builtin_amdgcn_exp2f(s[r]);
                lsum += s[r];
            }
            if (__any(!(lsum <= kLazyLimit))) {
                // Too low a reference: redo this block's scores from zero.
                s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int m = 0; m < 16; ++m)
                    s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[m >> 2][m & 3], q[gq][m], s, 0, 0, 0);
                if (tail) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (kk + 4 * grp + r >= k_end) s[r] = -INFINITY;
                }
                float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
                mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
                mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
                const float m_new = fmaxf(m_ref[gq], mt);
                const float alpha = __builtin_amdgcn_exp2f(m_ref[gq] - m_new);
                l_run[gq] *= alpha;
#pragma unroll
                for (int t = 0; t < 4; ++t) o[gq][t] *= alpha;
                neg_ref[gq] = -m_new;
                m_ref[gq] = m_new;
                lsum = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
                    lsum += s[r];
                }
            }
            l_run[gq] += lsum;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    o[gq][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[r][t], s[r], o[gq][t], 0, 0, 0);
        }
        fresh = false;
    };

    // Two register sets in turn: the next block's loads are always issued
    // (past the range they re-read its last key, a cached row) before the
    // current block's products, and no registers are copied between sets, so
    // each block waits only for its own loads.
    f32x4 k_a[4], v_a[4], k_b[4], v_b[4];
    int k0 = k_begin + 16 * wave;
    load(k0, k_a, v_a);
    while (k0 < k_end) {
        load(k0 + kStride, k_b, v_b);
        process(k0, k_a, v_a);
        k0 += kStride;
        if (k0 >= k_end) break;
        load(k0 + kStride, k_a, v_a);
        process(k0, k_b, v_b);
        k0 += kStride;
    }

    // Each wave's (reference, sum, unnormalised output) per query to LDS:
    // lane (grp, i16) holds dims 16 grp + 4 r + t of query 16 gq + i16.
#pragma unroll
    for (int gq = 0; gq < QG; ++gq) {
        float l = l_run[gq];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const int qi = 16 * gq + i16;
        if (grp == 0) red_m[wave][qi] = m_ref[gq], red_l[wave][qi] = l;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f32x4 v = {o[gq][0][r], o[gq][1][r], o[gq][2][r], o[gq][3][r]};
            *reinterpret_cast<f32x4 *>(&red_o[wave][qi * kDecodeOStride + 16 * grp + 4 * r]) = v;
        }
    }
    __syncthreads();
    // Merge: thread t takes query (t / 16) + 16 j and dims 4 (t % 16) .. +3.
    // A wave that got no block has reference -inf and sum 0.
#pragma unroll
    for (int j = 0; j < QG; ++j) {
        const int qi = (tid_x() >> 4) + 16 * j, d = 4 * (tid_x() & 15);
        if (qi >= p.q_rows) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) mx = fmaxf(mx, red_m[w][qi]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
            const float wgt = __builtin_amdgcn_exp2f(red_m[w][qi] - mx);
            acc += wgt * *reinterpret_cast<const f32x4 *>(&red_o[w][qi * kDecodeOStride + d]);
            den += wgt * red_l[w][qi];
        }
        const f32x4 out = acc * (1.0f / den);
        if constexpr (!SPLIT) {
            const int b = pair / kHeads, head = pair - b * kHeads;
            *reinterpret_cast<f32x4 *>(p.o + ((long long)b * p.q_rows + qi) * p.ldo + head * 64 + d) = out;
        } else {
            const long long row = ((long long)split * p.pairs + pair) * g.q_padded + qi;
            *reinterpret_cast<f32x4 *>(p.partial + row * 64 + d) = out;
            if (d == 0) p.partial[(long long)g.splits * p.pairs * g.q_padded * 64 + row] = mx + log2f(den);
        }
    }
}

// Few queries over the FP16 cache (optimize="auto"): as icl_decode_kernel,
// HBM-bound, now on half the bytes. Blocks of 32 keys on the 16x16x32 FP16
// MFMA, queries and probabilities split hi + lo as in the split kernel:
//   S^T block b (16 rows x 16 queries, 32 dims per product): row i is key
//     16 (i / 8) + 8 b + i % 8 of the block, A = K[that key][dims 32 m +
//     8 (lane / 16) .. +7], B = the lane's query; result register r of lane
//     l is row 4 (l / 16) + r, query l % 16;
//   O^T (16 dims x 16 queries per product, 32 keys): the lane's 8
//     probabilities (blocks 0 and 1, registers 0..3) are keys stored at
//     positions 8 (lane / 16) .. +7 of the block in V^T, so A is one 16-byte
//     load of V^T row dim.
// Every K load is 64 contiguous bytes per four lanes, every V^T load 64
// contiguous bytes of one dim row per four lanes.
// FP8: the same over the E4M3 cache, each load half as wide (8 bytes per
// lane) and converted to FP16 in registers; queries times the key scales
// rounded once to FP16, one product each, outputs times the value scales.
template <int QG, bool SPLIT, bool FP8 = false>
__global__ __launch_bounds__(kDecodeWaves * 64, 2) void icl_decode16_kernel(IclAttention p, IclLaunch g) {
    __shared__ float red_o[kDecodeWaves][QG * 16 * kDecodeOStride];
    __shared__ float red_m[kDecodeWaves][QG * 16], red_l[kDecodeWaves][QG * 16];
    const int wave = tid_x() >> 6, lane = tid_x() & 63, grp = lane >> 4, i16 = lane & 15;
    const int split = bid_x() % g.splits, pair = bid_x() / g.splits;
    const int k_begin = split * g.keys_per_split;
    const int k_end = min(p.kv_rows, k_begin + g.keys_per_split);
    const int n_pad = (p.kv_rows + kKeyTile - 1) / kKeyTile * kKeyTile;

    half8 qh[QG][2], ql[QG][2];
    {
        const float scale = 0.125f * kLog2e;
#pragma unroll
        for (int gq = 0; gq < QG; ++gq) {
            const int row = 16 * gq + i16;
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                float x[8];
                if (row < p.q_rows) {
                    const float *src = p.q + pair * p.q_pair_stride + (long long)row * 64 + 32 * m + 8 * grp;
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(src);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = a[e] * scale, x[4 + e] = b[e] * scale;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = 0.f;
                }
                if constexpr (FP8) {
                    const float *ks = p.kscale + pair * 64 + 32 * m + 8 * grp;
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] *= ks[e];
                    qh[gq][m] = round8(x);
                } else {
                    split8(x, qh[gq][m], ql[gq][m]);
                }
            }
        }
    }
    const unsigned short *kbase = p.k16 + (long long)pair * n_pad * 64;
    const unsigned short *vbase = p.v16 + (long long)pair * n_pad * 64;
    const unsigned char *kbase8 = p.k8 + (long long)pair * n_pad * 64;
    const unsigned char *vbase8 = p.v8 + (long long)pair * n_pad * 64;
    // The block's operands as loaded: 16 bytes per lane and operand (FP16),
    // or 8 (FP8, in the low half).
    // Block at k0 (a multiple of 32, at most n_pad - 32): K rows of S blocks
    // 0 and 1 (dims 32 m + 8 grp ..) and V^T rows 16 d + i16 at the block's
    // stored positions 8 grp ..
    auto load = [&](int k0, u32x4 *kd, u32x4 *vd) {
        const long long vt = (long long)(k0 >> 6) * 4096 + 32 * ((k0 >> 5) & 1) + 8 * grp;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int key = k0 + 16 * (i16 >> 3) + 8 * b + (i16 & 7);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const long long off = (long long)key * 64 + 32 * m + 8 * grp;
                if constexpr (FP8) {
                    const u32x2 w = *reinterpret_cast<const u32x2 *>(kbase8 + off);
                    kd[2 * b + m] = u32x4{w[0], w[1], 0u, 0u};
                } else {
                    kd[2 * b + m] = *reinterpret_cast<const u32x4 *>(kbase + off);
                }
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const long long off = vt + (long long)(16 * d + i16) * 64;
            if constexpr (FP8) {
                const u32x2 w = *reinterpret_cast<const u32x2 *>(vbase8 + off);
                vd[d] = u32x4{w[0], w[1], 0u, 0u};
            } else {
                vd[d] = *reinterpret_cast<const u32x4 *>(vbase + off);
            }
        }
    };
    auto operand = [](const u32x4 &w) {
        if constexpr (FP8)
            return fp8x8_to_half8(u32x2{w[0], w[1]});
        else
            return as_half8(w);
    };

    f32x4 o[QG][4];
    float neg_ref[QG], m_ref[QG], l_run[QG];
#pragma unroll
    for (int gq = 0; gq < QG; ++gq) {
#pragma unroll
        for (int d = 0; d < 4; ++d) o[gq][d] = f32x4{0.f, 0.f, 0.f, 0.f};
        neg_ref[gq] = 0.f, m_ref[gq] = -INFINITY, l_run[gq] = 0.f;
    }
    constexpr float kLazyLimit16 = 32768.0f;
    constexpr int kStride = 32 * kDecodeWaves;
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    bool fresh = true;  // the wave's first block sets the reference (as icl_decode_kernel)

    auto process = [&](int kk, const u32x4 *kf, const u32x4 *vf) {
        const bool tail = kk + 32 > k_end;
#pragma unroll
        for (int gq = 0; gq < QG; ++gq) {
            auto scores = [&](const f32x4 &init, f32x4 &s0, f32x4 &s1) {
                s0 = init, s1 = init;
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const half8 a0 = operand(kf[m]), a1 = operand(kf[2 + m]);
                    s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qh[gq][m], s0, 0, 0, 0);
                    s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qh[gq][m], s1, 0, 0, 0);
                    if constexpr (!FP8) {
                        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, ql[gq][m], s0, 0, 0, 0);
                        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, ql[gq][m], s1, 0, 0, 0);
                    }
                }
                if (tail) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * grp + r;
                        if (kk + 16 * (i >> 3) + (i & 7) >= k_end) s0[r] = -INFINITY;
                        if (kk + 16 * (i >> 3) + 8 + (i & 7) >= k_end) s1[r] = -INFINITY;
                    }
                }
            };
            const f32x4 nr = {neg_ref[gq], neg_ref[gq], neg_ref[gq], neg_ref[gq]};
            f32x4 s0, s1;
            scores(nr, s0, s1);
            if (fresh) {
                float mt = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                 fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
                mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
                mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
                neg_ref[gq] = -mt;
                m_ref[gq] = mt;
#pragma unroll
                for (int r = 0; r < 4; ++r) s0[r] -= mt, s1[r] -= mt;
            }
            float lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s0[r] = __builtin_amdgcn_exp2f(s0[r]);
                s1[r] = __builtin_amdgcn_exp2f(s1[r]);
                lsum += s0[r] + s1[r];
            }
            if (__any(!(lsum <= kLazyLimit16))) {
                f32x4 t0, t1;
                scores(zero4, t0, t1);
                float mt = fmaxf(fmaxf(fmaxf(t0[0], t0[1]), fmaxf(t0[2], t0[3])),
                                 fmaxf(fmaxf(t1[0], t1[1]), fmaxf(t1[2], t1[3])));
                mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
                mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
                const float m_new = fmaxf(m_ref[gq], mt);
                const float alpha = __builtin_amdgcn_exp2f(m_ref[gq] - m_new);
                l_run[gq] *= alpha;
#pragma unroll
                for (int d = 0; d < 4; ++d) o[gq][d] *= alpha;
                neg_ref[gq] = -m_new;
                m_ref[gq] = m_new;
                lsum = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s0[r] = __builtin_amdgcn_exp2f(t0[r] - m_new);
                    s1[r] = __builtin_amdgcn_exp2f(t1[r] - m_new);
                    lsum += s0[r] + s1[r];
                }
            }
            l_run[gq] += lsum;
            float x[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) x[r] = s0[r], x[4 + r] = s1[r];
            half8 ph, pl;
            if constexpr (FP8)
                ph = round8(x);
            else
                split8(x, ph, pl);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const half8 a = operand(vf[d]);
                o[gq][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, o[gq][d], 0, 0, 0);
                if constexpr (!FP8) o[gq][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, o[gq][d], 0, 0, 0);
            }
        }
        fresh = false;
    };

    // Two register sets in turn; loads past the range re-read the range's
    // own last block (just loaded, so served by the cache; results unused).
    // Clamping to the end of the whole cache instead would fetch one round of
    // the next range's keys per workgroup from HBM: a seventh more traffic at
    // 896 keys per range.
    u32x4 k_a[4], v_a[4], k_b[4], v_b[4];
    const int last = min(n_pad, (k_end + 31) / 32 * 32) - 32;
    int k0 = k_begin + 32 * wave;
    load(min(k0, last), k_a, v_a);
    while (k0 < k_end) {
        load(min(k0 + kStride, last), k_b, v_b);
        process(k0, k_a, v_a);
        k0 += kStride;
        if (k0 >= k_end) break;
        load(min(k0 + kStride, last), k_a, v_a);
        process(k0, k_b, v_b);
        k0 += kStride;
    }

    // Per-wave partials to LDS: lane (grp, i16) holds dims 16 d + 4 grp + r of query 16 gq + i16.
#pragma unroll
    for (int gq = 0; gq < QG; ++gq) {
        float l = l_run[gq];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const int qi = 16 * gq + i16;
        if (grp == 0) red_m[wave][qi] = m_ref[gq], red_l[wave][qi] = l;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            f32x4 v;
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = o[gq][d][r];
            *reinterpret_cast<f32x4 *>(&red_o[wave][qi * kDecodeOStride + 16 * d + 4 * grp]) = v;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < QG; ++j) {
        const int qi = (tid_x() >> 4) + 16 * j, d = 4 * (tid_x() & 15);
        if (qi >= p.q_rows) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) mx = fmaxf(mx, red_m[w][qi]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
            const float wgt = __builtin_amdgcn_exp2f(red_m[w][qi] - mx);
            acc += wgt * *reinterpret_cast<const f32x4 *>(&red_o[w][qi * kDecodeOStride + d]);
            den += wgt * red_l[w][qi];
        }
        f32x4 out = acc * (1.0f / den);
        if constexpr (FP8) out *= *reinterpret_cast<const f32x4 *>(p.vscale + pair * 64 + d);
        if constexpr (!SPLIT) {
            const int b = pair / kHeads, head = pair - b * kHeads;
            *reinterpret_cast<f32x4 *>(p.o + ((long long)b * p.q_rows + qi) * p.ldo + head * 64 + d) = out;
        } else {
            const long long row = ((long long)split * p.pairs + pair) * g.q_padded + qi;
            *reinterpret_cast<f32x4 *>(p.partial + row * 64 + d) = out;
            if (d == 0) p.partial[(long long)g.splits * p.pairs * g.q_padded * 64 + row] = mx + log2f(den);
        }
    }
}

// Merge of split partials by their log2-sum-exp, into tokens [b * q_rows +
// row, head * 64 + d]. Partial outputs are [splits, pairs, q_padded, 64],
// followed by the log2-sum-exps [splits, pairs, q_padded]. One single-wave
// workgroup per (pair, row), so even a one-row pass's eight merges spread
// over eight CUs: lane = split group (lane / 16, every fourth split) x four
// dims. Each round loads sixteen splits per group at once (the 64 splits of
// a decode pass in one round) and folds them into the lane's running
// reference; the four groups are combined at the end.
constexpr int kMergePerGroup = 16;
__global__ __launch_bounds__(64) void icl_merge_kernel(IclAttention p, int splits, int q_padded) {
    const long long pq = bid_x();
    if (pq >= (long long)p.pairs * p.q_rows) return;
    const int lane = tid_x() & 63, sg = lane >> 4, d = (lane & 15) * 4;
    const int qrow = (int)(pq % p.q_rows);
    const int pair = (int)(pq / p.q_rows);
    const long long step = (long long)p.pairs * q_padded;  // rows between splits
    const long long row0 = (long long)pair * q_padded + qrow;
    const float *lse = p.partial + (long long)splits * step * 64 + row0;
    float m_run = -INFINITY, den = 0.f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = sg; s0 < splits; s0 += 4 * kMergePerGroup) {
        float l8[kMergePerGroup];
        f32x4 v8[kMergePerGroup];
        // Slots past the splits re-read the last split and get weight 0
        // (unconditional loads, as in icl_merge_rows_kernel).
#pragma unroll
        for (int j = 0; j < kMergePerGroup; ++j) {
            const int s = s0 + 4 * j, sl = min(s, splits - 1);
            const float ls = lse[sl * step];
            v8[j] = *reinterpret_cast<const f32x4 *>(p.partial + (row0 + sl * step) * 64 + d);
            l8[j] = s < splits ? ls : -INFINITY;
        }
        float m_new = m_run;
#pragma unroll
        for (int j = 0; j < kMergePerGroup; ++j) m_new = fmaxf(m_new, l8[j]);
        const float a = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 while m_run is -inf
        num *= a, den *= a;
#pragma unroll
        for (int j = 0; j < kMergePerGroup; ++j) {
            const float w = __builtin_amdgcn_exp2f(l8[j] - m_new);
            num += w * v8[j];
            den += w;
        }
        m_run = m_new;
    }
#pragma unroll
    for (int off = 16; off <= 32; off *= 2) {
        const float m_o = __shfl_xor(m_run, off, 64), den_o = __shfl_xor(den, off, 64);
        f32x4 num_o;
#pragma unroll
        for (int e = 0; e < 4; ++e) num_o[e] = __shfl_xor(num[e], off, 64);
        const float m_new = fmaxf(m_run, m_o);
        if (m_new != -INFINITY) {  // both groups empty: nothing to combine
            const float a = __builtin_amdgcn_exp2f(m_run - m_new), b = __builtin_amdgcn_exp2f(m_o - m_new);
            num = a * num + b * num_o;
            den = a * den + b * den_o;
            m_run = m_new;
        }
    }
    if (sg != 0) return;
    const int b = pair / kHeads, head = pair - b * kHeads;
    *reinterpret_cast<f32x4 *>(p.o + ((long long)b * p.q_rows + qrow) * p.ldo + head * 64 + d) = num * (1.0f / den);
}

// Few splits (the build's self-attention, passes of many rows): a 16-lane
// group per (pair, query row), lane d4 taking dims 4 d4 .. +3, with every
// split's log2-sum-exp and partial row loaded at once; consecutive groups take
// consecutive rows of one pair, so a workgroup's loads of one split are one
// contiguous 4 KB run. A wave per row (icl_merge_kernel) leaves too few bytes
// in flight for these launches (the build's 5-split merge of 50,000 rows ran
// at 2.7 TB/s).
// pq0: the first (pair, query row) to merge, pair * q_rows + row (a tail
// launch's partials cover only the rows from its first unit on).
template <int MAXS>
__global__ __launch_bounds__(256) void icl_merge_rows_kernel(IclAttention p, IclLaunch g, long long pq0) {
    const long long pq = pq0 + (long long)bid_x() * 16 + (tid_x() >> 4);
    if (pq >= (long long)p.pairs * p.q_rows) return;
    const int splits = g.splits;
    const int d = (tid_x() & 15) * 4;
    const int qrow = (int)(pq % p.q_rows);
    const int pair = (int)(pq / p.q_rows);
    const long long step = g.part_rows;
    long long row0;
    if (g.tail_units) {
        const int qt = qrow / kIclQueries;
        row0 = (long long)(pair * g.qtiles + qt - g.unit0) * kIclQueries + (qrow - qt * kIclQueries);
    } else {
        row0 = (long long)pair * g.q_padded + qrow;
    }
    const float *lse = p.partial + (long long)splits * step * 64 + row0;
    // Branch-free loads: slots past the splits re-read the last split (a
    // cache hit) and get weight 0, so every slot is one unconditional load
    // (with a branch per slot the compiler duplicated the code per split
    // count and needed 212 registers at MAXS = 8).
    float l[MAXS];
    f32x4 v[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
        const int sl = min(s, splits - 1);
        const float ls = lse[sl * step];
        v[s] = *reinterpret_cast<const f32x4 *>(p.partial + (row0 + sl * step) * 64 + d);
        l[s] = s < splits ? ls : -INFINITY;
    }
    float m = l[0];
#pragma unroll
    for (int s = 1; s < MAXS; ++s) m = fmaxf(m, l[s]);
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
        const float w = __builtin_amdgcn_exp2f(l[s] - m);  // 0 past the splits
        num += w * v[s];
        den += w;
    }
    const int b = pair / kHeads, head = pair - b * kHeads;
    *reinterpret_cast<f32x4 *>(p.o + ((long long)b * p.q_rows + qrow) * p.ldo + head * 64 + d) = num * (1.0f / den);
}

IclLaunch plan_icl(int pairs, int q_rows, int kv_rows, int compute_units, bool f16 = false) {
    IclLaunch g{};
    if (q_rows <= kDecodeQueries) {
        // One workgroup per (pair, key range), about two per CU, at least 256
        // keys each. FP32 ranges are whole 16-key blocks, so the ranges come
        // out even and the grid is exactly two workgroups per CU where the keys
        // allow (50,000 keys x 8 pairs: 64 ranges of 784 keys; in whole rounds
        // of the four waves' blocks it was 61 and 12 CUs took one workgroup);
        // FP16 ranges are whole rounds of the waves' 32-key blocks (the
        // transposed V tiles hold 64 keys).
        g.qtiles = 1;
        g.q_padded = kDecodeQueries;
        const int want = std::max(1, (int)ceil_div(2LL * compute_units, pairs));
        const int splits = std::max(1, std::min(want, kv_rows / 256));
        const int round = f16 ? 32 * kDecodeWaves : 16;
        const int per = (int)ceil_div(ceil_div(kv_rows, splits), round) * round;
        g.keys_per_split = per;
        g.splits = (int)ceil_div(kv_rows, per);
        g.per_xcd = 0;
        g.count = pairs * g.splits;
        g.part_rows = (long long)pairs * g.q_padded;
        return g;
    }
    g.qtiles = (int)ceil_div(q_rows, kIclQueries);
    g.q_padded = g.qtiles * kIclQueries;
    const long long base = (long long)g.qtiles * pairs;
    const long long slots = compute_units;  // one workgroup per CU (its waves use up to 512 registers)
    const int max_splits = std::max(1, kv_rows / 512);
    int splits = 1;
    if (base < slots) {
        // Few queries: split the keys until one round of workgroups fills the chip.
        splits = std::min((int)ceil_div(slots, base), max_splits);
    } else {
        // Many: take the split count (up to 8) whose last round of workgroups is
        // fullest, preferring fewer splits unless more are clearly better.
        double best = 0.0;
        for (int s = 1; s <= std::min(8, max_splits); ++s) {
            const long long units = base * s, rounds = (units + slots - 1) / slots;
            const double fill = (double)units / (double)(rounds * slots);
            if (fill > best + 0.02) best = fill, splits = s;
        }
    }
    const int per = (int)ceil_div(ceil_div(kv_rows, splits), kKeyTile) * kKeyTile;
    g.keys_per_split = per;
    g.splits = (int)ceil_div(kv_rows, per);
    g.per_xcd = (int)ceil_div((long long)g.qtiles * pairs * g.splits, 8);
    g.count = g.qtiles * pairs * g.splits;
    g.part_rows = (long long)pairs * g.q_padded;
    return g;
}

// The FP32 wide kernel's plan. When its (query tile, pair) units fill at
// least one round of workgroups (one per CU), the whole rounds run every
// key in one workgroup each (final outputs: no partials, no merge) and the
// units left over, fewer than a round, are split over key ranges so that
// they fill one more round (the build's 50,000-row self-attention: 1,568
// units = six rounds and 32 units in 8 splits, where one plan for all units
// needed 5 splits, 30.6 rounds and a merge of every row). Otherwise the
// units are split as plan_icl says. tail.count = 0: no tail launch.
struct IclPlan {
    IclLaunch main, tail;
};

IclPlan plan_icl_fp32(int pairs, int q_rows, int kv_rows, int compute_units) {
    IclPlan pl{};
    pl.main = plan_icl(pairs, q_rows, kv_rows, compute_units, false);
    if (q_rows <= kDecodeQueries) return pl;
    const long long units = (long long)pl.main.qtiles * pairs, slots = std::max(1, compute_units);
    if (units < slots) return pl;
    const long long full = units / slots * slots, rest = units - full;
    IclLaunch &m = pl.main;
    m.splits = 1, m.keys_per_split = kv_rows, m.count = (int)full, m.per_xcd = (int)ceil_div(full, 8);
    if (rest > 0) {
        IclLaunch &t = pl.tail;
        t = m;
        // At most 16 splits: the rows merge kernel's limit.
        const long long max_splits = std::min(16, std::max(1, kv_rows / 512));
        const int want = (int)std::max<long long>(1, std::min(slots / rest, max_splits));
        t.keys_per_split = (int)ceil_div(ceil_div(kv_rows, want), kKeyTile) * kKeyTile;
        t.splits = (int)ceil_div(kv_rows, t.keys_per_split);
        t.unit0 = (int)full, t.tail_units = (int)rest;
        t.count = (int)(rest * t.splits);
        t.per_xcd = (int)ceil_div(t.count, 8);
        t.part_rows = rest * kIclQueries;
    }
    return pl;
}

// ---- 16-wide heads on matrix cores, many keys ----
//
// The inducing points of the column stage (128 queries per column and head)
// attend to every train row of the column (multihead_attn1 of the ISAB,
// cpu.rs:1180-1207), and a row's tokens attend to each other when the row
// has more than 128. One workgroup of four waves per (sequence, head, chunk
// of up to 128 queries, key range): wave w takes the range's 16-key blocks
// w, w + 4, ... for all of the chunk's queries, with the lazy running
// softmax of the ICL decode kernel (exp2 against a reference maximum that is
// raised only when a sum passes 2^64), and the four waves' results are
// merged through LDS. Products on v_mfma_f32_16x16x4f32:
//   S^T (16 keys x 16 queries): K-step st pairs lane group g with dim 4 g +
//     st, so a lane's K operands over the four steps are one 16-byte load
//     (key lane % 16, dims 4 g .. +3), and so are its Q operands; register r
//     of lane (j, g) is key 4 g + r, query j;
//   O^T (16 dims x 16 queries): step i puts key 4 g + i in k slot g, so the
//     score registers are the B operand as they are and lane (d, g) loads
//     V[4 g + i][d]; register r of lane (j, g) is dim 4 g + r of query j.
// When the chunks do not fill the chip the keys are also split over
// workgroups, which write normalised partial outputs and their log2 sums
// into the caller's partial buffer for small_merge_kernel.
constexpr int kLongWaves = 4;
constexpr int kLongQueries = 128;
constexpr int kLongOStride = 20;  // LDS rows of 16 outputs, padded

template <int QG, bool ROPE>
__global__ __launch_bounds__(64 * kLongWaves) void small_attention_long_kernel(SmallAttention p, int qchunks,
                                                                               int splits, int keys_per_split,
                                                                               int per_xcd, int count) {
    __shared__ __attribute__((aligned(16))) float red_o[kLongWaves][QG * 16 * kLongOStride];
    __shared__ float red_m[kLongWaves][QG * 16], red_l[kLongWaves][QG * 16];
    const int wave = tid_x() >> 6, lane = tid_x() & 63, g = lane >> 4, l16 = lane & 15;
    // Workgroups of one XCD take consecutive (split, chunk, head, sequence)
    // units: a token's heads share its cache lines (two 16-wide heads per
    // 128-byte line), which they then fetch into one L2.
    const int t = (int)(bid_x() & 7) * per_xcd + (int)(bid_x() >> 3);
    if (t >= count) return;
    const int split = t % splits;
    const int unit = t / splits;
    const int qc = unit % qchunks, item = unit / qchunks;
    const int head = item % p.heads, seq = item / p.heads;
    const int gs = seq / p.group, sq = seq - gs * p.group;
    const float *qb = p.q + gs * p.q_group + sq * p.q_seq + head * p.q_head;
    const float *kb = p.k + gs * p.k_group + sq * p.k_seq + head * p.k_head;
    const float *vb = p.v + gs * p.v_group + sq * p.v_seq + head * p.v_head;
    const int k_begin = split * keys_per_split;
    const int k_end = min(p.kv_rows, k_begin + keys_per_split);
    const int q0 = qc * kLongQueries;

    // Queries: lane (j, g) holds dims 4 g .. +3 of query q0 + 16 gq + j, RoPE'd and scaled.
    f32x4 qf[QG];
    {
        const float scale = p.scale * kLog2e;
#pragma unroll
        for (int gq = 0; gq < QG; ++gq) {
            const int row = q0 + 16 * gq + l16;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if (row < p.q_rows) {
                const float *src = qb + (long long)row * p.q_row;
                x = *reinterpret_cast<const f32x4 *>(src + 4 * g);
                if constexpr (ROPE) {
                    // dims (4 g + e) ^ 8 = (4 g ^ 8) + e
                    const f32x4 y = *reinterpret_cast<const f32x4 *>(src + (4 * g ^ 8));
                    const f32x4 c = *reinterpret_cast<const f32x4 *>(p.rope_cos + row * 16 + 4 * g);
                    const f32x4 s = *reinterpret_cast<const f32x4 *>(p.rope_sin + row * 16 + 4 * g);
                    x = x * c + y * s;
                }
            }
            qf[gq] = x * scale;
        }
    }

    // Block at kk: K dims 4 g .. +3 of key kk + lane % 16, and V dim lane % 16
    // of keys kk + 4 g + i. Keys past the range repeat its last key (masked).
    // Addresses are 32-bit byte offsets from the item's uniform bases (the
    // launcher checks that the keys' rows fit).
    const unsigned k_row = 4u * (unsigned)p.k_row, v_row = 4u * (unsigned)p.v_row;
    const char *kb8 = reinterpret_cast<const char *>(kb), *vb8 = reinterpret_cast<const char *>(vb);
    auto load = [&](int kk, f32x4 &kd, f32x4 &vd) {
        const unsigned key = (unsigned)min(kk + l16, k_end - 1);
        const unsigned ks = key * k_row;
        kd = *reinterpret_cast<const f32x4 *>(kb8 + (ks + 16u * g));
        if constexpr (ROPE) {
            const f32x4 y = *reinterpret_cast<const f32x4 *>(kb8 + (ks + 4u * (4 * g ^ 8)));
            const f32x4 c = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(p.rope_cos) + (key * 64u + 16u * g));
            const f32x4 s = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(p.rope_sin) + (key * 64u + 16u * g));
            kd = kd * c + y * s;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            vd[i] = *reinterpret_cast<const float *>(vb8 + ((unsigned)min(kk + 4 * g + i, k_end - 1) * v_row + 4u * l16));
    };

    f32x4 o[QG];
    float neg_ref[QG], m_ref[QG], l_run[QG];
#pragma unroll
    for (int gq = 0; gq < QG; ++gq) {
        o[gq] = f32x4{0.f, 0.f, 0.f, 0.f};
        neg_ref[gq] = INFINITY, m_ref[gq] = -INFINITY, l_run[gq] = 0.f;
    }
    constexpr float kLazyLimit = 18446744073709551616.0f;  // 2^64
    constexpr int kStride = 16 * kLongWaves;
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

    auto process = [&](int kk, const f32x4 &kf, const f32x4 &vf) {
        const bool tail = kk + 16 > k_end;
#pragma unroll
        for (int gq = 0; gq < QG; ++gq) {
            auto scores = [&](const f32x4 &init) {
                f32x4 s = init;
#pragma unroll
                for (int st = 0; st < 4; ++st) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[gq][st], s, 0, 0, 0);
                if (tail) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (kk + 4 * g + r >= k_end) s[r] = -INFINITY;
                }
                return s;
            };
            f32x4 s = scores(f32x4{neg_ref[gq], neg_ref[gq], neg_ref[gq], neg_ref[gq]});
            float lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = __builtin_amdgcn_exp2f(s[r]);
                lsum += s[r];
            }
            if (__any(!(lsum <= kLazyLimit))) {
                const f32x4 t = scores(zero4);
                float mt = fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]));
                mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
                mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
                const float m_new = fmaxf(m_ref[gq], mt);
                const float alpha = __builtin_amdgcn_exp2f(m_ref[gq] - m_new);
                l_run[gq] *= alpha;
                o[gq] *= alpha;
                neg_ref[gq] = -m_new;
                m_ref[gq] = m_new;
                lsum = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s[r] = __builtin_amdgcn_exp2f(t[r] - m_new);
                    lsum += s[r];
                }
            }
            l_run[gq] += lsum;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[gq] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[i], s[i], o[gq], 0, 0, 0);
        }
    };

    // Two register sets in turn: the next block's loads are issued before the
    // current block's products.
    f32x4 k_a, v_a, k_b, v_b;
    int kk = k_begin + 16 * wave;
    load(kk, k_a, v_a);
    while (kk < k_end) {
        load(kk + kStride, k_b, v_b);
        process(kk, k_a, v_a);
        kk += kStride;
        if (kk >= k_end) break;
        load(kk + kStride, k_a, v_a);
        process(kk, k_b, v_b);
        kk += kStride;
    }

    // Each wave's (reference, sum, unnormalised output) per query to LDS.
#pragma unroll
    for (int gq = 0; gq < QG; ++gq) {
        float l = l_run[gq];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const int qi = 16 * gq + l16;
        if (g == 0) red_m[wave][qi] = m_ref[gq], red_l[wave][qi] = l;
        *reinterpret_cast<f32x4 *>(&red_o[wave][qi * kLongOStride + 4 * g]) = o[gq];
    }
    __syncthreads();
    // Merge: thread t takes query t / 2 of the chunk, dims 8 (t % 2) .. +7. A
    // wave that got no block has reference -inf and sum 0; wave 0 always has one.
    const int qi = tid_x() >> 1, d0 = 8 * (tid_x() & 1);
    const int row = q0 + qi;
    if (qi >= QG * 16 || row >= p.q_rows) return;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kLongWaves; ++w) mx = fmaxf(mx, red_m[w][qi]);
    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
    float den = 0.f;
#pragma unroll
    for (int w = 0; w < kLongWaves; ++w) {
        const float wgt = __builtin_amdgcn_exp2f(red_m[w][qi] - mx);
        a0 += wgt * *reinterpret_cast<const f32x4 *>(&red_o[w][qi * kLongOStride + d0]);
        a1 += wgt * *reinterpret_cast<const f32x4 *>(&red_o[w][qi * kLongOStride + d0 + 4]);
        den += wgt * red_l[w][qi];
    }
    const float inv = 1.0f / den;
    float *dst;
    if (splits == 1) {
        dst = p.o + gs * p.o_group + sq * p.o_seq + (long long)row * p.o_row + head * p.o_head + d0;
    } else {
        const long long prow = ((long long)split * p.seqs * p.heads + item) * p.q_rows + row;
        dst = p.partial + prow * 16 + d0;
        if (d0 == 0) p.partial[(long long)splits * p.seqs * p.heads * p.q_rows * 16 + prow] = mx + log2f(den);
    }
    *reinterpret_cast<f32x4 *>(dst) = a0 * inv;
    *reinterpret_cast<f32x4 *>(dst + 4) = a1 * inv;
}

// Combines the key ranges of small_attention_long_kernel: thread per (sequence
// and head, query, four dims).
__global__ __launch_bounds__(256) void small_merge_kernel(SmallAttention p, int splits) {
    const long long items = (long long)p.seqs * p.heads;
    const long long idx = (long long)bid_x() * 256 + tid_x();
    const int c = (int)(idx & 3);
    const long long unit = idx >> 2;
    if (unit >= items * p.q_rows) return;
    const int row = (int)(unit % p.q_rows);
    const long long item = unit / p.q_rows;
    const long long stride = items * p.q_rows;
    const float *lse = p.partial + (long long)splits * stride * 16;
    float mx = -INFINITY;
    for (int s = 0; s < splits; ++s) mx = fmaxf(mx, lse[s * stride + unit]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
    for (int s = 0; s < splits; ++s) {
        const float wgt = __builtin_amdgcn_exp2f(lse[s * stride + unit] - mx);
        acc += wgt * *reinterpret_cast<const f32x4 *>(p.partial + (s * stride + unit) * 16 + 4 * c);
        den += wgt;
    }
    const int head = (int)(item % p.heads), seq = (int)(item / p.heads);
    const int gs = seq / p.group, sq = seq - gs * p.group;
    float *dst = p.o + gs * p.o_group + sq * p.o_seq + (long long)row * p.o_row + head * p.o_head + 4 * c;
    *reinterpret_cast<f32x4 *>(dst) = acc * (1.0f / den);
}

// ---- 16-wide heads on matrix cores, up to 128 keys ----
//
// One wave per (sequence, head) and a chunk of 16 * QB queries (the wave
// loops over every waves_per_seq-th chunk). The wave stages its keys (RoPE
// applied) and the transposed values into its own LDS, then per chunk
// computes S^T = K Q^T with v_mfma_f32_16x16x4f32 and keeps every score of
// its queries in registers: lane l holds keys 16 b + 4 (l / 16) + r of query
// l % 16 of each block. The softmax is exact (no running rescale); O^T = V^T
// P^T takes the score registers as its operand, the four k slots of MFMA i
// being keys 16 b + 4 g + i. K-step st of the first product pairs lane group
// g with dim 4 g + st, so each lane's Q and K operands are one 16-byte load.
constexpr int kShortKeys = 128;     // keys the matrix-core path takes
constexpr int kShortKStride = 20;   // K rows padded to 20 floats

template <int QB, int KB, bool ROPE, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void small_attention_mfma_kernel(SmallAttention p, int groups_per_seq,
                                                                          int per_xcd, int count) {
    // Rows are padded against bank conflicts, except for 80 keys (the
    // 68-token rows of 64 features): unpadded, one item's K and V^T take
    // exactly 10 KB, so sixteen single-wave workgroups fit a CU's LDS and a
    // 512-row pass (4,096 items) runs in one round.
    constexpr int KEYS = KB * 16, KSTRIDE = KB == 5 ? 16 : kShortKStride, VSTRIDE = KB == 5 ? KEYS : KEYS + 4;
    __shared__ __attribute__((aligned(16))) float Ks[KEYS * KSTRIDE];
    __shared__ __attribute__((aligned(16))) float Vt[16 * VSTRIDE];
    // Workgroup j of a (sequence, head) item: its WAVES waves take query chunks
    // (j * WAVES + wave) + k * groups_per_seq * WAVES and share the staged keys.
    // Workgroups of one XCD take consecutive (group, head, sequence) units,
    // so a token's heads fetch its cache lines into one L2.
    const int t = (int)(bid_x() & 7) * per_xcd + (int)(bid_x() >> 3);
    if (t >= count) return;
    const int item = t / groups_per_seq;
    const int wave = tid_x() >> 6;
    const int c_first = (t - item * groups_per_seq) * WAVES + wave;
    const int c_step = groups_per_seq * WAVES;
    const int head = item % p.heads, seq = item / p.heads;
    const int gq = seq / p.group, sq = seq - gq * p.group;
    const float *qb = p.q + gq * p.q_group + sq * p.q_seq + head * p.q_head;
    const float *kb = p.k + gq * p.k_group + sq * p.k_seq + head * p.k_head;
    const float *vb = p.v + gq * p.v_group + sq * p.v_seq + head * p.v_head;
    float *ob = p.o + gq * p.o_group + sq * p.o_seq + head * p.o_head;
    const int lane = tid_x() & 63, g = lane >> 4, l16 = lane & 15;
    const int kv = p.kv_rows;
    const int kblocks = (kv + 15) / 16;

    // Stage K (rotated) as [key][20] and V transposed as [dim][KEYS + 4]; keys past kv are zero.
    for (int key = tid_x(); key < kblocks * 16; key += 64 * WAVES) {
        float kr[16], vr[16];
        if (key < kv) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const f32x4 a = *reinterpret_cast<const f32x4 *>(kb + (long long)key * p.k_row + 4 * c);
                const f32x4 b = *reinterpret_cast<const f32x4 *>(vb + (long long)key * p.v_row + 4 * c);
#pragma unroll
                for (int e = 0; e < 4; ++e) kr[4 * c + e] = a[e], vr[4 * c + e] = b[e];
            }
            if constexpr (ROPE) {
                const float *cs = p.rope_cos + key * 16, *sn = p.rope_sin + key * 16;
                float r[16];
#pragma unroll
                for (int d = 0; d < 16; ++d) r[d] = kr[d] * cs[d] + kr[d ^ 8] * sn[d];
#pragma unroll
                for (int d = 0; d < 16; ++d) kr[d] = r[d];
            }
        } else {
#pragma unroll
            for (int d = 0; d < 16; ++d) kr[d] = 0.f, vr[d] = 0.f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f32x4 a;
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] = kr[4 * c + e];
            *reinterpret_cast<f32x4 *>(&Ks[key * KSTRIDE + 4 * c]) = a;
        }
#pragma unroll
        for (int d = 0; d < 16; ++d) Vt[d * VSTRIDE + key] = vr[d];
    }
    __syncthreads();

    const float scale = p.scale * kLog2e;
    // Query blocks J0 .. J0 + NJ - 1 of the chunk at q0: scores, softmax and
    // output. A chunk of more than three blocks runs in two such groups, so
    // the scores of at most three blocks are live at once (at five, the
    // 80-query chunk of a 68-token row held 148 registers, three waves per
    // SIMD, and a 512-row pass's 4,096 workgroups took a second round).
    auto blocks_of = [&]<int J0, int NJ>(int q0) {
        // This lane's query operands: dims 4g .. 4g+3 of query q0 + 16 (J0 + j) + l16.
        f32x4 qf[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int row = q0 + 16 * (J0 + j) + l16;
            f32x4 q = {0.f, 0.f, 0.f, 0.f};
            if (row < p.q_rows) {
                const float *src = qb + (long long)row * p.q_row;
                q = *reinterpret_cast<const f32x4 *>(src + 4 * g);
                if constexpr (ROPE) {
                    // Rotate-half pairs dim d with d ^ 8, held in dims 4 (g ^ 2) .. of the same row.
                    const f32x4 qp = *reinterpret_cast<const f32x4 *>(src + 4 * (g ^ 2));
                    const f32x4 cs = *reinterpret_cast<const f32x4 *>(p.rope_cos + row * 16 + 4 * g);
                    const f32x4 sn = *reinterpret_cast<const f32x4 *>(p.rope_sin + row * 16 + 4 * g);
                    q = q * cs + qp * sn;
                }
            }
            qf[j] = q * scale;
        }
        // Scores S^T for every key block.
        f32x4 s[NJ][KB];
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            if (b < kblocks) {
                const f32x4 kf = *reinterpret_cast<const f32x4 *>(&Ks[(16 * b + l16) * KSTRIDE + 4 * g]);
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int st = 0; st < 4; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[j][st], acc, 0, 0, 0);
                    s[j][b] = acc;
                }
            } else {
#pragma unroll
                for (int j = 0; j < NJ; ++j) s[j][b] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            }
        }
        if (kv < kblocks * 16) {
            const int b = kblocks - 1;
#pragma unroll
            for (int bb = 0; bb < KB; ++bb) {
                if (bb != b) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (16 * bb + 4 * g + r >= kv)
#pragma unroll
                        for (int j = 0; j < NJ; ++j) s[j][bb][r] = -INFINITY;
            }
        }
        // Exact softmax per query: lanes l16, l16 + 16, l16 + 32, l16 + 48 share a query.
        float inv[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            float m = -INFINITY;
#pragma unroll
            for (int b = 0; b < KB; ++b)
                if (b < kblocks) m = fmaxf(m, fmaxf(fmaxf(s[j][b][0], s[j][b][1]), fmaxf(s[j][b][2], s[j][b][3])));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            float l = 0.f;
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                if (b < kblocks) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        s[j][b][r] = __builtin_amdgcn_exp2f(s[j][b][r] - m);
                        l += s[j][b][r];
                    }
                }
            }
            l += __shfl_xor(l, 16, 64);
            l += __shfl_xor(l, 32, 64);
            inv[j] = 1.0f / l;
        }
        // O^T = V^T P^T.
        f32x4 o[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            if (b < kblocks) {
                const f32x4 vf = *reinterpret_cast<const f32x4 *>(&Vt[l16 * VSTRIDE + 16 * b + 4 * g]);
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[i], s[j][b][i], o[j], 0, 0, 0);
            }
        }
        // Lane l holds O[query q0 + 16 (J0 + j) + l16][dims 4g .. 4g+3].
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int row = q0 + 16 * (J0 + j) + l16;
            if (row < p.q_rows) *reinterpret_cast<f32x4 *>(ob + (long long)row * p.o_row + 4 * g) = o[j] * inv[j];
        }
    };
    const int chunks = (p.q_rows + 16 * QB - 1) / (16 * QB);
    for (int c = c_first; c < chunks; c += c_step) {
        const int q0 = c * 16 * QB;
        if constexpr (QB <= 3) {
            blocks_of.template operator()<0, QB>(q0);
        } else {
            constexpr int kFirst = (QB + 1) / 2;
            blocks_of.template operator()<0, kFirst>(q0);
            blocks_of.template operator()<kFirst, QB - kFirst>(q0);
        }
    }
}

// ---- 16-wide heads, every key staged once per item, query blocks over waves ----
//
// The row transformer's self-attention (row_embedding, cpu.rs:1226-1266:
// H + 4 tokens per row, RoPE on queries and keys) and the CLS block's four
// queries over every token. One workgroup of W waves per (sequence, head,
// chunk of W * NG query blocks of 16): its threads stage the item's keys once
// (RoPE applied, rows padded to 20 floats) and the values transposed into
// LDS, then wave w takes the chunk's blocks w, w + W, ... (NG of them) over
// every key, with the lazy running softmax of the long kernel: the scores
// are exp2 against a reference that moves only when a lane's four
// probabilities would sum past 2^64. The first key block sets the reference
// from its own maxima, so no block is computed twice unless a score rises
// 64 (log2 units) above it. A wave ends with its queries' final outputs: no
// merge between waves or workgroups. Products on v_mfma_f32_16x16x4f32 in
// the long kernel's transposed layout (S^T = K Q^T, O^T = V^T P^T).
// Workgroups of one XCD take consecutive items, so the 8 heads of a
// sequence, which share each token's 128-byte lines, are read into one L2.
constexpr int kStagedKStride = 20;

template <int NG, int KMAX, bool ROPE>
__global__ __launch_bounds__(1024, NG == 1 ? 8 : NG == 2 ? 6 : 4) void staged_attention_kernel(SmallAttention p, int chunks, int per_xcd) {
    constexpr int VSTRIDE = KMAX + 4;
    __shared__ __attribute__((aligned(16))) float Ks[KMAX * kStagedKStride];
    __shared__ __attribute__((aligned(16))) float Vt[16 * VSTRIDE];
    // Index arithmetic in 32 bits (the launcher caps units below 2^31), with
    // shifts for the row transformer's 8 heads and one chunk per item.
    const int unit = (int)(bid_x() & 7) * per_xcd + (int)(bid_x() >> 3);
    if (unit >= p.seqs * p.heads * chunks) return;
    const int chunk = chunks == 1 ? 0 : unit % chunks;
    const int item = chunks == 1 ? unit : unit / chunks;
    const int head = p.heads == 8 ? (item & 7) : item % p.heads;
    const int seq = p.heads == 8 ? (item >> 3) : item / p.heads;
    const int gs = p.group >= p.seqs ? 0 : seq / p.group, sq = seq - gs * p.group;
    const float *qb = p.q + gs * p.q_group + sq * p.q_seq + head * p.q_head;
    const float *kb = p.k + gs * p.k_group + sq * p.k_seq + head * p.k_head;
    const float *vb = p.v + gs * p.v_group + sq * p.v_seq + head * p.v_head;
    float *ob = p.o + gs * p.o_group + sq * p.o_seq + head * p.o_head;
    const int waves = bdim_x() >> 6, wave = tid_x() >> 6;
    const int lane = tid_x() & 63, g = lane >> 4, l16 = lane & 15;
    const int kv = p.kv_rows, kblocks = (kv + 15) >> 4;
    const int first_block = chunk * waves * NG + wave;

    // Stage K (rotated) as [key][20] and V^T as [dim][KMAX + 4]; keys past kv
    // (in the last block only) repeat key kv - 1, whose scores the last block
    // masks. Thread t takes dims 4 c .. +3 (c = t / 16 % 4) of key
    // 16 (t / 64) + t % 16: each 16-lane phase of a store covers 16
    // consecutive keys of one chunk, which no two lanes' banks share in
    // either layout. RoPE pairs dim d with d ^ 8, chunk c with c ^ 2.
    // Offsets within an item are 32-bit byte offsets (the launcher checks)
    // from the workgroup-uniform bases, so every load takes a scalar base.
    const unsigned k_row = 4u * (unsigned)p.k_row, v_row = 4u * (unsigned)p.v_row;
    const unsigned q_row = 4u * (unsigned)p.q_row, o_row = 4u * (unsigned)p.o_row;
    auto ld4 = [](const float *base, unsigned bytes) {
        return *reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(base) + bytes);
    };
    auto stage = [&](int t) {
        const unsigned key = ((t >> 6) << 4) | (t & 15), c = (t >> 4) & 3;
        const unsigned src = min(key, (unsigned)kv - 1);
        f32x4 kc = ld4(kb, src * k_row + 16 * c);
        const f32x4 vc = ld4(vb, src * v_row + 16 * c);
        if constexpr (ROPE) {
            const f32x4 kp = ld4(kb, src * k_row + 16 * (c ^ 2));
            const f32x4 cs = ld4(p.rope_cos, src * 64 + 16 * c);
            const f32x4 sn = ld4(p.rope_sin, src * 64 + 16 * c);
            kc = kc * cs + kp * sn;
        }
        *reinterpret_cast<f32x4 *>(&Ks[key * kStagedKStride + 4 * c]) = kc;
#pragma unroll
        for (int e = 0; e < 4; ++e) Vt[(4 * c + e) * VSTRIDE + key] = vc[e];
    };
    if (kblocks * 64 <= (int)bdim_x()) {
        // One pass covers every key (self-attention: a wave per 16-key block).
        if (tid_x() < kblocks * 64) stage(tid_x());
    } else {
        for (int t = tid_x(); t < kblocks * 64; t += bdim_x()) stage(t);
    }

    // This wave's queries, rotated and scaled into the exp2 domain: lane
    // (j, g) holds dims 4 g .. +3 of query 16 (first_block + n waves) + j.
    f32x4 qf[NG];
    {
        const float scale = p.scale * kLog2e;
#pragma unroll
        for (int n = 0; n < NG; ++n) {
            // Rows past q_rows repeat the last query (their outputs are not stored).
            const unsigned row = min(16u * (first_block + n * waves) + l16, (unsigned)p.q_rows - 1);
            f32x4 q = ld4(qb, row * q_row + 16 * g);
            if constexpr (ROPE) {
                const f32x4 qp = ld4(qb, row * q_row + 16 * (g ^ 2));
                const f32x4 cs = ld4(p.rope_cos, row * 64 + 16 * g);
                const f32x4 sn = ld4(p.rope_sin, row * 64 + 16 * g);
                q = q * cs + qp * sn;
            }
            qf[n] = q * scale;
        }
    }
    __syncthreads();

    f32x4 o[NG], neg[NG];
    float l_run[NG];
    constexpr float kLazyLimit = 18446744073709551616.0f;  // 2^64
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    // Maximum / sum over the four lanes l16 + 16 g that share a query.
    auto quad_max = [](float m) {
        auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
        m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
        auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
        return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
    };
    auto quad_sum = [](float m) {
        auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
        m = __uint_as_float(a[0]) + __uint_as_float(a[1]);
        auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
        return __uint_as_float(b[0]) + __uint_as_float(b[1]);
    };
    const float *k_lane = &Ks[l16 * kStagedKStride + 4 * g], *v_lane = &Vt[l16 * VSTRIDE + 4 * g];
    auto load_k = [&](int b) { return *reinterpret_cast<const f32x4 *>(k_lane + b * (16 * kStagedKStride)); };
    auto load_v = [&](int b) { return *reinterpret_cast<const f32x4 *>(v_lane + b * 16); };
    // Key block b with operands kf, vf. FIRST: the reference is this block's
    // maximum. MASK: keys at or past kv score -inf (only the last block can
    // hold them).
    auto block = [&]<bool FIRST, bool MASK>(int b, const f32x4 &kf, const f32x4 &vf) {
        auto scores = [&](int n, const f32x4 &init) {
            f32x4 s = init;
#pragma unroll
            for (int st = 0; st < 4; ++st) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[n][st], s, 0, 0, 0);
            if constexpr (MASK) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (16 * b + 4 * g + r >= kv) s[r] = -INFINITY;
            }
            return s;
        };
#pragma unroll
        for (int n = 0; n < NG; ++n) {
            f32x4 s;
            if constexpr (FIRST) {
                const f32x4 t = scores(n, zero4);
                const float m = quad_max(fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3])));
                neg[n] = f32x4{-m, -m, -m, -m};
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = __builtin_amdgcn_exp2f(t[r] - m);
                l_run[n] = (s[0] + s[1]) + (s[2] + s[3]);
            } else {
                s = scores(n, neg[n]);
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = __builtin_amdgcn_exp2f(s[r]);
                float lsum = (s[0] + s[1]) + (s[2] + s[3]);
                if (__any(!(lsum <= kLazyLimit))) {
                    const f32x4 t = scores(n, zero4);
                    const float m_old = -neg[n][0];
                    const float m_new = fmaxf(m_old, quad_max(fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]))));
                    const float alpha = __builtin_amdgcn_exp2f(m_old - m_new);
                    l_run[n] *= alpha;
                    o[n] *= alpha;
                    neg[n] = f32x4{-m_new, -m_new, -m_new, -m_new};
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[r] = __builtin_amdgcn_exp2f(t[r] - m_new);
                    lsum = (s[0] + s[1]) + (s[2] + s[3]);
                }
                l_run[n] += lsum;
            }
            f32x4 acc = FIRST ? zero4 : o[n];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[i], s[i], acc, 0, 0, 0);
            o[n] = acc;
        }
    };
    const bool ragged = kv < kblocks * 16;
    if (kblocks == 1) {
        if (ragged)
            block.template operator()<true, true>(0, load_k(0), load_v(0));
        else
            block.template operator()<true, false>(0, load_k(0), load_v(0));
    } else {
        // Each block's operands are read from LDS a block ahead, into two
        // register sets in turn: (ka, va) holds block b's at the loop's top.
        f32x4 ka = load_k(1), va = load_v(1);
        block.template operator()<true, false>(0, load_k(0), load_v(0));
        const int full_end = ragged ? kblocks - 1 : kblocks;
        int b = 1;
        for (; b + 2 <= full_end; b += 2) {
            const f32x4 kb2 = load_k(b + 1), vb2 = load_v(b + 1);
            block.template operator()<false, false>(b, ka, va);
            const int nb = min(b + 2, kblocks - 1);
            ka = load_k(nb), va = load_v(nb);
            block.template operator()<false, false>(b + 1, kb2, vb2);
        }
        if (b < full_end) {
            block.template operator()<false, false>(b, ka, va);
            ++b;
            ka = load_k(min(b, kblocks - 1)), va = load_v(min(b, kblocks - 1));
        }
        if (ragged) block.template operator()<false, true>(kblocks - 1, ka, va);
    }

    // Lane (j, g) holds O[query][dims 4 g .. +3]; the query's sum is over its four lanes.
#pragma unroll
    for (int n = 0; n < NG; ++n) {
        const float l = quad_sum(l_run[n]);
        const unsigned row = 16 * (first_block + n * waves) + l16;
        if (row < (unsigned)p.q_rows)
            *reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(ob) + (row * o_row + 16 * g)) =
                o[n] * __builtin_amdgcn_rcpf(l);
    }
}

}  // namespace

size_t icl_attention_partial_floats(int pairs, int q_rows, int kv_rows, int compute_units, bool f16) {
    if (pairs <= 0 || q_rows <= 0 || kv_rows <= 0) return 0;
    auto floats = [](const IclLaunch &g) { return g.splits > 1 ? (size_t)g.splits * g.part_rows * 65 : (size_t)0; };
    if (!f16) {
        const IclPlan pl = plan_icl_fp32(pairs, q_rows, kv_rows, compute_units);
        return std::max(floats(pl.main), pl.tail.count ? floats(pl.tail) : (size_t)0);
    }
    return floats(plan_icl(pairs, q_rows, kv_rows, compute_units, true));
}

void icl_attention(const IclAttention &args, hipStream_t stream) {
    if (args.pairs <= 0 || args.q_rows <= 0) return;
    if (args.kv_rows <= 0) fail(3, "ICL attention needs at least one key");
    if ((reinterpret_cast<uintptr_t>(args.q) & 15) || (reinterpret_cast<uintptr_t>(args.k) & 15) ||
        (reinterpret_cast<uintptr_t>(args.v) & 15) || (reinterpret_cast<uintptr_t>(args.o) & 15) ||
        (reinterpret_cast<uintptr_t>(args.partial) & 15) || (args.q_pair_stride & 3) || (args.kv_pair_stride & 3) ||
        (args.ldo & 3))
        fail(3, "ICL attention operands must be 16-byte aligned");
    const bool fp8 = args.k8 != nullptr;
    if (args.k16 && (!args.v16 || (reinterpret_cast<uintptr_t>(args.k16) & 15) || (reinterpret_cast<uintptr_t>(args.v16) & 15)))
        fail(3, "ICL attention FP16 cache must be 16-byte aligned");
    if (fp8 && (!args.v8 || !args.kscale || !args.vscale || (reinterpret_cast<uintptr_t>(args.k8) & 15) ||
                (reinterpret_cast<uintptr_t>(args.v8) & 15) || (reinterpret_cast<uintptr_t>(args.kscale) & 15) ||
                (reinterpret_cast<uintptr_t>(args.vscale) & 15)))
        fail(3, "ICL attention FP8 cache and scales must be 16-byte aligned");
    // The FP8 cache uses the FP16 cache's tiling.
    const bool f16 = args.k16 != nullptr || fp8;
    // Workgroup indices and unit counts are 32-bit in the kernels.
    if ((long long)ceil_div((size_t)args.q_rows, kIclQueries) * args.pairs * 64 > INT32_MAX)
        fail(3, "ICL attention shape exceeds the kernels' 32-bit workgroup indices");
    IclPlan pl{};
    if (f16)
        pl.main = plan_icl(args.pairs, args.q_rows, args.kv_rows, args.compute_units, true);
    else
        pl = plan_icl_fp32(args.pairs, args.q_rows, args.kv_rows, args.compute_units);
    const IclLaunch &g = pl.main;
    const bool tail = pl.tail.count > 0;
    {
        const size_t need = icl_attention_partial_floats(args.pairs, args.q_rows, args.kv_rows, args.compute_units, f16);
        if (need && (!args.partial || args.partial_floats < need)) fail(3, "ICL attention partial buffer is too small");
    }
    {
        const double pairs = args.pairs, q = args.q_rows, kv = args.kv_rows;
        const double elem = fp8 ? 1.0 : f16 ? 2.0 : 4.0;
        const double kv_bytes = elem * 64.0 * pairs * 2.0 * kv;
        KernelTimer timer(kFamIcl, stream, 4.0 * pairs * q * kv * 64.0, kv_bytes + 4.0 * 64.0 * pairs * 2.0 * q);
        auto decode16 = [&]<bool FP8>() {
            const dim3 blocks((unsigned)((long long)args.pairs * g.splits)), threads(kDecodeWaves * 64);
            if (args.q_rows <= 16) {
                if (g.splits > 1)
                    hipLaunchKernelGGL((icl_decode16_kernel<1, true, FP8>), blocks, threads, 0, stream, args, g);
                else
                    hipLaunchKernelGGL((icl_decode16_kernel<1, false, FP8>), blocks, threads, 0, stream, args, g);
            } else {
                if (g.splits > 1)
                    hipLaunchKernelGGL((icl_decode16_kernel<2, true, FP8>), blocks, threads, 0, stream, args, g);
                else
                    hipLaunchKernelGGL((icl_decode16_kernel<2, false, FP8>), blocks, threads, 0, stream, args, g);
            }
        };
        auto wide16 = [&]<bool FP8>() {
            if (g.splits > 1)
                hipLaunchKernelGGL((icl_attention_split_kernel<true, FP8>), dim3(g.per_xcd * 8), dim3(kIclWaves * 64),
                                   0, stream, args, g);
            else
                hipLaunchKernelGGL((icl_attention_split_kernel<false, FP8>), dim3(g.per_xcd * 8),
                                   dim3(kIclWaves * 64), 0, stream, args, g);
        };
        if (f16 && args.q_rows <= kDecodeQueries) {
            if (fp8)
                decode16.template operator()<true>();
            else
                decode16.template operator()<false>();
        } else if (f16) {
            if (fp8)
                wide16.template operator()<true>();
            else
                wide16.template operator()<false>();
        } else if (args.q_rows <= kDecodeQueries) {
            if ((long long)args.kv_rows * 256 > 0xffffffffLL) fail(3, "ICL attention: too many keys for the decode kernel");
            const dim3 blocks((unsigned)((long long)args.pairs * g.splits)), threads(kDecodeWaves * 64);
            if (args.q_rows <= 16) {
                if (g.splits > 1)
                    hipLaunchKernelGGL((icl_decode_kernel<1, true>), blocks, threads, 0, stream, args, g);
                else
                    hipLaunchKernelGGL((icl_decode_kernel<1, false>), blocks, threads, 0, stream, args, g);
            } else {
                if (g.splits > 1)
                    hipLaunchKernelGGL((icl_decode_kernel<2, true>), blocks, threads, 0, stream, args, g);
                else
                    hipLaunchKernelGGL((icl_decode_kernel<2, false>), blocks, threads, 0, stream, args, g);
            }
        } else {
            // Ranges of more than 2 x kFlushTiles tiles accumulate in two levels.
            auto wide = [&](const IclLaunch &l) {
                const dim3 grid(l.per_xcd * 8), block(kIclWaves * 64);
                const bool flush = l.keys_per_split > 2 * kFlushTiles * kKeyTile;
                if (l.splits > 1 && flush)
                    hipLaunchKernelGGL((icl_attention_kernel<true, true>), grid, block, 0, stream, args, l);
                else if (l.splits > 1)
                    hipLaunchKernelGGL((icl_attention_kernel<true, false>), grid, block, 0, stream, args, l);
                else if (flush)
                    hipLaunchKernelGGL((icl_attention_kernel<false, true>), grid, block, 0, stream, args, l);
                else
                    hipLaunchKernelGGL((icl_attention_kernel<false, false>), grid, block, 0, stream, args, l);
            };
            wide(g);
            if (tail) wide(pl.tail);
        }
        IRX_HIP(hipGetLastError());
    }
    // Merge the split rows: every row, or the tail launch's rows from its
    // first unit on.
    const IclLaunch &split = tail ? pl.tail : g;
    if (split.splits > 1) {
        long long pq0 = 0;
        if (tail) {
            const int pair0 = split.unit0 / split.qtiles, qt0 = split.unit0 - pair0 * split.qtiles;
            pq0 = (long long)pair0 * args.q_rows + (long long)qt0 * kIclQueries;
        }
        const long long rows = (long long)args.pairs * args.q_rows - pq0;
        KernelTimer timer(kFamIclMerge, stream, 0.0,
                          4.0 * ((double)split.splits * rows * 65.0 + (double)rows * 64.0));
        if (split.splits <= 2)
            hipLaunchKernelGGL(icl_merge_rows_kernel<2>, dim3(ceil_div(rows, 16)), dim3(256), 0, stream, args, split,
                               pq0);
        else if (split.splits <= 4)
            hipLaunchKernelGGL(icl_merge_rows_kernel<4>, dim3(ceil_div(rows, 16)), dim3(256), 0, stream, args, split,
                               pq0);
        else if (split.splits <= 8)
            hipLaunchKernelGGL(icl_merge_rows_kernel<8>, dim3(ceil_div(rows, 16)), dim3(256), 0, stream, args, split,
                               pq0);
        else if (split.splits <= 16)
            hipLaunchKernelGGL(icl_merge_rows_kernel<16>, dim3(ceil_div(rows, 16)), dim3(256), 0, stream, args, split,
                               pq0);
        else if (!tail)
            hipLaunchKernelGGL(icl_merge_kernel, dim3((unsigned)rows), dim3(64), 0, stream, args, split.splits,
                               split.q_padded);
        else
            fail(3, "ICL attention tail split exceeds the merge's 16 splits");
        IRX_HIP(hipGetLastError());
    }
}

// Launch shape of small_attention_long_kernel: one workgroup per (sequence,
// head, query chunk), and the keys split until about two workgroups per CU
// are in flight (ranges of at least 512 keys, in whole rounds of the four
// waves' 16-key blocks).
struct LongPlan {
    long long units;
    int qchunks, splits, keys_per_split;
    long long partial_floats;
};

LongPlan plan_long(const SmallAttention &a) {
    LongPlan p{};
    p.qchunks = (int)ceil_div(a.q_rows, kLongQueries);
    p.units = (long long)a.seqs * a.heads * p.qchunks;
    const long long want = ceil_div(2LL * 256, p.units);
    const int splits = (int)std::max<long long>(1, std::min<long long>({want, 64, a.kv_rows / 512}));
    const int round = 16 * kLongWaves;
    p.keys_per_split = (int)ceil_div(ceil_div(a.kv_rows, splits), round) * round;
    p.splits = (int)ceil_div(a.kv_rows, p.keys_per_split);
    p.partial_floats = (long long)p.splits * a.seqs * a.heads * a.q_rows * 17;
    return p;
}

// Launch shape of staged_attention_kernel: one chunk of query blocks per item
// where a workgroup of at most 16 waves holds them (one block per wave up to
// 16 blocks, two up to 32), else chunks of 64 blocks (16 waves of four).
struct StagedPlan {
    int ng, waves, chunks, kmax;
};

StagedPlan plan_staged(const SmallAttention &a) {
    StagedPlan p{};
    const int groups = (int)ceil_div(a.q_rows, 16);
    if (groups <= 16) {
        p.ng = 1, p.waves = groups, p.chunks = 1;
    } else if (groups <= 32) {
        p.ng = 2, p.waves = (int)ceil_div(groups, 2), p.chunks = 1;
    } else {
        p.ng = 4, p.waves = 16, p.chunks = (int)ceil_div(groups, 64);
    }
    const int kp = (int)ceil_div(a.kv_rows, 16) * 16;
    p.kmax = kp <= 80 ? 80 : kp <= 128 ? 128 : kp <= 256 ? 256 : kp <= 512 ? 512 : 0;
    return p;
}

// The staged kernel serves self-attention-shaped items: more than one query
// block and at most 512 keys.
bool staged_applies(const SmallAttention &a) { return a.q_rows > 16 && a.kv_rows <= 512; }

void launch_staged(const SmallAttention &a, hipStream_t stream) {
    const StagedPlan plan = plan_staged(a);
    const long long units = (long long)a.seqs * a.heads * plan.chunks;
    const long long per_xcd = ceil_div(units, 8);
    if (per_xcd * 8 > 0x7fffffffLL) fail(3, "small attention grid is too large");
    const long long span = std::max<long long>({(long long)a.q_rows * a.q_row, (long long)a.kv_rows * a.k_row,
                                                (long long)a.kv_rows * a.v_row, (long long)a.q_rows * a.o_row});
    if (4 * (span + 64) > 0xffffffffLL) fail(3, "small attention rows are too far apart for the staged kernel");
    const dim3 blocks((unsigned)(per_xcd * 8)), threads(64 * plan.waves);
    const bool rope = a.rope_cos != nullptr;
#define IRX_STAGED_CASE(NG, KMAX)                                                                               \
    if (plan.ng == NG && plan.kmax == KMAX) {                                                                   \
        if (rope)                                                                                               \
            hipLaunchKernelGGL((staged_attention_kernel<NG, KMAX, true>), blocks, threads, 0, stream, a,        \
                               plan.chunks, (int)per_xcd);                                                      \
        else                                                                                                    \
            hipLaunchKernelGGL((staged_attention_kernel<NG, KMAX, false>), blocks, threads, 0, stream, a,       \
                               plan.chunks, (int)per_xcd);                                                      \
    }
    IRX_STAGED_CASE(1, 80)
    IRX_STAGED_CASE(1, 128)
    IRX_STAGED_CASE(1, 256)
    IRX_STAGED_CASE(1, 512)
    IRX_STAGED_CASE(2, 80)
    IRX_STAGED_CASE(2, 128)
    IRX_STAGED_CASE(2, 256)
    IRX_STAGED_CASE(2, 512)
    IRX_STAGED_CASE(4, 80)
    IRX_STAGED_CASE(4, 128)
    IRX_STAGED_CASE(4, 256)
    IRX_STAGED_CASE(4, 512)
#undef IRX_STAGED_CASE
    IRX_HIP(hipGetLastError());
}

void small_attention(const SmallAttention &args, hipStream_t stream) {
    if (args.seqs <= 0 || args.q_rows <= 0) return;
    if (args.kv_rows <= 0 || args.group <= 0) fail(3, "small attention needs keys and a group size");
    if ((reinterpret_cast<uintptr_t>(args.q) & 15) || (reinterpret_cast<uintptr_t>(args.k) & 15) ||
        (reinterpret_cast<uintptr_t>(args.v) & 15) || (reinterpret_cast<uintptr_t>(args.o) & 15) ||
        ((args.q_row | args.k_row | args.v_row | args.o_row | args.q_seq | args.k_seq | args.v_seq | args.o_seq |
          args.q_group | args.k_group | args.v_group | args.o_group | args.q_head | args.k_head | args.v_head |
          args.o_head) & 3))
        fail(3, "small attention operands must be 16-byte aligned");
    if (args.method < 0 || args.method > 2) fail(3, "small attention method must be 0, 1 or 2");
    const double sh = (double)args.seqs * args.heads;
    KernelTimer timer(kFamSmall, stream, 4.0 * sh * args.q_rows * args.kv_rows * 16.0,
                      4.0 * sh * 32.0 * (args.q_rows + args.kv_rows));
    if (args.method == 2 && !staged_applies(args)) fail(3, "the staged kernel needs more than 16 queries and at most 512 keys");
    if (args.method == 2 || (args.method == 0 && staged_applies(args) && args.rope_cos != nullptr)) {
        launch_staged(args, stream);
        return;
    }
    if (args.kv_rows <= kShortKeys) {
        // Matrix cores: 16 * qb queries per wave; about 8192 waves in flight.
        // Long query sets share each item's staged keys among four waves.
        // With few items (passes of a few rows) every 16-query block gets a
        // wave of its own, which stages the item's keys again.
        const long long items = (long long)args.seqs * args.heads;
        const int qb = (args.q_rows <= 16 || items * ceil_div(args.q_rows, 80) < 1024) ? 1
                       : (args.q_rows <= 80 ? 5 : 4);
        const int kb = args.kv_rows <= 80 ? 5 : 8;
        const long long chunks = ceil_div(args.q_rows, 16 * qb);
        const int waves = (qb == 4 && chunks >= 4) ? 4 : 1;
        const long long groups = std::max<long long>(
            1, std::min<long long>(ceil_div(chunks, waves), ceil_div(8192, items * waves)));
        const long long blocks = items * groups, per_xcd = ceil_div(blocks, 8);
        if (per_xcd * 8 > 0x7fffffffLL) fail(3, "small attention grid is too large");
        const bool rope = args.rope_cos != nullptr;
#define IRX_SMALL_CASE(QB, KB, W)                                                                                 \
    if (qb == QB && kb == KB && waves == W) {                                                                    \
        if (rope)                                                                                                \
            hipLaunchKernelGGL((small_attention_mfma_kernel<QB, KB, true, W>), dim3((unsigned)(per_xcd * 8)),    \
                               dim3(64 * W), 0, stream, args, (int)groups, (int)per_xcd, (int)blocks);          \
        else                                                                                                     \
            hipLaunchKernelGGL((small_attention_mfma_kernel<QB, KB, false, W>), dim3((unsigned)(per_xcd * 8)),   \
                               dim3(64 * W), 0, stream, args, (int)groups, (int)per_xcd, (int)blocks);          \
    }
        IRX_SMALL_CASE(1, 5, 1)
        IRX_SMALL_CASE(1, 8, 1)
        IRX_SMALL_CASE(5, 5, 1)
        IRX_SMALL_CASE(5, 8, 1)
        IRX_SMALL_CASE(4, 5, 1)
        IRX_SMALL_CASE(4, 8, 1)
        IRX_SMALL_CASE(4, 5, 4)
        IRX_SMALL_CASE(4, 8, 4)
#undef IRX_SMALL_CASE
    } else {
        const LongPlan plan = plan_long(args);
        const bool split = plan.splits > 1 && args.partial && args.partial_floats >= plan.partial_floats;
        const int splits = split ? plan.splits : 1;
        const int per = split ? plan.keys_per_split : args.kv_rows;
        const long long blocks = plan.units * splits, per_xcd = ceil_div(blocks, 8);
        if (per_xcd * 8 > 0x7fffffffLL) fail(3, "small attention grid is too large");
        if (4LL * ((long long)args.kv_rows * std::max(args.k_row, args.v_row) + 64) > 0xffffffffLL)
            fail(3, "small attention keys are too far apart for the long-range kernel");
        const bool rope = args.rope_cos != nullptr;
        const int qg = args.q_rows >= kLongQueries ? 8 : (args.q_rows > 32 ? 4 : (args.q_rows > 16 ? 2 : 1));
#define IRX_LONG_CASE(QG)                                                                                      \
    if (qg == QG) {                                                                                            \
        if (rope)                                                                                              \
            hipLaunchKernelGGL((small_attention_long_kernel<QG, true>), dim3((unsigned)(per_xcd * 8)),         \
                               dim3(64 * kLongWaves), 0, stream, args, plan.qchunks, splits, per,              \
                               (int)per_xcd, (int)blocks);                                                     \
        else                                                                                                   \
            hipLaunchKernelGGL((small_attention_long_kernel<QG, false>), dim3((unsigned)(per_xcd * 8)),        \
                               dim3(64 * kLongWaves), 0, stream, args, plan.qchunks, splits, per,              \
                               (int)per_xcd, (int)blocks);                                                     \
    }
        IRX_LONG_CASE(1)
        IRX_LONG_CASE(2)
        IRX_LONG_CASE(4)
        IRX_LONG_CASE(8)
#undef IRX_LONG_CASE
        IRX_HIP(hipGetLastError());
        if (split) {
            const long long threads = (long long)args.seqs * args.heads * args.q_rows * 4;
            hipLaunchKernelGGL(small_merge_kernel, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, stream, args,
                               splits);
        }
    }
    IRX_HIP(hipGetLastError());
}

long long small_attention_partial_floats(const SmallAttention &args) {
    if (args.kv_rows <= kShortKeys || args.seqs <= 0 || args.q_rows <= 0) return 0;
    const LongPlan plan = plan_long(args);
    return plan.splits > 1 ? plan.partial_floats : 0;
}

void pack_icl16(const void *k, const void *v, bool src_f16, long long rows, int pairs, unsigned short *k16,
                unsigned short *v16, unsigned *bad, hipStream_t stream) {
    if (rows <= 0 || pairs <= 0) return;
    const unsigned blocks = (unsigned)(pairs * ((rows + kKeyTile - 1) / kKeyTile));
    if (src_f16)
        hipLaunchKernelGGL(pack_icl16_kernel<_Float16>, dim3(blocks), dim3(256), 0, stream,
                           static_cast<const _Float16 *>(k), static_cast<const _Float16 *>(v), rows, pairs, k16, v16,
                           bad);
    else
        hipLaunchKernelGGL(pack_icl16_kernel<float>, dim3(blocks), dim3(256), 0, stream, static_cast<const float *>(k),
                           static_cast<const float *>(v), rows, pairs, k16, v16, bad);
    IRX_HIP(hipGetLastError());
}

void unpack_icl16(const unsigned short *k16, const unsigned short *v16, long long rows, int pairs, unsigned short *k,
                  unsigned short *v, hipStream_t stream) {
    if (rows <= 0 || pairs <= 0) return;
    const unsigned blocks = (unsigned)(pairs * ((rows + kKeyTile - 1) / kKeyTile));
    hipLaunchKernelGGL(unpack_icl16_kernel, dim3(blocks), dim3(256), 0, stream, k16, v16, rows, pairs, k, v);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
