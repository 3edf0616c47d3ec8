// Attention kernels of the gfx950 backend.
//
// 1. ICL attention, 64-wide heads, FP32 on matrix cores. It serves both the
//    build's train-row self-attention (N queries x N keys) and prediction's
//    cross-attention of a pass's queries against the resident K/V: the role
//    of icl_attention_f32 + icl_attention_merge in the reference's CUDA
//    backend (src/kernels/cuda/kernels.rs:183-213, 1523-1702), with the
//    semantics of softmax(q k^T / 8) v in FP32 (src/kernels/reference.rs:792-1024).
//
//    A wave owns 32 queries. It computes the transposed products
//      S^T[key, q] = K Q^T       (v_mfma_f32_32x32x2f32, k = head dim)
//      O^T[d, q]  += V^T P^T     (k = keys)
//    so that in the accumulator layout lane (q = lane % 32, half = lane / 32)
//    holds all of one query's scores for half of each 32-key block, and all of
//    its 64 output dims across the two 32-row output tiles. The online softmax
//    state (running max, sum) is therefore per lane: a tile needs one swap
//    between the lane halves for the max, and the output rescale is a scalar
//    multiply (skipped when no lane's maximum moved). Scores live in the exp2
//    domain (q pre-scaled by log2(e)/8). The P^T operand of the second
//    product is the first product's accumulator register as is; each lane
//    fetches the V elements of the key that register holds. The two output
//    tiles take the even and the odd dims, so one 8-byte LDS read serves both.
//    Keys stream through double-buffered LDS tiles of 64 (K rows padded to 68
//    floats); only a range's last tile is clamped and masked.
//
//    Few queries (a prediction pass) split the keys over workgroups; each
//    split writes its normalized partial output and log2-sum-exp, and a merge
//    kernel combines them. Workgroups sharing a (pair, split) K/V range are
//    placed on the same XCD so the range is read into one L2.
//
// 2. Attention of 16-wide heads on the vector ALUs (column ISAB and row
//    transformer), one thread per (sequence, head, query row), keys staged
//    through LDS in chunks of 64, optional RoPE on queries and keys.
#include "common.hpp"

namespace irx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kKeyTile = 64;
constexpr int kKStride = 68;
constexpr float kLog2e = 1.44269504088896340736f;

struct IclLaunch {
    int qtiles, splits, keys_per_split, per_xcd, q_padded;
};

// SPLIT: the keys are split over workgroups and each writes a partial output
// and its log2-sum-exp (prediction passes); otherwise the output is final
// (the build's self-attention over all training rows).
template <int WAVES, bool SPLIT>
__global__ __launch_bounds__(WAVES * 64) void icl_attention_kernel(IclAttention p, IclLaunch g) {
    constexpr int THREADS = WAVES * 64;
    constexpr int LOADS = kKeyTile * 16 / THREADS;  // float4 loads of K and of V per thread per tile
    constexpr int KEY_STEP = THREADS / 16;
    __shared__ __attribute__((aligned(16))) float Ks[2][kKeyTile * kKStride];
    __shared__ __attribute__((aligned(16))) float Vs[2][kKeyTile * 64];

    const int total = g.qtiles * p.pairs * g.splits;
    const int bid = blockIdx.x;
    const int t_id = (bid % 8) * g.per_xcd + bid / 8;
    if (t_id >= total) return;
    const int qt = t_id % g.qtiles;
    const int rest = t_id / g.qtiles;
    const int split = rest % g.splits;
    const int pair = rest / g.splits;
    const int k_begin = split * g.keys_per_split;
    const int k_end = min(p.kv_rows, k_begin + g.keys_per_split);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    const int qrow = qt * (WAVES * 32) + wave * 32 + r32;

    // This lane's query: dims 32*half .. 32*half + 31, scaled into the exp2 domain.
    float qreg[32];
    {
        const float scale = 0.125f * kLog2e;
        if (qrow < p.q_rows) {
            const float *src = p.q + pair * p.q_pair_stride + (long long)qrow * 64 + 32 * half;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                f32x4 v = *reinterpret_cast<const f32x4 *>(src + 4 * c);
                qreg[4 * c + 0] = v[0] * scale;
                qreg[4 * c + 1] = v[1] * scale;
                qreg[4 * c + 2] = v[2] * scale;
                qreg[4 * c + 3] = v[3] * scale;
            }
        } else {
#pragma unroll
            for (int t = 0; t < 32; ++t) qreg[t] = 0.f;
        }
    }

    // Tile staging: this thread moves keys (tid / 16) + KEY_STEP i, float4 column tid % 16.
    const float *kbase = p.k + pair * p.kv_pair_stride;
    const float *vbase = p.v + pair * p.kv_pair_stride;
    const int lkey = tid >> 4, lcol = (tid & 15) * 4;
    f32x4 kload[LOADS], vload[LOADS];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int key = min(k0 + lkey + KEY_STEP * i, k_end - 1);
            const long long off = (long long)key * 64 + lcol;
            kload[i] = *reinterpret_cast<const f32x4 *>(kbase + off);
            vload[i] = *reinterpret_cast<const f32x4 *>(vbase + off);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int key = lkey + KEY_STEP * i;
            *reinterpret_cast<f32x4 *>(&Ks[buf][key * kKStride + lcol]) = kload[i];
            *reinterpret_cast<f32x4 *>(&Vs[buf][key * 64 + lcol]) = vload[i];
        }
    };

    // O^T accumulators: o0 holds even dims d = 2i, o1 odd dims d = 2i + 1, where
    // i = half*4 + (r&3) + 8*(r>>2) is the accumulator row of register r.
    f32x16 o0, o1;
#pragma unroll
    for (int r = 0; r < 16; ++r) o0[r] = 0.f, o1[r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    load_tile(k_begin);
    store_tile(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += kKeyTile) {
        const bool more = k0 + kKeyTile < k_end;
        if (more) load_tile(k0 + kKeyTile);

        // S^T for both 32-key blocks, accumulations interleaved.
        f32x4 ka[8], kb[8];
        const float *krow = &Ks[buf][r32 * kKStride + 32 * half];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            ka[c] = *reinterpret_cast<const f32x4 *>(krow + 4 * c);
            kb[c] = *reinterpret_cast<const f32x4 *>(krow + 32 * kKStride + 4 * c);
        }
        f32x16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) s0[r] = 0.f, s1[r] = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[c][e], qreg[4 * c + e], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kb[c][e], qreg[4 * c + e], s1, 0, 0, 0);
            }
        // Only the last tile of a range can hold keys past it.
        if (k0 + kKeyTile > k_end) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + half * 4 + (r & 3) + 8 * (r >> 2);
                if (key >= k_end) s0[r] = -INFINITY;
                if (key + 32 >= k_end) s1[r] = -INFINITY;
            }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(s0[r], s1[r]));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);
        // Rescale only when some lane's running maximum moved (rare after the first tiles).
        if (__any(m_new > m_run)) {
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int r = 0; r < 16; ++r) o0[r] *= alpha, o1[r] *= alpha;
        }
        m_run = m_new;
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = __builtin_amdgcn_exp2f(s0[r] - m_new);
            s1[r] = __builtin_amdgcn_exp2f(s1[r] - m_new);
            lsum += s0[r] + s1[r];
        }
        l_run += lsum;
        // O^T += V^T P^T: register r of s0 / s1 is key (half*4 + (r&3) + 8*(r>>2)) of block 0 / 1.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = half * 4 + (r & 3) + 8 * (r >> 2);
            const f32x2 v0 = *reinterpret_cast<const f32x2 *>(&Vs[buf][key * 64 + 2 * r32]);
            const f32x2 v1 = *reinterpret_cast<const f32x2 *>(&Vs[buf][(key + 32) * 64 + 2 * r32]);
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[0], s0[r], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[1], s0[r], o1, 0, 0, 0);
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[0], s1[r], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[1], s1[r], o1, 0, 0, 0);
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    if (qrow >= p.q_rows) return;
    const float inv = 1.0f / l_tot;
    float *dst;
    if constexpr (!SPLIT) {
        const int b = pair / kHeads, head = pair - b * kHeads;
        dst = p.o + ((long long)b * p.q_rows + qrow) * p.ldo + head * 64;
    } else {
        dst = p.partial + (((long long)split * p.pairs + pair) * g.q_padded + qrow) * 65;
        if (half == 0) dst[64] = m_run + log2f(l_tot);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = half * 4 + (r & 3) + 8 * (r >> 2);
        dst[2 * i] = o0[r] * inv;
        dst[2 * i + 1] = o1[r] * inv;
    }
}

// Merge of split partials by their log2-sum-exp, into tokens [b * q_rows + row, head * 64 + d].
__global__ __launch_bounds__(256) void icl_merge_kernel(IclAttention p, int splits, int q_padded) {
    long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    long long total = (long long)p.pairs * p.q_rows * 64;
    if (idx >= total) return;
    int d = idx & 63;
    long long pq = idx >> 6;
    int qrow = (int)(pq % p.q_rows);
    int pair = (int)(pq / p.q_rows);
    float mx = -INFINITY;
    for (int s = 0; s < splits; ++s)
        mx = fmaxf(mx, p.partial[(((long long)s * p.pairs + pair) * q_padded + qrow) * 65 + 64]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < splits; ++s) {
        const float *part = p.partial + (((long long)s * p.pairs + pair) * q_padded + qrow) * 65;
        float w = __builtin_amdgcn_exp2f(part[64] - mx);
        num += w * part[d];
        den += w;
    }
    int b = pair / kHeads, head = pair - b * kHeads;
    p.o[((long long)b * p.q_rows + qrow) * p.ldo + head * 64 + d] = num / den;
}

constexpr int kIclWaves = 4;

IclLaunch plan_icl(int pairs, int q_rows, int kv_rows, int compute_units) {
    IclLaunch g{};
    g.qtiles = (int)ceil_div(q_rows, kIclWaves * 32);
    g.q_padded = g.qtiles * kIclWaves * 32;
    long long base = (long long)g.qtiles * pairs;
    long long want = 2LL * compute_units;
    int splits = 1;
    if (base < want) {
        splits = (int)ceil_div(want, base);
        int max_splits = (int)ceil_div(kv_rows, 512);
        splits = splits < max_splits ? splits : max_splits;
        if (splits < 1) splits = 1;
    }
    int per = (int)ceil_div(ceil_div(kv_rows, splits), kKeyTile) * kKeyTile;
    g.keys_per_split = per;
    g.splits = (int)ceil_div(kv_rows, per);
    g.per_xcd = (int)ceil_div((long long)g.qtiles * pairs * g.splits, 8);
    return g;
}

// ---- 16-wide heads on the vector ALUs ----

constexpr int kSmallChunk = 64;

__global__ __launch_bounds__(64) void small_attention_kernel(SmallAttention p, int qtiles) {
    __shared__ __attribute__((aligned(16))) float Ks[kSmallChunk * 16];
    __shared__ __attribute__((aligned(16))) float Vs[kSmallChunk * 16];
    const int bid = blockIdx.x;
    const int qt = bid % qtiles;
    const int head = (bid / qtiles) % p.heads;
    const int seq = bid / (qtiles * p.heads);
    const int lane = threadIdx.x;
    const int row = qt * 64 + lane;
    const int gq = seq / p.group, sq = seq - gq * p.group;
    const float *qb = p.q + gq * p.q_group + sq * p.q_seq + head * p.q_head;
    const float *kb = p.k + gq * p.k_group + sq * p.k_seq + head * p.k_head;
    const float *vb = p.v + gq * p.v_group + sq * p.v_seq + head * p.v_head;

    float q[16], o[16];
    const float scale = p.scale * kLog2e;
    if (row < p.q_rows) {
        const float *src = qb + (long long)row * p.q_row;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f32x4 v = *reinterpret_cast<const f32x4 *>(src + 4 * c);
            q[4 * c] = v[0], q[4 * c + 1] = v[1], q[4 * c + 2] = v[2], q[4 * c + 3] = v[3];
        }
        if (p.rope_cos) {
            float r[16];
            const float *cs = p.rope_cos + row * 16, *sn = p.rope_sin + row * 16;
#pragma unroll
            for (int d = 0; d < 16; ++d) r[d] = q[d] * cs[d] + q[d ^ 8] * sn[d];
#pragma unroll
            for (int d = 0; d < 16; ++d) q[d] = r[d];
        }
    } else {
#pragma unroll
        for (int d = 0; d < 16; ++d) q[d] = 0.f;
    }
#pragma unroll
    for (int d = 0; d < 16; ++d) q[d] *= scale, o[d] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    for (int k0 = 0; k0 < p.kv_rows; k0 += kSmallChunk) {
        const int count = min(kSmallChunk, p.kv_rows - k0);
        __syncthreads();
        if (lane < count) {
            const int key = k0 + lane;
            const float *ks = kb + (long long)key * p.k_row;
            const float *vs = vb + (long long)key * p.v_row;
            float kr[16];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                f32x4 v = *reinterpret_cast<const f32x4 *>(ks + 4 * c);
                kr[4 * c] = v[0], kr[4 * c + 1] = v[1], kr[4 * c + 2] = v[2], kr[4 * c + 3] = v[3];
                *reinterpret_cast<f32x4 *>(&Vs[lane * 16 + 4 * c]) = *reinterpret_cast<const f32x4 *>(vs + 4 * c);
            }
            if (p.rope_cos) {
                const float *cs = p.rope_cos + key * 16, *sn = p.rope_sin + key * 16;
                float r[16];
#pragma unroll
                for (int d = 0; d < 16; ++d) r[d] = kr[d] * cs[d] + kr[d ^ 8] * sn[d];
#pragma unroll
                for (int d = 0; d < 16; ++d) kr[d] = r[d];
            }
#pragma unroll
            for (int c = 0; c < 4; ++c)
                *reinterpret_cast<f32x4 *>(&Ks[lane * 16 + 4 * c]) =
                    f32x4{kr[4 * c], kr[4 * c + 1], kr[4 * c + 2], kr[4 * c + 3]};
        }
        __syncthreads();
        for (int j0 = 0; j0 < count; j0 += 16) {
            const int nj = min(16, count - j0);
            float s[16];
            float mt = -INFINITY;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (j < nj) {
                    const float *kr = &Ks[(j0 + j) * 16];
                    float acc = 0.f;
#pragma unroll
                    for (int d = 0; d < 16; ++d) acc = fmaf(q[d], kr[d], acc);
                    s[j] = acc;
                } else {
                    s[j] = -INFINITY;
                }
                mt = fmaxf(mt, s[j]);
            }
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int d = 0; d < 16; ++d) o[d] *= alpha;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (j < nj) {
                    const float e = __builtin_amdgcn_exp2f(s[j] - m_new);
                    l_run += e;
                    const float *vr = &Vs[(j0 + j) * 16];
#pragma unroll
                    for (int d = 0; d < 16; ++d) o[d] = fmaf(e, vr[d], o[d]);
                }
            }
        }
    }
    if (row >= p.q_rows) return;
    const float inv = 1.0f / l_run;
    float *dst = p.o + gq * p.o_group + sq * p.o_seq + (long long)row * p.o_row + head * p.o_head;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        *reinterpret_cast<f32x4 *>(dst + 4 * c) =
            f32x4{o[4 * c] * inv, o[4 * c + 1] * inv, o[4 * c + 2] * inv, o[4 * c + 3] * inv};
}

}  // namespace

int icl_attention_splits(int pairs, int q_rows, int kv_rows, int compute_units) {
    return plan_icl(pairs, q_rows, kv_rows, compute_units).splits;
}

size_t icl_attention_partial_floats(int pairs, int q_rows, int splits) {
    if (splits <= 1) return 0;
    size_t q_padded = ceil_div(q_rows, kIclWaves * 32) * (size_t)(kIclWaves * 32);
    return (size_t)splits * pairs * q_padded * 65;
}

void icl_attention(const IclAttention &args, hipStream_t stream) {
    if (args.pairs <= 0 || args.q_rows <= 0) return;
    if (args.kv_rows <= 0) fail(3, "ICL attention needs at least one key");
    if ((reinterpret_cast<uintptr_t>(args.q) & 15) || (reinterpret_cast<uintptr_t>(args.k) & 15) ||
        (reinterpret_cast<uintptr_t>(args.v) & 15) || (args.q_pair_stride & 3) || (args.kv_pair_stride & 3))
        fail(3, "ICL attention operands must be 16-byte aligned");
    IclLaunch g = plan_icl(args.pairs, args.q_rows, args.kv_rows, args.compute_units);
    if (g.splits > 1) {
        size_t need = icl_attention_partial_floats(args.pairs, args.q_rows, g.splits);
        if (!args.partial || args.partial_floats < need) fail(3, "ICL attention partial buffer is too small");
    }
    {
        const double pairs = args.pairs, q = args.q_rows, kv = args.kv_rows;
        KernelTimer timer(kFamIcl, stream, 4.0 * pairs * q * kv * 64.0, 4.0 * 64.0 * pairs * (2.0 * kv + 2.0 * q));
        if (g.splits > 1)
            hipLaunchKernelGGL((icl_attention_kernel<kIclWaves, true>), dim3(g.per_xcd * 8), dim3(kIclWaves * 64), 0,
                               stream, args, g);
        else
            hipLaunchKernelGGL((icl_attention_kernel<kIclWaves, false>), dim3(g.per_xcd * 8), dim3(kIclWaves * 64), 0,
                               stream, args, g);
        IRX_HIP(hipGetLastError());
    }
    if (g.splits > 1) {
        long long total = (long long)args.pairs * args.q_rows * 64;
        KernelTimer timer(kFamIclMerge, stream, 0.0,
                          4.0 * ((double)g.splits * args.pairs * args.q_rows * 65.0 + (double)total));
        hipLaunchKernelGGL(icl_merge_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, stream, args, g.splits,
                           g.q_padded);
        IRX_HIP(hipGetLastError());
    }
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
    int qtiles = (int)ceil_div(args.q_rows, 64);
    long long blocks = (long long)qtiles * args.heads * args.seqs;
    if (blocks > 0x7fffffffLL) fail(3, "small attention grid is too large");
    const double sh = (double)args.seqs * args.heads;
    KernelTimer timer(kFamSmall, stream, 4.0 * sh * args.q_rows * args.kv_rows * 16.0,
                      4.0 * sh * 32.0 * (args.q_rows + args.kv_rows));
    hipLaunchKernelGGL(small_attention_kernel, dim3((unsigned)blocks), dim3(64), 0, stream, args, qtiles);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
