// Fused tail of a 128-wide transformer block on gfx950 matrix cores.
//
// The post-attention half of every column and row block (cpu.rs:1555-1601):
//   s1    = state + (att Wo^T + bo)
//   state = s1 + (gelu(LN2(s1) W1^T + b1) W2^T + b2)
// as one kernel instead of four launches (out-projection, LayerNorm, FFN up,
// FFN down), so s1, LN2(s1) and the 256-wide hidden layer never leave
// registers.
//
// Each wave owns 16 rows for the whole chain. Products are computed
// transposed, D = W X^T, on v_mfma_f32_16x16x4f32: the weights are the A
// operand and the rows the B operand. In D, lane (m, g) = (lane % 16,
// lane / 16) holds row m's features 16 b + 4 g + r in register r of block b,
// which is exactly what the next product's B operand needs at step r of
// k-block b, so the chain runs without moving data between lanes. The same
// per-lane layout is used to load att and state and to store the result.
//
// The weights are packed once (tail128_pack) into A-operand fragments, 1 KB
// per 16 x 16 block, lane after lane, in the order the kernel consumes them:
// ten 32 KB chunks (Wo in two, then per 32-unit slice of the hidden layer the
// W1 rows and W2 columns it touches). A workgroup streams each chunk as two
// 16 KB halves (out-projection k-blocks, or a slice's W1 rows then its W2
// columns) through two 16 KB LDS buffers with direct global -> LDS loads, so
// three workgroups share a CU; every LDS read is one 16-byte read per lane
// of consecutive addresses (no bank conflicts).
#include "common.hpp"

#include <algorithm>

namespace irx {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kChunkFloats = 8192;  // 32 KB: the packing unit
constexpr int kChunks = 10;
// Chunks stream through LDS in halves of 16 KB (two 16 KB buffers), so a
// workgroup takes 32 KB and three fit a CU.
constexpr int kHalfFloats = kChunkFloats / 2;
constexpr int kHalves = 2 * kChunks;
constexpr int kTailWaves = 4;
constexpr int kTailRows = 16 * kTailWaves;  // rows per workgroup

__device__ __forceinline__ void wait_vm() {
    // vmcnt(0); expcnt and lgkmcnt left at their maxima (no wait).
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

__device__ __forceinline__ f32x4 mfma(float a, float b, const f32x4 &acc) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
}

__device__ __forceinline__ f32x4 lds4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }

// The chain after a 128-wide block's attention (cpu.rs:1555-1601): x holds
// the row's attention output and s1 its state, in the per-wave layout above;
// the packed weights arrive as half-chunks h0 .. h0 + 19 from next(h), which
// returns the lane's base in the half's LDS buffer. The new state goes to
// out (the lane's first feature, 4 g) when the row is live.
template <class Next>
__device__ __forceinline__ void tail_chain(f32x4 (&x)[8], f32x4 (&s1)[8], Next &&next, int h0, const Tail128 &t,
                                           float *out, bool live, int g) {
    f32x4 acc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Out-projection: half-chunks 0 .. 3 hold k-blocks 2 hc and 2 hc + 1,
    // each with the eight output blocks' fragments. The second k-block's
    // fragments are read while the first one's 32 products (8 independent
    // accumulators) run.
#pragma unroll
    for (int hc = 0; hc < 4; ++hc) {
        const float *frag = next(h0 + hc);
        f32x4 fa[2][8];
#pragma unroll
        for (int ob = 0; ob < 8; ++ob) fa[0][ob] = lds4(frag + ob * 256);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            if (kb == 0) {
#pragma unroll
                for (int ob = 0; ob < 8; ++ob) fa[1][ob] = lds4(frag + (8 + ob) * 256);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ob = 0; ob < 8; ++ob) acc[ob] = mfma(fa[kb][ob][e], x[2 * hc + kb][e], acc[ob]);
        }
    }

    // s1 = state + (acc + bo), then LN2 over the row's 128 features, held by
    // lanes m, m + 16, m + 32, m + 48.
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const f32x4 bo = *reinterpret_cast<const f32x4 *>(t.bo + 16 * b + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s1[b][e] = s1[b][e] + (acc[b][e] + bo[e]);
            sum += s1[b][e];
        }
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float mean = sum / 128.f;
    float sq = 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = s1[b][e] - mean;
            sq = fmaf(d, d, sq);
        }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    const float rstd = 1.0f / sqrtf(sq / 128.f + 1e-5f);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const f32x4 w = *reinterpret_cast<const f32x4 *>(t.n2w + 16 * b + 4 * g);
        const f32x4 bb = *reinterpret_cast<const f32x4 *>(t.n2b + 16 * b + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[b][e] = (s1[b][e] - mean) * rstd * w[e] + bb[e];
        acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // FFN, 32 hidden units per slice c: h = gelu(W1 x + b1) for units 32 c +
    // 16 hb + 4 g + e from half-chunk 4 + 2 c (even and odd k-blocks in
    // separate accumulators, four independent chains), then acc += W2 h from
    // half-chunk 5 + 2 c.
#pragma unroll 1
    for (int c = 0; c < 8; ++c) {
        const float *frag = next(h0 + 4 + 2 * c);
        f32x4 h[2][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i >> 1][i & 1] = f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 fw[2][2];
        fw[0][0] = lds4(frag), fw[0][1] = lds4(frag + 256);
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            if (kb < 7) {
                fw[(kb + 1) & 1][0] = lds4(frag + ((kb + 1) * 2) * 256);
                fw[(kb + 1) & 1][1] = lds4(frag + ((kb + 1) * 2 + 1) * 256);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) h[hb][kb & 1] = mfma(fw[kb & 1][hb][e], x[kb][e], h[hb][kb & 1]);
        }
        f32x4 hg[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const f32x4 b1 = *reinterpret_cast<const f32x4 *>(t.b1 + 32 * c + 16 * hb + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) hg[hb][e] = gelu_erf((h[hb][0][e] + h[hb][1][e]) + b1[e]);
        }
        const float *frag2 = next(h0 + 5 + 2 * c);
        f32x4 f2[2][8];
#pragma unroll
        for (int ob = 0; ob < 8; ++ob) f2[0][ob] = lds4(frag2 + ob * 256);
#pragma unroll
        for (int ob = 0; ob < 8; ++ob) f2[1][ob] = lds4(frag2 + (8 + ob) * 256);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ob = 0; ob < 8; ++ob) acc[ob] = mfma(f2[j][ob][e], hg[j][e], acc[ob]);
    }

    if (!live) return;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const f32x4 b2 = *reinterpret_cast<const f32x4 *>(t.b2 + 16 * b + 4 * g);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (acc[b][e] + b2[e]) + s1[b][e];
        *reinterpret_cast<f32x4 *>(out + 16 * b) = v;
    }
}

__global__ __launch_bounds__(256, 3) void tail128_kernel(Tail128 p) {
    __shared__ __attribute__((aligned(16))) float buf[2][kHalfFloats];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;
    const long long row = (long long)blockIdx.x * kTailRows + wv * 16 + m16;
    const bool live = row < p.m;
    const long long r = live ? row : p.m - 1;

    // Half-chunk hc (16 KB) goes to buffer hc % 2; wave w moves its 1 KB
    // blocks 4 w .. 4 w + 3.
    auto issue = [&](int hc) {
        const float *src = p.pack + (long long)hc * kHalfFloats + (4 * wv) * 256 + lane * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(src + i * 256, (lds_void *)&buf[hc & 1][(4 * wv + i) * 256], 16, 0, 0);
    };
    // Before half-chunk hc is read: its loads done, every wave past the
    // previous one (whose buffer the next half-chunk then overwrites).
    auto next = [&](int hc) {
        wait_vm();
        __syncthreads();
        if (hc + 1 < kHalves) issue(hc + 1);
        return &buf[hc & 1][lane * 4];
    };
    issue(0);

    // x: row m's features 16 kb + 4 g + e (att now, LN2(s1) later).
    f32x4 x[8], s1[8];
    const float *att = p.att + r * p.lda + 4 * g;
    const float *st = p.state + r * p.ldx + 4 * g;
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = *reinterpret_cast<const f32x4 *>(att + 16 * b);
#pragma unroll
    for (int b = 0; b < 8; ++b) s1[b] = *reinterpret_cast<const f32x4 *>(st + 16 * b);
    tail_chain(x, s1, next, 0, p, p.state + r * p.ldx + 4 * g, live, g);
}

// A cached column block in one kernel: 64 rows of one column per workgroup,
// wave w carrying rows 16 w .. 16 w + 15 through LN1, the query projection
// (head128's order), the attention of its 8 heads to the column's 128 cached
// inducing keys and values (the 16-wide attention kernel's exact softmax and
// order) and tail128's chain, so q and the attention output never leave
// registers. 32 half-chunks of 16 KB stream through two LDS buffers: 0..3 the
// query rows' fragments, 4..11 head h's keys (fragment order, 8 KB) and values
// (8 KB: per 16-key block, four planes of 64 lanes, lane (d, g) of plane r
// holding key 16 kb + 4 g + r's dim d, gathered by 4-byte loads from the
// cache's [key][16] rows), 12..31 tail128's pack. Workgroups of one XCD take
// consecutive units, so a column's tiles share its K/V in one L2. Three
// workgroups share a CU (168 registers, as tail128; the compiler keeps a few
// values of the prologue in scratch until the epilogue): at two, the
// build's 3.2M-row blocks ran 6% slower than the three launches.
constexpr int kColumnHalves = 32;

__global__ __launch_bounds__(256, 3) void column_block_kernel(ColumnBlock p, int tiles, int per_xcd) {
    __shared__ __attribute__((aligned(16))) float buf[2][kHalfFloats];
    const int unit = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    if (unit >= p.cols * tiles) return;  // workgroup-uniform, before any barrier
    const int col = unit / tiles, tile = unit - col * tiles;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;
    const long long row = (long long)tile * kTailRows + wv * 16 + m16;
    const bool live = row < p.rows;
    const long long r = live ? row : p.rows - 1;
    float *xrow = p.state + ((long long)col * p.rows + r) * 128 + 4 * g;
    const long long coff = (long long)(col / p.group) * p.group_stride + (long long)(col % p.group) * kColumnCache;
    const float *kcol = p.k + coff, *vcol = p.v + coff;

    auto issue = [&](int h) {
        float *dst = buf[h & 1];
        if (h < 4 || h >= 12) {
            const float *src = (h < 4 ? p.qpack + h * kHalfFloats : p.pack + (h - 12) * kHalfFloats) + (4 * wv) * 256 +
                               lane * 4;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_amdgcn_global_load_lds(src + i * 256, (lds_void *)&dst[(4 * wv + i) * 256], 16, 0, 0);
        } else {
            // Head h - 4: wave w moves key blocks 2 w and 2 w + 1.
            const float *kh = kcol + (h - 4) * (kInducing * kColumnHead), *vh = vcol + (h - 4) * (kInducing * kColumnHead);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int kb = 2 * wv + i;
                __builtin_amdgcn_global_load_lds(kh + (16 * kb + m16) * 16 + 4 * g, (lds_void *)&dst[kb * 256], 16, 0, 0);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    __builtin_amdgcn_global_load_lds(vh + (16 * kb + 4 * g + rr) * 16 + m16,
                                                     (lds_void *)&dst[2048 + (kb * 4 + rr) * 64], 4, 0, 0);
            }
        }
    };
    // Half h's buffer once its loads are done and every wave is past half
    // h - 1 (whose buffer half h + 1 then overwrites).
    auto next = [&](int h) {
        wait_vm();
        __syncthreads();
        if (h + 1 < kColumnHalves) issue(h + 1);
        return &buf[h & 1][0];
    };
    issue(0);

    // The rows' states (kept for the residual) and LN1, as head128.
    f32x4 s1[8], x[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) s1[b] = *reinterpret_cast<const f32x4 *>(xrow + 16 * b);
    {
        float sum = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b) sum += (s1[b][0] + s1[b][1]) + (s1[b][2] + s1[b][3]);
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        const float mean = sum / 128.f;
        float sq = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = s1[b][e] - mean;
                sq = fmaf(d, d, sq);
            }
        sq += __shfl_xor(sq, 16, 64);
        sq += __shfl_xor(sq, 32, 64);
        const float rstd = 1.0f / sqrtf(sq / 128.f + 1e-5f);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const f32x4 w = *reinterpret_cast<const f32x4 *>(p.lnw + 16 * b + 4 * g);
            const f32x4 bb = *reinterpret_cast<const f32x4 *>(p.lnb + 16 * b + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[b][e] = (s1[b][e] - mean) * rstd * w[e] + bb[e];
        }
    }

    // q: lane (m, g) holds head h's dims 4 g .. 4 g + 3 of row m in q[h],
    // scaled into the exp2 domain (1 / sqrt(16) = 0.25).
    f32x4 q[8];
#pragma unroll
    for (int ob = 0; ob < 8; ++ob) q[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float *frag = next(c) + lane * 4;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int f = 16 * c + i, kb = f / 8, ob = f % 8;
            const f32x4 a = lds4(frag + i * 256);
#pragma unroll
            for (int e = 0; e < 4; ++e) q[ob] = mfma(a[e], x[kb][e], q[ob]);
        }
    }
    const float scale = 0.25f * kLog2e;
#pragma unroll
    for (int ob = 0; ob < 8; ++ob) q[ob] = (q[ob] + *reinterpret_cast<const f32x4 *>(p.qb + 16 * ob + 4 * g)) * scale;

    // Per head: S^T = K Q^T (lane (m, g) holds keys 16 kb + 4 g + r of row
    // m), the exact softmax over the 128 keys, O^T = V^T P^T, which leaves
    // head h's output in tail128's layout for feature block h.
    f32x4 att[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) {
        const float *hb = next(4 + h);
        f32x4 s[8];
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            const f32x4 kf = lds4(hb + kb * 256 + lane * 4);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) acc = mfma(kf[st], q[h][st], acc);
            s[kb] = acc;
        }
        float m = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) m = fmaxf(m, fmaxf(fmaxf(s[kb][0], s[kb][1]), fmaxf(s[kb][2], s[kb][3])));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float l = 0.f;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                s[kb][rr] = __builtin_amdgcn_exp2f(s[kb][rr] - m);
                l += s[kb][rr];
            }
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float inv = 1.0f / l;
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            const float *vp = hb + 2048 + kb * 256 + lane;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) o = mfma(vp[rr * 64], s[kb][rr], o);
        }
        att[h] = o * inv;
    }

    Tail128 t{};
    t.bo = p.bo, t.n2w = p.n2w, t.n2b = p.n2b, t.b1 = p.b1, t.b2 = p.b2;
    tail_chain(att, s1, [&](int h) { return next(h) + lane * 4; }, 12, t, xrow, live, g);
}

// The same tail for small passes (a few thousand rows or fewer), where
// tail128's 64-row workgroups would leave most CUs idle and each wave would
// carry its rows through all 320 products alone: one workgroup per 16 rows,
// wave w producing output blocks 2 w and 2 w + 1 (of the out-projection and
// of the FFN's second layer) and hidden slices 2 w and 2 w + 1. The waves
// swap s1 and the GELU layer through LDS; every wave takes LN2 of the whole
// rows itself. Fragments are read from the tail128 pack in global memory
// (320 KB, shared by every workgroup through L2), each wave's W1 fragments
// issued with its first loads. Every accumulator takes its products in
// tail128's order, so the results are tail128's bit for bit.
// tail128_rows16's chain from the out-projection on, for wave w of a
// workgroup of 16 rows: x holds the lane's row's attention output (all eight
// blocks), s1 its state's blocks 2 w and 2 w + 1, fo and f1 the wave's Wo and
// W1 fragments; s1s and hs are the workgroup's LDS exchange buffers, pk the
// lane's base in the tail128 pack. The new state's blocks 2 w, 2 w + 1 go to
// out (the lane's first feature, 4 g) when the row is live.
constexpr int kRows16S1Stride = 132, kRows16HidStride = 260;

__device__ __forceinline__ void rows16_chain(const Tail128 &t, const f32x4 (&x)[8], f32x4 (&s1)[2],
                                             const f32x4 (&fo)[8][2], const f32x4 (&f1)[2][8][2], float *s1s,
                                             float *hs, const float *pk, int w, int m16, int g, float *out,
                                             bool live) {
    constexpr int kS1Stride = kRows16S1Stride, kHidStride = kRows16HidStride;
    auto w2_frag = [&](int c, int j, int ob) {
        return *reinterpret_cast<const f32x4 *>(pk + (2 + c) * kChunkFloats + 4096 + (j * 8 + ob) * 256);
    };
    f32x4 xn[8];
    // Out-projection of output blocks 2 w + j; s1 = state + (acc + bo) to LDS.
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[j] = mfma(fo[kb][j][e], x[kb][e], acc[j]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c0 = 16 * (2 * w + j) + 4 * g;
        const f32x4 bo = *reinterpret_cast<const f32x4 *>(t.bo + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) s1[j][e] = s1[j][e] + (acc[j][e] + bo[e]);
        *reinterpret_cast<f32x4 *>(&s1s[m16 * kS1Stride + c0]) = s1[j];
    }
    __syncthreads();

    // LN2 of the 16 rows (as tail128: row m's features over lanes m, m + 16,
    // m + 32, m + 48).
#pragma unroll
    for (int b = 0; b < 8; ++b) xn[b] = *reinterpret_cast<const f32x4 *>(&s1s[m16 * kS1Stride + 16 * b + 4 * g]);
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += xn[b][e];
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float mean = sum / 128.f;
    float sq = 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = xn[b][e] - mean;
            sq = fmaf(d, d, sq);
        }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    const float rstd = 1.0f / sqrtf(sq / 128.f + 1e-5f);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const f32x4 nw = *reinterpret_cast<const f32x4 *>(t.n2w + 16 * b + 4 * g);
        const f32x4 nb = *reinterpret_cast<const f32x4 *>(t.n2b + 16 * b + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) xn[b][e] = (xn[b][e] - mean) * rstd * nw[e] + nb[e];
    }

    // Hidden slices c = 2 w + sl: gelu(W1 x + b1) to LDS.
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
        const int c = 2 * w + sl;
        f32x4 h[2][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i >> 1][i & 1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) h[hb][kb & 1] = mfma(f1[sl][kb][hb][e], xn[kb][e], h[hb][kb & 1]);
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const f32x4 b1 = *reinterpret_cast<const f32x4 *>(t.b1 + 32 * c + 16 * hb + 4 * g);
            f32x4 hg;
#pragma unroll
            for (int e = 0; e < 4; ++e) hg[e] = gelu_erf((h[hb][0][e] + h[hb][1][e]) + b1[e]);
            *reinterpret_cast<f32x4 *>(&hs[m16 * kHidStride + 32 * c + 16 * hb + 4 * g]) = hg;
        }
    }
    // This wave's W2 fragments (output blocks 2 w + j), in flight over the barrier.
    f32x4 f2[8][2][2];
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int ob = 0; ob < 2; ++ob) f2[c][j][ob] = w2_frag(c, j, 2 * w + ob);
    __syncthreads();

    // FFN down over the 256 hidden units, slice by slice as tail128 does.
    f32x4 acc2[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f32x4 hv = *reinterpret_cast<const f32x4 *>(&hs[m16 * kHidStride + 32 * c + 16 * j + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ob = 0; ob < 2; ++ob) acc2[ob] = mfma(f2[c][j][ob][e], hv[e], acc2[ob]);
        }
    if (!live) return;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c0 = 16 * (2 * w + j);
        const f32x4 b2 = *reinterpret_cast<const f32x4 *>(t.b2 + c0 + 4 * g);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (acc2[j][e] + b2[e]) + s1[j][e];
        *reinterpret_cast<f32x4 *>(out + c0) = v;
    }
}

__global__ __launch_bounds__(256) void tail128_rows16_kernel(Tail128 p) {
    constexpr int kS1Stride = kRows16S1Stride, kHidStride = kRows16HidStride;
    __shared__ __attribute__((aligned(16))) float s1s[16 * kS1Stride];
    __shared__ __attribute__((aligned(16))) float hs[16 * kHidStride];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;
    const long long row = (long long)blockIdx.x * 16 + m16;
    const bool live = row < p.m;
    const long long r = live ? row : p.m - 1;
    const float *pk = p.pack + lane * 4;
    // Fragment (k-block kb, output block ob) of Wo; (kb, hb) of slice c's W1
    // rows (tail128_pack's order).
    auto wo_frag = [&](int kb, int ob) { return *reinterpret_cast<const f32x4 *>(pk + kb * 2048 + ob * 256); };
    auto w1_frag = [&](int c, int kb, int hb) {
        return *reinterpret_cast<const f32x4 *>(pk + (2 + c) * kChunkFloats + (kb * 2 + hb) * 256);
    };

    f32x4 fo[8][2], x[8], s1[2];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) fo[kb][j] = wo_frag(kb, 2 * w + j);
    const float *att = p.att + r * p.lda + 4 * g;
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = *reinterpret_cast<const f32x4 *>(att + 16 * b);
    const float *st = p.state + r * p.ldx + 4 * g;
#pragma unroll
    for (int j = 0; j < 2; ++j) s1[j] = *reinterpret_cast<const f32x4 *>(st + 16 * (2 * w + j));
    f32x4 f1[2][8][2];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) f1[sl][kb][hb] = w1_frag(2 * w + sl, kb, hb);

    rows16_chain(p, x, s1, fo, f1, s1s, hs, pk, w, m16, g, p.state + r * p.ldx + 4 * g, live);
}

// The cached column block for small passes: one workgroup per 16 rows of
// one column, wave w taking query heads and output blocks 2 w and 2 w + 1
// (tail128_rows16's split). Every wave takes LN1 of the whole rows; its
// query fragments, its heads' keys (fragment order) and values (lane (d, g)
// value r of key block kb = key 16 kb + 4 g + r's dim d) come straight from
// global memory, all issued with its first loads, and the tail's Wo and W1
// fragments follow while the attention runs. The attention outputs meet in
// LDS for the out-projection; from there on this is tail128_rows16. The
// arithmetic is column_block_kernel's, so the results are its bits.
__global__ __launch_bounds__(256) void column_block_rows16_kernel(ColumnBlock p, int groups) {
    constexpr int kS1Stride = kRows16S1Stride, kHidStride = kRows16HidStride;
    __shared__ __attribute__((aligned(16))) float as[16 * kS1Stride];
    __shared__ __attribute__((aligned(16))) float s1s[16 * kS1Stride];
    __shared__ __attribute__((aligned(16))) float hs[16 * kHidStride];
    const int unit = blockIdx.x;
    const int col = unit / groups, grp = unit - col * groups;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;
    const long long row = (long long)grp * 16 + m16;
    const bool live = row < p.rows;
    const long long r = live ? row : p.rows - 1;
    float *xrow = p.state + ((long long)col * p.rows + r) * 128 + 4 * g;
    const long long coff = (long long)(col / p.group) * p.group_stride + (long long)(col % p.group) * kColumnCache;
    const float *kh = p.k + coff + (2 * w) * (kInducing * kColumnHead);
    const float *vh = p.v + coff + (2 * w) * (kInducing * kColumnHead);
    const float *qk = p.qpack + lane * 4, *pk = p.pack + lane * 4;

    f32x4 x[8], fq[8][2], kf[2][8];
    float vv[2][8][4];
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = *reinterpret_cast<const f32x4 *>(xrow + 16 * b);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) fq[kb][j] = *reinterpret_cast<const f32x4 *>(qk + (kb * 8 + 2 * w + j) * 256);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            kf[j][kb] = *reinterpret_cast<const f32x4 *>(kh + j * 2048 + (16 * kb + m16) * 16 + 4 * g);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) vv[j][kb][rr] = vh[j * 2048 + (16 * kb + 4 * g + rr) * 16 + m16];
        }

    // LN1 over the rows, as head128.
    {
        float sum = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b) sum += (x[b][0] + x[b][1]) + (x[b][2] + x[b][3]);
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        const float mean = sum / 128.f;
        float sq = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = x[b][e] - mean;
                sq = fmaf(d, d, sq);
            }
        sq += __shfl_xor(sq, 16, 64);
        sq += __shfl_xor(sq, 32, 64);
        const float rstd = 1.0f / sqrtf(sq / 128.f + 1e-5f);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const f32x4 lw = *reinterpret_cast<const f32x4 *>(p.lnw + 16 * b + 4 * g);
            const f32x4 lb = *reinterpret_cast<const f32x4 *>(p.lnb + 16 * b + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[b][e] = (x[b][e] - mean) * rstd * lw[e] + lb[e];
        }
    }
    f32x4 q[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int j = 0; j < 2; ++j) q[j] = mfma(fq[kb][j][e], x[kb][e], q[j]);
    const float scale = 0.25f * kLog2e;
#pragma unroll
    for (int j = 0; j < 2; ++j) q[j] = (q[j] + *reinterpret_cast<const f32x4 *>(p.qb + 16 * (2 * w + j) + 4 * g)) * scale;

    // The tail's fragments for this wave and its state blocks, in flight
    // during the attention.
    f32x4 fo[8][2], f1[2][8][2], s1[2];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) fo[kb][j] = *reinterpret_cast<const f32x4 *>(pk + kb * 2048 + (2 * w + j) * 256);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
                f1[sl][kb][hb] =
                    *reinterpret_cast<const f32x4 *>(pk + (2 + 2 * w + sl) * kChunkFloats + (kb * 2 + hb) * 256);
#pragma unroll
    for (int j = 0; j < 2; ++j) s1[j] = *reinterpret_cast<const f32x4 *>(xrow + 16 * (2 * w + j));

    // Heads 2 w + j, as column_block_kernel.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        f32x4 s[8];
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) acc = mfma(kf[j][kb][st], q[j][st], acc);
            s[kb] = acc;
        }
        float m = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) m = fmaxf(m, fmaxf(fmaxf(s[kb][0], s[kb][1]), fmaxf(s[kb][2], s[kb][3])));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float l = 0.f;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                s[kb][rr] = __builtin_amdgcn_exp2f(s[kb][rr] - m);
                l += s[kb][rr];
            }
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float inv = 1.0f / l;
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) o = mfma(vv[j][kb][rr], s[kb][rr], o);
        *reinterpret_cast<f32x4 *>(&as[m16 * kS1Stride + 16 * (2 * w + j) + 4 * g]) = o * inv;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = *reinterpret_cast<const f32x4 *>(&as[m16 * kS1Stride + 16 * b + 4 * g]);
    Tail128 t{};
    t.bo = p.bo, t.n2w = p.n2w, t.n2b = p.n2b, t.b1 = p.b1, t.b2 = p.b2;
    rows16_chain(t, x, s1, fo, f1, s1s, hs, pk, w, m16, g, xrow, live);
}

// The head of a 128-wide block: y = LN1(x) W^T + b over 16 NB outputs,
// written row-major; the same per-wave layout as tail128, the fragments of W
// in (k-block, output block) order streamed through the same LDS buffers.
template <int NB>
__global__ __launch_bounds__(256, 3) void head128_kernel(Head128 p) {
    // 16 KB halves of the packed chunks, as tail128 streams them: 32 KB of LDS
    // per workgroup, so three (four at 8 and 16 output blocks, whose
    // registers allow it) share a CU.
    __shared__ __attribute__((aligned(16))) float buf[2][kHalfFloats];
    constexpr int kFrags = 8 * NB, kHeadHalves = (kFrags + 15) / 16;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;
    const long long row = (long long)blockIdx.x * kTailRows + wv * 16 + m16;
    const bool live = row < p.m;
    const long long r = live ? row : p.m - 1;
    auto issue = [&](int hc) {
        // A short last half still moves 16 KB: the pack is padded to whole chunks.
        const float *src = p.pack + (long long)hc * kHalfFloats + (4 * wv) * 256 + lane * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(src + i * 256, (lds_void *)&buf[hc & 1][(4 * wv + i) * 256], 16, 0, 0);
    };
    issue(0);

    f32x4 x[8];
    const float *xr = p.x + r * p.ldx + 4 * g;
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = *reinterpret_cast<const f32x4 *>(xr + 16 * b);
    // LN1 over the row's 128 features (lanes m, m + 16, m + 32, m + 48).
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b) sum += (x[b][0] + x[b][1]) + (x[b][2] + x[b][3]);
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float mean = sum / 128.f;
    float sq = 0.f;
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = x[b][e] - mean;
            sq = fmaf(d, d, sq);
        }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    const float rstd = 1.0f / sqrtf(sq / 128.f + 1e-5f);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const f32x4 w = *reinterpret_cast<const f32x4 *>(p.lnw + 16 * b + 4 * g);
        const f32x4 bb = *reinterpret_cast<const f32x4 *>(p.lnb + 16 * b + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[b][e] = (x[b][e] - mean) * rstd * w[e] + bb[e];
    }

    f32x4 acc[NB];
#pragma unroll
    for (int ob = 0; ob < NB; ++ob) acc[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kHeadHalves; ++c) {
        wait_vm();
        __syncthreads();
        if (c + 1 < kHeadHalves) issue(c + 1);
        const float *frag = &buf[c & 1][lane * 4];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int f = 16 * c + i;
            if (f < kFrags) {
                const int kb = f / NB, ob = f % NB;
                const f32x4 a = lds4(frag + i * 256);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[ob] = mfma(a[e], x[kb][e], acc[ob]);
            }
        }
    }
    if (!live) return;
    float *out = p.out + row * p.ldo + 4 * g;
#pragma unroll
    for (int ob = 0; ob < NB; ++ob)
        *reinterpret_cast<f32x4 *>(out + 16 * ob) = acc[ob] + *reinterpret_cast<const f32x4 *>(p.b + 16 * ob + 4 * g);
}

}  // namespace

size_t head128_pack_floats(int outputs) { return (size_t)(8 * (outputs / 16) + 31) / 32 * kChunkFloats; }

void head128_pack(const float *w, int outputs, float *out) {
    const int nb = outputs / 16;
    std::fill(out, out + head128_pack_floats(outputs), 0.f);
    for (int kb = 0; kb < 8; ++kb)
        for (int ob = 0; ob < nb; ++ob) {
            float *dst = out + (size_t)(kb * nb + ob) * 256;
            for (int l = 0; l < 64; ++l)
                for (int e = 0; e < 4; ++e) dst[l * 4 + e] = w[(long long)(16 * ob + (l & 15)) * 128 + 16 * kb + 4 * (l >> 4) + e];
        }
}

void head128(const Head128 &h, hipStream_t stream) {
    if (h.m <= 0) return;
    if (!h.x || !h.out || !h.pack || !h.lnw || !h.lnb || !h.b || (h.nb != 8 && h.nb != 16 && h.nb != 24))
        fail(3, "head128: unsupported arguments");
    if ((h.ldx & 3) || (h.ldo & 3) || (reinterpret_cast<uintptr_t>(h.x) & 15) ||
        (reinterpret_cast<uintptr_t>(h.out) & 15) || (reinterpret_cast<uintptr_t>(h.pack) & 15))
        fail(3, "head128: rows must be 16-byte aligned");
    const double m = (double)h.m, n = 16.0 * h.nb;
    KernelTimer timer(kFamGemm, stream, 2.0 * m * 128.0 * n, 4.0 * m * (128.0 + n) + 4.0 * 128.0 * n);
    const dim3 grid((unsigned)ceil_div(h.m, (long long)kTailRows)), block(256);
    if (h.nb == 8)
        hipLaunchKernelGGL(head128_kernel<8>, grid, block, 0, stream, h);
    else if (h.nb == 16)
        hipLaunchKernelGGL(head128_kernel<16>, grid, block, 0, stream, h);
    else
        hipLaunchKernelGGL(head128_kernel<24>, grid, block, 0, stream, h);
    IRX_HIP(hipGetLastError());
}

void tail128_pack(const float *wo, const float *w1, const float *w2, float *out) {
    // Fragment (rows r0.., columns c0..) of a row-major [.., ld] matrix:
    // lane (n, g) = (l % 16, l / 16) holds W[r0 + n][c0 + 4 g .. c0 + 4 g + 3].
    auto fragment = [](const float *w, int ld, int r0, int c0, float *dst) {
        for (int l = 0; l < 64; ++l)
            for (int e = 0; e < 4; ++e) dst[l * 4 + e] = w[(long long)(r0 + (l & 15)) * ld + c0 + 4 * (l >> 4) + e];
    };
    for (int c = 0; c < 2; ++c)
        for (int kb = 0; kb < 4; ++kb)
            for (int ob = 0; ob < 8; ++ob)
                fragment(wo, 128, 16 * ob, 16 * (4 * c + kb), out + c * kChunkFloats + (kb * 8 + ob) * 256);
    for (int c = 0; c < 8; ++c) {
        float *chunk = out + (2 + c) * kChunkFloats;
        for (int kb = 0; kb < 8; ++kb)
            for (int hb = 0; hb < 2; ++hb) fragment(w1, 128, 32 * c + 16 * hb, 16 * kb, chunk + (kb * 2 + hb) * 256);
        for (int j = 0; j < 2; ++j)
            for (int ob = 0; ob < 8; ++ob) fragment(w2, 256, 16 * ob, 32 * c + 16 * j, chunk + 4096 + (j * 8 + ob) * 256);
    }
}

void tail128(const Tail128 &t, hipStream_t stream, bool rows16) {
    if (t.m <= 0) return;
    if (!t.att || !t.state || !t.pack || !t.bo || !t.n2w || !t.n2b || !t.b1 || !t.b2)
        fail(3, "tail128: missing tensor");
    if ((t.lda & 3) || (t.ldx & 3) || (reinterpret_cast<uintptr_t>(t.att) & 15) ||
        (reinterpret_cast<uintptr_t>(t.state) & 15) || (reinterpret_cast<uintptr_t>(t.pack) & 15))
        fail(3, "tail128: rows must be 16-byte aligned");
    const double m = (double)t.m;
    // Products 2 m (128*128 + 2 * 128*256); bytes: att and state in, state out, weights.
    KernelTimer timer(kFamGemm, stream, m * 2.0 * (128.0 * 128 + 2 * 128.0 * 256), m * 128 * 4 * 3.0 + kTail128PackFloats * 4.0);
    if (rows16)
        hipLaunchKernelGGL(tail128_rows16_kernel, dim3((unsigned)ceil_div(t.m, 16LL)), dim3(256), 0, stream, t);
    else
        hipLaunchKernelGGL(tail128_kernel, dim3((unsigned)ceil_div(t.m, (long long)kTailRows)), dim3(256), 0, stream, t);
    IRX_HIP(hipGetLastError());
}

void column_block(const ColumnBlock &c, hipStream_t stream, bool rows16) {
    if (c.cols <= 0 || c.rows <= 0) return;
    if (!c.state || !c.k || !c.v || !c.lnw || !c.lnb || !c.qpack || !c.qb || !c.pack || !c.bo || !c.n2w || !c.n2b ||
        !c.b1 || !c.b2 || c.group <= 0)
        fail(3, "column_block: missing tensor");
    if ((reinterpret_cast<uintptr_t>(c.state) & 15) || (reinterpret_cast<uintptr_t>(c.k) & 15) ||
        (reinterpret_cast<uintptr_t>(c.v) & 15) || (reinterpret_cast<uintptr_t>(c.qpack) & 15) ||
        (reinterpret_cast<uintptr_t>(c.pack) & 15) || (c.group_stride & 3))
        fail(3, "column_block: operands must be 16-byte aligned");
    const long long tiles = (c.rows + kTailRows - 1) / kTailRows, units = tiles * c.cols;
    const long long per_xcd = (units + 7) / 8;
    if (per_xcd * 8 > 0x7fffffffLL) fail(3, "column_block: too many rows");
    const double m = (double)c.cols * (double)c.rows;
    // q, attention (scores and values over 128 keys x 8 heads of 16), the tail.
    const double flops = m * 2.0 * (128.0 * 128 + 2.0 * 128 * 128 + 128.0 * 128 + 2 * 128.0 * 256);
    KernelTimer timer(kFamGemm, stream, flops, m * 128 * 4 * 2.0 + (double)c.cols * kColumnCache * 8.0);
    if (rows16) {
        const long long groups = (c.rows + 15) / 16;
        if (groups * c.cols > 0x7fffffffLL) fail(3, "column_block: too many rows");
        hipLaunchKernelGGL(column_block_rows16_kernel, dim3((unsigned)(groups * c.cols)), dim3(256), 0, stream, c,
                           (int)groups);
    } else {
        hipLaunchKernelGGL(column_block_kernel, dim3((unsigned)(per_xcd * 8)), dim3(256), 0, stream, c, (int)tiles,
                           (int)per_xcd);
    }
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
