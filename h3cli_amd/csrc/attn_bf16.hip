// FlashAttention-style BF16 self-attention for gfx950 (D = 128, non-causal).
//
// Semantics follow the reference's online-softmax operator
// (src/cuda/cuda_attention.cuh:7-51): softmax(scale * Q K^T) V with FP32 scores,
// FP32 running max / denominator and FP32 P.V accumulation, BF16 output. The
// difference is where P meets V: P is rounded to BF16 so that P.V runs on the
// BF16 matrix cores, as the reference's tensor-core path and FlashAttention do.
//
// Work decomposition (MI355X-first, not a translation of the CUDA kernels):
//  * one workgroup = WAVES wavefronts x 64 queries of one head; the query
//    fragments of a wave stay in VGPRs for the whole key sweep;
//  * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16:
//    each lane then owns one query column, so the row max is a register max
//    plus one exchange between the two 32-lane halves, and the FP32 score
//    accumulator is already laid out as the B operand of O^T += V^T P^T;
//  * K tiles (64 keys) are staged row-major in LDS, V tiles transposed in LDS
//    with a key permutation matching the score accumulator, both double
//    buffered with one barrier per tile; global loads of tile t+1 are issued
//    before the MFMAs of tile t;
//  * workgroup ids are remapped so that the workgroups of one head share an XCD
//    (and its L2), which is where their K/V tiles are re-read.
#include "common.h"
#include "internal.h"
#include "attn_common.h"

namespace {

constexpr int D = 128;
constexpr int BN = 64;                     // keys per tile
constexpr int K_STRIDE = D + 8;            // LDS row stride of the K tile (elements)
constexpr int V_STRIDE = BN + 8;           // LDS row stride of the transposed V tile
constexpr int K_ELEMS = BN * K_STRIDE;
constexpr int V_ELEMS = D * V_STRIDE;
constexpr int STAGE_ELEMS = K_ELEMS + V_ELEMS;

struct Args {
    uint16_t *out;
    const uint16_t *q, *k, *v;
    unsigned seq, heads;
    float scale_log2;                      // softmax scale * log2(e)
    int head_major;
    const uint32_t *kv_list;               // sparse: per 128-query block, kept 64-key tile ids (all heads)
    const uint32_t *kv_count;              // sparse: number of kept tiles per 128-query block
    unsigned list_stride;
    unsigned *fault;
};

// Position of key j (0..63) inside a transposed V row: keys are grouped by 16
// and, inside a group, ordered the way a lane half holds them in the S^T
// accumulator (rows (r/4)*8 + half*4 + r%4 of a 32x32 MFMA output).
__device__ inline unsigned v_position(unsigned j) {
    unsigned k16 = j & 15;
    return (j & ~15u) + ((k16 >> 2) & 1) * 8 + (k16 >> 3) * 4 + (k16 & 3);
}

template <int WAVES, bool SPARSE>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WAVES, 64 * WAVES), amdgpu_waves_per_eu(1, 1)))
void attn_bf16_kernel(Args a) {
    constexpr int T = 64 * WAVES;
    constexpr int BM = 64 * WAVES;
    constexpr int KCH = (BN * D / 8) / T;  // 16-byte K chunks per thread per tile
    constexpr int VU = (BN / 4) * (D / 8) / T;  // 4-key x 8-channel V units per thread
    static_assert(KCH * T == BN * D / 8 && VU * T == (BN / 4) * (D / 8), "tile split");
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned nqb = (a.seq + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = id / nqb, qb = id % nqb;
    const unsigned q0 = qb * BM;
    const size_t stride = (size_t)a.heads * D;
    const uint16_t *qh = a.q + (size_t)head * D;
    const uint16_t *kh = a.k + (size_t)head * D;
    const uint16_t *vh = a.v + (size_t)head * D;

    unsigned count;
    const uint32_t *list = nullptr;
    if constexpr (SPARSE) {
        count = a.kv_count[qb];
        list = a.kv_list + (size_t)qb * a.list_stride;
    } else {
        count = (a.seq + BN - 1) / BN;
    }

    // Query fragments: B operand of S^T = K Q^T, 8 k-steps of 16 channels.
    bf16x8 qf[2][8];
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
        unsigned row = q0 + wave * 64 + nb * 32 + n;
        row = row < a.seq ? row : a.seq - 1;
        const uint16_t *p = qh + (size_t)row * stride + hf * 8;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) qf[nb][ks] = *reinterpret_cast<const bf16x8 *>(p + ks * 16);
    }

    f32x16 o[4][2];
#pragma unroll
    for (int md = 0; md < 4; md++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++) o[md][nb] = f32x16{};
    float m[2] = {-1e30f, -1e30f}, l[2] = {0.f, 0.f};

    u16x8 rk[KCH];
    u16x8 rv[VU][4];
    auto load_tile = [&](unsigned tile) {
        const unsigned key0 = tile * BN;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            unsigned c = tid + T * j, key = key0 + c / 16, ch = c % 16;
            rk[j] = key < a.seq ? *reinterpret_cast<const u16x8 *>(kh + (size_t)key * stride + ch * 8) : u16x8{};
        }
#pragma unroll
        for (int j = 0; j < VU; j++) {
            unsigned u = tid + T * j, kg = u % 16, dc = u / 16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                unsigned key = key0 + kg * 4 + i;
                rv[j][i] = key < a.seq ? *reinterpret_cast<const u16x8 *>(vh + (size_t)key * stride + dc * 8) : u16x8{};
            }
        }
    };
    auto store_tile = [&](int stage) {
        uint16_t *ks = smem + stage * STAGE_ELEMS;
        uint16_t *vs = ks + K_ELEMS;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            unsigned c = tid + T * j, key = c / 16, ch = c % 16;
            *reinterpret_cast<u16x8 *>(ks + key * K_STRIDE + ch * 8) = rk[j];
        }
#pragma unroll
        for (int j = 0; j < VU; j++) {
            unsigned u = tid + T * j, kg = u % 16, dc = u / 16;
            unsigned pos = v_position(kg * 4);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                u16x4 col = {rv[j][0][e], rv[j][1][e], rv[j][2][e], rv[j][3][e]};
                *reinterpret_cast<u16x4 *>(vs + (dc * 8 + e) * V_STRIDE + pos) = col;
            }
        }
    };

    if (count) {
        load_tile(SPARSE ? list[0] : 0);
        store_tile(0);
    }
    __syncthreads();

    for (unsigned it = 0; it < count; it++) {
        const int cur = it & 1;
        const unsigned tile = SPARSE ? list[it] : it;
        const bool more = it + 1 < count;
        if (more) load_tile(SPARSE ? list[it + 1] : it + 1);

        const uint16_t *ks = smem + cur * STAGE_ELEMS;
        const uint16_t *vs = ks + K_ELEMS;

        // S^T[mb][nb]: 32 keys x 32 queries.
        f32x16 s[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
            for (int nb = 0; nb < 2; nb++) s[mb][nb] = f32x16{};
#pragma unroll
        for (int kstep = 0; kstep < 8; kstep++) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                bf16x8 kf = *reinterpret_cast<const bf16x8 *>(ks + (mb * 32 + n) * K_STRIDE + kstep * 16 + hf * 8);
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
                    s[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[nb][kstep], s[mb][nb], 0, 0, 0);
            }
        }
        if (tile * BN + BN > a.seq) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                    if (key >= a.seq) { s[mb][0][r] = -INFINITY; s[mb][1][r] = -INFINITY; }
                }
        }

        // Online softmax in the log2 domain; P rounded to BF16 as the PV operand.
        bf16x8 pb[2][4];
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            float mx = -INFINITY;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[mb][nb][r]);
            mx = fmaxf(mx, half_swap(mx));
            const float mnew = fmaxf(m[nb], mx * a.scale_log2);
            const float alpha = exp2f_fast(m[nb] - mnew);
            m[nb] = mnew;
            float psum = 0.f;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float p = exp2f_fast(fmaf(s[mb][nb][r], a.scale_log2, -mnew));
                    psum += p;
                    pb[nb][mb * 2 + r / 8][r % 8] = (__bf16)p;
                }
            l[nb] = fmaf(l[nb], alpha, psum);
#pragma unroll
            for (int md = 0; md < 4; md++) o[md][nb] *= alpha;
        }

        // O^T[md][nb] += V^T[md] P^T[nb]: 32 channels x 32 queries, 4 k-steps of 16 keys.
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
#pragma unroll
            for (int md = 0; md < 4; md++) {
                bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vs + (md * 32 + n) * V_STRIDE + kk * 16 + hf * 8);
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
                    o[md][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[nb][kk], o[md][nb], 0, 0, 0);
            }
        }

        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

    // Normalize and store. Lane holds query column n, channels (r/4)*8 + hf*4 + r%4.
    bool bad = false;
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
        const float total = l[nb] + half_swap(l[nb]);
        const float inv = total > 0.f ? 1.f / total : 0.f;
        const unsigned q = q0 + wave * 64 + nb * 32 + n;
        if (q >= a.seq) continue;
        uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
        for (int md = 0; md < 4; md++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                u16x4 w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float x = o[md][nb][g4 * 4 + i] * inv;
                    bad |= !__builtin_isfinite(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    if (bad) a.fault[0] = 1u;
}

template <int WAVES, bool SPARSE>
int launch(h3_gpu *g, const Args &a, unsigned groups) {
    constexpr size_t shared = 2 * STAGE_ELEMS * sizeof(uint16_t);
    static bool configured = false;
    auto kernel = attn_bf16_kernel<WAVES, SPARSE>;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shared),
                          "attention shared memory"))
            return 0;
        configured = true;
    }
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(64 * WAVES), shared, g->compute, a);
    return h3_launch_status(g, "BF16 attention");
}

}  // namespace

unsigned h3_attention_query_block(bool sparse) { return sparse ? 128u : 256u; }

int h3_launch_attention_bf16(h3_gpu *g, uint16_t *out, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                             uint32_t seq, uint32_t heads, float scale, bool head_major,
                             const uint32_t *kv_list, const uint32_t *kv_count, uint32_t list_stride) {
    Args a;
    a.out = out; a.q = q; a.k = k; a.v = v; a.seq = seq; a.heads = heads;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_major = head_major ? 1 : 0;
    a.kv_list = kv_list; a.kv_count = kv_count; a.list_stride = list_stride;
    a.fault = g->fault;
    if (kv_list) {
        unsigned nqb = (seq + 127) / 128;
        return launch<2, true>(g, a, nqb * heads);
    }
    unsigned nqb = (seq + 255) / 256;
    return launch<4, false>(g, a, nqb * heads);
}
