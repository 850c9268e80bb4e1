// Projection GEMMs of the DiT block for gfx950: y[M,N] = x[M,K] . W[N,K]^T (+bias)
// (+GELU-tanh), BF16 activations and output, FP32 accumulation.
//
// Weights are either BF16 (reference h3_gpu_linear_bf16, src/cuda/gpu_cuda.cu:927-1011)
// or W8A16 q8: int8 codes [N,K] with fp32 scales per (row, K-group); the group is
// 64 in the reference q8 recipe (src/weights/q8.c:26-56) or K for one scale per
// output channel. The q8 arithmetic is the reference's Metal kernel
// (src/metal/shaders.metal:799-855): every weight is reconstructed as
// w = bf16(code * scale) and multiplied in FP32 accumulation, bf16 output (+bias).
//
// MI355X design:
//  * C^T = W . X^T on v_mfma_f32_32x32x16_bf16, so a lane owns one output row and
//    four consecutive columns per register group (8-byte row-major stores);
//  * 256 x 256 output tile per workgroup of 8 waves (each 128 x 64, 8
//    accumulator blocks, two waves per SIMD), K staged 64 at a time, double
//    buffered in LDS, operand fragments of the next k-step read during MFMAs;
//  * X tiles go global -> LDS directly (global_load_lds_dwordx4, XOR-swizzled
//    16-byte chunks); int8 weight tiles are loaded into registers one tile ahead,
//    dequantized in registers (w = bf16(code * scale)) and written to LDS as BF16,
//    so each weight is converted once per workgroup, not per wave;
//  * tile ids are XCD-remapped and grouped along M so that the workgroups an XCD
//    runs together share weight columns in its L2;
//  * per-channel q8 (group == K) runs gemm_q8_staged: the int8 tile two steps
//    ahead goes straight to LDS, and the next step's dequantization shares a
//    basic block with this step's MFMAs, so its VALU work issues between them.
#include "common.h"
#include "internal.h"
#include <cmath>


namespace {

constexpr int TM = 256, TN = 256, TK = 64;
constexpr int ROW_BYTES = TK * 2;               // 128 B per BF16 tile row
constexpr int TILE_BYTES = 256 * ROW_BYTES;     // 32 KB per operand tile
constexpr int STAGE = 2 * TILE_BYTES;           // X tile + W tile
constexpr int GROUP_M = 8;                      // tile rows per grouped band

// 16-byte chunk swizzle of a 128-byte LDS row. A ds_read_b128 serves sixteen
// lanes (sixteen consecutive rows) per cycle across 256 bytes of banks: rows
// 2i and 2i+1 sit in different halves, and (row >> 1) & 7 spreads the eight
// pairs over eight chunks. Writes are served eight lanes per cycle across 128
// bytes; the weight store therefore gives eight consecutive lanes eight rows
// of the same parity (see w_row).
__device__ inline unsigned swz(unsigned row, unsigned ch) { return ch ^ ((row >> 1) & 7); }

// Weight staging map: chunk c (0..1023) of a 256 x 64 int8 tile -> (row, part).
// A wave covers 16 rows x 4 parts; lanes 8i..8i+7 of a part take rows of one
// parity, so their LDS stores hit eight different chunks.
__device__ inline unsigned w_row(unsigned c) { const unsigned l = c % 16; return (c / 64) * 16 + 2 * (l % 8) + l / 8; }
__device__ inline unsigned w_part(unsigned c) { return (c / 16) % 4; }

struct GemmArgs {
    uint16_t *y;
    const uint16_t *x;
    const void *w;            // bf16 [N,K] or int8 [N,K]
    const float *scales;      // q8: [N, groups]
    const uint16_t *bias;     // optional [N]
    const float *alpha;       // EPI bit 2: device scalar multiplying the accumulator
    unsigned m, n, k, group, groups;
    int gelu;
};

__device__ inline float gelu_tanh(float v) {
    // Reference h3_gelu_bf16, approximate form (src/cuda/cuda_kernels.cuh:879-902);
    // tanh(t) = 1 - 2 / (exp(2t) + 1) on the exp unit, |t| < 10 here.
    float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    if (inner <= -10.0f) return 0.0f;
    if (inner >= 10.0f) return v;
    float t = 1.0f - 2.0f / (__expf(2.0f * inner) + 1.0f);
    return 0.5f * v * (1.0f + t);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// WM x WN waves; each wave owns a (256 / WM) x (256 / WN) output tile of
// 32 x 32 MFMA blocks. 2 x 4 waves (128 x 64 per wave, two waves per SIMD) or
// 2 x 2 waves (128 x 128 per wave, one wave per SIMD: the 256 accumulator
// registers sit in AGPRs, and each fragment read from LDS feeds four MFMAs
// instead of two or four). CHANNEL: one scale per output row (group == K),
// loaded once. EPI bit 0: bias, bit 1: GELU, bit 2: alpha (before the bias).
template <bool Q8, bool CHANNEL, int EPI, int WM = 2, int WN = 4>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WM * WN, 64 * WM * WN),
                          amdgpu_waves_per_eu(WM * WN / 4, WM * WN / 4)))
void gemm_kernel(GemmArgs a) {
    constexpr int T = 64 * WM * WN;            // threads
    constexpr int NBM = TM / WM / 32, NBN = TN / WN / 32;
    constexpr int WCH = 1024 / T;              // weight chunks per thread
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64, n32 = lane % 32, hf = lane / 32;
    const unsigned tiles_m = (a.m + TM - 1) / TM, tiles_n = a.n / TN;
    // XCD-aware id, then grouped ordering: GROUP_M tile rows sweep the columns together.
    const unsigned pid = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned band = pid / (GROUP_M * tiles_n), first_m = band * GROUP_M;
    const unsigned rows_in_band = min(tiles_m - first_m, (unsigned)GROUP_M);
    const unsigned tm = first_m + (pid % (GROUP_M * tiles_n)) % rows_in_band;
    const unsigned tn = (pid % (GROUP_M * tiles_n)) / rows_in_band;
    const unsigned m0 = tm * TM, n0 = tn * TN;
    const unsigned wm = wave / WN, wn = wave % WN;   // wave rows m0 + wm*32*NBM, columns n0 + wn*32*NBN
    const unsigned ksteps = a.k / TK;

    f32x16 acc[NBN][NBM];   // [n block][m block], C^T layout: lane = output row, regs = columns
#pragma unroll
    for (int i = 0; i < NBN; i++)
#pragma unroll
        for (int j = 0; j < NBM; j++) acc[i][j] = f32x16{};

    // Weight staging (q8): 256 rows x 64 int8 = 1024 16-byte chunks, WCH per thread.
    i32x4 wq[WCH];
    float wscale[WCH];
    if constexpr (Q8 && CHANNEL) {
#pragma unroll
        for (int j = 0; j < WCH; j++) wscale[j] = a.scales[n0 + w_row(tid + T * j)];
    }
    auto load_w = [&](unsigned kt) {
        if constexpr (Q8) {
            const int8_t *w8 = reinterpret_cast<const int8_t *>(a.w);
#pragma unroll
            for (int j = 0; j < WCH; j++) {
                unsigned c = tid + T * j, row = w_row(c), part = w_part(c);
                wq[j] = *reinterpret_cast<const i32x4 *>(w8 + (size_t)(n0 + row) * a.k + kt * TK + part * 16);
                if constexpr (!CHANNEL)
                    wscale[j] = a.scales[(size_t)(n0 + row) * a.groups + (kt * TK + part * 16) / a.group];
            }
        }
    };
    auto x_stage = [&](int stage) { return lds + stage * STAGE; };
    auto w_stage = [&](int stage) { return lds + stage * STAGE + TILE_BYTES; };
    auto store_w = [&](int stage) {
        if constexpr (Q8) {
            uint8_t *ws = w_stage(stage);
#pragma unroll
            for (int j = 0; j < WCH; j++) {
                unsigned c = tid + T * j, row = w_row(c), part = w_part(c);
                bf16x8 half[2];
#pragma unroll
                for (int e = 0; e < 16; e += 2) {
                    int word = wq[j][e / 4];
                    f32x2 f = {(float)(int8_t)(word >> (8 * (e % 4))) * wscale[j],
                               (float)(int8_t)(word >> (8 * (e % 4 + 1))) * wscale[j]};
                    bf16x2 b = __builtin_convertvector(f, bf16x2);
                    half[e / 8][e % 8] = b[0];
                    half[e / 8][e % 8 + 1] = b[1];
                }
                *reinterpret_cast<bf16x8 *>(ws + row * ROW_BYTES + swz(row, part * 2) * 16) = half[0];
                *reinterpret_cast<bf16x8 *>(ws + row * ROW_BYTES + swz(row, part * 2 + 1) * 16) = half[1];
            }
        }
    };
    // Direct global -> LDS loads: X rows (clamped at M) and, for BF16 weights, W rows.
    auto load_direct = [&](unsigned kt, int stage) {
        uint8_t *xs = x_stage(stage);
#pragma unroll
        for (unsigned b = wave; b < 32; b += WM * WN) {
            unsigned row = 8 * b + lane / 8, ph = lane % 8;
            unsigned gm = min(m0 + row, a.m - 1);
            const uint16_t *src = a.x + (size_t)gm * a.k + kt * TK + swz(row, ph) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(xs + b * 1024), 16, 0, 0);
            if constexpr (!Q8) {
                const uint16_t *wsrc = reinterpret_cast<const uint16_t *>(a.w) + (size_t)(n0 + row) * a.k + kt * TK + swz(row, ph) * 8;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)wsrc,
                                                 (__attribute__((address_space(3))) void *)(xs + TILE_BYTES + b * 1024), 16, 0, 0);
            }
        }
    };
    auto frags = [&](const uint8_t *xs, const uint8_t *ws, int ks, bf16x8 *wf, bf16x8 *xf) {
#pragma unroll
        for (int i = 0; i < NBN; i++) {
            unsigned wr = wn * 32 * NBN + i * 32 + n32;
            wf[i] = *reinterpret_cast<const bf16x8 *>(ws + wr * ROW_BYTES + swz(wr, ks * 2 + hf) * 16);
        }
#pragma unroll
        for (int j = 0; j < NBM; j++) {
            unsigned xr = wm * 32 * NBM + j * 32 + n32;
            xf[j] = *reinterpret_cast<const bf16x8 *>(xs + xr * ROW_BYTES + swz(xr, ks * 2 + hf) * 16);
        }
    };

    {
    load_direct(0, 0);
    load_w(0);
    store_w(0);
    wait_vm_loads();
    __syncthreads();

    for (unsigned kt = 0; kt < ksteps; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < ksteps;
        if (more) { load_direct(kt + 1, cur ^ 1); load_w(kt + 1); }
        const uint8_t *xs = x_stage(cur);
        const uint8_t *ws = w_stage(cur);
        // Fragments of k-step ks+1 are read while the MFMAs of ks run.
        bf16x8 wf[2][NBN], xf[2][NBM];
        frags(xs, ws, 0, wf[0], xf[0]);
#pragma unroll
        for (int ks = 0; ks < TK / 16; ks++) {
            if (ks + 1 < TK / 16) frags(xs, ws, ks + 1, wf[(ks + 1) & 1], xf[(ks + 1) & 1]);
#pragma unroll
            for (int i = 0; i < NBN; i++)
#pragma unroll
                for (int j = 0; j < NBM; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][i], xf[ks & 1][j], acc[i][j], 0, 0, 0);
        }
        if (more) store_w(cur ^ 1);
        wait_vm_loads();
        __syncthreads();
    }
    }

    // Epilogue: lane holds output row m = m0 + wm*32*NBM + j*32 + n32 and columns
    // n0 + wn*32*NBN + i*32 + g*8 + hf*4 + 0..3 for register group g.
#pragma unroll
    for (int j = 0; j < NBM; j++) {
        const unsigned row = m0 + wm * 32 * NBM + j * 32 + n32;
        if (row >= a.m) continue;
        uint16_t *dst = a.y + (size_t)row * a.n;
#pragma unroll
        for (int i = 0; i < NBN; i++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const unsigned col = n0 + wn * 32 * NBN + i * 32 + g4 * 8 + hf * 4;
                u16x4 out;
                u16x4 bias4 = {};
                if constexpr (EPI & 1) bias4 = *reinterpret_cast<const u16x4 *>(a.bias + col);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = acc[i][j][g4 * 4 + e];
                    if constexpr (EPI & 4) v *= a.alpha[0];
                    if constexpr (EPI & 1) v += bf16_to_f32(bias4[e]);
                    uint16_t b = f32_to_bf16(v);
                    if constexpr (EPI & 2) b = f32_to_bf16(gelu_tanh(bf16_to_f32(b)));
                    out[e] = b;
                }
                *reinterpret_cast<u16x4 *>(dst + col) = out;
            }
    }
}

// W8A16 with the int8 weight tile staged in LDS: 8 waves (2 x 4, 128 x 64
// per wave, two per SIMD) as gemm_kernel, but the int8 tile of step kt + 2 is
// fetched straight into LDS (buffer_load ... lds) during step kt, and the
// dequantization of step kt + 1 (LDS int8 -> registers -> BF16 LDS tile) runs
// in the same basic block as step kt's MFMAs, so its VALU work can issue
// between them instead of after them. No register is held across a step for
// the weights. LDS: two stages of X and BF16 W (128 KB) plus two int8 stages
// (32 KB). X rows past M load zeros (BUFFER_OOB lane offsets); W8 rows never
// pass N, a multiple of 256.
constexpr int W8_BYTES = 256 * TK;                  // 16 KB int8 tile
// Per-output-channel scales (group == K) only: they are loaded once.
template <int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void gemm_q8_staged(GemmArgs a) {
    constexpr int WM = 2, WN = 4, T = 512;
    constexpr int NBM = TM / WM / 32, NBN = TN / WN / 32;
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    uint8_t *const w8s = lds + 2 * STAGE;
    // wave is read as a uniform value, so LDS destinations and buffer offsets
    // stay scalar (no waterfall loop around the buffer loads).
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n32 = lane % 32, hf = lane / 32;
    const unsigned tiles_m = (a.m + TM - 1) / TM, tiles_n = a.n / TN;
    const unsigned pid = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned band = pid / (GROUP_M * tiles_n), first_m = band * GROUP_M;
    const unsigned rows_in_band = min(tiles_m - first_m, (unsigned)GROUP_M);
    const unsigned tm = first_m + (pid % (GROUP_M * tiles_n)) % rows_in_band;
    const unsigned tn = (pid % (GROUP_M * tiles_n)) / rows_in_band;
    const unsigned m0 = __builtin_amdgcn_readfirstlane(tm * TM), n0 = __builtin_amdgcn_readfirstlane(tn * TN);
    const unsigned wm = wave / WN, wn = wave % WN;
    const unsigned ksteps = a.k / TK;

    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, (int)((size_t)a.m * a.k * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.w, (short)0, (int)((size_t)a.n * a.k), 0x00020000);
    // X block b = wave + 8 t: rows 8 b + lane / 8, 16-byte chunk lane % 8
    // (swizzled); the swizzle does not depend on t, so one lane offset serves
    // all four loads.
    const uint32_t xoff = ((8 * wave + lane / 8) * a.k + swz(8 * wave + lane / 8, lane % 8) * 8) * 2;
    // Weight chunks c = tid + 512 j: row w_row(c) = w_row(tid) + 128 j, part w_part(tid).
    const unsigned wrow = w_row(tid), wpart = w_part(tid);
    const uint32_t woff = wrow * a.k + wpart * 16;

    f32x16 acc[NBN][NBM];
#pragma unroll
    for (int i = 0; i < NBN; i++)
#pragma unroll
        for (int j = 0; j < NBM; j++) acc[i][j] = f32x16{};

    float wscale[2];
#pragma unroll
    for (int j = 0; j < 2; j++) wscale[j] = a.scales[n0 + wrow + 128 * j];
    // Loads of step kt's data into the stages of step `at` (the step numbers
    // of the stages are unclamped, so a clamped reload never lands in a stage
    // that the current step reads).
    // In the last row tile, lanes whose row is at or past M take BUFFER_OOB
    // and load zeros (those output rows are not stored).
    const bool m_tail = m0 + TM > a.m;
    // TAIL: compiled in only for the last row tile's loop.
    auto load_x = [&](unsigned kt, unsigned at, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        uint8_t *xs = lds + (at & 1) * STAGE;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            auto *dst = (__attribute__((address_space(3))) void *)(xs + (wave + 8 * t) * 1024);
            const uint32_t so = (uint32_t)(((size_t)m0 + 64 * t) * a.k * 2 + kt * TK * 2);
            if constexpr (TAIL) {
                const unsigned row = m0 + 64 * t + 8 * wave + lane / 8;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst, 16, row < a.m ? xoff : BUFFER_OOB, so, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst, 16, xoff, so, 0, 0);
            }
        }
    };
    auto load_w8 = [&](unsigned kt, unsigned at) {
        uint8_t *ws8 = w8s + (at & 1) * W8_BYTES;
#pragma unroll
        for (int j = 0; j < 2; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wr, (__attribute__((address_space(3))) void *)(ws8 + (wave + 8 * j) * 1024), 16, woff,
                (uint32_t)(((size_t)n0 + 128 * j) * a.k + kt * TK), 0, 0);
    };
    // int8 chunks of stage `at` (this thread's own two) -> BF16 W stage at & 1.
    auto dequant = [&](unsigned at) {
        const uint8_t *ws8 = w8s + (at & 1) * W8_BYTES;
        uint8_t *ws = lds + (at & 1) * STAGE + TILE_BYTES;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const i32x4 q = *reinterpret_cast<const i32x4 *>(ws8 + (tid + T * j) * 16);
            const unsigned row = wrow + 128 * j;
            bf16x8 half[2];
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                int word = q[e / 4];
                f32x2 f = {(float)(int8_t)(word >> (8 * (e % 4))) * wscale[j],
                           (float)(int8_t)(word >> (8 * (e % 4 + 1))) * wscale[j]};
                bf16x2 b = __builtin_convertvector(f, bf16x2);
                half[e / 8][e % 8] = b[0];
                half[e / 8][e % 8 + 1] = b[1];
            }
            *reinterpret_cast<bf16x8 *>(ws + row * ROW_BYTES + swz(row, wpart * 2) * 16) = half[0];
            *reinterpret_cast<bf16x8 *>(ws + row * ROW_BYTES + swz(row, wpart * 2 + 1) * 16) = half[1];
        }
    };
    auto frags = [&](const uint8_t *xs, const uint8_t *ws, int ks, bf16x8 *wf, bf16x8 *xf) {
#pragma unroll
        for (int i = 0; i < NBN; i++) {
            unsigned wr_ = wn * 32 * NBN + i * 32 + n32;
            wf[i] = *reinterpret_cast<const bf16x8 *>(ws + wr_ * ROW_BYTES + swz(wr_, ks * 2 + hf) * 16);
        }
#pragma unroll
        for (int j = 0; j < NBM; j++) {
            unsigned xr_ = wm * 32 * NBM + j * 32 + n32;
            xf[j] = *reinterpret_cast<const bf16x8 *>(xs + xr_ * ROW_BYTES + swz(xr_, ks * 2 + hf) * 16);
        }
    };

    // Prologue: X(0), W8(0), W8(1); W(0) dequantized.
    if (m_tail) load_x(0, 0, std::true_type{});
    else load_x(0, 0, std::false_type{});
    load_w8(0, 0);
    load_w8(min(1u, ksteps - 1), 1);
    wait_vm_loads();
    __syncthreads();
    dequant(0);
    __syncthreads();

    // The K loop, instantiated for the last row tile and for the others.
    // Fragments are read one sub-step ahead of their MFMAs; in the last
    // sub-step the barrier comes first and the next tile's first fragments are
    // read before this sub-step's MFMAs, so their LDS latency sits under them
    // (after the last tile those reads land in registers nobody uses). The
    // sched_barrier keeps hipcc from sinking the reads below the MFMAs.
    auto kloop = [&](auto tail_tag) {
    bf16x8 wf[2][NBN], xf[2][NBM];
    frags(lds, lds + TILE_BYTES, 0, wf[0], xf[0]);
    for (unsigned kt = 0; kt < ksteps; kt++) {
        const unsigned k1 = min(kt + 1, ksteps - 1), k2 = min(kt + 2, ksteps - 1);
        load_x(k1, kt + 1, tail_tag);
        load_w8(k2, kt + 2);
        const uint8_t *xs = lds + (kt & 1) * STAGE;
        const uint8_t *ws = xs + TILE_BYTES;
#pragma unroll
        for (int ks = 0; ks < TK / 16; ks++) {
            if (ks + 1 < TK / 16) {
                frags(xs, ws, ks + 1, wf[(ks + 1) & 1], xf[(ks + 1) & 1]);
            } else {
                wait_vm_loads();
                __syncthreads();
                const uint8_t *nx = lds + ((kt + 1) & 1) * STAGE;
                frags(nx, nx + TILE_BYTES, 0, wf[0], xf[0]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NBN; i++)
#pragma unroll
                for (int j = 0; j < NBM; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][i], xf[ks & 1][j], acc[i][j], 0, 0, 0);
            if (ks == 0) dequant(kt + 1);
        }
    }
    };
    if (m_tail) kloop(std::true_type{});
    else kloop(std::false_type{});

#pragma unroll
    for (int j = 0; j < NBM; j++) {
        const unsigned row = m0 + wm * 32 * NBM + j * 32 + n32;
        if (row >= a.m) continue;
        uint16_t *dst = a.y + (size_t)row * a.n;
#pragma unroll
        for (int i = 0; i < NBN; i++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const unsigned col = n0 + wn * 32 * NBN + i * 32 + g4 * 8 + hf * 4;
                u16x4 out;
                u16x4 bias4 = {};
                if constexpr (EPI & 1) bias4 = *reinterpret_cast<const u16x4 *>(a.bias + col);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = acc[i][j][g4 * 4 + e];
                    if constexpr (EPI & 1) v += bf16_to_f32(bias4[e]);
                    uint16_t b = f32_to_bf16(v);
                    if constexpr (EPI & 2) b = f32_to_bf16(gelu_tanh(bf16_to_f32(b)));
                    out[e] = b;
                }
                *reinterpret_cast<u16x4 *>(dst + col) = out;
            }
    }
}

template <int EPI>
int launch_staged(h3_gpu *g, const GemmArgs &a) {
    constexpr size_t shared = 2 * STAGE + 2 * W8_BYTES;
    static bool configured = false;
    auto kernel = gemm_q8_staged<EPI>;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)shared), "GEMM shared memory"))
            return 0;
        configured = true;
    }
    unsigned tiles = (a.m + TM - 1) / TM * (a.n / TN);
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(kernel, dim3(tiles), dim3(512), shared, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "W8A16 GEMM");
}

// Any-shape fallback (small or unaligned projections): one thread per output,
// FP32 accumulation in k order. Same weight reconstruction as the tiled kernel.
__global__ __launch_bounds__(256) void gemm_small(GemmArgs a, int q8) {
    size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)a.m * a.n) return;
    unsigned row = idx / a.n, col = idx % a.n;
    const uint16_t *xr = a.x + (size_t)row * a.k;
    float acc = 0.f;
    for (unsigned kk = 0; kk < a.k; kk++) {
        float w;
        if (q8) {
            int q = reinterpret_cast<const int8_t *>(a.w)[(size_t)col * a.k + kk];
            w = bf16_to_f32(f32_to_bf16((float)q * a.scales[(size_t)col * a.groups + kk / a.group]));
        } else {
            w = bf16_to_f32(reinterpret_cast<const uint16_t *>(a.w)[(size_t)col * a.k + kk]);
        }
        acc = fmaf(bf16_to_f32(xr[kk]), w, acc);
    }
    if (a.alpha) acc *= a.alpha[0];
    if (a.bias) acc += bf16_to_f32(a.bias[col]);
    uint16_t b = f32_to_bf16(acc);
    if (a.gelu) b = f32_to_bf16(gelu_tanh(bf16_to_f32(b)));
    a.y[idx] = b;
}

template <bool Q8, bool CHANNEL, int EPI, int WM = 2, int WN = 4>
int launch_tiled(h3_gpu *g, const GemmArgs &a) {
    constexpr size_t shared = 2 * STAGE;
    static bool configured = false;
    auto kernel = gemm_kernel<Q8, CHANNEL, EPI, WM, WN>;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)shared), "GEMM shared memory"))
            return 0;
        configured = true;
    }
    unsigned tiles = (a.m + TM - 1) / TM * (a.n / TN);
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(kernel, dim3(tiles), dim3(64 * WM * WN), shared, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, Q8 ? "W8A16 GEMM" : "BF16 GEMM");
}

template <bool Q8, bool CHANNEL>
int launch_epi(h3_gpu *g, const GemmArgs &a) {
    const int epi = (a.bias ? 1 : 0) | (a.gelu ? 2 : 0);
    if constexpr (Q8 && CHANNEL) {
        // Per-channel W8A16 (the synthetic DiT): int8 tiles
        // staged in LDS (buffer offsets are 32-bit). Variant 2 keeps the
        // register-staged weights of gemm_kernel (3-4% slower on config 4).
        if (g->gemm_variant != 2 && (size_t)a.m * a.k * 2 < (1ull << 31) && (size_t)a.n * a.k < (1ull << 31)) {
            switch (epi) {
            case 0: return launch_staged<0>(g, a);
            case 1: return launch_staged<1>(g, a);
            case 2: return launch_staged<2>(g, a);
            default: return launch_staged<3>(g, a);
            }
        }
    }
    // Variant 1: 2 x 2 waves of 128 x 128 (one wave per SIMD), about 10% slower.
    if (g->gemm_variant == 1) {
        switch (epi) {
        case 0: return launch_tiled<Q8, CHANNEL, 0, 2, 2>(g, a);
        case 1: return launch_tiled<Q8, CHANNEL, 1, 2, 2>(g, a);
        case 2: return launch_tiled<Q8, CHANNEL, 2, 2, 2>(g, a);
        default: return launch_tiled<Q8, CHANNEL, 3, 2, 2>(g, a);
        }
    }
    switch (epi) {
    case 0: return launch_tiled<Q8, CHANNEL, 0>(g, a);
    case 1: return launch_tiled<Q8, CHANNEL, 1>(g, a);
    case 2: return launch_tiled<Q8, CHANNEL, 2>(g, a);
    default: return launch_tiled<Q8, CHANNEL, 3>(g, a);
    }
}

}  // namespace

// y[M,N] = bf16(alpha[0] * x[M,K] . w[N,K]^T) with BF16 device operands and a
// device scalar alpha (the NVFP4 projections' dequantized operands).
int h3_gemm_bf16_alpha(h3_gpu *g, uint16_t *y, const uint16_t *x, const uint16_t *w, const float *alpha, uint32_t m,
                       uint32_t k, uint32_t n) {
    GemmArgs a{};
    a.y = y; a.x = x; a.w = w; a.alpha = alpha; a.m = m; a.n = n; a.k = k; a.group = 1; a.groups = 1;
    if (n % TN == 0 && k % TK == 0 && m >= 32) return launch_tiled<false, false, 4>(g, a);
    const size_t total = (size_t)m * n;
    hipLaunchKernelGGL(gemm_small, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g->compute, a, 0);
    return h3_launch_status(g, "small scaled GEMM");
}

int h3_gemm(h3_gpu *g, uint16_t *y, const uint16_t *x, const h3_gpu_tensor *w, const uint16_t *bias, uint32_t m,
            uint32_t k, uint32_t n, int gelu) {
    GemmArgs a{};
    a.y = y; a.x = x; a.w = w->data; a.bias = bias; a.m = m; a.n = n; a.k = k; a.gelu = gelu;
    a.scales = w->q8 ? w->q8_scales : nullptr;
    a.group = w->q8 ? w->q8_group : 1;
    a.groups = w->q8 ? (k + a.group - 1) / a.group : 1;
    if (!h3_tensor_acquire(g, w)) return 0;
    int ok;
    const bool tiled = n % TN == 0 && k % TK == 0 && m >= 32 && (!w->q8 || a.group % 16 == 0);
    if (tiled) {
        if (!w->q8) ok = launch_epi<false, false>(g, a);
        else if (a.group == k) ok = launch_epi<true, true>(g, a);
        else ok = launch_epi<true, false>(g, a);
    }
    else {
        size_t total = (size_t)m * n;
        hipLaunchKernelGGL(gemm_small, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g->compute, a, w->q8 ? 1 : 0);
        ok = h3_launch_status(g, "small GEMM");
    }
    if (ok) {
        g->stats.linear_dispatches++;
        if (w->q8) { g->stats.q8_dispatches++; g->stats.quant_projection_dispatches++; }
    }
    return ok && h3_tensor_release(g, w);
}
