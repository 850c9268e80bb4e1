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
// Shapes with K % 128 == 0 and N % 256 == 0 (every DiT projection) run
// gemm_bf16_pipe instead: a hand-scheduled K loop at one wave per SIMD (see
// its comment). For W8A16 weights a dequantization pass first writes
// w = bf16(code * scale) for the whole weight into a BF16 buffer of the
// context (in registers, 16 codes per thread: the same reconstruction as
// above), which costs about 1% of the GEMM at M = 32400 and leaves the MFMA
// loop free of VALU work. gemm_q8_staged and gemm_kernel remain for the other
// shapes (and as H3_HIP_GEMM_VARIANT=3 for comparison).
#include "common.h"
#include "internal.h"
#include <cmath>


namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

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
    // Reference h3_gelu_bf16, approximate form (src/cuda/cuda_kernels.cuh:879-902):
    // 0.5 v (1 + tanh(c (v + 0.044715 v^3))), c = sqrt(2 / pi), written as
    // v / (1 + exp(-2 c (v + 0.044715 v^3))) with the hardware exp and
    // reciprocal (no IEEE division, no branches). Large |v| saturate through
    // exp: to v (exp -> 0) or to a signed zero (exp -> inf, reciprocal 0).
    const float u = v * (1.5957691216057308f + 0.071354816272192f * v * v);
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-u));
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

// ------------------------------------------------------------ hand-scheduled BF16 GEMM
// gemm_bf16_pipe: the same 256 x 256 output tile as gemm_kernel, computed by
// four waves of 128 x 128 (one per SIMD, 2 x 2) on v_mfma_f32_16x16x32_bf16,
// each wave with 8 x 8 accumulator blocks of 16 x 16 in AGPRs, so one
// fragment read from LDS feeds eight MFMAs. (The same loop on 32 x 32 x 16
// MFMAs, 4 x 4 blocks of 16 AGPRs, measured 6% slower on the config-4 shapes.)
// The whole K loop is one inline-asm block, because its value is the order of
// the instructions; with one wave per SIMD nothing else hides a stall:
//  * a K tile (64) is two substeps of 64 MFMAs (32 K each); the 16 fragments
//    of the next substep are read during the first half of the current one,
//    one ds_read_b128 after every second MFMA, into the other register set;
//  * the 16 global -> LDS loads of a K tile (buffer_load ... lds, 1 KB each)
//    are issued two tiles ahead, two per eight MFMAs of the second substep,
//    into the stage this tile has finished reading;
//  * one barrier per tile, between the substeps: every wave has then read
//    all fragments of this tile and its loads of the next tile (issued a
//    tile earlier) have landed; the next tile's first reads follow it.
// LDS (128 KB): X stage 0 at 0, X stage 1 at 32 KB, W stage 0 at 64 KB,
// W stage 1 at 96 KB; rows of 64 BF16 (128 B) with the 16-byte chunk swizzle
// of swz(). Requirements: K % 128 == 0 (tiles come in stage pairs),
// N % 256 == 0, M * K * 2 < 2^31 and N * K * 2 < 2^31 (32-bit offsets).
constexpr int PIPE_LDS = 4 * TILE_BYTES;     // 128 KB
// Tile rows per grouped band of the pipe kernel: an XCD's 32 resident
// workgroups then cover 4 row tiles x 8 column tiles (measured on the config-4
// shapes: 4 and 8 within 1% of each other, 4 ahead; 16 rows 13% slower).
constexpr int PIPE_GROUP_M = 4;

// Load T (0..7) of a K tile's X (PIPE_LD_X) or W (PIPE_LD_W) into stage ST:
// LDS block wave + 4 T (1 KB), rows 8 wave + lane / 8 + 32 T from the lane
// offset o<T>. The offsets are precomputed so that the loop holds no VALU
// instruction besides the MFMAs (with one wave per SIMD each one delays the
// next MFMA); kc is the tile's K byte offset.
#define PIPE_LD_X(ST, T) "s_add_u32 m0, %[mb], 32768*" #ST "+4096*" #T "\n"                                  \
    "buffer_load_dwordx4 %[o" #T "], %[sx], %[kc] offen lds\n"
#define PIPE_LD_W(ST, T) "s_add_u32 m0, %[mb], 65536+32768*" #ST "+4096*" #T "\n"                            \
    "buffer_load_dwordx4 %[o" #T "], %[sw], %[kc] offen lds\n"
#define PIPE_LOADS_X(ST) PIPE_LD_X(ST, 0) PIPE_LD_X(ST, 1) PIPE_LD_X(ST, 2) PIPE_LD_X(ST, 3)                      \
    PIPE_LD_X(ST, 4) PIPE_LD_X(ST, 5) PIPE_LD_X(ST, 6) PIPE_LD_X(ST, 7)
#define PIPE_LOADS_W(ST) PIPE_LD_W(ST, 0) PIPE_LD_W(ST, 1) PIPE_LD_W(ST, 2) PIPE_LD_W(ST, 3)                      \
    PIPE_LD_W(ST, 4) PIPE_LD_W(ST, 5) PIPE_LD_W(ST, 6) PIPE_LD_W(ST, 7)

#define PIPE_X8(ST) PIPE_LD_X(ST, 0), PIPE_LD_X(ST, 1), PIPE_LD_X(ST, 2), PIPE_LD_X(ST, 3), PIPE_LD_X(ST, 4),      \
    PIPE_LD_X(ST, 5), PIPE_LD_X(ST, 6), PIPE_LD_X(ST, 7)
#define PIPE_W8(ST) PIPE_LD_W(ST, 0), PIPE_LD_W(ST, 1), PIPE_LD_W(ST, 2), PIPE_LD_W(ST, 3), PIPE_LD_W(ST, 4),      \
    PIPE_LD_W(ST, 5), PIPE_LD_W(ST, 6), PIPE_LD_W(ST, 7)

// MFMA (i, j) of set S: W block i (16 rows) x X block j.
#define P16_MFMA(S, I, J) "v_mfma_f32_16x16x32_bf16 %[c" #I #J "], %[" #S "w" #I "], %[" #S "x" #J "], %[c" #I #J "]\n"
#define P16_ROW(S, I, E0, E1, E2, E3, E4, E5, E6, E7)                                                        \
    P16_MFMA(S, I, 0) E0 P16_MFMA(S, I, 1) E1 P16_MFMA(S, I, 2) E2 P16_MFMA(S, I, 3) E3                        \
    P16_MFMA(S, I, 4) E4 P16_MFMA(S, I, 5) E5 P16_MFMA(S, I, 6) E6 P16_MFMA(S, I, 7) E7
// Fragment reads of substep KS (0, 1) from stage ST into set T: W block F
// (16 rows) at base pwKS + 2048 F, X block F at pxKS + 2048 F.
#define P16_RW(T, F, KS, ST) "ds_read_b128 %[" #T "w" #F "], %[pw" #KS "] offset:32768*" #ST "+2048*" #F "\n"
#define P16_RX(T, F, KS, ST) "ds_read_b128 %[" #T "x" #F "], %[px" #KS "] offset:32768*" #ST "+2048*" #F "\n"
// A substep of set S; rows 0..3 read the 16 fragments of substep KS / stage
// ST into set T at their even slots; L0..L15 go to the odd slots 1 and 5 of
// rows 0..7.
#define P16_SUB(S, T, KS, ST, L0, L1, L2, L3, L4, L5, L6, L7, L8, L9, L10, L11, L12, L13, L14, L15)            \
    P16_ROW(S, 0, P16_RW(T, 0, KS, ST), L0, P16_RW(T, 1, KS, ST), "", P16_RW(T, 2, KS, ST), L1,                \
            P16_RW(T, 3, KS, ST), "")                                                                        \
    P16_ROW(S, 1, P16_RW(T, 4, KS, ST), L2, P16_RW(T, 5, KS, ST), "", P16_RW(T, 6, KS, ST), L3,                \
            P16_RW(T, 7, KS, ST), "")                                                                        \
    P16_ROW(S, 2, P16_RX(T, 0, KS, ST), L4, P16_RX(T, 1, KS, ST), "", P16_RX(T, 2, KS, ST), L5,                \
            P16_RX(T, 3, KS, ST), "")                                                                        \
    P16_ROW(S, 3, P16_RX(T, 4, KS, ST), L6, P16_RX(T, 5, KS, ST), "", P16_RX(T, 6, KS, ST), L7,                \
            P16_RX(T, 7, KS, ST), "")                                                                        \
    P16_ROW(S, 4, "", L8, "", "", "", L9, "", "")                                                             \
    P16_ROW(S, 5, "", L10, "", "", "", L11, "", "")                                                           \
    P16_ROW(S, 6, "", L12, "", "", "", L13, "", "")                                                           \
    P16_ROW(S, 7, "", L14, "", "", "", L15, "", "")
#define P16_SUB_EXP(...) P16_SUB(__VA_ARGS__)
#define P16_NONE "", "", "", "", "", "", "", "", "", "", "", "", "", "", "", ""
// One K tile in stage ST: substep 0 (set a) reads substep 1 of this tile
// into set b; the barrier; substep 1 (set b) reads substep 0 of the next tile
// (stage OT) into set a and loads the tile two ahead into ST.
#define P16_TILE(ST, OT)                                                                                      \
    P16_SUB_EXP(a, b, 1, ST, P16_NONE)                                                                        \
    "s_waitcnt vmcnt(0) lgkmcnt(0)\n"                                                                         \
    "s_barrier\n"                                                                                             \
    "s_min_u32 %[kc], %[kn], %[kmax]\n"                                                                       \
    "s_add_u32 %[kn], %[kn], 128\n"                                                                           \
    P16_SUB_EXP(b, a, 0, OT, PIPE_X8(ST), PIPE_W8(ST))                                                        \
    "s_waitcnt lgkmcnt(0)\n"

#define P16_ACC8(I) [c##I##0] "+a"(c[I][0]), [c##I##1] "+a"(c[I][1]), [c##I##2] "+a"(c[I][2]),               \
    [c##I##3] "+a"(c[I][3]), [c##I##4] "+a"(c[I][4]), [c##I##5] "+a"(c[I][5]), [c##I##6] "+a"(c[I][6]),      \
    [c##I##7] "+a"(c[I][7])
#define P16_SET(S) [S##w0] "=&v"(S##f[0]), [S##w1] "=&v"(S##f[1]), [S##w2] "=&v"(S##f[2]),                    \
    [S##w3] "=&v"(S##f[3]), [S##w4] "=&v"(S##f[4]), [S##w5] "=&v"(S##f[5]), [S##w6] "=&v"(S##f[6]),          \
    [S##w7] "=&v"(S##f[7]), [S##x0] "=&v"(S##f[8]), [S##x1] "=&v"(S##f[9]), [S##x2] "=&v"(S##f[10]),          \
    [S##x3] "=&v"(S##f[11]), [S##x4] "=&v"(S##f[12]), [S##x5] "=&v"(S##f[13]), [S##x6] "=&v"(S##f[14]),      \
    [S##x7] "=&v"(S##f[15])

template <int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_pipe(GemmArgs a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const unsigned tid = threadIdx.x, lane = tid % 64, n16 = lane % 16, q4 = lane / 16;
    const unsigned wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const unsigned wm = wave / 2, wn = wave % 2;
    const unsigned tiles_m = (a.m + TM - 1) / TM, tiles_n = a.n / TN;
    const unsigned pid = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned band = pid / (PIPE_GROUP_M * tiles_n), first_m = band * PIPE_GROUP_M;
    const unsigned rows_in_band = min(tiles_m - first_m, (unsigned)PIPE_GROUP_M);
    const unsigned tm = first_m + (pid % (PIPE_GROUP_M * tiles_n)) % rows_in_band;
    const unsigned tn = (pid % (PIPE_GROUP_M * tiles_n)) / rows_in_band;
    const unsigned m0 = __builtin_amdgcn_readfirstlane(tm * TM), n0 = __builtin_amdgcn_readfirstlane(tn * TN);
    const unsigned ksteps = a.k / TK;

    const uint64_t xbase = (uint64_t)(a.x + (size_t)m0 * a.k);
    const uint64_t wbase = (uint64_t)((const uint16_t *)a.w + (size_t)n0 * a.k);
    const unsigned xrows = min(a.m - m0, (unsigned)TM);
    const i32x4 sx = {(int)__builtin_amdgcn_readfirstlane((unsigned)xbase),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)(xbase >> 32)),
                      (int)__builtin_amdgcn_readfirstlane(xrows * a.k * 2), 0x00020000};
    const i32x4 sw = {(int)__builtin_amdgcn_readfirstlane((unsigned)wbase),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)(wbase >> 32)),
                      (int)__builtin_amdgcn_readfirstlane(TN * a.k * 2), 0x00020000};
    const unsigned lrow = 8 * wave + lane / 8;
    // X and W tiles share the lane offsets: row lrow + 32 t, swizzled chunk.
    unsigned o[8];
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] = (lrow + 32 * t) * a.k * 2 + swz(lrow, lane % 8) * 16;
    const unsigned mb = __builtin_amdgcn_readfirstlane(wave * 1024);
    unsigned kn = 2 * TK * 2, kc = 0;
    const unsigned kmax = __builtin_amdgcn_readfirstlane((ksteps - 1) * TK * 2);
    unsigned pairs = __builtin_amdgcn_readfirstlane(ksteps / 2);
    // Fragment bases of substep ks (32 K) in stage 0: row n16 of the wave's
    // 128-row half, logical chunk 4 ks + q4.
    unsigned pw[2], px[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const unsigned part = n16 * ROW_BYTES + swz(n16, 4 * ks + q4) * 16;
        pw[ks] = 2 * TILE_BYTES + wn * 128 * ROW_BYTES + part;
        px[ks] = wm * 128 * ROW_BYTES + part;
    }
    f32x4 c[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) c[i][j] = f32x4{};
    bf16x8 af[16], bf[16];
    // Prologue: tiles 0 and 1 into stages 0 and 1, substep 0 of tile 0 into
    // set a. Then the tiles in stage pairs; the last pair's loads are clamped
    // reloads of the last tile into a stage nobody reads again, and its
    // closing reads land in registers nobody uses.
    asm volatile(
        "s_mov_b32 %[kc], 0\n" PIPE_LOADS_X(0) PIPE_LOADS_W(0)
        "s_mov_b32 %[kc], 128\n" PIPE_LOADS_X(1) PIPE_LOADS_W(1)
        "s_waitcnt vmcnt(0)\n"
        "s_barrier\n"
        P16_RW(a, 0, 0, 0) P16_RW(a, 1, 0, 0) P16_RW(a, 2, 0, 0) P16_RW(a, 3, 0, 0)
        P16_RW(a, 4, 0, 0) P16_RW(a, 5, 0, 0) P16_RW(a, 6, 0, 0) P16_RW(a, 7, 0, 0)
        P16_RX(a, 0, 0, 0) P16_RX(a, 1, 0, 0) P16_RX(a, 2, 0, 0) P16_RX(a, 3, 0, 0)
        P16_RX(a, 4, 0, 0) P16_RX(a, 5, 0, 0) P16_RX(a, 6, 0, 0) P16_RX(a, 7, 0, 0)
        "s_waitcnt lgkmcnt(0)\n"
        "p16_loop_%=:\n"
        P16_TILE(0, 1)
        P16_TILE(1, 0)
        "s_sub_u32 %[pairs], %[pairs], 1\n"
        "s_cmp_lg_u32 %[pairs], 0\n"
        "s_cbranch_scc1 p16_loop_%=\n"
        "s_waitcnt vmcnt(0) lgkmcnt(0)\n"
        // The last MFMAs' results are complete before the epilogue reads the
        // accumulators (hipcc does not see the MFMAs inside this block).
        "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"
        : P16_ACC8(0), P16_ACC8(1), P16_ACC8(2), P16_ACC8(3), P16_ACC8(4), P16_ACC8(5), P16_ACC8(6), P16_ACC8(7),
          P16_SET(a), P16_SET(b),
          [kc] "+s"(kc), [kn] "+s"(kn), [pairs] "+s"(pairs)
        : [sx] "s"(sx), [sw] "s"(sw), [o0] "v"(o[0]), [o1] "v"(o[1]), [o2] "v"(o[2]), [o3] "v"(o[3]),
          [o4] "v"(o[4]), [o5] "v"(o[5]), [o6] "v"(o[6]), [o7] "v"(o[7]), [mb] "s"(mb), [kmax] "s"(kmax),
          [pw0] "v"(pw[0]), [pw1] "v"(pw[1]), [px0] "v"(px[0]), [px1] "v"(px[1])
        : "m0", "scc", "memory");

    // Block (i, j): lane holds output row m0 + wm*128 + j*16 + n16 and columns
    // n0 + wn*128 + i*16 + 4*q4 + 0..3. Blocks i and i + 1 go out together
    // as 16-byte stores: v_permlane16_swap hands the odd lane rows' block-i
    // values to the even rows and the even rows' block-(i+1) values to the
    // odd rows, so each lane holds eight consecutive columns.
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const unsigned row = m0 + wm * 128 + j * 16 + n16;
        if (row >= a.m) continue;
        uint16_t *dst = a.y + (size_t)row * a.n;
#pragma unroll
        for (int ip = 0; ip < 4; ip++) {
            unsigned w[2][2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int i = 2 * ip + h;
                const unsigned col = n0 + wn * 128 + i * 16 + 4 * q4;
                u16x4 out;
                u16x4 bias4 = {};
                if constexpr (EPI & 1) bias4 = *reinterpret_cast<const u16x4 *>(a.bias + col);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x = c[i][j][e];
                    if constexpr (EPI & 4) x *= a.alpha[0];
                    if constexpr (EPI & 1) x += bf16_to_f32(bias4[e]);
                    uint16_t b = f32_to_bf16(x);
                    if constexpr (EPI & 2) b = f32_to_bf16(gelu_tanh(bf16_to_f32(b)));
                    out[e] = b;
                }
                w[h][0] = out[0] | ((unsigned)out[1] << 16);
                w[h][1] = out[2] | ((unsigned)out[3] << 16);
            }
            const auto s0 = __builtin_amdgcn_permlane16_swap(w[0][0], w[1][0], false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(w[0][1], w[1][1], false, false);
            const unsigned col = n0 + wn * 128 + 2 * ip * 16 + ((q4 & 1) ? 16 + 4 * (q4 - 1) : 4 * q4);
            u32x4 v = {s0[0], s1[0], s0[1], s1[1]};
            *reinterpret_cast<u32x4 *>(dst + col) = v;
        }
    }
}
template <int EPI>
int launch_pipe(h3_gpu *g, const GemmArgs &a, bool timed = true) {
    constexpr size_t shared = PIPE_LDS;
    static bool configured = false;
    auto kernel = gemm_bf16_pipe<EPI>;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)shared), "GEMM shared memory"))
            return 0;
        configured = true;
    }
    unsigned tiles = (a.m + TM - 1) / TM * (a.n / TN);
    hipEvent_t timing = timed ? h3_kernel_timing_begin(g) : nullptr;
    hipLaunchKernelGGL(kernel, dim3(tiles), dim3(256), shared, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "BF16 GEMM");
}

bool pipe_fits(const GemmArgs &a) {
    return a.n % TN == 0 && a.k % (2 * TK) == 0 && a.m >= 32 && (size_t)a.m * a.k * 2 < (1ull << 31) &&
           (size_t)a.n * a.k * 2 < (1ull << 31);
}
int launch_pipe_epi(h3_gpu *g, const GemmArgs &a, int epi, bool timed = true) {
    switch (epi) {
    case 0: return launch_pipe<0>(g, a, timed);
    case 1: return launch_pipe<1>(g, a, timed);
    case 2: return launch_pipe<2>(g, a, timed);
    case 3: return launch_pipe<3>(g, a, timed);
    default: return launch_pipe<4>(g, a, timed);
    }
}

// W8A16 weights -> BF16 values w = bf16(code * scale[row, k / group]), the
// reconstruction of gemm_kernel and of the reference's Metal kernel
// (shaders.metal:825-827), written once per projection call for
// gemm_bf16_pipe. HBM-bound: each thread reads 16 codes (one 16-byte load)
// and writes 32 bytes. group is a multiple of 16, so one scale covers them.
__global__ __launch_bounds__(256) void q8_dequant_bf16(const int8_t *codes, const float *scales, uint16_t *out,
                                                     unsigned k, unsigned group, unsigned groups, size_t chunks) {
    const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const size_t first = c * 16;
    const unsigned row = (unsigned)(first / k), col = (unsigned)(first % k);
    const float s = scales[(size_t)row * groups + col / group];
    const i32x4 q = *reinterpret_cast<const i32x4 *>(codes + first);
    bf16x8 half[2];
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
        const int word = q[e / 4];
        f32x2 f = {(float)(int8_t)(word >> (8 * (e % 4))) * s, (float)(int8_t)(word >> (8 * (e % 4 + 1))) * s};
        bf16x2 b = __builtin_convertvector(f, bf16x2);
        half[e / 8][e % 8] = b[0];
        half[e / 8][e % 8 + 1] = b[1];
    }
    *reinterpret_cast<bf16x8 *>(out + first) = half[0];
    *reinterpret_cast<bf16x8 *>(out + first + 8) = half[1];
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
    if (pipe_fits(a) && g->gemm_variant != 3) return launch_pipe<4>(g, a);
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
    const int epi = (bias ? 1 : 0) | (gelu ? 2 : 0);
    // Variant 3 keeps the earlier kernels (gemm_q8_staged, gemm_kernel) for A/B.
    const bool pipe = tiled && pipe_fits(a) && g->gemm_variant != 3;
    if (pipe && !w->q8) {
        ok = launch_pipe_epi(g, a, epi);
    } else if (pipe) {
        // W8A16: a dequantization pass into the context's BF16 weight buffer
        // (HBM-bound, ~1% of the GEMM at M = 32400), then the BF16 GEMM on it;
        // both inside one kernel-timing window.
        const size_t bytes = (size_t)n * k * 2;
        if (g->gemm_weights_bytes < bytes) {
            // An earlier projection may still read the old buffer.
            if (g->gemm_weights && !h3_hip_check(g, hipStreamSynchronize(g->compute), "GEMM weight buffer")) return 0;
            if (g->gemm_weights) hipFree(g->gemm_weights);
            g->gemm_weights = nullptr;
            g->gemm_weights_bytes = 0;
            if (!h3_hip_check(g, hipMalloc(&g->gemm_weights, bytes), "GEMM weight buffer")) {
                g->gemm_weights = nullptr;
                return 0;
            }
            g->gemm_weights_bytes = bytes;
        }
        const size_t chunks = (size_t)n * k / 16;
        hipEvent_t timing = h3_kernel_timing_begin(g);
        hipLaunchKernelGGL(q8_dequant_bf16, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, g->compute,
                           (const int8_t *)w->data, w->q8_scales, (uint16_t *)g->gemm_weights, k, a.group, a.groups,
                           chunks);
        GemmArgs b = a;
        b.w = g->gemm_weights;
        ok = h3_launch_status(g, "W8A16 dequantization") && launch_pipe_epi(g, b, epi, false);
        h3_kernel_timing_end(g, timing);
    } else if (tiled) {
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
