// delta_rule.hip - chunked gated delta rule (Gated DeltaNet recurrence) for gfx950.
//
// Computes exactly the reference's per-token recurrence (crates/huncho-backend/src/
// delta_cpu.rs:95-131, == qwen3_5.rs:950-987): for each token t of a sequence and head,
//   S <- S * exp(g_t);  m = S^T k_t;  delta_t = (v_t - m) * beta_t;  S <- S + k_t delta_t^T;
//   o_t = S^T q_t
// with S [dk, dv] fp32, in the algebraically equal chunked form (chunk C = 64). With
// G_t = sum_{s<=t} g_s inside a chunk and S0 the state entering it:
//   A[t,s]   = beta_t exp(G_t - G_s) (k_t . k_s)        s < t   (strictly lower)
//   T        = (I + A)^-1                              (forward substitution, fp32)
//   delta    = T [ beta * (V - exp(G) * (K S0)) ]
//   O        = exp(G) * (Q S0) + Aqk delta,  Aqk[t,s] = exp(G_t - G_s) (q_t . k_s), s <= t
//   S_next   = exp(G_last) S0 + K^T [exp(G_last - G) * delta]
// Only decay ratios exp(G_t - G_s) with t >= s (each <= 1) are formed.
//
// One workgroup = one (sequence, head); 4 waves; wave w owns value columns 32w..32w+31 of
// the state, held as four 32x32 MFMA accumulators for the whole sequence, so the state
// never leaves registers between chunks and is read/written in HBM only at the start (an
// optional initial state) and the end (the optional final state). Every intermediate
// (K S, R, delta) stays in accumulator layout and feeds the next MFMA as its B operand:
// the reduction index of each product is permuted to match the accumulator's row order
// instead of transposing the data. Inputs stream from HBM once: q, k, v, g, beta in, o out.
//
// This file holds the fp32 variant (v_mfma_f32_32x32x2_f32, the fp32 model path); the 16-bit
// variants and the fused Gated DeltaNet layer kernel live in gdn16_kernel.hpp.
#include "common.hpp"
#include "kernel_args.hpp"

namespace hk {

constexpr int CH = 64;
constexpr int DK = 128;
constexpr int DV = 128;

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ float wave_incl_scan(float x, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        float y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

// 16x16 fp32 tiles on v_mfma_f32_16x16x4_f32: operand lane l holds row/column l % 16 and
// reduction index l / 16; accumulator lane l holds column l % 16, rows (l / 16) * 4 + j.
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// D = X[16][K] . Y[K][16] from fp32 LDS tiles (K a multiple of 4).
__device__ __forceinline__ f32x4 tile16_mm(const float* X, int ldx, const float* Y, int ldy, int K, int lane) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, kq = lane >> 4;
    for (int k = 0; k < K; k += 4) acc = mfma16(X[r * ldx + k + kq], Y[(k + kq) * ldy + r], acc);
    return acc;
}

// D = -W[16][16] . Xacc where Xacc is a 16x16 accumulator tile: the reduction index of
// step j is paired with the accumulator row 4 * (l / 16) + j the lane already holds.
__device__ __forceinline__ f32x4 tile16_neg_mm_acc(const float* W, int ldw, f32x4 xacc, int lane) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = mfma16(-W[r * ldw + 4 * kq + j], xacc[j], acc);
    return acc;
}

__device__ __forceinline__ void tile16_store(float* D, int ldd, f32x4 acc, int lane) {
    const int c = lane & 15, r0 = (lane >> 4) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) D[(r0 + j) * ldd + c] = acc[j];
}

// T = (I + A)^-1 for strictly lower A [64][lda] (fp32, LDS), all 4 waves, blocked:
//   1. wave w inverts the unit-lower diagonal block w (16x16) by forward substitution;
//   2. T[1][0] = -T11 A10 T00 and T[3][2] = -T33 A32 T22 (16 -> 32);
//   3. T[2:4][0:2] = -T[2:4][2:4] A[2:4][0:2] T[0:2][0:2] (32 -> 64), one 16x16 tile per wave.
// T is written to Tf [64][lda] with its upper triangle zeroed; Xs is a [32][ldx] scratch.
// Contains __syncthreads(): every thread of the workgroup must call it.
__device__ void invert_unit_lower(const float* Am, float* Tf, int lda, float* Xs, int ldx, int wave, int lane) {
    {
        const int b = wave * 16;
        if (lane < 16) {
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float acc = (i == lane) ? 1.0f : 0.0f;
                const float* row = Am + (b + i) * lda + b;
#pragma unroll
                for (int k = 0; k < i; ++k) acc -= row[k] * x[k];
                x[i] = acc;
                Tf[(b + i) * lda + b + lane] = acc;
            }
        }
        // zero the blocks right of the diagonal in this block row
        for (int idx = lane; idx < 16 * (48 - b); idx += 64) {
            const int i = idx / (48 - b), j = idx % (48 - b);
            Tf[(b + i) * lda + b + 16 + j] = 0.0f;
        }
    }
    __syncthreads();
    if (wave < 2) {
        const int b = wave * 32;  // diagonal 32-block: [b, b+32)
        f32x4 x = tile16_mm(Am + (b + 16) * lda + b, lda, Tf + b * lda + b, lda, 16, lane);
        f32x4 t = tile16_neg_mm_acc(Tf + (b + 16) * lda + b + 16, lda, x, lane);
        tile16_store(Tf + (b + 16) * lda + b, lda, t, lane);
    }
    __syncthreads();
    {
        const int rt = wave >> 1, ct = wave & 1;
        f32x4 x = tile16_mm(Am + (32 + 16 * rt) * lda, lda, Tf + 16 * ct, lda, 32, lane);
        tile16_store(Xs + 16 * rt * ldx + 16 * ct, ldx, x, lane);
    }
    __syncthreads();
    {
        const int rt = wave >> 1, ct = wave & 1;
        f32x4 t = tile16_mm(Tf + (32 + 16 * rt) * lda + 32, lda, Xs + 16 * ct, ldx, 32, lane);
        t = -t;
        tile16_store(Tf + (32 + 16 * rt) * lda + 16 * ct, lda, t, lane);
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// fp32 variant
// ---------------------------------------------------------------------------
constexpr int F_KSTR = DK + 4;  // fp32 row stride of Kc/Qc
constexpr int F_ASTR = CH + 4;  // fp32 row stride of A/T and Aqk
constexpr int XSTR = 32 + 4;    // fp32 row stride of the inversion scratch
constexpr size_t GDN_F32_LDS = sizeof(float) * (2 * CH * F_KSTR + 3 * CH * F_ASTR + 32 * XSTR + 2 * CH);

__global__ __launch_bounds__(256, 1) void gdn_chunk_f32(GdnArgs a) {
    extern __shared__ __attribute__((aligned(16))) float smem_f[];
    float* Kc = smem_f;
    float* Qc = Kc + CH * F_KSTR;
    float* Am = Qc + CH * F_KSTR;
    float* Aq = Am + CH * F_ASTR;
    float* Tf = Aq + CH * F_ASTR;
    float* Xs = Tf + CH * F_ASTR;
    float* Gs = Xs + 32 * XSTR;
    float* Bs = Gs + CH;

    const int h = blockIdx.x, seq = blockIdx.y, H = a.H;
    const int t0 = a.cu_seqlens[seq];
    const int T = a.cu_seqlens[seq + 1] - t0;
    if (t0 < 0 || T < 0 || t0 + T > a.n_tokens) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, col = lane & 31;
    const int dvc = wave * 32 + col;  // this lane's value column
    const int kh = h / a.qk_rep;
    const float* qg = (const float*)a.q + (long)kh * DK;
    const float* kg = (const float*)a.k + (long)kh * DK;
    const float* vg = (const float*)a.v + (long)h * DV;
    float* og = (float*)a.o + (long)h * DV;
    // this sequence's state rows [H][dk][dv] (per-row pointer tables or contiguous arrays)
    const float* const s0 = a.init_rows ? a.init_rows[seq]
                                        : (a.initial_state ? a.initial_state + (long)seq * H * DK * DV : nullptr);
    float* const s1 = a.final_rows ? a.final_rows[seq]
                                   : (a.final_state ? a.final_state + (long)seq * H * DK * DV : nullptr);
    const long sbase = (long)h * DK * DV;

    f32x16 S[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int j = 0; j < 16; ++j)
            S[rb][j] = s0 ? s0[sbase + (long)(rb * 32 + acc_row(j, g)) * DV + dvc] : 0.0f;

    for (int c0 = 0; c0 < T; c0 += CH) {
        const int Lc = min(CH, T - c0);
        __syncthreads();
        // q, k chunk -> LDS (zero rows past the end); g, beta -> registers of wave 0
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int idx = tid + 256 * i, r = idx >> 5, c4 = (idx & 31) * 4;
            f32x4 qv = {0.f, 0.f, 0.f, 0.f}, kv = {0.f, 0.f, 0.f, 0.f};
            if (r < Lc) {
                qv = *(const f32x4*)(qg + (long)(t0 + c0 + r) * a.q_tok + c4);
                kv = *(const f32x4*)(kg + (long)(t0 + c0 + r) * a.k_tok + c4);
            }
            *(f32x4*)(Qc + r * F_KSTR + c4) = qv;
            *(f32x4*)(Kc + r * F_KSTR + c4) = kv;
        }
        if (wave == 0) {
            float gv = 0.f, bv = 0.f;
            if (lane < Lc) {
                gv = a.g[(long)(t0 + c0 + lane) * a.gb_tok + h];
                bv = a.beta[(long)(t0 + c0 + lane) * a.gb_tok + h];
            }
            Gs[lane] = wave_incl_scan(gv, lane);
            Bs[lane] = bv;
        }
        __syncthreads();
        // A (strictly lower, beta and decay folded in) and Aqk (lower incl. diagonal)
        if (wave < 3) {
            const int tb = wave == 0 ? 0 : 1, sb = wave == 2 ? 1 : 0;
            f32x16 kk = f32x16{}, qk = f32x16{};
            const float* ka = Kc + (tb * 32 + col) * F_KSTR + 2 * g;
            const float* qa = Qc + (tb * 32 + col) * F_KSTR + 2 * g;
            const float* kbp = Kc + (sb * 32 + col) * F_KSTR + 2 * g;
#pragma unroll 8
            for (int u = 0; u < 32; ++u) {
                f32x2 av = *(const f32x2*)(ka + 4 * u);
                f32x2 qv = *(const f32x2*)(qa + 4 * u);
                f32x2 bv = *(const f32x2*)(kbp + 4 * u);
                kk = mfma_f32(av[0], bv[0], kk);
                kk = mfma_f32(av[1], bv[1], kk);
                qk = mfma_f32(qv[0], bv[0], qk);
                qk = mfma_f32(qv[1], bv[1], qk);
            }
            const int s = sb * 32 + col;
            const float Gs_s = Gs[s];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = tb * 32 + acc_row(j, g);
                const float dec = s <= t ? __expf(Gs[t] - Gs_s) : 0.0f;
                Am[t * F_ASTR + s] = s < t ? Bs[t] * dec * kk[j] : 0.0f;
                Aq[t * F_ASTR + s] = s <= t ? dec * qk[j] : 0.0f;
            }
        } else {
            for (int idx = lane; idx < 32 * 32; idx += 64) {
                const int t = idx >> 5, s = 32 + (idx & 31);
                Am[t * F_ASTR + s] = 0.0f;
                Aq[t * F_ASTR + s] = 0.0f;
            }
        }
        __syncthreads();
        invert_unit_lower(Am, Tf, F_ASTR, Xs, XSTR, wave, lane);
        // K S0 and Q S0 for this wave's value columns
        f32x16 ks[2], qs[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            ks[tb] = f32x16{};
            qs[tb] = f32x16{};
            const float* kr = Kc + (tb * 32 + col) * F_KSTR + g * 4;
            const float* qr = Qc + (tb * 32 + col) * F_KSTR + g * 4;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    f32x4 kv = *(const f32x4*)(kr + rb * 32 + jj * 8);
                    f32x4 qv = *(const f32x4*)(qr + rb * 32 + jj * 8);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ks[tb] = mfma_f32(kv[e], S[rb][jj * 4 + e], ks[tb]);
                        qs[tb] = mfma_f32(qv[e], S[rb][jj * 4 + e], qs[tb]);
                    }
                }
        }
        // R = beta * (V - exp(G) K S0); O starts as exp(G) Q S0
        f32x16 R[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = tb * 32 + acc_row(j, g);
                const float eg = __expf(Gs[t]);
                const float vv = t < Lc ? vg[(long)(t0 + c0 + t) * a.v_tok + dvc] : 0.0f;
                R[tb][j] = Bs[t] * (vv - eg * ks[tb][j]);
                qs[tb][j] *= eg;
            }
        // delta = T R
        f32x16 dl[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            dl[tb] = f32x16{};
            const float* tr = Tf + (tb * 32 + col) * F_ASTR + g * 4;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    f32x4 tv = *(const f32x4*)(tr + sb * 32 + jj * 8);
#pragma unroll
                    for (int e = 0; e < 4; ++e) dl[tb] = mfma_f32(tv[e], R[sb][jj * 4 + e], dl[tb]);
                }
        }
        // O = exp(G) Q S0 + Aqk delta -> HBM
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const float* ar = Aq + (tb * 32 + col) * F_ASTR + g * 4;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    f32x4 av = *(const f32x4*)(ar + sb * 32 + jj * 8);
#pragma unroll
                    for (int e = 0; e < 4; ++e) qs[tb] = mfma_f32(av[e], dl[sb][jj * 4 + e], qs[tb]);
                }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = tb * 32 + acc_row(j, g);
                if (t < Lc) og[(long)(t0 + c0 + t) * a.o_tok + dvc] = qs[tb][j];
            }
        }
        // S = exp(G_last) S + K^T (exp(G_last - G) delta)
        const float glast = Gs[CH - 1];
        const float eglast = __expf(glast);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 16; ++j) dl[tb][j] *= __expf(glast - Gs[tb * 32 + acc_row(j, g)]);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
            for (int j = 0; j < 16; ++j) S[rb][j] *= eglast;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    S[rb] = mfma_f32(Kc[(tb * 32 + acc_row(j, g)) * F_KSTR + rb * 32 + col], dl[tb][j], S[rb]);
        }
    }
    if (s1) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int j = 0; j < 16; ++j) s1[sbase + (long)(rb * 32 + acc_row(j, g)) * DV + dvc] = S[rb][j];
    }
}

}  // namespace hk

extern "C" int hk_launch_gated_delta_chunked(int dtype, const hk::GdnArgs* args, int n_seqs, hipStream_t stream) {
    if (dtype != hk::DT_F32) return hk_launch_gdn16(dtype, 0, args, nullptr, n_seqs, stream);
    dim3 grid(args->H, n_seqs);
    // set once, under C++'s thread-safe static initialisation (replicas launch from several threads)
    static const bool configured = hipFuncSetAttribute((const void*)hk::gdn_chunk_f32,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)hk::GDN_F32_LDS) == hipSuccess;
    if (!configured) return HK_ERR_DEVICE;
    hipLaunchKernelGGL(hk::gdn_chunk_f32, grid, dim3(256), hk::GDN_F32_LDS, stream, *args);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}
