// gdn_v2.hip - chunked gated delta rule for 16-bit activations (bf16 / fp16) on gfx950, with
// an optional fused Gated DeltaNet prologue and epilogue.
//
// Recurrence (crates/huncho-backend/src/delta_cpu.rs:95-131, qwen3_5.rs:950-987), per token t:
//   S <- S exp(g_t); delta_t = beta_t (v_t - S^T k_t); S <- S + k_t delta_t^T; o_t = S^T q_t
// evaluated in the equal chunked form (chunk 64, G = inclusive cumsum of g in the chunk):
//   A = strict_lower(beta_t exp(G_t - G_s) k_t.k_s),  T = (I + A)^-1
//   delta = T [beta (V - exp(G) K S0)],  O = exp(G) Q S0 + lower(exp(G_t - G_s) q_t.k_s) delta
//   S1 = exp(G_last) S0 + K^T [exp(G_last - G) delta]
// State S stays in fp32 MFMA accumulators for the whole sequence (wave w owns value columns
// 32w..32w+31); products use 16-bit operands with fp32 accumulation; T is formed in fp32.
//
// Two modes (template FUSED):
//   standalone  q, k [tokens][k_heads][128], v [tokens][heads][128], g, beta fp32 -> o
//   fused       the Gated DeltaNet layer body of LinearAttn::forward (qwen3_5.rs:846-940)
//               straight from the fused in_proj output rows [q | k | v | z | b | a]:
//               causal depthwise conv (K = 4, ascending taps, conv_cpu.rs:34-48) + SiLU,
//               l2norm of q and k, q * 128^-1/2, beta = sigmoid(b),
//               g = -exp(A_log) softplus(a + dt_bias), the recurrence, then the gated
//               RMSNorm rms(o) * w * silu(z) (193-201) -> out_proj input
// so one kernel streams each layer's q|k|v|z|b|a once and writes one output row per token.
//
// Chunk pipeline, one workgroup (4 waves) per (sequence, value head), two workgroups per CU
// (78 KB of LDS, <= 256 registers per lane) so one workgroup's VALU prologue overlaps the
// other's MFMA phases:
//   P0  global -> LDS: q, v rows (padded) and k rows (swizzled) (fused: waves 0-2 run the
//       conv for q, k, v); wave 3: g scan and beta
//   P1  waves 0-2: K K^T and Q K^T blocks -> A (fp32) and Aqk; wave 3 zeroes the upper
//       blocks; every wave: K S0, Q S0 for its columns -> R and exp(G) Q S0 in registers
//   P2  in-place blocked inverse of I + A (four 16x16 diagonal solves, two merges; the
//       merge scratch lives in V's buffer, which is dead by then)
//   P3  delta = T R, O = exp(G) Q S0 + Aqk delta (staged in LDS), S update with the K^T
//       operand read through transposing LDS reads
//   P4  O (or the gated-normed O) -> HBM with 16-byte stores
#include "common.hpp"
#include "kernel_args.hpp"

namespace hk {
namespace gdn2 {

template <typename T> using Ops = Mma16<T>;

template <typename T> __device__ __forceinline__ float f(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ float rnd(float x) { return (float)(T)x; }

constexpr int CH = 64, DK = 128, DV = 128;
constexpr int RS = DK + 8;  // row stride (elements) of Qc / Vc / O staging
constexpr int TS = CH + 8;  // row stride of Aq [64][72]
constexpr int AS = CH + 4;  // fp32 row stride of A / T [64][68]
constexpr int XS = 32 + 4;  // fp32 row stride of the merge scratch [32][36] (in V's buffer)
// Qc, Vc padded; Kc [64][128] unpadded with an XOR chunk swizzle; A; Aq; g scan; beta:
// 78,336 B, so two workgroups share a CU (160 KiB of LDS)
constexpr size_t LDS_BYTES = 2 * CH * RS * 2 + CH * DK * 2 + CH * AS * 4 + CH * TS * 2 + 2 * CH * 4;

// K rows: 16-byte chunk c of row r sits at chunk c ^ kswz(r). Row writes, the row-major
// operand reads of K K^T / Q K^T, the permuted reads of K S and the transposing reads of
// the K^T operand of the state update all reach every LDS bank evenly with this swizzle.
__device__ __forceinline__ int kswz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ float silu(float x) { return fast_silu(x); }

__device__ __forceinline__ float wave_incl_scan(float x, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        float y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

// ---- 16x16 fp32 tiles on v_mfma_f32_16x16x4_f32 (operand lane l: row/col l % 16, reduction
// index l / 16; accumulator lane l: column l % 16, rows 4 (l / 16) + j) ----
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
template <int K>
__device__ __forceinline__ f32x4 tile_mm(const float* X, int ldx, const float* Y, int ldy, int lane) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int k = 0; k < K; k += 4) acc = mfma16(X[r * ldx + k + kq], Y[(k + kq) * ldy + r], acc);
    return acc;
}
// -W[16][16] . Xacc, pairing reduction step j with the accumulator row 4 (l / 16) + j
__device__ __forceinline__ f32x4 tile_neg_mm_acc(const float* W, int ldw, f32x4 xacc, int lane) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = mfma16(-W[r * ldw + 4 * kq + j], xacc[j], acc);
    return acc;
}
__device__ __forceinline__ void tile_store(float* D, int ldd, f32x4 acc, int lane) {
    const int c = lane & 15, r0 = (lane >> 4) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) D[(r0 + j) * ldd + c] = acc[j];
}

// In-place T = (I + A)^-1 for strictly lower A [64][AS] whose upper triangle is zero.
// Diagonal 16x16 blocks by forward substitution (wave w: block w, lane j: column j), then T10 = -T11 A10 T00 and T32 = -T33 A32 T22, then
// T[2:4][0:2] = -T[2:4][2:4] (A[2:4][0:2] T[0:2][0:2]). Every thread must call it.
__device__ void invert_in_place(float* Am, float* Xs, int wave, int lane) {
    {
        const int b = wave * 16, j = lane & 15;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float* row = Am + (b + i) * AS + b;
            float a0 = (i == j) ? 1.0f : 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
            for (int k = 0; k + 3 < i; k += 4) {
                f32x4 rv = *(const f32x4*)(row + k);
                a0 -= rv[0] * x[k];
                a1 -= rv[1] * x[k + 1];
                a2 -= rv[2] * x[k + 2];
                a3 -= rv[3] * x[k + 3];
            }
#pragma unroll
            for (int k = i & ~3; k < i; ++k) a0 -= row[k] * x[k];
            x[i] = (a0 + a1) + (a2 + a3);
        }
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 16; ++i) Am[(b + i) * AS + b + j] = x[i];
        }
    }
    __syncthreads();
    if (wave < 2) {
        const int b = wave * 32;
        f32x4 xa = tile_mm<16>(Am + (b + 16) * AS + b, AS, Am + b * AS + b, AS, lane);
        f32x4 t = tile_neg_mm_acc(Am + (b + 16) * AS + b + 16, AS, xa, lane);
        tile_store(Am + (b + 16) * AS + b, AS, t, lane);
    }
    __syncthreads();
    const int rt = wave >> 1, ct = wave & 1;
    {
        f32x4 xa = tile_mm<32>(Am + (32 + 16 * rt) * AS, AS, Am + 16 * ct, AS, lane);
        tile_store(Xs + 16 * rt * XS + 16 * ct, XS, xa, lane);
    }
    __syncthreads();
    {
        f32x4 t = tile_mm<32>(Am + (32 + 16 * rt) * AS + 32, AS, Xs + 16 * ct, XS, lane);
        t = -t;
        tile_store(Am + (32 + 16 * rt) * AS + 16 * ct, AS, t, lane);
    }
    __syncthreads();
}

// 8 operands whose reduction index g*8+i pairs with accumulator rows acc_row(hh*8+i, g) of the
// 32-block at `base`: two runs of four, base+16hh+4g and base+16hh+8+4g.
template <typename T>
__device__ __forceinline__ typename Ops<T>::v8 ld_perm(const T* row, int base, int hh, int g) {
    typedef typename Ops<T>::v4 v4;
    v4 lo = *(const v4*)(row + base + 16 * hh + 4 * g);
    v4 hi = *(const v4*)(row + base + 16 * hh + 8 + 4 * g);
    return typename Ops<T>::v8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// ld_perm for a swizzled K row (row's swizzle key swk): the same elements as ld_perm at base 32 rb
template <typename T>
__device__ __forceinline__ typename Ops<T>::v8 ld_perm_k(const T* row, int swk, int rb, int hh, int g) {
    typedef typename Ops<T>::v4 v4;
    v4 lo = *(const v4*)(row + 8 * ((4 * rb + 2 * hh) ^ swk) + 4 * g);
    v4 hi = *(const v4*)(row + 8 * ((4 * rb + 2 * hh + 1) ^ swk) + 4 * g);
    return typename Ops<T>::v8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
template <typename T>
__device__ __forceinline__ typename Ops<T>::v8 ld_perm_f32(const float* row, int base, int hh, int g) {
    f32x4 lo = *(const f32x4*)(row + base + 16 * hh + 4 * g);
    f32x4 hi = *(const f32x4*)(row + base + 16 * hh + 8 + 4 * g);
    return typename Ops<T>::v8{(T)lo[0], (T)lo[1], (T)lo[2], (T)lo[3], (T)hi[0], (T)hi[1], (T)hi[2], (T)hi[3]};
}
template <typename T>
__device__ __forceinline__ typename Ops<T>::v8 pack(const f32x16& v, int hh) {
    typename Ops<T>::v8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (T)v[hh * 8 + i];
    return r;
}

// Row of accumulator element j minus the lane's 4 g: a compile-time constant, so per-lane
// addresses are one base (holding the 4 g term) plus an instruction immediate.
__device__ __forceinline__ constexpr int arow(int j) { return (j >> 2) * 8 + (j & 3); }

template <typename T, bool FUSED>
__global__ __launch_bounds__(256, 2) void gdn_chunk(GdnArgs a, GdnFusedArgs fa) {
    typedef typename Ops<T>::v8 v8;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    T* Qc = (T*)smem;                       // [64][RS]; later O staging
    T* Vc = Qc + CH * RS;                   // [64][RS]
    T* Kc = Vc + CH * RS;                   // [64][DK], chunks swizzled by kswz
    float* Am = (float*)(Kc + CH * DK);     // [64][AS]: A, then T
    T* Aq = (T*)(Am + CH * AS);             // [64][TS]
    float* Gs = (float*)(Aq + CH * TS);
    float* Bs = Gs + CH;
    float* Xs = (float*)Vc;                 // [32][XS] merge scratch while V is dead (inversion)

    const int h = blockIdx.x, seq = blockIdx.y, H = a.H;
    const int t0 = a.cu_seqlens[seq];
    const int Tn = a.cu_seqlens[seq + 1] - t0;
    if (t0 < 0 || Tn < 0 || t0 + Tn > a.n_tokens) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, col = lane & 31;
    const int dvc = wave * 32 + col;
    const int kh = h / a.qk_rep;
    // this sequence's state rows and conv rows (per-row pointer tables or contiguous arrays)
    const float* const s0 = a.init_rows ? a.init_rows[seq]
                                        : (a.initial_state ? a.initial_state + (long)seq * H * DK * DV : nullptr);
    float* const s1 = a.final_rows ? a.final_rows[seq]
                                   : (a.final_state ? a.final_state + (long)seq * H * DK * DV : nullptr);
    const T* const hist = !FUSED ? nullptr
                          : fa.hist_rows ? (const T*)fa.hist_rows[seq]
                                         : (fa.hist ? (const T*)fa.hist + (long)seq * fa.conv_dim * 3 : nullptr);
    T* const tail = !FUSED ? nullptr
                    : fa.tail_rows ? (T*)fa.tail_rows[seq]
                                   : (fa.tail_out ? (T*)fa.tail_out + (long)seq * fa.conv_dim * 3 : nullptr);
    const long sbase = (long)h * DK * DV;
    // loader mapping (waves 0..2): slice = wave (q, k, v); 8 channels 8*sub..; rows 16*rg..
    const int sub = lane & 15, rg = lane >> 4;

    f32x16 S[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int j = 0; j < 16; ++j)
            S[rb][j] = s0 ? s0[sbase + (long)(4 * g) * DV + dvc + (rb * 32 + arow(j)) * DV] : 0.0f;

    // fused loader: this lane's 8 q channels; k channels follow at + Hk*128, v channels of
    // value head h at + 2 Hk*128 + (h - kh)*128
    const long mcol = (long)kh * 128 + 8 * sub;

    for (int c0 = 0; c0 < Tn; c0 += CH) {
        const int Lc = min(CH, Tn - c0);
        __syncthreads();
        // ---------------- P0: inputs -> LDS ----------------
        if (FUSED && wave < 3) {
            // wave ts (q, k, v) convolves chunk rows 16 rg .. 16 rg + 15 of its tensor, channels
            // 8 sub .. + 7, in two passes of 8 rows, each from an 11-row window of raw conv
            // inputs (sequence positions c0 + row - 3 ..). Positions past the sequence end are
            // loaded clamped: they only reach rows past the end, whose beta is 0 and whose
            // outputs are not stored. Positions before the start are the conv history or 0.
            typedef typename Ops<T>::v2 v2;
            const int ts = wave;
            const long mc = mcol + ts * (long)fa.Hk * 128 + (ts == 2 ? (long)(h - kh) * 128 : 0);
            T* dst = ts == 0 ? Qc : ts == 1 ? Kc : Vc;
            // taps (0, 1) and (2, 3) of each channel as 16-bit pairs (the weights are the model
            // dtype's values, exact in T), re-read per chunk rather than held in registers
            v2 w01[8], w23[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const f32x4 w4 = *(const f32x4*)(fa.conv_w + (mc + e) * 4);
                w01[e] = v2{(T)w4[0], (T)w4[1]};
                w23[e] = v2{(T)w4[2], (T)w4[3]};
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int r0 = 16 * rg + 8 * hf;
                v8 raw[11];
#pragma unroll
                for (int i = 0; i < 11; ++i) {
                    const int p = c0 + r0 - 3 + i;
                    const int pc = p < 0 ? 0 : (p >= Tn ? Tn - 1 : p);
                    raw[i] = *(const v8*)((const T*)fa.mixed + (long)(t0 + pc) * fa.mixed_tok + mc);
                }
                if (c0 + r0 == 0) {  // window starts 3 positions before the sequence
#pragma unroll
                    for (int i = 0; i < 3; ++i)
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            raw[i][e] = hist ? hist[((long)mc + e) * 3 + i] : (T)0.0f;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float y[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float acc = dot2(w23[e], v2{raw[i + 2][e], raw[i + 3][e]},
                                               dot2(w01[e], v2{raw[i][e], raw[i + 1][e]}, 0.0f));
                        y[e] = silu(acc);
                    }
                    if (ts < 2) {  // conv output stored in the activation dtype, then l2norm over
                                   // the head's 128 channels (16 lanes)
                        float ss = 0.0f;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            y[e] = rnd<T>(y[e]);
                            ss += y[e] * y[e];
                        }
                        ss = sum16(ss);
                        const float inv = fast_rsqrt(ss + 1e-6f);
#pragma unroll
                        for (int e = 0; e < 8; ++e) y[e] = ts == 0 ? (y[e] * inv) * fa.scale : y[e] * inv;
                    }
                    const int r = r0 + i;
                    v8 o;
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[e] = (T)y[e];
                    *(v8*)(dst + (ts == 1 ? r * DK + 8 * (sub ^ kswz(r)) : r * RS + 8 * sub)) = o;
                }
            }
        } else if (wave < 3) {
            T* dst = wave == 0 ? Qc : wave == 1 ? Kc : Vc;
            const T* src = wave == 0 ? (const T*)a.q + (long)kh * DK
                         : wave == 1 ? (const T*)a.k + (long)kh * DK : (const T*)a.v + (long)h * DV;
            const long tok = wave == 0 ? a.q_tok : wave == 1 ? a.k_tok : a.v_tok;
            v8 x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 16 * rg + i;
                x[i] = *(const v8*)(src + (long)(t0 + c0 + (r < Lc ? r : Lc - 1)) * tok + 8 * sub);
                if (r >= Lc) x[i] = v8{};
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 16 * rg + i;
                *(v8*)(dst + (wave == 1 ? r * DK + 8 * (sub ^ kswz(r)) : r * RS + 8 * sub)) = x[i];
            }
        }
        if (wave == 3) {  // g (inclusive scan over the chunk) and beta
            float gv = 0.0f, bv = 0.0f;
            if (lane < Lc) {
                const long tt = t0 + c0 + lane;
                if (FUSED) {
                    const T* row = (const T*)fa.ba + tt * fa.ba_tok;
                    const float b = f(row[fa.b_col + h]);
                    const float av = f(row[fa.a_col + h]);
                    bv = rnd<T>(fast_sigmoid(b));
                    gv = fa.base_g[h] * __logf(__expf(av + fa.dt_bias[h]) + 1.0f);
                } else {
                    gv = a.g[tt * a.gb_tok + h];
                    bv = a.beta[tt * a.gb_tok + h];
                }
            }
            Gs[lane] = wave_incl_scan(gv, lane);
            Bs[lane] = bv;
        }
        __syncthreads();
        // ---------------- P1: A, Aqk; K S0, Q S0 ----------------
        if (wave < 3) {
            const int tb = wave == 0 ? 0 : 1, sb = wave == 2 ? 1 : 0;
            f32x16 kk = f32x16{}, qk = f32x16{};
            int swk = kswz(col);  // K rows tb*32 + col and sb*32 + col share it
            asm volatile("" : "+v"(swk));  // recompute the swizzled addresses here, not hoisted and spilled
            const T* ka = Kc + (tb * 32 + col) * DK;
            const T* qa = Qc + (tb * 32 + col) * RS + g * 8;
            const T* kbp = Kc + (sb * 32 + col) * DK;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int ko = 8 * ((2 * ks + g) ^ swk);
                v8 bv = *(const v8*)(kbp + ko);
                kk = Ops<T>::mma(*(const v8*)(ka + ko), bv, kk);
                qk = Ops<T>::mma(*(const v8*)(qa + ks * 16), bv, qk);
            }
            const int s = sb * 32 + col;
            const float gs = Gs[s];
            const int t4 = tb * 32 + 4 * g;  // this lane's accumulator rows: t4 + arow(j)
            const float* gt = Gs + t4;
            const float* bt = Bs + t4;
            float* am = Am + t4 * AS + s;
            T* aq = Aq + t4 * TS + s;
            // G and beta of this lane's 16 rows (runs of 4 at t4 + 8 i), read before the masks
            // so the selects below compile without branches
            f32x4 gq[4], bq[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                gq[i] = *(const f32x4*)(gt + 8 * i);
                bq[i] = *(const f32x4*)(bt + 8 * i);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = t4 + arow(j);
                // exp(G_t - G_s) may overflow above the diagonal; the selects drop it there
                const float ex = __expf(gq[j >> 2][j & 3] - gs);
                const float dec = s <= t ? ex : 0.0f;
                am[arow(j) * AS] = s < t ? bq[j >> 2][j & 3] * dec * kk[j] : 0.0f;
                aq[arow(j) * TS] = (T)(dec * qk[j]);
            }
        } else {
            for (int idx = lane; idx < 32 * 32; idx += 64) {
                const int t = idx >> 5, s = 32 + (idx & 31);
                Am[t * AS + s] = 0.0f;
                Aq[t * TS + s] = (T)0.0f;
            }
        }
        v8 Sb[4][2];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            Sb[rb][0] = pack<T>(S[rb], 0);
            Sb[rb][1] = pack<T>(S[rb], 1);
        }
        v8 Rb[2][2];  // R = beta (V - exp(G) K S0), packed as the B operand of T R
        f32x16 Og[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            f32x16 ks = f32x16{}, qs = f32x16{};
            const T* kr = Kc + (tb * 32 + col) * DK;
            const T* qr = Qc + (tb * 32 + col) * RS;
            int swk = kswz(col);
            asm volatile("" : "+v"(swk));
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    ks = Ops<T>::mma(ld_perm_k<T>(kr, swk, rb, hh, g), Sb[rb][hh], ks);
                    qs = Ops<T>::mma(ld_perm<T>(qr, rb * 32, hh, g), Sb[rb][hh], qs);
                }
            const int t4 = tb * 32 + 4 * g;
            const float* gt = Gs + t4;
            const float* bt = Bs + t4;
            const T* vt = Vc + t4 * RS + dvc;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float eg = __expf(gt[arow(j)]);
                Rb[tb][j >> 3][j & 7] = (T)(bt[arow(j)] * (f(vt[arow(j) * RS]) - eg * ks[j]));
                Og[tb][j] = eg * qs[j];
            }
        }
        __syncthreads();
        // ---------------- P2: T = (I + A)^-1 in place ----------------
        invert_in_place(Am, Xs, wave, lane);
        // ---------------- P3: delta, O, state ----------------
        // (independent accumulation chains alternate in every product below)
        f32x16 dl[2] = {f32x16{}, f32x16{}};
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
                    dl[tb] = Ops<T>::mma(ld_perm_f32<T>(Am + (tb * 32 + col) * AS, sb * 32, hh, g), Rb[sb][hh], dl[tb]);
        v8 Db[2][2];
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            Db[sb][0] = pack<T>(dl[sb], 0);
            Db[sb][1] = pack<T>(dl[sb], 1);
        }
        T* Os = Qc;  // Q is no longer read in this chunk
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
                    Og[tb] = Ops<T>::mma(ld_perm<T>(Aq + (tb * 32 + col) * TS, sb * 32, hh, g), Db[sb][hh], Og[tb]);
        // every wave finished reading Qc (K S0 / Q S0) before the inversion's barriers
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 16; ++j) Os[(4 * g) * RS + dvc + (tb * 32 + arow(j)) * RS] = (T)Og[tb][j];
        const float glast = Gs[CH - 1];
        const float eglast = __expf(glast);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 16; ++j) dl[tb][j] *= __expf(glast - Gs[4 * g + tb * 32 + arow(j)]);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            Db[tb][0] = pack<T>(dl[tb], 0);
            Db[tb][1] = pack<T>(dl[tb], 1);
        }
        // S = e^{G_last} S + K^T (e^{G_last - G} delta). The A operand K^T[dk][t] (tokens
        // 32 tb + 16 hh + 8 x + 4 g + [0..3] for x = 0, 1) comes from transposing reads of K:
        // in 16-lane group G, lane j reads token 4 (G >> 1) + 8 x + (j >> 2) + 32 tb + 16 hh,
        // dims 32 rb + 16 (G & 1) + 4 (j & 3) .. + 3
        {
            int G = lane >> 4, j = lane & 15;
            asm volatile("" : "+v"(G), "+v"(j));
            int tofs[2][4];
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const int rr = 8 * x + 4 * (G >> 1) + (j >> 2);  // token row mod 32, without 16 hh
                    const int sw = ((j >> 2) << 2) | ((2 * x + (G >> 1)) & 3);
                    tofs[x][rb] = rr * DK + 8 * ((4 * rb + 2 * (G & 1) + ((j & 3) >> 1)) ^ sw) + 4 * (j & 1);
                }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) S[rb][jj] *= eglast;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int rb = 0; rb < 4; ++rb) {
                        const T* kb = Kc + (tb * 32 + 16 * hh) * DK;
                        const i16x4 lo = lds_read_tr16(kb + tofs[0][rb]);
                        const i16x4 hi = lds_read_tr16(kb + tofs[1][rb]);
                        const v8 af = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                        S[rb] = Ops<T>::mma(af, Db[tb][hh], S[rb]);
                    }
        }
        // P4 operands that do not depend on O: the gate norm_w * silu(z) of this thread's rows,
        // computed before the barrier (rows past the end read a clamped row and are not stored)
        const int rsub = tid & 15, rrow = tid >> 4;  // 16 lanes per row, 16 rows per pass
        float gz[4][8];
        if (FUSED) {
            v8 zv[4];
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const long tt = t0 + c0 + min(pass * 16 + rrow, Lc - 1);
                zv[pass] = *(const v8*)((const T*)fa.z + tt * fa.z_tok + (long)h * DV + 8 * rsub);
            }
#pragma unroll
            for (int pass = 0; pass < 4; ++pass)
#pragma unroll
                for (int e = 0; e < 8; ++e) gz[pass][e] = fa.norm_w[8 * rsub + e] * silu(f(zv[pass][e]));
        }
        __syncthreads();
        // ---------------- P4: O -> HBM (gated RMSNorm when fused) ----------------
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int r = pass * 16 + rrow;
            const v8 ov = *(const v8*)(Os + r * RS + 8 * rsub);
            const long tt = t0 + c0 + r;
            if (FUSED) {
                float x[8], ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x[e] = f(ov[e]);
                    ss += x[e] * x[e];
                }
                ss = sum16(ss);
                const float inv = fast_rsqrt(ss * (1.0f / 128.0f) + fa.eps);
                v8 y;
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = (T)((x[e] * inv) * gz[pass][e]);
                if (r < Lc) *(v8*)((T*)a.o + tt * a.o_tok + (long)h * DV + 8 * rsub) = y;
            } else if (r < Lc) {
                *(v8*)((T*)a.o + tt * a.o_tok + (long)h * DV + 8 * rsub) = ov;
            }
        }
    }
    if (s1) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int j = 0; j < 16; ++j) s1[sbase + (long)(4 * g) * DV + dvc + (rb * 32 + arow(j)) * DV] = S[rb][j];
    }
    if (FUSED && tail && wave < 3 && rg == 0) {
        // cache tail: the last 3 raw conv inputs of [history, sequence]; wave ts writes the
        // channels of q, k or v (16 lanes x 8 channels)
        const long mc = mcol + wave * (long)fa.Hk * 128 + (wave == 2 ? (long)(h - kh) * 128 : 0);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int p = Tn - 3 + i;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.0f;
            if (p >= 0) {
                v8 x = *(const v8*)((const T*)fa.mixed + (long)(t0 + p) * fa.mixed_tok + mc);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = f(x[e]);
            } else if (hist) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = f(hist[((long)mc + e) * 3 + (p + 3)]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) tail[((long)mc + e) * 3 + i] = (T)v[e];
        }
    }
}

}  // namespace gdn2
}  // namespace hk

template <typename T, bool FUSED>
static int launch_v2(const hk::GdnArgs* a, const hk::GdnFusedArgs* fa, int n_seqs, hipStream_t stream) {
    static bool configured = false;
    auto kern = hk::gdn2::gdn_chunk<T, FUSED>;
    if (!configured) {
        if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)hk::gdn2::LDS_BYTES) != hipSuccess)
            return HK_ERR_DEVICE;
        configured = true;
    }
    hipLaunchKernelGGL(kern, dim3(a->H, n_seqs), dim3(256), hk::gdn2::LDS_BYTES, stream, *a, *fa);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

// dtype16: 1 = bf16, 2 = fp16
extern "C" int hk_launch_gdn_v2(int dtype16, int fused, const hk::GdnArgs* a, const hk::GdnFusedArgs* fa, int n_seqs,
                                hipStream_t stream) {
    hk::GdnFusedArgs none{};
    if (!fa) fa = &none;
    if (dtype16 == 1)
        return fused ? launch_v2<hk::bf16, true>(a, fa, n_seqs, stream) : launch_v2<hk::bf16, false>(a, fa, n_seqs, stream);
    return fused ? launch_v2<hk::f16, true>(a, fa, n_seqs, stream) : launch_v2<hk::f16, false>(a, fa, n_seqs, stream);
}
