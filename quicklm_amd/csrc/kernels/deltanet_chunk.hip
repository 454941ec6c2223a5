// Chunked prefill of a Gated DeltaNet layer (one sequence, T prompt rows at
// positions p0 .. p0+T-1). The reference runs the recurrence row by row
// (Qwen3_5GatedDeltaNet::forward_chunk, attention.cpp:600-758); this is the
// same recurrence in the chunked "WY" form, with every contraction on the
// fp32 matrix cores (v_mfma_f32_16x16x4f32).
//
// Per head, with the state S [d_k, d_v] before a chunk of C = 64 rows,
// alpha_t = log-decay, G_t = sum_{s<=t} alpha_s within the chunk,
// gamma_t = exp(G_t), beta_t the write strength and q, k L2-normalised:
//   S_t = gamma_t S + sum_{s<=t} (gamma_t/gamma_s) k_s w_s^T, where
//   (I + A) W = diag(beta) (V - diag(gamma) K S),
//   A[t][s] = beta_t (gamma_t/gamma_s) (k_t . k_s) for s < t.
// With T = (I + A)^-1 diag(beta): U = T V, Wk = T diag(gamma) K, W = U - Wk S,
//   o_t = (gamma_t (Q S)[t] + sum_{s<=t} (gamma_t/gamma_s)(q_t . k_s) w_s) / sqrt(d),
//   S_next = gamma_end S + K^T diag(gamma_end/gamma) W.
// Every decay factor is exp of a non-positive number (ratios, never 1/gamma).
//
// Kernels (one stream, in order):
//   k_dn_chunk_prep   per (16 rows, head): conv taps from the prompt rows or
//                     the ring (positions before p0), SiLU, L2 norms, gates --
//                     the decode step's arithmetic;
//   k_dn_chunk_intra  per (chunk, head): K K^T and the masked, decayed Q K^T
//                     on the matrix cores, the triangular solve for T (one
//                     column per lane, unrolled), U and Wk on the matrix cores;
//   k_dn_chunk_inter  per (head, 16 value columns): chunks in order; W and
//                     the state update on the matrix cores, the state slice
//                     living in the accumulators, and on other waves O of
//                     the chunk before;
//   k_dn_chunk_post   per (16 rows, head): head RMSNorm + SiLU(z) gate (decode
//                     arithmetic) and the conv ring rows of the last positions.

#include "common.hpp"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;      // head dim (d_k = d_v)
constexpr int kC = 64;       // chunk rows
constexpr int KP = kD + 4;   // padded LDS row of a [64][128] tile
constexpr int TP = kC + 4;   // padded LDS row of a [64][64] tile
constexpr int CB = 16;       // value columns per inter-chunk workgroup

// Makes the compiler wait here for the load that produced v.
__device__ __forceinline__ void landed(float v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void landed(const float4& v) {
    landed(v.x);
    landed(v.y);
    landed(v.z);
    landed(v.w);
}

// D += A B on a 16x16 tile, K = 4: lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; it holds D[(l/16)*4 + i][l%16].
__device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ size_t rix(int t, int h, int H) { return ((size_t)t * H + h) * kD; }

// Rows a prep or post workgroup handles (a conv window slides down them).
constexpr int kPR = 16;

// Per (16 rows, head): thread (section, column) slides the conv window down
// the rows, the q and k outputs wait in LDS for their row norms (6 waves, a
// norm each at a time), v goes straight out.
__global__ __launch_bounds__(3 * kD) void k_dn_chunk_prep(
    const float* __restrict__ proj, int ldp, int T, const float* __restrict__ conv_state,
    const float* __restrict__ wt, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, int p0, int H, float* __restrict__ qn,
    float* __restrict__ kn, float* __restrict__ vv, float* __restrict__ alpha,
    float* __restrict__ beta) {
    __shared__ float ys[2][kPR][kD];
    const int t0 = blockIdx.x * kPR, h = blockIdx.y, tid = threadIdx.x;
    const int nt = min(kPR, T - t0);
    const int lane = tid & 63, wave = tid >> 6;
    const int HD = H * kD, C = 3 * HD;
    const int sec = tid / kD, tt = tid % kD, ch = sec * HD + h * kD + tt;
    const float w0 = wt[ch], w1 = wt[(size_t)C + ch], w2 = wt[(size_t)2 * C + ch],
                w3 = wt[(size_t)3 * C + ch];
    // inputs of positions t-3, t-2, t-1; positions before p0 come from the
    // ring, row (position mod 3), as the decode step reads it (zero rows on a
    // fresh sequence)
    float xw[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int r = t0 - 3 + j;
        if (r >= 0) {
            xw[j] = proj[(size_t)r * ldp + ch];
        } else {
            const int row = ((p0 + r) % 3 + 3) % 3;
            xw[j] = conv_state[(size_t)row * C + ch];
        }
    }
    float xr[kPR];  // rows past T read row T-1 and are never stored
#pragma unroll
    for (int r = 0; r < kPR; ++r) xr[r] = proj[(size_t)min(t0 + r, T - 1) * ldp + ch];
#pragma unroll
    for (int r = 0; r < kPR; ++r) {
        float acc = 0.0f;
        acc = nc_add_mul(acc, xw[0], w0);
        acc = nc_add_mul(acc, xw[1], w1);
        acc = nc_add_mul(acc, xw[2], w2);
        acc = nc_add_mul(acc, xr[r], w3);
        const float y = silu_f(acc);
        if (sec < 2) ys[sec][r][tt] = y;
        else if (r < nt) vv[rix(t0 + r, h, H) + tt] = y;
        xw[0] = xw[1];
        xw[1] = xw[2];
        xw[2] = xr[r];
    }
    if (tid >= 2 * kD && tid - 2 * kD < nt) {
        const int t = t0 + tid - 2 * kD;
        const float* pr = proj + (size_t)t * ldp;
        const float dt = pr[4 * HD + H + h] + dt_bias[h];
        const float sp = dt > 20.0f ? dt : log1pf(expf(dt));
        alpha[(size_t)t * H + h] = -expf(A_log[h]) * sp;
        beta[(size_t)t * H + h] = 1.0f / (1.0f + expf(-pr[4 * HD + h]));
    }
    __syncthreads();
    for (int i = wave; i < 2 * kPR; i += 3 * kD / 64) {
        const int which = i & 1, r = i >> 1;
        if (r >= nt) break;
        const float a0 = ys[which][r][lane], a1 = ys[which][r][lane + 64];
        float ss = fmaf(a0, a0, a1 * a1);
        ss = wave_sum(ss);
        const float nrm = sqrtf(ss + 1e-6f);
        float* dst = (which == 0 ? qn : kn) + rix(t0 + r, h, H);
        dst[lane] = a0 / nrm;
        dst[lane + 64] = a1 / nrm;
    }
}

// Global operands that feed the matrix cores straight from registers (the
// wave's q rows for Q K^T, its 32 value columns for U = T V) are loaded at
// the start, so their latency passes under the K staging, K K^T and the
// solve instead of stalling each product step.
__global__ __launch_bounds__(256, 2) void k_dn_chunk_intra(
    const float* __restrict__ qn, const float* __restrict__ kn, const float* __restrict__ vv,
    const float* __restrict__ alpha, const float* __restrict__ beta, int T, int H,
    float* __restrict__ U, float* __restrict__ Wk, float* __restrict__ Mq,
    float* __restrict__ Gc) {
    __shared__ __attribute__((aligned(16))) float Ks[kC * KP];
    __shared__ float Ts[kC * TP];
    __shared__ float gs[kC], bs[kC], gam[kC];
    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, l4 = lane >> 4;
    const int t0 = c * kC;
    const int nt = min(kC, T - t0);
    auto row = [&](int t) { return rix(t0 + min(t, nt - 1), h, H); };  // clamped; masked at use

    // q[tq][k0 + l4] for k0 = 0, 4, .., 124 (rows of Q K^T)
    const int tq = wave * 16 + l16;
    float qv[kD / 4];
    {
        const float* qrow = qn + row(tq);
#pragma unroll
        for (int i = 0; i < kD / 4; ++i) qv[i] = qrow[4 * i + l4];
    }
    // V[k0 + l4][32 wave + 16 ct + l16] for k0 = 0, 4, .., 60 (columns of U)
    float vr[kC / 4][2];
#pragma unroll
    for (int i = 0; i < kC / 4; ++i) {
        const float* vrow = vv + row(4 * i + l4) + 32 * wave + l16;
        vr[i][0] = vrow[0];
        vr[i][1] = vrow[16];
    }
    for (int i = tid; i < kC * (kD / 4); i += 256) {
        const int r = i / (kD / 4), c4 = i % (kD / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nt) v = *reinterpret_cast<const float4*>(kn + rix(t0 + r, h, H) + c4 * 4);
        *reinterpret_cast<float4*>(&Ks[r * KP + c4 * 4]) = v;
    }
    if (tid < kC) {
        gs[tid] = tid < nt ? alpha[(size_t)(t0 + tid) * H + h] : 0.0f;
        bs[tid] = tid < nt ? beta[(size_t)(t0 + tid) * H + h] : 0.0f;
    }
    __syncthreads();
    if (tid == 0) {  // cumulative log-decay, in row order
        float a = 0.0f;
        for (int t = 0; t < kC; ++t) {
            a += gs[t];
            gs[t] = a;
        }
    }
    __syncthreads();
    if (tid < kC) {
        gam[tid] = expf(gs[tid]);
        if (tid < nt) Gc[(size_t)(t0 + tid) * H + h] = gs[tid];
    }

    // A = beta_t (gamma_t/gamma_s) K K^T, strictly lower; wave w: rows 16w..16w+15
    {
        f32x4 acc[4];
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) acc[tc] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < kD; k0 += 4) {
            const float a = Ks[(wave * 16 + l16) * KP + k0 + l4];
#pragma unroll
            for (int tc = 0; tc < 4; ++tc) acc[tc] = mma(a, Ks[(tc * 16 + l16) * KP + k0 + l4], acc[tc]);
        }
#pragma unroll
        for (int tc = 0; tc < 4; ++tc)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = wave * 16 + l4 * 4 + i, s = tc * 16 + l16;
                Ts[t * TP + s] = s < t ? bs[t] * expf(gs[t] - gs[s]) * acc[tc][i] : 0.0f;
            }
    }

    // Mq[t][s] = (gamma_t/gamma_s) q_t . k_s for s <= t; wave w: rows 16w..
    {
        f32x4 m[4];
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) m[tc] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < kD / 4; ++i) {
            const float a = tq < nt ? qv[i] : 0.0f;
#pragma unroll
            for (int tc = 0; tc < 4; ++tc)
                m[tc] = mma(a, Ks[(tc * 16 + l16) * KP + 4 * i + l4], m[tc]);
        }
        float* mq = Mq + ((size_t)c * H + h) * kC * kC;
#pragma unroll
        for (int tc = 0; tc < 4; ++tc)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = wave * 16 + l4 * 4 + i, s = tc * 16 + l16;
                mq[t * kC + s] = (s <= t && t < nt) ? expf(gs[t] - gs[s]) * m[tc][i] : 0.0f;
            }
    }
    __syncthreads();

    // T = (I + A)^-1 diag(beta) by forward substitution; lane s < 64 owns
    // column s (T[t][s] = beta_t [t == s] - sum_{r<t} A[t][r] T[r][s]).
    float col[kC];
    if (tid < kC) {
#pragma unroll
        for (int t = 0; t < kC; ++t) {
            float v = t == tid ? bs[t] : 0.0f;
#pragma unroll
            for (int r = 0; r < t; ++r) v = fmaf(-Ts[t * TP + r], col[r], v);
            col[t] = v;
        }
    }
    __syncthreads();  // every read of A is done before T overwrites it
    if (tid < kC) {
#pragma unroll
        for (int t = 0; t < kC; ++t) Ts[t * TP + tid] = col[t];
    }
    __syncthreads();

    // Wk = T diag(gamma) K and U = T V: wave w columns 32w..32w+31, all 64
    // rows (four row tiles)
    {
        f32x4 wk[4][2], u[4][2];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                wk[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
                u[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int i = 0; i < kC / 4; ++i) {
            const int s = 4 * i + l4;
            const bool ok = s < nt;
            const float g = gam[s];
            const float kb0 = Ks[s * KP + 32 * wave + l16], kb1 = Ks[s * KP + 32 * wave + 16 + l16];
            const float vb0 = ok ? vr[i][0] : 0.0f, vb1 = ok ? vr[i][1] : 0.0f;
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const float tv = Ts[(rt * 16 + l16) * TP + s];
                const float tg = tv * g;
                wk[rt][0] = mma(tg, kb0, wk[rt][0]);
                wk[rt][1] = mma(tg, kb1, wk[rt][1]);
                u[rt][0] = mma(tv, vb0, u[rt][0]);
                u[rt][1] = mma(tv, vb1, u[rt][1]);
            }
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = rt * 16 + l4 * 4 + i;
                    if (t < nt) {
                        const size_t o = rix(t0 + t, h, H) + 32 * wave + 16 * ct + l16;
                        Wk[o] = wk[rt][ct][i];
                        U[o] = u[rt][ct][i];
                    }
                }
    }
}

// Per (head, 16 value columns), chunks in order, with two roles a SIMD:
// waves 0-3 run the state chain of chunk c,
//   W = U - Wk S,  S = gamma_end S + K^T diag(gamma_end / gamma) W,
// the only products that depend on the state (wave w: W rows 16w.., state
// rows 32w..); waves 4-7 meanwhile form the outputs of chunk c-1,
//   O = (gamma_t (Q S) + Mq W) / sqrt(d),
// Q S beside the chain's W and Mq W beside its state update, from the state
// and W that chunk left in LDS, so that work fills the chain's waits instead
// of lengthening it. The output waves also stage each chunk's k rows in LDS
// (whole rows, 16-byte loads) for the state update. The state is kept in
// three LDS slots (S_c read by the chain, S_{c+1} written, S_{c-1} read by
// the output waves), W and the cumulative gates in two. The chunk operands
// do not depend on the state: each is loaded for the next chunk right after
// its last use in this one, from buffers padded to whole chunks (rows past T
// are never used: every operand from them is replaced by zero with a
// select). Every product runs its K index as 16 kb + 4 l4 + j on lane
// (l16, l4), so the LDS operand of four consecutive products is one 16-byte
// read: the state and W slices are stored transposed ([16][K + 4]).
constexpr int KT = kD + 4;  // pitch of a transposed state slice
constexpr int TT = kC + 4;  // pitch of a transposed W slice

__global__ __launch_bounds__(512) void k_dn_chunk_inter(
    const float* __restrict__ qn, const float* __restrict__ kn, const float* __restrict__ U,
    const float* __restrict__ Wk, const float* __restrict__ Mq, const float* __restrict__ Gc,
    int T, int H, float* __restrict__ state, float* __restrict__ O) {
    __shared__ __attribute__((aligned(16))) float St[3][CB * KT];
    __shared__ __attribute__((aligned(16))) float Wt[2][CB * TT];
    __shared__ __attribute__((aligned(16))) float gs[2][kC];
    __shared__ __attribute__((aligned(16))) float dec[kC];
    __shared__ __attribute__((aligned(16))) float Ks[kC * KP];
    const int h = blockIdx.x, jb = blockIdx.y * CB;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the roles branch on it
    const int l16 = lane & 15, l4 = lane >> 4;
    const int w4 = wave & 3;
    const int nch = (T + kC - 1) / kC;
    const size_t RS = (size_t)H * kD;  // a row of every head
    const size_t CS = kC * RS;         // a chunk of rows
    const int tr = w4 * 16 + l16;      // A-operand row of this wave's tiles
    auto lds4 = [](const float* p) { return *reinterpret_cast<const float4*>(p); };
    auto sto4 = [](float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; };

    // Each role runs its own loop (so each loop's load waits count only its
    // own loads); both meet two barriers a pass, nch + 1 passes.
    if (wave < 4) {
        // state rows 32w .. 32w+31 (two 16-row tiles), columns jb .. jb+15
        float* Sg = state + (size_t)h * kD * kD;
        f32x4 sacc[2];
        float4 pw[8];
        float pu[4], pg = 0.0f, pge = 0.0f;
        const float* wk_b = Wk + tr * RS + h * kD + 4 * l4;
        const float* u_b = U + (w4 * 16 + l4 * 4) * RS + h * kD + jb + l16;
        auto load_g = [&](int c) {
            pg = Gc[((size_t)c * kC + lane) * H + h];  // row lane of the chunk (wave 0 uses it)
            pge = Gc[((size_t)c * kC + min(kC, T - c * kC) - 1) * H + h];
        };
        auto load_wu = [&](int c) {
            const size_t cs = (size_t)c * CS;
#pragma unroll
            for (int kb = 0; kb < 8; ++kb) pw[kb] = *reinterpret_cast<const float4*>(wk_b + cs + 16 * kb);
#pragma unroll
            for (int i = 0; i < 4; ++i) pu[i] = u_b[cs + i * RS];
        };
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int r0 = (2 * w4 + tt) * 16 + l4 * 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) sacc[tt][i] = Sg[(size_t)(r0 + i) * kD + jb + l16];
            sto4(&St[0][l16 * KT + r0], sacc[tt]);
        }
        load_g(0);
        load_wu(0);
        // Every load of the preamble lands before the loop: the wait counts
        // inside it then follow the loop's own load order (entered with the
        // preamble's loads pending, in another order, they wait for all).
        landed(pg);
        landed(pge);
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) landed(pw[kb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) landed(pu[i]);
        __syncthreads();
        for (int c = 0; c < nch; ++c) {
            const int cn = min(c + 1, nch - 1);
            const int nt = min(kC, T - c * kC);
            const bool tv = tr < nt;
            const float* Sc = St[c % 3] + l16 * KT + 4 * l4;
            if (wave == 0) {
                gs[c & 1][lane] = lane < nt ? pg : 0.0f;
                dec[lane] = lane < nt ? expf(pge - pg) : 0.0f;  // gamma_end / gamma_t
            }
            const float ge = expf(pge);
            load_g(cn);
            // W = U - Wk S (four independent chains: a chain of dependent
            // products waits out each one's latency)
            f32x4 wc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) wc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 8; ++kb) {
                const float a[4] = {pw[kb].x, pw[kb].y, pw[kb].z, pw[kb].w};
                const float4 b4 = lds4(Sc + 16 * kb);
                const float b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) wc[j] = mma(tv ? a[j] : 0.0f, b[j], wc[j]);
            }
            f32x4 wv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = w4 * 16 + l4 * 4 + i;
                wv[i] = t < nt ? pu[i] - ((wc[0][i] + wc[1][i]) + (wc[2][i] + wc[3][i])) : 0.0f;
            }
            sto4(&Wt[c & 1][l16 * TT + w4 * 16 + l4 * 4], wv);
            load_wu(cn);
            __syncthreads();  // W of chunk c and its gates are in LDS
            // S = gamma_end S + K^T diag(gamma_end / gamma) W
            const float* Wc = Wt[c & 1] + l16 * TT + 4 * l4;
            const float* Kc = Ks + 4 * l4 * KP + 2 * w4 * 16 + l16;
            f32x4 du[2][2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) du[tt][0] = du[tt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const float4 w4v = lds4(Wc + 16 * kb);
                const float4 d4 = lds4(&dec[16 * kb + 4 * l4]);
                const float b[4] = {w4v.x * d4.x, w4v.y * d4.y, w4v.z * d4.z, w4v.w * d4.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool ok = 16 * kb + 4 * l4 + j < nt;
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const float kv = Kc[(16 * kb + j) * KP + 16 * tt];
                        du[tt][j & 1] = mma(ok ? kv : 0.0f, b[j], du[tt][j & 1]);
                    }
                }
            }
            float* Sn = St[(c + 1) % 3];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    sacc[tt][i] = sacc[tt][i] * ge + (du[tt][0][i] + du[tt][1][i]);
                sto4(&Sn[l16 * KT + (2 * w4 + tt) * 16 + l4 * 4], sacc[tt]);
            }
            __syncthreads();  // S of chunk c+1 is in LDS; this pass's slot reads are done
        }
        __syncthreads();  // the output waves' last pass
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                Sg[(size_t)((2 * w4 + tt) * 16 + l4 * 4 + i) * kD + jb + l16] = sacc[tt][i];
    } else {
        // outputs of the chunk before: q and Mq rows 16w'.. of it
        const float rsd = 1.0f / sqrtf((float)kD);
        const size_t MS = (size_t)H * kC * kC;
        float4 pq[8], pm[4];
        const float* q_b = qn + tr * RS + h * kD + 4 * l4;
        const float* m_b = Mq + ((size_t)h * kC + tr) * kC + 4 * l4;
        auto load_out = [&](int c) {
#pragma unroll
            for (int kb = 0; kb < 8; ++kb)
                pq[kb] = *reinterpret_cast<const float4*>(q_b + (size_t)c * CS + 16 * kb);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                pm[kb] = *reinterpret_cast<const float4*>(m_b + (size_t)c * MS + 16 * kb);
        };
        // k rows of a chunk: thread o = tid - 256 moves float4 o + 256 i
        float4 pkk[8];
        const int o = tid - 256;
        auto load_kk = [&](int c) {
            const float* base = kn + (size_t)c * CS + h * kD;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = o + 256 * i;
                pkk[i] = *reinterpret_cast<const float4*>(base + (e >> 5) * RS + (e & 31) * 4);
            }
        };
        auto store_kk = [&]() {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = o + 256 * i;
                *reinterpret_cast<float4*>(&Ks[(e >> 5) * KP + (e & 31) * 4]) = pkk[i];
            }
        };
        load_out(0);
        load_kk(0);
        store_kk();
        if (nch > 1) load_kk(1);
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) landed(pq[kb]);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) landed(pm[kb]);
#pragma unroll
        for (int i = 0; i < 8; ++i) landed(pkk[i]);
        __syncthreads();
        for (int c = 0; c <= nch; ++c) {
            const int cp = c - 1;
            const int nt = min(kC, T - cp * kC);
            const bool tv = tr < nt;
            f32x4 qc[4];
            if (c > 0 && c < nch) {  // k rows of chunk c for its state update
                store_kk();
                if (c + 1 < nch) load_kk(c + 1);
            }
            if (c > 0) {  // Q S, beside the chain's W = U - Wk S
                const float* Sp = St[cp % 3] + l16 * KT + 4 * l4;
#pragma unroll
                for (int r = 0; r < 4; ++r) qc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < 8; ++kb) {
                    const float a[4] = {pq[kb].x, pq[kb].y, pq[kb].z, pq[kb].w};
                    const float4 b4 = lds4(Sp + 16 * kb);
                    const float b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) qc[j] = mma(tv ? a[j] : 0.0f, b[j], qc[j]);
                }
            }
            __syncthreads();
            if (c > 0) {  // Mq W and the outputs, beside the chain's state update
                const float* Wp = Wt[cp & 1] + l16 * TT + 4 * l4;
                f32x4 mc[2];
                mc[0] = mc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const float a[4] = {pm[kb].x, pm[kb].y, pm[kb].z, pm[kb].w};
                    const float4 b4 = lds4(Wp + 16 * kb);
                    const float b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) mc[j & 1] = mma(tv ? a[j] : 0.0f, b[j], mc[j & 1]);
                }
                if (c < nch) load_out(c);
                const float4 g4 = lds4(&gs[cp & 1][w4 * 16 + l4 * 4]);
                const float g[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = w4 * 16 + l4 * 4 + i;
                    if (t < nt)
                        O[((size_t)cp * kC + t) * RS + h * kD + jb + l16] =
                            (expf(g[i]) * ((qc[0][i] + qc[2][i]) + (qc[1][i] + qc[3][i])) +
                             (mc[0][i] + mc[1][i])) * rsd;
                }
            }
            __syncthreads();
        }
    }
}

// Per (16 rows, head): a wave a row at a time (its two 64-column halves
// summed as the decode step's two waves are), and the conv ring rows of the
// last three positions.
__global__ __launch_bounds__(256) void k_dn_chunk_post(
    const float* __restrict__ O, const float* __restrict__ proj, int ldp, int T,
    const float* __restrict__ norm_w, float* __restrict__ out, int ldo, int H,
    float* __restrict__ conv_state, int p0) {
    const int t0 = blockIdx.x * kPR, h = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nt = min(kPR, T - t0);
    const int HD = H * kD, C = 3 * HD;
    const float nw0 = norm_w[lane], nw1 = norm_w[lane + 64];
    for (int r = wave; r < nt; r += 4) {
        const int t = t0 + r;
        const float* pr = proj + (size_t)t * ldp;
        const float o0 = O[rix(t, h, H) + lane], o1 = O[rix(t, h, H) + lane + 64];
        const float z0 = pr[3 * HD + h * kD + lane], z1 = pr[3 * HD + h * kD + lane + 64];
        const float tot = wave_sum(o0 * o0) + wave_sum(o1 * o1);
        const float sn = 1.0f / sqrtf(tot / (float)kD + 1e-6f);
        out[(size_t)t * ldo + h * kD + lane] = ((o0 * sn) * nw0) * silu_f(z0);
        out[(size_t)t * ldo + h * kD + lane + 64] = ((o1 * sn) * nw1) * silu_f(z1);
        if (t >= T - 3) {  // ring row of position p0 + t keeps its conv input
            const int row = (p0 + t) % 3;
            for (int i = lane; i < 3 * kD; i += 64) {
                const int ch = (i / kD) * HD + h * kD + i % kD;
                conv_state[(size_t)row * C + ch] = pr[ch];
            }
        }
    }
}

size_t a256(size_t b) { return (b + 255) & ~(size_t)255; }

struct ChunkWork {
    float *qn, *kn, *vv, *U, *Wk, *O, *alpha, *beta, *Gc, *Mq;
    size_t bytes;
};

ChunkWork carve(void* base, int T, int H) {
    ChunkWork w{};
    // rows and gates padded to whole chunks: the state chain reads a whole
    // chunk's operands and masks the rows past T
    const int nch = (T + kC - 1) / kC;
    const size_t rows = a256((size_t)nch * kC * H * kD * sizeof(float));
    const size_t sc = a256((size_t)nch * kC * H * sizeof(float));
    char* p = reinterpret_cast<char*>(base);
    auto take = [&](size_t b) {
        float* r = reinterpret_cast<float*>(p);
        if (p) p += b;
        return r;
    };
    w.qn = take(rows);
    w.kn = take(rows);
    w.vv = take(rows);
    w.U = take(rows);
    w.Wk = take(rows);
    w.O = take(rows);
    w.alpha = take(sc);
    w.beta = take(sc);
    w.Gc = take(sc);
    w.Mq = take(a256((size_t)nch * H * kC * kC * sizeof(float)));
    w.bytes = 6 * rows + 3 * sc + a256((size_t)nch * H * kC * kC * sizeof(float));
    return w;
}

}  // namespace

extern "C" size_t qlm_deltanet_chunk_workspace_bytes(int T, int H, int d) {
    if (T <= 0 || H <= 0 || d != kD) return 0;
    return carve(nullptr, T, H).bytes;
}

extern "C" int qlm_deltanet_prefill_chunked(const float* proj, int ldp, int T, float* conv_state,
                                            const float* conv_w_t, const float* A_log,
                                            const float* dt_bias, const float* norm_w,
                                            float* state, int p0, float* out, int ldo, int H,
                                            int d, void* work, size_t work_bytes,
                                            void* stream) {
    if (!proj || !conv_state || !conv_w_t || !A_log || !dt_bias || !norm_w || !state || !out ||
        !work || T <= 0 || H <= 0 || p0 < 0)
        return QLM_ERR_ARG;
    if (d != kD) return QLM_ERR_SHAPE;
    if (ldp < 4 * H * d + 2 * H || ldo < H * d) return QLM_ERR_SHAPE;
    const ChunkWork w = carve(work, T, H);
    if (work_bytes < w.bytes || ((uintptr_t)work & 255u)) return QLM_ERR_ARG;
    hipStream_t st = as_stream(stream);
    const int nch = (T + kC - 1) / kC;
    const int nrb = (T + kPR - 1) / kPR;
    hipLaunchKernelGGL(k_dn_chunk_prep, dim3(nrb, H), dim3(3 * kD), 0, st, proj, ldp, T, conv_state,
                       conv_w_t, A_log, dt_bias, p0, H, w.qn, w.kn, w.vv, w.alpha, w.beta);
    int rc = qlm_launch_status();
    if (rc != QLM_OK) return rc;
    hipLaunchKernelGGL(k_dn_chunk_intra, dim3(nch, H), dim3(256), 0, st, w.qn, w.kn, w.vv,
                       w.alpha, w.beta, T, H, w.U, w.Wk, w.Mq, w.Gc);
    rc = qlm_launch_status();
    if (rc != QLM_OK) return rc;
    hipLaunchKernelGGL(k_dn_chunk_inter, dim3(H, kD / CB), dim3(512), 0, st, w.qn, w.kn, w.U,
                       w.Wk, w.Mq, w.Gc, T, H, state, w.O);
    rc = qlm_launch_status();
    if (rc != QLM_OK) return rc;
    hipLaunchKernelGGL(k_dn_chunk_post, dim3(nrb, H), dim3(256), 0, st, w.O, proj, ldp, T, norm_w,
                       out, ldo, H, conv_state, p0);
    return qlm_launch_status();
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_deltanet_chunk() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(k_dn_chunk_prep));
}
