// Gated DeltaNet decode step (reference: Qwen3_5GatedDeltaNet::forward,
// attention.cpp:414-590; recurrence :498-571).
//
// One workgroup per (sequence, head), 512 threads. The head's fp32 state
// S[d=128][d=128] (key i, value j) is read once into registers, updated in
// place and written once: thread (ig, jg) owns rows ig*8..ig*8+7 and columns
// jg*4..jg*4+3 (8 float4 = 32 values). A wave covers two 512-byte row
// segments per load, so state traffic is fully coalesced.
//
// The reference reduces kv[j] and o[j] sequentially over i; here each thread
// reduces its 8 rows sequentially and the 16 row-groups are then summed in
// fixed order through LDS (deterministic, not bit-identical).
//
// The fused decode form also does the head's slice of the causal conv1d
// (3 x 128 channels, tap-major ring indexed by pos % 3), SiLU, L2 norm of q
// and k, the decay/beta gates, head RMSNorm and the SiLU(z) output gate, so
// one launch replaces steps 2-9 of the reference forward.

#include "common.hpp"
#include "l2_prefetch.hpp"

namespace {

constexpr int kD = 128;
constexpr int kThreads = 512;
constexpr int kRowGroups = kThreads / 32;     // 16
constexpr int kRowsPer = kD / kRowGroups;      // 8

// The position of a call without a position array: a zero in device
// memory, so the position is read by an unconditional load (a load under a
// branch is waited for where the branch ends, before every other operand
// has even been requested).
__device__ int g_pos_zero = 0;

struct DnShared {
    float q[kD], k[kD], v[kD];
    float pad[kD];  // conv results of the threads past the 3d channels (unused)
    float red[kRowGroups][kD];
    float vec[kD];
    float scal[8];
};

// Thread (ig, jg)'s slice of the head state: rows ig*8..ig*8+7, float4
// column jg. Requested at kernel start so the 64 KiB read overlaps the
// prologue.
__device__ __forceinline__ void dn_load_state(const float* __restrict__ S,
                                              float4 (&s)[kRowsPer]) {
    const int tid = threadIdx.x;
    const int jg = tid & 31;
    const int ig = tid >> 5;
    const float4* S4 = reinterpret_cast<const float4*>(S);
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) s[r] = S4[(ig * kRowsPer + r) * (kD / 4) + jg];
}

// Recurrence core. q,k,v in LDS (q already L2-normalised, k too), the state
// slice in s (updated in place; also stored to S unless S is null). Leaves
// the un-normalised, 1/sqrt(d)-scaled output in sh.vec.
__device__ __forceinline__ void dn_recurrence(DnShared& sh, float* __restrict__ S,
                                              float4 (&s)[kRowsPer], float dec, float beta) {
    const int tid = threadIdx.x;
    const int jg = tid & 31;
    const int ig = tid >> 5;
    float4* S4 = reinterpret_cast<float4*>(S);

    // (1) decay and kv = k . S_decayed
    float4 kv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) {
        const float ki = sh.k[ig * kRowsPer + r];
        s[r].x *= dec;
        s[r].y *= dec;
        s[r].z *= dec;
        s[r].w *= dec;
        kv.x = fmaf(ki, s[r].x, kv.x);
        kv.y = fmaf(ki, s[r].y, kv.y);
        kv.z = fmaf(ki, s[r].z, kv.z);
        kv.w = fmaf(ki, s[r].w, kv.w);
    }
    reinterpret_cast<float4*>(sh.red[ig])[jg] = kv;
    __syncthreads();
    if (tid < kD) {
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < kRowGroups; ++g) t += sh.red[g][tid];
        sh.vec[tid] = sh.v[tid] - t;  // delta
    }
    __syncthreads();

    // (2) S += (beta*k) delta^T ; (3) o = q . S_new
    const float4 dl = reinterpret_cast<const float4*>(sh.vec)[jg];
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) {
        const int i = ig * kRowsPer + r;
        const float bk = beta * sh.k[i];
        const float qi = sh.q[i];
        s[r].x = fmaf(bk, dl.x, s[r].x);
        s[r].y = fmaf(bk, dl.y, s[r].y);
        s[r].z = fmaf(bk, dl.z, s[r].z);
        s[r].w = fmaf(bk, dl.w, s[r].w);
        o.x = fmaf(qi, s[r].x, o.x);
        o.y = fmaf(qi, s[r].y, o.y);
        o.z = fmaf(qi, s[r].z, o.z);
        o.w = fmaf(qi, s[r].w, o.w);
        if (S4) S4[i * (kD / 4) + jg] = s[r];
    }
    __syncthreads();  // everyone has consumed sh.vec (delta)
    reinterpret_cast<float4*>(sh.red[ig])[jg] = o;
    __syncthreads();
    if (tid < kD) {
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < kRowGroups; ++g) t += sh.red[g][tid];
        sh.vec[tid] = t * (1.0f / sqrtf((float)kD));
    }
    __syncthreads();
}

// Isolated step: q,k,v,o [B,H,d], decay/beta [B,H], state [B,H,d,d].
__global__ __launch_bounds__(kThreads) void k_gated_delta_step(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ decay, const float* __restrict__ beta, float* __restrict__ state,
    float* __restrict__ out, int H) {
    __shared__ DnShared sh;
    const int bh = blockIdx.x;  // b*H + h
    const int tid = threadIdx.x;
    float4 s[kRowsPer];
    dn_load_state(state + (size_t)bh * kD * kD, s);
    const float dec = decay[bh], bt = beta[bh];
    if (tid < kD) {
        sh.q[tid] = q[(size_t)bh * kD + tid];
        sh.k[tid] = k[(size_t)bh * kD + tid];
        sh.v[tid] = v[(size_t)bh * kD + tid];
    }
    __syncthreads();
    dn_recurrence(sh, state + (size_t)bh * kD * kD, s, dec, bt);
    if (tid < kD) out[(size_t)bh * kD + tid] = sh.vec[tid];
}

// Fused decode mixer core. proj row: [qkv 3*H*d | z H*d | b H | a H].
// Every operand (state slice, the three conv ring rows, conv taps, gate
// inputs, z, gain) is requested at kernel start; the ring row order is
// resolved once pos has arrived.
__global__ __launch_bounds__(kThreads) void k_deltanet_decode(
    const float* __restrict__ proj, int ldp, float* __restrict__ conv_state,
    const float* __restrict__ wt, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ norm_w,
    float* __restrict__ state, const int* __restrict__ pos, float* __restrict__ out, int ldo,
    int H) {
    __shared__ DnShared sh;
    // every argument is read before the position is requested, so the
    // first wait for arguments does not also wait for the position
    asm volatile("" ::"s"(proj), "s"(ldp), "s"(conv_state), "s"(wt), "s"(A_log), "s"(dt_bias),
                 "s"(norm_w), "s"(state), "s"(pos), "s"(out), "s"(ldo), "s"(H));
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int HD = H * kD;
    const int C = 3 * HD;
    const float* pr = proj + (size_t)b * ldp;
    float* cs = conv_state + (size_t)b * 3 * C;
    float* Sh = state + ((size_t)b * H + h) * kD * kD;

    // The small operands are requested first, then the 64 KiB state slice:
    // loads complete in order, so the conv, norms and gates below wait only
    // for their own operands while the state is still arriving. Every load
    // is unconditional (clamped index; unused values are dropped), since a
    // load under a branch is waited for where the branch ends. The position
    // stays a vector value until every operand is requested: moved to a
    // scalar register at once, it would be waited for before them.
    int pbv = *(pos ? pos + b : &g_pos_zero);
    // conv operands: channel ch = sec*HD + h*d + t for tid < 3d
    const bool conv_t = tid < 3 * kD;
    const int sec = tid / kD, t = tid % kD;
    const int ch = conv_t ? sec * HD + h * kD + t : h * kD + t;
    float ring[3], w4[4];
#pragma unroll
    for (int j = 0; j < 3; ++j) ring[j] = cs[(size_t)j * C + ch];
#pragma unroll
    for (int j = 0; j < 4; ++j) w4[j] = wt[(size_t)j * C + ch];
    const float xin = pr[ch];
    // gate operands (used by wave 2, lane 0) and the output gate / gain
    // (used by waves 0-1)
    const float ga = pr[4 * HD + H + h], gb = pr[4 * HD + h];
    const float gdt = dt_bias[h], galog = A_log[h];
    const float zj = pr[3 * HD + h * kD + (tid & (kD - 1))];
    const float nwj = norm_w[tid & (kD - 1)];
    float4 s[kRowsPer];
    dn_load_state(Sh, s);
    asm volatile("" : "+v"(pbv));
    const int pb = __builtin_amdgcn_readfirstlane(pbv);

    // conv1d (kernel 4, taps chronological from the oldest ring row) + SiLU,
    // computed and stored to LDS by every thread (the others into a pad row),
    // so that no branch holds the operand loads, which the compiler would
    // otherwise sink behind the state's; the conv ring is updated by the 3d
    // conv threads
    {
        const int oldest = pb % 3;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int row = (oldest + j) % 3;
            const float rv = row == 0 ? ring[0] : (row == 1 ? ring[1] : ring[2]);
            acc = nc_add_mul(acc, rv, w4[j]);
        }
        acc = nc_add_mul(acc, xin, w4[3]);
        const float y = silu_f(acc);
        float* dst = !conv_t ? sh.pad : sec == 0 ? sh.q : sec == 1 ? sh.k : sh.v;
        dst[t] = y;
        if (conv_t) cs[(size_t)oldest * C + ch] = xin;
    }
    __syncthreads();

    // L2 norms (wave 0: q, wave 1: k) and gates (wave 2)
    if (wave < 2) {
        float* vv = wave == 0 ? sh.q : sh.k;
        const float a0 = vv[lane], a1 = vv[lane + 64];
        float ss = fmaf(a0, a0, a1 * a1);
        ss = wave_sum(ss);
        const float nrm = sqrtf(ss + 1e-6f);
        vv[lane] = a0 / nrm;
        vv[lane + 64] = a1 / nrm;
    } else if (wave == 2 && lane == 0) {
        const float dt = ga + gdt;
        const float sp = dt > 20.0f ? dt : log1pf(expf(dt));
        const float alpha = -expf(galog) * sp;
        sh.scal[0] = expf(alpha);
        sh.scal[1] = 1.0f / (1.0f + expf(-gb));
    }
    __syncthreads();

    dn_recurrence(sh, Sh, s, sh.scal[0], sh.scal[1]);

    // head RMSNorm (plain gain, attention.cpp:574-578) + SiLU(z) gate (:582-585)
    float o = 0.0f;
    if (wave < 2) {
        o = sh.vec[tid];
        const float ss = wave_sum(o * o);
        if (lane == 0) sh.scal[2 + wave] = ss;
    }
    __syncthreads();
    if (wave < 2) {
        const float tot = sh.scal[2] + sh.scal[3];
        const float sn = 1.0f / sqrtf(tot / (float)kD + 1e-6f);
        const float r = (o * sn) * nwj;
        out[(size_t)b * ldo + h * kD + tid] = r * silu_f(zj);
    }
}

// Column-split form of the decode mixer, for small batches: the 128 value
// columns of a head are spread over kSplit workgroups of kColW columns, so
// a batch-1 step runs H * kSplit workgroups instead of H (the recurrence is
// independent per value column j: kv[j], delta[j] and o[j] reduce over the
// key index i only, attention.cpp:513-569). Each workgroup recomputes the
// head's conv1d + SiLU + L2 norm of q and k (256 channels) and the gates,
// and owns its 16 v channels and the state columns [16 s, 16 s + 16) of all
// 128 rows. The head RMSNorm needs all 128 outputs, so it is left to the
// consumer: the workgroup writes u[j] = o[j] * w[j] * silu(z[j]) and the sum
// of o[j]^2 over its columns (ss[b, h, s]); the mixer output is
// u[j] / sqrt(sum_s ss[b, h, s] / d + 1e-6) (the out-projection GEMV applies
// it in its prologue).
//
// Every workgroup of a head reads the q/k channels' oldest ring row, which
// this step overwrites with the new input. The workgroup that overwrites it
// is the last one to have read it: each workgroup takes a ticket (one
// atomic add on ticket[b, h], each in a 128-byte line of its own: atomics
// on one line serialise) once its ring values have arrived and looks
// at it at its end; the one holding ticket kSplit - 1 (mod kSplit) writes
// the q/k ring row. No workgroup waits for another; the tickets stay a
// multiple of kSplit between launches (and wrap consistently, kSplit
// dividing 2^32). The L2 norms of q and k enter as the scalars 1/|q| and
// 1/|k| on the reductions (the reference divides each element; the same
// value to rounding).
//
// Thread (rg, j) owns state rows rg*8 .. rg*8+7 of column 16 s + j and
// computes one q or k channel of those rows (lanes j < 8 of its 16-lane row
// q, lanes j >= 8 k), so every q and k value a thread needs is a row
// broadcast away (DPP, no LDS): the sums of squares and the kv partial sums
// meet in one LDS round, the output sums in a second. Every thread forms
// its own column's v channel and the gates.
constexpr int kColW = 16;                       // value columns per workgroup
constexpr int kSplit = kD / kColW;              // workgroups per head
constexpr int kColThreads = 256;
constexpr int kColRG = kColThreads / kColW;     // row groups
constexpr int kColRows = kD / kColRG;           // state rows per thread
static_assert(kColRows == 8 && kColW == 16, "a row group is one 16-lane DPP row: 8 q + 8 k");
static_assert(kSplit % 8 == 0, "prefetching workgroups start on XCD 0");

// lane n of this lane's 16-lane row
template <int n>
__device__ __forceinline__ float row_lane(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + n, 0xf, 0xf, false));
}

__global__ __launch_bounds__(kColThreads) void k_deltanet_cols(
    const float* __restrict__ proj, int ldp, float* __restrict__ conv_state,
    const float* __restrict__ wt, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ norm_w,
    float* __restrict__ state, const int* __restrict__ pos, float* __restrict__ u, int ldu,
    float* __restrict__ ss, unsigned* __restrict__ ticket, int H, qlm_l2_plan plan) {
    // The mixer's arguments are read together with H, before the branch
    // below: otherwise the compiler reads H alone, branches, and only then
    // requests the rest, one more round trip before the first operand load.
    asm volatile("" ::"s"(proj), "s"(ldp), "s"(conv_state), "s"(wt), "s"(A_log), "s"(dt_bias),
                 "s"(norm_w), "s"(state), "s"(pos), "s"(u), "s"(ldu), "s"(ss), "s"(ticket));
    // workgroups past the mixer's carry out the L2 plan (B = 1: blockIdx.x
    // is the dispatch order; H * kSplit is a multiple of 8, so prefetching
    // workgroup p sits on XCD p % 8)
    if ((int)blockIdx.x >= H * kSplit) {
        const int p = (int)blockIdx.x - H * kSplit;
        l2_prefetch(plan, p % 8, p / 8, ((int)gridDim.x - H * kSplit) / 8);
        return;
    }
    constexpr int NWV = kColThreads / QLM_WAVE;
    __shared__ float red[NWV][kColW], red2[NWV][kColW];
    __shared__ float ssq[NWV][2];
    const int h = blockIdx.x / kSplit, sp = blockIdx.x % kSplit;
    const int b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int HD = H * kD;
    const int C = 3 * HD;
    const float* pr = proj + (size_t)b * ldp;
    float* cs = conv_state + (size_t)b * 3 * C;
    float* Sh = state + ((size_t)b * H + h) * kD * kD;
    const int j = tid & (kColW - 1), rg = tid / kColW;
    const int col = sp * kColW + j;  // value column of this thread
    const bool isk = j >= 8;

    // Operands, all unconditional: the position, this thread's q/k channel
    // (row rg*8 + j%8 of q or k), the v channel of column col, z, gain and
    // gates, then the state slice rows rg*8 .. rg*8+7 of column col.
    const int pb = *(pos ? pos + b : &g_pos_zero);
    const int chqk = (isk ? HD : 0) + h * kD + rg * kColRows + (j & 7);
    const int chv = 2 * HD + h * kD + col;
    float rq[3], wq[4], rv[3], wv[4];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        rq[t] = cs[(size_t)t * C + chqk];
        rv[t] = cs[(size_t)t * C + chv];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        wq[t] = wt[(size_t)t * C + chqk];
        wv[t] = wt[(size_t)t * C + chv];
    }
    const float xq = pr[chqk], xv = pr[chv];
    const float zj = pr[3 * HD + h * kD + col];
    const float nwj = norm_w[col];
    const float ga = pr[4 * HD + H + h], gb = pr[4 * HD + h];
    const float gdt = dt_bias[h], galog = A_log[h];
    float sr[kColRows];
#pragma unroll
    for (int r = 0; r < kColRows; ++r) sr[r] = Sh[(size_t)(rg * kColRows + r) * kD + col];

    // conv1d (taps chronological from the oldest ring row) + SiLU
    const int oldest = pb % 3;
    auto conv = [&](const float (&ring)[3], const float (&w)[4], float x) {
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            const int row = (oldest + t) % 3;
            const float r = row == 0 ? ring[0] : (row == 1 ? ring[1] : ring[2]);
            acc = nc_add_mul(acc, r, w[t]);
        }
        acc = nc_add_mul(acc, x, w[3]);
        return silu_f(acc);
    };
    const float yq = conv(rq, wq, xq);
    const float yv = conv(rv, wv, xv);
    // gates (attention.cpp:472-483), in every thread
    const float dt = ga + gdt;
    const float spl = dt > 20.0f ? dt : log1pf(expf(dt));
    const float dec = expf(-expf(galog) * spl);
    const float beta = 1.0f / (1.0f + expf(-gb));

    // this row group's k and q values
    float kr[kColRows], qr[kColRows];
    kr[0] = row_lane<8>(yq);
    kr[1] = row_lane<9>(yq);
    kr[2] = row_lane<10>(yq);
    kr[3] = row_lane<11>(yq);
    kr[4] = row_lane<12>(yq);
    kr[5] = row_lane<13>(yq);
    kr[6] = row_lane<14>(yq);
    kr[7] = row_lane<15>(yq);
    qr[0] = row_lane<0>(yq);
    qr[1] = row_lane<1>(yq);
    qr[2] = row_lane<2>(yq);
    qr[3] = row_lane<3>(yq);
    qr[4] = row_lane<4>(yq);
    qr[5] = row_lane<5>(yq);
    qr[6] = row_lane<6>(yq);
    qr[7] = row_lane<7>(yq);

    // (1) decay and kv[col] = k . S_decayed[:, col] (k not yet normalised),
    // with the wave's q and k sums of squares
    float kv = 0.0f;
#pragma unroll
    for (int r = 0; r < kColRows; ++r) {
        sr[r] *= dec;
        kv = fmaf(kr[r], sr[r], kv);
    }
    // the 4 row groups of a wave share column j at lanes j, j+16, j+32, j+48
    kv = xor32_add(xor16_add(kv));
    const float sq = wave_sum(isk ? 0.0f : yq * yq), sk = wave_sum(isk ? yq * yq : 0.0f);
    if (lane < kColW) red[wave][lane] = kv;
    if (lane == 0) {
        ssq[wave][0] = sq;
        ssq[wave][1] = sk;
    }
    __syncthreads();  // every thread's ring values have arrived
    if (tid < kColW) cs[(size_t)oldest * C + chv] = xv;  // this workgroup's own v channels
    // Ticket, taken now; its value is needed only at the end. The workgroup
    // drawing the last ticket of the head overwrites the q/k ring row.
    unsigned t0 = 0;
    if (tid == 0) t0 = atomicAdd(&ticket[((size_t)b * H + h) * QLM_DN_TICKET_STRIDE], 1u);
    const float rqn = 1.0f / sqrtf(((ssq[0][0] + ssq[1][0]) + (ssq[2][0] + ssq[3][0])) + 1e-6f);
    const float rkn = 1.0f / sqrtf(((ssq[0][1] + ssq[1][1]) + (ssq[2][1] + ssq[3][1])) + 1e-6f);
    const float dj = yv - ((red[0][j] + red[1][j]) + (red[2][j] + red[3][j])) * rkn;

    // (2) S += (beta k) delta^T ; (3) o[col] = q . S_new[:, col]
    const float bk = beta * rkn;
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < kColRows; ++r) {
        const int i = rg * kColRows + r;
        sr[r] = fmaf(bk * kr[r], dj, sr[r]);
        o = fmaf(qr[r], sr[r], o);
        Sh[(size_t)i * kD + col] = sr[r];
    }
    o = xor32_add(xor16_add(o));
    if (lane < kColW) red2[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        float oj = 0.0f;
        if (lane < kColW) {
            oj = ((red2[0][lane] + red2[1][lane]) + (red2[2][lane] + red2[3][lane])) *
                 (rqn * (1.0f / sqrtf((float)kD)));
            u[(size_t)b * ldu + h * kD + col] = (oj * nwj) * silu_f(zj);
        }
        const float sq2 = group_sum<kColW>(oj * oj);
        if (lane == 0) ss[((size_t)b * H + h) * kSplit + sp] = sq2;
        // the last workgroup of the head to have read the q/k ring row
        // overwrites it with this step's inputs (lane l copies 4 of the 256)
        t0 = __shfl(t0, 0, QLM_WAVE);
        if (t0 % kSplit == kSplit - 1) {
            const int c = h * kD + (lane & 31) * 4 + (lane < 32 ? 0 : HD);
            *reinterpret_cast<float4*>(cs + (size_t)oldest * C + c) =
                *reinterpret_cast<const float4*>(pr + c);
        }
    }
}

// Column split of the isolated step, for few (sequence, head) pairs: the
// 128 value columns of a head over kSplit workgroups of kColW columns (the
// recurrence is independent per value column, attention.cpp:513-569), so
// B = 1 x 32 heads runs 256 workgroups instead of 32. Thread (rg, j) owns
// rows rg*8 .. rg*8+7 of column 16 s + j; the sums over rows meet by lane
// shuffles within a wave and through LDS across the 4 waves.
__global__ __launch_bounds__(kColThreads) void k_gated_delta_step_cols(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ decay, const float* __restrict__ beta, float* __restrict__ state,
    float* __restrict__ out, int H) {
    constexpr int NWV = kColThreads / QLM_WAVE;
    __shared__ float qs[kD], ks[kD], dl[kColW];
    __shared__ float red[NWV][kColW];
    const int bh = blockIdx.x / kSplit, sp = blockIdx.x % kSplit;  // bh = b*H + h
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = tid & (kColW - 1), rg = tid / kColW;
    const int col = sp * kColW + j;
    float* Sh = state + (size_t)bh * kD * kD;
    // operands, unconditional: this thread's q or k element, v of its
    // column, the gates, then its state rows
    const float qk = tid < kD ? q[(size_t)bh * kD + tid] : k[(size_t)bh * kD + tid - kD];
    const float vj = v[(size_t)bh * kD + col];
    const float dec = decay[bh], bt = beta[bh];
    float sr[kColRows];
#pragma unroll
    for (int r = 0; r < kColRows; ++r) sr[r] = Sh[(size_t)(rg * kColRows + r) * kD + col];
    if (tid < kD) qs[tid] = qk;
    else ks[tid - kD] = qk;
    __syncthreads();
    // (1) decay and kv[col] = k . S_decayed[:, col]
    float kv = 0.0f;
#pragma unroll
    for (int r = 0; r < kColRows; ++r) {
        sr[r] *= dec;
        kv = fmaf(ks[rg * kColRows + r], sr[r], kv);
    }
    kv = xor32_add(xor16_add(kv));
    if (lane < kColW) red[wave][lane] = kv;
    __syncthreads();
    if (tid < kColW) dl[tid] = vj - ((red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]));
    __syncthreads();
    // (2) S += (beta k) delta^T ; (3) o[col] = q . S_new[:, col]
    const float dj = dl[j];
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < kColRows; ++r) {
        const int i = rg * kColRows + r;
        sr[r] = fmaf(bt * ks[i], dj, sr[r]);
        o = fmaf(qs[i], sr[r], o);
        Sh[(size_t)i * kD + col] = sr[r];
    }
    o = xor32_add(xor16_add(o));
    if (lane < kColW) red[wave][lane] = o;  // red's kv sums were read before the last barrier
    __syncthreads();
    if (tid < kColW)
        out[(size_t)bh * kD + col] = ((red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid])) *
                                     (1.0f / sqrtf((float)kD));
}

// Prefill of one sequence over T consecutive rows of proj (positions
// p0 .. p0+T-1), one workgroup per head: the reference processes the rows of
// a prompt one after another through the same recurrence
// (Qwen3_5GatedDeltaNet::forward_chunk, attention.cpp:600-758), and so does
// this kernel, with the decode step's arithmetic (bit-identical to T calls of
// k_deltanet_decode). The head's state slice and its conv ring live in
// registers for all T steps and are written back once; each row's operands
// are requested while the previous row is being processed.
__global__ __launch_bounds__(kThreads) void k_deltanet_prefill(
    const float* __restrict__ proj, int ldp, int T, float* __restrict__ conv_state,
    const float* __restrict__ wt, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* __restrict__ norm_w,
    float* __restrict__ state, int p0, float* __restrict__ out, int ldo, int H) {
    __shared__ DnShared sh;
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int HD = H * kD;
    const int C = 3 * HD;
    float* Sh = state + (size_t)h * kD * kD;

    float4 s[kRowsPer];
    dn_load_state(Sh, s);
    const bool conv_t = tid < 3 * kD;
    const int sec = tid / kD, t = tid % kD;
    const int ch = sec * HD + h * kD + t;
    // ring in chronological order: r0 = x[p-3], r1 = x[p-2], r2 = x[p-1]
    float w4[4] = {0.f, 0.f, 0.f, 0.f}, r0 = 0.f, r1 = 0.f, r2 = 0.f;
    if (conv_t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w4[j] = wt[(size_t)j * C + ch];
        r0 = conv_state[(size_t)(p0 % 3) * C + ch];
        r1 = conv_state[(size_t)((p0 + 1) % 3) * C + ch];
        r2 = conv_state[(size_t)((p0 + 2) % 3) * C + ch];
    }
    const bool gate_t = wave == 2 && lane == 0;
    const float gdt = gate_t ? dt_bias[h] : 0.0f, galog = gate_t ? A_log[h] : 0.0f;
    const float nwj = tid < kD ? norm_w[tid] : 0.0f;

    float xin = 0.f, ga = 0.f, gb = 0.f, zj = 0.f;
    auto fetch = [&](int row) {
        const float* pr = proj + (size_t)row * ldp;
        if (conv_t) xin = pr[ch];
        if (gate_t) {
            ga = pr[4 * HD + H + h];
            gb = pr[4 * HD + h];
        }
        if (tid < kD) zj = pr[3 * HD + h * kD + tid];
    };
    fetch(0);
    for (int r = 0; r < T; ++r) {
        const float xc = xin, gac = ga, gbc = gb, zc = zj;
        if (r + 1 < T) fetch(r + 1);

        if (conv_t) {
            float acc = 0.0f;
            acc = nc_add_mul(acc, r0, w4[0]);
            acc = nc_add_mul(acc, r1, w4[1]);
            acc = nc_add_mul(acc, r2, w4[2]);
            acc = nc_add_mul(acc, xc, w4[3]);
            r0 = r1;
            r1 = r2;
            r2 = xc;
            const float y = silu_f(acc);
            if (sec == 0) sh.q[t] = y;
            else if (sec == 1) sh.k[t] = y;
            else sh.v[t] = y;
        }
        __syncthreads();

        if (wave < 2) {
            float* vv = wave == 0 ? sh.q : sh.k;
            const float a0 = vv[lane], a1 = vv[lane + 64];
            float ss = fmaf(a0, a0, a1 * a1);
            ss = wave_sum(ss);
            const float nrm = sqrtf(ss + 1e-6f);
            vv[lane] = a0 / nrm;
            vv[lane + 64] = a1 / nrm;
        } else if (gate_t) {
            const float dt = gac + gdt;
            const float sp = dt > 20.0f ? dt : log1pf(expf(dt));
            const float alpha = -expf(galog) * sp;
            sh.scal[0] = expf(alpha);
            sh.scal[1] = 1.0f / (1.0f + expf(-gbc));
        }
        __syncthreads();

        dn_recurrence(sh, nullptr, s, sh.scal[0], sh.scal[1]);

        float o = 0.0f;
        if (wave < 2) {
            o = sh.vec[tid];
            const float ss = wave_sum(o * o);
            if (lane == 0) sh.scal[2 + wave] = ss;
        }
        __syncthreads();
        if (wave < 2) {
            const float tot = sh.scal[2] + sh.scal[3];
            const float sn = 1.0f / sqrtf(tot / (float)kD + 1e-6f);
            const float rr = (o * sn) * nwj;
            out[(size_t)r * ldo + h * kD + tid] = rr * silu_f(zc);
        }
    }

    // state and ring as the decode step expects them at position p0 + T
    float4* S4 = reinterpret_cast<float4*>(Sh);
    const int jg = tid & 31, ig = tid >> 5;
#pragma unroll
    for (int rr = 0; rr < kRowsPer; ++rr) S4[(ig * kRowsPer + rr) * (kD / 4) + jg] = s[rr];
    if (conv_t) {
        const int p = p0 + T;
        conv_state[(size_t)(p % 3) * C + ch] = r0;
        conv_state[(size_t)((p + 1) % 3) * C + ch] = r1;
        conv_state[(size_t)((p + 2) % 3) * C + ch] = r2;
    }
}

}  // namespace

extern "C" int qlm_gated_delta_step(const float* q, const float* k, const float* v,
                                    const float* decay, const float* beta, float* state,
                                    float* out, int B, int H, int d, void* stream) {
    if (!q || !k || !v || !decay || !beta || !state || !out || B <= 0 || H <= 0)
        return QLM_ERR_ARG;
    if (d != kD) return QLM_ERR_SHAPE;
    // few (sequence, head) pairs: the column split keeps more of the GPU busy
    // (measured at 32 heads: B = 1 and 4 faster split, B >= 8 one workgroup
    // a head)
    if (B <= 4)
        hipLaunchKernelGGL(k_gated_delta_step_cols, dim3(B * H * kSplit), dim3(kColThreads), 0,
                           as_stream(stream), q, k, v, decay, beta, state, out, H);
    else
        hipLaunchKernelGGL(k_gated_delta_step, dim3(B * H), dim3(kThreads), 0, as_stream(stream),
                           q, k, v, decay, beta, state, out, H);
    return qlm_launch_status();
}

extern "C" int qlm_deltanet_decode(const float* proj, int ldp, float* conv_state,
                                   const float* conv_w_t, const float* A_log, const float* dt_bias,
                                   const float* norm_w, float* state, const int* pos, float* out,
                                   int ldo, int B, int H, int d, void* stream) {
    if (!proj || !conv_state || !conv_w_t || !A_log || !dt_bias || !norm_w || !state || !out ||
        B <= 0 || H <= 0)
        return QLM_ERR_ARG;
    if (d != kD) return QLM_ERR_SHAPE;
    if (ldp < 4 * H * d + 2 * H || ldo < H * d) return QLM_ERR_SHAPE;
    hipLaunchKernelGGL(k_deltanet_decode, dim3(H, B), dim3(kThreads), 0, as_stream(stream), proj,
                       ldp, conv_state, conv_w_t, A_log, dt_bias, norm_w, state, pos, out, ldo, H);
    return qlm_launch_status();
}

extern "C" int qlm_deltanet_decode_cols_pf(const float* proj, int ldp, float* conv_state,
                                           const float* conv_w_t, const float* A_log,
                                           const float* dt_bias, const float* norm_w,
                                           float* state, const int* pos, float* u, int ldu,
                                           float* ss, unsigned* ticket, int B, int H, int d,
                                           const qlm_l2_plan* plan, void* stream) {
    if (!proj || !conv_state || !conv_w_t || !A_log || !dt_bias || !norm_w || !state || !u ||
        !ss || !ticket || B <= 0 || H <= 0)
        return QLM_ERR_ARG;
    if (d != kD) return QLM_ERR_SHAPE;
    if (ldp < 4 * H * d + 2 * H || ldu < H * d) return QLM_ERR_SHAPE;
    // the last workgroup copies the q/k inputs into the ring as float4
    if (ldp % 4 != 0 || (((uintptr_t)proj | (uintptr_t)conv_state) & 15u)) return QLM_ERR_SHAPE;
    qlm_l2_plan pl{};
    if (plan) {
        if (!l2_plan_valid(*plan)) return QLM_ERR_ARG;
        pl = *plan;
    }
    const int npf = l2_plan_workgroups(pl);
    if (npf > 0 && B != 1) return QLM_ERR_SHAPE;  // XCD placement assumes a 1-D grid
    hipLaunchKernelGGL(k_deltanet_cols, dim3(H * kSplit + npf, B), dim3(kColThreads), 0,
                       as_stream(stream), proj, ldp, conv_state, conv_w_t, A_log, dt_bias, norm_w,
                       state, pos, u, ldu, ss, ticket, H, pl);
    return qlm_launch_status();
}

extern "C" int qlm_deltanet_decode_cols(const float* proj, int ldp, float* conv_state,
                                        const float* conv_w_t, const float* A_log,
                                        const float* dt_bias, const float* norm_w, float* state,
                                        const int* pos, float* u, int ldu, float* ss,
                                        unsigned* ticket, int B, int H, int d, void* stream) {
    return qlm_deltanet_decode_cols_pf(proj, ldp, conv_state, conv_w_t, A_log, dt_bias, norm_w,
                                       state, pos, u, ldu, ss, ticket, B, H, d, nullptr, stream);
}

extern "C" int qlm_deltanet_prefill(const float* proj, int ldp, int T, float* conv_state,
                                    const float* conv_w_t, const float* A_log,
                                    const float* dt_bias, const float* norm_w, float* state,
                                    int p0, float* out, int ldo, int H, int d, void* stream) {
    if (!proj || !conv_state || !conv_w_t || !A_log || !dt_bias || !norm_w || !state || !out ||
        T <= 0 || H <= 0 || p0 < 0)
        return QLM_ERR_ARG;
    if (d != kD) return QLM_ERR_SHAPE;
    if (ldp < 4 * H * d + 2 * H || ldo < H * d) return QLM_ERR_SHAPE;
    hipLaunchKernelGGL(k_deltanet_prefill, dim3(H), dim3(kThreads), 0, as_stream(stream), proj,
                       ldp, T, conv_state, conv_w_t, A_log, dt_bias, norm_w, state, p0, out, ldo,
                       H);
    return qlm_launch_status();
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_deltanet() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(k_deltanet_cols));
}
