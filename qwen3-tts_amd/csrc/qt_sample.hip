// qt_sample.hip — codec-token sampling on the device: the reference's qwen_tts_sample
// (qwen_tts_sampling.c:160-202) with its LCG state (sampling.c:38-49) as an argument, and
// optionally the codec-head rule in front of it (qwen_tts.c:1652-1679: clip to +-100,
// tokens >= 2048 except EOS masked, EOS masked for frames < 2, EOS boost).
//
// One 1024-thread workgroup; thread t owns the vocabulary entries 4t..4t+3 (n <= 4096), so
// every sum, scan and selection is a workgroup reduction instead of the reference's
// sequential loops:
//   repetition penalty   sequential over prev (a token listed twice is penalised twice)
//   greedy (temp < 1e-6) first index of the maximum
//   softmax              exp((l - max) * (1/temp)), / sum
//   top-k                radix select (4-bit digits, MSB first) of the k-th largest
//                        probability (with multiplicity, as the reference's quickselect),
//                        entries below it zeroed
//   top-p                bitonic sort of the nonzero probabilities by (probability desc,
//                        index asc), prefix sum over the sorted order, cutoff = first
//                        position whose prefix exceeds top_p, every later position zeroed
//   renormalise          / sum when the sum is positive
//   draw                 r = LCG; first index whose prefix sum (index order) exceeds r,
//                        else n - 1
// The sums run in a tree order where the reference runs (and, built with -ffast-math,
// vectorises) sequential loops, so a probability can differ in its last bits and a draw
// that lands within rounding of a cumulative boundary can pick the neighbouring token.
// Tied probabilities straddling the top-p cutoff keep the lowest indices (the reference's
// selection sort keeps the ties its swap history puts first).
#include "qt_device.h"

#define QS_T 1024
#define QS_NMAX 4096

struct QsArgs {
    const float *logits;
    int n, rule, frame;
    float eos_boost, temp;
    int top_k;
    float top_p, rep;
    const int *prev;
    int n_prev;
    uint32_t *seed;
    int *tok;
    int *done;      // nullable: once a token equal to EOS is drawn under the rule, later
                    // calls write EOS without drawing (the reference's loop ends there)
};

__device__ __forceinline__ void qs_put(const QsArgs &a, int t) {
    a.tok[0] = t;
    if (a.done && a.rule && t == 2150) a.done[0] = 1;
}

// total of v over the workgroup, in every thread (wave butterflies, then the 16 wave sums
// in wave order)
__device__ __forceinline__ float qs_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = group_sum<64>(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < QS_T / 64; w++) t += red[w];
    __syncthreads();
    return t;
}

// exclusive prefix of v over thread order
__device__ __forceinline__ float qs_scan_excl(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) red[wave] = x;
    const float ex = __shfl_up(x, 1, 64);
    __syncthreads();
    float base = 0.f;
    for (int w = 0; w < wave; w++) base += red[w];
    __syncthreads();
    return lane == 0 ? base : base + ex;
}

// smallest c over the workgroup (c = INT_MAX for none)
__device__ __forceinline__ int qs_min(int c, int *slot) {
    if (threadIdx.x == 0) *slot = 0x7FFFFFFF;
    __syncthreads();
    if (c != 0x7FFFFFFF) atomicMin(slot, c);
    __syncthreads();
    const int r = *slot;
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(QS_T) void k_sample(QsArgs a) {
    __shared__ float p[QS_NMAX];
    __shared__ unsigned long long srt[QS_NMAX];
    __shared__ float red[QS_T / 64];
    __shared__ unsigned hist[16];
    __shared__ int s_min;
    const int tid = threadIdx.x, n = a.n;
    if (a.done && a.done[0]) {           // uniform: every thread reads the same flag
        if (tid == 0) a.tok[0] = 2150;
        return;
    }

    // logits (and the codec-head rule) into LDS
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = 4 * tid + k;
        if (i >= n) continue;
        float v = a.logits[i];
        if (a.rule) {
            v = fminf(fmaxf(v, -100.0f), 100.0f);
            if (i >= 2048 && i != 2150) v = -1e30f;
            if (i == 2150) v = (a.frame < 2) ? -1e30f : __fadd_rn(v, a.eos_boost);
        }
        p[i] = v;
    }
    __syncthreads();
    if (a.rep != 1.0f && a.n_prev > 0) {
        if (tid == 0)
            for (int j = 0; j < a.n_prev; j++) {
                const int t = a.prev[j];
                if (t >= 0 && t < n) p[t] = p[t] > 0.f ? __fdiv_rn(p[t], a.rep) : __fmul_rn(p[t], a.rep);
            }
        __syncthreads();
    }
    float e[4];
#pragma unroll
    for (int k = 0; k < 4; k++) e[k] = (4 * tid + k < n) ? p[4 * tid + k] : -INFINITY;

    if (a.temp < 1e-6f) {
        // greedy: first index of the maximum
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (4 * tid + k < n && (e[k] > bv || bi == 0x7FFFFFFF)) { bv = e[k]; bi = 4 * tid + k; }
        const float m = group_max<64>(bv);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        float M = red[0];
        for (int w = 1; w < QS_T / 64; w++) M = fmaxf(M, red[w]);
        const int best = qs_min(bv == M ? bi : 0x7FFFFFFF, &s_min);
        if (tid == 0) qs_put(a, best == 0x7FFFFFFF ? 0 : best);
        return;
    }

    // softmax with temperature
    float m = fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3]));
    m = group_max<64>(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < QS_T / 64; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    const float inv = __fdiv_rn(1.0f, a.temp);
#pragma unroll
    for (int k = 0; k < 4; k++) e[k] = (4 * tid + k < n) ? expf(__fmul_rn(__fsub_rn(e[k], M), inv)) : 0.f;
    const float sum = qs_sum(((e[0] + e[1]) + e[2]) + e[3], red);
#pragma unroll
    for (int k = 0; k < 4; k++) e[k] = __fdiv_rn(e[k], sum);

    // top-k: the k-th largest probability by a 4-bit radix select on the bits (p >= 0)
    if (a.top_k > 0 && a.top_k < n) {
        unsigned prefix = 0, mask = 0;
        int kk = a.top_k;
        for (int sh = 28; sh >= 0; sh -= 4) {
            if (tid < 16) hist[tid] = 0;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const unsigned u = __float_as_uint(e[k]);
                if (4 * tid + k < n && (u & mask) == prefix) atomicAdd(&hist[(u >> sh) & 15u], 1u);
            }
            __syncthreads();
            int d = 15;
            for (; d > 0; d--) {
                if (kk <= (int)hist[d]) break;
                kk -= (int)hist[d];
            }
            prefix |= (unsigned)d << sh;
            mask |= 15u << sh;
            __syncthreads();
        }
        const float thr = __uint_as_float(prefix);
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (e[k] < thr) e[k] = 0.f;
    }

    // top-p over the probabilities sorted descending (ties: lower index first).  Only the
    // nonzero ones are sorted (compacted in index order; after top-k about k of them): a
    // zero adds nothing to the running sum, so the cutoff falls among them or nowhere.
    if (a.top_p < 1.0f && a.top_p > 0.0f) {
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) cnt += (4 * tid + k < n && e[k] > 0.f) ? 1 : 0;
        int at = (int)qs_scan_excl((float)cnt, red);        // exact: counts < 2^24
        const int nzc = (int)qs_sum((float)cnt, red);
        int np = 1;
        while (np < nzc) np <<= 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = 4 * tid + k;
            p[i] = e[k];
            if (i < n && e[k] > 0.f) srt[at++] = ((unsigned long long)__float_as_uint(e[k]) << 16) | (unsigned)(0xFFFF - i);
        }
        for (int i = nzc + tid; i < np; i += QS_T) srt[i] = 0ull;
        __syncthreads();
        for (int kb = 2; kb <= np; kb <<= 1)
            for (int j = kb >> 1; j > 0; j >>= 1) {
                for (int t = tid; t < np / 2; t += QS_T) {
                    const int i = 2 * j * (t / j) + (t % j), l = i + j;
                    const unsigned long long x = srt[i], y = srt[l];
                    if (((i & kb) == 0) ? (x < y) : (x > y)) { srt[i] = y; srt[l] = x; }
                }
                __syncthreads();
            }
        float c[4], run = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            run += (4 * tid + k < nzc) ? __uint_as_float((unsigned)(srt[4 * tid + k] >> 16)) : 0.f;
            c[k] = run;
        }
        const float base = qs_scan_excl(run, red);
        int cand = 0x7FFFFFFF;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (cand == 0x7FFFFFFF && 4 * tid + k < nzc && base + c[k] > a.top_p) cand = 4 * tid + k;
        const int first = qs_min(cand, &s_min);
        const int cutoff = first == 0x7FFFFFFF ? nzc : first + 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int s = 4 * tid + k;
            if (s >= cutoff && s < nzc) p[0xFFFF - (int)(srt[s] & 0xFFFFull)] = 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) e[k] = (4 * tid + k < n) ? p[4 * tid + k] : 0.f;
    }

    // renormalise and draw
    const float s2 = qs_sum(((e[0] + e[1]) + e[2]) + e[3], red);
    if (s2 > 0.f) {
#pragma unroll
        for (int k = 0; k < 4; k++) e[k] = __fdiv_rn(e[k], s2);
    }
    const uint32_t seed = *a.seed * 1103515245u + 12345u;
    const float r = (float)((seed >> 16) & 0x7FFFu) / 32768.0f;
    float c[4], run = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) { run += e[k]; c[k] = run; }
    const float base = qs_scan_excl(run, red);
    int cand = 0x7FFFFFFF;
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (cand == 0x7FFFFFFF && 4 * tid + k < n && r < base + c[k]) cand = 4 * tid + k;
    const int first = qs_min(cand, &s_min);
    if (tid == 0) {
        qs_put(a, first == 0x7FFFFFFF ? n - 1 : first);
        a.seed[0] = seed;
    }
}

extern "C" hipError_t qt_launch_sample(const float *logits, int n, int rule, int frame, float eos_boost, float temp,
                                       int top_k, float top_p, float rep, const int *prev, int n_prev,
                                       uint32_t *seed, int *tok, int *done, hipStream_t st) {
    if (n <= 0 || n > QS_NMAX || n_prev < 0 || (n_prev > 0 && !prev) || !seed || !tok || !logits ||
        (done && (!rule || n <= 2150)))
        return hipErrorInvalidValue;
    QsArgs a = {logits, n, rule, frame, eos_boost, temp, top_k, top_p, rep, prev, n_prev, seed, tok, done};
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(QS_T), 0, st, a);
    return hipGetLastError();
}
