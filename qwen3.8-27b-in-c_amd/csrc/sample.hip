// Token sampling on the device: the reference sampler_sample (sampler.c:62-162)
// on device logits, for the non-speculative decode loop (main.c:232-248).
//
//   1. k_smp_select: block b stages logits [4096 b, 4096 b + 4096) in LDS as
//      64-bit keys (order-preserving value bits << 32 | ~index: larger value
//      first, then smaller index), applies the repeat penalty to the window
//      tokens that fall in its range (each token once per occurrence, in window
//      order, written back to the logits: the reference changes them in place)
//      and finds its K largest keys by radix select (8-bit digits from the top,
//      a 256-bin LDS histogram per digit, stopping as soon as the digit's bin
//      holds exactly the keys still needed).  The K keys leave unsorted, with
//      the smallest of them (the block's K-th).  When the lists of all blocks
//      exceed what the final block holds, the same kernel selects again over
//      the keys (groups of 4096).
//   2. k_smp_final: one block drops the keys below the largest block K-th
//      (the global K-th is at least that), selects the K largest the same way,
//      orders them by rank and runs the reference's arithmetic with its
//      results: K exponentials in parallel; the double sum (a tree when every
//      term is at least 2^-21, where every partial sum is exact, else in order
//      on one thread); the float scaling; the one float sequence of cumulative
//      sums that the nucleus cut, the total and the draw all use (one thread),
//      with the cut and the draw as first-index searches over it; the
//      xorshift64 draw (state in device memory).  Greedy (temp <= 0 or
//      top_k == 1) is the same pipeline with K = 1: the first maximum under
//      strict > (-0.0 and +0.0 compare equal, as there).
// The candidates are the reference's: the K largest logits in descending order.
// Where logits are exactly equal, the reference's order (and, at the K-th place,
// which of them it keeps) follows its heap and the C library's qsort; here equal
// values order by index.  The exponential is exp in double rounded once to float:
// the correctly rounded expf, which the C library's expf returns except within
// about 2^-34 of a rounding midpoint.  Logits are taken to be free of NaN.
#include <utility>

#include "qgpu_internal.h"

#define SMP_CHUNK 4096          // keys per selection block (4 per thread)
#define SMP_FINAL 16384         // keys the final block holds (16 per thread)
#define SMP_MAXK  256
#define SMP_MAXW  4096          // repeat-penalty window

namespace qg {
static uint64_t *ws_smp = nullptr;
static size_t ws_smp_keys = 0;
}

// Key 0 is padding: every key of a logit is non-zero (its low half is ~index).
static __device__ __forceinline__ uint64_t smp_key(float v, uint32_t i)
{
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0;                // -0.0 == +0.0
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)(0xFFFFFFFFu - i);
}
static __device__ __forceinline__ float key_val(uint64_t k)
{
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
static __device__ __forceinline__ uint32_t key_idx(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)k; }

struct SelShared {
    uint32_t hist[256];
    uint64_t prefix, mask, kmin, bound;
    int need, done;
    uint32_t nout, nreal;
};

// Radix select of the `want` largest non-zero keys among the E keys of every thread of the block
// (want <= the number of non-zero keys; non-zero keys are distinct).  8-bit digits from the top: a
// histogram of the digit over the keys that match the digits chosen so far, then the bin holding the
// want-th largest.  Stops when that bin holds exactly the keys still needed (at the latest on the last
// digit, where every bin holds at most one key).  The keys taken are the non-zero ones with
// (key & mask) >= prefix.
template <int E>
static __device__ void radix_select(const uint64_t (&k)[E], int want, SelShared &sh, uint64_t &prefix,
                                    uint64_t &mask)
{
    const int tid = threadIdx.x;
    prefix = 0;
    mask = 0;
    int need = want;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += blockDim.x) sh.hist[i] = 0;
        __syncthreads();
        for (int j = 0; j < E; j++)
            if (k[j] && (k[j] & mask) == prefix) atomicAdd(&sh.hist[(uint32_t)(k[j] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid < 64) {
            const int b0 = 255 - 4 * tid;       // lane l: bins 255-4l .. 252-4l, largest first
            uint32_t h[4];
            for (int j = 0; j < 4; j++) h[j] = sh.hist[b0 - j];
            const uint32_t sl = h[0] + h[1] + h[2] + h[3];
            uint32_t inc = sl;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(inc, o, 64);
                if (tid >= o) inc += t;
            }
            uint32_t above = inc - sl;          // keys in bins above this lane's
            if (above < (uint32_t)need && (uint32_t)need <= inc) {
                int j = 0;
                while (above + h[j] < (uint32_t)need) above += h[j++];
                const uint32_t left = (uint32_t)need - above;
                sh.prefix = prefix | ((uint64_t)(b0 - j) << shift);
                sh.mask = mask | (0xFFull << shift);
                sh.need = (int)left;
                sh.done = h[j] == left;
            }
        }
        __syncthreads();
        prefix = sh.prefix;
        mask = sh.mask;
        need = sh.need;
        if (sh.done) break;                     // the same value in every thread
    }
}

// Wave-aggregated LDS counters: one atomic per wave instead of one per lane (atomics of many lanes on
// one LDS word serialise).  Every lane of the wave calls these.
static __device__ __forceinline__ uint32_t wave_sum(uint32_t v)
{
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
static __device__ __forceinline__ uint64_t wave_min64(uint64_t v)
{
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)v, o, 64), hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
        v = min(v, ((uint64_t)hi << 32) | lo);
    }
    return v;
}
// the first of n consecutive slots of *ctr for this lane
static __device__ __forceinline__ uint32_t wave_alloc(uint32_t *ctr, uint32_t n)
{
    const int lane = threadIdx.x & 63;
    uint32_t inc = n;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    uint32_t base = 0;
    if (lane == 63 && inc) base = atomicAdd(ctr, inc);
    return __shfl(base, 63, 64) + inc - n;
}

// one wave: the largest of kth[0, n)
static __device__ uint64_t lists_bound(const uint64_t *__restrict__ kth, uint32_t n)
{
    uint64_t b = 0;
    for (uint32_t l = threadIdx.x; l < n; l += 64) b = max(b, kth[l]);
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)b, o, 64), hi = __shfl_xor((uint32_t)(b >> 32), o, 64);
        b = max(b, ((uint64_t)hi << 32) | lo);
    }
    return b;
}

struct SmpArgs {
    float *logits;              // first pass: the logits (penalised in place) ...
    const uint64_t *keys;       // ... or a later pass: the lists of the pass before
    const uint64_t *kth;        // later pass: the K-th largest key of each of those lists
    uint32_t nlists;
    uint32_t n;                 // logits or keys in all
    const uint32_t *tokens;     // penalty window tokens[w0, w0 + W) (first pass only)
    uint32_t w0, W;
    float penalty;
    int K;
};

// block b: the K largest keys of [4096 b, 4096 b + 4096) -> cand[K b, K b + K) (unsorted, zero-padded),
// and the smallest of them -> kth[b] (0 when the range holds fewer than K keys).  The K-th largest key
// over all ranges is at least the largest kth[b], so later selections drop every key below it.
__global__ __launch_bounds__(1024) void k_smp_select(const SmpArgs a, uint64_t *__restrict__ cand,
                                                     uint64_t *__restrict__ kth)
{
    __shared__ uint64_t s[SMP_CHUNK];
    __shared__ __align__(16) uint32_t win[SMP_MAXW];
    __shared__ uint32_t negz[SMP_CHUNK / 32];  // logits that are -0.0 (their keys are those of +0.0)
    __shared__ SelShared sh;
    const int tid = threadIdx.x;
    const uint32_t c0 = blockIdx.x * SMP_CHUNK;
    if (tid == 0) {
        sh.nout = sh.nreal = 0;
        sh.kmin = ~0ull;
    }
    for (int i = tid; i < SMP_CHUNK; i += 1024) {
        const uint32_t g = c0 + i;
        const float v = g < a.n && !a.keys ? a.logits[g] : 0.0f;
        s[i] = g >= a.n ? 0ull : a.keys ? a.keys[g] : smp_key(v, g);
        const uint64_t nz = __ballot(__float_as_uint(v) == 0x80000000u);   // lanes: i - lane .. i - lane + 63
        if ((tid & 63) == 0) {
            negz[i >> 5] = (uint32_t)nz;
            negz[(i >> 5) + 1] = (uint32_t)(nz >> 32);
        }
    }
    const uint32_t w4 = (a.W + 3) & ~3u;       // padding never equals a token below 2^24
    for (uint32_t t = tid; t < w4; t += 1024) win[t] = t < a.W ? a.tokens[a.w0 + t] : 0xFFFFFFFFu;
    if (a.keys && tid < 64) {                   // the largest K-th key of the lists bounds the selection
        const uint64_t b = lists_bound(a.kth, a.nlists);
        if (tid == 0) sh.bound = b;
    }
    __syncthreads();
    const uint64_t bound = a.keys ? sh.bound : 0ull;
    if (a.W) {
        // occurrence t of the window owns its token if no earlier occurrence has it; the owner
        // applies the penalty once per occurrence (sampler.c:65-77: x > 0 ? x / p : x * p)
        for (uint32_t t = tid; t < a.W; t += 1024) {
            const uint32_t tk = win[t];
            if (tk >= a.n || tk < c0 || tk >= c0 + SMP_CHUNK) continue;
            uint32_t before = 0, n = 0;           // occurrences ahead of t, from t on
            for (uint32_t u = 0; u < w4; u += 4) {
                const uint4 w = *(const uint4 *)&win[u];
                const uint32_t e4[4] = {w.x, w.y, w.z, w.w};
                for (int c = 0; c < 4; c++)
                    if (e4[c] == tk) {
                        if (u + c < t) before++;
                        else n++;
                    }
            }
            if (before) continue;
            const uint32_t e = tk - c0;
            float x = ((negz[e >> 5] >> (e & 31)) & 1u) ? -0.0f : key_val(s[e]);
            for (uint32_t r = 0; r < n; r++) x = x > 0.0f ? x / a.penalty : x * a.penalty;
            s[e] = smp_key(x, tk);
            a.logits[tk] = x;
        }
        __syncthreads();
    }
    uint64_t k[4];
    uint32_t cnt = 0;
    for (int j = 0; j < 4; j++) {
        k[j] = s[4 * tid + j];
        if (k[j] < bound) k[j] = 0;
        cnt += k[j] != 0;
    }
    cnt = wave_sum(cnt);
    if ((tid & 63) == 0) atomicAdd(&sh.nreal, cnt);
    __syncthreads();
    const int want = min(a.K, (int)sh.nreal);
    uint64_t prefix, mask;
    radix_select<4>(k, want, sh, prefix, mask);
    uint64_t *o = cand + (uint64_t)blockIdx.x * a.K;
    uint64_t mine = ~0ull;
    uint32_t nt = 0;
    for (int j = 0; j < 4; j++) nt += k[j] && (k[j] & mask) >= prefix;
    uint32_t slot = wave_alloc(&sh.nout, nt);
    for (int j = 0; j < 4; j++)
        if (k[j] && (k[j] & mask) >= prefix) {
            if (slot < (uint32_t)want) o[slot] = k[j];
            slot++;
            mine = min(mine, k[j]);
        }
    if (tid >= want && tid < a.K) o[tid] = 0ull;
    mine = wave_min64(mine);
    if ((tid & 63) == 0 && mine != ~0ull) atomicMin(&sh.kmin, mine);
    __syncthreads();
    if (tid == 0) kth[blockIdx.x] = want == a.K ? sh.kmin : 0ull;
}

// first index i < n (n <= 256) with pred, else `none`; every thread of the block calls it (each call
// site with its own slot: the slot is read after the last barrier)
static __device__ int block_first(bool pred, int n, int none, int *slot)
{
    const int tid = threadIdx.x;
    if (tid == 0) *slot = none;
    __syncthreads();
    const uint64_t m = __ballot(tid < n && pred);
    if ((tid & 63) == 0 && m) atomicMin(slot, (tid & ~63) + __builtin_ctzll(m));
    __syncthreads();
    return *slot;
}

// sampler.c:79-161 on the K largest of the M keys of cand (one block).  The cumulative sums of the
// reference's nucleus cut, its total and its draw are the one float sequence S_i = S_{i-1} + p_i,
// computed once; the cut and the draw are then first-index searches over it.
__global__ __launch_bounds__(1024) void k_smp_final(const uint64_t *__restrict__ cand, int M,
                                                    const uint64_t *__restrict__ kth, int K, int greedy,
                                                    float temp, float top_p, uint64_t *__restrict__ rng,
                                                    uint32_t *__restrict__ out)
{
#pragma clang fp contract(off)
    __shared__ SelShared sh;
    __shared__ uint64_t sel[SMP_MAXK], srt[SMP_MAXK];
    __shared__ __align__(16) float p[SMP_MAXK];
    __shared__ __align__(16) float ps[SMP_MAXK];
    __shared__ double part[4];
    __shared__ float inv_sh;
    __shared__ int first_cut, first_draw;
    const int tid = threadIdx.x;
    const uint64_t x0 = greedy ? 0ull : *rng;   // read before the one write at the end
    if (tid == 0) sh.nout = sh.nreal = 0;
    if (tid < 64) {
        const uint64_t b = lists_bound(kth, (uint32_t)(M / K));
        if (tid == 0) sh.bound = b;
    }
    uint64_t k[SMP_FINAL / 1024];
    for (int j = 0; j < SMP_FINAL / 1024; j++) {
        const int i = tid + 1024 * j;
        k[j] = i < M ? cand[i] : 0ull;
    }
    __syncthreads();
    uint32_t cnt = 0;
    for (int j = 0; j < SMP_FINAL / 1024; j++) {
        if (k[j] < sh.bound) k[j] = 0;
        cnt += k[j] != 0;
    }
    cnt = wave_sum(cnt);
    if ((tid & 63) == 0) atomicAdd(&sh.nreal, cnt);
    __syncthreads();
    const int want = min(K, (int)sh.nreal);
    uint64_t prefix, mask;
    radix_select<SMP_FINAL / 1024>(k, want, sh, prefix, mask);
    uint32_t nt = 0;
    for (int j = 0; j < SMP_FINAL / 1024; j++) nt += k[j] && (k[j] & mask) >= prefix;
    uint32_t slot = wave_alloc(&sh.nout, nt);
    for (int j = 0; j < SMP_FINAL / 1024; j++)
        if (k[j] && (k[j] & mask) >= prefix) {
            if (slot < (uint32_t)want) sel[slot] = k[j];
            slot++;
        }
    __syncthreads();
    if (tid < want) {                           // distinct keys: the rank is the sorted position
        const uint64_t key = sel[tid];
        int r = 0;
#pragma unroll 8
        for (int u = 0; u < want; u++) r += sel[u] > key;
        srt[r] = key;
    }
    __syncthreads();
    if (greedy) {
        if (tid == 0) *out = key_idx(srt[0]);
        return;
    }
    // p_i = expf(l_i / temp - l_0 / temp) (exp in double, rounded once)
    const float top = key_val(srt[0]) / temp;
    const float pv = tid < want ? (float)exp((double)(key_val(srt[tid]) / temp - top)) : 0.0f;
    if (tid < SMP_MAXK) p[tid] = pv;
    // the double sum: when every p_i >= 2^-21, each is a multiple of 2^-44 and every partial sum
    // (below 2^9) is exact in double, so any order gives the sequential sum; otherwise sequential
    if (__syncthreads_and(tid >= want || pv >= 0x1p-21f)) {
        if (tid < SMP_MAXK) {
            double d = pv;
            for (int o = 32; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
            if ((tid & 63) == 0) part[tid >> 6] = d;
        }
        __syncthreads();
        if (tid == 0) {
            const double sum = (part[0] + part[1]) + (part[2] + part[3]);
            inv_sh = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
        }
    } else if (tid == 0) {
        double sum = 0.0;
        for (int i = 0; i < want; i++) sum += p[i];
        inv_sh = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
    }
    __syncthreads();
    if (tid < want) p[tid] *= inv_sh;
    __syncthreads();
    if (tid == 0) {                             // S_i, four per load (p is zero past want)
        float c = 0.0f;
        for (int i = 0; i < want; i += 4) {
            const float4 v = *(const float4 *)&p[i];
            float4 o;
            c += v.x; o.x = c;
            c += v.y; o.y = c;
            c += v.z; o.z = c;
            c += v.w; o.w = c;
            *(float4 *)&ps[i] = o;
        }
    }
    __syncthreads();
    const float s_t = tid < want ? ps[tid] : 0.0f;
    // nucleus cut: the first i with S_i >= top_p, else the last candidate
    const int nc = top_p < 1.0f ? block_first(s_t >= top_p, want, want - 1, &first_cut) + 1 : want;
    const float tot = ps[nc - 1];
    uint64_t x = x0;                            // xorshift64 (sampler.c:8-15)
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    const float r = ((float)(x % 10000000) / 10000000.0f) * tot;
    // the draw: the first i < nc with S_i >= r, else the first candidate
    const int pick = block_first(s_t >= r, nc, 0x7FFFFFFF, &first_draw);
    if (tid == 0) {
        *rng = x;
        *out = key_idx(srt[pick == 0x7FFFFFFF ? 0 : pick]);
    }
}

extern "C" int qgpu_sample(float *logits, uint32_t vocab, const uint32_t *tokens, uint32_t n_tokens, float temp,
                           float top_p, uint32_t top_k, float repeat_penalty, uint32_t repeat_last_n,
                           uint64_t *rng_state, uint32_t *out_token)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!logits || !out_token || vocab < 1 || top_k < 1 || (n_tokens && !tokens)) return QGPU_E_ARG;
    if (vocab > (1u << 24)) return QGPU_E_RANGE;
    const bool greedy = temp <= 0.0f || top_k == 1;
    if (!greedy && !rng_state) return QGPU_E_ARG;
    uint32_t K = greedy ? 1 : (top_k < SMP_MAXK ? top_k : SMP_MAXK);
    if (K > vocab) K = vocab;
    SmpArgs a = {};
    a.logits = logits;
    a.n = vocab;
    a.K = (int)K;
    a.penalty = repeat_penalty;
    if (repeat_penalty != 1.0f && tokens && n_tokens) {
        a.tokens = tokens;
        a.w0 = n_tokens > repeat_last_n ? n_tokens - repeat_last_n : 0;
        a.W = n_tokens - a.w0;
        if (a.W > SMP_MAXW) return QGPU_E_RANGE;
    }
    const uint32_t nblk = (vocab + SMP_CHUNK - 1) / SMP_CHUNK;
    const size_t need = 2 * (size_t)nblk * (K + 1);     // two list buffers, two K-th key arrays
    if (need > qg::ws_smp_keys) {
        if (qg::ws_smp) {
            QG_CHECK(hipStreamSynchronize(qg::stream));
            QG_CHECK(hipFree(qg::ws_smp));
        }
        qg::ws_smp = nullptr;
        qg::ws_smp_keys = 0;
        QG_CHECK(hipMalloc(&qg::ws_smp, need * sizeof(uint64_t)));
        qg::ws_smp_keys = need;
    }
    uint64_t *c0 = qg::ws_smp, *c1 = c0 + (size_t)nblk * K, *m0 = c1 + (size_t)nblk * K, *m1 = m0 + nblk;
    hipLaunchKernelGGL(k_smp_select, dim3(nblk), dim3(1024), 0, qg::stream, a, c0, m0);
    QG_LAUNCH_CHECK();
    uint32_t n = nblk * K;
    while (n > SMP_FINAL) {                     // further passes over the lists (groups of 4096 keys)
        SmpArgs b = {};
        b.keys = c0;
        b.kth = m0;
        b.nlists = n / K;
        b.n = n;
        b.K = (int)K;
        const uint32_t nb = (n + SMP_CHUNK - 1) / SMP_CHUNK;
        hipLaunchKernelGGL(k_smp_select, dim3(nb), dim3(1024), 0, qg::stream, b, c1, m1);
        QG_LAUNCH_CHECK();
        std::swap(c0, c1);
        std::swap(m0, m1);
        n = nb * K;
    }
    hipLaunchKernelGGL(k_smp_final, dim3(1), dim3(1024), 0, qg::stream, c0, (int)n, m0, (int)K, greedy ? 1 : 0, temp,
                       top_p, rng_state, out_token);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}
