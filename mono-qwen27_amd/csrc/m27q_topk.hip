// m27q_topk.hip -- exact top-k (k <= 64) over a logits vector.
//
// Each candidate becomes a 64-bit key: the float mapped to an order-preserving
// unsigned (with -0.0 folded onto +0.0 and NaN below every number) in the high
// word, the bitwise-inverted index in the low word, so one descending order on
// keys is (value desc, index asc), all keys are distinct, and no key is 0
// (0 marks an empty slot).
//
// Three launches:
//   1. chunk maxima: workgroup c writes the largest key of its chunk;
//   2. filter: every workgroup takes T = the k-th largest chunk maximum (k
//      chunks hold a key >= T, so the k-th largest key overall is >= T) and
//      writes the keys >= T of its chunk to the chunk's own k candidate slots,
//      and their count beside them (no atomic across workgroups: one counter
//      serialized the workgroups' reservations);
//      A chunk with more than k such keys first reduces them to its own top k
//      (radix select within the workgroup);
//   3. select (one workgroup): the chunks' counts give each candidate its
//      place; with at most 1024 candidates (the usual case: about 75 for
//      248320 i.i.d. logits) each candidate's rank is counted directly and the
//      first k are written in rank order; with more, a radix select runs over
//      the candidate slots.
// Replaces the CPU selection of sample() (src/mono27b_chat.cpp:211-227) and
// k_argmax (exec:211-239).
#include <atomic>

#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

constexpr int kTopkBlock = 256;      // threads of a chunk workgroup
constexpr int kTopkSelBlock = 1024;  // threads of the select workgroup
constexpr int kTopkMaxK = 64;
constexpr int kTopkMaxChunks = 256;
constexpr int kTopkCap = kTopkMaxChunks * kTopkMaxK;  // candidate list capacity

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t idx) {
    uint32_t o = 0u;  // NaN
    if (v == v) {
        const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
        o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return ((uint64_t)o << 32) | (uint64_t)(~idx);
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, mask, kWave);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), mask, kWave);
    return ((uint64_t)hi << 32) | lo;
}

// Scratch layout: chunk maxima, each chunk's candidate count, each chunk's k
// candidate slots (chunk c: cand[c * k .. c * k + count[c])).
struct TopkScratch {
    uint64_t *maxkey;  // [kTopkMaxChunks]
    uint32_t *count;   // [kTopkMaxChunks]
    uint64_t *cand;    // [kTopkCap]
};
constexpr size_t kTopkScratchWords = (size_t)kTopkMaxChunks + kTopkMaxChunks / 2 + kTopkCap;
__host__ __device__ inline TopkScratch topk_scratch(void *base) {
    uint64_t *p = (uint64_t *)base;
    return {p, (uint32_t *)(p + kTopkMaxChunks), p + kTopkMaxChunks + kTopkMaxChunks / 2};
}

// 1. Largest key of each chunk.
__global__ __launch_bounds__(kTopkBlock) void k_topk_chunk_max(const float *__restrict__ v, int n, int chunk,
                                                               TopkScratch sc) {
    __shared__ uint64_t wmax[kTopkBlock / kWave];
    const long long base = (long long)blockIdx.x * chunk;
    const int end = (int)min((long long)n, base + chunk);
    uint64_t m = 0;
    // four independent loads per thread and round (a chunk of 1024 is one round)
    int i = (int)base + (int)threadIdx.x;
    for (; i + 3 * kTopkBlock < end; i += 4 * kTopkBlock) {
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = v[i + u * kTopkBlock];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint64_t key = topk_key(x[u], (uint32_t)(i + u * kTopkBlock));
            m = key > m ? key : m;
        }
    }
    for (; i < end; i += kTopkBlock) {
        const uint64_t key = topk_key(v[i], (uint32_t)i);
        m = key > m ? key : m;
    }
#pragma unroll
    for (int s = 1; s < kWave; s <<= 1) {
        const uint64_t o = shfl_xor64(m, s);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t r = wmax[0];
#pragma unroll
        for (int w = 1; w < kTopkBlock / kWave; ++w) r = wmax[w] > r ? wmax[w] : r;
        sc.maxkey[blockIdx.x] = r;
    }
}

struct SelectShared {
    uint32_t hist[256];
    uint32_t above[256];
    int need, done, count;
    uint64_t prefix;
    int shift;
};

// hist[bin] += 1 for every active lane; the first lanes' bins are counted with
// one ballot each (keys crowd into a few bins at the top digits), the rest with
// LDS atomics.
__device__ __forceinline__ void hist_add(uint32_t *hist, bool active, uint32_t bin) {
    const int lane = (int)(threadIdx.x & (kWave - 1));
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const uint64_t m = __ballot(active);
        if (m == 0) return;  // wave-uniform
        const int leader = __ffsll((long long)m) - 1;
        const uint32_t lb = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
        const bool same = active && bin == lb;
        const uint64_t sm = __ballot(same);
        if (lane == leader) atomicAdd(&hist[lb], (uint32_t)__popcll(sm));
        active = active && !same;
    }
    if (active) atomicAdd(&hist[bin], 1u);
}

// Radix select, 8 bits per pass from the top, over the keys get(0 .. count)
// (0 = empty), read again on every pass: writes the min(k, non-empty count)
// largest, in no particular order, to out[] and zeros to the rest of out[0..k).
template <class Get>
__device__ void block_select_stream(Get get, int count, int k, uint64_t *out, SelectShared &sh) {
    const int t = (int)threadIdx.x, nth = (int)blockDim.x;
    const int rounds = (count + nth - 1) / nth;  // same trip count for every lane (ballots)
    if (t == 0) {
        sh.count = 0;
        sh.prefix = 0;
        sh.shift = 64;
        sh.done = 0;
    }
    __syncthreads();
    int mine = 0;
    for (int r = 0; r < rounds; ++r) {
        const int i = r * nth + t;
        mine += i < count && get(i) != 0;
    }
    if (mine) atomicAdd(&sh.count, mine);
    __syncthreads();
    const int avail = sh.count;
    if (t == 0) sh.need = min(k, avail);
    __syncthreads();
    for (int shift = 56; shift >= 0 && sh.need > 0 && !sh.done; shift -= 8) {
        for (int b = t; b < 256; b += nth) sh.hist[b] = 0;
        __syncthreads();
        const uint64_t pre = sh.prefix;
        for (int r = 0; r < rounds; ++r) {
            const int i = r * nth + t;
            const uint64_t kk = i < count ? get(i) : 0ull;
            const bool match = kk != 0 && (shift == 56 || (kk >> (shift + 8)) == (pre >> (shift + 8)));
            hist_add(sh.hist, match, (uint32_t)(kk >> shift) & 255u);
        }
        __syncthreads();
        if (t < kWave) {  // suffix sums over the 256 bins, 4 per lane from the top
            const int b0 = 255 - 4 * t;
            uint32_t c[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c[i] = sh.hist[b0 - i];
                s += c[i];
            }
            uint32_t incl = s;
#pragma unroll
            for (int d = 1; d < kWave; d <<= 1) {
                const uint32_t o = __shfl_up(incl, d, kWave);
                if (t >= d) incl += o;
            }
            uint32_t run = incl - s;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sh.above[b0 - i] = run;
                run += c[i];
            }
        }
        __syncthreads();
        if (t < 256) {
            const int need = sh.need;
            const uint32_t a = sh.above[t], h = sh.hist[t];
            if ((int)a < need && need <= (int)(a + h)) {  // exactly one bin
                sh.prefix = pre | ((uint64_t)t << shift);
                sh.shift = shift;
                sh.need = need - (int)a;
                if ((int)h == need - (int)a) sh.done = 1;
            }
        }
        __syncthreads();
    }
    const uint64_t pre = sh.prefix;
    const int shift = sh.shift;
    if (t == 0) sh.count = 0;
    __syncthreads();
    const int total = min(k, avail);
    for (int r = 0; r < rounds; ++r) {
        const int i = r * nth + t;
        const uint64_t kk = i < count ? get(i) : 0ull;
        if (kk != 0 && (shift >= 64 || (kk >> shift) >= (pre >> shift))) {
            const int slot = atomicAdd(&sh.count, 1);
            if (slot < total) out[slot] = kk;
        }
    }
    for (int i = total + t; i < k; i += nth) out[i] = 0;
    __syncthreads();
}

// 2. Keys >= T of each chunk into its k candidate slots.  A chunk with more
// than k of them (ties, sorted input) contributes only its own top k.
__global__ __launch_bounds__(kTopkBlock) void k_topk_filter(const float *__restrict__ v, int n, int k, int chunk,
                                                            int nchunks, TopkScratch sc) {
    __shared__ uint64_t mk[kTopkMaxChunks];
    __shared__ uint64_t bound;
    __shared__ uint32_t local;
    __shared__ SelectShared sh;
    __shared__ uint64_t best[kTopkMaxK];
    const int t = (int)threadIdx.x;
    const int base = (int)blockIdx.x * chunk;
    const int len = min(n - base, chunk);
    // The chunk's first 4 x 256 values, loaded while T is found.
    float x0[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = t + u * kTopkBlock;
        x0[u] = i < len ? v[base + i] : 0.f;
    }
    // Slots past nchunks hold 0, which ranks below every key (no key is 0), so
    // the rank loop runs over all kTopkMaxChunks slots, fully unrolled, in
    // batches of 8 keys read while the previous batch is compared: with one
    // wave per SIMD nothing else hides the LDS latency (top-64 of 248320:
    // 11.1 us against 12.2 with a loop over nchunks, 11.6 fully unrolled
    // without the batches).
    static_assert(kTopkBlock == kTopkMaxChunks, "one thread per chunk-maximum slot");
    mk[t] = t < nchunks ? sc.maxkey[t] : 0ull;
    if (t == 0) {
        bound = 0ull;  // fewer than k chunks: no bound
        local = 0u;
    }
    __syncthreads();
    if (t < nchunks) {
        const uint64_t me = mk[t];
        constexpr int B = 8;
        static_assert(kTopkMaxChunks % (2 * B) == 0, "whole pairs of batches");
        uint64_t ka[B], kb[B];
        int rank = 0;
#pragma unroll
        for (int i = 0; i < B; ++i) ka[i] = mk[i];
#pragma unroll
        for (int j0 = 0; j0 < kTopkMaxChunks; j0 += 2 * B) {
#pragma unroll
            for (int i = 0; i < B; ++i) kb[i] = mk[j0 + B + i];
#pragma unroll
            for (int i = 0; i < B; ++i) rank += ka[i] > me;
            if (j0 + 2 * B < kTopkMaxChunks) {
#pragma unroll
                for (int i = 0; i < B; ++i) ka[i] = mk[j0 + 2 * B + i];
            }
#pragma unroll
            for (int i = 0; i < B; ++i) rank += kb[i] > me;
        }
        if (rank == k - 1) bound = me;  // the maxima are distinct keys: one thread
    }
    __syncthreads();
    const uint64_t T = bound;
    // Count, reserve, write (the chunk is L2-resident after the first sweep).
    uint32_t mine = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = t + u * kTopkBlock;
        mine += i < len && topk_key(x0[u], (uint32_t)(base + i)) >= T;
    }
    for (int i = t + 4 * kTopkBlock; i < len; i += kTopkBlock)
        mine += topk_key(v[base + i], (uint32_t)(base + i)) >= T;
    if (mine) atomicAdd(&local, mine);
    __syncthreads();
    const uint32_t found = local;
    __syncthreads();  // every thread has read local before it is reset
    if (found > (uint32_t)k) {
        block_select_stream(
            [&](int i) {
                const uint64_t key = topk_key(v[base + i], (uint32_t)(base + i));
                return key >= T ? key : 0ull;
            },
            len, k, best, sh);
        if (t < k) sc.cand[(size_t)blockIdx.x * k + t] = best[t];
        if (t == 0) sc.count[blockIdx.x] = (uint32_t)k;
        return;
    }
    if (t == 0) {
        sc.count[blockIdx.x] = found;
        local = 0u;
    }
    __syncthreads();
    if (!mine) return;
    uint32_t off = (uint32_t)blockIdx.x * (uint32_t)k + atomicAdd(&local, mine);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = t + u * kTopkBlock;
        const uint64_t key = topk_key(x0[u], (uint32_t)(base + i));
        if (i < len && key >= T) sc.cand[off++] = key;
    }
    for (int i = t + 4 * kTopkBlock; i < len; i += kTopkBlock) {
        const uint64_t key = topk_key(v[base + i], (uint32_t)(base + i));
        if (key >= T) sc.cand[off++] = key;
    }
}

// Sort one key per lane descending across the 64 lanes (bitonic).
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t key, int lane) {
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint64_t o = shfl_xor64(key, stride);
            const bool desc = (lane & size) == 0;
            const bool lower = (lane & stride) == 0;
            key = (lower == desc) ? (key > o ? key : o) : (key < o ? key : o);
        }
    }
    return key;
}

__device__ __forceinline__ void topk_emit(const float *v, uint64_t key, int rank, int32_t *idx, float *val) {
    const uint32_t id = ~(uint32_t)key;
    idx[rank] = (int32_t)id;
    val[rank] = v[id];  // the original bits (keeps -0.0 and NaN payloads)
}

// 3. The top k of the candidates (k <= their number <= nchunks * k).
__global__ __launch_bounds__(kTopkSelBlock) void k_topk_select(const float *__restrict__ v, int k, int nchunks,
                                                               TopkScratch sc, int32_t *__restrict__ idx,
                                                               float *__restrict__ val) {
    __shared__ uint64_t keys[kTopkSelBlock];
    __shared__ uint32_t cnt[kTopkMaxChunks], start[kTopkMaxChunks];
    __shared__ int total_s;
    __shared__ SelectShared sh;
    __shared__ uint64_t best[kTopkMaxK];
    const int t = (int)threadIdx.x;
    static_assert(kTopkSelBlock >= kTopkMaxChunks, "one thread per chunk count");
    static_assert(kTopkMaxChunks == 4 * kWave, "the prefix below runs on one wave, 4 chunks per lane");
    if (t < kTopkMaxChunks) cnt[t] = t < nchunks ? sc.count[t] : 0u;
    __syncthreads();
    if (t < kWave) {  // exclusive prefix of the counts, 4 chunks per lane
        uint32_t c[4], s4 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = cnt[4 * t + i];
            s4 += c[i];
        }
        uint32_t incl = s4;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t o = __shfl_up(incl, d, kWave);
            if (t >= d) incl += o;
        }
        uint32_t run = incl - s4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            start[4 * t + i] = run;
            run += c[i];
        }
        if (t == kWave - 1) total_s = (int)incl;
    }
    __syncthreads();
    const int total = total_s;
    if (total <= kTopkSelBlock) {
        keys[t] = 0ull;
        __syncthreads();
        if (t < nchunks)
            for (uint32_t i = 0; i < cnt[t]; ++i) keys[start[t] + i] = sc.cand[(size_t)t * k + i];
        __syncthreads();
        const uint64_t me = keys[t];
        if (t < total) {
            int rank = 0;
            for (int j = 0; j < total; ++j) rank += keys[j] > me;
            if (rank < k) topk_emit(v, me, rank, idx, val);
        }
        return;
    }
    const uint64_t *cand = sc.cand;
    block_select_stream([&](int i) { return (uint32_t)(i % k) < cnt[i / k] ? cand[i] : 0ull; }, nchunks * k, k,
                        best, sh);
    if (t < kWave) {
        const uint64_t s = wave_sort_desc(t < k ? best[t] : 0ull, t);
        if (t < k) topk_emit(v, s, t, idx, val);
    }
}

// Sampling from the top-k candidates, in the steps and order of sample()
// (src/mono27b_chat.cpp:203-270) after its top-k: probabilities
// e^((v_i - v_0) / T) computed per lane (exp_cw; 0 below e^-87, NaN kept),
// then one lane runs the sum, the normalization, the min_p and top_p cuts and
// the pick in candidate order, so the float sums round as the reference's
// sequential loop does.
__global__ __launch_bounds__(kWave) void k_sample(const int32_t *__restrict__ idx, const float *__restrict__ val,
                                                  int k, float temperature, float min_p, float top_p,
                                                  const float *__restrict__ u, int32_t *__restrict__ token) {
    __shared__ float p[kTopkMaxK];
    __shared__ int kept[kTopkMaxK];
    const int lane = (int)threadIdx.x;
    const int best = idx[0];
    if (!(temperature > 0.f)) {
        if (lane == 0) *token = best;
        return;
    }
    if (lane < k) {
        const float a = (val[lane] - val[0]) / temperature;
        p[lane] = a >= -87.0f ? exp_cw(a) : (a < -87.0f ? 0.0f : a);
    }
    __syncthreads();
    if (lane != 0) return;
    float sum = 0.f;
    for (int i = 0; i < k; ++i) sum += p[i];
    if (!(sum > 0.f) || !isfinite(sum)) {
        *token = best;
        return;
    }
    for (int i = 0; i < k; ++i) p[i] /= sum;
    // min_p: drop candidates below p_0 * min_p (kept in order); p_0 itself
    // always stays unless min_p > 1, and then the pick falls back to best.
    const float thresh = p[0] * min_p;
    int n = 0;
    for (int i = 0; i < k; ++i)
        if (!(p[i] < thresh)) kept[n++] = i;
    if (n == 0) {
        *token = best;
        return;
    }
    if (top_p < 1.f) {
        float acc = 0.f;
        for (int i = 0; i < n; ++i) {
            acc += p[kept[i]];
            if (acc >= top_p) {
                n = i + 1;
                break;
            }
        }
    }
    float total = 0.f;
    for (int i = 0; i < n; ++i) total += p[kept[i]];
    const float pick = *u * total;
    float run = 0.f;
    for (int i = 0; i < n; ++i) {
        run += p[kept[i]];
        if (pick <= run) {
            *token = idx[kept[i]];
            return;
        }
    }
    *token = idx[kept[n - 1]];
}

hipError_t launch_sample(const int32_t *idx, const float *val, int k, float temperature, float min_p, float top_p,
                         const float *u, int32_t *token, hipStream_t s) {
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(kWave), 0, s, idx, val, k, temperature, min_p, top_p, u, token);
    return hipGetLastError();
}

// Values per chunk workgroup: 1024 for the vocab (243 chunks), doubled until
// the chunk count fits.
static int topk_chunk(int n) {
    for (int c = 1024; c <= (1 << 16); c *= 2)
        if ((n + c - 1) / c <= kTopkMaxChunks) return c;
    return 0;
}

int topk_max_n() { return (1 << 16) * kTopkMaxChunks; }

size_t topk_scratch_bytes(int n) {
    if (!topk_chunk(n)) return 0;
    return kTopkScratchWords * sizeof(uint64_t);
}

// The library's own top-k scratch for callers that cannot allocate
// (m27q_topk_noalloc): one fixed-size array per device, held until the
// process ends.  Host code never passes the array's name to a kernel: its
// device address is resolved once per device with hipGetSymbolAddress and
// cached.  Every call on a device shares that device's array (every call
// writes each chunk's maximum, count and candidates before they are read), so
// calls that overlap on one device race.
static __device__ __align__(256) uint64_t scratch[kTopkScratchWords];

size_t topk_static_scratch_bytes() { return sizeof(scratch); }

hipError_t topk_static_scratch(void **ptr) {
    constexpr int kMaxDevices = 64;
    static std::atomic<void *> cache[kMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void *p = cache[dev].load(std::memory_order_acquire);
    if (!p) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        cache[dev].store(p, std::memory_order_release);
    }
    *ptr = p;
    return hipSuccess;
}

hipError_t launch_topk(const float *v, int n, int k, int32_t *idx, float *val, void *scratch, hipStream_t s) {
    const int chunk = topk_chunk(n);
    if (!chunk) return hipErrorInvalidValue;
    const int nchunks = (n + chunk - 1) / chunk;
    const TopkScratch sc = topk_scratch(scratch);
    hipLaunchKernelGGL(k_topk_chunk_max, dim3(nchunks), dim3(kTopkBlock), 0, s, v, n, chunk, sc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_topk_filter, dim3(nchunks), dim3(kTopkBlock), 0, s, v, n, k, chunk, nchunks, sc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_topk_select, dim3(1), dim3(kTopkSelBlock), 0, s, v, k, nchunks, sc, idx, val);
    return hipGetLastError();
}

}  // namespace m27q
