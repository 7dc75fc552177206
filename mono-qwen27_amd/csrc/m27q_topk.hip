// m27q_topk.hip -- exact top-k (k <= 64) over a logits vector.
//
// Each candidate becomes a 64-bit key: the float mapped to an order-preserving
// unsigned (with -0.0 folded onto +0.0 and NaN below every number) in the high
// word, the bitwise-inverted index in the low word, so one descending order on
// keys is (value desc, index asc), all keys are distinct, and no key is 0
// (0 marks an empty slot).
//
// Selection is a radix select on the keys, 8 bits per pass from the top, with
// a 256-bin histogram in LDS: each pass narrows the prefix of the k-th largest
// key until the keys sharing it are exactly the ones still needed; the k keys
// at or above that prefix are then compacted.  Pass 1 (one workgroup per chunk
// of the vector) writes each chunk's top k; pass 2 (one workgroup) selects the
// top k of those and sorts them with a wavefront bitonic sort.
// Replaces the CPU selection of sample() (src/mono27b_chat.cpp:211-227) and
// k_argmax (exec:211-239).
#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

constexpr int kTopkBlock1 = 256;   // threads of a pass-1 workgroup
constexpr int kTopkBlock2 = 1024;  // threads of the pass-2 workgroup
constexpr int kTopkMaxK = 64;
constexpr int kTopkMaxChunks = 256;  // pass-2 capacity: 256 x 64 keys = 16 per thread

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t idx) {
    uint32_t o = 0u;  // NaN
    if (v == v) {
        const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
        o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return ((uint64_t)o << 32) | (uint64_t)(~idx);
}

struct SelectShared {
    uint32_t hist[256];
    uint32_t above[256];
    int need, done, count;
    uint64_t prefix, minkey;
    int shift;
};

// hist[bin] += 1 for every active lane.  Logits crowd into a few bins at the
// top digits, where plain LDS atomics on one address serialize lane by lane:
// the first lanes' bins are counted with one ballot each, the rest atomically.
__device__ __forceinline__ void hist_add(uint32_t *hist, bool active, uint32_t bin) {
    const int lane = (int)(threadIdx.x & (kWave - 1));
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const uint64_t m = __ballot(active);
        if (m == 0) return;  // wave-uniform
        const int leader = __ffsll((long long)m) - 1;
        const uint32_t lb = (uint32_t)__shfl((int)bin, leader, kWave);
        const bool same = active && bin == lb;
        const uint64_t sm = __ballot(same);
        if (lane == leader) atomicAdd(&hist[lb], (uint32_t)__popcll(sm));
        active = active && !same;
    }
    if (active) atomicAdd(&hist[bin], 1u);
}

// Select the k largest of the keys held by the block (KPT per thread, 0 =
// empty) and write them, in no particular order, to out[0..k); slots past the
// number of non-empty keys are written as 0.  With kth non-null, thread 0
// also writes the smallest selected key there (0 if fewer than k keys).
template <int KPT>
__device__ void block_select(const uint64_t (&key)[KPT], int k, uint64_t *out, SelectShared &sh,
                             uint64_t *kth = nullptr) {
    const int t = (int)threadIdx.x, nth = (int)blockDim.x;
    // number of non-empty keys
    if (t == 0) {
        sh.count = 0;
        sh.prefix = 0;
        sh.shift = 64;
        sh.done = 0;
    }
    __syncthreads();
    int mine = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j) mine += key[j] != 0;
    if (mine) atomicAdd(&sh.count, mine);
    __syncthreads();
    const int avail = sh.count;
    if (t == 0) sh.need = min(k, avail);
    __syncthreads();
    // Narrow the prefix of the need-th largest key, 8 bits at a time.
    for (int shift = 56; shift >= 0 && sh.need > 0 && !sh.done; shift -= 8) {
        for (int b = t; b < 256; b += nth) sh.hist[b] = 0;
        __syncthreads();
        const uint64_t pre = sh.prefix;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint64_t kk = key[j];
            const bool match = kk != 0 && (shift == 56 || (kk >> (shift + 8)) == (pre >> (shift + 8)));
            hist_add(sh.hist, match, (uint32_t)(kk >> shift) & 255u);
        }
        __syncthreads();
        if (t < 64) {  // one wave: suffix sums over the 256 bins (4 per lane, from the top)
            const int b0 = 255 - 4 * t;
            uint32_t c[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c[i] = sh.hist[b0 - i];
                s += c[i];
            }
            // inclusive scan of the lane totals over lanes 0..63 (bins from the top)
            uint32_t incl = s;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = __shfl_up(incl, d, 64);
                if (t >= d) incl += o;
            }
            uint32_t run = incl - s;  // keys in bins above b0
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
                if ((int)h == need - (int)a) sh.done = 1;  // every key of the bin is needed
            }
        }
        __syncthreads();
    }
    // Compact: keys whose top (64 - shift) bits are >= the prefix's (exactly
    // min(k, avail) of them).
    const uint64_t pre = sh.prefix;
    const int shift = sh.shift;
    if (t == 0) {
        sh.count = 0;
        sh.minkey = ~0ull;
    }
    __syncthreads();
    const int total = min(k, avail);
    uint64_t mn = ~0ull;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const uint64_t kk = key[j];
        const bool sel = kk != 0 && (shift >= 64 || (kk >> shift) >= (pre >> shift));
        if (sel) {
            const int slot = atomicAdd(&sh.count, 1);
            if (slot < total) out[slot] = kk;
            mn = kk < mn ? kk : mn;
        }
    }
    if (kth && mn != ~0ull) atomicMin((unsigned long long *)&sh.minkey, (unsigned long long)mn);
    for (int i = total + t; i < k; i += nth) out[i] = 0;
    __syncthreads();
    if (kth && t == 0) *kth = total == k ? sh.minkey : 0ull;
}

// Pass 1: workgroup g selects the top k of values [g * chunk, (g + 1) * chunk).
template <int KPT>
__global__ __launch_bounds__(kTopkBlock1) void k_topk_chunks(const float *__restrict__ v, int n, int k,
                                                             uint64_t *__restrict__ lists,
                                                             uint64_t *__restrict__ kth) {
    __shared__ SelectShared sh;
    const int chunk = KPT * kTopkBlock1;
    const long long base = (long long)blockIdx.x * chunk;
    uint64_t key[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const long long i = base + (long long)j * kTopkBlock1 + threadIdx.x;
        key[j] = i < n ? topk_key(v[i], (uint32_t)i) : 0ull;
    }
    block_select<KPT>(key, k, lists + (size_t)blockIdx.x * k, sh, kth + blockIdx.x);
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, mask, kWave);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), mask, kWave);
    return ((uint64_t)hi << 32) | lo;
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

// Pass 2: one workgroup selects the top k of the nchunks x k candidates and
// writes them in rank order.  A chunk's k-th key is a lower bound of the
// overall k-th key (that chunk alone holds k keys at or above it), so every
// candidate below the largest such bound is dropped before the selection.
__global__ __launch_bounds__(kTopkBlock2) void k_topk_final(const uint64_t *__restrict__ lists,
                                                            const uint64_t *__restrict__ kth, int nchunks, int k,
                                                            const float *__restrict__ v, int32_t *__restrict__ idx,
                                                            float *__restrict__ val) {
    constexpr int KPT = kTopkMaxChunks * kTopkMaxK / kTopkBlock2;  // 16
    __shared__ SelectShared sh;
    __shared__ uint64_t best[kTopkMaxK];
    __shared__ uint64_t bound;
    const int ncand = nchunks * k;
    uint64_t key[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const int i = j * kTopkBlock2 + (int)threadIdx.x;
        key[j] = i < ncand ? lists[i] : 0ull;
    }
    if (threadIdx.x == 0) bound = 0ull;
    __syncthreads();
    if ((int)threadIdx.x < nchunks) atomicMax((unsigned long long *)&bound, (unsigned long long)kth[threadIdx.x]);
    __syncthreads();
    const uint64_t lb = bound;
#pragma unroll
    for (int j = 0; j < KPT; ++j) key[j] = key[j] >= lb ? key[j] : 0ull;
    block_select<KPT>(key, k, best, sh);
    if (threadIdx.x < kWave) {
        const int lane = (int)threadIdx.x;
        const uint64_t s = wave_sort_desc(lane < k ? best[lane] : 0ull, lane);
        if (lane < k) {
            const uint32_t id = ~(uint32_t)s;
            idx[lane] = (int32_t)id;
            val[lane] = v[id];  // the original bits (keeps -0.0 and NaN payloads)
        }
    }
}

// Values per pass-1 workgroup: 1024 for the vocab (243 chunks), doubled until
// the chunks fit pass 2.
static int topk_kpt(int n) {
    for (int kpt = 4; kpt <= 64; kpt *= 2)
        if ((n + kpt * kTopkBlock1 - 1) / (kpt * kTopkBlock1) <= kTopkMaxChunks) return kpt;
    return 0;
}

int topk_max_n() { return 64 * kTopkBlock1 * kTopkMaxChunks; }

size_t topk_scratch_bytes(int n) {
    const int kpt = topk_kpt(n);
    if (!kpt) return 0;
    const int chunks = (n + kpt * kTopkBlock1 - 1) / (kpt * kTopkBlock1);
    return (size_t)chunks * (kTopkMaxK + 1) * sizeof(uint64_t);  // lists, then one k-th key per chunk
}

hipError_t launch_topk(const float *v, int n, int k, int32_t *idx, float *val, void *scratch, hipStream_t s) {
    const int kpt = topk_kpt(n);
    if (!kpt) return hipErrorInvalidValue;
    const int chunks = (n + kpt * kTopkBlock1 - 1) / (kpt * kTopkBlock1);
    uint64_t *lists = (uint64_t *)scratch;
    uint64_t *kth = lists + (size_t)chunks * kTopkMaxK;
    const dim3 g(chunks), b(kTopkBlock1);
    switch (kpt) {
        case 4: hipLaunchKernelGGL((k_topk_chunks<4>), g, b, 0, s, v, n, k, lists, kth); break;
        case 8: hipLaunchKernelGGL((k_topk_chunks<8>), g, b, 0, s, v, n, k, lists, kth); break;
        case 16: hipLaunchKernelGGL((k_topk_chunks<16>), g, b, 0, s, v, n, k, lists, kth); break;
        case 32: hipLaunchKernelGGL((k_topk_chunks<32>), g, b, 0, s, v, n, k, lists, kth); break;
        default: hipLaunchKernelGGL((k_topk_chunks<64>), g, b, 0, s, v, n, k, lists, kth); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_topk_final, dim3(1), dim3(kTopkBlock2), 0, s, lists, kth, chunks, k, v, idx, val);
    return hipGetLastError();
}

}  // namespace m27q
