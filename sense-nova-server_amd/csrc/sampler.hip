// The device half of the reference's sampler (src/sampler.rs:98-141): the repetition / presence /
// frequency penalties on a logits row, then its k largest entries in the order top_k_small
// produces (value descending, index ascending among equal values), so that only k (token,
// logit) pairs leave the device.  Temperature, softmax, min-p, top-p and the draw run on the host
// over those pairs.
//
// Top-k: every entry becomes a 64-bit key (order-preserving bits of the value << 32 | ~index), so
// one descending sort of keys gives the reference's order.  Chunks of 4096 keys are sorted in LDS
// (bitonic, 1024 threads) and keep their first k; the survivors are sorted again in chunks until
// one chunk remains.  Every step is a fixed comparison network, so the result is deterministic.
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int kChunk = 4096, kSortThreads = 1024;

__device__ __forceinline__ uint32_t order_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// src/sampler.rs:99-106, applied to the row in place
__global__ __launch_bounds__(256) void penalty_kernel(float* logits, const uint32_t* tok, const uint32_t* cnt, int n,
                                                      int V, float rep, float presence, float frequency) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n || tok[i] >= (uint32_t)V) return;
    float l = logits[tok[i]];
    if (rep != 1.0f) l = l > 0.0f ? l / rep : l * rep;
    l = l - (presence + frequency * (float)cnt[i]);
    logits[tok[i]] = l;
}

__device__ __forceinline__ void bitonic_desc(unsigned long long* s) {
    const int tid = threadIdx.x;
    for (int size = 2; size <= kChunk; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kChunk / 2 / kSortThreads; ++q) {
                const int p = tid + q * kSortThreads;               // pair index
                const int i = 2 * p - (p & (stride - 1));            // lower element of the pair
                const int j = i + stride;
                const bool desc = (i & size) == 0;                   // direction of this run
                const unsigned long long a = s[i], b = s[j];
                if ((a < b) == desc) {
                    s[i] = b;
                    s[j] = a;
                }
            }
        }
    }
    __syncthreads();
}

// level 0: keys of logits[c*kChunk ..] sorted, the first k kept per chunk
__global__ __launch_bounds__(kSortThreads) void topk_logits_kernel(const float* logits, int V, int k,
                                                                   unsigned long long* out) {
    __shared__ unsigned long long s[kChunk];
    const int c = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < kChunk; e += kSortThreads) {
        const int i = c * kChunk + e;
        s[e] = i < V ? ((unsigned long long)order_bits(logits[i]) << 32) | (0xFFFFFFFFu - (uint32_t)i) : 0ull;
    }
    bitonic_desc(s);
    for (int e = tid; e < k; e += kSortThreads) out[(size_t)c * k + e] = s[e];
}

// later levels: n keys in chunks, the first k of each chunk kept
__global__ __launch_bounds__(kSortThreads) void topk_keys_kernel(const unsigned long long* in, int n, int k,
                                                                 unsigned long long* out) {
    __shared__ unsigned long long s[kChunk];
    const int c = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < kChunk; e += kSortThreads) {
        const int i = c * kChunk + e;
        s[e] = i < n ? in[i] : 0ull;
    }
    bitonic_desc(s);
    for (int e = tid; e < k; e += kSortThreads) out[(size_t)c * k + e] = s[e];
}

}  // namespace

size_t topk_scratch_keys(int V, int k) { return 2 * (size_t)((V + kChunk - 1) / kChunk) * k + kChunk; }

int launch_penalties(float* logits, int V, const uint32_t* tok, const uint32_t* cnt, int n, float rep, float presence,
                     float frequency, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(penalty_kernel, dim3((n + 255) / 256), dim3(256), 0, s, logits, tok, cnt, n, V, rep, presence,
                       frequency);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_topk(const float* logits, int V, int k, unsigned long long* scratch, unsigned long long** result,
                hipStream_t s) {
    if (k < 1 || k > kChunk / 2 || V < 1) return -1;
    unsigned long long* a = scratch;
    unsigned long long* b = scratch + (size_t)((V + kChunk - 1) / kChunk) * k;
    int chunks = (V + kChunk - 1) / kChunk;
    hipLaunchKernelGGL(topk_logits_kernel, dim3(chunks), dim3(kSortThreads), 0, s, logits, V, k, a);
    int n = chunks * k;
    while (chunks > 1) {
        chunks = (n + kChunk - 1) / kChunk;
        hipLaunchKernelGGL(topk_keys_kernel, dim3(chunks), dim3(kSortThreads), 0, s, a, n, k, b);
        n = chunks * k;
        unsigned long long* t = a;
        a = b;
        b = t;
    }
    *result = a;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
