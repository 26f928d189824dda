// The range exchange of a kernel that quantizes its own output: a producer of a
// DynamicQuantizeLinear's input whose blocks are all resident at once (one wave of blocks)
// can compute the per-tensor scale and zero point itself, once every block knows every
// other block's (min, max), and write the DQL's u8 output directly.
//
// Exchange buffer (kQoutSyncBytes, zeroed before its first use, left valid by every launch):
//   word 0    launch number E
//   word 1    blocks past the exchange (bits 0-15) and those whose wait ran out (bits 16-31)
//   word 2    launches that ended with a wait run out (sticky: only the host clears it, after
//             reading it, so a failure of any launch reaches the caller as an error status)
//   byte 256+ two 64-bit slots per block, min and max, each tagged with E + 1 in its high
//             half, so a reader takes a slot as this launch's as soon as it sees the tag
//             (zeroed memory never matches).
// Every block reads E before it publishes, and the last block past the exchange increments
// E, so all blocks of a launch agree on it.  Every access is a device-scope atomic (they
// bypass the per-XCD L2s); no release / acquire fences, whose per-block L2 write-back and
// invalidate cost more than the exchange.  Waits are bounded in time (the constant-rate
// wall clock, kExchangeWaitUs microseconds from the start of a block's wait): a block whose
// wait runs out must write its part of y as 0, and the last block past the exchange then writes the scale
// as NaN, so that every consumer shows the failure, and counts the launch in word 2.
//
// All blocks of a launch must be resident together for the waits to end in time.  The host
// sizes the launch from the occupancy calculator, which knows nothing of other kernels that
// may occupy CUs at the same time (another stream, another process): that is the case the
// bounded waits and word 2 exist for.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "dql_core.hpp"
#include "internal.hpp"

namespace icx {
namespace qx {

__device__ __forceinline__ unsigned long long* slots(unsigned* sync) {
    return reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(sync) + 256);
}

// E + 1 for this launch; read it early (before the main work) to hide the latency, in one
// thread of the block, and share it through LDS after a barrier: a read by every thread puts
// thousands of loads on one address at once, and since a wave's loads complete in issue
// order, that wave's later loads would wait behind the queue.
__device__ __forceinline__ unsigned read_tag(unsigned* sync) {
    return __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}

// Thread 0 of a block: publish the block's (min, max).
__device__ __forceinline__ void publish(unsigned* sync, unsigned tag, float mn, float mx) {
    const unsigned long long hi = (unsigned long long)tag << 32;
    unsigned long long* s = slots(sync) + 2 * blockIdx.x;
    __hip_atomic_store(s, hi | __float_as_uint(mn), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s + 1, hi | __float_as_uint(mx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// dql::block_minmax that also ORs `flag` over the block through the same LDS exchange and
// barrier (__syncthreads_or would add a barrier and, forming the block-linear thread id from
// all three work-item ids, keep the packed id register alive for the whole kernel).
template <int NT>
__device__ __forceinline__ bool block_minmax_any(float& mn, float& mx, int flag) {
    __shared__ float smn[NT / 64], smx[NT / 64];
    __shared__ int sfl[NT / 64];
    dql::wave_minmax(mn, mx);
    const int any = __any(flag) ? 1 : 0;
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        smn[wid] = mn;
        smx[wid] = mx;
        sfl[wid] = any;
    }
    __syncthreads();
    mn = smn[0];
    mx = smx[0];
    int f = sfl[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
        dql::acc_minmax(smn[w], mn, mx);
        dql::acc_minmax(smx[w], mn, mx);
        f |= sfl[w];
    }
    return f != 0;
}

// Every thread of a block of NT threads: wait for all gridDim.x blocks' pairs (thread t polls
// blocks t, t + NT, ...), fold them as the DQL launch does and return its parameters.
// `ok` is false in every thread if any wait of this block ran out: a thread gives up on the
// slots still untagged once `limit` ticks of the wall clock (wall_clock64, a constant-rate
// counter; the host converts microseconds with the device's rate) have passed since its
// wait began.  `tag` is the value published (read_tag); a test hook passes a tag that no
// block publishes instead.
template <int NT>
__device__ __forceinline__ dql::DqlParams gather(unsigned* sync, unsigned tag, unsigned long long limit,
                                                 bool& ok) {
    const unsigned long long* s = slots(sync);
    float mn = 0.0f, mx = 0.0f;
    int late = 0;
    const unsigned long long t0 = wall_clock64();
    for (int b = threadIdx.x; b < (int)gridDim.x; b += NT) {
        unsigned long long lo, hi;
        for (;;) {
            lo = __hip_atomic_load(s + 2 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            hi = __hip_atomic_load(s + 2 * b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((unsigned)(lo >> 32) == tag && (unsigned)(hi >> 32) == tag) break;
            if (late || wall_clock64() - t0 > limit) {
                late = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        dql::acc_minmax(__uint_as_float((uint32_t)lo), mn, mx);
        dql::acc_minmax(__uint_as_float((uint32_t)hi), mn, mx);
    }
    ok = !block_minmax_any<NT>(mn, mx, late);
    return dql::make_params(mn, mx);
}

// Thread 0 of a block, after its part of y is written: count the block out; the last one
// writes the scale and zero point (NaN and 0 if any wait ran out) and starts the next
// launch number.
__device__ __forceinline__ void finish(unsigned* sync, bool ok, const dql::DqlParams& p, float* y_scale,
                                       uint8_t* y_zp) {
    const unsigned old = __hip_atomic_fetch_add(sync + 1, ok ? 1u : 0x10001u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if ((old & 0xffffu) == gridDim.x - 1) {
        const bool err = !ok || (old >> 16) != 0;
        *y_scale = err ? __builtin_nanf("") : (float)p.s;
        *y_zp = err ? (uint8_t)0 : (uint8_t)p.zp;
        if (err) __hip_atomic_fetch_add(sync + kQoutErrWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(sync + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace qx
}  // namespace icx
