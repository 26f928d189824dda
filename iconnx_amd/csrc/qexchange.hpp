// The range exchange of a kernel that quantizes its own output: a producer of a
// DynamicQuantizeLinear's input whose blocks are all resident at once (one wave of blocks)
// can compute the per-tensor scale and zero point itself, once every block knows every
// other block's (min, max), and write the DQL's u8 output directly.
//
// Exchange buffer (kQoutSyncBytes, zeroed before its first use, left valid by every launch):
//   word 0      launch number E
//   word 2      launches that ended with a wait run out (sticky: only the host clears it,
//               after reading it, so a failure of any launch reaches the caller as an error
//               status)
//   bytes 128+  the launch's (min, max), two 64-bit words tagged with E + 1 in their high
//               halves, written by block 0
//   bytes 256+  two such tagged words per block: its own (min, max)
//   then        kGroups + 1 counters of published blocks, one per 128-byte line
//   then        one word per block, tagged E + 1 when the block's slice of a GEMM's
//               quantized input is in memory (the fused DQL + GEMM launch: the blocks of a
//               row panel wait for each other's slices before their main loop)
// A tag tells a reader that a word is this launch's as soon as it sees it (zeroed memory
// never matches), so nothing is cleared between launches.  Each block publishes its pair;
// block 0 alone polls all pairs (one round trip per round for the whole grid; polls by
// every block would cost G^2 loads a round), folds them, and publishes the result, which
// the other blocks poll.  The serial chain after the last block publishes is three round
// trips to memory: its pair reaching block 0's poll, the result reaching the others'.  A
// launch of at most 256 blocks may instead have every block poll and fold every pair (two
// round trips; gather's ALL).
//
// E must advance exactly once per launch, and only after every block has read it (a block
// that read the next launch's number would tag its pair with that launch's tag, and that
// launch could take the stale pair for a fresh one).  Every block reads E before it
// publishes and then counts itself into one of kGroups counters (same-address atomics
// serialise at the memory, ~8 ns each: one counter for 768 blocks would take microseconds);
// the last of a group counts the group into the top counter, and the last group's last
// block resets the counters and increments E.  This holds also when a block starts late.
//
// Every access is a device-scope atomic (they bypass the per-XCD L2s); no release /
// acquire fences, whose per-block L2 write-back and invalidate cost more than the exchange.
// Waits are bounded in time (the constant-rate wall clock, kExchangeWaitUs microseconds from
// the start of a block's wait).  A block whose wait runs out writes its part of y as 0 and
// counts itself in word 2; if block 0's wait runs out, it publishes a NaN range, which every
// other block takes as a failure, and writes the scale as NaN.
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

constexpr int kGroups = 8;
constexpr size_t kCountOff = 256 + 16 * (size_t)kQoutMaxBlocks;
constexpr size_t kPanelOff = kCountOff + 128 * (kGroups + 1);
static_assert(kPanelOff + 4 * (size_t)kQoutMaxBlocks == kQoutSyncBytes, "exchange buffer layout");

__device__ __forceinline__ unsigned long long* slots(unsigned* sync) {
    return reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(sync) + 256);
}
__device__ __forceinline__ unsigned long long* result(unsigned* sync) {
    return reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(sync) + 128);
}
__device__ __forceinline__ unsigned* counter(unsigned* sync, int k) {  // k < kGroups: group, kGroups: top
    return reinterpret_cast<unsigned*>(reinterpret_cast<char*>(sync) + kCountOff + 128 * k);
}
__device__ __forceinline__ unsigned* panel(unsigned* sync) {
    return reinterpret_cast<unsigned*>(reinterpret_cast<char*>(sync) + kPanelOff);
}

// E + 1 for this launch; read it early (before the main work) to hide the latency, in one
// thread of the block, and share it through LDS after a barrier: a read by every thread puts
// thousands of loads on one address at once, and since a wave's loads complete in issue
// order, that wave's later loads would wait behind the queue.
__device__ __forceinline__ unsigned read_tag(unsigned* sync) {
    return __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}

__device__ __forceinline__ unsigned long long tagged(unsigned tag, float v) {
    return ((unsigned long long)tag << 32) | __float_as_uint(v);
}

// Thread 0 of a block, after read_tag has returned: publish the block's (min, max), then
// count the block in; the last block of the launch starts the next launch number.
__device__ __forceinline__ void publish(unsigned* sync, unsigned tag, float mn, float mx) {
    unsigned long long* s = slots(sync) + 2 * blockIdx.x;
    __hip_atomic_store(s, tagged(tag, mn), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s + 1, tagged(tag, mx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned G = gridDim.x, g = blockIdx.x % kGroups;
    const unsigned gsize = (G - g + kGroups - 1) / kGroups, ngroups = G < kGroups ? G : kGroups;
    if (__hip_atomic_fetch_add(counter(sync, g), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gsize - 1) {
        __hip_atomic_store(counter(sync, g), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__hip_atomic_fetch_add(counter(sync, kGroups), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            ngroups - 1) {
            __hip_atomic_store(counter(sync, kGroups), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
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

// With ALL, grids of at most this many blocks fold every pair in every block (one round trip
// less after the last block publishes; at most 2 x 256 polled words per block per round).
// Measured: the one-launch DQL + GEMM 34.3 -> 33.7 us; the encoder's FFN-up, whose blocks
// reach the exchange while others still compute and store, ~0.5 us slower — it keeps the
// single folding block.
constexpr int kAllPollMax = 256;

// Every thread of a block of NT threads, after thread 0's publish: return the launch's DQL
// parameters.  Block 0 waits for all gridDim.x pairs tagged `want` (thread t polls blocks
// t, t + NT, ... together, so the wait after the last block publishes is one round trip),
// folds them as the DQL launch does and publishes the result tagged `tag`; the other blocks
// wait for that result — or, with ALL in a grid of at most kAllPollMax blocks, fold every
// pair themselves the same way (min and max are exact, so every block gets the same result).
// `ok` is false in every thread of a block whose wait ran out (a wait gives up once `limit`
// ticks of the wall clock, a constant-rate counter the host converts from microseconds with
// the device's rate, have passed since it began) and in every block when block 0's did.
// `want` is `tag` but for a test hook, which passes a tag that no block publishes.
template <int NT, bool ALL = false>
__device__ __forceinline__ dql::DqlParams gather(unsigned* sync, unsigned tag, unsigned want,
                                                 unsigned long long limit, bool& ok) {
    const bool all = ALL && (int)gridDim.x <= kAllPollMax;
    if (blockIdx.x == 0 || all) {
        constexpr int MAXS = (kQoutMaxBlocks + NT - 1) / NT;
        const unsigned long long* s = slots(sync);
        float mn = 0.0f, mx = 0.0f;
        int late = 0;
        unsigned pending = 0;
#pragma unroll
        for (int i = 0; i < MAXS; ++i)
            if ((int)threadIdx.x + i * NT < (int)gridDim.x) pending |= 1u << i;
        const unsigned long long t0 = wall_clock64();
        while (pending) {
            unsigned long long lo[MAXS], hi[MAXS];
#pragma unroll
            for (int i = 0; i < MAXS; ++i) {
                if (pending & (1u << i)) {
                    const int b = threadIdx.x + i * NT;
                    lo[i] = __hip_atomic_load(s + 2 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    hi[i] = __hip_atomic_load(s + 2 * b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
#pragma unroll
            for (int i = 0; i < MAXS; ++i) {
                if ((pending & (1u << i)) && (unsigned)(lo[i] >> 32) == want && (unsigned)(hi[i] >> 32) == want) {
                    dql::acc_minmax(__uint_as_float((uint32_t)lo[i]), mn, mx);
                    dql::acc_minmax(__uint_as_float((uint32_t)hi[i]), mn, mx);
                    pending &= ~(1u << i);
                }
            }
            if (!pending) break;
            if (wall_clock64() - t0 > limit) {
                late = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        ok = !block_minmax_any<NT>(mn, mx, late);
        if (blockIdx.x == 0 && !all && threadIdx.x == 0) {
            const float nan = __builtin_nanf("");
            unsigned long long* r = result(sync);
            __hip_atomic_store(r, tagged(tag, ok ? mn : nan), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(r + 1, tagged(tag, ok ? mx : nan), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return dql::make_params(mn, mx);
    }
    __shared__ float s_mn, s_mx;
    __shared__ int s_ok;
    if (threadIdx.x == 0) {
        const unsigned long long* r = result(sync);
        unsigned long long r0 = 0, r1 = 0;
        int good = 0;
        const unsigned long long t0 = wall_clock64();
        for (;;) {
            r0 = __hip_atomic_load(r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            r1 = __hip_atomic_load(r + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((unsigned)(r0 >> 32) == tag && (unsigned)(r1 >> 32) == tag) {
                good = 1;
                break;
            }
            if (wall_clock64() - t0 > limit) break;
            __builtin_amdgcn_s_sleep(1);
        }
        const float mn = __uint_as_float((uint32_t)r0), mx = __uint_as_float((uint32_t)r1);
        good = good && mn == mn && mx == mx;  // block 0 publishes NaN when its wait ran out
        s_mn = good ? mn : 0.0f;
        s_mx = good ? mx : 0.0f;
        s_ok = good;
    }
    __syncthreads();
    ok = s_ok != 0;
    return dql::make_params(s_mn, s_mx);
}

// Thread 0 of a block, after its part of y is written: a block whose wait ran out counts
// itself in the error word; block 0 writes the scale and zero point (NaN and 0 if its wait
// ran out).
__device__ __forceinline__ void finish(unsigned* sync, bool ok, const dql::DqlParams& p, float* y_scale,
                                       uint8_t* y_zp) {
    if (!ok) __hip_atomic_fetch_add(sync + kQoutErrWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (blockIdx.x == 0) {
        *y_scale = ok ? (float)p.s : __builtin_nanf("");
        *y_zp = ok ? (uint8_t)p.zp : (uint8_t)0;
    }
}

}  // namespace qx
}  // namespace icx
