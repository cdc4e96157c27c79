// gfx950 top-k per row of float32 logits: the sparse indexer's selection of
// the cache entries each query attends (its indices feed
// compute_global_topk_indices_and_lens and sparse MLA decode).
//
// Reference: src/flaggems_vllm/ops/top_k_per_row_decode.py:1263-1399 (rows
// [0, seq_lens[r / next_n] - next_n + r % next_n + 1)) and
// src/flaggems_vllm/ops/top_k_per_row_prefill.py:1232-1331 (rows
// [row_starts[r], row_ends[r]), indices relative to row_starts[r]); shared
// job :877-1043 of the decode file.  Each row's top_k largest values' column
// indices, in no particular order, or all of the row's indices followed by
// -1 when the row holds at most top_k values.  The reference's radix select
// keeps an arbitrary subset of values equal to the k-th largest; this one
// keeps those with the smallest indices, so the selected set is determined
// by the values (NaN ordered above +inf, as torch.topk orders it).
//
// One workgroup per row.  Values map to 32-bit keys in the order of the
// floats; the k-th largest key is found by a radix select over three
// histograms in LDS (bits 31..21, 20..10, 9..0), each level counting only the
// values whose higher bits match the level above and picking the bin that
// holds the k-th largest:
//   - rows up to CACHE values are read from HBM once into LDS as keys, and
//     every level runs over LDS;
//   - longer rows are read once: an evenly spaced sample of the row (1/32 of
//     it, at least 2048 values) gives a key that about 4k of the row's values
//     reach, and one pass keeps every value at or above it, (key, index), in
//     LDS, where the select runs.  When at least k and at most CACHE / 2
//     values reach it, the row's top k are among them (ties at the k-th key
//     included); otherwise the row is read again for its first histogram and
//     once more for the threshold bin's values (twice more, when that bin
//     holds more than CACHE / 2 values);
//   - rows of 12 or more parts (192K+ values), when few and the caller gives
//     a workspace, are split into parts of at most 16384 values, one
//     workgroup each (read once into LDS), whose top k go to the workspace,
//     and a merge kernel selects each row's top k among its parts' candidates.
// Long rows get a 1024-thread workgroup each while there are no more rows
// than CUs, 512 threads (two rows per CU) beyond that.
// Every phase streams the row with several 16-byte loads per thread in flight.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kBins = 2048;

struct TopkArgs {
    const float* logits;
    int64_t s0, s1;
    const int32_t* row_starts;  // prefill rows, or null
    const int32_t* row_ends;
    const int32_t* seq_lens;    // decode rows
    int32_t next_n;
    int32_t* out;
    int64_t os0, os1;
    int32_t width, k;
    int32_t parts;        // parts per row (split rows), or 1
    uint32_t* cand_key;   // split rows: [rows][parts][k] candidates in the workspace
    int32_t* cand_idx;
};

__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t u = __float_as_uint(x);
    if (x != x)
        return 0xffffffffu;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int THREADS>
struct Block {
    static constexpr int kWaves = THREADS / 64;

    // Exclusive prefix of v over the block's threads in order, and the total.
    // Ends with every thread past its reads of wsum (a barrier).
    __device__ __forceinline__ static uint32_t scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        uint32_t incl = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t t = __shfl_up(incl, d);
            if (lane >= d)
                incl += t;
        }
        if (lane == 63)
            wsum[wave] = incl;
        __syncthreads();
        uint32_t before = 0, all = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t s = wsum[w];
            before += w < wave ? s : 0;
            all += s;
        }
        total = all;
        __syncthreads();
        return before + incl - v;
    }

    // The bin holding the rem-th largest counted value (rem >= 1, bins taken
    // from the top): sel[0] = the bin, sel[1] = the count above it.  Reads
    // hist after a barrier and ends after one.
    __device__ __forceinline__ static void find_bin(const uint32_t* hist, uint32_t rem, uint32_t* wsum,
                                                    int32_t* sel) {
        constexpr int per = kBins / THREADS;
        const int t = threadIdx.x;
        uint32_t c[per], local = 0;
#pragma unroll
        for (int j = 0; j < per; ++j) {
            c[j] = hist[kBins - 1 - (per * t + j)];
            local += c[j];
        }
        uint32_t total;
        uint32_t above = scan(local, wsum, total);
#pragma unroll
        for (int j = 0; j < per; ++j) {
            if (above < rem && rem <= above + c[j]) {
                sel[0] = kBins - 1 - (per * t + j);
                sel[1] = (int32_t)above;
            }
            above += c[j];
        }
        __syncthreads();
    }
};

// 16-byte loads in flight per thread while streaming a long row.
constexpr int kLoadDepth = 8;

// Word 3 of a raw buffer resource on gfx9: 32-bit data format, no swizzle.
constexpr int kBufferWord3 = 0x00020000;

// Calls f(value, index) for each of the row's len values (index i at
// x[i * s1]) for which keep(value) holds.  A unit-stride row is read in
// steps of DEPTH 16-byte buffer loads per thread, all issued before any is
// used (a load past the row's end reads zero and is not used); keep is
// evaluated over the whole step first, so a step none of whose values a
// lane keeps costs that lane one compare per value.  Other strides read
// single floats, DEPTH at a time.
struct KeepAll {
    __device__ __forceinline__ bool operator()(float) const { return true; }
};

template <int THREADS, int DEPTH, class K, class F>
__device__ __forceinline__ void for_each_if(const float* x, int64_t s1, int32_t len, K&& keep, F&& f) {
    const int t = threadIdx.x;
    if (s1 != 1) {
        for (int64_t i0 = 0; i0 < len; i0 += (int64_t)THREADS * DEPTH) {
            float v[DEPTH];
#pragma unroll
            for (int u = 0; u < DEPTH; ++u) {
                const int64_t i = i0 + u * THREADS + t;
                v[u] = i < len ? x[i * s1] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < DEPTH; ++u) {
                const int64_t i = i0 + u * THREADS + t;
                if (i < len && keep(v[u]))
                    f(v[u], (int32_t)i);
            }
        }
        return;
    }
    const int32_t head = (int32_t)(((16 - ((uintptr_t)x & 15)) & 15) >> 2);  // floats to a 16-byte boundary
    const int32_t h = head < len ? head : len;
    if (t < h && keep(x[t]))
        f(x[t], t);
    const float4* v = reinterpret_cast<const float4*>(x + h);
    const int32_t n4 = (len - h) >> 2;
    constexpr int32_t kStep = THREADS * DEPTH;
    for (int32_t j0 = 0; j0 < n4; j0 += kStep) {
        // a resource over this step's float4s only: offsets stay small and
        // loads past the row's end return zero
        const int32_t nstep = n4 - j0 < kStep ? n4 - j0 : kStep;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)(v + j0), (short)0, nstep * 16, kBufferWord3);
        uint32_t __attribute__((ext_vector_type(4))) q[DEPTH];
#pragma unroll
        for (int u = 0; u < DEPTH; ++u)
            q[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, t * 16, u * THREADS * 16, 0);
        bool any = false;
#pragma unroll
        for (int u = 0; u < DEPTH; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                any |= keep(__uint_as_float(q[u][c]));
        if (!any)
            continue;
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            const int32_t j = u * THREADS + t;
            if (j < nstep) {
                const int32_t i = h + 4 * (j0 + j);
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (keep(__uint_as_float(q[u][c])))
                        f(__uint_as_float(q[u][c]), i + c);
            }
        }
    }
    for (int32_t i = h + 4 * n4 + t; i < len; i += THREADS)
        if (keep(x[i]))
            f(x[i], i);
}

template <int THREADS, int DEPTH, class F>
__device__ __forceinline__ void for_each(const float* x, int64_t s1, int32_t len, F&& f) {
    for_each_if<THREADS, DEPTH>(x, s1, len, KeepAll{}, f);
}

// The float a key stands for (NaN for the keys above +inf's).
__device__ __forceinline__ float key_value(uint32_t key) {
    return __uint_as_float(key & 0x80000000u ? key ^ 0x80000000u : ~key);
}

// The k-th largest of n keys held in LDS (keys[0..n), 1 <= k <= n), the
// first histogram (bits 31..21) already counted in hist (read after a
// barrier).  Returns the key; cnt = how many keys equal it, need = how many of
// those are among the k largest.  hist is left holding the last level's
// counts, and every thread is past a barrier but may still read hist[b3]:
// clear it only after another barrier.
template <int THREADS>
__device__ __forceinline__ uint32_t lds_kth(const uint32_t* keys, int32_t n, uint32_t k, uint32_t* hist,
                                            uint32_t* wsum, int32_t* sel, uint32_t& need, uint32_t& cnt) {
    using B = Block<THREADS>;
    const int t = threadIdx.x;
    auto clear = [&]() {
        for (int b = t; b < kBins; b += THREADS)
            hist[b] = 0;
    };
    need = k;
    B::find_bin(hist, need, wsum, sel);
    const uint32_t b1 = sel[0];
    need -= sel[1];
    clear();
    __syncthreads();
    for (int32_t j = t; j < n; j += THREADS)
        if ((keys[j] >> 21) == b1)
            atomicAdd(&hist[(keys[j] >> 10) & 0x7ff], 1u);
    __syncthreads();
    B::find_bin(hist, need, wsum, sel);
    const uint32_t b2 = sel[0];
    need -= sel[1];
    clear();
    __syncthreads();
    const uint32_t p2 = (b1 << 11) | b2;
    for (int32_t j = t; j < n; j += THREADS)
        if ((keys[j] >> 10) == p2)
            atomicAdd(&hist[keys[j] & 0x3ff], 1u);
    __syncthreads();
    B::find_bin(hist, need, wsum, sel);
    const uint32_t b3 = sel[0];
    need -= sel[1];
    cnt = hist[b3];
    return (p2 << 10) | b3;
}

// Selection among n keys held in LDS, as lds_kth: keeps k positions, ties
// at the k-th key taken lowest index first, the index of position j being j
// itself (a row) or idx[j] (candidates; idx non-null).  Calls emit(keep, j),
// keep set for the kept j.
template <int THREADS, class Emit>
__device__ __forceinline__ void lds_select(const uint32_t* keys, const int32_t* idx, int32_t n, uint32_t k,
                                           uint32_t* hist, uint32_t* wsum, int32_t* sel, Emit&& emit) {
    using B = Block<THREADS>;
    const int t = threadIdx.x;
    uint32_t need, cnt_t;
    const uint32_t key_t = lds_kth<THREADS>(keys, n, k, hist, wsum, sel, need, cnt_t);
    for (int32_t j = t; j < n; j += THREADS)
        emit(keys[j] > key_t || (keys[j] == key_t && need == cnt_t), j);
    if (need == cnt_t)
        return;
    // ties at the k-th key: the `need` of them with the smallest indices
    if (idx) {
        for (int32_t j = t; j < n; j += THREADS) {
            bool keep = false;
            if (keys[j] == key_t) {
                const int32_t mine = idx[j];
                uint32_t rank = 0;
                for (int32_t l = 0; l < n; ++l)
                    rank += keys[l] == key_t && idx[l] < mine;
                keep = rank < need;
            }
            emit(keep, j);
        }
        return;
    }
    uint32_t base = 0;
    for (int32_t c0 = 0; c0 < n && base < need; c0 += THREADS) {
        const int32_t j = c0 + t;
        const bool tie = j < n && keys[j] == key_t;
        uint32_t total;
        const uint32_t rank = base + B::scan(tie ? 1u : 0u, wsum, total);
        emit(tie && rank < need, j);
        base += total;
    }
}

// The row's candidate range [start, end) clamped to [0, width), and its length.
__device__ __forceinline__ int32_t row_range(const TopkArgs& a, int32_t r, int32_t& start) {
    int32_t end;
    start = 0;
    if (a.row_starts) {
        start = a.row_starts[r];
        end = a.row_ends[r];
    } else {
        end = a.seq_lens[r / a.next_n] - a.next_n + r % a.next_n + 1;
    }
    start = start < 0 ? 0 : start;
    end = end > a.width ? a.width : end;
    return end > start ? end - start : 0;
}

template <int THREADS>
__device__ __forceinline__ void write_short_row(int32_t* orow, int64_t os1, int32_t len, int32_t k) {
    for (int32_t i = threadIdx.x; i < k; i += THREADS)
        orow[(int64_t)i * os1] = i < len ? i : -1;
}

// A row longer than the LDS cache (hist zeroed, counters zero, after a
// barrier): every phase streams it from HBM.
template <int CACHE, int THREADS, class Emit>
__device__ __forceinline__ void long_row(const TopkArgs& a, const float* x, int32_t len, int32_t k, uint32_t* cache,
                                         uint32_t* hist, uint32_t* wsum, int32_t* sel, uint32_t* counters,
                                         Emit&& emit) {
    using B = Block<THREADS>;
    constexpr int kCand = CACHE / 2;
    const int t = threadIdx.x;
    auto clear = [&]() {
        for (int b = t; b < kBins; b += THREADS)
            hist[b] = 0;
    };
    uint32_t need = (uint32_t)k, b1, b2, b3, cnt_t;
    uint32_t* ckey = cache;
    int32_t* cidx = reinterpret_cast<int32_t*>(cache + kCand);
    if (2 * k <= kCand) {
        // ---- longer rows, read once: a threshold from a sample of the row
        // (nch chunks of 256 contiguous values, one every `stride` values)
        int32_t ns = (len / 32) & ~255;
        ns = ns < 2048 ? 2048 : ns > CACHE ? CACHE : ns;
        const int32_t nch = ns >> 8, stride = len / nch;
        for (int32_t s0 = 0; s0 < ns; s0 += THREADS * kLoadDepth) {
            float v[kLoadDepth];
#pragma unroll
            for (int u = 0; u < kLoadDepth; ++u) {
                const int32_t q = s0 + u * THREADS + t;
                v[u] = q < ns ? x[(int64_t)((q >> 8) * stride + (q & 255)) * a.s1] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < kLoadDepth; ++u) {
                const int32_t q = s0 + u * THREADS + t;
                if (q < ns) {
                    const uint32_t key = order_key(v[u]);
                    cache[q] = key;
                    atomicAdd(&hist[key >> 21], 1u);
                }
            }
        }
        __syncthreads();
        // the sample's rank-th largest key: about `target` of the row's values reach it
        const int64_t target = min(4 * (int64_t)k, ((int64_t)k + kCand) / 2);
        int64_t rank = (target * ns + len - 1) / len;
        rank = rank < 1 ? 1 : rank > ns ? ns : rank;
        uint32_t sneed, scnt;
        const uint32_t key_e = lds_kth<THREADS>(cache, ns, (uint32_t)rank, hist, wsum, sel, sneed, scnt);
        __syncthreads();
        clear();
        __syncthreads();
        // !(v < fe) holds for every value whose key is at least key_e (NaN
        // included) and for -0 against +0: an up-set of the key order, so
        // when it holds k or more values it holds the row's top k
        const float fe = key_value(key_e);
        for_each_if<THREADS, kLoadDepth>(
            x, a.s1, len, [&](float v) { return !(v < fe); },
            [&](float v, int32_t i) {
                const uint32_t p = atomicAdd(&counters[1], 1u);
                if (p < (uint32_t)kCand) {
                    const uint32_t key = order_key(v);
                    ckey[p] = key;
                    cidx[p] = i;
                    atomicAdd(&hist[key >> 21], 1u);
                }
            });
        __syncthreads();
        const uint32_t m = counters[1];
        if (m >= (uint32_t)k && m <= (uint32_t)kCand) {
            lds_select<THREADS>(ckey, cidx, (int32_t)m, (uint32_t)k, hist, wsum, sel,
                                [&](bool keep, int32_t j) { emit(keep, cidx[j]); });
            return;
        }
        __syncthreads();
        clear();
        if (t == 0)
            counters[1] = 0;
        __syncthreads();
    }

    // ---- the first histogram from HBM (these passes are the exception:
    // shallower loads keep the kernel's code small)
    for_each<THREADS, kLoadDepth / 2>(x, a.s1, len, [&](float v, int32_t) { atomicAdd(&hist[order_key(v) >> 21], 1u); });
    __syncthreads();
    B::find_bin(hist, need, wsum, sel);
    b1 = sel[0];
    need -= sel[1];
    const uint32_t c1 = hist[b1];
    __syncthreads();
    clear();
    __syncthreads();
    if (c1 <= (uint32_t)kCand) {
        for_each<THREADS, kLoadDepth / 2>(x, a.s1, len, [&](float v, int32_t i) {
            const uint32_t key = order_key(v), b = key >> 21;
            emit(b > b1, i);
            if (b == b1) {
                const uint32_t p = atomicAdd(&counters[1], 1u);
                ckey[p] = key;
                cidx[p] = i;
                atomicAdd(&hist[(key >> 10) & 0x7ff], 1u);
            }
        });
        __syncthreads();
        const uint32_t m = counters[1];
        B::find_bin(hist, need, wsum, sel);
        b2 = sel[0];
        need -= sel[1];
        clear();
        __syncthreads();
        for (uint32_t j = t; j < m; j += THREADS)
            if (((ckey[j] >> 10) & 0x7ff) == b2)
                atomicAdd(&hist[ckey[j] & 0x3ff], 1u);
        __syncthreads();
        B::find_bin(hist, need, wsum, sel);
        b3 = sel[0];
        need -= sel[1];
        cnt_t = hist[b3];
        const uint32_t key_t = (((b1 << 11) | b2) << 10) | b3;
        for (uint32_t j = t; j < m; j += THREADS) {
            const uint32_t key = ckey[j];
            bool keep = key > key_t || (key == key_t && need == cnt_t);
            if (!keep && key == key_t) {
                // rank among the tied candidates by index (ties beyond the
                // k-th value are rare: a scan of the candidates each)
                const int32_t mine = cidx[j];
                uint32_t rank = 0;
                for (uint32_t l = 0; l < m; ++l)
                    rank += ckey[l] == key_t && cidx[l] < mine;
                keep = rank < need;
            }
            emit(keep, cidx[j]);
        }
        return;
    }

    // ---- a threshold bin too large for LDS: the lower levels from HBM too
    for_each<THREADS, kLoadDepth / 2>(x, a.s1, len, [&](float v, int32_t) {
        const uint32_t key = order_key(v);
        if ((key >> 21) == b1)
            atomicAdd(&hist[(key >> 10) & 0x7ff], 1u);
    });
    __syncthreads();
    B::find_bin(hist, need, wsum, sel);
    b2 = sel[0];
    need -= sel[1];
    clear();
    __syncthreads();
    const uint32_t p2 = (b1 << 11) | b2;
    for_each<THREADS, kLoadDepth / 2>(x, a.s1, len, [&](float v, int32_t) {
        const uint32_t key = order_key(v);
        if ((key >> 10) == p2)
            atomicAdd(&hist[key & 0x3ff], 1u);
    });
    __syncthreads();
    B::find_bin(hist, need, wsum, sel);
    b3 = sel[0];
    need -= sel[1];
    cnt_t = hist[b3];
    const uint32_t key_t = (p2 << 10) | b3;
    for_each<THREADS, kLoadDepth / 2>(x, a.s1, len, [&](float v, int32_t i) {
        const uint32_t key = order_key(v);
        emit(key > key_t || (key == key_t && need == cnt_t), i);
    });
    if (need < cnt_t) {
        uint32_t base = 0;
        for (int32_t c0 = 0; c0 < len && base < need; c0 += THREADS) {
            const int32_t i = c0 + t;
            const bool tie = i < len && order_key(x[(int64_t)i * a.s1]) == key_t;
            uint32_t total;
            const uint32_t rank = base + B::scan(tie ? 1u : 0u, wsum, total);
            emit(tie && rank < need, i);
            base += total;
        }
    }
}

// LONG = false: rows of at most CACHE values (the launcher's width), held in
// LDS.  LONG = true: any row; longer ones are streamed.
template <int CACHE, int THREADS, bool LONG>
__global__ void __launch_bounds__(THREADS)
top_k_per_row_kernel(TopkArgs a) {
    using B = Block<THREADS>;
    __shared__ uint32_t hist[kBins];
    __shared__ uint32_t cache[CACHE];  // the row's keys, or (key, index) candidates in the two halves
    __shared__ uint32_t wsum[B::kWaves];
    __shared__ int32_t sel[2];
    __shared__ uint32_t counters[2];   // values written, candidates kept
    constexpr int kCand = CACHE / 2;   // (key, index) candidates the cache holds
    constexpr int kRowDepth = CACHE / (4 * THREADS) < kLoadDepth ? CACHE / (4 * THREADS) : kLoadDepth;

    const int t = threadIdx.x;
    const int32_t r = blockIdx.x;
    int32_t start;
    int32_t len = row_range(a, r, start);
    int32_t* orow = a.out + (int64_t)r * a.os0;
    const int32_t k = a.k;
    if (len <= k) {
        write_short_row<THREADS>(orow, a.os1, len, k);
        return;
    }
    if (!LONG && len > CACHE)
        len = CACHE;  // not reached: the launcher keeps width <= CACHE here
    const float* x = a.logits + (int64_t)r * a.s0 + (int64_t)start * a.s1;
    auto clear = [&]() {
        for (int b = t; b < kBins; b += THREADS)
            hist[b] = 0;
    };
    auto emit = [&](bool keep, int32_t i) {
        if (keep) {
            const uint32_t p = atomicAdd(&counters[0], 1u);
            if (p < (uint32_t)k)
                orow[(int64_t)p * a.os1] = i;
        }
    };
    clear();
    if (t == 0) {
        counters[0] = counters[1] = 0;
        sel[0] = sel[1] = 0;
    }
    __syncthreads();

    if (!LONG || len <= CACHE) {
        // ---- the row in LDS
        for_each<THREADS, kRowDepth>(x, a.s1, len, [&](float v, int32_t i) {
            const uint32_t key = order_key(v);
            cache[i] = key;
            atomicAdd(&hist[key >> 21], 1u);
        });
        __syncthreads();
        lds_select<THREADS>(cache, nullptr, len, (uint32_t)k, hist, wsum, sel, emit);
        return;
    }
    if constexpr (LONG)
        long_row<CACHE, THREADS>(a, x, len, k, cache, hist, wsum, sel, counters, emit);
}
// ---- Rows split into parts: rows longer than the LDS row cache, when the
// caller's workspace holds every part's candidates.  Part p of a row is
// [p * cl, min(len, (p + 1) * cl)), cl = ceil(len / parts) <= kPartCache; its
// top k (by the same order: key, then index) go to the workspace as (key,
// row-relative index) pairs, key 0 (below every value's key) and index -1
// padding a part of fewer than k values; the merge then selects the row's
// top k among the parts' candidates.  Every element of the row's top k is
// among its part's top k (fewer than k elements of the row, so of its part,
// come before it), so the merge's choice is the row's.
constexpr int kPartCache = 16384;
constexpr int kMergeCap = 8192;

template <int THREADS>
__global__ void __launch_bounds__(THREADS)
top_k_part_kernel(TopkArgs a) {
    using B = Block<THREADS>;
    __shared__ uint32_t hist[kBins];
    __shared__ uint32_t cache[kPartCache];
    __shared__ uint32_t wsum[B::kWaves];
    __shared__ int32_t sel[2];
    __shared__ uint32_t counter;
    const int t = threadIdx.x;
    const int32_t r = blockIdx.x, part = blockIdx.y, parts = gridDim.y;
    int32_t start;
    const int32_t len = row_range(a, r, start);
    const int32_t k = a.k;
    if (len <= k) {  // the row's output, written by its first part; the merge skips the row
        if (part == 0)
            write_short_row<THREADS>(a.out + (int64_t)r * a.os0, a.os1, len, k);
        return;
    }
    const int32_t cl = (len + parts - 1) / parts;
    const int32_t p0 = part * cl;
    const int32_t plen = max(0, min(len - p0, cl));
    const int64_t slot = ((int64_t)r * parts + part) * k;
    uint32_t* wkey = a.cand_key + slot;
    int32_t* widx = a.cand_idx + slot;
    if (plen <= k) {
        const float* x = a.logits + (int64_t)r * a.s0 + (int64_t)(start + p0) * a.s1;
        for (int32_t i = t; i < k; i += THREADS) {
            wkey[i] = i < plen ? order_key(x[(int64_t)i * a.s1]) : 0u;
            widx[i] = i < plen ? p0 + i : -1;
        }
        return;
    }
    for (int b = t; b < kBins; b += THREADS)
        hist[b] = 0;
    if (t == 0) {
        counter = 0;
        sel[0] = sel[1] = 0;
    }
    __syncthreads();
    const float* x = a.logits + (int64_t)r * a.s0 + (int64_t)(start + p0) * a.s1;
    for_each<THREADS, kLoadDepth>(x, a.s1, plen, [&](float v, int32_t i) {
        const uint32_t key = order_key(v);
        cache[i] = key;
        atomicAdd(&hist[key >> 21], 1u);
    });
    __syncthreads();
    lds_select<THREADS>(cache, nullptr, plen, (uint32_t)k, hist, wsum, sel, [&](bool keep, int32_t j) {
        if (keep) {
            const uint32_t q = atomicAdd(&counter, 1u);
            if (q < (uint32_t)k) {
                wkey[q] = cache[j];
                widx[q] = p0 + j;
            }
        }
    });
}

template <int THREADS>
__global__ void __launch_bounds__(THREADS)
top_k_merge_kernel(TopkArgs a) {
    using B = Block<THREADS>;
    __shared__ uint32_t hist[kBins];
    __shared__ uint32_t ckey[kMergeCap];
    __shared__ int32_t cidx[kMergeCap];
    __shared__ uint32_t wsum[B::kWaves];
    __shared__ int32_t sel[2];
    __shared__ uint32_t counter;
    const int t = threadIdx.x;
    const int32_t r = blockIdx.x;
    int32_t start;
    const int32_t len = row_range(a, r, start);
    const int32_t k = a.k;
    if (len <= k)
        return;
    const int32_t n = a.parts * k;
    for (int b = t; b < kBins; b += THREADS)
        hist[b] = 0;
    if (t == 0) {
        counter = 0;
        sel[0] = sel[1] = 0;
    }
    __syncthreads();
    const int64_t slot = (int64_t)r * n;
    for (int32_t j = t; j < n; j += THREADS) {
        const uint32_t key = a.cand_key[slot + j];
        ckey[j] = key;
        cidx[j] = a.cand_idx[slot + j];
        atomicAdd(&hist[key >> 21], 1u);
    }
    __syncthreads();
    int32_t* orow = a.out + (int64_t)r * a.os0;
    lds_select<THREADS>(ckey, cidx, n, (uint32_t)k, hist, wsum, sel, [&](bool keep, int32_t j) {
        if (keep) {
            const uint32_t q = atomicAdd(&counter, 1u);
            if (q < (uint32_t)k)
                orow[(int64_t)q * a.os1] = cidx[j];
        }
    });
}

// Parts per row for the split: rows longer than one part's LDS cache, as
// many parts as keep each within it, when the merge can hold their candidates.
int64_t topk_parts(int64_t width, int64_t k) {
    if (width <= kPartCache || k <= 0)
        return 1;
    const int64_t parts = (width + kPartCache - 1) / kPartCache;
    return parts * k <= kMergeCap ? parts : 1;
}

// Long rows (12 parts or more, 192K+ values) are split while their parts fit
// one round of part workgroups (two per CU): streaming such a row takes one
// workgroup ~42 us (262144 values, MI355X), the split 32-37 us up to 32 rows
// and more once the parts run in two rounds.  Shorter rows stream faster than
// the split's two kernels finish.
bool topk_split(int64_t num_rows, int64_t width, int64_t k) {
    const int64_t parts = topk_parts(width, k);
    return parts >= 12 && num_rows * parts <= 2 * (int64_t)cu_count();
}

int64_t topk_workspace_bytes(int64_t num_rows, int64_t width, int64_t k) {
    return topk_split(num_rows, width, k) ? num_rows * topk_parts(width, k) * k * 8 : 0;
}

int launch_topk(TopkArgs a, int64_t num_rows, void* workspace, int64_t workspace_bytes, void* stream) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t need = topk_workspace_bytes(num_rows, a.width, a.k);
    a.parts = 1;
    a.cand_key = nullptr;
    a.cand_idx = nullptr;
    if (need > 0 && workspace && workspace_bytes >= need) {
        if (!aligned(workspace, 16))
            return fail(FGV_E_MISALIGNED, "workspace must be 16-byte aligned");
        a.parts = (int32_t)topk_parts(a.width, a.k);
        a.cand_key = static_cast<uint32_t*>(workspace);
        a.cand_idx = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + need / 2);
        hipLaunchKernelGGL(top_k_part_kernel<512>, dim3((unsigned)num_rows, (unsigned)a.parts), dim3(512), 0, st,
                           a);
        const int rc = launch_status();
        if (rc)
            return rc;
        hipLaunchKernelGGL(top_k_merge_kernel<512>, dim3((unsigned)num_rows), dim3(512), 0, st, a);
        return launch_status();
    }
    const dim3 grid((unsigned)num_rows);
    if (a.width <= 4096)
        hipLaunchKernelGGL((top_k_per_row_kernel<4096, 256, false>), grid, dim3(256), 0, st, a);
    else if (a.width <= 8192)
        hipLaunchKernelGGL((top_k_per_row_kernel<8192, 512, false>), grid, dim3(512), 0, st, a);
    else if (a.width <= 16384)
        hipLaunchKernelGGL((top_k_per_row_kernel<16384, 512, false>), grid, dim3(512), 0, st, a);
    else if (num_rows <= cu_count())  // a CU per row: 1024 threads stream it faster
        hipLaunchKernelGGL((top_k_per_row_kernel<8192, 1024, true>), grid, dim3(1024), 0, st, a);
    else  // two rows per CU
        hipLaunchKernelGGL((top_k_per_row_kernel<12288, 512, true>), grid, dim3(512), 0, st, a);
    return launch_status();
}

int check_topk(const float* logits, int64_t num_rows, int64_t width, int32_t* indices, int64_t top_k) {
    if (num_rows < 0 || width < 0 || top_k < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_rows > 0x7fffffffLL || width > 0x7fffffffLL || top_k > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "rows, width and top_k must fit in int32");
    if (num_rows > 0 && (!logits || !indices))
        return fail(FGV_E_NULL_POINTER, "null logits or indices");
    if (!aligned(logits, 4) || !aligned(indices, 4))
        return fail(FGV_E_MISALIGNED, "logits and indices must be 4-byte aligned");
    return FGV_OK;
}

}  // namespace
}  // namespace fgv

extern "C" int64_t fgv_top_k_per_row_workspace_bytes(int64_t num_rows, int64_t width, int64_t top_k) {
    if (num_rows <= 0 || width <= 0 || top_k <= 0 || num_rows > 0x7fffffffLL || width > 0x7fffffffLL ||
        top_k > 0x7fffffffLL)
        return 0;
    return fgv::topk_workspace_bytes(num_rows, width, top_k);
}

extern "C" int fgv_top_k_per_row_decode(const float* logits, int64_t stride0, int64_t stride1, int64_t num_rows,
                                        int64_t width, int64_t next_n, const int32_t* seq_lens, int32_t* indices,
                                        int64_t out_stride0, int64_t out_stride1, int64_t top_k, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
    using namespace fgv;
    int rc = check_topk(logits, num_rows, width, indices, top_k);
    if (rc)
        return rc;
    if (next_n <= 0 || next_n > 0x7fffffffLL)
        return fail(FGV_E_BAD_SHAPE, "next_n must be positive");
    if (num_rows == 0 || top_k == 0)
        return FGV_OK;
    if (!seq_lens)
        return fail(FGV_E_NULL_POINTER, "null seq_lens");
    TopkArgs a{logits, stride0, stride1, nullptr, nullptr, seq_lens, (int32_t)next_n, indices, out_stride0,
               out_stride1, (int32_t)width, (int32_t)top_k, 1, nullptr, nullptr};
    return launch_topk(a, num_rows, workspace, workspace_bytes, stream);
}

extern "C" int fgv_top_k_per_row_prefill(const float* logits, int64_t stride0, int64_t stride1, int64_t num_rows,
                                         int64_t width, const int32_t* row_starts, const int32_t* row_ends,
                                         int32_t* indices, int64_t out_stride0, int64_t out_stride1, int64_t top_k,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace fgv;
    int rc = check_topk(logits, num_rows, width, indices, top_k);
    if (rc)
        return rc;
    if (num_rows == 0 || top_k == 0)
        return FGV_OK;
    if (!row_starts || !row_ends)
        return fail(FGV_E_NULL_POINTER, "null row_starts or row_ends");
    TopkArgs a{logits, stride0, stride1, row_starts, row_ends, nullptr, 1, indices, out_stride0, out_stride1,
               (int32_t)width, (int32_t)top_k, 1, nullptr, nullptr};
    return launch_topk(a, num_rows, workspace, workspace_bytes, stream);
}
