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
//   - longer rows are read twice: the first histogram, then one pass that
//     writes out every value above the threshold bin and keeps the bin's own
//     values (key, index) in LDS, where the two lower levels run; only a
//     threshold bin of more than CACHE / 2 values reads the row twice more.
// Indices are written through an LDS counter, so their order within a row
// varies from call to call (the set does not).
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

// Calls f(value, index) for each of the row's len values (index i at x[i * s1]),
// with 16-byte loads where the row allows them.
template <int THREADS, class F>
__device__ __forceinline__ void for_each(const float* x, int64_t s1, int32_t len, F&& f) {
    const int t = threadIdx.x;
    if (s1 != 1) {
        for (int32_t i = t; i < len; i += THREADS)
            f(x[(int64_t)i * s1], i);
        return;
    }
    const int32_t head = (int32_t)(((16 - ((uintptr_t)x & 15)) & 15) >> 2);  // floats to a 16-byte boundary
    const int32_t h = head < len ? head : len;
    if (t < h)
        f(x[t], t);
    const float4* v = reinterpret_cast<const float4*>(x + h);
    const int32_t n4 = (len - h) >> 2;
    for (int32_t j = t; j < n4; j += THREADS) {
        const float4 q = v[j];
        const int32_t i = h + 4 * j;
        f(q.x, i);
        f(q.y, i + 1);
        f(q.z, i + 2);
        f(q.w, i + 3);
    }
    for (int32_t i = h + 4 * n4 + t; i < len; i += THREADS)
        f(x[i], i);
}

template <int CACHE, int THREADS>
__global__ void __launch_bounds__(THREADS)
top_k_per_row_kernel(TopkArgs a) {
    using B = Block<THREADS>;
    __shared__ uint32_t hist[kBins];
    __shared__ uint32_t cache[CACHE];  // the row's keys, or (key, index) candidates in the two halves
    __shared__ uint32_t wsum[B::kWaves];
    __shared__ int32_t sel[2];
    __shared__ uint32_t counters[2];   // values written, candidates kept
    constexpr int kCand = CACHE / 2;

    const int t = threadIdx.x;
    const int32_t r = blockIdx.x;
    int32_t start = 0, end;
    if (a.row_starts) {
        start = a.row_starts[r];
        end = a.row_ends[r];
    } else {
        end = a.seq_lens[r / a.next_n] - a.next_n + r % a.next_n + 1;
    }
    start = start < 0 ? 0 : start;
    end = end > a.width ? a.width : end;
    const int32_t len = end > start ? end - start : 0;
    int32_t* orow = a.out + (int64_t)r * a.os0;
    const int32_t k = a.k;
    if (len <= k) {
        for (int32_t i = t; i < k; i += THREADS)
            orow[(int64_t)i * a.os1] = i < len ? i : -1;
        return;
    }
    const float* x = a.logits + (int64_t)r * a.s0 + (int64_t)start * a.s1;
    auto clear = [&]() {
        for (int b = t; b < kBins; b += THREADS)
            hist[b] = 0;
    };
    auto emit = [&](int32_t i) {
        const uint32_t p = atomicAdd(&counters[0], 1u);
        if (p < (uint32_t)k)
            orow[(int64_t)p * a.os1] = i;
    };
    clear();
    if (t == 0) {
        counters[0] = counters[1] = 0;
        sel[0] = sel[1] = 0;
    }
    __syncthreads();

    uint32_t need = (uint32_t)k, b1, b2, b3, cnt_t;
    if (len <= CACHE) {
        // ---- the row in LDS
        for_each<THREADS>(x, a.s1, len, [&](float v, int32_t i) {
            const uint32_t key = order_key(v);
            cache[i] = key;
            atomicAdd(&hist[key >> 21], 1u);
        });
        __syncthreads();
        B::find_bin(hist, need, wsum, sel);
        b1 = sel[0];
        need -= sel[1];
        clear();
        __syncthreads();
        for (int32_t i = t; i < len; i += THREADS)
            if ((cache[i] >> 21) == b1)
                atomicAdd(&hist[(cache[i] >> 10) & 0x7ff], 1u);
        __syncthreads();
        B::find_bin(hist, need, wsum, sel);
        b2 = sel[0];
        need -= sel[1];
        clear();
        __syncthreads();
        const uint32_t p2 = (b1 << 11) | b2;
        for (int32_t i = t; i < len; i += THREADS)
            if ((cache[i] >> 10) == p2)
                atomicAdd(&hist[cache[i] & 0x3ff], 1u);
        __syncthreads();
        B::find_bin(hist, need, wsum, sel);
        b3 = sel[0];
        need -= sel[1];
        cnt_t = hist[b3];
        const uint32_t key_t = (p2 << 10) | b3;
        for (int32_t i = t; i < len; i += THREADS)
            if (cache[i] > key_t || (cache[i] == key_t && need == cnt_t))
                emit(i);
        if (need < cnt_t) {
            // ties at the k-th value: the `need` of them with the smallest indices
            uint32_t base = 0;
            for (int32_t c0 = 0; c0 < len && base < need; c0 += THREADS) {
                const int32_t i = c0 + t;
                const bool tie = i < len && cache[i] == key_t;
                uint32_t total;
                const uint32_t rank = base + B::scan(tie ? 1u : 0u, wsum, total);
                if (tie && rank < need)
                    emit(i);
                base += total;
            }
        }
        return;
    }

    // ---- longer rows: the first histogram from HBM
    for_each<THREADS>(x, a.s1, len, [&](float v, int32_t) { atomicAdd(&hist[order_key(v) >> 21], 1u); });
    __syncthreads();
    B::find_bin(hist, need, wsum, sel);
    b1 = sel[0];
    need -= sel[1];
    const uint32_t c1 = hist[b1];
    __syncthreads();
    clear();
    __syncthreads();
    if (c1 <= (uint32_t)kCand) {
        uint32_t* ckey = cache;
        int32_t* cidx = reinterpret_cast<int32_t*>(cache + kCand);
        for_each<THREADS>(x, a.s1, len, [&](float v, int32_t i) {
            const uint32_t key = order_key(v), b = key >> 21;
            if (b > b1) {
                emit(i);
            } else if (b == b1) {
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
            if (key > key_t || (key == key_t && need == cnt_t)) {
                emit(cidx[j]);
            } else if (key == key_t) {
                // rank among the tied candidates by index (ties beyond the
                // k-th value are rare: a scan of the candidates each)
                const int32_t mine = cidx[j];
                uint32_t rank = 0;
                for (uint32_t l = 0; l < m; ++l)
                    rank += ckey[l] == key_t && cidx[l] < mine;
                if (rank < need)
                    emit(mine);
            }
        }
        return;
    }

    // ---- a threshold bin too large for LDS: the lower levels from HBM too
    for_each<THREADS>(x, a.s1, len, [&](float v, int32_t) {
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
    for_each<THREADS>(x, a.s1, len, [&](float v, int32_t) {
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
    for_each<THREADS>(x, a.s1, len, [&](float v, int32_t i) {
        const uint32_t key = order_key(v);
        if (key > key_t || (key == key_t && need == cnt_t))
            emit(i);
    });
    if (need < cnt_t) {
        uint32_t base = 0;
        for (int32_t c0 = 0; c0 < len && base < need; c0 += THREADS) {
            const int32_t i = c0 + t;
            const bool tie = i < len && order_key(x[(int64_t)i * a.s1]) == key_t;
            uint32_t total;
            const uint32_t rank = base + B::scan(tie ? 1u : 0u, wsum, total);
            if (tie && rank < need)
                emit(i);
            base += total;
        }
    }
}

int launch_topk(const TopkArgs& a, int64_t num_rows, void* stream) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)num_rows);
    if (a.width <= 6144)
        hipLaunchKernelGGL((top_k_per_row_kernel<6144, 256>), grid, dim3(256), 0, st, a);
    else if (a.width <= 16384)
        hipLaunchKernelGGL((top_k_per_row_kernel<16384, 512>), grid, dim3(512), 0, st, a);
    else
        hipLaunchKernelGGL((top_k_per_row_kernel<12288, 512>), grid, dim3(512), 0, st, a);
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

extern "C" int fgv_top_k_per_row_decode(const float* logits, int64_t stride0, int64_t stride1, int64_t num_rows,
                                        int64_t width, int64_t next_n, const int32_t* seq_lens, int32_t* indices,
                                        int64_t out_stride0, int64_t out_stride1, int64_t top_k, void* stream) {
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
               out_stride1, (int32_t)width, (int32_t)top_k};
    return launch_topk(a, num_rows, stream);
}

extern "C" int fgv_top_k_per_row_prefill(const float* logits, int64_t stride0, int64_t stride1, int64_t num_rows,
                                         int64_t width, const int32_t* row_starts, const int32_t* row_ends,
                                         int32_t* indices, int64_t out_stride0, int64_t out_stride1, int64_t top_k,
                                         void* stream) {
    using namespace fgv;
    int rc = check_topk(logits, num_rows, width, indices, top_k);
    if (rc)
        return rc;
    if (num_rows == 0 || top_k == 0)
        return FGV_OK;
    if (!row_starts || !row_ends)
        return fail(FGV_E_NULL_POINTER, "null row_starts or row_ends");
    TopkArgs a{logits, stride0, stride1, row_starts, row_ends, nullptr, 1, indices, out_stride0, out_stride1,
               (int32_t)width, (int32_t)top_k};
    return launch_topk(a, num_rows, stream);
}
