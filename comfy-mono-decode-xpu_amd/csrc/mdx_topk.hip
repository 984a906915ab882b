// Exact top-k of long rows in torch's XPU order, one launch: fast_topk / fast_pick (one bf16 row,
// k <= 8, optional argmax) and topk_rows (up to 16 fp32 or bf16 rows, k <= 64).
//
// Reference semantics (comfy-mono-decode-xpu): csrc/fast_topk.sycl:4-40 (bf16 radix key, argmax rank,
// gather order of 1024 threads x 4 loads of 8), csrc/fast_topk.sycl:145-157 (index back-mapping),
// csrc/topk_rows.sycl:7-11,33-43 (fp32 radix key, gather order of 1024 threads x 8 loads of 4).
// Every element gets a unique 64-bit rank (radix key in the high word, the complement of its gather
// position in the low word); the k largest ranks, in descending order, are the result.
//
// Launch: rows x nseg work-groups of 256 (4 waves), each owning a contiguous segment of its row.
//   1. every thread streams its elements (stride 256) and keeps its largest rank;
//   2. theta = the k-th largest of the 256 thread maxima (each thread counts the maxima above its own;
//      ranks are unique, so exactly one thread sees k - 1). Every element >= theta belongs to one of
//      the k threads whose maximum is >= theta, so at most k * ceil(seg / 256) elements qualify and
//      the candidate buffer in LDS never overflows, ties or not;
//   3. the candidates are ranked by counting (position = number of larger candidates); the segment's
//      top-k goes to the workspace as a descending, zero-padded list;
//   4. the row's last work-group (device-scope counter, reset by that work-group) merges the nseg
//      lists: theta2 = the k-th largest list head bounds the row's top k from below (k lists hold an
//      entry >= theta2), and only the entries >= theta2 are ranked among themselves by counting.
// The counting loops read LDS eight words per round trip (indices clamped, masked).
// Ranks are never 0 (the radix key of a non-NaN value is nonzero, and a NaN's rank has a nonzero
// gather word), so 0 marks an empty slot.
#include <algorithm>

#include <mutex>

#include "mdx_common.hpp"
#include "mdx_rank.hpp"

namespace mdx {
namespace {

constexpr int TK_T = 256;
constexpr int TK_MAXK = 64;
constexpr int TK_MAXR = 16;
constexpr int TK_MAXSEG = 64;
constexpr int TK_E = 24;  // elements per thread held in registers per pass (segments of 6144 in one pass)

struct TopkArgs {
    const void* x;       // [rows, n] bf16 or fp32
    int64_t n;
    int rows, k, nseg, seg, f32;
    int pick;            // also the argmax (ORDER_ARGMAX rank) of the row
    void* values;        // [rows, k]: bf16 (ORDER_BF16 / ORDER_ARGMAX) or fp32 (ORDER_F32)
    int64_t* indices;    // [rows, k]
    int64_t* argmax;     // [rows] when pick
    uint64_t* lists;     // workspace: [rows][nseg][k] ranks, [rows][nseg] argmax ranks
    uint64_t* amax;
    unsigned* counter;   // [rows], zero between launches
};

__device__ __forceinline__ void st_c64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    return v;
}


// the number of entries of buf[b0, b1) above v, eight reads per LDS round trip
__device__ __forceinline__ int count_above(const uint64_t* buf, int b0, int b1, uint64_t v) {
    int n = 0;
    for (int f0 = b0; f0 < b1; f0 += 8) {
        uint64_t c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = buf[min(f0 + j, b1 - 1)];
#pragma unroll
        for (int j = 0; j < 8; ++j) n += (f0 + j < b1 && c[j] > v) ? 1 : 0;
    }
    return n;
}

template <int ORD, bool XF32>
__global__ __launch_bounds__(TK_T) void topk_kernel(TopkArgs a) {
    extern __shared__ __align__(16) uint64_t sm[];
    uint64_t* tmax = sm;             // [256] thread maxima
    uint64_t* cand = sm + TK_T;      // candidates (k * ceil(seg / 256)) or, in the merge, nseg * k lists + their survivors
    __shared__ uint64_t theta_s, theta2_s, am_s[TK_T / 64];
    __shared__ unsigned ncand, last_s, nc2_s;
    const int t = threadIdx.x;
    const int row = blockIdx.x / a.nseg, sg = blockIdx.x % a.nseg;
    const int K = a.k;
    const bool f32 = a.f32;
    const void* xr = f32 ? static_cast<const void*>(static_cast<const uint32_t*>(a.x) + row * a.n)
                         : static_cast<const void*>(static_cast<const uint16_t*>(a.x) + row * a.n);
    const uint32_t lo = uint32_t(sg) * uint32_t(a.seg);
    const int64_t end = int64_t(lo) + a.seg;
    const uint32_t hi = uint32_t(end < a.n ? end : a.n);

    // 1. thread maxima (and the argmax rank for a pick). The thread's elements lo + t + 256 j are read
    // TK_E at a time into registers, every load of a pass issued before the first use (addresses
    // clamped into the segment, no branches around the loads): one memory round trip per pass, where
    // a load per iteration would wait for each element in turn. A segment of at most TK_E * 256
    // elements takes one pass and stays in registers for step 3.
    const int nb = (a.seg + TK_T - 1) / TK_T, npass = (nb + TK_E - 1) / TK_E;  // (uniform)
    uint32_t rv[TK_E];
    auto load_pass = [&](int p) {
#pragma unroll
        for (int j = 0; j < TK_E; ++j) rv[j] = raw_of<ORD, XF32>(xr, min(lo + t + uint32_t(TK_T * (p * TK_E + j)), hi - 1));
    };
    uint64_t mx = 0, am = 0;
    for (int p = 0; p < npass; ++p) {
        load_pass(p);
#pragma unroll
        for (int j = 0; j < TK_E; ++j) {
            const uint32_t i = lo + t + uint32_t(TK_T * (p * TK_E + j));
            if (p * TK_E + j < nb && i < hi) {
                const uint64_t r = rank_raw<ORD, XF32>(rv[j], i);
                mx = r > mx ? r : mx;
                if (a.pick) {
                    const uint64_t q = rank_raw<ORDER_ARGMAX>(rv[j], i);
                    am = q > am ? q : am;
                }
            }
        }
    }
    tmax[t] = mx;
    if (t == 0) ncand = 0;
    if (a.pick) {
        am = wave_max_u64(am);
        if ((t & 63) == 0) am_s[t >> 6] = am;
    }
    __syncthreads();
    // 2. theta: the k-th largest thread maximum (or the smallest nonzero one if fewer than k)
    const int nz = __syncthreads_count(mx != 0);
    if (nz <= K) {
        if (t == 0) theta_s = 1;
    } else if (mx != 0) {
        int above = 0;
        for (int q = 0; q < TK_T; ++q) above += tmax[q] > mx;
        if (above == K - 1) theta_s = mx;
    }
    __syncthreads();
    const uint64_t theta = theta_s;
    // 3. candidates >= theta, ranked by counting
    if (mx >= theta)
        for (int p = 0; p < npass; ++p) {
            if (npass > 1) load_pass(p);  // (one pass: the registers still hold it)
#pragma unroll
            for (int j = 0; j < TK_E; ++j) {
                const uint32_t i = lo + t + uint32_t(TK_T * (p * TK_E + j));
                if (p * TK_E + j < nb && i < hi) {
                    const uint64_t r = rank_raw<ORD, XF32>(rv[j], i);
                    if (r >= theta) cand[atomicAdd(&ncand, 1u)] = r;
                }
            }
        }
    __syncthreads();
    const int nc = int(ncand);
    uint64_t* mylist = a.lists + (int64_t(row) * a.nseg + sg) * K;
    for (int j = t; j < nc; j += TK_T) {
        const uint64_t v = cand[j];
        const int pos = count_above(cand, 0, nc, v);
        if (pos < K) st_c64(mylist + pos, v);
    }
    for (int j = nc + t; j < K; j += TK_T) st_c64(mylist + j, uint64_t(0));
    if (a.pick && t == 0) {
        uint64_t b = am_s[0];
        for (int w = 1; w < TK_T / 64; ++w) b = am_s[w] > b ? am_s[w] : b;
        st_c64(a.amax + int64_t(row) * a.nseg + sg, b);
    }
    // 4. the row's last work-group merges. Hand-off without fences (an agent-scope fence writes back
    // and invalidates whole caches on this chip): the lists are coherent stores, complete (vector
    // memory counter at zero) before the counter bump; the last work-group reads them coherently.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0)
        last_s = __hip_atomic_fetch_add(a.counter + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 unsigned(a.nseg - 1);
    __syncthreads();
    if (!last_s) return;
    const int total = a.nseg * K;
    const uint64_t* rl = a.lists + int64_t(row) * a.nseg * K;
    {
        // every list entry's load issued before the first LDS store (one memory round trip)
        constexpr int LP = TK_MAXSEG * TK_MAXK / TK_T;
        uint64_t lv[LP];
#pragma unroll
        for (int j = 0; j < LP; ++j)
            if (TK_T * j < total)  // (uniform)
                lv[j] = __hip_atomic_load(rl + min(t + TK_T * j, total - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int j = 0; j < LP; ++j)
            if (t + TK_T * j < total) cand[t + TK_T * j] = lv[j];
    }
    __syncthreads();
    // the merge: theta2 = the K-th largest list head (the lists are descending, so K lists hold an
    // entry >= theta2 and every one of the row's top K is >= it), or 1 when at most K heads are nonzero;
    // only the entries >= theta2 (typically little more than K) are ranked, by counting
    const uint64_t hd = t < a.nseg ? cand[t * K] : 0;
    if (t == 0) {
        theta2_s = 1;
        nc2_s = 0;
    }
    const int nzh = __syncthreads_count(hd != 0);
    if (nzh > K && hd != 0) {
        int above = 0;
        for (int l0 = 0; l0 < a.nseg; l0 += 8) {  // eight heads per LDS round trip
            uint64_t c[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) c[j] = cand[min(l0 + j, a.nseg - 1) * K];
#pragma unroll
            for (int j = 0; j < 8; ++j) above += (l0 + j < a.nseg && c[j] > hd) ? 1 : 0;
        }
        if (above == K - 1) theta2_s = hd;
    }
    __syncthreads();
    const uint64_t theta2 = theta2_s;
    uint64_t* c2 = cand + total;  // [total]
    for (int j = t; j < total; j += TK_T) {
        const uint64_t v = cand[j];
        if (v != 0 && v >= theta2) c2[atomicAdd(&nc2_s, 1u)] = v;
    }
    __syncthreads();
    const int nc2 = int(nc2_s);
    for (int e = t; e < nc2; e += TK_T) {
        const uint64_t v = c2[e];
        const int pos = count_above(c2, 0, nc2, v);
        if (pos < K) {
            const uint32_t idx = index_of<ORD>(v);
            a.indices[int64_t(row) * K + pos] = idx;
            if (ORD == ORDER_F32) {
                const uint32_t u = f32 ? static_cast<const uint32_t*>(xr)[idx]
                                       : uint32_t(static_cast<const uint16_t*>(xr)[idx]) << 16;
                static_cast<float*>(a.values)[int64_t(row) * K + pos] = __uint_as_float(u);
            } else {
                static_cast<uint16_t*>(a.values)[int64_t(row) * K + pos] = static_cast<const uint16_t*>(xr)[idx];
            }
        }
    }
    if (a.pick && t == 0) {
        uint64_t b = 0;
        for (int w = 0; w < a.nseg; ++w) {
            const uint64_t q = __hip_atomic_load(a.amax + int64_t(row) * a.nseg + w, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            b = q > b ? q : b;
        }
        a.argmax[row] = index_of<ORDER_ARGMAX>(b);
    }
    if (t == 0) __hip_atomic_store(a.counter + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// segments: about 2 x 256 work-groups over all rows, at least 1024 elements each, at most 640 / k
void plan(int64_t rows, int64_t n, int64_t k, int& nseg, int& seg) {
    int64_t s = std::max<int64_t>(1, std::min<int64_t>(TK_MAXSEG, 512 / rows));
    s = std::min<int64_t>(s, std::max<int64_t>(1, n / 1024));
    s = std::min<int64_t>(s, std::max<int64_t>(4, 640 / k));  // the merge holds the lists twice in LDS
    int64_t len = (n + s - 1) / s;
    len = (len + 63) / 64 * 64;
    nseg = int((n + len - 1) / len);
    seg = int(len);
}

size_t lds_bytes(int k, int nseg, int seg) {
    const size_t cand = size_t(k) * size_t((seg + TK_T - 1) / TK_T);
    return (TK_T + std::max(cand, 2 * size_t(nseg) * k)) * sizeof(uint64_t);
}

size_t workspace_bytes(int64_t rows) {
    return size_t(rows) * TK_MAXSEG * (TK_MAXK + 1) * sizeof(uint64_t) + 256;
}

int launch(const void* x, bool f32, int ord, int64_t rows, int64_t n, int64_t k, bool pick, void* values,
           int64_t* indices, int64_t* argmax, void* ws, size_t ws_bytes, hipStream_t stream) {
    MDX_CHECK(ws && aligned(ws, 256) && ws_bytes >= workspace_bytes(rows), "workspace: %zu bytes, 256-byte aligned",
              workspace_bytes(rows));
    int nseg, seg;
    plan(rows, n, k, nseg, seg);
    TopkArgs a{};
    a.x = x;
    a.n = n;
    a.rows = int(rows);
    a.k = int(k);
    a.nseg = nseg;
    a.seg = seg;
    a.f32 = f32;
    a.pick = pick;
    a.values = values;
    a.indices = indices;
    a.argmax = argmax;
    a.counter = static_cast<unsigned*>(ws);
    a.lists = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + 256);
    a.amax = a.lists + size_t(rows) * TK_MAXSEG * TK_MAXK;
    const size_t lds = lds_bytes(int(k), nseg, seg);
    MDX_CHECK(lds <= 64 * 1024, "top-k LDS plan %zu bytes exceeds 64 KiB", lds);
    const dim3 grid(unsigned(rows * nseg)), block(TK_T);
    if (ord == ORDER_BF16)
        hipLaunchKernelGGL((topk_kernel<ORDER_BF16, false>), grid, block, lds, stream, a);
    else if (ord == ORDER_ARGMAX)
        hipLaunchKernelGGL((topk_kernel<ORDER_ARGMAX, false>), grid, block, lds, stream, a);
    else if (f32)
        hipLaunchKernelGGL((topk_kernel<ORDER_F32, true>), grid, block, lds, stream, a);
    else
        hipLaunchKernelGGL((topk_kernel<ORDER_F32, false>), grid, block, lds, stream, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

namespace mdx {
namespace {

// Gumbel-max pick over each row's top k: score_j = vals[r, j] * (1 / temperature) + g_j, with
// g_j = -log(-log(clamp(u[r, j], 1e-20, 1))), every operation an fp32 rounding as torch's elementwise
// kernels round them (a tensor divided by a scalar is multiplied by the scalar's fp32 reciprocal);
// the first maximal score wins, as torch.argmax picks; out[r] = idx[r, j*]. One wave per row (k <= 64).
// The uniform of (seed, counter, row r, slot j): the SplitMix64 output (Steele, Lea and Flood 2014: state
// += 0x9E3779B97F4A7C15, then the two xor-shift-multiply rounds and a final xor-shift) of the state
// seed + (n + 1) * 0x9E3779B97F4A7C15, n = counter * 1024 + 64 r + j, whose top 23 bits k give
// (k + 0.5) * 2^-23, in (0, 1) and exact in fp32.
__device__ __forceinline__ float mix_uniform(uint64_t seed, int64_t counter, int r, int j) {
    const uint64_t n = uint64_t(counter) * 1024u + uint64_t(r) * 64u + uint64_t(j);
    uint64_t z = seed + (n + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float(uint32_t(z >> 41)) + 0.5f) * 1.1920928955078125e-7f;
}

// u == nullptr: the uniforms are mix_uniform(seed, counter[0], r, j) (counter read on the device)
__global__ __launch_bounds__(64) void topk_sample_kernel(const float* vals, const int64_t* idx, const float* u, float temp,
                                                         int64_t k, int64_t* out, const int64_t* counter, uint64_t seed) {
    const int r = blockIdx.x, j = threadIdx.x;
    float sc = -INFINITY;
    int at = 64;
    if (j < k) {
        const float uu = fminf(fmaxf(u ? u[r * k + j] : mix_uniform(seed, counter[0], r, j), 1e-20f), 1.0f);
        const float g = -logf(-logf(uu));
        sc = __fadd_rn(__fmul_rn(vals[r * k + j], __fdiv_rn(1.f, temp)), g);
        at = j;
    }
    // (max score, then the smaller position) over the wave; NaN scores lose to numbers
    for (int d = 32; d >= 1; d >>= 1) {
        const float os = __shfl_xor(sc, d, 64);
        const int oa = __shfl_xor(at, d, 64);
        const bool take = (os > sc) || (os == sc && oa < at) || (sc != sc && os == os);
        sc = take ? os : sc;
        at = take ? oa : at;
    }
    if (j == 0) out[r] = idx[r * k + (at < k ? at : 0)];
}

}  // namespace
}  // namespace mdx

extern "C" size_t mdx_topk_workspace(int64_t rows) { return workspace_bytes(std::max<int64_t>(rows, 1)); }

extern "C" int mdx_fast_topk(const uint16_t* x, int64_t V, int64_t k, int32_t argmax_order, uint16_t* values,
                             int64_t* indices, void* workspace, size_t workspace_bytes, void* stream) {
    MDX_CHECK(x && values && indices, "null pointer");
    MDX_CHECK(k >= 1 && k <= 8, "1 <= k <= 8");
    MDX_CHECK(!argmax_order || k == 1, "argmax order takes k = 1");
    MDX_CHECK(V >= 32768 && V < (int64_t(1) << 31), "one long row (32768 <= V < 2^31)");
    return launch(x, false, argmax_order ? ORDER_ARGMAX : ORDER_BF16, 1, V, k, false, values, indices, nullptr,
                  workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_fast_pick(const uint16_t* x, int64_t V, int64_t k, uint16_t* values, int64_t* indices,
                             int64_t* argmax, void* workspace, size_t workspace_bytes, void* stream) {
    MDX_CHECK(x && values && indices && argmax, "null pointer");
    MDX_CHECK(k >= 1 && k <= 8, "1 <= k <= 8");
    MDX_CHECK(V >= 32768 && V < (int64_t(1) << 31), "one long row (32768 <= V < 2^31)");
    return launch(x, false, ORDER_BF16, 1, V, k, true, values, indices, argmax, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream));
}

extern "C" int mdx_topk_rows(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t k, float* values,
                             int64_t* indices, void* workspace, size_t workspace_bytes, void* stream) {
    MDX_CHECK(x && values && indices, "null pointer");
    MDX_CHECK(x_dtype == MDX_DT_F32 || x_dtype == MDX_DT_BF16, "x: fp32 or bf16");
    MDX_CHECK(rows >= 1 && rows <= TK_MAXR, "1 <= rows <= 16");
    MDX_CHECK(k >= 1 && k <= TK_MAXK && n >= 4096 && n < (int64_t(1) << 31), "1 <= k <= 64, 4096 <= N < 2^31");
    return launch(x, x_dtype == MDX_DT_F32, ORDER_F32, rows, n, k, false, values, indices, nullptr, workspace,
                  workspace_bytes, static_cast<hipStream_t>(stream));
}

// ---- the allocation-free entry point --------------------------------------------------------------
// A file-scope device array stands in for the caller's workspace, sized for the largest call (16 rows):
// 16 x 64 segments x (64 + 1) ranks x 8 B + 256 B of counters = 532,736 B per device, held until the
// process ends. Host code never uses its name as an address: the per-device address comes from
// hipGetSymbolAddress with that device current.
namespace mdx {
namespace {
constexpr size_t TOPK_SCRATCH_BYTES = size_t(TK_MAXR) * TK_MAXSEG * (TK_MAXK + 1) * sizeof(uint64_t) + 256;
constexpr int SCRATCH_MAX_DEVICES = 64;

__global__ __launch_bounds__(64) void zero_words_kernel(unsigned* p) { p[threadIdx.x] = 0u; }

std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAX_DEVICES];
}  // namespace
}  // namespace mdx

static __device__ __align__(256) uint8_t scratch[mdx::TOPK_SCRATCH_BYTES];

namespace mdx {
namespace {
// The current device's copy of `scratch`; at the first call on a device its counter words (the first
// 256 bytes) are cleared by a fill kernel on `st` (a kernel, not a memset: it may be captured).
int scratch_of_current_device(hipStream_t st, void** out) {
    int dev = -1;
    MDX_HIP(hipGetDevice(&dev));
    MDX_CHECK(dev >= 0 && dev < SCRATCH_MAX_DEVICES, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        MDX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        MDX_CHECK(p != nullptr && aligned(p, 256), "scratch symbol address");
        hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(64), 0, st, static_cast<unsigned*>(p));
        MDX_LAUNCHED();
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MDX_OK;
}
}  // namespace
}  // namespace mdx

extern "C" int mdx_topk_rows_noalloc(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t k,
                                     float* values, int64_t* indices, void* stream) {
    MDX_CHECK(x && values && indices, "null pointer");
    MDX_CHECK(x_dtype == MDX_DT_F32 || x_dtype == MDX_DT_BF16, "x: fp32 or bf16");
    MDX_CHECK(rows >= 1 && rows <= TK_MAXR,
              "1 <= rows <= %d (the library's static top-k scratch holds %d rows; got %lld)", TK_MAXR, TK_MAXR,
              (long long)rows);
    MDX_CHECK(k >= 1 && k <= TK_MAXK && n >= 4096 && n < (int64_t(1) << 31), "1 <= k <= 64, 4096 <= N < 2^31");
    MDX_CHECK(workspace_bytes(rows) <= TOPK_SCRATCH_BYTES, "scratch size");
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = nullptr;
    if (int rc = scratch_of_current_device(st, &ws)) return rc;
    return launch(x, x_dtype == MDX_DT_F32, ORDER_F32, rows, n, k, false, values, indices, nullptr, ws,
                  TOPK_SCRATCH_BYTES, st);
}

extern "C" int mdx_topk_sample(const float* values, const int64_t* indices, const float* uniform, float temperature,
                               int64_t rows, int64_t k, int64_t* out, void* stream) {
    MDX_CHECK(values && indices && uniform && out, "null pointer");
    MDX_CHECK(rows >= 1 && rows <= 65535 && k >= 1 && k <= 64, "1 <= rows, 1 <= k <= 64");
    MDX_CHECK(temperature > 0.f, "temperature > 0");
    hipLaunchKernelGGL(mdx::topk_sample_kernel, dim3(unsigned(rows)), dim3(64), 0, static_cast<hipStream_t>(stream),
                       values, indices, uniform, temperature, k, out, nullptr, uint64_t(0));
    MDX_LAUNCHED();
    return MDX_OK;
}

extern "C" int mdx_topk_sample_seeded(const float* values, const int64_t* indices, uint64_t seed, const int64_t* counter,
                                      float temperature, int64_t rows, int64_t k, int64_t* out, void* stream) {
    MDX_CHECK(values && indices && counter && out, "null pointer");
    MDX_CHECK(rows >= 1 && rows <= 16 && k >= 1 && k <= 64, "1 <= rows <= 16, 1 <= k <= 64");
    MDX_CHECK(temperature > 0.f, "temperature > 0");
    hipLaunchKernelGGL(mdx::topk_sample_kernel, dim3(unsigned(rows)), dim3(64), 0, static_cast<hipStream_t>(stream),
                       values, indices, nullptr, temperature, k, out, counter, seed);
    MDX_LAUNCHED();
    return MDX_OK;
}
