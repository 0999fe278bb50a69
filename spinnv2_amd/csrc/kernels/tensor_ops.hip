// Indexing and layout ops of the YOLO op set: Split, Slice, Transpose, Tile,
// Gather, GatherElements, TopK.  Reference semantics:
//   runtime/kernels/reference/tensor/split.c, slice.c, gather.c,
//   gather_elements.c, topk.c and shape/transpose.c, shape/tile.c.
// Tensors are float (index tensors hold integral floats, as in the
// reference).  Every kernel is a grid-stride loop in which consecutive lanes
// write consecutive output elements; source addresses come from per-node
// stride tables computed on the host.  Scalar parameters the reference reads
// from constant input tensors (Slice starts/ends/axes/steps, TopK k) are read
// from the package on the host; index tensors (Gather, GatherElements) are
// read on the device, so they may be produced by earlier nodes (TopK).
// Out-of-range indices, undefined in the reference, read 0 here.
#include <algorithm>
#include <cstring>

#include "common.hpp"
#include "kernels.hpp"

namespace spk::kern {

namespace {

constexpr int kRank = 8;

struct StrideMap {
    int rank;
    int64_t ydim[kRank];    // output shape
    int64_t src[kRank];     // source element stride per output dim (Transpose), or source dims (Tile)
    int64_t sstride[kRank]; // source strides (Tile)
};

// y[i] = x[sum_d coord_d(i) * src[d]]  (Transpose: src = input stride of
// the permuted axis)
__global__ void __launch_bounds__(256) permute_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n,
                                                      StrideMap m) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        size_t t = i;
        int64_t off = 0;
        for (int d = m.rank - 1; d >= 0; d--) {
            const int64_t c = static_cast<int64_t>(t % m.ydim[d]);
            t /= m.ydim[d];
            off += c * m.src[d];
        }
        y[i] = x[off];
    }
}

// Permutations that keep the last axis: every output row (the last axis, L
// elements) is one contiguous input row.  One workgroup per output row
// (grid-stride over rows), lanes along the row, 16-byte accesses when L
// and the row starts allow them.
__global__ void __launch_bounds__(256) permute_rows(const float *__restrict__ x, float *__restrict__ y, size_t rows,
                                                    int L, StrideMap m) {
    const bool vec = (L & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    for (size_t r = blockIdx.x; r < rows; r += gridDim.x) {
        // the output row's coordinates over ranks 0 .. rank-2 give the source row
        size_t t = r;
        int64_t off = 0;
        for (int d = m.rank - 2; d >= 0; d--) {
            const int64_t c = static_cast<int64_t>(t % m.ydim[d]);
            t /= m.ydim[d];
            off += c * m.src[d];
        }
        const float *src = x + off;
        float *dst = y + r * static_cast<size_t>(L);
        if (vec && (off & 3) == 0) {
            const floatx4 *s4 = reinterpret_cast<const floatx4 *>(src);
            floatx4 *d4 = reinterpret_cast<floatx4 *>(dst);
            for (int i = threadIdx.x; i < L / 4; i += 256) d4[i] = s4[i];
        } else {
            for (int i = threadIdx.x; i < L; i += 256) dst[i] = src[i];
        }
    }
}

// Permutations that swap the last two axes and keep the rest: batched
// transposes y[b][c][r] = x[b][r][c] of R x C matrices.  A workgroup moves a
// 32 x 32 tile through LDS (row pitch 33: the column reads hit 32 different
// banks), reading rows of x and writing rows of y coalesced.
constexpr int kTp = 32;

__global__ void __launch_bounds__(256) transpose_tiles(const float *__restrict__ x, float *__restrict__ y, int R, int C,
                                                       int tiles_c, int tiles_per_mat, size_t total_tiles) {
    __shared__ float tile[kTp][kTp + 1];
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
    for (size_t t = blockIdx.x; t < total_tiles; t += gridDim.x) {
        const size_t b = t / tiles_per_mat;
        const int tm = static_cast<int>(t - b * tiles_per_mat);
        const int r0 = (tm / tiles_c) * kTp, c0 = (tm % tiles_c) * kTp;
        const float *xb = x + b * static_cast<size_t>(R) * C;
        float *yb = y + b * static_cast<size_t>(R) * C;
        __syncthreads();  // the previous tile's reads of `tile` are done
#pragma unroll
        for (int i = 0; i < kTp; i += 8) {
            const int r = r0 + ty + i, c = c0 + tx;
            if (r < R && c < C) tile[ty + i][tx] = xb[static_cast<size_t>(r) * C + c];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kTp; i += 8) {
            const int c = c0 + ty + i, r = r0 + tx;
            if (r < R && c < C) yb[static_cast<size_t>(c) * R + r] = tile[tx][ty + i];
        }
    }
}

// y[i] = x[coords(i) mod xdim]  (reference shape/tile.c:13-19)
__global__ void __launch_bounds__(256) tile_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n,
                                                   StrideMap m) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        size_t t = i;
        int64_t off = 0;
        for (int d = m.rank - 1; d >= 0; d--) {
            const int64_t c = static_cast<int64_t>(t % m.ydim[d]);
            t /= m.ydim[d];
            off += (c % m.src[d]) * m.sstride[d];
        }
        y[i] = x[off];
    }
}

// Block copy: y[o * y_stride + j] = x[x_base + o * x_stride + j] for j < block
// (Split outputs, Slice with step 1).
__global__ void __launch_bounds__(256) block_copy(const float *__restrict__ x, float *__restrict__ y, size_t outer,
                                                  size_t block, size_t x_stride, size_t x_base, size_t y_stride) {
    const size_t n = outer * block;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        const size_t o = i / block, j = i - o * block;
        y[o * y_stride + j] = x[x_base + o * x_stride + j];
    }
}

// The same copy in 16-byte units: grid.y walks the blocks, grid.x the
// float4s of a block, so no division per element.
__global__ void __launch_bounds__(256) block_copy4(const floatx4 *__restrict__ x, floatx4 *__restrict__ y, size_t outer,
                                                   size_t block4, size_t x_stride4, size_t y_stride4) {
    for (size_t o = blockIdx.y; o < outer; o += gridDim.y)
        for (size_t j = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; j < block4;
             j += static_cast<size_t>(gridDim.x) * 256)
            y[o * y_stride4 + j] = x[o * x_stride4 + j];
}

// Several block copies in one launch: grid.z is the segment, grid.y walks
// its blocks, grid.x the float4s of a block.
constexpr int kMaxCopySegs = 8;
struct CopySegs4 {
    const floatx4 *x[kMaxCopySegs];
    floatx4 *y[kMaxCopySegs];
    size_t block4[kMaxCopySegs], x_stride4[kMaxCopySegs], y_stride4[kMaxCopySegs];
};
__global__ void __launch_bounds__(256) block_copy4_multi(CopySegs4 c, size_t outer) {
    const int k = static_cast<int>(blockIdx.z);
    const floatx4 *x = c.x[k];
    floatx4 *y = c.y[k];
    const size_t block4 = c.block4[k], xs = c.x_stride4[k], ys = c.y_stride4[k];
    for (size_t o = blockIdx.y; o < outer; o += gridDim.y)
        for (size_t j = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; j < block4;
             j += static_cast<size_t>(gridDim.x) * 256)
            y[o * ys + j] = x[o * xs + j];
}

// Slice with a step: y[(o*out + s)*inner + t] = x[(o*dim + start + s*step)*inner + t]
__global__ void __launch_bounds__(256) slice_kernel(const float *__restrict__ x, float *__restrict__ y, size_t outer,
                                                    int64_t out, int64_t dim, int64_t start, int64_t step, size_t inner) {
    const size_t n = outer * static_cast<size_t>(out) * inner;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        const size_t t = i % inner;
        const size_t q = i / inner;
        const int64_t s = static_cast<int64_t>(q % out);
        const size_t o = q / out;
        y[i] = x[(o * dim + start + s * step) * inner + t];
    }
}

// Gather (reference tensor/gather.c:28-36):
// y[(o*J + j)*inner + t] = data[(o*dim + ix_j)*inner + t], ix = (int)idx, +dim if negative
__global__ void __launch_bounds__(256) gather_kernel(const float *__restrict__ data, const float *__restrict__ idx,
                                                     float *__restrict__ y, size_t outer, size_t J, int64_t dim,
                                                     size_t inner) {
    const size_t n = outer * J * inner;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        const size_t t = i % inner;
        const size_t q = i / inner;
        const size_t j = q % J;
        const size_t o = q / J;
        int ix = static_cast<int>(idx[j]);
        if (ix < 0) ix += static_cast<int>(dim);
        y[i] = (ix >= 0 && ix < dim) ? data[(o * dim + ix) * inner + t] : 0.0f;
    }
}

// GatherElements (reference tensor/gather_elements.c:17-25): y has the
// index tensor's shape; coordinate `axis` is replaced by the index value.
__global__ void __launch_bounds__(256) gather_elements_kernel(const float *__restrict__ data,
                                                              const float *__restrict__ idx, float *__restrict__ y,
                                                              size_t n, StrideMap m, int axis, int64_t dim) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        size_t t = i;
        int64_t off = 0;
        for (int d = m.rank - 1; d >= 0; d--) {
            const int64_t c = static_cast<int64_t>(t % m.ydim[d]);
            t /= m.ydim[d];
            if (d != axis) off += c * m.sstride[d];
        }
        int g = static_cast<int>(idx[i]);
        if (g < 0) g += static_cast<int>(dim);
        y[i] = (g >= 0 && g < dim) ? data[off + static_cast<int64_t>(g) * m.sstride[axis]] : 0.0f;
    }
}

// ---------------------------------------------------------------- TopK

constexpr int kTopkMaxK = 1024;
constexpr int kTopkRowLds = 16384;  // rows up to this length are staged in LDS

// order-preserving key of a float: larger float -> larger unsigned
__device__ __forceinline__ uint32_t fkey(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct HeapPair {
    float v;
    uint32_t idx;
};

// The reference's sift-down from node i of a heap of n (tensor/topk.c:8-30):
// the smaller child (the larger one for largest = 0) moves up while it is
// strictly better-placed than the sifted element, the left child winning
// ties.  The sifted element is carried down and stored once.
__device__ __forceinline__ void topk_sift(HeapPair *h, int n, int i, int largest) {
    const HeapPair e = h[i];
    for (;;) {
        const int l = 2 * i + 1;
        if (l >= n) break;
        const int r = l + 1;
        // both children in one round trip (the right one clamped into the heap)
        const HeapPair cl = h[l];
        const HeapPair cr = h[min(r, n - 1)];
        int m = i;
        HeapPair mv = e;
        if (largest ? (cl.v < mv.v) : (cl.v > mv.v)) {
            m = l;
            mv = cl;
        }
        if (r < n && (largest ? (cr.v < mv.v) : (cr.v > mv.v))) {
            m = r;
            mv = cr;
        }
        if (m == i) break;
        h[i] = mv;
        i = m;
    }
    h[i] = e;
}

// The reference's insertion (tensor/topk.c:87-92 and 97-101): e replaces
// the root and is sifted down (topk_sift's rule), two levels per round trip
// to LDS (a node's children and grandchildren are read together; only the
// path's nodes are written).  Returns the value left at the root.
__device__ __forceinline__ float topk_sift_root(HeapPair *h, int n, HeapPair e, int largest) {
    auto above = [&](float a, float b) { return largest ? (a < b) : (a > b); };  // a belongs above b
    int i = 0;
    float rootv = e.v;
    for (;;) {
        const int l = 2 * i + 1;
        if (l >= n) break;
        const int g = 2 * l + 1;  // children of l: g, g + 1; of l + 1: g + 2, g + 3
        const HeapPair c0 = h[l], c1 = h[min(l + 1, n - 1)];
        const HeapPair g0 = h[min(g, n - 1)], g1 = h[min(g + 1, n - 1)];
        const HeapPair g2 = h[min(g + 2, n - 1)], g3 = h[min(g + 3, n - 1)];
        int m = i;
        HeapPair mv = e;
        if (above(c0.v, mv.v)) {
            m = l;
            mv = c0;
        }
        if (l + 1 < n && above(c1.v, mv.v)) {
            m = l + 1;
            mv = c1;
        }
        if (m == i) break;
        h[i] = mv;
        if (i == 0) rootv = mv.v;
        const bool left = m == l;
        i = m;
        const int l2 = 2 * i + 1;
        if (l2 >= n) break;
        const HeapPair d0 = left ? g0 : g2, d1 = left ? g1 : g3;
        m = i;
        mv = e;
        if (above(d0.v, mv.v)) {
            m = l2;
            mv = d0;
        }
        if (l2 + 1 < n && above(d1.v, mv.v)) {
            m = l2 + 1;
            mv = d1;
        }
        if (m == i) break;
        h[i] = mv;
        i = m;
    }
    h[i] = e;
    return rootv;
}

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;

// Inclusive prefix sum of v over the workgroup's threads in thread order:
// shuffles within each wave, the wave totals through LDS.
__device__ __forceinline__ uint32_t topk_scan(uint32_t v, uint32_t *wsum, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    for (int w = 0; w < wave; w++) v += wsum[w];
    return v;
}

// One workgroup of 1024 threads per (outer, inner) row.  Radix select over
// order-preserving keys finds the k-th best value T; when exactly k elements
// are at least as good as T (no tie straddles the k-th place, the usual
// case) they are the reference's selection; otherwise the reference's heap
// is replayed.  The selection is then ordered by (value, best first; index
// ascending), the reference's comparator (tensor/topk.c:28-41): its k keys
// (value key, inverted index) are distinct, so each one's output position is
// the number of keys above it.
//
// Rows of up to kTopkRowLds elements are read from memory once, into LDS
// (several loads per thread in flight), and every later pass reads LDS.  The
// replay of the reference's heap (tensor/topk.c:71-101) when values tie
// across the k-th place:
//   * the heap of the first k elements is built by all threads, Floyd's
//     sift-downs level by level from the deepest (the nodes of one level
//     root disjoint subtrees, so their order within the level is free, and
//     every deeper level precedes them, as in the reference's descending
//     loop);
//   * the heap's root only gets better as elements enter, so an element no
//     better than the root after heapify never enters: all threads mark the
//     others first (a bit per element), and one wave walks only the marked
//     ones in element order, testing 64 at a time against the current root;
//     lane 0 inserts the first that enters and the rest are re-tested
//     against the new root.
template <bool STAGED>
__global__ void __launch_bounds__(kTopkThreads) topk_kernel(const float *__restrict__ x, float *__restrict__ values,
                                                            float *__restrict__ indices, size_t inner, int dim, int k,
                                                            int largest) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wsum[kTopkWaves];
    __shared__ uint32_t s_prefix, s_remaining, s_count;
    __shared__ unsigned long long keys[kTopkMaxK];
    __shared__ HeapPair heap[kTopkMaxK];
    __shared__ unsigned long long cmask[STAGED ? kTopkRowLds / 64 : 1];
    __shared__ float rowbuf[STAGED ? kTopkRowLds : 1];
    const size_t row = blockIdx.x;
    const size_t o = row / inner, in = row % inner;
    const size_t base = o * static_cast<size_t>(dim) * inner + in;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // -0 and +0 compare equal in the reference: give them one key
    auto key_of = [&](float v) -> uint32_t {
        const uint32_t kk = fkey(v == 0.0f ? 0.0f : v);
        return largest ? kk : ~kk;
    };
    // (a compile-time choice: a run-time one merges both into generic loads)
    auto at = [&](int d) -> float {
        if constexpr (STAGED)
            return rowbuf[d];
        else
            return x[base + static_cast<size_t>(d) * inner];
    };

    if constexpr (STAGED) {
        constexpr int U = 4;
        for (int d0 = 0; d0 < dim; d0 += kTopkThreads * U) {
            float v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int d = d0 + u * kTopkThreads + tid;
                v[u] = d < dim ? x[base + static_cast<size_t>(d) * inner] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int d = d0 + u * kTopkThreads + tid;
                if (d < dim) rowbuf[d] = v[u];
            }
        }
    }

    uint32_t prefix = 0, mask = 0, remaining = static_cast<uint32_t>(k), eq_count = 0;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int d0 = 0; d0 < dim; d0 += kTopkThreads) {
            const int d = d0 + tid;
            const uint32_t kk = d < dim ? key_of(at(d)) : 0u;
            const bool act = d < dim && (kk & mask) == prefix;
            const uint32_t bin = (kk >> shift) & 255u;
            // a wave whose counted elements all fall in one bin (ties) adds
            // them with one atomic
            const unsigned long long am = __ballot(act);
            if (am == 0ull) continue;
            const int first = __ffsll(static_cast<long long>(am)) - 1;
            const uint32_t b0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bin), first));
            if (__ballot(act && bin == b0) == am) {
                if (lane == first) atomicAdd(&hist[b0], static_cast<uint32_t>(__popcll(am)));
            } else if (act) {
                atomicAdd(&hist[bin], 1u);
            }
        }
        __syncthreads();
        // digit: the largest b whose suffix count S(b) = hist[b] + ... +
        // hist[255] reaches `remaining` (thread t < 256 holds bin 255 - t)
        const uint32_t b = 255u - static_cast<uint32_t>(tid & 255);
        const uint32_t hb = tid < 256 ? hist[b] : 0u;
        const uint32_t S = topk_scan(hb, wsum, tid);
        if (tid < 256 && S >= remaining && S - hb < remaining) {
            s_prefix = prefix | (b << shift);
            s_remaining = remaining - (S - hb);
            s_count = hb;
        }
        __syncthreads();
        prefix = s_prefix;
        remaining = s_remaining;
        eq_count = s_count;
        mask |= 255u << shift;
        __syncthreads();
    }
    // T = prefix; `remaining` of the eq_count elements equal to T are needed
    const bool ambiguous = eq_count != remaining;
    if (tid == 0) s_count = 0;
    __syncthreads();
    if (!ambiguous) {
        for (int d0 = 0; d0 < dim; d0 += kTopkThreads) {
            const int d = d0 + tid;
            const uint32_t kk = d < dim ? key_of(at(d)) : 0u;
            const bool sel = d < dim && kk >= prefix;
            const unsigned long long sm = __ballot(sel);
            if (sm == 0ull) continue;
            const int first = __ffsll(static_cast<long long>(sm)) - 1;
            uint32_t slot = 0;
            if (lane == first) slot = atomicAdd(&s_count, static_cast<uint32_t>(__popcll(sm)));
            slot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(slot), first));
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(sm >> 32),
                                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(sm), 0u));
            if (sel) keys[slot + below] = (static_cast<unsigned long long>(kk) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(d));
        }
    } else {
        for (int i = tid; i < k; i += kTopkThreads) heap[i] = HeapPair{at(i), static_cast<uint32_t>(i)};
        __syncthreads();
        const int last = k / 2 - 1;  // the reference sifts nodes last .. 0
        for (int D = last >= 0 ? 31 - __clz(last + 1) : -1; D >= 0; D--) {
            const int hi = min((2 << D) - 2, last);
            for (int i = (1 << D) - 1 + tid; i <= hi; i += kTopkThreads) topk_sift(heap, k, i, largest);
            __syncthreads();
        }
        const float root0 = heap[0].v;
        if constexpr (STAGED) {
            const int nblk = (dim - k + 63) / 64;
            for (int bk = wave; bk < nblk; bk += kTopkWaves) {
                const int d = k + 64 * bk + lane;
                const float v = d < dim ? rowbuf[d] : 0.0f;
                const unsigned long long cm = __ballot(d < dim && (largest ? (v > root0) : (v < root0)));
                if (lane == 0) cmask[bk] = cm;
            }
            __syncthreads();
            if (wave == 0) {
                float root = root0;
                for (int b0 = 0; b0 < nblk; b0 += 64) {
                    const unsigned long long mine = b0 + lane < nblk ? cmask[b0 + lane] : 0ull;
                    unsigned long long nz = __ballot(mine != 0ull);
                    while (nz) {
                        const int jb = __ffsll(static_cast<long long>(nz)) - 1;
                        nz &= nz - 1;
                        const unsigned long long cm = __shfl(mine, jb);
                        const int d0 = k + 64 * (b0 + jb);
                        const bool cand = (cm >> lane) & 1ull;
                        const float v = cand ? rowbuf[d0 + lane] : 0.0f;
                        unsigned long long m = __ballot(cand && (largest ? (v > root) : (v < root)));
                        while (m) {
                            const int j = __ffsll(static_cast<long long>(m)) - 1;
                            const float vj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
                            float r = 0.0f;
                            if (lane == 0) r = topk_sift_root(heap, k, HeapPair{vj, static_cast<uint32_t>(d0 + j)}, largest);
                            root = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
                            m = __ballot(cand && lane > j && (largest ? (v > root) : (v < root)));
                        }
                    }
                }
            }
        } else if (wave == 0) {  // rows beyond the LDS: the same walk over every element, from memory
            float root = root0;
            for (int d0 = k; d0 < dim; d0 += 64) {
                const int d = d0 + lane;
                const bool live = d < dim;
                const float v = live ? x[base + static_cast<size_t>(d) * inner] : 0.0f;
                unsigned long long m = __ballot(live && (largest ? (v > root) : (v < root)));
                while (m) {
                    const int j = __ffsll(static_cast<long long>(m)) - 1;
                    const float vj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
                    float r = 0.0f;
                    if (lane == 0) r = topk_sift_root(heap, k, HeapPair{vj, static_cast<uint32_t>(d0 + j)}, largest);
                    root = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
                    m = __ballot(live && lane > j && (largest ? (v > root) : (v < root)));
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < k; i += kTopkThreads)
            keys[i] = (static_cast<unsigned long long>(key_of(heap[i].v)) << 32) | (0xFFFFFFFFu - heap[i].idx);
    }
    __syncthreads();
    // output position of each selected key: the number of keys above it
    // (descending order, as the reference's comparator sorts)
    for (int i = tid; i < k; i += kTopkThreads) {
        const unsigned long long ki = keys[i];
        int rank = 0;
#pragma unroll 8
        for (int j = 0; j < k; j++) rank += keys[j] > ki ? 1 : 0;
        const uint32_t d = 0xFFFFFFFFu - static_cast<uint32_t>(ki & 0xFFFFFFFFull);
        const size_t out = (o * static_cast<size_t>(k) + rank) * inner + in;
        values[out] = at(static_cast<int>(d));
        indices[out] = static_cast<float>(d);
    }
}

void shape_of(const Spkv2TensorRecord *r, int64_t *dims) {
    for (int i = 0; i < kRank; i++) dims[i] = i < r->rank ? r->shape[i] : 1;
}

void strides_of(const Spkv2TensorRecord *r, int64_t *st) {
    int64_t s = 1;
    for (int i = r->rank - 1; i >= 0; i--) {
        st[i] = s;
        s *= r->shape[i];
    }
}

int norm_axis(int axis, int rank) { return axis < 0 ? axis + rank : axis; }

// first value of a constant float tensor (from the package), or `fallback`
// when the input is absent
bool const_scalar(Spkv2Context *ctx, const Spkv2NodeRecord *node, int input, float *out) {
    if (node->input_count <= input || node->inputs[input] == 0xFFFFu) return false;
    const uint8_t *h = host_weight_data(ctx, node->inputs[input]);
    if (!h) return false;
    memcpy(out, h, sizeof(float));
    return true;
}

}  // namespace

int transpose_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]), *yr = rec(ctx, node->outputs[0]);
    if (xr->rank > kRank) return -11;
    StrideMap m{};
    m.rank = yr->rank;
    shape_of(yr, m.ydim);
    int64_t xs[kRank];
    strides_of(xr, xs);
    // reference shape/transpose.c:14-18: x coord perm[d] = y coord d
    for (int d = 0; d < xr->rank; d++) {
        const int src_axis = attr.extra_count > 0 ? attr.extra[d] : d;
        if (src_axis < 0 || src_axis >= xr->rank) return -11;
        m.src[d] = xs[src_axis];
    }
    const size_t n = elem_count(yr);
    if (n == 0) return 0;
    const int rank = xr->rank;
    auto perm = [&](int d) { return attr.extra_count > 0 ? static_cast<int>(attr.extra[d]) : d; };
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    float *y = dptr<float>(ctx, node->outputs[0]);
    bool keeps_last = rank >= 2 && perm(rank - 1) == rank - 1;
    bool swaps_last2 = rank >= 2 && perm(rank - 1) == rank - 2 && perm(rank - 2) == rank - 1;
    for (int d = 0; d + 2 < rank; d++) swaps_last2 = swaps_last2 && perm(d) == d;
    if (keeps_last && xr->shape[rank - 1] >= 64) {
        set_kernel_name(ctx, node, "transpose_rows");
        const int L = static_cast<int>(xr->shape[rank - 1]);
        const size_t rows = n / static_cast<size_t>(L);
        hipLaunchKernelGGL(permute_rows, dim3(static_cast<unsigned>(std::min<size_t>(rows, 65536))), dim3(256), 0,
                           ctx->stream, x, y, rows, L, m);
        return launch_status("transpose");
    }
    if (swaps_last2) {
        set_kernel_name(ctx, node, "transpose_tiles");
        const int R = static_cast<int>(xr->shape[rank - 2]), C = static_cast<int>(xr->shape[rank - 1]);
        const int tiles_r = (R + kTp - 1) / kTp, tiles_c = (C + kTp - 1) / kTp;
        const size_t total = n / (static_cast<size_t>(R) * C) * tiles_r * tiles_c;
        hipLaunchKernelGGL(transpose_tiles, dim3(static_cast<unsigned>(std::min<size_t>(total, 65536))), dim3(256), 0,
                           ctx->stream, x, y, R, C, tiles_c, tiles_r * tiles_c, total);
        return launch_status("transpose");
    }
    set_kernel_name(ctx, node, "transpose");
    hipLaunchKernelGGL(permute_kernel, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream, x, y, n, m);
    return launch_status("transpose");
}

int tile_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]), *yr = rec(ctx, node->outputs[0]);
    if (xr->rank != yr->rank || xr->rank > kRank) return -11;
    StrideMap m{};
    m.rank = yr->rank;
    shape_of(yr, m.ydim);
    shape_of(xr, m.src);
    strides_of(xr, m.sstride);
    const size_t n = elem_count(yr);
    if (n == 0) return 0;
    set_kernel_name(ctx, node, "tile");
    hipLaunchKernelGGL(tile_kernel, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream,
                       dptr<const float>(ctx, node->inputs[0]), dptr<float>(ctx, node->outputs[0]), n, m);
    return launch_status("tile");
}

// y[o * y_stride + j] = x[x_base + o * x_stride + j] for o < outer, j < block
// (elements): 16-byte copies when every offset and both pointers allow it.
int strided_block_copy(hipStream_t s, const float *x, float *y, size_t outer, size_t block, size_t x_stride,
                       size_t x_base, size_t y_stride) {
    if (outer * block == 0) return 0;
    const bool vec = block % 4 == 0 && x_stride % 4 == 0 && x_base % 4 == 0 && y_stride % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    if (vec) {
        const size_t block4 = block / 4;
        const unsigned gx = static_cast<unsigned>(std::min<size_t>((block4 + 255) / 256, 1024));
        const unsigned gy = static_cast<unsigned>(std::min<size_t>(outer, 65535));
        hipLaunchKernelGGL(block_copy4, dim3(gx, gy), dim3(256), 0, s, reinterpret_cast<const floatx4 *>(x + x_base),
                           reinterpret_cast<floatx4 *>(y), outer, block4, x_stride / 4, y_stride / 4);
    } else {
        hipLaunchKernelGGL(block_copy, dim3(grid_for(outer * block, 256)), dim3(256), 0, s, x, y, outer, block,
                           x_stride, x_base, y_stride);
    }
    return launch_status("block_copy");
}

int multi_block_copy(hipStream_t s, const CopySeg *segs, int count, size_t outer) {
    CopySegs4 c = {};
    int k = 0;
    size_t max4 = 0;
    auto flush = [&]() -> int {
        if (k == 0) return 0;
        const unsigned gx = static_cast<unsigned>(std::min<size_t>((max4 + 255) / 256, 1024));
        const unsigned gy = static_cast<unsigned>(std::min<size_t>(outer, 65535));
        hipLaunchKernelGGL(block_copy4_multi, dim3(gx, gy, static_cast<unsigned>(k)), dim3(256), 0, s, c, outer);
        k = 0;
        max4 = 0;
        return launch_status("block_copy");
    };
    for (int i = 0; i < count; i++) {
        const CopySeg &g = segs[i];
        if (outer * g.block == 0) continue;
        const bool vec = g.block % 4 == 0 && g.x_stride % 4 == 0 && g.x_base % 4 == 0 && g.y_stride % 4 == 0 &&
                         reinterpret_cast<uintptr_t>(g.x) % 16 == 0 && reinterpret_cast<uintptr_t>(g.y) % 16 == 0;
        if (!vec) {
            if (int rc = strided_block_copy(s, g.x, g.y, outer, g.block, g.x_stride, g.x_base, g.y_stride)) return rc;
            continue;
        }
        c.x[k] = reinterpret_cast<const floatx4 *>(g.x + g.x_base);
        c.y[k] = reinterpret_cast<floatx4 *>(g.y);
        c.block4[k] = g.block / 4;
        c.x_stride4[k] = g.x_stride / 4;
        c.y_stride4[k] = g.y_stride / 4;
        max4 = std::max(max4, g.block / 4);
        if (++k == kMaxCopySegs)
            if (int rc = flush()) return rc;
    }
    return flush();
}

int split_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    const int axis = norm_axis(attr.axis, xr->rank);
    if (axis < 0 || axis >= xr->rank) return -11;
    size_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= xr->shape[i];
    for (int i = axis + 1; i < xr->rank; i++) inner *= xr->shape[i];
    const size_t x_axis = xr->shape[axis];
    size_t axis_offset = 0;
    // every output a channel-slice view of the input (set up at prepare):
    // the outputs already are the input's channel ranges
    if (node->id < ctx->view_split.size() && ctx->view_split[node->id] && live_view(ctx, node->inputs[0])) {
        set_kernel_name(ctx, node, "split_views");
        return 0;
    }
    // the input as a view in its natural layout (the buffer a detection-head
    // chain's convs wrote in place)
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    if (const Spkv2TensorView *v = live_view(ctx, node->inputs[0])) {
        if (v->img_elems != static_cast<int64_t>(x_axis * inner) || (v->ch_elems != 0 && axis == 1 &&
                                                                    v->ch_elems != static_cast<int64_t>(inner)))
            return SPKV2_E_UNSUPPORTED;  // not set up that way
        x = reinterpret_cast<const float *>(v->base);
    }
    set_kernel_name(ctx, node, "split");
    CopySeg segs[4];  // a node record has at most four outputs
    int count = 0;
    for (uint16_t k = 0; k < node->output_count && k < 4; k++) {
        const Spkv2TensorRecord *yr = rec(ctx, node->outputs[k]);
        const size_t block = static_cast<size_t>(yr->shape[axis]) * inner;
        if (axis_offset + yr->shape[axis] > x_axis) return -11;
        segs[count++] = CopySeg{x, dptr<float>(ctx, node->outputs[k]), block, x_axis * inner, axis_offset * inner, block};
        axis_offset += yr->shape[axis];
    }
    return multi_block_copy(ctx->stream, segs, count, outer);  // one launch for the aligned outputs
}

int slice_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    // reference tensor/slice.c:12-49: starts/ends (and optional axes, steps)
    // are float constant inputs; only their first value is used
    float fs = 0.0f, fe = 0.0f, fa = 0.0f, fst = 1.0f;
    if (!const_scalar(ctx, node, 1, &fs) || !const_scalar(ctx, node, 2, &fe)) return SPKV2_E_UNSUPPORTED;
    (void)const_scalar(ctx, node, 3, &fa);
    (void)const_scalar(ctx, node, 4, &fst);
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    int64_t start = static_cast<int64_t>(fs), end = static_cast<int64_t>(fe);
    int axis = static_cast<int>(fa);
    const int64_t step = static_cast<int64_t>(static_cast<int>(fst));
    if (axis < 0) axis += xr->rank;
    if (axis < 0 || axis >= xr->rank || step <= 0) return -11;
    size_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= xr->shape[i];
    for (int i = axis + 1; i < xr->rank; i++) inner *= xr->shape[i];
    const int64_t dim = xr->shape[axis];
    if (start < 0) start += dim;
    if (end < 0) end += dim;
    if (end > dim) end = dim;
    if (start < 0) start = 0;
    const int64_t out = (end - start + step - 1) / step;
    if (out <= 0 || outer * inner == 0) return 0;
    if (start + (out - 1) * step >= dim) return -11;
    set_kernel_name(ctx, node, "slice");
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    float *y = dptr<float>(ctx, node->outputs[0]);
    const size_t n = outer * static_cast<size_t>(out) * inner;
    if (step == 1)
        return strided_block_copy(ctx->stream, x, y, outer, static_cast<size_t>(out) * inner,
                                  static_cast<size_t>(dim) * inner, static_cast<size_t>(start) * inner,
                                  static_cast<size_t>(out) * inner);
    else
        hipLaunchKernelGGL(slice_kernel, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream, x, y, outer, out, dim,
                           start, step, inner);
    return launch_status("slice");
}

int gather_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *dr = rec(ctx, node->inputs[0]), *ir = rec(ctx, node->inputs[1]);
    const int axis = norm_axis(attr.axis, dr->rank);
    if (axis < 0 || axis >= dr->rank) return -11;
    size_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= dr->shape[i];
    for (int i = axis + 1; i < dr->rank; i++) inner *= dr->shape[i];
    const size_t J = elem_count(ir);
    const size_t n = outer * J * inner;
    if (n == 0) return 0;
    set_kernel_name(ctx, node, "gather");
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream,
                       dptr<const float>(ctx, node->inputs[0]), dptr<const float>(ctx, node->inputs[1]),
                       dptr<float>(ctx, node->outputs[0]), outer, J, static_cast<int64_t>(dr->shape[axis]), inner);
    return launch_status("gather");
}

int gather_elements_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *dr = rec(ctx, node->inputs[0]), *ir = rec(ctx, node->inputs[1]);
    const int axis = norm_axis(attr.axis, dr->rank);
    if (axis < 0 || axis >= dr->rank || ir->rank != dr->rank || dr->rank > kRank) return -11;
    StrideMap m{};
    m.rank = ir->rank;
    shape_of(ir, m.ydim);
    strides_of(dr, m.sstride);
    const size_t n = elem_count(ir);
    if (n == 0) return 0;
    set_kernel_name(ctx, node, "gather_elements");
    hipLaunchKernelGGL(gather_elements_kernel, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream,
                       dptr<const float>(ctx, node->inputs[0]), dptr<const float>(ctx, node->inputs[1]),
                       dptr<float>(ctx, node->outputs[0]), n, m, axis, static_cast<int64_t>(dr->shape[axis]));
    return launch_status("gather_elements");
}

int topk_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    if (node->output_count < 2) return -11;
    float fk = 0.0f;
    if (!const_scalar(ctx, node, 1, &fk)) return SPKV2_E_UNSUPPORTED;  // k computed at run time
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    const int axis = norm_axis(attr.axis, xr->rank);
    if (axis < 0 || axis >= xr->rank) return -11;
    const int dim = static_cast<int>(xr->shape[axis]);
    int k = static_cast<int>(fk);
    if (k <= 0 || dim == 0) return 0;
    if (k > dim) k = dim;
    if (k > kTopkMaxK) return SPKV2_E_UNSUPPORTED;
    size_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= xr->shape[i];
    for (int i = axis + 1; i < xr->rank; i++) inner *= xr->shape[i];
    const size_t rows = outer * inner;
    if (rows == 0) return 0;
    if (rows > 0x7fffffffULL) return SPKV2_E_UNSUPPORTED;
    set_kernel_name(ctx, node, "topk");
    auto kernel = dim <= kTopkRowLds ? topk_kernel<true> : topk_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(rows)), dim3(kTopkThreads), 0, ctx->stream,
                       dptr<const float>(ctx, node->inputs[0]), dptr<float>(ctx, node->outputs[0]),
                       dptr<float>(ctx, node->outputs[1]), inner, dim, k, attr.largest ? 1 : 0);
    return launch_status("topk");
}

}  // namespace spk::kern
