// lhip_elem.hip -- elementwise and gather/scatter kernels: fill, add, SwiGLU fwd/bwd,
// RoPE, embedding gather and deterministic scatter-add.
//
// HBM-bound; 128-bit (float4) loads and stores wherever the shape and
// alignment allow, grid-stride loops sized to a few waves per CU.
// Semantics follow the CPU LMTrain path (ai/core/tensor2.lua):
//   mul :167-183, silu :272-303 (sigmoid by sign), rope :410-473 with the
//   angle table of ai/nn/transformer.lua:30-48, embed :572-607;
// and the batched contracts of cuda/luaTL_train.cu (swiglu :647-686 with
// leading dimensions, rope :719-767 with pos_ids / pos_offset / half-split /
// inverse, embed :771-806).
#include <cmath>

#include "lhip_internal.h"

namespace lhip {
namespace {

// One unit (usually a float4) per thread: on MI355X a grid-stride loop over a
// few blocks per CU streams at ~4.8 TB/s, one float4 per thread at ~6.2 TB/s
// (measured on a 1 GiB copy).  The cap only matters for enormous arrays, which
// the kernels' grid-stride loops then cover.
inline int grid_for(long long units, int threads)
{
    const long long cap = 1LL << 22;
    long long g = (units + threads - 1) / threads;
    if (g > cap) g = cap;
    return static_cast<int>(g < 1 ? 1 : g);
}

typedef float vf4 __attribute__((ext_vector_type(4)));

// 128-bit load of data read exactly once (non-temporal hint)
__device__ __forceinline__ float4 ld_stream(const float* p)
{
    const vf4 v = __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// 128-bit store of data written once and not read back by this kernel
// (non-temporal hint: streamed out rather than held dirty in L2 until the
// end-of-kernel write-back).
__device__ __forceinline__ void st_stream(float* p, const float4& v)
{
    __builtin_nontemporal_store(vf4{v.x, v.y, v.z, v.w}, reinterpret_cast<vf4*>(p));
}

__global__ void fill_kernel(float* __restrict__ p, long long n, float v)
{
    const long long n4 = n >> 2;
    float4* p4 = reinterpret_cast<float4*>(p);
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n4; i += stride)
        p4[i] = make_float4(v, v, v, v);
    for (long long i = 4 * n4 + blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n; i += stride)
        p[i] = v;
}

__global__ void fill_bytes_kernel(unsigned char* __restrict__ p, long long n)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n; i += stride)
        p[i] = 0;
}

// sigmoid evaluated by sign (tensor2.lua:272-291): 1/(1+e^-v) for v >= 0,
// e^v/(1+e^v) below, so neither branch overflows
__device__ __forceinline__ float silu_sign(float v)
{
    if (v >= 0.f) return v / (1.0f + expf(-v));
    const float z = expf(v);
    return v * z / (1.0f + z);
}

// out = silu(x) elementwise (in place allowed: each element is read, then written)
__global__ void silu_kernel(const float* x, float* o, long long n, int vec)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (vec) {
        const long long n4 = n >> 2;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        float4* o4 = reinterpret_cast<float4*>(o);
        for (long long i = t0; i < n4; i += stride) {
            const float4 v = x4[i];
            st_stream(reinterpret_cast<float*>(o4 + i),
                      make_float4(silu_sign(v.x), silu_sign(v.y), silu_sign(v.z), silu_sign(v.w)));
        }
        for (long long i = 4 * n4 + t0; i < n; i += stride) o[i] = silu_sign(x[i]);
    } else {
        for (long long i = t0; i < n; i += stride) o[i] = silu_sign(x[i]);
    }
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ o,
                           long long n, int vec)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (vec) {
        const long long n4 = n >> 2;
        const float4* a4 = reinterpret_cast<const float4*>(a);
        const float4* b4 = reinterpret_cast<const float4*>(b);
        float4* o4 = reinterpret_cast<float4*>(o);
        for (long long i = t0; i < n4; i += stride) {
            const float4 x = a4[i], y = b4[i];
            st_stream(reinterpret_cast<float*>(o4 + i), make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
        }
        for (long long i = 4 * n4 + t0; i < n; i += stride) o[i] = a[i] + b[i];
    } else {
        for (long long i = t0; i < n; i += stride) o[i] = a[i] + b[i];
    }
}

// sigmoid evaluated by sign (tensor2.lua:272-291)
__device__ __forceinline__ float sigmoid_by_sign(float v)
{
    if (v >= 0.f) return 1.0f / (1.0f + expf(-v));
    const float z = expf(v);
    return z / (1.0f + z);
}

// h = silu(g) * u over a rows x cols block with leading dimensions.
__global__ void swiglu_fwd_kernel(const float* __restrict__ g, int ldg, const float* __restrict__ u, int ldu,
                                  float* __restrict__ h, int ldh, int rows, int cols, int vec)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (vec) {
        const int c4n = cols >> 2;
        const long long n = static_cast<long long>(rows) * c4n;
        const bool flat = ldg == cols && ldu == cols && ldh == cols;
        for (long long i = t0; i < n; i += stride) {
            long long og, ou, oh;
            if (flat) {
                og = ou = oh = 4 * i;
            } else {
                const unsigned r = static_cast<unsigned>(i) / static_cast<unsigned>(c4n);
                const unsigned c = 4 * (static_cast<unsigned>(i) - r * static_cast<unsigned>(c4n));
                og = static_cast<long long>(r) * ldg + c;
                ou = static_cast<long long>(r) * ldu + c;
                oh = static_cast<long long>(r) * ldh + c;
            }
            const float4 gv = ld_stream(g + og);
            const float4 uv = ld_stream(u + ou);
            float4 o;
            o.x = gv.x * sigmoid_by_sign(gv.x) * uv.x;
            o.y = gv.y * sigmoid_by_sign(gv.y) * uv.y;
            o.z = gv.z * sigmoid_by_sign(gv.z) * uv.z;
            o.w = gv.w * sigmoid_by_sign(gv.w) * uv.w;
            st_stream(h + oh, o);
        }
    } else {
        const long long n = static_cast<long long>(rows) * cols;
        for (long long i = t0; i < n; i += stride) {
            const int r = static_cast<int>(i / cols), c = static_cast<int>(i % cols);
            const float gv = g[static_cast<long long>(r) * ldg + c];
            h[static_cast<long long>(r) * ldh + c] = gv * sigmoid_by_sign(gv) * u[static_cast<long long>(r) * ldu + c];
        }
    }
}

// dg = s*(1 + g*(1-s)) * (u*dh), du = silu(g)*dh  (BACKWARD.mul then BACKWARD.silu,
// tensor2.lua:172-183, 293-303); acc adds into dg/du.
__device__ __forceinline__ void swiglu_bwd_one(float gv, float uv, float dhv, float& dg, float& du)
{
    const float s = sigmoid_by_sign(gv);
    du = (gv * s) * dhv;
    dg = (s * (1.0f + gv * (1.0f - s))) * (uv * dhv);
}

__global__ void swiglu_bwd_kernel(const float* __restrict__ g, int ldg, const float* __restrict__ u, int ldu,
                                  const float* __restrict__ dh, int lddh, float* __restrict__ dg, int lddg,
                                  float* __restrict__ du, int lddu, int rows, int cols, int acc, int vec)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (vec) {
        const int c4n = cols >> 2;
        const long long n = static_cast<long long>(rows) * c4n;
        const bool flat = ldg == cols && ldu == cols && lddh == cols && lddg == cols && lddu == cols;
        for (long long i = t0; i < n; i += stride) {
            long long r, c;
            if (flat) {
                r = 0;
                c = 4 * i;
            } else {
                const unsigned ru = static_cast<unsigned>(i) / static_cast<unsigned>(c4n);
                r = ru;
                c = 4 * (static_cast<unsigned>(i) - ru * static_cast<unsigned>(c4n));
            }
            const float4 gv = ld_stream(g + r * ldg + c);
            const float4 uv = ld_stream(u + r * ldu + c);
            const float4 hv = ld_stream(dh + r * lddh + c);
            float4 a, b;
            swiglu_bwd_one(gv.x, uv.x, hv.x, a.x, b.x);
            swiglu_bwd_one(gv.y, uv.y, hv.y, a.y, b.y);
            swiglu_bwd_one(gv.z, uv.z, hv.z, a.z, b.z);
            swiglu_bwd_one(gv.w, uv.w, hv.w, a.w, b.w);
            float4* pg = reinterpret_cast<float4*>(dg + r * lddg + c);
            float4* pu = reinterpret_cast<float4*>(du + r * lddu + c);
            if (acc) {
                const float4 og = *pg, ou = *pu;
                a.x += og.x; a.y += og.y; a.z += og.z; a.w += og.w;
                b.x += ou.x; b.y += ou.y; b.z += ou.z; b.w += ou.w;
            }
            st_stream(dg + r * lddg + c, a);
            st_stream(du + r * lddu + c, b);
        }
    } else {
        const long long n = static_cast<long long>(rows) * cols;
        for (long long i = t0; i < n; i += stride) {
            const long long r = i / cols, c = i % cols;
            float a, b;
            swiglu_bwd_one(g[r * ldg + c], u[r * ldu + c], dh[r * lddh + c], a, b);
            float* pg = dg + r * lddg + c;
            float* pu = du + r * lddu + c;
            *pg = acc ? *pg + a : a;
            *pu = acc ? *pu + b : b;
        }
    }
}

// Contiguous operands (every leading dimension equal to cols, 16-byte
// aligned): U float4 per thread, block-contiguous (thread t of block b takes
// float4 b*256*U + t + 256*k), every load of a thread issued before its
// first store and none behind a branch: indices past the end are clamped
// (their stores skipped).  At 4096 x 4096 the forward (U = 1) streams at 82%
// of HBM and the backward (U = 2) at 78%, against 73% for one float4 per
// iteration of a grid-stride loop.
template <int U>
__global__ void __launch_bounds__(256)
swiglu_fwd_flat(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ h, long long n4)
{
    const long long base = static_cast<long long>(blockIdx.x) * 256 * U + threadIdx.x;
    const float4* g4 = reinterpret_cast<const float4*>(g);
    const float4* u4 = reinterpret_cast<const float4*>(u);
    float4 gv[U], uv[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const long long i = min(base + 256 * k, n4 - 1);
        gv[k] = ld_stream(reinterpret_cast<const float*>(g4 + i));
        uv[k] = ld_stream(reinterpret_cast<const float*>(u4 + i));
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const long long i = base + 256 * k;
        if (i >= n4) break;
        float4 o;
        o.x = gv[k].x * sigmoid_by_sign(gv[k].x) * uv[k].x;
        o.y = gv[k].y * sigmoid_by_sign(gv[k].y) * uv[k].y;
        o.z = gv[k].z * sigmoid_by_sign(gv[k].z) * uv[k].z;
        o.w = gv[k].w * sigmoid_by_sign(gv[k].w) * uv[k].w;
        st_stream(h + 4 * i, o);
    }
}

template <int U>
__global__ void __launch_bounds__(256)
swiglu_bwd_flat(const float* __restrict__ g, const float* __restrict__ u, const float* __restrict__ dh,
                float* __restrict__ dg, float* __restrict__ du, long long n4, int acc)
{
    const long long base = static_cast<long long>(blockIdx.x) * 256 * U + threadIdx.x;
    float4 gv[U], uv[U], hv[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const long long i = 4 * min(base + 256 * k, n4 - 1);
        gv[k] = ld_stream(g + i);
        uv[k] = ld_stream(u + i);
        hv[k] = ld_stream(dh + i);
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const long long i = base + 256 * k;
        if (i >= n4) break;
        float4 a, b;
        swiglu_bwd_one(gv[k].x, uv[k].x, hv[k].x, a.x, b.x);
        swiglu_bwd_one(gv[k].y, uv[k].y, hv[k].y, a.y, b.y);
        swiglu_bwd_one(gv[k].z, uv[k].z, hv[k].z, a.z, b.z);
        swiglu_bwd_one(gv[k].w, uv[k].w, hv[k].w, a.w, b.w);
        if (acc) {
            const float4 og = reinterpret_cast<const float4*>(dg)[i], ou = reinterpret_cast<const float4*>(du)[i];
            a.x += og.x; a.y += og.y; a.z += og.z; a.w += og.w;
            b.x += ou.x; b.y += ou.y; b.z += ou.z; b.w += ou.w;
        }
        st_stream(dg + 4 * i, a);
        st_stream(du + 4 * i, b);
    }
}

// --------------------------------------------------------------------- RoPE
// In place on x[rows][row_stride], heads of hd columns starting at column 0.
// pos = pos_ids ? pos_ids[r] : (period > 0 ? r % period : r) + pos_offset.
// Angle of pair p: pos * inv[p], inv[p] = 1 / base^(2p/hd), evaluated in
// double like the Lua table (transformer.lua:30-48); cos/sin in double, then
// rounded to fp32.  The table for the block's rows is built once in LDS and
// shared by every head.  inverse negates sin (the backward rotation).
constexpr int kRopeMaxPairs = 128;
constexpr int kRopeRowsPerBlock = 8;

struct RopeFreqs {
    double inv[kRopeMaxPairs];
};

// Vector access modes of one unit (a run of pairs sharing the row and head):
//   ROPE_IL4: interleaved, two pairs (x0,y0,x1,y1) in one float4;
//   ROPE_HS4: half-split, four pairs: float4 of first halves at p, float4 of
//             second halves at p + hd/2;
//   ROPE_HS2: half-split, two pairs as two float2 (8-byte alignment only).
enum { ROPE_IL4 = 0, ROPE_HS4 = 1, ROPE_HS2 = 2, ROPE_SCALAR = 3 };

__device__ __forceinline__ float2 rope_rot(float a, float b, float2 cs)
{
    return make_float2(a * cs.x - b * cs.y, b * cs.x + a * cs.y);
}

template <int MODE>
__global__ void __launch_bounds__(256)
rope_kernel(float* __restrict__ x, const int* __restrict__ pos_ids, int rows, int heads, int hd, int row_stride,
            int pos_offset, int period, int interleaved, int inverse, RopeFreqs fr)
{
    __shared__ float2 tab[kRopeRowsPerBlock * kRopeMaxPairs];   // (cos, sin)
    const int pairs = hd >> 1;
    const int r0 = blockIdx.x * kRopeRowsPerBlock;
    const int nr = min(kRopeRowsPerBlock, rows - r0);
    auto make_table = [&]() {
        for (int i = threadIdx.x; i < nr * pairs; i += blockDim.x) {
            const int rr = i / pairs, p = i % pairs;
            const int r = r0 + rr;
            const int pos = pos_ids ? pos_ids[r] : (period > 0 ? r % period : r) + pos_offset;
            const double ang = static_cast<double>(pos) * fr.inv[p];
            double sn, cs;
            sincos(ang, &sn, &cs);
            tab[rr * kRopeMaxPairs + p] = make_float2(static_cast<float>(cs), static_cast<float>(inverse ? -sn : sn));
        }
        __syncthreads();
    };
    if constexpr (MODE == ROPE_SCALAR) {
        make_table();
        const int units = nr * heads * pairs;
        for (int i = threadIdx.x; i < units; i += blockDim.x) {
            const int rr = i / (heads * pairs);
            const int rem = i % (heads * pairs);
            const int h = rem / pairs, p = rem % pairs;
            float* base = x + static_cast<long long>(r0 + rr) * row_stride + static_cast<long long>(h) * hd;
            const float2 cs = tab[rr * kRopeMaxPairs + p];
            float* a = interleaved ? base + 2 * p : base + p;
            float* b = interleaved ? base + 2 * p + 1 : base + p + pairs;
            const float x0 = *a, x1 = *b;
            const float2 o = rope_rot(x0, x1, cs);
            *a = o.x;
            *b = o.y;
        }
    } else {
        // A thread takes kU units per batch: the batch's loads are all issued
        // first (the first batch's before the angle table is computed, so the
        // two overlap), then rotated and stored.
        constexpr int kPPU = MODE == ROPE_HS4 ? 4 : 2;     // pairs per unit
        constexpr int kU = MODE == ROPE_HS4 ? 4 : 8;       // units per thread per batch
        const int units_per_head = pairs / kPPU;
        const int per_row = heads * units_per_head;
        const int units = nr * per_row;
        float4 va[kU], vb[kU];
        float* ptr[kU];
        int slot[kU];
        auto load = [&](int i0) {
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int i = i0 + u * static_cast<int>(blockDim.x);
                ptr[u] = nullptr;
                if (i < units) {
                    const int rr = i / per_row, rem = i - rr * per_row;
                    const int h = rem / units_per_head, p = kPPU * (rem - h * units_per_head);
                    float* base = x + static_cast<long long>(r0 + rr) * row_stride + static_cast<long long>(h) * hd;
                    slot[u] = rr * kRopeMaxPairs + p;
                    if constexpr (MODE == ROPE_IL4) {
                        ptr[u] = base + 2 * p;
                        va[u] = ld_stream(ptr[u]);
                    } else if constexpr (MODE == ROPE_HS4) {
                        ptr[u] = base + p;
                        va[u] = ld_stream(ptr[u]);
                        vb[u] = ld_stream(ptr[u] + pairs);
                    } else {
                        ptr[u] = base + p;
                        const float2 a = *reinterpret_cast<const float2*>(ptr[u]);
                        const float2 b = *reinterpret_cast<const float2*>(ptr[u] + pairs);
                        va[u] = make_float4(a.x, a.y, b.x, b.y);
                    }
                }
            }
        };
        auto rotate_store = [&]() {
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                if (!ptr[u]) continue;
                const float4 t = va[u];
                const float2 c0 = tab[slot[u]], c1 = tab[slot[u] + 1];
                if constexpr (MODE == ROPE_IL4) {
                    const float2 o0 = rope_rot(t.x, t.y, c0), o1 = rope_rot(t.z, t.w, c1);
                    st_stream(ptr[u], make_float4(o0.x, o0.y, o1.x, o1.y));
                } else if constexpr (MODE == ROPE_HS4) {
                    const float2 c2 = tab[slot[u] + 2], c3 = tab[slot[u] + 3];
                    const float4 b = vb[u];
                    const float2 o0 = rope_rot(t.x, b.x, c0), o1 = rope_rot(t.y, b.y, c1);
                    const float2 o2 = rope_rot(t.z, b.z, c2), o3 = rope_rot(t.w, b.w, c3);
                    st_stream(ptr[u], make_float4(o0.x, o1.x, o2.x, o3.x));
                    st_stream(ptr[u] + pairs, make_float4(o0.y, o1.y, o2.y, o3.y));
                } else {
                    // t = (a0, a1, b0, b1): pairs (a0, b0) at p and (a1, b1) at p + 1
                    const float2 o0 = rope_rot(t.x, t.z, c0), o1 = rope_rot(t.y, t.w, c1);
                    *reinterpret_cast<float2*>(ptr[u]) = make_float2(o0.x, o1.x);
                    *reinterpret_cast<float2*>(ptr[u] + pairs) = make_float2(o0.y, o1.y);
                }
            }
        };
        const int step = kU * static_cast<int>(blockDim.x);
        load(threadIdx.x);
        make_table();
        rotate_store();
        for (int i0 = threadIdx.x + step; i0 < units; i0 += step) {
            load(i0);
            rotate_store();
        }
    }
}

// ---------------------------------------------------------------- embedding
// out[i] = table[ids[i]] (exact copy); an id outside [0, vocab) gives a zero row.
__global__ void embed_fwd_kernel(const float* __restrict__ table, const int* __restrict__ ids,
                                 float* __restrict__ out, int n, int dim, int vocab, int vec)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (vec) {
        const int d4 = dim >> 2;
        const long long total = static_cast<long long>(n) * d4;
        for (long long i = t0; i < total; i += stride) {
            const int t = static_cast<int>(i / d4), c = static_cast<int>(i % d4);
            const int id = ids[t];
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (id >= 0 && id < vocab) v = reinterpret_cast<const float4*>(table + static_cast<long long>(id) * dim)[c];
            reinterpret_cast<float4*>(out + static_cast<long long>(t) * dim)[c] = v;
        }
    } else {
        const long long total = static_cast<long long>(n) * dim;
        for (long long i = t0; i < total; i += stride) {
            const int t = static_cast<int>(i / dim), c = static_cast<int>(i % dim);
            const int id = ids[t];
            out[i] = (id >= 0 && id < vocab) ? table[static_cast<long long>(id) * dim + c] : 0.f;
        }
    }
}

// dtable[v] (+)= scale * sum over tokens i with ids[i] == v, added in token
// order (the Lua loop order, tensor2.lua:592-607), one wave per vocabulary row:
// the ids are loaded 1024 at a time (16 per lane, all issued before the first
// compare) and matches found 64 at a time with a wave ballot.  No atomics, so
// the result is deterministic.  Ids outside [0, vocab) are skipped.
constexpr int kEmbedChunk = 512;  // columns per pass (8 per lane)
constexpr int kEmbedIds = 16;     // id chunks of 64 per scan pass

__global__ void __launch_bounds__(64)
embed_bwd_kernel(const float* __restrict__ g, const int* __restrict__ ids, float* __restrict__ dtable,
                 int n, int dim, int vocab, float scale, int acc)
{
    const int v = blockIdx.x;
    const int lane = threadIdx.x;
    for (int d0 = 0; d0 < dim; d0 += kEmbedChunk) {
        float a[kEmbedChunk / 64];
        float* row = dtable + static_cast<long long>(v) * dim;
#pragma unroll
        for (int k = 0; k < kEmbedChunk / 64; ++k) {
            const int d = d0 + lane + 64 * k;
            a[k] = (acc && d < dim) ? row[d] : 0.f;
        }
        for (int c0 = 0; c0 < n; c0 += 64 * kEmbedIds) {
            int idv[kEmbedIds];
#pragma unroll
            for (int k = 0; k < kEmbedIds; ++k) {
                if (c0 + 64 * k >= n) break;                  // uniform
                const int i = c0 + 64 * k + lane;
                idv[k] = ids[min(i, n - 1)];
            }
#pragma unroll
            for (int k = 0; k < kEmbedIds; ++k) {
                if (c0 + 64 * k >= n) break;
                const int i0 = c0 + 64 * k;
                unsigned long long mask = __ballot(i0 + lane < n && idv[k] == v);
                while (mask) {
                    const int b = __ffsll(static_cast<long long>(mask)) - 1;
                    mask &= mask - 1;
                    const float* gr = g + static_cast<long long>(i0 + b) * dim;
#pragma unroll
                    for (int j = 0; j < kEmbedChunk / 64; ++j) {
                        const int d = d0 + lane + 64 * j;
                        if (d < dim) a[j] = a[j] + scale * gr[d];
                    }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kEmbedChunk / 64; ++k) {
            const int d = d0 + lane + 64 * k;
            if (d < dim) row[d] = a[k];
        }
    }
    (void)vocab;
}

}  // namespace

int fill(float* p, long long n, float v, hipStream_t s)
{
    if (n <= 0) return LHIP_OK;
    if (!p) return fail(LHIP_E_NULL, "fill: NULL pointer");
    if (!aligned16(p)) return fail(LHIP_E_ARG, "fill: pointer must be 16-byte aligned");
    klaunch(fill_kernel, grid_for((n + 3) / 4, 256), 256, 0, s, p, n, v);
    return check_launch("fill");
}

int zero_bytes(void* p, size_t bytes, hipStream_t s)
{
    if (bytes == 0) return LHIP_OK;
    if (!p) return fail(LHIP_E_NULL, "zero: NULL pointer");
    if (aligned16(p) && bytes % 4 == 0) return fill(static_cast<float*>(p), static_cast<long long>(bytes / 4), 0.f, s);
    klaunch(fill_bytes_kernel, grid_for(static_cast<long long>(bytes), 256), 256, 0, s, static_cast<unsigned char*>(p),
                                                                                  static_cast<long long>(bytes));
    return check_launch("zero");
}

int add(const float* a, const float* b, float* o, long long n, hipStream_t s)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "add: n < 0");
    if (n == 0) return LHIP_OK;
    if (!a || !b || !o) return fail(LHIP_E_NULL, "add: NULL pointer");
    const int vec = aligned16(a) && aligned16(b) && aligned16(o);
    klaunch(add_kernel, grid_for(vec ? (n + 3) / 4 : n, 256), 256, 0, s, a, b, o, n, vec);
    return check_launch("add");
}

int silu(const float* x, float* o, long long n, hipStream_t s)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "silu: n < 0");
    if (n == 0) return LHIP_OK;
    if (!x || !o) return fail(LHIP_E_NULL, "silu: NULL pointer");
    const int vec = aligned16(x) && aligned16(o);
    klaunch(silu_kernel, grid_for(vec ? (n + 3) / 4 : n, 256), 256, 0, s, x, o, n, vec);
    return check_launch("silu");
}

int swiglu_fwd(const float* g, int ldg, const float* u, int ldu, float* h, int ldh, int rows, int cols,
               hipStream_t s)
{
    if (rows < 0 || cols < 0) return fail(LHIP_E_SHAPE, "swiglu_fwd: rows=%d cols=%d", rows, cols);
    if (rows == 0 || cols == 0) return LHIP_OK;
    if (!g || !u || !h) return fail(LHIP_E_NULL, "swiglu_fwd: NULL pointer");
    if (ldg < cols || ldu < cols || ldh < cols) return fail(LHIP_E_SHAPE, "swiglu_fwd: leading dimension < cols");
    const int vec = cols % 4 == 0 && ldg % 4 == 0 && ldu % 4 == 0 && ldh % 4 == 0 && aligned16(g) &&
                    aligned16(u) && aligned16(h) &&
                    static_cast<long long>(rows) * (cols / 4) < (1LL << 31);
    const long long units = static_cast<long long>(rows) * (vec ? cols / 4 : cols);
    if (vec && ldg == cols && ldu == cols && ldh == cols && units <= (1LL << 30))
        klaunch(swiglu_fwd_flat<1>, grid_for(units, 256), 256, 0, s, g, u, h, units);
    else
        klaunch(swiglu_fwd_kernel, grid_for(units, 256), 256, 0, s, g, ldg, u, ldu, h, ldh, rows, cols, vec);
    return check_launch("swiglu_fwd");
}

int swiglu_bwd(const float* g, int ldg, const float* u, int ldu, const float* dh, int lddh, float* dg, int lddg,
               float* du, int lddu, int rows, int cols, int acc, hipStream_t s)
{
    if (rows < 0 || cols < 0) return fail(LHIP_E_SHAPE, "swiglu_bwd: rows=%d cols=%d", rows, cols);
    if (rows == 0 || cols == 0) return LHIP_OK;
    if (!g || !u || !dh || !dg || !du) return fail(LHIP_E_NULL, "swiglu_bwd: NULL pointer");
    if (ldg < cols || ldu < cols || lddh < cols || lddg < cols || lddu < cols)
        return fail(LHIP_E_SHAPE, "swiglu_bwd: leading dimension < cols");
    const int vec = cols % 4 == 0 && ldg % 4 == 0 && ldu % 4 == 0 && lddh % 4 == 0 && lddg % 4 == 0 &&
                    lddu % 4 == 0 && aligned16(g) && aligned16(u) && aligned16(dh) && aligned16(dg) && aligned16(du) &&
                    static_cast<long long>(rows) * (cols / 4) < (1LL << 31);
    const long long units = static_cast<long long>(rows) * (vec ? cols / 4 : cols);
    if (vec && ldg == cols && ldu == cols && lddh == cols && lddg == cols && lddu == cols && units <= (1LL << 30))
        klaunch(swiglu_bwd_flat<2>, grid_for(units, 512), 256, 0, s, g, u, dh, dg, du, units, acc);
    else
        klaunch(swiglu_bwd_kernel, grid_for(units, 256), 256, 0, s, g, ldg, u, ldu, dh, lddh, dg, lddg, du, lddu, rows,
                cols, acc, vec);
    return check_launch("swiglu_bwd");
}

int rope(float* x, const int* pos_ids, int rows, int heads, int hd, int row_stride, int pos_offset, int period,
         double base, int interleaved, int inverse, hipStream_t s)
{
    if (rows < 0 || heads <= 0 || hd <= 0) return fail(LHIP_E_SHAPE, "rope: rows=%d heads=%d hd=%d", rows, heads, hd);
    if (rows == 0) return LHIP_OK;
    if (!x) return fail(LHIP_E_NULL, "rope: x is NULL");
    if (hd % 2) return fail(LHIP_E_ARG, "rope: head_dim %d must be even", hd);
    if (hd / 2 > kRopeMaxPairs) return fail(LHIP_E_CAPACITY, "rope: head_dim %d > %d", hd, 2 * kRopeMaxPairs);
    if (row_stride < heads * hd) return fail(LHIP_E_SHAPE, "rope: row_stride %d < heads*hd %d", row_stride, heads * hd);
    if (!(base > 0.0)) return fail(LHIP_E_ARG, "rope: base must be > 0");
    if (period < 0) return fail(LHIP_E_ARG, "rope: period must be >= 0");
    RopeFreqs fr;
    const int pairs = hd / 2;
    for (int p = 0; p < kRopeMaxPairs; ++p)
        fr.inv[p] = p < pairs ? 1.0 / std::pow(base, static_cast<double>(2 * p) / hd) : 0.0;
    // vector units: two pairs per float4 (interleaved), four pairs as two
    // float4 (half-split, pairs % 4 == 0), or two pairs as two float2
    // (half-split, 8-byte alignment); anything else takes scalar accesses
    const bool il4 = interleaved && pairs % 2 == 0 && row_stride % 4 == 0 && hd % 4 == 0 && aligned16(x);
    const bool hs4 = !interleaved && pairs % 4 == 0 && row_stride % 4 == 0 && aligned16(x);
    const bool hs2 = !interleaved && pairs % 2 == 0 && row_stride % 2 == 0 &&
                     (reinterpret_cast<uintptr_t>(x) & 7u) == 0;
    const dim3 grid(ceil_div(rows, kRopeRowsPerBlock));
#define LHIP_ROPE(M_) klaunch(rope_kernel<M_>, grid, 256, 0, s, x, pos_ids, rows, heads, hd, row_stride, pos_offset, \
                                                           period, interleaved, inverse, fr)
    if (il4) LHIP_ROPE(ROPE_IL4);
    else if (hs4) LHIP_ROPE(ROPE_HS4);
    else if (hs2) LHIP_ROPE(ROPE_HS2);
    else LHIP_ROPE(ROPE_SCALAR);
#undef LHIP_ROPE
    return check_launch("rope");
}

int embed_fwd(const float* table, const int* ids, float* out, int n, int dim, int vocab, hipStream_t s)
{
    if (n < 0 || dim <= 0 || vocab <= 0) return fail(LHIP_E_SHAPE, "embed_fwd: n=%d dim=%d vocab=%d", n, dim, vocab);
    if (n == 0) return LHIP_OK;
    if (!table || !ids || !out) return fail(LHIP_E_NULL, "embed_fwd: NULL pointer");
    const int vec = dim % 4 == 0 && aligned16(table) && aligned16(out);
    const long long units = static_cast<long long>(n) * (vec ? dim / 4 : dim);
    klaunch(embed_fwd_kernel, grid_for(units, 256), 256, 0, s, table, ids, out, n, dim, vocab, vec);
    return check_launch("embed_fwd");
}

int embed_bwd(const float* g, const int* ids, float* dtable, int n, int dim, int vocab, float scale, int acc,
              hipStream_t s)
{
    if (n < 0 || dim <= 0 || vocab <= 0) return fail(LHIP_E_SHAPE, "embed_bwd: n=%d dim=%d vocab=%d", n, dim, vocab);
    if (!dtable) return fail(LHIP_E_NULL, "embed_bwd: dtable is NULL");
    if (n > 0 && (!g || !ids)) return fail(LHIP_E_NULL, "embed_bwd: NULL g/ids");
    klaunch(embed_bwd_kernel, vocab, 64, 0, s, g, ids, dtable, n, dim, vocab, scale, acc);
    return check_launch("embed_bwd");
}

}  // namespace lhip

using lhip::st;

extern "C" {

LHIP_API int lhip_fill(float* x, long long n, float value)
{
    LHIP_REQUIRE_READY();
    return lhip::fill(x, n, value, st().stream);
}

LHIP_API int lhip_add(const float* a, const float* b, float* out, long long n)
{
    LHIP_REQUIRE_READY();
    return lhip::add(a, b, out, n, st().stream);
}

LHIP_API int lhip_silu(const float* x, float* out, long long n)
{
    LHIP_REQUIRE_READY();
    return lhip::silu(x, out, n, st().stream);
}

LHIP_API int lhip_swiglu_fwd(const float* gate, int ld_gate, const float* up, int ld_up, float* out, int ld_out,
                             int rows, int cols)
{
    LHIP_REQUIRE_READY();
    return lhip::swiglu_fwd(gate, ld_gate, up, ld_up, out, ld_out, rows, cols, st().stream);
}

LHIP_API int lhip_swiglu_bwd(const float* gate, int ld_gate, const float* up, int ld_up, const float* dout,
                             int ld_dout, float* dgate, int ld_dgate, float* dup, int ld_dup, int rows, int cols,
                             int accumulate)
{
    LHIP_REQUIRE_READY();
    return lhip::swiglu_bwd(gate, ld_gate, up, ld_up, dout, ld_dout, dgate, ld_dgate, dup, ld_dup, rows, cols,
                            accumulate, st().stream);
}

LHIP_API int lhip_rope(float* x, const int* pos_ids, int rows, int heads, int head_dim, int row_stride,
                       int pos_offset, int pos_period, double base, int interleaved, int inverse)
{
    LHIP_REQUIRE_READY();
    return lhip::rope(x, pos_ids, rows, heads, head_dim, row_stride, pos_offset, pos_period, base, interleaved,
                      inverse, st().stream);
}

LHIP_API int lhip_embed_fwd(const float* table, const int* ids, float* out, int n, int dim, int vocab)
{
    LHIP_REQUIRE_READY();
    return lhip::embed_fwd(table, ids, out, n, dim, vocab, st().stream);
}

LHIP_API int lhip_embed_bwd(const float* dout, const int* ids, float* dtable, int n, int dim, int vocab,
                            float scale, int accumulate)
{
    LHIP_REQUIRE_READY();
    return lhip::embed_bwd(dout, ids, dtable, n, dim, vocab, scale, accumulate, st().stream);
}

}  // extern "C"
