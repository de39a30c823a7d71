// (Skip)SimplifiedLayerNormalization and the elementwise/gather glue of the int4
// decoder graph, for gfx950.
#include "common.h"

namespace ortmi {

// One workgroup per row. r = x (+ skip) (+ bias), rounded to T when a sum was
// formed (the reference adds in the op dtype, rust/src/ops/norm.rs:237-238);
// y = r * rsqrt(mean(r^2) + eps) * gamma with one rounding (norm.rs:239).
// Rows of D <= 2048 2-byte values, D % 8 == 0: each thread owns one 16-byte
// vector of x (and of skip, bias, gamma), all requested before any is used, so
// a row costs one memory round trip. Vectors past D, and absent skip / bias, read
// zeros without an access.
template <typename T>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const T* __restrict__ x,
                                                           const T* __restrict__ skip,
                                                           const T* __restrict__ bias,
                                                           const T* __restrict__ gamma,
                                                           T* __restrict__ y, T* __restrict__ res,
                                                           int64_t D, float eps) {
    static_assert(sizeof(T) == 2, "2-byte elements");
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    const uint32_t bytes = (uint32_t)(D * 2);
    const uint32_t off = 16u * (uint32_t)t < bytes ? 16u * (uint32_t)t : bytes;
    const u32x4_t xv = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(x + row * D, bytes), off, 0, 0);
    const u32x4_t sv = __builtin_amdgcn_raw_buffer_load_b128(
        buffer_rsrc(skip ? skip + row * D : x, skip ? bytes : 0u), off, 0, 0);
    const u32x4_t bv = __builtin_amdgcn_raw_buffer_load_b128(
        buffer_rsrc(bias ? bias : x, bias ? bytes : 0u), off, 0, 0);
    const u32x4_t gv = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(gamma, bytes), off, 0, 0);
    const bool live = 16u * (uint32_t)t < bytes;
    const bool summed = skip || bias;
    const T* xe = reinterpret_cast<const T*>(&xv);
    const T* se = reinterpret_cast<const T*>(&sv);
    const T* be = reinterpret_cast<const T*>(&bv);
    float v[8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float a = to_f32(xe[i]) + to_f32(se[i]) + to_f32(be[i]);  // absent terms read 0
        if (summed) a = round_to<T>(a);
        v[i] = a;
        ss += a * a;
    }
    if (res && live) {
        T r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = from_f32<T>(v[i]);
        *reinterpret_cast<uint4*>(res + row * D + 8 * t) = *reinterpret_cast<const uint4*>(r);
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(tot / (float)D + eps);
    if (!live) return;
    const T* ge = reinterpret_cast<const T*>(&gv);
    T o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(v[i] * inv * to_f32(ge[i]));
    *reinterpret_cast<uint4*>(y + row * D + 8 * t) = *reinterpret_cast<const uint4*>(o);
}

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T* __restrict__ x,
                                                       const T* __restrict__ skip,
                                                       const T* __restrict__ bias,
                                                       const T* __restrict__ gamma,
                                                       T* __restrict__ y, T* __restrict__ res,
                                                       int64_t D, float eps) {
    extern __shared__ float sr[];  // D floats
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const T* xr = x + row * D;
    const T* sk = skip ? skip + row * D : nullptr;
    const bool summed = skip || bias;
    float ss = 0.f;
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
        float v = to_f32(xr[d]);
        if (sk) v += to_f32(sk[d]);
        if (bias) v += to_f32(bias[d]);
        if (summed) v = round_to<T>(v);
        sr[d] = v;
        ss += v * v;
        if (res) res[row * D + d] = from_f32<T>(v);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(tot / (float)D + eps);
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x)
        y[row * D + d] = from_f32<T>(sr[d] * inv * to_f32(gamma[d]));
}

template <typename T>
__global__ void gather_rows_kernel(const T* __restrict__ table, const int64_t* __restrict__ ids,
                                   T* __restrict__ out, int64_t V, int64_t D) {
    const int64_t r = blockIdx.x;
    int64_t id = ids[r];
    if (id < 0) id += V;
    const bool ok = id >= 0 && id < V;
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x)
        out[r * D + d] = ok ? table[id * D + d] : from_f32<T>(0.f);
}

// Sigmoid -> Mul(g, sig) -> Mul(., u), each result rounded to T.
template <typename T>
__global__ void swiglu_kernel(const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ o,
                              int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = to_f32(g[i]);
    const float sig = round_to<T>(1.0f / (1.0f + __expf(-gv)));
    const float t = round_to<T>(gv * sig);
    o[i] = from_f32<T>(t * to_f32(u[i]));
}

// SwiGLU over interleaved gate/up columns: y is [rows, 2P] with column 2i the
// gate and 2i+1 the up projection of output i; out is [rows, P].
template <typename T>
__global__ void swiglu_pairs_kernel(const T* __restrict__ y, T* __restrict__ o, int64_t pairs,
                                    int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t row = i / pairs, p = i % pairs;
    const T* yr = y + row * 2 * pairs + 2 * p;
    const float gv = to_f32(yr[0]);
    const float sig = round_to<T>(1.0f / (1.0f + __expf(-gv)));
    o[i] = from_f32<T>(round_to<T>(gv * sig) * to_f32(yr[1]));
}

template <typename T>
__global__ void binary_kernel(int op, const T* __restrict__ a, const T* __restrict__ b,
                              T* __restrict__ o, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = to_f32(a[i]), y = to_f32(b[i]);
    const float r = op == 0 ? x + y : (op == 1 ? x * y : x - y);
    o[i] = from_f32<T>(r);
}

template <typename T>
__global__ void sigmoid_kernel(const T* __restrict__ x, T* __restrict__ o, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    o[i] = from_f32<T>(1.0f / (1.0f + __expf(-to_f32(x[i]))));
}

// Index of the maximum of each row, the first on ties (the last with LAST, ONNX
// select_last_index = 1); NaNs are skipped, an all-NaN row gives 0.
template <typename T, bool LAST = false>
__global__ __launch_bounds__(256) void argmax_rows_kernel(const T* __restrict__ x,
                                                          int64_t* __restrict__ out,
                                                          int64_t cols) {
    __shared__ float sv[256];
    __shared__ int64_t si[256];
    const int64_t row = blockIdx.x;
    const T* xr = x + row * cols;
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float v = to_f32(xr[c]);
        if (v > best || (v == best && (LAST || bi < 0))) {
            best = v;
            bi = c;
        }
    }
    sv[threadIdx.x] = best;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = sv[threadIdx.x + s];
            const int64_t oi = si[threadIdx.x + s];
            const float mv = sv[threadIdx.x];
            const int64_t mi = si[threadIdx.x];
            const bool take =
                oi >= 0 && (mi < 0 || ov > mv || (ov == mv && (LAST ? oi > mi : oi < mi)));
            if (take) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[row] = si[0] < 0 ? 0 : si[0];
}

// Arg max along the middle axis of x viewed as [outer, dim, inner] (inner > 1):
// one thread per (outer, inner) column walks the axis, consecutive threads reading
// consecutive inner elements. Ties and NaNs as argmax_rows_kernel.
template <typename T, bool LAST>
__global__ __launch_bounds__(256) void argmax_axis_kernel(const T* __restrict__ x,
                                                          int64_t* __restrict__ out,
                                                          int64_t cols_total, int64_t dim,
                                                          int64_t inner) {
    const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= cols_total) return;
    const int64_t o = col / inner, i = col - o * inner;
    const T* p = x + o * dim * inner + i;
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t d = 0; d < dim; ++d) {
        const float v = to_f32(p[d * inner]);
        if (v > best || (v == best && (LAST || bi < 0))) {
            best = v;
            bi = d;
        }
    }
    out[col] = bi < 0 ? 0 : bi;
}

// Block-wide argmax of (value, index) pairs held one per thread; the lowest index
// wins ties. Returns the winner in thread 0.
__device__ __forceinline__ void argmax_block(float& best, int64_t& bi, float* sv, int64_t* si) {
    sv[threadIdx.x] = best;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = sv[threadIdx.x + s];
            const int64_t oi = si[threadIdx.x + s];
            const float mv = sv[threadIdx.x];
            const int64_t mi = si[threadIdx.x];
            if (oi >= 0 && (mi < 0 || ov > mv || (ov == mv && oi < mi))) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    best = sv[0];
    bi = si[0];
}

// Two-pass argmax for long rows: `parts` workgroups per row each reduce a
// contiguous slice to one (value, index) partial, then one workgroup per row
// reduces the partials.
struct ArgPartial {
    float v;
    int32_t pad;
    int64_t i;
};

template <typename T>
__global__ __launch_bounds__(256) void argmax_partial_kernel(const T* __restrict__ x,
                                                             ArgPartial* __restrict__ part,
                                                             int64_t cols, int parts,
                                                             int64_t slice) {
    __shared__ float sv[256];
    __shared__ int64_t si[256];
    const int64_t row = blockIdx.y;
    const int p = blockIdx.x;
    const T* xr = x + row * cols;
    const int64_t c0 = (int64_t)p * slice;
    const int64_t c1 = min(cols, c0 + slice);
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t c = c0 + threadIdx.x; c < c1; c += blockDim.x) {
        const float v = to_f32(xr[c]);
        if (v > best || (bi < 0 && v == best)) {
            best = v;
            bi = c;
        }
    }
    argmax_block(best, bi, sv, si);
    if (threadIdx.x == 0) part[row * parts + p] = ArgPartial{best, 0, bi};
}

// The same partials from 16-byte loads: each thread issues its kArgVec vectors of
// the 2048-column slice at once (one memory round trip per workgroup instead of a
// dependent load per element). Elements past the slice or the row read as zeros
// without a memory access and are skipped by index.
constexpr int kArgSlice = 2048;
template <typename T>
__global__ __launch_bounds__(256) void argmax_partial_vec_kernel(const T* __restrict__ x,
                                                                 ArgPartial* __restrict__ part,
                                                                 int64_t cols, int parts) {
    constexpr int E = 16 / (int)sizeof(T);     // elements per vector
    constexpr int NV = kArgSlice / (256 * E);  // vectors per thread
    __shared__ float sv[256];
    __shared__ int64_t si[256];
    const int64_t row = blockIdx.y;
    const int p = blockIdx.x;
    const int64_t c0 = (int64_t)p * kArgSlice;
    const uint32_t row_bytes = (uint32_t)(cols * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(x + row * cols, row_bytes);
    uint4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t c = c0 + (int64_t)(j * 256 + (int)threadIdx.x) * E;
        const uint32_t off = c < cols ? (uint32_t)(c * (int64_t)sizeof(T)) : row_bytes;
        const auto w = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        v[j] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    float best = -INFINITY;
    int64_t bi = -1;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const T* e = reinterpret_cast<const T*>(&v[j]);
        const int64_t cb = c0 + (int64_t)(j * 256 + (int)threadIdx.x) * E;
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const float val = to_f32(e[k]);
            if (cb + k < cols && (val > best || (bi < 0 && val == best))) {
                best = val;
                bi = cb + k;
            }
        }
    }
    argmax_block(best, bi, sv, si);
    if (threadIdx.x == 0) part[row * parts + p] = ArgPartial{best, 0, bi};
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const ArgPartial* __restrict__ part,
                                                           int64_t* __restrict__ out,
                                                           int parts) {
    __shared__ float sv[256];
    __shared__ int64_t si[256];
    const int64_t row = blockIdx.x;
    float best = -INFINITY;
    int64_t bi = -1;
    for (int p = threadIdx.x; p < parts; p += blockDim.x) {
        const ArgPartial a = part[row * parts + p];
        if (a.i >= 0 && (bi < 0 || a.v > best || (a.v == best && a.i < bi))) {
            best = a.v;
            bi = a.i;
        }
    }
    argmax_block(best, bi, sv, si);
    if (threadIdx.x == 0) out[row] = bi < 0 ? 0 : bi;
}

static int64_t dtype_bytes(int32_t dtype) { return dtype == ORTMI_F32 ? 4 : 2; }

static int argmax_parts(int64_t cols) {
    // 2048 columns per workgroup, at most 256 partials per row.
    int64_t p = (cols + kArgSlice - 1) / kArgSlice;
    return (int)std::min<int64_t>(std::max<int64_t>(p, 1), 256);
}

template <typename S, typename D>
__global__ void cast_kernel(const S* __restrict__ x, D* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = from_f32<D>(to_f32(x[i]));
}

static unsigned blocks_for(int64_t n, int t = 256) { return (unsigned)((n + t - 1) / t); }

}  // namespace ortmi

using namespace ortmi;

#define ORTMI_DISPATCH_FLOAT(dtype, MACRO)                                      \
    switch (dtype) {                                                            \
        case ORTMI_F32: MACRO(float);                                           \
        case ORTMI_F16: MACRO(half_t);                                          \
        case ORTMI_BF16: MACRO(uint16_t);                                       \
        default: return fail(ORTMI_E_INVALID, "unsupported dtype");             \
    }

extern "C" int ortmi_rms_norm(const void* x, const void* skip, const void* bias,
                              const void* gamma, void* y, void* residual_out, int64_t rows,
                              int64_t D, float eps, int32_t dtype, void* stream) {
    ORTMI_REQUIRE(rows >= 0 && D > 0, "SimplifiedLayerNormalization: bad shape");
    ORTMI_REQUIRE(D <= 16384, "SimplifiedLayerNormalization: normalized axis too long");
    if (rows == 0) return ORTMI_OK;
    ORTMI_REQUIRE(x && gamma && y, "SimplifiedLayerNormalization: null tensor");
    ORTMI_REQUIRE(rows < (1LL << 31), "SimplifiedLayerNormalization: too many rows");
    hipStream_t st = as_stream(stream);
    const auto a16 = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vec = D % 8 == 0 && D <= 2048 && a16(x) && a16(skip) && a16(bias) && a16(gamma) &&
                     a16(y) && a16(residual_out);
#define ORTMI_RMS(T)                                                                          \
    if constexpr (sizeof(T) == 2) {                                                           \
        if (vec) {                                                                            \
            hipLaunchKernelGGL((rms_norm_vec_kernel<T>), dim3((unsigned)rows), dim3(256), 0, st, \
                               static_cast<const T*>(x), static_cast<const T*>(skip),         \
                               static_cast<const T*>(bias), static_cast<const T*>(gamma),     \
                               static_cast<T*>(y), static_cast<T*>(residual_out), D, eps);    \
            return check_launch("rms_norm");                                                  \
        }                                                                                     \
    }                                                                                         \
    hipLaunchKernelGGL((rms_norm_kernel<T>), dim3((unsigned)rows), dim3(256), D * sizeof(float), \
                       st, static_cast<const T*>(x), static_cast<const T*>(skip),             \
                       static_cast<const T*>(bias), static_cast<const T*>(gamma),             \
                       static_cast<T*>(y), static_cast<T*>(residual_out), D, eps);            \
    return check_launch("rms_norm")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_RMS)
#undef ORTMI_RMS
}

extern "C" int ortmi_gather_rows(const void* table, const int64_t* ids, void* out,
                                 int64_t num_ids, int64_t vocab, int64_t D, int32_t dtype,
                                 void* stream) {
    ORTMI_REQUIRE(num_ids >= 0 && vocab > 0 && D > 0, "Gather: bad shape");
    if (num_ids == 0) return ORTMI_OK;
    ORTMI_REQUIRE(table && ids && out, "Gather: null tensor");
    hipStream_t st = as_stream(stream);
#define ORTMI_GATHER(T)                                                                     \
    hipLaunchKernelGGL((gather_rows_kernel<T>), dim3((unsigned)num_ids), dim3(256), 0, st,  \
                       static_cast<const T*>(table), ids, static_cast<T*>(out), vocab, D); \
    return check_launch("gather_rows")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_GATHER)
#undef ORTMI_GATHER
}

extern "C" int ortmi_swiglu(const void* gate, const void* up, void* out, int64_t n,
                            int32_t dtype, void* stream) {
    ORTMI_REQUIRE(n >= 0, "SwiGLU: bad size");
    if (n == 0) return ORTMI_OK;
    ORTMI_REQUIRE(gate && up && out, "SwiGLU: null tensor");
    hipStream_t st = as_stream(stream);
#define ORTMI_SWIGLU(T)                                                                      \
    hipLaunchKernelGGL((swiglu_kernel<T>), dim3(blocks_for(n)), dim3(256), 0, st,            \
                       static_cast<const T*>(gate), static_cast<const T*>(up),               \
                       static_cast<T*>(out), n);                                             \
    return check_launch("swiglu")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_SWIGLU)
#undef ORTMI_SWIGLU
}

extern "C" int ortmi_swiglu_pairs(const void* y, void* out, int64_t rows, int64_t pairs,
                                  int32_t dtype, void* stream) {
    ORTMI_REQUIRE(rows >= 0 && pairs >= 0, "SwiGLU pairs: bad shape");
    const int64_t n = rows * pairs;
    if (n == 0) return ORTMI_OK;
    ORTMI_REQUIRE(y && out, "SwiGLU pairs: null tensor");
    hipStream_t st = as_stream(stream);
#define ORTMI_SWIGLU_PAIRS(T)                                                                \
    hipLaunchKernelGGL((swiglu_pairs_kernel<T>), dim3(blocks_for(n)), dim3(256), 0, st,      \
                       static_cast<const T*>(y), static_cast<T*>(out), pairs, n);            \
    return check_launch("swiglu_pairs")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_SWIGLU_PAIRS)
#undef ORTMI_SWIGLU_PAIRS
}

extern "C" int ortmi_binary(int32_t op, const void* a, const void* b, void* out, int64_t n,
                            int32_t dtype, void* stream) {
    ORTMI_REQUIRE(op >= 0 && op <= 2, "binary: op must be 0 (Add), 1 (Mul) or 2 (Sub)");
    ORTMI_REQUIRE(n >= 0, "binary: bad size");
    if (n == 0) return ORTMI_OK;
    ORTMI_REQUIRE(a && b && out, "binary: null tensor");
    hipStream_t st = as_stream(stream);
#define ORTMI_BIN(T)                                                                          \
    hipLaunchKernelGGL((binary_kernel<T>), dim3(blocks_for(n)), dim3(256), 0, st, (int)op,   \
                       static_cast<const T*>(a), static_cast<const T*>(b),                   \
                       static_cast<T*>(out), n);                                             \
    return check_launch("binary")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_BIN)
#undef ORTMI_BIN
}

extern "C" int ortmi_sigmoid(const void* x, void* out, int64_t n, int32_t dtype, void* stream) {
    ORTMI_REQUIRE(n >= 0, "Sigmoid: bad size");
    if (n == 0) return ORTMI_OK;
    ORTMI_REQUIRE(x && out, "Sigmoid: null tensor");
    hipStream_t st = as_stream(stream);
#define ORTMI_SIG(T)                                                                           \
    hipLaunchKernelGGL((sigmoid_kernel<T>), dim3(blocks_for(n)), dim3(256), 0, st,             \
                       static_cast<const T*>(x), static_cast<T*>(out), n);                     \
    return check_launch("sigmoid")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_SIG)
#undef ORTMI_SIG
}

extern "C" size_t ortmi_argmax_rows_workspace_size(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0) return 0;
    return (size_t)rows * (size_t)argmax_parts(cols) * sizeof(ArgPartial);
}

extern "C" int ortmi_argmax_rows(const void* x, int64_t* out, int64_t rows, int64_t cols,
                                 int32_t dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    ORTMI_REQUIRE(rows >= 0 && cols > 0, "ArgMax: bad shape");
    if (rows == 0) return ORTMI_OK;
    ORTMI_REQUIRE(x && out, "ArgMax: null tensor");
    ORTMI_REQUIRE(rows <= 65535, "ArgMax: too many rows");
    hipStream_t st = as_stream(stream);
    const int parts = argmax_parts(cols);
    const bool split = parts > 1 && workspace &&
                       workspace_bytes >= ortmi_argmax_rows_workspace_size(rows, cols);
    const int64_t slice = (cols + parts - 1) / parts;
    // 16-byte loads need aligned rows and a slice that fits the 256 partials.
    const bool vec = split && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                     (cols * dtype_bytes(dtype)) % 16 == 0 &&
                     cols <= (int64_t)kArgSlice * 256 && cols * dtype_bytes(dtype) < (1LL << 31);
#define ORTMI_ARGMAX(T)                                                                         \
    if (vec) {                                                                                  \
        hipLaunchKernelGGL((argmax_partial_vec_kernel<T>), dim3((unsigned)parts, (unsigned)rows), \
                           dim3(256), 0, st, static_cast<const T*>(x),                          \
                           static_cast<ArgPartial*>(workspace), cols, parts);                   \
        if (int rc = check_launch("argmax_partial")) return rc;                                 \
        hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(256), 0, st,         \
                           static_cast<const ArgPartial*>(workspace), out, parts);              \
        return check_launch("argmax_final");                                                    \
    }                                                                                           \
    if (split) {                                                                                \
        hipLaunchKernelGGL((argmax_partial_kernel<T>), dim3((unsigned)parts, (unsigned)rows),   \
                           dim3(256), 0, st, static_cast<const T*>(x),                          \
                           static_cast<ArgPartial*>(workspace), cols, parts, slice);            \
        if (int rc = check_launch("argmax_partial")) return rc;                                 \
        hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(256), 0, st,         \
                           static_cast<const ArgPartial*>(workspace), out, parts);              \
        return check_launch("argmax_final");                                                    \
    }                                                                                           \
    hipLaunchKernelGGL((argmax_rows_kernel<T>), dim3((unsigned)rows), dim3(256), 0, st,         \
                       static_cast<const T*>(x), out, cols);                                    \
    return check_launch("argmax_rows")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_ARGMAX)
#undef ORTMI_ARGMAX
}

extern "C" int ortmi_argmax_axis(const void* x, int64_t* out, int64_t outer, int64_t dim,
                                 int64_t inner, int32_t select_last_index, int32_t dtype,
                                 void* stream) {
    ORTMI_REQUIRE(outer >= 0 && inner >= 0 && dim > 0, "ArgMax: bad shape");
    ORTMI_REQUIRE(select_last_index == 0 || select_last_index == 1,
                  "ArgMax: select_last_index must be 0 or 1");
    if (outer == 0 || inner == 0) return ORTMI_OK;
    ORTMI_REQUIRE(x && out, "ArgMax: null tensor");
    ORTMI_REQUIRE(outer <= INT32_MAX && outer * dim <= (INT64_MAX / 4) / (inner > 0 ? inner : 1),
                  "ArgMax: tensor too large");
    hipStream_t st = as_stream(stream);
    const bool last = select_last_index != 0;
    const int64_t cols = outer * inner;
#define ORTMI_ARGMAX_AXIS(T)                                                                        if (inner == 1) {                                                                                   if (last)                                                                                           hipLaunchKernelGGL((argmax_rows_kernel<T, true>), dim3((unsigned)outer), dim3(256),                                0, st, static_cast<const T*>(x), out, dim);                              else                                                                                                hipLaunchKernelGGL((argmax_rows_kernel<T, false>), dim3((unsigned)outer),                                          dim3(256), 0, st, static_cast<const T*>(x), out, dim);               } else {                                                                                            const unsigned blocks = (unsigned)((cols + 255) / 256);                                         if (last)                                                                                           hipLaunchKernelGGL((argmax_axis_kernel<T, true>), dim3(blocks), dim3(256), 0, st,                                  static_cast<const T*>(x), out, cols, dim, inner);                        else                                                                                                hipLaunchKernelGGL((argmax_axis_kernel<T, false>), dim3(blocks), dim3(256), 0, st,                                 static_cast<const T*>(x), out, cols, dim, inner);                    }                                                                                               return check_launch("argmax_axis")
    ORTMI_DISPATCH_FLOAT(dtype, ORTMI_ARGMAX_AXIS)
#undef ORTMI_ARGMAX_AXIS
}

extern "C" int ortmi_cast(const void* x, int32_t src_dtype, void* y, int32_t dst_dtype, int64_t n,
                          void* stream) {
    ORTMI_REQUIRE(n >= 0, "Cast: bad size");
    if (n == 0) return ORTMI_OK;
    ORTMI_REQUIRE(x && y, "Cast: null tensor");
    hipStream_t st = as_stream(stream);
#define ORTMI_CAST2(S, D)                                                                    \
    hipLaunchKernelGGL((cast_kernel<S, D>), dim3(blocks_for(n)), dim3(256), 0, st,           \
                       static_cast<const S*>(x), static_cast<D*>(y), n);                     \
    return check_launch("cast")
#define ORTMI_CAST_FROM(S)                                                                   \
    switch (dst_dtype) {                                                                     \
        case ORTMI_F32: ORTMI_CAST2(S, float);                                               \
        case ORTMI_F16: ORTMI_CAST2(S, half_t);                                              \
        case ORTMI_BF16: ORTMI_CAST2(S, uint16_t);                                           \
        default: return fail(ORTMI_E_INVALID, "Cast: unsupported destination dtype");       \
    }
    switch (src_dtype) {
        case ORTMI_F32: ORTMI_CAST_FROM(float)
        case ORTMI_F16: ORTMI_CAST_FROM(half_t)
        case ORTMI_BF16: ORTMI_CAST_FROM(uint16_t)
        default: return fail(ORTMI_E_INVALID, "Cast: unsupported source dtype");
    }
#undef ORTMI_CAST_FROM
#undef ORTMI_CAST2
}
