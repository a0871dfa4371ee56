// C ABI of fp8lin: argument validation (the reference's TORCH_CHECK
// preconditions turned into status codes), kernel dispatch and the
// Engine::linear decision table.  No allocation, no host synchronisation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <string>

#include "../../include/fp8lin.h"
#include "internal.hpp"

namespace {

thread_local std::string g_last_error;

struct Failure {
    int code;
    std::string msg;
};

[[noreturn]] void fail(int code, const std::string& msg) { throw Failure{code, msg}; }

void require(bool ok, int code, const char* msg) {
    if (!ok) fail(code, msg);
}

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(FP8LIN_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
}

template <class F>
int guarded(F&& body) {
    try {
        body();
        g_last_error.clear();
        return FP8LIN_OK;
    } catch (const Failure& f) {
        g_last_error = f.msg;
        return f.code;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return FP8LIN_ERR_LAUNCH;
    } catch (...) {
        g_last_error = "unknown failure";
        return FP8LIN_ERR_LAUNCH;
    }
}

constexpr int kMaxDevices = 64;
std::mutex g_device_mutex;
int g_device_state[kMaxDevices];  // 0 unknown, 1 gfx950, -1 other
// Device address of `scratch` on each GPU (each holds its own copy).
void* g_scratch[kMaxDevices];

}  // namespace

// Scratch of the allocation-free entry point fp8lin_linear_candidates_static:
// the head logits and the candidate chunk pairs.  Every GPU the library runs
// on holds FP8LIN_STATIC_SCRATCH_BYTES of it until the process ends.  In host
// code `scratch` is only a host-side stand-in for the symbol: its device
// address comes from hipGetSymbolAddress (ensure_device, once per device) and
// only that address is ever passed to a kernel.
static __device__ __align__(256) uint8_t scratch[FP8LIN_STATIC_SCRATCH_BYTES];

namespace {

// Checks that the current device is a gfx950 and, the first time on each
// device, looks up that device's copy of `scratch`.  Returns the device id.
int ensure_device() {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) fail(FP8LIN_ERR_DEVICE, std::string("hipGetDevice: ") + hipGetErrorString(e));
    require(dev >= 0 && dev < kMaxDevices, FP8LIN_ERR_DEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_device_mutex);
    if (g_device_state[dev] == 0) {
        hipDeviceProp_t prop;
        check_hip(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) {
            void* ptr = nullptr;
            check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
            require(ptr != nullptr, FP8LIN_ERR_LAUNCH, "hipGetSymbolAddress(scratch) returned null");
            g_scratch[dev] = ptr;
            g_device_state[dev] = 1;
        } else {
            g_device_state[dev] = -1;
        }
    }
    require(g_device_state[dev] == 1, FP8LIN_ERR_DEVICE,
            "fp8lin kernels are built for gfx950 (MI355X) only");
    return dev;
}

hipStream_t as_stream(fp8lin_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int64_t kMaxDim = (int64_t)1 << 31;
constexpr int64_t kMaxGridRows = (int64_t)1 << 22;  // one workgroup of up to 1024 threads per row

void check_dims(int64_t M, int64_t N, int64_t K) {
    require(M > 0 && N > 0 && K > 0, FP8LIN_ERR_SHAPE, "Empty GEMM: M, N and K must be positive");
    require(M < kMaxDim && N < kMaxDim && K < kMaxDim, FP8LIN_ERR_SHAPE,
            "dimension exceeds 2^31-1");
}

// src/optimized.cu:64: scales are [N] or [N, ceil(K/128)].
void check_scales(const float* scales, int64_t scale_cols, int64_t K) {
    require(scales != nullptr, FP8LIN_ERR_ARGUMENT, "Invalid FP8 scales: null pointer");
    require(scale_cols == 1 || scale_cols == ceil_div(K, 128), FP8LIN_ERR_ARGUMENT,
            "Invalid FP8 scales: scale_cols must be 1 or ceil(K/128)");
}

// Whether fp8lin_linear's 2..8-row call runs the small-M matrix-core kernel
// instead of the multi-row GEMV.  The reference's fp8_linear sends these rows
// to its GEMV, one pass over the weights per activation row
// (src/optimized.cu:62-68), and asks for no particular summation order there:
// its only bit-equality checks are the shared GEMV's FP8 vs decoded-BF16
// weights and the vector vs scalar GEMV on an unaligned one-row view
// (tests/optimized_test.cpp:7-14, :57-62), which stay on the GEMV kernels.
// The matrix-core kernel reads the weights once for all rows and
// dequantizes each code once (measured 1.4-2.2x faster than the 4- and
// 8-row GEMV at the decode shapes).  It takes block scales [N, K/128],
// K % 128 == 0, 16-byte aligned x and codes and 16 K < 2^31; weights of at
// most 1024 rows keep the GEMV (four rows or fewer per CU), and so do two
// rows at K <= 5120 except on the weights where the matrix-core kernel
// measured faster (small_m_two_rows: the output heads, 25..40 rows per CU).
bool linear_small_m(const uint16_t* x, const uint8_t* codes, int64_t S, int64_t M, int64_t N, int64_t K) {
    if (!(M >= 2 && M <= 8 && N > 1024 && K % 128 == 0 && S == K / 128 && aligned16(x) && aligned16(codes) &&
          16 * K < kMaxDim && N * S * 4 < kMaxDim))
        return false;
    return M > 2 || K > 5120 || fp8lin::small_m_two_rows((int)N, (int)K);
}

// K-split partials of fp8_linear's prefill GEMM (M > 8) for output row stride
// ldy: the engine branch's plan (few tiles, or a small last round, split K);
// 0 where nothing splits.  Block scales are assumed: per-row scales take the
// same plan.
size_t linear_ws(int64_t M, int64_t N, int64_t K, int64_t ldy) {
    if (M <= 8 || M >= kMaxDim || N <= 0 || N >= kMaxDim || K <= 0 || K >= kMaxDim) return 0;
    return fp8lin::gemm_workspace_bytes((int)ceil_div(K, 128), ldy, (int)M, (int)N, (int)K, false);
}

// ws: the K-split partials of the prefill GEMM (linear_ws bytes), or null to
// run every GEMM tile whole.
void linear_impl(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t S,
                 uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream,
                 void* ws = nullptr, size_t ws_bytes = 0) {
    if (linear_small_m(x, codes, S, M, N, K)) {
        check_hip(fp8lin::launch_small_m(x, codes, scales, y, ldy, (int)M, (int)N, (int)K, 1, false, stream),
                  "fp8 small-M launch");
    } else if (M <= 8) {
        const bool wide = K % 16 == 0 && aligned16(x) && aligned16(codes);
        check_hip(fp8lin::launch_gemv(x, codes, true, scales, (int)S, y, ldy, (int)M, (int)N, (int)K,
                                      wide, stream),
                  "fp8 gemv launch");
    } else {
        check_hip(fp8lin::launch_gemm_ws(x, codes, scales, (int)S, y, ldy, (int)M, (int)N, (int)K, false,
                                         ws_bytes ? ws : nullptr, ws_bytes, stream),
                  "fp8 gemm launch");
    }
}

// Gate/up + SwiGLU for M <= 8 rows: the kernel fp8lin_linear runs for the
// same (M, N, K) and pointers, with the SwiGLU epilogue, so the output is
// fused_swiglu of fp8lin_linear's bit for bit.
void decode_swiglu(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t S, uint16_t* y, int64_t M,
                   int64_t N, int64_t K, hipStream_t stream) {
    if (linear_small_m(x, codes, S, M, N, K)) {
        check_hip(fp8lin::launch_small_m(x, codes, scales, y, N / 2, (int)M, (int)N, (int)K, 1, true, stream),
                  "fp8 small-M+swiglu launch");
        return;
    }
    const bool wide = K % 16 == 0 && aligned16(x) && aligned16(codes);
    check_hip(fp8lin::launch_gemv_swiglu(x, codes, scales, (int)S, y, N / 2, (int)M, (int)N, (int)K, wide, stream),
              "fp8 gemv+swiglu launch");
}

// fp8lin_linear(x, W) followed by its vocabulary candidates, in `ws`
// (linear_candidates_ws bytes).  Where the linear runs the ring GEMV, the
// candidates come from that kernel's epilogue (the same per-row sums, rounded
// to the same BF16 logits, never stored) and one finishing launch; otherwise
// the logits go to the workspace and the two-stage candidate kernels read
// them.
void linear_candidates_impl(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t S, int64_t M,
                            int64_t N, int64_t K, int64_t offset, void* ws, double* out, hipStream_t stream);

void gemm_bf16_impl(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, hipStream_t stream) {
    if (M <= 8) {
        const bool wide = K % 16 == 0 && aligned16(x) && aligned16(w);
        check_hip(fp8lin::launch_gemv(x, w, false, nullptr, 1, y, ldy, (int)M, (int)N, (int)K, wide,
                                      stream),
                  "bf16 gemv launch");
    } else {
        check_hip(fp8lin::launch_gemm(x, w, nullptr, 1, y, ldy, (int)M, (int)N, (int)K, false,
                                      stream),
                  "bf16 gemm launch");
    }
}

// The split-4 partials are summed inside each workgroup (small_m.hip).
size_t tensor_small_ws(int64_t, int64_t, int) { return 0; }

// Whether fp8_tensor_small runs the matrix-core kernel (else the GEMV).
bool tensor_small_matrix_core(const uint16_t* x, const uint8_t* codes, int64_t K) {
    return aligned16(x) && aligned16(codes) && 16 * K < kMaxDim;
}

void tensor_small_impl(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, int split, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
    // src/fp8_tensor.cu:54-59
    require(x && codes && scales && y, FP8LIN_ERR_ARGUMENT, "Invalid FP8 W8A16 inputs: null pointer");
    require(M >= 2 && M <= 8 && N > 0 && K > 0 && K % 128 == 0 && N < kMaxDim && K < kMaxDim,
            FP8LIN_ERR_SHAPE, "Invalid FP8 W8A16 geometry: need 2 <= M <= 8, N > 0, K % 128 == 0");
    require(split == 1 || split == 4, FP8LIN_ERR_ARGUMENT, "Invalid FP8 W8A16 split: must be 1 or 4");
    (void)ws;
    (void)ws_bytes;
    ensure_device();
    // The matrix-core kernel DMAs 16-byte chunks of x and codes with 32-bit
    // buffer offsets.  The reference accepts any contiguous tensor
    // (src/fp8_tensor.cu:54-59), so an unaligned view or a K too large for
    // those offsets runs the multi-row GEMV instead: same operator, same
    // parity bar, only the FP32 summation order differs.
    if (!tensor_small_matrix_core(x, codes, K)) {
        check_hip(fp8lin::launch_gemv(x, codes, true, scales, (int)(K / 128), y, ldy, (int)M, (int)N, (int)K,
                                      K % 16 == 0 && aligned16(x) && aligned16(codes), stream),
                  "fp8 small-M fallback gemv launch");
        return;
    }
    check_hip(fp8lin::launch_small_m(x, codes, scales, y, ldy, (int)M, (int)N, (int)K, split, false, stream),
              "fp8 small-M launch");
}

void shared_impl(const uint16_t* x, const void* weight, const float* scales, int64_t S, uint16_t* y,
                 int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    // src/deep_kernels.cu:135-146
    require(x && weight && y, FP8LIN_ERR_ARGUMENT, "Invalid shared GEMV inputs: null pointer");
    require(M >= 1 && M <= 8 && N > 0 && K > 0 && N < kMaxDim && K < kMaxDim, FP8LIN_ERR_SHAPE,
            "Shared GEMV requires 1..8 rows and N, K > 0");
    if (scales) check_scales(scales, S, K);
    ensure_device();
    const bool wide = K % 16 == 0 && aligned16(x) && aligned16(weight);
    check_hip(fp8lin::launch_gemv(x, weight, scales != nullptr, scales, scales ? (int)S : 1, y, ldy,
                                  (int)M, (int)N, (int)K, wide, stream),
              "shared gemv launch");
}

constexpr int64_t kSlabRows = 2048;  // src/engine.cpp:229

size_t dequant_gemm_ws(int64_t N, int64_t K) {
    const int64_t rows = N < kSlabRows ? N : kSlabRows;
    return (size_t)rows * (size_t)K * 2;
}

bool tensor_small_eligible(const fp8lin_linear_options& o, const fp8lin_weight& w, int64_t rows) {
    return (o.fp8_tensor_small || o.tilelang_fp8) && rows >= 2 && rows <= 8 && w.scales &&
           w.K % 128 == 0 && w.scale_cols == w.K / 128 && (!o.tilelang_fp8 || w.N % 16 == 0);
}

// K-split partials of the FP8 GEMM branch (rows > 8): outputs whose tile
// count leaves CUs idle (few tiles, or a small last round) split K.
size_t engine_gemm_ws(const fp8lin_weight& w, int64_t rows, int64_t ldy) {
    if (rows <= 8 || rows >= kMaxDim) return 0;
    return fp8lin::gemm_workspace_bytes((int)w.scale_cols, ldy, (int)rows, (int)w.N, (int)w.K, false);
}

size_t engine_ws(const fp8lin_linear_options& o, const fp8lin_weight& w, int64_t rows) {
    if (tensor_small_eligible(o, w, rows)) return tensor_small_ws(rows, w.N, o.fp8_tensor_split);
    if (o.multi_token_gemv && rows > 1 && rows <= 8) return 0;
    if (w.cached_bf16 && rows > 1) return 0;
    // (the plan for ldy = N: a wider ldy never needs more)
    if (w.scales && o.optimized && !(o.cublas_prefill && rows > 8)) return engine_gemm_ws(w, rows, w.N);
    if (w.scales) return dequant_gemm_ws(w.N, w.K);
    return 0;
}

// The branch Engine::linear takes (src/engine.cpp:206-237), without running it.
int engine_path(const fp8lin_linear_options& o, const fp8lin_weight& w, int64_t rows) {
    if (tensor_small_eligible(o, w, rows)) return FP8LIN_PATH_TENSOR_SMALL;
    if (o.multi_token_gemv && rows > 1 && rows <= 8) return FP8LIN_PATH_SHARED_GEMV;
    if (w.cached_bf16 && rows > 1) return FP8LIN_PATH_CACHED_BF16;
    if (w.scales && o.optimized && !(o.cublas_prefill && rows > 8))
        return rows <= 8 ? FP8LIN_PATH_FP8_GEMV : FP8LIN_PATH_FP8_GEMM;
    if (w.scales) return FP8LIN_PATH_DEQUANT_GEMM;
    return FP8LIN_PATH_BF16;
}

// The option combinations the reference's Engine constructor rejects
// (src/engine.cpp:78-81).
bool options_consistent(const fp8lin_linear_options& o) {
    return !(o.fp8_tensor_small && o.tilelang_fp8) && (o.fp8_tensor_split == 1 || o.fp8_tensor_split == 4) &&
           (!(o.fp8_tensor_small || o.tilelang_fp8) || o.optimized);
}

void check_options(const fp8lin_linear_options& o) {
    require(!(o.fp8_tensor_small && o.tilelang_fp8), FP8LIN_ERR_ARGUMENT, "Choose one FP8 Tensor Core backend");
    require(o.fp8_tensor_split == 1 || o.fp8_tensor_split == 4, FP8LIN_ERR_ARGUMENT,
            "FP8 Tensor Core split must be 1 or 4");
    require(!(o.fp8_tensor_small || o.tilelang_fp8) || o.optimized, FP8LIN_ERR_ARGUMENT,
            "FP8 Tensor Core requires optimized mode");
}

void validate_engine(const fp8lin_linear_options& o, const fp8lin_weight& w, const uint16_t* x,
                     int64_t rows, const uint16_t* y, int64_t ldy) {
    check_options(o);
    require(x && y && w.data, FP8LIN_ERR_ARGUMENT, "Engine linear: null pointer");
    check_dims(rows, w.N, w.K);
    require(ldy >= w.N, FP8LIN_ERR_SHAPE, "Engine linear: ldy < N");
    if (w.scales) check_scales(w.scales, w.scale_cols, w.K);
}

int engine_branch(const fp8lin_linear_options& o, const fp8lin_weight& w, const uint16_t* x,
                  int64_t rows, uint16_t* y, int64_t ldy, void* ws, size_t ws_bytes,
                  hipStream_t stream) {
    const auto* codes = static_cast<const uint8_t*>(w.data);
    // src/engine.cpp:206-213
    if (tensor_small_eligible(o, w, rows)) {
        tensor_small_impl(x, codes, w.scales, y, ldy, rows, w.N, w.K, o.fp8_tensor_split, ws,
                          ws_bytes, stream);
        return FP8LIN_PATH_TENSOR_SMALL;
    }
    // :214-219
    if (o.multi_token_gemv && rows > 1 && rows <= 8) {
        const bool use_cached = w.cached_bf16 && !(o.shared_gemv_fp8 && w.scales);
        if (use_cached)
            shared_impl(x, w.cached_bf16, nullptr, 1, y, ldy, rows, w.N, w.K, stream);
        else
            shared_impl(x, w.data, w.scales, w.scale_cols, y, ldy, rows, w.N, w.K, stream);
        return FP8LIN_PATH_SHARED_GEMV;
    }
    // :220-221
    if (w.cached_bf16 && rows > 1) {
        gemm_bf16_impl(x, w.cached_bf16, y, ldy, rows, w.N, w.K, stream);
        return FP8LIN_PATH_CACHED_BF16;
    }
    // :222-224
    if (w.scales && o.optimized && !(o.cublas_prefill && rows > 8)) {
        if (rows > 8) {
            const size_t need = engine_gemm_ws(w, rows, ldy);
            require(need == 0 || (ws != nullptr && ws_bytes >= need && aligned16(ws)), FP8LIN_ERR_WORKSPACE,
                    "FP8 GEMM split-K partial workspace missing, too small or unaligned");
            check_hip(fp8lin::launch_gemm_ws(x, codes, w.scales, (int)w.scale_cols, y, ldy, (int)rows, (int)w.N,
                                             (int)w.K, false, need ? ws : nullptr, need, stream),
                      "fp8 gemm launch");
        } else {
            linear_impl(x, codes, w.scales, w.scale_cols, y, ldy, rows, w.N, w.K, stream);
        }
        return rows <= 8 ? FP8LIN_PATH_FP8_GEMV : FP8LIN_PATH_FP8_GEMM;
    }
    // :225-233, 2048-row BF16 slabs, each GEMM writing its column slice of y.
    if (w.scales) {
        const size_t need = dequant_gemm_ws(w.N, w.K);
        require(ws != nullptr && ws_bytes >= need && aligned16(ws), FP8LIN_ERR_WORKSPACE,
                "dequant-then-GEMM slab workspace missing, too small or unaligned");
        auto* slab = static_cast<uint16_t*>(ws);
        for (int64_t begin = 0; begin < w.N; begin += kSlabRows) {
            const int64_t count = w.N - begin < kSlabRows ? w.N - begin : kSlabRows;
            const float* s = w.scales + begin * w.scale_cols;
            check_hip(fp8lin::launch_dequant(codes + begin * w.K, s, w.scale_cols, slab, w.K, count,
                                             w.K, stream),
                      "dequant launch");
            gemm_bf16_impl(x, slab, y + begin, ldy, rows, count, w.K, stream);
        }
        return FP8LIN_PATH_DEQUANT_GEMM;
    }
    // :234-237
    gemm_bf16_impl(x, static_cast<const uint16_t*>(w.data), y, ldy, rows, w.N, w.K, stream);
    return FP8LIN_PATH_BF16;
}

// The branch, then the weight's bias (src/engine.cpp:240).
int engine_impl(const fp8lin_linear_options& o, const fp8lin_weight& w, const uint16_t* x,
                int64_t rows, uint16_t* y, int64_t ldy, void* ws, size_t ws_bytes,
                hipStream_t stream) {
    validate_engine(o, w, x, rows, y, ldy);
    const int path = engine_branch(o, w, x, rows, y, ldy, ws, ws_bytes, stream);
    if (w.bias) check_hip(fp8lin::launch_bias(y, ldy, w.bias, rows, w.N, stream), "bias launch");
    return path;
}

// src/dual_path.cu:69-72 (residual form) and src/optimized.cu:72 (plain form).
// Only the residual form checks eps (src/dual_path.cu:72); the plain form
// takes it as given (src/optimized.cu:72).
void check_rms(const uint16_t* x, const uint16_t* w, const uint16_t* y, int64_t rows, int64_t D,
               double eps, bool check_eps) {
    require(x && w && y, FP8LIN_ERR_ARGUMENT, "Invalid RMS input: null pointer");
    require(rows > 0 && D > 0 && D < kMaxDim, FP8LIN_ERR_SHAPE, "Invalid RMS input shape");
    require(rows < kMaxGridRows, FP8LIN_ERR_SHAPE, "RMS input: more than 2^22-1 rows");
    require(!check_eps || (std::isfinite(eps) && eps > 0), FP8LIN_ERR_ARGUMENT,
            "Invalid fused residual RMS input: eps must be finite and > 0");
}

// The sections only gate "f < 3 * section" for f < R/2 <= 2048: clamping
// them to [0, 4096] keeps that test unchanged and the product in range.
int clamp_section(int64_t s) { return s < 0 ? 0 : (s > 4096 ? 4096 : (int)s); }

// src/optimized.cu:78: r > 0, r even, r <= D, positions [3, T].  Heads are
// the second grid dimension, 4 per workgroup (at most 65535 workgroups).
constexpr int64_t kMaxRopeHeads = 4 * 65535;
void check_rope(int64_t T, int64_t H, int64_t D, int64_t rotary, int64_t max_d) {
    require(T > 0 && H > 0 && D > 0 && T < kMaxDim && H <= kMaxRopeHeads, FP8LIN_ERR_SHAPE, "Invalid RoPE input");
    require(D <= max_d, FP8LIN_ERR_SHAPE, "RoPE input: head dimension above the kernel's limit");
    require(T * H < kMaxDim, FP8LIN_ERR_SHAPE, "RoPE input: 2^31 rows or more");
    require(rotary > 0 && rotary % 2 == 0 && rotary <= D, FP8LIN_ERR_ARGUMENT, "Invalid RoPE input: rotary size");
}

// src/dual_path.cu:73-75
void check_candidates(int64_t M, int64_t N, int64_t offset, const double* out) {
    require(out != nullptr, FP8LIN_ERR_ARGUMENT, "Invalid vocabulary candidates: null output");
    require(M > 0 && M <= 65535 && N > 0 && offset >= 0 && offset <= INT32_MAX - N, FP8LIN_ERR_SHAPE,
            "Invalid vocabulary candidates");
}

void check_workspace(const void* ws, size_t have, size_t need, const char* what) {
    require(have >= need && (need == 0 || ws != nullptr), FP8LIN_ERR_WORKSPACE, what);
    require(aligned16(ws), FP8LIN_ERR_WORKSPACE, "workspace must be 16-byte aligned");
}

size_t vocab_ws(int64_t M, int64_t N) { return (size_t)(M * fp8lin::vocab_chunks(N) * 8); }

// Output head: the logits (padded to 256 bytes), then the chunk partials.
int64_t logits_bytes(int64_t M, int64_t N) { return (M * N * 2 + 255) / 256 * 256; }
// Either candidate form: the logits and chunk pairs of the two-stage form, or
// the ring GEMV's candidate pairs, slices and counters (M <= 2; no logits).
// The small-M row-range kernel's candidate pairs (M x at most CUs) fit in the
// two-stage form's logits (M x N BF16, N >= 32 CUs there).
size_t linear_candidates_ws(int64_t M, int64_t N) {
    const size_t two_stage = (size_t)logits_bytes(M, N) + vocab_ws(M, N);
    return M <= 2 ? std::max(two_stage, fp8lin::gemv_candidates_ws_bytes((int)M, (int)N)) : two_stage;
}

// Whether fp8lin_linear runs the small-M matrix-core kernel for this call
// (3..8 rows, or 2 at K > 5120 or on a weight of its row-range form, through
// linear_small_m; 9..32 rows through the GEMM dispatch's mid-rows rule).
bool linear_runs_small_m(const uint16_t* x, const uint8_t* codes, int64_t S, int64_t M, int64_t N, int64_t K) {
    return linear_small_m(x, codes, S, M, N, K) || fp8lin::gemm_mid_rows(x, codes, (int)S, M, N, K);
}

void linear_candidates_impl(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t S, int64_t M,
                            int64_t N, int64_t K, int64_t offset, void* ws, double* out, hipStream_t stream) {
    const bool wide = K % 16 == 0 && aligned16(x) && aligned16(codes);
    if (M <= 8 && !linear_runs_small_m(x, codes, S, M, N, K) &&
        fp8lin::gemv_candidates_supported((int)M, (int)N, (int)K, wide)) {
        check_hip(fp8lin::launch_gemv_candidates(x, codes, scales, (int)S, (int)M, (int)N, (int)K, offset, ws, out,
                                                 stream),
                  "fp8 gemv candidates launch");
        return;
    }
    // where fp8lin_linear runs the small-M row-range kernel: its candidate
    // form (the same logits, never stored; at most CUs pairs per row) and one
    // finishing workgroup per row
    if (M <= 32 && linear_runs_small_m(x, codes, S, M, N, K) &&
        fp8lin::small_m_candidates_supported((int)M, (int)N, (int)K)) {
        auto* part = static_cast<uint32_t*>(ws);
        int64_t groups = 0;
        check_hip(fp8lin::launch_small_m_candidates(x, codes, scales, (int)M, (int)N, (int)K, part, groups, stream),
                  "fp8 small-M candidates launch");
        check_hip(fp8lin::launch_candidates_finish(part, (int)M, groups, offset, out, stream),
                  "candidates finish launch");
        return;
    }
    auto* logits = static_cast<uint16_t*>(ws);
    auto* part = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + logits_bytes(M, N));
    linear_impl(x, codes, scales, S, logits, N, M, N, K, stream);
    check_hip(fp8lin::launch_vocab_candidates(logits, (int)M, (int)N, offset, part, out, stream),
              "vocabulary candidates launch");
}

}  // namespace

extern "C" {

int fp8lin_version(void) { return FP8LIN_VERSION; }

const char* fp8lin_last_error(void) { return g_last_error.c_str(); }

int fp8lin_init(void) {
    return guarded([&] { ensure_device(); });
}

int fp8lin_decode(const uint8_t* codes, const float* scales, int64_t scale_cols, uint16_t* y,
                  int64_t rows, int64_t cols, fp8lin_stream_t stream) {
    return guarded([&] {
        // src/kernels.cu:18-19
        require(rows >= 0 && cols >= 0, FP8LIN_ERR_SHAPE, "FP8 codes must be a [rows, cols] matrix");
        if (rows == 0 || cols == 0) return;
        require(codes && y, FP8LIN_ERR_ARGUMENT, "fp8_decode: null pointer");
        check_scales(scales, scale_cols, cols);
        ensure_device();
        check_hip(fp8lin::launch_dequant(codes, scales, scale_cols, y, cols, rows, cols,
                                         as_stream(stream)),
                  "dequant launch");
    });
}

int fp8lin_linear_ld(const uint16_t* x, const uint8_t* codes, const float* scales,
                     int64_t scale_cols, uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                     int vector_gemv, fp8lin_stream_t stream) {
    (void)vector_gemv;  // wide and byte loads give identical bits; alignment decides
    return guarded([&] {
        // src/optimized.cu:62-65
        require(x && codes && y, FP8LIN_ERR_ARGUMENT, "FP8 linear: null pointer");
        check_dims(M, N, K);
        check_scales(scales, scale_cols, K);
        require(ldy >= N, FP8LIN_ERR_SHAPE, "FP8 linear: ldy < N");
        ensure_device();
        linear_impl(x, codes, scales, scale_cols, y, ldy, M, N, K, as_stream(stream));
    });
}

int fp8lin_linear(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t scale_cols,
                  uint16_t* y, int64_t M, int64_t N, int64_t K, int vector_gemv,
                  fp8lin_stream_t stream) {
    return fp8lin_linear_ld(x, codes, scales, scale_cols, y, N, M, N, K, vector_gemv, stream);
}

size_t fp8lin_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) { return linear_ws(M, N, K, N); }

int fp8lin_linear_ws(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t scale_cols,
                     uint16_t* y, int64_t M, int64_t N, int64_t K, int vector_gemv, void* workspace,
                     size_t workspace_bytes, fp8lin_stream_t stream) {
    (void)vector_gemv;
    return guarded([&] {
        // src/optimized.cu:62-65
        require(x && codes && y, FP8LIN_ERR_ARGUMENT, "FP8 linear: null pointer");
        check_dims(M, N, K);
        check_scales(scales, scale_cols, K);
        const size_t need = linear_ws(M, N, K, N);
        check_workspace(workspace, workspace_bytes, need, "FP8 linear: workspace too small");
        ensure_device();
        linear_impl(x, codes, scales, scale_cols, y, N, M, N, K, as_stream(stream), need ? workspace : nullptr,
                    need);
    });
}

int fp8lin_linear_swiglu(const uint16_t* x, const uint8_t* codes, const float* scales,
                         int64_t scale_cols, uint16_t* y, int64_t M, int64_t N, int64_t K,
                         fp8lin_stream_t stream) {
    return guarded([&] {
        require(x && codes && y, FP8LIN_ERR_ARGUMENT, "FP8 linear+SwiGLU: null pointer");
        check_dims(M, N, K);
        require(N % 2 == 0, FP8LIN_ERR_SHAPE, "Invalid SwiGLU input: N must be even");
        check_scales(scales, scale_cols, K);
        ensure_device();
        if (M <= 8) {
            decode_swiglu(x, codes, scales, scale_cols, y, M, N, K, as_stream(stream));
        } else {
            check_hip(fp8lin::launch_gemm(x, codes, scales, (int)scale_cols, y, N / 2, (int)M,
                                          (int)N, (int)K, true, as_stream(stream)),
                      "fp8 gemm+swiglu launch");
        }
    });
}

int fp8lin_add_bias(uint16_t* y, int64_t ldy, const uint16_t* bias, int64_t rows, int64_t N,
                    fp8lin_stream_t stream) {
    return guarded([&] {
        require(rows >= 0 && N >= 0 && N < kMaxDim && rows < kMaxDim, FP8LIN_ERR_SHAPE, "Invalid bias add shape");
        if (rows == 0 || N == 0) return;
        require(y && bias, FP8LIN_ERR_ARGUMENT, "Bias add: null pointer");
        require(ldy >= N, FP8LIN_ERR_SHAPE, "Bias add: ldy < N");
        ensure_device();
        check_hip(fp8lin::launch_bias(y, ldy, bias, rows, N, as_stream(stream)), "bias launch");
    });
}

size_t fp8lin_linear_swiglu_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 8 || N <= 0 || K <= 0 || N % 2 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return 0;
    return fp8lin::gemm_workspace_bytes((int)ceil_div(K, 128), N / 2, (int)M, (int)N, (int)K, true);
}

int fp8lin_linear_swiglu_ws(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t scale_cols,
                            uint16_t* y, int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                            fp8lin_stream_t stream) {
    return guarded([&] {
        require(x && codes && y, FP8LIN_ERR_ARGUMENT, "FP8 linear+SwiGLU: null pointer");
        check_dims(M, N, K);
        require(N % 2 == 0, FP8LIN_ERR_SHAPE, "Invalid SwiGLU input: N must be even");
        check_scales(scales, scale_cols, K);
        const size_t need = fp8lin_linear_swiglu_workspace_bytes(M, N, K);
        check_workspace(workspace, workspace_bytes, need, "linear+SwiGLU: workspace too small");
        ensure_device();
        if (M <= 8) {
            decode_swiglu(x, codes, scales, scale_cols, y, M, N, K, as_stream(stream));
        } else {
            check_hip(fp8lin::launch_gemm_ws(x, codes, scales, (int)scale_cols, y, N / 2, (int)M, (int)N, (int)K,
                                             true, need ? workspace : nullptr, need, as_stream(stream)),
                      "fp8 gemm+swiglu launch");
        }
    });
}

int fp8lin_swiglu(const uint16_t* gate_up, uint16_t* y, int64_t M, int64_t D,
                  fp8lin_stream_t stream) {
    return guarded([&] {
        // src/optimized.cu:74
        require(M >= 0 && D >= 0, FP8LIN_ERR_SHAPE, "Invalid SwiGLU input shape");
        if (M == 0 || D == 0) return;
        require(gate_up && y, FP8LIN_ERR_ARGUMENT, "SwiGLU: null pointer");
        ensure_device();
        check_hip(fp8lin::launch_swiglu(gate_up, y, M, D, as_stream(stream)), "swiglu launch");
    });
}

int fp8lin_linear_shared(const uint16_t* x, const void* weight, const float* scales,
                         int64_t scale_cols, uint16_t* y, int64_t M, int64_t N, int64_t K,
                         fp8lin_stream_t stream) {
    return guarded([&] {
        shared_impl(x, weight, scales, scale_cols, y, N, M, N, K, as_stream(stream));
    });
}

size_t fp8lin_tensor_small_workspace_bytes(int64_t M, int64_t N, int split) {
    if (M <= 0 || N <= 0) return 0;
    return tensor_small_ws(M, N, split);
}

int fp8lin_tensor_small(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                        int64_t M, int64_t N, int64_t K, int split, void* workspace,
                        size_t workspace_bytes, fp8lin_stream_t stream) {
    return guarded([&] {
        tensor_small_impl(x, codes, scales, y, N, M, N, K, split, workspace, workspace_bytes,
                          as_stream(stream));
    });
}

int fp8lin_gemm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t ldy, int64_t M,
                     int64_t N, int64_t K, fp8lin_stream_t stream) {
    return guarded([&] {
        require(x && w && y, FP8LIN_ERR_ARGUMENT, "BF16 GEMM: null pointer");
        check_dims(M, N, K);
        require(ldy >= N, FP8LIN_ERR_SHAPE, "BF16 GEMM: ldy < N");
        ensure_device();
        gemm_bf16_impl(x, w, y, ldy, M, N, K, as_stream(stream));
    });
}

size_t fp8lin_engine_linear_workspace_bytes(const fp8lin_linear_options* options,
                                            const fp8lin_weight* weight, int64_t rows) {
    if (!options || !weight || rows <= 0 || !options_consistent(*options)) return 0;
    return engine_ws(*options, *weight, rows);
}

int fp8lin_engine_linear_path(const fp8lin_linear_options* options, const fp8lin_weight* weight,
                              int64_t rows) {
    if (!options || !weight || rows <= 0 || !options_consistent(*options)) return 0;
    return engine_path(*options, *weight, rows);
}

int fp8lin_engine_linear(const fp8lin_linear_options* options, const fp8lin_weight* weight,
                         const uint16_t* x, int64_t rows, uint16_t* y, int64_t ldy, void* workspace,
                         size_t workspace_bytes, int* path_out, fp8lin_stream_t stream) {
    return guarded([&] {
        require(options && weight, FP8LIN_ERR_ARGUMENT, "Engine linear: null options or weight");
        validate_engine(*options, *weight, x, rows, y, ldy);
        ensure_device();
        const int path = engine_impl(*options, *weight, x, rows, y, ldy, workspace, workspace_bytes,
                                     as_stream(stream));
        if (path_out) *path_out = path;
    });
}

int fp8lin_engine_linear_groups(const fp8lin_linear_options* options, const fp8lin_weight* groups,
                                int ngroups, const uint16_t* x, int64_t rows, uint16_t* y,
                                int64_t ldy, void* workspace, size_t workspace_bytes,
                                fp8lin_stream_t stream) {
    return guarded([&] {
        require(options && groups && ngroups > 0, FP8LIN_ERR_ARGUMENT,
                "Engine linear groups: null options/groups or no group");
        int64_t total = 0;
        for (int g = 0; g < ngroups; ++g) {
            require(groups[g].K == groups[0].K, FP8LIN_ERR_SHAPE,
                    "Engine linear groups: every group must share K");
            total += groups[g].N;
        }
        require(ldy >= total, FP8LIN_ERR_SHAPE, "Engine linear groups: ldy < sum of group N");
        for (int g = 0; g < ngroups; ++g) validate_engine(*options, groups[g], x, rows, y, ldy);
        ensure_device();
        // An FP8 weight then a BF16 weight at one row, both on the ring GEMV
        // (the GDN in_proj_all group): one launch, the same bits.
        if (ngroups == 2 && rows == 1) {
            const fp8lin_weight& a = groups[0];
            const fp8lin_weight& b = groups[1];
            if (engine_path(*options, a, rows) == FP8LIN_PATH_FP8_GEMV &&
                engine_path(*options, b, rows) == FP8LIN_PATH_BF16 && !a.bias && !b.bias && a.K % 16 == 0 &&
                aligned16(x) && aligned16(a.data) && aligned16(b.data)) {
                const hipError_t e = fp8lin::launch_gemv_pair(
                    x, static_cast<const uint8_t*>(a.data), a.scales, (int)a.scale_cols, y, (int)a.N,
                    static_cast<const uint16_t*>(b.data), y + a.N, (int)b.N, ldy, (int)a.K, as_stream(stream));
                if (e != hipErrorNotSupported) {
                    check_hip(e, "gemv pair launch");
                    return;
                }
            }
        }
        int64_t offset = 0;
        for (int g = 0; g < ngroups; ++g) {
            engine_impl(*options, groups[g], x, rows, y + offset, ldy, workspace, workspace_bytes,
                        as_stream(stream));
            offset += groups[g].N;
        }
    });
}

// ---- decode epilogue and output head ----

int fp8lin_rms(const uint16_t* x, const uint16_t* weight, uint16_t* y, int64_t rows, int64_t D,
               double eps, int centered, fp8lin_stream_t stream) {
    return guarded([&] {
        if (rows == 0) return;
        check_rms(x, weight, y, rows, D, eps, false);
        ensure_device();
        check_hip(fp8lin::launch_rms(x, nullptr, weight, nullptr, y, rows, (int)D, (float)eps, centered != 0,
                                     as_stream(stream)),
                  "rms launch");
    });
}

int fp8lin_residual_rms(const uint16_t* x, const uint16_t* update, const uint16_t* weight,
                        uint16_t* residual, uint16_t* y, int64_t rows, int64_t D, double eps,
                        int centered, fp8lin_stream_t stream) {
    return guarded([&] {
        check_rms(x, weight, y, rows, D, eps, true);
        require(update && residual, FP8LIN_ERR_ARGUMENT, "Invalid fused residual RMS input: null pointer");
        ensure_device();
        check_hip(fp8lin::launch_rms(x, update, weight, residual, y, rows, (int)D, (float)eps, centered != 0,
                                     as_stream(stream)),
                  "residual rms launch");
    });
}

int fp8lin_reduce_residual_rms(const uint16_t* x, const uint16_t* partials, int64_t ranks,
                               const uint16_t* weight, uint16_t* residual, uint16_t* y, int64_t rows,
                               int64_t D, double eps, int centered, fp8lin_stream_t stream) {
    return guarded([&] {
        check_rms(x, weight, y, rows, D, eps, true);
        require(partials && residual, FP8LIN_ERR_ARGUMENT, "Invalid reduce + residual RMS input: null pointer");
        require(ranks >= 1 && ranks <= 8, FP8LIN_ERR_SHAPE, "Invalid reduce + residual RMS input: 1..8 ranks");
        ensure_device();
        check_hip(fp8lin::launch_reduce_rms(x, partials, (int)ranks, weight, residual, y, rows, (int)D, (float)eps,
                                            centered != 0, as_stream(stream)),
                  "reduce residual rms launch");
    });
}

int fp8lin_rope(const uint16_t* x, const int64_t* positions, uint16_t* y, int64_t T, int64_t H, int64_t D,
                int64_t rotary, double theta, int64_t height_section, int64_t width_section,
                fp8lin_stream_t stream) {
    return guarded([&] {
        if (T == 0) return;
        require(x && positions && y, FP8LIN_ERR_ARGUMENT, "Invalid RoPE input: null pointer");
        check_rope(T, H, D, rotary, fp8lin::kRopeMaxD);
        ensure_device();
        check_hip(fp8lin::launch_rope(x, positions, y, (int)T, (int)H, (int)D, (int)rotary, (float)theta,
                                      clamp_section(height_section), clamp_section(width_section),
                                      as_stream(stream)),
                  "rope launch");
    });
}

int fp8lin_qk_norm_rope(const uint16_t* projected, int64_t ld, const uint16_t* q_norm, const uint16_t* k_norm,
                        const int64_t* positions, uint16_t* q, uint16_t* k, int64_t T, int64_t H, int64_t HK,
                        int64_t D, int64_t rotary, double theta, int64_t height_section, int64_t width_section,
                        double eps, fp8lin_stream_t stream) {
    return guarded([&] {
        if (T == 0) return;
        require(projected && q_norm && k_norm && positions && q && k, FP8LIN_ERR_ARGUMENT,
                "Invalid Q/K norm + RoPE input: null pointer");
        require(H > 0 && H < kMaxDim, FP8LIN_ERR_SHAPE, "Invalid Q/K norm + RoPE input: query heads");
        require(HK > 0 && HK < kMaxDim, FP8LIN_ERR_SHAPE, "Invalid Q/K norm + RoPE input: key heads");
        check_rope(T, H + HK, D, rotary, 512);
        require(ld >= 2 * (H + HK) * D && ld < kMaxDim, FP8LIN_ERR_SHAPE,
                "Invalid Q/K norm + RoPE input: row stride below H*2D + 2*HK*D");
        ensure_device();
        check_hip(fp8lin::launch_qk_norm_rope(projected, ld, q_norm, k_norm, positions, q, k, (int)T, (int)H,
                                              (int)HK, (int)D, (int)rotary, (float)theta,
                                              clamp_section(height_section), clamp_section(width_section),
                                              (float)eps, true, as_stream(stream)),
                  "qk norm rope launch");
    });
}

size_t fp8lin_vocab_candidates_workspace_bytes(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0 || M >= kMaxDim || N >= kMaxDim) return 0;
    return vocab_ws(M, N);
}

int fp8lin_vocab_candidates(const uint16_t* logits, int64_t M, int64_t N, int64_t offset, double* out,
                            void* workspace, size_t workspace_bytes, fp8lin_stream_t stream) {
    return guarded([&] {
        require(logits != nullptr, FP8LIN_ERR_ARGUMENT, "Invalid vocabulary candidates: null logits");
        check_candidates(M, N, offset, out);
        check_workspace(workspace, workspace_bytes, vocab_ws(M, N), "vocabulary candidates: workspace too small");
        ensure_device();
        check_hip(fp8lin::launch_vocab_candidates(logits, (int)M, (int)N, offset, static_cast<uint32_t*>(workspace),
                                                  out, as_stream(stream)),
                  "vocabulary candidates launch");
    });
}

int fp8lin_merge_candidates(const double* gathered, int64_t ranks, int64_t rows, int64_t* out,
                            fp8lin_stream_t stream) {
    return guarded([&] {
        // src/dual_path.cu:86-88
        require(gathered && out, FP8LIN_ERR_ARGUMENT, "Invalid gathered candidates: null pointer");
        require(ranks > 0 && ranks <= 8 && rows > 0 && rows <= 65535, FP8LIN_ERR_SHAPE,
                "Invalid gathered candidates");
        ensure_device();
        check_hip(fp8lin::launch_merge_candidates(gathered, (int)ranks, rows, out, as_stream(stream)),
                  "merge candidates launch");
    });
}

size_t fp8lin_linear_candidates_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return 0;
    return linear_candidates_ws(M, N);
}

int fp8lin_linear_candidates(const uint16_t* x, const uint8_t* codes, const float* scales,
                             int64_t scale_cols, int64_t M, int64_t N, int64_t K, int64_t offset,
                             double* out, void* workspace, size_t workspace_bytes,
                             fp8lin_stream_t stream) {
    return guarded([&] {
        // src/speculative.cpp:25-27: linear(normalized, "lm_head") then
        // vocabulary_candidates(projected, offset)
        require(x && codes, FP8LIN_ERR_ARGUMENT, "FP8 linear candidates: null pointer");
        check_dims(M, N, K);
        check_scales(scales, scale_cols, K);
        check_candidates(M, N, offset, out);
        check_workspace(workspace, workspace_bytes, linear_candidates_ws(M, N),
                        "linear candidates: workspace too small");
        ensure_device();
        const hipStream_t s = as_stream(stream);
        linear_candidates_impl(x, codes, scales, scale_cols, M, N, K, offset, workspace, out, s);
    });
}

int fp8lin_linear_candidates_static(const uint16_t* x, const uint8_t* codes, const float* scales,
                                    int64_t scale_cols, int64_t M, int64_t N, int64_t K, int64_t offset,
                                    double* out, fp8lin_stream_t stream) {
    return guarded([&] {
        require(x && codes, FP8LIN_ERR_ARGUMENT, "FP8 linear candidates: null pointer");
        check_dims(M, N, K);
        check_scales(scales, scale_cols, K);
        check_candidates(M, N, offset, out);
        require(linear_candidates_ws(M, N) <= (size_t)FP8LIN_STATIC_SCRATCH_BYTES, FP8LIN_ERR_UNSUPPORTED,
                "static linear candidates: the logits and candidate pairs of M x N exceed the "
                "FP8LIN_STATIC_SCRATCH_BYTES scratch; use fp8lin_linear_candidates with a workspace");
        const int dev = ensure_device();
        const hipStream_t s = as_stream(stream);
        char* base = static_cast<char*>(g_scratch[dev]);
        linear_candidates_impl(x, codes, scales, scale_cols, M, N, K, offset, base, out, s);
    });
}

size_t engine_candidates_head(int64_t rows, int64_t N) {
    return (linear_candidates_ws(rows, N) + 255) / 256 * 256;
}

size_t engine_candidates_ws(const fp8lin_linear_options& o, const fp8lin_weight& w, int64_t rows) {
    return engine_candidates_head(rows, w.N) + engine_ws(o, w, rows);
}

size_t fp8lin_engine_linear_candidates_workspace_bytes(const fp8lin_linear_options* options,
                                                       const fp8lin_weight* weight, int64_t rows) {
    if (!options || !weight || rows <= 0 || weight->N <= 0 || rows >= kMaxDim || weight->N >= kMaxDim ||
        !options_consistent(*options))
        return 0;
    return engine_candidates_ws(*options, *weight, rows);
}

int fp8lin_engine_linear_candidates(const fp8lin_linear_options* options, const fp8lin_weight* weight,
                                    const uint16_t* x, int64_t rows, int64_t offset, double* out,
                                    void* workspace, size_t workspace_bytes, int* path_out,
                                    fp8lin_stream_t stream) {
    return guarded([&] {
        // src/speculative.cpp:25-27 with gpu_candidates: Engine::linear(normalized,
        // "lm_head"), then vocabulary_candidates(projected, offset)
        require(options && weight, FP8LIN_ERR_ARGUMENT, "Engine linear candidates: null options or weight");
        require(x != nullptr, FP8LIN_ERR_ARGUMENT, "Engine linear: null pointer");
        check_dims(rows, weight->N, weight->K);
        check_candidates(rows, weight->N, offset, out);
        check_workspace(workspace, workspace_bytes, engine_candidates_ws(*options, *weight, rows),
                        "engine linear candidates: workspace too small");
        char* base = static_cast<char*>(workspace);
        auto* logits = reinterpret_cast<uint16_t*>(base);
        auto* part = reinterpret_cast<uint32_t*>(base + logits_bytes(rows, weight->N));
        const size_t head = engine_candidates_head(rows, weight->N);
        validate_engine(*options, *weight, x, rows, logits, weight->N);
        ensure_device();
        const hipStream_t s = as_stream(stream);
        int path = engine_path(*options, *weight, rows);
        const auto* codes = static_cast<const uint8_t*>(weight->data);
        if (path == FP8LIN_PATH_FP8_GEMV && !weight->bias) {
            // the FP8 GEMV branch is fp8lin_linear: its candidate form
            linear_candidates_impl(x, codes, weight->scales, weight->scale_cols, rows, weight->N, weight->K, offset,
                                   base, out, s);
        } else if (path == FP8LIN_PATH_TENSOR_SMALL && !weight->bias && tensor_small_matrix_core(x, codes, weight->K) &&
                   fp8lin::small_m_candidates_supported((int)rows, (int)weight->N, (int)weight->K)) {
            // the tensor-small branch runs the small-M row-range kernel here:
            // its candidate form gives the candidates of the same logits; its
            // pairs (rows x at most CUs) go where the logits would (rows x N
            // BF16, N >= 32 CUs on this path)
            auto* pairs = reinterpret_cast<uint32_t*>(base);
            int64_t groups = 0;
            check_hip(fp8lin::launch_small_m_candidates(x, codes, weight->scales, (int)rows, (int)weight->N,
                                                        (int)weight->K, pairs, groups, s),
                      "fp8 small-M candidates launch");
            check_hip(fp8lin::launch_candidates_finish(pairs, (int)rows, groups, offset, out, s),
                      "candidates finish launch");
        } else {
            path = engine_impl(*options, *weight, x, rows, logits, weight->N, base + head, workspace_bytes - head, s);
            check_hip(fp8lin::launch_vocab_candidates(logits, (int)rows, (int)weight->N, offset, part, out, s),
                      "vocabulary candidates launch");
        }
        if (path_out) *path_out = path;
    });
}

size_t fp8lin_decode_chain_workspace_bytes(int nlinks) {
    if (nlinks < 1 || nlinks > FP8LIN_CHAIN_MAX_LINKS) return 0;
    return (fp8lin::chain_sync_words(nlinks) * 8 + 255) / 256 * 256;
}

int fp8lin_decode_chain(const fp8lin_chain_link* links, int nlinks, void* workspace, size_t workspace_bytes,
                        fp8lin_stream_t stream) {
    return guarded([&] {
        require(links != nullptr, FP8LIN_ERR_ARGUMENT, "decode chain: null links");
        require(nlinks >= 1 && nlinks <= FP8LIN_CHAIN_MAX_LINKS, FP8LIN_ERR_SHAPE,
                "decode chain: 1 to FP8LIN_CHAIN_MAX_LINKS links");
        fp8lin::ChainLink dev[FP8LIN_CHAIN_MAX_LINKS];
        for (int L = 0; L < nlinks; ++L) {
            const fp8lin_chain_link& k = links[L];
            require(k.codes && k.scales && k.x && k.y, FP8LIN_ERR_ARGUMENT, "decode chain: null pointer in a link");
            check_dims(1, k.N, k.K);
            check_scales(k.scales, k.scale_cols, k.K);
            require(k.after >= -1 && k.after < L, FP8LIN_ERR_ARGUMENT,
                    "decode chain: a link may only wait for an earlier link");
            require(fp8lin::chain_link_supported(k.N, k.K, k.scale_cols, k.swiglu != 0), FP8LIN_ERR_UNSUPPORTED,
                    "decode chain: a link needs K % 16 == 0, K <= 9216 (5120 with SwiGLU, N even) and "
                    "N * K < 2^31");
            dev[L] = fp8lin::ChainLink{k.codes, k.scales, k.scale_cols, k.N, k.K, k.x, k.y, k.swiglu != 0, k.after};
        }
        check_workspace(workspace, workspace_bytes, fp8lin_decode_chain_workspace_bytes(nlinks),
                        "decode chain: workspace too small");
        require(workspace != nullptr, FP8LIN_ERR_WORKSPACE, "decode chain: null workspace");
        ensure_device();
        check_hip(fp8lin::launch_chain(dev, nlinks, static_cast<uint64_t*>(workspace), as_stream(stream)),
                  "decode chain launch");
    });
}

int fp8lin_gen_weights(uint64_t seed, uint32_t tag, int64_t N, int64_t K, float std_dev,
                       uint8_t* codes, float* scales, fp8lin_stream_t stream) {
    return guarded([&] {
        require(codes && scales, FP8LIN_ERR_ARGUMENT, "gen_weights: null pointer");
        require(N > 0 && K > 0 && N < kMaxDim && K < kMaxDim, FP8LIN_ERR_SHAPE,
                "gen_weights: N and K must be positive");
        ensure_device();
        check_hip(fp8lin::launch_gen_weights(seed, tag, N, K, std_dev, codes, scales,
                                             as_stream(stream)),
                  "gen_weights launch");
    });
}

int fp8lin_gen_activations(uint64_t seed, uint32_t tag, int64_t M, int64_t K, uint16_t* x,
                           fp8lin_stream_t stream) {
    return guarded([&] {
        require(x != nullptr, FP8LIN_ERR_ARGUMENT, "gen_activations: null pointer");
        require(M > 0 && K > 0, FP8LIN_ERR_SHAPE, "gen_activations: M and K must be positive");
        ensure_device();
        check_hip(fp8lin::launch_gen_activations(seed, tag, M, K, x, as_stream(stream)),
                  "gen_activations launch");
    });
}

int fp8lin_gen_normal(uint64_t seed, uint32_t tag, uint64_t first, int64_t n, float* out,
                      fp8lin_stream_t stream) {
    return guarded([&] {
        require(out != nullptr && n > 0, FP8LIN_ERR_ARGUMENT, "gen_normal: bad arguments");
        ensure_device();
        check_hip(fp8lin::launch_gen_normal(seed, tag, first, n, out, as_stream(stream)),
                  "gen_normal launch");
    });
}

int fp8lin_stream_read(const void* src, size_t bytes, float* sink, fp8lin_stream_t stream) {
    return guarded([&] {
        require(src && sink && bytes >= 16 && bytes < ((size_t)1 << 40), FP8LIN_ERR_ARGUMENT,
                "stream_read: bad arguments");
        require(aligned16(src), FP8LIN_ERR_ARGUMENT, "stream_read: source must be 16-byte aligned");
        ensure_device();
        check_hip(fp8lin::launch_stream_read(src, bytes, sink, as_stream(stream)),
                  "stream_read launch");
    });
}

int fp8lin_mfma_ceiling(int64_t iters, float* sink, uint64_t* clocks, fp8lin_stream_t stream) {
    return guarded([&] {
        require(sink && clocks && iters > 0, FP8LIN_ERR_ARGUMENT, "mfma_ceiling: bad arguments");
        ensure_device();
        check_hip(fp8lin::launch_mfma_ceiling(iters, sink, clocks, as_stream(stream)), "mfma_ceiling launch");
    });
}

}  // extern "C"
