// stream_exec.cpp -- the reference's C-ABI boundary, re-implemented as a host
// decoder that launches the gfx950 kernels.
//
// Reference: extern "C" void stream_exec(const uint8_t*, size_t)
// (include/ane/ane.hpp:37-39), implemented there by the SME2 interpreter
// loop of src/bytecode_interpreter.s:11-36 (fetch opcode byte, jump through a
// 128-entry table, stop at data+size; slot 0x00 exits).  Records are the
// packed little-endian serialisation made by ane::dispatch
// (include/ane/ane.hpp:206-220): [op:u8] then each argument's object bytes.
//
// Differences from the reference, all additive:
//  * operands are device pointers; every operand extent is checked against
//    its HIP allocation before anything is launched, so a short or host
//    buffer becomes an error instead of a GPU memory fault;
//  * opt-in host staging (ane_set_host_staging, or ANE_HOST_STAGING=1 in
//    the environment): operands in plain host memory (malloc,
//    aligned_alloc) are copied to a device staging buffer, the record runs
//    on the copies, and its outputs are copied back before the record
//    returns, so the reference's callers can keep their host allocations;
//  * scalar outputs (quantize scale_out, channelwise scales) may also be
//    host memory: they are computed on the device and copied back;
//  * errors are recorded per thread (ane_last_error) since the signature
//    returns void; execution stops at the first failing record.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <functional>
#include <vector>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "../../include/ane_decode.h"
#include "../../include/ane_hip.h"

namespace {

thread_local int t_status = ANE_OK;
thread_local std::string t_message;
thread_local hipStream_t t_stream = nullptr;
thread_local bool t_ran_fused = false;  // a dense_fused_i8 record ran in this stream_exec call
thread_local int t_staging = -1;        // host staging: -1 = ANE_HOST_STAGING, 0 off, 1 on

bool staging_on() {
    if (t_staging < 0) {
        const char* e = std::getenv("ANE_HOST_STAGING");
        t_staging = (e && e[0] && std::strcmp(e, "0") != 0) ? 1 : 0;
    }
    return t_staging == 1;
}

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_message = buf;
    return status;
}

// ---------------------------------------------------------------- workspace
// One grow-only device buffer per (device, stream).  Work on one stream is
// ordered, so reusing its buffer between records is safe.  A record holds
// the buffer's lock (a Lease) from the moment it takes the pointer until its
// kernels are enqueued: another host thread on the same stream that needs a
// bigger buffer waits for that, then synchronises the stream (so the
// enqueued kernels have finished) before it frees the old buffer.  Freed at
// process exit.
struct Workspace {
    std::mutex mu;
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
// pool 0: the records' workspaces; pool 1: host staging copies
std::map<std::pair<int, hipStream_t>, Workspace>* g_ws[2] = {nullptr, nullptr};

struct Lease {
    std::unique_lock<std::mutex> lock;
    void* ptr = nullptr;
};

int get_workspace(hipStream_t s, size_t bytes, Lease& lease, int pool = 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(ANE_ERR_HIP, "hipGetDevice failed");
    Workspace* w = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        if (!g_ws[pool]) g_ws[pool] = new std::map<std::pair<int, hipStream_t>, Workspace>();
        w = &(*g_ws[pool])[{dev, s}];  // map nodes never move
    }
    lease.lock = std::unique_lock<std::mutex>(w->mu);
    if (w->bytes < bytes) {
        if (w->ptr) {
            if (hipStreamSynchronize(s) != hipSuccess) return fail(ANE_ERR_HIP, "stream sync failed");
            (void)hipFree(w->ptr);
            w->ptr = nullptr;
            w->bytes = 0;
        }
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        if (hipMalloc(&w->ptr, want) != hipSuccess) {
            (void)hipGetLastError();
            w->ptr = nullptr;
            return fail(ANE_ERR_HIP, "workspace hipMalloc(%zu) failed", want);
        }
        w->bytes = want;
    }
    lease.ptr = w->ptr;
    return ANE_OK;
}

// ------------------------------------------------------------ pointer checks
enum class Where { kDevice, kHost };

// Returns ANE_OK if [p, p+bytes) lies inside one device-accessible
// allocation.  *where reports unregistered host memory when host_ok.
int check_range(const void* p, uint64_t bytes, const char* name, bool host_ok, Where* where) {
    if (where) *where = Where::kDevice;
    if (bytes == 0) return ANE_OK;
    if (!p) return fail(ANE_ERR_BAD_POINTER, "%s is null", name);
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof attr);
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess || attr.type == hipMemoryTypeUnregistered) {
        (void)hipGetLastError();
        if (host_ok) {
            if (where) *where = Where::kHost;
            return ANE_OK;
        }
        return fail(ANE_ERR_BAD_POINTER,
                    "%s (%p) is not device-accessible memory (use hipMalloc/hipMallocManaged/"
                    "hipHostMalloc)",
                    name, p);
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    e = hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p);
    if (e != hipSuccess || !base) {
        (void)hipGetLastError();
        return fail(ANE_ERR_BAD_POINTER, "%s (%p): allocation extent unknown", name, p);
    }
    const uint64_t off = (uint64_t)((const char*)p - (const char*)base);
    if (off > size || bytes > size - off)
        return fail(ANE_ERR_BUFFER_TOO_SMALL, "%s needs %llu bytes at %p, allocation holds %llu", name,
                    (unsigned long long)bytes, p, (unsigned long long)(size - (off > size ? size : off)));
    return ANE_OK;
}

#define CHECK(expr)                 \
    do {                            \
        int st__ = (expr);          \
        if (st__ != ANE_OK) return st__; \
    } while (0)

// ------------------------------------------------------------ host staging
// A record's operands, checked and (in staging mode) mapped.  operand()
// checks one operand's extent as before; in staging mode an operand in
// unregistered host memory is instead given a slot in the stream's staging
// buffer, and commit() then copies the inputs there and repoints the
// record's pointers at the copies.  finish() copies the outputs back and
// waits for them.  Without staging, host memory stays an error.
enum Dir { kIn = 1, kOut = 2, kInOut = 3 };

class Stager {
  public:
    explicit Stager(hipStream_t s) : s_(s) {}

    template <typename T>
    int operand(T*& p, uint64_t bytes, const char* name, Dir dir) {
        if (bytes == 0) return ANE_OK;
        Where w = Where::kDevice;
        CHECK(check_range(p, bytes, name, staging_on(), &w));
        if (w == Where::kHost) {
            T** slot = &p;
            items_.push_back({(void*)p, 0, bytes, dir, [slot](void* d) { *slot = reinterpret_cast<T*>(d); }});
        }
        return ANE_OK;
    }

    int commit() {
        if (items_.empty()) return ANE_OK;
        size_t total = 0;
        for (Item& it : items_) {
            it.offset = total;
            total += (it.bytes + 255) & ~(size_t)255;
        }
        CHECK(get_workspace(s_, total, lease_, 1));
        for (Item& it : items_) {
            void* d = (uint8_t*)lease_.ptr + it.offset;
            if ((it.dir & kIn) && hipMemcpyAsync(d, it.host, it.bytes, hipMemcpyHostToDevice, s_) != hipSuccess) {
                (void)hipGetLastError();
                return fail(ANE_ERR_HIP, "host staging: copy of %zu input bytes failed", it.bytes);
            }
            it.set(d);
        }
        return ANE_OK;
    }

    int finish(int st) {
        if (items_.empty() || st != ANE_OK) return st;
        for (Item& it : items_) {
            if (!(it.dir & kOut)) continue;
            const void* d = (uint8_t*)lease_.ptr + it.offset;
            if (hipMemcpyAsync(it.host, d, it.bytes, hipMemcpyDeviceToHost, s_) != hipSuccess) {
                (void)hipGetLastError();
                return fail(ANE_ERR_HIP, "host staging: copy of %zu output bytes failed", it.bytes);
            }
        }
        if (hipStreamSynchronize(s_) != hipSuccess) {
            (void)hipGetLastError();
            return fail(ANE_ERR_HIP, "host staging: stream synchronize failed");
        }
        return st;
    }

  private:
    struct Item {
        void* host;
        size_t offset;
        uint64_t bytes;
        Dir dir;
        std::function<void(void*)> set;
    };
    hipStream_t s_;
    std::vector<Item> items_;
    Lease lease_;
};

uint64_t ceil_u(uint64_t x, uint64_t m) { return (x + m - 1) / m * m; }

// ------------------------------------------------------------ record reader
struct Reader {
    const uint8_t* p;
    size_t left;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if (left < sizeof(T)) {
            ok = false;
            left = 0;
            return v;
        }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        left -= sizeof(T);
        return v;
    }
    template <typename T>
    T* ptr() {
        uint64_t v = get<uint64_t>();
        return reinterpret_cast<T*>((uintptr_t)v);
    }
};

int hip_status(int st, const char* what) {
    if (st == ANE_OK) return ANE_OK;
    if (t_message.empty()) return fail(st, "%s failed with status %d", what, st);
    return st;
}

// Runs a quantize-type record whose scalar outputs may live in host memory.
int copy_back(hipStream_t s, void* host_dst, const void* dev_src, size_t bytes) {
    if (hipMemcpyAsync(host_dst, dev_src, bytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        (void)hipGetLastError();
        return fail(ANE_ERR_HIP, "copy of scalar outputs to host failed");
    }
    return ANE_OK;
}

// 0x19 [count:u32][src][dst][scale_out]  (bytecode_interpreter.s:1885-1890)
int op_quantize(Reader& r, hipStream_t s) {
    const uint32_t count = r.get<uint32_t>();
    const float* src = r.ptr<const float>();
    int8_t* dst = r.ptr<int8_t>();
    float* scale_out = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "quantize_fp32_i8 record truncated");
    uint64_t n = ceil_u(count, 16);
    if (n == 0) n = 16;
    Where w;
    Stager st(s);
    CHECK(st.operand(src, n * 4, "quantize_fp32_i8 src", kIn));
    CHECK(st.operand(dst, n, "quantize_fp32_i8 dst", kOut));
    CHECK(check_range(scale_out, 4, "quantize_fp32_i8 scale_out", true, &w));
    CHECK(st.commit());
    const size_t wsb = ane_hip_quantize_workspace_size(n) + 256;
    Lease lease;
    CHECK(get_workspace(s, wsb, lease));
    void* ws = lease.ptr;
    float* dev_scale = w == Where::kHost ? (float*)ws : scale_out;
    void* part = (uint8_t*)ws + 256;
    CHECK(hip_status(ane_hip_quantize_fp32_i8(count, 1, src, dst, dev_scale, part, wsb - 256, s),
                     "quantize_fp32_i8"));
    if (w == Where::kHost) CHECK(copy_back(s, scale_out, dev_scale, 4));
    return st.finish(ANE_OK);
}

// 0x1A [count:u32][scale:f32][src][dst]  (bytecode_interpreter.s:1959-1963)
int op_dequantize(Reader& r, hipStream_t s) {
    const uint32_t count = r.get<uint32_t>();
    const float scale = r.get<float>();
    const int8_t* src = r.ptr<const int8_t>();
    float* dst = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "dequantize_i8_fp32 record truncated");
    const uint64_t n = ceil_u(count, 16);
    Stager st(s);
    CHECK(st.operand(src, n, "dequantize_i8_fp32 src", kIn));
    CHECK(st.operand(dst, n * 4, "dequantize_i8_fp32 dst", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_dequantize_i8_fp32(count, scale, src, dst, s), "dequantize_i8_fp32"));
}

// 0x1B [K:u32][N:u32][src][dst]  (bytecode_interpreter.s:2460-2464)
int op_pack_b(Reader& r, hipStream_t s) {
    const uint32_t K = r.get<uint32_t>();
    const uint32_t N = r.get<uint32_t>();
    const int8_t* src = r.ptr<const int8_t>();
    int8_t* dst = r.ptr<int8_t>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "pack_b_i8 record truncated");
    Stager st(s);
    CHECK(st.operand(src, (uint64_t)K * N, "pack_b_i8 src", kIn));
    CHECK(st.operand(dst, ane_hip_packed_b_size(K, N), "pack_b_i8 dst", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_pack_b_i8(K, N, src, dst, s), "pack_b_i8"));
}

// 0x1C [rows:u32][cols:u32][src][dst][scales]  (bytecode_interpreter.s:2592-2597)
int op_channelwise(Reader& r, hipStream_t s) {
    const uint32_t rows = r.get<uint32_t>();
    const uint32_t cols = r.get<uint32_t>();
    const float* src = r.ptr<const float>();
    int8_t* dst = r.ptr<int8_t>();
    float* scales = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "quantize_fp32_i8_channelwise record truncated");
    if (rows == 0) return ANE_OK;
    uint64_t cpad = ceil_u(cols, 16);
    if (cpad == 0) cpad = 16;
    Where w;
    Stager st(s);
    CHECK(st.operand(src, (uint64_t)rows * cpad * 4, "channelwise src", kIn));
    CHECK(st.operand(dst, (uint64_t)rows * cpad, "channelwise dst", kOut));
    CHECK(check_range(scales, (uint64_t)rows * 4, "channelwise scales", true, &w));
    CHECK(st.commit());
    float* dev_scales = scales;
    Lease lease;
    if (w == Where::kHost) {
        CHECK(get_workspace(s, (size_t)rows * 4, lease));
        dev_scales = (float*)lease.ptr;
    }
    CHECK(hip_status(ane_hip_quantize_channelwise(rows, cols, src, dst, dev_scales, s),
                     "quantize_fp32_i8_channelwise"));
    if (w == Where::kHost) CHECK(copy_back(s, scales, dev_scales, (size_t)rows * 4));
    return st.finish(ANE_OK);
}

// 0x18 / 0x1E [M][N][K][sa][sb][flags:u8][A][Bp][bias][C]
// (bytecode_interpreter.s:1997-2007, 2851-2861)
int op_dense(Reader& r, hipStream_t s, bool a_unsigned) {
    const uint32_t M = r.get<uint32_t>();
    const uint32_t N = r.get<uint32_t>();
    const uint32_t K = r.get<uint32_t>();
    const float sa = r.get<float>();
    const float sb = r.get<float>();
    const uint8_t flags = r.get<uint8_t>();
    const void* A = r.ptr<const void>();
    const int8_t* Bp = r.ptr<const int8_t>();
    const float* bias = r.ptr<const float>();
    float* C = r.ptr<float>();
    const char* nm = a_unsigned ? "dense_u8s8" : "dense_i8";
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "%s record truncated", nm);
    if (N == 0) return ANE_OK;  // every column store is predicated off
    const uint64_t Kp = ceil_u(K, 64);
    uint64_t Mp = ceil_u(M, 16);
    if (Mp == 0) Mp = 16;
    const uint64_t P = ceil_u(N, 16) / 16, G = Kp / 4;
    if (((uintptr_t)A & 15) || ((uintptr_t)Bp & 15))
        return fail(ANE_ERR_INVALID_ARG, "%s: A and B_packed must be 16-byte aligned", nm);
    Stager st(s);
    CHECK(st.operand(A, Mp * Kp, "dense A", kIn));
    CHECK(st.operand(Bp, P * G * 64, "dense B_packed", kIn));
    CHECK(st.operand(bias, (uint64_t)N * 4, "dense bias", kIn));
    CHECK(st.operand(C, Mp * N * 4, "dense C", kOut));
    CHECK(st.commit());
    return st.finish(
        hip_status(ane_hip_dense_i8(M, N, K, sa, sb, flags, A, Bp, bias, C, a_unsigned ? 1 : 0, s), nm));
}

// 0x57 [M:u32][K:u32][x][W][y]  (bytecode_interpreter.s:7017-7023)
int op_q8_0_gemv(Reader& r, hipStream_t s) {
    const uint32_t M = r.get<uint32_t>();
    const uint32_t K = r.get<uint32_t>();
    const float* x = r.ptr<const float>();
    const void* W = r.ptr<const void>();
    float* y = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "q8_0_gemv record truncated");
    if (M == 0) return ANE_OK;
    const uint64_t nb = K >> 5;
    if ((uintptr_t)W & 1) return fail(ANE_ERR_INVALID_ARG, "q8_0_gemv: W must be 2-byte aligned");
    Stager st(s);
    CHECK(st.operand(x, nb * 32 * 4, "q8_0_gemv x", kIn));
    CHECK(st.operand(W, (uint64_t)M * nb * 34, "q8_0_gemv W", kIn));
    CHECK(st.operand(y, (uint64_t)M * 4, "q8_0_gemv y", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_q8_0_gemv(M, K, x, W, y, s), "q8_0_gemv"));
}

// 0x80 [M:i32][N:i32][K:i32][scale:f32][relu:bool][A][B][C]  (README.md:87-97)
int op_dense_fused(Reader& r, hipStream_t s) {
    const int32_t M = r.get<int32_t>();
    const int32_t N = r.get<int32_t>();
    const int32_t K = r.get<int32_t>();
    const float scale = r.get<float>();
    const uint8_t relu = r.get<uint8_t>();
    const float* A = r.ptr<const float>();
    const float* B = r.ptr<const float>();
    float* C = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "dense_fused_i8 record truncated");
    if (M < 0 || N < 0 || K < 0) return fail(ANE_ERR_INVALID_ARG, "dense_fused_i8: negative shape");
    if (M == 0 || N == 0) return ANE_OK;
    Stager st(s);
    CHECK(st.operand(A, (uint64_t)M * K * 4, "dense_fused_i8 A", kIn));
    CHECK(st.operand(B, (uint64_t)K * N * 4, "dense_fused_i8 B", kIn));
    CHECK(st.operand(C, (uint64_t)M * N * 4, "dense_fused_i8 C", kOut));
    CHECK(st.commit());
    const size_t wsb = ane_hip_dense_fused_i8_workspace_size(M, N, K);
    Lease lease;
    CHECK(get_workspace(s, wsb, lease));
    t_ran_fused = true;
    return st.finish(hip_status(
        ane_hip_dense_fused_i8(M, N, K, scale, relu & 1, A, B, C, nullptr, lease.ptr, wsb, s), "dense_fused_i8"));
}

// 0x61 / 0x62 / 0x63 [flags:u8][M][N][K][lda][ldb][ldc:u32][alpha:f32][beta:f32][A][B][C]
// (bytecode_interpreter.s:8355-8369).  The extents checked are exactly the
// bytes the handler's arithmetic uses: A and B only over the K/64 whole
// blocks, C over rows < M and columns < N (read too when beta's bits are
// nonzero).
int op_cblas_igemm(Reader& r, hipStream_t s, int variant) {
    static const char* const kName[3] = {"cblas_igemm", "cblas_ugemm", "cblas_usgemm"};
    const char* nm = kName[variant];
    const uint8_t flags = r.get<uint8_t>();
    const uint32_t M = r.get<uint32_t>();
    const uint32_t N = r.get<uint32_t>();
    const uint32_t K = r.get<uint32_t>();
    const uint32_t lda = r.get<uint32_t>();
    const uint32_t ldb = r.get<uint32_t>();
    const uint32_t ldc = r.get<uint32_t>();
    const float alpha = r.get<float>();
    const float beta = r.get<float>();
    const void* A = r.ptr<const void>();
    const void* B = r.ptr<const void>();
    float* C = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "%s record truncated", nm);
    if (M == 0 || N == 0) return ANE_OK;
    if (ldc < N) return fail(ANE_ERR_INVALID_ARG, "%s: ldc %u < N %u (overlapping output rows)", nm, ldc, N);
    if ((uintptr_t)C & 3) return fail(ANE_ERR_INVALID_ARG, "%s: C must be 4-byte aligned", nm);
    const uint64_t Ke = (uint64_t)(K / 64) * 64;
    Stager st(s);
    if (Ke) {
        uint64_t a_ext;
        if (!(flags & 1)) {
            a_ext = (uint64_t)(M - 1) * lda + Ke;
        } else {  // row i reads from (i%16)*lda + (i - i%16)
            const uint64_t g = (uint64_t)(M - 1) - (M - 1) % 16;
            uint64_t mx = (uint64_t)((M - 1) % 16) * lda + g;
            if (M > 16) mx = std::max(mx, (uint64_t)15 * lda + g - 16);
            a_ext = mx + Ke;
        }
        const uint64_t b_ext = (flags & 2) ? (uint64_t)(N - 1) * ldb + Ke : (Ke - 1) * ldb + N;
        CHECK(st.operand(A, a_ext, nm, kIn));
        CHECK(st.operand(B, b_ext, nm, kIn));
    }
    // C is read too (beta, and the gaps between rows when ldc > N)
    CHECK(st.operand(C, ((uint64_t)(M - 1) * ldc + N) * 4, nm, kInOut));
    CHECK(st.commit());
    const size_t wsb = ane_hip_cblas_igemm_workspace_size(M, N, K);
    Lease lease;
    CHECK(get_workspace(s, wsb, lease));
    return st.finish(hip_status(ane_hip_cblas_igemm(variant, ANE_IGEMM_REFERENCE, flags, M, N, K, lda, ldb, ldc,
                                                    alpha, beta, A, B, C, lease.ptr, wsb, s),
                                nm));
}

// The decode-step handlers (bytecode_interpreter.s:6508-7009).  Their loops
// step 16 lanes with no tail, so a dim or count that is not a multiple of 16
// (which never ends there) is refused.
// 0x51 [dim:u32][eps:f32][in][w][out]  (:6509-6514)
int op_rms_norm(Reader& r, hipStream_t s) {
    const uint32_t dim = r.get<uint32_t>();
    const float eps = r.get<float>();
    const float* in = r.ptr<const float>();
    const float* w = r.ptr<const float>();
    float* out = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "rms_norm_fp32 record truncated");
    if (dim == 0) return ANE_OK;
    if (dim % 16) return fail(ANE_ERR_INVALID_ARG, "rms_norm_fp32: dim %u is not a multiple of 16", dim);
    Stager st(s);
    CHECK(st.operand(in, (uint64_t)dim * 4, "rms_norm_fp32 in", kIn));
    CHECK(st.operand(w, (uint64_t)dim * 4, "rms_norm_fp32 weight", kIn));
    CHECK(st.operand(out, (uint64_t)dim * 4, "rms_norm_fp32 out", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_rms_norm_fp32(1, dim, eps, in, w, out, s), "rms_norm_fp32"));
}

// 0x54 [count:u32][in][out]  (:6618-6621)
int op_silu(Reader& r, hipStream_t s) {
    const uint32_t count = r.get<uint32_t>();
    const float* in = r.ptr<const float>();
    float* out = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "silu_fp32 record truncated");
    if (count == 0) return ANE_OK;
    if (count % 16) return fail(ANE_ERR_INVALID_ARG, "silu_fp32: count %u is not a multiple of 16", count);
    Stager st(s);
    CHECK(st.operand(in, (uint64_t)count * 4, "silu_fp32 in", kIn));
    CHECK(st.operand(out, (uint64_t)count * 4, "silu_fp32 out", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_silu_fp32(count, in, out, s), "silu_fp32"));
}

// 0x55 [dim:u32][pos:u32][theta:f32][in][out]  (:6715-6720); pairs dim/2
int op_rope(Reader& r, hipStream_t s) {
    const uint32_t dim = r.get<uint32_t>();
    const uint32_t pos = r.get<uint32_t>();
    const float theta = r.get<float>();
    const float* in = r.ptr<const float>();
    float* out = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "rope_fp32 record truncated");
    const uint64_t n = (uint64_t)(dim / 2) * 2;
    if (n == 0) return ANE_OK;
    Stager st(s);
    CHECK(st.operand(in, n * 4, "rope_fp32 in", kIn));
    CHECK(st.operand(out, n * 4, "rope_fp32 out", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_rope_fp32(1, dim, pos, theta, in, out, s), "rope_fp32"));
}

// 0x56 [dim:u32][in][out]  (:6914-6917)
int op_softmax(Reader& r, hipStream_t s) {
    const uint32_t dim = r.get<uint32_t>();
    const float* in = r.ptr<const float>();
    float* out = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "softmax_fp32 record truncated");
    if (dim == 0) return ANE_OK;
    if (dim % 16) return fail(ANE_ERR_INVALID_ARG, "softmax_fp32: dim %u is not a multiple of 16", dim);
    Stager st(s);
    CHECK(st.operand(in, (uint64_t)dim * 4, "softmax_fp32 in", kIn));
    CHECK(st.operand(out, (uint64_t)dim * 4, "softmax_fp32 out", kOut));
    CHECK(st.commit());
    return st.finish(hip_status(ane_hip_softmax_fp32(1, dim, in, out, s), "softmax_fp32"));
}

// 0x58, 0x75-0x79 [M:u32][K:u32][x][W][y]: the other weight formats' GEMVs
// (bytecode_interpreter.s:7071-7079, 11024-11032 and the same prologue in
// each K-quant handler).
struct QGemv {
    uint8_t op;
    const char* name;
    uint32_t bytes, values;
    int (*fn)(uint32_t, uint32_t, const float*, const void*, float*, void*);
};
const QGemv kQGemv[] = {
    {ANE_OP_Q4_0_GEMV, "q4_0_gemv", 18, 32, ane_hip_q4_0_gemv},
    {ANE_OP_Q4_K_GEMV, "q4_k_gemv", 144, 256, ane_hip_q4_k_gemv},
    {ANE_OP_Q2_K_GEMV, "q2_k_gemv", 84, 256, ane_hip_q2_k_gemv},
    {ANE_OP_Q3_K_GEMV, "q3_k_gemv", 110, 256, ane_hip_q3_k_gemv},
    {ANE_OP_Q5_K_GEMV, "q5_k_gemv", 176, 256, ane_hip_q5_k_gemv},
    {ANE_OP_Q6_K_GEMV, "q6_k_gemv", 210, 256, ane_hip_q6_k_gemv},
};

int op_q_gemv(Reader& r, hipStream_t s, const QGemv& f) {
    const uint32_t M = r.get<uint32_t>();
    const uint32_t K = r.get<uint32_t>();
    const float* x = r.ptr<const float>();
    const void* W = r.ptr<const void>();
    float* y = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "%s record truncated", f.name);
    if (M == 0) return ANE_OK;
    const uint64_t nsb = K / f.values;
    Stager st(s);
    CHECK(st.operand(x, nsb * f.values * 4, f.name, kIn));
    CHECK(st.operand(W, (uint64_t)M * nsb * f.bytes, f.name, kIn));
    CHECK(st.operand(y, (uint64_t)M * 4, f.name, kOut));
    CHECK(st.commit());
    return st.finish(hip_status(f.fn(M, K, x, W, y, s), f.name));
}

// 0x7C / 0x7D [n_rows:u32][dim:u32][table][indices][out]
// (bytecode_interpreter.s:12363-12370, 12419-12426).  The indices are read
// back (after the stream's earlier work) to check every row against the
// table's allocation, which the reference does not do.
int op_get_rows(Reader& r, hipStream_t s, bool q4) {
    const char* name = q4 ? "get_rows_q4_0" : "get_rows_q8_0";
    const uint32_t n = r.get<uint32_t>();
    const uint32_t dim = r.get<uint32_t>();
    const void* table = r.ptr<const void>();
    const uint32_t* idx = r.ptr<const uint32_t>();
    float* out = r.ptr<float>();
    if (!r.ok) return fail(ANE_ERR_TRUNCATED, "%s record truncated", name);
    const uint64_t nb = dim >> 5;
    if (n == 0 || nb == 0) return ANE_OK;
    if (dim & 31) return fail(ANE_ERR_INVALID_ARG, "%s: dim %u is not a multiple of 32", name, dim);
    CHECK(check_range(idx, (uint64_t)n * 4, name, staging_on(), nullptr));
    CHECK(check_range(out, (uint64_t)n * nb * 32 * 4, name, staging_on(), nullptr));
    CHECK(check_range(table, 1, name, staging_on(), nullptr));
    std::vector<uint32_t> h(n);
    if (hipStreamSynchronize(s) != hipSuccess || hipMemcpy(h.data(), idx, (size_t)n * 4, hipMemcpyDefault) != hipSuccess) {
        (void)hipGetLastError();
        return fail(ANE_ERR_HIP, "%s: reading the indices failed", name);
    }
    uint32_t mx = 0;
    for (uint32_t v : h) mx = v > mx ? v : mx;
    const uint64_t rb = nb * (q4 ? 18 : 34);
    Stager st(s);
    CHECK(st.operand(table, ((uint64_t)mx + 1) * rb, name, kIn));
    CHECK(st.operand(idx, (uint64_t)n * 4, name, kIn));
    CHECK(st.operand(out, (uint64_t)n * nb * 32 * 4, name, kOut));
    CHECK(st.commit());
    const uint64_t rows = (uint64_t)mx + 1;
    return st.finish(hip_status(q4 ? ane_hip_get_rows_q4_0(n, dim, table, rows, idx, out, s)
                                   : ane_hip_get_rows_q8_0(n, dim, table, rows, idx, out, s),
                                name));
}

int run(const uint8_t* data, size_t size, hipStream_t s) {
    t_message.clear();
    if (size && !data) return fail(ANE_ERR_BAD_POINTER, "stream is null");
    Reader r{data, size};
    while (r.left > 0) {
        const size_t at = size - r.left;
        const uint8_t op = r.get<uint8_t>();
        int st = ANE_OK;
        switch (op) {
            case 0x00:
                return ANE_OK;  // jump-table slot 0 is .L_exit
            case ANE_OP_DENSE_I8: st = op_dense(r, s, false); break;
            case ANE_OP_QUANTIZE_FP32_I8: st = op_quantize(r, s); break;
            case ANE_OP_DEQUANTIZE_I8_FP32: st = op_dequantize(r, s); break;
            case ANE_OP_PACK_B_I8: st = op_pack_b(r, s); break;
            case ANE_OP_QUANTIZE_FP32_I8_CHANNELWISE: st = op_channelwise(r, s); break;
            case ANE_OP_DENSE_U8S8: st = op_dense(r, s, true); break;
            case ANE_OP_Q8_0_GEMV: st = op_q8_0_gemv(r, s); break;
            case ANE_OP_DENSE_FUSED_I8: st = op_dense_fused(r, s); break;
            case ANE_OP_GET_ROWS_Q8_0: st = op_get_rows(r, s, false); break;
            case ANE_OP_GET_ROWS_Q4_0: st = op_get_rows(r, s, true); break;
            case ANE_OP_RMS_NORM_FP32: st = op_rms_norm(r, s); break;
            case ANE_OP_SILU_FP32: st = op_silu(r, s); break;
            case ANE_OP_ROPE_FP32: st = op_rope(r, s); break;
            case ANE_OP_SOFTMAX_FP32: st = op_softmax(r, s); break;
            case ANE_OP_CBLAS_IGEMM: st = op_cblas_igemm(r, s, ANE_IGEMM_SIGNED); break;
            case ANE_OP_CBLAS_UGEMM: st = op_cblas_igemm(r, s, ANE_IGEMM_UNSIGNED); break;
            case ANE_OP_CBLAS_USGEMM: st = op_cblas_igemm(r, s, ANE_IGEMM_MIXED); break;
            default: {
                const QGemv* f = nullptr;
                for (const QGemv& q : kQGemv)
                    if (q.op == op) f = &q;
                if (f) {
                    st = op_q_gemv(r, s, *f);
                    break;
                }
                return fail(ANE_ERR_UNKNOWN_OPCODE,
                            "opcode 0x%02x at byte %zu is not part of the quantized path served by "
                            "this build",
                            op, at);
            }
        }
        if (st != ANE_OK) {
            if (t_message.empty()) fail(st, "record at byte %zu failed", at);
            return st;
        }
    }
    return ANE_OK;
}

}  // namespace

extern "C" void stream_exec(const uint8_t* data, size_t size) {
    hipStream_t s = t_stream;
    t_ran_fused = false;
    int st = run(data, size, s);
    if (hipStreamSynchronize(s) != hipSuccess) {
        (void)hipGetLastError();
        if (st == ANE_OK) st = fail(ANE_ERR_HIP, "hipStreamSynchronize failed");
    }
    if (t_ran_fused) {
        const int ws = ane_hip_grid_wait_status(s);
        if (ws != ANE_OK && st == ANE_OK)
            st = fail(ws, "dense_fused_i8: the quantizer's grid-wide wait gave up or saw another launch's "
                          "arrivals; C is not valid");
    }
    t_status = st;
}

extern "C" int ane_stream_exec_async(const uint8_t* data, size_t size, void* stream) {
    int st = run(data, size, (hipStream_t)stream);
    t_status = st;
    return st;
}

extern "C" int ane_last_error(void) { return t_status; }

extern "C" const char* ane_last_error_message(void) {
    return t_status == ANE_OK ? "" : t_message.c_str();
}

extern "C" void ane_set_stream(void* stream) { t_stream = (hipStream_t)stream; }

extern "C" void ane_set_host_staging(int mode) { t_staging = mode < 0 ? -1 : (mode ? 1 : 0); }

extern "C" int ane_hip_device_check(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return ANE_ERR_NO_DEVICE;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ANE_ERR_HIP;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return ANE_ERR_HIP;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return ANE_ERR_NO_DEVICE;
    return ANE_OK;
}

extern "C" const char* ane_hip_version(void) { return "ane_amd 0.1 (gfx950)"; }
