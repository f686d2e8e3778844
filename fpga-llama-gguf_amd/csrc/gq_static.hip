// The allocation-free batched GEMV (gemvq_gemm_static in include/gemvq_hip.h): the GEMM command's two kernels on
// caller-owned device buffers. The quantized activation rows, which the GEMM command stages in its context's
// buffers, are staged here in `scratch`, a fixed device array of this file (one copy per device, held until the
// process ends). Nothing here allocates: the array's address on a device is looked up once, on the first call on
// that device, and kept.
#include "gemvq_hip.h"
#include "gq_kernels.h"

#include <hip/hip_runtime.h>

#include <mutex>

using namespace gq;

namespace {

constexpr size_t Q_BYTES = size_t(GEMM_MAX_TOK) * GEMV_MAXK;          // quants of up to 32 token rows
constexpr size_t BLOCKS = size_t(GEMM_MAX_TOK) * (GEMV_MAXK / 32);    // their per-block scale words
constexpr size_t SCRATCH_BYTES = Q_BYTES + 2 * BLOCKS * sizeof(float);  // 640 KiB
static_assert(SCRATCH_BYTES == GEMVQ_STATIC_SCRATCH_BYTES, "scratch size in the header");

__device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mutex;
uint8_t * g_scratch[MAX_DEVICES];  // scratch's device address on each device (the host-side name is not one)

// The address of `scratch` on the current device, looked up on the first call there.
int scratch_on(int dev, uint8_t ** out) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_scratch[dev]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return -int(e);
        g_scratch[dev] = static_cast<uint8_t *>(p);
    }
    *out = g_scratch[dev];
    return 0;
}

bool aligned(const void * p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

extern "C" int gemvq_gemm_static(int type, int rows, int cols, const void * w, const float * x, int n_tok, int x_stride,
                                 float * y, int y_stride, void * stream) {
    if (type != T_Q4_0 && type != T_Q4_1 && type != T_Q8_0) return GEMVQ_EINVAL;
    if (rows < 1 || cols < 512 || cols % 512 || cols > int(GEMVQ_MAX_COLS)) return GEMVQ_EINVAL;
    if (n_tok < 1 || n_tok > int(GEMVQ_GEMM_MAX_TOK)) return GEMVQ_EINVAL;  // the scratch holds 32 token rows
    if (x_stride < cols || x_stride % 16 || y_stride < rows || y_stride % 16) return GEMVQ_EINVAL;
    if (!w || !x || !y || !aligned(w, 256) || !aligned(x, 64) || !aligned(y, 64)) return GEMVQ_EINVAL;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return -int(e);
    if (dev < 0 || dev >= MAX_DEVICES) return GEMVQ_EINVAL;
    uint8_t * base = nullptr;
    const int st = scratch_on(dev, &base);
    if (st) return st;
    GemmQuantArgs q{};
    q.x = x;
    q.norm_w = nullptr;
    q.q = reinterpret_cast<int8_t *>(base);
    q.d40 = reinterpret_cast<float *>(base + Q_BYTES);
    q.s40 = q.d40 + BLOCKS;
    q.n_tok = n_tok;
    q.n_pad = (n_tok + 15) / 16 * 16;  // the quantizer writes the padding rows too: nothing needs clearing
    q.cols = cols;
    q.x_stride = x_stride;
    GemmArgs g{};
    g.w = weight_view(static_cast<const uint8_t *>(w), type, rows, cols);
    g.q = q.q;
    g.d40 = q.d40;
    g.s40 = q.s40;
    g.y = y;
    g.rows = rows;
    g.cols = cols;
    g.n_tok = n_tok;
    g.y_stride = y_stride;
    g.epi = EPI_PLAIN;
    g.wbound[0] = INFINITY;  // the caller's matrix was never scanned: every round's terms are summed in int64
    const hipStream_t s = static_cast<hipStream_t>(stream);
    e = launch_gemm_quant(q, s);
    if (e == hipSuccess) e = launch_gemm(g, type, s);
    return e == hipSuccess ? 0 : -int(e);
}
