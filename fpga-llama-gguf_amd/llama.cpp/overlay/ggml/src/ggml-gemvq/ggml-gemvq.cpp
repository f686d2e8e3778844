// ggml backend for AMD Instinct MI355X (gfx950) over the gemvq command lists.
//
// This file only translates. The planner (fused command lists per split), the plan cache, the recurrent-state and KV
// buffers and the device runtime (HIP kernels, captured hipGraphs) are in libgemvq_hip.so, behind gemvq_ggml.h.
//
// Each ggml_tensor the backend is shown gets a gqg_tensor mirror holding the fields the planner reads, under the
// same names. A mirror lives as long as the backend: the library keys weight uploads and cached plans by the
// addresses of the mirrors of tensors outside a split (weights, states, host inputs), so a tensor keeps its mirror
// from one graph to the next. ggml reuses compute memory for the next graph's tensors, so a mirror's fields are
// copied again once per call (an epoch stamp) before the planner reads them.
//
// Counterparts in the reference (llama.cpp/overlay/ggml/src/ggml-xrt/ggml-xrt.cpp): the backend interface
// (:2773-2782), the device interface and registration (:2784-3063), the recurrent-state buffer type (:405-622),
// the CPU_REPACK weights (:655-710). What differs: weights are uploaded to HBM once, keyed by tensor; the KV caches
// can live on the device too (ggml_backend_gemvq_kv_buffer_type), so attention is one more command of the list.

#include "ggml-gemvq.h"

#include "ggml-backend-impl.h"
#include "ggml-impl.h"

#include "gemvq_ggml.h"
#include "gemvq_gguf.h"
#include "gemvq_hip.h"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <vector>

#ifndef GGML_SCHED_MARKS_SPLIT_OUTPUTS
#error "ggml-gemvq copies back only the tensors a later split reads: apply patches/0002 (GGML_TENSOR_FLAG_SPLIT_OUTPUT)"
#endif

static_assert(GGML_MAX_SRC <= GQG_MAX_SRC, "gqg_tensor holds every ggml source");
static_assert(GGML_MAX_DIMS == GQG_MAX_DIMS, "gqg_tensor has ggml's dimensions");
static_assert(sizeof(((ggml_tensor *) nullptr)->op_params) == GQG_MAX_OP_PARAMS * sizeof(int32_t),
              "gqg_tensor has ggml's op_params");
static_assert(GGML_MAX_NAME <= 64, "gqg_tensor names hold ggml's");

namespace {

// ---- the process's device and its one backend (gqg_backend_init allows one, as ggml-xrt.cpp:381-387) ----

ggml_backend_device g_device;
ggml_backend_reg g_reg;
ggml_backend_buffer_type g_rs_buft;
ggml_backend_buffer_type g_kv_buft;

struct Mirror {
    struct Entry {
        gqg_tensor t{};
        uint64_t epoch = 0;
        int depth = -1;  // source levels translated in that epoch
    };
    std::unordered_map<const ggml_tensor *, std::unique_ptr<Entry>> map;
    std::unordered_map<const ggml_tensor *, std::vector<uint8_t>> gguf_rows;  // CPU_REPACK weights, unpacked once
    gqg_tensor opaque{};  // stands for sources past a shallow translation: no op, no type the planner takes
    uint64_t epoch = 0;
    std::vector<gqg_tensor *> nodes;

    Mirror() { opaque.type = -1; }
    gqg_tensor * of(const ggml_tensor * t, int depth);
    void clear() {
        map.clear();
        gguf_rows.clear();
        nodes.clear();
    }
};

struct DeviceState {
    std::mutex mutex;
    gqg_backend * active = nullptr;
    Mirror mirror;
} g_state;

// Shallow translations (supports_op, buffer calls) go this many source levels deep: enough for every check
// gqg_supports_op makes (a CONCAT's state rows sit behind a few views and one GET_ROWS).
constexpr int SHALLOW = 8;
constexpr int FULL = INT_MAX;

bool is_repack_buft(ggml_backend_buffer_type_t buft) {
    return buft != nullptr && std::strcmp(ggml_backend_buft_name(buft), "CPU_REPACK") == 0;
}

// ggml's CPU_REPACK keeps Q4_0 rows in block_q4_0x8 on x86 (AVX2 and later, rows a multiple of 8); any other layout
// it uses is unknown here and such weights stay on the CPU.
bool repack_layout_known(const ggml_tensor * w) {
#if defined(__x86_64__)
    return w->type == GGML_TYPE_Q4_0 && w->ne[1] % 8 == 0 && w->ne[2] == 1 && w->ne[3] == 1;
#else
    (void) w;
    return false;
#endif
}

int op_of(const ggml_tensor * t) {
    switch (t->op) {
        case GGML_OP_NONE: return GQG_OP_NONE;
        case GGML_OP_ADD: return GQG_OP_ADD;
        case GGML_OP_MUL: return GQG_OP_MUL;
        case GGML_OP_SCALE: return GQG_OP_SCALE;
        case GGML_OP_RMS_NORM: return GQG_OP_RMS_NORM;
        case GGML_OP_L2_NORM: return GQG_OP_L2_NORM;
        case GGML_OP_MUL_MAT: return GQG_OP_MUL_MAT;
        case GGML_OP_CPY: return GQG_OP_CPY;
        case GGML_OP_CONT: return GQG_OP_CONT;
        case GGML_OP_RESHAPE: return GQG_OP_RESHAPE;
        case GGML_OP_VIEW: return GQG_OP_VIEW;
        case GGML_OP_PERMUTE: return GQG_OP_PERMUTE;
        case GGML_OP_TRANSPOSE: return GQG_OP_TRANSPOSE;
        case GGML_OP_GET_ROWS: return GQG_OP_GET_ROWS;
        case GGML_OP_SET_ROWS: return GQG_OP_SET_ROWS;
        case GGML_OP_CONCAT: return GQG_OP_CONCAT;
        case GGML_OP_ROPE: return GQG_OP_ROPE;
        case GGML_OP_FLASH_ATTN_EXT: return GQG_OP_FLASH_ATTN_EXT;
        case GGML_OP_SSM_CONV: return GQG_OP_SSM_CONV;
        case GGML_OP_GATED_DELTA_NET: return GQG_OP_GATED_DELTA_NET;
        case GGML_OP_UNARY: return GQG_OP_UNARY;
        case GGML_OP_GLU: return GQG_OP_GLU;
        case GGML_OP_SOFT_MAX: return GQG_OP_SOFT_MAX;
        default: return GQG_OP_COUNT;  // unknown to the planner: declined
    }
}

int unary_of(const ggml_tensor * t) {
    switch (ggml_get_unary_op(t)) {
        case GGML_UNARY_OP_SILU: return GQG_UNARY_SILU;
        case GGML_UNARY_OP_SIGMOID: return GQG_UNARY_SIGMOID;
        case GGML_UNARY_OP_SOFTPLUS: return GQG_UNARY_SOFTPLUS;
        default: return 0;
    }
}

int buffer_of(const ggml_tensor * t) {
    const ggml_tensor * owner = t->view_src != nullptr ? t->view_src : t;
    const ggml_backend_buffer_t buf = owner->buffer != nullptr ? owner->buffer : t->buffer;
    if (buf == nullptr) return GQG_BUF_HOST;
    if (buf->buft == &g_rs_buft) return GQG_BUF_RS;
    if (buf->buft == &g_kv_buft) return GQG_BUF_KV;
    if (ggml_backend_buffer_get_usage(buf) == GGML_BACKEND_BUFFER_USAGE_WEIGHTS) return GQG_BUF_WEIGHTS;
    return GQG_BUF_HOST;
}

gqg_tensor * Mirror::of(const ggml_tensor * t, int depth) {
    if (t == nullptr) return nullptr;
    if (depth < 0) return &opaque;
    std::unique_ptr<Entry> & slot = map[t];
    if (!slot) slot = std::make_unique<Entry>();
    Entry & e = *slot;
    if (e.epoch == epoch && e.depth >= depth) return &e.t;
    e.epoch = epoch;
    e.depth = depth;
    gqg_tensor & g = e.t;
    g.type = int32_t(t->type);
    g.op = op_of(t);
    std::memcpy(g.ne, t->ne, sizeof g.ne);
    for (int d = 0; d < GQG_MAX_DIMS; ++d) g.nb[d] = t->nb[d];
    std::memcpy(g.op_params, t->op_params, sizeof g.op_params);
    if (t->op == GGML_OP_UNARY) g.op_params[0] = unary_of(t);
    if (t->op == GGML_OP_GLU) g.op_params[0] = ggml_get_glu_op(t) == GGML_GLU_OP_SWIGLU ? GQG_GLU_SWIGLU : 0;
    g.flags = ((t->flags & GGML_TENSOR_FLAG_INPUT) ? GQG_FLAG_INPUT : 0) |
              ((t->flags & GGML_TENSOR_FLAG_OUTPUT) ? GQG_FLAG_OUTPUT : 0) |
              ((t->flags & GGML_TENSOR_FLAG_SPLIT_OUTPUT) ? GQG_FLAG_SPLIT_OUTPUT : 0);
    g.buffer = buffer_of(t);
    g.data = t->data;
    g.view_offs = t->view_offs;
    std::memset(g.name, 0, sizeof g.name);
    std::strncpy(g.name, t->name, sizeof g.name - 1);
    if (t->view_src == nullptr && t->buffer != nullptr && is_repack_buft(t->buffer->buft)) {
        if (!repack_layout_known(t)) {
            g.type = -1;
        } else {
            std::vector<uint8_t> & rows = gguf_rows[t];
            if (rows.empty()) {
                rows.resize(ggml_row_size(GGML_TYPE_Q4_0, t->ne[0]) * size_t(t->ne[1]));
                if (gemvq_unrepack_q4_0x8(int(t->ne[1]), int(t->ne[0]), t->data, rows.data()) != 0) {
                    GGML_ABORT("gemvq: %s: cannot unpack its block_q4_0x8 rows", t->name);
                }
            }
            g.data = rows.data();  // the strides stay ggml's Q4_0 ones: repacking moves bytes within row groups
        }
    }
    for (int i = 0; i < GQG_MAX_SRC; ++i) g.src[i] = i < GGML_MAX_SRC ? of(t->src[i], depth == FULL ? FULL : depth - 1) : nullptr;
    g.view_src = of(t->view_src, depth == FULL ? FULL : depth - 1);
    return &g;
}

[[noreturn]] void device_failure(const char * what) {
    GGML_ABORT("gemvq: %s: %s", what, gqg_backend_error(g_state.active));
}

// ---- RS and KV buffers (ggml-xrt.cpp:405-622; the KV type is new) ----

gqg_buffer * buffer_ctx(ggml_backend_buffer_t buffer) { return static_cast<gqg_buffer *>(buffer->context); }

void buffer_free(ggml_backend_buffer_t buffer) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    gqg_buffer_free(buffer_ctx(buffer));
}

void * buffer_base(ggml_backend_buffer_t buffer) { return gqg_buffer_base(buffer_ctx(buffer)); }

gqg_tensor * shallow(const ggml_tensor * t) {
    ++g_state.mirror.epoch;
    return g_state.mirror.of(t, SHALLOW);
}

ggml_status buffer_init_tensor(ggml_backend_buffer_t buffer, ggml_tensor * tensor) {
    if (tensor->view_src != nullptr) return GGML_STATUS_SUCCESS;
    std::lock_guard<std::mutex> lock(g_state.mutex);
    const int st = gqg_buffer_init_tensor(buffer_ctx(buffer), shallow(tensor));
    if (st != GQG_STATUS_SUCCESS) GGML_LOG_ERROR("gemvq: %s: %s\n", tensor->name, gqg_backend_error(g_state.active));
    return ggml_status(st);
}

void buffer_set_tensor(ggml_backend_buffer_t buffer, ggml_tensor * tensor, const void * data, size_t offset, size_t size) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    if (gqg_buffer_set(buffer_ctx(buffer), shallow(tensor), data, offset, size) != GQG_STATUS_SUCCESS) {
        device_failure(tensor->name);
    }
}

void buffer_get_tensor(ggml_backend_buffer_t buffer, const ggml_tensor * tensor, void * data, size_t offset, size_t size) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    if (gqg_buffer_get(buffer_ctx(buffer), shallow(tensor), data, offset, size) != GQG_STATUS_SUCCESS) {
        device_failure(tensor->name);
    }
}

void buffer_memset_tensor(ggml_backend_buffer_t buffer, ggml_tensor * tensor, uint8_t value, size_t offset, size_t size) {
    const std::vector<uint8_t> fill(size, value);
    buffer_set_tensor(buffer, tensor, fill.data(), offset, size);
}

void buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    if (gqg_buffer_clear(buffer_ctx(buffer), value) != GQG_STATUS_SUCCESS) device_failure("clear");
}

const ggml_backend_buffer_i k_buffer_iface = [] {
    ggml_backend_buffer_i i{};
    i.free_buffer = buffer_free;
    i.get_base = buffer_base;
    i.init_tensor = buffer_init_tensor;
    i.memset_tensor = buffer_memset_tensor;
    i.set_tensor = buffer_set_tensor;
    i.get_tensor = buffer_get_tensor;
    i.clear = buffer_clear;
    return i;
}();

const char * rs_buft_name(ggml_backend_buffer_type_t) { return "GEMVQ_RS"; }
const char * kv_buft_name(ggml_backend_buffer_type_t) { return "GEMVQ_KV"; }

ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    if (g_state.active == nullptr) return nullptr;
    gqg_buffer * b = buft == &g_rs_buft ? gqg_rs_buffer_alloc(g_state.active, size)
                                        : gqg_kv_buffer_alloc(g_state.active, size);
    if (b == nullptr) return nullptr;
    ggml_backend_buffer_t buffer = ggml_backend_buffer_init(buft, k_buffer_iface, b, size);
    if (buffer == nullptr) gqg_buffer_free(b);
    return buffer;
}

// State rows are read and written whole (128 floats); tensors start on a row.
size_t buft_alignment(ggml_backend_buffer_type_t) { return 512; }
bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

ggml_backend_buffer_type_i buft_iface(const char * (*name)(ggml_backend_buffer_type_t)) {
    ggml_backend_buffer_type_i i{};
    i.get_name = name;
    i.alloc_buffer = buft_alloc;
    i.get_alignment = buft_alignment;
    i.is_host = buft_is_host;
    return i;
}

// ---- backend (ggml-xrt.cpp:2747-2782) ----

ggml_guid * backend_guid() {
    static ggml_guid guid = {0x67, 0x65, 0x6d, 0x76, 0x71, 0x2d, 0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x67, 0x66, 0x78};
    return &guid;
}

const char * backend_name(ggml_backend_t) { return "GEMVQ"; }

void backend_free(ggml_backend_t backend) {
    {
        std::lock_guard<std::mutex> lock(g_state.mutex);
        auto * b = static_cast<gqg_backend *>(backend->context);
        if (g_state.active == b) {
            g_state.active = nullptr;
            g_state.mirror.clear();
        }
        gqg_backend_free(b);
    }
    delete backend;
}

// One split: its nodes in graph order, mirrored (sources come before their readers, so the translation of node i
// finds its operands already refreshed), then planned, run and read back by the library. A failure latches the
// backend: later calls fail too (ggml-xrt.cpp:2761-2770).
ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph * cgraph) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    auto * b = static_cast<gqg_backend *>(backend->context);
    Mirror & m = g_state.mirror;
    ++m.epoch;
    m.nodes.clear();
    for (int i = 0; i < cgraph->n_nodes; ++i) m.nodes.push_back(m.of(cgraph->nodes[i], FULL));
    gqg_cgraph g{int(m.nodes.size()), m.nodes.data()};
    const int st = gqg_graph_compute(b, &g);
    if (st != GQG_STATUS_SUCCESS) GGML_LOG_ERROR("gemvq: graph_compute: %s\n", gqg_backend_error(b));
    return ggml_status(st);
}

const ggml_backend_i k_backend_iface = [] {
    ggml_backend_i i{};
    i.get_name = backend_name;
    i.free = backend_free;
    i.graph_compute = backend_graph_compute;
    return i;
}();

// ---- device (ggml-xrt.cpp:2784-3063) ----

size_t env_size(const char * name, size_t fallback) {
    const char * v = std::getenv(name);
    return v != nullptr && *v != '\0' ? size_t(std::strtoull(v, nullptr, 0)) : fallback;
}

const char * dev_name(ggml_backend_dev_t) { return "GEMVQ"; }
const char * dev_description(ggml_backend_dev_t) { return gqg_backend_get_reg()->get_description(); }

void dev_memory(ggml_backend_dev_t, size_t * free_bytes, size_t * total_bytes) {
    size_t f = 0, t = 0;
    gemvq_device_memory(int(env_size("GGML_GEMVQ_DEVICE", 0)), &f, &t);
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
}

ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_props(ggml_backend_dev_t dev, ggml_backend_dev_props * props) {
    props->name = dev_name(dev);
    props->description = dev_description(dev);
    dev_memory(dev, &props->memory_free, &props->memory_total);
    props->type = dev_type(dev);
    props->caps.async = false;
    props->caps.host_buffer = false;
    props->caps.buffer_from_host_ptr = false;
    props->caps.events = false;
}

// Sizes of the device context, from the environment:
//   GGML_GEMVQ_DEVICE        HIP device (0)
//   GGML_GEMVQ_WEIGHT_BYTES  weight arena (half the device's free HBM, at most 64 GiB)
//   GGML_GEMVQ_ACT_FLOATS    activation buffer: a transient half for split inputs and outputs, a resident half for
//                            constants, rope tables and conv windows (2^26 floats)
//   GGML_GEMVQ_STATE_ROWS    recurrent-state rows of 128 floats (2^20 rows, 512 MiB)
ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *) {
    gqg_params p{};
    p.device = int(env_size("GGML_GEMVQ_DEVICE", 0));
    size_t free_b = 0, total_b = 0;
    gemvq_device_memory(p.device, &free_b, &total_b);
    p.weight_bytes = env_size("GGML_GEMVQ_WEIGHT_BYTES", std::min<size_t>(free_b / 2, size_t(64) << 30) >> 20 << 20);
    p.act_floats = env_size("GGML_GEMVQ_ACT_FLOATS", size_t(1) << 26);
    p.state_rows = env_size("GGML_GEMVQ_STATE_ROWS", size_t(1) << 20);
    std::lock_guard<std::mutex> lock(g_state.mutex);
    if (g_state.active != nullptr) {
        GGML_LOG_ERROR("gemvq: one backend per process; free the other first\n");
        return nullptr;
    }
    gqg_backend * b = gqg_backend_init(&p);
    if (b == nullptr) {
        GGML_LOG_ERROR("gemvq: cannot create a context on HIP device %d (weight arena %zu MiB)\n", p.device,
                       p.weight_bytes >> 20);
        return nullptr;
    }
    g_state.active = b;
    GGML_LOG_INFO("gemvq: %s, device %d, weight arena %zu MiB\n", dev_description(dev), p.device, p.weight_bytes >> 20);
    auto * backend = new ggml_backend{};
    backend->guid = backend_guid();
    backend->iface = k_backend_iface;
    backend->device = dev;
    backend->context = b;
    return backend;
}

// Weights stay in llama's host buffers; the backend uploads each quantized matrix and F32 constant once.
ggml_backend_buffer_type_t dev_buffer_type(ggml_backend_dev_t) { return ggml_backend_cpu_buffer_type(); }

bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor * op) {
    std::lock_guard<std::mutex> lock(g_state.mutex);
    if (g_state.active == nullptr) return false;
    return gqg_supports_op(g_state.active, shallow(op)) != 0;
}

bool dev_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t buft) {
    return ggml_backend_buft_is_host(buft) || buft == &g_rs_buft || buft == &g_kv_buft || is_repack_buft(buft);
}

const char * reg_name(ggml_backend_reg_t) { return "GEMVQ"; }
size_t reg_device_count(ggml_backend_reg_t) { return 1; }
ggml_backend_dev_t reg_device(ggml_backend_reg_t, size_t i) { return i == 0 ? &g_device : nullptr; }

void * reg_proc_address(ggml_backend_reg_t, const char * name) {
    if (std::strcmp(name, "ggml_backend_gemvq_rs_buffer_type") == 0) return (void *) ggml_backend_gemvq_rs_buffer_type;
    if (std::strcmp(name, "ggml_backend_gemvq_kv_buffer_type") == 0) return (void *) ggml_backend_gemvq_kv_buffer_type;
    return nullptr;
}

ggml_backend_buffer_type_t device_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type * buft) {
    if (dev != &g_device) return nullptr;
    std::lock_guard<std::mutex> lock(g_state.mutex);
    return g_state.active != nullptr ? buft : nullptr;
}

}  // namespace

extern "C" ggml_backend_reg_t ggml_backend_gemvq_reg(void) {
    static const bool once = [] {
        g_reg.api_version = GGML_BACKEND_API_VERSION;
        g_reg.iface.get_name = reg_name;
        g_reg.iface.get_device_count = reg_device_count;
        g_reg.iface.get_device = reg_device;
        g_reg.iface.get_proc_address = reg_proc_address;
        g_reg.context = nullptr;

        g_device.iface.get_name = dev_name;
        g_device.iface.get_description = dev_description;
        g_device.iface.get_memory = dev_memory;
        g_device.iface.get_type = dev_type;
        g_device.iface.get_props = dev_props;
        g_device.iface.init_backend = dev_init_backend;
        g_device.iface.get_buffer_type = dev_buffer_type;
        g_device.iface.get_host_buffer_type = dev_buffer_type;
        g_device.iface.supports_op = dev_supports_op;
        g_device.iface.offload_op = dev_supports_op;
        g_device.iface.supports_buft = dev_supports_buft;
        g_device.reg = &g_reg;
        g_device.context = &g_state;

        g_rs_buft.iface = buft_iface(rs_buft_name);
        g_rs_buft.device = &g_device;
        g_rs_buft.context = nullptr;
        g_kv_buft.iface = buft_iface(kv_buft_name);
        g_kv_buft.device = &g_device;
        g_kv_buft.context = nullptr;
        return true;
    }();
    (void) once;
    return &g_reg;
}

extern "C" ggml_backend_buffer_type_t ggml_backend_gemvq_rs_buffer_type(ggml_backend_dev_t dev) {
    return device_buft(dev, &g_rs_buft);
}

extern "C" ggml_backend_buffer_type_t ggml_backend_gemvq_kv_buffer_type(ggml_backend_dev_t dev) {
    return device_buft(dev, &g_kv_buft);
}

GGML_BACKEND_DL_IMPL(ggml_backend_gemvq_reg)
