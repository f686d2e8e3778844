// Host side of the MI355X decode backend: device buffers, the load-time weight repack, the command processor that
// validates a command list and fuses it into kernel launches (the role of gemvqc16's run_list,
// fpga/src/gemvqc16.cpp:552-958, moved to the host because a GPU launch sequence can be captured once), and the
// hipGraph capture and replay of per-token lists. C ABI in include/gemvq_hip.h.
#include "gemvq_hip.h"
#include "gq_kernels.h"
#include "gq_ref.h"
#include "gq_refmath.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <variant>
#include <vector>

using namespace gq;

namespace gq {
thread_local hipEvent_t g_prof_start = nullptr, g_prof_stop = nullptr;
}

namespace {

struct Weight {
    int type, rows, cols;
    size_t bytes;
    float wbound;  // Q4_0 / Q4_1 / Q8_0: the largest block term magnitude over |d_x| * 2^40 (see weight_bound)
};

// IEEE binary16 to float (subnormals, infinities and NaN included).
float half_to_float_host(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    const float v = e == 0 ? std::ldexp(float(m), -24) : e == 31 ? (m ? NAN : INFINITY) : std::ldexp(float(1024 + m), e - 25);
    return (h & 0x8000) ? -v : v;
}

// The largest |block term| / (|d_x| 2^40) of a Q4_0 / Q4_1 / Q8_0 matrix: over its blocks, |d_w| times the largest
// |sum of products| with Q8_0 quants (|q_x| <= 127: 32 * 8 * 127 for Q4_0, 32 * 15 * 127 for Q4_1, 32 * 128 * 127
// for Q8_0), plus for Q4_1 |m_w| times the largest |s_x| / d_x (32 * 127); rounded up to FP32. 0 for other types.
float weight_bound(int type, int rows, int cols, const uint8_t * gguf) {
    if (type != T_Q4_0 && type != T_Q4_1 && type != T_Q8_0) return 0.0f;
    const size_t nb = size_t(rows) * size_t(cols / 32), bb = type == T_Q4_0 ? 18 : type == T_Q4_1 ? 20 : 34;
    const double smax = type == T_Q4_0 ? 32.0 * 8 * 127 : type == T_Q4_1 ? 32.0 * 15 * 127 : 32.0 * 128 * 127;
    const auto h = [](const uint8_t * p) {
        uint16_t u;
        std::memcpy(&u, p, 2);
        return std::fabs(double(half_to_float_host(u)));
    };
    double best = 0.0;
    for (size_t i = 0; i < nb; ++i) {
        const uint8_t * blk = gguf + i * bb;
        double t = h(blk) * smax;
        if (type == T_Q4_1) t += h(blk + 2) * (32.0 * 127);
        if (!(t <= best)) best = t;  // a NaN scale makes the bound NaN: every launch on it sums in int64
    }
    return std::nextafter(float(best), INFINITY);
}

struct KvBuf {
    uint16_t * k = nullptr;
    uint16_t * v = nullptr;
    float * part = nullptr;       // attention partials and counters: one set per token of a GEMM_MAX_TOK batch
    unsigned * counter = nullptr;
    float * qr = nullptr;         // a batch's rotated queries [GEMM_MAX_TOK][ATTN_MAXG * n_head_kv][head_dim]
    int n_ctx = 0, n_head_kv = 0, head_dim = 0;
};

// ref: the launch runs in the reference arithmetic (gq_ref.h); tok: the one token of a CONV, GDN or ATTN command
// that such a launch runs (the command's tokens run as launches in order)
struct LGemv { GemvArgs a; int type; int ref = 0; };
struct LNorm { NormArgs a; int ref = 0; };
struct LEw { EwArgs a; int ref = 0; };
struct LConv { ConvArgs a; int ref = 0, tok = 0; };
struct LRope { RopeArgs a; };
struct LGdn { GdnArgs a; int ref = 0, tok = 0; };
struct LGdnOut { GdnOutArgs a; int type; };
struct LGated { GatedNormArgs a; };
struct LAttn { AttnArgs a; int ref = 0, tok = 0; };
struct LRows { GetRowsArgs a; };
struct LArgmax { const float * x; int n; unsigned long long * key; int rows, stride; };
struct LNext { NextTokenArgs a; };
struct LGemmQ { GemmQuantArgs a; };
struct LGemm { GemmArgs a; int type; };
struct LTok { TokArgs a; int type; uint32_t x_off, x_len; };  // x_off, x_len: the token rows read (activation floats)
using Launch = std::variant<LGemv, LNorm, LEw, LConv, LRope, LGdn, LGated, LAttn, LRows, LArgmax, LNext, LGemmQ, LGemm,
                            LGdnOut, LTok>;

}  // namespace

struct gemvq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    float * act = nullptr;
    size_t act_floats = 0;
    uint8_t * warena = nullptr;
    size_t wbytes = 0, wused = 0;
    float * state = nullptr;
    size_t state_rows = 0;
    std::map<uint64_t, Weight> weights;
    std::vector<KvBuf> kvs;
    std::vector<hipGraphExec_t> graphs;
    std::vector<hipGraph_t> graph_defs;
    int32_t * dbg = nullptr;      // device buffer of the armed block-sum dump
    size_t dbg_n = 0;
    int32_t * dbg_dst = nullptr;  // host destination; non-NULL while armed
    bool dbg_used = false;        // the list being compiled writes the dump
    float * gdn_raw = nullptr;    // raw DeltaNet output when its gated norm is folded into the next GEMV
    float * dsnap = nullptr;      // a deferred norm's row, computed before a command overwrote its source
    float * xsnap = nullptr;      // a GEMV group's activation, copied before a member overwrites it
    unsigned long long * gdn_xch = nullptr;  // the fused DeltaNet step + ssm_out's exchange area (GDN_XCH_WORDS, zero)
    uint32_t * gdn_fault = nullptr;  // host word the fused launch sets when a wait for its heads ran out of polls
    unsigned xch_polls = 0;          // that wait's bound in polls (set at creation)
    int8_t * gemm_q = nullptr;    // a batched GEMV's quantized activation rows (GEMM_MAX_TOK x GEMV_MAXK)
    float * gemm_d = nullptr;     // and their block scales
    float * gemm_s = nullptr;     // and their Q8_1 block sums (for Q4_1 weights)
    float * ref_x = nullptr;      // the reference arithmetic's copy of a GEMM's token rows and norm weight
    int arith = GEMVQ_ARITH_CANONICAL;  // the arithmetic lists are compiled in (gemvq_set_arith)
    int last_launches = 0;
    std::string err;
    // Failure handling (ggml-xrt.cpp:69-78, 1258-1264, 2761-2770): every wait for the device is bounded by wait_ms;
    // a launch or copy that failed or did not finish in time leaves the device in an unknown state, so the context
    // refuses further device work (usable = false) until it is destroyed.
    unsigned wait_ms = 180000;
    bool usable = true;
};

static std::string g_create_error;

namespace {

int fail(gemvq_ctx * c, hipError_t e, const char * what) {
    if (c) {
        c->err = std::string(what) + ": " + hipGetErrorString(e);
        c->usable = false;
    }
    return -int(e);
}

// The status of an entry point on a context that an earlier device failure made unusable.
int unusable(gemvq_ctx * c) {
    c->err = "context unusable after a failed or timed-out device operation (" + c->err + ")";
    return GEMVQ_EUNUSABLE;
}

// Waits for the context's stream for at most c->wait_ms (polling; a yield between polls). 0, a negated HIP error
// (the stream reported a failure) or GEMVQ_ETIMEDOUT; either failure makes the context unusable.
int wait_stream(gemvq_ctx * c, const char * what) {
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::milliseconds(c->wait_ms);
    for (;;) {
        const hipError_t e = hipStreamQuery(c->stream);
        if (e == hipSuccess) {
            if (c->gdn_fault && __atomic_load_n(c->gdn_fault, __ATOMIC_ACQUIRE)) {
                c->err = std::string(what) + ": a fused DeltaNet step + ssm_out launch's wait for its heads ran out "
                         "of polls (its output was not written)";
                c->usable = false;
                return GEMVQ_ETIMEDOUT;
            }
            return 0;
        }
        if (e != hipErrorNotReady) return fail(c, e, what);
        if (std::chrono::steady_clock::now() > deadline) {
            c->err = std::string(what) + ": the device did not finish within " + std::to_string(c->wait_ms) + " ms";
            c->usable = false;
            return GEMVQ_ETIMEDOUT;
        }
        std::this_thread::yield();
    }
}

// Host copies of pageable memory run synchronously behind the work already queued on the stream, outside any
// bound: every such copy first waits (bounded) for that work, so the copy itself has nothing to wait behind.
int drain(gemvq_ctx * c, const char * what) { return wait_stream(c, what); }

int einval(gemvq_ctx * c, const std::string & what) {
    if (c) c->err = what;
    return GEMVQ_EINVAL;
}

float bits_f(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// ---- layout-only repack (gq_kernels.h: the GGUF block fields split into field-major regions) ----
void repack_rows(int type, int rows, int cols, const uint8_t * src, uint8_t * dst, bool inverse) {
    const size_t R = size_t(rows);
    if (type == T_Q4_1) {  // qs, then d | m << 16 per block
        const size_t nb = size_t(cols / 32);
        uint8_t * qa = dst, * dm = dst + R * nb * 16;
        for (size_t i = 0; i < R * nb; ++i) {
            uint8_t * blk = const_cast<uint8_t *>(src) + i * 20;
            if (!inverse) {
                std::memcpy(dm + 4 * i, blk, 4);
                std::memcpy(qa + 16 * i, blk + 4, 16);
            } else {
                std::memcpy(blk, dm + 4 * i, 4);
                std::memcpy(blk + 4, qa + 16 * i, 16);
            }
        }
    } else if (type == T_Q4_0 || type == T_Q8_0) {
        const size_t nb = size_t(cols / 32), bb = type == T_Q4_0 ? 18 : 34;
        uint8_t * qa = dst;
        uint8_t * qb = dst + R * nb * 16;
        uint8_t * dd = type == T_Q4_0 ? qb : dst + R * nb * 32;
        for (size_t i = 0; i < R * nb; ++i) {
            uint8_t * blk = const_cast<uint8_t *>(src) + i * bb;
            if (!inverse) {
                std::memcpy(dd + 2 * i, blk, 2);
                std::memcpy(qa + 16 * i, blk + 2, 16);
                if (type == T_Q8_0) std::memcpy(qb + 16 * i, blk + 18, 16);
            } else {
                std::memcpy(blk, dd + 2 * i, 2);
                std::memcpy(blk + 2, qa + 16 * i, 16);
                if (type == T_Q8_0) std::memcpy(blk + 18, qb + 16 * i, 16);
            }
        }
    } else if (type == T_Q5_K) {
        const size_t ns = size_t(cols / 256);
        uint8_t * qs = dst, * qh = dst + R * ns * 128, * meta = dst + R * ns * 160;
        for (size_t i = 0; i < R * ns; ++i) {
            uint8_t * blk = const_cast<uint8_t *>(src) + i * 176;
            if (!inverse) {
                std::memcpy(meta + 16 * i, blk, 16);
                std::memcpy(qh + 32 * i, blk + 16, 32);
                std::memcpy(qs + 128 * i, blk + 48, 128);
            } else {
                std::memcpy(blk, meta + 16 * i, 16);
                std::memcpy(blk + 16, qh + 32 * i, 32);
                std::memcpy(blk + 48, qs + 128 * i, 128);
            }
        }
    } else if (type == T_Q6_K) {
        // ql and d as they are. The high bits and scales are regrouped per 64-weight unit j = 2n + p (the quants
        // 32p + l of half n, group A, and 64 + 32p + l, group B, l < 32), so a unit reads one contiguous piece of
        // each: its 16 high-bit bytes, where byte b of word k holds, from bit 0, the 2-bit fields of A at l = 4k + b
        // and 4k + 16 + b, then of B at the same l (GGUF bits 2p and 2p + 4 of qh[32n + l]); and its 4 scale bytes
        // sc[8n + 2p], sc[8n + 2p + 1], sc[8n + 4 + 2p], sc[8n + 5 + 2p]. Every bit keeps its value.
        const size_t ns = size_t(cols / 256);
        uint8_t * ql = dst, * qh = dst + R * ns * 128, * sc = dst + R * ns * 192, * dd = dst + R * ns * 208;
        for (size_t i = 0; i < R * ns; ++i) {
            uint8_t * blk = const_cast<uint8_t *>(src) + i * 210;
            uint8_t * h = qh + 64 * i, * s = sc + 16 * i;
            if (!inverse) {
                std::memcpy(ql + 128 * i, blk, 128);
                std::memcpy(dd + 2 * i, blk + 208, 2);
                std::memset(h, 0, 64);
                for (int j = 0; j < 4; ++j) {
                    const int n = j >> 1, p = j & 1;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t v = blk[128 + 32 * n + l];
                        const int a2 = (v >> (2 * p)) & 3, b2 = (v >> (2 * p + 4)) & 3, k = (l >> 2) & 3, up = 2 * (l >> 4);
                        h[16 * j + 4 * k + (l & 3)] |= uint8_t((a2 << up) | (b2 << (4 + up)));
                    }
                    for (int q = 0; q < 4; ++q) s[4 * j + q] = blk[192 + 8 * n + 2 * p + (q & 1) + 4 * (q >> 1)];
                }
            } else {
                std::memcpy(blk, ql + 128 * i, 128);
                std::memcpy(blk + 208, dd + 2 * i, 2);
                std::memset(blk + 128, 0, 64);
                for (int j = 0; j < 4; ++j) {
                    const int n = j >> 1, p = j & 1;
                    for (int l = 0; l < 32; ++l) {
                        const int k = (l >> 2) & 3, up = 2 * (l >> 4);
                        const uint8_t v = h[16 * j + 4 * k + (l & 3)];
                        const int a2 = (v >> up) & 3, b2 = (v >> (4 + up)) & 3;
                        blk[128 + 32 * n + l] |= uint8_t((a2 << (2 * p)) | (b2 << (2 * p + 4)));
                    }
                    for (int q = 0; q < 4; ++q) blk[192 + 8 * n + 2 * p + (q & 1) + 4 * (q >> 1)] = s[4 * j + q];
                }
            }
        }
    }
}

bool type_ok(int t) { return t == T_Q4_0 || t == T_Q4_1 || t == T_Q8_0 || t == T_Q5_K || t == T_Q6_K; }

bool shape_ok(int t, int rows, int cols) {
    if (rows <= 0 || cols <= 0 || cols > int(GEMVQ_MAX_COLS)) return false;
    return (t == T_Q5_K || t == T_Q6_K) ? cols % 256 == 0 : cols % 32 == 0;
}

// ---- command processor ----
struct Compiler {
    gemvq_ctx * c;
    std::vector<Launch> out;
    std::vector<std::pair<int, int>> spans;  // per launch: first command, number of commands
    int bad = 0;  // 1-based index of the first invalid command
    std::string why;

    bool range(uint32_t off, uint64_t n) const { return off % 16 == 0 && uint64_t(off) + n <= c->act_floats; }
    // the list is compiled in the reference arithmetic (gq_ref.h): no fused forms whose arithmetic differs from it
    int ref() const { return c->arith == GEMVQ_ARITH_REFERENCE ? 1 : 0; }
    float * A(uint32_t off) const { return c->act + off; }

    bool reject(unsigned i, const std::string & w) {
        bad = int(i) + 1;
        why = "command " + std::to_string(i + 1) + ": " + w;
        return false;
    }

    const Weight * weight(uint64_t off, int type, int rows, int cols) const {
        auto it = c->weights.find(off);
        if (it == c->weights.end()) return nullptr;
        const Weight & w = it->second;
        return (w.type == type && w.rows == rows && w.cols == cols) ? &w : nullptr;
    }

    // Act ranges (in floats) and their overlap.
    struct Rng { uint64_t lo, hi; };
    static bool meet(Rng a, Rng b) { return a.lo < b.hi && b.lo < a.hi; }
    static bool meet_any(const std::vector<Rng> & a, const std::vector<Rng> & b) {
        for (const Rng & x : a)
            for (const Rng & y : b)
                if (meet(x, y)) return true;
        return false;
    }

    // What the GEMV at command i writes while its pass runs (its output; a CONV epilog's new state; an ARGMAX key)
    // and what its epilog reads meanwhile (the residual; the conv state and kernel). Validation happens elsewhere.
    void gemv_io(const uint32_t * cmds, unsigned n, unsigned i, std::vector<Rng> & wr, std::vector<Rng> & rd) const {
        const uint32_t * k = cmds + size_t(i) * GEMVQ_CMD_WORDS;
        const uint64_t rows = k[2];
        const uint32_t flags = k[1] & ~0xffu;
        const uint32_t * e = i + 1 < n ? k + GEMVQ_CMD_WORDS : nullptr;
        if ((flags & GEMVQ_GEMV_SWIGLU) && e) {
            wr.push_back({e[7], e[7] + rows});
        } else if ((flags & GEMVQ_GEMV_ADD) && e) {
            const uint64_t r = e[2] == k[7] ? e[3] : e[2];
            wr.push_back({e[4], e[4] + rows});
            rd.push_back({r, r + rows});
        } else if ((flags & GEMVQ_GEMV_CONV) && e) {
            wr.push_back({e[4], e[4] + rows});
            wr.push_back({e[6], e[6] + 3 * rows});
            rd.push_back({e[5], e[5] + 3 * rows});
            rd.push_back({e[3], e[3] + 4 * rows});
        } else if ((flags & GEMVQ_GEMV_ARGMAX) && e) {
            wr.push_back({k[7], k[7] + rows});
            wr.push_back({e[3], e[3] + 2});
        } else {
            wr.push_back({k[7], k[7] + rows});
        }
    }

    // Act ranges the commands i .. i + used - 1 write (a superset is fine: it only costs a snapshot).
    void cmd_writes(const uint32_t * cmds, unsigned n, unsigned i, unsigned used, std::vector<Rng> & wr) const {
        for (unsigned j = i; j < i + used && j < n;) {
            const uint32_t * k = cmds + size_t(j) * GEMVQ_CMD_WORDS;
            const uint32_t * k2 = j + 1 < n ? k + GEMVQ_CMD_WORDS : nullptr;
            unsigned step = 1;
            switch (k[0]) {
            case GEMVQ_OP_GEMV: wr.push_back({k[7], k[7] + uint64_t(k[2])}); break;
            case GEMVQ_OP_RMSNORM:
                if (!(k[7] & GEMVQ_NORM_DEFER)) wr.push_back({k[4], k[4] + uint64_t(k[1]) * (k[6] ? k[6] : 1)});
                break;
            case GEMVQ_OP_ADD: case GEMVQ_OP_MUL: case GEMVQ_OP_SILU_MUL: case GEMVQ_OP_UNARY:
                wr.push_back({k[4], k[4] + uint64_t(k[1])});
                break;
            case GEMVQ_OP_FILL: wr.push_back({k[2], k[2] + uint64_t(k[1])}); break;
            case GEMVQ_OP_CONV: {
                const uint64_t nt = (k[7] >> 16) ? (k[7] >> 16) : 1;
                wr.push_back({k[4], k[4] + uint64_t(k[1]) * nt});
                wr.push_back({k[6], k[6] + 3ull * k[1] * ((k[7] & GEMVQ_CONV_SEQS) ? nt : 1)});
                break;
            }
            case GEMVQ_OP_ROPE: wr.push_back({k[4], k[4] + uint64_t(k[5]) * k[6]}); break;
            case GEMVQ_OP_GDN: {
                const bool gates = k2 && (k2[3] & GEMVQ_GDN_GATES);
                const uint32_t * k3 = gates && j + 2 < n ? k2 + GEMVQ_CMD_WORDS : nullptr;
                const uint64_t nt = k3 && k3[2] ? k3[2] : 1;
                wr.push_back({k[7], k[7] + uint64_t(k[1] & 0xffffu) * 128 * nt});
                step = gates ? 3 : 2;
                break;
            }
            case GEMVQ_OP_ATTN: {
                const uint64_t nt = (k[7] >> 16) & 0xffu ? (k[7] >> 16) & 0xffu : 1;
                wr.push_back({k[4], k[4] + uint64_t(k[1] & 0xffffu) * (k[5] & 0xffffu) * nt});
                step = 2;
                break;
            }
            case GEMVQ_OP_GET_ROWS: {
                const uint64_t nt = (k[1] >> 16) & 0xffu ? (k[1] >> 16) & 0xffu : 1;
                wr.push_back({k[7], k[7] + uint64_t(k[3]) * nt});
                break;
            }
            case GEMVQ_OP_ARGMAX: wr.push_back({k[3], k[3] + 16ull * ((k[4] ? k[4] : 1) - 1) + 2}); break;
            case GEMVQ_OP_NEXT_TOKEN: {
                const uint64_t ns = (k[7] & 0xffu) > 1 ? (k[7] & 0xffu) : 1, sl = 16 * (ns - 1);
                wr.push_back({k[1], k[1] + sl + 2});
                wr.push_back({k[2], k[2] + sl + 1});
                wr.push_back({k[3], k[3] + sl + 1});
                wr.push_back({k[6], ns > 1 ? k[6] + uint64_t(k[7] >> 8) * ns : c->act_floats});
                break;
            }
            case GEMVQ_OP_GEMM:
                if (k2) wr.push_back({k[7], k[7] + uint64_t(k2[2]) * (k2[0] ? k2[0] - 1 : 0) + k[2]});
                step = 2;
                break;
            default: break;
            }
            j += step;
        }
    }

    // A GDN's gated output norm pending for the GEMV group that reads its output next: the gated vector goes to y
    // (written by workgroup 0 of that group), computed from the raw step output (a private buffer), z and w.
    struct Gated { bool on = false; uint32_t y, cols; const float * z; const float * w; float eps; int z_silu; } gated;

    std::vector<Rng> gated_ranges() const {
        const uint64_t z = uint64_t(gated.z - c->act), w = uint64_t(gated.w - c->act);
        return {{gated.y, gated.y + uint64_t(gated.cols)}, {z, z + gated.cols}, {w, w + 128}};
    }

    // The DeltaNet layer shape the fused step + ssm_out serves (the reference's GDN_WITH_OUT, gemvqc16.cpp:872-903):
    // the one-token GDN with the gated norm whose next command `next` is a Q4_0 / Q8_0 GEMV on its whole output
    // (hv a multiple of 4 up to 32, rows a multiple of 16 and at least 16 hv) with the ADD epilog, its ADD writing
    // y2 = ssm_out + res. Every workgroup of the fused launch reads its rows' residuals at its start and writes y2
    // after all heads are stepped, so y2 is res itself or apart from it, and neither meets anything the step reads
    // or writes (q, k, v, the gates, z, the norm weight, y). y2 and res are returned.
    bool fuse_out(const uint32_t * cmds, unsigned n, unsigned next, const std::vector<Rng> & step_io, uint32_t gy,
                  uint32_t hv, uint32_t & y2, uint32_t & res) const {
        if (next + 1 >= n) return false;
        const uint32_t * g = cmds + size_t(next) * GEMVQ_CMD_WORDS, * e = g + GEMVQ_CMD_WORDS;
        const int t = int(g[1] & 0xffu);
        const uint32_t rows = g[2];
        const uint64_t woff = uint64_t(g[4]) | (uint64_t(g[5]) << 32);
        if (g[0] != GEMVQ_OP_GEMV || (g[1] & ~0xffu) != GEMVQ_GEMV_ADD || (t != T_Q4_0 && t != T_Q8_0) || g[6] != gy ||
            g[3] != hv * 128 || !gdn_out_fits(int(hv), int(rows)) || !weight(woff, t, int(rows), int(hv * 128)))
            return false;
        if (e[0] != GEMVQ_OP_ADD || e[1] != rows || (e[2] != g[7] && e[3] != g[7])) return false;
        res = e[2] == g[7] ? e[3] : e[2];
        y2 = e[4];
        if (!range(res, rows) || !range(y2, rows) || (y2 != res && meet({y2, uint64_t(y2) + rows}, {res, uint64_t(res) + rows})))
            return false;
        return !meet_any({{y2, uint64_t(y2) + rows}, {res, uint64_t(res) + rows}}, step_io);
    }

    // The command at `next` is a Q4_0 / Q8_0 GEMV that reads exactly the GDN output y (cols = heads * 128 <= 8192)
    // and whose pass neither writes nor reads what the gated prologue reads and writes (y, z, the norm weight).
    bool fold_gated(const uint32_t * cmds, unsigned n, unsigned next, uint32_t y, uint32_t cols, uint32_t z_off,
                    uint32_t w_off) const {
        if (next >= n || cols > 8192) return false;
        const uint32_t * g = cmds + size_t(next) * GEMVQ_CMD_WORDS;
        const int t = int(g[1] & 0xffu);
        if (!(g[0] == GEMVQ_OP_GEMV && g[6] == y && g[3] == cols && (t == T_Q4_0 || t == T_Q8_0) &&
              !(g[1] & GEMVQ_GEMV_SWIGLU)))  // the gated prologue has no SwiGLU-pair variant
            return false;
        std::vector<Rng> wr, rd;
        gemv_io(cmds, n, next, wr, rd);
        const std::vector<Rng> gr = {{y, uint64_t(y) + cols}, {z_off, uint64_t(z_off) + cols}, {w_off, uint64_t(w_off) + 128}};
        return !meet_any(wr, gr) && !meet_any(rd, gr);
    }

    // The deferred RMSNORM pending for the GEMVs on its output (gemvqc16.h:46-51: its normalized row is fixed when
    // the command runs; y is never written). `dirty`: the first launch of a later command that overwrote its row or
    // weight (-1: none). A GEMV on the norm after that reads the row from the context's snapshot buffer (`snap`),
    // into which the row is computed right before that launch.
    struct Deferred { bool on = false, snap = false; long dirty = -1; uint32_t n, x, w, y; float eps; uint32_t flags; } defer;

    std::vector<Rng> defer_ranges() const {
        std::vector<Rng> r = {{defer.x, uint64_t(defer.x) + defer.n}};
        if (!(defer.flags & GEMVQ_NORM_NO_WEIGHT)) r.push_back({defer.w, uint64_t(defer.w) + defer.n});
        return r;
    }

    // The deferred row computed into the snapshot buffer, as launch `at` (before the launches that overwrite it).
    void snapshot_defer(size_t at, int cmd) {
        NormArgs a{A(defer.x), (defer.flags & GEMVQ_NORM_NO_WEIGHT) ? nullptr : A(defer.w), c->dsnap, int(defer.n), 1,
                   int(defer.n), defer.eps, int(defer.flags & 3)};
        out.insert(out.begin() + long(at), LNorm{a, ref()});
        spans.insert(spans.begin() + long(at), {cmd, 1});
        defer.snap = true;
    }

    // The activation rows a batched GEMV quantized last, while nothing since could have changed them: the next GEMM
    // on the same rows (same norm) reuses the scratch instead of quantizing again.
    struct LastQuant { bool on = false; GemmQuantArgs q; uint32_t x_off, x_len; } lastq;

    int fused_out = 0;  // fused DeltaNet step + ssm_out launches so far: launch j uses exchange counter slot j % 2

    bool compile(const uint32_t * cmds, unsigned n) {
        for (unsigned i = 0; i < n;) {
            const size_t before = out.size();
            const unsigned at = i;
            if (!compile_one(cmds, n, i)) return false;
            // a command that overwrote the row or the weight of a pending deferred norm: a later GEMV on the norm
            // reads a snapshot computed before that command. A command that added no launch joined the last one
            // (a GEMM merged into the previous GEMM's launch), which then does the writing: the snapshot goes
            // before that launch.
            if (defer.on && !defer.snap && defer.dirty < 0) {
                std::vector<Rng> wr;
                cmd_writes(cmds, n, at, i - at, wr);
                if (meet_any(wr, defer_ranges())) defer.dirty = long(out.size() == before && before > 0 ? before - 1 : before);
            }
        }
        if (fused_out % 2) {  // the last fused launch used slot 0: clear its tags for the next list (slot 1 is clear)
            EwArgs z{nullptr, nullptr, reinterpret_cast<float *>(c->gdn_xch), 2 * GDN_XCH_COPIES * GDN_XCH_SLOT, 0, 0,
                     EW_FILL, 0.0f};
            out.push_back(LEw{z});
            spans.push_back({int(n) - 1, 1});
        }
        return true;
    }

    // Compiles the command at i (with the commands it consumes); advances i past them.
    bool compile_one(const uint32_t * cmds, unsigned n, unsigned & i) {
        {
            const uint32_t * k = cmds + size_t(i) * GEMVQ_CMD_WORDS;
            const uint32_t op = k[0];
            if (op != GEMVQ_OP_GEMM) lastq.on = tok_open = false;
            switch (op) {
            case GEMVQ_OP_GEMV: {
                unsigned used = 0;
                if (!gemv_group(cmds, n, i, used)) return false;
                i += used;
                return true;
            }
            case GEMVQ_OP_RMSNORM: {
                const uint32_t nn = k[1], rows = k[6] ? k[6] : 1, flags = k[7], stride = ((flags >> 8) & 0xffffu) * 16;
                const uint32_t st = stride ? stride : nn;
                if (nn == 0 || nn % 16 || nn > GEMVQ_MAX_COLS || stride % 16) return reject(i, "RMSNORM n");
                if (stride && stride < nn) return reject(i, "RMSNORM stride");
                if (!range(k[2], uint64_t(st) * (rows - 1) + nn) || !range(k[4], uint64_t(nn) * rows)) return reject(i, "RMSNORM range");
                if (!(flags & GEMVQ_NORM_NO_WEIGHT) && !range(k[3], nn)) return reject(i, "RMSNORM weight");
                if (flags & GEMVQ_NORM_DEFER) {
                    if (rows != 1 || stride) return reject(i, "deferred RMSNORM needs one packed row");
                    defer.on = true;
                    defer.snap = false;
                    defer.dirty = -1;
                    defer.n = nn;
                    defer.x = k[2];
                    defer.w = k[3];
                    defer.y = k[4];
                    defer.eps = bits_f(k[5]);
                    defer.flags = flags;
                } else {
                    NormArgs a{A(k[2]), (flags & GEMVQ_NORM_NO_WEIGHT) ? nullptr : A(k[3]), A(k[4]), int(nn), int(rows),
                               int(st), bits_f(k[5]), int(flags & 3)};
                    out.push_back(LNorm{a, ref()});
                    spans.push_back({int(i), 1});
                }
                break;
            }
            case GEMVQ_OP_ADD:
            case GEMVQ_OP_MUL: {
                const uint32_t nn = k[1];
                if (nn == 0 || !range(k[2], nn) || !range(k[3], nn) || !range(k[4], nn)) return reject(i, "ADD/MUL range");
                EwArgs a{A(k[2]), A(k[3]), A(k[4]), int(nn), 0, 0, op == GEMVQ_OP_ADD ? EW_ADD : EW_MUL, 0.0f};
                out.push_back(LEw{a});
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_SILU_MUL: {
                const uint32_t nn = k[1], row = k[6], stride = k[7];
                if (nn == 0 || !range(k[3], nn) || !range(k[4], nn)) return reject(i, "SILU_MUL range");
                if (row) {
                    if (nn % row || row % 16 || stride % 16 || stride < row || !range(k[2], uint64_t(stride) * (nn / row - 1) + row))
                        return reject(i, "SILU_MUL rows");
                } else if (!range(k[2], nn)) {
                    return reject(i, "SILU_MUL range");
                }
                EwArgs a{A(k[2]), A(k[3]), A(k[4]), int(nn), int(row), int(stride),
                         (k[5] & GEMVQ_SILU_MUL_SIGMOID) ? EW_SIGMOID_MUL : EW_SILU_MUL, 0.0f};
                out.push_back(LEw{a, ref()});
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_UNARY: {
                const uint32_t nn = k[1], kind = k[3], row = k[5], stride = k[6];
                if (nn == 0 || kind < 1 || kind > 4 || !range(k[4], nn)) return reject(i, "UNARY");
                if (row) {
                    if (nn % row || row % 16 || stride % 16 || stride < row || !range(k[2], uint64_t(stride) * (nn / row - 1) + row))
                        return reject(i, "UNARY rows");
                } else if (!range(k[2], nn)) {
                    return reject(i, "UNARY range");
                }
                const int ops[5] = {0, EW_SILU, EW_SIGMOID, EW_SOFTPLUS, EW_COPY};
                EwArgs a{A(k[2]), nullptr, A(k[4]), int(nn), int(row), int(stride), ops[kind], 0.0f};
                out.push_back(LEw{a, ref()});
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_GDN: {
                if (i + 1 >= n) return reject(i, "GDN needs its second slot");
                const uint32_t * k2 = k + GEMVQ_CMD_WORDS;
                const uint32_t hv = k[1] & 0xffffu, hk = k[1] >> 16, flags = k2[3];
                const bool gates = flags & GEMVQ_GDN_GATES;
                if (gates && i + 2 >= n) return reject(i, "GDN needs its gates slot");
                const uint32_t * k3 = gates ? k2 + GEMVQ_CMD_WORDS : nullptr;
                if (hv == 0 || hk == 0 || hv > GDN_MAX_HEADS || hv % hk) return reject(i, "GDN heads");
                // tokens (gates slot words 2..4): n_tok, the q / k / v row stride, the g / beta row stride; y and
                // z rows are packed (hv * 128 floats apart)
                const uint32_t ntok = gates && k3[2] ? k3[2] : 1, sq = ntok > 1 ? k3[3] : 0, sg = ntok > 1 ? k3[4] : 0;
                const uint64_t yz = uint64_t(hv) * 128 * (ntok - 1);
                if (ntok > GEMVQ_GEMM_MAX_TOK || (ntok > 1 && (sq % 16 || sg % 16))) return reject(i, "GDN tokens");
                if (!range(k[2], uint64_t(sq) * (ntok - 1) + hk * 128) || !range(k[3], uint64_t(sq) * (ntok - 1) + hk * 128) ||
                    !range(k[4], uint64_t(sq) * (ntok - 1) + hv * 128) || !range(k[5], uint64_t(sg) * (ntok - 1) + hv) ||
                    !range(k[6], uint64_t(sg) * (ntok - 1) + hv) || !range(k[7], yz + hv * 128))
                    return reject(i, "GDN range");
                const uint64_t src = k2[0], dst = k2[1];
                const bool seqs = flags & GEMVQ_GDN_SEQS;  // token t of sequence t on state rows + t hv 128
                const uint64_t srows = uint64_t(hv) * 128 * (seqs ? ntok : 1);
                if (src + srows > c->state_rows || dst + srows > c->state_rows) return reject(i, "GDN state rows");
                if (src != dst && (src < dst + srows && dst < src + srows)) return reject(i, "GDN state overlap");
                if (gates && (!range(k3[0], hv) || !range(k3[1], hv))) return reject(i, "GDN gates range");
                if ((flags & GEMVQ_GDN_GATED) && (!range(k2[6], 128) || !range(k2[7], yz + hv * 128))) return reject(i, "GDN gated range");
                GdnArgs a{};
                a.q = A(k[2]);
                a.k = A(k[3]);
                a.v = A(k[4]);
                a.g = A(k[5]);
                a.beta = A(k[6]);
                a.y = A(k[7]);
                a.dt = gates ? A(k3[0]) : nullptr;
                a.a = gates ? A(k3[1]) : nullptr;
                a.src = c->state + src * 128;
                a.dst = c->state + dst * 128;
                a.hv = int(hv);
                a.hk = int(hk);
                a.scale = bits_f(k2[2]);
                a.l2_eps = bits_f(k2[4]);
                a.flags = int(flags);
                a.n_tok = int(ntok);
                a.s_qkv = int(sq);
                a.s_gb = int(sg);
                a.s_y = int(hv * 128);
                a.seqs = int(seqs && ntok > 1);
                const unsigned next = i + (gates ? 3 : 2);
                uint32_t fy = 0, fres = 0;
                if (ref()) {  // the tokens one launch each, in order, each with the gated norm of its heads
                    if (flags & GEMVQ_GDN_GATED) {
                        a.gz = A(k2[7]);
                        a.gw = A(k2[6]);
                        a.rms_eps = bits_f(k2[5]);
                    }
                    for (uint32_t t = 0; t < ntok; ++t) {
                        out.push_back(LGdn{a, 1, int(t)});
                        spans.push_back({int(i), gates ? 3 : 2});
                    }
                    i = next;
                    return true;
                }
                // what the step reads and writes in the act buffer (the fused launch's rows must stay apart)
                std::vector<Rng> step_io = {{k[2], uint64_t(k[2]) + hk * 128}, {k[3], uint64_t(k[3]) + hk * 128},
                                            {k[4], uint64_t(k[4]) + hv * 128}, {k[5], uint64_t(k[5]) + hv},
                                            {k[6], uint64_t(k[6]) + hv}, {k[7], uint64_t(k[7]) + hv * 128},
                                            {k2[6], uint64_t(k2[6]) + 128}, {k2[7], uint64_t(k2[7]) + hv * 128}};
                if (gates) {
                    step_io.push_back({k3[0], uint64_t(k3[0]) + hv});
                    step_io.push_back({k3[1], uint64_t(k3[1]) + hv});
                }
                if ((flags & GEMVQ_GDN_GATED) && (flags & GEMVQ_GDN_WITH_OUT) && ntok == 1 &&
                    fuse_out(cmds, n, next, step_io, k[7], hv, fy, fres)) {
                    // asked for with GEMVQ_GDN_WITH_OUT: the step, the gated norm, ssm_out and its ADD in one launch
                    const uint32_t * g = cmds + size_t(next) * GEMVQ_CMD_WORDS;
                    const int t = int(g[1] & 0xffu);
                    GdnOutArgs o{};
                    o.g = a;
                    o.z = A(k2[7]);
                    o.nw = A(k2[6]);
                    o.rms_eps = bits_f(k2[5]);
                    o.z_silu = int(bool(flags & GEMVQ_GDN_Z_SILU));
                    o.y = A(k[7]);
                    o.rows = int(g[2]);
                    o.w = weight_view(c->warena + (uint64_t(g[4]) | (uint64_t(g[5]) << 32)), t, o.rows, int(hv * 128));
                    o.res = A(fres);
                    o.out = A(fy);
                    o.xch = c->gdn_xch;
                    o.fault = c->gdn_fault;
                    o.polls = c->xch_polls;
                    o.slot = fused_out++ % 2;
                    out.push_back(LGdnOut{o, t});
                    spans.push_back({int(i), int(next + 2 - i)});
                    i = next + 2;
                    return true;
                }
                if ((flags & GEMVQ_GDN_GATED) && ntok == 1 && fold_gated(cmds, n, next, k[7], hv * 128, k2[7], k2[6])) {
                    // the gated norm runs in the next GEMV's activation prologue: the step writes its raw output
                    // to scratch, and that GEMV writes the gated values to y as the norm would have
                    a.y = c->gdn_raw;
                    a.flags = int(flags & ~GEMVQ_GDN_GATED);
                    gated = {true, k[7], hv * 128, A(k2[7]), A(k2[6]), bits_f(k2[5]), int(bool(flags & GEMVQ_GDN_Z_SILU))};
                }
                out.push_back(LGdn{a});
                spans.push_back({int(i), gates ? 3 : 2});
                if ((flags & GEMVQ_GDN_GATED) && !gated.on) {
                    GatedNormArgs g{A(k[7]), A(k2[7]), A(k2[6]), int(hv * ntok), bits_f(k2[5]), int(bool(flags & GEMVQ_GDN_Z_SILU))};
                    out.push_back(LGated{g});
                    spans.push_back({int(i), gates ? 3 : 2});
                }
                i = next;
                return true;
            }
            case GEMVQ_OP_CONV: {
                const uint32_t ch = k[1], ntok = (k[7] >> 16) ? (k[7] >> 16) : 1;  // packed token rows
                const bool seqs = k[7] & GEMVQ_CONV_SEQS;  // token t of sequence t: windows packed, 3 ch apart
                const uint64_t sw = 3ull * ch * (seqs ? ntok : 1);
                if (ch == 0 || ch % 16 || ntok > GEMVQ_GEMM_MAX_TOK || !range(k[2], uint64_t(ch) * ntok) ||
                    !range(k[3], 4ull * ch) || !range(k[4], uint64_t(ch) * ntok) || !range(k[5], sw) ||
                    !range(k[6], sw))
                    return reject(i, "CONV range");
                if (seqs && k[5] != k[6] && meet({k[5], k[5] + sw}, {k[6], k[6] + sw})) return reject(i, "CONV state overlap");
                ConvArgs a{A(k[2]), A(k[3]), A(k[5]), A(k[6]), A(k[4]), int(ch), int(k[7] & 1), int(ntok), int(seqs)};
                if (ref()) {  // the tokens one launch each, in order
                    for (uint32_t t = 0; t + 1 < ntok; ++t) {
                        out.push_back(LConv{a, 1, int(t)});
                        spans.push_back({int(i), 1});
                    }
                    out.push_back(LConv{a, 1, int(ntok - 1)});
                } else {
                    out.push_back(LConv{a});
                }
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_STATE_LOAD:
            case GEMVQ_OP_TRACE:
                break;
            case GEMVQ_OP_ROPE: {
                const uint32_t nd = k[1], ne0 = k[5], rows = k[6], pos_off = k[7];
                if (nd == 0 || nd % 2 || nd > ne0 || ne0 % 16 || ne0 > 1024 || rows == 0) return reject(i, "ROPE shape");
                if (!range(k[2], uint64_t(ne0) * rows) || !range(k[4], uint64_t(ne0) * rows)) return reject(i, "ROPE range");
                if (pos_off && !range(pos_off, 1)) return reject(i, "ROPE pos");
                if (!pos_off && k[3] + uint64_t(nd) > c->act_floats) return reject(i, "ROPE cache");
                RopeArgs a{A(k[2]), A(k[3]), pos_off ? reinterpret_cast<const int32_t *>(A(pos_off)) : nullptr, A(k[4]),
                           int(nd), int(ne0), int(rows)};
                out.push_back(LRope{a});
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_ATTN: {
                if (i + 1 >= n) return reject(i, "ATTN needs its second slot");
                const uint32_t * k2 = k + GEMVQ_CMD_WORDS;
                const uint32_t nh = k[1] & 0xffffu, nkv = k[1] >> 16, hd = k[5] & 0xffffu, nrot = k[5] >> 16;
                const uint32_t kv = k[3], flags = k[7];
                if (kv >= c->kvs.size()) return reject(i, "ATTN kv buffer");
                const KvBuf & b = c->kvs[kv];
                if (nkv == 0 || nh % nkv || nh / nkv > ATTN_MAXG || int(nkv) != b.n_head_kv || int(hd) != b.head_dim || hd > 256 ||
                    hd < 16 || (hd & (hd - 1)) || nrot > hd || nrot % 2)
                    return reject(i, "ATTN shape");
                const uint32_t qstride = (flags & 1) ? 2 * hd : hd, ntok = (flags >> 16) & 0xffu ? (flags >> 16) & 0xffu : 1;
                if (ntok > GEMVQ_GEMM_MAX_TOK) return reject(i, "ATTN tokens");
                // token t of sequence t: position at pos + 16 t, the cache split into ntok equal regions
                const bool seqs = (flags & GEMVQ_ATTN_SEQS) && ntok > 1;
                if (seqs && (b.n_ctx % int(ntok) || !range(k[6], 16ull * (ntok - 1) + 1))) return reject(i, "ATTN sequences");
                const uint64_t qt = uint64_t(nh) * qstride * (ntok - 1), kvt = uint64_t(nkv) * hd * ntok;  // packed tokens
                if (!range(k[2], qt + uint64_t(qstride) * (nh - 1) + hd) || !range(k[4], uint64_t(nh) * hd * ntok) ||
                    !range(k[6], 1) || !range(k2[0], kvt) || !range(k2[1], kvt) || !range(k2[4], hd) ||
                    !range(k2[5], hd) || k2[6] + uint64_t(seqs ? b.n_ctx / int(ntok) : b.n_ctx) * nrot > c->act_floats)
                    return reject(i, "ATTN range");
                if ((flags & 1) && !range(k2[7], qt + uint64_t(2 * hd) * (nh - 1) + hd)) return reject(i, "ATTN gate range");
                AttnArgs a{};
                a.q = A(k[2]);
                a.k = A(k2[0]);
                a.v = A(k2[1]);
                a.qn = A(k2[4]);
                a.kn = A(k2[5]);
                a.cs = A(k2[6]);
                a.pos = reinterpret_cast<const int32_t *>(A(k[6]));
                a.gate = (flags & 1) ? A(k2[7]) : nullptr;
                a.y = A(k[4]);
                a.kc = b.k;
                a.vc = b.v;
                a.part = b.part;
                a.counter = b.counter;
                a.n_head = int(nh);
                a.n_head_kv = int(nkv);
                a.head_dim = int(hd);
                a.n_rot = int(nrot);
                a.q_stride = int(qstride);
                a.n_ctx = seqs ? b.n_ctx / int(ntok) : b.n_ctx;
                a.seq_ctx = seqs ? a.n_ctx : 0;
                a.scale = bits_f(k2[2]);
                a.eps = bits_f(k2[3]);
                a.n_tok = int(ntok);
                a.qr = b.qr;
                if (ref()) {  // the tokens one launch pair each, in order
                    for (uint32_t t = 0; t < ntok; ++t) {
                        out.push_back(LAttn{a, 1, int(t)});
                        spans.push_back({int(i), 2});
                    }
                } else {
                    out.push_back(LAttn{a});
                    spans.push_back({int(i), 2});
                }
                i += 2;
                return true;
            }
            case GEMVQ_OP_GEMM: {
                unsigned used = 0;
                if (!gemm(cmds, n, i, used)) return false;
                i += used;
                return true;
            }
            case GEMVQ_OP_GET_ROWS: {
                const int type = int(k[1] & 0xffu), rows = int(k[2]), cols = int(k[3]);
                const uint32_t ntok = (k[1] >> 16) & 0xffu ? (k[1] >> 16) & 0xffu : 1;  // ids 16 floats apart
                const uint64_t woff = uint64_t(k[4]) | (uint64_t(k[5]) << 32);
                if (type != T_Q6_K && type != T_Q4_0 && type != T_Q8_0) return reject(i, "GET_ROWS type");
                if (ntok > GEMVQ_GEMM_MAX_TOK) return reject(i, "GET_ROWS tokens");
                if (!weight(woff, type, rows, cols)) return reject(i, "GET_ROWS weight");
                if (!range(k[6], 16ull * (ntok - 1) + 1) || !range(k[7], uint64_t(cols) * ntok)) return reject(i, "GET_ROWS range");
                GetRowsArgs a{weight_view(c->warena + woff, type, rows, cols), reinterpret_cast<const int32_t *>(A(k[6])),
                              A(k[7]), rows, cols, type, int(ntok)};
                out.push_back(LRows{a});
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_ARGMAX: {
                const uint32_t rows = k[4] ? k[4] : 1, stride = rows > 1 ? k[5] : 0;  // rows: keys 16 floats apart
                if (k[1] == 0 || rows > GEMVQ_GEMM_MAX_TOK || (rows > 1 && (stride < k[1] || stride % 16)) ||
                    !range(k[2], uint64_t(stride) * (rows - 1) + k[1]) || !range(k[3], 16ull * (rows - 1) + 2))
                    return reject(i, "ARGMAX range");
                out.push_back(LArgmax{A(k[2]), int(k[1]), reinterpret_cast<unsigned long long *>(A(k[3])), int(rows),
                                      int(stride)});
                spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_NEXT_TOKEN: {
                const uint32_t ns = k[7] & 0xffu, cap = k[7] >> 8;  // sequences (2..): slots 16 floats apart
                if (ns > 1) {
                    const uint64_t sl = 16ull * (ns - 1);
                    if (ns > GEMVQ_GEMM_MAX_TOK || cap == 0 || !range(k[1], sl + 2) || !range(k[2], sl + 1) ||
                        !range(k[3], sl + 1) || !range(k[5], sl + 1) || !range(k[4], uint64_t(cap) * ns) ||
                        !range(k[6], uint64_t(cap) * ns))
                        return reject(i, "NEXT_TOKEN sequences");
                    NextTokenArgs a{};
                    a.key = reinterpret_cast<unsigned long long *>(A(k[1]));
                    a.tok = reinterpret_cast<int32_t *>(A(k[2]));
                    a.pos = reinterpret_cast<int32_t *>(A(k[3]));
                    a.prompt = reinterpret_cast<const int32_t *>(A(k[4]));
                    a.out = reinterpret_cast<int32_t *>(A(k[6]));
                    a.n_seq = int(ns);
                    a.n_prompt_of = reinterpret_cast<const int32_t *>(A(k[5]));
                    a.seq_cap = int(cap);
                    out.push_back(LNext{a});
                    spans.push_back({int(i), 1});
                    break;
                }
                if (!range(k[1], 2) || !range(k[2], 1) || !range(k[3], 1) || (k[5] && !range(k[4], k[5])) ||
                    !range(k[6], 1))
                    return reject(i, "NEXT_TOKEN range");
                NextTokenArgs a{};
                a.key = reinterpret_cast<unsigned long long *>(A(k[1]));
                a.tok = reinterpret_cast<int32_t *>(A(k[2]));
                a.pos = reinterpret_cast<int32_t *>(A(k[3]));
                a.prompt = reinterpret_cast<const int32_t *>(A(k[4]));
                a.n_prompt = int(k[5]);
                a.out = reinterpret_cast<int32_t *>(A(k[6]));
                a.max_pos = int(c->act_floats - k[6]);
                out.push_back(LNext{a});
                    spans.push_back({int(i), 1});
                break;
            }
            case GEMVQ_OP_FILL: {
                if (k[1] == 0 || !range(k[2], k[1])) return reject(i, "FILL range");
                EwArgs a{nullptr, nullptr, A(k[2]), int(k[1]), 0, 0, EW_FILL, bits_f(k[3])};
                out.push_back(LEw{a});
                    spans.push_back({int(i), 1});
                break;
            }
            default:
                return reject(i, "unknown opcode " + std::to_string(op));
            }
            ++i;
        }
        return true;
    }

    // A batched GEMV at command i (two slots; a SwiGLU g takes its u command too): the activation rows are
    // quantized once into the context's scratch rows, then every weight row is read once for all the tokens.
    bool gemm(const uint32_t * cmds, unsigned n, unsigned i, unsigned & used) {
        if (i + 1 >= n) return reject(i, "GEMM needs its second slot");
        const uint32_t * k = cmds + size_t(i) * GEMVQ_CMD_WORDS, * k2 = k + GEMVQ_CMD_WORDS;
        const int t = int(k[1] & 0xffu), rows = int(k[2]);
        const uint32_t flags = k[1] & ~0xffu, cols = k[3], ntok = k2[0], xs = k2[1], ys = k2[2], nflags = k2[7];
        const bool kq = t == T_Q5_K || t == T_Q6_K;  // no MFMA form: launches of up to 4 tokens of the small-token GEMV
        if (t != T_Q4_0 && t != T_Q4_1 && t != T_Q8_0 && !kq) return reject(i, "GEMM format (Q4_0, Q4_1, Q8_0, Q5_K or Q6_K)");
        if (rows <= 0 || cols == 0 || cols % 512 || cols > GEMVQ_MAX_COLS) return reject(i, "GEMM shape (cols a multiple of 512)");
        if (flags & ~(GEMVQ_GEMV_SWIGLU | GEMVQ_GEMV_ADD | GEMVQ_GEMV_SILU) || __builtin_popcount(flags) > 1)
            return reject(i, "GEMM flags");
        if (kq && ((flags & GEMVQ_GEMV_SWIGLU) || !gemv_tok_ok(t, int(cols), 1, false)))
            return reject(i, "GEMM on K-quant weights: no SwiGLU pair, at most 12288 columns");
        if (ntok < 1 || ntok > GEMVQ_GEMM_MAX_TOK) return reject(i, "GEMM token count");
        if (xs % 16 || xs < cols || ys % 16 || ys < uint32_t(rows)) return reject(i, "GEMM strides");
        const uint64_t woff = uint64_t(k[4]) | (uint64_t(k[5]) << 32);
        const Weight * gw = weight(woff, t, rows, int(cols));
        if (!gw) return reject(i, "GEMM weight offset, format or shape does not match an uploaded weight");
        if (!range(k[6], uint64_t(xs) * (ntok - 1) + cols) || !range(k[7], uint64_t(ys) * (ntok - 1) + rows))
            return reject(i, "GEMM range");
        const bool norm = nflags & GEMVQ_NORM_DEFER, normw = norm && !(nflags & GEMVQ_NORM_NO_WEIGHT);
        if (nflags & ~(GEMVQ_NORM_DEFER | GEMVQ_NORM_NO_WEIGHT | GEMVQ_NORM_L2) || (normw && !range(k2[5], cols)))
            return reject(i, "GEMM norm");
        GemmArgs g{};
        g.w = weight_view(c->warena + woff, t, rows, int(cols));
        g.wbound[0] = gw->wbound;
        g.rows = rows;
        g.cols = int(cols);
        g.n_tok = int(ntok);
        g.y = A(k[7]);
        g.y_stride = int(ys);
        g.epi = EPI_PLAIN;
        used = 2;
        if (flags & GEMVQ_GEMV_SWIGLU) {
            if (i + 3 >= n) return reject(i, "SwiGLU GEMM without its u GEMM");
            const uint32_t * u = k + 2 * GEMVQ_CMD_WORDS, * u2 = u + GEMVQ_CMD_WORDS;
            const uint64_t uoff = uint64_t(u[4]) | (uint64_t(u[5]) << 32);
            if (u[0] != GEMVQ_OP_GEMM || u[1] != uint32_t(t) || int(u[2]) != rows || u[3] != cols || u[6] != k[6] ||
                u2[0] != ntok || u2[1] != xs || u2[5] != k2[5] || u2[6] != k2[6] || u2[7] != nflags)
                return reject(i + 2, "SwiGLU u GEMM must match its g GEMM");
            const Weight * uw = weight(uoff, t, rows, int(cols));
            if (u2[2] % 16 || u2[2] < uint32_t(rows) || !uw || !range(u[7], uint64_t(u2[2]) * (ntok - 1) + rows))
                return reject(i + 2, "SwiGLU u GEMM weight, stride or range");
            if (!(uw->wbound <= g.wbound[0])) g.wbound[0] = uw->wbound;
            g.epi = EPI_SWIGLU;
            g.w2 = weight_view(c->warena + uoff, t, rows, int(cols));
            g.y = A(u[7]);
            g.y_stride = int(u2[2]);
            used = 4;
        } else if (flags & GEMVQ_GEMV_ADD) {
            const uint32_t rs = k2[4];
            if (rs % 16 || rs < uint32_t(rows) || !range(k2[3], uint64_t(rs) * (ntok - 1) + rows)) return reject(i, "GEMM residual");
            g.epi = EPI_ADD;
            g.res = A(k2[3]);
            g.res_stride = int(rs);
        } else if (flags & GEMVQ_GEMV_SILU) {
            g.epi = EPI_SILU;
        }
        const uint32_t x_len = xs * (ntok - 1) + cols;
        const uint32_t y_off = uint32_t(g.y - c->act), y_len = uint32_t(g.y_stride) * (ntok - 1) + uint32_t(rows);
        // 2-4 tokens (K-quants: any count, in launches of up to 4): the small-token GEMV, which quantizes the rows in
        // every workgroup's prologue, so no output may fall on the rows or the norm weight (other workgroups may still
        // be reading them)
        const bool over = (y_off < k[6] + x_len && k[6] < y_off + y_len) || (normw && y_off < k2[5] + cols && k2[5] < y_off + y_len);
        if (kq && over && !ref()) return reject(i, "GEMM on K-quant weights: the output falls on the input rows or the norm weight");
        if (ref()) return gemm_ref(g, t, k, k2, over, normw, i, used);
        if (kq || (!over && gemv_tok_ok(t, int(cols), int(ntok), g.epi == EPI_SWIGLU))) {
            const uint32_t cs = kq ? (gemv_tok_ok(t, int(cols), TOK_MAX, false) ? TOK_MAX : 2) : ntok;  // tokens a launch
            for (uint32_t c0 = 0; c0 < ntok; c0 += cs) {
                const uint32_t nt = std::min(cs, ntok - c0);
                TokArgs ta{};
                ta.x = A(k[6]) + size_t(c0) * xs;
                ta.norm_w = normw ? A(k2[5]) : nullptr;
                ta.eps = bits_f(k2[6]);
                ta.norm = norm ? 1 : 0;
                ta.norm_l2 = (nflags & GEMVQ_NORM_L2) ? 1 : 0;
                ta.cols = int(cols);
                ta.n_tok = int(nt);
                ta.x_stride = int(xs);
                ta.n_members = 1;
                ta.wbound[0] = g.wbound[0];
                TokMember & m = ta.m[0];
                m.w = g.w;
                m.w2 = g.w2;
                m.y = g.y + size_t(c0) * g.y_stride;
                m.res = g.res ? g.res + size_t(c0) * g.res_stride : nullptr;
                m.rows = rows;
                m.y_stride = g.y_stride;
                m.res_stride = g.res_stride;
                m.epi = g.epi;
                if (!(nt == ntok && merge_tok(ta, t, k[6], x_len, int(i), int(used)))) {
                    out.push_back(LTok{ta, t, uint32_t(k[6] + c0 * xs), xs * (nt - 1) + cols});
                    spans.push_back({int(i), int(used)});
                }
            }
            tok_open = cs >= ntok;  // a later GEMM on the same rows may join a launch that holds all of them
            // the outputs end a reuse of the last batched GEMV's quantized rows if they fall on its rows or weight
            const bool hits_x = y_off < lastq.x_off + lastq.x_len && lastq.x_off < y_off + y_len;
            const uint32_t w_off = lastq.q.norm_w ? uint32_t(lastq.q.norm_w - c->act) : 0;
            if (hits_x || (lastq.q.norm_w && y_off < w_off + lastq.q.cols && w_off < y_off + y_len)) lastq.on = false;
            return true;
        }
        tok_open = false;
        GemmQuantArgs q{};
        q.x = A(k[6]);
        q.norm_w = normw ? A(k2[5]) : nullptr;
        q.q = c->gemm_q;
        q.d40 = c->gemm_d;
        q.s40 = c->gemm_s;
        q.n_tok = int(ntok);
        q.n_pad = int((ntok + 15) / 16 * 16);
        q.cols = int(cols);
        q.x_stride = int(xs);
        q.norm = norm ? 1 : 0;
        q.norm_l2 = (nflags & GEMVQ_NORM_L2) ? 1 : 0;
        q.eps = bits_f(k2[6]);
        g.q = c->gemm_q;
        g.d40 = c->gemm_d;
        g.s40 = c->gemm_s;
        const bool same = lastq.on && lastq.x_off == k[6] && lastq.x_len == x_len && lastq.q.n_tok == q.n_tok &&
                          lastq.q.cols == q.cols && lastq.q.x_stride == q.x_stride && lastq.q.norm == q.norm &&
                          lastq.q.norm_l2 == q.norm_l2 && lastq.q.norm_w == q.norm_w && lastq.q.eps == q.eps;
        if (!same) {
            out.push_back(LGemmQ{q});
            spans.push_back({int(i), int(used)});
            lastq = {true, q, k[6], x_len};
        }
        if (!(same && merge_gemm(g, t, int(i), int(used)))) {
            out.push_back(LGemm{g, t});
            spans.push_back({int(i), int(used)});
        }
        // outputs written over the quantized rows (or the norm weight) end the reuse
        const bool hits_x = y_off < lastq.x_off + lastq.x_len && lastq.x_off < y_off + y_len;
        const uint32_t w_off = q.norm_w ? uint32_t(q.norm_w - c->act) : 0;
        const bool hits_w = q.norm_w && y_off < w_off + cols && w_off < y_off + y_len;
        if (hits_x || hits_w) lastq.on = false;
        return true;
    }

    // The reference arithmetic has no batched form: token t of a GEMM runs as the GEMV command on its row (with the
    // per-token norm as a deferred norm), one launch each. An output that falls on the token rows or the norm weight
    // would change what a later token reads, so those are copied first (as the batched kernels read them all before
    // writing).
    bool gemm_ref(const GemmArgs & g, int t, const uint32_t * k, const uint32_t * k2, bool over, bool normw, unsigned i,
                  unsigned used) {
        const uint32_t cols = k[3], ntok = k2[0], xs = k2[1], nflags = k2[7];
        const float * x = A(k[6]);
        size_t xstride = xs;
        const float * nw = normw ? A(k2[5]) : nullptr;
        if (over) {
            EwArgs cp{x, nullptr, c->ref_x, int(cols * ntok), int(cols), int(xs), EW_COPY, 0.0f};
            out.push_back(LEw{cp});
            spans.push_back({int(i), int(used)});
            x = c->ref_x;
            xstride = cols;
            if (nw) {
                EwArgs cw{nw, nullptr, c->ref_x + size_t(GEMM_MAX_TOK) * GEMV_MAXK, int(cols), 0, 0, EW_COPY, 0.0f};
                out.push_back(LEw{cw});
                spans.push_back({int(i), int(used)});
                nw = c->ref_x + size_t(GEMM_MAX_TOK) * GEMV_MAXK;
            }
        }
        for (uint32_t tk = 0; tk < ntok; ++tk) {
            GemvArgs a{};
            a.x = x + tk * xstride;
            a.cols = int(cols);
            a.xsrc = (nflags & GEMVQ_NORM_DEFER) ? XSRC_NORM : XSRC_RAW;
            a.norm_w = nw;
            a.norm_eps = bits_f(k2[6]);
            a.norm_l2 = (nflags & GEMVQ_NORM_L2) ? 1 : 0;
            a.n_members = 1;
            a.total_tasks = g.rows;
            GemvMember & m = a.m[0];
            m.w = g.w;
            m.w2 = g.w2;
            m.rows = g.rows;
            m.epi = g.epi;
            m.y = g.y + size_t(tk) * g.y_stride;
            m.res = g.res ? g.res + size_t(tk) * g.res_stride : nullptr;
            a.wbound[0] = g.wbound[0];
            out.push_back(LGemv{a, t, 1});
            spans.push_back({int(i), int(used)});
        }
        lastq.on = tok_open = false;
        return true;
    }

    // A small-token GEMM right after another on the same rows (the same token count, stride and norm) joins its launch
    // as a further member (up to four, none a SwiGLU pair), under the rules of merge_gemm; no member writes the rows
    // or the norm weight (checked before).
    bool tok_open = false;  // the last command was a GEMM that made or joined the last launch, an LTok
    bool merge_tok(const TokArgs & g, int t, uint32_t x_off, uint32_t x_len, int i, int used) {
        auto * p = out.empty() || !tok_open ? nullptr : std::get_if<LTok>(&out.back());
        if (!p || p->type != t || p->x_off != x_off || p->x_len != x_len || p->a.n_members >= 4 ||
            p->a.m[0].epi == EPI_SWIGLU || g.m[0].epi == EPI_SWIGLU || p->a.n_tok != g.n_tok || p->a.cols != g.cols ||
            p->a.x_stride != g.x_stride || p->a.norm != g.norm || p->a.norm_l2 != g.norm_l2 || p->a.norm_w != g.norm_w ||
            p->a.eps != g.eps)
            return false;
        struct R { uint64_t lo, hi; };
        auto span = [&](const float * base, int stride, int rows) {
            const uint64_t lo = uint64_t(base - c->act);
            return R{lo, lo + uint64_t(stride) * uint64_t(g.n_tok - 1) + uint64_t(rows)};
        };
        auto meet = [](R x, R y) { return x.lo < y.hi && y.lo < x.hi; };
        const TokMember & nm = g.m[0];
        const R ny = span(nm.y, nm.y_stride, nm.rows);
        const bool nres = nm.epi == EPI_ADD;
        const R nr = nres ? span(nm.res, nm.res_stride, nm.rows) : R{0, 0};
        for (int m = 0; m < p->a.n_members; ++m) {
            const TokMember & o = p->a.m[m];
            const R y = span(o.y, o.y_stride, o.rows);
            const R res = o.epi == EPI_ADD ? span(o.res, o.res_stride, o.rows) : R{0, 0};
            if (meet(ny, y) || (o.epi == EPI_ADD && meet(ny, res)) || (nres && meet(nr, y))) return false;
        }
        p->a.wbound[p->a.n_members] = g.wbound[0];
        p->a.m[p->a.n_members++] = nm;
        spans.back().second = i + used - spans.back().first;
        return true;
    }

    // A GEMM on the rows the previous GEMM launch quantized joins that launch as a further member (up to four, none a
    // SwiGLU pair) when no member's output overlaps another's output or residual (so the order between them does not
    // matter); its command span extends the launch's.
    bool merge_gemm(const GemmArgs & g, int t, int i, int used) {
        auto * p = out.empty() ? nullptr : std::get_if<LGemm>(&out.back());
        if (!p || p->type != t || p->a.epi == EPI_SWIGLU || g.epi == EPI_SWIGLU || p->a.n_more >= GEMM_MAX_MORE ||
            p->a.n_tok != g.n_tok || p->a.cols != g.cols || p->a.q != g.q)
            return false;
        struct R { uint64_t lo, hi; };
        auto span = [&](const float * base, int stride, int rows) {
            const uint64_t lo = uint64_t(base - c->act);
            return R{lo, lo + uint64_t(stride) * uint64_t(g.n_tok - 1) + uint64_t(rows)};
        };
        auto meet = [](R x, R y) { return x.lo < y.hi && y.lo < x.hi; };
        const R ny = span(g.y, g.y_stride, g.rows);
        const bool nres = g.epi == EPI_ADD;
        const R nr = nres ? span(g.res, g.res_stride, g.rows) : R{0, 0};
        int tiles = 0;
        for (int m = 0; m <= p->a.n_more; ++m) {
            const bool first = m == 0;
            const GemmMore * o = first ? nullptr : &p->a.more[m - 1];
            const R y = first ? span(p->a.y, p->a.y_stride, p->a.rows) : span(o->y, o->y_stride, o->rows);
            const int epi = first ? p->a.epi : o->epi;
            const R res = epi == EPI_ADD ? (first ? span(p->a.res, p->a.res_stride, p->a.rows) : span(o->res, o->res_stride, o->rows))
                                         : R{0, 0};
            if (meet(ny, y) || (epi == EPI_ADD && meet(ny, res)) || (nres && meet(nr, y))) return false;
            tiles += ((first ? p->a.rows : o->rows) + 15) / 16;
        }
        p->a.wbound[p->a.n_more + 1] = g.wbound[0];
        p->a.more[p->a.n_more++] = GemmMore{g.w, g.y, g.res, g.rows, g.y_stride, g.res_stride, g.epi, tiles};
        spans.back().second = i + used - spans.back().first;
        return true;
    }

    // A GEMV group starting at command i (gemvqc16.h:26-45, gemvqc16.cpp:646-733). Its members run in one launch,
    // so a member joins only if the order against the earlier members cannot matter: it writes nothing an earlier
    // member writes or reads, and reads nothing an earlier member writes (a residual loaded while another member's
    // rows are stored; gemvqc16.cpp:470-474, 686). A group ends after a member that writes over x.
    bool gemv_group(const uint32_t * cmds, unsigned n, unsigned i0, unsigned & used) {
        GemvArgs a{};
        int type = -1;
        uint32_t x_off = 0, cols = 0;
        unsigned i = i0, gemvs = 0;
        int tasks = 0;
        std::vector<Rng> W, R;  // what the members so far write and read during the pass
        while (i < n && a.n_members < 4) {
            const uint32_t * k = cmds + size_t(i) * GEMVQ_CMD_WORDS;
            if (k[0] != GEMVQ_OP_GEMV) break;
            const int t = int(k[1] & 0xffu);
            const uint32_t flags = k[1] & ~0xffu;
            const int rows = int(k[2]);
            if (gemvs > 0 && (k[6] != x_off || k[3] != cols || t != type)) break;
            if (!type_ok(t) || !shape_ok(t, rows, int(k[3]))) return reject(i, "GEMV format or shape");
            if (flags & ~(GEMVQ_GEMV_SWIGLU | GEMVQ_GEMV_CONV | GEMVQ_GEMV_ADD | GEMVQ_GEMV_ARGMAX | GEMVQ_GEMV_SILU))
                return reject(i, "GEMV flags");
            if (__builtin_popcount(flags) > 1) return reject(i, "GEMV: at most one epilog bit");
            const uint64_t woff = uint64_t(k[4]) | (uint64_t(k[5]) << 32);
            const Weight * w = weight(woff, t, rows, int(k[3]));
            if (!w) return reject(i, "GEMV weight offset, format or shape does not match an uploaded weight");
            if (!range(k[6], k[3]) || !range(k[7], uint64_t(rows))) return reject(i, "GEMV range");
            if (gemvs + ((flags & GEMVQ_GEMV_SWIGLU) ? 2 : 1) > GEMVQ_GROUP) break;
            std::vector<Rng> mw, mr;
            gemv_io(cmds, n, i, mw, mr);
            if (gemvs > 0 && (meet_any(mw, W) || meet_any(mw, R) || meet_any(mr, W))) break;
            // workgroup 0 writes the gated activation while the group runs, from z and the norm weight: no member
            // may write or read those
            if (gated.on && gemvs > 0 && (meet_any(mw, gated_ranges()) || meet_any(mr, gated_ranges()))) break;
            if (gated.on && (flags & GEMVQ_GEMV_SWIGLU)) break;
            if (gemvs == 0) {
                type = t;
                x_off = k[6];
                cols = k[3];
            }
            GemvMember m{};
            float wb = w->wbound;  // the member's term bound (a SwiGLU pair: the larger of its two matrices)
            m.w = weight_view(c->warena + woff, t, rows, int(cols));
            m.rows = rows;
            m.task_begin = tasks;
            m.epi = EPI_PLAIN;
            m.y = A(k[7]);
            unsigned step = 1;
            if (flags & GEMVQ_GEMV_SWIGLU) {
                if (i + 1 >= n) return reject(i, "SwiGLU GEMV without its u GEMV");
                const uint32_t * u = k + GEMVQ_CMD_WORDS;
                const uint64_t uoff = uint64_t(u[4]) | (uint64_t(u[5]) << 32);
                if (u[0] != GEMVQ_OP_GEMV || int(u[1] & 0xffu) != t || (u[1] & ~0xffu) || int(u[2]) != rows || u[3] != cols ||
                    u[6] != x_off)
                    return reject(i + 1, "SwiGLU u GEMV must match its g GEMV");
                const Weight * uw = weight(uoff, t, rows, int(cols));
                if (!uw || !range(u[7], uint64_t(rows))) return reject(i + 1, "SwiGLU u weight or range");
                if (!(uw->wbound <= wb)) wb = uw->wbound;
                m.epi = EPI_SWIGLU;
                m.w2 = weight_view(c->warena + uoff, t, rows, int(cols));
                m.y = A(u[7]);
                step = 2;
            } else if (flags & GEMVQ_GEMV_SILU) {
                m.epi = EPI_SILU;
            } else if (flags & (GEMVQ_GEMV_CONV | GEMVQ_GEMV_ADD | GEMVQ_GEMV_ARGMAX)) {
                if (i + 1 >= n) return reject(i, "GEMV epilog without its command");
                const uint32_t * e = k + GEMVQ_CMD_WORDS;
                if (flags & GEMVQ_GEMV_CONV) {
                    if (e[0] != GEMVQ_OP_CONV || e[1] != uint32_t(rows) || e[2] != k[7] || rows % 16 || (e[7] >> 16) > 1)
                        return reject(i + 1, "CONV epilog");
                    if (!range(e[3], 4ull * rows) || !range(e[4], uint64_t(rows)) || !range(e[5], 3ull * rows) ||
                        !range(e[6], 3ull * rows))
                        return reject(i + 1, "CONV epilog range");
                    m.epi = EPI_CONV;
                    m.conv_w = A(e[3]);
                    m.conv_src = A(e[5]);
                    m.conv_dst = A(e[6]);
                    m.conv_silu = int(e[7] & 1);
                    m.y = A(e[4]);
                } else if (flags & GEMVQ_GEMV_ADD) {
                    if (e[0] != GEMVQ_OP_ADD || e[1] != uint32_t(rows) || (e[2] != k[7] && e[3] != k[7]))
                        return reject(i + 1, "ADD epilog");
                    const uint32_t r_off = e[2] == k[7] ? e[3] : e[2];
                    if (!range(r_off, uint64_t(rows)) || !range(e[4], uint64_t(rows))) return reject(i + 1, "ADD epilog range");
                    m.epi = EPI_ADD;
                    m.res = A(r_off);
                    m.y = A(e[4]);
                } else {
                    if (e[0] != GEMVQ_OP_ARGMAX || e[1] != uint32_t(rows) || e[2] != k[7] || !range(e[3], 2))
                        return reject(i + 1, "ARGMAX epilog");
                    if (a.n_members != 0) return reject(i, "ARGMAX epilog must be on the first GEMV of a group");
                    a.argmax_key = reinterpret_cast<unsigned long long *>(A(e[3]));
                }
                step = 2;
            }
            a.wbound[a.n_members] = wb;
            a.m[a.n_members++] = m;
            tasks += rows;
            gemvs += (flags & GEMVQ_GEMV_SWIGLU) ? 2 : 1;
            i += step;
            W.insert(W.end(), mw.begin(), mw.end());
            R.insert(R.end(), mr.begin(), mr.end());
            // a group ends after a GEMV whose output (or new conv state) overlaps x (gemvqc16.cpp:468-474)
            if (meet_any(mw, {{x_off, uint64_t(x_off) + cols}})) break;
        }
        if (a.n_members == 0) return reject(i0, "GEMV");
        a.cols = int(cols);
        a.total_tasks = tasks;
        a.x = A(x_off);
        a.xsrc = XSRC_RAW;
        if (gated.on) {  // the group right after the GDN whose output it reads (checked when the GDN compiled)
            a.xsrc = XSRC_GATED;
            a.x = c->gdn_raw;
            a.gate_z = gated.z;
            a.norm_w = gated.w;
            a.norm_eps = gated.eps;
            a.x_out = A(gated.y);
            a.gate_silu = gated.z_silu;
            gated.on = false;
        } else if (defer.on && defer.y == x_off && defer.n == cols) {
            // every workgroup reads the norm's row and weight in its prologue while others store rows: with a member
            // writing over them, or after an earlier command did, the launch reads the snapshot instead
            if (!defer.snap && defer.dirty >= 0) snapshot_defer(size_t(defer.dirty), int(i0));
            else if (!defer.snap && meet_any(W, defer_ranges())) snapshot_defer(out.size(), int(i0));
            if (defer.snap) {
                a.x = c->dsnap;
            } else {
                a.xsrc = XSRC_NORM;
                a.x = A(defer.x);
                a.norm_w = (defer.flags & GEMVQ_NORM_NO_WEIGHT) ? nullptr : A(defer.w);
                a.norm_eps = defer.eps;
                a.norm_l2 = int(defer.flags & GEMVQ_NORM_L2);
            }
        } else if (meet_any(W, {{x_off, uint64_t(x_off) + cols}})) {
            // a member writes over x while other workgroups still read it: the launch reads a copy taken before
            EwArgs cp{A(x_off), nullptr, c->xsnap, int(cols), 0, 0, EW_COPY, 0.0f};
            out.push_back(LEw{cp});
            spans.push_back({int(i0), 1});
            a.x = c->xsnap;
        }
        if (c->dbg_dst && !c->dbg_used && ref()) return reject(i0, "debug block sums are not written in the reference arithmetic");
        if (c->dbg_dst && !c->dbg_used) {
            const Weight * w0 = &c->weights[uint64_t(cmds[size_t(i0) * GEMVQ_CMD_WORDS + 4]) |
                                            (uint64_t(cmds[size_t(i0) * GEMVQ_CMD_WORDS + 5]) << 32)];
            const size_t need = (type == T_Q5_K || type == T_Q6_K) ? size_t(w0->rows) * (cols / 256) * 2
                                                                   : size_t(w0->rows) * (cols / 32);
            if (need > c->dbg_n) return reject(i0, "debug block-sum buffer too small for this GEMV");
            a.dbg = c->dbg;
            c->dbg_used = true;
        }
        out.push_back(LGemv{a, type, ref()});
        spans.push_back({int(i0), int(i - i0)});
        used = i - i0;
        return true;
    }
};

// Kernel name (template instance) and algorithmic bytes of a launch: GGUF-sized weights, fp32 vectors read and
// written once, recurrent state and KV cache read and written. `pos` is the token position (attention reads
// pos + 1 cached keys and values).
std::pair<std::string, uint64_t> describe(const Launch & l, int pos) {
    if (auto * g = std::get_if<LGemv>(&l)) {
        const GemvArgs & a = g->a;
        const bool kq = g->type == T_Q5_K || g->type == T_Q6_K;
        const int nu = (a.cols / (kq ? 64 : 32) + 63) / 64;
        uint64_t b = uint64_t(a.cols) * 4 * (a.xsrc == XSRC_GATED ? 3 : a.xsrc == XSRC_NORM && a.norm_w ? 2 : 1);
        for (int i = 0; i < a.n_members; ++i) {
            const GemvMember & m = a.m[i];
            const uint64_t rows = uint64_t(m.rows);
            b += rows * gguf_row_bytes(g->type, a.cols) * (m.epi == EPI_SWIGLU ? 2 : 1) + rows * 4;
            if (m.epi == EPI_ADD) b += rows * 4;
            if (m.epi == EPI_CONV) b += rows * 40;
        }
        return {std::string(g->ref ? "gemv_ref_kernel<" : "gemv_kernel<") + std::to_string(g->type) + "," + std::to_string(nu) + ">", b};
    }
    if (auto * x = std::get_if<LNorm>(&l))
        return {x->ref ? "norm_ref_kernel" : "norm_kernel", uint64_t(x->a.n) * x->a.rows * 8 + (x->a.w ? uint64_t(x->a.n) * 4 : 0)};
    if (auto * x = std::get_if<LEw>(&l))
        return {x->ref ? "ew_ref_kernel" : "ew_kernel", uint64_t(x->a.n) * 4 * (x->a.op == EW_FILL ? 1 : x->a.b ? 3 : 2)};
    if (auto * x = std::get_if<LConv>(&l))
        return {x->ref ? "conv_ref_kernel" : "conv_kernel", uint64_t(x->a.ch) * (40 + 8 * (x->ref ? 1 : x->a.n_tok))};
    if (auto * x = std::get_if<LRope>(&l))
        return {"rope_kernel", uint64_t(x->a.ne0) * x->a.rows * 8 + uint64_t(x->a.n_dims) * 4};
    if (auto * x = std::get_if<LGdn>(&l)) {
        const uint64_t hv = uint64_t(x->a.hv), hk = uint64_t(x->a.hk);
        return {x->ref ? "gdn_ref_kernel" : "gdn_kernel",
                2 * hv * 128 * 128 * 4 + ((2 * hk + 2 * hv) * 128 * 4 + hv * 16) * uint64_t(x->ref ? 1 : x->a.n_tok)};
    }
    if (auto * x = std::get_if<LGated>(&l))
        return {"gated_norm_kernel", uint64_t(x->a.heads) * 128 * 12 + 512};
    if (auto * x = std::get_if<LGdnOut>(&l)) {
        const GdnOutArgs & o = x->a;
        const uint64_t hv = uint64_t(o.g.hv), hk = uint64_t(o.g.hk), rows = uint64_t(o.rows);
        const uint64_t state = 2 * hv * 128 * 128 * 4, vec = (2 * hk + 3 * hv) * 128 * 4 + 512 + hv * 16;
        return {"gdn_out_kernel<" + std::to_string(x->type) + ">",
                state + vec + rows * gguf_row_bytes(x->type, int(hv * 128)) + rows * 8};
    }
    if (auto * x = std::get_if<LAttn>(&l)) {
        const AttnArgs & a = x->a;
        const uint64_t nt = uint64_t(a.n_tok > 1 && !x->ref ? a.n_tok : 1);  // token t reads positions 0 .. pos + t
        const uint64_t kv = (uint64_t(pos + 1) * nt + nt * (nt - 1) / 2) * a.n_head_kv * a.head_dim * 2 * 2;
        const uint64_t vec = (uint64_t(a.n_head) * a.head_dim * 4 * (a.gate ? 3 : 2) + uint64_t(a.n_head_kv) * a.head_dim * 8) * nt;
        return {x->ref ? "attn_ref_kernel" : "attn_kernel", kv + vec};
    }
    if (auto * x = std::get_if<LRows>(&l))
        return {"get_rows_kernel", uint64_t(x->a.cols) * 4 + gguf_row_bytes(x->a.type, x->a.cols)};
    if (auto * x = std::get_if<LArgmax>(&l)) return {"argmax_kernel", uint64_t(x->n) * 4 * uint64_t(x->rows)};
    if (auto * x = std::get_if<LGemmQ>(&l)) {
        const GemmQuantArgs & a = x->a;
        return {"gemm_quant_kernel", uint64_t(a.n_tok) * a.cols * (4 + 1) + uint64_t(a.n_tok) * (a.cols / 32) * 4 +
                                         (a.norm_w ? uint64_t(a.cols) * 4 : 0)};
    }
    if (auto * x = std::get_if<LGemm>(&l)) {
        const GemmArgs & a = x->a;
        uint64_t w = uint64_t(a.rows) * gguf_row_bytes(x->type, a.cols) * (a.epi == EPI_SWIGLU ? 2 : 1);
        uint64_t out = uint64_t(a.n_tok) * a.rows * 4 * (a.epi == EPI_ADD ? 2 : 1);
        for (int m = 0; m < a.n_more; ++m) {
            w += uint64_t(a.more[m].rows) * gguf_row_bytes(x->type, a.cols);
            out += uint64_t(a.n_tok) * a.more[m].rows * 4 * (a.more[m].epi == EPI_ADD ? 2 : 1);
        }
        const uint64_t act = uint64_t(a.n_tok) * (a.cols + (a.cols / 32) * 4);
        return {"gemm_kernel<" + std::to_string(x->type) + ">", w + act + out};
    }
    if (auto * x = std::get_if<LTok>(&l)) {
        const TokArgs & a = x->a;
        uint64_t w = 0, out = 0;
        for (int m = 0; m < a.n_members; ++m) {
            w += uint64_t(a.m[m].rows) * gguf_row_bytes(x->type, a.cols) * (a.m[m].epi == EPI_SWIGLU ? 2 : 1);
            out += uint64_t(a.n_tok) * a.m[m].rows * 4 * (a.m[m].epi == EPI_ADD ? 2 : 1);
        }
        const uint64_t act = uint64_t(a.n_tok) * a.cols * 4 + (a.norm_w ? uint64_t(a.cols) * 4 : 0);
        return {"gemv_tok_kernel<" + std::to_string(x->type) + "," + std::to_string(a.n_tok) + ">", w + act + out};
    }
    return {"next_token_kernel", 32};
}

hipError_t issue(const std::vector<Launch> & ls, hipStream_t s) {
    for (const Launch & l : ls) {
        hipError_t e = hipSuccess;
        if (auto * g = std::get_if<LGemv>(&l)) e = g->ref ? launch_gemv_ref(g->a, g->type, s) : launch_gemv(g->a, g->type, s);
        else if (auto * x = std::get_if<LNorm>(&l)) e = x->ref ? launch_norm_ref(x->a, s) : launch_norm(x->a, s);
        else if (auto * x = std::get_if<LEw>(&l)) e = x->ref ? launch_ew_ref(x->a, s) : launch_ew(x->a, s);
        else if (auto * x = std::get_if<LConv>(&l)) e = x->ref ? launch_conv_ref(x->a, x->tok, s) : launch_conv(x->a, s);
        else if (auto * x = std::get_if<LRope>(&l)) e = launch_rope(x->a, s);
        else if (auto * x = std::get_if<LGdn>(&l)) e = x->ref ? launch_gdn_ref(x->a, x->tok, s) : launch_gdn(x->a, s);
        else if (auto * x = std::get_if<LGated>(&l)) e = launch_gated_norm(x->a, s);
        else if (auto * x = std::get_if<LAttn>(&l)) e = x->ref ? launch_attn_ref(x->a, x->tok, s) : launch_attn(x->a, s);
        else if (auto * x = std::get_if<LRows>(&l)) e = launch_get_rows(x->a, s);
        else if (auto * x = std::get_if<LArgmax>(&l)) e = launch_argmax(x->x, x->n, x->key, x->rows, x->stride, s);
        else if (auto * x = std::get_if<LNext>(&l)) e = launch_next_token(x->a, s);
        else if (auto * x = std::get_if<LGemmQ>(&l)) e = launch_gemm_quant(x->a, s);
        else if (auto * x = std::get_if<LGemm>(&l)) e = launch_gemm(x->a, x->type, s);
        else if (auto * x = std::get_if<LGdnOut>(&l)) e = launch_gdn_out(x->a, x->type, s);
        else if (auto * x = std::get_if<LTok>(&l)) e = launch_gemv_tok(x->a, x->type, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int compile_list(gemvq_ctx * c, const uint32_t * cmds, unsigned n, std::vector<Launch> & out,
                 std::vector<std::pair<int, int>> * spans = nullptr) {
    if (n > GEMVQ_MAX_CMDS) {
        c->err = "command list too long";
        return int(GEMVQ_MAX_CMDS) + 1;
    }
    Compiler cp{c, {}, {}, 0, {}};
    if (!cp.compile(cmds, n)) {
        c->err = cp.why;
        return cp.bad;
    }
    out = std::move(cp.out);
    if (spans) *spans = std::move(cp.spans);
    c->last_launches = int(out.size());
    return 0;
}

}  // namespace

extern "C" {

gemvq_ctx * gemvq_ctx_create(int device, size_t act_floats, size_t weight_bytes, size_t state_rows) {
    unsigned wait_ms = 180000;  // GEMVQ_WAIT_TIMEOUT_MS (ggml-xrt.cpp:69-78's GGML_XRT_WAIT_TIMEOUT_MS)
    if (const char * v = std::getenv("GEMVQ_WAIT_TIMEOUT_MS")) {
        char * end = nullptr;
        const unsigned long ms = std::strtoul(v, &end, 10);
        if (end == v || *end != '\0' || ms == 0 || ms > 0xffffffffUL) {
            g_create_error = "gemvq_ctx_create: GEMVQ_WAIT_TIMEOUT_MS must be a positive integer";
            return nullptr;
        }
        wait_ms = unsigned(ms);
    }
    // the bound of the fused DeltaNet launch's in-kernel wait for its heads, in polls of at least a microsecond: 1000
    // per millisecond of the wait bound, at most 2^22 (seconds, against the microseconds the heads take); or
    // GEMVQ_EXCHANGE_POLLS (0 makes every such wait fail at once, which tests use to reach the failure path)
    unsigned polls = wait_ms >= 4194u ? 4194304u : wait_ms * 1000u;
    if (const char * v = std::getenv("GEMVQ_EXCHANGE_POLLS")) {
        char * end = nullptr;
        const unsigned long p = std::strtoul(v, &end, 10);
        if (end == v || *end != '\0' || p > 0xffffffffUL) {
            g_create_error = "gemvq_ctx_create: GEMVQ_EXCHANGE_POLLS must be a non-negative integer";
            return nullptr;
        }
        polls = unsigned(p);
    }
    auto * c = new gemvq_ctx();
    c->device = device;
    c->wait_ms = wait_ms;
    c->xch_polls = polls;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&c->act, std::max<size_t>(act_floats, 16) * sizeof(float));
    if (e == hipSuccess) e = hipMemset(c->act, 0, std::max<size_t>(act_floats, 16) * sizeof(float));
    if (e == hipSuccess && weight_bytes) e = hipMalloc(&c->warena, weight_bytes);
    if (e == hipSuccess && state_rows) e = hipMalloc(&c->state, state_rows * 128 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->gdn_raw, size_t(GDN_MAX_HEADS) * 128 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->dsnap, size_t(GEMV_MAXK) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->xsnap, size_t(GEMV_MAXK) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->gdn_xch, size_t(GDN_XCH_WORDS) * 8);
    if (e == hipSuccess) e = hipMemset(c->gdn_xch, 0, size_t(GDN_XCH_WORDS) * 8);
    if (e == hipSuccess) e = hipHostMalloc(&c->gdn_fault, sizeof(uint32_t), hipHostMallocCoherent);
    if (e == hipSuccess) *c->gdn_fault = 0;
    if (e == hipSuccess) e = hipMalloc(&c->gemm_q, size_t(GEMM_MAX_TOK) * GEMV_MAXK);
    if (e == hipSuccess) e = hipMalloc(&c->gemm_d, size_t(GEMM_MAX_TOK) * (GEMV_MAXK / 32) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->gemm_s, size_t(GEMM_MAX_TOK) * (GEMV_MAXK / 32) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->ref_x, size_t(GEMM_MAX_TOK + 1) * GEMV_MAXK * sizeof(float));
    if (e == hipSuccess && state_rows) e = hipMemset(c->state, 0, state_rows * 128 * sizeof(float));
    if (e != hipSuccess) {
        g_create_error = std::string("gemvq_ctx_create: ") + hipGetErrorString(e);
        gemvq_ctx_destroy(c);
        return nullptr;
    }
    c->act_floats = act_floats;
    c->wbytes = weight_bytes;
    c->state_rows = state_rows;
    return c;
}

void gemvq_ctx_destroy(gemvq_ctx * c) {
    if (!c) return;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    for (auto g : c->graphs)
        if (g) hipGraphExecDestroy(g);
    for (auto g : c->graph_defs)
        if (g) hipGraphDestroy(g);
    for (auto & b : c->kvs) {
        hipFree(b.k);
        hipFree(b.v);
        hipFree(b.part);
        hipFree(b.counter);
        hipFree(b.qr);
    }
    hipFree(c->act);
    hipFree(c->warena);
    hipFree(c->state);
    hipFree(c->gdn_raw);
    hipFree(c->dsnap);
    hipFree(c->xsnap);
    hipFree(c->gdn_xch);
    if (c->gdn_fault) hipHostFree(c->gdn_fault);
    hipFree(c->gemm_q);
    hipFree(c->gemm_d);
    hipFree(c->gemm_s);
    hipFree(c->ref_x);
    hipFree(c->dbg);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

const char * gemvq_last_error(const gemvq_ctx * c) { return c ? c->err.c_str() : g_create_error.c_str(); }

// Internal (not part of the public ABI): lets the model driver report its own errors through gemvq_last_error.
__attribute__((visibility("hidden"))) void gq_set_error(gemvq_ctx * c, const char * what) {
    if (c) c->err = what;
}

int gemvq_device_memory(int device, size_t * free_bytes, size_t * total_bytes) {
    size_t f = 0, t = 0;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipMemGetInfo(&f, &t);
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return e == hipSuccess ? 0 : -int(e);
}

void gemvq_features(gemvq_ctx *, uint32_t out[2]) {
    out[0] = GEMVQ_FEATURES;
    out[1] = GEMVQ_FEATURES2;
}

int gemvq_repack(int type, int rows, int cols, const void * gguf_rows, void * dst) {
    if (!type_ok(type) || !shape_ok(type, rows, cols) || !gguf_rows || !dst) return GEMVQ_EINVAL;
    repack_rows(type, rows, cols, static_cast<const uint8_t *>(gguf_rows), static_cast<uint8_t *>(dst), false);
    return 0;
}

int gemvq_unpack(int type, int rows, int cols, const void * packed, void * gguf_rows) {
    if (!type_ok(type) || !shape_ok(type, rows, cols) || !gguf_rows || !packed) return GEMVQ_EINVAL;
    repack_rows(type, rows, cols, static_cast<uint8_t *>(gguf_rows), const_cast<uint8_t *>(static_cast<const uint8_t *>(packed)),
                true);
    return 0;
}

int gemvq_upload_weight(gemvq_ctx * c, int type, int rows, int cols, const void * gguf_rows, uint64_t * w_off) {
    if (!c || !w_off || !gguf_rows) return einval(c, "gemvq_upload_weight: null argument");
    if (!c->usable) return unusable(c);
    if (!type_ok(type) || !shape_ok(type, rows, cols)) return einval(c, "gemvq_upload_weight: unsupported type or shape");
    const size_t bytes = gguf_row_bytes(type, cols) * size_t(rows);
    const size_t off = (c->wused + 255) & ~size_t(255);
    if (off + bytes > c->wbytes) return einval(c, "gemvq_upload_weight: weight arena full");
    hipSetDevice(c->device);
    void * host = nullptr;
    hipError_t e = hipHostMalloc(&host, bytes, hipHostMallocDefault);
    if (e != hipSuccess) return fail(c, e, "hipHostMalloc");
    repack_rows(type, rows, cols, static_cast<const uint8_t *>(gguf_rows), static_cast<uint8_t *>(host), false);
    e = hipMemcpyAsync(c->warena + off, host, bytes, hipMemcpyHostToDevice, c->stream);
    const int ws = e == hipSuccess ? wait_stream(c, "weight upload") : fail(c, e, "weight upload");
    if (ws == 0 || ws == GEMVQ_ETIMEDOUT) hipHostFree(host);  // a failed stream may still read it: kept
    if (ws) return ws;
    c->weights[off] = Weight{type, rows, cols, bytes, weight_bound(type, rows, cols, static_cast<const uint8_t *>(gguf_rows))};
    c->wused = off + bytes;
    *w_off = off;
    return 0;
}

uint64_t gemvq_weight_bytes_used(const gemvq_ctx * c) { return c ? c->wused : 0; }

int gemvq_act_write(gemvq_ctx * c, size_t off, const void * src, size_t n) {
    if (!c || !src || off + n > c->act_floats) return einval(c, "gemvq_act_write: range");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    if (const int w = drain(c, "act write")) return w;
    hipError_t e = hipMemcpyAsync(c->act + off, src, n * 4, hipMemcpyHostToDevice, c->stream);
    return e == hipSuccess ? wait_stream(c, "act write") : fail(c, e, "act write");
}

int gemvq_act_read(gemvq_ctx * c, size_t off, void * dst, size_t n) {
    if (!c || !dst || off + n > c->act_floats) return einval(c, "gemvq_act_read: range");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    if (const int w = drain(c, "act read")) return w;
    hipError_t e = hipMemcpyAsync(dst, c->act + off, n * 4, hipMemcpyDeviceToHost, c->stream);
    return e == hipSuccess ? wait_stream(c, "act read") : fail(c, e, "act read");
}

int gemvq_state_write(gemvq_ctx * c, size_t row, const float * src, size_t rows) {
    if (!c || !src || row + rows > c->state_rows) return einval(c, "gemvq_state_write: range");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    if (const int w = drain(c, "state write")) return w;
    hipError_t e = hipMemcpyAsync(c->state + row * 128, src, rows * 512, hipMemcpyHostToDevice, c->stream);
    return e == hipSuccess ? wait_stream(c, "state write") : fail(c, e, "state write");
}

int gemvq_state_read(gemvq_ctx * c, size_t row, float * dst, size_t rows) {
    if (!c || !dst || row + rows > c->state_rows) return einval(c, "gemvq_state_read: range");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    if (const int w = drain(c, "state read")) return w;
    hipError_t e = hipMemcpyAsync(dst, c->state + row * 128, rows * 512, hipMemcpyDeviceToHost, c->stream);
    return e == hipSuccess ? wait_stream(c, "state read") : fail(c, e, "state read");
}

int gemvq_state_clear(gemvq_ctx * c) {
    if (!c) return GEMVQ_EINVAL;
    if (!c->usable) return unusable(c);
    if (!c->state_rows) return 0;
    hipSetDevice(c->device);
    hipError_t e = hipMemsetAsync(c->state, 0, c->state_rows * 512, c->stream);
    return e == hipSuccess ? wait_stream(c, "state clear") : fail(c, e, "state clear");
}

int gemvq_kv_create(gemvq_ctx * c, int n_ctx, int n_head_kv, int head_dim) {
    if (!c || n_ctx <= 0 || n_head_kv <= 0 || head_dim <= 0 || head_dim > 256 || head_dim % 16)
        return einval(c, "gemvq_kv_create: shape");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    KvBuf b;
    b.n_ctx = n_ctx;
    b.n_head_kv = n_head_kv;
    b.head_dim = head_dim;
    const size_t kvn = size_t(n_ctx) * n_head_kv * head_dim;
    const size_t nch = size_t(n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    const size_t heads = size_t(ATTN_MAXG) * n_head_kv * GEMM_MAX_TOK;  // (token, q head) sets of a batch
    const size_t partn = heads * nch * (2 + head_dim);
    hipError_t e = hipMalloc(&b.k, kvn * 2);
    if (e == hipSuccess) e = hipMalloc(&b.v, kvn * 2);
    if (e == hipSuccess) e = hipMalloc(&b.part, partn * 4);
    if (e == hipSuccess) e = hipMalloc(&b.counter, heads * 4);
    if (e == hipSuccess) e = hipMalloc(&b.qr, heads * head_dim * 4);
    if (e == hipSuccess) e = hipMemset(b.k, 0, kvn * 2);
    if (e == hipSuccess) e = hipMemset(b.v, 0, kvn * 2);
    if (e == hipSuccess) e = hipMemset(b.counter, 0, heads * 4);
    if (e != hipSuccess) {
        hipFree(b.k);
        hipFree(b.v);
        hipFree(b.part);
        hipFree(b.counter);
        hipFree(b.qr);
        return fail(c, e, "kv create");
    }
    c->kvs.push_back(b);
    return int(c->kvs.size()) - 1;
}

int gemvq_kv_read(gemvq_ctx * c, int kv, int pos0, int npos, uint16_t * k, uint16_t * v) {
    if (!c || kv < 0 || size_t(kv) >= c->kvs.size()) return einval(c, "gemvq_kv_read: buffer");
    if (!c->usable) return unusable(c);
    const KvBuf & b = c->kvs[kv];
    if (pos0 < 0 || npos < 0 || pos0 + npos > b.n_ctx) return einval(c, "gemvq_kv_read: range");
    hipSetDevice(c->device);
    const size_t row = size_t(b.n_head_kv) * b.head_dim, off = size_t(pos0) * row, n = size_t(npos) * row;
    if (const int w = drain(c, "kv read")) return w;
    hipError_t e = hipSuccess;
    if (k) e = hipMemcpyAsync(k, b.k + off, n * 2, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && v) e = hipMemcpyAsync(v, b.v + off, n * 2, hipMemcpyDeviceToHost, c->stream);
    return e == hipSuccess ? wait_stream(c, "kv read") : fail(c, e, "kv read");
}

int gemvq_kv_clear(gemvq_ctx * c) {
    if (!c) return GEMVQ_EINVAL;
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    hipError_t e = hipSuccess;
    for (auto & b : c->kvs) {
        const size_t kvn = size_t(b.n_ctx) * b.n_head_kv * b.head_dim;
        if (e == hipSuccess) e = hipMemsetAsync(b.k, 0, kvn * 2, c->stream);
        if (e == hipSuccess) e = hipMemsetAsync(b.v, 0, kvn * 2, c->stream);
        const size_t heads = size_t(ATTN_MAXG) * b.n_head_kv * GEMM_MAX_TOK;  // every (token, q head) set, as created
        if (e == hipSuccess) e = hipMemsetAsync(b.counter, 0, heads * 4, c->stream);
    }
    return e == hipSuccess ? wait_stream(c, "kv clear") : fail(c, e, "kv clear");
}

int gemvq_run(gemvq_ctx * c, const uint32_t * cmds, unsigned n) {
    if (!c || (n && !cmds)) return einval(c, "gemvq_run: null argument");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    if (n == 0) {  // feature probe (gemvqc16.cpp:1076-1082)
        const uint32_t f[2] = {GEMVQ_FEATURES, GEMVQ_FEATURES2};
        return gemvq_act_write(c, 0, f, 2);
    }
    std::vector<Launch> ls;
    c->dbg_used = false;
    const int st = compile_list(c, cmds, n, ls);
    if (st) {
        c->dbg_used = false;
        return st;
    }
    hipError_t e = issue(ls, c->stream);
    if (e != hipSuccess) return fail(c, e, "run");
    const int ws = wait_stream(c, "run");
    if (ws) return ws;
    if (c->dbg_used) {
        e = hipMemcpy(c->dbg_dst, c->dbg, c->dbg_n * 4, hipMemcpyDeviceToHost);
        c->dbg_dst = nullptr;
        c->dbg_used = false;
    }
    return e == hipSuccess ? 0 : fail(c, e, "run");
}

int gemvq_graph_create(gemvq_ctx * c, const uint32_t * cmds, unsigned n, int * graph) {
    if (!c || !cmds || !graph || n == 0) return einval(c, "gemvq_graph_create: arguments");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    std::vector<Launch> ls;
    int32_t * const armed = c->dbg_dst;
    c->dbg_dst = nullptr;  // block-sum dumps are for gemvq_run only
    const int st = compile_list(c, cmds, n, ls);
    c->dbg_dst = armed;
    c->dbg_used = false;
    if (st) return st;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(c, e, "begin capture");
    hipError_t le = issue(ls, c->stream);
    e = hipStreamEndCapture(c->stream, &g);
    if (le != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return fail(c, le, "launch during capture");
    }
    if (e != hipSuccess) return fail(c, e, "end capture");
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g);
        return fail(c, e, "graph instantiate");
    }
    c->graphs.push_back(ge);
    c->graph_defs.push_back(g);
    *graph = int(c->graphs.size()) - 1;
    return 0;
}

int gemvq_graph_replay(gemvq_ctx * c, int graph, int times) {
    if (!c || graph < 0 || size_t(graph) >= c->graphs.size() || !c->graphs[graph] || times < 0)
        return einval(c, "gemvq_graph_replay: graph");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    for (int t = 0; t < times; ++t) {
        const hipError_t e = hipGraphLaunch(c->graphs[graph], c->stream);
        if (e != hipSuccess) return fail(c, e, "graph launch");
    }
    return 0;
}

int gemvq_graph_destroy(gemvq_ctx * c, int graph) {
    if (!c || graph < 0 || size_t(graph) >= c->graphs.size()) return einval(c, "gemvq_graph_destroy: graph");
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    if (c->graphs[graph]) hipGraphExecDestroy(c->graphs[graph]);
    if (c->graph_defs[graph]) hipGraphDestroy(c->graph_defs[graph]);
    c->graphs[graph] = nullptr;
    c->graph_defs[graph] = nullptr;
    return 0;
}

int gemvq_sync(gemvq_ctx * c) {
    if (!c) return GEMVQ_EINVAL;
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    return wait_stream(c, "sync");
}

int gemvq_set_wait_timeout(gemvq_ctx * c, unsigned ms) {
    if (!c || ms == 0) return einval(c, "gemvq_set_wait_timeout: a positive number of milliseconds");
    c->wait_ms = ms;
    return 0;
}

int gemvq_usable(const gemvq_ctx * c) { return c && c->usable ? 1 : 0; }

int gemvq_last_launch_count(const gemvq_ctx * c) { return c ? c->last_launches : -1; }

int gemvq_set_arith(gemvq_ctx * c, int arith) {
    if (!c || (arith != GEMVQ_ARITH_CANONICAL && arith != GEMVQ_ARITH_REFERENCE)) return einval(c, "gemvq_set_arith: mode");
    c->arith = arith;
    return 0;
}

int gemvq_arith(const gemvq_ctx * c) { return c ? c->arith : GEMVQ_EINVAL; }

float gemvq_cr_expf(float x) { return cr::expf(x); }
float gemvq_cr_logf(float x) { return cr::logf(x); }

int gemvq_crmath_hash(gemvq_ctx * c, int fn, uint64_t * hashes) {
    if (!c || !hashes || (fn != 0 && fn != 1)) return einval(c, "gemvq_crmath_hash: arguments");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    unsigned long long * d = nullptr;
    hipError_t e = hipMalloc(&d, 4096 * 8);
    if (e != hipSuccess) return fail(c, e, "crmath hash");
    e = launch_crmath_hash(fn, d, c->stream);
    if (e != hipSuccess) {
        hipFree(d);
        return fail(c, e, "crmath hash");
    }
    int st = wait_stream(c, "crmath hash");
    if (!st) {
        e = hipMemcpy(hashes, d, 4096 * 8, hipMemcpyDeviceToHost);
        if (e != hipSuccess) st = fail(c, e, "crmath hash copy");
    }
    hipFree(d);
    return st;
}

int gemvq_debug_blocksums(gemvq_ctx * c, int32_t * dst, size_t n) {
    if (!c || !dst || n == 0) return einval(c, "gemvq_debug_blocksums: arguments");
    hipSetDevice(c->device);
    hipFree(c->dbg);
    hipError_t e = hipMalloc(&c->dbg, n * 4);
    if (e != hipSuccess) return fail(c, e, "debug buffer");
    c->dbg_n = n;
    c->dbg_dst = dst;
    c->dbg_used = false;
    return 0;
}

int gemvq_graph_time(gemvq_ctx * c, int graph, int times, double * us) {
    if (!c || !us || times <= 0 || graph < 0 || size_t(graph) >= c->graphs.size() || !c->graphs[graph])
        return einval(c, "gemvq_graph_time: arguments");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    hipError_t e = hipEventRecord(a, c->stream);
    for (int t = 0; t < times && e == hipSuccess; ++t) e = hipGraphLaunch(c->graphs[graph], c->stream);
    if (e == hipSuccess) e = hipEventRecord(b, c->stream);
    const int ws = e == hipSuccess ? wait_stream(c, "graph time") : fail(c, e, "graph time");
    float ms = 0.0f;
    if (ws == 0) e = hipEventElapsedTime(&ms, a, b);
    hipEventDestroy(a);
    hipEventDestroy(b);
    if (ws) return ws;
    if (e != hipSuccess) return fail(c, e, "graph time");
    *us = double(ms) * 1000.0 / times;
    return 0;
}

int gemvq_profile(gemvq_ctx * c, const uint32_t * cmds, unsigned n, int reps, gemvq_launch_stat * out, int max_out) {
    if (!c || !cmds || n == 0 || reps <= 0) return einval(c, "gemvq_profile: arguments");
    if (!c->usable) return unusable(c);
    hipSetDevice(c->device);
    std::vector<Launch> ls;
    std::vector<std::pair<int, int>> spans;
    const int st = compile_list(c, cmds, n, ls, &spans);
    if (st) return st;
    // the token position (attention bytes depend on it): the first ATTN's pos operand
    int pos = 0;
    for (const Launch & l : ls)
        if (auto * x = std::get_if<LAttn>(&l)) {
            hipMemcpy(&pos, x->a.pos, 4, hipMemcpyDeviceToHost);
            break;
        }
    const size_t L = ls.size();
    std::vector<hipEvent_t> e0(L), e1(L);
    std::vector<std::vector<float>> ms_of(L);  // per launch, one duration per repetition
    hipError_t e = hipSuccess;
    int ws = 0;
    for (size_t i = 0; i < L && e == hipSuccess; ++i) {
        e = hipEventCreate(&e0[i]);
        if (e == hipSuccess) e = hipEventCreate(&e1[i]);
    }
    for (int r = 0; r < reps && e == hipSuccess && ws == 0; ++r) {
        for (size_t i = 0; i < L && e == hipSuccess; ++i) {
            g_prof_start = e0[i];
            g_prof_stop = e1[i];
            e = issue({ls[i]}, c->stream);
        }
        g_prof_start = g_prof_stop = nullptr;
        if (e == hipSuccess) ws = wait_stream(c, "profile");
        if (ws) break;
        for (size_t i = 0; i < L && e == hipSuccess; ++i) {
            float ms = 0.0f;
            e = hipEventElapsedTime(&ms, e0[i], e1[i]);
            ms_of[i].push_back(ms);
        }
    }
    g_prof_start = g_prof_stop = nullptr;
    for (size_t i = 0; i < L; ++i) {
        if (e0[i]) hipEventDestroy(e0[i]);
        if (e1[i]) hipEventDestroy(e1[i]);
    }
    if (ws) return ws;
    if (e != hipSuccess) return fail(c, e, "profile");
    for (size_t i = 0; i < L && int(i) < max_out; ++i) {
        const auto d = describe(ls[i], pos);
        gemvq_launch_stat & o = out[i];
        std::memset(&o, 0, sizeof(o));
        std::strncpy(o.name, d.first.c_str(), sizeof(o.name) - 1);
        o.first_cmd = spans[i].first;
        o.n_cmds = spans[i].second;
        o.bytes = d.second;
        // the median over the repetitions (a repetition slowed by something outside the launch does not move it)
        std::vector<float> & v = ms_of[i];
        std::sort(v.begin(), v.end());
        const size_t h = v.size() / 2;
        o.us = (v.size() % 2 ? double(v[h]) : 0.5 * (double(v[h - 1]) + double(v[h]))) * 1000.0;
    }
    return int(L);
}

}  // extern "C"
