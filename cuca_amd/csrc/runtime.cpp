// runtime.cpp -- implementation of the C ABI in include/cuca_hip.h.
//
// The kernels are one gfx950 code object (kernels/cuca_kernels.hip) that
// the build embeds into this library (CUCA_CODE_OBJECT, .incbin below).  A
// context loads it with hipModuleLoadData, resolves every kernel once with
// hipModuleGetFunction and launches with hipModuleLaunchKernel, each kernel
// taking one by-value argument block (kernel_args.h).  Host code only: no
// device code is compiled into this file.  The one device variable of the
// library, the allocation-free entry points' scratch array, is defined in
// noalloc.hip; this file takes only its per-device address.
#include "cuca_hip.h"
#include "kernel_args.h"
#include "noalloc.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

// hipExtModuleLaunchKernel (libamdhip64): the module launch whose events
// stamp the kernel's own start and end.  Declared here because hip_ext.h
// also carries device-side templates a host-only C++ compiler cannot parse.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams,
                                               void **extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

#ifndef CUCA_CODE_OBJECT
#error "CUCA_CODE_OBJECT must name the gfx950 code object to embed"
#endif

extern "C" const unsigned char cuca_code_object_start[];
extern "C" const unsigned char cuca_code_object_end[];
__asm__(".section .rodata\n"
        ".global cuca_code_object_start\n"
        ".balign 4096\n"
        "cuca_code_object_start:\n"
        ".incbin \"" CUCA_CODE_OBJECT "\"\n"
        ".global cuca_code_object_end\n"
        "cuca_code_object_end:\n"
        ".previous\n");

namespace {

// Every kernel of the code object, resolved at context creation.
enum Kernel {
#define K(name) name,
#include "kernel_list.inc"
#undef K
    KERNEL_COUNT
};
const char *const kKernelNames[] = {
#define K(name) #name,
#include "kernel_list.inc"
#undef K
};

thread_local std::string g_thread_error;

// The context's scratch for the slices' results of argmax / top-k.
constexpr size_t kPickScratchBytes = 4 << 20;

}  // namespace

struct cuca_hip_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t fn[KERNEL_COUNT] = {};
    unsigned long long *status = nullptr;  // CUCA_STATUS_WORDS device words
    hipEvent_t t0 = nullptr, t1 = nullptr;
    bool capturing = false;
    int64_t last_vocab = 0;       // for the out-of-range message
    int64_t last_kv_blocks = 0;   // the pool size of the last K/V store (for messages)
    int64_t last_table_rows = 0;
    int64_t last_moe_tokens = 0;  // the activation rows of the last MoE up call
    int64_t last_head_rows = 0;   // the vocabulary of the last indexed LM head
    // device scratch for the per-slice results of cuca_hip_argmax / _top_k
    // (allocated with the context: ops never allocate)
    void *pscratch = nullptr;
    // this device's copy of the allocation-free entry points' scratch array
    // (noalloc.hip), resolved at creation; its failure, if any, is reported
    // by those entry points only
    void *noalloc = nullptr;
    std::string noalloc_error;
    int cu_count = 256;
    std::string error;
    // per-kernel timing (cuca_hip_profile_start/stop)
    struct ProfRec { int kernel; hipEvent_t start, stop; };
    std::vector<ProfRec> prof;    // event pairs, created once and reused
    size_t prof_used = 0;
    size_t prof_limit = 0;
    bool profiling = false;
};

struct cuca_hip_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

cuca_status fail(cuca_hip_ctx *ctx, cuca_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->error = buf;
    else g_thread_error = buf;
    return st;
}

cuca_status hip_fail(cuca_hip_ctx *ctx, hipError_t e, const char *what) {
    return fail(ctx, CUCA_HIP_ERROR, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(ctx, call)                                    \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
    } while (0)

// Make the context's device current for the calling thread.
cuca_status use(cuca_hip_ctx *ctx) {
    if (!ctx) return fail(nullptr, CUCA_INVALID_ARG, "null context");
    int cur = -1;
    HIP_TRY(ctx, hipGetDevice(&cur));
    if (cur != ctx->device) HIP_TRY(ctx, hipSetDevice(ctx->device));
    return CUCA_OK;
}

// A grid of grid x grid_y workgroups of `block` threads.
template <typename Args>
cuca_status launch2(cuca_hip_ctx *ctx, Kernel k, unsigned grid, unsigned grid_y, unsigned block, unsigned lds,
                    Args &args) {
    if (grid == 0 || grid_y == 0) return CUCA_OK;
    void *params[] = {&args};
    hipError_t e;
    if (ctx->profiling && !ctx->capturing && ctx->prof_used < ctx->prof_limit) {
        cuca_hip_ctx::ProfRec &r = ctx->prof[ctx->prof_used++];
        r.kernel = k;
        // work sizes in work-items; the events stamp the kernel's own start and end
        e = hipExtModuleLaunchKernel(ctx->fn[k], grid * block, grid_y, 1, block, 1, 1, lds, ctx->stream,
                                     params, nullptr, r.start, r.stop, 0);
    } else {
        e = hipModuleLaunchKernel(ctx->fn[k], grid, grid_y, 1, block, 1, 1, lds, ctx->stream, params,
                                  nullptr);
    }
    if (e != hipSuccess) return fail(ctx, CUCA_HIP_ERROR, "launching %s: %s", kKernelNames[k],
                                     hipGetErrorString(e));
    return CUCA_OK;
}

template <typename Args>
cuca_status launch(cuca_hip_ctx *ctx, Kernel k, unsigned grid, unsigned block, unsigned lds, Args &args) {
    return launch2(ctx, k, grid, 1u, block, lds, args);
}

inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t esize(cuca_dtype t) { return t == CUCA_F16 ? 2 : 4; }
inline bool dtype_ok(cuca_dtype t) { return t == CUCA_F32 || t == CUCA_F16; }
inline int chunk_elems(cuca_dtype t) { return t == CUCA_F16 ? 8 : 4; }
inline unsigned div_up(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }
constexpr unsigned CUCA_BLOCK_THREADS = 256; // every kernel's workgroup size but the norm's

}  // namespace

extern "C" {

const char *cuca_hip_last_error(const cuca_hip_ctx *ctx) {
    return ctx ? ctx->error.c_str() : g_thread_error.c_str();
}

cuca_status cuca_hip_ctx_create(int device, cuca_hip_ctx **out) {
    if (!out) return fail(nullptr, CUCA_INVALID_ARG, "null output pointer");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return fail(nullptr, CUCA_HIP_ERROR, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n)
        return fail(nullptr, CUCA_INVALID_ARG, "device %d outside 0..%d", device, n - 1);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(nullptr, CUCA_HIP_ERROR, "hipGetDeviceProperties: %s",
                                     hipGetErrorString(e));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, CUCA_NOT_GFX950, "device %d is %s; this library is built for gfx950 only",
                    device, prop.gcnArchName);
    cuca_hip_ctx *ctx = new cuca_hip_ctx();
    ctx->device = device;
    cuca_status st = CUCA_OK;
    do {
        if ((e = hipSetDevice(device)) != hipSuccess) { st = hip_fail(ctx, e, "hipSetDevice"); break; }
        // default priority: streams of other priorities are not used anywhere
        if ((e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking)) != hipSuccess) {
            st = hip_fail(ctx, e, "hipStreamCreateWithFlags"); break;
        }
        ctx->stream = ctx->own_stream;
        if ((e = hipModuleLoadData(&ctx->module, cuca_code_object_start)) != hipSuccess) {
            st = hip_fail(ctx, e, "hipModuleLoadData(gfx950 code object)"); break;
        }
        for (int k = 0; k < KERNEL_COUNT; k++) {
            if ((e = hipModuleGetFunction(&ctx->fn[k], ctx->module, kKernelNames[k])) != hipSuccess) {
                st = fail(ctx, CUCA_HIP_ERROR, "kernel %s: %s", kKernelNames[k], hipGetErrorString(e));
                break;
            }
        }
        if (st != CUCA_OK) break;
        ctx->cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
        if ((e = hipMalloc(&ctx->pscratch, kPickScratchBytes)) != hipSuccess) {
            st = hip_fail(ctx, e, "hipMalloc(selection scratch)"); break;
        }
        if ((e = hipMalloc(&ctx->status, CUCA_STATUS_WORDS * sizeof(unsigned long long))) != hipSuccess) {
            st = hip_fail(ctx, e, "hipMalloc(status)"); break;
        }
        unsigned long long ones[CUCA_STATUS_WORDS];
        std::memset(ones, 0xff, sizeof ones);
        if ((e = hipMemcpy(ctx->status, ones, sizeof ones, hipMemcpyHostToDevice)) != hipSuccess) {
            st = hip_fail(ctx, e, "hipMemcpy(status)"); break;
        }
        if ((e = hipEventCreate(&ctx->t0)) != hipSuccess || (e = hipEventCreate(&ctx->t1)) != hipSuccess) {
            st = hip_fail(ctx, e, "hipEventCreate"); break;
        }
        // the device is current: resolve its copy of the allocation-free scratch
        if ((e = cuca_noalloc_scratch(device, &ctx->noalloc)) != hipSuccess) {
            ctx->noalloc = nullptr;
            ctx->noalloc_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            (void)hipGetLastError();
        }
    } while (0);
    if (st != CUCA_OK) {
        g_thread_error = ctx->error;
        cuca_hip_ctx_destroy(ctx);
        return st;
    }
    *out = ctx;
    return CUCA_OK;
}

void cuca_hip_ctx_destroy(cuca_hip_ctx *ctx) {
    if (!ctx) return;
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != ctx->device) (void)hipSetDevice(ctx->device);
    if (ctx->own_stream) (void)hipStreamSynchronize(ctx->own_stream);
    if (ctx->stream && ctx->stream != ctx->own_stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->t0) (void)hipEventDestroy(ctx->t0);
    if (ctx->t1) (void)hipEventDestroy(ctx->t1);
    for (auto &r : ctx->prof) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    if (ctx->status) (void)hipFree(ctx->status);
    if (ctx->pscratch) (void)hipFree(ctx->pscratch);
    if (ctx->module) (void)hipModuleUnload(ctx->module);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

cuca_status cuca_hip_set_stream(cuca_hip_ctx *ctx, void *stream) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (ctx->capturing) return fail(ctx, CUCA_INVALID_ARG, "cannot change the stream during a capture");
    ctx->stream = stream ? static_cast<hipStream_t>(stream) : ctx->own_stream;
    return CUCA_OK;
}

void *cuca_hip_get_stream(const cuca_hip_ctx *ctx) { return ctx ? ctx->stream : nullptr; }

int cuca_hip_device(const cuca_hip_ctx *ctx) { return ctx ? ctx->device : -1; }

cuca_status cuca_hip_malloc(cuca_hip_ctx *ctx, size_t bytes, void **out) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!out) return fail(ctx, CUCA_INVALID_ARG, "null output pointer");
    *out = nullptr;
    if (bytes == 0) return CUCA_OK;
    HIP_TRY(ctx, hipMalloc(out, bytes));
    return CUCA_OK;
}

cuca_status cuca_hip_free(cuca_hip_ctx *ctx, void *ptr) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (ptr) HIP_TRY(ctx, hipFree(ptr));
    return CUCA_OK;
}

static cuca_status copy_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes,
                              hipMemcpyKind kind) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (bytes == 0) return CUCA_OK;
    if (!dst || !src) return fail(ctx, CUCA_INVALID_ARG, "null copy pointer");
    HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
    return CUCA_OK;
}

cuca_status cuca_hip_memcpy_h2d_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_async(ctx, dst, src, bytes, hipMemcpyHostToDevice);
}
cuca_status cuca_hip_memcpy_d2h_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_async(ctx, dst, src, bytes, hipMemcpyDeviceToHost);
}
cuca_status cuca_hip_memcpy_d2d_async(cuca_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_async(ctx, dst, src, bytes, hipMemcpyDeviceToDevice);
}

cuca_status cuca_hip_stream_sync(cuca_hip_ctx *ctx) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return CUCA_OK;
}

cuca_status cuca_hip_check_device(cuca_hip_ctx *ctx) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (ctx->capturing) return fail(ctx, CUCA_INVALID_ARG, "cannot check the device during a capture");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    unsigned long long w[CUCA_STATUS_WORDS];
    HIP_TRY(ctx, hipMemcpy(w, ctx->status, sizeof w, hipMemcpyDeviceToHost));
    const unsigned long long none = ~0ull;
    bool bad = false;
    for (int i = 0; i < CUCA_STATUS_WORDS; i++) bad |= w[i] != none;
    if (!bad) return CUCA_OK;
    unsigned long long ones[CUCA_STATUS_WORDS];
    std::memset(ones, 0xff, sizeof ones);
    HIP_TRY(ctx, hipMemcpy(ctx->status, ones, sizeof ones, hipMemcpyHostToDevice));
    if (w[CUCA_STATUS_EMBED_ID] != none) {
        unsigned long long v = w[CUCA_STATUS_EMBED_ID];
        return fail(ctx, CUCA_OUT_OF_RANGE, "token id %u outside the embedding table of %lld rows (row %u)",
                    (unsigned)(v & 0xffffffffu), (long long)ctx->last_vocab, (unsigned)(v >> 32));
    }
    if (w[CUCA_STATUS_ROPE_POS] != none) {
        unsigned long long v = w[CUCA_STATUS_ROPE_POS];
        return fail(ctx, CUCA_OUT_OF_RANGE, "position %d outside the rope table of %lld rows (row %u)",
                    (int)(v & 0xffffffffu), (long long)ctx->last_table_rows, (unsigned)(v >> 32));
    }
    if (w[CUCA_STATUS_KV_SLOT] != none) {
        unsigned long long v = w[CUCA_STATUS_KV_SLOT];
        return fail(ctx, CUCA_OUT_OF_RANGE, "K/V slot %d outside the pool of %lld blocks (row %u)",
                    (int)(v & 0xffffffffu), (long long)ctx->last_kv_blocks, (unsigned)(v >> 32));
    }
    if (w[CUCA_STATUS_HEAD_ROW] != none) {
        unsigned long long v = w[CUCA_STATUS_HEAD_ROW];
        return fail(ctx, CUCA_OUT_OF_RANGE, "qmm: weight row %u out of range (%lld) (index %u)",
                    (unsigned)(v & 0xffffffffu), (long long)ctx->last_head_rows, (unsigned)(v >> 32));
    }
    if (w[CUCA_STATUS_MOE_PAIR] != none) {
        unsigned long long v = w[CUCA_STATUS_MOE_PAIR];
        return fail(ctx, CUCA_OUT_OF_RANGE, "a routed token (%d) outside the %lld rows (pair %u)",
                    (int)(v & 0xffffffffu), (long long)ctx->last_moe_tokens, (unsigned)(v >> 32));
    }
    unsigned long long v = w[CUCA_STATUS_KV_RANGE];
    if ((v & 0xffffffffu) == 0xffffffffu)
        return fail(ctx, CUCA_OUT_OF_RANGE, "attention row %u: empty key range, or one past its block table",
                    (unsigned)(v >> 32));
    return fail(ctx, CUCA_OUT_OF_RANGE,
                "attention row %u: position %u has no K/V block (it left the window or was never allocated)",
                (unsigned)(v >> 32), (unsigned)(v & 0xffffffffu));
}

// ---------------------------------------------------------------------
// embedding
// ---------------------------------------------------------------------

// mode 0: the gather; 1: with rms_norm_rows (norm_eps); 2: with the first
// block's RMSNorm into h_out (rms_w, rms_eps)
static cuca_status embed_common(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type, int64_t vocab,
                                int64_t hidden, const uint32_t *ids, int64_t n, float scale, int mode,
                                float norm_eps, const float *rms_w, float rms_eps, void *out, void *h_out,
                                cuca_dtype out_dtype) {
    const bool norm = mode == 1;
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (ggml_type != CUCA_GGML_Q4_0 && ggml_type != CUCA_GGML_Q8_0)
        return fail(ctx, CUCA_UNSUPPORTED, "ggml type %u: only Q4_0 (2) and Q8_0 (8) are supported", ggml_type);
    if (!dtype_ok(out_dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad output dtype %d", (int)out_dtype);
    if (hidden <= 0 || hidden % 32 != 0)
        return fail(ctx, CUCA_INVALID_ARG,
                    "token embedding: row length %lld is not a whole number of %s blocks",
                    (long long)hidden, ggml_type == CUCA_GGML_Q4_0 ? "Q4_0" : "Q8_0");
    if (vocab <= 0 || vocab > 0xffffffffll) return fail(ctx, CUCA_INVALID_ARG, "bad vocab %lld", (long long)vocab);
    if (n < 0 || n > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "bad token count %lld", (long long)n);
    if (n == 0) return CUCA_OK;
    if (!table || !ids || !out) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!al16(out)) return fail(ctx, CUCA_INVALID_ARG, "output must be 16-byte aligned");
    const int64_t row_bytes = hidden / 32 * (ggml_type == CUCA_GGML_Q4_0 ? 18 : 34);
    if (hidden > (1 << 28)) return fail(ctx, CUCA_UNSUPPORTED, "hidden size %lld too large", (long long)hidden);
    if (reinterpret_cast<uintptr_t>(table) & 1u) return fail(ctx, CUCA_INVALID_ARG, "table must be 2-byte aligned");
    if (norm && !(norm_eps >= 0.0f)) return fail(ctx, CUCA_INVALID_ARG, "embedding norm eps must be >= 0");
    if (mode == 2) {
        if (!h_out) return fail(ctx, CUCA_INVALID_ARG, "null h_out");
        if (!al16(h_out) || (rms_w && !al16(rms_w)))
            return fail(ctx, CUCA_INVALID_ARG, "h_out and the norm weights must be 16-byte aligned");
        if (!(rms_eps >= 0.0f)) return fail(ctx, CUCA_INVALID_ARG, "eps must be >= 0");
    }
    const bool f16 = out_dtype == CUCA_F16;
    // a wave per token, lane units of 8 values, up to 8 units per lane per round
    const int64_t per_lane = (hidden / 8 + 63) / 64;
    const int ui = per_lane <= 1 ? 0 : per_lane <= 2 ? 1 : per_lane <= 4 ? 2 : 3;
    static const Kernel table_k[3][2][2][4] = {
        {{{cuca_embed_q4_0_f32_u1, cuca_embed_q4_0_f32_u2, cuca_embed_q4_0_f32_u4, cuca_embed_q4_0_f32_u8},
          {cuca_embed_q4_0_f16_u1, cuca_embed_q4_0_f16_u2, cuca_embed_q4_0_f16_u4, cuca_embed_q4_0_f16_u8}},
         {{cuca_embed_q8_0_f32_u1, cuca_embed_q8_0_f32_u2, cuca_embed_q8_0_f32_u4, cuca_embed_q8_0_f32_u8},
          {cuca_embed_q8_0_f16_u1, cuca_embed_q8_0_f16_u2, cuca_embed_q8_0_f16_u4, cuca_embed_q8_0_f16_u8}}},
        {{{cuca_embed_q4_0_f32_norm_u1, cuca_embed_q4_0_f32_norm_u2, cuca_embed_q4_0_f32_norm_u4,
           cuca_embed_q4_0_f32_norm_u8},
          {cuca_embed_q4_0_f16_norm_u1, cuca_embed_q4_0_f16_norm_u2, cuca_embed_q4_0_f16_norm_u4,
           cuca_embed_q4_0_f16_norm_u8}},
         {{cuca_embed_q8_0_f32_norm_u1, cuca_embed_q8_0_f32_norm_u2, cuca_embed_q8_0_f32_norm_u4,
           cuca_embed_q8_0_f32_norm_u8},
          {cuca_embed_q8_0_f16_norm_u1, cuca_embed_q8_0_f16_norm_u2, cuca_embed_q8_0_f16_norm_u4,
           cuca_embed_q8_0_f16_norm_u8}}},
        {{{cuca_embed_q4_0_f32_rms_u1, cuca_embed_q4_0_f32_rms_u2, cuca_embed_q4_0_f32_rms_u4,
           cuca_embed_q4_0_f32_rms_u8},
          {cuca_embed_q4_0_f16_rms_u1, cuca_embed_q4_0_f16_rms_u2, cuca_embed_q4_0_f16_rms_u4,
           cuca_embed_q4_0_f16_rms_u8}},
         {{cuca_embed_q8_0_f32_rms_u1, cuca_embed_q8_0_f32_rms_u2, cuca_embed_q8_0_f32_rms_u4,
           cuca_embed_q8_0_f32_rms_u8},
          {cuca_embed_q8_0_f16_rms_u1, cuca_embed_q8_0_f16_rms_u2, cuca_embed_q8_0_f16_rms_u4,
           cuca_embed_q8_0_f16_rms_u8}}}};
    const Kernel k = table_k[mode][ggml_type == CUCA_GGML_Q8_0][f16][ui];
    // The fused norm with a workgroup per token (TPR threads of one unit, or
    // 1024 of two) up to 8192 tokens: measured in the prefill steps on
    // MI355X, 13.9 against 15.3 us at 4096 tokens of 4096 (Q8_0 -> f16) and
    // 13.4 against 14.7 us at 8192 tokens of 2048 (Q4_0); at 16384 tokens of
    // 4096 the wave-per-token kernel is faster (69 against 76 us).
    int tpr_i = -1, tpr = 0;
    if (mode == 2 && n <= 8192) {
        const int64_t nu = hidden / 8;
        if (nu <= 1024) {
            tpr = 64;
            tpr_i = 0;
            while (tpr < nu) { tpr <<= 1; tpr_i++; }
        } else if (nu <= 2048) {
            tpr = 1024;
            tpr_i = 5;
        }
    }
    static const Kernel table_t[2][2][6] = {
        {{cuca_embed_q4_0_f32_rms_t64, cuca_embed_q4_0_f32_rms_t128, cuca_embed_q4_0_f32_rms_t256,
          cuca_embed_q4_0_f32_rms_t512, cuca_embed_q4_0_f32_rms_t1024, cuca_embed_q4_0_f32_rms_t1024_c2},
         {cuca_embed_q4_0_f16_rms_t64, cuca_embed_q4_0_f16_rms_t128, cuca_embed_q4_0_f16_rms_t256,
          cuca_embed_q4_0_f16_rms_t512, cuca_embed_q4_0_f16_rms_t1024, cuca_embed_q4_0_f16_rms_t1024_c2}},
        {{cuca_embed_q8_0_f32_rms_t64, cuca_embed_q8_0_f32_rms_t128, cuca_embed_q8_0_f32_rms_t256,
          cuca_embed_q8_0_f32_rms_t512, cuca_embed_q8_0_f32_rms_t1024, cuca_embed_q8_0_f32_rms_t1024_c2},
         {cuca_embed_q8_0_f16_rms_t64, cuca_embed_q8_0_f16_rms_t128, cuca_embed_q8_0_f16_rms_t256,
          cuca_embed_q8_0_f16_rms_t512, cuca_embed_q8_0_f16_rms_t1024, cuca_embed_q8_0_f16_rms_t1024_c2}}};
    EmbedArgs a{};
    a.table = static_cast<const uint8_t *>(table);
    a.ids = ids;
    a.out = out;
    a.status = ctx->status;
    a.vocab = vocab;
    a.row_bytes = row_bytes;
    a.hidden = (int32_t)hidden;
    a.n = (int32_t)n;
    a.scale = scale;
    a.norm_eps = norm_eps;
    a.h_out = h_out;
    a.rms_w = rms_w;
    a.rms_eps = rms_eps;
    ctx->last_vocab = vocab;
    // [q8][f16][u2, u4, u8]
    static const Kernel table_l[2][2][3] = {
        {{cuca_embed_q4_0_f32_rms_lds_u2, cuca_embed_q4_0_f32_rms_lds_u4, cuca_embed_q4_0_f32_rms_lds_u8},
         {cuca_embed_q4_0_f16_rms_lds_u2, cuca_embed_q4_0_f16_rms_lds_u4, cuca_embed_q4_0_f16_rms_lds_u8}},
        {{cuca_embed_q8_0_f32_rms_lds_u2, cuca_embed_q8_0_f32_rms_lds_u4, cuca_embed_q8_0_f32_rms_lds_u8},
         {cuca_embed_q8_0_f16_rms_lds_u2, cuca_embed_q8_0_f16_rms_lds_u4, cuca_embed_q8_0_f16_rms_lds_u8}}};
    // Beyond 8192 tokens (rows of up to 512 units per lane round) the fused
    // norm stages its weights in LDS once per workgroup and each wave loops
    // over tpw tokens (about 1024 workgroups, 4 per CU).  Measured in the
    // config C prefill step at 16384 tokens on MI355X: 65.8 us against 72-73
    // for the wave-per-token kernel (tpw 1: 67.6, 2: 67.0, 4: 65.8); at 4096
    // and 8192 tokens it is slower than the workgroup-per-token kernel (18.1
    // against 15.3, 17.1 against 15.5 us), too few tokens per CU to hide
    // the staging.
    // Beyond 8192 tokens, rows of 256 or 512 units (hidden 2048 or 4096) take
    // persistent workgroups of one thread per unit, each workgroup looping
    // over TPW tokens, with a grid the device holds at once (8 waves per
    // SIMD): TPW the smallest of 8, 16, 32 that fits the tokens in that grid.
    // Measured in the config C prefill step at 16384 tokens on MI355X:
    // 61.3-61.6 us against 65.2-65.4 for the LDS-weights kernel below.
    const int64_t nu = hidden / 8;
    if (mode == 2 && n > 8192 && (nu == 256 || nu == 512)) {
        // [q8][f16][tpr 512][tpw 8, 16, 32]
        static const Kernel table_p[2][2][2][3] = {
            {{{cuca_embed_q4_0_f32_rms_p256_w8, cuca_embed_q4_0_f32_rms_p256_w16, cuca_embed_q4_0_f32_rms_p256_w32},
              {cuca_embed_q4_0_f32_rms_p512_w8, cuca_embed_q4_0_f32_rms_p512_w16, cuca_embed_q4_0_f32_rms_p512_w32}},
             {{cuca_embed_q4_0_f16_rms_p256_w8, cuca_embed_q4_0_f16_rms_p256_w16, cuca_embed_q4_0_f16_rms_p256_w32},
              {cuca_embed_q4_0_f16_rms_p512_w8, cuca_embed_q4_0_f16_rms_p512_w16, cuca_embed_q4_0_f16_rms_p512_w32}}},
            {{{cuca_embed_q8_0_f32_rms_p256_w8, cuca_embed_q8_0_f32_rms_p256_w16, cuca_embed_q8_0_f32_rms_p256_w32},
              {cuca_embed_q8_0_f32_rms_p512_w8, cuca_embed_q8_0_f32_rms_p512_w16, cuca_embed_q8_0_f32_rms_p512_w32}},
             {{cuca_embed_q8_0_f16_rms_p256_w8, cuca_embed_q8_0_f16_rms_p256_w16, cuca_embed_q8_0_f16_rms_p256_w32},
              {cuca_embed_q8_0_f16_rms_p512_w8, cuca_embed_q8_0_f16_rms_p512_w16, cuca_embed_q8_0_f16_rms_p512_w32}}}};
        const int tpr = (int)nu;
        const int64_t resident = (int64_t)ctx->cu_count * (2048 / tpr);
        int wi = 0, tpw = 8;
        while (wi < 2 && div_up(n, tpw) > resident) { wi++; tpw <<= 1; }
        return launch(ctx, table_p[ggml_type == CUCA_GGML_Q8_0][f16][tpr == 512][wi], (unsigned)div_up(n, tpw),
                      (unsigned)tpr, 0u, a);
    }
    if (mode == 2 && per_lane <= 8 && n > 8192) {
        const int li = per_lane <= 2 ? 0 : per_lane <= 4 ? 1 : 2;
        a.tpw = (int32_t)std::max<int64_t>(1, std::min<int64_t>(8, n / 4096));
        return launch(ctx, table_l[ggml_type == CUCA_GGML_Q8_0][f16][li], div_up(n, 4 * a.tpw), 256,
                      rms_w ? (unsigned)(hidden * 4) : 0u, a);
    }
    if (tpr_i >= 0)
        return launch(ctx, table_t[ggml_type == CUCA_GGML_Q8_0][f16][tpr_i], (unsigned)n, (unsigned)tpr, 0, a);
    return launch(ctx, k, div_up(n, 4), 256, 0, a); // 4 waves, one token each
}

cuca_status cuca_hip_embed_gguf(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type,
                                int64_t vocab, int64_t hidden, const uint32_t *ids, int64_t n,
                                float scale, void *out, cuca_dtype out_dtype) {
    return embed_common(ctx, table, ggml_type, vocab, hidden, ids, n, scale, 0, 0.0f, nullptr, 0.0f, out,
                        nullptr, out_dtype);
}

cuca_status cuca_hip_embed_gguf_norm(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type,
                                     int64_t vocab, int64_t hidden, const uint32_t *ids, int64_t n,
                                     float scale, float norm_eps, void *out, cuca_dtype out_dtype) {
    return embed_common(ctx, table, ggml_type, vocab, hidden, ids, n, scale, 1, norm_eps, nullptr, 0.0f, out,
                        nullptr, out_dtype);
}

cuca_status cuca_hip_embed_gguf_rms(cuca_hip_ctx *ctx, const void *table, uint32_t ggml_type, int64_t vocab,
                                    int64_t hidden, const uint32_t *ids, int64_t n, float scale, const float *w,
                                    float eps, void *x_out, void *h_out, cuca_dtype out_dtype) {
    return embed_common(ctx, table, ggml_type, vocab, hidden, ids, n, scale, 2, 0.0f, w, eps, x_out, h_out,
                        out_dtype);
}

// ---------------------------------------------------------------------
// residual add + RMSNorm
// ---------------------------------------------------------------------

// Inputs at least this large stream through with nontemporal loads: they
// cannot stay in the 256 MiB last-level cache (MALL) anyway, and streaming
// them keeps it for data that is reused (+5 to +15 % measured at the
// 16384-token shapes; no gain below the cache size).
// Norm and SwiGLU calls whose inputs reach these sizes read them with
// streaming (nontemporal) loads: a prefill-sized op's inputs are read once,
// and left in the caches (L2, the 256 MB MALL) they displace what the next
// kernels read.  Set by measurement on MI355X (five-op prefill steps, f16):
// - at 4096 tokens (norm inputs 64 MiB, SwiGLU 224 MiB) streaming both
//   took the step from 146 to 134 us (SwiGLU 74 -> 81 % of HBM peak, the
//   norms 66 -> 70 %); the thresholds were 256 MiB before;
// - Gemma-2 shapes at 2048 tokens (norm 28 MiB, GeGLU 112 MiB) ran slower
//   streamed (GeGLU 86 -> 76 %, the norms 59 -> 49 %);
// - RoPE, which rewrites its rows in place, ran slower streamed at every
//   size (66 -> 61 % at 4096 tokens); it reads with device-scope loads
//   instead (rope_common), except the prefill-sized QK-norm calls.
static const int64_t kStreamBytes = 48ll << 20;
static const int64_t kGluStreamBytes = 192ll << 20;

// Launch shape of the vector norm kernel for rows of `nch` 16-byte chunks:
// `tpr` threads per row, one chunk each, up to 1024 threads (one row per
// workgroup beyond 64); wider rows give each of 1024 threads 2, 4 or 8
// chunks.  One chunk per thread keeps a row's registers small, lets a
// decode row issue all its loads at once, and measured best at prefill
// (67 % of peak per 4096 f16 rows of 4096, 88 % per 16384, against 44 % and
// 55 % for one wave per row).  Returns false when no vector kernel fits.
static bool norm_shape(int64_t nch, int *tpr, int *per) {
    if (nch <= 1024) {
        int t = 1;
        while (t < nch) t <<= 1;
        *tpr = t;
        *per = 1;
        return true;
    }
    const int64_t need = (nch + 1023) / 1024;
    int p = 2;
    while (p < need) p <<= 1;
    if (p > 8) return false;
    *tpr = 1024;
    *per = p;
    return true;
}

static Kernel norm_kernel(bool f16, int tpr, int per, bool nt) {
    struct E { int tpr, per; bool nt; Kernel k32, k16; };
    static const E table[] = {
        {1, 1, false, cuca_norm_f32_t1, cuca_norm_f16_t1},
        {2, 1, false, cuca_norm_f32_t2, cuca_norm_f16_t2},
        {4, 1, false, cuca_norm_f32_t4, cuca_norm_f16_t4},
        {8, 1, false, cuca_norm_f32_t8, cuca_norm_f16_t8},
        {16, 1, false, cuca_norm_f32_t16, cuca_norm_f16_t16},
        {32, 1, false, cuca_norm_f32_t32, cuca_norm_f16_t32},
        {64, 1, false, cuca_norm_f32_t64, cuca_norm_f16_t64},
        {128, 1, false, cuca_norm_f32_t128, cuca_norm_f16_t128},
        {256, 1, false, cuca_norm_f32_t256, cuca_norm_f16_t256},
        {512, 1, false, cuca_norm_f32_t512, cuca_norm_f16_t512},
        {1024, 1, false, cuca_norm_f32_t1024, cuca_norm_f16_t1024},
        {1024, 2, false, cuca_norm_f32_t1024_c2, cuca_norm_f16_t1024_c2},
        {1024, 4, false, cuca_norm_f32_t1024_c4, cuca_norm_f16_t1024_c4},
        {1024, 8, false, cuca_norm_f32_t1024_c8, KERNEL_COUNT},
        {128, 1, true, cuca_norm_f32_t128_nt, cuca_norm_f16_t128_nt},
        {256, 1, true, cuca_norm_f32_t256_nt, cuca_norm_f16_t256_nt},
        {512, 1, true, cuca_norm_f32_t512_nt, cuca_norm_f16_t512_nt},
        {1024, 1, true, cuca_norm_f32_t1024_nt, cuca_norm_f16_t1024_nt},
        {1024, 2, true, cuca_norm_f32_t1024_c2_nt, cuca_norm_f16_t1024_c2_nt},
    };
    Kernel plain = KERNEL_COUNT;
    for (const E &e : table) {
        if (e.tpr != tpr || e.per != per) continue;
        if (e.nt == nt) return f16 ? e.k16 : e.k32;
        if (!e.nt) plain = f16 ? e.k16 : e.k32;
    }
    return plain;
}

cuca_status cuca_hip_add_rmsnorm(cuca_hip_ctx *ctx, const void *x, const void *branch,
                                 const float *w, const float *w_post, float eps, float post_eps,
                                 float residual_scale, int64_t rows, int64_t hidden, void *x_out,
                                 void *h_out, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (hidden <= 0 || hidden > (1 << 30)) return fail(ctx, CUCA_INVALID_ARG, "bad hidden size %lld", (long long)hidden);
    if (rows < 0) return fail(ctx, CUCA_INVALID_ARG, "bad row count %lld", (long long)rows);
    if (rows == 0) return CUCA_OK;
    if (!x || !h_out) return fail(ctx, CUCA_INVALID_ARG, "null x or h_out");
    if (w_post && !branch) return fail(ctx, CUCA_INVALID_ARG, "w_post needs a branch");
    if (!(eps >= 0.0f) || !(post_eps >= 0.0f)) return fail(ctx, CUCA_INVALID_ARG, "eps must be >= 0");
    const size_t es = esize(dtype);
    NormArgs a{};
    a.x = x;
    a.branch = branch;
    a.w = w;
    a.w_post = w_post;
    a.x_out = x_out;
    a.h_out = h_out;
    a.rows = rows;
    a.hidden = (int32_t)hidden;
    a.eps = eps;
    a.post_eps = post_eps;
    a.rs = residual_scale;
    const int N = chunk_elems(dtype);
    const bool vec = hidden % N == 0 && al16(x) && al16(h_out) && (!branch || al16(branch)) &&
                     (!x_out || al16(x_out)) && (!w || al16(w)) && (!w_post || al16(w_post)) &&
                     ((size_t)hidden * es) % 16 == 0;
    const int64_t nch = hidden / N;
    const bool f16 = dtype == CUCA_F16;
    if (rows > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "too many rows (%lld)", (long long)rows);
    int tpr = 0, per = 0;
    const bool stream = (int64_t)(branch ? 2 : 1) * rows * hidden * (int64_t)es >= kStreamBytes;
    Kernel k = vec && norm_shape(nch, &tpr, &per) ? norm_kernel(f16, tpr, per, stream) : KERNEL_COUNT;
    // the prefill form of the plain residual step (streamed, a branch and
    // weights, no sandwich, rs 1, x' written, one chunk a thread over the
    // whole row): the streamlined kernels, the same bits
    if (k != KERNEL_COUNT && stream && per == 1 && nch == tpr && branch && w && !w_post && x_out &&
        residual_scale == 1.0f && (tpr == 256 || tpr == 512 || tpr == 1024)) {
        static const Kernel plain[2][3] = {{cuca_norm_f32_t256_nts, cuca_norm_f32_t512_nts, cuca_norm_f32_t1024_nts},
                                           {cuca_norm_f16_t256_nts, cuca_norm_f16_t512_nts, cuca_norm_f16_t1024_nts}};
        k = plain[f16][tpr == 256 ? 0 : tpr == 512 ? 1 : 2];
    }
    if (k == KERNEL_COUNT)
        return launch(ctx, f16 ? cuca_norm_f16_generic : cuca_norm_f32_generic, (unsigned)rows, 256, 0, a);
    // (rows of 256 threads go two to a block: the _t256 kernels)
    const int64_t rows_per_block = tpr == 256 ? 2 : tpr > 64 ? 1 : 256 / tpr;
    const unsigned threads = tpr == 256 ? 512u : tpr > 64 ? (unsigned)tpr : 256u;
    return launch(ctx, k, div_up(rows, rows_per_block), threads, 0, a);
}

cuca_status cuca_hip_selftest_group_sum(cuca_hip_ctx *ctx, const float *input, int64_t n, float *out) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (n <= 0 || n % 256 != 0 || n > (1ll << 30))
        return fail(ctx, CUCA_INVALID_ARG, "self-test length %lld must be a positive multiple of 256", (long long)n);
    if (!input || !out) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    SelftestArgs a{};
    a.in = input;
    a.out = out;
    a.n = n;
    return launch(ctx, cuca_selftest_group_sum, (unsigned)(n / 256), 256, 0, a);
}

// ---------------------------------------------------------------------
// gated activation
// ---------------------------------------------------------------------

static cuca_status glu_common(cuca_hip_ctx *ctx, const void *gate, int64_t gate_ld, const void *up,
                              int64_t up_ld, const int32_t *offsets, int32_t n_experts, int64_t rows,
                              int64_t ff, cuca_act act, float clamp, void *out, int64_t out_ld,
                              cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    if (ff <= 0 || ff > (1 << 30)) return fail(ctx, CUCA_INVALID_ARG, "bad ff %lld", (long long)ff);
    if (rows < 0) return fail(ctx, CUCA_INVALID_ARG, "bad row count %lld", (long long)rows);
    if (gate_ld < ff || up_ld < ff || out_ld < ff)
        return fail(ctx, CUCA_INVALID_ARG, "row strides (%lld, %lld, %lld) shorter than ff %lld",
                    (long long)gate_ld, (long long)up_ld, (long long)out_ld, (long long)ff);
    if (rows == 0) return CUCA_OK;
    if (!gate || !up || !out) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    const bool ragged = offsets != nullptr;
    const size_t es = esize(dtype);
    const int N = chunk_elems(dtype);
    const bool vec = ff % N == 0 && al16(gate) && al16(up) && al16(out) && (gate_ld * es) % 16 == 0 &&
                     (up_ld * es) % 16 == 0 && (out_ld * es) % 16 == 0;
    const bool f16 = dtype == CUCA_F16, gelu = act == CUCA_ACT_GELU_TANH;
    Kernel k;
    int64_t bpr;
    // prefill-sized dense calls stream gate and up (kStreamBytes)
    const bool stream = !ragged && 2 * rows * ff * (int64_t)es >= kGluStreamBytes;
    if (vec) {
        bpr = (ff / N + 255) / 256;
        if (ragged)
            k = f16 ? (gelu ? cuca_glu_f16_gelu_ragged : cuca_glu_f16_silu_ragged)
                    : (gelu ? cuca_glu_f32_gelu_ragged : cuca_glu_f32_silu_ragged);
        else if (stream) {
            k = f16 ? (gelu ? cuca_glu_f16_gelu_nt : cuca_glu_f16_silu_nt)
                    : (gelu ? cuca_glu_f32_gelu_nt : cuca_glu_f32_silu_nt);
            bpr = (ff / N + CUCA_GLU_NT_BLOCK - 1) / CUCA_GLU_NT_BLOCK;
        } else
            k = f16 ? (gelu ? cuca_glu_f16_gelu : cuca_glu_f16_silu)
                    : (gelu ? cuca_glu_f32_gelu : cuca_glu_f32_silu);
    } else {
        bpr = (ff + 255) / 256;
        k = f16 ? (gelu ? (ragged ? cuca_glu_f16_gelu_ragged_generic : cuca_glu_f16_gelu_generic)
                        : (ragged ? cuca_glu_f16_silu_ragged_generic : cuca_glu_f16_silu_generic))
                : (gelu ? (ragged ? cuca_glu_f32_gelu_ragged_generic : cuca_glu_f32_gelu_generic)
                        : (ragged ? cuca_glu_f32_silu_ragged_generic : cuca_glu_f32_silu_generic));
    }
    if (rows * bpr > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "grid too large (%lld rows)", (long long)rows);
    GluArgs a{};
    a.gate = gate;
    a.up = up;
    a.out = out;
    a.offsets = offsets;
    a.rows = rows;
    a.gate_ld = gate_ld;
    a.up_ld = up_ld;
    a.out_ld = out_ld;
    a.ff = (int32_t)ff;
    a.blocks_per_row = (int32_t)bpr;
    a.n_experts = n_experts;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    return launch(ctx, k, (unsigned)(rows * bpr), vec && stream ? CUCA_GLU_NT_BLOCK : 256, 0, a);
}

cuca_status cuca_hip_glu(cuca_hip_ctx *ctx, const void *gate, int64_t gate_ld, const void *up,
                         int64_t up_ld, int64_t rows, int64_t ff, cuca_act act, float clamp,
                         void *out, int64_t out_ld, cuca_dtype dtype) {
    return glu_common(ctx, gate, gate_ld, up, up_ld, nullptr, 0, rows, ff, act, clamp, out, out_ld, dtype);
}

cuca_status cuca_hip_glu_ragged(cuca_hip_ctx *ctx, const void *gate, int64_t gate_ld, const void *up,
                                int64_t up_ld, const int32_t *expert_offsets, int32_t n_experts,
                                int64_t max_rows, int64_t ff, cuca_act act, float clamp, void *out,
                                int64_t out_ld, cuca_dtype dtype) {
    if (!expert_offsets) return fail(ctx, CUCA_INVALID_ARG, "null expert_offsets");
    if (n_experts <= 0) return fail(ctx, CUCA_INVALID_ARG, "bad expert count %d", n_experts);
    return glu_common(ctx, gate, gate_ld, up, up_ld, expert_offsets, n_experts, max_rows, ff, act, clamp,
                      out, out_ld, dtype);
}

// ---------------------------------------------------------------------
// RoPE
// ---------------------------------------------------------------------

// The store (STORE kernels) is on when `slots` is given.
static cuca_status rope_common(cuca_hip_ctx *ctx, void *q, int64_t q_ld, const void *k, int64_t k_ld,
                               const void *v, int64_t v_ld, int64_t rows, int32_t nq, int32_t nk,
                               int32_t head_dim, int32_t n_dims, cuca_rope_kind kind, const float *cos,
                               const float *sin, int64_t table_rows, const int32_t *positions,
                               const float *q_norm_w, const float *k_norm_w, int32_t v_norm, float eps,
                               void *pool_k, void *pool_v, int64_t n_blocks, const int32_t *slots,
                               cuca_dtype dtype, bool full = false) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    const bool store = slots != nullptr;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (kind != CUCA_ROPE_NORM && kind != CUCA_ROPE_NEOX)
        return fail(ctx, CUCA_INVALID_ARG, "bad rope kind %d", (int)kind);
    if (head_dim <= 0 || n_dims <= 0 || n_dims > head_dim || n_dims % 2 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "n_dims %d must be even and within head_dim %d", n_dims, head_dim);
    if (nq < 0 || nk < 0 || rows < 0) return fail(ctx, CUCA_INVALID_ARG, "negative count");
    if (nq > 0 && (!q || q_ld < (int64_t)nq * head_dim))
        return fail(ctx, CUCA_INVALID_ARG, "q row stride %lld shorter than %d heads of %d", (long long)q_ld, nq, head_dim);
    if (nk > 0 && (!k || k_ld < (int64_t)nk * head_dim))
        return fail(ctx, CUCA_INVALID_ARG, "k row stride %lld shorter than %d heads of %d", (long long)k_ld, nk, head_dim);
    if (store) {
        if (nk > 0 && (!v || v_ld < (int64_t)nk * head_dim))
            return fail(ctx, CUCA_INVALID_ARG, "v row stride %lld shorter than %d heads of %d", (long long)v_ld, nk, head_dim);
        if (nk > 0 && (!pool_k || !pool_v)) return fail(ctx, CUCA_INVALID_ARG, "null K/V pool");
        if (n_blocks <= 0 || n_blocks > 0x7fffffffll / CUCA_KV_BLOCK)
            return fail(ctx, CUCA_INVALID_ARG, "bad pool size %lld blocks", (long long)n_blocks);
        if (v_norm != 0 && v_norm != 1) return fail(ctx, CUCA_INVALID_ARG, "v_norm must be 0 or 1");
    }
    const int32_t nv = store ? nk : 0;
    if (rows == 0 || nq + nk == 0) return CUCA_OK;
    if (!cos || !sin || !positions) return fail(ctx, CUCA_INVALID_ARG, "null table or positions");
    if (table_rows <= 0) return fail(ctx, CUCA_INVALID_ARG, "empty rope table");
    if (!(eps >= 0.0f)) return fail(ctx, CUCA_INVALID_ARG, "eps must be >= 0");
    if (rows * (int64_t)(nq + nk + nv) > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "too many heads");
    const size_t es = esize(dtype);
    const int VP = chunk_elems(dtype);
    const bool norm = q_norm_w || k_norm_w || (store && v_norm);
    RopeArgs a{};
    a.q = q;
    a.k = const_cast<void *>(k);
    a.cos_t = cos;
    a.sin_t = sin;
    a.pos = positions;
    a.q_norm_w = q_norm_w;
    a.k_norm_w = k_norm_w;
    a.status = ctx->status;
    a.q_ld = q_ld;
    a.k_ld = k_ld;
    a.table_rows = table_rows;
    a.rows = (int32_t)rows;
    a.nq = nq;
    a.nk = nk;
    a.head_dim = head_dim;
    a.n_dims = n_dims;
    a.eps = eps;
    a.kind = (int32_t)kind;
    if (store) {
        a.v = v;
        a.v_ld = v_ld;
        a.pool_k = pool_k;
        a.pool_v = pool_v;
        a.slots = slots;
        a.n_slots = n_blocks * CUCA_KV_BLOCK;
        a.nv = nv;
        a.v_norm = v_norm;
        ctx->last_kv_blocks = n_blocks;
    }
    ctx->last_table_rows = table_rows;
    // lanes per head: NEOX pairs chunk u with chunk u + n/(2 VP) (two per
    // lane); NORM gives each lane one chunk of whole (2i, 2i+1) pairs
    const bool neox_k = kind == CUCA_ROPE_NEOX;
    const int per_lane = neox_k ? 2 * VP : VP;
    const int tph = head_dim / per_lane;
    const bool pow2 = tph > 0 && (tph & (tph - 1)) == 0 && tph <= 64;
    const bool vec = head_dim % per_lane == 0 && n_dims % (2 * VP) == 0 && pow2 &&
                     (nq == 0 || (al16(q) && (q_ld * es) % 16 == 0)) &&
                     (nk == 0 || (al16(k) && (k_ld * es) % 16 == 0)) && al16(cos) && al16(sin) &&
                     (!q_norm_w || al16(q_norm_w)) && (!k_norm_w || al16(k_norm_w)) &&
                     (!store || nk == 0 ||
                      (al16(v) && (v_ld * es) % 16 == 0 && al16(pool_k) && al16(pool_v)));
    const bool f16 = dtype == CUCA_F16, neox = kind == CUCA_ROPE_NEOX;
    const int64_t heads = rows * (nq + nk + nv);
    if (full) {
        // a workgroup per row over its (head, lane) slots, 4 per thread
        if (!vec)
            return fail(ctx, CUCA_UNSUPPORTED,
                        "full-width QK-norm needs head_dim and n_dims in whole 16-byte chunks per lane "
                        "and 16-byte aligned rows, tables and weights");
        const int64_t total = (int64_t)(nq + nk + nv) * tph;
        if (total > 4096)
            return fail(ctx, CUCA_UNSUPPORTED, "full-width QK-norm: %lld head lanes per row, above 4096",
                        (long long)total);
        int lg = 0;
        while ((1 << lg) < tph) lg++;
        a.tph_log2 = lg;
        unsigned block = 64;
        while ((int64_t)block * 4 < total) block <<= 1;
        static const Kernel table_f[2][2][2] = {
            {{cuca_rope_f32_norm_full, cuca_rope_f32_norm_full_kv}, {cuca_rope_f32_neox_full, cuca_rope_f32_neox_full_kv}},
            {{cuca_rope_f16_norm_full, cuca_rope_f16_norm_full_kv}, {cuca_rope_f16_neox_full, cuca_rope_f16_neox_full_kv}}};
        return launch(ctx, table_f[f16][neox][store], (unsigned)rows, block, 0, a);
    }
    if (!vec) {
        Kernel kk = f16 ? cuca_rope_f16_generic : cuca_rope_f32_generic;
        return launch(ctx, kk, div_up(heads, 4), 256, 0, a);
    }
    int lg = 0;
    while ((1 << lg) < tph) lg++;
    a.tph_log2 = lg;
    // [device-scope loads][dtype][kind][norm][store]: the device-scope
    // kernels address a row's chunks by 32-bit byte offsets from q, k and v
    static const Kernel table_k[2][2][2][2][2] = {
        {{{{cuca_rope_f32_norm_g, cuca_rope_f32_norm_kv_g}, {cuca_rope_f32_norm_qkn_g, cuca_rope_f32_norm_qkn_kv_g}},
          {{cuca_rope_f32_neox_g, cuca_rope_f32_neox_kv_g}, {cuca_rope_f32_neox_qkn_g, cuca_rope_f32_neox_qkn_kv_g}}},
         {{{cuca_rope_f16_norm_g, cuca_rope_f16_norm_kv_g}, {cuca_rope_f16_norm_qkn_g, cuca_rope_f16_norm_qkn_kv_g}},
          {{cuca_rope_f16_neox_g, cuca_rope_f16_neox_kv_g}, {cuca_rope_f16_neox_qkn_g, cuca_rope_f16_neox_qkn_kv_g}}}},
        {{{{cuca_rope_f32_norm, cuca_rope_f32_norm_kv}, {cuca_rope_f32_norm_qkn, cuca_rope_f32_norm_qkn_kv}},
          {{cuca_rope_f32_neox, cuca_rope_f32_neox_kv}, {cuca_rope_f32_neox_qkn, cuca_rope_f32_neox_qkn_kv}}},
         {{{cuca_rope_f16_norm, cuca_rope_f16_norm_kv}, {cuca_rope_f16_norm_qkn, cuca_rope_f16_norm_qkn_kv}},
          {{cuca_rope_f16_neox, cuca_rope_f16_neox_kv}, {cuca_rope_f16_neox_qkn, cuca_rope_f16_neox_qkn_kv}}}}};
    const int64_t lim = 1ll << 32;
    const bool dev = (nq == 0 || rows * q_ld * (int64_t)es <= lim) && (nk == 0 || rows * k_ld * (int64_t)es <= lim) &&
                     (!store || nk == 0 || rows * v_ld * (int64_t)es <= lim);
    static const Kernel table_nt[2][2][2] = {
        {{cuca_rope_f32_norm_qkn_nt, cuca_rope_f32_norm_qkn_kv_nt}, {cuca_rope_f32_neox_qkn_nt, cuca_rope_f32_neox_qkn_kv_nt}},
        {{cuca_rope_f16_norm_qkn_nt, cuca_rope_f16_norm_qkn_kv_nt}, {cuca_rope_f16_neox_qkn_nt, cuca_rope_f16_neox_qkn_kv_nt}}};
    // Head chunks are read with device-scope loads (the rope kernels' load
    // policies), except that prefill-sized QK-norm calls stream them with
    // nontemporal loads.  Measured on MI355X in the config E prefill step
    // (8192 tokens, QK-norm NEOX RoPE): RoPE takes 31.4 us either way, but
    // with device-scope loads the ragged SwiGLU after it slows from 48.3 to
    // 54.7 us and the next gather from 15.4 to 20.8 us.
    const bool stream = norm && heads * (int64_t)head_dim * (int64_t)esize(dtype) >= kStreamBytes;
    const Kernel kk = stream ? table_nt[f16][neox][store] : table_k[dev][f16][neox][norm][store];
    static const Kernel table_h2[2][2][2][2] = {
        {{{cuca_rope_f32_norm_h2, cuca_rope_f32_norm_kv_h2}, {cuca_rope_f32_norm_qkn_h2, cuca_rope_f32_norm_qkn_kv_h2}},
         {{cuca_rope_f32_neox_h2, cuca_rope_f32_neox_kv_h2}, {cuca_rope_f32_neox_qkn_h2, cuca_rope_f32_neox_qkn_kv_h2}}},
        {{{cuca_rope_f16_norm_h2, cuca_rope_f16_norm_kv_h2}, {cuca_rope_f16_norm_qkn_h2, cuca_rope_f16_norm_qkn_kv_h2}},
         {{cuca_rope_f16_neox_h2, cuca_rope_f16_neox_kv_h2}, {cuca_rope_f16_neox_qkn_h2, cuca_rope_f16_neox_qkn_kv_h2}}}};
    static const Kernel table_nt_h2[2][2][2] = {
        {{cuca_rope_f32_norm_qkn_nt_h2, cuca_rope_f32_norm_qkn_kv_nt_h2}, {cuca_rope_f32_neox_qkn_nt_h2, cuca_rope_f32_neox_qkn_kv_nt_h2}},
        {{cuca_rope_f16_norm_qkn_nt_h2, cuca_rope_f16_norm_qkn_kv_nt_h2}, {cuca_rope_f16_neox_qkn_nt_h2, cuca_rope_f16_neox_qkn_kv_nt_h2}}};
    // Two heads per lane when both projections have an even head count: a
    // lane then loads its cos/sin entries and norm weights once for two heads
    // of a row.  Measured on MI355X in the prefill steps: config C RoPE
    // 15.3 -> 14.1 us at 4096 tokens and 54.6 -> 49.4 us at 16384, the fused
    // K/V store 17.9 -> 16.7 and 65.1 -> 59.5 us, config E's QK-norm RoPE
    // 29.8 -> 27.9 us and its fused store 31.4 -> 30.4 us; four heads per
    // lane ran config E's QK-norm kernels slower (99 registers).
    // In-place RoPE of whole heads (the rotated dims cover the head; with
    // QK-norm, norm weights for both projections) takes the _h2w kernels:
    // the same arithmetic without the per-value selects of pass-through
    // lanes and weightless heads, and each QK-norm factor computed once per
    // lane pair.  Measured on MI355X in the prefill steps, the two forms A/B in
    // one process (same bits): config E's QK-norm RoPE 27.3-27.7 -> 26.8-27.1
    // us at 8192 tokens, config C's RoPE 13.9-14.1 -> 13.6-13.8 us at 4096
    // and 49.3-49.4 -> 49.0 us at 16384.
    static const Kernel table_h2w[2][2][2] = {
        {{cuca_rope_f32_norm_h2w, cuca_rope_f32_norm_qkn_h2w}, {cuca_rope_f32_neox_h2w, cuca_rope_f32_neox_qkn_h2w}},
        {{cuca_rope_f16_norm_h2w, cuca_rope_f16_norm_qkn_h2w}, {cuca_rope_f16_neox_h2w, cuca_rope_f16_neox_qkn_h2w}}};
    static const Kernel table_nt_h2w[2][2] = {{cuca_rope_f32_norm_qkn_nt_h2w, cuca_rope_f32_neox_qkn_nt_h2w},
                                              {cuca_rope_f16_norm_qkn_nt_h2w, cuca_rope_f16_neox_qkn_nt_h2w}};
    const bool whole = !store && n_dims == head_dim && tph >= 2 && (!norm || (q_norm_w && k_norm_w));
    if (dev && nq % 2 == 0 && nk % 2 == 0) {
        const Kernel k2 = whole ? (stream ? table_nt_h2w[f16][neox] : table_h2w[f16][neox][norm])
                                : (stream ? table_nt_h2[f16][neox][store] : table_h2[f16][neox][norm][store]);
        return launch(ctx, k2, div_up(heads / 2, 256 / tph), 256, 0, a);
    }
    return launch(ctx, kk, div_up(heads, 256 / tph), 256, 0, a);
}

cuca_status cuca_hip_rope(cuca_hip_ctx *ctx, void *q, int64_t q_ld, void *k, int64_t k_ld, int64_t rows,
                          int32_t nq, int32_t nk, int32_t head_dim, int32_t n_dims, cuca_rope_kind kind,
                          const float *cos, const float *sin, int64_t table_rows, const int32_t *positions,
                          const float *q_norm_w, const float *k_norm_w, float eps, cuca_dtype dtype) {
    return rope_common(ctx, q, q_ld, k, k_ld, nullptr, 0, rows, nq, nk, head_dim, n_dims, kind, cos, sin,
                       table_rows, positions, q_norm_w, k_norm_w, 0, eps, nullptr, nullptr, 0, nullptr, dtype);
}

cuca_status cuca_hip_rope_full(cuca_hip_ctx *ctx, void *q, int64_t q_ld, void *k, int64_t k_ld, int64_t rows,
                               int32_t nq, int32_t nk, int32_t head_dim, int32_t n_dims, cuca_rope_kind kind,
                               const float *cos, const float *sin, int64_t table_rows, const int32_t *positions,
                               const float *q_norm_w, const float *k_norm_w, float eps, cuca_dtype dtype) {
    return rope_common(ctx, q, q_ld, k, k_ld, nullptr, 0, rows, nq, nk, head_dim, n_dims, kind, cos, sin,
                       table_rows, positions, q_norm_w, k_norm_w, 0, eps, nullptr, nullptr, 0, nullptr, dtype,
                       true);
}

cuca_status cuca_hip_rope_store_kv_full(cuca_hip_ctx *ctx, void *q, int64_t q_ld, const void *k, int64_t k_ld,
                                        const void *v, int64_t v_ld, int64_t rows, int32_t nq, int32_t nk,
                                        int32_t head_dim, int32_t n_dims, cuca_rope_kind kind, const float *cos,
                                        const float *sin, int64_t table_rows, const int32_t *positions,
                                        const float *q_norm_w, const float *k_norm_w, int32_t v_norm, float eps,
                                        void *pool_k, void *pool_v, int64_t n_blocks, const int32_t *slots,
                                        cuca_dtype dtype) {
    if (!slots) return fail(ctx, CUCA_INVALID_ARG, "null slots");
    return rope_common(ctx, q, q_ld, k, k_ld, v, v_ld, rows, nq, nk, head_dim, n_dims, kind, cos, sin,
                       table_rows, positions, q_norm_w, k_norm_w, v_norm, eps, pool_k, pool_v, n_blocks,
                       slots, dtype, true);
}

cuca_status cuca_hip_rope_store_kv(cuca_hip_ctx *ctx, void *q, int64_t q_ld, const void *k, int64_t k_ld,
                                   const void *v, int64_t v_ld, int64_t rows, int32_t nq, int32_t nk,
                                   int32_t head_dim, int32_t n_dims, cuca_rope_kind kind, const float *cos,
                                   const float *sin, int64_t table_rows, const int32_t *positions,
                                   const float *q_norm_w, const float *k_norm_w, int32_t v_norm, float eps,
                                   void *pool_k, void *pool_v, int64_t n_blocks, const int32_t *slots,
                                   cuca_dtype dtype) {
    if (!slots) return fail(ctx, CUCA_INVALID_ARG, "null slots");
    return rope_common(ctx, q, q_ld, k, k_ld, v, v_ld, rows, nq, nk, head_dim, n_dims, kind, cos, sin,
                       table_rows, positions, q_norm_w, k_norm_w, v_norm, eps, pool_k, pool_v, n_blocks,
                       slots, dtype);
}

// The pool rows of cache indices start..start+t (paged.rs:9-16): position p
// is row p % 16 of block table[p / 16]; a missing, released or out-of-pool
// block fails like check_range (cpu/paged_attn.rs:42-65).
cuca_status cuca_hip_kv_slots(const uint32_t *table, int64_t table_len, int64_t start, int64_t t,
                              int64_t n_blocks, int32_t *slots_out) {
    if (start < 0 || t < 0 || table_len < 0) return fail(nullptr, CUCA_INVALID_ARG, "negative count");
    if (t == 0) return CUCA_OK;
    if (!slots_out || (!table && table_len > 0)) return fail(nullptr, CUCA_INVALID_ARG, "null pointer");
    if (n_blocks <= 0 || n_blocks > 0x7fffffffll / CUCA_KV_BLOCK)
        return fail(nullptr, CUCA_INVALID_ARG, "bad pool size %lld blocks", (long long)n_blocks);
    for (int64_t i = 0; i < t; i++) {
        const int64_t p = start + i;
        const int64_t bi = p / CUCA_KV_BLOCK;
        const uint32_t id = bi < table_len ? table[bi] : CUCA_NO_BLOCK;
        if (id == CUCA_NO_BLOCK || (int64_t)id >= n_blocks)
            return fail(nullptr, CUCA_OUT_OF_RANGE,
                        "position %lld has no K/V block (it left the window or was never allocated)",
                        (long long)(bi * CUCA_KV_BLOCK));
        slots_out[i] = (int32_t)((int64_t)id * CUCA_KV_BLOCK + p % CUCA_KV_BLOCK);
    }
    return CUCA_OK;
}

// ---------------------------------------------------------------------
// paged decode attention
// ---------------------------------------------------------------------

// Partials a row of max_blocks blocks can need: parts are never shorter
// than CUCA_ATTN_MIN_PART positions.
static int64_t attn_max_parts(int64_t max_blocks, int64_t part_positions) {
    return (max_blocks * CUCA_KV_BLOCK + part_positions - 1) / part_positions;
}

cuca_status cuca_hip_paged_decode_workspace(int64_t rows, int32_t n_head, int32_t head_dim,
                                            int64_t max_blocks, size_t *bytes) {
    if (!bytes) return fail(nullptr, CUCA_INVALID_ARG, "null output pointer");
    if (rows < 0 || n_head <= 0 || head_dim <= 0 || max_blocks <= 0)
        return fail(nullptr, CUCA_INVALID_ARG, "bad attention shape");
    *bytes = (size_t)rows * (size_t)n_head * (size_t)attn_max_parts(max_blocks, CUCA_ATTN_MIN_PART) *
             (size_t)(head_dim + 2) * sizeof(float);
    return CUCA_OK;
}

// The paged decode of a caller's workspace (noalloc false) or of the
// library's scratch array (noalloc true: workspace is ignored).
static cuca_status paged_decode_run(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool_k,
                                    const void *pool_v, int64_t n_blocks, const uint32_t *tables,
                                    int64_t max_blocks, const int32_t *ranges, int64_t rows, int32_t n_head,
                                    int32_t n_kv, int32_t head_dim, float scale, void *workspace,
                                    size_t workspace_bytes, bool noalloc, void *out, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (rows < 0) return fail(ctx, CUCA_INVALID_ARG, "negative count");
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv != 0)
        return fail(ctx, CUCA_INVALID_ARG, "attention: query shape mismatch (%d heads over %d KV heads)",
                    n_head, n_kv);
    if (head_dim <= 0 || head_dim > 512) return fail(ctx, CUCA_UNSUPPORTED, "head_dim %d above 512", head_dim);
    if (max_blocks <= 0 || max_blocks > (1 << 22))
        return fail(ctx, CUCA_INVALID_ARG, "bad block table width %lld", (long long)max_blocks);
    if (n_blocks <= 0) return fail(ctx, CUCA_INVALID_ARG, "bad pool size %lld blocks", (long long)n_blocks);
    if (rows == 0) return CUCA_OK;
    if (!q || !pool_k || !pool_v || !tables || !ranges || !out || (!noalloc && !workspace))
        return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (q_ld < (int64_t)n_head * head_dim)
        return fail(ctx, CUCA_INVALID_ARG, "q row stride %lld below %d heads of %d", (long long)q_ld, n_head,
                    head_dim);
    if (((size_t)q_ld * esize(dtype)) % 4 != 0 || (reinterpret_cast<uintptr_t>(q) & 3) != 0)
        return fail(ctx, CUCA_INVALID_ARG, "q rows must be 4-byte aligned");
    if (!noalloc) {
        size_t need = 0;
        cuca_hip_paged_decode_workspace(rows, n_head, head_dim, max_blocks, &need);
        if (workspace_bytes < need)
            return fail(ctx, CUCA_INVALID_ARG, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
        if (!al16(workspace)) return fail(ctx, CUCA_INVALID_ARG, "workspace must be 16-byte aligned");
    }
    const bool f16 = dtype == CUCA_F16;
    const size_t es = esize(dtype);
    const int G = n_head / n_kv;
    const int di = head_dim == 64 ? 0 : head_dim == 128 ? 1 : head_dim == 256 ? 2 : -1;
    const int gi = G == 1 ? 0 : G == 2 ? 1 : G == 4 ? 2 : G == 8 ? 3 : -1;
    const bool vec = di >= 0 && gi >= 0 && !(di == 2 && gi == 3) && al16(pool_k) && al16(pool_v) &&
                     ((size_t)head_dim * es) % 16 == 0;
    // vector kernel: a part = 4 waves x CP positions, CP = 64 / LPP with
    // LPP = max(1, row bytes / 256), and at least 2 for a group of 8 (the
    // 8-wave f16 group-4 kernels: 8 waves x CP / 2, the same length);
    // generic: a part = 64 positions
    int64_t part_positions = CUCA_ATTN_MIN_PART;
    if (vec) {
        const int64_t rowb = (int64_t)head_dim * (int64_t)es;
        int64_t lpp = rowb > 256 ? rowb / 256 : 1;
        if (G >= 8 && lpp < 2) lpp = 2;
        part_positions = 4 * (64 / lpp);
    }
    const int64_t parts = attn_max_parts(max_blocks, part_positions);
    if (rows * n_head * parts > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "too many attention parts");
    if (noalloc) {
        // the partials this call writes and reads: [rows, n_head, parts, head_dim + 2] f32
        const double used = (double)rows * (double)n_head * (double)parts * (double)(head_dim + 2) * 4.0;
        if (used > (double)CUCA_NOALLOC_SCRATCH_BYTES)
            return fail(ctx, CUCA_INVALID_ARG,
                        "paged_decode_noalloc: %lld rows x %d heads x %lld parts of %d values need %.0f bytes "
                        "of scratch, above the library's %u (use cuca_hip_paged_decode with a workspace)",
                        (long long)rows, n_head, (long long)parts, head_dim + 2, used,
                        (unsigned)CUCA_NOALLOC_SCRATCH_BYTES);
        if (!ctx->noalloc) return fail(ctx, CUCA_HIP_ERROR, "paged_decode_noalloc: no scratch on device %d: %s",
                                       ctx->device, ctx->noalloc_error.c_str());
        workspace = ctx->noalloc;
    }
    AttnArgs a{};
    a.q = q;
    a.q_ld = q_ld;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = tables;
    a.ranges = ranges;
    a.part = static_cast<float *>(workspace);
    a.out = out;
    a.status = ctx->status;
    a.n_blocks = n_blocks;
    a.rows = (int32_t)rows;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.head_dim = head_dim;
    a.max_blocks = (int32_t)max_blocks;
    a.max_parts = (int32_t)parts;
    a.part_positions = (int32_t)part_positions;
    a.scale = scale;
    // one part a row (short contexts): the split writes the outputs itself
    a.direct = vec && parts == 1 ? 1 : 0;
    Kernel split;
    unsigned grid;
    if (vec) {
        // [dtype][head_dim 64/128/256][group 1/2/4/8]; no d256 x 8 kernel
        static const Kernel ks[2][3][4] = {
            {{cuca_attn_split_f32_d64_g1, cuca_attn_split_f32_d64_g2, cuca_attn_split_f32_d64_g4,
              cuca_attn_split_f32_d64_g8},
             {cuca_attn_split_f32_d128_g1, cuca_attn_split_f32_d128_g2, cuca_attn_split_f32_d128_g4,
              cuca_attn_split_f32_d128_g8},
             {cuca_attn_split_f32_d256_g1, cuca_attn_split_f32_d256_g2, cuca_attn_split_f32_d256_g4, KERNEL_COUNT}},
            {{cuca_attn_split_f16_d64_g1, cuca_attn_split_f16_d64_g2, cuca_attn_split_f16_d64_g4,
              cuca_attn_split_f16_d64_g8},
             {cuca_attn_split_f16_d128_g1, cuca_attn_split_f16_d128_g2, cuca_attn_split_f16_d128_g4,
              cuca_attn_split_f16_d128_g8},
             {cuca_attn_split_f16_d256_g1, cuca_attn_split_f16_d256_g2, cuca_attn_split_f16_d256_g4, KERNEL_COUNT}}};
        split = ks[f16][di][gi];
        grid = (unsigned)(rows * n_kv * parts); // a workgroup per (row, KV head, part)
    } else {
        split = f16 ? cuca_attn_split_f16_generic : cuca_attn_split_f32_generic;
        grid = div_up(rows * n_head * parts, 4); // a wave per (row, head, part)
    }
    // (f16 group-4 splits at head_dim 64 / 128 are 8-wave workgroups)
    const unsigned split_threads = vec && f16 && gi == 2 && di < 2 ? 512u : 256u;
    if ((st = launch(ctx, split, grid, split_threads, 0, a)) != CUCA_OK) return st;
    if (a.direct) return CUCA_OK;
    static const Kernel km[2][4] = {
        {cuca_attn_merge_f32_c1, cuca_attn_merge_f32_c2, cuca_attn_merge_f32_c4, cuca_attn_merge_f32_c8},
        {cuca_attn_merge_f16_c1, cuca_attn_merge_f16_c2, cuca_attn_merge_f16_c4, cuca_attn_merge_f16_c8}};
    const int cpl = (head_dim + 63) / 64;
    // (the two-column merge reads column pairs: an even head_dim; an odd one
    // takes the four-column kernel, whose columns sum in the same order)
    const int ci = cpl <= 1 ? 0 : (cpl <= 2 && head_dim % 2 == 0) ? 1 : cpl <= 4 ? 2 : 3;
    return launch(ctx, km[f16][ci], div_up(rows * n_head, 4), 256, 0, a);
}

cuca_status cuca_hip_paged_decode(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool_k,
                                  const void *pool_v, int64_t n_blocks, const uint32_t *tables, int64_t max_blocks,
                                  const int32_t *ranges, int64_t rows, int32_t n_head, int32_t n_kv,
                                  int32_t head_dim, float scale, void *workspace, size_t workspace_bytes,
                                  void *out, cuca_dtype dtype) {
    return paged_decode_run(ctx, q, q_ld, pool_k, pool_v, n_blocks, tables, max_blocks, ranges, rows, n_head,
                            n_kv, head_dim, scale, workspace, workspace_bytes, false, out, dtype);
}

cuca_status cuca_hip_paged_decode_noalloc(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool_k,
                                          const void *pool_v, int64_t n_blocks, const uint32_t *tables,
                                          int64_t max_blocks, const int32_t *ranges, int64_t rows, int32_t n_head,
                                          int32_t n_kv, int32_t head_dim, float scale, void *out,
                                          cuca_dtype dtype) {
    return paged_decode_run(ctx, q, q_ld, pool_k, pool_v, n_blocks, tables, max_blocks, ranges, rows, n_head,
                            n_kv, head_dim, scale, nullptr, 0, true, out, dtype);
}

// ---------------------------------------------------------------------
// paged attention of many rows of one sequence (attend_paged_rows)
// ---------------------------------------------------------------------

// pool_v NULL: the latent form (values = the key rows' first v_width columns)
static cuca_status attend_rows_run(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool_k,
                                   const void *pool_v, int64_t n_blocks, const uint32_t *table, int64_t max_blocks,
                                   const int32_t *ranges, int64_t rows, int32_t n_head, int32_t n_kv,
                                   int32_t head_dim, int32_t v_width, float scale, void *out, int64_t out_ld,
                                   cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (rows < 0 || rows > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "bad row count %lld", (long long)rows);
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv != 0)
        return fail(ctx, CUCA_INVALID_ARG, "attention: query shape mismatch (%d heads over %d KV heads)",
                    n_head, n_kv);
    if (head_dim <= 0 || head_dim > 1024)
        return fail(ctx, CUCA_UNSUPPORTED, "head_dim %d above 1024", head_dim);
    if (v_width <= 0 || v_width > head_dim) return fail(ctx, CUCA_INVALID_ARG, "attention: bad latent value width");
    if (v_width > 512) return fail(ctx, CUCA_UNSUPPORTED, "value width %d above 512", v_width);
    if (max_blocks <= 0 || max_blocks > (1 << 22))
        return fail(ctx, CUCA_INVALID_ARG, "bad block table width %lld", (long long)max_blocks);
    if (n_blocks <= 0) return fail(ctx, CUCA_INVALID_ARG, "bad pool size %lld blocks", (long long)n_blocks);
    if (rows == 0) return CUCA_OK;
    if (!q || !pool_k || !table || !ranges || !out) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (q_ld < (int64_t)n_head * head_dim)
        return fail(ctx, CUCA_INVALID_ARG, "q row stride %lld below %d heads of %d", (long long)q_ld, n_head,
                    head_dim);
    if (out_ld < (int64_t)n_head * v_width)
        return fail(ctx, CUCA_INVALID_ARG, "out row stride %lld below %d heads of %d", (long long)out_ld, n_head,
                    v_width);
    const size_t es = esize(dtype);
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) % es != 0)
        return fail(ctx, CUCA_INVALID_ARG, "q and out must be aligned to their element");
    const bool f16 = dtype == CUCA_F16;
    const int G = n_head / n_kv;
    const int di = head_dim == 64 ? 0 : head_dim == 128 ? 1 : head_dim == 256 ? 2 : -1;
    const int gi = G == 1 ? 0 : G == 2 ? 1 : G == 4 ? 2 : G == 8 ? 3 : -1;
    // the matrix-core kernel: its own value pool, 16-byte pool rows and
    // loads, 8-byte (f16) or 16-byte (f32) query and output pieces
    const uintptr_t qa = reinterpret_cast<uintptr_t>(q), oa = reinterpret_cast<uintptr_t>(out);
    const bool mfma = pool_v && di >= 0 && gi >= 0 && al16(pool_k) && al16(pool_v) &&
                      (f16 ? (qa % 8 == 0 && q_ld % 4 == 0 && oa % 8 == 0 && out_ld % 4 == 0)
                           : (oa % 16 == 0 && out_ld % 4 == 0));
    AttnRowsArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.table = table;
    a.ranges = ranges;
    a.out = out;
    a.status = ctx->status;
    a.q_ld = q_ld;
    a.out_ld = out_ld;
    a.n_blocks = n_blocks;
    a.rows = (int32_t)rows;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.head_dim = head_dim;
    a.v_width = v_width;
    a.max_blocks = (int32_t)max_blocks;
    a.scale = scale;
    if (mfma) {
        // [f16][head_dim 64/128/256][group 1/2/4/8]
        static const Kernel table_k[2][3][4] = {
            {{cuca_attn_rows_f32_d64_g1, cuca_attn_rows_f32_d64_g2, cuca_attn_rows_f32_d64_g4, cuca_attn_rows_f32_d64_g8},
             {cuca_attn_rows_f32_d128_g1, cuca_attn_rows_f32_d128_g2, cuca_attn_rows_f32_d128_g4,
              cuca_attn_rows_f32_d128_g8},
             {cuca_attn_rows_f32_d256_g1, cuca_attn_rows_f32_d256_g2, cuca_attn_rows_f32_d256_g4,
              cuca_attn_rows_f32_d256_g8}},
            {{cuca_attn_rows_f16_d64_g1, cuca_attn_rows_f16_d64_g2, cuca_attn_rows_f16_d64_g4, cuca_attn_rows_f16_d64_g8},
             {cuca_attn_rows_f16_d128_g1, cuca_attn_rows_f16_d128_g2, cuca_attn_rows_f16_d128_g4,
              cuca_attn_rows_f16_d128_g8},
             {cuca_attn_rows_f16_d256_g1, cuca_attn_rows_f16_d256_g2, cuca_attn_rows_f16_d256_g4,
              cuca_attn_rows_f16_d256_g8}}};
        // a workgroup: RT tiles of 16 rows x the G query heads, one wave each
        // (the kernels' launch shape: RT = 4 at groups 1 and 2, 8 / G beyond)
        const int rt = G <= 2 ? 4 : 8 / G;
        const int64_t tiles = (rows + 16 * rt - 1) / (16 * rt);
        if (tiles * n_kv > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "too many attention tiles");
        return launch(ctx, table_k[f16][di][gi], (unsigned)(tiles * n_kv), (unsigned)(64 * G * rt), 0u, a);
    }
    const int64_t jobs = rows * n_head;
    if ((jobs + 3) / 4 > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "too many attention rows");
    return launch(ctx, f16 ? cuca_attn_rows_f16_generic : cuca_attn_rows_f32_generic, div_up(jobs, 4), 256u, 0u, a);
}

cuca_status cuca_hip_attend_rows(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool_k,
                                 const void *pool_v, int64_t n_blocks, const uint32_t *table, int64_t max_blocks,
                                 const int32_t *ranges, int64_t rows, int32_t n_head, int32_t n_kv, int32_t head_dim,
                                 float scale, void *out, int64_t out_ld, cuca_dtype dtype) {
    if (!pool_v) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    return attend_rows_run(ctx, q, q_ld, pool_k, pool_v, n_blocks, table, max_blocks, ranges, rows, n_head, n_kv,
                           head_dim, head_dim, scale, out, out_ld, dtype);
}

cuca_status cuca_hip_attend_latent_rows(cuca_hip_ctx *ctx, const void *q, int64_t q_ld, const void *pool,
                                        int64_t n_blocks, const uint32_t *table, int64_t max_blocks,
                                        const int32_t *ranges, int64_t rows, int32_t n_head, int32_t head_dim,
                                        int32_t v_width, float scale, void *out, int64_t out_ld, cuca_dtype dtype) {
    return attend_rows_run(ctx, q, q_ld, pool, nullptr, n_blocks, table, max_blocks, ranges, rows, n_head, 1,
                           head_dim, v_width, scale, out, out_ld, dtype);
}

// ---------------------------------------------------------------------
// quantized matmul (QmmWeight, qmm.rs)
// ---------------------------------------------------------------------

// Packed layout of qmm.hip: groups of G blocks of GB bytes per row.
static bool qfmt(uint32_t t, int *g, int *gb) {
    if (t == CUCA_GGML_Q4_0) { *g = 16; *gb = 288; return true; }
    if (t == CUCA_GGML_Q8_0) { *g = 8; *gb = 272; return true; }
    return false;
}

// from_raw's checks (qmm.rs:1769-1782): a served type, whole blocks, n > 0.
static cuca_status qweight_shape(cuca_hip_ctx *ctx, uint32_t t, int64_t n, int64_t k, int *g,
                                 int *gb) {
    if (!qfmt(t, g, gb))
        return fail(ctx, CUCA_UNSUPPORTED, "ggml type %u: the quantized matmul serves Q4_0 (2) and Q8_0 (8)", t);
    if (n <= 0 || n > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "qmm: bad weight row count %lld", (long long)n);
    if (k <= 0 || k % 32 != 0 || k / 32 > 0x7fffffffll)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: row length %lld is not a whole number of blocks", (long long)k);
    return CUCA_OK;
}

cuca_status cuca_hip_qweight_bytes(uint32_t ggml_type, int64_t n, int64_t k, size_t *bytes) {
    if (!bytes) return fail(nullptr, CUCA_INVALID_ARG, "null output pointer");
    int g = 0, gb = 0;
    cuca_status st = qweight_shape(nullptr, ggml_type, n, k, &g, &gb);
    if (st != CUCA_OK) return st;
    const int64_t ng = (k / 32 + g - 1) / g;
    *bytes = (size_t)n * (size_t)ng * (size_t)gb;
    return CUCA_OK;
}

cuca_status cuca_hip_qweight_pack(cuca_hip_ctx *ctx, const void *gguf, uint32_t ggml_type, int64_t n,
                                  int64_t k, void *packed) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!gguf || !packed) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!al16(packed)) return fail(ctx, CUCA_INVALID_ARG, "packed weight must be 16-byte aligned");
    const int64_t nb = k / 32, ng = (nb + g - 1) / g;
    const int64_t pieces = n * ng * (gb / 16);
    if (pieces / CUCA_BLOCK_THREADS + 1 > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "weight too large");
    QPackArgs a{};
    a.src = static_cast<const uint8_t *>(gguf);
    a.dst = static_cast<uint8_t *>(packed);
    a.n = (int32_t)n;
    a.nb = (int32_t)nb;
    a.ng = (int32_t)ng;
    return launch(ctx, ggml_type == CUCA_GGML_Q4_0 ? cuca_qpack_q4_0 : cuca_qpack_q8_0,
                  div_up(pieces, CUCA_BLOCK_THREADS), CUCA_BLOCK_THREADS, 0, a);
}

// The LM head epilogue of cap_logits (cpu.rs:2603-2617); all 1 / 0 = none.
struct LogitCap {
    float logit_scale = 1.0f, logit_mult = 1.0f, softcap = 0.0f;
};

// LDS of a qmv workgroup (qmv.hip QMV_LDS_BYTES) for MT rows, nbp padded
// blocks of groups of G; the kernel is used when it fits in 64 KiB.
static size_t qmv_lds(int64_t mt, int64_t nbp, int g) {
    return (size_t)(mt * 16 * (nbp + 2) * 8 + mt * nbp * 4 + 4 * mt * 2 * 4 * g * 4 + 4 * 32 * mt * 2 * 4 * 4);
}
static bool qmv_fits(int64_t m, int64_t nbp, int g) {
    return m >= 1 && m <= 2 && qmv_lds(m, nbp, g) <= (64u << 10);
}
// qmm routes one or two rows to the decode GEMV only where its persistent
// waves (four workgroups of four per CU) each get at least two four-row
// tasks, so the per-workgroup expansion of the quants is shared: the LM
// head.  Below that the one-pass kernel is faster (it has no separate
// quantisation launch and fills the chip with more, shorter waves).
static bool qmv_wins(const cuca_hip_ctx *ctx, int64_t rows) {
    return (rows + 3) / 4 >= 2 * 16 * (int64_t)ctx->cu_count;
}

static cuca_status q8_acts_launch(cuca_hip_ctx *ctx, const void *x, int64_t ldx, int64_t m, int64_t k,
                                  cuca_dtype dtype, int8_t *quants, int64_t q_ld, float *scales) {
    Q8ActsArgs a{};
    a.x = x;
    a.quants = quants;
    a.scales = scales;
    a.ldx = ldx;
    a.q_ld = q_ld;
    a.m = (int32_t)m;
    a.nb = (int32_t)(k / 32);
    return launch(ctx, dtype == CUCA_F16 ? cuca_q8_acts_f16 : cuca_q8_acts_f32, div_up(m * (k / 32), CUCA_BLOCK_THREADS),
                  CUCA_BLOCK_THREADS, 0, a);
}

// The decode GEMV (m <= 2, qmv_fits checked): mode 0 on quantised rows
// (quants, scales), mode 3 on the rows of x.  glu: 0 plain, 1 SiLU, 2 GELU-tanh.
static cuca_status qmv_launch(cuca_hip_ctx *ctx, int mode, const void *w, const void *w_up, uint32_t ggml_type,
                              int64_t n, int64_t k, const int8_t *quants, int64_t q_ld, const float *scales,
                              const void *x, int64_t ldx, int64_t m, int64_t rows, int glu, float clamp, void *out,
                              int64_t out_ld, cuca_dtype dtype, const LogitCap &cap);

// The decode matmul of one activation row (qmd.hip): rows up to 16384
// values (n2 kernels to 4096), the workgroup's LDS copy of the expanded row
// within 64 KiB, and the weight rows' bytes addressable by a 32-bit buffer
// offset.  mode 0: plain / GLU (glu 1 SiLU, 2 GELU-tanh); 3: Q|K|V with RoPE
// and the K/V store (a carries the epilogue's fields).
static size_t qmd_lds(int64_t ng, int g) { return (size_t)(16 * (ng * g + 2) * 8 + (ng + 1) * g * 4); }
static bool qmd_fits(int64_t m, int64_t k, int64_t ng, int g, int64_t rows, int64_t row_bytes) {
    return m == 1 && k <= 16384 && qmd_lds(ng, g) <= (64u << 10) && rows * row_bytes < (1ll << 31);
}
static cuca_status qmd_launch(cuca_hip_ctx *ctx, int mode, int glu, uint32_t ggml_type, int64_t k, int g,
                              cuca_dtype dtype, QmmArgs &a, bool rn = false) {
    // [dtype][format][n2, n8][plain, silu, gelu, rope_kv]
    static const Kernel table_k[2][2][2][4] = {
        {{{cuca_qmd_f32_q4_0_n2, cuca_qmd_glu_f32_q4_0_silu_n2, cuca_qmd_glu_f32_q4_0_gelu_n2,
           cuca_qmd_rope_kv_f32_q4_0_n2},
          {cuca_qmd_f32_q4_0_n8, cuca_qmd_glu_f32_q4_0_silu_n8, cuca_qmd_glu_f32_q4_0_gelu_n8,
           cuca_qmd_rope_kv_f32_q4_0_n8}},
         {{cuca_qmd_f32_q8_0_n2, cuca_qmd_glu_f32_q8_0_silu_n2, cuca_qmd_glu_f32_q8_0_gelu_n2,
           cuca_qmd_rope_kv_f32_q8_0_n2},
          {cuca_qmd_f32_q8_0_n8, cuca_qmd_glu_f32_q8_0_silu_n8, cuca_qmd_glu_f32_q8_0_gelu_n8,
           cuca_qmd_rope_kv_f32_q8_0_n8}}},
        {{{cuca_qmd_f16_q4_0_n2, cuca_qmd_glu_f16_q4_0_silu_n2, cuca_qmd_glu_f16_q4_0_gelu_n2,
           cuca_qmd_rope_kv_f16_q4_0_n2},
          {cuca_qmd_f16_q4_0_n8, cuca_qmd_glu_f16_q4_0_silu_n8, cuca_qmd_glu_f16_q4_0_gelu_n8,
           cuca_qmd_rope_kv_f16_q4_0_n8}},
         {{cuca_qmd_f16_q8_0_n2, cuca_qmd_glu_f16_q8_0_silu_n2, cuca_qmd_glu_f16_q8_0_gelu_n2,
           cuca_qmd_rope_kv_f16_q8_0_n2},
          {cuca_qmd_f16_q8_0_n8, cuca_qmd_glu_f16_q8_0_silu_n8, cuca_qmd_glu_f16_q8_0_gelu_n8,
           cuca_qmd_rope_kv_f16_q8_0_n8}}}};
    // the same with the residual add + RMSNorm prologue
    static const Kernel table_rn[2][2][2][4] = {
        {{{cuca_qmd_f32_q4_0_n2_rn, cuca_qmd_glu_f32_q4_0_silu_n2_rn, cuca_qmd_glu_f32_q4_0_gelu_n2_rn,
           cuca_qmd_rope_kv_f32_q4_0_n2_rn},
          {cuca_qmd_f32_q4_0_n8_rn, cuca_qmd_glu_f32_q4_0_silu_n8_rn, cuca_qmd_glu_f32_q4_0_gelu_n8_rn,
           cuca_qmd_rope_kv_f32_q4_0_n8_rn}},
         {{cuca_qmd_f32_q8_0_n2_rn, cuca_qmd_glu_f32_q8_0_silu_n2_rn, cuca_qmd_glu_f32_q8_0_gelu_n2_rn,
           cuca_qmd_rope_kv_f32_q8_0_n2_rn},
          {cuca_qmd_f32_q8_0_n8_rn, cuca_qmd_glu_f32_q8_0_silu_n8_rn, cuca_qmd_glu_f32_q8_0_gelu_n8_rn,
           cuca_qmd_rope_kv_f32_q8_0_n8_rn}}},
        {{{cuca_qmd_f16_q4_0_n2_rn, cuca_qmd_glu_f16_q4_0_silu_n2_rn, cuca_qmd_glu_f16_q4_0_gelu_n2_rn,
           cuca_qmd_rope_kv_f16_q4_0_n2_rn},
          {cuca_qmd_f16_q4_0_n8_rn, cuca_qmd_glu_f16_q4_0_silu_n8_rn, cuca_qmd_glu_f16_q4_0_gelu_n8_rn,
           cuca_qmd_rope_kv_f16_q4_0_n8_rn}},
         {{cuca_qmd_f16_q8_0_n2_rn, cuca_qmd_glu_f16_q8_0_silu_n2_rn, cuca_qmd_glu_f16_q8_0_gelu_n2_rn,
           cuca_qmd_rope_kv_f16_q8_0_n2_rn},
          {cuca_qmd_f16_q8_0_n8_rn, cuca_qmd_glu_f16_q8_0_silu_n8_rn, cuca_qmd_glu_f16_q8_0_gelu_n8_rn,
           cuca_qmd_rope_kv_f16_q8_0_n8_rn}}}};
    const int kind = mode == 3 ? 3 : glu;
    // a plain matmul of at least 32 rows per compute unit (the LM head, or
    // the final norm and the head) as 8-wave workgroups
    if (kind == 0 && div_up(a.rows, 32) >= (int64_t)ctx->cu_count) {
        // [norm prologue][dtype][format][n2, n8]
        static const Kernel table_p8[2][2][2][2] = {{{{cuca_qmd_f32_q4_0_n2w8, cuca_qmd_f32_q4_0_n8w8},
            {cuca_qmd_f32_q8_0_n2w8, cuca_qmd_f32_q8_0_n8w8}},
            {{cuca_qmd_f16_q4_0_n2w8, cuca_qmd_f16_q4_0_n8w8},
            {cuca_qmd_f16_q8_0_n2w8, cuca_qmd_f16_q8_0_n8w8}}},
            {{{cuca_qmd_f32_q4_0_n2w8_rn, cuca_qmd_f32_q4_0_n8w8_rn},
            {cuca_qmd_f32_q8_0_n2w8_rn, cuca_qmd_f32_q8_0_n8w8_rn}},
            {{cuca_qmd_f16_q4_0_n2w8_rn, cuca_qmd_f16_q4_0_n8w8_rn},
            {cuca_qmd_f16_q8_0_n2w8_rn, cuca_qmd_f16_q8_0_n8w8_rn}}}};
        return launch(ctx, table_p8[rn][dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][k > 4096], div_up(a.rows, 32),
                      8 * 64, (unsigned)qmd_lds(a.ng, g), a);
    }
    // the Q|K|V with the norm prologue as 8-wave workgroups
    if (kind == 3 && rn) {
        // [dtype][format][n2, n8]
        static const Kernel table_q8[2][2][2] = {{{cuca_qmd_rope_kv_f32_q4_0_n2w8_rn, cuca_qmd_rope_kv_f32_q4_0_n8w8_rn},
            {cuca_qmd_rope_kv_f32_q8_0_n2w8_rn, cuca_qmd_rope_kv_f32_q8_0_n8w8_rn}},
            {{cuca_qmd_rope_kv_f16_q4_0_n2w8_rn, cuca_qmd_rope_kv_f16_q4_0_n8w8_rn},
            {cuca_qmd_rope_kv_f16_q8_0_n2w8_rn, cuca_qmd_rope_kv_f16_q8_0_n8w8_rn}}};
        return launch(ctx, table_q8[dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][k > 4096], div_up(a.rows, 32),
                      8 * 64, (unsigned)qmd_lds(a.ng, g), a);
    }
    // the GLU as 8-wave workgroups (32 rows each) when every compute unit
    // gets one: half the workgroups quantise (and normalise) the row
    if ((kind == 1 || kind == 2) && div_up(a.rows, 32) >= (int64_t)ctx->cu_count) {
        // [rn][dtype][format][n2, n8][silu, gelu]
        static const Kernel table_w8[2][2][2][2][2] = {{{{{cuca_qmd_glu_f32_q4_0_silu_n2w8, cuca_qmd_glu_f32_q4_0_gelu_n2w8},
            {cuca_qmd_glu_f32_q4_0_silu_n8w8, cuca_qmd_glu_f32_q4_0_gelu_n8w8}},
            {{cuca_qmd_glu_f32_q8_0_silu_n2w8, cuca_qmd_glu_f32_q8_0_gelu_n2w8},
            {cuca_qmd_glu_f32_q8_0_silu_n8w8, cuca_qmd_glu_f32_q8_0_gelu_n8w8}}},
            {{{cuca_qmd_glu_f16_q4_0_silu_n2w8, cuca_qmd_glu_f16_q4_0_gelu_n2w8},
            {cuca_qmd_glu_f16_q4_0_silu_n8w8, cuca_qmd_glu_f16_q4_0_gelu_n8w8}},
            {{cuca_qmd_glu_f16_q8_0_silu_n2w8, cuca_qmd_glu_f16_q8_0_gelu_n2w8},
            {cuca_qmd_glu_f16_q8_0_silu_n8w8, cuca_qmd_glu_f16_q8_0_gelu_n8w8}}}},
            {{{{cuca_qmd_glu_f32_q4_0_silu_n2w8_rn, cuca_qmd_glu_f32_q4_0_gelu_n2w8_rn},
            {cuca_qmd_glu_f32_q4_0_silu_n8w8_rn, cuca_qmd_glu_f32_q4_0_gelu_n8w8_rn}},
            {{cuca_qmd_glu_f32_q8_0_silu_n2w8_rn, cuca_qmd_glu_f32_q8_0_gelu_n2w8_rn},
            {cuca_qmd_glu_f32_q8_0_silu_n8w8_rn, cuca_qmd_glu_f32_q8_0_gelu_n8w8_rn}}},
            {{{cuca_qmd_glu_f16_q4_0_silu_n2w8_rn, cuca_qmd_glu_f16_q4_0_gelu_n2w8_rn},
            {cuca_qmd_glu_f16_q4_0_silu_n8w8_rn, cuca_qmd_glu_f16_q4_0_gelu_n8w8_rn}},
            {{cuca_qmd_glu_f16_q8_0_silu_n2w8_rn, cuca_qmd_glu_f16_q8_0_gelu_n2w8_rn},
            {cuca_qmd_glu_f16_q8_0_silu_n8w8_rn, cuca_qmd_glu_f16_q8_0_gelu_n8w8_rn}}}}};
        const Kernel k8 = table_w8[rn][dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][k > 4096][kind - 1];
        return launch(ctx, k8, div_up(a.rows, 32), 8 * 64, (unsigned)qmd_lds(a.ng, g), a);
    }
    const Kernel kk = (rn ? table_rn : table_k)[dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][k > 4096][kind];
    return launch(ctx, kk, div_up(a.rows, 16), CUCA_BLOCK_THREADS, (unsigned)qmd_lds(a.ng, g), a);
}

// The residual add + RMSNorm in front of a matmul (the
// cuca_hip_add_rmsnorm_qmm* entry points): cuca_hip_add_rmsnorm(x, branch,
// w, eps, rs) into x_out and h_out, then the matmul of h_out.
struct NormIn {
    const void *x, *branch;
    const float *w;
    float eps, rs;
    void *x_out, *h_out;
};

static bool ranges_overlap(const void *p, const void *q, size_t bytes) {
    if (!p || !q) return false;
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return a < b + bytes && b < a + bytes;
}

// What cuca_hip_add_rmsnorm checks, and that neither output overlaps an
// input (workgroup 0 writes them while the others still read x and branch).
static cuca_status norm_in_check(cuca_hip_ctx *ctx, const NormIn &rn, int64_t m, int64_t k, cuca_dtype dtype) {
    if (!rn.x || !rn.h_out) return fail(ctx, CUCA_INVALID_ARG, "null x or h_out");
    if (!(rn.eps >= 0.0f)) return fail(ctx, CUCA_INVALID_ARG, "eps must be >= 0");
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    const size_t bytes = (size_t)m * (size_t)k * esize(dtype);
    if (ranges_overlap(rn.x_out, rn.x, bytes) || ranges_overlap(rn.x_out, rn.branch, bytes) ||
        ranges_overlap(rn.h_out, rn.x, bytes) || ranges_overlap(rn.h_out, rn.branch, bytes) ||
        ranges_overlap(rn.h_out, rn.x_out, bytes))
        return fail(ctx, CUCA_INVALID_ARG, "add_rmsnorm_qmm: x_out and h_out must not overlap x, branch or each other");
    return CUCA_OK;
}

// Whether the one-row matmul can run the norm as its prologue (with the
// bits of cuca_hip_add_rmsnorm's vector kernel: its shape goes into a).
static bool norm_prologue(const NormIn &rn, int64_t m, int64_t k, cuca_dtype dtype, QmmArgs &a) {
    const int N = chunk_elems(dtype);
    const size_t es = esize(dtype);
    const bool vec = m == 1 && k % N == 0 && al16(rn.x) && al16(rn.h_out) && (!rn.branch || al16(rn.branch)) &&
                     (!rn.x_out || al16(rn.x_out)) && (!rn.w || al16(rn.w)) && ((size_t)k * es) % 16 == 0;
    int tpr = 0, per = 0;
    if (!vec || !norm_shape(k / N, &tpr, &per) || norm_kernel(dtype == CUCA_F16, tpr, per, false) == KERNEL_COUNT)
        return false;
    a.x = rn.x;
    a.rn_branch = rn.branch;
    a.rn_w = rn.w;
    a.rn_x_out = rn.x_out;
    a.rn_h_out = rn.h_out;
    a.rn_eps = rn.eps;
    a.rn_rs = rn.rs;
    a.rn_tpr = tpr;
    a.rn_per = per;
    return true;
}

// The norm as a launch of its own (when the matmul does not take it).
static cuca_status norm_in_launch(cuca_hip_ctx *ctx, const NormIn &rn, int64_t m, int64_t k, cuca_dtype dtype) {
    return cuca_hip_add_rmsnorm(ctx, rn.x, rn.branch, rn.w, nullptr, rn.eps, rn.eps, rn.rs, m, k, rn.x_out,
                                rn.h_out, dtype);
}

// glu: 0 plain, 1 SiLU, 2 GELU-tanh
static cuca_status qmm_common(cuca_hip_ctx *ctx, const void *w, const void *w_up, uint32_t ggml_type,
                              int64_t n, int64_t k, const void *x, int64_t ldx, int64_t m, int64_t rows,
                              int glu, float clamp, void *out, int64_t out_ld, cuca_dtype dtype,
                              const LogitCap &cap = LogitCap(), const NormIn *rn = nullptr) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    // forward_rows (qmm.rs:1823-1825)
    if (rows <= 0 || rows > n)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: %lld weight rows of %lld", (long long)rows, (long long)n);
    if (m < 0 || m > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "qmm: bad activation row count %lld", (long long)m);
    if (ldx < k)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: activation row stride %lld shorter than %lld", (long long)ldx,
                    (long long)k);
    if (out_ld < rows)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: output row stride %lld shorter than %lld", (long long)out_ld,
                    (long long)rows);
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    if (m == 0) return CUCA_OK;
    if (!w || !x || !out || (glu && !w_up)) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    const size_t es = esize(dtype);
    if (!al16(w) || (w_up && !al16(w_up)))
        return fail(ctx, CUCA_INVALID_ARG, "packed weights must be 16-byte aligned");
    if (!al16(x) || ((size_t)ldx * es) % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: activation rows must start 16-byte aligned");
    const int64_t nb = k / 32, ng = (nb + g - 1) / g;
    // one or two rows of a tall matrix whose tile fits the LDS: the decode
    // GEMV stream, each workgroup quantising the rows itself -- except that
    // one row the one-row kernel takes runs there (measured on MI355X, the
    // 128256 x 4096 LM head at one row: Q8_0 101-103 -> 88-89 us, Q4_0 59-60
    // -> 51 us as 8-wave workgroups)
    const bool qmv = m <= 2 && qmv_wins(ctx, rows) && qmv_fits(m, ng * g, g) &&
                     !(m == 1 && qmd_fits(m, k, ng, g, rows, ng * gb));
    if (qmv) {
        if (rn && (st = norm_in_launch(ctx, *rn, m, k, dtype)) != CUCA_OK) return st;
        return qmv_launch(ctx, 3, w, w_up, ggml_type, n, k, nullptr, 0, nullptr, x, ldx, m, rows, glu, clamp, out,
                          out_ld, dtype, cap);
    }
    const bool qmd = qmd_fits(m, k, ng, g, rows, ng * gb);
    const int mt = m == 1 ? 1 : m == 2 ? 2 : 4;
    const int mi = mt == 1 ? 0 : mt == 2 ? 1 : 2;
    const int64_t ntile = (m + mt - 1) / mt;
    const int64_t nrb = (rows + 15) / 16;
    const int64_t nrb8 = (nrb + 7) / 8 * 8;
    if (nrb8 * ntile > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "qmm: grid too large");
    // [dtype][format][plain, silu, gelu][tile rows 1, 2, 4]
    static const Kernel table_k[2][2][3][3] = {
        {{{cuca_qmm_f32_q4_0_m1, cuca_qmm_f32_q4_0_m2, cuca_qmm_f32_q4_0_m4},
          {cuca_qmm_glu_f32_q4_0_silu_m1, cuca_qmm_glu_f32_q4_0_silu_m2, cuca_qmm_glu_f32_q4_0_silu_m4},
          {cuca_qmm_glu_f32_q4_0_gelu_m1, cuca_qmm_glu_f32_q4_0_gelu_m2, cuca_qmm_glu_f32_q4_0_gelu_m4}},
         {{cuca_qmm_f32_q8_0_m1, cuca_qmm_f32_q8_0_m2, cuca_qmm_f32_q8_0_m4},
          {cuca_qmm_glu_f32_q8_0_silu_m1, cuca_qmm_glu_f32_q8_0_silu_m2, cuca_qmm_glu_f32_q8_0_silu_m4},
          {cuca_qmm_glu_f32_q8_0_gelu_m1, cuca_qmm_glu_f32_q8_0_gelu_m2, cuca_qmm_glu_f32_q8_0_gelu_m4}}},
        {{{cuca_qmm_f16_q4_0_m1, cuca_qmm_f16_q4_0_m2, cuca_qmm_f16_q4_0_m4},
          {cuca_qmm_glu_f16_q4_0_silu_m1, cuca_qmm_glu_f16_q4_0_silu_m2, cuca_qmm_glu_f16_q4_0_silu_m4},
          {cuca_qmm_glu_f16_q4_0_gelu_m1, cuca_qmm_glu_f16_q4_0_gelu_m2, cuca_qmm_glu_f16_q4_0_gelu_m4}},
         {{cuca_qmm_f16_q8_0_m1, cuca_qmm_f16_q8_0_m2, cuca_qmm_f16_q8_0_m4},
          {cuca_qmm_glu_f16_q8_0_silu_m1, cuca_qmm_glu_f16_q8_0_silu_m2, cuca_qmm_glu_f16_q8_0_silu_m4},
          {cuca_qmm_glu_f16_q8_0_gelu_m1, cuca_qmm_glu_f16_q8_0_gelu_m2, cuca_qmm_glu_f16_q8_0_gelu_m4}}}};
    const Kernel kk = table_k[dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][glu][mi];
    QmmArgs a{};
    a.w = static_cast<const uint8_t *>(w);
    a.w_up = static_cast<const uint8_t *>(w_up);
    a.x = x;
    a.out = out;
    a.ldx = ldx;
    a.out_ld = out_ld;
    a.row_bytes = ng * gb;
    a.rows = (int32_t)rows;
    a.m = (int32_t)m;
    a.nb = (int32_t)nb;
    a.ng = (int32_t)ng;
    a.nrb = (int32_t)nrb;
    a.ntile = (int32_t)ntile;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    // candle's affine takes its factor as f64 and converts it to f32
    if (cap.logit_scale != 1.0f) { a.cap_flags |= 1; a.mul1 = (float)(1.0 / (double)cap.logit_scale); }
    if (cap.logit_mult != 1.0f) { a.cap_flags |= 2; a.mul2 = cap.logit_mult; }
    if (cap.softcap > 0.0f) {
        a.cap_flags |= 4;
        a.softcap_inv = (float)(1.0 / (double)cap.softcap);
        a.softcap = cap.softcap;
    }
    // one activation row: the decode matmul (the same bits), with the norm
    // as its prologue when asked and its shape allows
    const bool fused = rn && qmd && norm_prologue(*rn, m, k, dtype, a);
    if (rn && !fused && (st = norm_in_launch(ctx, *rn, m, k, dtype)) != CUCA_OK) return st;
    if (qmd) return qmd_launch(ctx, 0, glu, ggml_type, k, g, dtype, a, fused);
    return launch(ctx, kk, (unsigned)(nrb8 * ntile), CUCA_BLOCK_THREADS, 0, a);
}

static cuca_status qmm_rope_kv_common(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t k,
                                      const void *x, int64_t ldx, int64_t m, int32_t nq, int32_t nk,
                                      int32_t head_dim, int32_t n_dims, cuca_rope_kind kind, const float *cos,
                                      const float *sin, int64_t table_rows, const int32_t *positions, void *q_out,
                                      int64_t q_ld, void *pool_k, void *pool_v, int64_t n_blocks,
                                      const int32_t *slots, cuca_dtype dtype, const NormIn *rn) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (kind != CUCA_ROPE_NORM)
        return fail(ctx, kind == CUCA_ROPE_NEOX ? CUCA_UNSUPPORTED : CUCA_INVALID_ARG,
                    "qmm_rope_store_kv: only NORM (adjacent-pair) RoPE rides in the matmul's epilogue; NEOX "
                    "models take cuca_hip_qmm + cuca_hip_rope_store_kv");
    if (nq <= 0 || nk <= 0 || head_dim <= 0 || head_dim % 2 != 0 || n_dims <= 0 || n_dims > head_dim ||
        n_dims % 2 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "qmm_rope_store_kv: bad heads %d/%d x %d, n_dims %d", nq, nk, head_dim,
                    n_dims);
    const int64_t n = (int64_t)(nq + 2 * nk) * head_dim;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (m < 0 || m > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "qmm: bad activation row count %lld", (long long)m);
    if (ldx < k) return fail(ctx, CUCA_INVALID_ARG, "qmm: activation row stride %lld shorter than %lld",
                             (long long)ldx, (long long)k);
    if (q_ld < (int64_t)nq * head_dim)
        return fail(ctx, CUCA_INVALID_ARG, "q row stride %lld shorter than %d heads of %d", (long long)q_ld, nq,
                    head_dim);
    if (n_blocks <= 0 || n_blocks > 0x7fffffffll / CUCA_KV_BLOCK)
        return fail(ctx, CUCA_INVALID_ARG, "bad pool size %lld blocks", (long long)n_blocks);
    if (m == 0) return CUCA_OK;
    if (!w || !x || !q_out || !cos || !sin || !positions || !pool_k || !pool_v || !slots)
        return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (table_rows <= 0) return fail(ctx, CUCA_INVALID_ARG, "empty rope table");
    const size_t es = esize(dtype);
    if (!al16(w)) return fail(ctx, CUCA_INVALID_ARG, "packed weights must be 16-byte aligned");
    if (!al16(x) || ((size_t)ldx * es) % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: activation rows must start 16-byte aligned");
    const int64_t nb = k / 32, ng = (nb + g - 1) / g;
    const int mt = m == 1 ? 1 : m == 2 ? 2 : 4;
    const int mi = mt == 1 ? 0 : mt == 2 ? 1 : 2;
    const int64_t ntile = (m + mt - 1) / mt;
    const int64_t nrb = (n + 15) / 16;
    const int64_t nrb8 = (nrb + 7) / 8 * 8;
    if (nrb8 * ntile > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "qmm: grid too large");
    static const Kernel table_k[2][2][3] = {
        {{cuca_qmm_rope_kv_f32_q4_0_m1, cuca_qmm_rope_kv_f32_q4_0_m2, cuca_qmm_rope_kv_f32_q4_0_m4},
         {cuca_qmm_rope_kv_f32_q8_0_m1, cuca_qmm_rope_kv_f32_q8_0_m2, cuca_qmm_rope_kv_f32_q8_0_m4}},
        {{cuca_qmm_rope_kv_f16_q4_0_m1, cuca_qmm_rope_kv_f16_q4_0_m2, cuca_qmm_rope_kv_f16_q4_0_m4},
         {cuca_qmm_rope_kv_f16_q8_0_m1, cuca_qmm_rope_kv_f16_q8_0_m2, cuca_qmm_rope_kv_f16_q8_0_m4}}};
    QmmArgs a{};
    a.w = static_cast<const uint8_t *>(w);
    a.x = x;
    a.out = q_out;
    a.ldx = ldx;
    a.out_ld = q_ld;
    a.row_bytes = ng * gb;
    a.rows = (int32_t)n;
    a.m = (int32_t)m;
    a.nb = (int32_t)nb;
    a.ng = (int32_t)ng;
    a.nrb = (int32_t)nrb;
    a.ntile = (int32_t)ntile;
    a.status = ctx->status;
    a.cos_t = cos;
    a.sin_t = sin;
    a.pos = positions;
    a.slots = slots;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.table_rows = table_rows;
    a.n_slots = n_blocks * CUCA_KV_BLOCK;
    a.nq = nq;
    a.nk = nk;
    a.head_dim = head_dim;
    a.n_dims = n_dims;
    ctx->last_table_rows = table_rows;
    ctx->last_kv_blocks = n_blocks;
    const bool qmd = qmd_fits(m, k, ng, g, n, ng * gb);
    const bool fused = rn && qmd && norm_prologue(*rn, m, k, dtype, a);
    if (rn && !fused && (st = norm_in_launch(ctx, *rn, m, k, dtype)) != CUCA_OK) return st;
    if (qmd) return qmd_launch(ctx, 3, 0, ggml_type, k, g, dtype, a, fused);
    return launch(ctx, table_k[dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][mi], (unsigned)(nrb8 * ntile),
                  CUCA_BLOCK_THREADS, 0, a);
}

cuca_status cuca_hip_qmm_rope_store_kv(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t k, const void *x,
                                       int64_t ldx, int64_t m, int32_t nq, int32_t nk, int32_t head_dim,
                                       int32_t n_dims, cuca_rope_kind kind, const float *cos, const float *sin,
                                       int64_t table_rows, const int32_t *positions, void *q_out, int64_t q_ld,
                                       void *pool_k, void *pool_v, int64_t n_blocks, const int32_t *slots,
                                       cuca_dtype dtype) {
    return qmm_rope_kv_common(ctx, w, ggml_type, k, x, ldx, m, nq, nk, head_dim, n_dims, kind, cos, sin, table_rows,
                              positions, q_out, q_ld, pool_k, pool_v, n_blocks, slots, dtype, nullptr);
}

cuca_status cuca_hip_add_rmsnorm_qmm_rope_store_kv(cuca_hip_ctx *ctx, const void *x, const void *branch,
                                                   const float *norm_w, float eps, float residual_scale,
                                                   void *x_out, void *h_out, const void *w, uint32_t ggml_type,
                                                   int64_t k, int64_t m, int32_t nq, int32_t nk, int32_t head_dim,
                                                   int32_t n_dims, cuca_rope_kind kind, const float *cos,
                                                   const float *sin, int64_t table_rows, const int32_t *positions,
                                                   void *q_out, int64_t q_ld, void *pool_k, void *pool_v,
                                                   int64_t n_blocks, const int32_t *slots, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    const NormIn rn{x, branch, norm_w, eps, residual_scale, x_out, h_out};
    if (m > 0 && (st = norm_in_check(ctx, rn, m, k, dtype)) != CUCA_OK) return st;
    return qmm_rope_kv_common(ctx, w, ggml_type, k, h_out, k, m, nq, nk, head_dim, n_dims, kind, cos, sin, table_rows,
                              positions, q_out, q_ld, pool_k, pool_v, n_blocks, slots, dtype, &rn);
}

cuca_status cuca_hip_lm_head(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t vocab, int64_t n_embd,
                             const void *x, int64_t ldx, int64_t m, int64_t rows, float logit_scale,
                             float logit_mult, float softcap, void *logits, int64_t logits_ld, cuca_dtype dtype) {
    if (!(logit_scale > 0.0f) || !std::isfinite(logit_scale) || !std::isfinite(logit_mult) ||
        !(softcap >= 0.0f) || !std::isfinite(softcap))
        return fail(ctx, CUCA_INVALID_ARG, "lm head: bad logit scale, multiplier or soft-cap");
    LogitCap cap;
    cap.logit_scale = logit_scale;
    cap.logit_mult = logit_mult;
    cap.softcap = softcap;
    return qmm_common(ctx, w, nullptr, ggml_type, vocab, n_embd, x, ldx, m, rows, 0, 0.0f, logits, logits_ld,
                      dtype, cap);
}

cuca_status cuca_hip_lm_head_indexed_workspace(uint32_t ggml_type, int64_t n_embd, int64_t n_ids, size_t *bytes) {
    if (!bytes) return fail(nullptr, CUCA_INVALID_ARG, "null output pointer");
    if (n_ids < 0) return fail(nullptr, CUCA_INVALID_ARG, "negative count");
    if (n_ids == 0) {
        *bytes = 0;
        return CUCA_OK;
    }
    return cuca_hip_qweight_bytes(ggml_type, n_ids, n_embd, bytes);
}

cuca_status cuca_hip_lm_head_indexed(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t vocab,
                                     int64_t n_embd, const void *x, int64_t ldx, int64_t m, const uint32_t *ids,
                                     int64_t n_ids, float logit_scale, float logit_mult, float softcap,
                                     void *workspace, size_t workspace_bytes, void *logits, int64_t logits_ld,
                                     cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!(logit_scale > 0.0f) || !std::isfinite(logit_scale) || !std::isfinite(logit_mult) ||
        !(softcap >= 0.0f) || !std::isfinite(softcap))
        return fail(ctx, CUCA_INVALID_ARG, "lm head: bad logit scale, multiplier or soft-cap");
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, vocab, n_embd, &g, &gb)) != CUCA_OK) return st;
    if (n_ids < 0 || n_ids > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "bad id count %lld", (long long)n_ids);
    if (m < 0) return fail(ctx, CUCA_INVALID_ARG, "negative count");
    if (n_ids == 0 || m == 0) return CUCA_OK;
    size_t need = 0;
    if ((st = cuca_hip_lm_head_indexed_workspace(ggml_type, n_embd, n_ids, &need)) != CUCA_OK) return st;
    if (!w || !ids || !workspace || !logits) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (workspace_bytes < need)
        return fail(ctx, CUCA_INVALID_ARG, "lm head: workspace of %zu bytes, %zu needed", workspace_bytes, need);
    if (!al16(w) || !al16(workspace)) return fail(ctx, CUCA_INVALID_ARG, "weights and workspace must be 16-byte aligned");
    RowGatherArgs ga{};
    ga.src = static_cast<const uint8_t *>(w);
    ga.ids = ids;
    ga.dst = static_cast<uint8_t *>(workspace);
    ga.status = ctx->status;
    ga.n_src = vocab;
    ga.row_bytes = (int64_t)((n_embd / 32 + g - 1) / g) * gb;
    ga.n = (int32_t)n_ids;
    ctx->last_head_rows = vocab;
    if ((st = launch(ctx, cuca_gather_rows, (unsigned)n_ids, 256u, 0u, ga)) != CUCA_OK) return st;
    LogitCap cap;
    cap.logit_scale = logit_scale;
    cap.logit_mult = logit_mult;
    cap.softcap = softcap;
    return qmm_common(ctx, workspace, nullptr, ggml_type, n_ids, n_embd, x, ldx, m, n_ids, 0, 0.0f, logits, logits_ld,
                      dtype, cap);
}

static cuca_status pick_check(cuca_hip_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t vocab,
                              cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (rows < 0 || rows > 0x7fffffffll || vocab <= 0 || vocab > 0x7fffffffll || ld < vocab)
        return fail(ctx, CUCA_INVALID_ARG, "bad logits shape (%lld rows of %lld, stride %lld)", (long long)rows,
                    (long long)vocab, (long long)ld);
    if (rows > 0 && !logits) return fail(ctx, CUCA_INVALID_ARG, "null logits");
    return CUCA_OK;
}

cuca_status cuca_hip_argmax(cuca_hip_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t vocab,
                            cuca_dtype dtype, uint32_t *ids) {
    cuca_status st = pick_check(ctx, logits, ld, rows, vocab, dtype);
    if (st != CUCA_OK || rows == 0) return st;
    if (!ids) return fail(ctx, CUCA_INVALID_ARG, "null output");
    PickArgs a{};
    a.logits = logits;
    a.out_ids = ids;
    a.ld = ld;
    a.rows = (int32_t)rows;
    a.vocab = (int32_t)vocab;
    // slices of at least 2048 values, enough of them to give the chip four
    // workgroups per CU
    int64_t slices = std::min<int64_t>((vocab + 2047) / 2048, std::max<int64_t>(1, 4 * ctx->cu_count / rows));
    slices = std::min<int64_t>(slices, (int64_t)(kPickScratchBytes / 8) / rows);
    if (slices < 2) slices = 1;
    a.slices = (int32_t)slices;
    a.slice_len = (int32_t)((vocab + slices - 1) / slices);
    a.mode = slices > 1;
    a.cand = static_cast<unsigned long long *>(ctx->pscratch);
    if ((st = launch(ctx, dtype == CUCA_F16 ? cuca_argmax_f16 : cuca_argmax_f32, (unsigned)(rows * slices),
                     CUCA_BLOCK_THREADS, 0, a)) != CUCA_OK || slices == 1)
        return st;
    return launch(ctx, cuca_argmax_merge, (unsigned)div_up(rows, CUCA_BLOCK_THREADS / 64), CUCA_BLOCK_THREADS, 0, a);
}

cuca_status cuca_hip_top_k(cuca_hip_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t vocab,
                           cuca_dtype dtype, int32_t k, float temperature, float *out_logits, uint32_t *out_ids,
                           int32_t *out_count) {
    cuca_status st = pick_check(ctx, logits, ld, rows, vocab, dtype);
    if (st != CUCA_OK || rows == 0) return st;
    if (k <= 0 || k > CUCA_TOP_K_MAX)
        return fail(ctx, CUCA_UNSUPPORTED, "top-k of %d: 1..%d candidates are selected on the device", k,
                    CUCA_TOP_K_MAX);
    if (!(temperature > 0.0f) || !std::isfinite(temperature))
        return fail(ctx, CUCA_INVALID_ARG, "temperature must be positive (greedy is cuca_hip_argmax)");
    if (!out_logits || !out_ids || !out_count) return fail(ctx, CUCA_INVALID_ARG, "null output");
    PickArgs a{};
    a.logits = logits;
    a.out_logits = out_logits;
    a.out_ids = out_ids;
    a.out_count = out_count;
    a.ld = ld;
    a.rows = (int32_t)rows;
    a.vocab = (int32_t)vocab;
    a.k = k;
    a.temperature = temperature;
    // slices of at least 2048 values, two workgroups per CU, at most
    // CUCA_PICK_CAP candidates per row for the merge (one LDS round) and
    // the candidates within the context's scratch
    const int64_t per_slice = (int64_t)k * 8 + 4;
    int64_t slices = std::min<int64_t>((vocab + 2047) / 2048, std::max<int64_t>(1, 2 * ctx->cu_count / rows));
    slices = std::min<int64_t>(slices, std::min<int64_t>(CUCA_PICK_CAP / k, CUCA_PICK_MAX_SLICES));
    slices = std::min<int64_t>(slices, (int64_t)kPickScratchBytes / (rows * per_slice));
    if (slices < 2) slices = 1;
    a.slices = (int32_t)slices;
    a.slice_len = (int32_t)((vocab + slices - 1) / slices);
    a.mode = slices > 1;
    a.cand = static_cast<unsigned long long *>(ctx->pscratch);
    a.cand_count = reinterpret_cast<int32_t *>(static_cast<char *>(ctx->pscratch) + rows * slices * k * 8);
    if ((st = launch(ctx, dtype == CUCA_F16 ? cuca_topk_f16 : cuca_topk_f32, (unsigned)(rows * slices), 1024, 0,
                     a)) != CUCA_OK || slices == 1)
        return st;
    return launch(ctx, cuca_topk_merge, (unsigned)rows, 1024, 0, a);
}

// The rest of sample() after select_top_k (sampler.rs:166-185 and
// :308-334), on the host: softmax of the candidates from the first (the
// largest), probabilities of zero dropped, cut_top_p, one SplitMix64 draw.
// With no candidate the draw still happens, over the greedy fallback.
cuca_status cuca_hip_sample_candidates(const float *logits, const uint32_t *ids, int32_t count, float top_p,
                                       uint32_t fallback, uint64_t *rng_state, uint32_t *out_id) {
    if (!rng_state || !out_id || (count > 0 && (!logits || !ids)))
        return fail(nullptr, CUCA_INVALID_ARG, "null pointer");
    if (count < 0) return fail(nullptr, CUCA_INVALID_ARG, "negative candidate count");
    std::vector<float> p;
    std::vector<uint32_t> id;
    p.reserve((size_t)count);
    id.reserve((size_t)count);
    if (count > 0) {
        const float max = logits[0];
        float sum = 0.0f;
        std::vector<float> e((size_t)count);
        for (int32_t i = 0; i < count; i++) {
            e[(size_t)i] = std::exp(logits[i] - max); // the platform's expf, as Rust's f32::exp
            sum += e[(size_t)i];
        }
        for (int32_t i = 0; i < count; i++) {
            const float v = e[(size_t)i] / sum;
            if (v > 0.0f) { p.push_back(v); id.push_back(ids[i]); }
        }
    }
    if (p.empty()) {
        p.push_back(1.0f);
        id.push_back(fallback);
    } else {
        // cut_top_p (sampler.rs:288-300)
        float cumulative = 0.0f;
        for (size_t i = 0; i < p.size(); i++) {
            cumulative += p[i];
            if (cumulative >= top_p) { p.resize(i + 1); id.resize(i + 1); break; }
        }
    }
    float total = 0.0f;
    for (float v : p) total += v;
    // SplitMix64::next_f32 (sampler.rs:21-35)
    uint64_t z = (*rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const float target = (float)(z >> 40) / 16777216.0f * total;
    float acc = 0.0f;
    *out_id = id.back();
    for (size_t i = 0; i < p.size(); i++) {
        acc += p[i];
        if (target < acc) { *out_id = id[i]; break; }
    }
    return CUCA_OK;
}

cuca_status cuca_hip_qmm(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t n, int64_t k,
                         const void *x, int64_t ldx, int64_t m, int64_t rows, void *out, int64_t out_ld,
                         cuca_dtype dtype) {
    return qmm_common(ctx, w, nullptr, ggml_type, n, k, x, ldx, m, rows, 0, 0.0f, out, out_ld, dtype);
}

cuca_status cuca_hip_qmm_glu(cuca_hip_ctx *ctx, const void *gate, const void *up, uint32_t ggml_type,
                             int64_t ff, int64_t k, const void *x, int64_t ldx, int64_t m, cuca_act act,
                             float clamp, void *out, int64_t out_ld, cuca_dtype dtype) {
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    return qmm_common(ctx, gate, up, ggml_type, ff, k, x, ldx, m, ff, act == CUCA_ACT_SILU ? 1 : 2, clamp,
                      out, out_ld, dtype);
}

cuca_status cuca_hip_add_rmsnorm_qmm(cuca_hip_ctx *ctx, const void *x, const void *branch, const float *norm_w,
                                     float eps, float residual_scale, void *x_out, void *h_out, const void *w,
                                     uint32_t ggml_type, int64_t n, int64_t k, int64_t m, int64_t rows, void *out,
                                     int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    const NormIn rn{x, branch, norm_w, eps, residual_scale, x_out, h_out};
    if (m > 0 && (st = norm_in_check(ctx, rn, m, k, dtype)) != CUCA_OK) return st;
    return qmm_common(ctx, w, nullptr, ggml_type, n, k, h_out, k, m, rows, 0, 0.0f, out, out_ld, dtype, LogitCap(),
                      &rn);
}

cuca_status cuca_hip_add_rmsnorm_qmm_glu(cuca_hip_ctx *ctx, const void *x, const void *branch, const float *norm_w,
                                         float eps, float residual_scale, void *x_out, void *h_out, const void *gate,
                                         const void *up, uint32_t ggml_type, int64_t ff, int64_t k, int64_t m,
                                         cuca_act act, float clamp, void *out, int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    const NormIn rn{x, branch, norm_w, eps, residual_scale, x_out, h_out};
    if (m > 0 && (st = norm_in_check(ctx, rn, m, k, dtype)) != CUCA_OK) return st;
    return qmm_common(ctx, gate, up, ggml_type, ff, k, h_out, k, m, ff, act == CUCA_ACT_SILU ? 1 : 2, clamp, out,
                      out_ld, dtype, LogitCap(), &rn);
}

// ---------------------------------------------------------------------
// the dense f16 path for many rows: a resident f16 copy of the weight and
// the library's f16 GEMM on the matrix cores (gemm16.hip, f32 accumulation)
// ---------------------------------------------------------------------

cuca_status cuca_hip_qweight_dequant(cuca_hip_ctx *ctx, const void *packed, uint32_t ggml_type, int64_t n, int64_t k,
                                     void *w16) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!packed || !w16) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!al16(packed)) return fail(ctx, CUCA_INVALID_ARG, "packed weights must be 16-byte aligned");
    const int64_t nb = k / 32, ng = (nb + g - 1) / g;
    if (n * ng * 16 > 0x7fffffffll * 256) return fail(ctx, CUCA_UNSUPPORTED, "dequant: weight too large");
    QDequantArgs a{};
    a.w = static_cast<const uint8_t *>(packed);
    a.out = w16;
    a.row_bytes = ng * gb;
    a.out_ld = k;
    a.n = n;
    a.k = (int32_t)k;
    a.nb = (int32_t)nb;
    a.ng = (int32_t)ng;
    return launch(ctx, ggml_type == CUCA_GGML_Q8_0 ? cuca_qdequant_q8_0 : cuca_qdequant_q4_0,
                  (unsigned)div_up(n * ng * 16, CUCA_BLOCK_THREADS), CUCA_BLOCK_THREADS, 0, a);
}

// Tiles of 256 (GLU 128) output columns x 256 rows.  A call of fewer than
// 128 tiles splits k (up to 8 ways into equal splits of at least 8 stages of
// 32 values) so that about 256 workgroups run; the splits' f32 sums go to
// the workspace and a reduce launch adds them in split order.  The split
// count follows from the shape alone, so a call's bits do not depend on the
// device.
static int gemm16_splits(int64_t n, int64_t k, int64_t m, bool glu) {
    const int64_t tiles = ((n + (glu ? 127 : 255)) / (glu ? 128 : 256)) * ((m + 255) / 256);
    if (tiles >= 128) return 1;
    const int64_t nst = k / 32;
    int64_t s = std::min<int64_t>(std::min<int64_t>(8, (256 + tiles - 1) / tiles), std::max<int64_t>(1, nst / 8));
    while (nst % s) s--; // equal splits
    return (int)s;
}
// The workspace: the activations rounded to f16 when they come as f32, then
// the split sums.
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
static size_t gemm_w16_ws_x(int64_t k, int64_t m, cuca_dtype dtype) {
    return dtype == CUCA_F32 ? align256((size_t)m * (size_t)k * 2) : 0;
}
static size_t gemm_w16_ws_bytes(int64_t n, int64_t k, int64_t m, bool glu, cuca_dtype dtype) {
    const int sp = gemm16_splits(n, k, m, glu);
    return gemm_w16_ws_x(k, m, dtype) + (sp > 1 ? (size_t)sp * (glu ? 2 : 1) * (size_t)m * (size_t)n * 4 : 0);
}

cuca_status cuca_hip_gemm_w16_workspace(int64_t n, int64_t k, int64_t m, int32_t glu, cuca_dtype dtype,
                                        size_t *bytes) {
    if (!bytes) return fail(nullptr, CUCA_INVALID_ARG, "null pointer");
    if (n <= 0 || k <= 0 || k % 32 != 0 || m < 0 || m > 0x7fffffffll || !dtype_ok(dtype))
        return fail(nullptr, CUCA_INVALID_ARG, "gemm: bad shape %lld x %lld, %lld rows", (long long)n, (long long)k,
                    (long long)m);
    *bytes = gemm_w16_ws_bytes(n, k, m, glu != 0, dtype);
    return CUCA_OK;
}

// Row strides the kernel addresses with 32-bit byte offsets within a tile
// of 256 rows.
constexpr int64_t kGemm16MaxLd = 1ll << 22;

// glu: 0 plain, 1 SiLU, 2 GELU-tanh; w16 [n][k] (gate rows, then up rows
// for the GLU: n = 2 ff).
static cuca_status gemm_w16_common(cuca_hip_ctx *ctx, const void *w16, int64_t n, int64_t k, const void *x,
                                   int64_t ldx, int64_t m, int64_t rows, int glu, float clamp, void *ws,
                                   size_t ws_bytes, void *out, int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (n <= 0 || k <= 0 || k % 32 != 0 || k > 0x7fffffffll)
        return fail(ctx, CUCA_INVALID_ARG, "gemm: bad weight shape %lld x %lld", (long long)n, (long long)k);
    if (rows <= 0 || rows > n)
        return fail(ctx, CUCA_INVALID_ARG, "gemm: %lld weight rows of %lld", (long long)rows, (long long)n);
    if (m < 0 || m > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "gemm: bad activation row count %lld", (long long)m);
    if (ldx < k)
        return fail(ctx, CUCA_INVALID_ARG, "gemm: activation row stride %lld shorter than %lld", (long long)ldx,
                    (long long)k);
    if (out_ld < (glu ? n / 2 : rows))
        return fail(ctx, CUCA_INVALID_ARG, "gemm: output row stride %lld too short", (long long)out_ld);
    if (k >= kGemm16MaxLd || ldx >= kGemm16MaxLd)
        return fail(ctx, CUCA_UNSUPPORTED, "gemm: row strides from %lld values on are not supported",
                    (long long)kGemm16MaxLd);
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    if (m == 0) return CUCA_OK;
    const int64_t ncols = glu ? n / 2 : rows; // output columns
    const size_t need = gemm_w16_ws_bytes(ncols, k, m, glu != 0, dtype);
    if (!w16 || !x || !out || (need && !ws)) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    const size_t es = esize(dtype);
    if (!al16(w16) || !al16(x) || !al16(out) || (ws && !al16(ws)) || ((size_t)ldx * es) % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "gemm: weights, rows, output and workspace must be 16-byte aligned");
    if (ws_bytes < need)
        return fail(ctx, CUCA_INVALID_ARG, "gemm: workspace of %zu bytes, %zu needed (cuca_hip_gemm_w16_workspace)",
                    ws_bytes, need);
    const void *xh = x;
    int64_t ldxh = ldx;
    if (dtype == CUCA_F32) { // the activations rounded to f16 once
        QDequantArgs c{};
        c.x = x;
        c.out = ws;
        c.ldx = ldx;
        c.out_ld = k;
        c.m = (int32_t)m;
        c.k = (int32_t)k;
        if ((st = launch(ctx, cuca_cvt_f16_f32, (unsigned)div_up(m * (k / 8), CUCA_BLOCK_THREADS),
                         CUCA_BLOCK_THREADS, 0, c)) != CUCA_OK)
            return st;
        xh = ws;
        ldxh = k;
    }
    const bool f16 = dtype == CUCA_F16;
    const int splits = gemm16_splits(ncols, k, m, glu != 0);
    Gemm16Args a{};
    a.w = w16;
    a.x = xh;
    a.ldw = k;
    a.ldx = ldxh;
    a.m = (int32_t)m;
    a.n_tm = (int32_t)div_up(m, 256);
    a.gn = 8;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    a.splits = splits;
    // The GLU form runs as 8 waves a workgroup (two a SIMD), the plain form
    // as 4 (gemm16.hip: measured with the launches of the forms interleaved,
    // the 8-wave GLU 7 % faster at 4096 rows, the 8-wave plain form no faster).
    // [f16 output][SiLU, GELU]
    static const Kernel k8[2][2] = {{cuca_gemm16_w8_glu_f32_silu, cuca_gemm16_w8_glu_f32_gelu},
                                    {cuca_gemm16_w8_glu_f16_silu, cuca_gemm16_w8_glu_f16_gelu}};
    Kernel kern;
    bool w8;
    if (splits == 1) {
        a.out = out;
        a.out_ld = out_ld;
        a.up_row = glu ? n / 2 : 0;
        a.n = (int32_t)ncols;
        a.k = (int32_t)k;
        a.n_tn = (int32_t)div_up(ncols, glu ? 128 : 256);
        a.vec = out_ld % 4 == 0 ? 1 : 0;
        w8 = glu != 0;
        kern = w8 ? k8[f16][glu - 1] : (f16 ? cuca_gemm16_f16 : cuca_gemm16_f32);
    } else {
        // the plain form over every weight row the call reads (the GLU's gate
        // rows, then its up rows), k / splits values per split, each split's
        // f32 sums to its own [m][width] matrix of the workspace
        const int64_t width = glu ? n : ncols;
        a.part = reinterpret_cast<float *>(static_cast<char *>(ws) + gemm_w16_ws_x(k, m, dtype));
        a.out = a.part;
        a.out_ld = width;
        a.n = (int32_t)width;
        a.k = (int32_t)(k / splits);
        a.n_tn = (int32_t)div_up(width, 256);
        a.vec = width % 4 == 0 ? 1 : 0;
        w8 = false;
        kern = cuca_gemm16_f32;
    }
    const int64_t tiles = (int64_t)a.n_tn * a.n_tm;
    if (tiles > 0x7ffffff8ll) return fail(ctx, CUCA_UNSUPPORTED, "gemm: grid too large");
    // every XCD (workgroups x, x + 8, ...) gets ceil(tiles / 8) workgroups
    if ((st = launch2(ctx, kern, (unsigned)(8 * div_up(tiles, 8)), (unsigned)splits, w8 ? 512u : 256u, 0, a)) !=
            CUCA_OK ||
        splits == 1)
        return st;
    Gemm16Args r{};
    r.part = a.part;
    r.out = out;
    r.out_ld = out_ld;
    r.n = (int32_t)ncols;
    r.m = (int32_t)m;
    r.splits = splits;
    r.clamp = a.clamp;
    static const Kernel red_k[2][3] = {
        {cuca_gemm16_reduce_f32, cuca_gemm16_reduce_glu_f32_silu, cuca_gemm16_reduce_glu_f32_gelu},
        {cuca_gemm16_reduce_f16, cuca_gemm16_reduce_glu_f16_silu, cuca_gemm16_reduce_glu_f16_gelu}};
    return launch(ctx, red_k[f16][glu], div_up(m * ncols, CUCA_BLOCK_THREADS), CUCA_BLOCK_THREADS, 0, r);
}

cuca_status cuca_hip_gemm_w16(cuca_hip_ctx *ctx, const void *w16, int64_t n, int64_t k, const void *x, int64_t ldx,
                              int64_t m, int64_t rows, void *workspace, size_t workspace_bytes, void *out,
                              int64_t out_ld, cuca_dtype dtype) {
    return gemm_w16_common(ctx, w16, n, k, x, ldx, m, rows, 0, 0.0f, workspace, workspace_bytes, out, out_ld, dtype);
}

cuca_status cuca_hip_gemm_w16_glu(cuca_hip_ctx *ctx, const void *w16, int64_t ff, int64_t k, const void *x,
                                  int64_t ldx, int64_t m, cuca_act act, float clamp, void *workspace,
                                  size_t workspace_bytes, void *out, int64_t out_ld, cuca_dtype dtype) {
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    if (ff <= 0 || ff > 0x3fffffffll) return fail(ctx, CUCA_INVALID_ARG, "gemm glu: bad ff %lld", (long long)ff);
    return gemm_w16_common(ctx, w16, 2 * ff, k, x, ldx, m, 2 * ff, act == CUCA_ACT_SILU ? 1 : 2, clamp, workspace,
                           workspace_bytes, out, out_ld, dtype);
}

// The matrix-core matmul (qgemm.hip): the workspace holds the activations
// in slot order (f16, kp values per row) and, up to 2048 rows, the split
// sums (up to kQgMaxSplits splits of f32 rows, two per output with the GLU)
// that grids of fewer workgroups than CUs use.
constexpr int64_t kQgMaxSplits = 8;
constexpr int64_t kQgMaxK = 1ll << 28; // in-kernel offsets of a few rows of kp values stay within int32

static int64_t qgemm_kp(int g, int64_t k) {
    const int64_t ng = (k / 32 + g - 1) / g;
    return ng * g * 32;
}
// tokens per tile, and the activation rows of the workspace: whole tiles,
// the rows past m zero
static int qgemm_tm(int64_t m) { return m <= 32 ? 32 : m <= 64 ? 64 : 128; }
static int64_t qgemm_mp(int64_t m) {
    const int tm = qgemm_tm(m);
    return (m + tm - 1) / tm * tm;
}
static size_t qgemm_xp_bytes(int g, int64_t k, int64_t m) {
    return ((size_t)qgemm_mp(m) * (size_t)qgemm_kp(g, k) * 2 + 255) / 256 * 256;
}
static size_t qgemm_ws_bytes(int g, int64_t n, int64_t k, int64_t m, bool glu) {
    const size_t xp = qgemm_xp_bytes(g, k, m);
    const size_t part = m <= 2048 ? (size_t)kQgMaxSplits * (glu ? 2 : 1) * (size_t)m * (size_t)n * 4 : 0;
    return xp + part;
}

cuca_status cuca_hip_qgemm_workspace(uint32_t ggml_type, int64_t n, int64_t k, int64_t m, int32_t glu, size_t *bytes) {
    if (!bytes) return fail(nullptr, CUCA_INVALID_ARG, "null pointer");
    int g = 0, gb = 0;
    if (!qfmt(ggml_type, &g, &gb)) return fail(nullptr, CUCA_UNSUPPORTED, "qgemm: ggml type %u", ggml_type);
    if (n <= 0 || k <= 0 || k % 32 != 0 || m < 0 || m > 0x7fffffffll)
        return fail(nullptr, CUCA_INVALID_ARG, "qgemm: bad shape %lld x %lld, %lld rows", (long long)n, (long long)k,
                    (long long)m);
    if (k > kQgMaxK) return fail(nullptr, CUCA_UNSUPPORTED, "qgemm: rows of more than %lld values", (long long)kQgMaxK);
    *bytes = qgemm_ws_bytes(g, n, k, m, glu != 0);
    return CUCA_OK;
}

// glu: 0 plain, 1 SiLU, 2 GELU-tanh.
static cuca_status qgemm_common(cuca_hip_ctx *ctx, const void *w, const void *w_up, uint32_t ggml_type, int64_t n,
                                int64_t k, const void *x, int64_t ldx, int64_t m, int64_t rows, int glu, float clamp,
                                void *ws, size_t ws_bytes, void *out, int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (rows <= 0 || rows > n)
        return fail(ctx, CUCA_INVALID_ARG, "qgemm: %lld weight rows of %lld", (long long)rows, (long long)n);
    if (m < 0 || m > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "qgemm: bad activation row count %lld", (long long)m);
    if (k > kQgMaxK) return fail(ctx, CUCA_UNSUPPORTED, "qgemm: rows of more than %lld values", (long long)kQgMaxK);
    if (ldx < k)
        return fail(ctx, CUCA_INVALID_ARG, "qgemm: activation row stride %lld shorter than %lld", (long long)ldx,
                    (long long)k);
    if (out_ld < rows)
        return fail(ctx, CUCA_INVALID_ARG, "qgemm: output row stride %lld shorter than %lld", (long long)out_ld,
                    (long long)rows);
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    if (m == 0) return CUCA_OK;
    if (!w || !x || !out || !ws || (glu && !w_up)) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!al16(w) || (w_up && !al16(w_up)) || !al16(ws))
        return fail(ctx, CUCA_INVALID_ARG, "packed weights and the workspace must be 16-byte aligned");
    const int64_t kp = qgemm_kp(g, k);
    const size_t xp_bytes = qgemm_xp_bytes(g, k, m);
    if (ws_bytes < xp_bytes)
        return fail(ctx, CUCA_INVALID_ARG, "qgemm: workspace of %zu bytes, %zu needed (cuca_hip_qgemm_workspace)",
                    ws_bytes, xp_bytes);
    const int tm = qgemm_tm(m);
    const int ti = tm == 32 ? 0 : tm == 64 ? 1 : 2;
    const int64_t n_rt = (rows + 127) / 128, n_ct = qgemm_mp(m) / tm;
    const int64_t tiles = (n_rt + 7) / 8 * 8 * n_ct;
    const int64_t nkc = kp / 128;
    if (tiles > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "qgemm: grid too large");
    // split k for grids smaller than the CU count: up to two workgroups per
    // CU, at least 4 k-chunks per split, within the workspace given
    int64_t splits = 1;
    const size_t split_row = (size_t)(glu ? 2 : 1) * (size_t)m * (size_t)rows * 4;
    if (m <= 2048 && tiles < ctx->cu_count) {
        splits = std::min<int64_t>(kQgMaxSplits, std::min<int64_t>((2 * ctx->cu_count + tiles - 1) / tiles, nkc / 4));
        splits = std::min<int64_t>(splits, (int64_t)((ws_bytes - xp_bytes) / split_row));
        if (splits < 2) splits = 1;
    }
    const int64_t kcs = (nkc + splits - 1) / splits;
    splits = (nkc + kcs - 1) / kcs;
    QGemmArgs a{};
    a.w = static_cast<const uint8_t *>(w);
    a.w_up = static_cast<const uint8_t *>(w_up);
    a.x = x;
    a.xp = static_cast<uint16_t *>(ws);
    a.part = reinterpret_cast<float *>(static_cast<char *>(ws) + xp_bytes);
    a.out = out;
    a.ldx = ldx;
    a.out_ld = out_ld;
    a.row_bytes = (kp / 32 / g) * gb;
    a.kp = kp;
    a.rows = (int32_t)rows;
    a.m = (int32_t)m;
    a.k = (int32_t)k;
    a.nkc = (int32_t)nkc;
    a.n_rt = (int32_t)n_rt;
    a.n_ct = (int32_t)n_ct;
    a.kcs = (int32_t)kcs;
    a.splits = (int32_t)splits;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    a.mp = (int32_t)(n_ct * tm);
    const bool f16 = dtype == CUCA_F16, q8 = ggml_type == CUCA_GGML_Q8_0;
    static const Kernel prep_k[2][2] = {{cuca_qgemm_prep_f32_q4_0, cuca_qgemm_prep_f32_q8_0},
                                        {cuca_qgemm_prep_f16_q4_0, cuca_qgemm_prep_f16_q8_0}};
    if ((st = launch(ctx, prep_k[f16][q8], div_up((int64_t)a.mp * nkc * 16, CUCA_BLOCK_THREADS), CUCA_BLOCK_THREADS, 0,
                     a)) != CUCA_OK)
        return st;
    // [dtype][format][plain, silu, gelu][tokens per tile 32, 64, 128]
    static const Kernel table_k[2][2][3][3] = {
        {{{cuca_qgemm_f32_q4_0_t32, cuca_qgemm_f32_q4_0_t64, cuca_qgemm_f32_q4_0_t128},
          {cuca_qgemm_glu_f32_q4_0_silu_t32, cuca_qgemm_glu_f32_q4_0_silu_t64, cuca_qgemm_glu_f32_q4_0_silu_t128},
          {cuca_qgemm_glu_f32_q4_0_gelu_t32, cuca_qgemm_glu_f32_q4_0_gelu_t64, cuca_qgemm_glu_f32_q4_0_gelu_t128}},
         {{cuca_qgemm_f32_q8_0_t32, cuca_qgemm_f32_q8_0_t64, cuca_qgemm_f32_q8_0_t128},
          {cuca_qgemm_glu_f32_q8_0_silu_t32, cuca_qgemm_glu_f32_q8_0_silu_t64, cuca_qgemm_glu_f32_q8_0_silu_t128},
          {cuca_qgemm_glu_f32_q8_0_gelu_t32, cuca_qgemm_glu_f32_q8_0_gelu_t64, cuca_qgemm_glu_f32_q8_0_gelu_t128}}},
        {{{cuca_qgemm_f16_q4_0_t32, cuca_qgemm_f16_q4_0_t64, cuca_qgemm_f16_q4_0_t128},
          {cuca_qgemm_glu_f16_q4_0_silu_t32, cuca_qgemm_glu_f16_q4_0_silu_t64, cuca_qgemm_glu_f16_q4_0_silu_t128},
          {cuca_qgemm_glu_f16_q4_0_gelu_t32, cuca_qgemm_glu_f16_q4_0_gelu_t64, cuca_qgemm_glu_f16_q4_0_gelu_t128}},
         {{cuca_qgemm_f16_q8_0_t32, cuca_qgemm_f16_q8_0_t64, cuca_qgemm_f16_q8_0_t128},
          {cuca_qgemm_glu_f16_q8_0_silu_t32, cuca_qgemm_glu_f16_q8_0_silu_t64, cuca_qgemm_glu_f16_q8_0_silu_t128},
          {cuca_qgemm_glu_f16_q8_0_gelu_t32, cuca_qgemm_glu_f16_q8_0_gelu_t64, cuca_qgemm_glu_f16_q8_0_gelu_t128}}}};
    // [dtype][format][plain, glu][tokens per tile]
    static const Kernel split_k[2][2][2][3] = {
        {{{cuca_qgemm_f32_q4_0_t32_split, cuca_qgemm_f32_q4_0_t64_split, cuca_qgemm_f32_q4_0_t128_split},
          {cuca_qgemm_glu_f32_q4_0_t32_split, cuca_qgemm_glu_f32_q4_0_t64_split, cuca_qgemm_glu_f32_q4_0_t128_split}},
         {{cuca_qgemm_f32_q8_0_t32_split, cuca_qgemm_f32_q8_0_t64_split, cuca_qgemm_f32_q8_0_t128_split},
          {cuca_qgemm_glu_f32_q8_0_t32_split, cuca_qgemm_glu_f32_q8_0_t64_split, cuca_qgemm_glu_f32_q8_0_t128_split}}},
        {{{cuca_qgemm_f16_q4_0_t32_split, cuca_qgemm_f16_q4_0_t64_split, cuca_qgemm_f16_q4_0_t128_split},
          {cuca_qgemm_glu_f16_q4_0_t32_split, cuca_qgemm_glu_f16_q4_0_t64_split, cuca_qgemm_glu_f16_q4_0_t128_split}},
         {{cuca_qgemm_f16_q8_0_t32_split, cuca_qgemm_f16_q8_0_t64_split, cuca_qgemm_f16_q8_0_t128_split},
          {cuca_qgemm_glu_f16_q8_0_t32_split, cuca_qgemm_glu_f16_q8_0_t64_split, cuca_qgemm_glu_f16_q8_0_t128_split}}}};
    if (splits == 1) return launch(ctx, table_k[f16][q8][glu][ti], (unsigned)tiles, 256, 0, a);
    if ((st = launch2(ctx, split_k[f16][q8][glu != 0][ti], (unsigned)tiles, (unsigned)splits, 256, 0, a)) != CUCA_OK)
        return st;
    static const Kernel red_k[2][3] = {{cuca_qgemm_reduce_f32, cuca_qgemm_reduce_glu_f32_silu, cuca_qgemm_reduce_glu_f32_gelu},
                                       {cuca_qgemm_reduce_f16, cuca_qgemm_reduce_glu_f16_silu, cuca_qgemm_reduce_glu_f16_gelu}};
    return launch(ctx, red_k[f16][glu], div_up(m * rows, CUCA_BLOCK_THREADS), CUCA_BLOCK_THREADS, 0, a);
}

cuca_status cuca_hip_qgemm(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t n, int64_t k, const void *x,
                           int64_t ldx, int64_t m, int64_t rows, void *workspace, size_t workspace_bytes, void *out,
                           int64_t out_ld, cuca_dtype dtype) {
    return qgemm_common(ctx, w, nullptr, ggml_type, n, k, x, ldx, m, rows, 0, 0.0f, workspace, workspace_bytes, out,
                        out_ld, dtype);
}

cuca_status cuca_hip_qgemm_glu(cuca_hip_ctx *ctx, const void *gate, const void *up, uint32_t ggml_type, int64_t ff,
                               int64_t k, const void *x, int64_t ldx, int64_t m, cuca_act act, float clamp,
                               void *workspace, size_t workspace_bytes, void *out, int64_t out_ld, cuca_dtype dtype) {
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    return qgemm_common(ctx, gate, up, ggml_type, ff, k, x, ldx, m, ff, act == CUCA_ACT_SILU ? 1 : 2, clamp, workspace,
                        workspace_bytes, out, out_ld, dtype);
}

static cuca_status qmv_launch(cuca_hip_ctx *ctx, int mode, const void *w, const void *w_up, uint32_t ggml_type,
                              int64_t n, int64_t k, const int8_t *quants, int64_t q_ld, const float *scales,
                              const void *x, int64_t ldx, int64_t m, int64_t rows, int glu, float clamp, void *out,
                              int64_t out_ld, cuca_dtype dtype, const LogitCap &cap) {
    int g = 0, gb = 0;
    qfmt(ggml_type, &g, &gb);
    const int64_t nb = k / 32, ng = (nb + g - 1) / g, nbp = ng * g;
    const int64_t ntask = (rows + 3) / 4;
    int64_t grid = (ntask + 3) / 4;
    const int64_t cap_wg = (int64_t)ctx->cu_count * 4; // persistent beyond four workgroups per CU
    if (grid > cap_wg) grid = cap_wg;
    // [rows of x][dtype][format][plain, silu, gelu][rows 1, 2]
    static const Kernel table_k[2][2][2][3][2] = {
        {{{{cuca_qmv_q4_0_m1_f32, cuca_qmv_q4_0_m2_f32},
           {cuca_qmv_glu_q4_0_silu_m1_f32, cuca_qmv_glu_q4_0_silu_m2_f32},
           {cuca_qmv_glu_q4_0_gelu_m1_f32, cuca_qmv_glu_q4_0_gelu_m2_f32}},
          {{cuca_qmv_q8_0_m1_f32, cuca_qmv_q8_0_m2_f32},
           {cuca_qmv_glu_q8_0_silu_m1_f32, cuca_qmv_glu_q8_0_silu_m2_f32},
           {cuca_qmv_glu_q8_0_gelu_m1_f32, cuca_qmv_glu_q8_0_gelu_m2_f32}}},
         {{{cuca_qmv_q4_0_m1_f16, cuca_qmv_q4_0_m2_f16},
           {cuca_qmv_glu_q4_0_silu_m1_f16, cuca_qmv_glu_q4_0_silu_m2_f16},
           {cuca_qmv_glu_q4_0_gelu_m1_f16, cuca_qmv_glu_q4_0_gelu_m2_f16}},
          {{cuca_qmv_q8_0_m1_f16, cuca_qmv_q8_0_m2_f16},
           {cuca_qmv_glu_q8_0_silu_m1_f16, cuca_qmv_glu_q8_0_silu_m2_f16},
           {cuca_qmv_glu_q8_0_gelu_m1_f16, cuca_qmv_glu_q8_0_gelu_m2_f16}}}},
        {{{{cuca_qmvx_q4_0_m1_f32, cuca_qmvx_q4_0_m2_f32},
           {cuca_qmvx_glu_q4_0_silu_m1_f32, cuca_qmvx_glu_q4_0_silu_m2_f32},
           {cuca_qmvx_glu_q4_0_gelu_m1_f32, cuca_qmvx_glu_q4_0_gelu_m2_f32}},
          {{cuca_qmvx_q8_0_m1_f32, cuca_qmvx_q8_0_m2_f32},
           {cuca_qmvx_glu_q8_0_silu_m1_f32, cuca_qmvx_glu_q8_0_silu_m2_f32},
           {cuca_qmvx_glu_q8_0_gelu_m1_f32, cuca_qmvx_glu_q8_0_gelu_m2_f32}}},
         {{{cuca_qmvx_q4_0_m1_f16, cuca_qmvx_q4_0_m2_f16},
           {cuca_qmvx_glu_q4_0_silu_m1_f16, cuca_qmvx_glu_q4_0_silu_m2_f16},
           {cuca_qmvx_glu_q4_0_gelu_m1_f16, cuca_qmvx_glu_q4_0_gelu_m2_f16}},
          {{cuca_qmvx_q8_0_m1_f16, cuca_qmvx_q8_0_m2_f16},
           {cuca_qmvx_glu_q8_0_silu_m1_f16, cuca_qmvx_glu_q8_0_silu_m2_f16},
           {cuca_qmvx_glu_q8_0_gelu_m1_f16, cuca_qmvx_glu_q8_0_gelu_m2_f16}}}}};
    const Kernel kk = table_k[mode == 3][dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][glu][m == 2];
    QmvArgs a{};
    a.w = static_cast<const uint8_t *>(w);
    a.w_up = static_cast<const uint8_t *>(w_up);
    a.quants = quants;
    a.scales = scales;
    a.x = x;
    a.out = out;
    a.q_ld = q_ld;
    a.ldx = ldx;
    a.out_ld = out_ld;
    a.row_bytes = ng * gb;
    a.rows = (int32_t)rows;
    a.m = (int32_t)m;
    a.nb = (int32_t)nb;
    a.ng = (int32_t)ng;
    a.nbp = (int32_t)nbp;
    a.ntask = (int32_t)ntask;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    if (cap.logit_scale != 1.0f) { a.cap_flags |= 1; a.mul1 = (float)(1.0 / (double)cap.logit_scale); }
    if (cap.logit_mult != 1.0f) { a.cap_flags |= 2; a.mul2 = cap.logit_mult; }
    if (cap.softcap > 0.0f) {
        a.cap_flags |= 4;
        a.softcap_inv = (float)(1.0 / (double)cap.softcap);
        a.softcap = cap.softcap;
    }
    return launch(ctx, kk, (unsigned)grid, CUCA_BLOCK_THREADS, (unsigned)qmv_lds(m, nbp, g), a);
}

cuca_status cuca_hip_q8_acts(cuca_hip_ctx *ctx, const void *x, int64_t ldx, int64_t m, int64_t k, cuca_dtype dtype,
                             int8_t *quants, float *scales) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (k <= 0 || k % 32 != 0 || k / 32 > 0x7fffffffll)
        return fail(ctx, CUCA_INVALID_ARG, "q8 acts: row length %lld is not a whole number of blocks", (long long)k);
    if (m < 0 || m * (k / 32) > 0x7fffffffll) return fail(ctx, CUCA_INVALID_ARG, "q8 acts: bad row count %lld", (long long)m);
    if (ldx < k) return fail(ctx, CUCA_INVALID_ARG, "q8 acts: row stride %lld shorter than %lld", (long long)ldx, (long long)k);
    if (m == 0) return CUCA_OK;
    if (!x || !quants || !scales) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!al16(x) || ((size_t)ldx * esize(dtype)) % 16 != 0 || !al16(quants) || k % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "q8 acts: rows must start 16-byte aligned");
    return q8_acts_launch(ctx, x, ldx, m, k, dtype, quants, k, scales);
}

static cuca_status qmv_common(cuca_hip_ctx *ctx, const void *w, const void *w_up, uint32_t ggml_type, int64_t n,
                              int64_t k, const int8_t *quants, const float *scales, int64_t m, int64_t rows, int glu,
                              float clamp, void *out, int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (rows <= 0 || rows > n)
        return fail(ctx, CUCA_INVALID_ARG, "qmm: %lld weight rows of %lld", (long long)rows, (long long)n);
    if (out_ld < rows) return fail(ctx, CUCA_INVALID_ARG, "qmm: output row stride %lld shorter than %lld",
                                   (long long)out_ld, (long long)rows);
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    const int64_t ng = (k / 32 + g - 1) / g;
    if (m == 0) return CUCA_OK;
    if (!qmv_fits(m, ng * g, g))
        return fail(ctx, CUCA_UNSUPPORTED, "qmv: %lld rows of %lld values do not fit the decode GEMV (1 or 2 rows; "
                    "cuca_hip_qmm takes any)", (long long)m, (long long)k);
    if (!w || !quants || !scales || !out || (glu && !w_up)) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (!al16(w) || (w_up && !al16(w_up))) return fail(ctx, CUCA_INVALID_ARG, "packed weights must be 16-byte aligned");
    return qmv_launch(ctx, 0, w, w_up, ggml_type, n, k, quants, k, scales, nullptr, 0, m, rows, glu, clamp, out,
                      out_ld, dtype, LogitCap());
}

cuca_status cuca_hip_qmv(cuca_hip_ctx *ctx, const void *w, uint32_t ggml_type, int64_t n, int64_t k,
                         const int8_t *quants, const float *scales, int64_t m, int64_t rows, void *out, int64_t out_ld,
                         cuca_dtype dtype) {
    return qmv_common(ctx, w, nullptr, ggml_type, n, k, quants, scales, m, rows, 0, 0.0f, out, out_ld, dtype);
}

cuca_status cuca_hip_qmv_glu(cuca_hip_ctx *ctx, const void *gate, const void *up, uint32_t ggml_type, int64_t ff,
                             int64_t k, const int8_t *quants, const float *scales, int64_t m, cuca_act act, float clamp,
                             void *out, int64_t out_ld, cuca_dtype dtype) {
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    return qmv_common(ctx, gate, up, ggml_type, ff, k, quants, scales, m, ff, act == CUCA_ACT_SILU ? 1 : 2, clamp,
                      out, out_ld, dtype);
}

// MoE (expert_sum, cpu.rs:3599-3642; the reference GPU engine's moe_up /
// moe_down / moe_sum, moe_kernel.rs:1163-1385).  Pairs are grouped by
// expert: expert e owns pairs [offsets[e], offsets[e+1]) of the pair arrays,
// which hold max_pairs entries; the counts are read on the device.
// up: 1 SiLU, 2 GELU-tanh; 0 = down.
static cuca_status moe_common(cuca_hip_ctx *ctx, const void *w, const void *w_up, int64_t estride,
                              uint32_t ggml_type, int64_t n, int64_t k, int32_t n_experts, const void *x,
                              int64_t ldx, int64_t n_tokens, const int32_t *offsets, const int32_t *pair_token,
                              const float *pair_weight, int64_t max_pairs, int up, float clamp, void *out,
                              int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (n_experts <= 0) return fail(ctx, CUCA_INVALID_ARG, "moe: bad expert count %d", n_experts);
    if (max_pairs < 0 || max_pairs > 0x7fffffffll)
        return fail(ctx, CUCA_INVALID_ARG, "moe: bad pair capacity %lld", (long long)max_pairs);
    if (ldx < k) return fail(ctx, CUCA_INVALID_ARG, "moe: activation row stride %lld shorter than %lld",
                             (long long)ldx, (long long)k);
    if (out_ld < n) return fail(ctx, CUCA_INVALID_ARG, "moe: output row stride %lld shorter than %lld",
                                (long long)out_ld, (long long)n);
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    if (max_pairs == 0) return CUCA_OK;
    if (!w || !x || !out || !offsets || (up && (!w_up || !pair_token)) || (!up && !pair_weight))
        return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (up && (n_tokens <= 0 || n_tokens > 0x7fffffffll))
        return fail(ctx, CUCA_INVALID_ARG, "moe: bad token count %lld", (long long)n_tokens);
    const int64_t nb = k / 32, ng = (nb + g - 1) / g;
    const int64_t packed = n * ng * gb;
    if (estride < packed || estride % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "moe: expert stride %lld bytes, at least %lld (a multiple of 16) needed",
                    (long long)estride, (long long)packed);
    const size_t es = esize(dtype);
    if (!al16(w) || (w_up && !al16(w_up))) return fail(ctx, CUCA_INVALID_ARG, "packed weights must be 16-byte aligned");
    if (!al16(x) || ((size_t)ldx * es) % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "moe: activation rows must start 16-byte aligned");
    // tile rows from the mean pairs per expert
    const double mean = (double)max_pairs / (double)n_experts;
    const int mt = mean <= 1.5 ? 1 : mean <= 3.0 ? 2 : 4;
    const int mi = mt == 1 ? 0 : mt == 2 ? 1 : 2;
    // an upper bound of the tiles, sum over experts of ceil(n_e / mt): at
    // most min(n_experts, pairs) experts hold pairs, each adding at most
    // (mt - 1) / mt of a tile to pairs / mt
    const int64_t ntile = (max_pairs + (mt - 1) * std::min<int64_t>(n_experts, max_pairs)) / mt;
    // the decode GEMV, a workgroup per (tile, split of the expert's rows),
    // when the tile's rows fit its LDS, from two tokens' pairs up (16 pairs
    // over 128 experts; measured at Qwen3-30B-A3B's shapes: 34 vs 36 us at
    // two tokens, 159 vs 448 us at 32); a single token's pairs keep the
    // one-pass kernel (25 vs 30 us)
    if (16 * max_pairs > n_experts && qmv_lds(mt, ng * g, g) <= (64u << 10)) {
        const int64_t ntask = (n + 3) / 4;
        int64_t splits = std::max<int64_t>(1, ((int64_t)ctx->cu_count * 4 + ntile - 1) / ntile);
        splits = std::min<int64_t>(splits, (ntask + 3) / 4);
        const int64_t tps = ((ntask + splits - 1) / splits + 3) / 4 * 4;
        splits = (ntask + tps - 1) / tps;
        if (ntile * splits > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "moe: grid too large");
        // [dtype][format][up silu, up gelu, down][tile rows 1, 2, 4]
        static const Kernel table_v[2][2][3][3] = {
            {{{cuca_qmv_moe_up_q4_0_silu_m1_f32, cuca_qmv_moe_up_q4_0_silu_m2_f32, cuca_qmv_moe_up_q4_0_silu_m4_f32},
              {cuca_qmv_moe_up_q4_0_gelu_m1_f32, cuca_qmv_moe_up_q4_0_gelu_m2_f32, cuca_qmv_moe_up_q4_0_gelu_m4_f32},
              {cuca_qmv_moe_down_q4_0_m1_f32, cuca_qmv_moe_down_q4_0_m2_f32, cuca_qmv_moe_down_q4_0_m4_f32}},
             {{cuca_qmv_moe_up_q8_0_silu_m1_f32, cuca_qmv_moe_up_q8_0_silu_m2_f32, cuca_qmv_moe_up_q8_0_silu_m4_f32},
              {cuca_qmv_moe_up_q8_0_gelu_m1_f32, cuca_qmv_moe_up_q8_0_gelu_m2_f32, cuca_qmv_moe_up_q8_0_gelu_m4_f32},
              {cuca_qmv_moe_down_q8_0_m1_f32, cuca_qmv_moe_down_q8_0_m2_f32, cuca_qmv_moe_down_q8_0_m4_f32}}},
            {{{cuca_qmv_moe_up_q4_0_silu_m1_f16, cuca_qmv_moe_up_q4_0_silu_m2_f16, cuca_qmv_moe_up_q4_0_silu_m4_f16},
              {cuca_qmv_moe_up_q4_0_gelu_m1_f16, cuca_qmv_moe_up_q4_0_gelu_m2_f16, cuca_qmv_moe_up_q4_0_gelu_m4_f16},
              {cuca_qmv_moe_down_q4_0_m1_f16, cuca_qmv_moe_down_q4_0_m2_f16, cuca_qmv_moe_down_q4_0_m4_f16}},
             {{cuca_qmv_moe_up_q8_0_silu_m1_f16, cuca_qmv_moe_up_q8_0_silu_m2_f16, cuca_qmv_moe_up_q8_0_silu_m4_f16},
              {cuca_qmv_moe_up_q8_0_gelu_m1_f16, cuca_qmv_moe_up_q8_0_gelu_m2_f16, cuca_qmv_moe_up_q8_0_gelu_m4_f16},
              {cuca_qmv_moe_down_q8_0_m1_f16, cuca_qmv_moe_down_q8_0_m2_f16, cuca_qmv_moe_down_q8_0_m4_f16}}}};
        QmvArgs v{};
        v.w = static_cast<const uint8_t *>(w);
        v.w_up = static_cast<const uint8_t *>(w_up);
        v.x = x;
        v.out = out;
        v.offsets = offsets;
        v.pair_token = pair_token;
        v.pair_weight = pair_weight;
        v.status = ctx->status;
        v.ldx = ldx;
        v.out_ld = out_ld;
        v.w_estride = estride;
        v.row_bytes = ng * gb;
        v.rows = (int32_t)n;
        v.m = mt;
        v.nb = (int32_t)nb;
        v.ng = (int32_t)ng;
        v.nbp = (int32_t)(ng * g);
        v.ntask = (int32_t)ntask;
        v.n_experts = n_experts;
        v.max_pairs = (int32_t)max_pairs;
        v.n_tokens = (int32_t)(up ? n_tokens : max_pairs);
        v.splits = (int32_t)splits;
        v.tps = (int32_t)tps;
        v.clamp = clamp > 0.0f ? clamp : 0.0f;
        if (up) ctx->last_moe_tokens = n_tokens;
        return launch(ctx, table_v[dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][up ? up - 1 : 2][mi],
                      (unsigned)(ntile * splits), CUCA_BLOCK_THREADS, (unsigned)qmv_lds(mt, ng * g, g), v);
    }
    const int64_t nrb = (n + 15) / 16, nrb8 = (nrb + 7) / 8 * 8;
    if (nrb8 * ntile > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "moe: grid too large");
    // [dtype][format][up silu, up gelu, down][tile rows 1, 2, 4]
    static const Kernel table_k[2][2][3][3] = {
        {{{cuca_moe_up_f32_q4_0_silu_m1, cuca_moe_up_f32_q4_0_silu_m2, cuca_moe_up_f32_q4_0_silu_m4},
          {cuca_moe_up_f32_q4_0_gelu_m1, cuca_moe_up_f32_q4_0_gelu_m2, cuca_moe_up_f32_q4_0_gelu_m4},
          {cuca_moe_down_f32_q4_0_m1, cuca_moe_down_f32_q4_0_m2, cuca_moe_down_f32_q4_0_m4}},
         {{cuca_moe_up_f32_q8_0_silu_m1, cuca_moe_up_f32_q8_0_silu_m2, cuca_moe_up_f32_q8_0_silu_m4},
          {cuca_moe_up_f32_q8_0_gelu_m1, cuca_moe_up_f32_q8_0_gelu_m2, cuca_moe_up_f32_q8_0_gelu_m4},
          {cuca_moe_down_f32_q8_0_m1, cuca_moe_down_f32_q8_0_m2, cuca_moe_down_f32_q8_0_m4}}},
        {{{cuca_moe_up_f16_q4_0_silu_m1, cuca_moe_up_f16_q4_0_silu_m2, cuca_moe_up_f16_q4_0_silu_m4},
          {cuca_moe_up_f16_q4_0_gelu_m1, cuca_moe_up_f16_q4_0_gelu_m2, cuca_moe_up_f16_q4_0_gelu_m4},
          {cuca_moe_down_f16_q4_0_m1, cuca_moe_down_f16_q4_0_m2, cuca_moe_down_f16_q4_0_m4}},
         {{cuca_moe_up_f16_q8_0_silu_m1, cuca_moe_up_f16_q8_0_silu_m2, cuca_moe_up_f16_q8_0_silu_m4},
          {cuca_moe_up_f16_q8_0_gelu_m1, cuca_moe_up_f16_q8_0_gelu_m2, cuca_moe_up_f16_q8_0_gelu_m4},
          {cuca_moe_down_f16_q8_0_m1, cuca_moe_down_f16_q8_0_m2, cuca_moe_down_f16_q8_0_m4}}}};
    const Kernel kk = table_k[dtype == CUCA_F16][ggml_type == CUCA_GGML_Q8_0][up ? up - 1 : 2][mi];
    QmmArgs a{};
    a.w = static_cast<const uint8_t *>(w);
    a.w_up = static_cast<const uint8_t *>(w_up);
    a.x = x;
    a.out = out;
    a.ldx = ldx;
    a.out_ld = out_ld;
    a.row_bytes = ng * gb;
    a.rows = (int32_t)n;
    a.m = (int32_t)max_pairs;
    a.nb = (int32_t)nb;
    a.ng = (int32_t)ng;
    a.nrb = (int32_t)nrb;
    a.ntile = (int32_t)ntile;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    a.n_tokens = (int32_t)(up ? n_tokens : max_pairs);
    a.offsets = offsets;
    a.pair_token = pair_token;
    a.pair_weight = pair_weight;
    a.status = ctx->status;
    a.w_estride = estride;
    a.n_experts = n_experts;
    a.max_pairs = (int32_t)max_pairs;
    if (up) ctx->last_moe_tokens = n_tokens;
    return launch(ctx, kk, (unsigned)(nrb8 * ntile), CUCA_BLOCK_THREADS, 0, a);
}

cuca_status cuca_hip_moe_up(cuca_hip_ctx *ctx, const void *gate, const void *up, int64_t expert_stride,
                            uint32_t ggml_type, int64_t ff, int64_t n_embd, int32_t n_experts, const void *x,
                            int64_t ldx, int64_t n_tokens, const int32_t *offsets, const int32_t *pair_token,
                            int64_t max_pairs, cuca_act act, float clamp, void *hidden, int64_t hidden_ld,
                            cuca_dtype dtype) {
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    return moe_common(ctx, gate, up, expert_stride, ggml_type, ff, n_embd, n_experts, x, ldx, n_tokens, offsets,
                      pair_token, nullptr, max_pairs, act == CUCA_ACT_SILU ? 1 : 2, clamp, hidden, hidden_ld,
                      dtype);
}

cuca_status cuca_hip_moe_down(cuca_hip_ctx *ctx, const void *down, int64_t expert_stride, uint32_t ggml_type,
                              int64_t n_embd, int64_t ff, int32_t n_experts, const void *hidden,
                              int64_t hidden_ld, const int32_t *offsets, const float *pair_weight,
                              int64_t max_pairs, float *scratch, int64_t scratch_ld, cuca_dtype dtype) {
    return moe_common(ctx, down, nullptr, expert_stride, ggml_type, n_embd, ff, n_experts, hidden, hidden_ld, 0,
                      offsets, nullptr, pair_weight, max_pairs, 0, 0.0f, scratch, scratch_ld, dtype);
}

cuca_status cuca_hip_moe_sum(cuca_hip_ctx *ctx, const float *scratch, int64_t scratch_ld, int64_t max_pairs,
                             const int32_t *token_pairs, int32_t n_used, int64_t n_tokens, int64_t n_embd,
                             void *out, int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (n_tokens < 0 || n_tokens > 0x7fffffffll || n_embd <= 0 || n_embd > 0x7fffffffll || n_used <= 0 ||
        max_pairs < 0 || max_pairs > 0x7fffffffll)
        return fail(ctx, CUCA_INVALID_ARG, "moe sum: bad shape");
    if (scratch_ld < n_embd || out_ld < n_embd) return fail(ctx, CUCA_INVALID_ARG, "moe sum: row strides shorter than n_embd");
    if (n_tokens == 0) return CUCA_OK;
    if (!scratch || !token_pairs || !out) return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    const int64_t nq = (n_embd + 3) / 4;
    if (n_tokens * nq / CUCA_BLOCK_THREADS + 1 > 0x7fffffffll) return fail(ctx, CUCA_UNSUPPORTED, "moe sum: grid too large");
    MoeSumArgs a{};
    a.scratch = scratch;
    a.pairs = token_pairs;
    a.out = out;
    a.scratch_ld = scratch_ld;
    a.out_ld = out_ld;
    a.n_tokens = (int32_t)n_tokens;
    a.n_used = n_used;
    a.n_embd = (int32_t)n_embd;
    a.max_pairs = (int32_t)max_pairs;
    return launch(ctx, dtype == CUCA_F16 ? cuca_moe_sum_f16 : cuca_moe_sum_f32, div_up(n_tokens * nq, CUCA_BLOCK_THREADS),
                  CUCA_BLOCK_THREADS, 0, a);
}

// Routed experts on the matrix cores (qgemm.hip, the qgemm_moe kernels): a
// plan of the token tiles (cuca_qgemm_moe_plan), the pairs' activation rows
// rewritten into the tile layout, then one grouped GEMM launch over (weight
// row tile, token tile), each token tile one expert's.  Tiles of 128 pairs
// from a mean of 96 pairs per expert, else 64.  The tile count is bounded
// by ceil(max_pairs / tm) + min(n_experts, max_pairs) (each expert with
// pairs adds at most one partial tile).
static int moe_qgemm_tm(int64_t max_pairs, int32_t n_experts) {
    return (double)max_pairs / (double)n_experts >= 96.0 ? 128 : 64;
}
static int64_t moe_qgemm_tiles(int64_t max_pairs, int32_t n_experts, int tm) {
    return (max_pairs + tm - 1) / tm + std::min<int64_t>(n_experts, max_pairs);
}
static size_t moe_qgemm_ws_bytes(int g, int64_t k, int32_t n_experts, int64_t max_pairs) {
    const int tm = moe_qgemm_tm(max_pairs, n_experts);
    const int64_t tiles = moe_qgemm_tiles(max_pairs, n_experts, tm);
    const size_t plan = ((size_t)tiles * 3 * 4 + 255) / 256 * 256;
    return plan + (size_t)tiles * (size_t)tm * (size_t)qgemm_kp(g, k) * 2;
}

cuca_status cuca_hip_moe_qgemm_workspace(uint32_t ggml_type, int64_t k, int32_t n_experts, int64_t max_pairs,
                                         size_t *bytes) {
    if (!bytes) return fail(nullptr, CUCA_INVALID_ARG, "null pointer");
    int g = 0, gb = 0;
    if (!qfmt(ggml_type, &g, &gb)) return fail(nullptr, CUCA_UNSUPPORTED, "moe qgemm: ggml type %u", ggml_type);
    if (k <= 0 || k % 32 != 0 || k > kQgMaxK || n_experts <= 0 || max_pairs < 0 || max_pairs > 0x7fffffffll)
        return fail(nullptr, CUCA_INVALID_ARG, "moe qgemm: bad shape");
    *bytes = moe_qgemm_ws_bytes(g, k, n_experts, max_pairs);
    return CUCA_OK;
}

// up: 1 SiLU, 2 GELU-tanh; 0 down.
static cuca_status moe_qgemm_common(cuca_hip_ctx *ctx, const void *w, const void *w_up, int64_t estride,
                                    uint32_t ggml_type, int64_t n, int64_t k, int32_t n_experts, const void *x,
                                    int64_t ldx, int64_t n_tokens, const int32_t *offsets, const int32_t *pair_token,
                                    const float *pair_weight, int64_t max_pairs, int up, float clamp, void *ws,
                                    size_t ws_bytes, void *out, int64_t out_ld, cuca_dtype dtype) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    int g = 0, gb = 0;
    if ((st = qweight_shape(ctx, ggml_type, n, k, &g, &gb)) != CUCA_OK) return st;
    if (!dtype_ok(dtype)) return fail(ctx, CUCA_INVALID_ARG, "bad dtype %d", (int)dtype);
    if (n_experts <= 0 || n_experts > 4096)
        return fail(ctx, CUCA_INVALID_ARG, "moe qgemm: %d experts (1 to 4096)", n_experts);
    if (max_pairs < 0 || max_pairs > 0x7fffffffll)
        return fail(ctx, CUCA_INVALID_ARG, "moe: bad pair capacity %lld", (long long)max_pairs);
    if (k > kQgMaxK) return fail(ctx, CUCA_UNSUPPORTED, "moe qgemm: rows of more than %lld values", (long long)kQgMaxK);
    if (ldx < k) return fail(ctx, CUCA_INVALID_ARG, "moe: activation row stride %lld shorter than %lld",
                             (long long)ldx, (long long)k);
    if (out_ld < n) return fail(ctx, CUCA_INVALID_ARG, "moe: output row stride %lld shorter than %lld",
                                (long long)out_ld, (long long)n);
    if (!(clamp == clamp)) return fail(ctx, CUCA_INVALID_ARG, "clamp is NaN");
    if (max_pairs == 0) return CUCA_OK;
    if (!w || !x || !out || !offsets || !ws || (up && (!w_up || !pair_token)) || (!up && !pair_weight))
        return fail(ctx, CUCA_INVALID_ARG, "null pointer");
    if (up && (n_tokens <= 0 || n_tokens > 0x7fffffffll))
        return fail(ctx, CUCA_INVALID_ARG, "moe: bad token count %lld", (long long)n_tokens);
    const int64_t nb = k / 32, ng = (nb + g - 1) / g;
    const int64_t packed = n * ng * gb;
    if (estride < packed || estride % 16 != 0)
        return fail(ctx, CUCA_INVALID_ARG, "moe: expert stride %lld bytes, at least %lld (a multiple of 16) needed",
                    (long long)estride, (long long)packed);
    if (!al16(w) || (w_up && !al16(w_up)) || !al16(ws))
        return fail(ctx, CUCA_INVALID_ARG, "packed weights and the workspace must be 16-byte aligned");
    const size_t need = moe_qgemm_ws_bytes(g, k, n_experts, max_pairs);
    if (ws_bytes < need)
        return fail(ctx, CUCA_INVALID_ARG, "moe qgemm: workspace of %zu bytes, %zu needed (cuca_hip_moe_qgemm_workspace)",
                    ws_bytes, need);
    const int tm = moe_qgemm_tm(max_pairs, n_experts);
    const int64_t tiles = moe_qgemm_tiles(max_pairs, n_experts, tm);
    const int64_t kp = qgemm_kp(g, k), nkc = kp / 128;
    const int64_t n_rt = (n + 127) / 128;
    const int64_t grid = (n_rt + 7) / 8 * 8 * tiles;
    if (grid > 0x7fffffffll || tiles * tm * nkc * 16 / CUCA_BLOCK_THREADS + 1 > 0x7fffffffll)
        return fail(ctx, CUCA_UNSUPPORTED, "moe qgemm: grid too large");
    const size_t plan = ((size_t)tiles * 3 * 4 + 255) / 256 * 256;
    QGemmArgs a{};
    a.w = static_cast<const uint8_t *>(w);
    a.w_up = static_cast<const uint8_t *>(w_up);
    a.x = x;
    a.tile_e = static_cast<int32_t *>(ws);
    a.tile_p0 = a.tile_e + tiles;
    a.tile_n = a.tile_p0 + tiles;
    a.xp = reinterpret_cast<uint16_t *>(static_cast<char *>(ws) + plan);
    a.out = out;
    a.ldx = ldx;
    a.out_ld = out_ld;
    a.row_bytes = (kp / 32 / g) * gb;
    a.kp = kp;
    a.rows = (int32_t)n;
    a.m = up ? (int32_t)n_tokens : (int32_t)max_pairs;
    a.k = (int32_t)k;
    a.nkc = (int32_t)nkc;
    a.n_rt = (int32_t)n_rt;
    a.n_ct = (int32_t)tiles;
    a.kcs = (int32_t)nkc;
    a.splits = 1;
    a.clamp = clamp > 0.0f ? clamp : 0.0f;
    a.mp = (int32_t)(tiles * tm);
    a.offsets = offsets;
    a.pair_token = pair_token;
    a.pair_weight = pair_weight;
    a.status = ctx->status;
    a.estride = estride;
    a.n_experts = n_experts;
    a.max_pairs = (int32_t)max_pairs;
    a.tm = tm;
    a.moe_up = up ? 1 : 0;
    if ((st = launch(ctx, cuca_qgemm_moe_plan, 1, CUCA_BLOCK_THREADS, 0, a)) != CUCA_OK) return st;
    const bool f16 = dtype == CUCA_F16, q8 = ggml_type == CUCA_GGML_Q8_0;
    static const Kernel prep_k[2][2] = {{cuca_qgemm_moe_prep_f32_q4_0, cuca_qgemm_moe_prep_f32_q8_0},
                                        {cuca_qgemm_moe_prep_f16_q4_0, cuca_qgemm_moe_prep_f16_q8_0}};
    if ((st = launch(ctx, prep_k[f16][q8], div_up((int64_t)a.mp * nkc * 16, CUCA_BLOCK_THREADS), CUCA_BLOCK_THREADS,
                     0, a)) != CUCA_OK)
        return st;
    // [dtype][format][down, up silu, up gelu][tile pairs 64, 128]
    static const Kernel table_k[2][2][3][2] = {
        {{{cuca_qgemm_moe_down_f32_q4_0_t64, cuca_qgemm_moe_down_f32_q4_0_t128},
          {cuca_qgemm_moe_up_f32_q4_0_silu_t64, cuca_qgemm_moe_up_f32_q4_0_silu_t128},
          {cuca_qgemm_moe_up_f32_q4_0_gelu_t64, cuca_qgemm_moe_up_f32_q4_0_gelu_t128}},
         {{cuca_qgemm_moe_down_f32_q8_0_t64, cuca_qgemm_moe_down_f32_q8_0_t128},
          {cuca_qgemm_moe_up_f32_q8_0_silu_t64, cuca_qgemm_moe_up_f32_q8_0_silu_t128},
          {cuca_qgemm_moe_up_f32_q8_0_gelu_t64, cuca_qgemm_moe_up_f32_q8_0_gelu_t128}}},
        {{{cuca_qgemm_moe_down_f16_q4_0_t64, cuca_qgemm_moe_down_f16_q4_0_t128},
          {cuca_qgemm_moe_up_f16_q4_0_silu_t64, cuca_qgemm_moe_up_f16_q4_0_silu_t128},
          {cuca_qgemm_moe_up_f16_q4_0_gelu_t64, cuca_qgemm_moe_up_f16_q4_0_gelu_t128}},
         {{cuca_qgemm_moe_down_f16_q8_0_t64, cuca_qgemm_moe_down_f16_q8_0_t128},
          {cuca_qgemm_moe_up_f16_q8_0_silu_t64, cuca_qgemm_moe_up_f16_q8_0_silu_t128},
          {cuca_qgemm_moe_up_f16_q8_0_gelu_t64, cuca_qgemm_moe_up_f16_q8_0_gelu_t128}}}};
    return launch(ctx, table_k[f16][q8][up][tm == 128], (unsigned)grid, CUCA_BLOCK_THREADS, 0, a);
}

cuca_status cuca_hip_moe_up_qgemm(cuca_hip_ctx *ctx, const void *gate, const void *up, int64_t expert_stride,
                                  uint32_t ggml_type, int64_t ff, int64_t n_embd, int32_t n_experts, const void *x,
                                  int64_t ldx, int64_t n_tokens, const int32_t *offsets, const int32_t *pair_token,
                                  int64_t max_pairs, cuca_act act, float clamp, void *workspace,
                                  size_t workspace_bytes, void *hidden, int64_t hidden_ld, cuca_dtype dtype) {
    if (act != CUCA_ACT_SILU && act != CUCA_ACT_GELU_TANH)
        return fail(ctx, CUCA_INVALID_ARG, "bad activation %d", (int)act);
    return moe_qgemm_common(ctx, gate, up, expert_stride, ggml_type, ff, n_embd, n_experts, x, ldx, n_tokens,
                            offsets, pair_token, nullptr, max_pairs, act == CUCA_ACT_SILU ? 1 : 2, clamp, workspace,
                            workspace_bytes, hidden, hidden_ld, dtype);
}

cuca_status cuca_hip_moe_down_qgemm(cuca_hip_ctx *ctx, const void *down, int64_t expert_stride, uint32_t ggml_type,
                                    int64_t n_embd, int64_t ff, int32_t n_experts, const void *hidden,
                                    int64_t hidden_ld, const int32_t *offsets, const float *pair_weight,
                                    int64_t max_pairs, void *workspace, size_t workspace_bytes, float *scratch,
                                    int64_t scratch_ld, cuca_dtype dtype) {
    return moe_qgemm_common(ctx, down, nullptr, expert_stride, ggml_type, n_embd, ff, n_experts, hidden, hidden_ld, 0,
                            offsets, nullptr, pair_weight, max_pairs, 0, 0.0f, workspace, workspace_bytes, scratch,
                            scratch_ld, dtype);
}

// RopeSpec::tables (rope.rs:118-151): f64 angles with the platform libm,
// `cos(theta) * mscale` rounded to f32.
cuca_status cuca_hip_rope_tables(const cuca_rope_spec *spec, const float *factors, int64_t positions,
                                 float *cos_out, float *sin_out) {
    if (!spec || !cos_out || !sin_out) return fail(nullptr, CUCA_INVALID_ARG, "null pointer");
    const int n_dims = spec->n_dims;
    if (n_dims <= 0 || n_dims % 2 != 0) return fail(nullptr, CUCA_INVALID_ARG, "n_dims %d must be even", n_dims);
    if (positions < 0) return fail(nullptr, CUCA_INVALID_ARG, "negative position count");
    if (!(spec->base > 0.0) || !(spec->freq_scale > 0.0))
        return fail(nullptr, CUCA_INVALID_ARG, "base and freq_scale must be positive");
    const int half = n_dims / 2;
    if (factors)
        for (int i = 0; i < half; i++)
            if (!(factors[i] > 0.0f) || !std::isfinite(factors[i]))
                return fail(nullptr, CUCA_INVALID_ARG, "factors must be finite and positive");
    const bool yarn = spec->yarn_ext_factor != 0.0;
    double c0 = 0.0, c1 = 0.0;
    if (yarn) {
        // ggml rope_yarn_corr_dims (rope.rs:86-99)
        auto corr = [&](double n_rot) {
            return (double)n_dims * std::log((double)spec->yarn_n_ctx_orig / (n_rot * 2.0 * M_PI)) /
                   (2.0 * std::log(spec->base));
        };
        c0 = std::fmax(0.0, std::floor(corr(spec->yarn_beta_fast)));
        c1 = std::fmin((double)(n_dims - 1), std::ceil(corr(spec->yarn_beta_slow)));
    }
    for (int64_t pos = 0; pos < positions; pos++) {
        for (int i = 0; i < half; i++) {
            const double factor = factors ? (double)factors[i] : 1.0;
            const int i0 = 2 * i;
            const double extrap = (double)pos * std::pow(spec->base, -(double)i0 / (double)n_dims) / factor;
            const double interp = spec->freq_scale * extrap;
            double theta = interp, mscale = spec->attn_factor;
            if (yarn) {
                double r = ((double)(i0 / 2) - c0) / std::fmax(c1 - c0, 0.001);
                r = r < 0.0 ? 0.0 : (r > 1.0 ? 1.0 : r);
                const double mix = (1.0 - r) * spec->yarn_ext_factor;
                mscale = spec->attn_factor * (1.0 + 0.1 * std::log(1.0 / spec->freq_scale));
                theta = interp * (1.0 - mix) + extrap * mix;
            }
            cos_out[pos * half + i] = (float)(std::cos(theta) * mscale);
            sin_out[pos * half + i] = (float)(std::sin(theta) * mscale);
        }
    }
    return CUCA_OK;
}

// ---------------------------------------------------------------------
// graphs and timing
// ---------------------------------------------------------------------

cuca_status cuca_hip_graph_begin(cuca_hip_ctx *ctx) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (ctx->capturing) return fail(ctx, CUCA_INVALID_ARG, "a capture is already open");
    HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return CUCA_OK;
}

cuca_status cuca_hip_graph_end(cuca_hip_ctx *ctx, cuca_hip_graph **out) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!out) return fail(ctx, CUCA_INVALID_ARG, "null output pointer");
    *out = nullptr;
    if (!ctx->capturing) return fail(ctx, CUCA_INVALID_ARG, "no capture is open");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    HIP_TRY(ctx, hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_fail(ctx, e, "hipGraphInstantiate");
    }
    *out = new cuca_hip_graph{g, exec};
    return CUCA_OK;
}

cuca_status cuca_hip_graph_launch(cuca_hip_ctx *ctx, cuca_hip_graph *graph) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!graph) return fail(ctx, CUCA_INVALID_ARG, "null graph");
    HIP_TRY(ctx, hipGraphLaunch(graph->exec, ctx->stream));
    return CUCA_OK;
}

void cuca_hip_graph_destroy(cuca_hip_graph *graph) {
    if (!graph) return;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

cuca_status cuca_hip_timer_start(cuca_hip_ctx *ctx) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    HIP_TRY(ctx, hipEventRecord(ctx->t0, ctx->stream));
    return CUCA_OK;
}

cuca_status cuca_hip_timer_stop(cuca_hip_ctx *ctx, float *ms) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!ms) return fail(ctx, CUCA_INVALID_ARG, "null output pointer");
    HIP_TRY(ctx, hipEventRecord(ctx->t1, ctx->stream));
    HIP_TRY(ctx, hipEventSynchronize(ctx->t1));
    HIP_TRY(ctx, hipEventElapsedTime(ms, ctx->t0, ctx->t1));
    return CUCA_OK;
}

cuca_status cuca_hip_profile_start(cuca_hip_ctx *ctx, int32_t max_launches) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (ctx->capturing) return fail(ctx, CUCA_INVALID_ARG, "cannot profile during a capture");
    if (max_launches < 0 || max_launches > (1 << 20))
        return fail(ctx, CUCA_INVALID_ARG, "bad launch count %d", max_launches);
    while (ctx->prof.size() < (size_t)max_launches) {
        cuca_hip_ctx::ProfRec r{0, nullptr, nullptr};
        HIP_TRY(ctx, hipEventCreate(&r.start));
        hipError_t e = hipEventCreate(&r.stop);
        if (e != hipSuccess) {
            (void)hipEventDestroy(r.start);
            return hip_fail(ctx, e, "hipEventCreate");
        }
        ctx->prof.push_back(r);
    }
    ctx->prof_used = 0;
    ctx->prof_limit = (size_t)max_launches;
    ctx->profiling = true;
    return CUCA_OK;
}

cuca_status cuca_hip_profile_stop(cuca_hip_ctx *ctx, cuca_hip_kernel_time *out, int32_t max,
                                  int32_t *count) {
    cuca_status st = use(ctx);
    if (st != CUCA_OK) return st;
    if (!count || (max > 0 && !out)) return fail(ctx, CUCA_INVALID_ARG, "null output pointer");
    if (!ctx->profiling) return fail(ctx, CUCA_INVALID_ARG, "profiling was not started");
    ctx->profiling = false;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    const int32_t n = (int32_t)ctx->prof_used < max ? (int32_t)ctx->prof_used : max;
    for (int32_t i = 0; i < n; i++) {
        const cuca_hip_ctx::ProfRec &r = ctx->prof[i];
        out[i].kernel = kKernelNames[r.kernel];
        HIP_TRY(ctx, hipEventElapsedTime(&out[i].ms, r.start, r.stop));
    }
    *count = n;
    return CUCA_OK;
}

}  // extern "C"
