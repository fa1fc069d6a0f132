// core.hip -- context, device memory, events and status strings of libemuhip.
#include "internal.hpp"

#include <stdio.h>
#include <string.h>

int emu_hip_fail(emu_ctx *ctx, hipError_t e, const char *what)
{
    if (ctx) snprintf(ctx->last_error, sizeof ctx->last_error, "%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? EMU_E_NOMEM : EMU_E_HIP;
}

extern "C" const char *emu_strerror(int status)
{
    switch (status) {
    case EMU_OK: return "ok";
    case EMU_E_SHORT: return "byte length is not a whole number of blocks";
    case EMU_E_SHAPE: return "weight count does not match the declared shape";
    case EMU_E_ACTIVATION_LEN: return "activation vector shorter than the input dimension";
    case EMU_E_TRUNCATED: return "stream ended before the matrix did";
    case EMU_E_UNSUPPORTED: return "unsupported encoding";
    case EMU_E_CONTEXT_FULL: return "KV context exhausted";
    case EMU_E_CONFIG: return "invalid configuration";
    case EMU_E_HIP: return "HIP runtime error";
    case EMU_E_ARG: return "invalid argument";
    case EMU_E_NOMEM: return "allocation refused";
    case EMU_E_FORMAT: return "file refused by its reader";
    case EMU_E_IO: return "file read failed";
    default: return "unknown status";
    }
}

extern "C" const char *emu_last_error(const emu_ctx *ctx) { return ctx ? ctx->last_error : ""; }

extern "C" int emu_block_layout(int encoding, uint32_t *block_elems, uint32_t *block_bytes)
{
    if (!block_elems || !block_bytes) return EMU_E_ARG;
    // spm-gguf/src/parse.rs:10-29, the dtypes on the token-loop path
    switch (encoding) {
    case EMU_ENC_F32: *block_elems = 1; *block_bytes = 4; return EMU_OK;
    case EMU_ENC_F16: *block_elems = 1; *block_bytes = 2; return EMU_OK;
    case EMU_ENC_Q8_0: *block_elems = 32; *block_bytes = 34; return EMU_OK;
    case EMU_ENC_Q2_K: *block_elems = 256; *block_bytes = 84; return EMU_OK;
    case EMU_ENC_Q5_K: *block_elems = 256; *block_bytes = 176; return EMU_OK;
    case EMU_ENC_Q6_K: *block_elems = 256; *block_bytes = 210; return EMU_OK;
    default: return EMU_E_UNSUPPORTED;
    }
}

extern "C" int emu_ctx_create(int device, emu_ctx **out)
{
    if (!out) return EMU_E_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return EMU_E_HIP;
    if (device < 0 || device >= count) return EMU_E_ARG;
    emu_ctx *ctx = new (std::nothrow) emu_ctx();
    if (!ctx) return EMU_E_NOMEM;
    ctx->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    for (int i = 0; e == hipSuccess && i < 16; ++i) e = hipEventCreate(&ctx->events[i]);
    if (e != hipSuccess) {
        delete ctx;
        return EMU_E_HIP;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
        ctx->cus = prop.multiProcessorCount;
        snprintf(ctx->arch, sizeof ctx->arch, "%s", prop.gcnArchName);
    }
    if (emu_ops_device_init(ctx) != EMU_OK) {
        emu_ctx_destroy(ctx);
        return EMU_E_HIP;
    }
    *out = ctx;
    return EMU_OK;
}

extern "C" int emu_ctx_destroy(emu_ctx *ctx)
{
    if (!ctx) return EMU_E_ARG;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto &ev : ctx->events)
        if (ev) (void)hipEventDestroy(ev);
    if (ctx->mfma_ws) (void)hipFree(ctx->mfma_ws);
    for (int i = 0; i < 2; ++i) {
        if (ctx->stage_ev[i]) (void)hipEventDestroy(ctx->stage_ev[i]);
        if (ctx->stage[i]) (void)hipHostFree(ctx->stage[i]);
    }
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return EMU_OK;
}

extern "C" int emu_ctx_sync(emu_ctx *ctx)
{
    if (!ctx) return EMU_E_ARG;
    EMU_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return EMU_OK;
}

extern "C" int emu_ctx_stream(emu_ctx *ctx, void **stream)
{
    if (!ctx || !stream) return EMU_E_ARG;
    *stream = (void *)ctx->stream;
    return EMU_OK;
}

extern "C" int emu_device_info(emu_ctx *ctx, int *compute_units, char *arch, size_t arch_len)
{
    if (!ctx) return EMU_E_ARG;
    if (compute_units) *compute_units = ctx->cus;
    if (arch && arch_len) snprintf(arch, arch_len, "%s", ctx->arch);
    return EMU_OK;
}

extern "C" int emu_malloc(emu_ctx *ctx, size_t bytes, void **d_out)
{
    if (!ctx || !d_out) return EMU_E_ARG;
    *d_out = nullptr;
    EMU_HIP(ctx, hipSetDevice(ctx->device));
    EMU_HIP(ctx, hipMalloc(d_out, bytes ? bytes : 1));
    return EMU_OK;
}

extern "C" int emu_free(emu_ctx *ctx, void *d_ptr)
{
    if (!ctx) return EMU_E_ARG;
    if (!d_ptr) return EMU_OK;
    EMU_HIP(ctx, hipStreamSynchronize(ctx->stream));
    EMU_HIP(ctx, hipFree(d_ptr));
    return EMU_OK;
}

extern "C" int emu_memcpy_htod(emu_ctx *ctx, void *d_dst, const void *h_src, size_t bytes)
{
    if (!ctx || (bytes && (!d_dst || !h_src))) return EMU_E_ARG;
    if (!bytes) return EMU_OK;
    EMU_HIP(ctx, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream));
    EMU_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return EMU_OK;
}

extern "C" int emu_memcpy_dtoh(emu_ctx *ctx, void *h_dst, const void *d_src, size_t bytes)
{
    if (!ctx || (bytes && (!d_src || !h_dst))) return EMU_E_ARG;
    if (!bytes) return EMU_OK;
    EMU_HIP(ctx, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    EMU_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return EMU_OK;
}

extern "C" int emu_memcpy_dtod(emu_ctx *ctx, void *d_dst, const void *d_src, size_t bytes)
{
    if (!ctx || (bytes && (!d_src || !d_dst))) return EMU_E_ARG;
    if (!bytes) return EMU_OK;
    EMU_HIP(ctx, hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return EMU_OK;
}

extern "C" int emu_memset(emu_ctx *ctx, void *d_dst, int value, size_t bytes)
{
    if (!ctx || (bytes && !d_dst)) return EMU_E_ARG;
    if (!bytes) return EMU_OK;
    EMU_HIP(ctx, hipMemsetAsync(d_dst, value, bytes, ctx->stream));
    return EMU_OK;
}

extern "C" int emu_event_record(emu_ctx *ctx, int slot)
{
    if (!ctx || slot < 0 || slot >= 16) return EMU_E_ARG;
    EMU_HIP(ctx, hipEventRecord(ctx->events[slot], ctx->stream));
    return EMU_OK;
}

extern "C" int emu_event_elapsed(emu_ctx *ctx, int start_slot, int end_slot, float *ms)
{
    if (!ctx || !ms || start_slot < 0 || start_slot >= 16 || end_slot < 0 || end_slot >= 16)
        return EMU_E_ARG;
    EMU_HIP(ctx, hipEventSynchronize(ctx->events[end_slot]));
    EMU_HIP(ctx, hipEventElapsedTime(ms, ctx->events[start_slot], ctx->events[end_slot]));
    return EMU_OK;
}
