/*
 * Host side of the MI355X attention path: the C ABI of include/q38_attn.h.
 *
 * Kernels live in gfx950 code objects (one .hsaco per source file) loaded
 * with hipModuleLoad and launched with hipModuleLaunchKernel; their argument
 * blocks (q38_kargs.h) travel by value in the kernarg segment, so a decode
 * step needs no host-to-device copy besides page-table updates.
 *
 * Validation happens here, before any launch, and turns every bad input
 * into -1 with a message (the reference's Err(-1), e.g. the KV bounds check
 * of src/model/ops.rs:858-864): no kernel ever sees an index it was not
 * sized for.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

/* From hip/hip_ext.h (whose templates need the HIP compiler): a module launch
 * whose start/stop events are stamped by the kernel dispatch itself. */
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams, void **extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent,
                                               uint32_t flags);

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../../include/q38_attn.h"
#include "../../../include/q38_bench.h"
#include "../q38_kargs.h"
#include "q38_scratch.h"

namespace {

thread_local std::string g_last_error;

int fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return -1;
}

}  // namespace

/* The error slot for the library's other host files (q38_gguf.cpp). */
__attribute__((visibility("hidden"))) int q38_fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return -1;
}

namespace {

#define Q38_HIP(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) return fail("%s: %s (%s:%d)", #call, hipGetErrorString(e_), \
                                          __FILE__, __LINE__);                          \
    } while (0)

std::string library_dir() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void *>(&library_dir), &info) == 0 || info.dli_fname == nullptr)
        return ".";
    std::string path(info.dli_fname);
    size_t slash = path.find_last_of('/');
    return slash == std::string::npos ? std::string(".") : path.substr(0, slash);
}

/* Full-attention layers: every fourth block and the MTP block 64
 * (ops.rs:38-41); their slot is layer/4 (ops.rs:858). */
bool is_full_attention(int layer) { return layer >= 0 && ((layer + 1) % 4 == 0 || layer == 64); }

/* The weight formats of the Q8_K GEMV (tensor_gemv_q8_k's types,
 * tensor.rs:70-75): the GEMV kernel, its many-token form on the int8
 * matrix unit and that form with a row's blocks split over 8, 16 or 4
 * waves (for small grids), f32 terms per block in a row's sum, and the bytes of the
 * lattice grid an IQ kernel copies into LDS. */
struct GemvType {
    int ggml_type;
    const char *kernel;
    const char *gemm_kernel;
    const char *gemm_ks_kernel;
    const char *gemm_ks16_kernel;
    const char *gemm_ks4_kernel;
    int terms;
    int grid_bytes;
};
constexpr GemvType kGemv[] = {
    {Q38_GGML_Q4_K, "q38_gemv_q8k_q4k", "q38_gemm_q8k_q4k", "q38_gemm_ks_q8k_q4k", "q38_gemm_ks16_q8k_q4k", "q38_gemm_ks4_q8k_q4k", 1, 0},
    {Q38_GGML_Q5_K, "q38_gemv_q8k_q5k", "q38_gemm_q8k_q5k", "q38_gemm_ks_q8k_q5k", "q38_gemm_ks16_q8k_q5k", "q38_gemm_ks4_q8k_q5k", 1, 0},
    {Q38_GGML_Q6_K, "q38_gemv_q8k_q6k", "q38_gemm_q8k_q6k", "q38_gemm_ks_q8k_q6k", "q38_gemm_ks16_q8k_q6k", "q38_gemm_ks4_q8k_q6k", 1, 0},
    {Q38_GGML_Q3_K, "q38_gemv_q8k_q3k", "q38_gemm_q8k_q3k", "q38_gemm_ks_q8k_q3k", "q38_gemm_ks16_q8k_q3k", "q38_gemm_ks4_q8k_q3k", 1, 0},
    {Q38_GGML_IQ4_XS, "q38_gemv_q8k_iq4xs", "q38_gemm_q8k_iq4xs", "q38_gemm_ks_q8k_iq4xs", "q38_gemm_ks16_q8k_iq4xs", "q38_gemm_ks4_q8k_iq4xs", 1, 0},
    {Q38_GGML_Q2_K, "q38_gemv_q8k_q2k", "q38_gemm_q8k_q2k", "q38_gemm_ks_q8k_q2k", "q38_gemm_ks16_q8k_q2k", "q38_gemm_ks4_q8k_q2k", 1, 0},
    {Q38_GGML_IQ4_NL, "q38_gemv_q8k_iq4nl", "q38_gemm_q8k_iq4nl", nullptr, nullptr, nullptr, 8, 0},
    {Q38_GGML_IQ2_XXS, "q38_gemv_q8k_iq2xxs", "q38_gemm_q8k_iq2xxs", "q38_gemm_ks_q8k_iq2xxs", "q38_gemm_ks16_q8k_iq2xxs", "q38_gemm_ks4_q8k_iq2xxs", 1, 256 * 8},
    {Q38_GGML_IQ2_XS, "q38_gemv_q8k_iq2xs", "q38_gemm_q8k_iq2xs", "q38_gemm_ks_q8k_iq2xs", "q38_gemm_ks16_q8k_iq2xs", "q38_gemm_ks4_q8k_iq2xs", 1, 512 * 8},
    {Q38_GGML_IQ2_S, "q38_gemv_q8k_iq2s", "q38_gemm_q8k_iq2s", "q38_gemm_ks_q8k_iq2s", "q38_gemm_ks16_q8k_iq2s", "q38_gemm_ks4_q8k_iq2s", 1, 1024 * 8},
    {Q38_GGML_IQ3_XXS, "q38_gemv_q8k_iq3xxs", "q38_gemm_q8k_iq3xxs", "q38_gemm_ks_q8k_iq3xxs", "q38_gemm_ks16_q8k_iq3xxs", "q38_gemm_ks4_q8k_iq3xxs", 1, 256 * 4},
    {Q38_GGML_IQ3_S, "q38_gemv_q8k_iq3s", "q38_gemm_q8k_iq3s", "q38_gemm_ks_q8k_iq3s", "q38_gemm_ks16_q8k_iq3s", "q38_gemm_ks4_q8k_iq3s", 1, 512 * 4},
    {Q38_GGML_IQ1_S, "q38_gemv_q8k_iq1s", "q38_gemm_q8k_iq1s", "q38_gemm_ks_q8k_iq1s", "q38_gemm_ks16_q8k_iq1s", "q38_gemm_ks4_q8k_iq1s", 1, 2048 * 8},
    {Q38_GGML_IQ1_M, "q38_gemv_q8k_iq1m", "q38_gemm_q8k_iq1m", "q38_gemm_ks_q8k_iq1m", "q38_gemm_ks16_q8k_iq1m", "q38_gemm_ks4_q8k_iq1m", 1, 2048 * 8},
};
constexpr int kGemvTypes = (int)(sizeof(kGemv) / sizeof(kGemv[0]));
/* The split-block GEMM's grid: at least this many workgroups (fewer: the
 * GEMV), at most this many per CU (more: the 128 x 64 tiles) */
constexpr long kGemmKsMinTiles = 64;
/* q38_quantize_project_q8_k folds the quantisation into the GEMV up to this
 * many tokens (a layer's four projections, measured at 1-7 tokens: one
 * token 65.5 against 68.0 us folded; two 84.5 against 74.8 us, every
 * workgroup quantising both tokens) */
constexpr int kQuantizeFoldMaxTokens = 1;
constexpr long kGemmKsMaxPerCu = 5;

}  // namespace

struct q38_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t mod_decode = nullptr;
    hipModule_t mod_gdn = nullptr;
    hipModule_t mod_prefill = nullptr;
    hipFunction_t f_prefill = nullptr;
    hipFunction_t f_kv_split = nullptr;
    hipFunction_t f_prefill_merge = nullptr;
    hipModule_t mod_gdn_chunk = nullptr;
    hipFunction_t f_chunk_prep = nullptr;
    hipFunction_t f_chunk_scan = nullptr;
    hipFunction_t f_gdn_post = nullptr;
    hipFunction_t f_decode_split = nullptr;
    hipFunction_t f_decode_split_many = nullptr; /* any number of splits */
    hipFunction_t f_decode_split_pre = nullptr; /* the same with full_core's pre step fused */
    hipFunction_t f_decode_split_pre_many = nullptr;
    hipFunction_t f_decode_split_one = nullptr;     /* one sequence: arguments in one load round */
    hipFunction_t f_decode_split_pre_one = nullptr;
    hipFunction_t f_decode_merge = nullptr;
    hipFunction_t f_kv_copy = nullptr;
    hipFunction_t f_attn_pre = nullptr;
    hipFunction_t f_gdn_decode = nullptr;
    hipFunction_t f_gdn_pre = nullptr;
    hipFunction_t f_gdn_step_rows = nullptr;
    hipModule_t mod_proj = nullptr;
    hipFunction_t f_quantize_q8k = nullptr;
    hipFunction_t f_gemm[kGemvTypes] = {};    /* by kGemv index: the int8 matrix-unit form */
    hipFunction_t f_gemm_ks[kGemvTypes] = {};   /* and its split-block form */
    hipFunction_t f_gemm_ks16[kGemvTypes] = {}; /* ... on 16 waves */
    hipFunction_t f_gemm_ks4[kGemvTypes] = {};  /* ... on 4 waves */
    hipFunction_t f_gemv_q8k[kGemvTypes] = {}; /* by kGemv index */
    hipFunction_t f_gemv_f32[3] = {nullptr, nullptr, nullptr}; /* F32, F16, BF16 weights */
    hipFunction_t f_gemm_f32[4] = {nullptr, nullptr, nullptr, nullptr}; /* the same, on the matrix unit */
    hipFunction_t f_gemm_f32s[4] = {nullptr, nullptr, nullptr, nullptr}; /* few tokens, k split over the waves */
    hipFunction_t f_gemm_f32w[4] = {nullptr, nullptr, nullptr, nullptr}; /* 128-token tiles (not F32) */
    hipFunction_t f_gemv_q80s[4] = {}; /* Q8_0, activations staged in LDS: TP 1, 2, 4 (RW 2), 8 (RW 4) */
    hipModule_t mod_synth = nullptr;
    hipFunction_t f_fill_normal = nullptr;
    hipFunction_t f_copy = nullptr;
    hipFunction_t f_noop = nullptr;
    /* per-kernel event timer (q38_kernel_timer_*) */
    hipFunction_t timed = nullptr;
    std::vector<hipEvent_t> timer_events;
    int timer_used = 0;
    int cu_count = 0;
    int decode_block = 64 * Q38_DECODE_WAVES; /* threads of a decode workgroup (the kernel's launch bound) */
    int gdn_decode_block = 512;               /* threads of a q38_gdn_decode workgroup (its launch bound) */
    int split_tokens = 0; /* context tokens per decode workgroup; 0: chosen per launch */
    int clock_khz = 0;
    int lds_bytes = 0;
    int lds_per_cu = 0;
    int gemv_occupancy[kGemvTypes] = {}; /* by kGemv index: GEMV workgroups a CU holds */
    char name[256] = {0};
    /* this device's copy of the fixed scratch array (q38_full_core_noalloc) */
    void *scratch = nullptr;
    /* grow-only device workspace (split-K partials, pre-kernel outputs) */
    void *work = nullptr;
    size_t work_bytes = 0;
    /* DeltaNet decode arrival counters [n_seq][Q38_GDN_ARRIVALS], zero
     * between calls */
    int32_t *arrivals = nullptr;
    int arrival_seqs = 0;

    int ensure_arrivals(int n_seq) {
        if (n_seq <= arrival_seqs) return 0;
        if (arrivals != nullptr) {
            Q38_HIP(hipStreamSynchronize(stream));
            Q38_HIP(hipFree(arrivals));
            arrivals = nullptr;
            arrival_seqs = 0;
        }
        const int want = std::max(n_seq, 64);
        const size_t bytes = (size_t)want * Q38_GDN_ARRIVALS * sizeof(int32_t);
        Q38_HIP(hipMalloc(&arrivals, bytes));
        Q38_HIP(hipMemsetAsync(arrivals, 0, bytes, stream));
        arrival_seqs = want;
        return 0;
    }
    float rope_theta_scale = 0.0f;

    int ensure_work(size_t bytes) {
        if (bytes <= work_bytes) return 0;
        if (work != nullptr) {
            Q38_HIP(hipStreamSynchronize(stream));
            Q38_HIP(hipFree(work));
            work = nullptr;
            work_bytes = 0;
        }
        size_t want = std::max(bytes, (size_t)1 << 20);
        Q38_HIP(hipMalloc(&work, want));
        work_bytes = want;
        return 0;
    }

    int launch(hipFunction_t f, unsigned gx, unsigned gy, unsigned gz, unsigned block, void *args,
               unsigned lds_bytes = 0) {
        void *params[] = {args};
        /* the stamped form takes the grid in threads, a 32-bit count */
        if ((uint64_t)gx * block > 0xFFFFFFFFull) return fail("grid of %u workgroups too large", gx);
        const bool timing = f == timed && timer_used + 2 <= (int)timer_events.size();
        if (timing) {
            /* start/stop timestamps taken by the dispatch itself */
            Q38_HIP(hipExtModuleLaunchKernel(f, gx * block, gy, gz, block, 1, 1, lds_bytes, stream, params,
                                             nullptr, timer_events[timer_used], timer_events[timer_used + 1], 0));
            timer_used += 2;
            return 0;
        }
        Q38_HIP(hipModuleLaunchKernel(f, gx, gy, gz, block, 1, 1, lds_bytes, stream, params, nullptr));
        return 0;
    }
};

struct q38_kv {
    q38_ctx *ctx = nullptr;
    int n_slots = 0;
    int max_pages = 0;
    int max_seqs = 0;
    int pt_stride = 0; /* pages per sequence at most */
    float *kpool = nullptr;
    float *vpool = nullptr;
    int32_t *d_page_table = nullptr;
    std::vector<int32_t> page_table; /* host mirror [max_seqs][pt_stride] */
    std::vector<int32_t> free_pages; /* stack */
    std::vector<char> seq_live;
    std::vector<int32_t> seq_pages; /* pages held per sequence */
    /* pinned staging for page-table uploads, used as a ring */
    int32_t *staging = nullptr;
    size_t staging_len = 0;
    size_t staging_head = 0;
    /* Prefill's bf16 hi/lo images of each (sequence, slot)'s 32-key blocks,
     * [4 kv heads][cap] x Q38_PREFILL_IMAGE_BYTES, kept between calls:
     * blocks [0, valid) are images of the keys and values now in the cache.
     * Every write at position p cuts valid to p / 32. */
    struct Images {
        void *buf = nullptr;
        int cap = 0;
        int valid = 0;
    };
    std::vector<Images> images; /* [max_seqs][n_slots] */
    bool image_cache = true;

    Images &img(int seq, int slot) { return images[(size_t)seq * n_slots + slot]; }

    /* positions >= pos of `seq` changed in `slot` (every slot when slot < 0) */
    void images_from(int seq, int slot, long pos) {
        const int b = (int)std::min<long>(std::max<long>(pos, 0) / Q38_PREFILL_KEYS, 1L << 30);
        for (int s = slot < 0 ? 0 : slot; s < (slot < 0 ? n_slots : slot + 1); ++s) {
            Images &im = img(seq, s);
            im.valid = std::min(im.valid, b);
        }
    }

    /* the sequence's image buffers released (no call may still read them) */
    void images_free(int seq) {
        bool any = false;
        for (int s = 0; s < n_slots; ++s) any |= img(seq, s).buf != nullptr;
        if (!any) return;
        (void)hipStreamSynchronize(ctx->stream);
        for (int s = 0; s < n_slots; ++s) {
            Images &im = img(seq, s);
            if (im.buf != nullptr) (void)hipFree(im.buf);
            im = Images();
        }
    }

    size_t slot_floats() const { return (size_t)max_pages * Q38_PAGE_FLOATS; }
    float *kslot(int slot) const { return kpool + (size_t)slot * slot_floats(); }
    float *vslot(int slot) const { return vpool + (size_t)slot * slot_floats(); }

    int check_seq(int seq) const {
        if (seq < 0 || seq >= max_seqs || !seq_live[seq]) return fail("sequence %d does not exist", seq);
        return 0;
    }

    /* Copy page-table entries [first, first+count) of `seq` to the device,
     * stream-ordered, through the pinned ring. */
    int upload_entries(int seq, int first, int count) {
        if (count <= 0) return 0;
        if ((size_t)count > staging_len) return fail("page-table update larger than staging");
        if (staging_head + count > staging_len) {
            Q38_HIP(hipStreamSynchronize(ctx->stream));
            staging_head = 0;
        }
        int32_t *src = staging + staging_head;
        memcpy(src, &page_table[(size_t)seq * pt_stride + first], sizeof(int32_t) * count);
        staging_head += count;
        Q38_HIP(hipMemcpyAsync(d_page_table + (size_t)seq * pt_stride + first, src,
                               sizeof(int32_t) * count, hipMemcpyHostToDevice, ctx->stream));
        return 0;
    }

    int reserve(int seq, int n_tokens) {
        if (n_tokens < 0) return fail("negative token count");
        const int need = (n_tokens + Q38_PAGE_TOKENS - 1) / Q38_PAGE_TOKENS;
        if (need > pt_stride)
            return fail("sequence %d: %d tokens exceed the per-sequence limit of %d", seq, n_tokens,
                        pt_stride * Q38_PAGE_TOKENS);
        const int have = seq_pages[seq];
        if (need <= have) return 0;
        if ((size_t)(need - have) > free_pages.size())
            return fail("KV pool exhausted: need %d pages, %zu free", need - have, free_pages.size());
        for (int p = have; p < need; ++p) {
            page_table[(size_t)seq * pt_stride + p] = free_pages.back();
            free_pages.pop_back();
        }
        seq_pages[seq] = need;
        return upload_entries(seq, have, need - have);
    }

    void release_from(int seq, int keep_pages) {
        images_from(seq, -1, (long)keep_pages * Q38_PAGE_TOKENS);
        for (int p = seq_pages[seq] - 1; p >= keep_pages; --p) {
            free_pages.push_back(page_table[(size_t)seq * pt_stride + p]);
            page_table[(size_t)seq * pt_stride + p] = -1;
        }
        seq_pages[seq] = std::min(seq_pages[seq], keep_pages);
    }

    int slot_of(int layer, int *slot) const {
        if (!is_full_attention(layer)) return fail("layer %d is not a full-attention layer", layer);
        if (layer / 4 >= n_slots) return fail("layer %d needs slot %d, cache has %d", layer, layer / 4, n_slots);
        *slot = layer / 4;
        return 0;
    }
};

/* ======================================================================= */

extern "C" {

const char *q38_last_error(void) { return g_last_error.c_str(); }

int q38_device_count(int *count) {
    if (count == nullptr) return fail("count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return 0;
}

int q38_ctx_create(q38_ctx **out, int device, const char *module_dir) {
    if (out == nullptr) return fail("out is NULL");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail("no HIP device available");
    if (device < 0 || device >= n) return fail("device %d out of range (%d devices)", device, n);
    /* a failure part-way through set-up releases what was created so far */
    std::unique_ptr<q38_ctx, int (*)(q38_ctx *)> ctx(new q38_ctx, q38_ctx_destroy);
    ctx->device = device;
    Q38_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    Q38_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail("device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    ctx->cu_count = prop.multiProcessorCount;
    ctx->clock_khz = prop.clockRate;
    ctx->lds_bytes = (int)prop.sharedMemPerBlock;
    ctx->lds_per_cu = (int)prop.maxSharedMemoryPerMultiProcessor;
    snprintf(ctx->name, sizeof(ctx->name), "%.200s (%.40s)", prop.name, prop.gcnArchName);
    Q38_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    {
        const int e = q38_scratch_address(device, &ctx->scratch);
        if (e != 0) return fail("device scratch lookup failed: %s", hipGetErrorString((hipError_t)e));
    }

    const std::string dir = module_dir != nullptr ? std::string(module_dir) : library_dir();
    const std::string p_decode = dir + "/attn_decode.hsaco";
    const std::string p_gdn = dir + "/gdn.hsaco";
    Q38_HIP(hipModuleLoad(&ctx->mod_decode, p_decode.c_str()));
    Q38_HIP(hipModuleLoad(&ctx->mod_gdn, p_gdn.c_str()));
    const std::string p_chunk = dir + "/gdn_chunk.hsaco";
    Q38_HIP(hipModuleLoad(&ctx->mod_gdn_chunk, p_chunk.c_str()));
    Q38_HIP(hipModuleGetFunction(&ctx->f_chunk_prep, ctx->mod_gdn_chunk, "q38_gdn_chunk_prep"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_chunk_scan, ctx->mod_gdn_chunk, "q38_gdn_chunk_scan"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gdn_post, ctx->mod_gdn_chunk, "q38_gdn_post"));
    const std::string p_prefill = dir + "/attn_prefill.hsaco";
    Q38_HIP(hipModuleLoad(&ctx->mod_prefill, p_prefill.c_str()));
    Q38_HIP(hipModuleGetFunction(&ctx->f_prefill, ctx->mod_prefill, "q38_attn_prefill_mfma"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_kv_split, ctx->mod_prefill, "q38_kv_split_mfma"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_prefill_merge, ctx->mod_prefill, "q38_prefill_merge"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_split, ctx->mod_decode, "q38_attn_decode_split"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_split_many, ctx->mod_decode, "q38_attn_decode_split_many"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_split_pre, ctx->mod_decode, "q38_attn_decode_split_pre"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_split_one, ctx->mod_decode, "q38_attn_decode_split_one"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_split_pre_one, ctx->mod_decode, "q38_attn_decode_split_pre_one"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_split_pre_many, ctx->mod_decode,
                                 "q38_attn_decode_split_pre_many"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_decode_merge, ctx->mod_decode, "q38_attn_decode_merge"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_kv_copy, ctx->mod_decode, "q38_kv_copy"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_attn_pre, ctx->mod_decode, "q38_attn_pre"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gdn_decode, ctx->mod_gdn, "q38_gdn_decode"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gdn_pre, ctx->mod_gdn, "q38_gdn_pre"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gdn_step_rows, ctx->mod_gdn, "q38_gdn_step_rows"));
    Q38_HIP(hipFuncGetAttribute(&ctx->decode_block, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                ctx->f_decode_split));
    Q38_HIP(hipFuncGetAttribute(&ctx->gdn_decode_block, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                ctx->f_gdn_decode));
    /* the decode kernel's reductions and its page-id array are sized for
     * exactly Q38_DECODE_WAVES waves */
    if (ctx->decode_block != 64 * Q38_DECODE_WAVES)
        return fail("decode kernel has block size %d, expected %d", ctx->decode_block, 64 * Q38_DECODE_WAVES);
    const std::string p_proj = dir + "/proj.hsaco";
    Q38_HIP(hipModuleLoad(&ctx->mod_proj, p_proj.c_str()));
    Q38_HIP(hipModuleGetFunction(&ctx->f_quantize_q8k, ctx->mod_proj, "q38_quantize_q8k"));
    for (int i = 0; i < kGemvTypes; ++i)
        Q38_HIP(hipModuleGetFunction(&ctx->f_gemv_q8k[i], ctx->mod_proj, kGemv[i].kernel));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemv_f32[0], ctx->mod_proj, "q38_gemv_f32_f32"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemv_f32[1], ctx->mod_proj, "q38_gemv_f32_f16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemv_f32[2], ctx->mod_proj, "q38_gemv_f32_bf16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32[0], ctx->mod_proj, "q38_gemm_f32_f32"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32[1], ctx->mod_proj, "q38_gemm_f32_f16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32[2], ctx->mod_proj, "q38_gemm_f32_bf16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32[3], ctx->mod_proj, "q38_gemm_f32_q8_0"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32s[0], ctx->mod_proj, "q38_gemm_f32s_f32"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32s[1], ctx->mod_proj, "q38_gemm_f32s_f16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32s[2], ctx->mod_proj, "q38_gemm_f32s_bf16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32s[3], ctx->mod_proj, "q38_gemm_f32s_q8_0"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32w[1], ctx->mod_proj, "q38_gemm_f32w_f16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32w[2], ctx->mod_proj, "q38_gemm_f32w_bf16"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_f32w[3], ctx->mod_proj, "q38_gemm_f32w_q8_0"));
    for (int t = 0; t < 4; ++t) {
        char nm[64];
        snprintf(nm, sizeof(nm), "q38_gemv_f32_q8_0s_r%d_t%d", t == 3 ? 4 : 2, 1 << t);
        Q38_HIP(hipModuleGetFunction(&ctx->f_gemv_q80s[t], ctx->mod_proj, nm));
    }
    for (int i = 0; i < kGemvTypes; ++i) {
        int n = 0;
        Q38_HIP(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, ctx->f_gemv_q8k[i], 256, 0));
        ctx->gemv_occupancy[i] = std::max(1, n);
    }
    for (int i = 0; i < kGemvTypes; ++i) {
        if (kGemv[i].gemm_kernel != nullptr)
            Q38_HIP(hipModuleGetFunction(&ctx->f_gemm[i], ctx->mod_proj, kGemv[i].gemm_kernel));
        if (kGemv[i].gemm_ks_kernel != nullptr)
            Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_ks[i], ctx->mod_proj, kGemv[i].gemm_ks_kernel));
        if (kGemv[i].gemm_ks16_kernel != nullptr)
            Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_ks16[i], ctx->mod_proj, kGemv[i].gemm_ks16_kernel));
        if (kGemv[i].gemm_ks4_kernel != nullptr)
            Q38_HIP(hipModuleGetFunction(&ctx->f_gemm_ks4[i], ctx->mod_proj, kGemv[i].gemm_ks4_kernel));
    }
    const std::string p_synth = dir + "/synth.hsaco";
    Q38_HIP(hipModuleLoad(&ctx->mod_synth, p_synth.c_str()));
    Q38_HIP(hipModuleGetFunction(&ctx->f_fill_normal, ctx->mod_synth, "q38_fill_normal"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_copy, ctx->mod_synth, "q38_copy_f32"));
    Q38_HIP(hipModuleGetFunction(&ctx->f_noop, ctx->mod_synth, "q38_noop"));
    /* ops.rs:596: 1e7^(-2/64) in f32, computed once with the host's powf */
    ctx->rope_theta_scale = powf(10000000.0f, -2.0f / 64.0f);
    *out = ctx.release();
    return 0;
}

int q38_ctx_destroy(q38_ctx *ctx) {
    if (ctx == nullptr) return 0;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->work) (void)hipFree(ctx->work);
    if (ctx->arrivals) (void)hipFree(ctx->arrivals);
    if (ctx->mod_decode) (void)hipModuleUnload(ctx->mod_decode);
    if (ctx->mod_gdn) (void)hipModuleUnload(ctx->mod_gdn);
    if (ctx->mod_prefill) (void)hipModuleUnload(ctx->mod_prefill);
    if (ctx->mod_gdn_chunk) (void)hipModuleUnload(ctx->mod_gdn_chunk);
    if (ctx->mod_synth) (void)hipModuleUnload(ctx->mod_synth);
    if (ctx->mod_proj) (void)hipModuleUnload(ctx->mod_proj);
    for (hipEvent_t e : ctx->timer_events) (void)hipEventDestroy(e);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return 0;
}

void *q38_ctx_stream(q38_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int q38_sync(q38_ctx *ctx) {
    if (ctx == nullptr) return fail("ctx is NULL");
    Q38_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int q38_set_decode_split(q38_ctx *ctx, int tokens) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (tokens != 0 && (tokens < Q38_PAGE_TOKENS || tokens > Q38_MAX_SPLIT_TOKENS || tokens % Q38_PAGE_TOKENS != 0))
        return fail("split of %d tokens: 0, or a multiple of %d in %d..%d", tokens, Q38_PAGE_TOKENS, Q38_PAGE_TOKENS,
                    Q38_MAX_SPLIT_TOKENS);
    ctx->split_tokens = tokens;
    return 0;
}

int q38_device_info(q38_ctx *ctx, int *cu_count, int *clock_khz, int *lds_bytes, char *name,
                    size_t name_len) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (cu_count) *cu_count = ctx->cu_count;
    if (clock_khz) *clock_khz = ctx->clock_khz;
    if (lds_bytes) *lds_bytes = ctx->lds_bytes;
    if (name && name_len) snprintf(name, name_len, "%s", ctx->name);
    return 0;
}

int q38_alloc(q38_ctx *ctx, size_t bytes, void **d_ptr) {
    if (ctx == nullptr || d_ptr == nullptr) return fail("NULL argument");
    *d_ptr = nullptr;
    Q38_HIP(hipMalloc(d_ptr, bytes ? bytes : 4));
    return 0;
}

int q38_free(q38_ctx *ctx, void *d_ptr) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (d_ptr == nullptr) return 0;
    Q38_HIP(hipStreamSynchronize(ctx->stream));
    Q38_HIP(hipFree(d_ptr));
    return 0;
}

int q38_upload(q38_ctx *ctx, void *d_dst, const void *src, size_t bytes) {
    if (ctx == nullptr || d_dst == nullptr || src == nullptr) return fail("NULL argument");
    Q38_HIP(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    Q38_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int q38_download(q38_ctx *ctx, void *dst, const void *d_src, size_t bytes) {
    if (ctx == nullptr || dst == nullptr || d_src == nullptr) return fail("NULL argument");
    Q38_HIP(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    Q38_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int q38_zero(q38_ctx *ctx, void *d_dst, size_t bytes) {
    if (ctx == nullptr || d_dst == nullptr) return fail("NULL argument");
    Q38_HIP(hipMemsetAsync(d_dst, 0, bytes, ctx->stream));
    return 0;
}

int q38_event_create(q38_ctx *ctx, void **event) {
    if (ctx == nullptr || event == nullptr) return fail("NULL argument");
    hipEvent_t e;
    Q38_HIP(hipEventCreate(&e));
    *event = (void *)e;
    return 0;
}

int q38_event_record(q38_ctx *ctx, void *event) {
    if (ctx == nullptr || event == nullptr) return fail("NULL argument");
    Q38_HIP(hipEventRecord((hipEvent_t)event, ctx->stream));
    return 0;
}

int q38_event_elapsed_ms(void *start, void *stop, float *ms) {
    if (start == nullptr || stop == nullptr || ms == nullptr) return fail("NULL argument");
    Q38_HIP(hipEventSynchronize((hipEvent_t)stop));
    Q38_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return 0;
}

int q38_event_destroy(void *event) {
    if (event == nullptr) return 0;
    Q38_HIP(hipEventDestroy((hipEvent_t)event));
    return 0;
}

int q38_fill_normal(q38_ctx *ctx, float *d_out, size_t n, uint64_t seed, float sigma, float mean) {
    if (ctx == nullptr || d_out == nullptr) return fail("NULL argument");
    if (n == 0) return 0;
    struct {
        float *out;
        uint64_t n;
        uint64_t seed;
        float sigma;
        float mean;
    } a = {d_out, (uint64_t)n, seed, sigma, mean};
    const uint64_t pairs = ((uint64_t)n + 1) / 2;
    const uint64_t blocks = (pairs + 255) / 256;
    if (blocks > 0x7FFFFFFFull) return fail("fill of %zu elements is too large", n);
    return ctx->launch(ctx->f_fill_normal, (unsigned)blocks, 1, 1, 256, &a);
}

int q38_device_copy(q38_ctx *ctx, void *d_dst, const void *d_src, size_t bytes) {
    if (ctx == nullptr || d_dst == nullptr || d_src == nullptr) return fail("NULL argument");
    if (bytes == 0) return 0;
    if (bytes % 16 != 0 || ((uintptr_t)d_dst | (uintptr_t)d_src) % 16 != 0)
        return fail("q38_device_copy needs 16-byte aligned pointers and a multiple of 16 bytes");
    struct {
        const void *src;
        void *dst;
        uint64_t n4;
    } a = {d_src, d_dst, (uint64_t)(bytes / 16)};
    const uint64_t blocks = (a.n4 + 255) / 256;
    if (blocks > 0x7FFFFFFFull) return fail("copy of %zu bytes is too large", bytes);
    return ctx->launch(ctx->f_copy, (unsigned)blocks, 1, 1, 256, &a);
}

int q38_device_noop(q38_ctx *ctx) {
    if (ctx == nullptr) return fail("ctx is NULL");
    int32_t unused = 0;
    return ctx->launch(ctx->f_noop, 1, 1, 1, 64, &unused);
}

int q38_kernel_timer_start(q38_ctx *ctx, const char *kernel_name, int max_launches) {
    if (ctx == nullptr || kernel_name == nullptr) return fail("NULL argument");
    if (max_launches < 1) return fail("max_launches must be positive");
    hipFunction_t f = nullptr;
    const std::string name(kernel_name);
    if (name == "q38_attn_decode_split") f = ctx->f_decode_split;
    else if (name == "q38_attn_decode_split_many") f = ctx->f_decode_split_many;
    else if (name == "q38_attn_decode_split_pre") f = ctx->f_decode_split_pre;
    else if (name == "q38_attn_decode_split_pre_many") f = ctx->f_decode_split_pre_many;
    else if (name == "q38_attn_decode_split_one") f = ctx->f_decode_split_one;
    else if (name == "q38_attn_decode_split_pre_one") f = ctx->f_decode_split_pre_one;
    else if (name == "q38_attn_decode_merge") f = ctx->f_decode_merge;
    else if (name == "q38_kv_copy") f = ctx->f_kv_copy;
    else if (name == "q38_attn_pre") f = ctx->f_attn_pre;
    else if (name == "q38_gdn_decode") f = ctx->f_gdn_decode;
    else if (name == "q38_gdn_pre") f = ctx->f_gdn_pre;
    else if (name == "q38_gdn_step_rows") f = ctx->f_gdn_step_rows;
    else if (name == "q38_copy_f32") f = ctx->f_copy;
    else if (name == "q38_noop") f = ctx->f_noop;
    else if (name == "q38_quantize_q8k") f = ctx->f_quantize_q8k;
    else if (name == "q38_gemv_f32_f32") f = ctx->f_gemv_f32[0];
    else if (name == "q38_gemv_f32_f16") f = ctx->f_gemv_f32[1];
    else if (name == "q38_gemv_f32_bf16") f = ctx->f_gemv_f32[2];
    else if (name == "q38_gemm_f32_f32") f = ctx->f_gemm_f32[0];
    else if (name == "q38_gemm_f32_f16") f = ctx->f_gemm_f32[1];
    else if (name == "q38_gemm_f32_bf16") f = ctx->f_gemm_f32[2];
    else if (name == "q38_gemm_f32_q8_0") f = ctx->f_gemm_f32[3];
    else if (name == "q38_gemm_f32s_f32") f = ctx->f_gemm_f32s[0];
    else if (name == "q38_gemm_f32s_f16") f = ctx->f_gemm_f32s[1];
    else if (name == "q38_gemm_f32s_bf16") f = ctx->f_gemm_f32s[2];
    else if (name == "q38_gemm_f32s_q8_0") f = ctx->f_gemm_f32s[3];
    else if (name == "q38_gemm_f32w_f16") f = ctx->f_gemm_f32w[1];
    else if (name == "q38_gemm_f32w_bf16") f = ctx->f_gemm_f32w[2];
    else if (name == "q38_gemm_f32w_q8_0") f = ctx->f_gemm_f32w[3];
    else if (name == "q38_gemv_f32_q8_0s_r2_t1") f = ctx->f_gemv_q80s[0];
    else if (name == "q38_gemv_f32_q8_0s_r2_t2") f = ctx->f_gemv_q80s[1];
    else if (name == "q38_gemv_f32_q8_0s_r2_t4") f = ctx->f_gemv_q80s[2];
    else if (name == "q38_gemv_f32_q8_0s_r4_t8") f = ctx->f_gemv_q80s[3];
    else if (name == "q38_attn_prefill_mfma") f = ctx->f_prefill;
    else if (name == "q38_kv_split_mfma") f = ctx->f_kv_split;
    else if (name == "q38_prefill_merge") f = ctx->f_prefill_merge;
    else if (name == "q38_gdn_chunk_prep") f = ctx->f_chunk_prep;
    else if (name == "q38_gdn_chunk_scan") f = ctx->f_chunk_scan;
    else if (name == "q38_gdn_post") f = ctx->f_gdn_post;
    else {
        for (int i = 0; i < kGemvTypes; ++i) {
            if (name == kGemv[i].kernel) f = ctx->f_gemv_q8k[i];
            if (kGemv[i].gemm_kernel != nullptr && name == kGemv[i].gemm_kernel) f = ctx->f_gemm[i];
            if (kGemv[i].gemm_ks_kernel != nullptr && name == kGemv[i].gemm_ks_kernel) f = ctx->f_gemm_ks[i];
            if (kGemv[i].gemm_ks16_kernel != nullptr && name == kGemv[i].gemm_ks16_kernel) f = ctx->f_gemm_ks16[i];
            if (kGemv[i].gemm_ks4_kernel != nullptr && name == kGemv[i].gemm_ks4_kernel) f = ctx->f_gemm_ks4[i];
        }
        if (f == nullptr) return fail("unknown kernel %s", kernel_name);
    }
    while ((int)ctx->timer_events.size() < 2 * max_launches) {
        hipEvent_t e;
        Q38_HIP(hipEventCreate(&e));
        ctx->timer_events.push_back(e);
    }
    ctx->timed = f;
    ctx->timer_used = 0;
    return 0;
}

int q38_kernel_timer_stop(q38_ctx *ctx, float *total_ms, int *launches) {
    if (ctx == nullptr || total_ms == nullptr || launches == nullptr) return fail("NULL argument");
    ctx->timed = nullptr;
    Q38_HIP(hipStreamSynchronize(ctx->stream));
    double total = 0.0;
    for (int i = 0; i + 1 < ctx->timer_used; i += 2) {
        float ms = 0.0f;
        Q38_HIP(hipEventElapsedTime(&ms, ctx->timer_events[i], ctx->timer_events[i + 1]));
        total += ms;
    }
    *total_ms = (float)total;
    *launches = ctx->timer_used / 2;
    ctx->timer_used = 0;
    return 0;
}

/* ------------------------------------------------------------------ KV cache */

int q38_kv_create(q38_ctx *ctx, int n_slots, int max_pages, int max_seqs, int max_tokens_per_seq,
                  q38_kv **out) {
    if (ctx == nullptr || out == nullptr) return fail("NULL argument");
    *out = nullptr;
    if (n_slots < 1 || n_slots > 17) return fail("n_slots %d outside 1..17", n_slots);
    if (max_pages < 1 || max_seqs < 1 || max_tokens_per_seq < 1)
        return fail("max_pages, max_seqs and max_tokens_per_seq must be positive");
    if ((long)max_tokens_per_seq > (long)Q38_MAX_SPLITS * Q38_MAX_SPLIT_TOKENS)
        return fail("max_tokens_per_seq %d above the decode limit of %ld", max_tokens_per_seq,
                    (long)Q38_MAX_SPLITS * Q38_MAX_SPLIT_TOKENS);
    std::unique_ptr<q38_kv> kv(new q38_kv);
    kv->ctx = ctx;
    kv->n_slots = n_slots;
    kv->max_pages = max_pages;
    kv->max_seqs = max_seqs;
    kv->pt_stride = (max_tokens_per_seq + Q38_PAGE_TOKENS - 1) / Q38_PAGE_TOKENS;
    const size_t pool_bytes = (size_t)n_slots * max_pages * Q38_PAGE_FLOATS * sizeof(float);
    Q38_HIP(hipSetDevice(ctx->device));
    Q38_HIP(hipMalloc(&kv->kpool, pool_bytes));
    if (hipMalloc(&kv->vpool, pool_bytes) != hipSuccess) {
        (void)hipFree(kv->kpool);
        return fail("cannot allocate %zu bytes for the V pool", pool_bytes);
    }
    /* zeroed once so that no page ever holds non-finite garbage */
    Q38_HIP(hipMemsetAsync(kv->kpool, 0, pool_bytes, ctx->stream));
    Q38_HIP(hipMemsetAsync(kv->vpool, 0, pool_bytes, ctx->stream));
    const size_t pt_entries = (size_t)max_seqs * kv->pt_stride;
    Q38_HIP(hipMalloc(&kv->d_page_table, pt_entries * sizeof(int32_t)));
    Q38_HIP(hipMemsetAsync(kv->d_page_table, 0xFF, pt_entries * sizeof(int32_t), ctx->stream));
    kv->page_table.assign(pt_entries, -1);
    kv->free_pages.resize(max_pages);
    for (int p = 0; p < max_pages; ++p) kv->free_pages[p] = max_pages - 1 - p; /* pop gives 0,1,2.. */
    kv->seq_live.assign(max_seqs, 0);
    kv->seq_pages.assign(max_seqs, 0);
    kv->images.assign((size_t)max_seqs * n_slots, q38_kv::Images());
    kv->staging_len = std::max<size_t>(1 << 16, (size_t)kv->pt_stride * 4);
    Q38_HIP(hipHostMalloc((void **)&kv->staging, kv->staging_len * sizeof(int32_t), hipHostMallocDefault));
    Q38_HIP(hipStreamSynchronize(ctx->stream));
    *out = kv.release();
    return 0;
}

int q38_kv_destroy(q38_kv *kv) {
    if (kv == nullptr) return 0;
    (void)hipStreamSynchronize(kv->ctx->stream);
    for (q38_kv::Images &im : kv->images)
        if (im.buf != nullptr) (void)hipFree(im.buf);
    (void)hipFree(kv->kpool);
    (void)hipFree(kv->vpool);
    (void)hipFree(kv->d_page_table);
    (void)hipHostFree(kv->staging);
    delete kv;
    return 0;
}

int q38_kv_set_prefill_cache(q38_kv *kv, int enable) {
    if (kv == nullptr) return fail("kv is NULL");
    if (!enable) {
        for (int s = 0; s < kv->max_seqs; ++s) kv->images_free(s);
    }
    kv->image_cache = enable != 0;
    return 0;
}

int q38_kv_free_pages(q38_kv *kv, int *n_free) {
    if (kv == nullptr || n_free == nullptr) return fail("NULL argument");
    *n_free = (int)kv->free_pages.size();
    return 0;
}

int q38_seq_create(q38_kv *kv, int *seq) {
    if (kv == nullptr || seq == nullptr) return fail("NULL argument");
    for (int s = 0; s < kv->max_seqs; ++s) {
        if (!kv->seq_live[s]) {
            kv->seq_live[s] = 1;
            kv->seq_pages[s] = 0;
            *seq = s;
            return 0;
        }
    }
    return fail("all %d sequence slots are in use", kv->max_seqs);
}

int q38_seq_free(q38_kv *kv, int seq) {
    if (kv == nullptr) return fail("kv is NULL");
    if (kv->check_seq(seq)) return -1;
    kv->release_from(seq, 0);
    kv->images_free(seq);
    kv->seq_live[seq] = 0;
    return 0;
}

int q38_seq_reset(q38_kv *kv, int seq) {
    if (kv == nullptr) return fail("kv is NULL");
    if (kv->check_seq(seq)) return -1;
    kv->release_from(seq, 0);
    return 0;
}

int q38_seq_truncate(q38_kv *kv, int seq, int n_tokens) {
    if (kv == nullptr) return fail("kv is NULL");
    if (kv->check_seq(seq)) return -1;
    if (n_tokens < 0) return fail("negative token count");
    kv->release_from(seq, (n_tokens + Q38_PAGE_TOKENS - 1) / Q38_PAGE_TOKENS);
    return 0;
}

int q38_seq_reserve(q38_kv *kv, int seq, int n_tokens) {
    if (kv == nullptr) return fail("kv is NULL");
    if (kv->check_seq(seq)) return -1;
    return kv->reserve(seq, n_tokens);
}

int q38_seq_set_pages(q38_kv *kv, int seq, int n_pages, const int32_t *page_ids) {
    if (kv == nullptr || (page_ids == nullptr && n_pages > 0)) return fail("NULL argument");
    if (kv->check_seq(seq)) return -1;
    if (n_pages < 0 || n_pages > kv->pt_stride)
        return fail("n_pages %d outside 0..%d", n_pages, kv->pt_stride);
    /* validate first (the sequence's own pages count as available), so a
     * rejected call keeps the sequence's mapping and the pool unchanged */
    std::vector<char> avail(kv->max_pages, 0);
    for (int32_t p : kv->free_pages) avail[p] = 1;
    for (int i = 0; i < kv->seq_pages[seq]; ++i) avail[kv->page_table[(size_t)seq * kv->pt_stride + i]] = 1;
    for (int i = 0; i < n_pages; ++i) {
        const int32_t p = page_ids[i];
        if (p < 0 || p >= kv->max_pages) return fail("page id %d outside the pool of %d", p, kv->max_pages);
        if (!avail[p]) return fail("page %d is not free (held, or listed twice)", p);
        avail[p] = 0;
    }
    kv->release_from(seq, 0);
    std::vector<int32_t> rest;
    rest.reserve(kv->free_pages.size());
    for (int32_t p : kv->free_pages)
        if (avail[p]) rest.push_back(p);
    kv->free_pages.swap(rest);
    for (int i = 0; i < n_pages; ++i) kv->page_table[(size_t)seq * kv->pt_stride + i] = page_ids[i];
    kv->seq_pages[seq] = n_pages;
    return kv->upload_entries(seq, 0, n_pages);
}

int q38_seq_capacity(q38_kv *kv, int seq, int *n_tokens) {
    if (kv == nullptr || n_tokens == nullptr) return fail("NULL argument");
    if (kv->check_seq(seq)) return -1;
    *n_tokens = kv->seq_pages[seq] * Q38_PAGE_TOKENS;
    return 0;
}

static int kv_copy(q38_kv *kv, int layer, int seq, int pos0, int n_tokens, float *d_k, float *d_v,
                   int to_pages) {
    if (kv == nullptr) return fail("kv is NULL");
    if (d_k == nullptr || d_v == nullptr) return fail("NULL row buffer");
    if (kv->check_seq(seq)) return -1;
    int slot = 0;
    if (kv->slot_of(layer, &slot)) return -1;
    if (pos0 < 0 || n_tokens < 0) return fail("negative position or count");
    if (n_tokens == 0) return 0;
    if (to_pages) {
        if (kv->reserve(seq, pos0 + n_tokens)) return -1;
        kv->images_from(seq, slot, pos0);
    } else if (pos0 + n_tokens > kv->seq_pages[seq] * Q38_PAGE_TOKENS) {
        return fail("positions %d..%d are not reserved", pos0, pos0 + n_tokens - 1);
    }
    q38_kv_copy_args a;
    memset(&a, 0, sizeof(a));
    a.kpool = kv->kslot(slot);
    a.vpool = kv->vslot(slot);
    a.page_table = kv->d_page_table;
    a.k_rows = d_k;
    a.v_rows = d_v;
    a.pt_stride = kv->pt_stride;
    a.seq = seq;
    a.pos0 = pos0;
    a.n_tokens = n_tokens;
    a.to_pages = to_pages;
    return kv->ctx->launch(kv->ctx->f_kv_copy, n_tokens, 2, 1, 256, &a);
}

int q38_kv_write(q38_kv *kv, int layer, int seq, int pos0, int n_tokens, const float *d_k,
                 const float *d_v) {
    return kv_copy(kv, layer, seq, pos0, n_tokens, const_cast<float *>(d_k), const_cast<float *>(d_v), 1);
}

int q38_kv_read(q38_kv *kv, int layer, int seq, int pos0, int n_tokens, float *d_k, float *d_v) {
    return kv_copy(kv, layer, seq, pos0, n_tokens, d_k, d_v, 0);
}

/* ------------------------------------------------------------ attention decode */

namespace {

/* Context tokens per decode workgroup: a whole number of pages, at most
 * Q38_MAX_SPLIT_TOKENS, chosen to give one workgroup per CU for one
 * sequence (the split kernel streams fastest so: 46 us at 32768 tokens
 * against 50 us with two per CU; at 1024 tokens 16-token splits, 256
 * workgroups, take 13.2-13.8 us per step against 14.4-14.8 us with 64),
 * unless q38_set_decode_split fixed it. */
constexpr int kMaxSplitsPerSeq = Q38_MAX_SPLITS; /* LDS weights of the merge kernel */

int choose_split_tokens(const q38_ctx *ctx, int n_seq, long total_tokens, long max_tokens, int *split_out) {
    long split = Q38_PAGE_TOKENS;
    if (ctx->split_tokens > 0) {
        split = ctx->split_tokens;
    } else {
        const long slots = std::max(ctx->cu_count, 1);
        const long per = (total_tokens * Q38_ATTN_KV_HEADS + slots - 1) / slots;
        split = std::min<long>((per + Q38_PAGE_TOKENS - 1) / Q38_PAGE_TOKENS * Q38_PAGE_TOKENS,
                               Q38_MAX_SPLIT_TOKENS);
        split = std::max<long>(split, Q38_PAGE_TOKENS);
        /* sequences of different lengths make workgroups of different
         * lengths; past one round of workgroups, 1024-token splits balance
         * them best (32 sequences of 1K-32K tokens: 74% of HBM against 64%
         * with 4096-token splits) */
        if (n_seq > 1) split = std::min<long>(split, 1024);
    }
    /* no sequence may need more splits than the merge kernel holds, and no
     * split more pages than the kernel's page-id array */
    while ((max_tokens + split - 1) / split > kMaxSplitsPerSeq && split < Q38_MAX_SPLIT_TOKENS)
        split = std::min<long>(split * 2, Q38_MAX_SPLIT_TOKENS);
    if ((max_tokens + split - 1) / split > kMaxSplitsPerSeq)
        return fail("context of %ld tokens exceeds %d splits of %d tokens", max_tokens, kMaxSplitsPerSeq,
                    Q38_MAX_SPLIT_TOKENS);
    *split_out = (int)split;
    return 0;
}

/* How one decode launch of n_seq sequences is split: tokens per split, the
 * total number of splits, and the workspace the split-K partials need (0
 * when every sequence fits one split). */
struct decode_plan {
    int split_tokens = 0;
    int total_splits = 0;
    size_t work_bytes = 0;
};

int plan_decode(const q38_ctx *ctx, int n_seq, const int32_t *positions, decode_plan *plan) {
    long total_tokens = 0, max_tokens = 0;
    for (int b = 0; b < n_seq; ++b) {
        total_tokens += positions[b] + 1;
        max_tokens = std::max<long>(max_tokens, positions[b] + 1);
    }
    if (choose_split_tokens(ctx, n_seq, total_tokens, max_tokens, &plan->split_tokens)) return -1;
    int total = 0;
    bool any_multi = false;
    for (int b = 0; b < n_seq; ++b) {
        const int ns = (positions[b] + plan->split_tokens) / plan->split_tokens; /* ceil((pos+1)/split) */
        any_multi |= ns > 1;
        total += ns;
    }
    plan->total_splits = total;
    plan->work_bytes = any_multi ? (size_t)total * Q38_ATTN_HEADS * (Q38_ATTN_HEAD_DIM + 2) * sizeof(float) : 0;
    return 0;
}

/* full_core's pre step fused into the decode kernel: d_q holds raw q|gate
 * rows, d_k_new raw keys; norm weights for both */
struct decode_pre {
    const float *q_norm;
    const float *k_norm;
};

/* The arguments of one decode launch: the split kernel, its grid, and the
 * merge that follows it when some sequence has more than one split. */
struct decode_launch {
    q38_decode_args a;
    q38_merge_args m;
    hipFunction_t f = nullptr;
    unsigned grid_x = 0;
    bool merge = false;
};

/* Arguments of one decode launch for n_seq <= Q38_MAX_BATCH sequences whose
 * pages are reserved; `work` holds plan.work_bytes.  `arg_pages` chooses the
 * split kernel that takes each split's first page ids in its arguments (at
 * most Q38_HEAD_PAGE_SPLITS splits), else the one reading every id from the
 * page table; -1 picks by the split count. */
int build_decode(q38_kv *kv, int slot, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                 const float *d_q, const float *d_k_new, const float *d_v_new, const float *d_gate, float *d_out,
                 const decode_plan &plan, void *work, const decode_pre *pre, int arg_pages_choice,
                 decode_launch *L) {
    q38_ctx *ctx = kv->ctx;
    const int split_tokens = plan.split_tokens;
    q38_decode_args &a = L->a;
    memset(&a, 0, sizeof(a));
    a.kpool = kv->kslot(slot);
    a.vpool = kv->vslot(slot);
    a.page_table = kv->d_page_table;
    a.q = d_q;
    a.k_new = d_k_new;
    a.v_new = d_v_new;
    a.gate = d_gate;
    a.out = d_out;
    a.gate_head_stride = Q38_ATTN_HEAD_DIM;
    if (pre != nullptr) {
        /* q|gate rows: the gate is the second half of each head's 512 */
        a.gate = d_q + Q38_ATTN_HEAD_DIM;
        a.gate_head_stride = 2 * Q38_ATTN_HEAD_DIM;
        a.q_norm = pre->q_norm;
        a.k_norm = pre->k_norm;
        a.theta_scale = ctx->rope_theta_scale;
    }
    a.pt_stride = kv->pt_stride;
    a.n_seq = n_seq;
    a.split_tokens = split_tokens;
    int total = 0;
    for (int b = 0; b < n_seq; ++b) {
        a.seq[b] = seq_ids[b];
        a.pos[b] = positions[b];
        a.split_base[b] = total;
        total += (positions[b] + split_tokens) / split_tokens; /* ceil((pos+1)/split) */
    }
    a.split_base[n_seq] = total;
    a.total_splits = total;
    /* up to 256 splits, each split's first two page ids ride in the launch
     * arguments (from the host mirror of the page table), so the kernel's
     * first row loads wait on no page-table load */
    const bool arg_pages = arg_pages_choice < 0 ? total <= Q38_HEAD_PAGE_SPLITS : arg_pages_choice > 0;
    if (arg_pages) {
        if (total > Q38_HEAD_PAGE_SPLITS)
            return fail("%d splits: at most %d carry their page ids in the arguments", total, Q38_HEAD_PAGE_SPLITS);
        for (int b = 0; b < n_seq; ++b) {
            const int32_t *row = &kv->page_table[(size_t)seq_ids[b] * kv->pt_stride];
            const int held = kv->seq_pages[seq_ids[b]];
            for (int g = a.split_base[b]; g < a.split_base[b + 1]; ++g) {
                const int lp = (int)(((long)(g - a.split_base[b]) * split_tokens) / Q38_PAGE_TOKENS);
                if (lp >= held) return fail("sequence %d: split page %d is not reserved", seq_ids[b], lp);
                a.head_pages[g][0] = row[lp];
                a.head_pages[g][1] = row[lp + 1 < held ? lp + 1 : lp];
            }
        }
    }

    L->merge = plan.work_bytes > 0;
    if (work != nullptr) {
        a.part_o = static_cast<float *>(work);
        a.part_ml = a.part_o + (size_t)total * Q38_ATTN_HEADS * Q38_ATTN_HEAD_DIM;
    } else if (L->merge) {
        return fail("decode workspace missing");
    }
    const bool one = arg_pages && n_seq == 1;
    L->f = pre != nullptr ? (one ? ctx->f_decode_split_pre_one
                                 : arg_pages ? ctx->f_decode_split_pre : ctx->f_decode_split_pre_many)
                          : (one ? ctx->f_decode_split_one : arg_pages ? ctx->f_decode_split : ctx->f_decode_split_many);
    L->grid_x = (unsigned)total;
    q38_merge_args &m = L->m;
    memset(&m, 0, sizeof(m));
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    m.gate = a.gate;
    m.gate_head_stride = a.gate_head_stride;
    m.out = d_out;
    m.n_seq = n_seq;
    memcpy(m.split_base, a.split_base, sizeof(m.split_base));
    return 0;
}

/* One decode launch (plus the merge) for n_seq <= Q38_MAX_BATCH sequences
 * whose pages are reserved; `work` holds plan.work_bytes. */
int decode_chunk(q38_kv *kv, int slot, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                 const float *d_q, const float *d_k_new, const float *d_v_new, const float *d_gate,
                 float *d_out, const decode_plan &plan, void *work, const decode_pre *pre = nullptr) {
    q38_ctx *ctx = kv->ctx;
    decode_launch L;
    if (build_decode(kv, slot, n_seq, seq_ids, positions, d_q, d_k_new, d_v_new, d_gate, d_out, plan,
                     plan.work_bytes > 0 ? work : nullptr, pre, -1, &L))
        return -1;
    if (ctx->launch(L.f, L.grid_x, Q38_ATTN_KV_HEADS, 1, ctx->decode_block, &L.a)) return -1;
    if (L.merge && ctx->launch(ctx->f_decode_merge, n_seq, Q38_ATTN_HEADS, 4, 256, &L.m)) return -1;
    return 0;
}

/* Every check of a decode call, with nothing changed: the layer is a
 * full-attention layer with a slot, sequences exist (and are distinct when
 * the call appends), positions are inside the context limit (the reference's
 * KV bounds check, ops.rs:860-864, and its context-full check, :1702), and
 * the pool holds the pages the whole batch must take for its appends; a
 * call that does not append must find its positions reserved. */
int validate_decode(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                    bool appends, int *slot) {
    if (kv == nullptr) return fail("kv is NULL");
    if (kv->slot_of(layer, slot)) return -1;
    if (n_seq < 0) return fail("negative n_seq");
    if (n_seq > 0 && (seq_ids == nullptr || positions == nullptr)) return fail("NULL seq_ids/positions");
    long pages_needed = 0;
    for (int b = 0; b < n_seq; ++b) {
        const int s = seq_ids[b];
        if (kv->check_seq(s)) return -1;
        if (positions[b] < 0) return fail("negative position %d", positions[b]);
        if ((long)positions[b] + 1 > (long)kv->pt_stride * Q38_PAGE_TOKENS)
            return fail("position %d is past the context limit %d", positions[b],
                        kv->pt_stride * Q38_PAGE_TOKENS);
        for (int c = 0; c < b; ++c)
            if (seq_ids[c] == s && appends) return fail("sequence %d appears twice", s);
        const int need = positions[b] / Q38_PAGE_TOKENS + 1;
        if (appends) {
            pages_needed += std::max(0, need - kv->seq_pages[s]);
        } else if (need > kv->seq_pages[s]) {
            return fail("sequence %d: position %d is not reserved", s, positions[b]);
        }
    }
    if (pages_needed > (long)kv->free_pages.size())
        return fail("KV pool exhausted: the batch needs %ld more pages, %zu free", pages_needed,
                    kv->free_pages.size());
    return 0;
}

/* The decode of n_seq sequences in launches of up to Q38_MAX_BATCH: every
 * check first, then the workspace, then the page reservations, so that a
 * call that fails leaves the cache as it was.  `pre` set: full_core's
 * norm + RoPE fused (d_q holds q|gate rows, d_k_new raw keys). */
int decode_all(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids, const int32_t *positions,
               const float *d_q, const float *d_k_new, const float *d_v_new, const float *d_gate, float *d_out,
               const decode_pre *pre, void *fixed_work = nullptr, size_t fixed_bytes = 0) {
    int slot = 0;
    const bool appends = d_k_new != nullptr;
    if (validate_decode(kv, layer, n_seq, seq_ids, positions, appends, &slot)) return -1;
    if (n_seq == 0) return 0;
    q38_ctx *ctx = kv->ctx;
    size_t work_bytes = 0;
    for (int b0 = 0; b0 < n_seq; b0 += Q38_MAX_BATCH) {
        decode_plan plan;
        if (plan_decode(ctx, std::min(Q38_MAX_BATCH, n_seq - b0), positions + b0, &plan)) return -1;
        work_bytes = std::max(work_bytes, plan.work_bytes);
    }
    void *work = nullptr;
    if (fixed_work != nullptr) {
        /* the caller's fixed area: no allocation, so the call must fit */
        if (work_bytes > fixed_bytes)
            return fail("split-K partials need %zu bytes, the fixed scratch holds %zu", work_bytes, fixed_bytes);
        work = fixed_work;
    } else {
        if (work_bytes > 0 && ctx->ensure_work(work_bytes)) return -1;
        work = ctx->work;
    }
    if (appends)
        for (int b = 0; b < n_seq; ++b) {
            if (kv->reserve(seq_ids[b], positions[b] + 1)) return -1;
            kv->images_from(seq_ids[b], slot, positions[b]);
        }
    const size_t q_rows = pre != nullptr ? Q38_ATTN_QG_DIM : Q38_ATTN_Q_DIM;
    for (int b0 = 0; b0 < n_seq; b0 += Q38_MAX_BATCH) {
        const int n = std::min(Q38_MAX_BATCH, n_seq - b0);
        decode_plan plan;
        if (plan_decode(ctx, n, positions + b0, &plan)) return -1;
        const size_t kvoff = (size_t)b0 * Q38_ATTN_KV_DIM;
        const size_t qoff = (size_t)b0 * Q38_ATTN_Q_DIM;
        if (decode_chunk(kv, slot, n, seq_ids + b0, positions + b0, d_q + (size_t)b0 * q_rows,
                         d_k_new ? d_k_new + kvoff : nullptr, d_v_new ? d_v_new + kvoff : nullptr,
                         d_gate ? d_gate + qoff : nullptr, d_out + qoff, plan, work, pre))
            return -1;
    }
    return 0;
}

}  // namespace

int q38_attn_decode(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids,
                    const int32_t *positions, const float *d_q, const float *d_k_new,
                    const float *d_v_new, const float *d_gate, float *d_out) {
    if ((d_k_new == nullptr) != (d_v_new == nullptr)) return fail("d_k_new and d_v_new go together");
    if (n_seq > 0 && (d_q == nullptr || d_out == nullptr)) return fail("NULL q/out");
    return decode_all(kv, layer, n_seq, seq_ids, positions, d_q, d_k_new, d_v_new, d_gate, d_out, nullptr);
}

int q38_attn_pre(q38_ctx *ctx, int n_tokens, int pos0, const float *d_q_norm, const float *d_k_norm,
                 const float *d_q_and_gate, const float *d_key, float *d_q_out, float *d_gate_out,
                 float *d_k_out) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (n_tokens < 0 || pos0 < 0) return fail("negative count or position");
    if (n_tokens == 0) return 0;
    if (!d_q_norm || !d_k_norm || !d_q_and_gate || !d_key || !d_q_out || !d_gate_out || !d_k_out)
        return fail("NULL argument");
    q38_attn_pre_args a;
    memset(&a, 0, sizeof(a));
    a.q_and_gate = d_q_and_gate;
    a.key = d_key;
    a.q_norm = d_q_norm;
    a.k_norm = d_k_norm;
    a.q_out = d_q_out;
    a.gate_out = d_gate_out;
    a.k_out = d_k_out;
    a.pos0 = pos0;
    a.n_tokens = n_tokens;
    a.theta_scale = ctx->rope_theta_scale;
    static_assert((Q38_ATTN_HEADS + Q38_ATTN_KV_HEADS) % 4 == 0, "4 heads per workgroup");
    return ctx->launch(ctx->f_attn_pre, n_tokens, (Q38_ATTN_HEADS + Q38_ATTN_KV_HEADS) / 4, 1, 256, &a);
}

int q38_full_core(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids,
                  const int32_t *positions, const float *d_q_norm, const float *d_k_norm,
                  const float *d_q_and_gate, const float *d_key, const float *d_value,
                  float *d_out) {
    if (n_seq > 0 && (!d_q_norm || !d_k_norm || !d_q_and_gate || !d_key || !d_value || !d_out))
        return fail("NULL argument");
    /* the pre step (q/gate split, q and k RMSNorm, RoPE) runs inside the
     * decode kernel: no separate launch and no intermediate rows */
    const decode_pre pre{d_q_norm, d_k_norm};
    return decode_all(kv, layer, n_seq, seq_ids, positions, d_q_and_gate, d_key, d_value, nullptr, d_out, &pre);
}

int q38_full_core_noalloc(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids,
                          const int32_t *positions, const float *d_q_norm, const float *d_k_norm,
                          const float *d_q_and_gate, const float *d_key, const float *d_value,
                          float *d_out) {
    if (kv == nullptr) return fail("kv is NULL");
    if (n_seq > 0 && (!d_q_norm || !d_k_norm || !d_q_and_gate || !d_key || !d_value || !d_out))
        return fail("NULL argument");
    if (kv->ctx->scratch == nullptr) return fail("device scratch is not set up");
    const decode_pre pre{d_q_norm, d_k_norm};
    return decode_all(kv, layer, n_seq, seq_ids, positions, d_q_and_gate, d_key, d_value, nullptr, d_out, &pre,
                      kv->ctx->scratch, Q38_NOALLOC_SCRATCH_BYTES);
}

/* ----------------------------------------------------- replayed token graph */

/* A token's work as one instantiated HIP graph, in the order it was added:
 * full-attention decode calls (a split node and a merge node each; the merge
 * exits at once when every sequence has one split), one-token linear_core
 * calls (one node each), and graphs of the caller's own work (one child node
 * each, copied at the add).  Only the decode calls depend on the positions;
 * their launch arguments and grids are rewritten in place by
 * q38_decode_graph_set_positions. */
struct q38_decode_graph {
    struct Call {
        q38_decode_call c;
        int slot = 0;
        bool appends = false;
        bool has_pre = false;
        decode_pre pre{nullptr, nullptr};
        hipGraphNode_t split_node = nullptr;
        hipGraphNode_t merge_node = nullptr;
        decode_launch L;
    };
    q38_kv *kv = nullptr;
    int n_seq = 0;
    int arg_pages = 0; /* the split kernel taking first page ids as arguments (batch 1) */
    int32_t seq_ids[Q38_MAX_BATCH] = {0};
    int32_t positions[Q38_MAX_BATCH] = {0};
    std::vector<Call> calls;
    void *work = nullptr;
    size_t work_bytes = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipGraphNode_t last = nullptr; /* the node the next step depends on */
    int steps = 0;

    ~q38_decode_graph() {
        if (exec != nullptr) (void)hipGraphExecDestroy(exec);
        if (graph != nullptr) (void)hipGraphDestroy(graph);
        if (work != nullptr) (void)hipFree(work);
    }

    /* The split-K workspace for `pos`, grown only while no replay runs
     * (the caller's stream has been waited for). */
    int ensure_work(const int32_t *pos, decode_plan *plan) {
        if (plan_decode(kv->ctx, n_seq, pos, plan)) return -1;
        if (arg_pages && plan->total_splits > Q38_HEAD_PAGE_SPLITS)
            return fail("%d splits: this graph's split kernel takes at most %d", plan->total_splits,
                        Q38_HEAD_PAGE_SPLITS);
        const size_t need = (size_t)plan->total_splits * Q38_ATTN_HEADS * (Q38_ATTN_HEAD_DIM + 2) * sizeof(float);
        if (need > work_bytes) {
            if (work != nullptr) {
                Q38_HIP(hipStreamSynchronize(kv->ctx->stream));
                Q38_HIP(hipFree(work));
                work = nullptr;
                work_bytes = 0;
            }
            const size_t want = std::max(need, (size_t)1 << 20);
            Q38_HIP(hipMalloc(&work, want));
            work_bytes = want;
        }
        return 0;
    }

    /* Checks of positions for every call, with nothing changed; then the
     * workspace, the page reservations and each call's launch arguments. */
    int prepare(const int32_t *pos) {
        if (pos == nullptr) return fail("NULL positions");
        for (const Call &k : calls) {
            int slot = 0;
            if (validate_decode(kv, k.c.layer, n_seq, seq_ids, pos, k.appends, &slot)) return -1;
        }
        decode_plan plan;
        if (ensure_work(pos, &plan)) return -1;
        bool any_append = false;
        for (const Call &k : calls) any_append |= k.appends;
        if (any_append)
            for (int b = 0; b < n_seq; ++b)
                if (kv->reserve(seq_ids[b], pos[b] + 1)) return -1;
        for (const Call &k : calls)
            if (k.appends)
                for (int b = 0; b < n_seq; ++b) kv->images_from(seq_ids[b], k.slot, pos[b]);
        for (Call &k : calls)
            if (build(k, pos, plan)) return -1;
        memcpy(positions, pos, sizeof(int32_t) * n_seq);
        return 0;
    }

    int build(Call &k, const int32_t *pos, const decode_plan &plan) {
        return build_decode(kv, k.slot, n_seq, seq_ids, pos, k.c.d_q, k.c.d_k_new, k.c.d_v_new,
                            k.has_pre ? nullptr : k.c.d_gate, k.c.d_out, plan, work, k.has_pre ? &k.pre : nullptr,
                            arg_pages, &k.L);
    }

    void node_params(Call &k, bool merge, hipKernelNodeParams *p, void **arg) {
        *p = hipKernelNodeParams{};
        if (!merge) {
            *arg = &k.L.a;
            p->func = reinterpret_cast<void *>(k.L.f);
            p->gridDim = dim3(k.L.grid_x, Q38_ATTN_KV_HEADS, 1);
            p->blockDim = dim3(kv->ctx->decode_block, 1, 1);
        } else {
            *arg = &k.L.m;
            p->func = reinterpret_cast<void *>(kv->ctx->f_decode_merge);
            p->gridDim = dim3(n_seq, Q38_ATTN_HEADS, 4);
            p->blockDim = dim3(256, 1, 1);
        }
        p->kernelParams = arg;
        p->sharedMemBytes = 0;
        p->extra = nullptr;
    }

    int open_for_steps() const {
        if (exec != nullptr) return fail("the graph is already instantiated");
        if (steps >= 4096) return fail("a token graph holds at most 4096 steps");
        return 0;
    }

    int add_kernel(hipGraphNode_t *node, const hipKernelNodeParams &p) {
        Q38_HIP(hipGraphAddKernelNode(node, graph, last ? &last : nullptr, last ? 1 : 0, &p));
        last = *node;
        ++steps;
        return 0;
    }
};

int q38_decode_graph_begin(q38_kv *kv, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                           q38_decode_graph **out) {
    if (out == nullptr) return fail("NULL out");
    *out = nullptr;
    if (kv == nullptr) return fail("kv is NULL");
    if (n_seq < 1 || n_seq > Q38_MAX_BATCH) return fail("n_seq %d outside 1..%d", n_seq, Q38_MAX_BATCH);
    if (seq_ids == nullptr || positions == nullptr) return fail("NULL seq_ids/positions");
    for (int b = 0; b < n_seq; ++b) {
        if (kv->check_seq(seq_ids[b])) return -1;
        for (int c = 0; c < b; ++c)
            if (seq_ids[c] == seq_ids[b]) return fail("sequence %d appears twice", seq_ids[b]);
    }
    std::unique_ptr<q38_decode_graph> g(new q38_decode_graph());
    g->kv = kv;
    g->n_seq = n_seq;
    memcpy(g->seq_ids, seq_ids, sizeof(int32_t) * n_seq);
    memcpy(g->positions, positions, sizeof(int32_t) * n_seq);
    g->arg_pages = n_seq == 1 && kv->ctx->split_tokens == 0 ? 1 : 0;
    Q38_HIP(hipGraphCreate(&g->graph, 0));
    *out = g.release();
    return 0;
}

int q38_decode_graph_add_decode(q38_decode_graph *g, const q38_decode_call *call) {
    if (g == nullptr || call == nullptr) return fail("NULL argument");
    if (g->open_for_steps()) return -1;
    q38_decode_graph::Call k;
    k.c = *call;
    q38_kv *kv = g->kv;
    if (kv->slot_of(k.c.layer, &k.slot)) return -1;
    if (k.c.d_q == nullptr || k.c.d_out == nullptr) return fail("NULL q/out");
    if ((k.c.d_q_norm == nullptr) != (k.c.d_k_norm == nullptr)) return fail("d_q_norm and d_k_norm go together");
    k.has_pre = k.c.d_q_norm != nullptr;
    if (k.has_pre && (k.c.d_k_new == nullptr || k.c.d_v_new == nullptr))
        return fail("the full_core form needs its key and value");
    if ((k.c.d_k_new == nullptr) != (k.c.d_v_new == nullptr)) return fail("d_k_new and d_v_new go together");
    k.appends = k.c.d_k_new != nullptr;
    k.pre = decode_pre{k.c.d_q_norm, k.c.d_k_norm};
    int slot = 0;
    if (validate_decode(kv, k.c.layer, g->n_seq, g->seq_ids, g->positions, k.appends, &slot)) return -1;
    decode_plan plan;
    if (g->ensure_work(g->positions, &plan)) return -1;
    if (k.appends)
        for (int b = 0; b < g->n_seq; ++b) {
            if (kv->reserve(g->seq_ids[b], g->positions[b] + 1)) return -1;
            kv->images_from(g->seq_ids[b], k.slot, g->positions[b]);
        }
    if (g->build(k, g->positions, plan)) return -1;
    /* the workspace may have moved: every call's arguments name the current one */
    for (q38_decode_graph::Call &o : g->calls) {
        if (g->build(o, g->positions, plan)) return -1;
        hipKernelNodeParams p;
        void *arg = nullptr;
        g->node_params(o, false, &p, &arg);
        Q38_HIP(hipGraphKernelNodeSetParams(o.split_node, &p));
        g->node_params(o, true, &p, &arg);
        Q38_HIP(hipGraphKernelNodeSetParams(o.merge_node, &p));
    }
    g->calls.push_back(k);
    q38_decode_graph::Call &kk = g->calls.back();
    hipKernelNodeParams p;
    void *arg = nullptr;
    g->node_params(kk, false, &p, &arg);
    if (g->add_kernel(&kk.split_node, p)) return -1;
    g->node_params(kk, true, &p, &arg);
    return g->add_kernel(&kk.merge_node, p);
}

int q38_decode_graph_add_linear_core(q38_decode_graph *g, int n_seq, const q38_linear_weights *w,
                                     float *d_conv_state, float *d_delta_state, const float *d_qkv,
                                     const float *d_z, const float *d_beta, const float *d_alpha, float *d_out) {
    if (g == nullptr || w == nullptr) return fail("NULL argument");
    if (g->open_for_steps()) return -1;
    if (n_seq < 1 || n_seq > 65535) return fail("n_seq %d outside 1..65535", n_seq);
    if (!w->d_conv_w || !w->d_dt || !w->d_a || !w->d_norm || !d_conv_state || !d_delta_state || !d_qkv || !d_z ||
        !d_beta || !d_alpha || !d_out)
        return fail("NULL argument");
    q38_ctx *ctx = g->kv->ctx;
    /* the arrival counters exist before any replay (no allocation or fill
     * inside the graph; the kernel leaves them zero) */
    if (ctx->ensure_arrivals(n_seq)) return -1;
    q38_gdn_decode_args a;
    memset(&a, 0, sizeof(a));
    a.qkv_raw = d_qkv;
    a.conv_w = w->d_conv_w;
    a.conv_state = d_conv_state;
    a.state = d_delta_state;
    a.z = d_z;
    a.beta_raw = d_beta;
    a.alpha_raw = d_alpha;
    a.dt = w->d_dt;
    a.a = w->d_a;
    a.norm_w = w->d_norm;
    a.out = d_out;
    a.arrivals = ctx->arrivals;
    void *arg = &a;
    hipKernelNodeParams p{};
    p.func = reinterpret_cast<void *>(ctx->f_gdn_decode);
    p.gridDim = dim3(Q38_LIN_V_HEADS, n_seq, 1);
    p.blockDim = dim3(ctx->gdn_decode_block, 1, 1);
    p.kernelParams = &arg;
    p.sharedMemBytes = 0;
    p.extra = nullptr;
    hipGraphNode_t node = nullptr;
    return g->add_kernel(&node, p);
}

int q38_decode_graph_add_graph(q38_decode_graph *g, void *hip_graph) {
    if (g == nullptr || hip_graph == nullptr) return fail("NULL argument");
    if (g->open_for_steps()) return -1;
    hipGraphNode_t node = nullptr;
    Q38_HIP(hipGraphAddChildGraphNode(&node, g->graph, g->last ? &g->last : nullptr, g->last ? 1 : 0,
                                      static_cast<hipGraph_t>(hip_graph)));
    g->last = node;
    ++g->steps;
    return 0;
}

int q38_decode_graph_end(q38_decode_graph *g) {
    if (g == nullptr) return fail("graph is NULL");
    if (g->exec != nullptr) return fail("the graph is already instantiated");
    if (g->steps == 0) return fail("the graph has no steps");
    Q38_HIP(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0));
    return 0;
}

int q38_decode_graph_create(q38_kv *kv, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                            int n_calls, const q38_decode_call *calls, q38_decode_graph **out) {
    if (out == nullptr) return fail("NULL out");
    *out = nullptr;
    if (n_calls < 1 || calls == nullptr) return fail("no decode calls");
    q38_decode_graph *g = nullptr;
    if (q38_decode_graph_begin(kv, n_seq, seq_ids, positions, &g)) return -1;
    for (int i = 0; i < n_calls; ++i) {
        if (q38_decode_graph_add_decode(g, &calls[i])) {
            const std::string why = g_last_error;
            delete g;
            return fail("call %d: %s", i, why.c_str());
        }
    }
    if (q38_decode_graph_end(g)) {
        delete g;
        return -1;
    }
    *out = g;
    return 0;
}

int q38_decode_graph_set_positions(q38_decode_graph *g, const int32_t *positions) {
    if (g == nullptr) return fail("graph is NULL");
    if (g->exec == nullptr) return fail("the graph is not instantiated (q38_decode_graph_end)");
    /* a replay still running reads the arguments being replaced */
    Q38_HIP(hipStreamSynchronize(g->kv->ctx->stream));
    if (g->prepare(positions)) return -1;
    for (q38_decode_graph::Call &k : g->calls) {
        hipKernelNodeParams p;
        void *arg = nullptr;
        g->node_params(k, false, &p, &arg);
        Q38_HIP(hipGraphExecKernelNodeSetParams(g->exec, k.split_node, &p));
        g->node_params(k, true, &p, &arg);
        Q38_HIP(hipGraphExecKernelNodeSetParams(g->exec, k.merge_node, &p));
    }
    return 0;
}

int q38_decode_graph_launch(q38_decode_graph *g) {
    if (g == nullptr) return fail("graph is NULL");
    if (g->exec == nullptr) return fail("the graph is not instantiated (q38_decode_graph_end)");
    Q38_HIP(hipGraphLaunch(g->exec, g->kv->ctx->stream));
    return 0;
}

int q38_decode_graph_destroy(q38_decode_graph *g) {
    if (g == nullptr) return 0;
    Q38_HIP(hipStreamSynchronize(g->kv->ctx->stream));
    delete g;
    return 0;
}

namespace {

/* Spread the 3 * n_qblocks (head pair, query block) jobs of one kv head over
 * Q38_PREFILL_BINS bins of at most Q38_PREFILL_JOBS_MAX jobs, a job weighing
 * the key blocks its workgroup streams: longest first onto the lightest bin,
 * then moves and swaps out of the heaviest bin while they lower it.  When a
 * job is longer than 1.35x the average bin's blocks (the last query blocks of a
 * short prompt, or every block of a prompt after a long prefix), jobs are
 * first cut into pieces of about a third of that share, of equal key ranges, each
 * starting on a block every row of the job sees whole; the pieces write partials (one slot each) that
 * q38_prefill_merge combines, and `splits` lists them.  Writes the table
 * (code 0xFFFF past a bin's last job) and returns the jobs per bin. */
int place_prefill_jobs(int base_pos, int n_tokens, int n_qblocks, q38_prefill_job *table,
                       q38_prefill_split *splits, int *n_split, int *n_slots) {
    constexpr int kBins = Q38_PREFILL_BINS, kMax = Q38_PREFILL_JOBS_MAX;
    constexpr int kMinPiece = 8; /* key blocks: a piece's own cost (its Q, its partials) is ~1 */
    struct Job {
        int weight;
        q38_prefill_job j;
    };
    long total = 0, longest = 0;
    for (int qb = 0; qb < n_qblocks; ++qb) {
        const int q_last = std::min((qb + 1) * Q38_PREFILL_QUERIES, n_tokens) - 1;
        const long n_kb = (base_pos + q_last) / Q38_PREFILL_KEYS + 1;
        total += Q38_PREFILL_HEAD_PAIRS * n_kb;
        longest = std::max(longest, n_kb);
    }
    const long avg = (total + kBins - 1) / kBins;
    /* pieces of a third of a bin's share, so that the bins can be evened out;
     * only when some job is longer than 1.35 shares: below that the pieces'
     * own costs outweigh the balance (2048 tokens, longest job 1.28 shares:
     * 0.224 ms cut against 0.198 ms whole; 1024 tokens after 9000, 48 jobs
     * of 1.39 shares for 64 bins, are cut) */
    long cap = longest * 20 > avg * 27 ? std::max<long>((avg + 2) / 3, kMinPiece) : longest;
    std::vector<Job> jobs;
    int slots = 0, ns = 0;
retry:
    jobs.clear();
    slots = ns = 0;
    for (int qb = 0; qb < n_qblocks; ++qb) {
        const int q_last = std::min((qb + 1) * Q38_PREFILL_QUERIES, n_tokens) - 1;
        const int n_kb = (base_pos + q_last) / Q38_PREFILL_KEYS + 1;
        /* the last block every row of the job sees whole: keys up to the
         * position of its first row */
        const int first_pos = base_pos + qb * Q38_PREFILL_QUERIES;
        const int seen = first_pos >= Q38_PREFILL_KEYS - 1 ? (first_pos - (Q38_PREFILL_KEYS - 1)) / Q38_PREFILL_KEYS
                                                           : -1;
        int np = n_kb > cap ? (int)((n_kb + cap - 1) / cap) : 1;
        while (np > 1 && (long)(np - 1) * n_kb / np > seen) --np; /* the last piece's start */
        for (int hp = 0; hp < Q38_PREFILL_HEAD_PAIRS; ++hp) {
            const uint16_t code = (uint16_t)(hp << 6 | qb);
            if (np == 1) {
                jobs.push_back({n_kb + 1, {code, 0xFFFF, 0, n_kb}});
                continue;
            }
            splits[ns++] = {code, (uint16_t)slots, (uint16_t)np, 0};
            for (int i = 0; i < np; ++i) {
                const int kb0 = (int)((long)i * n_kb / np), kb1 = (int)((long)(i + 1) * n_kb / np);
                jobs.push_back({kb1 - kb0 + 1, {code, (uint16_t)(slots + i), kb0, kb1}});
            }
            slots += np;
        }
    }
    if ((int)jobs.size() > kBins * kMax) {
        cap *= 2; /* more pieces than the table holds */
        goto retry;
    }
    *n_split = ns;
    *n_slots = slots;
    std::stable_sort(jobs.begin(), jobs.end(), [](const Job &x, const Job &y) { return x.weight > y.weight; });
    std::vector<std::vector<Job>> bins(kBins);
    std::vector<long> load(kBins, 0);
    for (const Job &jb : jobs) {
        int best = -1;
        for (int b = 0; b < kBins; ++b)
            if ((int)bins[b].size() < kMax && (best < 0 || load[b] < load[best])) best = b;
        bins[best].push_back(jb);
        load[best] += jb.weight;
    }
    for (int it = 0; it < 4096; ++it) {
        const int hi = (int)(std::max_element(load.begin(), load.end()) - load.begin());
        long best_max = load[hi];
        int bb = -1, bx = -1, by = -1; /* by < 0: a move */
        for (int b = 0; b < kBins; ++b) {
            if (b == hi) continue;
            for (int x = 0; x < (int)bins[hi].size(); ++x) {
                const long wx = bins[hi][x].weight;
                if ((int)bins[b].size() < kMax) {
                    const long m = std::max(load[hi] - wx, load[b] + wx);
                    if (m < best_max) best_max = m, bb = b, bx = x, by = -1;
                }
                for (int y = 0; y < (int)bins[b].size(); ++y) {
                    const long wy = bins[b][y].weight;
                    const long m = std::max(load[hi] - wx + wy, load[b] - wy + wx);
                    if (m < best_max) best_max = m, bb = b, bx = x, by = y;
                }
            }
        }
        if (bb < 0) break;
        const Job jx = bins[hi][bx];
        if (by < 0) {
            bins[hi].erase(bins[hi].begin() + bx);
            bins[bb].push_back(jx);
            load[hi] -= jx.weight;
            load[bb] += jx.weight;
        } else {
            const Job jy = bins[bb][by];
            bins[hi][bx] = jy;
            bins[bb][by] = jx;
            load[hi] += jy.weight - jx.weight;
            load[bb] += jx.weight - jy.weight;
        }
    }
    int per = 1;
    for (const auto &b : bins) per = std::max(per, (int)b.size());
    for (int i = 0; i < kBins * kMax; ++i) table[i] = {0xFFFF, 0xFFFF, 0, 0};
    for (int b = 0; b < kBins; ++b)
        for (int i = 0; i < (int)bins[b].size(); ++i) table[b * per + i] = bins[b][i].j;
    return per;
}

}  // namespace

/* kernel arguments travel by value; keep them within the 4 KiB a launch
 * carries on every HIP runtime */
static_assert(sizeof(q38_prefill_args) <= 4096, "prefill arguments exceed 4 KiB");
static_assert(sizeof(q38_decode_args) <= 4096, "decode arguments exceed 4 KiB");
static_assert(sizeof(q38_prefill_merge_args) <= 4096, "prefill merge arguments exceed 4 KiB");

int q38_attn_prefill(q38_kv *kv, int layer, int seq, int base_pos, int n_tokens, const float *d_q,
                     const float *d_k, const float *d_v, const float *d_gate, float *d_out) {
    if (kv == nullptr) return fail("kv is NULL");
    if (n_tokens < 0 || base_pos < 0) return fail("negative count or position");
    if (n_tokens == 0) return 0;
    if (!d_q || !d_k || !d_v || !d_out) return fail("NULL argument");
    if (kv->check_seq(seq)) return -1;
    int slot = 0;
    if (kv->slot_of(layer, &slot)) return -1;
    const long end = (long)base_pos + n_tokens;
    if (end > (long)kv->pt_stride * Q38_PAGE_TOKENS)
        return fail("positions %d..%ld are past the context limit %d", base_pos, end - 1,
                    kv->pt_stride * Q38_PAGE_TOKENS);
    const long need = (end + Q38_PAGE_TOKENS - 1) / Q38_PAGE_TOKENS - kv->seq_pages[seq];
    if (need > (long)kv->free_pages.size())
        return fail("KV pool exhausted: need %ld pages, %zu free", need, kv->free_pages.size());
    q38_ctx *ctx = kv->ctx;
    constexpr int kQueryBlock = Q38_PREFILL_QUERIES; /* query tokens per workgroup of the kernel */
    q38_prefill_args a;
    memset(&a, 0, sizeof(a));
    a.kpool = kv->kslot(slot);
    a.vpool = kv->vslot(slot);
    a.page_table = kv->d_page_table + (size_t)seq * kv->pt_stride;
    a.q = d_q;
    a.gate = d_gate;
    a.out = d_out;
    a.base_pos = base_pos;
    a.n_tokens = n_tokens;
    a.n_qblocks = (n_tokens + kQueryBlock - 1) / kQueryBlock;
    a.n_kblocks = (int)((end - 1) / Q38_PREFILL_KEYS + 1);
    size_t n_wg = (size_t)a.n_qblocks * Q38_ATTN_KV_HEADS * Q38_PREFILL_HEAD_PAIRS;
    if (n_wg > 0x7FFFFFFFull) return fail("prompt too long");
    q38_prefill_merge_args mg;
    memset(&mg, 0, sizeof(mg));
    if (a.n_qblocks <= 64) {
        /* few jobs per CU: placed here so that every bin (one workgroup per CU)
         * gets the same number of key blocks, which the hardware's
         * longest-first order cannot do with 3 jobs per CU */
        a.jobs_per_wg = place_prefill_jobs(base_pos, n_tokens, a.n_qblocks, a.jobs, mg.split, &mg.n_split, &a.n_slots);
        n_wg = (size_t)Q38_ATTN_KV_HEADS * Q38_PREFILL_BINS;
    }
    /* the block images: the (sequence, slot)'s own buffer, kept between
     * calls and grown to hold n_kblocks blocks (its valid images copied
     * over); with the cache switched off, or no memory for it, the
     * context's workspace, converted whole */
    q38_kv::Images *im = kv->image_cache ? &kv->img(seq, slot) : nullptr;
    if (im != nullptr && im->cap < a.n_kblocks) {
        const long max_blocks = ((long)kv->pt_stride * Q38_PAGE_TOKENS + Q38_PREFILL_KEYS - 1) / Q38_PREFILL_KEYS;
        const int cap = (int)std::min<long>(max_blocks, std::max<long>(a.n_kblocks, 2L * im->cap));
        const size_t block_bytes = Q38_PREFILL_IMAGE_BYTES;
        void *buf = nullptr;
        if (hipMalloc(&buf, (size_t)Q38_ATTN_KV_HEADS * cap * block_bytes) != hipSuccess) {
            (void)hipGetLastError();
            im = nullptr;
        } else {
            for (int j = 0; j < Q38_ATTN_KV_HEADS && im->valid > 0; ++j)
                Q38_HIP(hipMemcpyAsync(static_cast<char *>(buf) + (size_t)j * cap * block_bytes,
                                       static_cast<char *>(im->buf) + (size_t)j * im->cap * block_bytes,
                                       (size_t)im->valid * block_bytes, hipMemcpyDeviceToDevice, ctx->stream));
            if (im->buf != nullptr) {
                Q38_HIP(hipStreamSynchronize(ctx->stream));
                Q38_HIP(hipFree(im->buf));
            }
            im->buf = buf;
            im->cap = cap;
        }
    }
    /* the workspace for the pieces' partials (and the images without a
     * cache), before anything is changed */
    const size_t img_bytes =
        im != nullptr ? 0 : ((size_t)Q38_ATTN_KV_HEADS * a.n_kblocks * Q38_PREFILL_IMAGE_BYTES + 255) / 256 * 256;
    const size_t part_rows = (size_t)Q38_ATTN_KV_HEADS * a.n_slots * Q38_PREFILL_QUERIES * 2;
    if (ctx->ensure_work(img_bytes + part_rows * (Q38_ATTN_HEAD_DIM + 2) * sizeof(float))) return -1;
    a.images = im != nullptr ? im->buf : ctx->work;
    a.img_stride = im != nullptr ? im->cap : a.n_kblocks;
    a.part_o = reinterpret_cast<float *>(static_cast<char *>(ctx->work) + img_bytes);
    a.part_ml = a.part_o + part_rows * Q38_ATTN_HEAD_DIM;
    /* append the prompt's rows (reserves pages; the blocks from base_pos on
     * are no longer valid images) */
    if (q38_kv_write(kv, layer, seq, base_pos, n_tokens, d_k, d_v)) return -1;
    /* the K/V blocks without a valid image split once into bf16 hi/lo
     * images, then the attention kernel */
    a.kb0 = im != nullptr ? std::min(im->valid, a.n_kblocks) : 0;
    if (a.kb0 < a.n_kblocks &&
        ctx->launch(ctx->f_kv_split, a.n_kblocks - a.kb0, Q38_ATTN_KV_HEADS, 1, 256, &a))
        return -1;
    /* the blocks every key of which is now in the cache stay valid */
    if (im != nullptr) im->valid = (int)(end / Q38_PREFILL_KEYS);
    if (ctx->launch(ctx->f_prefill, (unsigned)n_wg, 1, 1, 256, &a)) return -1;
    if (mg.n_split == 0) return 0;
    mg.part_o = a.part_o;
    mg.part_ml = a.part_ml;
    mg.gate = d_gate;
    mg.out = d_out;
    mg.n_tokens = n_tokens;
    mg.n_slots = a.n_slots;
    return ctx->launch(ctx->f_prefill_merge, (unsigned)mg.n_split, Q38_ATTN_KV_HEADS, 2 * Q38_PREFILL_QUERIES / 4,
                       256, &mg);
}

/* ---------------------------------------------------------------- DeltaNet */

/* Chunked recurrence over n_tokens > 1 tokens of n_seq states (the token
 * loop of ops.rs:1088-1099 in 64-token chunks); work holds
 * chunk_work_floats(n_seq, n_tokens) floats. */
static size_t chunk_work_floats(int n_seq, int n_tokens) {
    const size_t n_chunks =
        std::min<size_t>(((size_t)n_tokens + Q38_GDN_CHUNK - 1) / Q38_GDN_CHUNK, Q38_GDN_STAGE_CHUNKS);
    return (size_t)n_seq * Q38_LIN_V_HEADS * n_chunks * (Q38_GDN_RECORD_BYTES / sizeof(float));
}

static int gdn_chunked(q38_ctx *ctx, int n_seq, int n_tokens, float *d_state, int64_t state_stride,
                       const float *d_q, const float *d_k, const float *d_v, const float *d_beta,
                       const float *d_g, float *d_out, int q_stride, int v_stride, float *work) {
    const int n_chunks = (n_tokens + Q38_GDN_CHUNK - 1) / Q38_GDN_CHUNK;
    if (n_chunks > 65535) return fail("%d tokens exceed the chunked prefill's 65535 chunks", n_tokens);
    q38_gdn_chunk_args a;
    memset(&a, 0, sizeof(a));
    a.state = d_state;
    a.q = d_q;
    a.k = d_k;
    a.v = d_v;
    a.beta = d_beta;
    a.g = d_g;
    a.out = d_out;
    a.work = work;
    a.state_stride = state_stride;
    a.q_stride = q_stride;
    a.v_stride = v_stride;
    a.n_tokens = n_tokens;
    /* stages of Q38_GDN_STAGE_CHUNKS chunks: the scan reads each stage's
     * records right after the prep wrote them */
    for (int c0 = 0; c0 < n_chunks; c0 += Q38_GDN_STAGE_CHUNKS) {
        a.chunk0 = c0;
        a.n_chunks = std::min(Q38_GDN_STAGE_CHUNKS, n_chunks - c0);
        if (ctx->launch(ctx->f_chunk_prep, Q38_LIN_QK_HEADS, a.n_chunks, n_seq, 512, &a)) return -1;
        if (ctx->launch(ctx->f_chunk_scan, Q38_LIN_V_HEADS * 4, n_seq, 1, 64 * Q38_GDN_SCAN_WAVES, &a)) return -1;
    }
    return 0;
}

int q38_gdn_step(q38_ctx *ctx, int n_seq, float *d_state, int64_t state_stride, const float *d_q,
                 const float *d_k, const float *d_v, const float *d_beta, const float *d_g,
                 float *d_out) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (n_seq < 0) return fail("negative n_seq");
    if (n_seq == 0) return 0;
    if (!d_state || !d_q || !d_k || !d_v || !d_beta || !d_g || !d_out) return fail("NULL argument");
    if (n_seq > 65535) return fail("n_seq %d above 65535", n_seq);
    if (n_seq > 1 && state_stride < (int64_t)Q38_LIN_STATE_FLOATS)
        return fail("state_stride %lld overlaps states", (long long)state_stride);
    /* one token: the row-parallel kernel (8 workgroups per value head) */
    q38_gdn_args a;
    memset(&a, 0, sizeof(a));
    a.state = d_state;
    a.q = d_q;
    a.k = d_k;
    a.v = d_v;
    a.beta = d_beta;
    a.g = d_g;
    a.out = d_out;
    a.state_stride = state_stride;
    a.q_stride = Q38_LIN_QK_DIM;
    a.v_stride = Q38_LIN_V_DIM;
    a.n_seq = n_seq;
    return ctx->launch(ctx->f_gdn_step_rows, Q38_LIN_V_HEADS * (Q38_LIN_HEAD_DIM / 16), n_seq, 1, 256, &a);
}

int q38_gdn_prefill(q38_ctx *ctx, float *d_state, int n_tokens, const float *d_q, const float *d_k,
                    const float *d_v, const float *d_beta, const float *d_g, float *d_out) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (n_tokens < 0) return fail("negative n_tokens");
    if (n_tokens == 0) return 0;
    if (!d_state || !d_q || !d_k || !d_v || !d_beta || !d_g || !d_out) return fail("NULL argument");
    if (n_tokens == 1)
        return q38_gdn_step(ctx, 1, d_state, Q38_LIN_STATE_FLOATS, d_q, d_k, d_v, d_beta, d_g, d_out);
    if (ctx->ensure_work(chunk_work_floats(1, n_tokens) * sizeof(float))) return -1;
    return gdn_chunked(ctx, 1, n_tokens, d_state, Q38_LIN_STATE_FLOATS, d_q, d_k, d_v, d_beta, d_g, d_out,
                       Q38_LIN_QK_DIM, Q38_LIN_V_DIM, static_cast<float *>(ctx->work));
}

int q38_linear_core(q38_ctx *ctx, int n_seq, int n_tokens, const q38_linear_weights *w,
                    float *d_conv_state, float *d_delta_state, const float *d_qkv,
                    const float *d_z, const float *d_beta, const float *d_alpha, float *d_out) {
    if (ctx == nullptr || w == nullptr) return fail("NULL argument");
    if (n_seq < 0 || n_tokens < 0) return fail("negative count");
    if (n_seq == 0 || n_tokens == 0) return 0;
    if (!w->d_conv_w || !w->d_dt || !w->d_a || !w->d_norm || !d_conv_state || !d_delta_state ||
        !d_qkv || !d_z || !d_beta || !d_alpha || !d_out)
        return fail("NULL argument");
    if (n_seq > 65535) return fail("n_seq %d above 65535", n_seq);
    if (n_tokens == 1) {
        /* decode: conv, gates, recurrence and gated norm in one launch */
        if (ctx->ensure_arrivals(n_seq)) return -1;
        q38_gdn_decode_args a;
        memset(&a, 0, sizeof(a));
        a.qkv_raw = d_qkv;
        a.conv_w = w->d_conv_w;
        a.conv_state = d_conv_state;
        a.state = d_delta_state;
        a.z = d_z;
        a.beta_raw = d_beta;
        a.alpha_raw = d_alpha;
        a.dt = w->d_dt;
        a.a = w->d_a;
        a.norm_w = w->d_norm;
        a.out = d_out;
        a.arrivals = ctx->arrivals;
        return ctx->launch(ctx->f_gdn_decode, Q38_LIN_V_HEADS, n_seq, 1, ctx->gdn_decode_block, &a);
    }
    if (((uintptr_t)d_conv_state | (uintptr_t)d_qkv | (uintptr_t)d_z | (uintptr_t)d_out) % 16 != 0)
        return fail("d_conv_state, d_qkv, d_z and d_out must be 16-byte aligned");
    /* the conv runs of q38_gdn_pre read conv_state_in while the last run
     * writes the shifted state: a separate buffer when there are several */
    const int pre_runs = (n_tokens + Q38_GDN_PRE_TOKENS - 1) / Q38_GDN_PRE_TOKENS;
    const size_t toks = (size_t)n_seq * n_tokens;
    /* workspace: qkv after conv/SiLU/L2 | beta | g | conv state out |
     * recurrence output before the norm | chunk products */
    const size_t conv_floats = (size_t)n_seq * Q38_LIN_QKV_DIM * 3;
    const size_t base_floats = toks * (Q38_LIN_QKV_DIM + 2 * Q38_LIN_V_HEADS) + (pre_runs > 1 ? conv_floats : 0);
    const size_t o_floats = toks * Q38_LIN_V_DIM;
    const size_t chunk_floats = chunk_work_floats(n_seq, n_tokens);
    if (toks > 0x7FFFFFFFull) return fail("too many tokens");
    if (ctx->ensure_work((base_floats + o_floats + chunk_floats) * sizeof(float))) return -1;
    float *x = static_cast<float *>(ctx->work);
    float *beta = x + toks * Q38_LIN_QKV_DIM;
    float *g = beta + toks * Q38_LIN_V_HEADS;
    float *conv_out = pre_runs > 1 ? g + toks * Q38_LIN_V_HEADS : d_conv_state;
    float *o_raw = x + base_floats;
    float *chunk_work = o_raw + o_floats;

    q38_gdn_pre_args p;
    memset(&p, 0, sizeof(p));
    p.qkv_raw = d_qkv;
    p.conv_w = w->d_conv_w;
    p.conv_state_in = d_conv_state;
    p.conv_state_out = conv_out;
    p.qkv_out = x;
    p.beta_raw = d_beta;
    p.alpha_raw = d_alpha;
    p.dt = w->d_dt;
    p.a = w->d_a;
    p.beta_out = beta;
    p.g_out = g;
    p.n_tokens = n_tokens;
    p.n_seq = n_seq;
    if (ctx->launch(ctx->f_gdn_pre, Q38_LIN_QKV_DIM / 1024 + 1, pre_runs, n_seq, 256, &p)) return -1;
    if (pre_runs > 1)
        Q38_HIP(hipMemcpyAsync(d_conv_state, conv_out, conv_floats * sizeof(float),
                               hipMemcpyDeviceToDevice, ctx->stream));
    /* prompt: chunked recurrence, then the gated RMSNorm */
    if (gdn_chunked(ctx, n_seq, n_tokens, d_delta_state, Q38_LIN_STATE_FLOATS, x, x + Q38_LIN_QK_DIM,
                    x + 2 * Q38_LIN_QK_DIM, beta, g, o_raw, Q38_LIN_QKV_DIM, Q38_LIN_QKV_DIM, chunk_work))
        return -1;
    q38_gdn_post_args pa;
    memset(&pa, 0, sizeof(pa));
    pa.o = o_raw;
    pa.z = d_z;
    pa.norm_w = w->d_norm;
    pa.out = d_out;
    /* 16 (token, value head) rows per workgroup; toks * 48 rows */
    return ctx->launch(ctx->f_gdn_post, (unsigned)(toks * (Q38_LIN_V_HEADS / 16)), 1, 1, 256, &pa);
}

/* ------------------------------------------------------------ projections */

int q38_q8k_bytes(int n_tokens, int width, size_t *bytes) {
    if (bytes == nullptr) return fail("bytes is NULL");
    if (n_tokens < 0 || width <= 0 || width % Q38_Q8K_BLOCK != 0)
        return fail("width %d is not a positive multiple of %d (or n_tokens %d < 0)", width, Q38_Q8K_BLOCK, n_tokens);
    *bytes = Q38_Q8K_BYTES(n_tokens, width);
    return 0;
}

int q38_quantize_q8_k(q38_ctx *ctx, int n_tokens, int width, const float *d_x, void *d_q8k) {
    if (ctx == nullptr) return fail("ctx is NULL");
    if (n_tokens < 0) return fail("negative n_tokens");
    if (width <= 0 || width % Q38_Q8K_BLOCK != 0)
        return fail("input length %d is not a multiple of %d", width, Q38_Q8K_BLOCK); /* quant.rs:100-104 */
    if (n_tokens == 0) return 0;
    if (d_x == nullptr || d_q8k == nullptr) return fail("NULL argument");
    if (((uintptr_t)d_x | (uintptr_t)d_q8k) % 16 != 0) return fail("d_x and d_q8k must be 16-byte aligned");
    if (width / Q38_Q8K_BLOCK > 65535 || n_tokens > 65535) return fail("too many blocks or tokens");
    q38_quantize_args a;
    memset(&a, 0, sizeof(a));
    a.x = d_x;
    a.q8k = d_q8k;
    a.width = width;
    a.n_tokens = n_tokens;
    return ctx->launch(ctx->f_quantize_q8k, (width / Q38_Q8K_BLOCK + 15) / 16, n_tokens, 1, 256, &a);
}

/* The projections of one input; d_x non-NULL: the f32 input, quantised into
 * d_q8k as q38_quantize_q8_k does (by the GEMV itself when every matrix
 * stays on it, else by a q38_quantize_q8k launch first). */
static int gemv_q8k_multi(q38_ctx *ctx, int ggml_type, int n_mats, const int *rows, int width,
                          const void *const *d_weights, const float *d_x, const void *d_q8k, int n_tokens,
                          float *const *d_out) {
    if (ctx == nullptr) return fail("ctx is NULL");
    int ti_occ = -1; /* kGemv index */
    for (int i = 0; i < kGemvTypes; ++i)
        if (kGemv[i].ggml_type == ggml_type) ti_occ = i;
    if (ti_occ < 0)
        return fail("unsupported quant type %d (Q2_K 10, Q3_K 11, Q4_K 12, Q5_K 13, Q6_K 14, IQ2_XXS 16, IQ2_XS 17, "
                    "IQ3_XXS 18, IQ1_S 19, IQ4_NL 20, IQ3_S 21, IQ2_S 22, IQ4_XS 23, IQ1_M 29; "
                    "F32, F16, BF16 and Q8_0 weights take q38_gemv_f32)",
                    ggml_type);
    const hipFunction_t f = ctx->f_gemv_q8k[ti_occ];
    /* f32 terms per block in the row sums (IQ4_NL adds one per 32-weight
     * group) and the LDS copy of an IQ format's lattice grid */
    const int nt = kGemv[ti_occ].terms;
    const int grid_lds = kGemv[ti_occ].grid_bytes;
    /* the int8 matrix-unit form */
    const bool has_gemm = ctx->f_gemm[ti_occ] != nullptr;
    if (n_mats < 1 || n_mats > Q38_GEMV_MAX_MATS) return fail("n_mats %d outside 1..%d", n_mats, Q38_GEMV_MAX_MATS);
    if (rows == nullptr || d_weights == nullptr || d_out == nullptr) return fail("NULL argument");
    if (n_tokens < 0) return fail("negative n_tokens");
    for (int i = 0; i < n_mats; ++i)
        if (rows[i] < 0) return fail("negative rows (matrix %d)", i);
    if (width <= 0 || width % Q38_Q8K_BLOCK != 0)
        return fail("width %d is not a multiple of %d", width, Q38_Q8K_BLOCK);
    if (width / Q38_Q8K_BLOCK > Q38_GEMV_MAX_BLOCKS)
        return fail("width %d above %d", width, Q38_GEMV_MAX_BLOCKS * Q38_Q8K_BLOCK);
    if (n_tokens == 0) return 0;
    int n_nonempty = 0;
    for (int i = 0; i < n_mats; ++i) {
        if (rows[i] == 0) continue; /* nothing to compute for an empty matrix */
        if (d_weights[i] == nullptr || d_out[i] == nullptr) return fail("NULL weights or output (matrix %d)", i);
        if ((uintptr_t)d_weights[i] % 16 != 0) return fail("d_weights[%d] must be 16-byte aligned", i);
        ++n_nonempty;
    }
    if (d_q8k == nullptr || (uintptr_t)d_q8k % 16 != 0) return fail("d_q8k is NULL or not 16-byte aligned");
    if (d_x != nullptr && (uintptr_t)d_x % 16 != 0) return fail("d_x must be 16-byte aligned");
    if (n_nonempty == 0) return d_x != nullptr ? q38_quantize_q8_k(ctx, n_tokens, width, d_x, const_cast<void *>(d_q8k)) : 0;
    if (((long)n_tokens + Q38_GEMM_KS_TOKENS - 1) / Q38_GEMM_KS_TOKENS > 65535) return fail("too many tokens");

    /* Many tokens: the int8 matrix-unit forms.  A matrix whose split-block
     * grid (32 rows x 32 tokens per workgroup) would exceed kGemmKsMaxPerCu
     * workgroups per CU takes the 128 x 64 tiles, a launch of its own; from
     * Q38_GEMM_MIN_TOKENS tokens on, the others share one split-block launch
     * where their grids add up to at least kGemmKsMinTiles workgroups (on
     * fewer, e.g. 1024 x 5120 alone below 64 tokens, the GEMV is faster)
     * (measured on the FFN, q|gate and k matrices, 4-512 tokens: at 8 tokens
     * as fast as the GEMV for one matrix, at 9-15 tokens 1.2-1.6x faster,
     * where the GEMV takes two passes; a layer's projections at 8-15 tokens
     * 1.4-2x faster).  IQ4_NL, which has only the 128 x 64 form, takes it
     * from Q38_GEMM_IQ4NL_MIN_TOKENS tokens (half as many for 8192+ rows). */
    const int ti = ti_occ;
    const long tok_tiles = ((long)n_tokens + Q38_GEMM_TOKENS - 1) / Q38_GEMM_TOKENS;
    const long ks_tok_tiles = ((long)n_tokens + Q38_GEMM_KS_TOKENS - 1) / Q38_GEMM_KS_TOKENS;
    bool on_gemv[Q38_GEMV_MAX_MATS] = {}, on_big[Q38_GEMV_MAX_MATS] = {};
    bool any_gemm = false, ks_call = false;
    long ks_total = 0; /* workgroups of the shared split-block launch */
    for (int i = 0; i < n_mats; ++i) {
        if (rows[i] == 0) continue;
        if (ctx->f_gemm_ks[ti] != nullptr) {
            const long ks_tiles = ((long)rows[i] + Q38_GEMM_KS_ROWS - 1) / Q38_GEMM_KS_ROWS * ks_tok_tiles;
            on_big[i] = n_tokens >= Q38_GEMM_MIN_TOKENS && ks_tiles > kGemmKsMaxPerCu * (long)ctx->cu_count;
            if (!on_big[i]) ks_total += ks_tiles;
        } else if (has_gemm) {
            on_big[i] = n_tokens >= Q38_GEMM_IQ4NL_MIN_TOKENS ||
                        (2 * n_tokens >= Q38_GEMM_IQ4NL_MIN_TOKENS && rows[i] >= 64L * Q38_GEMM_ROWS);
        }
        any_gemm = any_gemm || on_big[i];
    }
    if (ctx->f_gemm_ks[ti] != nullptr)
        ks_call = n_tokens >= Q38_GEMM_MIN_TOKENS && ks_total >= kGemmKsMinTiles;
    any_gemm = any_gemm || ks_call;
    for (int i = 0; i < n_mats; ++i) on_gemv[i] = rows[i] > 0 && !on_big[i] && !ks_call;
    /* the matrix-unit forms read the quantised input from memory; the GEMV
     * quantises it itself, in every workgroup, up to kQuantizeFoldMaxTokens
     * tokens (beyond, that repeated work costs more than the launch) */
    if (d_x != nullptr && (any_gemm || n_tokens > kQuantizeFoldMaxTokens)) {
        if (q38_quantize_q8_k(ctx, n_tokens, width, d_x, const_cast<void *>(d_q8k))) return -1;
        d_x = nullptr;
    }
    for (int i = 0; i < n_mats; ++i) {
        if (!on_big[i]) continue;
        const long row_tiles = ((long)rows[i] + Q38_GEMM_ROWS - 1) / Q38_GEMM_ROWS;
        q38_gemv_args g;
        memset(&g, 0, sizeof(g));
        g.weights[0] = static_cast<const uint8_t *>(d_weights[i]);
        g.out[0] = d_out[i];
        g.rows[0] = rows[i];
        g.n_mats = 1;
        g.q8k = d_q8k;
        g.width = width;
        g.n_tokens = n_tokens;
        if (ctx->launch(ctx->f_gemm[ti], (unsigned)row_tiles, (unsigned)tok_tiles, 1, 256, &g)) return -1;
    }
    if (ks_call) {
        /* workgroup x serves 32-row tile x - wg_begin[m] of the launch's
         * matrix m.  Waves per workgroup by workgroups per CU: up to one, 16
         * waves split the blocks; up to 1.5, 8; beyond, 4 (measured on the
         * FFN, q|gate and k matrices at 16-256 tokens) */
        q38_gemv_args g;
        memset(&g, 0, sizeof(g));
        long row_tiles = 0;
        int m = 0;
        for (int i = 0; i < n_mats; ++i) {
            if (rows[i] == 0 || on_big[i]) continue;
            g.weights[m] = static_cast<const uint8_t *>(d_weights[i]);
            g.out[m] = d_out[i];
            g.rows[m] = rows[i];
            g.wg_begin[m] = (int32_t)row_tiles;
            row_tiles += ((long)rows[i] + Q38_GEMM_KS_ROWS - 1) / Q38_GEMM_KS_ROWS;
            ++m;
        }
        g.wg_begin[m] = (int32_t)row_tiles;
        g.n_mats = m;
        g.q8k = d_q8k;
        g.width = width;
        g.n_tokens = n_tokens;
        hipFunction_t fk = ctx->f_gemm_ks[ti];
        int waves = Q38_GEMM_KS_WAVES;
        if (ks_total <= (long)ctx->cu_count && ctx->f_gemm_ks16[ti] != nullptr) {
            fk = ctx->f_gemm_ks16[ti];
            waves = Q38_GEMM_KS_WAVES_WIDE;
        } else if (2 * ks_total > 3L * ctx->cu_count && ctx->f_gemm_ks4[ti] != nullptr) {
            fk = ctx->f_gemm_ks4[ti];
            waves = Q38_GEMM_KS_WAVES_NARROW;
        }
        if (ctx->launch(fk, (unsigned)row_tiles, (unsigned)ks_tok_tiles, 1, 64 * waves, &g)) return -1;
    }

    /* The GEMV over the other matrices, in one launch.  Tokens per pass: as
     * many as Q38_GEMV_ACT_LDS holds (one at least), up to 8, spread evenly
     * over the passes that takes (8 tokens at most 3 per pass: 3, 3, 2) */
    const int blocks = width / Q38_Q8K_BLOCK;
    int tok_pass = std::max(1, std::min(Q38_GEMV_TOKENS, Q38_GEMV_ACT_LDS / (blocks * Q38_GEMV_REC_BYTES)));
    tok_pass = std::min(tok_pass, n_tokens);
    {
        const int passes = (n_tokens + tok_pass - 1) / tok_pass;
        tok_pass = (n_tokens + passes - 1) / passes;
    }
    /* rows per workgroup: up to Q38_GEMV_UNITS_MAX units (four per lane), the
     * per-token terms in at most 16 KiB of LDS, and few enough rows that the
     * launch has about as many workgroups as the CUs hold at once: a lane
     * keeps one 144-210 byte block in flight, so the bytes a CU has in
     * flight -- and with them its share of the bandwidth -- grow with the
     * workgroups it runs side by side */
    /* f32 terms a workgroup keeps in LDS: 16 KiB, or for IQ4_NL's eight
     * terms per block with several tokens 96 KiB (with at most 64 KiB of
     * staged activations, the 160 KiB of a CU), so that a workgroup still
     * holds a few rows (64 units would be 3 rows of a 5120-wide matrix) */
    const int term_floats = (nt > 1 && tok_pass > 1) ? 24576 : 4096;
    const int max_units = std::min(Q38_GEMV_UNITS_MAX, term_floats / (tok_pass * nt));
    const long tok_groups_all = ((long)n_tokens + tok_pass - 1) / tok_pass;
    int target_per_wg = max_units / blocks;
    {
        long all_rows = 0;
        for (int i = 0; i < n_mats; ++i)
            if (on_gemv[i]) all_rows += rows[i];
        const long lds_max =
            grid_lds + (long)tok_pass * blocks * Q38_GEMV_REC_BYTES + (long)tok_pass * max_units * 4 * nt;
        long occ = ctx->gemv_occupancy[ti_occ];
        if (ctx->lds_per_cu > 0) occ = std::max(1L, std::min(occ, ctx->lds_per_cu / lds_max));
        const long slots = std::max(1L, (long)ctx->cu_count * occ / std::max(1L, tok_groups_all));
        target_per_wg = (int)std::max(1L, std::min((long)target_per_wg, (all_rows + slots - 1) / slots));
    }
    q38_gemv_args a;
    memset(&a, 0, sizeof(a));
    long wgs = 0;
    int max_per_wg = 1;
    int kept = 0;
    for (int i = 0; i < n_mats; ++i) {
        if (!on_gemv[i]) continue;
        const int per_wg = target_per_wg;
        a.weights[kept] = static_cast<const uint8_t *>(d_weights[i]);
        a.out[kept] = d_out[i];
        a.rows[kept] = rows[i];
        a.rows_per_wg[kept] = per_wg;
        a.wg_begin[kept] = (int32_t)wgs;
        wgs += ((long)rows[i] + per_wg - 1) / per_wg;
        max_per_wg = std::max(max_per_wg, per_wg);
        ++kept;
    }
    if (kept == 0) return 0;
    const long tok_groups = ((long)n_tokens + tok_pass - 1) / tok_pass;
    /* one pass: a workgroup per row group; several: the passes of a row
     * group 8 workgroup ids apart (one XCD, dispatched together) */
    const long grid = tok_groups == 1 ? wgs : (wgs + 7) / 8 * 8 * tok_groups;
    if (grid > 0x7FFFFFFFL) return fail("too many rows or tokens");
    a.wg_begin[kept] = (int32_t)wgs;
    a.n_mats = kept;
    a.q8k = d_q8k;
    a.x = d_x;
    a.width = width;
    a.n_tokens = n_tokens;
    a.tok_pass = tok_pass;
    a.tok_groups = (int32_t)tok_groups;
    const unsigned lds =
        (unsigned)(grid_lds + tok_pass * blocks * Q38_GEMV_REC_BYTES + tok_pass * max_per_wg * blocks * 4 * nt);
    return ctx->launch(f, (unsigned)grid, 1, 1, 256, &a, lds);
}

int q38_gemv_q8_k_multi(q38_ctx *ctx, int ggml_type, int n_mats, const int *rows, int width,
                        const void *const *d_weights, const void *d_q8k, int n_tokens, float *const *d_out) {
    return gemv_q8k_multi(ctx, ggml_type, n_mats, rows, width, d_weights, nullptr, d_q8k, n_tokens, d_out);
}

int q38_quantize_project_q8_k(q38_ctx *ctx, int ggml_type, int n_mats, const int *rows, int width,
                              const void *const *d_weights, const float *d_x, int n_tokens, void *d_q8k,
                              float *const *d_out) {
    if (d_x == nullptr && n_tokens > 0) return fail("d_x is NULL");
    return gemv_q8k_multi(ctx, ggml_type, n_mats, rows, width, d_weights, d_x, d_q8k, n_tokens, d_out);
}

int q38_gemv_q8_k(q38_ctx *ctx, int ggml_type, int rows, int width, const void *d_weights, const void *d_q8k,
                  int n_tokens, float *d_out) {
    return q38_gemv_q8_k_multi(ctx, ggml_type, 1, &rows, width, &d_weights, d_q8k, n_tokens, &d_out);
}

static const int kF32UnitMinTokens = 4;
static const int kF32UnitMinTokensQ80 = 9;

int q38_gemv_f32(q38_ctx *ctx, int ggml_type, int rows, int width, const void *d_weights, const float *d_x,
                 int n_tokens, float *d_out) {
    if (ctx == nullptr) return fail("ctx is NULL");
    int ti = -1, block = 1, block_bytes = 0;
    if (ggml_type == Q38_GGML_F32) ti = 0, block_bytes = 4;
    else if (ggml_type == Q38_GGML_F16) ti = 1, block_bytes = 2;
    else if (ggml_type == Q38_GGML_BF16) ti = 2, block_bytes = 2;
    else if (ggml_type == Q38_GGML_Q8_0) ti = 3, block = 32, block_bytes = 34;
    else
        return fail("unsupported weight type %d for the f32 path (F32 0, F16 1, BF16 30, Q8_0 8)", ggml_type);
    if (rows < 0 || n_tokens < 0) return fail("negative rows or n_tokens");
    const int wmul = ti == 3 ? 64 : 8;
    if (width <= 0 || width % wmul != 0) return fail("width %d is not a positive multiple of %d", width, wmul);
    if (rows == 0 || n_tokens == 0) return 0;
    if (d_weights == nullptr || d_x == nullptr || d_out == nullptr) return fail("NULL argument");
    if ((uintptr_t)d_weights % (ti == 3 ? 4 : 16) != 0)
        return fail("d_weights must be %d-byte aligned", ti == 3 ? 4 : 16);
    if ((uintptr_t)d_x % 16 != 0) return fail("d_x must be 16-byte aligned");
    const long row_groups = ((long)rows + 3) / 4;
    const long tok_groups = ((long)n_tokens + Q38_GEMV_TOKENS - 1) / Q38_GEMV_TOKENS;
    if (row_groups > 0x7FFFFFFFL || tok_groups > 65535) return fail("too many rows or tokens");
    /* Widths a multiple of 64 take the bf16 matrix unit from 4 tokens on
     * (Q8_0: from 9, its staged GEMV being faster up to 8): up to 32 tokens,
     * or where the 128 x 64 tiles would give fewer than half a workgroup per
     * CU, 64 rows x 32 tokens per workgroup with k split over its waves;
     * otherwise the 128 x 64 tiles (measured on 48-17408 rows x 5120 and
     * 5120 x 17408, 2-4096 tokens: e.g. BF16 17408 x 5120 at 15 tokens 72
     * against 188 us as the GEMV, at 48 tokens 105 against 123 us on the
     * split-k form; 48 x 5120 at 4096 tokens 39 against 99 us) */
    const bool unit_width = width % Q38_GEMM_F32_K == 0;
    const long big_wgs = ((long)rows + Q38_GEMM_F32_ROWS - 1) / Q38_GEMM_F32_ROWS *
                         (((long)n_tokens + Q38_GEMM_F32_TOKENS - 1) / Q38_GEMM_F32_TOKENS);
    const bool on_unit_any = unit_width && n_tokens >= (ti == 3 ? kF32UnitMinTokensQ80 : kF32UnitMinTokens);
    const bool skinny = on_unit_any && (n_tokens <= 32 || 2 * big_wgs < (long)ctx->cu_count);
    const bool on_unit = on_unit_any && !skinny;
    if (skinny) {
        q38_gemv_f32_args s;
        memset(&s, 0, sizeof(s));
        s.weights = static_cast<const uint8_t *>(d_weights);
        s.x = d_x;
        s.out = d_out;
        s.row_bytes = (int64_t)(width / block) * block_bytes;
        s.rows = rows;
        s.width = width;
        s.n_tokens = n_tokens;
        return ctx->launch(ctx->f_gemm_f32s[ti], (unsigned)((rows + 63) / 64), (unsigned)((n_tokens + 31) / 32), 1,
                           256, &s);
    }
    q38_gemv_f32_args a;
    memset(&a, 0, sizeof(a));
    a.weights = static_cast<const uint8_t *>(d_weights);
    a.x = d_x;
    a.out = d_out;
    a.row_bytes = (int64_t)(width / block) * block_bytes;
    a.rows = rows;
    a.width = width;
    a.n_tokens = n_tokens;
    if (on_unit) {
        /* 128-token tiles where they still give 4+ workgroups per CU
         * (measured: 5-11% faster at 4096 tokens through 5120-17408 rows,
         * 12-25% slower at 512-1024 tokens, where the grid shrinks) */
        const long row_tiles = ((long)rows + Q38_GEMM_F32_ROWS - 1) / Q38_GEMM_F32_ROWS;
        const long wide_tok = ((long)n_tokens + Q38_GEMM_F32_WIDE_TOKENS - 1) / Q38_GEMM_F32_WIDE_TOKENS;
        if (ctx->f_gemm_f32w[ti] != nullptr && row_tiles * wide_tok >= 4L * ctx->cu_count)
            return ctx->launch(ctx->f_gemm_f32w[ti], (unsigned)row_tiles, (unsigned)wide_tok, 1, 256, &a);
        return ctx->launch(ctx->f_gemm_f32[ti], (unsigned)row_tiles,
                           (unsigned)((n_tokens + Q38_GEMM_F32_TOKENS - 1) / Q38_GEMM_F32_TOKENS), 1, 256, &a);
    }
    /* Q8_0: the activations staged in LDS once per 4 RW rows, TP tokens a
     * pass (the smallest of 1, 2, 4, 8 that holds min(T, 8)); 4 rows a wave
     * for 8-token passes, else 2 (measured on 1024-17408 rows x 5120 and
     * 5120 x 17408: 2 rows 5-20% faster at 1-4 tokens, 4 rows 2-20% at 8) */
    if (ti == 3) {
        const int tpi = n_tokens <= 1 ? 0 : n_tokens <= 2 ? 1 : n_tokens <= 4 ? 2 : 3;
        const int tp = 1 << tpi;
        const long wg_rows = tp == 8 ? 16 : 8;
        return ctx->launch(ctx->f_gemv_q80s[tpi], (unsigned)((rows + wg_rows - 1) / wg_rows),
                           (unsigned)((n_tokens + tp - 1) / tp), 1, 256, &a);
    }
    return ctx->launch(ctx->f_gemv_f32[ti], (unsigned)row_groups, (unsigned)tok_groups, 1, 256, &a); /* ti < 3 */
}

}  /* extern "C" */
