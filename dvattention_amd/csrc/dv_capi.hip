// C ABI of libdvattn_amd.so (declared in include/dvattn_amd.h).  Validates the
// arguments the reference's torch binding validated (src/binding.cu:41-296),
// rejects the shapes/dtypes it silently ignored, and launches the gfx950
// kernels on the caller's stream.  No exception crosses this boundary.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <initializer_list>
#include <mutex>
#include <vector>

#include "../../include/dvattn_amd.h"
#include "dv_common.h"
#include "dv_stream.h"

namespace {

thread_local char g_err[512] = "";

dvattn_status fail(dvattn_status st, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return st;
}

dvattn_status ok() {
    g_err[0] = '\0';
    return DVATTN_OK;
}

dvattn_status hip_fail(hipError_t e, const char* what) {
    return fail(DVATTN_ERR_HIP, "%s: %s (%s)", what, hipGetErrorString(e), dv::last_hip_site());
}

bool valid_dtype(int dt) { return dt == DVATTN_F32 || dt == DVATTN_F16 || dt == DVATTN_BF16; }

int log2_exact(int v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int s = 0;
    while ((1 << s) < v) ++s;
    return s;
}

int current_device(int device) {
    if (device >= 0) return device;
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) d = 0;
    return d;
}

// Checks shared by the attention entry points: GQA 16, E == Ev == 128
// (paged_kernel_v21.cuh:413, varlen:410, kernel_v21.cuh:400).
dvattn_status check_heads(const dvattn_shape* s) {
    if (s->Hkv <= 0) return fail(DVATTN_ERR_INVALID, "Hkv must be positive (got %d)", s->Hkv);
    if (s->Hq != 16 * s->Hkv)
        return fail(DVATTN_ERR_UNSUPPORTED, "only GQA 16 is implemented (Hq=%d, Hkv=%d)", s->Hq, s->Hkv);
    if (s->E != 128 || s->Ev != 128)
        return fail(DVATTN_ERR_UNSUPPORTED, "only head dims E == Ev == 128 are implemented (E=%d, Ev=%d)", s->E,
                    s->Ev);
    return DVATTN_OK;
}

dvattn_status check_rotary(int R, int E) {
    if (R < 0 || R > E || (R & 1))
        return fail(DVATTN_ERR_UNSUPPORTED, "rotary_dim must be even and in [0, E] (got %d, E=%d)", R, E);
    return DVATTN_OK;
}

dvattn_status check_pages(const dvattn_shape* s) {
    if (s->block_size <= 0) return fail(DVATTN_ERR_INVALID, "block_size must be positive (got %d)", s->block_size);
    if (s->max_blocks_per_seq < 0 || s->num_blocks < 0)
        return fail(DVATTN_ERR_INVALID, "max_blocks_per_seq / num_blocks must be >= 0");
    // the kernels index cache rows (block, slot, KV head) with 32-bit integers
    if ((long long)s->num_blocks * s->block_size * (s->Hkv > 0 ? s->Hkv : 1) >= (1ll << 32))
        return fail(DVATTN_ERR_UNSUPPORTED, "K/V cache of %lld rows exceeds 2^32 rows",
                    (long long)s->num_blocks * s->block_size * s->Hkv);
    return DVATTN_OK;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// The attention kernels move queries, outputs, cache and view rows and partial
// results as 16-byte vectors and LDS DMAs, update 8-byte merge flags in the
// workspace atomically and read the int32 / fp32 arrays as 4-byte words (the
// reference's kernels load 16-byte vectors too, paged_kernel_v21.cuh:58-62,
// unchecked).  A pointer off that alignment is refused here instead of reaching
// a kernel.  Null pointers pass: the null checks are separate.
struct Aligned {
    const void* ptr;
    const char* name;
    unsigned align;
};

unsigned elem_bytes(int dtype) { return dtype == DVATTN_F32 ? 4u : 2u; }

dvattn_status check_aligned(std::initializer_list<Aligned> ptrs) {
    for (const Aligned& a : ptrs)
        if ((uintptr_t)a.ptr & (a.align - 1))
            return fail(DVATTN_ERR_INVALID, "%s must be %u-byte aligned (got %p)", a.name, a.align, a.ptr);
    return DVATTN_OK;
}

// ---- static scratch of dvattn_paged_sdpa_noalloc ------------------------------
// Device memory for the partial results and merge directory of the paged entry
// point, for callers that cannot allocate.  Each GPU the library runs on holds
// its own copy of the array until the process ends.  In host code `scratch`
// names a host-side stand-in, never the device memory: the device address is
// taken once per device with hipGetSymbolAddress and only that address is used.
constexpr size_t kScratchBytes = (size_t)DVATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call on that device, with the device current).
dvattn_status scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(DVATTN_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(DVATTN_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(DVATTN_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_dev[dev] = ptr;
    }
    *out = g_scratch_dev[dev];
    return DVATTN_OK;
}

size_t contig_table_bytes(int F) {
    return F > dv::kMaxFragArgs ? align256((size_t)F * sizeof(dv::FragDesc)) : 0;
}

}  // namespace

namespace dv {

namespace {

// Option values; kUnset until first read (then from the environment).
constexpr int kUnset = -1;
std::atomic<int> g_options[kOptCount] = {kUnset};

int option_from_env(Option) {
    const char* e = getenv("DVATTN_SMALL_PATH");
    if (!e) return kSmallAuto;
    if (e[0] == '0') return kSmallOff;
    if (strcmp(e, "require") == 0) return kSmallRequire;
    if (strcmp(e, "force") == 0) return kSmallForce;
    return kSmallAuto;
}

}  // namespace

int option(Option o) {
    int v = g_options[o].load(std::memory_order_relaxed);
    if (v == kUnset) {
        int expected = kUnset;
        const int init = option_from_env(o);
        g_options[o].compare_exchange_strong(expected, init, std::memory_order_relaxed);
        v = g_options[o].load(std::memory_order_relaxed);
    }
    return v;
}

void set_option(Option o, int value) { g_options[o].store(value, std::memory_order_relaxed); }

// splitmix64 of a process-wide call counter, 48 bits, nonzero
unsigned long long next_call_tag() {
    static std::atomic<unsigned long long> calls{0x5eed5eedull};
    unsigned long long z = calls.fetch_add(0x9e3779b97f4a7c15ull, std::memory_order_relaxed);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    z &= (1ull << 48) - 1ull;
    return z ? z : 1ull;
}

}  // namespace dv

extern "C" {

const char* dvattn_last_error(void) { return g_err; }

dvattn_status dvattn_set_option(const char* name, int value) {
    if (!name) return fail(DVATTN_ERR_INVALID, "dvattn_set_option: null name");
    if (strcmp(name, "small_path") == 0) {
        if (value < dv::kSmallOff || value > dv::kSmallForce)
            return fail(DVATTN_ERR_INVALID, "small_path: 0 (off), 1 (auto), 2 (require) or 3 (force), not %d", value);
        dv::set_option(dv::kOptSmallPath, value);
        return ok();
    }
    return fail(DVATTN_ERR_INVALID, "unknown option \"%s\" (small_path)", name);
}

int dvattn_get_option(const char* name) {
    if (!name) return -1;
    if (strcmp(name, "small_path") == 0) return dv::option(dv::kOptSmallPath);
    return -1;
}

int dvattn_abi_version(void) { return DVATTN_ABI_VERSION; }

// ---------------------------------------------------------------------------
size_t dvattn_paged_sdpa_workspace_size(int dtype, const dvattn_shape* s, int device) {
    if (!s || !valid_dtype(dtype)) return 0;
    if (dv::use_chunk(dtype, s->S)) return dv::chunk_workspace_bytes(s->W, s->S, s->Hkv, current_device(device));
    return dv::decode_workspace_bytes(s->W * s->S, s->Hkv, current_device(device), dtype);
}

dvattn_status dvattn_paged_sdpa(int dtype, void* out, float scale, const int* locations, const void* queries,
                                const float* cosines, const float* sines, const int* fragment_lengths,
                                const void* k_cache, const void* v_cache, const int* block_tables,
                                const dvattn_shape* s, void* workspace, size_t workspace_bytes, void* stream) {
    if (!s) return fail(DVATTN_ERR_INVALID, "shape is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    if (s->F < 0 || s->W < 0 || s->S < 0) return fail(DVATTN_ERR_INVALID, "negative F/W/S");
    if ((long long)s->W * s->S == 0 || s->Hkv == 0) return ok();  // paged_kernel_v21.cuh:385-386
    dvattn_status st;
    if ((st = check_heads(s)) != DVATTN_OK) return st;
    if ((st = check_rotary(s->rotary_dim, s->E)) != DVATTN_OK) return st;
    if ((st = check_pages(s)) != DVATTN_OK) return st;
    if (!out || !queries) return fail(DVATTN_ERR_INVALID, "null output or query pointer");
    if (s->F > 0 && (!locations || !fragment_lengths || ((!cosines || !sines) && s->rotary_dim > 0)))
        return fail(DVATTN_ERR_INVALID, "null locations / fragment_lengths / cos / sin pointer");
    if (s->num_blocks > 0 && (!k_cache || !v_cache)) return fail(DVATTN_ERR_INVALID, "null k/v cache pointer");
    if (s->max_blocks_per_seq > 0 && !block_tables) return fail(DVATTN_ERR_INVALID, "null block_tables pointer");
    if ((st = check_aligned({{out, "out", 16}, {queries, "queries", 16}, {k_cache, "k_cache", 16},
                             {v_cache, "v_cache", 16}, {workspace, "workspace", 16}, {locations, "locations", 4},
                             {fragment_lengths, "fragment_lengths", 4}, {cosines, "cosines", 4},
                             {sines, "sines", 4}, {block_tables, "block_tables", 4}})) != DVATTN_OK)
        return st;
    const size_t need = dvattn_paged_sdpa_workspace_size(dtype, s, -1);
    if (workspace_bytes < need || (need && !workspace))
        return fail(DVATTN_ERR_WORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);

    dv::DecodeParams p;
    memset(&p, 0, sizeof(p));
    p.out = out;
    p.loc = locations;
    p.q = queries;
    p.cosv = cosines;
    p.sinv = sines;
    p.fl = fragment_lengths;
    p.kc = k_cache;
    p.vc = v_cache;
    p.bt = block_tables;
    p.l2scale = scale * 1.4426950408889634f;  // scale / ln 2 (paged_kernel_v21.cuh:47)
    p.F = s->F;
    p.W = s->W;
    p.S = s->S;
    p.Hq = s->Hq;
    p.Hkv = s->Hkv;
    p.R = s->rotary_dim;
    p.bs = s->block_size;
    p.bs_shift = log2_exact(s->block_size);
    p.maxB = s->max_blocks_per_seq;
    p.nblocks = s->num_blocks;
    p.min_keys = dv::kDecodeMinKeys;
    const long long max_keys = (long long)s->max_blocks_per_seq * s->block_size;
    hipError_t e;
    if (dv::use_chunk(dtype, s->S)) {
        p.min_keys = 256;
        e = dv::launch_chunk(dtype, dv::kQRotFull, dv::kKvPaged, p, max_keys, workspace, workspace_bytes,
                             (hipStream_t)stream);
    } else {
        e = dv::launch_decode(dtype, dv::kQRotFull, dv::kKvPaged, dv::kRowWS, p, s->W * s->S, max_keys, workspace,
                              workspace_bytes, (hipStream_t)stream);
    }
    if (e != hipSuccess) return hip_fail(e, "dvattn_paged_sdpa launch");
    return ok();
}

dvattn_status dvattn_paged_sdpa_noalloc(int dtype, void* out, float scale, const int* locations,
                                        const void* queries, const float* cosines, const float* sines,
                                        const int* fragment_lengths, const void* k_cache, const void* v_cache,
                                        const int* block_tables, const dvattn_shape* s, void* stream) {
    if (!s) return fail(DVATTN_ERR_INVALID, "shape is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    const size_t need = dvattn_paged_sdpa_workspace_size(dtype, s, -1);
    if (need > kScratchBytes)
        return fail(DVATTN_ERR_WORKSPACE,
                    "dvattn_paged_sdpa_noalloc: this shape needs %zu bytes of scratch, the static scratch "
                    "holds %zu (use dvattn_paged_sdpa with a workspace)",
                    need, kScratchBytes);
    void* ws = nullptr;
    const dvattn_status st = scratch_address(&ws);
    if (st != DVATTN_OK) return st;
    // nothing in the scratch has to start at zero: every call's kernels write the
    // partial slots and the merge directory before reading them
    return dvattn_paged_sdpa(dtype, out, scale, locations, queries, cosines, sines, fragment_lengths, k_cache,
                             v_cache, block_tables, s, ws, kScratchBytes, stream);
}

// ---------------------------------------------------------------------------
size_t dvattn_varlen_paged_sdpa_workspace_size(int dtype, const dvattn_shape* s, int device) {
    if (!s || !valid_dtype(dtype)) return 0;
    if (dv::use_varlen_chunk(dtype, s->total_q_tokens, s->W))
        return dv::varlen_chunk_workspace_bytes(s->total_q_tokens, s->W, s->Hkv, current_device(device));
    return dv::decode_workspace_bytes(s->total_q_tokens, s->Hkv, current_device(device), dtype);
}

dvattn_status dvattn_varlen_paged_sdpa(int dtype, void* out, float scale, const int* locations,
                                       const void* queries, const float* cosines, const float* sines,
                                       const int* fragment_lengths, const void* k_cache, const void* v_cache,
                                       const int* block_tables, const int* cu_seqlens_q, const int* cu_seqlens_k,
                                       const dvattn_shape* s, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    (void)cu_seqlens_k;  // passed but never read by the reference (binding.cu:279,290)
    if (!s) return fail(DVATTN_ERR_INVALID, "shape is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    if (s->F < 0 || s->W < 0 || s->total_q_tokens < 0) return fail(DVATTN_ERR_INVALID, "negative F/W/T");
    if (s->total_q_tokens == 0 || s->Hkv == 0) return ok();  // varlen_paged_kernel_v21.cuh:382-383
    dvattn_status st;
    if ((st = check_heads(s)) != DVATTN_OK) return st;
    if ((st = check_rotary(s->rotary_dim, s->E)) != DVATTN_OK) return st;
    if ((st = check_pages(s)) != DVATTN_OK) return st;
    if (!out || !queries) return fail(DVATTN_ERR_INVALID, "null output or query pointer");
    if (s->W > 0 && !cu_seqlens_q) return fail(DVATTN_ERR_INVALID, "null cu_seqlens_q pointer");
    if (s->F > 0 && (!locations || !fragment_lengths || ((!cosines || !sines) && s->rotary_dim > 0)))
        return fail(DVATTN_ERR_INVALID, "null locations / fragment_lengths / cos / sin pointer");
    if (s->num_blocks > 0 && (!k_cache || !v_cache)) return fail(DVATTN_ERR_INVALID, "null k/v cache pointer");
    if (s->max_blocks_per_seq > 0 && !block_tables) return fail(DVATTN_ERR_INVALID, "null block_tables pointer");
    if ((st = check_aligned({{out, "out", 16}, {queries, "queries", 16}, {k_cache, "k_cache", 16},
                             {v_cache, "v_cache", 16}, {workspace, "workspace", 16}, {locations, "locations", 4},
                             {fragment_lengths, "fragment_lengths", 4}, {cosines, "cosines", 4},
                             {sines, "sines", 4}, {block_tables, "block_tables", 4},
                             {cu_seqlens_q, "cu_seqlens_q", 4}})) != DVATTN_OK)
        return st;
    const size_t need = dvattn_varlen_paged_sdpa_workspace_size(dtype, s, -1);
    if (workspace_bytes < need || (need && !workspace))
        return fail(DVATTN_ERR_WORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);

    dv::DecodeParams p;
    memset(&p, 0, sizeof(p));
    p.out = out;
    p.loc = locations;
    p.q = queries;
    p.cosv = cosines;
    p.sinv = sines;
    p.fl = fragment_lengths;
    p.kc = k_cache;
    p.vc = v_cache;
    p.bt = block_tables;
    p.cu_q = cu_seqlens_q;
    p.l2scale = scale * 1.4426950408889634f;
    p.F = s->F;
    p.W = s->W;
    p.S = 1;
    p.T = s->total_q_tokens;
    p.Hq = s->Hq;
    p.Hkv = s->Hkv;
    p.R = s->rotary_dim;
    p.bs = s->block_size;
    p.bs_shift = log2_exact(s->block_size);
    p.maxB = s->max_blocks_per_seq;
    p.nblocks = s->num_blocks;
    p.min_keys = dv::kDecodeMinKeys;
    const long long max_keys = (long long)s->max_blocks_per_seq * s->block_size;
    hipError_t e;
    if (dv::use_varlen_chunk(dtype, s->total_q_tokens, s->W)) {
        // two or more packed tokens per sequence on average: each sequence's
        // tokens share one K/V stream (the reference re-reads K/V per token,
        // varlen_paged_kernel_v21.cuh:388)
        p.min_keys = 256;
        e = dv::launch_varlen_chunk(dtype, p, max_keys, workspace, workspace_bytes, (hipStream_t)stream);
    } else {
        e = dv::launch_decode(dtype, dv::kQRotHalf, dv::kKvPaged, dv::kRowVarlen, p, s->total_q_tokens, max_keys,
                              workspace, workspace_bytes, (hipStream_t)stream);
    }
    if (e != hipSuccess) return hip_fail(e, "dvattn_varlen_paged_sdpa launch");
    return ok();
}

// ---------------------------------------------------------------------------
size_t dvattn_sdpa_workspace_size(int dtype, const dvattn_shape* s, int device) {
    if (!s || !valid_dtype(dtype)) return 0;
    if (dv::use_chunk(dtype, s->S))
        return dv::chunk_workspace_bytes(s->W, s->S, s->Hkv, current_device(device)) + contig_table_bytes(s->F);
    return dv::decode_workspace_bytes(s->W * s->S, s->Hkv, current_device(device), dtype) +
           contig_table_bytes(s->F);
}

}  // extern "C"

namespace {

// dvattn_sdpa's argument checks (binding.cu:79-149, plus the shapes the
// reference ignored) and its launch parameters: p, the view table and the
// longest row's key count.  `empty`: nothing to compute.
dvattn_status sdpa_setup(int dtype, void* out, float scale, const int* locations, const void* rotated_queries,
                         const int* fragment_lengths, const void* const* key_fragments,
                         const void* const* value_fragments, const int* fragment_tokens, const int* fragment_batch,
                         const dvattn_shape* s, void* workspace, size_t workspace_bytes, dv::DecodeParams& p,
                         std::vector<dv::FragDesc>& tab, long long& max_keys, bool& empty) {
    empty = true;
    if (!s) return fail(DVATTN_ERR_INVALID, "shape is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    if (s->F < 0 || s->W < 0 || s->S < 0) return fail(DVATTN_ERR_INVALID, "negative F/W/S");
    if ((long long)s->W * s->S == 0 || s->Hkv == 0) return DVATTN_OK;
    dvattn_status st;
    if ((st = check_heads(s)) != DVATTN_OK) return st;
    if (!out || !rotated_queries) return fail(DVATTN_ERR_INVALID, "null output or query pointer");
    if (s->F > 0 && (!locations || !fragment_lengths || !key_fragments || !value_fragments || !fragment_tokens ||
                     !fragment_batch))
        return fail(DVATTN_ERR_INVALID, "null locations / fragment_lengths / fragment arrays");
    if ((st = check_aligned({{out, "out", 16}, {rotated_queries, "rotated_queries", 16},
                             {workspace, "workspace", 16}, {locations, "locations", 4},
                             {fragment_lengths, "fragment_lengths", 4}})) != DVATTN_OK)
        return st;
    const size_t need = dvattn_sdpa_workspace_size(dtype, s, -1);
    if (workspace_bytes < need || (need && !workspace))
        return fail(DVATTN_ERR_WORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);

    memset(&p, 0, sizeof(p));
    tab.assign((size_t)s->F, dv::FragDesc{});
    max_keys = 0;
    for (int f = 0; f < s->F; ++f) {
        const int L = fragment_tokens[f];
        const int B = fragment_batch[f];
        if (L < 0) return fail(DVATTN_ERR_INVALID, "fragment %d: negative token count", f);
        if (B != 1 && B != s->W)
            return fail(DVATTN_ERR_INVALID, "fragment %d: batch %d is neither 1 nor W=%d", f, B, s->W);
        if (L > 0 && (!key_fragments[f] || !value_fragments[f]))
            return fail(DVATTN_ERR_INVALID, "fragment %d: null pointer", f);
        if ((((uintptr_t)key_fragments[f]) | ((uintptr_t)value_fragments[f])) & 15)
            return fail(DVATTN_ERR_INVALID, "fragment %d: pointers must be 16-byte aligned", f);
        dv::FragDesc& d = tab[(size_t)f];
        d.k = key_fragments[f];
        d.v = value_fragments[f];
        d.L = L;
        d.bstride = B == 1 ? 0 : (long long)s->Hkv * L * 128;
        d.pad = 0;
        max_keys += L;
        if (f < dv::kMaxFragArgs) p.frags[f] = d;
    }
    p.out = out;
    p.loc = locations;
    p.q = rotated_queries;
    p.fl = fragment_lengths;
    p.l2scale = scale * 1.4426950408889634f;
    p.F = s->F;
    p.W = s->W;
    p.S = s->S;
    p.Hq = s->Hq;
    p.Hkv = s->Hkv;
    p.R = 0;
    p.bs = 1;
    p.bs_shift = 0;
    p.min_keys = dv::kDecodeMinKeys;
    empty = false;
    return DVATTN_OK;
}

// View descriptors written into the device view table by a kernel whose
// arguments carry them: the values travel with the launch (a captured graph
// keeps its own copy), so no host buffer has to outlive the call, as a
// host-to-device copy from the caller's memory would in a captured graph.
constexpr int kFragFillBatch = 64;  // descriptors per launch: 2 KiB of kernel arguments
struct FragFill {
    dv::FragDesc d[kFragFillBatch];
    int first, n;
};

__global__ __launch_bounds__(kFragFillBatch) void dv_frag_fill(dv::FragDesc* dst, const FragFill b) {
    const int i = threadIdx.x;
    if (i < b.n) dst[b.first + i] = b.d[i];
}

// The general contiguous-view launch: view table (F > kMaxFragArgs) to the
// workspace, then the decode or chunk kernel on already-rotated queries.
dvattn_status sdpa_launch(int dtype, dv::DecodeParams& p, const std::vector<dv::FragDesc>& tab, long long max_keys,
                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
    void* ws = workspace;
    size_t ws_left = workspace_bytes;
    const size_t tab_bytes = contig_table_bytes(p.F);
    if (tab_bytes) {
        dv::FragDesc* dst = reinterpret_cast<dv::FragDesc*>(workspace);
        for (int first = 0; first < p.F; first += kFragFillBatch) {
            FragFill b;
            memset(&b, 0, sizeof(b));
            b.first = first;
            b.n = p.F - first < kFragFillBatch ? p.F - first : kFragFillBatch;
            for (int i = 0; i < b.n; ++i) b.d[i] = tab[(size_t)(first + i)];
            hipLaunchKernelGGL(dv_frag_fill, dim3(1), dim3(kFragFillBatch), 0, stream, dst, b);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return hip_fail(e, "dvattn_sdpa view table");
        }
        p.frag_tab = dst;
        ws = reinterpret_cast<unsigned char*>(workspace) + tab_bytes;
        ws_left -= tab_bytes;
    }
    hipError_t e;
    if (dv::use_chunk(dtype, p.S)) {
        p.min_keys = 256;
        e = dv::launch_chunk(dtype, dv::kQPre, dv::kKvContig, p, max_keys, ws, ws_left, stream);
    } else {
        e = dv::launch_decode(dtype, dv::kQPre, dv::kKvContig, dv::kRowWS, p, p.W * p.S, max_keys, ws, ws_left,
                              stream);
    }
    if (e != hipSuccess) return hip_fail(e, "dvattn_sdpa launch");
    return ok();
}

// Whether the single-launch path takes a validated contiguous-view call (fp32,
// fp16 or bf16): at most kMaxFragArgs views of at most kSmallMaxChunks chunks
// together, and its partials within the documented workspace size of the shape
// (so the choice depends on the shape and the fragment lengths only); rotating
// calls (dvattn_fused) also need rotary_dim % 8 == 0.  Returns the chunk count,
// or -1 for the general path.
// Option small_path (dvattn_set_option; DVATTN_SMALL_PATH at first use): off
// turns the path off; require makes a call it cannot take fail with
// DVATTN_ERR_UNSUPPORTED (*refused); force takes it past the workgroup limit
// below as well (for measuring that limit: bench.py --small-crossover).
int small_path_chunks(int dtype, const dvattn_shape* s, const int* fragment_tokens, bool rotating, bool* refused) {
    *refused = false;
    const int mode = dv::option(dv::kOptSmallPath);
    if (mode == dv::kSmallOff) return -1;
    const bool require = mode == dv::kSmallRequire;
    const bool force = mode == dv::kSmallForce;
    int chunks = -1;
    if (s->F >= 1 && s->F <= dv::kMaxFragArgs && (!rotating || s->rotary_dim % 8 == 0)) {
        chunks = dv::small_chunks(s->F, fragment_tokens);
        const long long items = (long long)s->W * s->S * s->Hkv;
        // Only a single-chunk call (one view of at most kSmallChunk keys) needs
        // no merge.  Any other call (several chunks, from one long view or
        // from several views) merges its chunks in the launch, and every
        // workgroup pays the merge protocol's fences, whose cost grows with the
        // number of workgroups: past items x chunks = small_max_merged() the
        // general path (rotation, decode and merge launches) is faster
        // (measured crossover about 190 workgroups for fp32, about 110 for
        // 16-bit types, whose general path is faster).
        if (chunks > 1 && items * chunks > dv::small_max_merged(dtype) && !force) chunks = -1;
        if (chunks >= 1 && dv::small_workspace_bytes(items, chunks) > dvattn_sdpa_workspace_size(dtype, s, -1))
            chunks = -1;
    }
    if (chunks < 1 && require) {
        fail(DVATTN_ERR_UNSUPPORTED,
             "DVATTN_SMALL_PATH=require: the single-launch path takes calls of 1-%d views with at most %d "
             "chunks of %d keys per row, and at most %d (fp32) or %d (16-bit) workgroups in all when a row "
             "has more than one chunk (one per row, KV head and chunk); rotary_dim %% 8 == 0 when it rotates",
             dv::kMaxFragArgs, dv::kSmallMaxChunks, dv::kSmallChunk, dv::small_max_merged(DVATTN_F32),
             dv::small_max_merged(DVATTN_BF16));
        *refused = true;
    }
    return chunks;
}

dvattn_status small_launch(int dtype, int qmode, const dv::DecodeParams& p, int chunks, const int* fragment_tokens,
                           void* rq_out, void* workspace, hipStream_t stream) {
    dv::SmallParams sp;
    memset(&sp, 0, sizeof(sp));
    sp.d = p;
    sp.rq = rq_out;
    sp.chunks = chunks;
    int c = 0;
    for (int f = 0; f < p.F; ++f) {
        sp.first_chunk[f] = c;
        const int L = fragment_tokens[f];
        c += L > 0 ? (L + dv::kSmallChunk - 1) / dv::kSmallChunk : 1;
    }
    sp.first_chunk[p.F] = c;
    const hipError_t e = dv::launch_small(dtype, qmode, sp, workspace, stream);
    if (e != hipSuccess) return hip_fail(e, "single-launch attention");
    return ok();
}

// dvattn_rope's checks (rope.cuh:54-65) into p; `empty`: nothing to rotate.
dvattn_status rope_setup(int dtype, void* out, const void* queries, const float* cosines, const float* sines,
                         const dvattn_shape* s, dv::RopeParams& p, bool& empty) {
    empty = true;
    if (!s) return fail(DVATTN_ERR_INVALID, "shape is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    if (s->F < 0 || s->W < 0 || s->Hq < 0 || s->S < 0 || s->E < 0)
        return fail(DVATTN_ERR_INVALID, "negative size");
    dvattn_status st;
    if ((st = check_rotary(s->rotary_dim, s->E)) != DVATTN_OK) return st;
    if ((long long)s->F * s->W * s->Hq * s->S * s->E == 0) return DVATTN_OK;  // rope.cuh:58-60
    if (!out || !queries || (s->rotary_dim > 0 && (!cosines || !sines)))
        return fail(DVATTN_ERR_INVALID, "null pointer");
    if ((st = check_aligned({{out, "out", elem_bytes(dtype)}, {queries, "queries", elem_bytes(dtype)},
                             {cosines, "cosines", 4}, {sines, "sines", 4}})) != DVATTN_OK)
        return st;
    memset(&p, 0, sizeof(p));
    p.out = out;
    p.q = queries;
    p.cosv = cosines;
    p.sinv = sines;
    p.F = s->F;
    p.W = s->W;
    p.Hq = s->Hq;
    p.S = s->S;
    p.E = s->E;
    p.R = s->rotary_dim;
    p.half_width = 0;
    empty = false;
    return DVATTN_OK;
}

}  // namespace

extern "C" {

dvattn_status dvattn_sdpa(int dtype, void* out, float scale, const int* locations, const void* rotated_queries,
                          const int* fragment_lengths, const void* const* key_fragments,
                          const void* const* value_fragments, const int* fragment_tokens,
                          const int* fragment_batch, const dvattn_shape* s, void* workspace,
                          size_t workspace_bytes, void* stream) {
    dv::DecodeParams p;
    std::vector<dv::FragDesc> tab;
    long long max_keys = 0;
    bool empty = true;
    dvattn_status st = sdpa_setup(dtype, out, scale, locations, rotated_queries, fragment_lengths, key_fragments,
                                  value_fragments, fragment_tokens, fragment_batch, s, workspace, workspace_bytes, p,
                                  tab, max_keys, empty);
    if (st != DVATTN_OK) return st;
    if (empty) return ok();
    bool refused = false;
    const int chunks = small_path_chunks(dtype, s, fragment_tokens, false, &refused);
    if (refused) return DVATTN_ERR_UNSUPPORTED;
    if (chunks > 0)
        return small_launch(dtype, dv::kQPre, p, chunks, fragment_tokens, nullptr, workspace, (hipStream_t)stream);
    return sdpa_launch(dtype, p, tab, max_keys, workspace, workspace_bytes, (hipStream_t)stream);
}

// binding.cu:356-372: rotate the queries into rotated_queries, attend on them.
// Both steps' arguments are checked before anything runs; short views take the
// single launch that rotates, attends and merges.
dvattn_status dvattn_fused(int dtype, void* out, void* rotated_queries, float scale, const int* locations,
                           const void* queries, const int* fragment_lengths, const void* const* key_fragments,
                           const void* const* value_fragments, const int* fragment_tokens,
                           const int* fragment_batch, const float* cosines, const float* sines,
                           const dvattn_shape* s, void* workspace, size_t workspace_bytes, void* stream) {
    dv::RopeParams rp;
    bool no_rope = true;
    dvattn_status st = rope_setup(dtype, rotated_queries, queries, cosines, sines, s, rp, no_rope);
    if (st != DVATTN_OK) return st;
    dv::DecodeParams p;
    std::vector<dv::FragDesc> tab;
    long long max_keys = 0;
    bool empty = true;
    st = sdpa_setup(dtype, out, scale, locations, rotated_queries, fragment_lengths, key_fragments, value_fragments,
                    fragment_tokens, fragment_batch, s, workspace, workspace_bytes, p, tab, max_keys, empty);
    if (st != DVATTN_OK) return st;
    // the single launch reads the unrotated queries in vectors as well
    if (!no_rope && (st = check_aligned({{queries, "queries", 16}})) != DVATTN_OK) return st;
    bool refused = false;
    const int chunks = empty || no_rope ? -1 : small_path_chunks(dtype, s, fragment_tokens, true, &refused);
    if (refused) return DVATTN_ERR_UNSUPPORTED;
    if (chunks > 0) {
        p.q = queries;
        p.cosv = cosines;
        p.sinv = sines;
        p.R = s->rotary_dim;
        return small_launch(dtype, dv::kQRotFull, p, chunks, fragment_tokens, rotated_queries, workspace,
                            (hipStream_t)stream);
    }
    if (!no_rope) {
        const hipError_t e = dv::launch_rope(dtype, rp, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "dvattn_rope launch");
    }
    if (empty) return ok();
    return sdpa_launch(dtype, p, tab, max_keys, workspace, workspace_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
dvattn_status dvattn_rope(int dtype, void* out, const void* queries, const float* cosines, const float* sines,
                          const dvattn_shape* s, void* stream) {
    dv::RopeParams p;
    bool empty = true;
    const dvattn_status st = rope_setup(dtype, out, queries, cosines, sines, s, p, empty);
    if (st != DVATTN_OK) return st;
    if (empty) return ok();
    hipError_t e = dv::launch_rope(dtype, p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dvattn_rope launch");
    return ok();
}

dvattn_status dvattn_varlen_rope(int dtype, void* out, const void* queries, const float* cosines,
                                 const float* sines, const dvattn_shape* s, void* stream) {
    if (!s) return fail(DVATTN_ERR_INVALID, "shape is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    if (s->F < 0 || s->total_q_tokens < 0 || s->Hq < 0 || s->E < 0) return fail(DVATTN_ERR_INVALID, "negative size");
    dvattn_status st;
    if ((st = check_rotary(s->rotary_dim, s->E)) != DVATTN_OK) return st;
    if ((long long)s->F * s->total_q_tokens * s->Hq * s->E == 0) return ok();  // rope.cuh:106-108
    if (!out || !queries || (s->rotary_dim > 0 && (!cosines || !sines)))
        return fail(DVATTN_ERR_INVALID, "null pointer");
    if ((st = check_aligned({{out, "out", elem_bytes(dtype)}, {queries, "queries", elem_bytes(dtype)},
                             {cosines, "cosines", 4}, {sines, "sines", 4}})) != DVATTN_OK)
        return st;
    dv::RopeParams p;
    memset(&p, 0, sizeof(p));
    p.out = out;
    p.q = queries;
    p.cosv = cosines;
    p.sinv = sines;
    p.F = s->F;
    p.T = s->total_q_tokens;
    p.Hq = s->Hq;
    p.E = s->E;
    p.R = s->rotary_dim;
    p.half_width = 1;
    hipError_t e = dv::launch_rope(dtype, p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dvattn_varlen_rope launch");
    return ok();
}

// ---------------------------------------------------------------------------
dvattn_status dvattn_paged_kv_append(int dtype, int rope_dtype, void* k_cache, void* v_cache,
                                     const int* block_tables, const int* positions, const void* keys,
                                     const void* values, const void* cosines, const void* sines,
                                     const dvattn_shape* s, const dvattn_kv_layout* lay, void* stream) {
    if (!s || !lay) return fail(DVATTN_ERR_INVALID, "shape or layout is null");
    if (!valid_dtype(dtype)) return fail(DVATTN_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
    if (rope_dtype != DVATTN_F32 && rope_dtype != dtype)
        return fail(DVATTN_ERR_UNSUPPORTED, "cos/sin dtype code %d must be float32 or the storage dtype %d",
                    rope_dtype, dtype);
    if (s->W < 0 || s->S < 0 || s->Hkv < 0 || s->E < 0 || s->Ev < 0)
        return fail(DVATTN_ERR_INVALID, "negative W/S/Hkv/E/Ev");
    if ((long long)s->W * s->S * s->Hkv == 0 || (s->E == 0 && s->Ev == 0)) return ok();
    dvattn_status st;
    if ((st = check_rotary(s->rotary_dim, s->E)) != DVATTN_OK) return st;
    if (s->block_size <= 0) return fail(DVATTN_ERR_INVALID, "block_size must be positive (got %d)", s->block_size);
    if (s->max_blocks_per_seq < 0 || s->num_blocks < 0)
        return fail(DVATTN_ERR_INVALID, "max_blocks_per_seq / num_blocks must be >= 0");
    // the kernel indexes (token, head, element) in 32 bits
    if ((long long)s->W * s->S * s->Hkv * (s->E > s->Ev ? s->E : s->Ev) >= (1ll << 31))
        return fail(DVATTN_ERR_UNSUPPORTED, "%lld key elements in one call exceed 2^31",
                    (long long)s->W * s->S * s->Hkv * (s->E > s->Ev ? s->E : s->Ev));
    if (!k_cache || !v_cache || !keys || !values || !positions || (s->max_blocks_per_seq > 0 && !block_tables) ||
        (s->rotary_dim > 0 && (!cosines || !sines)))
        return fail(DVATTN_ERR_INVALID, "null pointer");
    // element-wise copies where the 16-byte vector form does not apply
    if ((st = check_aligned({{k_cache, "k_cache", elem_bytes(dtype)}, {v_cache, "v_cache", elem_bytes(dtype)},
                             {keys, "keys", elem_bytes(dtype)}, {values, "values", elem_bytes(dtype)},
                             {cosines, "cosines", elem_bytes(rope_dtype)}, {sines, "sines", elem_bytes(rope_dtype)},
                             {positions, "positions", 4}, {block_tables, "block_tables", 4}})) != DVATTN_OK)
        return st;
    dv::AppendParams p;
    memset(&p, 0, sizeof(p));
    p.kc = k_cache;
    p.vc = v_cache;
    p.bt = block_tables;
    p.pos = positions;
    p.k = keys;
    p.v = values;
    p.cosv = cosines;
    p.sinv = sines;
    for (int i = 0; i < 3; ++i) {
        p.kcs[i] = lay->k_cache_strides[i];
        p.vcs[i] = lay->v_cache_strides[i];
        p.ks[i] = lay->key_strides[i];
        p.vs[i] = lay->value_strides[i];
    }
    p.cs[0] = lay->rope_strides[0];
    p.cs[1] = lay->rope_strides[1];
    p.W = s->W;
    p.S = s->S;
    p.Hkv = s->Hkv;
    p.E = s->E;
    p.Ev = s->Ev;
    p.R = s->rotary_dim;
    p.bs = s->block_size;
    p.maxB = s->max_blocks_per_seq;
    p.nblocks = s->num_blocks;
    hipError_t e = dv::launch_kv_append(dtype, rope_dtype, p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dvattn_paged_kv_append launch");
    return ok();
}

dvattn_status dvattn_view_metadata(int* locations, float* cosines, float* sines, const int* fragment_lengths,
                                   const int* order, const float* inv_freq, float attention_scaling,
                                   int round_dtype, int F, int W, int S, int rotary_dim, void* stream) {
    if (F < 0 || W < 0 || S < 0) return fail(DVATTN_ERR_INVALID, "negative F/W/S");
    if (rotary_dim < 0 || (rotary_dim & 1))
        return fail(DVATTN_ERR_UNSUPPORTED, "rotary_dim must be even and >= 0 (got %d)", rotary_dim);
    if (round_dtype != -1 && round_dtype != DVATTN_F32 && round_dtype != DVATTN_F16 && round_dtype != DVATTN_BF16)
        return fail(DVATTN_ERR_UNSUPPORTED, "unsupported round_dtype code %d", round_dtype);
    if ((long long)F * W * S == 0) return ok();
    if (!locations || !fragment_lengths || !order || (rotary_dim > 0 && (!cosines || !sines || !inv_freq)))
        return fail(DVATTN_ERR_INVALID, "null pointer");
    dv::MetaParams p;
    memset(&p, 0, sizeof(p));
    p.loc = locations;
    p.cosv = cosines;
    p.sinv = sines;
    p.fl = fragment_lengths;
    p.order = order;
    p.inv_freq = inv_freq;
    p.scaling = attention_scaling;
    p.round_dt = round_dtype == DVATTN_F32 ? -1 : round_dtype;
    p.F = F;
    p.W = W;
    p.S = S;
    p.R = rotary_dim;
    hipError_t e = dv::launch_view_meta(p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dvattn_view_metadata launch");
    return ok();
}

}  // extern "C"
