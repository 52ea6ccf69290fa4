// Shared host/device definitions of the gfx950 DVAttn kernels: compile-time
// limits, the launch-parameter structs passed by value to the kernels, and the
// internal launcher API used by the C ABI layer (dv_capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include <atomic>
#include <stdint.h>
#include <stdlib.h>

namespace dv {

constexpr int kWave = 64;         // CDNA wavefront width
constexpr int kGqa = 16;          // query heads per KV head (reference hard-wires 16)
constexpr int kHeadDim = 128;     // E == Ev == 128 (reference hard-wires 128)
constexpr int kStep = 32;         // keys per wave per pipeline step (two 16-key MFMA blocks)
constexpr int kMaxRows = 2048;    // query rows per decode launch (schedule prefix lives in LDS)
constexpr int kMaxFragArgs = 16;  // contiguous views passed in kernel arguments
constexpr int kMaxWavesPerWg = 4; // KV heads per workgroup (one wave per KV head)

// Storage dtype codes (same values as dvattn_dtype in include/dvattn_amd.h).
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// How the query of (row, view) is obtained.
enum QMode : int {
    kQRotFull = 0,  // rotate queries [W,Hq,S,E] with full-width cos/sin [F,W,S,R]
    kQRotHalf = 1,  // rotate queries [T,Hq,E] with half-width cos/sin [F,T,R/2]
    kQPre = 2       // read rotated queries [F,W,Hq,S,E]
};

// Where the keys/values of (sequence, view, token) live.
enum KvMode : int {
    kKvPaged = 0,   // [num_blocks, block_size, Hkv, E] pages via block_tables
    kKvContig = 1   // per-view [B, Hkv, L, E] tensors
};

// How a query row maps to a sequence / query token.
enum RowMode : int {
    kRowWS = 0,     // row r = w*S + s
    kRowVarlen = 1  // row r = packed token t, sequence from cu_seqlens_q
};

struct FragDesc {
    const void* k;        // [B, Hkv, L, E]
    const void* v;        // [B, Hkv, L, Ev]
    long long bstride;    // elements between batch entries (0: one batch shared by all rows)
    int L;                // tokens in the tensor
    int pad;
};

struct DecodeParams {
    void* out;
    float* part;          // partial results, slot-major (layout: store_partial in dv_device.h)
    int* dir;             // per (row, head-group) segment: {first slot, piece count}
    const int* loc;
    const void* q;
    const float* cosv;
    const float* sinv;
    const int* fl;        // fragment_lengths [F] (device)
    const void* kc;
    const void* vc;
    const int* bt;
    const int* cu_q;
    const int* vgroups;   // varlen chunk path: per row group {first token, tokens, sequence, 0}
    const FragDesc* frag_tab;  // device table when F > kMaxFragArgs
    float l2scale;        // softmax scale / ln(2): scores are kept in base-2 units
    int F, W, S, Hq, Hkv, R;
    int bs, bs_shift, maxB, nblocks;
    int T;
    int row_begin, nrows;
    int hpw;              // KV heads (waves) per workgroup
    int nwg;              // workgroups launched
    int min_keys;         // smallest key range worth a workgroup
    int piece_cost;       // fixed cost of starting a segment, in keys (charged in the work split)
    int skew_pm;          // per mille of a chunk moved from each odd workgroup to the even one before it
    int slot_floats;      // floats per partial slot
    FragDesc frags[kMaxFragArgs];
};

// Single-launch path for short contiguous views (dv_small.hip): one workgroup
// per (query row, KV head, chunk of kSmallChunk tensor keys of one view).  The
// query rotation (dvattn_fused), the attention and the merge of the chunks all
// run in that one launch; the last workgroup of a (row, KV head) to finish
// merges its chunks.  Rotating mode needs rotary_dim % 8 == 0.
constexpr int kSmallChunk = 64;       // tensor keys per workgroup (16 per wave)
constexpr int kSmallMaxChunks = 64;   // chunks per (row, KV head): up to 4096 keys
// Most workgroups (items x chunks) of a call whose rows have several chunks.
inline int small_max_merged(int dtype) { return dtype == kF32 ? 160 : 96; }

struct SmallParams {
    DecodeParams d;                   // out, loc, q, cosv, sinv, fl, frags, l2scale, F, W, S, Hq, Hkv, R
    void* rq;                         // rotated queries [F,W,Hq,S,E] written here (rotating mode), or null
    float* part;                      // [items][chunks][kGqa * (kHeadDim + 1)]: normalised output, base-2 LSE
    unsigned long long* flags;        // [items][chunks] arrival flags (raised: == tag)
    unsigned long long tag;           // this call's flag value (48 bits, nonzero)
    int chunks;                       // chunks per item (row, KV head)
    int first_chunk[kMaxFragArgs + 1];  // first chunk of view f; first_chunk[F] = chunks
};

struct RopeParams {
    void* out;
    const void* q;
    const float* cosv;
    const float* sinv;
    int F, W, Hq, S, E, R;
    int T;                // varlen
    int half_width;       // 1: cos/sin rows hold R/2 entries (varlen layout)
};

// K/V append: new tokens' keys (rotated) and values written into their cache rows.
struct AppendParams {
    void* kc;                 // destination caches, element strides (page, row, head), last dim contiguous
    void* vc;
    long long kcs[3], vcs[3];
    const int* bt;            // block_tables [W, maxB]
    const int* pos;           // positions [W, S]: logical position of each new token (< 0: not written)
    const void* k;            // keys [W, Hkv, S, E], element strides (w, h, s)
    const void* v;            // values [W, Hkv, S, Ev]
    long long ks[3], vs[3];
    const void* cosv;         // cos/sin [W, S, R], element strides (w, s); 0 broadcasts
    const void* sinv;
    long long cs[2];
    int W, S, Hkv, E, Ev, R;
    int bs, maxB, nblocks;
};

// View metadata: per (view, sequence, new token) location and rotary cos/sin.
struct MetaParams {
    int* loc;                 // [F, W, S]
    float* cosv;              // [F, W, S, R] (full width, both halves equal)
    float* sinv;
    const int* fl;            // fragment_lengths [F]
    const int* order;         // [W, F]: view index of sequence w's j-th segment
    const float* inv_freq;    // [R/2]
    float scaling;            // attention scaling applied to cos and sin
    int round_dt;             // -1, or a 16-bit dtype code the values are rounded through
    int F, W, S, R;
};

// CU count of a device, queried once per device (thread-safe; 256 if unknown).
inline int device_cu_count(int device) {
    static std::atomic<int> cache[64];
    if (device < 0 || device >= 64) return 256;
    int c = cache[device].load(std::memory_order_relaxed);
    if (c == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || c <= 0) c = 256;
        cache[device].store(c, std::memory_order_relaxed);
    }
    return c;
}

// Runs set_up() the first time a kernel is launched on `device` (one bit per
// device in `done`).  set_up must be idempotent: two threads launching at once
// may both run it.
template <class F>
inline hipError_t once_per_device(std::atomic<unsigned long long>& done, int device, F&& set_up) {
    const unsigned long long bit = device >= 0 && device < 64 ? 1ull << device : 0ull;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    const hipError_t e = set_up();
    if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
    return e;
}

// Process-wide switches (dvattn_set_option): each starts from its environment
// variable, read once at first use, and a call of dvattn_set_option replaces it.
//   kOptSmallPath  (DVATTN_SMALL_PATH: "0" off, "require", "force"; default auto)
enum Option : int { kOptSmallPath = 0, kOptCount = 1 };
enum SmallPathMode : int { kSmallOff = 0, kSmallAuto = 1, kSmallRequire = 2, kSmallForce = 3 };
int option(Option o);
void set_option(Option o, int value);

// Per-call tags for arrival flags: 48 bits, nonzero, distinct for consecutive
// calls of the process.
unsigned long long next_call_tag();

// A per-mille tuning value from the environment, clamped to [0, 200].
inline int env_per_mille(const char* name, int dflt) {
    const char* e = getenv(name);
    const int x = e ? atoi(e) : dflt;
    return x < 0 ? 0 : (x > 200 ? 200 : x);
}

// Internal launchers (return a hipError_t; argument validation happens in the C ABI).
size_t decode_workspace_bytes(int nrows_total, int Hkv, int device, int dtype);
// max_keys_per_row: host-known upper bound of the visible keys of one row (sizes
// the grid for small problems).
hipError_t launch_decode(int dtype, int qmode, int kvmode, int rowmode, const DecodeParams& base,
                         int nrows_total, long long max_keys_per_row, void* workspace, size_t ws_bytes,
                         hipStream_t stream);
hipError_t launch_rope(int dtype, const RopeParams& p, hipStream_t stream);
// rope_dtype: kF32, or the storage dtype (cos/sin in the model's dtype).
hipError_t launch_kv_append(int dtype, int rope_dtype, const AppendParams& p, hipStream_t stream);
hipError_t launch_view_meta(const MetaParams& p, hipStream_t stream);

// Multi-query path (S >= 2 tokens per sequence; dv_chunk for 16-bit types,
// dv_chunk32 for fp32): K/V read once per block of 16 tokens.  Rows of
// DecodeParams are (sequence, 16-token block) groups.
inline bool use_chunk(int /*dtype*/, int S) { return S >= 2; }
size_t chunk_workspace_bytes(int W, int S, int Hkv, int device);
hipError_t launch_chunk(int dtype, int qmode, int kvmode, const DecodeParams& base, long long max_keys_per_group,
                        void* workspace, size_t ws_bytes, hipStream_t stream);
// Varlen calls whose packed tokens average two or more per sequence go through
// the chunk kernel too: the tokens of each sequence (token t: the first i with
// t < cu_seqlens_q[i + 1]) in groups of up to 16, one K/V stream per group.
constexpr int kVarlenChunkMaxW = 4096;  // sequences of the group-table pass (LDS)
inline bool use_varlen_chunk(int dtype, int T, int W) {
    (void)dtype;
    return W >= 1 && W <= kVarlenChunkMaxW && (long long)T >= 2ll * W;
}
size_t varlen_chunk_workspace_bytes(int T, int W, int Hkv, int device);
hipError_t launch_varlen_chunk(int dtype, const DecodeParams& base, long long max_keys_per_group, void* workspace,
                               size_t ws_bytes, hipStream_t stream);
// Single-launch path (contiguous views, any dtype): chunks per item for F views of
// fragment_tokens toks, or -1 when the views are too many or too long; the
// workspace it needs for `items` (row, KV head) items; the launch (qmode kQPre
// or kQRotFull).  launch_small fills p.part / p.flags / p.tag from the workspace.
int small_chunks(int F, const int* toks);
size_t small_workspace_bytes(long long items, int chunks);
hipError_t launch_small(int dtype, int qmode, SmallParams& p, void* workspace, hipStream_t stream);
// Which runtime call produced the last error returned by launch_decode (this thread).
const char* last_hip_site();

}  // namespace dv
