// torch.ops.libdvatt: the reference's operator schemas (src/binding.cu:407-430),
// registered for the CUDA dispatch key (which ROCm torch uses for HIP
// tensors).  Each op checks what the reference's binding checked
// (binding.cu:41-296) plus dtype / device / size consistency, allocates the
// workspace from torch's caching allocator, and calls the C ABI of
// libdvattn_amd.so on the tensors' current HIP stream.  Unsupported dtypes and
// shapes raise instead of silently doing nothing.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <string>
#include <vector>

#include "dvattn_amd.h"

namespace {

int dtype_code(const at::Tensor& t) {
    switch (t.scalar_type()) {
        case at::kFloat: return DVATTN_F32;
        case at::kHalf: return DVATTN_F16;
        case at::kBFloat16: return DVATTN_BF16;
        default:
            TORCH_CHECK(false, "dvattn: unsupported dtype ", t.scalar_type(),
                        " (float32, float16 and bfloat16 are supported)");
    }
    return -1;
}

void check_same(const at::Tensor& t, const at::Tensor& ref, const char* name) {
    TORCH_CHECK(t.scalar_type() == ref.scalar_type(), "dvattn: ", name, " must have dtype ", ref.scalar_type(),
                ", got ", t.scalar_type());
}

void check_dev(const at::Tensor& t, const at::Tensor& ref, const char* name) {
    TORCH_CHECK(t.is_cuda(), "dvattn: ", name, " must be a GPU tensor");
    TORCH_CHECK(t.device() == ref.device(), "dvattn: ", name, " is on ", t.device(), ", expected ", ref.device());
}

void check_i32(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.scalar_type() == at::kInt, "dvattn: ", name, " must be int32, got ", t.scalar_type());
}

void check_f32(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.scalar_type() == at::kFloat, "dvattn: ", name, " must be float32, got ", t.scalar_type());
}

void check_contig(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_contiguous(), "dvattn: ", name, " must be contiguous");
}

void check_dim(const at::Tensor& t, int64_t d, const char* name) {
    TORCH_CHECK(t.dim() == d, "dvattn: ", name, " must have ", d, " dims, got ", t.dim());
}

int as_int(int64_t v, const char* what) {
    TORCH_CHECK(v >= 0 && v <= INT32_MAX, "dvattn: ", what, " = ", v, " does not fit the kernels' int32 indexing");
    return (int)v;
}

void check_status(dvattn_status st, const char* op) {
    TORCH_CHECK(st == DVATTN_OK, "dvattn: ", op, " failed: ", dvattn_last_error());
}

hipStream_t stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
    return at::empty({(int64_t)(bytes ? bytes : 1)}, like.options().dtype(at::kByte));
}

// ---------------------------------------------------------------------------
// dvattn_rope(Tensor(a!) output, Tensor queries, Tensor cosines, Tensor sines)
// binding.cu:41-77: out [F,W,Hq,S,E], queries [W,Hq,S,E], cos/sin [F,W,S,R].
void dvattn_rope_op(at::Tensor& out, const at::Tensor& queries, const at::Tensor& cosines, const at::Tensor& sines) {
    const int dt = dtype_code(out);
    check_dim(out, 5, "output");
    check_dim(queries, 4, "queries");
    check_dim(cosines, 4, "cosines");
    check_dim(sines, 4, "sines");
    check_same(queries, out, "queries");
    check_f32(cosines, "cosines");
    check_f32(sines, "sines");
    check_contig(out, "output");
    check_contig(queries, "queries");
    check_contig(cosines, "cosines");
    check_contig(sines, "sines");
    check_dev(queries, out, "queries");
    check_dev(cosines, out, "cosines");
    check_dev(sines, out, "sines");
    const int64_t F = out.size(0), W = out.size(1), Hq = out.size(2), S = out.size(3), E = out.size(4);
    const int64_t R = cosines.size(3);
    TORCH_CHECK(queries.size(0) == W && queries.size(1) == Hq && queries.size(2) == S && queries.size(3) == E,
                "dvattn_rope: queries must be [W,Hq,S,E] = [", W, ",", Hq, ",", S, ",", E, "], got ", queries.sizes());
    TORCH_CHECK(cosines.size(0) == F && cosines.size(1) == W && cosines.size(2) == S,
                "dvattn_rope: cosines must be [F,W,S,R], got ", cosines.sizes());
    TORCH_CHECK(sines.sizes() == cosines.sizes(), "dvattn_rope: sines must match cosines, got ", sines.sizes());
    c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    dvattn_shape s{};
    s.F = as_int(F, "F");
    s.W = as_int(W, "W");
    s.Hq = as_int(Hq, "Hq");
    s.S = as_int(S, "S");
    s.E = as_int(E, "E");
    s.rotary_dim = as_int(R, "rotary_dim");
    check_status(dvattn_rope(dt, out.data_ptr(), queries.data_ptr(), cosines.data_ptr<float>(),
                             sines.data_ptr<float>(), &s, stream_of(out)),
                 "dvattn_rope");
}

// dvattn_varlen_rope(Tensor(a!) output, Tensor queries, Tensor cosines, Tensor sines)
// binding.cu:205-247: out [F,T,H,E], queries [T,H,E], cos/sin [F,T,R/2].
void dvattn_varlen_rope_op(at::Tensor& out, const at::Tensor& queries, const at::Tensor& cosines,
                           const at::Tensor& sines) {
    const int dt = dtype_code(out);
    check_dim(out, 4, "output");
    check_dim(queries, 3, "queries");
    check_dim(cosines, 3, "cosines");
    check_dim(sines, 3, "sines");
    check_same(queries, out, "queries");
    check_f32(cosines, "cosines");
    check_f32(sines, "sines");
    check_contig(out, "output");
    check_contig(queries, "queries");
    check_contig(cosines, "cosines");
    check_contig(sines, "sines");
    check_dev(queries, out, "queries");
    check_dev(cosines, out, "cosines");
    check_dev(sines, out, "sines");
    const int64_t F = out.size(0), T = out.size(1), H = out.size(2), E = out.size(3);
    TORCH_CHECK(queries.size(0) == T && queries.size(1) == H && queries.size(2) == E,
                "dvattn_varlen_rope: queries must be [T,H,E], got ", queries.sizes());
    TORCH_CHECK(cosines.size(0) == F && cosines.size(1) == T, "dvattn_varlen_rope: cosines must be [F,T,R/2], got ",
                cosines.sizes());
    TORCH_CHECK(sines.sizes() == cosines.sizes(), "dvattn_varlen_rope: sines must match cosines, got ",
                sines.sizes());
    c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    dvattn_shape s{};
    s.F = as_int(F, "F");
    s.total_q_tokens = as_int(T, "T");
    s.Hq = as_int(H, "H");
    s.E = as_int(E, "E");
    s.rotary_dim = as_int(2 * cosines.size(2), "rotary_dim");
    check_status(dvattn_varlen_rope(dt, out.data_ptr(), queries.data_ptr(), cosines.data_ptr<float>(),
                                    sines.data_ptr<float>(), &s, stream_of(out)),
                 "dvattn_varlen_rope");
}

// ---------------------------------------------------------------------------
// dvattn_paged_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries,
//   Tensor cosines, Tensor sines, Tensor fragment_lengths, Tensor k_cache, Tensor v_cache,
//   Tensor block_tables)    binding.cu:151-203
void dvattn_paged_sdpa_op(at::Tensor& out, double scale, const at::Tensor& locations, const at::Tensor& queries,
                          const at::Tensor& cosines, const at::Tensor& sines, const at::Tensor& fragment_lengths,
                          const at::Tensor& k_cache, const at::Tensor& v_cache, const at::Tensor& block_tables) {
    const int dt = dtype_code(out);
    check_dim(out, 4, "output");
    check_dim(locations, 3, "locations");
    check_dim(queries, 4, "queries");
    check_dim(cosines, 4, "cosines");
    check_dim(sines, 4, "sines");
    check_dim(fragment_lengths, 1, "fragment_lengths");
    check_dim(k_cache, 4, "k_cache");
    check_dim(v_cache, 4, "v_cache");
    check_dim(block_tables, 2, "block_tables");
    check_same(queries, out, "queries");
    check_same(k_cache, out, "k_cache");
    check_same(v_cache, out, "v_cache");
    check_i32(locations, "locations");
    check_i32(fragment_lengths, "fragment_lengths");
    check_i32(block_tables, "block_tables");
    check_f32(cosines, "cosines");
    check_f32(sines, "sines");
    const at::Tensor* all[] = {&out, &locations, &queries, &cosines, &sines, &fragment_lengths,
                               &k_cache, &v_cache, &block_tables};
    const char* names[] = {"output", "locations", "queries", "cosines", "sines", "fragment_lengths",
                           "k_cache", "v_cache", "block_tables"};
    for (int i = 0; i < 9; ++i) {
        check_contig(*all[i], names[i]);
        check_dev(*all[i], out, names[i]);
    }
    const int64_t W = out.size(0), Hq = out.size(1), S = out.size(2), Ev = out.size(3);
    const int64_t F = locations.size(0);
    TORCH_CHECK(locations.size(1) == W && locations.size(2) == S, "dvattn_paged_sdpa: locations must be [F,W,S], got ",
                locations.sizes());
    const int64_t E = queries.size(3);
    TORCH_CHECK(queries.size(0) == W && queries.size(1) == Hq && queries.size(2) == S,
                "dvattn_paged_sdpa: queries must be [W,Hq,S,E], got ", queries.sizes());
    TORCH_CHECK(cosines.size(0) == F && cosines.size(1) == W && cosines.size(2) == S,
                "dvattn_paged_sdpa: cosines must be [F,W,S,R], got ", cosines.sizes());
    TORCH_CHECK(sines.sizes() == cosines.sizes(), "dvattn_paged_sdpa: sines must match cosines");
    TORCH_CHECK(fragment_lengths.size(0) == F, "dvattn_paged_sdpa: fragment_lengths must be [F], got ",
                fragment_lengths.sizes());
    const int64_t P = k_cache.size(0), bs = k_cache.size(1), Hkv = k_cache.size(2);
    TORCH_CHECK(k_cache.size(3) == E, "dvattn_paged_sdpa: k_cache head dim ", k_cache.size(3), " != query dim ", E);
    TORCH_CHECK(v_cache.size(0) == P && v_cache.size(1) == bs && v_cache.size(2) == Hkv && v_cache.size(3) == Ev,
                "dvattn_paged_sdpa: v_cache must be [num_blocks, block_size, Hkv, Ev], got ", v_cache.sizes());
    TORCH_CHECK(block_tables.size(0) >= W, "dvattn_paged_sdpa: block_tables needs a row per sequence (", W,
                "), got ", block_tables.sizes());
    c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    dvattn_shape s{};
    s.F = as_int(F, "F");
    s.W = as_int(W, "W");
    s.Hq = as_int(Hq, "Hq");
    s.Hkv = as_int(Hkv, "Hkv");
    s.E = as_int(E, "E");
    s.Ev = as_int(Ev, "Ev");
    s.S = as_int(S, "S");
    s.block_size = as_int(bs, "block_size");
    s.max_blocks_per_seq = as_int(block_tables.size(1), "max_blocks_per_seq");
    s.num_blocks = as_int(P, "num_blocks");
    s.rotary_dim = as_int(cosines.size(3), "rotary_dim");
    const size_t ws = dvattn_paged_sdpa_workspace_size(dt, &s, out.device().index());
    at::Tensor w = workspace(ws, out);
    check_status(dvattn_paged_sdpa(dt, out.data_ptr(), (float)scale, locations.data_ptr<int>(), queries.data_ptr(),
                                   cosines.data_ptr<float>(), sines.data_ptr<float>(),
                                   fragment_lengths.data_ptr<int>(), k_cache.data_ptr(), v_cache.data_ptr(),
                                   block_tables.data_ptr<int>(), &s, w.data_ptr(), ws, stream_of(out)),
                 "dvattn_paged_sdpa");
}

// dvattn_varlen_paged_sdpa(..., Tensor cu_seqlens_q, Tensor cu_seqlens_k)   binding.cu:249-296
void dvattn_varlen_paged_sdpa_op(at::Tensor& out, double scale, const at::Tensor& locations,
                                 const at::Tensor& queries, const at::Tensor& cosines, const at::Tensor& sines,
                                 const at::Tensor& fragment_lengths, const at::Tensor& k_cache,
                                 const at::Tensor& v_cache, const at::Tensor& block_tables,
                                 const at::Tensor& cu_seqlens_q, const at::Tensor& cu_seqlens_k) {
    const int dt = dtype_code(out);
    check_dim(out, 3, "output");
    check_dim(locations, 2, "locations");
    check_dim(queries, 3, "queries");
    check_dim(cosines, 3, "cosines");
    check_dim(sines, 3, "sines");
    check_dim(fragment_lengths, 1, "fragment_lengths");
    check_dim(k_cache, 4, "k_cache");
    check_dim(v_cache, 4, "v_cache");
    check_dim(block_tables, 2, "block_tables");
    check_dim(cu_seqlens_q, 1, "cu_seqlens_q");
    check_same(queries, out, "queries");
    check_same(k_cache, out, "k_cache");
    check_same(v_cache, out, "v_cache");
    check_i32(locations, "locations");
    check_i32(fragment_lengths, "fragment_lengths");
    check_i32(block_tables, "block_tables");
    check_i32(cu_seqlens_q, "cu_seqlens_q");
    check_f32(cosines, "cosines");
    check_f32(sines, "sines");
    const at::Tensor* all[] = {&out, &locations, &queries, &cosines, &sines, &fragment_lengths,
                               &k_cache, &v_cache, &block_tables, &cu_seqlens_q};
    const char* names[] = {"output", "locations", "queries", "cosines", "sines", "fragment_lengths",
                           "k_cache", "v_cache", "block_tables", "cu_seqlens_q"};
    for (int i = 0; i < 10; ++i) {
        check_contig(*all[i], names[i]);
        check_dev(*all[i], out, names[i]);
    }
    const int64_t T = queries.size(0), Hq = queries.size(1), E = queries.size(2);
    const int64_t F = locations.size(0);
    const int64_t W = cu_seqlens_q.size(0) - 1;
    TORCH_CHECK(W >= 0, "dvattn_varlen_paged_sdpa: cu_seqlens_q must have W+1 >= 1 entries");
    const int64_t Ev = v_cache.size(3);
    TORCH_CHECK(out.size(0) == T && out.size(1) == Hq && out.size(2) == Ev,
                "dvattn_varlen_paged_sdpa: output must be [T,Hq,Ev], got ", out.sizes());
    TORCH_CHECK(locations.size(1) == T, "dvattn_varlen_paged_sdpa: locations must be [F,T], got ", locations.sizes());
    TORCH_CHECK(cosines.size(0) == F && cosines.size(1) == T,
                "dvattn_varlen_paged_sdpa: cosines must be [F,T,R/2], got ", cosines.sizes());
    TORCH_CHECK(sines.sizes() == cosines.sizes(), "dvattn_varlen_paged_sdpa: sines must match cosines");
    TORCH_CHECK(fragment_lengths.size(0) == F, "dvattn_varlen_paged_sdpa: fragment_lengths must be [F]");
    const int64_t P = k_cache.size(0), bs = k_cache.size(1), Hkv = k_cache.size(2);
    TORCH_CHECK(k_cache.size(3) == E, "dvattn_varlen_paged_sdpa: k_cache head dim != query dim");
    TORCH_CHECK(v_cache.size(0) == P && v_cache.size(1) == bs && v_cache.size(2) == Hkv,
                "dvattn_varlen_paged_sdpa: v_cache must match k_cache pages, got ", v_cache.sizes());
    TORCH_CHECK(block_tables.size(0) >= W || T == 0,
                "dvattn_varlen_paged_sdpa: block_tables needs a row per sequence (", W, "), got ",
                block_tables.sizes());
    TORCH_CHECK(W > 0 || T == 0, "dvattn_varlen_paged_sdpa: tokens without any sequence (cu_seqlens_q has 1 entry)");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    dvattn_shape s{};
    s.F = as_int(F, "F");
    s.W = as_int(W, "W");
    s.Hq = as_int(Hq, "Hq");
    s.Hkv = as_int(Hkv, "Hkv");
    s.E = as_int(E, "E");
    s.Ev = as_int(Ev, "Ev");
    s.S = 1;
    s.total_q_tokens = as_int(T, "T");
    s.block_size = as_int(bs, "block_size");
    s.max_blocks_per_seq = as_int(block_tables.size(1), "max_blocks_per_seq");
    s.num_blocks = as_int(P, "num_blocks");
    s.rotary_dim = as_int(2 * cosines.size(2), "rotary_dim");
    const size_t ws = dvattn_varlen_paged_sdpa_workspace_size(dt, &s, out.device().index());
    at::Tensor w = workspace(ws, out);
    // cu_seqlens_k is part of the schema but, as in the reference (binding.cu:279,290), never read.
    (void)cu_seqlens_k;
    check_status(dvattn_varlen_paged_sdpa(dt, out.data_ptr(), (float)scale, locations.data_ptr<int>(),
                                          queries.data_ptr(), cosines.data_ptr<float>(), sines.data_ptr<float>(),
                                          fragment_lengths.data_ptr<int>(), k_cache.data_ptr(), v_cache.data_ptr(),
                                          block_tables.data_ptr<int>(), cu_seqlens_q.data_ptr<int>(), nullptr, &s,
                                          w.data_ptr(), ws, stream_of(out)),
                 "dvattn_varlen_paged_sdpa");
}

// ---------------------------------------------------------------------------
// dvattn_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries,
//   Tensor fragment_lengths, Tensor[] key_fragments, Tensor[] value_fragments)  binding.cu:79-149
void sdpa_common(at::Tensor& out, double scale, const at::Tensor& locations, const at::Tensor& rq,
                 const at::Tensor& fragment_lengths, const std::vector<at::Tensor>& keys,
                 const std::vector<at::Tensor>& values, const at::Tensor* queries, at::Tensor* rq_out,
                 const at::Tensor* cosines, const at::Tensor* sines) {
    const int dt = dtype_code(out);
    check_dim(out, 4, "output");
    check_dim(locations, 3, "locations");
    check_dim(rq, 5, "queries");
    check_dim(fragment_lengths, 1, "fragment_lengths");
    check_same(rq, out, "queries");
    check_i32(locations, "locations");
    check_i32(fragment_lengths, "fragment_lengths");
    check_contig(out, "output");
    check_contig(locations, "locations");
    check_contig(rq, "queries");
    check_contig(fragment_lengths, "fragment_lengths");
    check_dev(locations, out, "locations");
    check_dev(rq, out, "queries");
    check_dev(fragment_lengths, out, "fragment_lengths");
    const int64_t W = out.size(0), Hq = out.size(1), S = out.size(2), Ev = out.size(3);
    const int64_t F = locations.size(0);
    TORCH_CHECK(locations.size(1) == W && locations.size(2) == S, "dvattn_sdpa: locations must be [F,W,S], got ",
                locations.sizes());
    const int64_t E = rq.size(4);
    TORCH_CHECK(rq.size(0) == F && rq.size(1) == W && rq.size(2) == Hq && rq.size(3) == S,
                "dvattn_sdpa: queries must be [F,W,Hq,S,E], got ", rq.sizes());
    TORCH_CHECK(fragment_lengths.size(0) == F, "dvattn_sdpa: fragment_lengths must be [F]");
    TORCH_CHECK((int64_t)keys.size() == F && (int64_t)values.size() == F,
                "dvattn_sdpa: need one key and one value fragment per view (F=", F, "), got ", keys.size(), " and ",
                values.size());
    int64_t Hkv = 0;
    std::vector<const void*> kp(F), vp(F);
    std::vector<int> toks(F), batch(F);
    for (int64_t f = 0; f < F; ++f) {
        const at::Tensor& k = keys[f];
        const at::Tensor& v = values[f];
        TORCH_CHECK(k.dim() == 3 || k.dim() == 4, "dvattn_sdpa: key fragment ", f, " must be [B,Hkv,L,E] or [Hkv,L,E]");
        TORCH_CHECK(v.dim() == k.dim(), "dvattn_sdpa: value fragment ", f, " rank differs from its key fragment");
        check_same(k, out, "key fragment");
        check_same(v, out, "value fragment");
        check_contig(k, "key fragment");
        check_contig(v, "value fragment");
        check_dev(k, out, "key fragment");
        check_dev(v, out, "value fragment");
        const int fo = k.dim() == 4 ? 1 : 0;
        const int64_t B = fo ? k.size(0) : 1;
        if (f == 0) Hkv = k.size(fo);
        TORCH_CHECK(k.size(fo) == Hkv && v.size(fo) == Hkv, "dvattn_sdpa: fragment ", f, " has ", k.size(fo),
                    " kv heads, expected ", Hkv);
        TORCH_CHECK(k.size(fo + 1) == v.size(fo + 1), "dvattn_sdpa: fragment ", f, " key/value lengths differ");
        TORCH_CHECK(k.size(fo + 2) == E, "dvattn_sdpa: fragment ", f, " key dim ", k.size(fo + 2), " != ", E);
        TORCH_CHECK(v.size(fo + 2) == Ev, "dvattn_sdpa: fragment ", f, " value dim ", v.size(fo + 2), " != ", Ev);
        TORCH_CHECK(!fo || v.size(0) == B, "dvattn_sdpa: fragment ", f, " key/value batch differs");
        TORCH_CHECK(B == 1 || B == W, "dvattn_sdpa: fragment ", f, " batch ", B, " must be 1 or W=", W);
        kp[f] = k.data_ptr();
        vp[f] = v.data_ptr();
        toks[f] = as_int(k.size(fo + 1), "fragment length");
        batch[f] = (int)B;
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    dvattn_shape s{};
    s.F = as_int(F, "F");
    s.W = as_int(W, "W");
    s.Hq = as_int(Hq, "Hq");
    s.Hkv = as_int(Hkv, "Hkv");
    s.E = as_int(E, "E");
    s.Ev = as_int(Ev, "Ev");
    s.S = as_int(S, "S");
    const size_t ws = dvattn_sdpa_workspace_size(dt, &s, out.device().index());
    at::Tensor w = workspace(ws, out);
    if (queries) {
        check_dim(*queries, 4, "queries");
        check_dim(*cosines, 4, "cosines");
        check_dim(*sines, 4, "sines");
        check_same(*queries, out, "queries");
        check_f32(*cosines, "cosines");
        check_f32(*sines, "sines");
        check_contig(*queries, "queries");
        check_contig(*cosines, "cosines");
        check_contig(*sines, "sines");
        check_dev(*queries, out, "queries");
        check_dev(*cosines, out, "cosines");
        check_dev(*sines, out, "sines");
        TORCH_CHECK(queries->size(0) == W && queries->size(1) == Hq && queries->size(2) == S && queries->size(3) == E,
                    "dvattn_fused: queries must be [W,Hq,S,E], got ", queries->sizes());
        TORCH_CHECK(cosines->size(0) == F && cosines->size(1) == W && cosines->size(2) == S,
                    "dvattn_fused: cosines must be [F,W,S,R], got ", cosines->sizes());
        TORCH_CHECK(sines->sizes() == cosines->sizes(), "dvattn_fused: sines must match cosines");
        s.rotary_dim = as_int(cosines->size(3), "rotary_dim");
        check_status(dvattn_fused(dt, out.data_ptr(), rq_out->data_ptr(), (float)scale, locations.data_ptr<int>(),
                                  queries->data_ptr(), fragment_lengths.data_ptr<int>(), kp.data(), vp.data(),
                                  toks.data(), batch.data(), cosines->data_ptr<float>(), sines->data_ptr<float>(), &s,
                                  w.data_ptr(), ws, stream_of(out)),
                     "dvattn_fused");
    } else {
        check_status(dvattn_sdpa(dt, out.data_ptr(), (float)scale, locations.data_ptr<int>(), rq.data_ptr(),
                                 fragment_lengths.data_ptr<int>(), kp.data(), vp.data(), toks.data(), batch.data(), &s,
                                 w.data_ptr(), ws, stream_of(out)),
                     "dvattn_sdpa");
    }
}

void dvattn_sdpa_op(at::Tensor& out, double scale, const at::Tensor& locations, const at::Tensor& queries,
                    const at::Tensor& fragment_lengths, at::TensorList key_fragments, at::TensorList value_fragments) {
    sdpa_common(out, scale, locations, queries, fragment_lengths, key_fragments.vec(), value_fragments.vec(), nullptr,
                nullptr, nullptr, nullptr);
}

// dvattn_fused(Tensor(a!) output, Tensor(b!) rq, float scale, Tensor locations, Tensor queries,
//   Tensor fragment_lengths, Tensor[] key_fragments, Tensor[] value_fragments, Tensor cosines,
//   Tensor sines)   binding.cu:356-372: rotate into rq, then attend on rq.
void dvattn_fused_op(at::Tensor& out, at::Tensor& rq, double scale, const at::Tensor& locations,
                     const at::Tensor& queries, const at::Tensor& fragment_lengths, at::TensorList key_fragments,
                     at::TensorList value_fragments, const at::Tensor& cosines, const at::Tensor& sines) {
    std::vector<at::Tensor> ks, vs;
    ks.reserve(key_fragments.size());
    vs.reserve(value_fragments.size());
    for (const auto& k : key_fragments) ks.push_back(k.contiguous());  // binding.cu:362-369
    for (const auto& v : value_fragments) vs.push_back(v.contiguous());
    check_dim(rq, 5, "rq");
    check_contig(rq, "rq");
    check_dev(rq, out, "rq");
    sdpa_common(out, scale, locations, rq, fragment_lengths, ks, vs, &queries, &rq, &cosines, &sines);
}

// ---------------------------------------------------------------------------
// dvattn_paged_kv_append(Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor block_tables,
//   Tensor positions, Tensor keys, Tensor values, Tensor cosines, Tensor sines)
// The K side of a decode step (attention.py:304 rotation + 141-152 cache append)
// and merge_caches' re-rotation (attention.py:245-251) on a paged cache.
// keys/values [W,Hkv,S,E|Ev] and the caches may be strided views (last dim
// contiguous); cos/sin [W|1, S|1, R] broadcast over size-1 dims.  Keys/values
// may live in the cache tensors (merge_caches between segments of one pool) but
// must not overlap the rows being written.
void dvattn_paged_kv_append_op(at::Tensor& k_cache, at::Tensor& v_cache, const at::Tensor& block_tables,
                               const at::Tensor& positions, const at::Tensor& keys, const at::Tensor& values,
                               const at::Tensor& cosines, const at::Tensor& sines) {
    const int dt = dtype_code(k_cache);
    check_dim(k_cache, 4, "k_cache");
    check_dim(v_cache, 4, "v_cache");
    check_dim(block_tables, 2, "block_tables");
    check_dim(positions, 2, "positions");
    check_dim(keys, 4, "keys");
    check_dim(values, 4, "values");
    check_dim(cosines, 3, "cosines");
    check_dim(sines, 3, "sines");
    check_same(v_cache, k_cache, "v_cache");
    check_same(keys, k_cache, "keys");
    check_same(values, k_cache, "values");
    check_i32(block_tables, "block_tables");
    check_i32(positions, "positions");
    TORCH_CHECK(cosines.scalar_type() == at::kFloat || cosines.scalar_type() == k_cache.scalar_type(),
                "dvattn_paged_kv_append: cosines must be float32 or ", k_cache.scalar_type(), ", got ",
                cosines.scalar_type());
    check_same(sines, cosines, "sines");
    const at::Tensor* all[] = {&k_cache, &v_cache, &block_tables, &positions, &keys, &values, &cosines, &sines};
    const char* names[] = {"k_cache", "v_cache", "block_tables", "positions", "keys", "values", "cosines", "sines"};
    for (int i = 0; i < 8; ++i) check_dev(*all[i], k_cache, names[i]);
    check_contig(block_tables, "block_tables");
    check_contig(positions, "positions");
    for (int i : {0, 1, 4, 5})
        TORCH_CHECK(all[i]->size(3) <= 1 || all[i]->stride(3) == 1, "dvattn_paged_kv_append: the last dim of ",
                    names[i], " must be contiguous");
    for (int i : {6, 7})
        TORCH_CHECK(all[i]->size(2) <= 1 || all[i]->stride(2) == 1, "dvattn_paged_kv_append: the last dim of ",
                    names[i], " must be contiguous");
    const int64_t W = keys.size(0), Hkv = keys.size(1), S = keys.size(2), E = keys.size(3);
    const int64_t Ev = values.size(3);
    TORCH_CHECK(values.size(0) == W && values.size(1) == Hkv && values.size(2) == S,
                "dvattn_paged_kv_append: values must be [W,Hkv,S,Ev] = [", W, ",", Hkv, ",", S, ",Ev], got ",
                values.sizes());
    const int64_t P = k_cache.size(0), bs = k_cache.size(1);
    TORCH_CHECK(k_cache.size(2) == Hkv && k_cache.size(3) == E,
                "dvattn_paged_kv_append: k_cache must be [num_blocks, block_size, Hkv, E] with Hkv=", Hkv, ", E=", E,
                ", got ", k_cache.sizes());
    TORCH_CHECK(v_cache.size(0) == P && v_cache.size(1) == bs && v_cache.size(2) == Hkv && v_cache.size(3) == Ev,
                "dvattn_paged_kv_append: v_cache must be [num_blocks, block_size, Hkv, Ev], got ", v_cache.sizes());
    TORCH_CHECK(positions.size(0) == W && positions.size(1) == S, "dvattn_paged_kv_append: positions must be [W,S] = [",
                W, ",", S, "], got ", positions.sizes());
    TORCH_CHECK(block_tables.size(0) >= W, "dvattn_paged_kv_append: block_tables needs a row per sequence (", W,
                "), got ", block_tables.sizes());
    const int64_t R = cosines.size(2);
    TORCH_CHECK((cosines.size(0) == W || cosines.size(0) == 1) && (cosines.size(1) == S || cosines.size(1) == 1),
                "dvattn_paged_kv_append: cosines must be [W|1, S|1, R], got ", cosines.sizes());
    TORCH_CHECK(sines.sizes() == cosines.sizes(), "dvattn_paged_kv_append: sines must match cosines, got ",
                sines.sizes());
    TORCH_CHECK(R <= E && R % 2 == 0, "dvattn_paged_kv_append: rotary dim ", R, " must be even and <= E=", E);
    TORCH_CHECK(cosines.stride(0) == sines.stride(0) && cosines.stride(1) == sines.stride(1),
                "dvattn_paged_kv_append: cosines and sines must have the same strides");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(k_cache.device());
    dvattn_shape s{};
    s.W = as_int(W, "W");
    s.S = as_int(S, "S");
    s.Hkv = as_int(Hkv, "Hkv");
    s.E = as_int(E, "E");
    s.Ev = as_int(Ev, "Ev");
    s.block_size = as_int(bs, "block_size");
    s.max_blocks_per_seq = as_int(block_tables.size(1), "max_blocks_per_seq");
    s.num_blocks = as_int(P, "num_blocks");
    s.rotary_dim = as_int(R, "rotary_dim");
    dvattn_kv_layout lay{};
    for (int i = 0; i < 3; ++i) {
        lay.key_strides[i] = keys.stride(i);
        lay.value_strides[i] = values.stride(i);
        lay.k_cache_strides[i] = k_cache.stride(i);
        lay.v_cache_strides[i] = v_cache.stride(i);
    }
    lay.rope_strides[0] = cosines.size(0) == 1 ? 0 : cosines.stride(0);
    lay.rope_strides[1] = cosines.size(1) == 1 ? 0 : cosines.stride(1);
    const int rope_dt = cosines.scalar_type() == at::kFloat ? DVATTN_F32 : dt;
    check_status(dvattn_paged_kv_append(dt, rope_dt, k_cache.data_ptr(), v_cache.data_ptr(),
                                        block_tables.data_ptr<int>(), positions.data_ptr<int>(), keys.data_ptr(),
                                        values.data_ptr(), cosines.data_ptr(), sines.data_ptr(), &s, &lay,
                                        stream_of(k_cache)),
                 "dvattn_paged_kv_append");
}

// dvattn_view_metadata(Tensor(a!) locations, Tensor(b!) cosines, Tensor(c!) sines,
//   Tensor fragment_lengths, Tensor order, Tensor inv_freq, float attention_scaling,
//   ScalarType? round_to=None)        attention.py:158-186
void dvattn_view_metadata_op(at::Tensor& locations, at::Tensor& cosines, at::Tensor& sines,
                             const at::Tensor& fragment_lengths, const at::Tensor& order, const at::Tensor& inv_freq,
                             double attention_scaling, std::optional<at::ScalarType> round_to) {
    check_dim(locations, 3, "locations");
    check_dim(cosines, 4, "cosines");
    check_dim(sines, 4, "sines");
    check_dim(fragment_lengths, 1, "fragment_lengths");
    check_dim(order, 2, "order");
    check_dim(inv_freq, 1, "inv_freq");
    check_i32(locations, "locations");
    check_i32(fragment_lengths, "fragment_lengths");
    check_i32(order, "order");
    check_f32(cosines, "cosines");
    check_f32(sines, "sines");
    check_f32(inv_freq, "inv_freq");
    const at::Tensor* all[] = {&locations, &cosines, &sines, &fragment_lengths, &order, &inv_freq};
    const char* names[] = {"locations", "cosines", "sines", "fragment_lengths", "order", "inv_freq"};
    for (int i = 0; i < 6; ++i) {
        check_contig(*all[i], names[i]);
        check_dev(*all[i], locations, names[i]);
    }
    const int64_t F = locations.size(0), W = locations.size(1), S = locations.size(2), R = cosines.size(3);
    TORCH_CHECK(cosines.size(0) == F && cosines.size(1) == W && cosines.size(2) == S,
                "dvattn_view_metadata: cosines must be [F,W,S,R], got ", cosines.sizes());
    TORCH_CHECK(sines.sizes() == cosines.sizes(), "dvattn_view_metadata: sines must match cosines");
    TORCH_CHECK(fragment_lengths.size(0) == F, "dvattn_view_metadata: fragment_lengths must be [F], got ",
                fragment_lengths.sizes());
    TORCH_CHECK(order.size(0) == W && order.size(1) == F, "dvattn_view_metadata: order must be [W,F], got ",
                order.sizes());
    TORCH_CHECK(R % 2 == 0 && inv_freq.size(0) >= R / 2, "dvattn_view_metadata: need an even rotary dim and R/2 ",
                "inverse frequencies (R=", R, ", got ", inv_freq.size(0), ")");
    int rd = -1;
    if (round_to.has_value()) {
        switch (*round_to) {
            case at::kFloat: rd = -1; break;
            case at::kHalf: rd = DVATTN_F16; break;
            case at::kBFloat16: rd = DVATTN_BF16; break;
            default: TORCH_CHECK(false, "dvattn_view_metadata: round_to must be float32, float16 or bfloat16");
        }
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(locations.device());
    check_status(dvattn_view_metadata(locations.data_ptr<int>(), cosines.data_ptr<float>(), sines.data_ptr<float>(),
                                      fragment_lengths.data_ptr<int>(), order.data_ptr<int>(),
                                      inv_freq.data_ptr<float>(), (float)attention_scaling, rd, as_int(F, "F"),
                                      as_int(W, "W"), as_int(S, "S"), as_int(R, "rotary_dim"),
                                      stream_of(locations)),
                 "dvattn_view_metadata");
}

}  // namespace

TORCH_LIBRARY(libdvatt, m) {
    std::vector<at::Tag> tags;
    tags.push_back(at::Tag::needs_fixed_stride_order);
    m.def("dvattn_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries, "
          "Tensor fragment_lengths, Tensor[] key_fragments, Tensor[] value_fragments) -> ()",
          tags, torch::_RegisterOrVerify::REGISTER);
    m.def("dvattn_paged_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries, "
          "Tensor cosines, Tensor sines, Tensor fragment_lengths, Tensor k_cache, Tensor v_cache, "
          "Tensor block_tables) -> ()",
          tags, torch::_RegisterOrVerify::REGISTER);
    m.def("dvattn_rope(Tensor(a!) output, Tensor queries, Tensor cosines, Tensor sines) -> ()", tags,
          torch::_RegisterOrVerify::REGISTER);
    m.def("dvattn_fused(Tensor(a!) output, Tensor(b!) rq, float scale, Tensor locations, Tensor queries, "
          "Tensor fragment_lengths, Tensor[] key_fragments, Tensor[] value_fragments, Tensor cosines, "
          "Tensor sines) -> ()",
          tags, torch::_RegisterOrVerify::REGISTER);
    m.def("dvattn_varlen_rope(Tensor(a!) output, Tensor queries, Tensor cosines, Tensor sines) -> ()", tags,
          torch::_RegisterOrVerify::REGISTER);
    m.def("dvattn_varlen_paged_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries, "
          "Tensor cosines, Tensor sines, Tensor fragment_lengths, Tensor k_cache, Tensor v_cache, "
          "Tensor block_tables, Tensor cu_seqlens_q, Tensor cu_seqlens_k) -> ()",
          tags, torch::_RegisterOrVerify::REGISTER);
    // around the path: the reference does these in Python (attention.py:141-192, 245-251, 304)
    m.def("dvattn_paged_kv_append(Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor block_tables, "
          "Tensor positions, Tensor keys, Tensor values, Tensor cosines, Tensor sines) -> ()");
    m.def("dvattn_view_metadata(Tensor(a!) locations, Tensor(b!) cosines, Tensor(c!) sines, "
          "Tensor fragment_lengths, Tensor order, Tensor inv_freq, float attention_scaling, "
          "ScalarType? round_to=None) -> ()");
}

TORCH_LIBRARY_IMPL(libdvatt, CUDA, m) {
    m.impl("dvattn_sdpa", dvattn_sdpa_op);
    m.impl("dvattn_paged_sdpa", dvattn_paged_sdpa_op);
    m.impl("dvattn_rope", dvattn_rope_op);
    m.impl("dvattn_fused", dvattn_fused_op);
    m.impl("dvattn_varlen_rope", dvattn_varlen_rope_op);
    m.impl("dvattn_varlen_paged_sdpa", dvattn_varlen_paged_sdpa_op);
    m.impl("dvattn_paged_kv_append", dvattn_paged_kv_append_op);
    m.impl("dvattn_view_metadata", dvattn_view_metadata_op);
}
