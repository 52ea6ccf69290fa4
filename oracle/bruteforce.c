/*
 * Float64 brute-force restatement of the DVAttn attention semantics --
 * TEST INFRASTRUCTURE ONLY (a checker for oracle/dvattn_oracle.py on tiny
 * inputs; never linked into the product).
 *
 * Plain loops written from the reference kernels' index arithmetic rather than
 * from the vectorised oracle:
 *   - paged:  src/kernels/paged_kernel_v21.cuh:80-120 (view offset off_f,
 *             page = block_tables[w*maxB + p/bs], row = p%bs, K/V address
 *             ((page*bs + row)*Hkv + hkv)*E), :198 (off_f += L_f)
 *   - varlen: src/kernels/varlen_paged_kernel_v21.cuh:40-47 (token -> sequence),
 *             :75-80 (loc < 0 skips the view), :88 (q address)
 *   - contig: src/kernels/kernel_v21.cuh:84-114 (view f, batch w, head hkv:
 *             ((w*Hkv + hkv)*L + l)*E; batch stride 0 broadcasts one batch)
 * Scores are scale * <q, k>, one softmax over all visible keys of all views,
 * output = sum p v / sum p, all in double.  A row with no visible key gives 0
 * (paged_kernel_v21.cuh:318-345).
 *
 * Inputs are float arrays (K/V/q already converted from their storage type;
 * q already rotated per view).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int n;
    double mx;
    double sum;
    double* acc; /* Ev */
} row_state;

static void state_init(row_state* st, double* acc, int Ev) {
    st->n = 0;
    st->mx = -INFINITY;
    st->sum = 0.0;
    st->acc = acc;
    memset(acc, 0, sizeof(double) * (size_t)Ev);
}

static void state_add(row_state* st, double score, const float* v, int Ev) {
    if (score > st->mx) {
        double r = (st->n == 0) ? 0.0 : exp(st->mx - score);
        st->sum *= r;
        for (int e = 0; e < Ev; ++e) st->acc[e] *= r;
        st->mx = score;
    }
    double p = exp(score - st->mx);
    st->sum += p;
    for (int e = 0; e < Ev; ++e) st->acc[e] += p * (double)v[e];
    st->n++;
}

static void state_store(const row_state* st, double* out, int Ev) {
    for (int e = 0; e < Ev; ++e) out[e] = st->n ? st->acc[e] / st->sum : 0.0;
}

static double dot(const float* a, const float* b, int E) {
    double s = 0.0;
    for (int e = 0; e < E; ++e) s += (double)a[e] * (double)b[e];
    return s;
}

/* rq [F,W,Hq,S,E]; loc [F,W,S]; fl [F]; kc [P,bs,Hkv,E]; vc [P,bs,Hkv,Ev];
 * bt [W,maxB]; out [W,Hq,S,Ev] (double). Returns 0, or -1 on an index outside
 * block_tables / the page pool. */
int bf_paged(double* out, double scale, const int* loc, const float* rq, const int* fl,
             const float* kc, const float* vc, const int* bt,
             int F, int W, int Hq, int S, int E, int Ev, int P, int bs, int Hkv, int maxB) {
    int G = Hq / Hkv;
    double* acc = (double*)malloc(sizeof(double) * (size_t)Ev);
    for (int w = 0; w < W; ++w)
        for (int h = 0; h < Hq; ++h)
            for (int s = 0; s < S; ++s) {
                row_state st;
                state_init(&st, acc, Ev);
                long off = 0;
                for (int f = 0; f < F; ++f) {
                    int ql = loc[(f * W + w) * S + s];
                    int L = fl[f];
                    int maxL = L < ql + 1 ? L : ql + 1;
                    const float* q = rq + ((((long)f * W + w) * Hq + h) * S + s) * E;
                    for (int l = 0; l < maxL; ++l) {
                        long p = off + l;
                        long lp = p / bs;
                        if (lp >= maxB) { free(acc); return -1; }
                        int page = bt[(long)w * maxB + lp];
                        if (page < 0 || page >= P) { free(acc); return -1; }
                        long row = ((long)page * bs + p % bs) * Hkv + h / G;
                        state_add(&st, scale * dot(q, kc + row * E, E), vc + row * Ev, Ev);
                    }
                    off += L;
                }
                state_store(&st, out + (((long)w * Hq + h) * S + s) * Ev, Ev);
            }
    free(acc);
    return 0;
}

/* rq [F,T,Hq,E]; loc [F,T]; cu_q [W+1]; out [T,Hq,Ev]. */
int bf_varlen(double* out, double scale, const int* loc, const float* rq, const int* fl,
              const float* kc, const float* vc, const int* bt, const int* cu_q,
              int F, int T, int W, int Hq, int E, int Ev, int P, int bs, int Hkv, int maxB) {
    int G = Hq / Hkv;
    double* acc = (double*)malloc(sizeof(double) * (size_t)Ev);
    for (int t = 0; t < T; ++t) {
        int w = 0;
        for (int i = 0; i < W; ++i)
            if (t < cu_q[i + 1]) { w = i; break; }
        for (int h = 0; h < Hq; ++h) {
            row_state st;
            state_init(&st, acc, Ev);
            long off = 0;
            for (int f = 0; f < F; ++f) {
                int ql = loc[(long)f * T + t];
                int L = fl[f];
                if (ql < 0) { off += L; continue; }
                int maxL = L < ql + 1 ? L : ql + 1;
                const float* q = rq + (((long)f * T + t) * Hq + h) * E;
                for (int l = 0; l < maxL; ++l) {
                    long p = off + l;
                    long lp = p / bs;
                    if (lp >= maxB) { free(acc); return -1; }
                    int page = bt[(long)w * maxB + lp];
                    if (page < 0 || page >= P) { free(acc); return -1; }
                    long row = ((long)page * bs + p % bs) * Hkv + h / G;
                    state_add(&st, scale * dot(q, kc + row * E, E), vc + row * Ev, Ev);
                }
                off += L;
            }
            state_store(&st, out + ((long)t * Hq + h) * Ev, Ev);
        }
    }
    free(acc);
    return 0;
}

/* Contiguous views. kf/vf: concatenation of the F fragments (float);
 * frag_off[f]: element offset of fragment f in kf (and vf scaled by Ev/E via
 * vfrag_off); frag_L[f]: token dim of fragment f; frag_bstride[f]: 1 if the
 * fragment has one batch entry per sequence, 0 if one batch is shared.
 * rq [F,W,Hq,S,E]; loc [F,W,S]; fl [F] (mask bound); out [W,Hq,S,Ev]. */
int bf_contig(double* out, double scale, const int* loc, const float* rq, const int* fl,
              const float* kf, const float* vf, const long* kfrag_off, const long* vfrag_off,
              const int* frag_L, const int* frag_bstride,
              int F, int W, int Hq, int S, int E, int Ev, int Hkv) {
    int G = Hq / Hkv;
    double* acc = (double*)malloc(sizeof(double) * (size_t)Ev);
    for (int w = 0; w < W; ++w)
        for (int h = 0; h < Hq; ++h)
            for (int s = 0; s < S; ++s) {
                row_state st;
                state_init(&st, acc, Ev);
                for (int f = 0; f < F; ++f) {
                    int ql = loc[(f * W + w) * S + s];
                    int L = fl[f] < frag_L[f] ? fl[f] : frag_L[f];
                    int maxL = L < ql + 1 ? L : ql + 1;
                    const float* q = rq + ((((long)f * W + w) * Hq + h) * S + s) * E;
                    long b = frag_bstride[f] ? w : 0;
                    for (int l = 0; l < maxL; ++l) {
                        long krow = (b * Hkv + h / G) * (long)frag_L[f] + l;
                        state_add(&st, scale * dot(q, kf + kfrag_off[f] + krow * E, E),
                                  vf + vfrag_off[f] + krow * Ev, Ev);
                    }
                }
                state_store(&st, out + (((long)w * Hq + h) * S + s) * Ev, Ev);
            }
    free(acc);
    return 0;
}
