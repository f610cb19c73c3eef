/*
 * nacho_oracle.c — CPU restatement of the reference's kernels, used ONLY as a checker.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load this library; the product (nacho_amd) never links or calls it.
 *
 * What is restated (own code, following the reference's generated CPU target):
 *   - csr_union / csr_intersect: the CPU entry point of csr_add / csr_mul.  One merge-path
 *     partition per hardware thread (stitch_and_generate_cpu.cpp:26-31, 138-154), then a
 *     count pass, a serial exclusive scan over threads (156-215), result allocation with
 *     pos[0] zeroed (stitch_and_generate.cpp:438-527) and a write pass.  The partition is the
 *     reference's: count = t * per_thread_work with per_thread_work = total_work / T + 1 and
 *     total_work = nnzA + nnzB (stitch_and_generate.cpp:90-112); boundary threads take
 *     (0, -1, -1) / (rows, nnzA-1, nnzB-1) (partition.cpp:143-267, base_lowerer.cpp:79-110);
 *     otherwise a binary search over rows on the work functions (partition.cpp:586-811,
 *     tensor.cpp:162-440) followed by the balanced merge-path search inside the row
 *     (partition.cpp:813-993).  Positions stored are "last consumed" (pos - 1).  The compute
 *     pass walks rows start_i..end_i and merges with the union / intersection lattice
 *     (compute.cpp:25-149, 619-1388): coordinates ascending, a+b / a*b where both exist,
 *     copies otherwise (union only), explicit zeros kept, pos[i+1] written for every row a
 *     thread finishes.
 *   - coo_union / coo_intersect / coo3_union: the merged-coordinate lowering of COO
 *     (Compile.cpp:66-154, tensor.cpp:447-577): the same pipeline over one level whose
 *     coordinates are tuples compared lexicographically.
 *   - csf3_union: the three-level union lattice (for i in A_i ∪ B_i, for j in A_ij ∪ B_ij,
 *     for k in A_ijk ∪ B_ijk), emitted in lexicographic order; every coordinate of each
 *     level's union is appended, and its child range is the union below it (never empty for
 *     operands without empty fibres, which is what to_csf3 builds).  Serial restatement of
 *     the lattice; the reference's nested partitioning (partition.cpp:286-461) only splits
 *     this work among threads.
 *   - csr_add3: the three-way union lattice of csr_add_3 (compiler.cpp:114), row by row,
 *     values evaluated as (a + b) + c with absent operands removed.
 *   - dcsr_union / dcsr_intersect: the two-level lattice of dcsr_add / dcsr_mul
 *     (compiler.cpp:124-133): i over A_i ∪ B_i (add) or A_i ∩ B_i (mul), j over the union /
 *     intersection of the two fibres; a row id is emitted at every i lattice point, with its
 *     fibre, even when a product fibre is empty.  Serial restatement of the lattice.
 *   - sssmm: masked SpGEMM (GPU-only in the reference, compiler.cpp:150-153), row by row
 *     with a dense mask marker; products in ascending j, summed in float64.
 *   - csf3_inner / coo3_inner: the full reductions inner_prod and inner_prod_coo
 *     (compiler.cpp:141, 143): the intersection lattice at every level, float32 products
 *     summed in float64 (details at oracle_csf3_inner below).
 *   - spgemm: the reference has no CPU SpGEMM (compiler.cpp:145-148 is GPU-only).  This is
 *     the ESC semantics of its GPU path (stitch_and_generate_gpu.cpp:14-138, 257-366) run
 *     row-parallel on the CPU: per row, expand a_ij * b_jk, sort by k, and sum runs.
 *     Products are f32 (one IEEE multiply, as the reference), sums accumulate in f64 in
 *     ascending (j) order and are rounded to f32 once.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define ORC_OK 0
#define ORC_ENOMEM (-3)
#define ORC_EOVERFLOW (-2)

/* ---------------------------------------------------------------------------------- */
/* thread pool: run fn(t, arg) for t in [0, n) on n threads                              */

typedef void (*task_fn)(int t, void *arg);
typedef struct {
    task_fn fn;
    void *arg;
    int t;
} task;

static void *task_main(void *p) {
    task *k = (task *)p;
    k->fn(k->t, k->arg);
    return NULL;
}

static void parallel_for(int n, task_fn fn, void *arg) {
    if (n <= 1) {
        if (n == 1) fn(0, arg);
        return;
    }
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n);
    task *ks = (task *)malloc(sizeof(task) * (size_t)n);
    int started = 0;
    for (int t = 1; t < n; ++t) {
        ks[t].fn = fn;
        ks[t].arg = arg;
        ks[t].t = t;
        if (pthread_create(&th[t], NULL, task_main, &ks[t]) == 0) {
            ++started;
        } else {
            fn(t, arg); /* could not spawn: run inline */
            th[t] = 0;
        }
    }
    fn(0, arg);
    for (int t = 1; t < n; ++t)
        if (th[t]) pthread_join(th[t], NULL);
    (void)started;
    free(th);
    free(ks);
}

int oracle_default_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

void oracle_free(void *p) { free(p); }

/* ---------------------------------------------------------------------------------- */
/* CSR union / intersection                                                            */

typedef struct {
    /* operands */
    int rows;
    const int32_t *pa, *ca, *pb, *cb;
    const float *va, *vb;
    int nnz_a, nnz_b;
    int intersect;
    /* partition */
    int nthreads;
    long per_thread_work, total_work;
    int *part_i, *part_a, *part_b; /* last-consumed positions */
    long *count;                   /* per-thread output counts, then exclusive offsets */
    /* result */
    int32_t *pz, *cz;
    float *vz;
} csr_job;

/* Work of rows [0, i) in one operand: the reference's work_ij_<t>_dim_i(t, i - 1) =
 * pos[i] - pos[0] (tensor.cpp:162-440). */
static long csr_work_rows(const int32_t *pos, int i) { return (long)pos[i] - pos[0]; }

static void csr_partition(csr_job *J, int t) {
    const long count = (long)t * J->per_thread_work;
    if (count == 0) {
        J->part_i[t] = 0;
        J->part_a[t] = -1;
        J->part_b[t] = -1;
        return;
    }
    if (J->total_work <= count) {
        J->part_i[t] = J->rows;
        J->part_a[t] = J->nnz_a - 1;
        J->part_b[t] = J->nnz_b - 1;
        return;
    }
    /* Row search over the dense i level (not the last loop): mid = start + (end-start+1)/2,
     * work of the rows before mid; keep the largest row whose preceding work < count. */
    long rem = count;
    int start = -1, end = J->rows - 1, i = 0;
    for (;;) {
        const int mid = start + (end - start + 1) / 2;
        const long work = csr_work_rows(J->pa, mid) + csr_work_rows(J->pb, mid);
        if (end <= start) {
            i = mid;
            rem -= work;
            break;
        }
        if (work < rem) {
            start = mid;
        } else {
            end = mid - 1;
        }
    }
    /* Balanced merge-path inside row i over last-consumed positions. */
    const int t1s = J->pa[i] - 1, t1e = J->pa[i + 1] - 1;
    const int t2s = J->pb[i] - 1, t2e = J->pb[i + 1] - 1;
    const int32_t *A = J->ca, *B = J->cb;
    int sj = t1s, ej = t1e;
    int t1 = sj + (ej - sj + 1) / 2;
    int t2 = t2s + (int)(rem - (t1 - t1s));
    while (sj < ej) {
        t1 = sj + (ej - sj + 1) / 2;
        t2 = t2s + (int)(rem - (t1 - t1s));
        if (t2s <= t2 && t2 <= t2e) {
            if (t2s < t2 && t1 + 1 <= t1e && A[t1 + 1] < B[t2]) {
                sj = t1 + 1;
            } else if (t1s < t1 && t2 + 1 <= t2e && B[t2 + 1] < A[t1]) {
                ej = t1 - 1;
            } else {
                sj = t1;
                ej = t1;
            }
        } else if (t2e < t2) {
            sj = t1 + 1;
        } else {
            ej = t1 - 1;
        }
    }
    t1 = sj + (ej - sj + 1) / 2;
    t2 = t2s + (int)(rem - (t1 - t1s));
    /* keep an equal pair in one partition */
    if (t2s < t2 && t1 + 1 <= t1e && A[t1 + 1] == B[t2]) {
        t1 += 1;
    } else if (t1s < t1 && t2 + 1 <= t2e && B[t2 + 1] == A[t1]) {
        t2 += 1;
    }
    J->part_i[t] = i;
    J->part_a[t] = t1;
    J->part_b[t] = t2;
}

static void csr_partition_task(int t, void *arg) { csr_partition((csr_job *)arg, t); }

/* Walk thread t's share.  write == 0: count outputs.  write == 1: emit them at offset. */
static long csr_walk(csr_job *J, int t, int write) {
    const int T = J->nthreads;
    const int start_i = J->part_i[t];
    const int end_i = t < T - 1 ? J->part_i[t + 1] : J->rows;
    const int start_a = J->part_a[t] + 1, start_b = J->part_b[t] + 1;
    const int end_a = t < T - 1 ? J->part_a[t + 1] : J->nnz_a - 1; /* inclusive */
    const int end_b = t < T - 1 ? J->part_b[t + 1] : J->nnz_b - 1;
    long off = write ? J->count[t] : 0;
    const long off0 = off;
    for (int it = start_i; it <= end_i; ++it) {
        if (it == J->rows) break;
        int ia = (it == start_i) ? start_a : J->pa[it];
        int ib = (it == start_i) ? start_b : J->pb[it];
        const int sa = (it == end_i) ? end_a : J->pa[it + 1] - 1;
        const int sb = (it == end_i) ? end_b : J->pb[it + 1] - 1;
        while (ia <= sa && ib <= sb) {
            const int32_t aj = J->ca[ia], bj = J->cb[ib];
            const int32_t j = bj < aj ? bj : aj;
            if (j == aj && j == bj) {
                if (write) {
                    J->cz[off] = j;
                    J->vz[off] = J->intersect ? J->va[ia] * J->vb[ib] : J->va[ia] + J->vb[ib];
                }
                ++off;
            } else if (!J->intersect && j == aj) {
                if (write) {
                    J->cz[off] = j;
                    J->vz[off] = J->va[ia];
                }
                ++off;
            } else if (!J->intersect && j == bj) {
                if (write) {
                    J->cz[off] = j;
                    J->vz[off] = J->vb[ib];
                }
                ++off;
            }
            ia += (aj == j);
            ib += (bj == j);
        }
        if (!J->intersect) {
            for (; ia <= sa; ++ia) {
                if (write) {
                    J->cz[off] = J->ca[ia];
                    J->vz[off] = J->va[ia];
                }
                ++off;
            }
            for (; ib <= sb; ++ib) {
                if (write) {
                    J->cz[off] = J->cb[ib];
                    J->vz[off] = J->vb[ib];
                }
                ++off;
            }
        }
        if (write && it < end_i) J->pz[it + 1] = (int32_t)off;
    }
    return off - off0;
}

static void csr_count_task(int t, void *arg) {
    csr_job *J = (csr_job *)arg;
    J->count[t] = csr_walk(J, t, 0);
}

static void csr_write_task(int t, void *arg) { (void)csr_walk((csr_job *)arg, t, 1); }

/* Z = A (+|*) B over CSR.  Outputs are malloc'd (free with oracle_free).  Returns 0 or an
 * error code.  nthreads <= 0 means one per online CPU. */
int oracle_csr_binary(int intersect, int rows, const int32_t *pa, const int32_t *ca,
                      const float *va, int nnz_a, const int32_t *pb, const int32_t *cb,
                      const float *vb, int nnz_b, int nthreads, int32_t **out_pos,
                      int32_t **out_crd, float **out_val, int *out_nnz) {
    csr_job J;
    memset(&J, 0, sizeof(J));
    J.rows = rows;
    J.pa = pa;
    J.ca = ca;
    J.va = va;
    J.pb = pb;
    J.cb = cb;
    J.vb = vb;
    J.nnz_a = nnz_a;
    J.nnz_b = nnz_b;
    J.intersect = intersect;
    J.nthreads = nthreads > 0 ? nthreads : oracle_default_threads();
    J.total_work = (long)nnz_a + nnz_b;
    J.per_thread_work = J.total_work / J.nthreads + 1;
    const int T = J.nthreads;
    J.part_i = (int *)malloc(sizeof(int) * (size_t)T);
    J.part_a = (int *)malloc(sizeof(int) * (size_t)T);
    J.part_b = (int *)malloc(sizeof(int) * (size_t)T);
    J.count = (long *)malloc(sizeof(long) * (size_t)T);
    if (!J.part_i || !J.part_a || !J.part_b || !J.count) goto oom;

    parallel_for(T, csr_partition_task, &J);
    parallel_for(T, csr_count_task, &J);
    long total = 0;
    for (int t = 0; t < T; ++t) { /* serial exclusive scan over threads */
        const long c = J.count[t];
        J.count[t] = total;
        total += c;
    }
    if (total > 0x7fffffffL) {
        free(J.part_i);
        free(J.part_a);
        free(J.part_b);
        free(J.count);
        return ORC_EOVERFLOW;
    }
    J.pz = (int32_t *)malloc(sizeof(int32_t) * ((size_t)rows + 1));
    J.cz = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    J.vz = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    if (!J.pz || !J.cz || !J.vz) goto oom;
    if (total == 0) { /* empty result: zeroed offsets (stitch_and_generate.cpp:168-220) */
        memset(J.pz, 0, sizeof(int32_t) * ((size_t)rows + 1));
    }
    J.pz[0] = 0;
    if (total > 0) parallel_for(T, csr_write_task, &J);
    free(J.part_i);
    free(J.part_a);
    free(J.part_b);
    free(J.count);
    *out_pos = J.pz;
    *out_crd = J.cz;
    *out_val = J.vz;
    *out_nnz = (int)total;
    return ORC_OK;
oom:
    free(J.part_i);
    free(J.part_a);
    free(J.part_b);
    free(J.count);
    free(J.pz);
    free(J.cz);
    free(J.vz);
    return ORC_ENOMEM;
}

/* ---------------------------------------------------------------------------------- */
/* COO (merged coordinate) union / intersection over 2- or 3-tuples                      */

typedef struct {
    int arity; /* 2 or 3 */
    const int32_t *a[3], *b[3];
    const float *va, *vb;
    int nnz_a, nnz_b;
    int intersect;
    int nthreads;
    long per_thread_work, total_work;
    int *part_a, *part_b;
    long *count;
    int32_t *z[3];
    float *vz;
} coo_job;

/* lexicographic compare of A[x] and B[y] */
static int coo_cmp(const coo_job *J, int x, int y) {
    for (int d = 0; d < J->arity; ++d) {
        const int32_t p = J->a[d][x], q = J->b[d][y];
        if (p != q) return p < q ? -1 : 1;
    }
    return 0;
}

static void coo_partition(coo_job *J, int t) {
    const long count = (long)t * J->per_thread_work;
    if (count == 0) {
        J->part_a[t] = -1;
        J->part_b[t] = -1;
        return;
    }
    if (J->total_work <= count) {
        J->part_a[t] = J->nnz_a - 1;
        J->part_b[t] = J->nnz_b - 1;
        return;
    }
    const long rem = count;
    const int t1s = -1, t1e = J->nnz_a - 1, t2s = -1, t2e = J->nnz_b - 1;
    int sj = t1s, ej = t1e;
    int t1 = sj + (ej - sj + 1) / 2;
    int t2 = t2s + (int)(rem - (t1 - t1s));
    while (sj < ej) {
        t1 = sj + (ej - sj + 1) / 2;
        t2 = t2s + (int)(rem - (t1 - t1s));
        if (t2s <= t2 && t2 <= t2e) {
            if (t2s < t2 && t1 + 1 <= t1e && coo_cmp(J, t1 + 1, t2) < 0) {
                sj = t1 + 1;
            } else if (t1s < t1 && t2 + 1 <= t2e && coo_cmp(J, t1, t2 + 1) > 0) {
                ej = t1 - 1;
            } else {
                sj = t1;
                ej = t1;
            }
        } else if (t2e < t2) {
            sj = t1 + 1;
        } else {
            ej = t1 - 1;
        }
    }
    t1 = sj + (ej - sj + 1) / 2;
    t2 = t2s + (int)(rem - (t1 - t1s));
    if (t2s < t2 && t1 + 1 <= t1e && coo_cmp(J, t1 + 1, t2) == 0) {
        t1 += 1;
    } else if (t1s < t1 && t2 + 1 <= t2e && coo_cmp(J, t1, t2 + 1) == 0) {
        t2 += 1;
    }
    J->part_a[t] = t1;
    J->part_b[t] = t2;
}

static void coo_partition_task(int t, void *arg) { coo_partition((coo_job *)arg, t); }

static void coo_emit(coo_job *J, long off, const int32_t *const *src, int idx, float v) {
    for (int d = 0; d < J->arity; ++d) J->z[d][off] = src[d][idx];
    J->vz[off] = v;
}

static long coo_walk(coo_job *J, int t, int write) {
    const int T = J->nthreads;
    int ia = J->part_a[t] + 1, ib = J->part_b[t] + 1;
    const int sa = t < T - 1 ? J->part_a[t + 1] : J->nnz_a - 1;
    const int sb = t < T - 1 ? J->part_b[t + 1] : J->nnz_b - 1;
    long off = write ? J->count[t] : 0;
    const long off0 = off;
    while (ia <= sa && ib <= sb) {
        const int c = coo_cmp(J, ia, ib);
        if (c == 0) {
            if (write)
                coo_emit(J, off, J->a, ia,
                         J->intersect ? J->va[ia] * J->vb[ib] : J->va[ia] + J->vb[ib]);
            ++off;
            ++ia;
            ++ib;
        } else if (c < 0) {
            if (!J->intersect) {
                if (write) coo_emit(J, off, J->a, ia, J->va[ia]);
                ++off;
            }
            ++ia;
        } else {
            if (!J->intersect) {
                if (write) coo_emit(J, off, J->b, ib, J->vb[ib]);
                ++off;
            }
            ++ib;
        }
    }
    if (!J->intersect) {
        for (; ia <= sa; ++ia) {
            if (write) coo_emit(J, off, J->a, ia, J->va[ia]);
            ++off;
        }
        for (; ib <= sb; ++ib) {
            if (write) coo_emit(J, off, J->b, ib, J->vb[ib]);
            ++off;
        }
    }
    return off - off0;
}

static void coo_count_task(int t, void *arg) {
    coo_job *J = (coo_job *)arg;
    J->count[t] = coo_walk(J, t, 0);
}

static void coo_write_task(int t, void *arg) { (void)coo_walk((coo_job *)arg, t, 1); }

/* Z = A (+|*) B over COO tuples of `arity` (2 or 3) coordinates.  a_crd/b_crd hold `arity`
 * coordinate arrays; out_crd receives `arity` malloc'd arrays. */
int oracle_coo_binary(int intersect, int arity, const int32_t *const *a_crd, const float *va,
                      int nnz_a, const int32_t *const *b_crd, const float *vb, int nnz_b,
                      int nthreads, int32_t **out_crd, float **out_val, int *out_nnz) {
    coo_job J;
    memset(&J, 0, sizeof(J));
    if (arity < 1 || arity > 3) return -1;
    J.arity = arity;
    for (int d = 0; d < arity; ++d) {
        J.a[d] = a_crd[d];
        J.b[d] = b_crd[d];
    }
    J.va = va;
    J.vb = vb;
    J.nnz_a = nnz_a;
    J.nnz_b = nnz_b;
    J.intersect = intersect;
    J.nthreads = nthreads > 0 ? nthreads : oracle_default_threads();
    J.total_work = (long)nnz_a + nnz_b;
    J.per_thread_work = J.total_work / J.nthreads + 1;
    const int T = J.nthreads;
    J.part_a = (int *)malloc(sizeof(int) * (size_t)T);
    J.part_b = (int *)malloc(sizeof(int) * (size_t)T);
    J.count = (long *)malloc(sizeof(long) * (size_t)T);
    if (!J.part_a || !J.part_b || !J.count) goto oom;
    parallel_for(T, coo_partition_task, &J);
    parallel_for(T, coo_count_task, &J);
    long total = 0;
    for (int t = 0; t < T; ++t) {
        const long c = J.count[t];
        J.count[t] = total;
        total += c;
    }
    for (int d = 0; d < arity; ++d) {
        J.z[d] = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
        if (!J.z[d]) goto oom;
    }
    J.vz = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    if (!J.vz) goto oom;
    if (total > 0) parallel_for(T, coo_write_task, &J);
    free(J.part_a);
    free(J.part_b);
    free(J.count);
    for (int d = 0; d < arity; ++d) out_crd[d] = J.z[d];
    *out_val = J.vz;
    *out_nnz = (int)total;
    return ORC_OK;
oom:
    free(J.part_a);
    free(J.part_b);
    free(J.count);
    for (int d = 0; d < 3; ++d) free(J.z[d]);
    free(J.vz);
    return ORC_ENOMEM;
}

/* ---------------------------------------------------------------------------------- */
/* CSF3 union                                                                            */

typedef struct {
    int32_t *ci, *pj, *cj, *pk, *ck;
    float *v;
    long ni, nj, nk;
} csf_out;

/* Append the union of k-fibres A[ka0,ka1) and B[kb0,kb1); returns entries appended. */
static long csf_k_union(csf_out *o, const int32_t *ak, const float *av, int ka0, int ka1,
                        const int32_t *bk, const float *bv, int kb0, int kb1) {
    long n0 = o->nk;
    int x = ka0, y = kb0;
    while (x < ka1 && y < kb1) {
        if (ak[x] == bk[y]) {
            o->ck[o->nk] = ak[x];
            o->v[o->nk++] = av[x++] + bv[y++];
        } else if (ak[x] < bk[y]) {
            o->ck[o->nk] = ak[x];
            o->v[o->nk++] = av[x++];
        } else {
            o->ck[o->nk] = bk[y];
            o->v[o->nk++] = bv[y++];
        }
    }
    for (; x < ka1; ++x) {
        o->ck[o->nk] = ak[x];
        o->v[o->nk++] = av[x];
    }
    for (; y < kb1; ++y) {
        o->ck[o->nk] = bk[y];
        o->v[o->nk++] = bv[y];
    }
    return o->nk - n0;
}

/* Z = A + B over CSF3.  Inputs: (crd_i[ni], pos_j[ni+1], crd_j[nj], pos_k[nj+1], crd_k[nk],
 * val[nk]) per operand.  Output arrays are malloc'd with capacity ni_a+ni_b etc. */
int oracle_csf3_union(const int32_t *a_ci, int a_ni, const int32_t *a_pj, const int32_t *a_cj,
                      int a_nj, const int32_t *a_pk, const int32_t *a_ck, const float *a_v,
                      int a_nk, const int32_t *b_ci, int b_ni, const int32_t *b_pj,
                      const int32_t *b_cj, int b_nj, const int32_t *b_pk, const int32_t *b_ck,
                      const float *b_v, int b_nk, int32_t **o_ci, int32_t **o_pj,
                      int32_t **o_cj, int32_t **o_pk, int32_t **o_ck, float **o_v, int *o_ni,
                      int *o_nj, int *o_nk) {
    csf_out o;
    memset(&o, 0, sizeof(o));
    const size_t ci_cap = (size_t)a_ni + b_ni + 1, cj_cap = (size_t)a_nj + b_nj + 1,
                 ck_cap = (size_t)a_nk + b_nk + 1;
    o.ci = (int32_t *)malloc(sizeof(int32_t) * ci_cap);
    o.pj = (int32_t *)malloc(sizeof(int32_t) * (ci_cap + 1));
    o.cj = (int32_t *)malloc(sizeof(int32_t) * cj_cap);
    o.pk = (int32_t *)malloc(sizeof(int32_t) * (cj_cap + 1));
    o.ck = (int32_t *)malloc(sizeof(int32_t) * ck_cap);
    o.v = (float *)malloc(sizeof(float) * ck_cap);
    if (!o.ci || !o.pj || !o.cj || !o.pk || !o.ck || !o.v) {
        free(o.ci);
        free(o.pj);
        free(o.cj);
        free(o.pk);
        free(o.ck);
        free(o.v);
        return ORC_ENOMEM;
    }
    o.pj[0] = 0;
    o.pk[0] = 0;
    int ia = 0, ib = 0;
    while (ia < a_ni || ib < b_ni) {
        int i;
        int ha = ia < a_ni, hb = ib < b_ni;
        if (ha && hb) {
            i = a_ci[ia] < b_ci[ib] ? a_ci[ia] : b_ci[ib];
            ha = a_ci[ia] == i;
            hb = b_ci[ib] == i;
        } else {
            i = ha ? a_ci[ia] : b_ci[ib];
        }
        /* j-level union inside fibre i */
        int ja = ha ? a_pj[ia] : 0, jae = ha ? a_pj[ia + 1] : 0;
        int jb = hb ? b_pj[ib] : 0, jbe = hb ? b_pj[ib + 1] : 0;
        const long nj0 = o.nj;
        while (ja < jae || jb < jbe) {
            int j;
            int ga = ja < jae, gb = jb < jbe;
            if (ga && gb) {
                j = a_cj[ja] < b_cj[jb] ? a_cj[ja] : b_cj[jb];
                ga = a_cj[ja] == j;
                gb = b_cj[jb] == j;
            } else {
                j = ga ? a_cj[ja] : b_cj[jb];
            }
            csf_k_union(&o, a_ck, a_v, ga ? a_pk[ja] : 0, ga ? a_pk[ja + 1] : 0, b_ck, b_v,
                        gb ? b_pk[jb] : 0, gb ? b_pk[jb + 1] : 0);
            o.cj[o.nj++] = j;
            o.pk[o.nj] = (int32_t)o.nk;
            ja += ga;
            jb += gb;
        }
        (void)nj0;
        o.ci[o.ni++] = i;
        o.pj[o.ni] = (int32_t)o.nj;
        ia += ha;
        ib += hb;
    }
    *o_ci = o.ci;
    *o_pj = o.pj;
    *o_cj = o.cj;
    *o_pk = o.pk;
    *o_ck = o.ck;
    *o_v = o.v;
    *o_ni = (int)o.ni;
    *o_nj = (int)o.nj;
    *o_nk = (int)o.nk;
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------- */
/* CSR three-way union (csr_add_3)                                                       */

/* Z = A + B + C over CSR (compiler.cpp:114).  Per row, the lattice of a + b + c: every
 * coordinate of the three rows' union in ascending order, valued by the expression with the
 * absent operands removed, evaluated as written ((a + b) + c, compute.cpp:413-491):
 * (a + b) + c, a + b, a + c, b + c or a copy.  Serial.  Outputs are malloc'd. */
int oracle_csr_add3(int rows, const int32_t *pa, const int32_t *ca, const float *va,
                    const int32_t *pb, const int32_t *cb, const float *vb, const int32_t *pc,
                    const int32_t *cc, const float *vc, int32_t **o_pos, int32_t **o_crd,
                    float **o_val, int *o_nnz) {
    const size_t cap = (size_t)pa[rows] + pb[rows] + pc[rows] + 1;
    int32_t *pos = (int32_t *)malloc(sizeof(int32_t) * ((size_t)rows + 1));
    int32_t *crd = (int32_t *)malloc(sizeof(int32_t) * cap);
    float *val = (float *)malloc(sizeof(float) * cap);
    if (!pos || !crd || !val) {
        free(pos);
        free(crd);
        free(val);
        return ORC_ENOMEM;
    }
    long n = 0;
    pos[0] = 0;
    for (int r = 0; r < rows; ++r) {
        int x = pa[r], y = pb[r], z = pc[r];
        const int xe = pa[r + 1], ye = pb[r + 1], ze = pc[r + 1];
        while (x < xe || y < ye || z < ze) {
            int j = INT32_MAX;
            if (x < xe && ca[x] < j) j = ca[x];
            if (y < ye && cb[y] < j) j = cb[y];
            if (z < ze && cc[z] < j) j = cc[z];
            const int ha = x < xe && ca[x] == j, hb = y < ye && cb[y] == j,
                      hc = z < ze && cc[z] == j;
            float v;
            if (ha && hb) {
                v = va[x] + vb[y];
                if (hc) v = v + vc[z];
            } else if (ha) {
                v = hc ? va[x] + vc[z] : va[x];
            } else if (hb) {
                v = hc ? vb[y] + vc[z] : vb[y];
            } else {
                v = vc[z];
            }
            crd[n] = j;
            val[n++] = v;
            x += ha;
            y += hb;
            z += hc;
        }
        pos[r + 1] = (int32_t)n;
    }
    *o_pos = pos;
    *o_crd = crd;
    *o_val = val;
    *o_nnz = (int)n;
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------- */
/* DCSR union / intersection                                                             */

/* Z = A (+|*) B over DCSR (i and j both compressed).  Follows the generated loop nest of
 * dcsr_add / dcsr_mul (compiler.cpp:124-133): the i level co-iterates the two row-id lists
 * (union for add; for mul only the ids present in both), and at every such i lattice point
 * the j level merges the two fibres (union / intersection, compute.cpp:1169-1198), appends
 * the fibre and counts the row id whether or not the fibre is empty (compute.cpp:945-990).
 * Values: a + b or a copy (add), a * b (mul), one float32 operation each.  Inputs:
 * (crd_i[ni], pos_j[ni+1], crd_j[nj], val[nj]) per operand.  Outputs are malloc'd. */
int oracle_dcsr_binary(int intersect, const int32_t *a_ci, int a_ni, const int32_t *a_pj,
                       const int32_t *a_cj, const float *a_v, const int32_t *b_ci, int b_ni,
                       const int32_t *b_pj, const int32_t *b_cj, const float *b_v,
                       int32_t **o_ci, int32_t **o_pj, int32_t **o_cj, float **o_v,
                       int *o_ni, int *o_nj) {
    const int a_nj = a_pj[a_ni], b_nj = b_pj[b_ni];
    const size_t ci_cap = (size_t)a_ni + b_ni + 1, cj_cap = (size_t)a_nj + b_nj + 1;
    int32_t *ci = (int32_t *)malloc(sizeof(int32_t) * ci_cap);
    int32_t *pj = (int32_t *)malloc(sizeof(int32_t) * (ci_cap + 1));
    int32_t *cj = (int32_t *)malloc(sizeof(int32_t) * cj_cap);
    float *v = (float *)malloc(sizeof(float) * cj_cap);
    if (!ci || !pj || !cj || !v) {
        free(ci);
        free(pj);
        free(cj);
        free(v);
        return ORC_ENOMEM;
    }
    long ni = 0, nj = 0;
    pj[0] = 0;
    int ia = 0, ib = 0;
    while (intersect ? (ia < a_ni && ib < b_ni) : (ia < a_ni || ib < b_ni)) {
        int ha = ia < a_ni, hb = ib < b_ni;
        int i;
        if (ha && hb) {
            i = a_ci[ia] < b_ci[ib] ? a_ci[ia] : b_ci[ib];
            ha = a_ci[ia] == i;
            hb = b_ci[ib] == i;
        } else {
            i = ha ? a_ci[ia] : b_ci[ib];
        }
        if (!intersect || (ha && hb)) {
            int x = ha ? a_pj[ia] : 0, xe = ha ? a_pj[ia + 1] : 0;
            int y = hb ? b_pj[ib] : 0, ye = hb ? b_pj[ib + 1] : 0;
            while (x < xe && y < ye) {
                if (a_cj[x] == b_cj[y]) {
                    cj[nj] = a_cj[x];
                    v[nj++] = intersect ? a_v[x] * b_v[y] : a_v[x] + b_v[y];
                    ++x;
                    ++y;
                } else if (a_cj[x] < b_cj[y]) {
                    if (!intersect) {
                        cj[nj] = a_cj[x];
                        v[nj++] = a_v[x];
                    }
                    ++x;
                } else {
                    if (!intersect) {
                        cj[nj] = b_cj[y];
                        v[nj++] = b_v[y];
                    }
                    ++y;
                }
            }
            if (!intersect) {
                for (; x < xe; ++x) {
                    cj[nj] = a_cj[x];
                    v[nj++] = a_v[x];
                }
                for (; y < ye; ++y) {
                    cj[nj] = b_cj[y];
                    v[nj++] = b_v[y];
                }
            }
            ci[ni++] = i;
            pj[ni] = (int32_t)nj;
        }
        ia += ha;
        ib += hb;
    }
    *o_ci = ci;
    *o_pj = pj;
    *o_cj = cj;
    *o_v = v;
    *o_ni = (int)ni;
    *o_nj = (int)nj;
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------- */
/* SpGEMM (ESC semantics, row-parallel)                                                  */

typedef struct {
    int rows, cols;
    const int32_t *pa, *ca, *pb, *cb;
    const float *va, *vb;
    int nthreads;
    int64_t *row_nnz; /* symbolic: distinct k per row, then exclusive offsets */
    int64_t *pz;
    int32_t *cz;
    float *vz;
    int phase;
    /* dynamic schedule: rows are claimed SP_CHUNK at a time; on a cache line of its own */
    _Alignas(64) int next_row;
    _Alignas(64) int failed;
} sp_job;

/* One row per claim: on power-law inputs the heaviest rows sit next to each other (R-MAT
 * puts them at the lowest indices), and a chunk of several would hand them all to one
 * thread. */
#define SP_CHUNK 1

/* Per-thread dense accumulator over k (an SPA): the row's distinct columns are the keys of
 * the expanded products; emitting them in ascending k order is the sort + compress. */
typedef struct {
    double *acc;
    int32_t *mark; /* row id + 1 that last touched k */
    int32_t *keys;
} spa;

/* Ascending sort of n column ids in [0, cols): insertion sort for short rows, else an LSD
 * radix sort with 11-bit digits over the bits `cols` needs (tmp holds n entries). */
static void sort_keys(int32_t *keys, int32_t *tmp, int n, int cols) {
    if (n < 64) {
        for (int i = 1; i < n; ++i) {
            const int32_t v = keys[i];
            int j = i - 1;
            while (j >= 0 && keys[j] > v) {
                keys[j + 1] = keys[j];
                --j;
            }
            keys[j + 1] = v;
        }
        return;
    }
    int bits = 1;
    while (bits < 31 && (1L << bits) < cols) ++bits;
    int32_t *src = keys, *dst = tmp;
    for (int shift = 0; shift < bits; shift += 11) {
        int count[2049];
        memset(count, 0, sizeof(count));
        for (int i = 0; i < n; ++i) ++count[((src[i] >> shift) & 2047) + 1];
        for (int d = 0; d < 2048; ++d) count[d + 1] += count[d];
        for (int i = 0; i < n; ++i) dst[count[(src[i] >> shift) & 2047]++] = src[i];
        int32_t *t = src;
        src = dst;
        dst = t;
    }
    if (src != keys) memcpy(keys, src, sizeof(int32_t) * (size_t)n);
}

/* One row of Z: scatter the row's products into the accumulator (float32 products summed in
 * float64), then emit the distinct columns in ascending order (phase 1) or count them
 * (phase 0). */
static void sp_row(sp_job *J, spa *s, int32_t *tmp, int r) {
    /* the job's fields are read once: the shared row counter sits near them, and other
     * threads' claims would otherwise invalidate the line under this loop */
    const int32_t *const pb = J->pb, *const cb = J->cb;
    const float *const vb = J->vb;
    const int phase = J->phase;
    int32_t *const mark = s->mark, *const keys = s->keys;
    double *const acc = s->acc;
    int nkeys = 0;
    for (int p = J->pa[r]; p < J->pa[r + 1]; ++p) {
        const int j = J->ca[p];
        const float a = J->va[p];
        for (int q = pb[j]; q < pb[j + 1]; ++q) {
            const int k = cb[q];
            if (mark[k] != r + 1) {
                mark[k] = r + 1;
                acc[k] = 0.0;
                keys[nkeys++] = k;
            }
            if (phase == 1) acc[k] += (double)(a * vb[q]); /* f32 product */
        }
    }
    if (phase == 0) {
        J->row_nnz[r] = nkeys;
        return;
    }
    sort_keys(s->keys, tmp, nkeys, J->cols);
    int64_t off = J->pz[r];
    for (int x = 0; x < nkeys; ++x) {
        J->cz[off] = s->keys[x];
        J->vz[off] = (float)s->acc[s->keys[x]];
        ++off;
    }
}

/* Rows are claimed dynamically in chunks (row costs are very uneven on power-law inputs). */
static void sp_task(int t, void *arg) {
    sp_job *J = (sp_job *)arg;
    (void)t;
    spa s;
    const size_t n = (size_t)J->cols + 1;
    s.acc = (double *)calloc(n, sizeof(double));
    s.mark = (int32_t *)calloc(n, sizeof(int32_t));
    s.keys = (int32_t *)malloc(sizeof(int32_t) * n);
    int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * n);
    if (!s.acc || !s.mark || !s.keys || !tmp) {
        __atomic_store_n(&J->failed, 1, __ATOMIC_RELAXED);
    } else {
        for (;;) {
            const int r0 = __atomic_fetch_add(&J->next_row, SP_CHUNK, __ATOMIC_RELAXED);
            if (r0 >= J->rows) break;
            const int r1 = r0 + SP_CHUNK < J->rows ? r0 + SP_CHUNK : J->rows;
            for (int r = r0; r < r1; ++r) sp_row(J, &s, tmp, r);
        }
    }
    free(s.acc);
    free(s.mark);
    free(s.keys);
    free(tmp);
}

/* Z = A B (rows x cols result).  Offsets are int64.  Returns 0 or error. */
int oracle_spgemm(int rows, int inner, int cols, const int32_t *pa, const int32_t *ca,
                  const float *va, const int32_t *pb, const int32_t *cb, const float *vb,
                  int nthreads, int64_t **out_pos, int32_t **out_crd, float **out_val,
                  int64_t *out_nnz) {
    (void)inner;
    sp_job J;
    memset(&J, 0, sizeof(J));
    J.rows = rows;
    J.cols = cols;
    J.pa = pa;
    J.ca = ca;
    J.va = va;
    J.pb = pb;
    J.cb = cb;
    J.vb = vb;
    J.nthreads = nthreads > 0 ? nthreads : oracle_default_threads();
    J.row_nnz = (int64_t *)malloc(sizeof(int64_t) * ((size_t)rows + 1));
    J.pz = (int64_t *)malloc(sizeof(int64_t) * ((size_t)rows + 1));
    if (!J.row_nnz || !J.pz) {
        free(J.row_nnz);
        free(J.pz);
        return ORC_ENOMEM;
    }
    J.phase = 0; /* symbolic */
    J.next_row = 0;
    parallel_for(J.nthreads, sp_task, &J);
    if (J.failed) {
        free(J.row_nnz);
        free(J.pz);
        return ORC_ENOMEM;
    }
    int64_t total = 0;
    for (int r = 0; r < rows; ++r) {
        J.pz[r] = total;
        total += J.row_nnz[r];
    }
    J.pz[rows] = total;
    J.cz = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    J.vz = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    if (!J.cz || !J.vz) {
        free(J.row_nnz);
        free(J.pz);
        free(J.cz);
        free(J.vz);
        return ORC_ENOMEM;
    }
    J.phase = 1; /* numeric */
    J.next_row = 0;
    parallel_for(J.nthreads, sp_task, &J);
    free(J.row_nnz);
    if (J.failed) {
        free(J.pz);
        free(J.cz);
        free(J.vz);
        return ORC_ENOMEM;
    }
    *out_pos = J.pz;
    *out_crd = J.cz;
    *out_val = J.vz;
    *out_nnz = total;
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------- */
/* Masked SpGEMM (sssmm)                                                                 */

/* Z_ik = sum_j a_ij * b_jk * c_ik for the (i, k) stored in C that at least one product
 * reaches (compiler.cpp:150-153; GPU-only in the reference, whose benchmark checks the
 * structure against cuSPARSE A*B followed by csr_mul with C, benchmarks/sssmm.py:46-51).
 * Row by row: the row's mask entries are marked in a dense array over k; every product
 * a_ij * b_jk (j ascending) that lands on a marked k adds (a_ij * b_jk) * c_ik, each product
 * rounded to float32 as written, to a float64 accumulator; the reached entries are emitted
 * in C's order with the sum rounded to float32. */
typedef struct {
    int rows, cols;
    const int32_t *pa, *ca, *pb, *cb, *pc, *cc;
    const float *va, *vb, *vc;
    const int32_t *row_list; /* rows to compute (NULL = all) */
    int n_list;
    int phase;
    int64_t *row_nnz;
    int64_t *pz;
    int32_t *cz;
    float *vz;
    _Alignas(64) int next; /* row claim counter, on a cache line of its own */
    _Alignas(64) int failed;
} ms_job;

static void ms_row(ms_job *J, int32_t *mark, double *acc, char *hit, int r) {
    const int c0 = J->pc[r], c1 = J->pc[r + 1];
    for (int q = c0; q < c1; ++q) {
        mark[J->cc[q]] = q - c0 + 1;
        acc[q - c0] = 0.0;
        hit[q - c0] = 0;
    }
    const int32_t *const pb = J->pb, *const cb = J->cb;
    const float *const vb = J->vb, *const vc = J->vc;
    for (int p = J->pa[r]; p < J->pa[r + 1]; ++p) {
        const int j = J->ca[p];
        const float a = J->va[p];
        for (int q = pb[j]; q < pb[j + 1]; ++q) {
            const int m = mark[cb[q]];
            if (m) {
                const float ab = a * vb[q];
                acc[m - 1] += (double)(ab * vc[c0 + m - 1]);
                hit[m - 1] = 1;
            }
        }
    }
    int64_t n = 0;
    int64_t off = J->phase == 1 ? J->pz[r] : 0;
    for (int q = c0; q < c1; ++q) {
        mark[J->cc[q]] = 0;
        if (hit[q - c0]) {
            if (J->phase == 1) {
                J->cz[off] = J->cc[q];
                J->vz[off] = (float)acc[q - c0];
                ++off;
            }
            ++n;
        }
    }
    if (J->phase == 0) J->row_nnz[r] = n;
}

static void ms_task(int t, void *arg) {
    ms_job *J = (ms_job *)arg;
    (void)t;
    int max_c = 1;
    for (int r = 0; r < J->rows; ++r) {
        const int len = J->pc[r + 1] - J->pc[r];
        if (len > max_c) max_c = len;
    }
    int32_t *mark = (int32_t *)calloc((size_t)J->cols + 1, sizeof(int32_t));
    double *acc = (double *)malloc(sizeof(double) * (size_t)max_c);
    char *hit = (char *)malloc((size_t)max_c);
    if (!mark || !acc || !hit) {
        __atomic_store_n(&J->failed, 1, __ATOMIC_RELAXED);
    } else {
        const int n = J->row_list ? J->n_list : J->rows;
        for (;;) {
            const int x0 = __atomic_fetch_add(&J->next, SP_CHUNK, __ATOMIC_RELAXED);
            if (x0 >= n) break;
            const int x1 = x0 + SP_CHUNK < n ? x0 + SP_CHUNK : n;
            for (int x = x0; x < x1; ++x) ms_row(J, mark, acc, hit, J->row_list ? J->row_list[x] : x);
        }
    }
    free(mark);
    free(acc);
    free(hit);
}

/* Z = (A B) masked by C, valued as above (rows x cols).  `row_list` (n_list rows, may be
 * NULL for all rows) restricts the work to those rows; the other rows of Z are empty.
 * Returns 0 or an error. */
int oracle_sssmm(int rows, int cols, const int32_t *pa, const int32_t *ca, const float *va,
                 const int32_t *pb, const int32_t *cb, const float *vb, const int32_t *pc,
                 const int32_t *cc, const float *vc, const int32_t *row_list, int n_list,
                 int nthreads, int32_t **out_pos, int32_t **out_crd, float **out_val,
                 int *out_nnz) {
    ms_job J;
    memset(&J, 0, sizeof(J));
    J.rows = rows;
    J.cols = cols;
    J.pa = pa;
    J.ca = ca;
    J.va = va;
    J.pb = pb;
    J.cb = cb;
    J.vb = vb;
    J.pc = pc;
    J.cc = cc;
    J.vc = vc;
    J.row_list = row_list;
    J.n_list = n_list;
    const int nt = nthreads > 0 ? nthreads : oracle_default_threads();
    J.row_nnz = (int64_t *)calloc((size_t)rows + 1, sizeof(int64_t));
    J.pz = (int64_t *)malloc(sizeof(int64_t) * ((size_t)rows + 1));
    int32_t *pos = (int32_t *)malloc(sizeof(int32_t) * ((size_t)rows + 1));
    if (!J.row_nnz || !J.pz || !pos) {
        free(J.row_nnz);
        free(J.pz);
        free(pos);
        return ORC_ENOMEM;
    }
    J.phase = 0;
    parallel_for(nt, ms_task, &J);
    int64_t total = 0;
    for (int r = 0; r < rows; ++r) {
        J.pz[r] = total;
        total += J.row_nnz[r];
    }
    J.pz[rows] = total;
    J.cz = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    J.vz = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    if (J.failed || !J.cz || !J.vz || total > INT32_MAX) {
        free(J.row_nnz);
        free(J.pz);
        free(pos);
        free(J.cz);
        free(J.vz);
        return J.failed || !J.cz || !J.vz ? ORC_ENOMEM : ORC_EOVERFLOW;
    }
    J.phase = 1;
    J.next = 0;
    parallel_for(nt, ms_task, &J);
    for (int r = 0; r <= rows; ++r) pos[r] = (int32_t)J.pz[r];
    free(J.row_nnz);
    free(J.pz);
    if (J.failed) {
        free(pos);
        free(J.cz);
        free(J.vz);
        return ORC_ENOMEM;
    }
    *out_pos = pos;
    *out_crd = J.cz;
    *out_val = J.vz;
    *out_nnz = (int)total;
    return ORC_OK;
}


/* ---------------------------------------------------------------------------------- */
/* Thread-parallel restatements of the serial lattices above (CPU baselines)            */
/*
 * The reference's CPU target runs one partition per hardware thread: a partition pass, a
 * count pass, a serial prefix of the counts, and a write pass (stitch_and_generate_cpu.cpp:
 * 26-31, 138-154).  These follow that structure for CSF3 union, DCSR union / intersection
 * and the three-way CSR union: the outermost level is cut into `nthreads` ranges of about
 * equal nonzero count (ranges never split a coordinate present in both operands), each
 * thread counts its range's outputs, a serial exclusive scan turns counts into offsets, and
 * each thread writes its range at its offsets.  The results are identical to the serial
 * functions' (tests/test_oracle_mt.py checks it).
 */

typedef struct {
    int ia0, ia1, ib0, ib1; /* top-level ranges of A and B (or rows: ia only)          */
    long n[3];              /* per-level output counts, then exclusive offsets          */
} top_range;

/* Cut the merged top-level id lists into `nt` ranges of about equal weight.  wa(i) / wb(i)
 * give the weight of A's / B's i-th fibre (pos arrays of the level holding the nonzeros). */
static void split_top(const int32_t *a_ci, int a_ni, const long *wa_pos, const int32_t *b_ci,
                      int b_ni, const long *wb_pos, int nt, top_range *r) {
    const long total = (a_ni ? wa_pos[a_ni] - wa_pos[0] : 0) +
                       (b_ni ? wb_pos[b_ni] - wb_pos[0] : 0) + (long)a_ni + b_ni;
    int ia = 0, ib = 0, t = 0;
    long acc = 0;
    r[0].ia0 = 0;
    r[0].ib0 = 0;
    while (ia < a_ni || ib < b_ni) {
        int ha = ia < a_ni, hb = ib < b_ni;
        if (ha && hb) {
            const int i = a_ci[ia] < b_ci[ib] ? a_ci[ia] : b_ci[ib];
            ha = a_ci[ia] == i;
            hb = b_ci[ib] == i;
        }
        if (ha) acc += wa_pos[ia + 1] - wa_pos[ia] + 1;
        if (hb) acc += wb_pos[ib + 1] - wb_pos[ib] + 1;
        ia += ha;
        ib += hb;
        while (t + 1 < nt && acc * nt >= total * (long)(t + 1)) {
            r[t].ia1 = ia;
            r[t].ib1 = ib;
            ++t;
            r[t].ia0 = ia;
            r[t].ib0 = ib;
        }
    }
    for (; t < nt; ++t) {
        r[t].ia1 = a_ni;
        r[t].ib1 = b_ni;
        if (t + 1 < nt) {
            r[t + 1].ia0 = a_ni;
            r[t + 1].ib0 = b_ni;
        }
    }
}

static void exclusive_offsets(top_range *r, int nt, int levels, long *totals) {
    for (int d = 0; d < levels; ++d) {
        long run = 0;
        for (int t = 0; t < nt; ++t) {
            const long c = r[t].n[d];
            r[t].n[d] = run;
            run += c;
        }
        totals[d] = run;
    }
}

/* -- CSF3 union ----------------------------------------------------------------------- */

typedef struct {
    const int32_t *ci, *pj, *cj, *pk, *ck;
    const float *v;
    int ni;
} csf_in;

typedef struct {
    const csf_in *A, *B;
    top_range *r;
    csf_out o; /* shared output arrays (write pass) */
    int write;
} csf_mt_job;

/* The serial CSF3 union loop over one top-level range, counting (write == 0) or writing at
 * the range's offsets. */
static void csf_union_range(csf_mt_job *J, int t) {
    const csf_in *A = J->A, *B = J->B;
    top_range *rg = &J->r[t];
    long ni = J->write ? rg->n[0] : 0, nj = J->write ? rg->n[1] : 0, nk = J->write ? rg->n[2] : 0;
    csf_out *o = &J->o;
    int ia = rg->ia0, ib = rg->ib0;
    while (ia < rg->ia1 || ib < rg->ib1) {
        int ha = ia < rg->ia1, hb = ib < rg->ib1, i;
        if (ha && hb) {
            i = A->ci[ia] < B->ci[ib] ? A->ci[ia] : B->ci[ib];
            ha = A->ci[ia] == i;
            hb = B->ci[ib] == i;
        } else {
            i = ha ? A->ci[ia] : B->ci[ib];
        }
        int ja = ha ? A->pj[ia] : 0, jae = ha ? A->pj[ia + 1] : 0;
        int jb = hb ? B->pj[ib] : 0, jbe = hb ? B->pj[ib + 1] : 0;
        while (ja < jae || jb < jbe) {
            int ga = ja < jae, gb = jb < jbe, j;
            if (ga && gb) {
                j = A->cj[ja] < B->cj[jb] ? A->cj[ja] : B->cj[jb];
                ga = A->cj[ja] == j;
                gb = B->cj[jb] == j;
            } else {
                j = ga ? A->cj[ja] : B->cj[jb];
            }
            int x = ga ? A->pk[ja] : 0, xe = ga ? A->pk[ja + 1] : 0;
            int y = gb ? B->pk[jb] : 0, ye = gb ? B->pk[jb + 1] : 0;
            while (x < xe || y < ye) {
                const int hx = x < xe, hy = y < ye;
                const int k = (hx && (!hy || A->ck[x] <= B->ck[y])) ? A->ck[x] : B->ck[y];
                const int ux = hx && A->ck[x] == k, uy = hy && B->ck[y] == k;
                if (J->write) {
                    o->ck[nk] = k;
                    o->v[nk] = ux && uy ? A->v[x] + B->v[y] : (ux ? A->v[x] : B->v[y]);
                }
                ++nk;
                x += ux;
                y += uy;
            }
            if (J->write) {
                o->cj[nj] = j;
                o->pk[nj + 1] = (int32_t)nk;
            }
            ++nj;
            ja += ga;
            jb += gb;
        }
        if (J->write) {
            o->ci[ni] = i;
            o->pj[ni + 1] = (int32_t)nj;
        }
        ++ni;
        ia += ha;
        ib += hb;
    }
    if (!J->write) {
        rg->n[0] = ni;
        rg->n[1] = nj;
        rg->n[2] = nk;
    }
}

static void csf_union_task(int t, void *arg) { csf_union_range((csf_mt_job *)arg, t); }

/* The same result as oracle_csf3_union, on `nthreads` threads (0: all online cores). */
int oracle_csf3_union_mt(const int32_t *a_ci, int a_ni, const int32_t *a_pj,
                         const int32_t *a_cj, int a_nj, const int32_t *a_pk,
                         const int32_t *a_ck, const float *a_v, int a_nk, const int32_t *b_ci,
                         int b_ni, const int32_t *b_pj, const int32_t *b_cj, int b_nj,
                         const int32_t *b_pk, const int32_t *b_ck, const float *b_v, int b_nk,
                         int nthreads, int32_t **o_ci, int32_t **o_pj, int32_t **o_cj,
                         int32_t **o_pk, int32_t **o_ck, float **o_v, int *o_ni, int *o_nj,
                         int *o_nk) {
    (void)a_nj;
    (void)b_nj;
    (void)a_nk;
    (void)b_nk;
    const int nt = nthreads > 0 ? nthreads : oracle_default_threads();
    const csf_in A = {a_ci, a_pj, a_cj, a_pk, a_ck, a_v, a_ni};
    const csf_in B = {b_ci, b_pj, b_cj, b_pk, b_ck, b_v, b_ni};
    /* weight of a top-level fibre: its k entries, from pos_k at the fibre's j range */
    long *wa = (long *)malloc(sizeof(long) * ((size_t)a_ni + 1));
    long *wb = (long *)malloc(sizeof(long) * ((size_t)b_ni + 1));
    top_range *r = (top_range *)calloc((size_t)nt, sizeof(top_range));
    if (!wa || !wb || !r) {
        free(wa);
        free(wb);
        free(r);
        return ORC_ENOMEM;
    }
    for (int i = 0; i <= a_ni; ++i) wa[i] = a_pk[a_pj[i]];
    for (int i = 0; i <= b_ni; ++i) wb[i] = b_pk[b_pj[i]];
    split_top(a_ci, a_ni, wa, b_ci, b_ni, wb, nt, r);
    free(wa);
    free(wb);
    csf_mt_job J;
    memset(&J, 0, sizeof(J));
    J.A = &A;
    J.B = &B;
    J.r = r;
    parallel_for(nt, csf_union_task, &J);
    long tot[3];
    exclusive_offsets(r, nt, 3, tot);
    J.o.ci = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[0] + 1));
    J.o.pj = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[0] + 1));
    J.o.cj = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[1] + 1));
    J.o.pk = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[1] + 1));
    J.o.ck = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[2] + 1));
    J.o.v = (float *)malloc(sizeof(float) * ((size_t)tot[2] + 1));
    if (!J.o.ci || !J.o.pj || !J.o.cj || !J.o.pk || !J.o.ck || !J.o.v) {
        free(J.o.ci);
        free(J.o.pj);
        free(J.o.cj);
        free(J.o.pk);
        free(J.o.ck);
        free(J.o.v);
        free(r);
        return ORC_ENOMEM;
    }
    J.o.pj[0] = 0;
    J.o.pk[0] = 0;
    J.write = 1;
    parallel_for(nt, csf_union_task, &J);
    free(r);
    *o_ci = J.o.ci;
    *o_pj = J.o.pj;
    *o_cj = J.o.cj;
    *o_pk = J.o.pk;
    *o_ck = J.o.ck;
    *o_v = J.o.v;
    *o_ni = (int)tot[0];
    *o_nj = (int)tot[1];
    *o_nk = (int)tot[2];
    return ORC_OK;
}

/* -- DCSR union / intersection --------------------------------------------------------- */

typedef struct {
    const int32_t *a_ci, *a_pj, *a_cj, *b_ci, *b_pj, *b_cj;
    const float *a_v, *b_v;
    int intersect, write;
    top_range *r;
    int32_t *ci, *pj, *cj;
    float *v;
} dcsr_mt_job;

static void dcsr_range(dcsr_mt_job *J, int t) {
    top_range *rg = &J->r[t];
    long ni = J->write ? rg->n[0] : 0, nj = J->write ? rg->n[1] : 0;
    int ia = rg->ia0, ib = rg->ib0;
    const int X = J->intersect;
    while (X ? (ia < rg->ia1 && ib < rg->ib1) : (ia < rg->ia1 || ib < rg->ib1)) {
        int ha = ia < rg->ia1, hb = ib < rg->ib1, i;
        if (ha && hb) {
            i = J->a_ci[ia] < J->b_ci[ib] ? J->a_ci[ia] : J->b_ci[ib];
            ha = J->a_ci[ia] == i;
            hb = J->b_ci[ib] == i;
        } else {
            i = ha ? J->a_ci[ia] : J->b_ci[ib];
        }
        if (!X || (ha && hb)) {
            int x = ha ? J->a_pj[ia] : 0, xe = ha ? J->a_pj[ia + 1] : 0;
            int y = hb ? J->b_pj[ib] : 0, ye = hb ? J->b_pj[ib + 1] : 0;
            while (X ? (x < xe && y < ye) : (x < xe || y < ye)) {
                const int hx = x < xe, hy = y < ye;
                const int j = (hx && (!hy || J->a_cj[x] <= J->b_cj[y])) ? J->a_cj[x] : J->b_cj[y];
                const int ux = hx && J->a_cj[x] == j, uy = hy && J->b_cj[y] == j;
                if (!X || (ux && uy)) {
                    if (J->write) {
                        J->cj[nj] = j;
                        J->v[nj] = ux && uy ? (X ? J->a_v[x] * J->b_v[y] : J->a_v[x] + J->b_v[y])
                                            : (ux ? J->a_v[x] : J->b_v[y]);
                    }
                    ++nj;
                }
                x += ux;
                y += uy;
            }
            if (J->write) {
                J->ci[ni] = i;
                J->pj[ni + 1] = (int32_t)nj;
            }
            ++ni;
        }
        ia += ha;
        ib += hb;
    }
    if (!J->write) {
        rg->n[0] = ni;
        rg->n[1] = nj;
    }
}

static void dcsr_task(int t, void *arg) { dcsr_range((dcsr_mt_job *)arg, t); }

/* The same result as oracle_dcsr_binary, on `nthreads` threads (0: all online cores). */
int oracle_dcsr_binary_mt(int intersect, const int32_t *a_ci, int a_ni, const int32_t *a_pj,
                          const int32_t *a_cj, const float *a_v, const int32_t *b_ci, int b_ni,
                          const int32_t *b_pj, const int32_t *b_cj, const float *b_v,
                          int nthreads, int32_t **o_ci, int32_t **o_pj, int32_t **o_cj,
                          float **o_v, int *o_ni, int *o_nj) {
    const int nt = nthreads > 0 ? nthreads : oracle_default_threads();
    long *wa = (long *)malloc(sizeof(long) * ((size_t)a_ni + 1));
    long *wb = (long *)malloc(sizeof(long) * ((size_t)b_ni + 1));
    top_range *r = (top_range *)calloc((size_t)nt, sizeof(top_range));
    if (!wa || !wb || !r) {
        free(wa);
        free(wb);
        free(r);
        return ORC_ENOMEM;
    }
    for (int i = 0; i <= a_ni; ++i) wa[i] = a_pj[i];
    for (int i = 0; i <= b_ni; ++i) wb[i] = b_pj[i];
    split_top(a_ci, a_ni, wa, b_ci, b_ni, wb, nt, r);
    free(wa);
    free(wb);
    dcsr_mt_job J;
    memset(&J, 0, sizeof(J));
    J.a_ci = a_ci;
    J.a_pj = a_pj;
    J.a_cj = a_cj;
    J.a_v = a_v;
    J.b_ci = b_ci;
    J.b_pj = b_pj;
    J.b_cj = b_cj;
    J.b_v = b_v;
    J.intersect = intersect;
    J.r = r;
    parallel_for(nt, dcsr_task, &J);
    long tot[2];
    exclusive_offsets(r, nt, 2, tot);
    J.ci = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[0] + 1));
    J.pj = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[0] + 1));
    J.cj = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[1] + 1));
    J.v = (float *)malloc(sizeof(float) * ((size_t)tot[1] + 1));
    if (!J.ci || !J.pj || !J.cj || !J.v) {
        free(J.ci);
        free(J.pj);
        free(J.cj);
        free(J.v);
        free(r);
        return ORC_ENOMEM;
    }
    J.pj[0] = 0;
    J.write = 1;
    parallel_for(nt, dcsr_task, &J);
    free(r);
    *o_ci = J.ci;
    *o_pj = J.pj;
    *o_cj = J.cj;
    *o_v = J.v;
    *o_ni = (int)tot[0];
    *o_nj = (int)tot[1];
    return ORC_OK;
}

/* -- three-way CSR union --------------------------------------------------------------- */

typedef struct {
    int rows;
    const int32_t *pa, *ca, *pb, *cb, *pc, *cc;
    const float *va, *vb, *vc;
    int write;
    top_range *r; /* ia0/ia1 = row range */
    int32_t *pos, *crd;
    float *val;
} add3_mt_job;

static void add3_range(add3_mt_job *J, int t) {
    top_range *rg = &J->r[t];
    long n = J->write ? rg->n[0] : 0;
    for (int row = rg->ia0; row < rg->ia1; ++row) {
        int x = J->pa[row], y = J->pb[row], z = J->pc[row];
        const int xe = J->pa[row + 1], ye = J->pb[row + 1], ze = J->pc[row + 1];
        while (x < xe || y < ye || z < ze) {
            int j = INT32_MAX;
            if (x < xe && J->ca[x] < j) j = J->ca[x];
            if (y < ye && J->cb[y] < j) j = J->cb[y];
            if (z < ze && J->cc[z] < j) j = J->cc[z];
            const int ha = x < xe && J->ca[x] == j, hb = y < ye && J->cb[y] == j,
                      hc = z < ze && J->cc[z] == j;
            if (J->write) {
                float v;
                if (ha && hb) {
                    v = J->va[x] + J->vb[y];
                    if (hc) v = v + J->vc[z];
                } else if (ha) {
                    v = hc ? J->va[x] + J->vc[z] : J->va[x];
                } else if (hb) {
                    v = hc ? J->vb[y] + J->vc[z] : J->vb[y];
                } else {
                    v = J->vc[z];
                }
                J->crd[n] = j;
                J->val[n] = v;
            }
            ++n;
            x += ha;
            y += hb;
            z += hc;
        }
        if (J->write) J->pos[row + 1] = (int32_t)n;
    }
    if (!J->write) rg->n[0] = n;
}

static void add3_task(int t, void *arg) { add3_range((add3_mt_job *)arg, t); }

/* The same result as oracle_csr_add3, on `nthreads` threads (0: all online cores): rows cut
 * into ranges of about equal (entries + rows). */
int oracle_csr_add3_mt(int rows, const int32_t *pa, const int32_t *ca, const float *va,
                       const int32_t *pb, const int32_t *cb, const float *vb, const int32_t *pc,
                       const int32_t *cc, const float *vc, int nthreads, int32_t **o_pos,
                       int32_t **o_crd, float **o_val, int *o_nnz) {
    const int nt = nthreads > 0 ? nthreads : oracle_default_threads();
    top_range *r = (top_range *)calloc((size_t)nt, sizeof(top_range));
    if (!r) return ORC_ENOMEM;
    const long total = (long)pa[rows] + pb[rows] + pc[rows] + rows;
    for (int t = 0; t < nt; ++t) {
        /* first row whose prefix weight reaches t * total / nt */
        const long target = total * t / nt;
        int lo = 0, hi = rows;
        while (lo < hi) {
            const int mid = (lo + hi) / 2;
            if ((long)pa[mid] + pb[mid] + pc[mid] + mid < target) {
                lo = mid + 1;
            } else {
                hi = mid;
            }
        }
        r[t].ia0 = t == 0 ? 0 : lo;
    }
    for (int t = 0; t < nt; ++t) r[t].ia1 = t + 1 < nt ? r[t + 1].ia0 : rows;
    add3_mt_job J;
    memset(&J, 0, sizeof(J));
    J.rows = rows;
    J.pa = pa;
    J.ca = ca;
    J.va = va;
    J.pb = pb;
    J.cb = cb;
    J.vb = vb;
    J.pc = pc;
    J.cc = cc;
    J.vc = vc;
    J.r = r;
    parallel_for(nt, add3_task, &J);
    long tot[1];
    exclusive_offsets(r, nt, 1, tot);
    J.pos = (int32_t *)malloc(sizeof(int32_t) * ((size_t)rows + 1));
    J.crd = (int32_t *)malloc(sizeof(int32_t) * ((size_t)tot[0] + 1));
    J.val = (float *)malloc(sizeof(float) * ((size_t)tot[0] + 1));
    if (!J.pos || !J.crd || !J.val) {
        free(J.pos);
        free(J.crd);
        free(J.val);
        free(r);
        return ORC_ENOMEM;
    }
    J.pos[0] = 0;
    J.write = 1;
    parallel_for(nt, add3_task, &J);
    free(r);
    *o_pos = J.pos;
    *o_crd = J.crd;
    *o_val = J.val;
    *o_nnz = (int)tot[0];
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------- */
/* inner products (inner_prod, inner_prod_coo)                                           */
/*
 * z = sum over the coordinates both operands hold of a * b (compiler.cpp:141, 143): the
 * intersection lattice at every level (for i in A_i ∩ B_i, for j in A_ij ∩ B_ij, for k in
 * A_ijk ∩ B_ijk), each product one float32 multiply (compute.cpp:476-491 evaluates a * b
 * in value_t).  The reference accumulates float32 partial sums per thread and adds them
 * with atomics (compute.cpp:498-520, runtime/nacho_kernel_utils.h:40-58), an order that
 * depends on its partitioning; here the products are summed in float64 (the product path's
 * arithmetic) over a range of the top level per thread, ranges in ascending order, and the
 * thread totals added in thread order.  The float64 total is returned; callers round it.
 */

/* Sum of a[k] * b[k] over the k both sorted fibres hold. */
static double k_intersect(const int32_t *ak, const float *av, int a0, int a1,
                          const int32_t *bk, const float *bv, int b0, int b1) {
    double s = 0.0;
    while (a0 < a1 && b0 < b1) {
        if (ak[a0] < bk[b0]) {
            ++a0;
        } else if (bk[b0] < ak[a0]) {
            ++b0;
        } else {
            s += (double)(av[a0] * bv[b0]);
            ++a0;
            ++b0;
        }
    }
    return s;
}

/* First index x in [lo, hi) with key[x] >= q (hi when none). */
static int lower_bound_i32(const int32_t *key, int lo, int hi, int32_t q) {
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (key[mid] < q) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

typedef struct {
    const int32_t *a_ci, *a_pj, *a_cj, *a_pk, *a_ck;
    const float *a_v;
    int a_ni;
    const int32_t *b_ci, *b_pj, *b_cj, *b_pk, *b_ck;
    const float *b_v;
    int b_ni;
    int nt;
    double *part;
} csf_inner_job;

/* First index x in [lo, hi] with key[x] >= q (hi + 1 when none), over int32 offsets. */
static int first_at_least(const int32_t *key, int lo, int hi, long q) {
    int h = hi + 1;
    while (lo < h) {
        const int mid = lo + (h - lo) / 2;
        if ((long)key[mid] < q) {
            lo = mid + 1;
        } else {
            h = mid;
        }
    }
    return lo;
}

/* Thread t: A's (i, j) fibres whose k entries start in [t*nk/nt, (t+1)*nk/nt), so threads
 * hold equal shares of A's entries however skewed the i level is; each fibre is matched
 * with B's fibre of the same (i, j) and their k lists intersected. */
static void csf_inner_task(int t, void *arg) {
    csf_inner_job *J = (csf_inner_job *)arg;
    const int a_nj = J->a_ni > 0 ? J->a_pj[J->a_ni] : 0;
    const long a_nk = a_nj > 0 ? J->a_pk[a_nj] : 0;
    const int f0 = first_at_least(J->a_pk, 0, a_nj, a_nk * t / J->nt);
    const int f1 = t + 1 == J->nt ? a_nj : first_at_least(J->a_pk, 0, a_nj, a_nk * (t + 1) / J->nt);
    double s = 0.0;
    if (f0 < f1) {
        /* the i entry holding fibre f0: the last ia with a_pj[ia] <= f0 */
        int ia = first_at_least(J->a_pj, 0, J->a_ni, (long)f0 + 1) - 1;
        int f = f0;
        while (f < f1) {
            const int fend = J->a_pj[ia + 1] < f1 ? J->a_pj[ia + 1] : f1;
            const int ib = lower_bound_i32(J->b_ci, 0, J->b_ni, J->a_ci[ia]);
            if (ib < J->b_ni && J->b_ci[ib] == J->a_ci[ia]) {
                const int jbe = J->b_pj[ib + 1];
                int jb = lower_bound_i32(J->b_cj, J->b_pj[ib], jbe, J->a_cj[f]);
                int fa = f;
                while (fa < fend && jb < jbe) {
                    if (J->a_cj[fa] < J->b_cj[jb]) {
                        ++fa;
                    } else if (J->b_cj[jb] < J->a_cj[fa]) {
                        ++jb;
                    } else {
                        s += k_intersect(J->a_ck, J->a_v, J->a_pk[fa], J->a_pk[fa + 1], J->b_ck,
                                         J->b_v, J->b_pk[jb], J->b_pk[jb + 1]);
                        ++fa;
                        ++jb;
                    }
                }
            }
            f = fend;
            ++ia;
        }
    }
    J->part[t] = s;
}

/* Inner product of two CSF3 tensors (arrays as oracle_csf3_union takes them), on nthreads
 * threads (<= 0: one per online CPU). */
int oracle_csf3_inner(const int32_t *a_ci, int a_ni, const int32_t *a_pj, const int32_t *a_cj,
                      const int32_t *a_pk, const int32_t *a_ck, const float *a_v,
                      const int32_t *b_ci, int b_ni, const int32_t *b_pj, const int32_t *b_cj,
                      const int32_t *b_pk, const int32_t *b_ck, const float *b_v, int nthreads,
                      double *out) {
    const int nt = nthreads > 0 ? nthreads : oracle_default_threads();
    double *part = (double *)calloc((size_t)nt, sizeof(double));
    if (!part) return ORC_ENOMEM;
    csf_inner_job J = {a_ci, a_pj, a_cj, a_pk, a_ck, a_v, a_ni,
                       b_ci, b_pj, b_cj, b_pk, b_ck, b_v, b_ni, nt, part};
    parallel_for(nt, csf_inner_task, &J);
    double s = 0.0;
    for (int t = 0; t < nt; ++t) s += part[t];
    free(part);
    *out = s;
    return ORC_OK;
}

typedef struct {
    const int32_t *ai, *aj, *ak;
    const float *av;
    int na;
    const int32_t *bi, *bj, *bk;
    const float *bv;
    int nb;
    int nt;
    double *part;
} coo3_inner_job;

static int tuple_cmp(const int32_t *xi, const int32_t *xj, const int32_t *xk, int x,
                     const int32_t *yi, const int32_t *yj, const int32_t *yk, int y) {
    if (xi[x] != yi[y]) return xi[x] < yi[y] ? -1 : 1;
    if (xj[x] != yj[y]) return xj[x] < yj[y] ? -1 : 1;
    if (xk[x] != yk[y]) return xk[x] < yk[y] ? -1 : 1;
    return 0;
}

/* Thread t: A's entries [t*na/nt, (t+1)*na/nt) merged against B from the first B tuple not
 * below the range's first A tuple. */
static void coo3_inner_task(int t, void *arg) {
    coo3_inner_job *J = (coo3_inner_job *)arg;
    int a = (int)((long)J->na * t / J->nt), a_end = (int)((long)J->na * (t + 1) / J->nt);
    double s = 0.0;
    int b = J->nb;
    if (a < a_end) {
        int lo = 0, hi = J->nb;
        while (lo < hi) {
            const int mid = lo + (hi - lo) / 2;
            if (tuple_cmp(J->bi, J->bj, J->bk, mid, J->ai, J->aj, J->ak, a) < 0) {
                lo = mid + 1;
            } else {
                hi = mid;
            }
        }
        b = lo;
    }
    while (a < a_end && b < J->nb) {
        const int c = tuple_cmp(J->ai, J->aj, J->ak, a, J->bi, J->bj, J->bk, b);
        if (c < 0) {
            ++a;
        } else if (c > 0) {
            ++b;
        } else {
            s += (double)(J->av[a] * J->bv[b]);
            ++a;
            ++b;
        }
    }
    J->part[t] = s;
}

/* Inner product of two COO3 tensors sorted by (i, j, k) without duplicates. */
int oracle_coo3_inner(const int32_t *ai, const int32_t *aj, const int32_t *ak, const float *av,
                      int na, const int32_t *bi, const int32_t *bj, const int32_t *bk,
                      const float *bv, int nb, int nthreads, double *out) {
    const int nt = nthreads > 0 ? nthreads : oracle_default_threads();
    double *part = (double *)calloc((size_t)nt, sizeof(double));
    if (!part) return ORC_ENOMEM;
    coo3_inner_job J = {ai, aj, ak, av, na, bi, bj, bk, bv, nb, nt, part};
    parallel_for(nt, coo3_inner_task, &J);
    double s = 0.0;
    for (int t = 0; t < nt; ++t) s += part[t];
    free(part);
    *out = s;
    return ORC_OK;
}
