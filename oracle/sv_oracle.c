/*
 * CPU oracle for SparseConv2D (SV-TAD, pcr-upm/eccv26_tad).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path (the HIP library, the
 * torch extension, the Python wrapper) links, loads or calls this file. It is
 * used by tests/ (as the checker), by __graft_entry__.smoke() (as the checker)
 * and by bench.py's cpu_baseline leg (timed as a restatement of the reference
 * dataflow, kind "port").
 *
 * Every function restates the reference's algorithm and cites the reference
 * file:line it follows (paths relative to the reference repository root):
 *   sparse_conv_layer.py  = opentad/models/bricks/sparse_conv_layer.py
 *   2d_sparse_v3.cu       = opentad/models/bricks/2d_sparse_v3.cu
 *   implicit_gemm_v2.cu   = opentad/models/bricks/implicit_gemm_v2.cu
 *   poguise.py            = opentad/models/backbones/vit_sparse_adapter_poguise.py
 *
 * Two precisions:
 *   *_f64 : float32 inputs, float64 accumulation and float64 outputs. This is
 *           the parity oracle.
 *   *_f32 : float32 accumulation in the reference's dataflow order (gather
 *           [9,N,C] -> 9 per-offset GEMMs into fp32 -> sum over the offsets),
 *           OpenMP-parallel. This is the timed CPU baseline.
 *
 * Index semantics shared by all functions (2d_sparse_v3.cu:432-436,674-677,
 * 728-731; implicit_gemm_v2.cu:67-72): entry nbr[i*9+k] == -1 means "missing";
 * otherwise the source row is nbr[i*9+k] + off(i) with
 * off(i) = (i / tpb) * tpb when tpb > 0, else 0 (the per-row rule of the
 * backward kernels). A source row outside [0, n) is treated as missing (the
 * reference reads out of bounds there, which is undefined).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline int64_t src_row(const int32_t* nbr, int64_t i, int k, int64_t n, int64_t tpb) {
    int32_t v = nbr[i * 9 + k];
    if (v < 0) return -1;
    int64_t r = (int64_t)v + (tpb > 0 ? (i / tpb) * tpb : 0);
    return (r < n) ? r : -1;
}

/* ------------------------------------------------------------------------- */
/* Neighbor table                                                             */
/* ------------------------------------------------------------------------- */

/* Number of kept cells in a B*T*H*W keep mask. */
int64_t svo_count(const uint8_t* mask, int64_t cells) {
    int64_t c = 0;
    for (int64_t p = 0; p < cells; ++p) c += mask[p] != 0;
    return c;
}

/*
 * Neighbor table from a keep mask [B,T,H,W] (row-major), closed form.
 *
 * The reference builds the full-grid table per frame by padding the h*w arange
 * with -1 and stacking the 9 shifted slices with dy outer and dx inner
 * (poguise.py:1629-1640), so k = (dy+1)*3 + (dx+1) and k = 4 is the cell
 * itself; it then adds t*h*w (:1651-1655) and b*T*h*w (:1664-1668) to valid
 * entries. After each prune it keeps the rows of the kept tokens (sorted
 * ascending, poguise.py:785-787) and maps every old global index through
 * old -> b*N_new + j (poguise.py:913-977). Both are captured by one formula:
 * table[rank(p), k] = rank(p + delta_k) if that cell is inside the frame and
 * kept, else -1, where rank is the exclusive prefix count of the flattened
 * B*T*H*W mask. Rows are written in rank order.
 */
void svo_build_table(const uint8_t* mask, int64_t B, int64_t T, int64_t H, int64_t W,
                     int32_t* table) {
    const int64_t cells = B * T * H * W;
    int64_t* rank = (int64_t*)malloc(sizeof(int64_t) * (size_t)(cells > 0 ? cells : 1));
    int64_t acc = 0;
    for (int64_t p = 0; p < cells; ++p) { rank[p] = acc; acc += mask[p] != 0; }
    const int64_t hw = H * W;
    for (int64_t p = 0; p < cells; ++p) {
        if (!mask[p]) continue;
        const int64_t frame = p / hw, q = p % hw, y = q / W, x = q % W;
        int32_t* row = table + rank[p] * 9;
        for (int dy = -1; dy <= 1; ++dy)
            for (int dx = -1; dx <= 1; ++dx) {
                const int k = (dy + 1) * 3 + (dx + 1);
                const int64_t yy = y + dy, xx = x + dx;
                int32_t v = -1;
                if (yy >= 0 && yy < H && xx >= 0 && xx < W) {
                    const int64_t pn = frame * hw + yy * W + xx;
                    if (mask[pn]) v = (int32_t)rank[pn];
                }
                row[k] = v;
            }
    }
    free(rank);
}

/*
 * Table remap after a prune, restating poguise.py:913-977 step by step:
 * gather the kept rows (:920-925), fill the global mapping with -1 (:928-929),
 * write mapping[b*N_prev + keep[b,j]] = b*N_new + j (:932-957), then map every
 * valid entry (:961-977). keep_idx is [B, N_new] local indices into N_prev.
 * mapping_ws must hold B*N_prev int32.
 */
void svo_remap_table(const int32_t* table, int64_t B, int64_t n_prev, const int64_t* keep_idx,
                     int64_t n_new, int32_t* mapping_ws, int32_t* out) {
    for (int64_t p = 0; p < B * n_prev; ++p) mapping_ws[p] = -1;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t j = 0; j < n_new; ++j)
            mapping_ws[b * n_prev + keep_idx[b * n_new + j]] = (int32_t)(b * n_new + j);
    for (int64_t b = 0; b < B; ++b)
        for (int64_t j = 0; j < n_new; ++j) {
            const int32_t* src = table + (b * n_prev + keep_idx[b * n_new + j]) * 9;
            int32_t* dst = out + (b * n_new + j) * 9;
            for (int k = 0; k < 9; ++k) dst[k] = src[k] != -1 ? mapping_ws[src[k] < 0 ? 0 : src[k]] : -1;
        }
}

/* ------------------------------------------------------------------------- */
/* Full (dense channel) SparseConv2D, fp64 oracle                             */
/* ------------------------------------------------------------------------- */

/*
 * Forward: out[i,co] = sum_k sum_ci x[src(i,k), ci] * W[k,ci,co] (+ bias[co]).
 * W layout (9, C_in, C_out) with k = ky*3 + kx (sparse_conv_layer.py:136,
 * 150-156). Math of sparse_fwd_tiled_v2/v3 (2d_sparse_v3.cu:439-512) and of
 * gather -> GEMM -> sum (implicit_gemm_v2.cu:43-79, 272-287, 131-161).
 * bias may be NULL.
 */
void svo_fwd_f64(const float* x, const int32_t* nbr, const float* w, const float* bias,
                 int64_t n, int ci, int co, int64_t tpb, double* out) {
    double* acc = (double*)malloc(sizeof(double) * (size_t)co);
    for (int64_t i = 0; i < n; ++i) {
        for (int c = 0; c < co; ++c) acc[c] = bias ? (double)bias[c] : 0.0;
        for (int k = 0; k < 9; ++k) {
            const int64_t r = src_row(nbr, i, k, n, tpb);
            if (r < 0) continue;
            const float* xr = x + r * ci;
            const float* wk = w + (int64_t)k * ci * co;
            for (int a = 0; a < ci; ++a) {
                const double xv = xr[a];
                const float* wr = wk + (int64_t)a * co;
                for (int c = 0; c < co; ++c) acc[c] += xv * (double)wr[c];
            }
        }
        for (int c = 0; c < co; ++c) out[i * co + c] = acc[c];
    }
    free(acc);
}

/*
 * Backward-input as the reference scatters it (2d_sparse_v3.cu:679-707):
 * gi[src(i,k), ci] += sum_co go[i,co] * W[k,ci,co]. gi is zeroed here
 * (2d_sparse_v3.cu:825).
 */
void svo_bwd_in_f64(const float* go, const int32_t* nbr, const float* w, int64_t n, int ci,
                    int co, int64_t tpb, double* gi) {
    memset(gi, 0, sizeof(double) * (size_t)(n * ci));
    for (int64_t i = 0; i < n; ++i) {
        const float* g = go + i * co;
        for (int k = 0; k < 9; ++k) {
            const int64_t r = src_row(nbr, i, k, n, tpb);
            if (r < 0) continue;
            const float* wk = w + (int64_t)k * ci * co;
            for (int a = 0; a < ci; ++a) {
                const float* wr = wk + (int64_t)a * co;
                double s = 0.0;
                for (int c = 0; c < co; ++c) s += (double)g[c] * (double)wr[c];
                gi[r * ci + a] += s;
            }
        }
    }
}

/*
 * Backward-weight (2d_sparse_v3.cu:733-744): gw[k,ci,co] = sum_i go[i,co] *
 * x[src(i,k), ci]; zero-initialised (:841).
 */
void svo_bwd_w_f64(const float* go, const float* x, const int32_t* nbr, int64_t n, int ci,
                   int co, int64_t tpb, double* gw) {
    memset(gw, 0, sizeof(double) * (size_t)(9 * (int64_t)ci * co));
    for (int64_t i = 0; i < n; ++i) {
        const float* g = go + i * co;
        for (int k = 0; k < 9; ++k) {
            const int64_t r = src_row(nbr, i, k, n, tpb);
            if (r < 0) continue;
            const float* xr = x + r * ci;
            double* gk = gw + (int64_t)k * ci * co;
            for (int a = 0; a < ci; ++a) {
                const double xv = xr[a];
                double* gr = gk + (int64_t)a * co;
                for (int c = 0; c < co; ++c) gr[c] += xv * (double)g[c];
            }
        }
    }
}

/* Bias gradient: gb[co] = sum_i go[i,co] (sparse_conv_layer.py:120-121). */
void svo_bias_grad_f64(const float* go, int64_t n, int co, double* gb) {
    for (int c = 0; c < co; ++c) gb[c] = 0.0;
    for (int64_t i = 0; i < n; ++i)
        for (int c = 0; c < co; ++c) gb[c] += go[i * co + c];
}

/* ------------------------------------------------------------------------- */
/* Depthwise SparseConv2D (groups = C), fp64 oracle                           */
/* Not in the reference (SparseConv2d has no groups, sparse_conv_layer.py:127)*/
/* W layout (9, C). Same index semantics as above.                            */
/* ------------------------------------------------------------------------- */

void svo_dw_fwd_f64(const float* x, const int32_t* nbr, const float* w, const float* bias,
                    int64_t n, int c, int64_t tpb, double* out) {
    for (int64_t i = 0; i < n; ++i)
        for (int a = 0; a < c; ++a) {
            double s = bias ? (double)bias[a] : 0.0;
            for (int k = 0; k < 9; ++k) {
                const int64_t r = src_row(nbr, i, k, n, tpb);
                if (r >= 0) s += (double)x[r * c + a] * (double)w[k * c + a];
            }
            out[i * c + a] = s;
        }
}

void svo_dw_bwd_in_f64(const float* go, const int32_t* nbr, const float* w, int64_t n, int c,
                       int64_t tpb, double* gi) {
    memset(gi, 0, sizeof(double) * (size_t)(n * c));
    for (int64_t i = 0; i < n; ++i)
        for (int k = 0; k < 9; ++k) {
            const int64_t r = src_row(nbr, i, k, n, tpb);
            if (r < 0) continue;
            for (int a = 0; a < c; ++a) gi[r * c + a] += (double)go[i * c + a] * (double)w[k * c + a];
        }
}

void svo_dw_bwd_w_f64(const float* go, const float* x, const int32_t* nbr, int64_t n, int c,
                      int64_t tpb, double* gw) {
    memset(gw, 0, sizeof(double) * (size_t)(9 * c));
    for (int64_t i = 0; i < n; ++i)
        for (int k = 0; k < 9; ++k) {
            const int64_t r = src_row(nbr, i, k, n, tpb);
            if (r < 0) continue;
            for (int a = 0; a < c; ++a) gw[k * c + a] += (double)go[i * c + a] * (double)x[r * c + a];
        }
}

/* ------------------------------------------------------------------------- */
/* fp32 "port" of the reference dataflow, OpenMP (timed CPU baseline)         */
/* ------------------------------------------------------------------------- */

/*
 * Forward in the order of implicit_gemm_fwd_v2 (implicit_gemm_v2.cu:197-300):
 * gather x_g[9,N,C_in] with zeros for missing neighbors (:43-79), nine GEMMs
 * x_g[k] @ W[k] into fp32 out_f[9,N,C_out] (:272-287), then
 * out = sum_k out_f[k] + bias in fp32 (:131-161). xg_ws holds 9*n*ci floats and
 * of_ws 9*n*co floats.
 */
void svo_fwd_f32(const float* x, const int32_t* nbr, const float* w, const float* bias,
                 int64_t n, int ci, int co, int64_t tpb, float* xg_ws, float* of_ws, float* out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        for (int k = 0; k < 9; ++k) {
            const int64_t r = src_row(nbr, i, k, n, tpb);
            float* dst = xg_ws + ((int64_t)k * n + i) * ci;
            if (r < 0) memset(dst, 0, sizeof(float) * (size_t)ci);
            else memcpy(dst, x + r * ci, sizeof(float) * (size_t)ci);
        }
    #pragma omp parallel for collapse(2) schedule(static)
    for (int k = 0; k < 9; ++k)
        for (int64_t i = 0; i < n; ++i) {
            const float* a = xg_ws + ((int64_t)k * n + i) * ci;
            const float* wk = w + (int64_t)k * ci * co;
            float* o = of_ws + ((int64_t)k * n + i) * co;
            for (int c = 0; c < co; ++c) o[c] = 0.f;
            for (int t = 0; t < ci; ++t) {
                const float av = a[t];
                const float* wr = wk + (int64_t)t * co;
                for (int c = 0; c < co; ++c) o[c] += av * wr[c];
            }
        }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        for (int c = 0; c < co; ++c) {
            float s = 0.f;
            for (int k = 0; k < 9; ++k) s += of_ws[((int64_t)k * n + i) * co + c];
            out[i * co + c] = s + (bias ? bias[c] : 0.f);
        }
}

/*
 * Backward-input, fp32, same sum as 2d_sparse_v3.cu:679-707. The reference
 * scatters with atomics; here each thread owns a block of C_in columns, so the
 * scatter needs no atomics.
 */
void svo_bwd_in_f32(const float* go, const int32_t* nbr, const float* w, int64_t n, int ci,
                    int co, int64_t tpb, float* gi) {
    memset(gi, 0, sizeof(float) * (size_t)(n * ci));
    #pragma omp parallel for schedule(static)
    for (int a = 0; a < ci; ++a)
        for (int64_t i = 0; i < n; ++i) {
            const float* g = go + i * co;
            for (int k = 0; k < 9; ++k) {
                const int64_t r = src_row(nbr, i, k, n, tpb);
                if (r < 0) continue;
                const float* wr = w + ((int64_t)k * ci + a) * co;
                float s = 0.f;
                for (int c = 0; c < co; ++c) s += g[c] * wr[c];
                gi[r * ci + a] += s;
            }
        }
}

/* Backward-weight, fp32 (2d_sparse_v3.cu:733-744); each thread owns (k, ci) rows of gw. */
void svo_bwd_w_f32(const float* go, const float* x, const int32_t* nbr, int64_t n, int ci,
                   int co, int64_t tpb, float* gw) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int k = 0; k < 9; ++k)
        for (int a = 0; a < ci; ++a) {
            float* gr = gw + ((int64_t)k * ci + a) * co;
            for (int c = 0; c < co; ++c) gr[c] = 0.f;
            for (int64_t i = 0; i < n; ++i) {
                const int64_t r = src_row(nbr, i, k, n, tpb);
                if (r < 0) continue;
                const float xv = x[r * ci + a];
                const float* g = go + i * co;
                for (int c = 0; c < co; ++c) gr[c] += xv * g[c];
            }
        }
}

int svo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
