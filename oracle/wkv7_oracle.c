/*
 * CPU oracle for the WKV7 slot-pool recurrence.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path (wkvm_amd/) links,
 * loads or calls this file. It is used by tests/ as the checker, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg
 * as the timed CPU restatement ("port").
 *
 * What it restates. The reference (xiaol/wkvm) drives the WKV7 arithmetic
 * through the third-party `fla` package (wkvm/models/rwkv7.py:113,
 * wkvm/runner/runner.py:3-7): the fused recurrent kernel for T < 64 and
 * `chunk_rwkv7` for T >= 64 (wkvm/models/rwkv7.py:108-111). `fla` is not
 * vendored, not version-pinned (pyproject.toml:14-30) and not installed here,
 * so the recurrence is restated from its mathematical definition, per head
 * with N = K = V:
 *
 *     S_t = S_{t-1} diag(w_t) + (S_{t-1} a_t) b_t^T + v_t k_t^T,   y_t = S_t r_t
 *
 * stored in the bank orientation h = S^T, i.e. state[j][i] = S[i][j] with j the
 * key index and i the value index (wkvm/models/rwkv7.py:15-16 documents the
 * per-layer state as [H, head_dim, head_v_dim]; wkvm/runner/state.py:35-39
 * allocates wkv as [L, S+1, H, K, V] fp32):
 *
 *     p_i         = sum_m a_t[m] h_{t-1}[m][i]
 *     h_t[j][i]   = exp(w_t[j]) h_{t-1}[j][i] + b_t[j] p_i + k_t[j] v_t[i]
 *     y_t[i]      = scale * sum_j r_t[j] h_t[j][i]
 *
 * `w` crosses every interface as log-decay (the multiplicative decay is
 * exp(w)), the convention of the fla wkv op the reference calls.
 *
 * Two families of functions:
 *   wkv7_oracle_scan_f64   float64 stepwise scan over ragged sequences; the
 *                          parity checker. Arbitrary N (tiny N for brute-force
 *                          tests).
 *   wkv7_port_*_f32        float32 restatements with the product's exact
 *                          interface semantics (bf16 inputs, in-place slot
 *                          pool, bf16 outputs). Used only as the timed CPU
 *                          baseline and checked against the f64 scan in tests.
 *
 * Parity pinning of this file (tests/test_oracle.py): closed forms CF1-CF4
 * (linear-attention prefix sum, constant-decay geometric sum, delta-rule
 * retrieval S_1 k = v, zero state), linearity in (S_0, v), an invariant that
 * fixes which side a and b act on, the explicit product of transition
 * matrices M_t = diag(w_t) + a_t b_t^T evaluated with numpy matmul, and
 * committed golden vectors produced by that product form.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static double bf16_to_double(uint16_t x)
{
    uint32_t u = (uint32_t)x << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return (double)f;
}

static float bf16_to_float(uint16_t x)
{
    uint32_t u = (uint32_t)x << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Round-to-nearest-even float -> bf16 (NaN kept quiet). */
static uint16_t float_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void wkv7_oracle_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0)
        omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int wkv7_oracle_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/*
 * float64 stepwise scan, written once and instantiated for two input types:
 *   wkv7_oracle_scan_f64   float64 inputs and initial state (any N)
 *   wkv7_oracle_scan_bf16  bf16 bit-pattern inputs, float32 initial state
 *                          rows gathered by slot id from a pool (N = any);
 *                          widened exactly to float64 on load
 * Arguments:
 *   cu_seqlens [nseq+1]: token offsets of each sequence in the [T, H, N] inputs
 *   h0: initial state [nseq, H, N, N] (f64 variant) or NULL for zero state;
 *       bf16 variant: pool [rows, H, N, N] float32 + slot_ids [nseq] (pool NULL
 *       for zero state)
 *   r, w (log-decay), k, v, a, b [T, H, N]
 *   y [T, H, N], hT [nseq, H, N, N] float64 outputs
 * Returns 0, or a negative code on bad arguments.
 */
#define SCAN_BODY(LOAD, INIT)                                                          \
    const int64_t NN = N * N;                                                          \
    int bad = 0;                                                                       \
    _Pragma("omp parallel for schedule(dynamic, 1) reduction(| : bad)")                \
    for (int64_t sh = 0; sh < nseq * H; ++sh) {                                         \
        const int64_t s = sh / H, hd = sh % H;                                         \
        double *h = hT + sh * NN;                                                      \
        double *p = (double *)malloc((size_t)(2 * N) * sizeof(double));                \
        if (!p) {                                                                      \
            bad = 1;                                                                   \
            continue;                                                                  \
        }                                                                              \
        double *dec = p + N;                                                           \
        INIT                                                                           \
        for (int64_t t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t) {                  \
            const int64_t o = (t * H + hd) * N;                                        \
            for (int64_t i = 0; i < N; ++i)                                            \
                p[i] = 0.0;                                                            \
            for (int64_t m = 0; m < N; ++m) {                                          \
                const double am = LOAD(a, o + m);                                      \
                for (int64_t i = 0; i < N; ++i)                                        \
                    p[i] += am * h[m * N + i];                                         \
            }                                                                          \
            for (int64_t j = 0; j < N; ++j)                                            \
                dec[j] = exp(LOAD(w, o + j));                                          \
            for (int64_t j = 0; j < N; ++j) {                                          \
                const double bj = LOAD(b, o + j), kj = LOAD(k, o + j);                 \
                for (int64_t i = 0; i < N; ++i)                                        \
                    h[j * N + i] = dec[j] * h[j * N + i] + bj * p[i] + kj * LOAD(v, o + i); \
            }                                                                          \
            for (int64_t i = 0; i < N; ++i) {                                          \
                double acc = 0.0;                                                      \
                for (int64_t j = 0; j < N; ++j)                                        \
                    acc += LOAD(r, o + j) * h[j * N + i];                              \
                y[o + i] = scale * acc;                                                \
            }                                                                          \
        }                                                                              \
        free(p);                                                                       \
    }                                                                                  \
    return bad ? -2 : 0;

#define LOAD_F64(x, i) ((x)[i])
#define LOAD_BF16(x, i) bf16_to_double((x)[i])

static int check_cu(int64_t nseq, const int64_t *cu_seqlens)
{
    for (int64_t s = 0; s < nseq; ++s)
        if (cu_seqlens[s + 1] < cu_seqlens[s])
            return -1;
    return 0;
}

int wkv7_oracle_scan_f64(int64_t nseq, int64_t H, int64_t N,
                         const int64_t *cu_seqlens, const double *h0,
                         const double *r, const double *w, const double *k,
                         const double *v, const double *a, const double *b,
                         double scale, double *y, double *hT)
{
    if (nseq < 0 || H < 1 || N < 1 || !cu_seqlens || !y || !hT || check_cu(nseq, cu_seqlens))
        return -1;
    SCAN_BODY(LOAD_F64,
              if (h0) memcpy(h, h0 + sh * NN, (size_t)NN * sizeof(double));
              else memset(h, 0, (size_t)NN * sizeof(double));)
}

int wkv7_oracle_scan_bf16(int64_t nseq, int64_t H, int64_t N,
                          const int64_t *cu_seqlens, const float *pool, int64_t rows,
                          const int32_t *slot_ids,
                          const uint16_t *r, const uint16_t *w, const uint16_t *k,
                          const uint16_t *v, const uint16_t *a, const uint16_t *b,
                          double scale, double *y, double *hT)
{
    if (nseq < 0 || H < 1 || N < 1 || !cu_seqlens || !y || !hT || check_cu(nseq, cu_seqlens))
        return -1;
    if (pool) {
        if (!slot_ids)
            return -1;
        for (int64_t s = 0; s < nseq; ++s)
            if (slot_ids[s] < 0 || slot_ids[s] >= rows)
                return -1;
    }
    SCAN_BODY(LOAD_BF16,
              if (pool) {
                  const float *src = pool + ((int64_t)slot_ids[s] * H + hd) * NN;
                  for (int64_t e = 0; e < NN; ++e) h[e] = (double)src[e];
              } else memset(h, 0, (size_t)NN * sizeof(double));)
}

/*
 * One head step of the float32 port, N = 64, state updated in place.
 */
#define PN 64
static void port_head_step(float *h, const uint16_t *r, const uint16_t *w, const uint16_t *k,
                           const uint16_t *v, const uint16_t *a, const uint16_t *b,
                           float scale, uint16_t *y)
{
    float p[PN], vv[PN], acc[PN];
    for (int i = 0; i < PN; ++i) {
        p[i] = 0.f;
        acc[i] = 0.f;
        vv[i] = bf16_to_float(v[i]);
    }
    for (int m = 0; m < PN; ++m) {
        const float am = bf16_to_float(a[m]);
        for (int i = 0; i < PN; ++i)
            p[i] += am * h[m * PN + i];
    }
    for (int j = 0; j < PN; ++j) {
        const float dj = expf(bf16_to_float(w[j]));
        const float bj = bf16_to_float(b[j]);
        const float kj = bf16_to_float(k[j]);
        const float rj = bf16_to_float(r[j]) * scale;
        for (int i = 0; i < PN; ++i) {
            const float hn = dj * h[j * PN + i] + bj * p[i] + kj * vv[i];
            h[j * PN + i] = hn;
            acc[i] += rj * hn;
        }
    }
    for (int i = 0; i < PN; ++i)
        y[i] = float_to_bf16(acc[i]);
}

/*
 * float32 port of the slot-indexed decode step (same semantics as the HIP
 * entry point wkv7_decode_slots): wkv_layer [num_rows, H, 64, 64] fp32 updated
 * in place at rows slot_ids[0..B); inputs [B, H, 64] bf16; y [B, H, 64] bf16.
 */
int wkv7_port_decode_slots_f32(float *wkv_layer, int64_t num_rows, int64_t H,
                               const int32_t *slot_ids, int64_t B,
                               const uint16_t *r, const uint16_t *w, const uint16_t *k,
                               const uint16_t *v, const uint16_t *a, const uint16_t *b,
                               float scale, uint16_t *y)
{
    for (int64_t i = 0; i < B; ++i)
        if (slot_ids[i] < 0 || slot_ids[i] >= num_rows)
            return -1;
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < B * H; ++bh) {
        const int64_t row = bh / H, hd = bh % H;
        float *h = wkv_layer + ((int64_t)slot_ids[row] * H + hd) * PN * PN;
        const int64_t o = bh * PN;
        port_head_step(h, r + o, w + o, k + o, v + o, a + o, b + o, scale, y + o);
    }
    return 0;
}

/*
 * float32 port of the varlen prefill (same semantics as the HIP entry point
 * wkv7_prefill_varlen): sequence s runs tokens [cu_seqlens[s], cu_seqlens[s+1])
 * of the [T, H, 64] inputs starting from slot slot_ids[s] (or zero when
 * zero_init) and leaves its final state in that slot.
 */
int wkv7_port_prefill_f32(float *wkv_layer, int64_t num_rows, int64_t H,
                          const int32_t *slot_ids, const int64_t *cu_seqlens, int64_t nseq,
                          const uint16_t *r, const uint16_t *w, const uint16_t *k,
                          const uint16_t *v, const uint16_t *a, const uint16_t *b,
                          int zero_init, float scale, uint16_t *y)
{
    for (int64_t s = 0; s < nseq; ++s)
        if (slot_ids[s] < 0 || slot_ids[s] >= num_rows || cu_seqlens[s + 1] < cu_seqlens[s])
            return -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t sh = 0; sh < nseq * H; ++sh) {
        const int64_t s = sh / H, hd = sh % H;
        float *h = wkv_layer + ((int64_t)slot_ids[s] * H + hd) * PN * PN;
        if (zero_init)
            memset(h, 0, sizeof(float) * PN * PN);
        for (int64_t t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t) {
            const int64_t o = (t * H + hd) * PN;
            port_head_step(h, r + o, w + o, k + o, v + o, a + o, b + o, scale, y + o);
        }
    }
    return 0;
}

/* Exposed for tests: the bf16 conversion helpers used above. */
double wkv7_oracle_bf16_to_double(uint16_t x) { return bf16_to_double(x); }
uint16_t wkv7_oracle_float_to_bf16(float f) { return float_to_bf16(f); }
