/* ORACLE -- test infrastructure only. Never linked or loaded by the product (seedpack_amd/).
 *
 * A plain-C restatement of llama.cpp's lattice ("grid") i-quant quantizers as vendored by the
 * reference (/root/reference/seedpack/ggml/ggml-quants.c, cited per function as
 * ggml-quants.c:LINES): IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S and IQ1_M (both formulations
 * of IQ1_M's split search), and the lattice tables they search (grid points, level-index map,
 * neighbour lists), built here from the compact codebooks.
 *
 * Formulation: the five IQ2/IQ3 quantizers share one sub-block routine driven by a parameter row
 * (group size, level count, step schedule, sign parity, start and refit rules); IQ1_S and IQ1_M
 * share the split search over sorted weights. Every float expression is evaluated in the C
 * reference's order (left to right, no contraction: built with -ffp-contract=off), every
 * reduction runs over the element index in order, and comparisons keep the reference's strict or
 * non-strict sense and its first-occurrence tie rule. Where the reference aborts (GGML_ASSERT, a
 * point left off the grid) the entry point returns -1.
 *
 * Pinned by tests/test_oracle_iq.py: the tables against the SHA-256 digests of the reference's
 * table fixture (tests/golden/iqtables_sha256.json) and a brute-force neighbour search; the
 * quantizers byte-for-byte against the reference's own C build (oracle/_ref) on seeded inputs and
 * against the committed golden vectors (tests/golden/quant_small.npz); the half conversion
 * against numpy's; planted mistakes (a dropped parity fix, a wrong refit rule) fail the goldens.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK 256

/* ------------------------------------------------------------------ scalar primitives */

/* ggml-quants.c:621-626: round half to even through the 1.5*2^23 bias (|v| < 2^22) */
static int rint_bias(float v) {
    float t = v + 12582912.f;
    int32_t b;
    memcpy(&b, &t, 4);
    return (b & 0x007fffff) - 0x00400000;
}

/* f32 -> IEEE half bits, round to nearest even, overflow to infinity, NaN -> 0x7E00 | sign
   (the conversion of ggml-impl.h:417-443) */
uint16_t og_half_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;
    if (a >= 0x477ff000u) return sign | 0x7c00u;          /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {                                 /* below 2^-14: a multiple of 2^-24 */
        float v;
        memcpy(&v, &a, 4);
        return sign | (uint16_t)lrintf(v * 16777216.f);   /* exact scaling, then nearest even */
    }
    uint32_t h = ((a >> 23) - 112u) << 10 | (a & 0x7fffffu) >> 13;
    uint32_t rest = a & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;   /* a carry moves into the exponent */
    return sign | (uint16_t)h;
}

/* the reference's MAX(a, b) macro: a when a > b, else b (so a NaN b wins) */
static float fmax_c(float a, float b) { return a > b ? a : b; }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

static void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static void put32(uint8_t* p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> 8 * i); }
static uint16_t get16(const uint8_t* p) { return (uint16_t)(p[0] | p[1] << 8); }

/* ------------------------------------------------------------------ lattice tables */

/* The six lattices, indexed as the reference's iq2_data[] / iq3_data[] (ggml-quants.c:2842-2846,
   :3683-3686): 0 IQ2_XXS, 1 IQ2_XS, 2 IQ1_S/IQ1_M, 3 IQ2_S (8 coordinates, 2-bit levels);
   4 IQ3_XXS, 5 IQ3_S (4 coordinates, 3-bit levels). nwant = distinct distances kept per list
   (:3120, :3781); map sizes 43692 and 4096 (:3118, :3780). */
static const int LAT_DIM[6] = {8, 8, 8, 8, 4, 4};
static const int LAT_BITS[6] = {2, 2, 2, 2, 3, 3};
static const int LAT_NPTS[6] = {256, 512, 2048, 1024, 256, 512};
static const int LAT_NWANT[6] = {2, 2, 3, 1, 2, 3};

typedef struct {
    int dim, bits, npts, nmap, nnb;
    uint8_t* pt;     /* npts x dim coordinate values 2l+1 */
    int32_t* map;    /* level index -> point, or -(offset + 1) of its neighbour list in nb */
    uint16_t* nb;    /* per off-grid index: count, then the points */
} Lattice;

static Lattice LAT[6];

static int level_index(const Lattice* T, const uint8_t* coords) {
    int u = 0;
    for (int c = 0; c < T->dim; ++c) u |= ((coords[c] - 1) / 2) << (T->bits * c);
    return u;
}

/* Lists the points nearest to off-grid index u: every point whose squared distance is one of the
   nwant smallest distinct values, ordered by (distance, point). That is the order of the
   reference's qsort over (d2, j) pairs with its lexicographic compare (ggml-quants.c:2848-2852,
   :3225-3252). Writes into out (or only counts when out is NULL); returns the count. */
static int neighbour_list(const Lattice* T, int nwant, int u, int* d2, uint16_t* out) {
    int pos[8];
    for (int c = 0; c < T->dim; ++c) pos[c] = 2 * ((u >> (T->bits * c)) & ((1 << T->bits) - 1)) + 1;
    for (int j = 0; j < T->npts; ++j) {
        int s = 0;
        for (int c = 0; c < T->dim; ++c) {
            int d = T->pt[j * T->dim + c] - pos[c];
            s += d * d;
        }
        d2[j] = s;
    }
    int n = 0, level = -1;
    for (int have = 0; have < nwant; ++have) {
        int next = 1 << 30;
        for (int j = 0; j < T->npts; ++j)
            if (d2[j] > level && d2[j] < next) next = d2[j];
        if (next == 1 << 30) break;
        for (int j = 0; j < T->npts; ++j)
            if (d2[j] == next) {
                if (out) out[n] = (uint16_t)j;
                ++n;
            }
        level = next;
    }
    return n;
}

/* ggml-quants.c:2854-3257 (8 coordinates), :3704-3913 (4 coordinates): points from the compact
   codebook (level l of coordinate c in bits [bits*c, bits*c + bits), value 2l+1), the index map,
   then the neighbour lists of every off-grid index in increasing index order. */
int og_lattice_init(int li, const uint16_t* code, int n) {
    if (li < 0 || li > 5 || n != LAT_NPTS[li]) return -1;
    Lattice* T = &LAT[li];
    if (T->pt) return 0;
    Lattice L = {LAT_DIM[li], LAT_BITS[li], n, LAT_DIM[li] == 8 ? 43692 : 4096, 0, NULL, NULL, NULL};
    L.pt = malloc((size_t)n * L.dim);
    L.map = malloc(sizeof(int32_t) * L.nmap);
    int* d2 = malloc(sizeof(int) * n);
    int* cnt = malloc(sizeof(int) * L.nmap);
    if (!L.pt || !L.map || !d2 || !cnt) return -1;
    for (int k = 0; k < n; ++k)
        for (int c = 0; c < L.dim; ++c) L.pt[k * L.dim + c] = (uint8_t)(2 * ((code[k] >> (L.bits * c)) & ((1 << L.bits) - 1)) + 1);
    for (int i = 0; i < L.nmap; ++i) L.map[i] = -1;
    for (int k = 0; k < n; ++k) L.map[level_index(&L, L.pt + k * L.dim)] = k;
    int total = 0;
    for (int i = 0; i < L.nmap; ++i) {
        cnt[i] = L.map[i] >= 0 ? -1 : neighbour_list(&L, LAT_NWANT[li], i, d2, NULL);
        if (cnt[i] >= 0) total += 1 + cnt[i];
    }
    L.nb = malloc(sizeof(uint16_t) * (total ? total : 1));
    if (!L.nb) return -1;
    int off = 0;
    for (int i = 0; i < L.nmap; ++i) {
        if (cnt[i] < 0) continue;
        L.map[i] = -(off + 1);
        L.nb[off] = (uint16_t)neighbour_list(&L, LAT_NWANT[li], i, d2, L.nb + off + 1);
        off += 1 + cnt[i];
    }
    L.nnb = total;
    free(d2);
    free(cnt);
    *T = L;
    return 0;
}

int og_lattice_table(int li, const uint8_t** pt, int* pt_bytes, const int32_t** map, int* map_n, const uint16_t** nb,
                     int* nb_n) {
    if (li < 0 || li > 5 || !LAT[li].pt) return -1;
    *pt = LAT[li].pt;
    *pt_bytes = LAT[li].npts * LAT[li].dim;
    *map = LAT[li].map;
    *map_n = LAT[li].nmap;
    *nb = LAT[li].nb;
    *nb_n = LAT[li].nnb;
    return 0;
}

/* The listed point nearest to xv/scale in the ws-weighted norm (ws = sqrt of the importance), first
   on ties, -1 when no distance is below FLT_MAX (ggml-quants.c:3271-3293, :3915-3937). */
static int nearest_listed(const Lattice* T, const uint16_t* list, const float* xv, const float* ws, float scale) {
    int best = -1;
    float bd = FLT_MAX;
    for (int j = 1; j <= list[0]; ++j) {
        const uint8_t* p = T->pt + (size_t)list[j] * T->dim;
        float d2 = 0;
        for (int c = 0; c < T->dim; ++c) {
            float diff = scale * (float)p[c] - xv[c];
            d2 += ws[c] * diff * diff;
        }
        if (d2 < bd) {
            bd = d2;
            best = list[j];
        }
    }
    return best;
}

/* ------------------------------------------------------------------ IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS / IQ3_S */

/* ggml-quants.c:1077-1148 (make_qp_quants). L is uint8_t in the reference: a negative level wraps
   when stored, the running sums take the int level, and later reads of L see the wrapped byte. */
static float qp_quants(int n, int nmax, const float* x, uint8_t* L, const float* qw) {
    float mx = 0;
    for (int i = 0; i < n; ++i) mx = fmax_c(mx, x[i]);
    if (mx < 1e-15f) {
        memset(L, 0, n);
        return 0.f;
    }
    float iscale = nmax / mx;
    for (int i = 0; i < n; ++i) L[i] = (uint8_t)rint_bias(iscale * x[i]);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        float diff = x[i] - scale * L[i];
        best += qw[i] * diff * diff;
    }
    for (int is = -4; is <= 4; ++is) {
        if (is == 0) continue;
        float isc = (0.1f * is + nmax) / mx;
        float sc = 1 / isc;
        float mse = 0;
        for (int i = 0; i < n; ++i) {
            int l = rint_bias(isc * x[i]);
            l = nmax < l ? nmax : l;
            float diff = x[i] - sc * l;
            mse += qw[i] * diff * diff;
        }
        if (mse < best) {
            best = mse;
            iscale = isc;
        }
    }
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = rint_bias(iscale * x[i]);
        l = nmax < l ? nmax : l;
        L[i] = (uint8_t)l;
        float w = qw[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    for (int itry = 0; itry < 5; ++itry) {
        int changed = 0;
        for (int i = 0; i < n; ++i) {
            float w = qw[i];
            float slx = sumlx - w * x[i] * L[i];
            float sl2 = suml2 - w * L[i] * L[i];
            if (slx > 0 && sl2 > 0) {
                int nl = rint_bias(x[i] * sl2 / slx);
                nl = nmax < nl ? nmax : nl;
                if (nl != L[i]) {
                    slx += w * x[i] * nl;
                    sl2 += w * nl * nl;
                    if (slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = (uint8_t)nl;
                        sumlx = slx;
                        suml2 = sl2;
                        ++changed;
                    }
                }
            }
        }
        if (!changed) break;
    }
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

/* What distinguishes the five lattice quantizers' sub-block searches. */
typedef struct {
    int lat;       /* lattice */
    int n;         /* weights per sub-block */
    int qmax;      /* levels per coordinate (kMaxQ) */
    int r;         /* scale steps -r..r */
    float step;    /* step of the level count per scale step */
    int parity;    /* sign groups keep 7 bits: an odd number of negatives flips the least important */
    float eps;     /* skip below this maximum; 0: skip only an all-zero sub-block */
    int start;     /* 1: the first scale and the step base come from make_qp_quants (IQ2_XXS) */
    int grid0;     /* initial "group on grid" flags when no step improves */
    int refit;     /* 0: off-grid groups, when any; 1: all groups, when any is off grid; 2: all groups */
    float fudge;   /* super-block scale factor in the stored half (1: none) */
} Sub;

/* OG_PLANT is for the tests' planted-mistake builds only (the default build has 0): 1 drops
   IQ2_XS's sign-parity fix, 2 refits only IQ3_S's off-grid groups, 3 starts IQ2_XXS from max/5. */
#ifndef OG_PLANT
#define OG_PLANT 0
#endif

/* ggml-quants.c:3295-3471 (IQ2_XXS), :3473-3651 (IQ2_XS), :5114-5281 (IQ2_S),
   :3939-4151 (IQ3_XXS), :4170-4351 (IQ3_S) */
static const Sub SUB_IQ2_XXS = {0, 32, 3, 6, 0.1f, 1, 1e-15f, OG_PLANT != 3, 1, 2, 1.f};
static const Sub SUB_IQ2_XS = {1, 16, 3, 9, 0.1f, OG_PLANT != 1, 1e-15f, 0, 1, 0, 1.f};
static const Sub SUB_IQ2_S = {3, 16, 3, 9, 0.1f, 0, 1e-8f, 0, 1, 0, 0.9875f};
static const Sub SUB_IQ3_XXS = {4, 32, 8, 15, 0.2f, 1, 1e-8f, 0, 1, 0, 1.0125f};
static const Sub SUB_IQ3_S = {5, 32, 8, 9, 0.2f, 0, 0.f, 0, 0, OG_PLANT == 2 ? 0 : 1, 1.033f};

/* One sub-block: signs and magnitudes, the scale search over lattice points, the refit. Returns 1
   (coded: scale, grid point per group, sign byte per 8 weights), 0 (skipped: the reference leaves
   the sub-block's scale 0 and writes nothing), -1 (the reference aborts). */
static int lattice_sub(const Sub* S, const float* xb, const float* w, float* scale_out, int* gidx, uint8_t* sgn) {
    const Lattice* T = &LAT[S->lat];
    const int n = S->n, D = T->dim, G = n / D, B = T->bits, qmax = S->qmax;
    float xv[32], ws[32];
    int8_t Lb[32], La[32];
    int on[8], on_a[8];
    for (int i = 0; i < n; ++i) ws[i] = sqrtf(w[i]);
    for (int k = 0; k < n / 8; ++k) {
        int flips = 0;
        uint8_t s = 0;
        for (int i = 0; i < 8; ++i) {
            float x = xb[8 * k + i];
            if (x >= 0) {
                xv[8 * k + i] = x;
            } else {
                xv[8 * k + i] = -x;
                ++flips;
                s |= (uint8_t)(1 << i);
            }
        }
        if (S->parity && flips % 2) {
            int imin = 0;
            float m = w[8 * k] * xb[8 * k] * xb[8 * k];
            for (int i = 1; i < 8; ++i) {
                float a = w[8 * k + i] * xb[8 * k + i] * xb[8 * k + i];
                if (a < m) {
                    m = a;
                    imin = i;
                }
            }
            xv[8 * k + imin] = -xv[8 * k + imin];
            s ^= (uint8_t)(1 << imin);
        }
        sgn[k] = S->parity ? (uint8_t)(s & 127) : s;
    }
    float mx = xv[0];
    for (int i = 1; i < n; ++i) mx = fmax_c(mx, xv[i]);
    memset(Lb, 0, sizeof Lb);
    if (S->eps > 0 ? mx < S->eps : mx == 0) return 0;
    float scale, base, best = 0;
    if (S->start) {
        scale = qp_quants(n, qmax + 1, xv, (uint8_t*)Lb, w);
        base = scale * qmax;
        if (base <= 0) return 0;
    } else {
        scale = mx / (2 * qmax - 1);
        base = mx;
    }
    for (int k = 0; k < G; ++k) on[k] = S->grid0;
    for (int is = -S->r; is <= S->r; ++is) {
        float id = (2 * qmax - 1 + is * S->step) / base;
        float this_scale = 1 / id;
        for (int k = 0; k < G; ++k) {
            int u = 0;
            for (int c = 0; c < D; ++c) {
                int l = clampi(rint_bias(0.5f * (id * xv[D * k + c] - 1)), 0, qmax - 1);
                La[D * k + c] = (int8_t)l;
                u |= l << (B * c);
            }
            int g = T->map[u];
            on_a[k] = g >= 0;
            if (g < 0) {
                g = nearest_listed(T, T->nb - T->map[u] - 1, xv + D * k, ws + D * k, this_scale);
                if (g < 0) return -1;
                for (int c = 0; c < D; ++c) La[D * k + c] = (int8_t)((T->pt[g * D + c] - 1) / 2);
            }
        }
        float sqx = 0, sq2 = 0;
        for (int i = 0; i < n; ++i) {
            float q = 2 * La[i] + 1;
            sqx += w[i] * xv[i] * q;
            sq2 += w[i] * q * q;
        }
        if (sq2 > 0 && sqx * sqx > best * sq2) {
            scale = sqx / sq2;
            best = scale * sqx;
            memcpy(Lb, La, n);
            memcpy(on, on_a, sizeof on);
        }
    }
    int off = 0;
    for (int k = 0; k < G; ++k) off += !on[k];
    if (S->refit == 2 ? scale > 0 : off > 0 && scale > 0) {
        float id = 1 / scale;
        for (int k = 0; k < G; ++k) {
            if (S->refit == 0 && on[k]) continue;
            int u = 0;
            for (int c = 0; c < D; ++c) u |= clampi(rint_bias(0.5f * (id * xv[D * k + c] - 1)), 0, qmax - 1) << (B * c);
            int g = T->map[u];
            if (g < 0) {
                g = nearest_listed(T, T->nb - T->map[u] - 1, xv + D * k, ws + D * k, scale);
                if (g < 0) return -1;
            }
            for (int c = 0; c < D; ++c) Lb[D * k + c] = (int8_t)((T->pt[g * D + c] - 1) / 2);
        }
        float sqx = 0, sq2 = 0;
        for (int i = 0; i < n; ++i) {
            float q = 2 * Lb[i] + 1;
            sqx += w[i] * xv[i] * q;
            sq2 += w[i] * q * q;
        }
        if (sq2 > 0) scale = sqx / sq2;
    }
    if (scale < 0) {
        scale = -scale;
        for (int k = 0; k < n / 8; ++k) sgn[k] = S->parity ? (uint8_t)(~sgn[k] & 127) : (uint8_t)~sgn[k];
    }
    for (int k = 0; k < G; ++k) {
        int u = 0;
        for (int c = 0; c < D; ++c) u |= Lb[D * k + c] << (B * c);
        u &= 0xffff;
        if (u >= T->nmap || T->map[u] < 0) return -1;
        gidx[k] = T->map[u];
    }
    *scale_out = scale;
    return 1;
}

enum { T_IQ2_XXS = 16, T_IQ2_XS = 17, T_IQ3_XXS = 18, T_IQ1_S = 19, T_IQ3_S = 21, T_IQ2_S = 22, T_IQ1_M = 29 };

/* One super-block of a lattice type: the sub-block searches, the packing of grid points, signs and
   4-bit sub-block scales, and the half super-block scale (layouts of ggml-common.h:381-421). */
static int lattice_block(int type, const float* xbl, const float* qw, uint8_t* y) {
    const Sub* S = type == T_IQ2_XXS ? &SUB_IQ2_XXS : type == T_IQ2_XS ? &SUB_IQ2_XS : type == T_IQ2_S ? &SUB_IQ2_S
                 : type == T_IQ3_XXS ? &SUB_IQ3_XXS : &SUB_IQ3_S;
    const int bytes = type == T_IQ2_XXS ? 66 : type == T_IQ2_XS ? 74 : type == T_IQ2_S ? 82 : type == T_IQ3_XXS ? 98 : 110;
    if (!qw && (type == T_IQ2_XXS || type == T_IQ2_XS)) return -1;   /* "missing quantization weights" */
    const int n = S->n, nsub = QK / n;
    memset(y, 0, bytes);
    float sumx2 = 0;
    for (int i = 0; i < QK; ++i) sumx2 += xbl[i] * xbl[i];
    float sigma2 = (type == T_IQ2_XXS || type == T_IQ2_XS) ? sumx2 / QK : 2 * sumx2 / QK;
    float scales[16], max_scale = 0;
    int qs_at = 0, sg_at = 0;   /* IQ3_S: cursors that advance past coded sub-blocks only */
    for (int ib = 0; ib < nsub; ++ib) {
        const float* xb = xbl + n * ib;
        float w[32];
        for (int i = 0; i < n; ++i)
            w[i] = qw ? qw[n * ib + i] * sqrtf(sigma2 + xb[i] * xb[i])
                 : type == T_IQ2_S ? 0.25f * sigma2 + xb[i] * xb[i] : xb[i] * xb[i];
        float sc;
        int g[8];
        uint8_t s[4];
        int r = lattice_sub(S, xb, w, &sc, g, s);
        if (r < 0) return -1;
        if (r == 0) {
            scales[ib] = 0;
            continue;
        }
        if (type == T_IQ2_XXS) {         /* qs: per sub-block a u32 of 4 point bytes, a u32 of 4 x 7 sign bits */
            uint32_t a = 0, b = 0;
            for (int k = 0; k < 4; ++k) {
                a |= (uint32_t)g[k] << 8 * k;
                b |= (uint32_t)s[k] << 7 * k;
            }
            put32(y + 2 + 8 * ib, a);
            put32(y + 6 + 8 * ib, b);
        } else if (type == T_IQ2_XS) {   /* qs: u16 per group, 9-bit point and 7 sign bits */
            for (int k = 0; k < 2; ++k) put16(y + 2 + 2 * (2 * ib + k), (uint16_t)(g[k] | s[k] << 9));
        } else if (type == T_IQ2_S) {    /* qs: point low bytes, then sign bytes; qh: 2 high bits per point */
            for (int k = 0; k < 2; ++k) {
                int j = 2 * ib + k;
                y[2 + j] = (uint8_t)g[k];
                y[66 + j / 4] |= (uint8_t)((g[k] >> 8) << 2 * (j % 4));
                y[2 + 32 + j] = s[k];
            }
        } else if (type == T_IQ3_XXS) {  /* qs: 8 point bytes per sub-block, then a u32 of 4 x 7 sign bits */
            for (int k = 0; k < 8; ++k) y[2 + 8 * ib + k] = (uint8_t)g[k];
            put32(y + 2 + 64 + 4 * ib, (uint32_t)s[0] | (uint32_t)s[1] << 7 | (uint32_t)s[2] << 14 | (uint32_t)s[3] << 21);
        } else {                         /* IQ3_S: qs/signs at the cursors, qh at the absolute point */
            for (int k = 0; k < 8; ++k) {
                int j = 8 * ib + k;
                y[2 + qs_at + k] = (uint8_t)g[k];
                y[66 + j / 8] |= (uint8_t)((g[k] >> 8) << (j % 8));
            }
            for (int k = 0; k < 4; ++k) y[74 + sg_at + k] = s[k];
            qs_at += 8;
            sg_at += 4;
        }
        if (!(sc >= 0)) return -1;
        scales[ib] = sc;
        max_scale = fmax_c(max_scale, sc);
    }
    if (!max_scale) {
        /* IQ2_XXS / IQ2_XS / IQ3_XXS clear qs (their sub-block data were staged); IQ2_S / IQ3_S keep theirs */
        if (type == T_IQ2_XXS || type == T_IQ2_XS || type == T_IQ3_XXS) memset(y, 0, bytes);
        return 0;
    }
    float d = max_scale / 31;
    put16(y, og_half_bits(S->fudge == 1.f ? d : d * S->fudge));
    float id = 1 / d;
    for (int ib = 0; ib < nsub; ++ib) {
        int l = clampi(rint_bias(0.5f * (id * scales[ib] - 1)), 0, 15);
        if (type == T_IQ2_XXS) y[2 + 8 * ib + 7] |= (uint8_t)(l << 4);
        else if (type == T_IQ3_XXS) y[2 + 64 + 4 * ib + 3] |= (uint8_t)(l << 4);
        else if (type == T_IQ3_S) y[106 + ib / 2] |= (uint8_t)(l << 4 * (ib % 2));
        else y[(type == T_IQ2_XS ? 66 : 74) + ib / 2] |= (uint8_t)(l << 4 * (ib % 2));
    }
    return 0;
}

/* ------------------------------------------------------------------ IQ1_S / IQ1_M */

static const float IQ1_XP[3] = {-1 + 0.125f, 0.125f, 1 + 0.125f};   /* IQ1S_DELTA = IQ1M_DELTA = 0.125 */
static const float IQ1_XM[3] = {-1 - 0.125f, -0.125f, 1 - 0.125f};

/* The listed point nearest to xb/scale where coordinate value c stands for xx[(c-1)/2], in the
   plain importance-weighted norm, first on ties (ggml-quants.c:4444-4464). The reference's
   whole-grid fallback (:4465-4480) runs only when no listed distance is below FLT_MAX; it indexes
   xval by the grid point and then asserts, so it is treated as the abort it ends in (-1). */
static int iq1_nearest_listed(const Lattice* T, const uint16_t* list, const float* xb, const float* w, float scale,
                              const float* xx) {
    int best = -1;
    float bd = FLT_MAX;
    for (int j = 1; j <= list[0]; ++j) {
        const uint8_t* p = T->pt + (size_t)list[j] * 8;
        float d2 = 0;
        for (int c = 0; c < 8; ++c) {
            float q = xx[(p[c] - 1) / 2];
            float diff = scale * q - xb[c];
            d2 += w[c] * diff * diff;
        }
        if (d2 < bd) {
            bd = d2;
            best = list[j];
        }
    }
    return best;
}

/* ascending by value, stable (the reference's qsort over (value, index) pairs compares values
   only, ggml-quants.c:4501-4505; glibc's merge sort and the reference GPU path's insertion sort
   both keep the index order of equal values) */
static void sort_order(const float* x, int n, int* ord) {
    for (int j = 0; j < n; ++j) {
        int i = j;
        while (i > 0 && x[ord[i - 1]] > x[j]) {
            ord[i] = ord[i - 1];
            --i;
        }
        ord[i] = j;
    }
}

/* The points of an IQ1 sub-block once its levels are fixed: each 8-weight group's point, the
   nearest listed point when its levels are off the grid, and the refit of the scale over the
   chosen points when any group moved (ggml-quants.c:4610-4637, :4820-4854). xx_of(k) selects
   the shifted level values of group k. */
static int iq1_points(const Lattice* T, int groups, const int8_t* L, const float* xb, const float* w,
                      const float* const* xx, float* scale, int* idx) {
    int all = 1;
    for (int k = 0; k < groups; ++k) {
        int u = 0;
        for (int c = 0; c < 8; ++c) u |= L[8 * k + c] << 2 * c;
        int g = T->map[u];
        if (g < 0) {
            all = 0;
            g = iq1_nearest_listed(T, T->nb - T->map[u] - 1, xb + 8 * k, w + 8 * k, *scale, xx[k]);
            if (g < 0) return -1;
        }
        idx[k] = g;
    }
    if (!all) {
        float sqx = 0, sq2 = 0;
        for (int k = 0; k < groups; ++k) {
            const uint8_t* p = T->pt + (size_t)idx[k] * 8;
            for (int c = 0; c < 8; ++c) {
                float ww = w[8 * k + c];
                float q = xx[k][(p[c] - 1) / 2];
                sqx += ww * q * xb[8 * k + c];
                sq2 += ww * q * q;
            }
        }
        if (sqx > 0 && sq2 > 0) *scale = sqx / sq2;
    }
    return 0;
}

static void split_levels(const int* ord, int n, int i1, int i2, int8_t* L) {
    for (int j = 0; j < n; ++j) L[ord[j]] = (int8_t)(j < i1 ? 0 : j < i2 ? 1 : 2);
}

/* ggml-quants.c:4509-4671: IQ1_S super-block. Per 32-weight sub-block an exhaustive search over
   the two split points of the sorted weights for levels {-1, 0, 1} + shift, with prefix sums. */
static int iq1s_block(const float* xbl, const float* qw, uint8_t* y) {
    const Lattice* T = &LAT[2];
    if (!qw) return -1;   /* "missing quantization weights" */
    memset(y, 0, 50);
    float sumx2 = 0;
    for (int i = 0; i < QK; ++i) sumx2 += xbl[i] * xbl[i];
    float sigma2 = 2 * sumx2 / QK;
    float scales[8], max_scale = 0;
    int shifts[8];
    for (int ib = 0; ib < 8; ++ib) {
        const float* xb = xbl + 32 * ib;
        float w[32];
        for (int i = 0; i < 32; ++i) w[i] = qw[32 * ib + i] * sqrtf(sigma2 + xb[i] * xb[i]);
        float mx = fabsf(xb[0]);
        for (int i = 1; i < 32; ++i) mx = fmax_c(mx, fabsf(xb[i]));
        scales[ib] = 0;
        shifts[ib] = 1;
        if (mx < 1e-12f) continue;
        int ord[32];
        sort_order(xb, 32, ord);
        float sx[33], sw[33];
        sx[0] = sw[0] = 0;
        for (int j = 0; j < 32; ++j) {
            int i = ord[j];
            sx[j + 1] = sx[j] + w[i] * xb[i];
            sw[j + 1] = sw[j] + w[i];
        }
        float best = -FLT_MAX, scale = mx;
        int b1 = -1, b2 = -1, shift = 0;
        for (int i1 = 0; i1 <= 32; ++i1)
            for (int i2 = i1; i2 <= 32; ++i2)
                for (int sgn = 1; sgn >= -1; sgn -= 2) {
                    const float* v = sgn == 1 ? IQ1_XP : IQ1_XM;
                    float sqx = (sx[i1] - sx[0]) * v[0] + (sx[i2] - sx[i1]) * v[1] + (sx[32] - sx[i2]) * v[2];
                    float sq2 = (sw[i1] - sw[0]) * v[0] * v[0] + (sw[i2] - sw[i1]) * v[1] * v[1] + (sw[32] - sw[i2]) * v[2] * v[2];
                    if (sq2 > 0 && sqx * sqx > best * sq2) {
                        scale = sqx / sq2;
                        best = scale * sqx;
                        b1 = i1;
                        b2 = i2;
                        shift = sgn;
                    }
                }
        if (b1 < 0 || b2 < 0 || shift == 0) continue;
        int8_t L[32];
        split_levels(ord, 32, b1, b2, L);
        if (scale < 0) {
            for (int j = 0; j < 32; ++j) L[j] = (int8_t)(2 - L[j]);
            scale = -scale;
            shift = -shift;
        }
        const float* xx = shift == 1 ? IQ1_XP : IQ1_XM;
        const float* xxs[4] = {xx, xx, xx, xx};
        int idx[4];
        if (iq1_points(T, 4, L, xb, w, xxs, &scale, idx) < 0) return -1;
        uint16_t h = 0;
        for (int k = 0; k < 4; ++k) {
            y[2 + 4 * ib + k] = (uint8_t)idx[k];
            h |= (uint16_t)((idx[k] >> 8) << 3 * k);
        }
        put16(y + 34 + 2 * ib, h);
        if (!(scale >= 0)) return -1;
        scales[ib] = scale;
        shifts[ib] = shift;
        max_scale = fmax_c(max_scale, scale);
    }
    if (!max_scale) return 0;
    float d = max_scale / 15;
    put16(y, og_half_bits(d * 1.125f));
    float id = 1 / d;
    for (int ib = 0; ib < 8; ++ib) {
        int l = clampi(rint_bias(0.5f * (id * scales[ib] - 1)), 0, 7);
        if (shifts[ib] == -1) l |= 8;
        put16(y + 34 + 2 * ib, (uint16_t)(get16(y + 34 + 2 * ib) | l << 12));
    }
    return 0;
}

/* shifted level values of IQ1_M group k (0: first 8 weights, 1: last 8) under sign pattern bk:
   0 (+,+), 1 (+,-), 2 (-,+), 3 (-,-) (ggml-quants.c:4754-4757, :4822-4823) */
static const float* iq1m_xx(int bk, int k) {
    return (k == 0 ? bk < 2 : bk % 2 == 0) ? IQ1_XP : IQ1_XM;
}

/* ggml-quants.c:4693-4916: IQ1_M super-block. 16-weight sub-blocks, each half with its own shift
   sign. variant 0 scores a split with per-half prefix sums (:4758-4803); variant 1 is the
   formulation before that change (variants/ggml-quants.pre-f95b0d9539.c: four running sums
   accumulated over the sorted weights for every split). */
static int iq1m_block(const float* xbl, const float* qw, uint8_t* y, int variant) {
    const Lattice* T = &LAT[2];
    static const uint8_t masks[4] = {0x00, 0x80, 0x08, 0x88};
    memset(y, 0, 56);
    float sumx2 = 0;
    for (int i = 0; i < QK; ++i) sumx2 += xbl[i] * xbl[i];
    float sigma2 = 2 * sumx2 / QK;
    float scales[16], max_scale = 0;
    int shifts[16];
    for (int ib = 0; ib < 16; ++ib) {
        const float* xb = xbl + 16 * ib;
        float w[16];
        for (int i = 0; i < 16; ++i) w[i] = qw ? qw[16 * ib + i] * sqrtf(sigma2 + xb[i] * xb[i]) : xb[i] * xb[i];
        float mx = fabsf(xb[0]);
        for (int i = 1; i < 16; ++i) mx = fmax_c(mx, fabsf(xb[i]));
        scales[ib] = 0;
        shifts[ib] = 0;
        if (mx < 1e-7f) continue;
        int ord[16];
        sort_order(xb, 16, ord);
        float best = -FLT_MAX, scale = mx;
        int b1 = -1, b2 = -1, bk = -1;
        float sqx[4], sq2[4];
        if (variant == 0) {
            float px[2][17], pw[2][17];
            px[0][0] = px[1][0] = pw[0][0] = pw[1][0] = 0;
            for (int j = 0; j < 16; ++j) {
                int i = ord[j], h = i < 8 ? 0 : 1;
                px[h][j + 1] = px[h][j] + w[i] * xb[i];
                px[1 - h][j + 1] = px[1 - h][j];
                pw[h][j + 1] = pw[h][j] + w[i];
                pw[1 - h][j + 1] = pw[1 - h][j];
            }
            const float tx[2] = {px[0][16], px[1][16]}, tw[2] = {pw[0][16], pw[1][16]};
            const float p2 = IQ1_XP[2], m2 = IQ1_XM[2];
            const float cp1 = IQ1_XP[0] * IQ1_XP[0] - IQ1_XP[1] * IQ1_XP[1], cp2 = IQ1_XP[1] * IQ1_XP[1] - IQ1_XP[2] * IQ1_XP[2];
            const float cm1 = IQ1_XM[0] * IQ1_XM[0] - IQ1_XM[1] * IQ1_XM[1], cm2 = IQ1_XM[1] * IQ1_XM[1] - IQ1_XM[2] * IQ1_XM[2];
            for (int i1 = 0; i1 <= 16; ++i1)
                for (int i2 = i1; i2 <= 16; ++i2) {
                    float qp[2], qm[2], rp[2], rm[2];
                    for (int h = 0; h < 2; ++h) {
                        float s = px[h][i1] + px[h][i2];
                        qp[h] = tx[h] * p2 - s;
                        qm[h] = tx[h] * m2 - s;
                        rp[h] = tw[h] * p2 * p2 + pw[h][i1] * cp1 + pw[h][i2] * cp2;
                        rm[h] = tw[h] * m2 * m2 + pw[h][i1] * cm1 + pw[h][i2] * cm2;
                    }
                    sqx[0] = qp[0] + qp[1]; sqx[1] = qp[0] + qm[1]; sqx[2] = qm[0] + qp[1]; sqx[3] = qm[0] + qm[1];
                    sq2[0] = rp[0] + rp[1]; sq2[1] = rp[0] + rm[1]; sq2[2] = rm[0] + rp[1]; sq2[3] = rm[0] + rm[1];
                    for (int k = 0; k < 4; ++k)
                        if (sq2[k] > 0 && sqx[k] * sqx[k] > best * sq2[k]) {
                            scale = sqx[k] / sq2[k];
                            best = scale * sqx[k];
                            b1 = i1; b2 = i2; bk = k;
                        }
                }
        } else {
            for (int i1 = 0; i1 <= 16; ++i1)
                for (int i2 = i1; i2 <= 16; ++i2) {
                    for (int k = 0; k < 4; ++k) sqx[k] = sq2[k] = 0;
                    for (int j = 0; j < 16; ++j) {
                        int i = ord[j], seg = j < i1 ? 0 : j < i2 ? 1 : 2;
                        for (int k = 0; k < 4; ++k) {
                            float v = iq1m_xx(k, i < 8 ? 0 : 1)[seg];
                            sqx[k] += w[i] * v * xb[i];
                            sq2[k] += w[i] * v * v;
                        }
                    }
                    for (int k = 0; k < 4; ++k)
                        if (sq2[k] > 0 && sqx[k] * sqx[k] > best * sq2[k]) {
                            scale = sqx[k] / sq2[k];
                            best = scale * sqx[k];
                            b1 = i1; b2 = i2; bk = k;
                        }
                }
        }
        if (b1 < 0 || b2 < 0 || bk < 0) continue;
        int8_t L[16];
        split_levels(ord, 16, b1, b2, L);
        if (scale < 0) {
            for (int j = 0; j < 16; ++j) L[j] = (int8_t)(2 - L[j]);
            scale = -scale;
            bk = 3 - bk;
        }
        const float* xxs[2] = {iq1m_xx(bk, 0), iq1m_xx(bk, 1)};
        int idx[2];
        if (iq1_points(T, 2, L, xb, w, xxs, &scale, idx) < 0) return -1;
        y[2 * ib] = (uint8_t)idx[0];
        y[2 * ib + 1] = (uint8_t)idx[1];
        y[32 + ib] = (uint8_t)((idx[0] >> 8) | (idx[1] >> 8) << 4);
        if (!(scale >= 0)) return -1;
        scales[ib] = scale;
        shifts[ib] = bk;
        max_scale = fmax_c(max_scale, scale);
    }
    if (!max_scale) return 0;
    /* sub-block scales (3 bits), shift bits, and the super-block scale refit over every sub-block's
       chosen points (skipped sub-blocks take part with point 0 and scale level 0) */
    float d = max_scale / 15;
    float id = 1 / d;
    float sqx = 0, sq2 = 0;
    uint16_t sc[4] = {0, 0, 0, 0};
    for (int ib = 0; ib < 16; ++ib) {
        int l = clampi(rint_bias(0.5f * (id * scales[ib] - 1)), 0, 7);
        sc[ib / 4] |= (uint16_t)(l << 3 * (ib % 4));
        y[32 + ib] |= masks[shifts[ib]];
        const float* xb = xbl + 16 * ib;
        float w[16];
        for (int i = 0; i < 16; ++i) w[i] = qw ? qw[16 * ib + i] * sqrtf(sigma2 + xb[i] * xb[i]) : xb[i] * xb[i];
        for (int k = 0; k < 2; ++k) {
            const float* xx = iq1m_xx(shifts[ib], k);
            int g = y[2 * ib + k] + ((y[32 + ib] << (8 - 4 * k)) & 0x700);
            const uint8_t* p = T->pt + (size_t)g * 8;
            for (int c = 0; c < 8; ++c) {
                float ww = w[8 * k + c];
                float q = xx[(p[c] - 1) / 2] * (2 * l + 1);
                sqx += ww * q * xb[8 * k + c];
                sq2 += ww * q * q;
            }
        }
    }
    if (sq2 > 0) d = sqx / sq2;
    uint16_t s = og_half_bits(d * 1.1125f);
    sc[0] |= (uint16_t)((s & 0x000f) << 12);
    sc[1] |= (uint16_t)((s & 0x00f0) << 8);
    sc[2] |= (uint16_t)((s & 0x0f00) << 4);
    sc[3] |= (uint16_t)(s & 0xf000);
    for (int j = 0; j < 4; ++j) put16(y + 48 + 2 * j, sc[j]);
    return 0;
}

/* ------------------------------------------------------------------ entry */

/* quantize_<type>(src, dst, nrow, n_per_row, imatrix) for the seven lattice types (the row loops of
   ggml-quants.c:3653-3675, :4153-4163, :4354-4375, :4673-4690, :4918-4935, :5283-5293): every row
   restarts the imatrix. Returns the bytes written, or -1 where the reference aborts / the type or
   its tables are not available. */
int64_t og_quantize(int type, int variant, const float* src, uint8_t* dst, int64_t nrow, int64_t n_per_row,
                    const float* imatrix) {
    int li, bytes;
    switch (type) {
        case T_IQ2_XXS: li = 0; bytes = 66; break;
        case T_IQ2_XS: li = 1; bytes = 74; break;
        case T_IQ2_S: li = 3; bytes = 82; break;
        case T_IQ3_XXS: li = 4; bytes = 98; break;
        case T_IQ3_S: li = 5; bytes = 110; break;
        case T_IQ1_S: li = 2; bytes = 50; break;
        case T_IQ1_M: li = 2; bytes = 56; break;
        default: return -1;
    }
    if (!LAT[li].pt || n_per_row % QK || (variant != 0 && type != T_IQ1_M) || variant < 0 || variant > 1) return -1;
    const int64_t nbl = n_per_row / QK;
    for (int64_t r = 0; r < nrow; ++r)
        for (int64_t b = 0; b < nbl; ++b) {
            const float* x = src + r * n_per_row + b * QK;
            const float* qw = imatrix ? imatrix + b * QK : NULL;
            uint8_t* y = dst + (r * nbl + b) * bytes;
            int rc = type == T_IQ1_S ? iq1s_block(x, qw, y) : type == T_IQ1_M ? iq1m_block(x, qw, y, variant)
                                                                               : lattice_block(type, x, qw, y);
            if (rc < 0) return -1;
        }
    return nrow * nbl * bytes;
}
