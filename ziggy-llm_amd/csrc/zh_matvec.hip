// zh_matvec.hip -- host-side planning and dispatch of the batch-1
// dequant-matvec kernels (templates in zh_mv.h, instantiated by the
// zh_mv_*.hip files), and the bit-exact dequant kernels.
#include <utility>

#include "zh_mv.h"

namespace zh {

// Rows per team so that the grid has at most target_wgs workgroups, or one
// row per team when the matrix is too small to fill them.
// Rows per team of each segment for an even byte budget per team: segment i
// takes rpt_i = max(1, W / row_bytes_i) rows per team, with W the smallest
// budget whose grid fits in target_wgs workgroups.  (A grid one workgroup
// over the CU count runs a second round on one CU and doubles the launch;
// equal row counts across a Q4_K and a Q6_K segment leave the Q6_K
// workgroups 1.46x the bytes.)
void plan_matvec(MvParams &p, int target_wgs) {
    p.slots = p.cols / 64;
    p.team = team_width(p.cols);
    const int teams = kThreads / p.team;
    if (target_wgs < 1) target_wgs = 1;
    auto rpt_of = [&](int i, uint64_t W) {
        const uint64_t rb = p.seg[i].stride ? p.seg[i].stride : 1;
        const uint64_t r = W / rb;
        return (int)(r < 1 ? 1 : r > (1u << 20) ? (1u << 20) : r);
    };
    auto wgs_of = [&](uint64_t W) {
        int64_t g = 0;
        for (int i = 0; i < p.nseg; i++) {
            const int per = teams * rpt_of(i, W);
            g += (p.seg[i].rows + per - 1) / per;
        }
        return g;
    };
    uint64_t lo = 1, hi = 1;
    for (int i = 0; i < p.nseg; i++) hi += (uint64_t)p.seg[i].rows * (p.seg[i].stride ? p.seg[i].stride : 1);
    while (lo < hi) {  // smallest W with wgs_of(W) <= target (wgs_of never grows with W)
        const uint64_t mid = lo + (hi - lo) / 2;
        if (wgs_of(mid) <= target_wgs) hi = mid;
        else lo = mid + 1;
    }
    int wg = 0, rmax = 1;
    for (int i = 0; i < p.nseg; i++) {
        const int rpt = rpt_of(i, lo);
        rmax = rpt > rmax ? rpt : rmax;
        p.seg[i].rows_per_wg = teams * rpt;
        p.seg[i].wg_begin = wg;
        wg += (p.seg[i].rows + teams * rpt - 1) / (teams * rpt);
    }
    p.rows_per_team = rmax;
    for (int i = p.nseg; i < kMaxSeg; i++) p.seg[i].wg_begin = 0x7fffffff;
}

static int total_wgs(const MvParams &p) {
    int wg = 0;
    for (int i = 0; i < p.nseg; i++) wg += (p.seg[i].rows + p.seg[i].rows_per_wg - 1) / p.seg[i].rows_per_wg;
    return wg;
}

// Ring batches of the fast path; ZIGGY_HIP_MATVEC_NB forces 1, 2 or 3 (a tuning knob).
int forced_nb() {
    static int v = [] {
        const char *e = getenv("ZIGGY_HIP_MATVEC_NB");
        const int n = e ? atoi(e) : 0;
        return n >= 1 && n <= 3 ? n : 0;
    }();
    return v;
}

static int device_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return cus;
}

// Workgroups per CU of a matvec grid.  Grids are whole multiples of the CU
// count: every CU then streams the same number of rows (within one), where a
// partial second round of workgroups would double the time of the CUs that
// take one.  ZIGGY_HIP_MATVEC_WPC overrides the default (a tuning knob).
static float workgroups_per_cu() {
    static float w = [] {
        const char *e = getenv("ZIGGY_HIP_MATVEC_WPC");
        const float v = e ? (float)atof(e) : 1.0f;
        return v > 0.f ? v : 1.0f;
    }();
    return w;
}

// Bytes of the first c columns of a row (c a multiple of the format's block).
static uint64_t column_bytes(int fmt, int c) {
    auto of = [&](auto geom) { return (uint64_t)c / decltype(geom)::kValues * decltype(geom)::kBytes; };
    switch (fmt) {
    case Q4_K: return of(Geom<Q4_K>{});
    case Q6_K: return of(Geom<Q6_K>{});
    case Q3_K: return of(Geom<Q3_K>{});
    case IQ4_XS: return of(Geom<IQ4_XS>{});
    case Q8_0: return of(Geom<Q8_0>{});
    case F16: return of(Geom<F16>{});
    default: return of(Geom<F32>{});
    }
}

static hipError_t launch_matvec_team(const MvParams &p_in, int in, int out, hipStream_t s);

int matvec_target_wgs() { return (int)(device_cus() * workgroups_per_cu() + 0.5f); }

// A row longer than one team covers (kMaxMatvecCols values: 256 lanes of 64)
// runs as column windows of that length, the first with the call's output
// mode and the rest adding onto it.  Plain and SiLU inputs only (a norm needs
// the whole row before any window); stored or added outputs only.
hipError_t launch_matvec(const MvParams &p_in, int in, int out, hipStream_t s) {
    if (p_in.cols <= kMaxMatvecCols) return launch_matvec_team(p_in, in, out, s);
    if ((in != IN_PLAIN && in != IN_SILU) || (out != OUT_STORE && out != OUT_ADD) || p_in.expert || p_in.pro_in)
        return hipErrorInvalidValue;
    for (int c0 = 0; c0 < p_in.cols; c0 += kMaxMatvecCols) {
        MvParams q = p_in;
        q.cols = p_in.cols - c0 < kMaxMatvecCols ? p_in.cols - c0 : kMaxMatvecCols;
        for (int i = 0; i < q.nseg; i++) {
            const uint64_t off = column_bytes(q.seg[i].fmt, c0);
            q.seg[i].w += off;
            if (q.seg[i].w2) q.seg[i].w2 += off;
            if (q.seg[i].x) q.seg[i].x += c0;
        }
        if (q.x) q.x += c0;
        if (q.x2) q.x2 += c0;
        const hipError_t e = launch_matvec_team(q, in, c0 == 0 ? out : OUT_ADD, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

static hipError_t launch_matvec_team(const MvParams &p_in, int in, int out, hipStream_t s) {
    MvParams p = p_in;
    int f1 = p.seg[0].fmt, f2 = f1;
    for (int i = 1; i < p.nseg; i++)
        if (p.seg[i].fmt != f1) f2 = p.seg[i].fmt;
    for (int i = 0; i < p.nseg; i++)
        if (p.seg[i].fmt != f1 && p.seg[i].fmt != f2) return hipErrorInvalidValue;
    plan_matvec(p, (int)(device_cus() * workgroups_per_cu() + 0.5f));
    const int n = p.rows_per_team;
    MvKernel k = nullptr;
    if (f1 == f2) {
        switch (f1) {
        case Q4_K: k = pick_mv_q4k(in, out, p.cols, n); break;
        case Q6_K: k = pick_mv_q6k(in, out, p.cols, n); break;
        case Q8_0: k = pick_mv_q8_0(in, out, p.cols, n); break;
        default: k = pick_mv_other(f1, in, out, p.cols, n); break;
        }
    } else if (in == IN_NORM && out == OUT_STORE && (f1 == Q4_K || f1 == Q6_K)) {
        // the q/k/v launch of a Q4_K_M layer: Q4_K and Q6_K segments
        k = pick_mv_mixed(f1, f2, p.cols, n);
    } else {
        // routed (IQ4_XS) and shared (Q3_K) experts of an MoE layer
        k = pick_mv_moe(f1, f2, in, out, p.cols);
    }
    if (!k) return hipErrorInvalidValue;
    int grid = total_wgs(p);
    if (grid <= 0) return hipSuccess;
    // the SWIGLU routing prologue: one more workgroup writes the route
    p.route_wg = out == OUT_SWIGLU && p.pro_in ? grid++ : -1;
    hipLaunchKernelGGL(k, dim3(grid), dim3(kThreads), 0, s, p);
    return hipGetLastError();
}

static bool seg_formats(const MvParams &p, int &f1, int &f2) {
    f1 = p.seg[0].fmt, f2 = f1;
    for (int i = 1; i < p.nseg; i++)
        if (p.seg[i].fmt != f1) f2 = p.seg[i].fmt;
    for (int i = 0; i < p.nseg; i++)
        if (p.seg[i].fmt != f1 && p.seg[i].fmt != f2) return false;
    return true;
}

bool moe_ffn_supported(int f1, int f2, int gate_cols, int down_cols) {
    return gate_cols <= kMaxMatvecCols && down_cols <= kPollRowMax && pick_moe_ffn(f1, f2, gate_cols, down_cols);
}

hipError_t launch_moe_ffn(const MvParams &gu, const MvParams &down, int *poll_err, float *refill, int refill_n,
                          hipStream_t s) {
    MvParams pg = gu, pd = down;
    int f1, f2, d1, d2;
    if (!seg_formats(pg, f1, f2) || !seg_formats(pd, d1, d2) || !poll_err || !pg.pro_in || !pd.pro_in ||
        pg.expert || pd.expert || (refill_n && !refill))
        return hipErrorInvalidValue;
    // the down segments take the gate/up launch's two formats
    if ((d1 != f1 && d1 != f2) || (d2 != f1 && d2 != f2)) return hipErrorInvalidValue;
    if (f1 != IQ4_XS) std::swap(f1, f2);
    const MoeFfnKernel k = pg.cols <= kMaxMatvecCols && pd.cols <= kPollRowMax ? pick_moe_ffn(f1, f2, pg.cols, pd.cols)
                                                                               : nullptr;
    if (!k) return hipErrorInvalidValue;
    // each part planned for the whole chip: the down workgroups wait while
    // gate/up streams, then stream their own rows
    const int target = (int)(device_cus() * workgroups_per_cu() + 0.5f);
    plan_matvec(pg, target);
    plan_matvec(pd, target);
    int ng = total_wgs(pg);
    pg.route_wg = ng++;  // the route writer: the last gate/up workgroup
    pd.route_wg = -1;
    const int nd = total_wgs(pd);
    if (ng <= 0 || nd <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k, dim3(ng + nd), dim3(kThreads), 0, s, pg, pd, ng, MvFuse{poll_err, refill, refill_n});
    return hipGetLastError();
}

// ---------------- bit-exact dequant (one thread per block) ----------------

template <int F>
__global__ void dequant_kernel(const uint8_t *__restrict__ w, uint64_t stride, float *__restrict__ out, int rows,
                               int cols) {
    constexpr int V = Geom<F>::kValues, B = Geom<F>::kBytes;
    const int blocks_per_row = cols / V;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * blocks_per_row) return;
    const int r = (int)(i / blocks_per_row), b = (int)(i % blocks_per_row);
    dequant_block<F>(w + (uint64_t)r * stride + (uint64_t)b * B, out + (uint64_t)r * cols + (uint64_t)b * V);
}

__global__ void dequant_dense_kernel(const uint8_t *__restrict__ w, uint64_t stride, float *__restrict__ out,
                                     int rows, int cols, int is_f16) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i % cols);
    const uint8_t *row = w + (uint64_t)r * stride;
    out[i] = is_f16 ? h2f(ld2(row + 2 * c)) : __uint_as_float(ld4(row + 4 * c));
}

hipError_t launch_dequant(int fmt, const uint8_t *w, uint64_t stride, float *out, int rows, int cols, hipStream_t s) {
    auto go = [&](auto kern, int values) {
        const long long n = (long long)rows * (cols / values);
        const int grid = (int)((n + 255) / 256);
        if (grid > 0) hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, s, w, stride, out, rows, cols);
        return hipGetLastError();
    };
    switch (fmt) {
    case Q4_K: return go(dequant_kernel<Q4_K>, 256);
    case Q6_K: return go(dequant_kernel<Q6_K>, 256);
    case Q8_0: return go(dequant_kernel<Q8_0>, 32);
    case Q3_K: return go(dequant_kernel<Q3_K>, 256);
    case IQ4_XS: return go(dequant_kernel<IQ4_XS>, 256);
    case F16:
    case F32: {
        const long long n = (long long)rows * cols;
        const int grid = (int)((n + 255) / 256);
        if (grid > 0)
            hipLaunchKernelGGL(dequant_dense_kernel, dim3(grid), dim3(256), 0, s, w, stride, out, rows, cols,
                               fmt == F16 ? 1 : 0);
        return hipGetLastError();
    }
    default: return hipErrorInvalidValue;
    }
}

}  // namespace zh
