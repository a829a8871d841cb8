// rmsnorm_wide.hpp -- the RMSNorm forward and backward for rows wider than the
// register-resident shapes hold (forward: more than 8192 16-byte slots, 32768
// fp32 or 65536 bf16 columns; backward: more than 16384 columns), with every
// row 16-byte aligned.  Included by rmsnorm.hip inside namespace agk.
//
// A row is cut into segments of kWideSegCols columns for its statistics and
// into chunks of kWideChunkCols columns for the element-wise pass, so a few
// long rows still spread over the whole GPU:
//
//   forward   wide_row_stats<S, kWideSumSq>  per (row, segment): sum of x^2
//             wide_row_finish<kWideSumSq>    per row: partials in a fixed
//                                            order -> inv_rms[row]
//             wide_fwd_scale<S>              per (row, chunk): y = (x*r)*gamma
//   backward  wide_row_stats<S, kWideDot>    per (row, segment): sum of g*x,
//                                            g = dy*gamma          (dx only)
//             wide_row_finish<kWideDot>      per row: s = r*r*dot/cols
//             wide_bwd_tiles<S, ACC>         per (row block, chunk): dx =
//                                            r*(g - x*s) and one fp32 dgamma
//                                            partial row per row block
//             dgamma_finalize                partial rows in fixed fp64 order
//                                            (more than one row block only)
//
// The formulas are the resident kernels' (same products, same association);
// only the order of the row sums differs (segment trees, then the segments
// over a fixed lane tree), and it depends only on cols.  Every launch shape depends only on
// rows and cols, so results are bit-identical run to run.
//
// The composition rms(x) * gamma (COMP: agk_rms_mul_bwd) runs the same
// kernels with g = gy*gamma rounded to storage (and written to dr) and the
// dgamma term gy * h, h = x*r rounded to storage.  Its dx is then the plain
// path's dx of dr with no gamma, and its tiles take the looped kernels' row
// blocking (bwd_rows_per_block), so its dgamma partial rows are the ones
// agk_mul_rowbcast_bwd writes for gy and h: both outputs bit-identical to the
// two calls it replaces.
//
// Scratch: the forward keeps its per-segment partial sums in the first
// nseg * 4 bytes of each row of y (y is written in full by the last kernel;
// x and y must not overlap -- the caller checks and takes the one-workgroup-
// per-row kernel when they do).  The backward keeps its partials and per-row
// coefficients in the caller's workspace (wide_ws_layout).

constexpr int kWideLanes = 256;         // lanes per workgroup of every wide kernel
constexpr int kWideSegCols = 4096;      // columns per segment of the row statistics
constexpr int kWideChunkCols = 2048;    // columns per chunk of the element-wise pass
constexpr int64_t kWideTiles = 2048;    // backward tiles aimed for (8 per CU)
constexpr int kWideMinCols = 16385;     // narrowest row the wide paths take (either dtype)
constexpr int kWideSumSq = 0;
constexpr int kWideDot = 1;
constexpr int kWideDotComp = 2;  // g rounded to storage (the composition)

inline int launch_finalize(const float* partials, float* dgamma, int64_t nblk, int cols,
                           int accumulate, hipStream_t st);

struct WidePlan {
    int64_t nseg = 0;  // segments per row
    int64_t nch = 0;   // chunks per row
    int64_t rb = 0;    // rows per backward tile
    int64_t nrb = 0;   // backward row blocks = dgamma partial rows
};

// Depends only on rows and cols (never on the dtype or the device), so the
// workspace size and the dgamma summation order are fixed by the shape.
inline WidePlan wide_plan(int64_t rows, int cols) {
    WidePlan p;
    p.nseg = (cols + kWideSegCols - 1) / kWideSegCols;
    p.nch = (cols + kWideChunkCols - 1) / kWideChunkCols;
    int64_t nrb = (kWideTiles + p.nch - 1) / p.nch;
    if (nrb > rows) nrb = rows;
    if (nrb < 1) nrb = 1;
    p.rb = (rows + nrb - 1) / nrb;
    p.nrb = (rows + p.rb - 1) / p.rb;
    return p;
}

inline size_t round256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Row blocking of the wide tiles: the plan's for the RMSNorm backward, the
// looped kernels' for the composition (see above).
inline void wide_blocking(int64_t rows, int cols, bool comp, int64_t& rb, int64_t& nrb) {
    if (comp) {
        rb = bwd_rows_per_block(rows);
        nrb = bwd_num_blocks(rows);
    } else {
        const WidePlan p = wide_plan(rows, cols);
        rb = p.rb;
        nrb = p.nrb;
    }
}

// Workspace layout of the wide backward: [segment sums: rows x nseg 8-byte
// slots] [coefficients: rows fp32] [dgamma partial rows: prows x cols fp32],
// each region 256-byte aligned.  The split path keeps each segment's fp32 sum
// in the low 4 bytes of its slot's place (float index row*nseg + seg of the
// region); the team path (wide_bwd_team) uses the whole 64-bit slot.  The row
// statistics come first, so a dx-only call needs only the bytes before the
// partial rows (wide_ws_stats_bytes).
struct WideWs {
    size_t partials = 0, segs = 0, coefs = 0, total = 0;
};
inline WideWs wide_ws_layout(int64_t rows, int cols, int64_t prows) {
    const WidePlan p = wide_plan(rows, cols);
    WideWs w;
    w.segs = 0;
    w.coefs = round256(static_cast<size_t>(rows) * static_cast<size_t>(p.nseg) * 8u);
    w.partials = w.coefs + round256(static_cast<size_t>(rows) * 4u);
    w.total = w.partials + round256(static_cast<size_t>(prows) * static_cast<size_t>(cols) * 4u);
    return w;
}
inline WideWs wide_ws_layout(int64_t rows, int cols, bool comp) {
    int64_t rb = 0, nrb = 0;
    wide_blocking(rows, cols, comp, rb, nrb);
    return wide_ws_layout(rows, cols, nrb);
}
// Bytes the wide backward (comp false) or the composition (comp true) needs.
inline size_t wide_ws_bytes(int64_t rows, int64_t cols, bool comp) {
    if (cols < kWideMinCols || rows <= 0) return 0;
    return wide_ws_layout(rows, static_cast<int>(cols), comp).total;
}
// Bytes the wide RMSNorm backward needs when it writes no dgamma: the row
// statistics only.
inline size_t wide_ws_stats_bytes(int64_t rows, int64_t cols) {
    if (cols < kWideMinCols || rows <= 0) return 0;
    return wide_ws_layout(rows, static_cast<int>(cols), int64_t{0}).partials;
}

// Per (row, segment): the segment's sum of x^2 (kWideSumSq) or of g*x with
// g = dy*gamma (kWideDot; kWideDotComp: g rounded to storage, gamma
// required), summed per lane over its slots in order, then over the wave's
// lanes (DPP tree) and the four waves in order.  Blocks are row-major over
// (row, segment).  Loads past the row end return zeros.
template <class S, int KIND>
__global__ __launch_bounds__(kWideLanes) void wide_row_stats(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ dy,
    const typename S::T* __restrict__ gamma, float* __restrict__ out, int64_t out_row_stride,
    int64_t rows, int cols, int64_t nseg) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NV = kWideSegCols / (W * kWideLanes);  // slots per lane
    __shared__ float red[2][kWideLanes / 64];
    const int64_t row = static_cast<int64_t>(blockIdx.x) / nseg;
    const int seg = static_cast<int>(static_cast<int64_t>(blockIdx.x) - row * nseg);
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    const rsrc_t rx = make_rsrc(x + row * static_cast<int64_t>(cols), row_bytes);
    const rsrc_t rd = make_rsrc(KIND != kWideSumSq ? dy + row * static_cast<int64_t>(cols) : x,
                                KIND != kWideSumSq ? row_bytes : 0u);
    const rsrc_t rg = make_rsrc(gamma, gamma ? row_bytes : 0u);
    uint32_t off[NV];
    u32x4 xv[NV], dv[NV], gv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = seg * kWideSegCols + (static_cast<int>(threadIdx.x) + k * kWideLanes) * W;
        off[k] = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
        xv[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off[k], 0, 0);
        if constexpr (KIND != kWideSumSq) {
            dv[k] = __builtin_amdgcn_raw_buffer_load_b128(rd, off[k], 0, 0);
            if (gamma) gv[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[k], 0, 0);
        }
    }
    float part[W];
#pragma unroll
    for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float fx[W];
        S::unpack(xv[k], fx);
        if constexpr (KIND == kWideSumSq) {
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] += fx[e] * fx[e];
        } else {
            float fd[W];
            S::unpack(dv[k], fd);
            if constexpr (KIND == kWideDotComp) {
                float gm[W];
                u32x4 q;
                S::unpack(gv[k], gm);
                stored_product<S>(fd, gm, q);
            } else if (gamma) {
                float gm[W];
                S::unpack(gv[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) fd[e] = fd[e] * gm[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] += fd[e] * fx[e];
        }
    }
    float v = 0.0f;
#pragma unroll
    for (int e = 0; e < W; ++e) v += part[e];
    v = row_sum<kWideLanes, 1>(v, red, 0);
    if (threadIdx.x == 0) out[row * out_row_stride + seg] = v;
    (void)rows;
}

// Per row (one wave of 64 lanes each, four rows per workgroup): the segment
// partials summed in a fixed order -- lane l adds partials l, l+64, l+128, ...
// in turn, then the lanes are added over the DPP tree of group_sum -- then
//   kWideSumSq: out[row] = 1/sqrt(sum/cols + eps)            (inv_rms)
//   otherwise:  out[row] = (r*r*dot) * (1/cols), r = inv_rms[row]
// Each lane's loads are issued before any is added, so a row of up to 256
// segments (1M columns) costs one round trip.
constexpr int kFinishRowsPerBlock = kWideLanes / 64;
template <int KIND>
__global__ __launch_bounds__(kWideLanes) void wide_row_finish(
    const float* __restrict__ partials, int64_t part_row_stride, const float* __restrict__ inv_rms,
    float* __restrict__ out, int64_t rows, int cols, int64_t nseg, float eps) {
    constexpr int kBatch = 4;
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kFinishRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform: the whole wave takes this row or none
    const float* p = partials + row * part_row_stride;
    float v = 0.0f;
    for (int64_t base = lane; base < nseg; base += 64 * kBatch) {
        float t[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int64_t i = base + 64 * u;
            t[u] = i < nseg ? p[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v += t[u];
    }
    v = group_sum<64>(v);
    if (lane != 0) return;
    if constexpr (KIND == kWideSumSq) {
        out[row] = 1.0f / sqrtf(v / static_cast<float>(cols) + eps);
        (void)inv_rms;
    } else {
        (void)eps;
        const float r = inv_rms[row];
        out[row] = (r * r * v) * (1.0f / static_cast<float>(cols));
    }
}

// Per (row, chunk): y = (x * r) * gamma (x * r without gamma), as the resident
// forward computes it.  Blocks are row-major over (row, chunk).
template <class S>
__global__ __launch_bounds__(kWideLanes) void wide_fwd_scale(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, typename S::T* __restrict__ y, int64_t rows, int cols,
    int64_t nch) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NV = kWideChunkCols / (W * kWideLanes);
    const int64_t row = static_cast<int64_t>(blockIdx.x) / nch;
    const int ch = static_cast<int>(static_cast<int64_t>(blockIdx.x) - row * nch);
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    const rsrc_t rx = make_rsrc(x + row * static_cast<int64_t>(cols), row_bytes);
    const rsrc_t ry = make_rsrc(y + row * static_cast<int64_t>(cols), row_bytes);
    const rsrc_t rg = make_rsrc(gamma, gamma ? row_bytes : 0u);
    const float r = inv_rms[row];
    uint32_t off[NV];
    u32x4 xv[NV], gv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = ch * kWideChunkCols + (static_cast<int>(threadIdx.x) + k * kWideLanes) * W;
        off[k] = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
        xv[k] = bload16_stream(rx, off[k]);
        if (gamma) gv[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[k], 0, 0);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float f[W];
        S::unpack(xv[k], f);
        if (gamma) {
            float gm[W];
            S::unpack(gv[k], gm);
#pragma unroll
            for (int e = 0; e < W; ++e) f[e] = (f[e] * r) * gm[e];
        } else {
#pragma unroll
            for (int e = 0; e < W; ++e) f[e] = f[e] * r;
        }
        bstore16_stream(ry, off[k], S::pack(f));
    }
    (void)rows;
}

// Per (row block, chunk): rows rb*RB .. of the block in order, each
//   g = dy*gamma, dx (+)= r*(g - x*s)     (s from wide_row_finish<kWideDot>)
// and each lane's dgamma terms dy*(x*r) added row by row in fp32, as the
// resident backward does (COMP: g rounded to storage and written to dr, the
// dgamma term dy*h with h = x*r rounded to storage).  The block's sums go to partial row rb (nrb > 1) or
// straight to dgamma (one row block: dgamma (+)= the sums).  The next row's
// slots are loaded while the current row is processed (a row past the block
// reads through a zero-size resource and returns zeros).  Blocks are
// row-major over (row block, chunk).  coefs == nullptr: no dx.
template <class S, bool ACC, bool COMP>
__global__ __launch_bounds__(kWideLanes) void wide_bwd_tiles(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, typename S::T* __restrict__ dr,
    const float* __restrict__ coefs, float* __restrict__ partials, float* __restrict__ dgamma,
    int64_t rows, int cols, int64_t nch, int64_t rb, int64_t nrb, int acc_dg) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NV = kWideChunkCols / (W * kWideLanes);
    const int64_t blk = static_cast<int64_t>(blockIdx.x) / nch;
    const int ch = static_cast<int>(static_cast<int64_t>(blockIdx.x) - blk * nch);
    const int64_t r0 = blk * rb;
    const int64_t r1 = r0 + rb < rows ? r0 + rb : rows;
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    const bool want_dx = coefs != nullptr;
    uint32_t off[NV];
    u32x4 gv[NV];
    const rsrc_t rg = make_rsrc(gamma, gamma ? row_bytes : 0u);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = ch * kWideChunkCols + (static_cast<int>(threadIdx.x) + k * kWideLanes) * W;
        off[k] = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
        gv[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[k], 0, 0);
    }
    float dg[NV][W];
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < W; ++e) dg[k][e] = 0.0f;

    struct Set {
        u32x4 xv[NV], dv[NV], ov[NV];
        float r, s;
    };
    auto issue = [&](Set& b, int64_t row) {
        const uint32_t n = row < r1 ? 1u : 0u;
        const int64_t rr = row < r1 ? row : r0;
        const int64_t e0 = rr * static_cast<int64_t>(cols);
        const rsrc_t rx = make_rsrc(x + e0, n * row_bytes);
        const rsrc_t rd = make_rsrc(dy + e0, n * row_bytes);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            b.xv[k] = bload16_stream(rx, off[k]);
            b.dv[k] = bload16_stream(rd, off[k]);
        }
        if constexpr (ACC) {
            const rsrc_t ro = make_rsrc(dx ? dx + e0 : dx, dx ? n * row_bytes : 0u);
#pragma unroll
            for (int k = 0; k < NV; ++k) b.ov[k] = bload16_stream(ro, off[k]);
        }
        b.r = inv_rms[rr];
        b.s = want_dx ? coefs[rr] : 0.0f;
    };
    Set cur, nxt;
    issue(cur, r0);
    for (int64_t row = r0; row < r1; ++row) {
        issue(nxt, row + 1);
        const float r = cur.r, s = cur.s;
        const rsrc_t rdx = make_rsrc(dx ? dx + row * static_cast<int64_t>(cols) : dx,
                                     (dx && want_dx) ? row_bytes : 0u);
        const rsrc_t rdr = make_rsrc(COMP ? dr + row * static_cast<int64_t>(cols) : dr,
                                     COMP ? row_bytes : 0u);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fx[W], fd[W], gk[W];
            S::unpack(cur.xv[k], fx);
            S::unpack(cur.dv[k], fd);
            if constexpr (COMP) {
                float gm[W];
                u32x4 q;
                S::unpack(gv[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) gk[e] = fd[e];
                stored_product<S>(gk, gm, q);
                bstore16_stream(rdr, off[k], q);
            } else if (gamma) {
                float gm[W];
                S::unpack(gv[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) gk[e] = fd[e] * gm[e];
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) gk[e] = fd[e];
            }
            if (want_dx) {
                float o[W];
#pragma unroll
                for (int e = 0; e < W; ++e) o[e] = r * (gk[e] - fx[e] * s);
                if constexpr (ACC) {
                    float old[W];
                    S::unpack(cur.ov[k], old);
#pragma unroll
                    for (int e = 0; e < W; ++e) o[e] = acc_add(old[e], o[e]);
                }
                bstore16_stream(rdx, off[k], S::pack(o));
            }
            if constexpr (COMP) {
                // as agk_mul_rowbcast_bwd's looped kernel: the product, then
                // an unfused add (the first row's term taken as it is)
                float h[W];
#pragma unroll
                for (int e = 0; e < W; ++e) h[e] = fx[e] * r;
                S::unpack(S::pack(h), h);
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const float t = fd[e] * h[e];
                    dg[k][e] = row == r0 ? t : acc_add(dg[k][e], t);
                }
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) dg[k][e] += fd[e] * (fx[e] * r);
            }
        }
        cur = nxt;
    }
    if (partials == nullptr && dgamma == nullptr) return;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (off[k] == kOffOut) continue;
        const int col = static_cast<int>(off[k] / sizeof(T));
        if (nrb > 1) {
            float* p = partials + blk * static_cast<int64_t>(cols) + col;
#pragma unroll
            for (int e = 0; e < W; e += 4)
                *reinterpret_cast<float4*>(p + e) =
                    make_float4(dg[k][e], dg[k][e + 1], dg[k][e + 2], dg[k][e + 3]);
        } else {
            // +0.0 + sum, as the finalize's fp64 sum from +0.0 gives it (a
            // lone -0.0 term becomes +0.0)
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const float v = 0.0f + dg[k][e];
                dgamma[col + e] = acc_dg ? dgamma[col + e] + v : v;
            }
        }
    }
}

// A row of cols elements the wide kernels can take: a multiple of the slot
// width, at least kWideMinCols, and short enough for 32-bit buffer offsets.
template <class S>
inline bool wide_cols_ok(int cols) {
    return cols >= kWideMinCols && (cols % S::kVec) == 0 &&
           static_cast<uint64_t>(cols) * sizeof(typename S::T) < 0x80000000ull;
}

// Whether [a, a+bytes) and [b, b+bytes) share a byte.
inline bool overlaps(const void* a, const void* b, size_t bytes) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + bytes && pb < pa + bytes;
}

// The wide forward's sizes: rows too wide for a resident shape (resident_plan
// false), any number of them (with many rows it still streams 1.6-2.9x faster
// than the one-workgroup-per-row kernel's element-wise passes).
template <class S>
inline bool wide_fwd_shape_ok(int64_t rows, int cols, bool resident_plan) {
    (void)rows;
    return !resident_plan && wide_cols_ok<S>(cols);
}

// ... and its pointers: 16-byte aligned, y not overlapping x (y holds the
// partial sums meanwhile).
template <class S>
inline bool wide_fwd_eligible(const void* x, const void* gamma, const void* y, int64_t rows,
                              int cols, bool resident_plan) {
    return wide_fwd_shape_ok<S>(rows, cols, resident_plan) && aligned16(x) && aligned16(y) &&
           (gamma == nullptr || aligned16(gamma)) &&
           !overlaps(x, y, static_cast<size_t>(rows) * static_cast<size_t>(cols) *
                               sizeof(typename S::T));
}

// The wide backward's arguments without the workspace: rows too wide for a
// resident shape, x, dy, dx (when given) and gamma (when given) 16-byte
// aligned.  The caller also needs a 16-byte aligned workspace of
// wide_ws_bytes(rows, cols).
template <class S>
inline bool wide_bwd_eligible(const void* x, const void* gamma, const void* dy, const void* dx,
                              int cols, bool resident_plan) {
    return !resident_plan && wide_cols_ok<S>(cols) && aligned16(x) && aligned16(dy) &&
           (dx == nullptr || aligned16(dx)) && (gamma == nullptr || aligned16(gamma));
}

template <class S>
int launch_wide_fwd(const void* x, const void* gamma, void* y, float* inv_rms, int64_t rows,
                    int cols, float eps, hipStream_t st) {
    using T = typename S::T;
    const WidePlan p = wide_plan(rows, cols);
    const int64_t nstat = rows * p.nseg, nscale = rows * p.nch;
    if (nstat > 0x7fffffffLL || nscale > 0x7fffffffLL) return AGK_EINVAL;
    const T* xp = static_cast<const T*>(x);
    T* yp = static_cast<T*>(y);
    // per-segment partials in the first nseg floats of each row of y
    float* part = static_cast<float*>(y);
    const int64_t stride = static_cast<int64_t>(cols) * static_cast<int64_t>(sizeof(T)) / 4;
    hipLaunchKernelGGL((wide_row_stats<S, kWideSumSq>), dim3(static_cast<unsigned>(nstat)),
                       dim3(kWideLanes), 0, st, xp, static_cast<const T*>(nullptr),
                       static_cast<const T*>(nullptr), part, stride, rows, cols, p.nseg);
    if (int rc = check_launch()) return rc;
    hipLaunchKernelGGL(wide_row_finish<kWideSumSq>,
                       dim3(static_cast<unsigned>((rows + kFinishRowsPerBlock - 1) /
                                                  kFinishRowsPerBlock)),
                       dim3(kWideLanes), 0, st, part, stride, static_cast<const float*>(nullptr),
                       inv_rms, rows, cols, p.nseg, eps);
    if (int rc = check_launch()) return rc;
    hipLaunchKernelGGL((wide_fwd_scale<S>), dim3(static_cast<unsigned>(nscale)), dim3(kWideLanes),
                       0, st, xp, static_cast<const T*>(gamma), inv_rms, yp, rows, cols, p.nch);
    return check_launch();
}

// ws: at least wide_ws_bytes(rows, cols, dr != nullptr) bytes, 16-byte
// aligned (checked by the caller).  dr != nullptr: the composition (gamma
// required), dr receiving g = gy*gamma rounded to storage.
template <class S>
int launch_wide_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
                    void* dx, void* dr, float* dgamma, void* ws, int64_t rows, int cols,
                    int acc_dx, int acc_dg, hipStream_t st) {
    using T = typename S::T;
    const bool comp = dr != nullptr;
    WidePlan p = wide_plan(rows, cols);
    wide_blocking(rows, cols, comp, p.rb, p.nrb);
    const WideWs w = wide_ws_layout(rows, cols, p.nrb);
    const int64_t nstat = rows * p.nseg, ntile = p.nrb * p.nch;
    if (nstat > 0x7fffffffLL || ntile > 0x7fffffffLL) return AGK_EINVAL;
    char* base = static_cast<char*>(ws);
    float* partials = reinterpret_cast<float*>(base + w.partials);
    float* segs = reinterpret_cast<float*>(base + w.segs);
    float* coefs = reinterpret_cast<float*>(base + w.coefs);
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* dyp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    T* drp = static_cast<T*>(dr);
    if (dx) {
        if (comp)
            hipLaunchKernelGGL((wide_row_stats<S, kWideDotComp>),
                               dim3(static_cast<unsigned>(nstat)), dim3(kWideLanes), 0, st, xp,
                               dyp, gp, segs, p.nseg, rows, cols, p.nseg);
        else
            hipLaunchKernelGGL((wide_row_stats<S, kWideDot>), dim3(static_cast<unsigned>(nstat)),
                               dim3(kWideLanes), 0, st, xp, dyp, gp, segs, p.nseg, rows, cols,
                               p.nseg);
        if (int rc = check_launch()) return rc;
        hipLaunchKernelGGL(wide_row_finish<kWideDot>,
                           dim3(static_cast<unsigned>((rows + kFinishRowsPerBlock - 1) /
                                                  kFinishRowsPerBlock)),
                           dim3(kWideLanes), 0, st, segs, p.nseg, inv_rms, coefs, rows, cols,
                           p.nseg, 0.0f);
        if (int rc = check_launch()) return rc;
    }
    float* part_arg = dgamma && p.nrb > 1 ? partials : nullptr;
    float* dg_arg = dgamma && p.nrb == 1 ? dgamma : nullptr;
    const float* coef_arg = dx ? coefs : nullptr;
    const dim3 grid(static_cast<unsigned>(ntile));
#define AGK_TILES(ACC_, COMP_)                                                               \
    hipLaunchKernelGGL((wide_bwd_tiles<S, ACC_, COMP_>), grid, dim3(kWideLanes), 0, st, xp, gp, \
                       inv_rms, dyp, dxp, drp, coef_arg, part_arg, dg_arg, rows, cols, p.nch,   \
                       p.rb, p.nrb, acc_dg)
    const bool acc = acc_dx && dx;
    if (comp) {
        if (acc) AGK_TILES(true, true);
        else AGK_TILES(false, true);
    } else {
        if (acc) AGK_TILES(true, false);
        else AGK_TILES(false, false);
    }
#undef AGK_TILES
    if (int rc = check_launch()) return rc;
    if (part_arg) return launch_finalize(partials, dgamma, p.nrb, cols, acc_dg, st);
    return AGK_OK;
}

// ---- one pass over rows of up to 32768 columns ----------------------------------
// Aligned rows of kWideMinCols..kWideResMaxCols columns and at least
// kWideResMinRows rows: one 1024-lane workgroup per row at a time, the row's x
// and dy in registers (NV 16-byte slots per lane: 8 fp32, 4 bf16), gamma
// re-read per row from L2, and each lane's dgamma columns in LDS (dgl,
// 128 KiB) instead of registers, which the row would not leave room for.
// Each lane adds to LDS only the columns it owns, so the accumulators need no
// barrier.  Before the row sum each slot yields g = dy*gamma, its share of
// the dot, the composition's dr and the dgamma term (which needs r, not the
// sum), so only x and g stay live across the sum.  x and dy are read once:
// the split path's second read disappears.
//   RMSNorm backward (COMP false): rows dealt round-robin to min(rows, 256)
//     workgroups (as the resident backward), the dgamma term dy*(x*r);
//   composition (COMP true): g rounded to storage and written to dr, the term
//     gy*h with h = x*r rounded to storage, added unfused in row order over
//     the looped kernels' contiguous row blocks (bwd_rows_per_block), so the
//     partial rows are agk_mul_rowbcast_bwd's.
// Both end with one fp32 partial row per workgroup (dgamma_finalize after);
// the dx arithmetic and its row sum are the same in both.
constexpr int kWideResLanes = 1024;
constexpr int kWideResMaxCols = 32768;
constexpr int64_t kWideResMinRows = 256;
constexpr int64_t kWideResBlocks = 256;

template <class S>
inline bool wide_res_eligible(const void* x, const void* gamma, const void* dy, const void* dx,
                              const void* dr, int64_t rows, int cols, bool resident_plan) {
    return !resident_plan && rows >= kWideResMinRows && cols <= kWideResMaxCols &&
           wide_cols_ok<S>(cols) && aligned16(x) && aligned16(dy) &&
           (dx == nullptr || aligned16(dx)) && (dr == nullptr || aligned16(dr)) &&
           (gamma == nullptr || aligned16(gamma));
}

// Row blocking of the one-pass kernel: (workgroups, contiguous rows per
// workgroup, 0 = round-robin).
inline void wide_res_blocking(int64_t rows, bool comp, int64_t& nblk, int64_t& rpb) {
    if (comp) {
        rpb = bwd_rows_per_block(rows);
        nblk = bwd_num_blocks(rows);
    } else {
        nblk = rows < kWideResBlocks ? rows : kWideResBlocks;
        rpb = 0;
    }
}

template <class S, bool ACC, bool COMP>
__global__ __launch_bounds__(kWideResLanes) void wide_bwd_resident(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, typename S::T* __restrict__ dr, float* __restrict__ partials,
    int64_t rows, int cols, int64_t rpb) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NV = kWideResMaxCols / (W * kWideResLanes);
    __shared__ float red[2][kWideResLanes / 64];
    __shared__ __align__(16) float dgl[kWideResMaxCols];
    const int t = threadIdx.x;
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    const bool want_dg = partials != nullptr;
    const bool want_dx = dx != nullptr;
    const float inv_cols = 1.0f / static_cast<float>(cols);
    // Slot k of lane t: columns (t + k*1024)*W ..  Offsets past the row end
    // read zeros and drop stores through the row's buffer resource.
    const uint32_t off0 = static_cast<uint32_t>(t * W) * sizeof(T);
    constexpr uint32_t kSlotStride = kWideResLanes * W * sizeof(T);
    const rsrc_t rg = make_rsrc(gamma, gamma ? row_bytes : 0u);
    if (want_dg) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = (t + k * kWideResLanes) * W;
            if (col < cols) {
#pragma unroll
                for (int e = 0; e < W; e += 4)
                    *reinterpret_cast<float4*>(dgl + col + e) = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }
    int64_t row, step, end;
    if (rpb > 0) {
        row = static_cast<int64_t>(blockIdx.x) * rpb;
        end = row + rpb < rows ? row + rpb : rows;
        step = 1;
    } else {
        row = blockIdx.x;
        end = rows;
        step = gridDim.x;
    }
    // The row's slots, and the next row's loaded into them slot by slot as
    // the dx loop frees them (a row past the end reads through a zero-size
    // resource).
    u32x4 xv[NV], dv[NV], gv[NV];
    float r_next = 0.0f;
    auto issue_slot = [&](int64_t rr, int k) {
        const uint32_t n = rr < end ? row_bytes : 0u;
        const int64_t e = (rr < end ? rr : 0) * static_cast<int64_t>(cols);
        xv[k] = bload16_stream(make_rsrc(x + e, n), off0 + k * kSlotStride);
        dv[k] = bload16_stream(make_rsrc(dy + e, n), off0 + k * kSlotStride);
        gv[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off0 + k * kSlotStride, 0, 0);
    };
    auto issue_r = [&](int64_t rr) { r_next = rr < end ? inv_rms[rr] : 0.0f; };
#pragma unroll
    for (int k = 0; k < NV; ++k) issue_slot(row, k);
    issue_r(row);
    int parity = 0;
    for (const int64_t first = row; row < end; row += step, parity ^= 1) {
        const int64_t e0 = row * static_cast<int64_t>(cols);
        const int64_t next = row + step;
        const rsrc_t rdr = make_rsrc(COMP ? dr + e0 : dr, COMP ? row_bytes : 0u);
        const float r = r_next;
        // Before the row sum: g = dy*gamma (kept for dx), its dot with x, the
        // composition's dr, and the dgamma terms (they need r, not the sum).
        float g[NV][W];
        float part[W];
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fx[W], fd[W];
            S::unpack(xv[k], fx);
            S::unpack(dv[k], fd);
#pragma unroll
            for (int e = 0; e < W; ++e) g[k][e] = fd[e];
            if constexpr (COMP) {
                float gm[W];
                u32x4 q;
                S::unpack(gv[k], gm);
                stored_product<S>(g[k], gm, q);
                bstore16_stream(rdr, off0 + k * kSlotStride, q);
            } else if (gamma) {
                float gm[W];
                S::unpack(gv[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) g[k][e] = fd[e] * gm[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] += g[k][e] * fx[e];
            const int col = (t + k * kWideResLanes) * W;
            if (want_dg && col < cols) {
                float* a = dgl + col;
                if constexpr (COMP) {
                    float h[W];
#pragma unroll
                    for (int e = 0; e < W; ++e) h[e] = fx[e] * r;
                    S::unpack(S::pack(h), h);
#pragma unroll
                    for (int e = 0; e < W; ++e) {
                        const float term = fd[e] * h[e];
                        a[e] = row == first ? term : acc_add(a[e], term);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) a[e] += fd[e] * (fx[e] * r);
                }
            }
        }
        if (!want_dx) {  // workgroup-uniform
#pragma unroll
            for (int k = 0; k < NV; ++k) issue_slot(next, k);
            issue_r(next);
            continue;
        }
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < W; ++e) dot += part[e];
        dot = row_sum<kWideResLanes, 1>(dot, red, parity);
        const float s = (r * r * dot) * inv_cols;
        const rsrc_t rdx = make_rsrc(dx + e0, row_bytes);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fx[W], o[W];
            S::unpack(xv[k], fx);
#pragma unroll
            for (int e = 0; e < W; ++e) o[e] = r * (g[k][e] - fx[e] * s);
            if constexpr (ACC) {
                float old[W];
                S::unpack(bload16_stream(rdx, off0 + k * kSlotStride), old);
#pragma unroll
                for (int e = 0; e < W; ++e) o[e] = acc_add(old[e], o[e]);
            }
            bstore16_stream(rdx, off0 + k * kSlotStride, S::pack(o));
            issue_slot(next, k);
        }
        issue_r(next);
    }
    if (!want_dg) return;
    float* prow = partials + static_cast<int64_t>(blockIdx.x) * cols;  // any 4-byte alignment
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int col = (t + k * kWideResLanes) * W;
        if (col < cols) {
#pragma unroll
            for (int e = 0; e < W; ++e) prow[col + e] = dgl[col + e];
        }
    }
}

// partials: nblk rows of cols floats when dgamma != nullptr (wide_res_blocking).
template <class S>
int launch_wide_res_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
                        void* dx, void* dr, float* partials, float* dgamma, int64_t rows,
                        int cols, int acc_dx, int acc_dg, hipStream_t st) {
    using T = typename S::T;
    const bool comp = dr != nullptr;
    int64_t nblk = 0, rpb = 0;
    wide_res_blocking(rows, comp, nblk, rpb);
    if (nblk > 0x7fffffffLL) return AGK_EINVAL;
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* dyp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    T* drp = static_cast<T*>(dr);
    float* part = dgamma ? partials : nullptr;
    const dim3 grid(static_cast<unsigned>(nblk));
#define AGK_RES(ACC_, COMP_)                                                                  \
    hipLaunchKernelGGL((wide_bwd_resident<S, ACC_, COMP_>), grid, dim3(kWideResLanes), 0, st, \
                       xp, gp, inv_rms, dyp, dxp, drp, part, rows, cols, rpb)
    const bool acc = acc_dx && dx;
    if (comp) {
        if (acc) AGK_RES(true, true);
        else AGK_RES(false, true);
    } else {
        if (acc) AGK_RES(true, false);
        else AGK_RES(false, false);
    }
#undef AGK_RES
    if (int rc = check_launch()) return rc;
    if (dgamma) return launch_finalize(partials, dgamma, nblk, cols, acc_dg, st);
    return AGK_OK;
}

// ---- one pass over rows wider than a workgroup holds: teams -----------------------
// Aligned rows of up to kTeamMaxSegs segments, at least kTeamMinRows of them,
// that the one-pass kernel above does not take (wider than 32768 columns, or
// fewer than 256 rows).  A team of P workgroups holds one row at a time in
// registers: workgroup p of the team owns segments [p*SEGS, (p+1)*SEGS) of
// kWideSegCols columns (SEGS = team_segs_for: 1 or 2 for fp32, 2 for bf16), with the
// same slots per lane as wide_row_stats.  Team t takes rows t, t+T, t+2T, ...
// (T = kTeamWorkgroups / P, at most the split path's row blocks, so the
// dgamma partial rows fit the same workspace region).  Per row each workgroup
//   1. sums g*x, g = dy*gamma, over each of its segments exactly as
//      wide_row_stats does (per lane over its slots in order, then the
//      wave's DPP tree and the four waves in order);
//   2. publishes each segment sum in the slot for (row, segment): one 64-bit
//      word holding a set flag in the high half and the float's bits in the
//      low half, stored at agent scope, so a reader sees either the cleared
//      word or the whole value;
//   3. reads the row's other slots: one wave polls them with agent-scope
//      loads, at most `wait_polls` times, and a sum still missing after that
//      is recomputed by the workgroup from x, dy and gamma with the same
//      arithmetic (the same bits), so the result never depends on which
//      workgroups are resident at once and every wait ends;
//   4. adds the segment sums as wide_row_finish does (lane l: segments l,
//      l+64, l+128, l+192 in turn from +0, then the DPP tree), so
//      s = (r*r*dot)/cols and every dx element r*(g - x*s) are the split
//      path's bits;
//   5. writes dx, while the loads of the team's next row, issued before
//      step 1, are in flight.
// Each lane adds its columns' dgamma terms dy*(x*r) in row order; at the end
// each workgroup writes its columns of partial row t, and dgamma_finalize
// adds the T partial rows in a fixed order.  The slots are cleared by a fill
// kernel ahead of the launch, in stream order, so a set flag means "written
// by this call".  x and dy are read once: the split path's second read
// disappears.  Without dx nothing is exchanged.
constexpr int64_t kTeamMaxSegs = 256;  // 1M columns; wider rows take the split path
constexpr int kTeamWaitPolls = 4096;   // polls before a missing sum is recomputed

constexpr int64_t kTeamMinRows = 4;   // fewer rows take the split path
// Workgroups a launch aims for: two 256-lane workgroups per CU of a 256-CU
// MI355X, all resident at once at the kernel's register use.  A constant, so
// the team count (and with it dgamma's summation order) depends only on the
// shape, never on the device.
constexpr int64_t kTeamWorkgroups = 512;

// Segments per workgroup, which the row's exchange is amortised over.  bf16:
// two (32 KiB of x and dy per row).  fp32: one (32 KiB), or two (64 KiB; gamma
// then staged in LDS instead of registers, so the row fits 237 VGPRs at two
// waves per SIMD) where one-segment parts would number 32 or more per row or
// a two-segment team gets at least 16 rows, and there are rows enough for
// two-segment teams to fill the grid (at [8, 262144] two segments took 16.9
// us against 16.5).  A function of rows and cols
// only, so the team count and dgamma's summation order are fixed by the
// shape.  Measured on MI355X (graph-replayed backward, dx and dgamma, us,
// one segment -> two): fp32 [2048, 65536] 284 -> 272, [4096, 65536] 559 ->
// 525, [2048, 131072] 704 -> 537, [256, 262144] 226 -> 161, [128, 524288]
// 246 -> 170, [4096, 40000] 358 -> 341; but [256, 65536] 46 -> 50 and
// [512, 65536] 81 -> 84 (four and eight rows per team: the pipeline of each
// team's rows too short).  bf16 [8192, 131072]: 1189 us with two segments
// against 1985 with one; gamma in LDS cost it 3 % (1179 -> 1212 us), and
// three segments (251 VGPRs) 1392 us.
inline int team_segs_for(int dtype, int64_t rows, int64_t cols) {
    if (dtype != AGK_F32) return 2;
    const int64_t parts1 = (cols + kWideSegCols - 1) / kWideSegCols;
    const int64_t parts2 = (cols + 2 * kWideSegCols - 1) / (2 * kWideSegCols);
    const int64_t teams2 = kTeamWorkgroups / parts2 > 0 ? kTeamWorkgroups / parts2 : 1;
    // two only where its teams still fill the grid (few rows want more parts)
    return rows >= teams2 && (parts1 >= 32 || rows >= 16 * teams2) ? 2 : 1;
}

struct TeamPlan {
    int64_t parts = 0;  // workgroups per row (team size)
    int64_t teams = 0;  // rows in flight = dgamma partial rows
};
inline TeamPlan team_plan(int64_t rows, int cols, int segs) {
    TeamPlan tp;
    const int64_t part_cols = static_cast<int64_t>(segs) * kWideSegCols;
    tp.parts = (cols + part_cols - 1) / part_cols;
    // at most the split path's row blocks (the workspace's partial rows)
    const int64_t nrb = wide_plan(rows, cols).nrb;
    const int64_t want = kTeamWorkgroups / tp.parts > 0 ? kTeamWorkgroups / tp.parts : 1;
    tp.teams = want < nrb ? want : nrb;
    return tp;
}

template <class S>
inline bool team_eligible(const void* x, const void* gamma, const void* dy, const void* dx,
                          int64_t rows, int cols, bool resident_plan) {
    const int64_t nseg = (cols + kWideSegCols - 1) / kWideSegCols;
    return wide_bwd_eligible<S>(x, gamma, dy, dx, cols, resident_plan) && nseg <= kTeamMaxSegs &&
           rows >= kTeamMinRows && !(rows >= kWideResMinRows && cols <= kWideResMaxCols);
}

__device__ __forceinline__ void slot_publish(uint64_t* p, float v) {
    const uint64_t w = (static_cast<uint64_t>(1) << 32) | __float_as_uint(v);
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t slot_read(uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Shared LDS of a team kernel's exchange: the row's segment sums, which of
// them a wait missed, and whether any did.  Each field is written for the
// next row only after a barrier that every wave reaches after reading it for
// the current one.
struct TeamXchg {
    float vals[kTeamMaxSegs];
    unsigned char missing[kTeamMaxSegs];
    int nmissing;
};

// Steps 2-3 of both team kernels (workgroup-uniform call, 256 lanes): this
// workgroup's kSegs segment sums v (segments seg0 ..) are published in the
// row's slots rs, wave 0 gathers the row's other segments' sums with at most
// `wait_polls` polls, and a sum still missing after that is recomputed by
// the whole workgroup with recompute(sg) (the publisher's arithmetic, so the
// same bits).  On return x.vals[0, nseg) holds every segment sum.
template <int kSegs, class Recompute>
__device__ __forceinline__ void team_gather(uint64_t* rs, const float (&v)[kSegs], int seg0,
                                            int nseg, int wait_polls, TeamXchg& x,
                                            Recompute recompute) {
    constexpr int kPerLane = static_cast<int>(kTeamMaxSegs / 64);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (t == 0) {
#pragma unroll
        for (int s = 0; s < kSegs; ++s)
            if (seg0 + s < nseg) slot_publish(rs + seg0 + s, v[s]);
    }
    if (wave == 0) {
        float val[kPerLane];
        bool have[kPerLane];
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int sg = lane + 64 * j;
            const bool own = sg >= seg0 && sg < seg0 + kSegs;
            have[j] = sg >= nseg || own;
            val[j] = 0.0f;
#pragma unroll
            for (int s = 0; s < kSegs; ++s)
                if (sg == seg0 + s) val[j] = v[s];
        }
        for (int it = 0;; ++it) {
            bool all = true;
#pragma unroll
            for (int j = 0; j < kPerLane; ++j) {
                if (!have[j]) {
                    const uint64_t w = slot_read(rs + lane + 64 * j);
                    if ((w >> 32) != 0) {
                        have[j] = true;
                        val[j] = __uint_as_float(static_cast<uint32_t>(w));
                    } else {
                        all = false;
                    }
                }
            }
            if (__all(all) || it >= wait_polls) break;
            __builtin_amdgcn_s_sleep(1);
        }
        bool miss = false;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int sg = lane + 64 * j;
            if (sg < nseg) {
                x.vals[sg] = val[j];
                x.missing[sg] = have[j] ? 0 : 1;
                miss = miss || !have[j];
            }
        }
        const int any_miss = __any(miss);
        if (lane == 0) x.nmissing = any_miss;
    }
    __syncthreads();
    if (x.nmissing != 0) {  // workgroup-uniform: a wait ran out
        for (int sg = 0; sg < nseg; ++sg) {
            if (!x.missing[sg]) continue;  // uniform (LDS)
            const float a = recompute(sg);
            if (t == 0) x.vals[sg] = a;
        }
        __syncthreads();
    }
}

// The row total of the segment sums in wide_row_finish's order: lane l adds
// segments l, l+64, l+128, l+192 in turn from +0, then the wave's lane tree.
__device__ __forceinline__ float team_row_total(const TeamXchg& x, int nseg) {
    constexpr int kPerLane = static_cast<int>(kTeamMaxSegs / 64);
    const int lane = threadIdx.x & 63;
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int sg = lane + 64 * j;
        a += sg < nseg ? x.vals[sg] : 0.0f;
    }
    return group_sum<64>(a);
}

template <class S, bool ACC, int kTeamSegs>
__global__ __launch_bounds__(kWideLanes) void wide_bwd_team(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    const float* __restrict__ inv_rms, const typename S::T* __restrict__ dy,
    typename S::T* __restrict__ dx, uint64_t* __restrict__ slots, float* __restrict__ partials,
    int64_t rows, int cols, int nseg, int nparts, int64_t nteams, int wait_polls) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NV = kWideSegCols / (W * kWideLanes);  // slots per lane per segment
    constexpr int NS = kTeamSegs * NV;
    constexpr int kWaves = kWideLanes / 64;
    // one buffer each: a wave writes red (and the exchange fields) for the
    // next row only after the barrier that follows the poll, which every wave
    // reaches after reading them
    __shared__ float red[kTeamSegs][kWaves];
    __shared__ float fb[kWaves];
    __shared__ TeamXchg xchg;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int64_t team = static_cast<int64_t>(blockIdx.x) / nparts;
    const int seg0 = (static_cast<int>(static_cast<int64_t>(blockIdx.x) - team * nparts)) * kTeamSegs;
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    const bool want_dx = dx != nullptr, want_dg = partials != nullptr;
    const float inv_cols = 1.0f / static_cast<float>(cols);
    // slot q = s*NV + k of lane t: columns (seg0+s)*kWideSegCols + (t + k*256)*W ..
    uint32_t off[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const int col = (seg0 + q / NV) * kWideSegCols + (t + (q % NV) * kWideLanes) * W;
        off[q] = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
    }
    const rsrc_t rg = make_rsrc(gamma, gamma ? row_bytes : 0u);
    // gamma of this workgroup's columns, loaded once: in LDS for fp32 parts of
    // two segments (registers for the rows), else in registers
    constexpr bool GLDS = std::is_same<S, F32>::value && kTeamSegs == 2;
    __shared__ u32x4 glds[GLDS ? NS : 1][GLDS ? kWideLanes : 1];
    u32x4 gv[GLDS ? 1 : NS];
    if constexpr (GLDS) {
#pragma unroll
        for (int q = 0; q < NS; ++q)
            glds[q][t] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[q], 0, 0);
        __syncthreads();
    } else {
#pragma unroll
        for (int q = 0; q < NS; ++q)
            gv[q] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[q], 0, 0);
    }
    auto gam = [&](int q) -> u32x4 {
        if constexpr (GLDS) return glds[q][t];
        else return gv[q];
    };
    float dg[NS][W];
#pragma unroll
    for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int e = 0; e < W; ++e) dg[q][e] = 0.0f;

    struct Set {
        u32x4 xv[NS], dv[NS];
        float r;
    };
    auto issue = [&](Set& b, int64_t row) {
        const bool live = row < rows;
        const int64_t e0 = (live ? row : 0) * static_cast<int64_t>(cols);
        const rsrc_t rx = make_rsrc(x + e0, live ? row_bytes : 0u);
        const rsrc_t rd = make_rsrc(dy + e0, live ? row_bytes : 0u);
#pragma unroll
        for (int q = 0; q < NS; ++q) {
            b.xv[q] = bload16_stream(rx, off[q]);
            b.dv[q] = bload16_stream(rd, off[q]);
        }
        b.r = live ? inv_rms[row] : 0.0f;
    };
    // segment sg's sum of g*x for `row`, recomputed by the whole workgroup
    // with wide_row_stats' arithmetic (workgroup-uniform call)
    auto recompute = [&](int64_t row, int sg) -> float {
        const int64_t e0 = row * static_cast<int64_t>(cols);
        const rsrc_t rx = make_rsrc(x + e0, row_bytes);
        const rsrc_t rd = make_rsrc(dy + e0, row_bytes);
        u32x4 xv[NV], dv[NV], gk[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = sg * kWideSegCols + (t + k * kWideLanes) * W;
            const uint32_t o = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
            xv[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
            dv[k] = __builtin_amdgcn_raw_buffer_load_b128(rd, o, 0, 0);
            gk[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, o, 0, 0);
        }
        float part[W];
#pragma unroll
        for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fx[W], fd[W];
            S::unpack(xv[k], fx);
            S::unpack(dv[k], fd);
            if (gamma) {
                float gm[W];
                S::unpack(gk[k], gm);
#pragma unroll
                for (int e = 0; e < W; ++e) fd[e] = fd[e] * gm[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] += fd[e] * fx[e];
        }
        float v = 0.0f;
#pragma unroll
        for (int e = 0; e < W; ++e) v += part[e];
        v = group_sum<64>(v);
        if (lane == 0) fb[wave] = v;
        __syncthreads();
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) a += fb[w];
        __syncthreads();
        return a;
    };

    // One row: `cur` holds it; the loads of row `ahead` go into `fill` first.
    auto step = [&](Set& cur, Set& fill, int64_t row, int64_t ahead) {
        issue(fill, ahead);
        const float r = cur.r;
        // 1. per segment: g*x summed as wide_row_stats sums it; the dgamma
        //    terms (they need r only)
        float v[kTeamSegs];
#pragma unroll
        for (int s = 0; s < kTeamSegs; ++s) {
            float part[W];
#pragma unroll
            for (int e = 0; e < W; ++e) part[e] = 0.0f;
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const int q = s * NV + k;
                float fx[W], fd[W];
                S::unpack(cur.xv[q], fx);
                S::unpack(cur.dv[q], fd);
                if (want_dg) {
#pragma unroll
                    for (int e = 0; e < W; ++e) dg[q][e] += fd[e] * (fx[e] * r);
                }
                if (gamma) {
                    float gm[W];
                    S::unpack(gam(q), gm);
#pragma unroll
                    for (int e = 0; e < W; ++e) fd[e] = fd[e] * gm[e];
                }
#pragma unroll
                for (int e = 0; e < W; ++e) part[e] += fd[e] * fx[e];
            }
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < W; ++e) a += part[e];
            v[s] = group_sum<64>(a);
        }
        if (!want_dx) return;  // workgroup-uniform
        if (lane == 0) {
#pragma unroll
            for (int s = 0; s < kTeamSegs; ++s) red[s][wave] = v[s];
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kTeamSegs; ++s) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) a += red[s][w];
            v[s] = a;
        }
        // 2.-3. publish this workgroup's sums, gather the row's others
        team_gather<kTeamSegs>(slots + row * static_cast<int64_t>(nseg), v, seg0, nseg,
                               wait_polls, xchg, [&](int sg) { return recompute(row, sg); });
        // 4. the row's dot as wide_row_finish adds it, then s
        const float dot = team_row_total(xchg, nseg);
        const float sc = (r * r * dot) * inv_cols;
        // 5. dx = r*(g - x*s)
        const rsrc_t rdx = make_rsrc(dx + row * static_cast<int64_t>(cols), row_bytes);
#pragma unroll
        for (int q = 0; q < NS; ++q) {
            float fx[W], gk[W], o[W];
            S::unpack(cur.xv[q], fx);
            S::unpack(cur.dv[q], gk);
            if (gamma) {
                float gm[W];
                S::unpack(gam(q), gm);
#pragma unroll
                for (int e = 0; e < W; ++e) gk[e] = gk[e] * gm[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) o[e] = r * (gk[e] - fx[e] * sc);
            if constexpr (ACC) {
                float old[W];
                S::unpack(bload16_stream(rdx, off[q]), old);
#pragma unroll
                for (int e = 0; e < W; ++e) o[e] = acc_add(old[e], o[e]);
            }
            bstore16_stream(rdx, off[q], S::pack(o));
        }
    };
    // Two register sets in turn, so the loads of the team's next row are in
    // flight while a row is summed, exchanged and written (unrolled by two,
    // so no set is copied).  A third set (two rows ahead) measured level.
    int64_t row = team;
    Set a, b;
    issue(a, row);
    for (;;) {
        step(a, b, row, row + nteams);
        if ((row += nteams) >= rows) break;
        step(b, a, row, row + nteams);
        if ((row += nteams) >= rows) break;
    }
    if (!want_dg) return;
    float* prow = partials + team * static_cast<int64_t>(cols);
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        if (off[q] == kOffOut) continue;
        float* p = prow + off[q] / sizeof(T);
#pragma unroll
        for (int e = 0; e < W; e += 4)
            *reinterpret_cast<float4*>(p + e) =
                make_float4(dg[q][e], dg[q][e + 1], dg[q][e + 2], dg[q][e + 3]);
    }
}

inline int zero_fill(float* p, int64_t n, hipStream_t st);
int team_wait_polls();

template <class S, int kSegs>
int launch_wide_team_bwd_segs(const void* x, const void* gamma, const float* inv_rms,
                              const void* dy, void* dx, float* dgamma, void* ws, int64_t rows,
                              int cols, int acc_dx, int acc_dg, hipStream_t st) {
    using T = typename S::T;
    const TeamPlan tp = team_plan(rows, cols, kSegs);
    const WideWs w = wide_ws_layout(rows, cols, tp.teams);
    const int64_t nseg = (cols + kWideSegCols - 1) / kWideSegCols;
    const int64_t grid = tp.teams * tp.parts;
    if (grid > 0x7fffffffLL || nseg > kTeamMaxSegs) return AGK_EINVAL;
    char* base = static_cast<char*>(ws);
    uint64_t* slots = reinterpret_cast<uint64_t*>(base + w.segs);
    float* partials = dgamma ? reinterpret_cast<float*>(base + w.partials) : nullptr;
    if (dx) {
        if (int rc = zero_fill(reinterpret_cast<float*>(slots), rows * nseg * 2, st)) return rc;
    }
    const T* xp = static_cast<const T*>(x);
    const T* gp = static_cast<const T*>(gamma);
    const T* dyp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    const int polls = team_wait_polls();
#define AGK_TEAM(ACC_)                                                                         \
    hipLaunchKernelGGL((wide_bwd_team<S, ACC_, kSegs>), dim3(static_cast<unsigned>(grid)),     \
                       dim3(kWideLanes), 0, st, xp, gp, inv_rms, dyp, dxp, slots, partials, rows, \
                       cols, static_cast<int>(nseg), static_cast<int>(tp.parts), tp.teams, polls)
    if (acc_dx && dx) AGK_TEAM(true);
    else AGK_TEAM(false);
#undef AGK_TEAM
    if (int rc = check_launch()) return rc;
    if (dgamma) return launch_finalize(partials, dgamma, tp.teams, cols, acc_dg, st);
    return AGK_OK;
}

// ws: at least wide_ws_bytes(rows, cols, false) bytes (wide_ws_stats_bytes
// without dgamma), 16-byte aligned (checked by the caller).
template <class S>
int launch_wide_team_bwd(const void* x, const void* gamma, const float* inv_rms, const void* dy,
                         void* dx, float* dgamma, void* ws, int64_t rows, int cols, int acc_dx,
                         int acc_dg, hipStream_t st) {
    if constexpr (std::is_same<S, F32>::value) {
        if (team_segs_for(AGK_F32, rows, cols) == 2)
            return launch_wide_team_bwd_segs<S, 2>(x, gamma, inv_rms, dy, dx, dgamma, ws, rows,
                                                   cols, acc_dx, acc_dg, st);
        return launch_wide_team_bwd_segs<S, 1>(x, gamma, inv_rms, dy, dx, dgamma, ws, rows, cols,
                                               acc_dx, acc_dg, st);
    } else {
        return launch_wide_team_bwd_segs<S, 2>(x, gamma, inv_rms, dy, dx, dgamma, ws, rows, cols,
                                               acc_dx, acc_dg, st);
    }
}

// ---- the forward in one read of x: teams ------------------------------------------
// Given a workspace (agk_rmsnorm_fwd_ws), the rows the split forward takes,
// of at most kTeamMaxSegs segments and at least kTeamMinRows rows, go to
// teams of P workgroups as in the team backward (all 512 workgroups resident
// at once at the kernel's register use): workgroup p owns segments
// [p*SEGS, (p+1)*SEGS) (SEGS = fwd_team_segs_for), team t takes rows t, t+T, ...
// (T = min(kFwdTeamWorkgroups / P, rows)).  Per row each workgroup
//   1. sums x^2 over each of its segments as wide_row_stats does;
//   2. publishes the sums in the row's slots and gathers the others with the
//      team backward's bounded wait, recomputing a sum still missing after
//      `wait_polls` polls from x itself (same arithmetic, same bits);
//   3. adds the row's segment sums as wide_row_finish does and takes
//      r = 1/sqrt(sum/cols + eps) (workgroup 0 of the team writes inv_rms);
//   4. writes y = (x*r)*gamma as wide_fwd_scale does,
// while the loads of the team's next row are in flight.  inv_rms and y are
// the split path's bits, and x is read once (the split path reads it twice).
// The slots are cleared by a fill kernel ahead of the launch, in stream
// order, so a set flag means "written by this call".
constexpr int64_t kFwdTeamWorkgroups = 512;

// Segments per workgroup, which the row's exchange is amortised over: 32 KiB
// of x per row (two fp32 or four bf16 segments), or for fp32 64 KiB (four
// segments, gamma then staged in LDS) where two-segment parts would number 16
// or more per row or a two-segment team would get at most 4 rows, and there
// are rows enough for four-segment teams to fill the grid (at [8, 262144] four
// segments ran 9.3 us against 7.7: 128 workgroups against 256).  A function
// of rows and cols only.  Measured on MI355X (graph-replayed
// agk_rmsnorm_fwd_ws, 512 workgroups): fp32 [2048, 65536] 200 -> 176 us with
// two segments against one, bf16 [8192, 131072] 925 -> 722 us with four
// against two.  fp32 two segments -> four: [512, 131072] 97 -> 94,
// [2048, 131072] 373 -> 360, [64, 262144] 31 -> 24, [256, 262144] 111 -> 96,
// [128, 524288] 121 -> 99, [256, 65536] 24 -> 23; but [1024, 65536] 91 -> 95,
// [2048, 65536] 178 -> 189, [4096, 40000] 223 -> 230.  Gamma in registers
// instead of LDS at four fp32 segments measured the same (241 VGPRs).  Eight
// bf16 segments need 256 VGPRs (one wave per SIMD: the 512 workgroups would
// not all be resident; measured 9-16 % slower), and 1024 workgroups of the
// narrower parts measured between one and two segments.
inline int fwd_team_segs_for(int dtype, int64_t rows, int64_t cols) {
    if (dtype != AGK_F32) return 4;
    const int64_t parts2 = (cols + 2 * kWideSegCols - 1) / (2 * kWideSegCols);
    const int64_t parts4 = (cols + 4 * kWideSegCols - 1) / (4 * kWideSegCols);
    const int64_t teams2 = kFwdTeamWorkgroups / parts2 > 0 ? kFwdTeamWorkgroups / parts2 : 1;
    const int64_t teams4 = kFwdTeamWorkgroups / parts4 > 0 ? kFwdTeamWorkgroups / parts4 : 1;
    // four only where its teams still fill the grid (few rows want more parts)
    return rows >= teams4 && (parts2 >= 16 || rows <= 4 * teams2) ? 4 : 2;
}

inline TeamPlan fwd_team_plan(int64_t rows, int cols, int segs) {
    TeamPlan tp;
    const int64_t part_cols = static_cast<int64_t>(segs) * kWideSegCols;
    tp.parts = (cols + part_cols - 1) / part_cols;
    const int64_t want = kFwdTeamWorkgroups / tp.parts > 0 ? kFwdTeamWorkgroups / tp.parts : 1;
    tp.teams = want < rows ? want : rows;
    return tp;
}

// The sizes the team forward can take (given the split forward's pointers):
// at most kTeamMaxSegs segments and at least kTeamMinRows rows.
inline bool fwd_team_shape_ok(int64_t rows, int64_t cols) {
    const int64_t nseg = (cols + kWideSegCols - 1) / kWideSegCols;
    return cols >= kWideMinCols && nseg <= kTeamMaxSegs && rows >= kTeamMinRows;
}
// Bytes of the team forward's slots: one 8-byte word per (row, segment).
// Depends only on rows and cols; 0 for sizes the team forward never takes.
inline size_t fwd_team_ws_bytes(int64_t rows, int64_t cols) {
    if (!fwd_team_shape_ok(rows, cols)) return 0;
    const int64_t nseg = (cols + kWideSegCols - 1) / kWideSegCols;
    return static_cast<size_t>(rows) * static_cast<size_t>(nseg) * 8u;
}

template <class S, int kSegs>
__global__ __launch_bounds__(kWideLanes) void wide_fwd_team(
    const typename S::T* __restrict__ x, const typename S::T* __restrict__ gamma,
    typename S::T* __restrict__ y, float* __restrict__ inv_rms, uint64_t* __restrict__ slots,
    int64_t rows, int cols, int nseg, int nparts, int64_t nteams, float eps, int wait_polls) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NV = kWideSegCols / (W * kWideLanes);  // slots per lane per segment
    constexpr int NS = kSegs * NV;
    constexpr int kWaves = kWideLanes / 64;
    // red and the exchange fields are written for the next row only after a
    // barrier that every wave reaches after reading them for this one
    __shared__ float red[kSegs][kWaves];
    __shared__ float fb[kWaves];
    __shared__ TeamXchg xchg;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int64_t team = static_cast<int64_t>(blockIdx.x) / nparts;
    const int part = static_cast<int>(static_cast<int64_t>(blockIdx.x) - team * nparts);
    const int seg0 = part * kSegs;
    const uint32_t row_bytes = static_cast<uint32_t>(cols) * sizeof(T);
    // slot q = s*NV + k of lane t: columns (seg0+s)*kWideSegCols + (t + k*256)*W ..
    uint32_t off[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const int col = (seg0 + q / NV) * kWideSegCols + (t + (q % NV) * kWideLanes) * W;
        off[q] = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
    }
    const rsrc_t rg = make_rsrc(gamma, gamma ? row_bytes : 0u);
    // gamma of this workgroup's columns, loaded once: in LDS for parts of more
    // than 8 slots per lane (registers for the rows), else in registers
    constexpr bool GLDS = NS > 8;
    __shared__ u32x4 glds[GLDS ? NS : 1][GLDS ? kWideLanes : 1];
    u32x4 gv[GLDS ? 1 : NS];
    if constexpr (GLDS) {
#pragma unroll
        for (int q = 0; q < NS; ++q)
            glds[q][t] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[q], 0, 0);
        __syncthreads();
    } else {
#pragma unroll
        for (int q = 0; q < NS; ++q)
            gv[q] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[q], 0, 0);
    }
    auto gam = [&](int q) -> u32x4 {
        if constexpr (GLDS) return glds[q][t];
        else return gv[q];
    };

    struct Set {
        u32x4 xv[NS];
    };
    auto issue = [&](Set& b, int64_t row) {
        const bool live = row < rows;
        const rsrc_t rx =
            make_rsrc(x + (live ? row : 0) * static_cast<int64_t>(cols), live ? row_bytes : 0u);
#pragma unroll
        for (int q = 0; q < NS; ++q) b.xv[q] = bload16_stream(rx, off[q]);
    };
    // segment sg's sum of x^2 for `row`, recomputed by the whole workgroup
    // with wide_row_stats' arithmetic (workgroup-uniform call)
    auto recompute = [&](int64_t row, int sg) -> float {
        const rsrc_t rx = make_rsrc(x + row * static_cast<int64_t>(cols), row_bytes);
        u32x4 xv[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int col = sg * kWideSegCols + (t + k * kWideLanes) * W;
            const uint32_t o = col < cols ? static_cast<uint32_t>(col) * sizeof(T) : kOffOut;
            xv[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
        }
        float part_sum[W];
#pragma unroll
        for (int e = 0; e < W; ++e) part_sum[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float fx[W];
            S::unpack(xv[k], fx);
#pragma unroll
            for (int e = 0; e < W; ++e) part_sum[e] += fx[e] * fx[e];
        }
        float v = 0.0f;
#pragma unroll
        for (int e = 0; e < W; ++e) v += part_sum[e];
        v = group_sum<64>(v);
        if (lane == 0) fb[wave] = v;
        __syncthreads();
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) a += fb[w];
        __syncthreads();
        return a;
    };

    // One row: `cur` holds it; the loads of row `ahead` go into `fill` first.
    auto step = [&](Set& cur, Set& fill, int64_t row, int64_t ahead) {
        issue(fill, ahead);
        // 1. per segment: x^2 summed as wide_row_stats sums it
        float v[kSegs];
#pragma unroll
        for (int s = 0; s < kSegs; ++s) {
            float part_sum[W];
#pragma unroll
            for (int e = 0; e < W; ++e) part_sum[e] = 0.0f;
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                float fx[W];
                S::unpack(cur.xv[s * NV + k], fx);
#pragma unroll
                for (int e = 0; e < W; ++e) part_sum[e] += fx[e] * fx[e];
            }
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < W; ++e) a += part_sum[e];
            v[s] = group_sum<64>(a);
        }
        if (lane == 0) {
#pragma unroll
            for (int s = 0; s < kSegs; ++s) red[s][wave] = v[s];
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kSegs; ++s) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) a += red[s][w];
            v[s] = a;
        }
        // 2. publish this workgroup's sums, gather the row's others
        team_gather<kSegs>(slots + row * static_cast<int64_t>(nseg), v, seg0, nseg, wait_polls,
                           xchg, [&](int sg) { return recompute(row, sg); });
        // 3. the row's sum as wide_row_finish adds it, then r
        const float ss = team_row_total(xchg, nseg);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
        if (part == 0 && t == 0) inv_rms[row] = r;
        // 4. y = (x*r)*gamma
        const rsrc_t ry = make_rsrc(y + row * static_cast<int64_t>(cols), row_bytes);
#pragma unroll
        for (int q = 0; q < NS; ++q) {
            float f[W];
            S::unpack(cur.xv[q], f);
            if (gamma) {
                float gm[W];
                S::unpack(gam(q), gm);
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = (f[e] * r) * gm[e];
            } else {
#pragma unroll
                for (int e = 0; e < W; ++e) f[e] = f[e] * r;
            }
            bstore16_stream(ry, off[q], S::pack(f));
        }
    };
    // Two register sets in turn, as the team backward (unrolled by two, so no
    // set is copied).
    int64_t row = team;
    Set a, b;
    issue(a, row);
    for (;;) {
        step(a, b, row, row + nteams);
        if ((row += nteams) >= rows) break;
        step(b, a, row, row + nteams);
        if ((row += nteams) >= rows) break;
    }
}

// ws: at least fwd_team_ws_bytes(rows, cols) bytes, 8-byte aligned (checked
// by the caller).
template <class S, int kSegs>
int launch_wide_team_fwd_segs(const void* x, const void* gamma, void* y, float* inv_rms,
                              void* ws, int64_t rows, int cols, float eps, hipStream_t st) {
    using T = typename S::T;
    const TeamPlan tp = fwd_team_plan(rows, cols, kSegs);
    const int64_t nseg = (cols + kWideSegCols - 1) / kWideSegCols;
    const int64_t grid = tp.teams * tp.parts;
    if (grid > 0x7fffffffLL || nseg > kTeamMaxSegs) return AGK_EINVAL;
    uint64_t* slots = static_cast<uint64_t*>(ws);
    if (int rc = zero_fill(static_cast<float*>(ws), rows * nseg * 2, st)) return rc;
    hipLaunchKernelGGL((wide_fwd_team<S, kSegs>), dim3(static_cast<unsigned>(grid)),
                       dim3(kWideLanes), 0, st, static_cast<const T*>(x),
                       static_cast<const T*>(gamma), static_cast<T*>(y), inv_rms, slots, rows,
                       cols, static_cast<int>(nseg), static_cast<int>(tp.parts), tp.teams, eps,
                       team_wait_polls());
    return check_launch();
}

template <class S>
int launch_wide_team_fwd(const void* x, const void* gamma, void* y, float* inv_rms, void* ws,
                         int64_t rows, int cols, float eps, hipStream_t st) {
    if constexpr (std::is_same<S, F32>::value) {
        if (fwd_team_segs_for(AGK_F32, rows, cols) == 4)
            return launch_wide_team_fwd_segs<S, 4>(x, gamma, y, inv_rms, ws, rows, cols, eps, st);
        return launch_wide_team_fwd_segs<S, 2>(x, gamma, y, inv_rms, ws, rows, cols, eps, st);
    } else {
        return launch_wide_team_fwd_segs<S, 4>(x, gamma, y, inv_rms, ws, rows, cols, eps, st);
    }
}
