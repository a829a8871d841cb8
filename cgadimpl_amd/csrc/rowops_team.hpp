// rowops_team.hpp -- row softmax, its backward and the log-sum-exp backward
// over rows too wide for one workgroup to hold in registers, with one read of
// each input row from HBM.  Included by rowops.hip inside namespace
// agk::rowops, after the ops.
//
// A row's 16-byte slots are cut into `parts` contiguous ranges of at most
// `ps` slots; a "team" of `parts` workgroups of 256 lanes holds one row at a
// time, workgroup p of the team holding range p in registers (lane t: slots
// t + k*256 of its range, k < NVL).  A row that does not start on a 16-byte
// boundary (every row tensor at the same offset from one) is a head of up to
// W-1 elements before its first boundary, which part 0 holds, a body of slots
// and a tail of up to W-1 elements, which the last part holds (lane t: head
// element t, tail element t).  Team t takes rows t, t+T, t+2T, ... (T teams).
// Per row each workgroup
//   1. reduces its range: the softmax backward sums y*dy; the softmax forward
//      and the log-sum-exp backward take the range's maximum M_p, then
//      S_p = sum of exp(z - M_p) over the same values in registers.  Per lane
//      over its slots in order, then the wave's lane tree and the four waves
//      in order;
//   2. publishes its value(s) in the row's slots: one 64-bit word per value,
//      a set flag in the high half and the float's bits in the low half,
//      stored at agent scope, so a reader sees the cleared word or the value;
//   3. reads the other parts' words: one wave polls them with agent-scope
//      loads, at most `polls` times, and a value still missing after that is
//      recomputed by the workgroup from the row with the same arithmetic (the
//      same bits), so the result never depends on which workgroups are
//      resident at once and every wait ends;
//   4. combines the parts in part order over a fixed lane tree, so every
//      workgroup of the team gets the same bits: dot = sum of the parts, or
//      M = max M_p and S = sum of S_p * exp(M_p - M) over the parts with
//      M_p > -inf (S = NaN for a row that is -inf throughout, as on the
//      other paths);
//   5. writes its range of the output row -- y * (dy - dot), exp(z - M) / S,
//      or dy[row] * (exp(z - M) / S), the last two as the exponentials of
//      step 1 kept in registers times exp(M_p - M) / S (the head and tail
//      elements: exp(z - M) / S) -- while the loads of the team's next row,
//      issued before step 1, are in flight.
// The words are cleared by a fill kernel ahead of the launch, in stream
// order, so a set flag means "written by this call".  The launch shape
// depends only on rows, cols and the storage type, so results are bit-
// identical run to run; they differ from the one-workgroup-per-row paths'
// in the order of the row sums and, for the forward and the log-sum-exp
// backward, by the rounding of exp(z - M_p) * exp(M_p - M) against
// exp(z - M) (a few fp32 units).

constexpr int kTeamLanes = 256;
constexpr int kTeamWaves = kTeamLanes / 64;
constexpr int kTeamMaxParts = 64;  // one polling lane per part
// Slots per lane per row tensor: a part covers NVL * 256 slots (32 KiB of
// each row tensor).  Measured on MI355X (graph-replayed, bf16 and fp32
// [8192, 128256], [8192, 50257], bf16 [4096, 151936]): 8 slots per lane
// with two workgroups per CU against 4 slots with four (the row exchanged
// twice as often: 5-14 points slower except bf16 softmax forward at 50257
// columns, 5 points faster) and, for the backward, 6 slots (1-6 points
// slower).
template <class Op>
constexpr int team_nvl(bool bf16, bool aligned) {
    (void)bf16;
    (void)aligned;
    return 8;
}
inline int team_nvl_of(int op, bool bf16, bool aligned) {  // op as agk_rowops_team_plan's
    return op == 1 ? team_nvl<SmBwd>(bf16, aligned) : team_nvl<SmFwd>(bf16, aligned);
}

// Values a team exchanges per row: 1 (a sum) or 2 (a maximum and a sum).
template <class Op>
struct TeamVals : std::integral_constant<int, 2> {};
template <>
struct TeamVals<SmBwd> : std::integral_constant<int, 1> {};

// Workgroups per CU a launch aims for, all resident at once at the kernel's
// register use (the kernel is built for that many waves per SIMD): three for
// the forward and the log-sum-exp backward (at most 168 registers per lane;
// they use 102-154), two for the softmax backward (up to 190).  Measured on
// MI355X (graph-replayed, three against two per CU, us): bf16 [8192, 50257]
// 313-319 -> 305-306, [4096, 151936] 464-466 -> 450, fp32 [8192, 128256]
// 1519-1525 -> 1502-1503; bf16 [8192, 128256] and [8192, 65536] and fp32
// [8192, 50257] within 1 %.
template <class Op>
constexpr int team_per_cu() {
    return TeamVals<Op>::value == 2 ? 3 : 2;
}
// Workgroups a launch aims for on a 256-CU MI355X.  A constant per op, so the
// team count depends only on the shape, never on the device.
template <class Op>
constexpr int64_t team_grid() {
    return 256 * team_per_cu<Op>();
}

struct TeamShape {
    int parts = 0;       // workgroups per row
    int ps = 0;          // slots per part
    int64_t teams = 0;   // rows in flight
};

// Depends only on rows, cols, the slot width W, the op's slots per lane and
// its grid (teams = grid / parts rows in flight; the grid never changes the
// arithmetic, only which workgroups run a row).
inline TeamShape team_shape(int64_t rows, int64_t cols, int W, int nvl, int64_t grid) {
    TeamShape s;
    const int64_t nslot = (cols + W - 1) / W;  // at least any row's body slots
    const int64_t per = static_cast<int64_t>(nvl) * kTeamLanes;  // slots per part
    const int64_t parts = (nslot + per - 1) / per;
    if (parts < 1 || parts > kTeamMaxParts) return s;
    s.parts = static_cast<int>(parts);
    s.ps = static_cast<int>((nslot + parts - 1) / parts);
    const int64_t want = grid / parts > 0 ? grid / parts : 1;
    s.teams = want < rows ? want : rows;
    return s;
}

// Bytes of the exchange words a launch of Op over [rows, cols] uses.
inline size_t team_words_bytes(int64_t rows, const TeamShape& s, int nvals) {
    return static_cast<size_t>(rows) * static_cast<size_t>(s.parts) *
           static_cast<size_t>(nvals) * sizeof(uint64_t);
}

// The workspace the *_ws entry points ask for: the most any op of either
// storage type and layout uses at this shape (two values per part and row;
// the fp32 plan has the most parts, or where it would need more than
// kTeamMaxParts the bf16 plan's) when a row has at least two parts, 0 for
// narrower rows (one workgroup holds them).
inline size_t team_ws_bytes(int64_t rows, int64_t cols) {
    size_t most = 0;
    for (int op = 0; op < 3; ++op)
        for (int bf16 = 0; bf16 < 2; ++bf16)
            for (int al = 0; al < 2; ++al) {
                const TeamShape s = team_shape(rows, cols, bf16 ? 8 : 4,
                                               team_nvl_of(op, bf16 != 0, al != 0), 1);
                const size_t n = s.parts >= 2 ? team_words_bytes(rows, s, op == 1 ? 1 : 2) : 0;
                most = n > most ? n : most;
            }
    return rows > 0 ? most : 0;
}

__device__ __forceinline__ void team_publish(uint64_t* p, float v) {
    const uint64_t w = (static_cast<uint64_t>(1) << 32) | __float_as_uint(v);
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t team_peek(uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void team_clear(uint64_t* __restrict__ p, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        p[i] = 0;
}

// Per-lane accumulation shared by the resident ranges and the recompute, so
// both produce the same bits.
template <class S>
__device__ __forceinline__ void team_dot_slot(float (&acc)[S::kVec], u32x4 a, u32x4 b) {
    float fa[S::kVec], fb[S::kVec];
    S::unpack(a, fa);
    S::unpack(b, fb);
#pragma unroll
    for (int e = 0; e < S::kVec; ++e) acc[e] += fa[e] * fb[e];
}
// A slot past the range (loaded as zeros) is masked: -inf for the maximum
// (max(m, -inf) = m, m is never NaN: v_max_f32 returns the other operand of
// a NaN), 0 for the sum.  The dot needs no mask: 0 * 0 adds nothing.
template <class S>
__device__ __forceinline__ float team_max_slot(float m, u32x4 a, bool valid) {
    float fa[S::kVec];
    S::unpack(a, fa);
#pragma unroll
    for (int e = 0; e < S::kVec; ++e) m = MaxR::op(m, valid ? fa[e] : -__builtin_inff());
    return m;
}
template <class S>
__device__ __forceinline__ void team_exp_slot(float (&acc)[S::kVec], u32x4 a, float M,
                                              bool valid) {
    float fa[S::kVec];
    S::unpack(a, fa);
#pragma unroll
    for (int e = 0; e < S::kVec; ++e) acc[e] += valid ? fast_exp(fa[e] - M) : 0.0f;
}
template <int W>
__device__ __forceinline__ float team_fold(const float (&acc)[W]) {
    float v = acc[0];
#pragma unroll
    for (int e = 1; e < W; ++e) v += acc[e];
    return v;
}

// team_per_cu<Op>() workgroups resident on every CU, as the grid assumes:
// that many waves per SIMD (2: at most 256 registers per lane, 3: 168).
template <class S, class Op, bool ALIGNED, bool ACC>
__global__ __launch_bounds__(kTeamLanes) __attribute__((amdgpu_waves_per_eu(team_per_cu<Op>()))) void row_team(const RowArgs p, uint64_t* __restrict__ words,
                                                       int64_t rows, int cols, int parts, int ps,
                                                       int64_t teams, int polls) {
    using T = typename S::T;
    constexpr int W = S::kVec;
    constexpr int NVL = team_nvl<Op>(std::is_same<S, BF16>::value, ALIGNED);
    constexpr int NIN = Op::kIn;
    constexpr int NVALS = TeamVals<Op>::value;
    constexpr bool kLse = std::is_same<Op, LseBwd>::value;
    constexpr float kNegInf = -__builtin_inff();
    __shared__ float red[2][kTeamWaves];
    __shared__ float vals[NVALS][kTeamMaxParts];
    __shared__ unsigned char missing[kTeamMaxParts];
    __shared__ int nmiss;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int64_t team = static_cast<int64_t>(blockIdx.x) / parts;
    const int part = static_cast<int>(static_cast<int64_t>(blockIdx.x) - team * parts);
    const T* in0 = static_cast<const T*>(p.in0);
    const T* in1 = static_cast<const T*>(p.in1);
    T* out = static_cast<T*>(p.out);
    int par = 0;

    // Workgroup-uniform reductions (double-buffered: one barrier each).
    auto wg_sum = [&](float v) -> float {
        v = group_sum<64>(v);
        if (lane == 0) red[par][wave] = v;
        __syncthreads();
        float s = red[par][0];
#pragma unroll
        for (int w = 1; w < kTeamWaves; ++w) s += red[par][w];
        par ^= 1;
        return s;
    };
    auto wg_max = [&](float v) -> float {
        v = group_reduce<64, MaxR>(v);
        if (lane == 0) red[par][wave] = v;
        __syncthreads();
        float s = red[par][0];
#pragma unroll
        for (int w = 1; w < kTeamWaves; ++w) s = MaxR::op(s, red[par][w]);
        par ^= 1;
        return s;
    };

    // A row's layout: elements before its first 16-byte boundary, whole slots
    // (from there), elements after them; the range of part q.
    struct Geo {
        int head, nslot, tail0, ntail;
    };
    auto geo_of = [&](int64_t row) -> Geo {
        Geo g;
        if constexpr (ALIGNED) {
            g.head = 0;
            g.nslot = cols / W;
            g.tail0 = cols;
            g.ntail = 0;
        } else {
            const T* x = in0 + row * static_cast<int64_t>(cols);
            const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x) & 15u);
            int head = mis ? static_cast<int>((16u - mis) / sizeof(T)) : 0;
            if (head > cols) head = cols;
            g.head = head;
            g.nslot = (cols - head) / W;
            g.tail0 = head + g.nslot * W;
            g.ntail = cols - g.tail0;
        }
        return g;
    };
    auto range_len = [&](const Geo& g, int q) -> int {
        const int n = g.nslot - q * ps;
        return n < 0 ? 0 : (n > ps ? ps : n);
    };
    // element offset of range q's first slot in the tensors
    auto range_base = [&](int64_t row, const Geo& g, int q) -> int64_t {
        return row * static_cast<int64_t>(cols) + g.head + static_cast<int64_t>(q) * ps * W;
    };

    // A row's registers.  Values that need no arithmetic before their use
    // are kept as loaded (storage bits), so no load is waited for before the
    // step that uses it.
    struct Set {
        u32x4 a[NVL];
        u32x4 b[NIN == 2 ? NVL : 1];
        T ha, hb, ta, tb;  // this lane's head / tail elements (own_h / own_t)
        bool own_h, own_t;
        T g;               // log-sum-exp backward: dy[row]
        Geo geo;
        int len;
    };
    auto issue = [&](Set& s, int64_t row) {
        const bool live = row < rows;
        const int64_t r = live ? row : 0;
        s.geo = geo_of(r);
        s.len = live ? range_len(s.geo, part) : 0;
        const int64_t base = range_base(r, s.geo, part);
        const uint32_t bytes = static_cast<uint32_t>(s.len) * 16u;
        s.own_h = false;
        s.own_t = false;
        // Straight-line loads (a slot past the range reads zeros): the
        // compiler's count of loads in flight stays exact, so the waits for
        // this row's slots never wait for the next row's.
        const rsrc_t ra = make_rsrc(in0 + base, bytes);
        const rsrc_t rb = make_rsrc(NIN == 2 ? in1 + base : in0, NIN == 2 ? bytes : 0u);
#pragma unroll
        for (int k = 0; k < NVL; ++k) {
            const uint32_t o = static_cast<uint32_t>(t + k * kTeamLanes) * 16u;
            s.a[k] = bload16_stream(ra, o);
            if constexpr (NIN == 2) s.b[k] = bload16_stream(rb, o);
        }
        if constexpr (!ALIGNED) {
            // every lane loads from inside the row; only owners use the value
            const int64_t r0 = r * static_cast<int64_t>(cols);
            s.own_h = live && part == 0 && t < s.geo.head;
            s.own_t = live && part == parts - 1 && t < s.geo.ntail;
            const int64_t ih = r0 + (s.own_h ? t : 0);
            const int64_t it = r0 + (s.own_t ? s.geo.tail0 + t : 0);
            s.ha = in0[ih];
            s.ta = in0[it];
            if constexpr (NIN == 2) {
                s.hb = in1[ih];
                s.tb = in1[it];
            }
        }
        if constexpr (kLse) s.g = static_cast<const T*>(p.rsv)[r];
    };
    auto val = [](const T& v) -> float { return S::get(&v); };

    // Range q of `row`, reduced from memory, one slot per lane at a time,
    // with the arithmetic of the resident range (workgroup-uniform call).
    auto recompute = [&](int64_t row, int q, float (&v)[NVALS]) {
        const Geo g = geo_of(row);
        const int len = range_len(g, q);
        const int64_t base = range_base(row, g, q);
        const uint32_t bytes = static_cast<uint32_t>(len) * 16u;
        const rsrc_t ra = make_rsrc(in0 + base, bytes);
        const rsrc_t rb = make_rsrc(NIN == 2 ? in1 + base : in0, NIN == 2 ? bytes : 0u);
        bool oh = false, ot = false;
        float ha = 0.0f, hb = 0.0f, ta = 0.0f, tb = 0.0f;
        if constexpr (!ALIGNED) {
            const int64_t r0 = row * static_cast<int64_t>(cols);
            oh = q == 0 && t < g.head;
            ot = q == parts - 1 && t < g.ntail;
            if (oh) {
                ha = S::get(in0 + r0 + t);
                if constexpr (NIN == 2) hb = S::get(in1 + r0 + t);
            }
            if (ot) {
                ta = S::get(in0 + r0 + g.tail0 + t);
                if constexpr (NIN == 2) tb = S::get(in1 + r0 + g.tail0 + t);
            }
        }
        float acc[W];
#pragma unroll
        for (int e = 0; e < W; ++e) acc[e] = 0.0f;
        if constexpr (NVALS == 1) {
#pragma unroll 1
            for (int k = 0; k < NVL; ++k) {
                const uint32_t o = static_cast<uint32_t>(t + k * kTeamLanes) * 16u;
                team_dot_slot<S>(acc, __builtin_amdgcn_raw_buffer_load_b128(ra, o, 0, 0),
                                 __builtin_amdgcn_raw_buffer_load_b128(rb, o, 0, 0));
            }
            float x = team_fold<W>(acc);
            if constexpr (!ALIGNED) x += (oh ? ha * hb : 0.0f) + (ot ? ta * tb : 0.0f);
            v[0] = wg_sum(x);
        } else {
            float m = kNegInf;
#pragma unroll 1
            for (int k = 0; k < NVL; ++k)
                m = team_max_slot<S>(m, __builtin_amdgcn_raw_buffer_load_b128(
                                            ra, static_cast<uint32_t>(t + k * kTeamLanes) * 16u,
                                            0, 0),
                                     t + k * kTeamLanes < len);
            if (oh) m = MaxR::op(m, ha);
            if (ot) m = MaxR::op(m, ta);
            const float M = wg_max(m);
#pragma unroll 1
            for (int k = 0; k < NVL; ++k)
                team_exp_slot<S>(acc, __builtin_amdgcn_raw_buffer_load_b128(
                                          ra, static_cast<uint32_t>(t + k * kTeamLanes) * 16u,
                                          0, 0),
                                 M, t + k * kTeamLanes < len);
            float x = team_fold<W>(acc);
            if constexpr (!ALIGNED) {
                float es = 0.0f;
                if (oh) es += fast_exp(ha - M);
                if (ot) es += fast_exp(ta - M);
                x += es;
            }
            v[0] = M;
            v[1] = wg_sum(x);
        }
    };

    // One row: `cur` holds it; the loads of row `ahead` go into `fill` first.
    auto step = [&](Set& cur, Set& fill, int64_t row, int64_t ahead) {
        issue(fill, ahead);
        // 1. this range's value(s), in every wave
        float mine[NVALS];
        float acc[W];
        float ex[NVALS == 2 ? NVL : 1][W];  // exp(a - this range's max)
#pragma unroll
        for (int e = 0; e < W; ++e) acc[e] = 0.0f;
        float ha = 0.0f, hb = 0.0f, ta = 0.0f, tb = 0.0f;
        if constexpr (!ALIGNED) {
            ha = val(cur.ha);
            ta = val(cur.ta);
            if constexpr (NIN == 2) {
                hb = val(cur.hb);
                tb = val(cur.tb);
            }
        }
        if constexpr (NVALS == 1) {
#pragma unroll
            for (int k = 0; k < NVL; ++k) team_dot_slot<S>(acc, cur.a[k], cur.b[k]);
            float x = team_fold<W>(acc);
            if constexpr (!ALIGNED)
                x += (cur.own_h ? ha * hb : 0.0f) + (cur.own_t ? ta * tb : 0.0f);
            mine[0] = wg_sum(x);
        } else {
            float m = kNegInf;
#pragma unroll
            for (int k = 0; k < NVL; ++k)
                m = team_max_slot<S>(m, cur.a[k], t + k * kTeamLanes < cur.len);
            if (cur.own_h) m = MaxR::op(m, ha);
            if (cur.own_t) m = MaxR::op(m, ta);
            const float M = wg_max(m);
            // Each element's exp(a - M) is kept for the output, which scales
            // it by exp(M - row max) / row sum: one exponential per element
            // instead of two.  The sum adds the same values in the same order
            // as team_exp_slot (the recompute's).  A range whose maximum is
            // -inf exponentiates against 0 instead: its elements are -inf or
            // masked, every kept value is 0, and the combine below ignores
            // its published sum.
            const float Mx = M == kNegInf ? 0.0f : M;
#pragma unroll
            for (int k = 0; k < NVL; ++k) {
                float fa[W];
                S::unpack(cur.a[k], fa);
                const bool valid = t + k * kTeamLanes < cur.len;
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    ex[k][e] = valid ? fast_exp(fa[e] - Mx) : 0.0f;
                    acc[e] += ex[k][e];
                }
            }
            float x = team_fold<W>(acc);
            if constexpr (!ALIGNED) {
                float es = 0.0f;
                if (cur.own_h) es += fast_exp(ha - M);
                if (cur.own_t) es += fast_exp(ta - M);
                x += es;
            }
            mine[0] = M;
            mine[1] = wg_sum(x);
        }
        // Two row tensors: the packed slots are made opaque here, so the
        // output below unpacks them again instead of the compiler holding
        // every unpacked value of the dot across the exchange (which would
        // not fit in registers).
        if constexpr (NIN == 2) {
#pragma unroll
            for (int k = 0; k < NVL; ++k) opaque(cur.a[k], cur.b[k]);
        }
        // 2.-3. publish this range's value(s); wave 0 gathers the other
        // parts' (its poll waits for the loads issued before it, the next
        // row's among them)
        uint64_t* rw = words + row * static_cast<int64_t>(parts) * NVALS;
        if (wave == 0) {
            if (lane == 0) {
#pragma unroll
                for (int i = 0; i < NVALS; ++i) team_publish(rw + part * NVALS + i, mine[i]);
            }
            const int j = lane;
            const bool need = j < parts && j != part;
            float got[NVALS];
            bool have[NVALS];
#pragma unroll
            for (int i = 0; i < NVALS; ++i) {
                got[i] = j == part ? mine[i] : 0.0f;
                have[i] = !need;
            }
            for (int it = 0;; ++it) {
                bool all = true;
                if (need) {
#pragma unroll
                    for (int i = 0; i < NVALS; ++i) {
                        if (!have[i]) {
                            const uint64_t w = team_peek(rw + j * NVALS + i);
                            if ((w >> 32) != 0) {
                                have[i] = true;
                                got[i] = __uint_as_float(static_cast<uint32_t>(w));
                            } else {
                                all = false;
                            }
                        }
                    }
                }
                if (__all(all) || it >= polls) break;
                __builtin_amdgcn_s_sleep(1);
            }
            bool miss = false;
#pragma unroll
            for (int i = 0; i < NVALS; ++i) miss = miss || !have[i];
            if (j < parts) {
#pragma unroll
                for (int i = 0; i < NVALS; ++i) vals[i][j] = got[i];
                missing[j] = miss ? 1 : 0;
            }
            const int any = __any(miss);
            if (lane == 0) nmiss = any;
        }
        __syncthreads();
        if (nmiss != 0) {  // workgroup-uniform: a wait ran out
            for (int q = 0; q < parts; ++q) {
                if (!missing[q]) continue;  // uniform (LDS)
                float v[NVALS];
                recompute(row, q, v);
                if (t == 0) {
#pragma unroll
                    for (int i = 0; i < NVALS; ++i) vals[i][q] = v[i];
                }
            }
            __syncthreads();
        }
        // 4. the row's statistics, in part order over the lane tree
        float dot = 0.0f, M = 0.0f, inv = 0.0f;
        if constexpr (NVALS == 1) {
            dot = group_sum<64>(lane < parts ? vals[0][lane] : 0.0f);
        } else {
            const float mj = lane < parts ? vals[0][lane] : kNegInf;
            const float sj = lane < parts ? vals[1][lane] : 0.0f;
            M = group_reduce<64, MaxR>(mj);
            float sum = group_sum<64>(mj == kNegInf ? 0.0f : sj * fast_exp(mj - M));
            if (M == kNegInf) sum = __builtin_nanf("");
            inv = 1.0f / sum;
        }
        // the kept exponentials' scale: exp(m - M) / sum for this range's
        // maximum m (exp(-inf - M) = 0 for a range of -inf; NaN where the
        // whole row is -inf, as exp(a - M) / sum gives there)
        float sc = 0.0f;
        if constexpr (NVALS == 2) sc = fast_exp(mine[0] - M) * inv;
        // 5. this range of the output row
        const int64_t base = range_base(row, cur.geo, part);
        const rsrc_t ro = make_rsrc(out + base, static_cast<uint32_t>(cur.len) * 16u);
        const float g = kLse ? val(cur.g) : 0.0f;
        auto f = [&](float a, float b) -> float {
            if constexpr (NVALS == 1) return a * (b - dot);
            else if constexpr (kLse) return g * (fast_exp(a - M) * inv);
            else return fast_exp(a - M) * inv;
        };
#pragma unroll
        for (int k = 0; k < NVL; ++k) {
            const uint32_t o = static_cast<uint32_t>(t + k * kTeamLanes) * 16u;
            float fa[W], fb[W], r[W];
            if constexpr (NVALS == 2) {
#pragma unroll
                for (int e = 0; e < W; ++e) r[e] = kLse ? g * (ex[k][e] * sc) : ex[k][e] * sc;
            } else {
                S::unpack(cur.a[k], fa);
                if constexpr (NIN == 2) S::unpack(cur.b[k], fb);
#pragma unroll
                for (int e = 0; e < W; ++e) r[e] = f(fa[e], NIN == 2 ? fb[e] : 0.0f);
            }
            if constexpr (ACC) {
                float old[W];
                S::unpack(bload16_stream(ro, o), old);
#pragma unroll
                for (int e = 0; e < W; ++e) r[e] = acc_add(old[e], r[e]);
            }
            bstore16_stream(ro, o, S::pack(r));  // past the range: dropped
        }
        if constexpr (!ALIGNED) {
            T* orow = out + row * static_cast<int64_t>(cols);
            if (cur.own_h) {
                float r = f(ha, hb);
                if constexpr (ACC) r = acc_add(S::get(orow + t), r);
                S::put(orow + t, r);
            }
            if (cur.own_t) {
                float r = f(ta, tb);
                if constexpr (ACC) r = acc_add(S::get(orow + cur.geo.tail0 + t), r);
                S::put(orow + cur.geo.tail0 + t, r);
            }
        }
    };

    // Two register sets in turn, so the loads of the team's next row are in
    // flight while a row is reduced, exchanged and written (unrolled by two,
    // so no set is copied).
    int64_t row = team;
    Set sa, sb;
    issue(sa, row);
    for (;;) {
        step(sa, sb, row, row + teams);
        if ((row += teams) >= rows) break;
        step(sb, sa, row, row + teams);
        if ((row += teams) >= rows) break;
    }
}

// Whether a [rows, cols] call of Op can take the team kernel: the rows'
// layout (every row tensor 16-byte aligned with whole slots, or all at one
// offset from a boundary), buffer offsets that fit 32 bits, at most
// kTeamMaxParts parts and at least `min_parts` of them.
template <class S, class Op>
inline bool team_fits(const RowArgs& p, int64_t rows, int cols, int min_parts, bool* aligned) {
    using T = typename S::T;
    if (rows <= 0 || rows > 0x7fffffffLL) return false;
    if (static_cast<uint64_t>(cols) * sizeof(T) >= 0x80000000ull) return false;
    *aligned = (cols % S::kVec) == 0 && aligned16(p.in0) && aligned_or_null(p.in1) &&
               aligned16(p.out);
    if (!*aligned && !same_offset<T>(p)) return false;
    const TeamShape s = team_shape(rows, cols, S::kVec,
                                   team_nvl<Op>(std::is_same<S, BF16>::value, *aligned),
                                   team_grid<Op>());
    return s.parts >= min_parts && s.parts != 0 && s.teams * s.parts <= 0x7fffffffLL;
}

int team_wait_limit();

template <class Op, class S>
int launch_team(const RowArgs& p, void* ws, int64_t rows, int cols, bool aligned, hipStream_t st) {
    const TeamShape s = team_shape(rows, cols, S::kVec,
                                   team_nvl<Op>(std::is_same<S, BF16>::value, aligned),
                                   team_grid<Op>());
    uint64_t* words = static_cast<uint64_t*>(ws);
    const int64_t nwords = rows * s.parts * TeamVals<Op>::value;
    {
        int64_t blocks = (nwords + 255) / 256;
        if (blocks > 1024) blocks = 1024;
        hipLaunchKernelGGL(team_clear, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, words,
                           nwords);
        if (int rc = check_launch()) return rc;
    }
    const dim3 grid(static_cast<unsigned>(s.teams * s.parts)), block(kTeamLanes);
    const int polls = team_wait_limit();
#define AGK_TEAM(AL, ACC_)                                                                      \
    hipLaunchKernelGGL((row_team<S, Op, AL, ACC_>), grid, block, 0, st, p, words, rows, cols,    \
                       s.parts, s.ps, s.teams, polls)
    if (aligned) {
        if (p.acc) AGK_TEAM(true, true);
        else AGK_TEAM(true, false);
    } else {
        if (p.acc) AGK_TEAM(false, true);
        else AGK_TEAM(false, false);
    }
#undef AGK_TEAM
    return check_launch();
}
