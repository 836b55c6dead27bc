// Few-row linear layer of the decoder hosts' decode step, gfx950.
//
// y[m, n] = sum_k x[m, k] W[n, k] (+ bias[n]) for M <= 8 rows of x: the
// nn.Linear / F.linear calls of one decode step (batch rows of one token
// each).  At that size the product is a read of W and nothing else, so the
// kernel is laid out for HBM: each wave owns one or two rows of W and requests
// all of their 16-byte pieces before any arithmetic (lane l takes pieces l, l + 64,
// ... of a row, so every request is a contiguous 1 KB row segment), the few x
// rows sit in LDS (staged once per workgroup, read by all its waves, reused
// over the row groups of wide outputs; their own requests leave before W's,
// since loads complete in order and x requested after W would wait for W),
// and the 64 lane partial sums of each output are added by xor-shuffles.  Accumulation
// is fp32 and the output is rounded once, as torch's GEMM does; the summation
// order differs from hipBLASLt's, so results agree to rounding, not bit for
// bit.
#include "gdn2_common.h"
#include "gdn2_internal.h"

namespace gdn2 {
namespace {

constexpr int kWaves = 4;
// Workgroups of a launch at most: enough to fill the chip several times over;
// wider outputs loop over row groups so that the staged x rows are reused.
constexpr int kMaxGroups = 2048;

__device__ __forceinline__ void widen8(uint4 u, float (&f)[8], bool bf)
{
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
        if (bf) {
            f[2 * i] = bf16_bits_to_f32(lo);
            f[2 * i + 1] = bf16_bits_to_f32(hi);
        } else {
            f[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
            f[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
        }
    }
}

template <typename T>
__device__ __forceinline__ uint4 narrow8(const float (&f)[8])
{
    unsigned w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint16_t lo, hi;
        if constexpr (std::is_same<T, bf16_t>::value) {
            lo = f32_to_bf16_bits(f[2 * i]);
            hi = f32_to_bf16_bits(f[2 * i + 1]);
        } else {
            lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f[2 * i]));
            hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f[2 * i + 1]));
        }
        w[i] = static_cast<unsigned>(lo) | (static_cast<unsigned>(hi) << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// MM: rows of x the instantiation holds (p.M <= MM, rows past p.M are zero
// and not stored); NP: 16-byte pieces of a row per lane (K = 512 NP); RPW:
// rows of W per wave; NW: waves per workgroup.  Workgroup b takes the groups
// of NW * RPW rows b, b + gridDim.x, ...
template <typename T, int MM, int NP, int RPW, int NW>
__global__ __launch_bounds__(64 * NW) void skinny_linear_kernel(SkinnyParams p)
{
    constexpr int kRowsPerWave = RPW;
    constexpr bool BF = std::is_same<T, bf16_t>::value;
    constexpr int PPR = 64 * NP;  // 16-byte pieces per row of x or W
    __shared__ __align__(16) uint4 sx[MM * PPR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int groups = (p.N + NW * kRowsPerWave - 1) / (NW * kRowsPerWave);
    const T *w = static_cast<const T *>(p.w);
    const T *x = static_cast<const T *>(p.x);

    // This wave's rows of W in a group (rows past N read row N-1); the first
    // group's are requested right after the x rows' own requests.
    uint4 wr[kRowsPerWave][NP];
    // Row r of the wave in group grp: rows n0 + r, or with the SwiGLU epilogue
    // (RPW = 2) rows c and c + N / 2 of output column c.
    auto row_of = [&](int grp, int r) __attribute__((always_inline)) {
        if constexpr (RPW == 2) {
            if (p.glu_out) return (grp * NW + wave) + r * (p.N / 2);
        }
        return (grp * NW + wave) * kRowsPerWave + r;
    };
    auto request = [&](int grp) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            const int rr = row_of(grp, r);
            const int row = rr < p.N ? rr : p.N - 1;
#pragma unroll
            for (int c = 0; c < NP; ++c)
                wr[r][c] = *reinterpret_cast<const uint4 *>(w + static_cast<int64_t>(row) * p.ldw + (c * 64 + lane) * 8);
        }
    };
    // The staging rows (x, the residual and the norm weight) are requested
    // before W: loads complete in order, so rows requested after W would wait
    // for all of W to land before the norm could start.
    uint4 xq[NP], rq[NP], nq[NP];
    if (p.norm && wave < MM) {
        const int mr = wave < p.M ? wave : 0;
        const T *xr = x + static_cast<int64_t>(mr) * p.ldx;
        const T *rr = static_cast<const T *>(p.res) + static_cast<int64_t>(mr) * p.ldres;
#pragma unroll
        for (int v = 0; v < NP; ++v) {
            xq[v] = *reinterpret_cast<const uint4 *>(xr + (v * 64 + lane) * 8);
            rq[v] = *reinterpret_cast<const uint4 *>(rr + (v * 64 + lane) * 8);
            nq[v] = *reinterpret_cast<const uint4 *>(static_cast<const T *>(p.nw) + (v * 64 + lane) * 8);
        }
    }
    // Plain staging: this thread's x pieces requested before W as well (rows
    // past M and pieces past the end read piece 0 of row 0 and become zeros).
    constexpr int XPT = (MM * PPR + 64 * NW - 1) / (64 * NW);
    uint4 xp[XPT];
    if (!p.norm) {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
            const int idx = i * 64 * NW + tid;
            const int m = idx / PPR, c = idx - m * PPR;
            const bool ok = idx < MM * PPR && m < p.M;
            xp[i] = *reinterpret_cast<const uint4 *>(x + (ok ? static_cast<int64_t>(m) * p.ldx + c * 8 : 0));
            if (!ok) xp[i] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    request(blockIdx.x);
    if (p.norm) {
        // x = RMSNorm(x + res) staged by wave m for row m (M <= 4, NP <= 4),
        // with gated_rmsnorm_vec_kernel's roundings and summation order (lane l
        // holds pieces l + 64 v, squares summed piece by piece, then the
        // xor-tree over the 64 lanes), so the staged rows equal
        // gdn2_add_rms_norm_fwd's output bit for bit.  Workgroup 0 stores the
        // residual sums.
        if (wave < MM) {
            uint4 st[NP];
            if (wave < p.M) {
                float sv[NP][8], sq = 0.0f;
#pragma unroll
                for (int v = 0; v < NP; ++v) {
                    float a[8], b[8];
                    widen8(xq[v], a, BF);
                    widen8(rq[v], b, BF);
#pragma unroll
                    for (int e = 0; e < 8; ++e) sv[v][e] = round_to<T>(a[e] + b[e]);
                }
#pragma unroll
                for (int v = 0; v < NP; ++v)
#pragma unroll
                    for (int e = 0; e < 8; ++e) sq += round_to<T>(sv[v][e] * sv[v][e]);
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) sq += __shfl_xor(sq, o, 64);
                const float var = round_to<T>(sq / static_cast<float>(p.K));
                const float inv = round_to<T>(rsqrtf(round_to<T>(var + p.eps)));
                T *so = static_cast<T *>(p.sum_out) + static_cast<int64_t>(wave) * p.ldsum;
#pragma unroll
                for (int v = 0; v < NP; ++v) {
                    if (blockIdx.x == 0) *reinterpret_cast<uint4 *>(so + (v * 64 + lane) * 8) = narrow8<T>(sv[v]);
                    float o8[8], wn[8];
                    widen8(nq[v], wn, BF);
#pragma unroll
                    for (int e = 0; e < 8; ++e) o8[e] = round_to<T>(round_to<T>(sv[v][e] * inv) * wn[e]);
                    st[v] = narrow8<T>(o8);
                }
            } else {
#pragma unroll
                for (int v = 0; v < NP; ++v) st[v] = make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int v = 0; v < NP; ++v) sx[wave * PPR + v * 64 + lane] = st[v];
        }
    } else {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const int idx = i * 64 * NW + tid;
        if (idx < MM * PPR) sx[idx] = xp[i];
    }
    }
    __syncthreads();

    for (int grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    const int n0 = (grp * NW + wave) * kRowsPerWave;
    float acc[kRowsPerWave][MM];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int c = 0; c < NP; ++c) {
        float wf[kRowsPerWave][8];
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) widen8(wr[r][c], wf[r], BF);
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            float xf[8];
            widen8(sx[m * PPR + c * 64 + lane], xf, BF);
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r][m] = fmaf(wf[r][e], xf[e], acc[r][m]);
        }
    }
    // The next group's rows are requested before this group's sums and stores.
    if (grp + static_cast<int>(gridDim.x) < groups) request(grp + gridDim.x);
    // Sum over the 64 lanes; every lane ends with every total.
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) acc[r][m] += __shfl_xor(acc[r][m], o, 64);
    if constexpr (RPW == 2) {
        if (p.glu_out) {
            // SwiGLU epilogue: lane m stores out[m, c] = round(round(silu(a)) * b)
            // from a = round(row c), b = round(row c + N / 2), as a product
            // followed by gdn2_silu_mul_fwd computes it.
            const int c = grp * NW + wave;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (lane == m && m < p.M && c < p.N / 2) {
                    float a = acc[0][m], b = acc[1][m];
                    if (p.bias) {
                        a += io<T>::ld(static_cast<const T *>(p.bias), c);
                        b += io<T>::ld(static_cast<const T *>(p.bias), c + p.N / 2);
                    }
                    a = round_to<T>(a);
                    b = round_to<T>(b);
                    const float sl = a / (1.0f + expf(-a));
                    io<T>::st(static_cast<T *>(p.y), static_cast<int64_t>(m) * p.ldy + c,
                              round_to<T>(round_to<T>(sl) * b));
                }
            }
            continue;
        }
    }
    // Lane r * MM + m stores output (m, n0 + r).
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const int row = n0 + r;
            if (lane == r * MM + m && m < p.M && row < p.N) {
                float v = acc[r][m];
                if (p.bias) v += io<T>::ld(static_cast<const T *>(p.bias), row);
                io<T>::st(static_cast<T *>(p.y), static_cast<int64_t>(m) * p.ldy + row, v);
            }
        }
    }
    }
}

template <typename T, int MM, int NP, int RPW, int NW>
hipError_t skinny_launch(const SkinnyParams &p, hipStream_t s)
{
    const int groups = (p.N + NW * RPW - 1) / (NW * RPW);
    const dim3 grid(static_cast<unsigned>(groups < kMaxGroups ? groups : kMaxGroups));
    hipLaunchKernelGGL((skinny_linear_kernel<T, MM, NP, RPW, NW>), grid, dim3(64 * NW), 0, s, p);
    return hipGetLastError();
}

// Rows of W per wave by output width (measured at K = 1024 and 3072, M = 4):
// one for narrow outputs (more waves, so more of the matrix requested at
// once), two beyond 2048 rows (four measured slower on a 151,936-row
// output); capped so that a wave's requests (RPW * NP pieces) and sums
// (RPW * MM) stay in registers.  Wide outputs run sixteen-wave workgroups
// where the 128 registers of a 1024-thread workgroup hold the wave's state
// (MM <= 4, NP <= 2): a quarter of the workgroups to dispatch and a quarter
// of the x stagings (config-3 decode step 0.95 vs 0.98 ms at four waves);
// narrow outputs keep four, which gives 256 workgroups at 1024 rows.
template <typename T, int MM, int NP>
hipError_t skinny_np(const SkinnyParams &p, hipStream_t s)
{
    if constexpr (MM * NP > 32) {
        return hipErrorInvalidValue;  // rejected by skinny_linear_supported (x pieces would not fit in registers)
    } else {
        constexpr int LIM = 8 / NP < 16 / MM ? 8 / NP : 16 / MM;
        if constexpr (LIM >= 2)
            if (p.N > 2048 || p.glu_out) return skinny_launch<T, MM, NP, 2, (MM <= 4 && NP <= 2) ? 16 : 4>(p, s);
        if (p.glu_out) return hipErrorInvalidValue;  // rejected before (the epilogue needs two rows per wave)
        return skinny_launch<T, MM, NP, 1, 4>(p, s);
    }
}

template <typename T, int MM>
hipError_t skinny_m(const SkinnyParams &p, hipStream_t s)
{
    switch (p.K / 512) {
    case 1: return skinny_np<T, MM, 1>(p, s);
    case 2: return skinny_np<T, MM, 2>(p, s);
    case 4: return skinny_np<T, MM, 4>(p, s);
    case 6: return skinny_np<T, MM, 6>(p, s);
    default: return skinny_np<T, MM, 8>(p, s);
    }
}

template <typename T>
hipError_t skinny_t(const SkinnyParams &p, hipStream_t s)
{
    if (p.M <= 1) return skinny_m<T, 1>(p, s);
    if (p.M <= 2) return skinny_m<T, 2>(p, s);
    if (p.M <= 4) return skinny_m<T, 4>(p, s);
    return skinny_m<T, 8>(p, s);
}

// Small inner dimension (K <= 256), up to two independent problems per launch
// (blockIdx.y): KP8 = K / 8 lanes share a row of W (one 16-byte piece each),
// so a wave instruction reads 64 / KP8 consecutive rows, one contiguous 1 KB
// segment; the row's dot products are completed by xor-shuffles over those
// lanes.
template <typename T, int MM, int KP8>
__global__ __launch_bounds__(256) void small_linear_kernel(SmallLinearParams p)
{
    constexpr bool BF = std::is_same<T, bf16_t>::value;
    constexpr int RPI = 64 / KP8;  // rows per wave
    __shared__ __align__(16) uint4 sx[MM * KP8];
    const SmallLinearProblem &q = p.prob[blockIdx.y];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rsub = lane / KP8, c = lane - (lane / KP8) * KP8;
    const int row = (static_cast<int>(blockIdx.x) * kWaves + wave) * RPI + rsub;
    const T *w = static_cast<const T *>(q.w);
    const int rowc = row < q.N ? row : q.N - 1;
    // The x piece is requested before the row of W (loads complete in order, so
    // the LDS staging and the barrier then overlap W's latency).
    uint4 xv = make_uint4(0u, 0u, 0u, 0u);
    const int xm = tid / KP8, xc = tid - (tid / KP8) * KP8;
    if (tid < MM * KP8 && xm < p.M)
        xv = *reinterpret_cast<const uint4 *>(static_cast<const T *>(q.x) + xm * q.ldx + xc * 8);
    const uint4 wv = *reinterpret_cast<const uint4 *>(w + static_cast<int64_t>(rowc) * p.K + c * 8);
    if (tid < MM * KP8) sx[tid] = xv;
    __syncthreads();
    float wf[8];
    widen8(wv, wf, BF);
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        float xf[8];
        widen8(sx[m * KP8 + c], xf, BF);
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a = fmaf(wf[e], xf[e], a);
#pragma unroll
        for (int o = 1; o < KP8; o <<= 1) a += __shfl_xor(a, o, 64);
        acc[m] = a;
    }
    if (row < q.N && c < MM && c < p.M) {
        // Lane c of the row's group stores output (c, row).
        float v = acc[0];
#pragma unroll
        for (int m = 1; m < MM; ++m)
            if (m == c) v = acc[m];
        if (q.bias) v += io<T>::ld(static_cast<const T *>(q.bias), row);
        io<T>::st(static_cast<T *>(q.y), static_cast<int64_t>(c) * q.ldy + row, v);
    }
}

template <typename T, int KP8>
hipError_t small_k(const SmallLinearParams &p, int nprob, hipStream_t s)
{
    constexpr int RPW = kWaves * (64 / KP8);
    int nmax = 0;
    for (int i = 0; i < nprob; ++i) nmax = p.prob[i].N > nmax ? p.prob[i].N : nmax;
    const dim3 grid(static_cast<unsigned>((nmax + RPW - 1) / RPW), static_cast<unsigned>(nprob));
    if (p.M <= 1) hipLaunchKernelGGL((small_linear_kernel<T, 1, KP8>), grid, dim3(256), 0, s, p);
    else if (p.M <= 2) hipLaunchKernelGGL((small_linear_kernel<T, 2, KP8>), grid, dim3(256), 0, s, p);
    else if (p.M <= 4) hipLaunchKernelGGL((small_linear_kernel<T, 4, KP8>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((small_linear_kernel<T, 8, KP8>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <typename T>
hipError_t small_t(const SmallLinearParams &p, int nprob, hipStream_t s)
{
    switch (p.K / 8) {
    case 8: return small_k<T, 8>(p, nprob, s);
    case 16: return small_k<T, 16>(p, nprob, s);
    case 32: return small_k<T, 32>(p, nprob, s);
    default: return small_k<T, 4>(p, nprob, s);
    }
}

}  // namespace

bool small_linear_supported(int io_dtype, int M, int K)
{
    // Lane c of a row's K / 8 lanes stores output row c, so M <= K / 8.
    return (io_dtype == GDN2_DTYPE_BF16 || io_dtype == GDN2_DTYPE_F16) && M >= 1 && M <= 8 && M <= K / 8 &&
           (K == 32 || K == 64 || K == 128 || K == 256);
}

hipError_t launch_small_linear(const SmallLinearParams &p, int nprob, int io_dtype, hipStream_t stream)
{
    return io_dtype == GDN2_DTYPE_BF16 ? small_t<bf16_t>(p, nprob, stream) : small_t<f16_t>(p, nprob, stream);
}

bool skinny_linear_supported(int io_dtype, int M, int K)
{
    if (io_dtype != GDN2_DTYPE_BF16 && io_dtype != GDN2_DTYPE_F16) return false;
    if (M < 1 || M > 8 || K % 512 != 0) return false;
    const int np = K / 512;
    if (M > 4 && np > 4) return false;  // eight rows of x with K > 2048: torch's GEMM
    return np == 1 || np == 2 || np == 4 || np == 6 || np == 8;
}

hipError_t launch_skinny_linear(const SkinnyParams &p, int io_dtype, hipStream_t stream)
{
    return io_dtype == GDN2_DTYPE_BF16 ? skinny_t<bf16_t>(p, stream) : skinny_t<f16_t>(p, stream);
}

}  // namespace gdn2
