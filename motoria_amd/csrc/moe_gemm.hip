// Expert products of the batched / prefill MoE layer on the matrix cores.
//
// For T tokens the T*K assignments are bucketed by expert (k_dispatch); each
// expert's bucket is a dense contraction with that expert's weights:
//
//   k_gateup_mfma  h = SwiGLU(Wg x, Wu x), then Q8_0(h)   forward.c:186-192
//   k_down_mfma    tmp = Wd Q8(h)                           forward.c:192-193
//
// gate/up is bit-exact. Its operands are the Q8_0 codes themselves, as fp16
// integers: v_mfma_f32_16x16x32_f16 over one 32-value block gives the exact
// int32 block dot (every partial sum is an integer below 2^24), and the
// reference's term ((float)acc * d_w) * d_x is added to the row sum in block
// order by the vector ALUs (matmul.c:19-28). h, and so Q8(h), are therefore
// the reference's bits. (Q8(h) is sensitive: an h off by 1e-4 moves ~3 % of
// its codes by one step, and one code step on a large down weight is a
// 1e-3 change of the output.)
//
// down takes the reference's dequantized values (d * q for the weights,
// d_h * q_h for h) rounded to fp16 on the matrix cores with fp32
// accumulation: ~1e-4 relative of the reference, within the path's 1e-3.
//
// Tiles: 128 assignments (rows of one expert's bucket) x 128 weight rows, one
// 32-value Q8_0 block of k per step (one 16x16x32 product per 16x16 tile).
// Wavefront w owns assignment rows 32w..32w+31 against all 128 weight rows:
// 2 x 8 tiles of 16x16, 64 accumulators per lane. Weight codes become fp16
// on the way into LDS (a byte permute and one packed fp16 subtract per two
// codes); the k loop double-buffers LDS and keeps the global loads two
// blocks ahead in registers.
#include "mhip_internal.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int GT = 256;           // threads per workgroup (4 wavefronts)
constexpr int TM = MHIP_GEMM_TM;  // assignment rows per tile
constexpr int TN = 128;           // weight rows per tile
constexpr int KB = 32;            // k per step: one Q8_0 block
constexpr int LDK = KB;           // LDS row: 32 halves = 4 chunks of 16 bytes, swizzled
constexpr int HLD = TN / 2 + 4;   // epilogue h tile row stride (floats)
constexpr int MT = 2, NTL = TN / 16;  // 16x16 tiles per wavefront: 2 (rows) x 8 (weight rows)

static_assert(TM == 128 && GT == 256, "4 wavefronts x 32 assignment rows");
static_assert(TM <= GT && TN == GT / 2, "staging: one thread per scale, two per B row");

// LDS: two buffers of two k steps each ([buffer][step][row][k]). The 16-byte
// chunk c of row r is stored at chunk c ^ ((r >> 2) & 3), so the 16 lanes of
// an operand read (16 consecutive rows, one chunk) hit 16 distinct groups of
// 4 banks.
struct KLds {
    alignas(16) _Float16 a[2][2][TM][LDK];
    alignas(16) _Float16 b[2][2][TN][LDK];
    alignas(16) float sa[2][2][TM];   // activation block scales (gate/up)
    alignas(16) float sb[2][2][TN];   // weight block scales (gate/up)
};
union alignas(16) GemmLds {
    KLds k;
    alignas(16) float h[TM][HLD];
};

// The group g with gtile[g] <= mt < gtile[g + 1] (gtile is non-decreasing).
__device__ __forceinline__ int find_group(const int *gtile, int G, int mt) {
    int lo = 0, hi = G;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (gtile[mid] <= mt)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

// 8 Q8_0 codes (two little-endian words) as fp16 integers, in byte order:
// flipping the sign bit gives the code + 128 as a byte u, the fp16 with bits
// 0x64 u is 1024 + u, and subtracting 1152 is exact.
__device__ __forceinline__ h8 codes8(unsigned w0, unsigned w1) {
    const unsigned u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    const unsigned d[4] = {__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)};
    const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 v = __builtin_bit_cast(h2, d[i]) - off;
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ ((row >> 2) & 3)) * 8; }

// v if keep, else zeros (a value select: no address is taken).
__device__ __forceinline__ int4 keep4(bool keep, const int4 v) {
    return make_int4(keep ? v.x : 0, keep ? v.y : 0, keep ? v.z : 0, keep ? v.w : 0);
}

// Generic grouped GEMM over one tile; EXACT selects gate/up (codes as fp16
// integers, exact per-block epilogue) or down (dequantized operands).
// A rows come from arow0/arow1 (fp16, KB halves per step; always readable:
// rows past the bucket's end point at a valid row and are zeroed by aval);
// B rows are Q8_0 codes bq with scales bs; ascale (gate/up) is the
// block-scale row of assignment row tid (threads < TM; always readable,
// zeroed by sval); nk = k steps.
// On return acc[i][j][r] holds
//   C[32*wave + 16*i + 4*(lane/16) + r][16*j + lane%16].
//
// Each iteration takes two k steps: it issues the global loads of the next
// two steps into registers, runs its own two steps from one LDS buffer, then
// stores the loaded steps into the other buffer and synchronises. No load is
// in flight across the loop's back edge, so the compiler's wait counts are
// exact, and the loads have two steps of products to arrive. Every load is
// unconditional (the step index is clamped to the last step).
template <bool EXACT>
__device__ __forceinline__ void gemm_tile(GemmLds &L, const _Float16 *arow0,
                                          const _Float16 *arow1, bool aval0, bool aval1,
                                          int am0, int ap0, int am1, int ap1,
                                          const int8_t *bq, const float *bs, int brow, int bh,
                                          const float *ascale, bool sval, int nk,
                                          f4v acc[MT][NTL]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int4 a0[2], a1[2], bw[2];
    float sw[2], sa[2];
#define GEMM_LOAD(S, KB_)                                                             \
    do {                                                                              \
        const size_t k_ = (size_t)min((KB_), nk - 1);                                 \
        a0[S] = *(const int4 *)(arow0 + k_ * KB);                                     \
        a1[S] = *(const int4 *)(arow1 + k_ * KB);                                     \
        bw[S] = *(const int4 *)(bq + k_ * KB);                                        \
        sw[S] = bs[k_];                                                               \
        if (EXACT) sa[S] = ascale[k_];                                                \
    } while (0)
#define GEMM_STORE(S, P)                                                              \
    do {                                                                              \
        *(int4 *)&L.k.a[P][S][am0][swz(am0, ap0)] = keep4(aval0, a0[S]);              \
        *(int4 *)&L.k.a[P][S][am1][swz(am1, ap1)] = keep4(aval1, a1[S]);              \
        h8 lo_ = codes8((unsigned)bw[S].x, (unsigned)bw[S].y);                        \
        h8 hi_ = codes8((unsigned)bw[S].z, (unsigned)bw[S].w);                        \
        if (EXACT) {                                                                  \
            if (bh == 0) L.k.sb[P][S][brow] = sw[S];                                  \
            if (tid < TM) L.k.sa[P][S][tid] = sval ? sa[S] : 0.0f;                    \
        } else {                                                                      \
            const _Float16 s_ = (_Float16)sw[S];                                      \
            const h8 s8_ = {s_, s_, s_, s_, s_, s_, s_, s_};                          \
            lo_ = lo_ * s8_;                                                          \
            hi_ = hi_ * s8_;                                                          \
        }                                                                             \
        *(h8 *)&L.k.b[P][S][brow][swz(brow, 2 * bh)] = lo_;                           \
        *(h8 *)&L.k.b[P][S][brow][swz(brow, 2 * bh + 1)] = hi_;                       \
    } while (0)
#define GEMM_MMA(P, S)                                                                 \
    do {                                                                              \
        const int ck = lane >> 4;                                                     \
        h8 av[MT];                                                                    \
        _Pragma("unroll") for (int i = 0; i < MT; i++) av[i] =                        \
            *(const h8 *)&L.k.a[P][S][32 * wave + 16 * i + (lane & 15)]               \
                                  [swz(32 * wave + 16 * i + (lane & 15), ck)];        \
        if (EXACT) {                                                                  \
            /* tile j's products are issued while tile j-1's are scaled and    */    \
            /* added; scheduling barriers keep two tiles' products live at most */   \
            float4 sx[MT];                                                            \
            _Pragma("unroll") for (int i = 0; i < MT; i++) sx[i] =                    \
                *(const float4 *)&L.k.sa[P][S][32 * wave + 16 * i + 4 * (lane >> 4)];    \
            f4v pc[MT], pn[MT];                                                       \
            float wc = 0.0f, wn = 0.0f;                                               \
            _Pragma("unroll") for (int j = 0; j <= NTL; j++) {                        \
                if (j < NTL) {                                                        \
                    const h8 bv = *(const h8 *)&L.k.b[P][S][16 * j + (lane & 15)]      \
                                                     [swz(16 * j + (lane & 15), ck)]; \
                    wn = L.k.sb[P][S][16 * j + (lane & 15)];                          \
                    _Pragma("unroll") for (int i = 0; i < MT; i++) {                  \
                        const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};                       \
                        pn[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv, z, 0, 0, 0); \
                    }                                                                 \
                }                                                                     \
                if (j > 0) {                                                          \
                    _Pragma("unroll") for (int i = 0; i < MT; i++) {                  \
                        f4v &c = acc[i][j - 1];                                       \
                        c[0] = c[0] + (pc[i][0] * wc) * sx[i].x;                      \
                        c[1] = c[1] + (pc[i][1] * wc) * sx[i].y;                      \
                        c[2] = c[2] + (pc[i][2] * wc) * sx[i].z;                      \
                        c[3] = c[3] + (pc[i][3] * wc) * sx[i].w;                      \
                    }                                                                 \
                }                                                                     \
                _Pragma("unroll") for (int i = 0; i < MT; i++) pc[i] = pn[i];         \
                wc = wn;                                                              \
                __builtin_amdgcn_sched_barrier(0);                                    \
            }                                                                         \
        } else {                                                                      \
            _Pragma("unroll") for (int j = 0; j < NTL; j++) {                         \
                const h8 bv = *(const h8 *)&L.k.b[P][S][16 * j + (lane & 15)]          \
                                                 [swz(16 * j + (lane & 15), ck)];     \
                _Pragma("unroll") for (int i = 0; i < MT; i++) acc[i][j] =            \
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv, acc[i][j], 0, 0, 0); \
            }                                                                         \
        }                                                                             \
    } while (0)
    // nk is even (gemm_path_fits): the loop moves in pairs of steps.
    GEMM_LOAD(0, 0);
    GEMM_LOAD(1, 1);
    GEMM_STORE(0, 0);
    GEMM_STORE(1, 0);
    __syncthreads();
    for (int kb = 0; kb < nk; kb += 2) {
        const int p = (kb >> 1) & 1;
        GEMM_LOAD(0, kb + 2);
        GEMM_LOAD(1, kb + 3);
        asm volatile("" ::: "memory");  // the prefetch goes out before this pair's work
        GEMM_MMA(p, 0);
        asm volatile("" ::: "memory");  // one step's operands and products at a time
        GEMM_MMA(p, 1);
        asm volatile("" ::: "memory");
        GEMM_STORE(0, p ^ 1);
        GEMM_STORE(1, p ^ 1);
        __syncthreads();
    }
#undef GEMM_LOAD
#undef GEMM_STORE
#undef GEMM_MMA
}

// Tile coordinates shared by both kernels.
struct TileRef {
    int e, base, nrows;
};
__device__ __forceinline__ bool tile_of(const int *groups, const int *gtile, int mt, TileRef &t) {
    const int G = groups[0];
    if (G == 0 || mt >= gtile[G]) return false;
    const int g = find_group(gtile, G, mt);
    t.e = groups[1 + 3 * g];
    t.base = groups[2 + 3 * g] + (mt - gtile[g]) * TM;
    t.nrows = min(TM, groups[3 + 3 * g] - t.base);
    return true;
}

// ---- gate/up + SwiGLU + Q8(h) ----------------------------------------------------
//
// blockIdx.x = tile of assignment rows (gtile numbering), blockIdx.y = 64
// consecutive h columns; the tile's 128 weight rows are those 64 gate rows
// and the 64 up rows of the same h columns, so SwiGLU pairs accumulator
// tiles j and j + 4 of a wavefront lane by lane.
__global__ __launch_bounds__(GT, 1) void k_gateup_mfma(
    const uint8_t *__restrict__ table, mhip_layout lay, const _Float16 *__restrict__ xq16,
    const float *__restrict__ xs, const int *__restrict__ groups, const int *__restrict__ gtile,
    const int *__restrict__ perm, _Float16 *__restrict__ hdq, int d, int eh, int K) {
    __shared__ GemmLds L;
    TileRef tr;
    if (!tile_of(groups, gtile, blockIdx.x, tr)) return;
    const int base = tr.base, nrows = tr.nrows;
    const int h0 = blockIdx.y * (TN / 2);
    const uint8_t *ex = table + (size_t)tr.e * lay.expert_bytes;
    const int nb = d / KB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // A: this thread's two 16-byte chunks per step (rows am, parts ap); rows
    // past the bucket's end read its first row and are zeroed
    const int am0 = tid >> 2, ap0 = tid & 3, am1 = (tid + GT) >> 2, ap1 = (tid + GT) & 3;
    const bool aval0 = am0 < nrows, aval1 = am1 < nrows;
    const int t0 = perm[base + (aval0 ? am0 : 0)] / K;
    const int t1 = perm[base + (aval1 ? am1 : 0)] / K;
    const _Float16 *arow0 = xq16 + (size_t)t0 * d + ap0 * 8;
    const _Float16 *arow1 = xq16 + (size_t)t1 * d + ap1 * 8;
    // block scales of assignment row tid (threads 0..TM-1; zeroed past the end)
    const bool sval = tid < nrows;
    const float *ascale = xs + (size_t)(perm[base + (sval ? tid : 0)] / K) * nb;
    // B: weight row brow (gate rows first, then up rows), 16-byte half bh
    const int brow = tid >> 1, bh = tid & 1;
    const bool isg = brow < TN / 2;
    const int wr = h0 + (isg ? brow : brow - TN / 2);
    const int8_t *bq = (const int8_t *)(ex + (isg ? lay.gate_q : lay.up_q)) + (size_t)wr * d + bh * 16;
    const float *bs = (const float *)(ex + (isg ? lay.gate_s : lay.up_s)) + (size_t)wr * nb;

    f4v acc[MT][NTL];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NTL; j++) acc[i][j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    gemm_tile<true>(L, arow0, arow1, aval0, aval1, am0, ap0, am1, ap1, bq, bs, brow, bh, ascale,
                    sval, nb, acc);

    __syncthreads();  // every wavefront is done with the k-loop LDS
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NTL / 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = 32 * wave + 16 * i + 4 * (lane >> 4) + r;
                const float gv = acc[i][j][r], uv = acc[i][j + NTL / 2][r];
                L.h[m][16 * j + (lane & 15)] = (gv / (1.0f + mia_expf_glibc(-gv))) * uv;
            }
    __syncthreads();
    {
        // Q8_0 of one 32-block of h (quant.c:11-27), stored dequantized
        const int m = tid >> 1, i = tid & 1;
        if (m < nrows) {
            const float4 *src = (const float4 *)&L.h[m][32 * i];
            float v[32];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 q = src[k];
                v[4 * k] = q.x;
                v[4 * k + 1] = q.y;
                v[4 * k + 2] = q.z;
                v[4 * k + 3] = q.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(v[k]));
            const float dsc = amax / 127.0f;
            const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
            h8 o[4];
#pragma unroll
            for (int k = 0; k < 32; k++) o[k >> 3][k & 7] = (_Float16)(roundf(v[k] * qi) * dsc);
            h8 *dst = (h8 *)(hdq + (size_t)(base + m) * eh + h0 + 32 * i);
#pragma unroll
            for (int k = 0; k < 4; k++) dst[k] = o[k];
        }
    }
}

// ---- down -----------------------------------------------------------------------------
//
// blockIdx.x = tile of assignment rows, blockIdx.y = 128 consecutive down
// rows. A rows are the tile's Q8(h) (fp16, bucketed order, contiguous).
__global__ __launch_bounds__(GT, 2) void k_down_mfma(const uint8_t *__restrict__ table,
                                                     mhip_layout lay,
                                                     const _Float16 *__restrict__ hdq,
                                                     const int *__restrict__ groups,
                                                     const int *__restrict__ gtile,
                                                     float *__restrict__ tmp, int d, int eh) {
    __shared__ GemmLds L;
    TileRef tr;
    if (!tile_of(groups, gtile, blockIdx.x, tr)) return;
    const int base = tr.base, nrows = tr.nrows;
    const int n0 = blockIdx.y * TN;
    const uint8_t *ex = table + (size_t)tr.e * lay.expert_bytes;
    const int nbh = eh / KB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    const int am0 = tid >> 2, ap0 = tid & 3, am1 = (tid + GT) >> 2, ap1 = (tid + GT) & 3;
    const bool aval0 = am0 < nrows, aval1 = am1 < nrows;
    const _Float16 *arow0 = hdq + (size_t)(base + (aval0 ? am0 : 0)) * eh + ap0 * 8;
    const _Float16 *arow1 = hdq + (size_t)(base + (aval1 ? am1 : 0)) * eh + ap1 * 8;
    const int brow = tid >> 1, bh = tid & 1;
    const int8_t *bq = (const int8_t *)(ex + lay.down_q) + (size_t)(n0 + brow) * eh + bh * 16;
    const float *bs = (const float *)(ex + lay.down_s) + (size_t)(n0 + brow) * nbh;

    f4v acc[MT][NTL];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NTL; j++) acc[i][j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    gemm_tile<false>(L, arow0, arow1, aval0, aval1, am0, ap0, am1, ap1, bq, bs, brow, bh, bs,
                     false, nbh, acc);

#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 32 * wave + 16 * i + 4 * (lane >> 4) + r;
            if (m < nrows) {
                float *dst = tmp + (size_t)(base + m) * d + n0 + (lane & 15);
#pragma unroll
                for (int j = 0; j < NTL; j++) dst[16 * j] = acc[i][j][r];
            }
        }
}

}  // namespace

namespace mhip {

bool gemm_path_fits(const mhip_dims *s) {
    // whole tiles of weight rows, and an even number of k steps
    return s->dim % TN == 0 && s->expert_hidden % (TN / 2) == 0 && s->dim % (2 * KB) == 0 &&
           s->expert_hidden % (2 * KB) == 0;
}

int gemm_max_tiles(int A, int E) { return (A + TM - 1) / TM + (A < E ? A : E); }

int launch_gateup_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                       const void *d_table_layer, const mhip_scratch *sc, int A) {
    const int d = s->dim, eh = s->expert_hidden;
    dim3 grid((unsigned)gemm_max_tiles(A, s->n_experts), (unsigned)(eh / (TN / 2)));
    k_gateup_mfma<<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                       (const _Float16 *)sc->xdq, sc->xs, sc->groups,
                                       sc->gtile, sc->perm, (_Float16 *)sc->hdq, d, eh,
                                       s->n_active);
    return (int)hipGetLastError();
}

int launch_down_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                     const void *d_table_layer, const mhip_scratch *sc, int A) {
    const int d = s->dim, eh = s->expert_hidden;
    dim3 grid((unsigned)gemm_max_tiles(A, s->n_experts), (unsigned)(d / TN));
    k_down_mfma<<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                     (const _Float16 *)sc->hdq, sc->groups, sc->gtile, sc->tmp,
                                     d, eh);
    return (int)hipGetLastError();
}

}  // namespace mhip
