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
// 32-value Q8_0 block of k per step. Wavefront w owns weight rows
// 32w..32w+31 against all 128 assignment rows: 8 x 2 tiles of 16x16 (one
// 16x16x32 product each per step), 64 accumulators per lane, and it alone
// turns those weight codes into fp16 operands.
//
// Operands move from global memory straight into an NS-stage LDS ring with
// global_load_lds (no registers on the way), NS-1 steps ahead of the
// products. Each wavefront issues exactly four such loads per step, so a
// wait for the oldest step is one immediate vmcnt count. The loads are
// issued from inline assembly (which sets M0, the LDS base they use) so the
// compiler does not wait for all of them before every LDS read; the waits
// are explicit. Rows past a bucket's end load a valid row; their results are
// never stored.
#include "mhip_internal.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int GT = 256;           // threads per workgroup (4 wavefronts)
constexpr int TM = MHIP_GEMM_TM;  // assignment rows per tile
constexpr int TN = 128;           // weight rows per tile
constexpr int KB = 32;            // k per step: one Q8_0 block
constexpr int MI = TM / 16;       // 16-row tiles of assignments (8)
constexpr int NJ = 2;             // 16-row tiles of weights per wavefront
constexpr int HLD = TN / 2 + 4;   // epilogue h tile row stride (floats)
constexpr int DMA_PER_STEP = 4;   // global_load_lds per wavefront per step

static_assert(TM == 128 && TN == 128 && GT == 256, "tiling");

// One step of the ring: A rows of 32 fp16 (4 chunks of 16 bytes; chunk c of
// row r at slot c ^ ((r >> 1) & 3), so the eight rows that eight consecutive
// lanes read at one chunk fall on distinct banks), B rows of 32 int8 codes,
// and block scales of the weight rows (sb) and of the assignment rows (sa).
struct alignas(16) Step {
    _Float16 a[TM][KB];  // 8 KB
    int8_t b[TN][KB];    // 4 KB
    float sb[TN];
    float sa[TM];
};
static_assert(sizeof(Step) == 13312, "step layout");

__device__ __forceinline__ int aslot(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

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

// Tile coordinates shared by both kernels.
//
// The 1-D grid is ordered for the XCDs' L2 caches: workgroup b runs on XCD
// b % 8, and XCD k takes a contiguous share of the row tiles (consecutive
// tiles of one expert share its weights), each row tile's ny weight-row
// tiles back to back (they share its A rows). The share is computed from
// the number of row tiles the dispatch produced; workgroups beyond it exit.
struct TileRef {
    int e, base, nrows, y;
};
constexpr int NXCD = 8;
__device__ __forceinline__ bool tile_of(const int *groups, const int *gtile, int ny,
                                        TileRef &t) {
    const int G = groups[0];
    if (G == 0) return false;
    const int nreal = gtile[G];
    const int b = blockIdx.x, xcd = b % NXCD, r = b / NXCD;
    const int share = (nreal + NXCD - 1) / NXCD;
    const int q = r / ny;
    if (q >= share) return false;
    const int mt = xcd * share + q;
    if (mt >= nreal) return false;
    t.y = r % ny;
    const int g = find_group(gtile, G, mt);
    t.e = groups[1 + 3 * g];
    t.base = groups[2 + 3 * g] + (mt - gtile[g]) * TM;
    t.nrows = min(TM, groups[3 + 3 * g] - t.base);
    return true;
}

// global -> LDS, 16 (resp. 4) bytes per lane; lane i writes LDS at
// lds + 16 i (resp. 4 i). lds must be wavefront-uniform.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(unsigned lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(unsigned lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return (unsigned)(uintptr_t)p;
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

// Per-thread global sources of one tile, advanced by one block per step.
struct Src {
    const _Float16 *a0, *a1;  // A chunks of rows ar0, ar1 (fp16, KB halves per step)
    const int8_t *b;          // B 16-byte half of weight row br (KB bytes per step)
    const float *s;           // a block scale in a block-major array ...
    int sstep;                // ... whose blocks are sstep floats apart
};

// The k loop over nk steps (nk >= NS - 1). On return acc[i][j][r] holds
//   C[16*i + 4*(lane/16) + r][32*wave + 16*j + lane%16].
template <int NS, bool EXACT>
__device__ __forceinline__ void gemm_tile(Step *ring, const Src &src, int nk, f4v acc[MI][NJ]) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // LDS destinations of this wavefront's four loads within a step
    const unsigned ring0 = lds_addr(ring);
    const unsigned oa0 = (unsigned)offsetof(Step, a) + (2 * wave) * 1024;
    const unsigned oa1 = oa0 + 1024;
    const unsigned ob = (unsigned)offsetof(Step, b) + wave * 1024;
    // waves 0, 1: the weight rows' scales; waves 2, 3: the assignment rows'
    const unsigned os = (wave < 2 ? (unsigned)offsetof(Step, sb) : (unsigned)offsetof(Step, sa)) +
                        (wave & 1) * 256;
    auto issue = [&](int kb) {
        const int k = min(kb, nk - 1);  // past the end: reload the last step
        const unsigned st = ring0 + (unsigned)((kb % NS) * sizeof(Step));
        dma16(st + oa0, src.a0 + (size_t)k * KB);
        dma16(st + oa1, src.a1 + (size_t)k * KB);
        dma16(st + ob, src.b + (size_t)k * KB);
        dma4(st + os, src.s + (size_t)k * src.sstep);
    };
#pragma unroll
    for (int s = 0; s < NS - 1; s++) issue(s);
    for (int kb = 0; kb < nk; kb++) {
        // this wavefront's loads of step kb are done (NS - 2 later steps may
        // still be in flight); then every wavefront's are
        wait_vm<(NS - 2) * DMA_PER_STEP>();
        __syncthreads();
        // step kb + NS - 1 reuses the slot read in step kb - 1, which every
        // wavefront has finished with (the LDS reads completed before the
        // barrier)
        issue(kb + NS - 1);
        const Step &S = ring[kb % NS];
        const int ck = lane >> 4;
        h8 bv[NJ];
        float sw[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int n = 32 * wave + 16 * j + (lane & 15);
            const uint2 q = *(const uint2 *)&S.b[n][8 * ck];
            bv[j] = codes8(q.x, q.y);
            sw[j] = S.sb[n];
            if (!EXACT) {
                const _Float16 s = (_Float16)sw[j];
                const h8 s8 = {s, s, s, s, s, s, s, s};
                bv[j] = bv[j] * s8;
            }
        }
#pragma unroll
        for (int i = 0; i < MI; i++) {
            const int m = 16 * i + (lane & 15);
            const h8 av = *(const h8 *)&S.a[m][8 * aslot(m, ck)];
            if (EXACT) {
                const float4 sx = *(const float4 *)&S.sa[16 * i + 4 * ck];
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
                    const f4v blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[j], z, 0, 0, 0);
                    acc[i][j][0] = acc[i][j][0] + (blk[0] * sw[j]) * sx.x;
                    acc[i][j][1] = acc[i][j][1] + (blk[1] * sw[j]) * sx.y;
                    acc[i][j][2] = acc[i][j][2] + (blk[2] * sw[j]) * sx.z;
                    acc[i][j][3] = acc[i][j][3] + (blk[3] * sw[j]) * sx.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[j], acc[i][j], 0, 0, 0);
            }
        }
    }
    wait_vm<0>();  // the reloads past the end
    __syncthreads();
}

// The A rows this thread loads: rows 32*wave + 16*q + lane/4 (q = 0, 1), in
// the chunk that lands in LDS slot lane % 4.
__device__ __forceinline__ void a_rows(int &r0, int &c0, int &r1, int &c1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    r0 = 32 * wave + (lane >> 2);
    r1 = r0 + 16;
    c0 = aslot(r0, lane & 3);  // slot ^ swizzle = the chunk stored there
    c1 = aslot(r1, lane & 3);
}

// ---- x block scales in bucketed, block-major order --------------------------------
//
// xsb[k][p] = xs[t][k] for the assignment p = (t, j) in bucketed order, so a
// tile's 128 rows read their scales of block k as one contiguous run.
__global__ __launch_bounds__(256) void k_xs_bucket(const float *__restrict__ xs,
                                                   const int *__restrict__ perm,
                                                   float *__restrict__ xsb, int A, int nb, int K) {
    const int p = blockIdx.x * 256 + threadIdx.x, k = blockIdx.y;
    if (p < A) xsb[(size_t)k * A + p] = xs[(size_t)(perm[p] / K) * nb + k];
}

// ---- gate/up + SwiGLU + Q8(h) ----------------------------------------------------
//
// blockIdx.x = tile of assignment rows (gtile numbering), blockIdx.y = 64
// consecutive h columns h0..h0+63. Wavefront w's 32 weight rows are the gate
// rows then the up rows of h columns h0+16w..h0+16w+15, so SwiGLU pairs its
// accumulator tiles 0 and 1 lane by lane.
constexpr int NS_GU = 4;
constexpr int NS_DN = 6;

union alignas(16) GateUpLds {
    Step ring[NS_GU];
    float h[TM][HLD];
};
union alignas(16) DownLds {
    Step ring[NS_DN];
};

__global__ __launch_bounds__(GT, 1) void k_gateup_mfma(
    const uint8_t *__restrict__ table, mhip_layout lay, const _Float16 *__restrict__ xq16,
    const float *__restrict__ xsb, const int *__restrict__ groups, const int *__restrict__ gtile,
    const int *__restrict__ perm, _Float16 *__restrict__ hdq, int d, int eh, int K, int A) {
    __shared__ GateUpLds L;
    TileRef tr;
    if (!tile_of(groups, gtile, eh / (TN / 2), tr)) return;
    const int base = tr.base, nrows = tr.nrows;
    const int h0 = tr.y * (TN / 2);
    const uint8_t *ex = table + (size_t)tr.e * lay.expert_bytes;
    const int nb = d / KB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    Src src;
    {
        int r0, c0, r1, c1;
        a_rows(r0, c0, r1, c1);
        const int t0 = perm[base + min(r0, nrows - 1)] / K;
        const int t1 = perm[base + min(r1, nrows - 1)] / K;
        src.a0 = xq16 + (size_t)t0 * d + c0 * 8;
        src.a1 = xq16 + (size_t)t1 * d + c1 * 8;
        // weight row of B row 32*wave + lane/2: gate rows then up rows
        const int bj = (lane >> 1) >> 4, br = (lane >> 1) & 15;
        const int wr = h0 + 16 * wave + br;
        src.b = (const int8_t *)(ex + (bj == 0 ? lay.gate_q : lay.up_q)) + (size_t)wr * d +
                (lane & 1) * 16;
        // block-major scales: the 128 rows of a step are 4 (waves 0, 1) or
        // 1 (waves 2, 3) contiguous runs
        if (wave < 2) {
            // scale of B row 64*wave + lane
            const int b = 64 * wave + lane;
            const int sw = h0 + 16 * (b >> 5) + (b & 15);
            src.s = (const float *)(ex + (((b >> 4) & 1) == 0 ? lay.gate_st : lay.up_st)) + sw;
            src.sstep = eh;
        } else {
            // scale of assignment row 64*(wave-2) + lane
            const int m = 64 * (wave - 2) + lane;
            src.s = xsb + base + min(m, nrows - 1);
            src.sstep = A;
        }
    }

    f4v acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    gemm_tile<NS_GU, true>(L.ring, src, nb, acc);

    // SwiGLU into the h tile (LDS, reused), then Q8_0 per 32-block
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * i + 4 * (lane >> 4) + r;
            const float gv = acc[i][0][r], uv = acc[i][1][r];
            L.h[m][16 * wave + (lane & 15)] = (gv / (1.0f + mia_expf_glibc(-gv))) * uv;
        }
    __syncthreads();
    {
        // Q8_0 of one 32-block of h (quant.c:11-27), stored dequantized
        const int m = tid >> 1, i = tid & 1;
        if (m < nrows) {
            const float4 *hs = (const float4 *)&L.h[m][32 * i];
            float v[32];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 q = hs[k];
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
    __shared__ DownLds L;
    TileRef tr;
    if (!tile_of(groups, gtile, d / TN, tr)) return;
    const int base = tr.base, nrows = tr.nrows;
    const int n0 = tr.y * TN;
    const uint8_t *ex = table + (size_t)tr.e * lay.expert_bytes;
    const int nbh = eh / KB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    Src src;
    {
        int r0, c0, r1, c1;
        a_rows(r0, c0, r1, c1);
        src.a0 = hdq + (size_t)(base + min(r0, nrows - 1)) * eh + c0 * 8;
        src.a1 = hdq + (size_t)(base + min(r1, nrows - 1)) * eh + c1 * 8;
        const int row = n0 + 32 * wave + (lane >> 1);
        src.b = (const int8_t *)(ex + lay.down_q) + (size_t)row * eh + (lane & 1) * 16;
        // scales of weight rows 64*(wave&1) + lane, block-major (waves 2, 3
        // repeat waves 0, 1 into the unused assignment-scale slot)
        src.s = (const float *)(ex + lay.down_st) + n0 + 64 * (wave & 1) + lane;
        src.sstep = d;
    }

    f4v acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    gemm_tile<NS_DN, false>(L.ring, src, nbh, acc);

#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * i + 4 * (lane >> 4) + r;
            if (m < nrows) {
                float *dst = tmp + (size_t)(base + m) * d + n0 + 32 * wave + (lane & 15);
#pragma unroll
                for (int j = 0; j < NJ; j++) dst[16 * j] = acc[i][j][r];
            }
        }
}

}  // namespace

namespace mhip {

bool gemm_path_fits(const mhip_dims *s) {
    // whole tiles of weight rows, and enough k steps to fill the rings
    return s->dim % TN == 0 && s->expert_hidden % (TN / 2) == 0 &&
           s->dim / KB >= NS_GU - 1 && s->expert_hidden / KB >= NS_DN - 1;
}

int gemm_max_tiles(int A, int E) { return (A + TM - 1) / TM + (A < E ? A : E); }

// Workgroups for ny weight-row tiles: every XCD's share can hold all row tiles.
static unsigned gemm_grid(int A, int E, int ny) {
    const int share = (gemm_max_tiles(A, E) + NXCD - 1) / NXCD;
    return (unsigned)(NXCD * share * ny);
}

int launch_gateup_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                       const void *d_table_layer, const mhip_scratch *sc, int A) {
    const int d = s->dim, eh = s->expert_hidden;
    k_xs_bucket<<<dim3((A + 255) / 256, d / KB), 256, 0, st>>>(sc->xs, sc->perm, sc->xsb, A,
                                                              d / KB, s->n_active);
    const unsigned grid = gemm_grid(A, s->n_experts, eh / (TN / 2));
    k_gateup_mfma<<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                       (const _Float16 *)sc->xdq, sc->xsb, sc->groups,
                                       sc->gtile, sc->perm, (_Float16 *)sc->hdq, d, eh,
                                       s->n_active, A);
    return (int)hipGetLastError();
}

int launch_down_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                     const void *d_table_layer, const mhip_scratch *sc, int A) {
    const int d = s->dim, eh = s->expert_hidden;
    const unsigned grid = gemm_grid(A, s->n_experts, d / TN);
    k_down_mfma<<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                     (const _Float16 *)sc->hdq, sc->groups, sc->gtile, sc->tmp,
                                     d, eh);
    return (int)hipGetLastError();
}

}  // namespace mhip
