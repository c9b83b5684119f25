// Expert products of the batched / prefill MoE layer on the matrix cores.
//
// For T tokens the T*K assignments are bucketed by expert (k_disp_*); each
// expert's bucket is a dense contraction with that expert's weights:
//
//   k_gateup_mfma  h = SwiGLU(Wg x, Wu x), then Q8_0(h)   forward.c:186-192
//   k_down_mfma    tmp = Wd Q8(h)                           forward.c:192-193
//
// Both products run on the Q8_0 codes themselves, as fp16 integers:
// v_mfma_f32_16x16x32_f16 over one 32-value block gives the exact int32
// block dot (every partial sum is an integer below 2^24). The reference's
// block term ((float)acc * d_w) * d_x is added to the row sum in block order
// by the vector ALUs (matmul.c:19-28). gate/up keeps the reference's three
// roundings, so h, and Q8(h) after it, are bit-equal to the reference's: h
// is requantized, and a code that flips on a last-ulp difference moves a
// token's layer output by up to ~1.5e-3 relative (measured over 48 layers of
// 4096 tokens with one fused multiply-add there). down, whose output is not
// requantized, adds each term with one fused multiply-add (the second
// product's rounding and the addition's become one): the expert outputs are
// within a few fp32 ulps of the reference's. gate/up writes Q8(h) as fp16
// codes plus block-major scales, which down reads the same way as gate/up
// reads Q8(xn); no operand is ever rounded to fp16.
//
// Tiles: 256 weight rows x 128 assignments (rows of one expert's bucket),
// one 32-value Q8_0 block of k per step. Wavefront w owns weight rows
// 64w..64w+63 against all 128 assignments: 4 x 8 tiles of 16x16 with the
// weights as the A operand, so each lane's four results share one
// assignment (one x scale) and four consecutive weight rows (one float4 of
// weight scales). Two gate/up or three down workgroups share a CU.
//
// Operands move from global memory straight into an NS-stage LDS ring with
// global_load_lds (no registers on the way), NS-1 steps ahead of the
// products. Each wavefront issues a fixed number of such loads per step, so
// a wait for the oldest step is one immediate vmcnt count. The loads are
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
constexpr int TN = 256;           // weight rows per tile
constexpr int KB = 32;            // k per step: one Q8_0 block
constexpr int WN = TN / 4;        // weight rows per wavefront (64)
constexpr int MI = WN / 16;       // 16-row weight tiles per wavefront (4)
constexpr int NJ = TM / 16;       // 16-row assignment tiles (8)
constexpr int NS = 4;             // ring stages (two workgroups per CU)
constexpr int OLD = TM + 4;       // gate/up epilogue tile row stride (floats): 128 columns + pad
constexpr int DLD = WN + 4;       // down epilogue tile row stride: 64 columns + pad

static_assert(TM == 128 && TN == 256 && GT == 256, "tiling");

// One step of the ring.
//   x:  assignment rows, 32 fp16 codes = 4 chunks of 16 bytes; chunk c
//       of row m sits at slot c ^ ((m >> 1) & 3), so the eight rows that
//       eight consecutive lanes read at one chunk fall on distinct banks;
//   w:  weight rows, 32 int8 codes = 2 halves of 16 bytes; half h of row n
//       sits at slot h ^ ((n >> 3) & 1), so the sixteen rows that sixteen
//       consecutive lanes read (8 bytes each) fall on distinct banks;
//   sw: block scales of the weight rows, sx: of the assignment rows.
struct alignas(16) Step {
    _Float16 x[TM][KB];  // 8 KB
    int8_t w[TN][KB];    // 8 KB
    float sw[TN];        // 1 KB
    float sx[TM];        // 512 B: the scale of bucket row 16 j + l at 8 l + j
};
static_assert(sizeof(Step) == 17920, "step layout");

__device__ __forceinline__ int xslot(int m, int chunk) { return chunk ^ ((m >> 1) & 3); }
__device__ __forceinline__ int wslot(int n, int half) { return half ^ ((n >> 3) & 1); }

// The group g < G with f(g) <= p < f(g + 1), for a non-decreasing f over
// 0..G with f(0) <= p < f(G).
template <typename F>
__device__ __forceinline__ int find_group(F f, int G, int p) {
    int lo = 0, hi = G;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (f(mid) <= p)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

// Tile coordinates shared by both kernels.
//
// A bucket's row tiles are TM rows each but its last, which holds the rest;
// that one is light when it has at most TM / 2 rows (its products run on at
// most four 16-row assignment tiles), heavy otherwise. The 1-D grid is
// ordered for balance and for the XCDs' L2 caches: workgroup b runs on XCD
// b % 8, and XCD k takes a contiguous eighth of the heavy row tiles (in
// bucket order, so consecutive tiles of one expert share its weights), then
// a contiguous eighth of the light ones, each row tile's ny weight-row tiles
// back to back (they share its A rows). Every XCD thus starts the same number
// of heavy tiles (within one) before any light tile, and the light tiles fill
// the last round. Workgroups beyond an XCD's shares exit.
struct TileRef {
    int e, base, nrows, y;
};
constexpr int NXCD = 8;
__device__ __forceinline__ bool tile_of(const int *groups, const int *gtile, const int *glight,
                                        int ny, TileRef &t) {
    const int G = groups[0];
    if (G == 0) return false;
    const int nl = glight[G], nh = gtile[G] - nl;
    const int hs = (nh + NXCD - 1) / NXCD, ls = (nl + NXCD - 1) / NXCD;
    const int b = blockIdx.x, xcd = b % NXCD, r = b / NXCD;
    const int q = r / ny;
    const int hk = max(0, min(hs, nh - xcd * hs)), lk = max(0, min(ls, nl - xcd * ls));
    int g, mt;
    if (q < hk) {
        // heavy tile p: group g's heavy tiles are its first
        // (gtile - glight)(g + 1) - (gtile - glight)(g)
        const int p = xcd * hs + q;
        auto heavy_before = [&](int k) { return gtile[k] - glight[k]; };
        g = find_group(heavy_before, G, p);
        mt = gtile[g] + (p - heavy_before(g));
    } else if (q < hk + lk) {
        // light tile p: the last tile of the group with glight(g) == p
        const int p = xcd * ls + (q - hk);
        g = find_group([&](int k) { return glight[k]; }, G, p);
        mt = gtile[g + 1] - 1;
    } else {
        return false;
    }
    t.y = r % ny;
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
    const _Float16 *x0, *x1;  // assignment-row chunks (KB halves per step)
    const int8_t *w0, *w1;    // weight-row halves (KB bytes per step)
    const float *sw;          // this lane's weight-row scale, block-major ...
    int swstep;               // ... blocks swstep floats apart
    const float *sx;          // this lane's assignment-row scale (lanes < 32)
    int sxstep;
};

// This thread's four 16-byte pieces of a step: x rows 32 w + lane / 4 and
// 32 w + 16 + lane / 4 (the chunk that lands in slot lane % 4), weight rows
// 64 w + lane / 2 and 64 w + 32 + lane / 2 (the half that lands in slot
// lane % 2).
struct Pieces {
    int xr0, xc0, xr1, xc1, wr0, wh0, wr1, wh1;
};
__device__ __forceinline__ Pieces pieces() {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    Pieces p;
    p.xr0 = 32 * wave + (lane >> 2);
    p.xr1 = p.xr0 + 16;
    p.xc0 = xslot(p.xr0, lane & 3);  // slot ^ swizzle = the chunk stored there
    p.xc1 = xslot(p.xr1, lane & 3);
    p.wr0 = 64 * wave + (lane >> 1);
    p.wr1 = p.wr0 + 32;
    p.wh0 = wslot(p.wr0, lane & 1);
    p.wh1 = wslot(p.wr1, lane & 1);
    return p;
}

// The k loop over nk steps (nk >= NS - 1). On return acc[i][j][r] holds
//   C[64*wave + 16*i + 4*(lane/16) + r][16*j + lane%16]
// (weight row, assignment row) for the assignment tiles j < NJA (the tiles
// that hold rows of the bucket; the others are not computed): the exact
// block dots, each block term added with its two scales in block order.
// EXACT: the reference's three roundings, s = s + ((float)acc * d_w) * d_x
// (bit-equal row sums); otherwise the second product and the addition are
// one fused multiply-add (within a few ulps).
template <bool EXACT, int NJA>
__device__ __forceinline__ void gemm_tile(Step *ring, const Src &src, int nk, f4v acc[MI][NJ]) {
    static_assert(NJA >= 1 && NJA <= NJ, "assignment tiles");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int NLOAD = 6;  // global_load_lds per wavefront per step
    const unsigned ring0 = lds_addr(ring);
    const unsigned ox = (unsigned)offsetof(Step, x) + (2 * wave) * 1024;
    const unsigned ow = (unsigned)offsetof(Step, w) + (2 * wave) * 1024;
    const unsigned osw = (unsigned)offsetof(Step, sw) + wave * 256;
    const unsigned osx = (unsigned)offsetof(Step, sx) + wave * 128;
    auto issue = [&](int kb) {
        const int k = min(kb, nk - 1);  // past the end: reload the last step
        const unsigned st = ring0 + (unsigned)((kb % NS) * sizeof(Step));
        dma16(st + ox, src.x0 + (size_t)k * KB);
        dma16(st + ox + 1024, src.x1 + (size_t)k * KB);
        dma16(st + ow, src.w0 + (size_t)k * KB);
        dma16(st + ow + 1024, src.w1 + (size_t)k * KB);
        dma4(st + osw, src.sw + (size_t)k * src.swstep);
        if (lane < 32) dma4(st + osx, src.sx + (size_t)k * src.sxstep);
    };
#pragma unroll
    for (int s = 0; s < NS - 1; s++) issue(s);
    const int c = lane >> 4, l16 = lane & 15;
    for (int kb = 0; kb < nk; kb++) {
        // this wavefront's loads of step kb are done (NS - 2 later steps may
        // still be in flight); then every wavefront's are
        wait_vm<(NS - 2) * NLOAD>();
        __syncthreads();
        // step kb + NS - 1 reuses the slot read in step kb - 1, which every
        // wavefront has finished with (the LDS reads completed before the
        // barrier)
        issue(kb + NS - 1);
        const Step &S = ring[kb % NS];
        h8 av[MI];
        f4v s4[MI];
#pragma unroll
        for (int i = 0; i < MI; i++) {
            // weight row n, codes 8c .. 8c+7
            const int n = WN * wave + 16 * i + l16;
            const uint2 q = *(const uint2 *)&S.w[n][16 * wslot(n, c >> 1) + 8 * (c & 1)];
            av[i] = codes8(q.x, q.y);
            s4[i] = *(const f4v *)&S.sw[WN * wave + 16 * i + 4 * c];
        }
        // The block dots of assignment tile j + 1 are started before the
        // terms of tile j are added, so the vector ALUs never wait for the
        // product they consume.
        const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
        // x scales of this lane's assignment rows 16 j + l16, j < 8
        const f4v sxa = *(const f4v *)&S.sx[8 * l16], sxb = *(const f4v *)&S.sx[8 * l16 + 4];
        f4v blk[2][MI];
        {
            const h8 bv = *(const h8 *)&S.x[l16][8 * xslot(l16, c)];
#pragma unroll
            for (int i = 0; i < MI; i++)
                blk[0][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv, z, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < NJA; j++) {
            if (j + 1 < NJA) {
                const int m1 = 16 * (j + 1) + l16;
                const h8 bv = *(const h8 *)&S.x[m1][8 * xslot(m1, c)];
#pragma unroll
                for (int i = 0; i < MI; i++)
                    blk[(j + 1) & 1][i] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv, z, 0, 0, 0);
            }
            const float sx = j < 4 ? sxa[j & 3] : sxb[j & 3];
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float t = blk[j & 1][i][r] * s4[i][r];
                    if (EXACT)
                        acc[i][j][r] = acc[i][j][r] + t * sx;  // no contraction (-ffp-contract=off)
                    else
                        acc[i][j][r] = __builtin_fmaf(t, sx, acc[i][j][r]);
                }
        }
    }
    wait_vm<0>();  // the reloads past the end
    __syncthreads();
}

// The assignment tiles that hold rows of the bucket (a bucket's last tile
// may hold few rows).
template <bool EXACT>
__device__ __forceinline__ void gemm_tile_rows(Step *ring, const Src &src, int nk, int nrows,
                                               f4v acc[MI][NJ]) {
    // one instantiation per count of 16-row tiles, so a bucket's last tile
    // runs no empty tile (gate/up 468 -> 459 us at T = 4096, 157 -> 149 us
    // at T = 512, against rounding the count up to a power of two)
    switch ((nrows + 15) / 16) {
    case 8: gemm_tile<EXACT, 8>(ring, src, nk, acc); break;
    case 7: gemm_tile<EXACT, 7>(ring, src, nk, acc); break;
    case 6: gemm_tile<EXACT, 6>(ring, src, nk, acc); break;
    case 5: gemm_tile<EXACT, 5>(ring, src, nk, acc); break;
    case 4: gemm_tile<EXACT, 4>(ring, src, nk, acc); break;
    case 3: gemm_tile<EXACT, 3>(ring, src, nk, acc); break;
    case 2: gemm_tile<EXACT, 2>(ring, src, nk, acc); break;
    default: gemm_tile<EXACT, 1>(ring, src, nk, acc); break;
    }
}

// ---- x block scales in bucketed, block-major order --------------------------------
//
// xsb[k][p] = xs[t][k] for the assignment p = (t, j) in bucketed order, so a
// tile's 128 rows read their scales of block k as one contiguous run.
// Thread p copies blocks XB y .. XB y + XB - 1 of its token's row: four
// 16-byte reads of one row (rather than a 4-byte gather per block), then
// stores that are contiguous across the wavefront for each block.
constexpr int XB = 16;
__global__ __launch_bounds__(256) void k_xs_bucket(const float *__restrict__ xs,
                                                   const int *__restrict__ perm,
                                                   float *__restrict__ xsb, int A, int nb, int K) {
    const int p = blockIdx.x * 256 + threadIdx.x, k0 = blockIdx.y * XB;
    if (p >= A) return;
    const float *row = xs + (size_t)(perm[p] / K) * nb + k0;
    float *dst = xsb + (size_t)k0 * A + p;
    if (nb % 4 == 0 && k0 + XB <= nb) {
        float v[XB];
#pragma unroll
        for (int q = 0; q < XB / 4; q++) {
            const float4 f = *(const float4 *)(row + 4 * q);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
#pragma unroll
        for (int k = 0; k < XB; k++) dst[(size_t)k * A] = v[k];
    } else {
        for (int k = 0; k < XB && k0 + k < nb; k++) dst[(size_t)k * A] = row[k];
    }
}

union alignas(16) GateUpLds {
    Step ring[NS];
    float o[TM][OLD];  // epilogue: 128 assignment rows x 128 h columns
};
union alignas(16) DownLds {
    Step ring[NS];
    float o[TM][DLD];  // epilogue: 128 assignment rows x 64 down rows
};
static_assert(sizeof(GateUpLds) == NS * sizeof(Step) && sizeof(DownLds) == NS * sizeof(Step),
              "epilogue tiles fit the rings");
static_assert(2 * sizeof(DownLds) <= 160 * 1024, "two workgroups per CU");

// ---- gate/up + SwiGLU + Q8(h) ----------------------------------------------------
//
// blockIdx.x = tile of assignment rows (gtile numbering) x 6 column tiles of
// 128 consecutive h columns h0..h0+127. Wavefront w's 64 weight rows are the
// gate rows then the up rows of h columns h0+32w..h0+32w+31, so SwiGLU pairs
// its accumulator tiles i and i + 2 lane by lane.
__global__ __launch_bounds__(GT, 2) void k_gateup_mfma(
    const uint8_t *__restrict__ table, mhip_layout lay, const _Float16 *__restrict__ xq16,
    const float *__restrict__ xsb, const int *__restrict__ groups, const int *__restrict__ gtile,
    const int *__restrict__ glight, const int *__restrict__ perm, _Float16 *__restrict__ hq16,
    float *__restrict__ hsb, int d, int eh, int K, int A) {
    __shared__ GateUpLds L;
    __shared__ uint64_t etab[32];  // the expf table, for the SwiGLU lookups
    TileRef tr;
    if (!tile_of(groups, gtile, glight, eh / (TN / 2), tr)) return;
    if (threadIdx.x < 32) etab[threadIdx.x] = mia_expf_tab[threadIdx.x];  // read after the k loop's barriers
    const int base = tr.base, nrows = tr.nrows;
    const int h0 = tr.y * (TN / 2);
    const uint8_t *ex = table + (size_t)tr.e * lay.expert_bytes;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    Src src;
    {
        const Pieces p = pieces();
        const int t0 = perm[base + min(p.xr0, nrows - 1)] / K;
        const int t1 = perm[base + min(p.xr1, nrows - 1)] / K;
        src.x0 = xq16 + (size_t)t0 * d + p.xc0 * 8;
        src.x1 = xq16 + (size_t)t1 * d + p.xc1 * 8;
        // tile row n: wavefront n / 64; within it gate rows then up rows
        auto wrow = [&](int n, int half) {
            const int r = n % WN;
            const int hc = h0 + (n / WN) * (WN / 2) + r % (WN / 2);
            return (const int8_t *)(ex + (r < WN / 2 ? lay.gate_q : lay.up_q)) + (size_t)hc * d +
                   16 * half;
        };
        src.w0 = wrow(p.wr0, p.wh0);
        src.w1 = wrow(p.wr1, p.wh1);
        {
            // scale of tile row 64 wave + lane
            const int hc = h0 + wave * (WN / 2) + lane % (WN / 2);
            src.sw = (const float *)(ex + (lane < WN / 2 ? lay.gate_st : lay.up_st)) + hc;
            src.swstep = eh;
        }
        {
            // sx slot p = 32 wave + lane holds bucket row 16 (p % 8) + p / 8
            const int p = 32 * wave + (lane & 31);
            src.sx = xsb + base + min(16 * (p & 7) + (p >> 3), nrows - 1);
        }
        src.sxstep = A;
    }

    f4v acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    gemm_tile_rows<true>(L.ring, src, d / KB, nrows, acc);

    // SwiGLU into the h tile (LDS, reused): row = assignment, column = h - h0
    const int c = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int i = 0; i < MI / 2; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            f4v hv;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float gv = acc[i][j][r], uv = acc[i + 2][j][r];
                hv[r] = (gv / (1.0f + mia_expf_glibc_tab(-gv, etab))) * uv;
            }
            *(f4v *)&L.o[16 * j + l16][(WN / 2) * wave + 16 * i + 4 * c] = hv;
        }
    __syncthreads();
    {
        // Q8_0 of 32-blocks of h (quant.c:11-27): the codes as fp16 integers
        // (bucketed rows) and the scales block-major (hsb[block][row], the
        // down kernel's x scales); thread (m, b2) does blocks 2 b2 and
        // 2 b2 + 1 of row m
        const int m = tid >> 1, b2 = tid & 1;
        if (m < nrows) {
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
                const int blk = 2 * b2 + bb;
                const f4v *hs = (const f4v *)&L.o[m][32 * blk];
                float v[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const f4v q = hs[k];
                    v[4 * k] = q[0];
                    v[4 * k + 1] = q[1];
                    v[4 * k + 2] = q[2];
                    v[4 * k + 3] = q[3];
                }
                float amax = 0.0f;
#pragma unroll
                for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(v[k]));
                const float dsc = amax / 127.0f;
                const float qi = dsc != 0.0f ? 1.0f / dsc : 0.0f;
                h8 o[4];
#pragma unroll
                for (int k = 0; k < 32; k++) o[k >> 3][k & 7] = (_Float16)roundf(v[k] * qi);
                h8 *dst = (h8 *)(hq16 + (size_t)(base + m) * eh + h0 + 32 * blk);
#pragma unroll
                for (int k = 0; k < 4; k++) dst[k] = o[k];
                hsb[(size_t)(h0 / KB + blk) * A + base + m] = dsc;
            }
        }
    }
}

// ---- down -----------------------------------------------------------------------------
//
// blockIdx.x = tile of assignment rows x 8 column tiles of 256 consecutive
// down rows n0..n0+255. The x operand is the tile's Q8(h) (fp16 codes,
// bucketed order, contiguous) with its block-major scales. Results go out
// through LDS a wavefront's 64 columns at a time, so every assignment row is
// written as 256 contiguous bytes.
// EXACT: the reference's roundings of each block term (the expert outputs
// bit-equal); otherwise one fused multiply-add per term (a few ulps).
template <bool EXACT>
__global__ __launch_bounds__(GT, 2) void k_down_mfma(const uint8_t *__restrict__ table,
                                                     mhip_layout lay,
                                                     const _Float16 *__restrict__ hq16,
                                                     const float *__restrict__ hsb,
                                                     const int *__restrict__ groups,
                                                     const int *__restrict__ gtile,
                                                     const int *__restrict__ glight,
                                                     float *__restrict__ tmp, int d, int eh,
                                                     int A) {
    __shared__ DownLds L;
    TileRef tr;
    if (!tile_of(groups, gtile, glight, d / TN, tr)) return;
    const int base = tr.base, nrows = tr.nrows;
    const int n0 = tr.y * TN;
    const uint8_t *ex = table + (size_t)tr.e * lay.expert_bytes;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    Src src;
    {
        const Pieces p = pieces();
        src.x0 = hq16 + (size_t)(base + min(p.xr0, nrows - 1)) * eh + p.xc0 * 8;
        src.x1 = hq16 + (size_t)(base + min(p.xr1, nrows - 1)) * eh + p.xc1 * 8;
        const int8_t *dq = (const int8_t *)(ex + lay.down_q);
        src.w0 = dq + (size_t)(n0 + p.wr0) * eh + 16 * p.wh0;
        src.w1 = dq + (size_t)(n0 + p.wr1) * eh + 16 * p.wh1;
        src.sw = (const float *)(ex + lay.down_st) + n0 + WN * wave + lane;
        src.swstep = d;
        // sx slot p = 32 wave + lane holds bucket row 16 (p % 8) + p / 8
        const int ps = 32 * wave + (lane & 31);
        src.sx = hsb + base + min(16 * (ps & 7) + (ps >> 3), nrows - 1);
        src.sxstep = A;
    }

    f4v acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = (f4v){0.0f, 0.0f, 0.0f, 0.0f};
    gemm_tile_rows<EXACT>(L.ring, src, eh / KB, nrows, acc);

    const int c = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int qw = 0; qw < 4; qw++) {
        // wavefront qw's 64 columns, then every thread writes them out
        if (wave == qw) {
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    *(f4v *)&L.o[16 * j + l16][16 * i + 4 * c] = acc[i][j];
        }
        __syncthreads();
        // 128 rows x 16 float4: thread tid writes float4 tid % 16 of rows tid / 16 + 16 k
#pragma unroll
        for (int k = 0; k < TM / 16; k++) {
            const int m = tid / 16 + 16 * k, f = tid % 16;
            if (m < nrows)
                *(f4v *)(tmp + (size_t)(base + m) * d + n0 + WN * qw + 4 * f) =
                    *(const f4v *)&L.o[m][4 * f];
        }
        __syncthreads();
    }
}

}  // namespace

namespace mhip {

bool gemm_path_fits(const mhip_dims *s) {
    // whole tiles of weight rows, and enough k steps to fill the rings
    return s->dim % TN == 0 && s->expert_hidden % (TN / 2) == 0 && s->dim / KB >= NS - 1 &&
           s->expert_hidden / KB >= NS - 1;
}

int gemm_max_tiles(int A, int E) { return (A + TM - 1) / TM + (A < E ? A : E); }

// Workgroups for ny weight-row tiles: every XCD's heavy and light shares
// (ceil(H / 8) + ceil(L / 8) <= ceil((H + L) / 8) + 1 row tiles) fit.
static unsigned gemm_grid(int A, int E, int ny) {
    const int share = (gemm_max_tiles(A, E) + NXCD - 1) / NXCD + 1;
    return (unsigned)(NXCD * share * ny);
}

int launch_gateup_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                       const void *d_table_layer, const mhip_scratch *sc, int A) {
    const int d = s->dim, eh = s->expert_hidden;
    k_xs_bucket<<<dim3((A + 255) / 256, (d / KB + XB - 1) / XB), 256, 0, st>>>(
        sc->xs, sc->perm, sc->xsb, A, d / KB, s->n_active);
    const unsigned grid = gemm_grid(A, s->n_experts, eh / (TN / 2));
    k_gateup_mfma<<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                       (const _Float16 *)sc->xdq, sc->xsb, sc->groups,
                                       sc->gtile, sc->glight, sc->perm, (_Float16 *)sc->hdq,
                                       sc->hs, d, eh, s->n_active, A);
    return (int)hipGetLastError();
}

int launch_down_mfma(hipStream_t st, const mhip_dims *s, const mhip_layout *lay,
                     const void *d_table_layer, const mhip_scratch *sc, int A, bool exact) {
    const int d = s->dim, eh = s->expert_hidden;
    const unsigned grid = gemm_grid(A, s->n_experts, d / TN);
    if (exact)
        k_down_mfma<true><<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                               (const _Float16 *)sc->hdq, sc->hs, sc->groups,
                                               sc->gtile, sc->glight, sc->tmp, d, eh, A);
    else
        k_down_mfma<false><<<grid, GT, 0, st>>>((const uint8_t *)d_table_layer, *lay,
                                                (const _Float16 *)sc->hdq, sc->hs, sc->groups,
                                                sc->gtile, sc->glight, sc->tmp, d, eh, A);
    return (int)hipGetLastError();
}

}  // namespace mhip
