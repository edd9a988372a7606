// et_expert_gemm.hip -- the expert grouped GEMM over the routing CSR (gfx950):
//
//   C[s, n] = sum_k A[row(s), k] * W[e(s), n, k]     bf16 operands, binary32
//                                                     accumulation, bf16 out
//
// for every slot s below min(S, slot_capacity), where e(s) is the expert whose
// slot block [expert_offsets[e], expert_offsets[e + 1]) holds s, and
// row(s) = sorted_token[s] in gather mode (the dispatch is fused into the
// operand load: A is X [T, K] and Xp is never written) or row(s) = s (A is a
// slot-major buffer [cap, K]).  W [E, N, K] holds each expert's weight in
// nn.Linear layout (row n of expert e is output feature n).
//
// Tiling.  A block of 4 waves owns 256 slots x 256 output features of one
// expert; wave (wm, wn) owns 128 x 128 of it: 8 x 8 tiles of
// v_mfma_f32_16x16x32_bf16 (bf16), or 4 x 4 tiles of
// v_mfma_scale_f32_32x32x64_f8f6f4 (fp8).  The 16 x 16 bf16 form moves half
// the accumulator bytes per FLOP of v_mfma_f32_32x32x16_bf16 and draws less
// power: with the same fragment reads, a sustained MFMA loop on every CU ran
// 16% faster with it, and this kernel runs at a 13% higher clock (its time
// changed by -3.4% to +0.4%: the operand stream, not the clock, bounds it).
// K advances in chunks of 64 through two LDS stages
// filled by gfx950's direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds),
// with no staging registers.  A wave holds a whole chunk's MFMA fragments in
// registers, so a stage is free again as soon as every wave has read it, and
// two chunks stream in while one is multiplied.  One direct load fills 1 KiB
// of LDS, lane i's 16 bytes at 16 i; it is given 8 operand rows x 128
// contiguous bytes (a whole cache line per row: streaming through L2 into LDS
// runs ~45% faster this way than with 32 rows x 32 bytes per instruction, the
// MFMA fragment's own shape).  So a stage holds each operand row-major, 128
// bytes (64 k) per row, and the 16-byte segment s of row R sits at slot
// s ^ key(R), key(R) = (R & 7) ^ ((R >> 3) & 1): the fragment reads (bf16:
// lane l reads row l % 16, segment 4 * kstep + l / 16) then hit 16 distinct
// slots of every 256-byte bank window, with no bank conflicts.  The output
// goes straight from the accumulators to memory (16 bytes per lane after a
// lane-row swap), leaving the stages to the next tile.
//
// MFMA 16x16x32 bf16 operand layout (checked on the device): lane l holds A
// row l % 16 and B column l % 16 at k = 8 (l / 16) + i; C column l % 16,
// acc[r] at row 4 (l / 16) + r.  The product is issued as mfma(W fragment, X
// fragment) so that C's columns are slots and its rows output features: each
// lane then holds 4 consecutive features of one slot.
//
// Order of the sum.  Every output sums its k-steps (32 k for bf16, 64 for
// fp8) in ascending k, each k-step inside one MFMA; so results depend on K
// only, not on the tile, the expert or the mode, and the gather and
// slot-major modes give identical bits.
//
// Schedule.  The grid is persistent (a multiple of 8 blocks, at most one per
// CU).  Each block computes the per-expert tile prefix once, then walks its
// tiles.  The 8 XCDs take blocks in turn (block b runs on XCD b % 8), so XCD
// x is given the contiguous range of tiles [x * per, (x + 1) * per); inside an
// expert, tiles are ordered in groups of 4 or 8 slot tiles x every feature
// tile, so the ~32 blocks running together on one XCD share a few A tiles and
// W tiles through that XCD's L2 (the larger A is fetched again less often; an
// expert's W is re-read from the last-level cache).  A block's tiles form one stream of chunks: the last
// two chunks of a tile load the next tile's first two, so the ~6 us a tile
// otherwise spent filling its pipeline and storing its output overlaps the
// neighbouring tiles' loads and MFMAs.
#include <algorithm>
#include <type_traits>

#include "et_common.hpp"

namespace et {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_t;

// Word 3 of a gfx9 buffer descriptor for raw (untyped, stride 0) access.
constexpr int kBufDword3 = 0x00020000;
// A byte offset past every descriptor's num_records (all < 2^31): loads return
// 0 and stores are dropped.
constexpr uint32_t kOOR = 0x80000000u;
// s_waitcnt immediate of gfx9 for lgkmcnt(0) alone (vmcnt 63, expcnt 7: no wait)
constexpr int kWaitLgkm0 = 0xC07F;

constexpr int kBM = 256;          // slots per tile
constexpr int kBN = 256;          // output features per tile
constexpr int kThreads = 256;
// Slot tiles per group in the tile order: 8 for K >= 2048 (the gate/up
// projections: 2.5-3% faster than 4 at C3 and C4), 4 below (the down
// projection: 4.6% faster than 8 at C3), except 8 again when the experts with
// slots average kGroupMBigExperts slot tiles or more (the down projection at
// C4, 32 experts of 32 tiles: 2% faster with 8).  The order changes no bits.
constexpr int kGroupMLargeK = 8;
constexpr int kGroupMSmallK = 4;
constexpr int kGroupMBigExperts = 24;
constexpr int kHalf = 256 * 128;  // one operand's chunk: 256 rows x 128 bytes
constexpr int kStage = 2 * kHalf; // A then W; two stages fill 128 KiB of LDS
constexpr int kSmemBytes = 2 * kStage;

struct GemmArgs {
    const unsigned char* a;         // gather: X [a_rows, K]; else A [cap, K] (bf16, or fp8 e4m3)
    const int32_t* sorted_token;    // [cap] (gather only)
    const unsigned char* w;         // [E, N, K] (bf16, or fp8 e4m3)
    const int32_t* expert_offsets;  // [E + 1]
    uint16_t* c;                    // [cap, N] bf16
    const float* row_scale;         // [cap] (EPI_ROW_SCALE only)
    const float* a_scale;           // fp8: [a_rows], the scale of each row of a
    const float* w_scale;           // fp8: [E, N], the scale of each weight row
    int64_t a_rows;
    int64_t cap;
    int K, N, E;                    // N: rows of each expert's weight (2 F for SwiGLU)
};

// Epilogues: the plain product; the product times a per-slot factor; or SwiGLU,
// h = silu(g) * u of the gate rows g (weight rows 0..F-1) and the up rows u
// (rows F..2F-1) of the same hidden unit.
constexpr int EPI_PLAIN = ET_GEMM_PLAIN;
constexpr int EPI_ROW_SCALE = ET_GEMM_ROW_SCALE;
constexpr int EPI_SWIGLU = ET_GEMM_SWIGLU;

// One direct-to-LDS load: this lane's 16 bytes at byte offset voff + soff of
// the buffer land at LDS address lds + 16 * lane (soff and lds are
// wave-uniform; lds goes in M0).  Every offset this file passes keeps
// voff + soff inside the operand row that voff names, or marks voff out of
// range, so the access is in bounds whether or not the range check counts
// soff.
// Written as inline assembly so that the compiler does not treat the load as
// an LDS store: it would otherwise wait for every such load in flight before
// each LDS read (a full drain of the ring).  The s_nop covers the one wait
// state an LDS DMA needs after M0 is written.
__device__ __forceinline__ void dma_b128(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t soff, uint32_t lds)
{
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(res), "s"(soff), "{m0}"(lds)
                 : "memory");
}

// The same for 4 bytes per lane: lane i's dword lands at lds + 4 * lane.
__device__ __forceinline__ void dma_b32(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t lds)
{
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(res), "{m0}"(lds) : "memory");
}

// Output of one 32 x 32 accumulator tile row segment: lane l (kh = l / 32)
// holds features 8 r + 4 kh + 0..3 of its slot in P[r] (two bf16x2 words),
// r = 0..3.  v_permlane32_swap exchanges lanes 32..63 of its first operand
// with lanes 0..31 of its second (lane layout checked on the device): swapping
// P[2p] with P[2p + 1] leaves lane l with features 16 p + 8 kh + 0..7, which it
// stores as one 16-byte write at that column (range-checked offset).
__device__ __forceinline__ void store_row_segment(u32x2_t (&P)[4], __amdgpu_buffer_rsrc_t res, bool row_ok,
                                                  uint32_t row_base, int col0, int ncols, int kh)
{
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        u32x2_t& a = P[2 * p];
        u32x2_t& b = P[2 * p + 1];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const auto r = __builtin_amdgcn_permlane32_swap(a[w], b[w], false, false);
            a[w] = r[0];
            b[w] = r[1];
        }
        const int col = col0 + 16 * p + 8 * kh;
        const u32x4_t v = {a[0], a[1], b[0], b[1]};
        const uint32_t off = (row_ok && col < ncols) ? (row_base + (uint32_t)col) * 2u : kOOR;
        __builtin_amdgcn_raw_buffer_store_b128(v, res, off, 0, 0);
    }
}

// Output of two 16 x 16 accumulator tiles side by side (output columns col0
// ... col0 + 31 of one slot): lane l (16-lane row rho = l / 16) holds columns
// 4 rho + 0..3 of the first tile in v[0..3] and of the second in v[4..7].
// v_permlane16_swap exchanges the odd 16-lane rows of its first operand with
// the even rows of its second (lane layout checked on the device), after
// which lane l holds columns 16 (rho & 1) + 8 (rho >> 1) + 0..7, stored as one
// 16-byte write (range-checked offset; ncols is a multiple of 8).
__device__ __forceinline__ void store_pair16(const float (&v)[8], __amdgpu_buffer_rsrc_t res, bool row_ok,
                                             uint32_t row_base, int col0, int ncols, int rho)
{
    const auto lo = __builtin_amdgcn_permlane16_swap(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[4], v[5]), false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap(pack_bf16x2(v[2], v[3]), pack_bf16x2(v[6], v[7]), false, false);
    const u32x4_t out = {lo[0], hi[0], lo[1], hi[1]};
    const int col = col0 + 16 * (rho & 1) + 8 * (rho >> 1);
    const uint32_t off = (row_ok && col < ncols) ? (row_base + (uint32_t)col) * 2u : kOOR;
    __builtin_amdgcn_raw_buffer_store_b128(out, res, off, 0, 0);
}

// Wait until at most N of this wave's vector-memory operations are in flight,
// then meet the other waves.  The direct-to-LDS loads count in vmcnt and are
// in LDS once it has dropped, so after the barrier every wave's loads of the
// chunk are visible.  The memory clobber and the scheduling barriers keep the
// LDS reads after this point.
template <int N>
__device__ __forceinline__ void dma_wait_barrier()
{
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// FP8: operands in OCP fp8 e4m3 (one byte per element) on
// v_mfma_scale_f32_32x32x64_f8f6f4 with unit block scales, and the products
// scaled by a_scale[row] * w_scale[e, n] in the epilogue.  A chunk row is the
// same 128 bytes, so a chunk holds 128 k in two k-steps of 64; lane l's
// fragment is row l % 32, the 32 bytes at 32 (l / 32) of the k-step (two
// 16-byte segments).  The MFMA's sum over a k-step is the same for any
// permutation of k applied to both operands (checked on the device), so the
// fragment layouts of A and W only have to agree.
template <bool GATHER, int EPI, bool FP8 = false>
__global__ __launch_bounds__(kThreads) void expert_gemm_kernel(GemmArgs g)
{
    constexpr int ES = FP8 ? 1 : 2;           // bytes per element
    constexpr int KC = 128 / ES;              // k per chunk (one 128-byte row)
    constexpr int NKS = 2;                    // k-steps per chunk (32 k bf16, 64 k fp8)
    constexpr int TS = FP8 ? 32 : 16;         // MFMA tile side
    constexpr int TM = 128 / TS;              // MFMA tiles per wave and dimension
    // the two operand stages
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kSmemBytes];
    __shared__ int ptile[ET_MAX_EXPERTS + 1];    // prefix of the per-expert slot-tile counts
    __shared__ int nexp;                         // experts with at least one slot tile
    __shared__ int32_t tokbuf[2][kBM];           // gather: the tokens of a tile's slots, by tile parity
    // fp8: the weight-row scales of a tile's columns and the scales of its
    // rows of a, by tile parity (read as float4 in the epilogue)
    __shared__ __attribute__((aligned(16))) float wsbuf[2][kBN];
    __shared__ __attribute__((aligned(16))) float asbuf[2][kBM];

    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = g.E, K = g.K, N = g.N;

    if (wave == 0) {
        int carry = 0, busy = 0;
        for (int e0 = 0; e0 < E; e0 += kWave) {
            const int e = e0 + lane;
            int n = 0;
            if (e < E) {
                const int64_t lo = min<int64_t>(g.expert_offsets[e], g.cap);
                const int64_t hi = min<int64_t>(g.expert_offsets[e + 1], g.cap);
                n = (int)((max<int64_t>(0, hi - lo) + kBM - 1) / kBM);
            }
            const int inc = wave_incl_scan(n) + carry;
            if (e < E) ptile[e + 1] = inc;
            carry = __shfl(inc, kWave - 1, kWave);
            busy += (int)__popcll(__ballot(n > 0));
        }
        if (lane == 0) {
            ptile[0] = 0;
            nexp = busy;
        }
    }
    __syncthreads();

    // A SwiGLU tile covers 128 hidden units: 128 gate rows and their 128 up
    // rows of the weight (256 rows, as every tile).
    const int F = N / 2;
    const int nN = EPI == EPI_SWIGLU ? (F + kBN / 2 - 1) / (kBN / 2) : (N + kBN - 1) / kBN;
    const int Q = ptile[E] * nN;
    const int per = (Q + 7) / 8;
    const int group_m = (K >= 2048 || ptile[E] >= kGroupMBigExperts * nexp) ? kGroupMLargeK : kGroupMSmallK;
    const int nloc = (int)(gridDim.x / 8);
    const int xcd = (int)(blockIdx.x & 7);
    const int r32 = lane & 31;
    const int kh = lane >> 5;
    const int r16 = lane & 15;
    const int rho = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (K + KC - 1) / KC;

    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_t*)smem;

    // Tile context: the block's k-th tile is q = xcd * per + l, l = blockIdx / 8
    // + k * nloc.  Direct loads of a chunk: wave w fills row groups 8 w + i (i <
    // 8) of A and of W, rows R = 64 w + 8 i + lane / 8 of the tile; lane puts
    // segment seg = (lane % 8) ^ key(R) of its row at slot lane % 8, key(R) =
    // (lane / 8) ^ (i & 1).  Rows past the tile's slots repeat its last slot
    // (their outputs are not stored); features past N and invalid tokens read 0
    // (offset marked out of range).
    int segk[2];              // first k of this lane's segment, by i & 1
#pragma unroll
    for (int p = 0; p < 2; ++p) segk[p] = (((lane & 7) ^ (lane >> 3) ^ p)) * (16 / ES);
    struct Tile {
        bool valid;
        int64_t s0;           // first slot
        int rows;             // slots in the tile
        int n0;               // first output column
        int e;                // expert
        __amdgpu_buffer_rsrc_t ares, wres;
    };
    struct Offsets {
        uint32_t a[8];        // gather: per load row, the byte offset of the lane's segment
    };
    // First half of a tile's setup: which tile, its descriptors, and (gather)
    // a direct load of its slots' tokens into tokbuf[buf] (one dword per
    // lane; slots past the tile read 0 and are never used).  It counts among
    // the wave's vector-memory operations like the operand loads, so the
    // waits of the chunk stream cover it.  Second half: the load offsets,
    // from the tokens in LDS.  Split so that a prefetched tile's offsets are
    // only computed (and held in registers) once the current tile's own loads
    // are done.
    auto setup_a = [&](int l, Tile& t, int buf) {
        const int q = xcd * per + l;
        t.valid = l < per && q < Q;
        if (!t.valid) return;
        // the tile's expert: the last e with ptile[e] <= q / nN
        const int v = q / nN;
        int lo = 0, hi = E;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (ptile[mid] <= v) lo = mid;
            else hi = mid;
        }
        const int e = lo;
        const int mte = ptile[e + 1] - ptile[e];
        const int qq = q - ptile[e] * nN;
        const int grp = qq / (group_m * nN);
        const int gm = min(group_m, mte - grp * group_m);
        const int idx = qq - grp * group_m * nN;
        const int mt = grp * group_m + idx % gm;
        const int nt = idx / gm;
        t.s0 = (int64_t)g.expert_offsets[e] + (int64_t)mt * kBM;
        const int64_t rend = min<int64_t>(g.expert_offsets[e + 1], g.cap);
        t.rows = (int)min<int64_t>(kBM, rend - t.s0);
        t.n0 = nt * (EPI == EPI_SWIGLU ? kBN / 2 : kBN);
        t.e = e;
        t.ares = GATHER ? __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(g.a), (short)0,
                                                            (int)(g.a_rows * K * ES), kBufDword3)
                        : __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(g.a + t.s0 * K * ES),
                                                            (short)0, t.rows * K * ES, kBufDword3);
        t.wres = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(g.w + (int64_t)e * N * K * ES),
                                                   (short)0, N * K * ES, kBufDword3);
        if constexpr (GATHER) {
            const __amdgpu_buffer_rsrc_t tres = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<int32_t*>(g.sorted_token + t.s0), (short)0, t.rows * 4, kBufDword3);
            dma_b32(tres, (uint32_t)(64 * wave + lane) * 4u,
                    (uint32_t)(uintptr_t)(lds_t*)&tokbuf[buf][64 * wave]);
        }
    };
    // fp8: direct loads of a tile's scales into wsbuf[buf] and asbuf[buf],
    // one dword per lane: its 256 weight-row scales in output-column order
    // (SwiGLU: 128 gate rows, then their 128 up rows; columns past the weight
    // read 0) and the scales of its 256 rows of a (by token in gather mode;
    // the tokens must have landed in tokbuf[buf]; rows past the tile's slots
    // and invalid tokens read 0).  Issued only after a barrier that follows
    // the previous tile's epilogue, the last reader of these buffers.
    auto setup_scales = [&](const Tile& t, int buf) {
        if constexpr (FP8) {
            const int ent = 64 * wave + lane;
            int n;
            if constexpr (EPI == EPI_SWIGLU) {
                const int hid = t.n0 + (ent & 127);
                n = hid < F ? (ent < 128 ? hid : F + hid) : N;
            } else {
                n = t.n0 + ent;
            }
            const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(g.w_scale + (int64_t)t.e * N), (short)0, N * 4, kBufDword3);
            dma_b32(sres, n < N ? (uint32_t)n * 4u : kOOR, (uint32_t)(uintptr_t)(lds_t*)&wsbuf[buf][64 * wave]);
            uint32_t aoff;
            if constexpr (GATHER) {
                const uint32_t tok = (uint32_t)tokbuf[buf][ent];
                aoff = ent < t.rows && tok < (uint32_t)g.a_rows ? tok * 4u : kOOR;
            } else {
                aoff = ent < t.rows ? (uint32_t)ent * 4u : kOOR;
            }
            // (base and size read from lane 0: the compiler cannot otherwise
            // tell that they are uniform, and the load needs them in scalar
            // registers)
            const uint64_t ab = (uint64_t)(uintptr_t)(g.a_scale + (GATHER ? 0 : t.s0));
            const int alo = __builtin_amdgcn_readfirstlane((int)(uint32_t)ab);
            const int ahi = __builtin_amdgcn_readfirstlane((int)(uint32_t)(ab >> 32));
            const int abytes = __builtin_amdgcn_readfirstlane(GATHER ? (int)(g.a_rows * 4) : t.rows * 4);
            const __amdgpu_buffer_rsrc_t rres = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(uintptr_t)(((uint64_t)(uint32_t)ahi << 32) | (uint32_t)alo), (short)0, abytes, kBufDword3);
            dma_b32(rres, aoff, (uint32_t)(uintptr_t)(lds_t*)&asbuf[buf][64 * wave]);
        }
    };
    // z is 0; a laundered z (opaque to the compiler) makes it compute the
    // offsets again instead of keeping an earlier copy in registers.
    auto setup_b = [&](const Tile& t, Offsets& o, uint32_t z, int buf) {
        if constexpr (GATHER) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int R = 64 * wave + 8 * i + (lane >> 3);
                const uint32_t seg = (uint32_t)segk[i & 1] * ES + z;
                const uint32_t tok = (uint32_t)tokbuf[buf][min(R, t.rows - 1)];
                o.a[i] = tok < (uint32_t)g.a_rows ? tok * ((uint32_t)K * ES) + seg : kOOR;
            }
        }
    };
    // Byte offset of the lane's segment in load row i of A (slot-major) or W:
    // computed at each load from the tile's scalars (registers are scarce in
    // the K loop).
    // (gather mode keeps its 8 offsets in registers: reading the token from
    // LDS at each load would put an LDS wait before every load)
    auto a_off = [&](const Tile& t, const Offsets& o, int i, [[maybe_unused]] int tb) -> uint32_t {
        const int R = 64 * wave + 8 * i + (lane >> 3);
        if constexpr (GATHER) {
            return o.a[i];
        } else {
            return (uint32_t)min(R, t.rows - 1) * ((uint32_t)K * ES) + (uint32_t)segk[i & 1] * ES;
        }
    };
    auto b_off = [&](const Tile& t, int i) -> uint32_t {
        const int R = 64 * wave + 8 * i + (lane >> 3);
        const uint32_t seg = (uint32_t)segk[i & 1] * ES;
        if constexpr (EPI == EPI_SWIGLU) {
            // tile row R -> wave column half R / 128, MFMA tile tt of the
            // half (bf16: 16 rows, 0..3 gate, 4..7 up; fp8: 32 rows, 0, 1
            // gate, 2, 3 up), so a wave's gate and up accumulators of one
            // hidden unit sit in the same lane and register
            const int tt = (R & 127) / TS;
            const int hid = t.n0 + (R >> 7) * 64 + (tt % (TM / 2)) * TS + (R & (TS - 1));
            return hid < F ? (uint32_t)(tt >= TM / 2 ? F + hid : hid) * ((uint32_t)K * ES) + seg : kOOR;
        } else {
            const int n = t.n0 + R;
            return n < N ? (uint32_t)n * ((uint32_t)K * ES) + seg : kOOR;
        }
    };

    // The block's tiles form one stream of chunks: chunk c of a tile goes to
    // stage (c + par) & 1, and the next tile's parity follows on (par += nk).
    // One direct load of a tile's chunk c: q even -> A block q / 2, q odd -> W
    // block q / 2.  A chunk that runs past K masks the segments at or past K
    // (K is a multiple of 8, so a segment is all in or all out).
    auto dma_one = [&](const Tile& t, const Offsets& o, int tb, int c, int par, int q) {
        const int i = q >> 1;
        const uint32_t sb =
            lds0 + (uint32_t)((c + par) & 1) * kStage + (uint32_t)wave * 8192u + (uint32_t)i * 1024u;
        const uint32_t soff = (uint32_t)c * 128u;
        const uint32_t kmask = (c + 1) * KC <= K || c * KC + segk[i & 1] < K ? 0u : kOOR;
        if (q & 1) dma_b128(t.wres, b_off(t, i) | kmask, soff, sb + kHalf);
        else dma_b128(t.ares, a_off(t, o, i, tb) | kmask, soff, sb);
    };

    using Acc = std::conditional_t<FP8, f32x16_t, f32x4_t>;
    Acc acc[TM][TM];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = Acc{};

    // Fragment of tile t (TS rows), k-step ks: lane l reads row R = TS t +
    // l % TS, at 1024 (R / 8) + 128 (R % 8) + 16 (segment ^ key(R)),
    // key(R) = (l % 8) ^ ((l / 8) & 1) (TS is a multiple of 16); the segment
    // is 4 ks + l / 16 (bf16) or 4 ks + 2 (l / 32) + piece (fp8).  A 16-lane
    // group reads 16 rows or one row group pair at 16 distinct slots of a
    // 256-byte window: no bank conflicts.
    const int fkey = (lane & 7) ^ ((lane >> 3) & 1);
    const int flane = ((lane & (TS - 1)) >> 3) * 1024 + (lane & 7) * 128;
    const unsigned char* const abase = smem + wm * 16384 + flane;
    const unsigned char* const bbase = smem + kHalf + wn * 16384 + flane;
    // A whole chunk's fragments, [k-step][A, W][tile]: 16 bytes per lane
    // (bf16) or 32 (fp8, filled by two reads).
    using Frag = std::conditional_t<FP8, u32x8_t, u32x4_t>;
    Frag f[NKS][2][TM];
    // Read r of k-step ks of the chunk in stage st, r < RPK: fragment q = r
    // (bf16) or r / 2 (fp8, piece r % 2); q < TM: A tile q, else W tile q - TM.
    constexpr int RPK = 16;
    auto read_r = [&](int st, int ks, int r) {
        const int q = FP8 ? r >> 1 : r;
        const int sgi = FP8 ? 4 * ks + 2 * (lane >> 5) + (r & 1) : 4 * ks + (lane >> 4);
        const int off = st * kStage + ((sgi ^ fkey) << 4) + (q % TM) * (TS * 128);
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>((q < TM ? abase : bbase) + off);
        if constexpr (FP8) {
            Frag& fr = f[ks][q / TM][q % TM];
            const int h = 4 * (r & 1);
#pragma unroll
            for (int w = 0; w < 4; ++w) fr[h + w] = v[w];
        } else {
            f[ks][q / TM][q % TM] = v;
        }
    };
    // MFMA m of k-step ks: slot tile m / TM, feature tile m % TM
    auto mfma_one = [&](int ks, int m) {
        const int i = m / TM, j = m % TM;
        if constexpr (FP8) {
            // formats 0, 0: fp8 e4m3 both; block scales 127: 2^0
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                __builtin_bit_cast(i32x8_t, f[ks][1][j]), __builtin_bit_cast(i32x8_t, f[ks][0][i]), acc[i][j], 0, 0,
                0, 127, 0, 127);
        } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, f[ks][1][j]),
                                                                __builtin_bit_cast(bf16x8_t, f[ks][0][i]),
                                                                acc[i][j], 0, 0, 0);
        }
    };
    auto pin = [&]() { __builtin_amdgcn_sched_barrier(0); };
    auto barrier = [&]() {
        pin();
        asm volatile("s_barrier" ::: "memory");
        pin();
    };

    Tile cur, nxt;
    Offsets co, no;           // load offsets of the current and the next tile
    int l = (int)(blockIdx.x >> 3);
    int buf = 0;              // tokbuf of the current tile
    setup_a(l, cur, buf);
    if (!cur.valid) return;
    if (GATHER) dma_wait_barrier<0>();
    setup_b(cur, co, 0u, buf);
    setup_scales(cur, buf);   // (older than the chunk loads below: their wait covers it)
    int par = 0;              // stage of chunk c: (c + par) & 1
    // First tile: chunks 0 and 1 in flight, wait for chunk 0, read its first
    // k-step.  Later tiles find theirs prefetched (below).
    {
#pragma unroll
        for (int q = 0; q < 16; ++q) dma_one(cur, co, buf, 0, par, q);
        if (nk > 1) {
#pragma unroll
            for (int q = 0; q < 16; ++q) dma_one(cur, co, buf, 1, par, q);
            dma_wait_barrier<16>();
        } else {
            dma_wait_barrier<0>();
        }
#pragma unroll
        for (int r = 0; r < (NKS - 1) * RPK; ++r) read_r(par & 1, r / RPK, r % RPK);
    }
    // With two chunks or more per tile, the last two chunks of a tile load the
    // next tile's chunks 0 and 1, so a tile starts with its data in LDS and the
    // previous tile's stores overlap its loads.
    const bool stream = nk >= 2;
    // Step c (chunk c in stage (c + par) & 1, its first k-step already in
    // registers).  Each wave reads the chunk's last k-step, so once it has
    // waited for its reads and met the others, nobody reads that stage any
    // more: the stream's chunk two ahead is loaded into it (load(q), q < 16)
    // while the next MFMAs run.  Then every wave waits for the stream's next
    // chunk (the one after may stay in flight), meets the others, and reads
    // its first k-step under the last MFMAs -- within the tile; the next
    // tile's first fragments are read after the epilogue.  Every load and
    // fragment read sits between two MFMAs (the order is pinned): the matrix
    // pipe keeps a queued MFMA while they issue.
    auto step = [&](int c, auto load, bool more2, bool more1) {
        const int st = (c + par) & 1;
        const int st1 = st ^ 1;                    // the stream's next chunk
        const bool rd1 = c + 1 < nk;
        if constexpr (!FP8) {
            // 128 MFMAs (two k-steps of 64): k-step 1's 16 reads under the
            // first 32, the 16 loads under the next 64 (one per four), the
            // next chunk's k-step 0 under the last 32
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                mfma_one(0, m);
                pin();
                if (m & 1) read_r(st, 1, m >> 1);
                pin();
            }
            // (the builtin, not inline assembly: the compiler then knows these
            // reads are complete and adds no waits for them later)
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            barrier();
#pragma unroll
            for (int m = 32; m < 96; ++m) {
                mfma_one(m >> 6, m & 63);
                pin();
                if (more2 && (m & 3) == 3) load((m - 32) >> 2);
                pin();
            }
            if (more1) {
                if (more2) dma_wait_barrier<16>();
                else dma_wait_barrier<0>();
            }
#pragma unroll
            for (int m = 96; m < 128; ++m) {
                mfma_one(1, m & 63);
                pin();
                if (rd1 && (m & 1)) read_r(st1, 0, (m - 96) >> 1);
                pin();
            }
        } else {
            // Two k-steps of 16 MFMAs (each twice a 32x32x16 bf16 MFMA's time), in the
            // same proportions: the last k-step's 16 reads under the first 8
            // MFMAs, the loads under the next 16, the next chunk's k-step 0
            // under the last 8.
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                mfma_one(0, m);
                pin();
                read_r(st, 1, 2 * m);
                read_r(st, 1, 2 * m + 1);
                pin();
            }
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            barrier();
#pragma unroll
            for (int m = 8; m < 24; ++m) {
                mfma_one(m >> 4, m & 15);
                pin();
                if (more2) load(m - 8);
                pin();
            }
            if (more1) {
                if (more2) dma_wait_barrier<16>();
                else dma_wait_barrier<0>();
            }
#pragma unroll
            for (int m = 8; m < 16; ++m) {
                mfma_one(1, m);
                pin();
                if (rd1) {
                    read_r(st1, 0, 2 * (m - 8));
                    read_r(st1, 0, 2 * (m - 8) + 1);
                }
                pin();
            }
        }
    };

    for (;;) {
        l += nloc;
        setup_a(l, nxt, buf ^ 1);
        const bool more_tiles = nxt.valid && stream;
        // chunks whose stream successor two ahead is this tile's own
        const int nmain = nk - 2;
        for (int c = 0; c < nmain; ++c)
            step(c, [&](int q) { dma_one(cur, co, buf, c + 2, par, q); }, true, true);
        // the last two chunks: the stream's chunks two ahead are the next
        // tile's 0 and 1
        // (the next tile's tokens: its token load is older than the stream's
        // last 16 loads, so any chunk wait of the loop above covered it; with
        // no such wait, wait here)
        // (fp8: the next tile's scales, now that every wave has met the others
        // after the last epilogue -- in the loop above or just here -- and
        // before the next tile's chunk loads, whose waits cover them)
        if (more_tiles) {
            if ((GATHER || FP8) && nmain <= 0) dma_wait_barrier<0>();
            setup_b(nxt, no, 0u, buf ^ 1);
            setup_scales(nxt, buf ^ 1);
        }
        for (int c = max(nmain, 0); c < nk; ++c)
            step(c, [&](int q) { dma_one(nxt, no, buf ^ 1, c + 2 - nk, par + nk, q); }, more_tiles,
                 c + 1 < nk || more_tiles);

        // Epilogue straight from the accumulators.  bf16: lane l holds slot
        // (wm * 8 + i) * 16 + l % 16 and tile columns (wn * 8 + j) * 16 +
        // 4 (l / 16) + 0..3 in acc[i][j]; tiles j and j + 1 swap 16-lane rows
        // (store_pair16).  fp8: lane l holds slot (wm * 4 + i) * 32 + l % 32
        // and tile columns (wn * 4 + j) * 32 + 8 r + 4 (l / 32) + 0..3 in
        // acc[i][j][4 r ..]; pairs of lanes swap halves (store_row_segment).
        // Either way each lane stores 16 bytes through a range-checked
        // descriptor (rows past the tile's slots and columns past the output
        // get an out-of-range offset and are dropped).  The LDS stages keep
        // the next tile's chunks meanwhile.  The accumulators stay in the
        // accumulation registers up to here (the epilogues' arithmetic would
        // otherwise lead the register allocator to keep some in the vector
        // registers the K loop needs).
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) asm volatile("" : "+a"(acc[i][j]));
        // fp8: the scale of slot tile i's row of a, and the weight-row scales
        // of 4 consecutive output columns, from the tile's copies in LDS
        // (wsbuf entry = output column of the tile; SwiGLU: gate column, or
        // 128 + its up column)
        auto a_row_scale = [&](int i) -> float { return asbuf[buf][(wm * 4 + i) * 32 + r32]; };
        auto w_scales = [&](int col) -> float4 { return *reinterpret_cast<const float4*>(&wsbuf[buf][col]); };
        if constexpr (EPI == EPI_SWIGLU) {
            // h = (g * sigmoid(g)) * u in binary32, from the gate tiles j = 0, 1
            // and the up tiles j + 2 of the same lane and register; 128 hidden
            // columns per tile, wave column half wn holds hidden wn * 64 ...
            const __amdgpu_buffer_rsrc_t cres = __builtin_amdgcn_make_buffer_rsrc(
                g.c + cur.s0 * F, (short)0, cur.rows * F * 2, kBufDword3);
            if constexpr (FP8) {
                float sa[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) sa[i] = a_row_scale(i);
                // hidden tile outermost: its gate and up weight-row scales are
                // loaded once
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    __builtin_amdgcn_sched_barrier(0);
                    float4 wg[4], wu[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int col = wn * 64 + j * 32 + 8 * r + 4 * kh;
                        wg[r] = w_scales(col);
                        wu[r] = w_scales(128 + col);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = (wm * 4 + i) * 32 + r32;
                        u32x2_t P[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            __builtin_amdgcn_sched_barrier(0);   // one 4-value group at a time
                            float h[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const float gv = (acc[i][j][4 * r + e] * sa[i]) * wg[r][e];
                                const float uv = (acc[i][j + 2][4 * r + e] * sa[i]) * wu[r][e];
                                h[e] = (gv * sigmoid(gv)) * uv;
                            }
                            P[r] = u32x2_t{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
                        }
                        store_row_segment(P, cres, row < cur.rows, (uint32_t)row * (uint32_t)F,
                                          cur.n0 + wn * 64 + j * 32, F, kh);
                    }
                }
            } else {
            // gate tiles j = 0..3, up tiles j + 4; hidden wn * 64 + 16 j + ...
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                __builtin_amdgcn_sched_barrier(0);       // one slot tile at a time: few temporaries
                const int row = (wm * TM + i) * TS + r16;
#pragma unroll
                for (int j = 0; j < TM / 2; j += 2) {
                    __builtin_amdgcn_sched_barrier(0);   // one pair of tiles at a time
                    float h[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int jj = j + (e >> 2);
                        const float gv = acc[i][jj][e & 3];
                        h[e] = (gv * sigmoid(gv)) * acc[i][jj + TM / 2][e & 3];
                    }
                    store_pair16(h, cres, row < cur.rows, (uint32_t)row * (uint32_t)F, cur.n0 + wn * 64 + j * TS,
                                 F, rho);
                }
            }
            }
        } else {
            const __amdgpu_buffer_rsrc_t cres = __builtin_amdgcn_make_buffer_rsrc(
                g.c + cur.s0 * N, (short)0, cur.rows * N * 2, kBufDword3);
            // (the compiler barrier keeps the row-scale loads here rather than
            // hoisted above the K loop, where their registers would be live)
            asm volatile("" ::: "memory");
            float sc[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                sc[i] = 1.0f;
                if constexpr (EPI == EPI_ROW_SCALE) {
                    const int row = (wm * TM + i) * TS + (lane & (TS - 1));
                    sc[i] = g.row_scale[cur.s0 + min(row, cur.rows - 1)];
                }
                if constexpr (FP8) sc[i] = a_row_scale(i);
            }
            if constexpr (FP8) {
                // feature tile outermost: its 16 weight-row scales are loaded once
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    __builtin_amdgcn_sched_barrier(0);
                    float4 ws[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) ws[r] = w_scales((wn * 4 + j) * 32 + 8 * r + 4 * kh);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        __builtin_amdgcn_sched_barrier(0);   // one 32 x 32 tile at a time
                        const int row = (wm * 4 + i) * 32 + r32;
                        u32x2_t P[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            float v[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = (sc[i] * acc[i][j][4 * r + e]) * ws[r][e];
                            P[r] = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                        }
                        store_row_segment(P, cres, row < cur.rows, (uint32_t)row * (uint32_t)N,
                                          cur.n0 + (wn * 4 + j) * 32, N, kh);
                    }
                }
            } else {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if constexpr (EPI == EPI_ROW_SCALE) __builtin_amdgcn_sched_barrier(0);   // one slot tile at a time
                const int row = (wm * TM + i) * TS + r16;
#pragma unroll
                for (int j = 0; j < TM; j += 2) {
                    __builtin_amdgcn_sched_barrier(0);       // one pair of 16 x 16 tiles at a time
                    float v[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float a = acc[i][j + (e >> 2)][e & 3];
                        v[e] = EPI == EPI_ROW_SCALE ? sc[i] * a : a;
                    }
                    store_pair16(v, cres, row < cur.rows, (uint32_t)row * (uint32_t)N, cur.n0 + (wn * TM + j) * TS,
                                 N, rho);
                }
            }
            }
        }
        if (!nxt.valid) break;
        // (nothing below moves into the epilogue, where it would hold registers)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = Acc{};
        if (!stream) {
            // one chunk per tile: load it now (every wave has finished reading
            // the stage: its reads were consumed by its MFMAs, and the
            // barrier makes that hold for all waves)
            dma_wait_barrier<0>();
            setup_b(nxt, no, 0u, buf ^ 1);
            setup_scales(nxt, buf ^ 1);
#pragma unroll
            for (int q = 0; q < 16; ++q) dma_one(nxt, no, buf ^ 1, 0, par + nk, q);
            dma_wait_barrier<0>();
        }
        // the next tile's chunk 0 is in its stage for every wave (the last
        // step's wait and barrier, or the one just above): its first k-step
#pragma unroll
        for (int r = 0; r < (NKS - 1) * RPK; ++r) read_r((par + nk) & 1, r / RPK, r % RPK);
        par = (par + nk) & 1;
        cur = nxt;
        buf ^= 1;
        // the offsets again, from the tokens in LDS (nothing was kept in
        // registers across the epilogue)
        uint32_t z = 0u;
        asm volatile("" : "+v"(z));
        setup_b(cur, co, z, buf);
    }
}


// Compute units of the current device (the persistent grid's size), looked
// up once per device.
int num_cus()
{
    static int cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    int* slot = dev < 64 ? &cache[dev] : nullptr;
    if (slot && *slot > 0) return *slot;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    if (slot) *slot = n;
    return n;
}

}  // namespace
}  // namespace et

using namespace et;

namespace {

// Argument checks and launch of both entry points (es = bytes per operand
// element: 2 for bf16, 1 for fp8).
int launch_expert_gemm(const char* fn, int es, const void* a, int64_t a_rows, const float* a_scale,
                       const int32_t* sorted_token, const void* w, const float* w_scale,
                       const int32_t* expert_offsets, int64_t num_experts, int64_t K, int64_t N,
                       int64_t slot_capacity, int epilogue, const float* row_scale, void* c, void* stream)
{
    const int64_t E = num_experts;
    const bool fp8 = es == 1;
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    const int64_t kq = 16 / es;   // k per 16-byte segment
    if (K < kq || K % kq != 0 || K >= (int64_t(1) << 22))
        return fail(ET_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": K must be a positive multiple of " + std::to_string(kq) + " below 2^22");
    if (N < 8 || N % 8 != 0)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": N must be a positive multiple of 8");
    if (epilogue != ET_GEMM_PLAIN && epilogue != ET_GEMM_ROW_SCALE && epilogue != ET_GEMM_SWIGLU)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": unknown epilogue " + std::to_string(epilogue));
    if (fp8 && epilogue == ET_GEMM_ROW_SCALE)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": the fp8 GEMM has the plain and SwiGLU epilogues");
    if (epilogue == ET_GEMM_SWIGLU && N % 16 != 0)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": SwiGLU needs N = 2 F with F a multiple of 8");
    if (N * K * es >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": one expert's weight (N * K * element bytes) must be below 2 GiB");
    if (kBM * N * 2 >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": N too large");
    if (slot_capacity < 0 || slot_capacity >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": slot_capacity out of range");
    const bool gather = sorted_token != nullptr;
    if (gather && (a_rows < 0 || a_rows * K * es >= (int64_t(1) << 31)))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) +
                                                 ": in gather mode the token rows (a_rows * K * element bytes) must "
                                                 "be below 2 GiB");
    if (slot_capacity == 0) return ET_OK;
    if (!a || !w || !expert_offsets || !c) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null pointer");
    if (epilogue == ET_GEMM_ROW_SCALE && !row_scale)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": the row-scale epilogue needs row_scale");
    if ((reinterpret_cast<uintptr_t>(a) & 15) || (reinterpret_cast<uintptr_t>(w) & 15) ||
        (reinterpret_cast<uintptr_t>(c) & 15))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": a, w and c must be 16-byte aligned");
    if (fp8 && (!a_scale || !w_scale || (reinterpret_cast<uintptr_t>(w_scale) & 3) ||
                (reinterpret_cast<uintptr_t>(a_scale) & 3)))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": a_scale and w_scale (4-byte aligned) are required");
    const int64_t nN = epilogue == ET_GEMM_SWIGLU ? (N / 2 + kBN / 2 - 1) / (kBN / 2) : (N + kBN - 1) / kBN;
    const int64_t qmax = ((slot_capacity + kBM - 1) / kBM + E) * nN;
    if (qmax >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": too many output tiles (slot_capacity / 256 * N / 256)");
    const int64_t blocks = std::min<int64_t>((int64_t)num_cus(), qmax);
    const dim3 grid((unsigned)(8 * ((blocks + 7) / 8)));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const GemmArgs args{static_cast<const unsigned char*>(a), sorted_token, static_cast<const unsigned char*>(w),
                        expert_offsets, static_cast<uint16_t*>(c), row_scale, a_scale, w_scale, a_rows,
                        slot_capacity, (int)K, (int)N, (int)E};
    const dim3 block(kThreads);
    if (fp8) {
        switch ((epilogue == ET_GEMM_SWIGLU ? 2 : 0) + (gather ? 1 : 0)) {
            case 0: expert_gemm_kernel<false, EPI_PLAIN, true><<<grid, block, 0, s>>>(args); break;
            case 1: expert_gemm_kernel<true, EPI_PLAIN, true><<<grid, block, 0, s>>>(args); break;
            case 2: expert_gemm_kernel<false, EPI_SWIGLU, true><<<grid, block, 0, s>>>(args); break;
            default: expert_gemm_kernel<true, EPI_SWIGLU, true><<<grid, block, 0, s>>>(args); break;
        }
    } else {
        switch (epilogue * 2 + (gather ? 1 : 0)) {
            case 0: expert_gemm_kernel<false, EPI_PLAIN><<<grid, block, 0, s>>>(args); break;
            case 1: expert_gemm_kernel<true, EPI_PLAIN><<<grid, block, 0, s>>>(args); break;
            case 2: expert_gemm_kernel<false, EPI_ROW_SCALE><<<grid, block, 0, s>>>(args); break;
            case 3: expert_gemm_kernel<true, EPI_ROW_SCALE><<<grid, block, 0, s>>>(args); break;
            case 4: expert_gemm_kernel<false, EPI_SWIGLU><<<grid, block, 0, s>>>(args); break;
            default: expert_gemm_kernel<true, EPI_SWIGLU><<<grid, block, 0, s>>>(args); break;
        }
    }
    return check_launch("expert_gemm_kernel");
}

}  // namespace

extern "C" int et_expert_gemm(const void* a, int64_t a_rows, const int32_t* sorted_token, const void* w,
                              const int32_t* expert_offsets, int64_t num_experts, int64_t K, int64_t N,
                              int64_t slot_capacity, int epilogue, const float* row_scale, void* c, void* stream)
{
    return launch_expert_gemm("et_expert_gemm", 2, a, a_rows, nullptr, sorted_token, w, nullptr, expert_offsets,
                              num_experts, K, N, slot_capacity, epilogue, row_scale, c, stream);
}

extern "C" int et_expert_gemm_fp8(const void* a, int64_t a_rows, const float* a_scale, const int32_t* sorted_token,
                                  const void* w, const float* w_scale, const int32_t* expert_offsets,
                                  int64_t num_experts, int64_t K, int64_t N, int64_t slot_capacity, int epilogue,
                                  void* c, void* stream)
{
    return launch_expert_gemm("et_expert_gemm_fp8", 1, a, a_rows, a_scale, sorted_token, w, w_scale, expert_offsets,
                              num_experts, K, N, slot_capacity, epilogue, nullptr, c, stream);
}

// ---------------------------------------------------------------------------
// Weight transpose for the input gradient: wt[e, k, n] = w[e, n, k] for the
// experts with slots, so that dA = dC . W_e is a product against wt in the
// layout the grouped GEMM above reads (nn.Linear: rows are output features).
// ---------------------------------------------------------------------------

namespace et {
namespace {

constexpr int kTrTile = 64;

// Block (x, y) owns the 64 x 64 tile (k0 = 64 x, n0 = 64 y) of every expert
// z, z + gridDim.z, ...; experts without slots are skipped.  Rows are read and
// written 16 bytes per thread (N and K are multiples of 8); the tile passes
// through LDS with rows padded by 16 bytes.
__global__ __launch_bounds__(256) void weight_transpose_kernel(const uint16_t* __restrict__ w,
                                                                uint16_t* __restrict__ wt,
                                                                const int32_t* __restrict__ expert_offsets, int E,
                                                                int N, int K, int64_t cap)
{
    __shared__ __attribute__((aligned(16))) uint16_t tile[kTrTile][kTrTile + 8];
    const int tid = threadIdx.x;
    const int k0 = blockIdx.x * kTrTile, n0 = blockIdx.y * kTrTile;
    const int r = tid >> 3, c8 = (tid & 7) * 8;
    for (int e = blockIdx.z; e < E; e += gridDim.z) {
        const int64_t lo = min<int64_t>(expert_offsets[e], cap);
        const int64_t hi = min<int64_t>(expert_offsets[e + 1], cap);
        if (hi <= lo) continue;                       // block-uniform
        const uint16_t* src = w + (int64_t)e * N * K;
        uint16_t* dst = wt + (int64_t)e * N * K;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int n = n0 + r + 32 * p, k = k0 + c8;
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (n < N && k < K) v = *reinterpret_cast<const u32x4_t*>(src + (int64_t)n * K + k);
            *reinterpret_cast<u32x4_t*>(&tile[r + 32 * p][c8]) = v;
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int k = k0 + r + 32 * p, n = n0 + c8;
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q[i] = (uint32_t)tile[c8 + 2 * i][r + 32 * p] | ((uint32_t)tile[c8 + 2 * i + 1][r + 32 * p] << 16);
            if (k < K && n < N) *reinterpret_cast<u32x4_t*>(dst + (int64_t)k * N + n) = u32x4_t{q[0], q[1], q[2], q[3]};
        }
        __syncthreads();
    }
}

}  // namespace
}  // namespace et

extern "C" int et_expert_weight_transpose(const void* w, const int32_t* expert_offsets, int64_t num_experts,
                                          int64_t N, int64_t K, int64_t slot_capacity, void* wt, void* stream)
{
    const char* fn = "et_expert_weight_transpose";
    if (num_experts < 1 || num_experts > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (N < 8 || N % 8 != 0 || K < 8 || K % 8 != 0 || N * K >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": N and K must be positive multiples of 8, N*K < 2^31");
    if (slot_capacity < 0) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": slot_capacity < 0");
    if (!w || !expert_offsets || !wt) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(w) & 15) || (reinterpret_cast<uintptr_t>(wt) & 15))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": w and wt must be 16-byte aligned");
    if (w == wt) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": w and wt must not alias");
    const dim3 grid((unsigned)((K + kTrTile - 1) / kTrTile), (unsigned)((N + kTrTile - 1) / kTrTile),
                    (unsigned)std::min<int64_t>(num_experts, 16));
    weight_transpose_kernel<<<grid, dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t*>(w), static_cast<uint16_t*>(wt), expert_offsets, (int)num_experts, (int)N,
        (int)K, slot_capacity);
    return check_launch("weight_transpose_kernel");
}

// ---------------------------------------------------------------------------
// Weight gradient of the expert GEMM:
//   dw[e, n, k] = sum over e's slots s of dc[s, n] * a[s, k]      (f32 out)
// with dc [cap, N] and a [cap, K] slot-major bf16.  The sum runs over the
// slot (row) dimension of both operands, so neither loads as an MFMA fragment
// directly: a stage holds each operand's 64-slot chunk row-major (64 rows x
// 256 columns x 2 bytes), and the fragments -- 8 consecutive slots of one
// column per lane -- come from gfx950's transposing LDS read
// ds_read_b64_tr_b16.  Within each 16-lane group, if lane j points at 4
// consecutive 16-bit elements M[j][0..3], lane i receives M[4 m + i / 4][i % 4]
// for m = 0..3 (checked on the device).  So with lane j pointing at row
// r0 + j / 4, columns c0 + 4 (j % 4), lane i gets column c0 + i of rows
// r0..r0+3: two such reads give an MFMA operand of 8 consecutive slots.
// Each 512-byte row stores its 16-byte segment s at slot s ^ (4 (row & 3)),
// which puts the four rows of one read on distinct 64-byte bank windows.
// The product is issued as mfma(dc fragment, a fragment): lane l holds column
// k = l % 32 of a tile and rows n = 8 (r / 4) + 4 (l / 32) + r % 4, stored as
// 128-byte row pieces.
// ---------------------------------------------------------------------------

namespace et {
namespace {

struct WgradArgs {
    const uint16_t* dc;             // [cap, N]
    const uint16_t* a;              // [cap, K]
    const int32_t* expert_offsets;  // [E + 1]
    float* dw;                      // [E, N, K]
    int64_t cap;
    int K, N, E;
};

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

__device__ __forceinline__ uint2 read_tr16(const unsigned char* p)
{
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4_t*)(__attribute__((address_space(3))) unsigned char*)p);
    return __builtin_bit_cast(uint2, v);
}

__global__ __launch_bounds__(kThreads) void expert_wgrad_kernel(WgradArgs g)
{
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * kStage];
    __shared__ int ecnt[ET_MAX_EXPERTS];           // slots per expert
    __shared__ int order[ET_MAX_EXPERTS];          // experts by decreasing slot count

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int E = g.E, K = g.K, N = g.N;
    const int wm = wave >> 1, wn = wave & 1;
    const int nNt = (N + kBN - 1) / kBN, nKt = (K + kBN - 1) / kBN;
    const int tpe = nNt * nKt;                     // tiles per expert
    const int Q = E * tpe;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_t*)smem;

    // Work balance with locality.  A tile reduces over all of its expert's
    // slots, so tiles of heavily routed experts cost up to thousands of times
    // more than the others.  Experts are ordered by decreasing slot count
    // (ties by index) and the tiles dealt out round-robin in that order:
    // every block gets the same number of heavy tiles (within one), and the
    // blocks running together work on tiles of the same expert, which share
    // its operand rows through L2.
    for (int e = threadIdx.x; e < E; e += kThreads) {
        const int64_t lo = min<int64_t>(g.expert_offsets[e], g.cap);
        const int64_t hi = min<int64_t>(g.expert_offsets[e + 1], g.cap);
        ecnt[e] = (int)max<int64_t>(0, hi - lo);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kThreads) {
        const int ce = ecnt[e];
        int rank = 0;
        for (int f = 0; f < E; ++f) {
            const int cf = ecnt[f];
            rank += (cf > ce || (cf == ce && f < e)) ? 1 : 0;
        }
        order[rank] = e;
    }
    __syncthreads();

    // Direct loads of a chunk: wave w fills row pairs 8 w + i (i < 8) of each
    // operand, rows r = 16 w + 2 i + lane / 32, 16-byte slot q = lane % 32,
    // holding column segment q ^ (4 (r & 3)).
    // Fragment reads (tile t of 32 columns, k-step ks of 16 slots, half h):
    // lane l reads row 16 ks + 8 (l / 32) + 4 h + j / 4 (j = l % 16), columns
    // 32 t + 16 ((l / 16) % 2) + 4 (j % 4) .. + 3.  Per-lane LDS offset of
    // tile t's fragment at k-step 0, half 0; k-step ks and half h add
    // (16 ks + 4 h) * 512 bytes (the row & 3 of the swizzle is j / 4 for
    // every ks and h).
    const int jj = lane & 15;
    uint32_t fb[2][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int o = 0; o < 2; ++o) {
            const int tile = (o == 0 ? wm : wn) * 4 + t;
            const int seg = 4 * tile + 2 * ((lane >> 4) & 1) + ((jj & 3) >> 1);
            const int slot = seg ^ (4 * (jj >> 2));
            fb[o][t] = (uint32_t)((8 * (lane >> 5) + (jj >> 2)) * 512 + slot * 16 + (jj & 1) * 8 + o * kHalf);
        }
    }
    for (int q = blockIdx.x; q < Q; q += gridDim.x) {
        const int e = order[q / tpe];
        const int rem = q % tpe;
        const int n0 = (rem / nKt) * kBN, k0 = (rem % nKt) * kBN;
        const int64_t lo = min<int64_t>(g.expert_offsets[e], g.cap);
        const int64_t hi = min<int64_t>(g.expert_offsets[e + 1], g.cap);
        const int se = (int)max<int64_t>(0, hi - lo);
        const int nk = (se + 63) / 64;

        uint32_t doff[8], aoff[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 16 * wave + 2 * i + (lane >> 5);
            const int seg = (lane & 31) ^ (4 * (r & 3));
            const int n = n0 + 8 * seg, k = k0 + 8 * seg;
            doff[i] = n < N ? ((uint32_t)r * (uint32_t)N + (uint32_t)n) * 2u : kOOR;
            aoff[i] = k < K ? ((uint32_t)r * (uint32_t)K + (uint32_t)k) * 2u : kOOR;
        }
        // chunk c: slots lo + 64 c ..; descriptors rebased per chunk, so slots
        // past the expert's read 0.  Load q of a chunk: row pair q / 2, dc for
        // q even, a for q odd.
        auto dma_one = [&](int c, int q) {
            const int64_t s0 = lo + 64 * (int64_t)c;
            const int nrow = min(64, (int)(hi - s0));
            const uint32_t sb = lds0 + (uint32_t)(c & 1) * kStage + (uint32_t)wave * 8192u + (uint32_t)(q >> 1) * 1024u;
            if (q & 1) {
                const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint16_t*>(g.a + s0 * K), (short)0, nrow * K * 2, kBufDword3);
                dma_b128(ares, aoff[q >> 1], 0u, sb + kHalf);
            } else {
                const __amdgpu_buffer_rsrc_t dres = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint16_t*>(g.dc + s0 * N), (short)0, nrow * N * 2, kBufDword3);
                dma_b128(dres, doff[q >> 1], 0u, sb);
            }
        };
        auto issue = [&](int c) {
#pragma unroll
            for (int q = 0; q < 16; ++q) dma_one(c, q);
        };

        f32x16_t acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

        u32x4_t f[4][2][4];       // [k-step][dc, a][tile]
        // read r of k-step ks (r < 16): operand r / 8, tile (r / 2) % 4, half
        // r % 2 (rows 4 h .. 4 h + 3 of the lane's 8) -> that half of the
        // fragment
        auto read_one = [&](int c, int ks, int r) {
            const int o = r >> 3, t = (r >> 1) & 3, h = r & 1;
            const unsigned char* st = smem + (c & 1) * kStage + ks * 16 * 512;
            const uint2 v = read_tr16(st + fb[o][t] + h * 4 * 512);
            if (h == 0) {
                f[ks][o][t][0] = v.x;
                f[ks][o][t][1] = v.y;
            } else {
                f[ks][o][t][2] = v.x;
                f[ks][o][t][3] = v.y;
            }
        };
        // MFMA m of k-step ks: dc tile m / 4, a tile m % 4
        auto mfma_one = [&](int ks, int m) {
            const int i = m >> 2, j = m & 3;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f[ks][0][i]),
                                                                __builtin_bit_cast(bf16x8_t, f[ks][1][j]),
                                                                acc[i][j], 0, 0, 0);
        };
        auto pin = [&]() { __builtin_amdgcn_sched_barrier(0); };
        auto barrier = [&]() {
            pin();
            asm volatile("s_barrier" ::: "memory");
            pin();
        };

        // The forward kernel's schedule: a whole chunk's fragments in
        // registers, two chunks streaming while one is multiplied, and every
        // load and fragment read between two MFMAs (the order pinned).
        barrier();
        if (nk > 0) {
            issue(0);
            if (nk > 1) issue(1);
            if (nk > 1) dma_wait_barrier<16>();
            else dma_wait_barrier<0>();
#pragma unroll
            for (int r = 0; r < 48; ++r) read_one(0, r >> 4, r & 15);
        }
        for (int c = 0; c < nk; ++c) {
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                mfma_one(0, m);
                pin();
                read_one(c, 3, m);
                pin();
            }
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            barrier();
            const bool more2 = c + 2 < nk;
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                mfma_one(1 + (m >> 4), m & 15);
                pin();
                if (more2 && (m & 1)) dma_one(c + 2, m >> 1);
                pin();
            }
            const bool more1 = c + 1 < nk;
            if (more1) {
                if (more2) dma_wait_barrier<16>();
                else dma_wait_barrier<0>();
            }
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                mfma_one(3, m);
                pin();
                if (more1) {
#pragma unroll
                    for (int r = 3 * m; r < 3 * m + 3; ++r) read_one(c + 1, r >> 4, r & 15);   // 48 reads
                }
                pin();
            }
        }

        // Epilogue: f32 straight from the accumulators, 128-byte row pieces.
        const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
            g.dw + (int64_t)e * N * K, (short)0, N * K * 4, kBufDword3);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = k0 + (wn * 4 + j) * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = n0 + (wm * 4 + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const uint32_t off = (n < N && k < K) ? ((uint32_t)n * (uint32_t)K + (uint32_t)k) * 4u : kOOR;
                    __builtin_amdgcn_raw_buffer_store_b32(f2u(acc[i][j][r]), wres, off, 0, 0);
                }
            }
    }
}

}  // namespace
}  // namespace et

extern "C" int et_expert_wgrad(const void* dc, const void* a, const int32_t* expert_offsets, int64_t num_experts,
                               int64_t N, int64_t K, int64_t slot_capacity, float* dw, void* stream)
{
    const char* fn = "et_expert_wgrad";
    if (num_experts < 1 || num_experts > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (N < 8 || N % 8 != 0 || K < 8 || K % 8 != 0)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": N and K must be positive multiples of 8");
    if (N * K * 4 >= (int64_t(1) << 31) || 64 * std::max(N, K) * 2 >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": one expert's gradient (N * K * 4 bytes) must be below 2 GiB");
    if (slot_capacity < 0 || slot_capacity >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": slot_capacity out of range");
    if (!expert_offsets || !dw || (slot_capacity > 0 && (!dc || !a)))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(dc) & 15) || (reinterpret_cast<uintptr_t>(a) & 15) ||
        (reinterpret_cast<uintptr_t>(dw) & 3))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": dc and a must be 16-byte aligned, dw 4-byte aligned");
    const int64_t tiles = num_experts * ((N + kBN - 1) / kBN) * ((K + kBN - 1) / kBN);
    if (tiles >= (int64_t(1) << 31)) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": too many tiles");
    const dim3 grid((unsigned)std::min<int64_t>((int64_t)num_cus(), tiles));
    const WgradArgs args{static_cast<const uint16_t*>(dc), static_cast<const uint16_t*>(a), expert_offsets, dw,
                         slot_capacity, (int)K, (int)N, (int)num_experts};
    expert_wgrad_kernel<<<grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(args);
    return check_launch("expert_wgrad_kernel");
}
