// Paged GQA decode attention on the matrix cores: fp16, q8_0 and q4_0 pages.
//
// Same semantics as the vector-ALU kernel (pkg/engine/forward.go:242-267
// with the online softmax), arranged for CDNA4's 16x16x32 f16 MFMA:
//
//   S^T[token][head] = K[token][d] * Q^T[d][head]     (A = K rows straight
//                                                       from the page)
//   O[head][d]      += P[head][token] * V[token][d]    (B = V from the
//                                                       dimension-major page)
//
// A wave walks 32-token blocks as two 16-row MFMA tiles.  The query is split
// into hi + lo halves (q = hi + lo up to 2^-22 |q|) and the probabilities
// likewise, so both products keep float32 accuracy while K/V feed the MFMA in
// their stored fp16 form: no conversion instructions on the bandwidth path.
//
// Token order inside a block: tile 0 row i holds token 8*(i/4) + i%4, tile 1
// row i token 8*(i/4) + 4 + i%4.  The S tile then leaves lane (col j, group
// g = lane/16) with the scores of tokens 8g .. 8g+7 -- exactly the eight
// k-slots that lane feeds to the P*V product -- so P never moves between
// lanes, and the lane's V operand (dimension 16*nb + j, tokens 8g .. 8g+7) is
// one contiguous 16-byte run of the dimension-major page.
//
// Each of the NW waves of a workgroup (4, or 8 when the grid fills the CUs
// only once) keeps its own running max / sum; the workgroup merges them at the
// end, and split-K partials are merged by merge_splits.
//
// Quantised pages (q8_0, q4_0) stay exact.  Their integer codes are exact
// fp16 values (a byte or nibble permute into 0x64XX, then a bias), and one
// 32-wide k-step of S^T is exactly one quantisation block of K, so each
// k-step's partial scores are multiplied by their K block scale in float32.
// The V block scale varies along the P*V reduction (tokens), so it is folded
// into P: w = p * vscale / vnorm, where vnorm is a running power of two >=
// every V scale the wave has seen (the accumulators hold O / vnorm and are
// rescaled exactly when it grows).  w is
// split into hi + lo halves like p, the lo rows carrying a further 2^11 so
// they keep full precision; both factors are taken out in the final merge.
// Quantised blocks reach the registers through a per-wave LDS staging area
// filled by direct global->LDS loads.
#include "gi_common.h"
#include "gi_kernels.h"
#include "mfma_ops.h"
#include "token_store.h"

#include <math.h>
#include <type_traits>

namespace gi {

using mfma_ops::h2;
using mfma_ops::h8;
using mfma_ops::f4;
using mfma_ops::u2;
using mfma_ops::u4;
using mfma_ops::i8x8_sub_to_h8;
using mfma_ops::i8x8_to_h8;
using mfma_ops::u4x8_masked_to_h8;
using mfma_ops::u4x8_sub_to_h8;
using mfma_ops::split_pair;
typedef uint16_t us2 __attribute__((ext_vector_type(2)));

// Cache policy of the direct global->LDS loads (2: non-temporal, 0: the
// default).  A step reads each layer's pages once, so they load
// non-temporally wherever they stream: the staged K of fp16 pages (same box,
// batch 32 x U[512, 4096]: 0.0619 / 0.0637 against 0.0639 / 0.0657 ms per
// launch; batch 256 x 8192 unchanged), as the register loads of V do, and the
// f32 and quantised stages of four-wave launches (batch 64 x 8192 f32 pages
// 0.651 against 0.707 ms; batch 256 x 8192 q8_0 0.710 / 0.712 against
// 0.760 / 0.756 ms, q4_0 0.445 / 0.446 against 0.457 / 0.458 ms).  The
// eight-wave launches of f32 and quantised pages (one round of workgroups)
// keep the default policy: in the batch-1 case the pages of every layer fit
// the caches between steps, and non-temporal stages measured 25.4 against
// 23.0 ms per step there.
constexpr int kDecodeF16KAux = 2;
template <int NW>
constexpr int stage_aux() { return NW == 8 ? 0 : 2; }

namespace mfma_decode {

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <bool NT>
__device__ __forceinline__ h8 ld16(const uint8_t *p)
{
    if (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const h8 *>(p));
    return *reinterpret_cast<const h8 *>(p);
}

// Pages holding tokens base and base+16 of a 32-token block (equal when one
// page holds both or the second half is past the end), and the in-page slots
// of those two tokens.  Each 16-token half lies inside one page (pages hold a
// multiple of 16 tokens, blocks start at multiples of 32), so token t < 32 of
// the block sits in slot sA + t (t < 16) or sB + t - 16.  Everything here is
// wave-uniform: the table entries are read through the scalar cache (the
// tables are not written while a decode kernel runs), so fetching them never
// waits for the vector loads in flight.  Ids outside the pool are reported
// and replaced by page 0; their tokens are masked.
// (Plain scalars rather than a struct: a struct carried across the loop is
// not promoted to registers by the compiler.)
__device__ __forceinline__ void block_pages(const DecodeArgs &a, const int32_t *bt, int base, int t1,
                                            int64_t &pA, int64_t &pB, int &sA, int &sB, int &ok)
{
    typedef const __attribute__((address_space(4))) int32_t *const_i32;
    const PoolLayout &L = a.L;
    const int P = L.page_tokens;
    base = __builtin_amdgcn_readfirstlane(base);
    const int ia = base / P, ib = (base + 16) / P;
    sA = base - ia * P;
    sB = base + 16 - ib * P;
    const const_i32 cb = (const_i32)bt;
    const int32_t idA = cb[ia], idB = base + 16 < t1 ? cb[ib] : idA;
    pA = idA;
    pB = idB;
    // one unsigned 32-bit compare per id (negative ids wrap above any
    // limit; a pool of 2^31 pages or more holds every non-negative id)
    const uint32_t lim = (uint32_t)(L.num_pages < 0x80000000ll ? L.num_pages : 0x80000000ll);
    const bool okA = (uint32_t)idA < lim;
    const bool okB = (uint32_t)idB < lim;
    // bit 0: tokens 0-15 of the block are on a page of the pool, bit 1:
    // tokens 16-31; the tokens of a rejected page are skipped
    ok = (okA ? 1 : 0) | (okB ? 2 : 0);
    if (ok != 3) {
        if ((threadIdx.x & 63) == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_PAGE);
        if (!okA)
            pA = 0;
        if (!okB)
            pB = 0;
    }
}

// K rows: tile 0 row j is token 8*(j/4) + j%4 of the block, tile 1 adds 4.
template <int HD, bool NT>
__device__ __forceinline__ void load_k(const DecodeArgs &a, int64_t pA, int64_t pB, int sA, int sB,
                                       int64_t koff, int j, int g, h8 *k0, h8 *k1)
{
    const PoolLayout &L = a.L;
    const int tk0 = 8 * (j >> 2) + (j & 3), tk1 = tk0 + 4;
    const int64_t pk0 = tk0 < 16 ? pA : pB, pk1 = tk1 < 16 ? pA : pB;
    const int sk0 = (tk0 < 16 ? sA : sB) + (tk0 & 15), sk1 = (tk1 < 16 ? sA : sB) + (tk1 & 15);
    const uint8_t *r0 = a.base + pk0 * L.page_bytes + koff + sk0 * HD * 2;
    const uint8_t *r1 = a.base + pk1 * L.page_bytes + koff + sk1 * HD * 2;
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) {
        k0[kk] = ld16<NT>(r0 + (32 * kk + 8 * g) * 2);
        k1[kk] = ld16<NT>(r1 + (32 * kk + 8 * g) * 2);
    }
}

// V: tokens 8g .. 8g+7 of the block, dimension 16*nb + j.
template <int HD, bool NT>
__device__ __forceinline__ void load_v(const DecodeArgs &a, int64_t pA, int64_t pB, int sA, int sB,
                                       int64_t voff, int j, int g, h8 *v)
{
    const PoolLayout &L = a.L;
    const int P = L.page_tokens;
    const int64_t pv = g < 2 ? pA : pB;
    const int sv = (g < 2 ? sA : sB) + 8 * (g & 1);
    const uint8_t *vr = a.base + pv * L.page_bytes + voff + sv * 2;
#pragma unroll
    for (int nb = 0; nb < HD / 16; nb++)
        v[nb] = ld16<NT>(vr + (int64_t)(16 * nb + j) * P * 2);
}

// Running state of one wave for head column j.
template <int HD>
struct State {
    float m2;   // running max, log2 units
    float lsum; // this lane's share of the running denominator
    f4 o[HD / 16];
};

// Scores of one block: lane holds column j, block-local tokens 8g + r (s0[r])
// and 8g + 4 + r (s1[r]).  Unpacked (GP == 0): column j is head j and the
// hi and lo query halves are accumulated by two products.  Packed (GP = G):
// column j < G holds q_hi of head j and column 2G-1-j holds q_lo of head j,
// so one product covers both and a lane-mirror add (partner j ^ (2G-1))
// completes every score in both columns.
template <int GP>
__device__ __forceinline__ float mirror(float x)
{
    // DPP within 16-lane rows: quad_perm [1,0,3,2] (^1), quad_perm [3,2,1,0]
    // (^3), row_half_mirror (^7 within 8 lanes), row_mirror (^15).
    // Every lane reads a lane of its own row, so the bound control never
    // applies; written as an update of 0 the move folds into the add that
    // uses it (one v_add_f32_dpp).
    constexpr int ctrl = GP == 1 ? 0xB1 : GP == 2 ? 0x1B : GP == 4 ? 0x141 : 0x140;
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), ctrl,
                                                                  0xF, 0xF, true));
}

// Half i of a run of uint32 words, widened to float by the hardware
// conversion: exact for every finite half, subnormals included, since these
// kernels run with fp16 denormals preserved (the default float mode, which
// the code object's kernel descriptor records as float_denorm_mode_16_64 3).
// Block scales are never NaN.
__device__ __forceinline__ float half_at(const u4 *w, int i)
{
    const h8 v = __builtin_bit_cast(h8, w[i >> 3]);
    return (float)v[i & 7];
}

// Codes and scales of one 32-token block of a quantised page, as this lane
// feeds them to the products.
//   k0/k1[kk]: 8 codes of K tile 0/1 row j (token 8*(j/4) + j%4, + 4 for
//              tile 1), dimensions 32*kk + 8*g .. + 7;
//   ks:        K scales of tokens 8g .. 8g+7, half t*KK + kk;
//   v[..]:     8 codes of V, tokens 8g .. 8g+7: q8_0 dimension 16*nb + j for
//              tile nb; q4_0 the byte of dimensions 32*db + j (low nibble,
//              tile 2*db) and 32*db + 16 + j (high nibble, tile 2*db + 1);
//   vs[db]:    V scales of block db, tokens 8g .. 8g+7.
// SPLIT (four heads per kv head): the scores of a block leave the products
// with tokens 8g .. 8g+3 in lanes j < 8 and 8g+4 .. 8g+7 in lanes j >= 8, and
// each lane holds the scales of its own four tokens only: ks half t*KK + kk
// and vs[db] half t for its token t of four.
template <int KT, int HD, bool SPLIT = false>
struct QBlock {
    static constexpr int KK = HD / 32;
    typedef std::conditional_t<SPLIT, u2, u4> VS;
    u2 k0[KK], k1[KK];
    u4 ks[SPLIT ? KK / 2 : KK];
    u2 v[KT == KV_Q4_0 ? KK : 2 * KK];
    VS vs[KK];
};

// One wave's staging area for a block of a quantised page, filled by direct
// global->LDS loads (16 bytes per lane for codes, 4 for scales) and read back
// into the QBlock operand registers.  Reading pages through LDS lets every
// global load fetch long contiguous runs -- the K operand otherwise makes each
// quarter-wave touch 16 token rows per load -- and the next block's loads
// need no registers, so they are issued a whole block ahead.
//   k:  token rows in order, RB bytes each, as the pages hold them; the
//       16-byte piece p of token t sits at position p ^ m(t) of its row,
//       m(t) = (t >> 3) & 3 (q4_0) or 2 * ((t >> 3) & 3) (q8_0), cut to the
//       row's pieces (head_dim 64 has fewer), so that the
//       operand reads of the 16 token rows of a tile spread over the banks
//       while every quarter-wave of a load still fetches whole rows (4 rows
//       of q4_0, 2 of q8_0: two 128-byte lines);
//   v:  half h (tokens 16h .. 16h+15) in bytes [h, h + 1) * CODE_BYTES / 2,
//       code row c (q8_0: dimension c; q4_0: the byte row of dimensions
//       32(c/16) + c%16 and that + 16) at 16c, so that the operand reads
//       of 32 lanes (16 rows, both 8-byte parts) cover every bank once;
//   ks: [half][16 tokens][KK halves], 128 bytes per half;
//   vs: [half][db][16 tokens], 32 bytes per block row, 128 per half.
template <int KT, int HD>
struct QStage {
    static constexpr int KK = HD / 32;
    static constexpr int RB = KT == KV_Q4_0 ? HD / 2 : HD; // bytes of one token's codes
    static constexpr int CB = RB / KK, NS = CB / 16;
    static constexpr int CODE_BYTES = 32 * RB;              // of K (and of V) per block
    static constexpr int NLOAD = CODE_BYTES / 1024;         // 16-byte loads of 64 lanes
    uint8_t k[CODE_BYTES];
    uint8_t v[CODE_BYTES];
    uint8_t ks[256];
    uint8_t vs[256];
};

typedef __attribute__((address_space(3))) void *lds_ptr;

// Swizzle of the 16-byte pieces of K token row t in the staging area (NP
// pieces per row; a power of two).
template <int KT, int NP>
__device__ __forceinline__ int qk_swz(int t)
{
    return ((KT == KV_Q4_0 ? 1 : 2) * ((t >> 3) & 3)) & (NP - 1);
}

// K codes of a block into the staging area: slot sl (16 bytes, lane order)
// is piece (sl % NP) ^ swizzle of token row sl / NP.  With two or more loads
// each load reads rows of one page only, so its address is a wave-uniform
// base (page, slot, kv head) plus a per-lane offset that is the same for
// every block.
template <int KT, int HD, int AUX>
__device__ __forceinline__ void issue_qk(const DecodeArgs &a, int64_t pA, int64_t pB, int sA, int sB,
                                         int64_t koff, int lane, QStage<KT, HD> &S)
{
    typedef QStage<KT, HD> Q;
    constexpr int RB = Q::RB, NP = RB / 16, NL = Q::NLOAD;
    const PoolLayout &L = a.L;
    // token 0 of the block, token 16 of the block
    const uint8_t *gA = a.base + pA * L.page_bytes + koff + (int64_t)sA * RB;
    const uint8_t *gB = a.base + pB * L.page_bytes + koff + (int64_t)sB * RB;
#pragma unroll
    for (int q = 0; q < NL; q++) {
        const int sl = 64 * q + lane;
        const int tk = sl / NP, pc = (sl % NP) ^ qk_swz<KT, NP>(tk);
        const bool onB = NL >= 2 ? q >= NL / 2 : tk >= 16;
        const uint32_t off = (uint32_t)((tk - (onB ? 16 : 0)) * RB + 16 * pc);
        const uint8_t *src = (onB ? gB : gA) + off;
        __builtin_amdgcn_global_load_lds(src, (lds_ptr)&S.k[1024 * q], 16, 0, AUX);
    }
}

// Both scale planes, then the V codes of a block, into the staging area (in
// this order: a wait for all but the last NLOAD loads covers the scales).
// V: half h of the block (tokens 16h .. 16h+15, one page) fills bytes
// [h * CODE_BYTES / 2, (h + 1) * CODE_BYTES / 2), code row r at 16 r; with two
// or more loads each load reads one half, so its address is a wave-uniform
// base plus a per-lane offset.
template <int KT, int HD, int AUX>
__device__ __forceinline__ void issue_qv(const DecodeArgs &a, int64_t pA, int64_t pB, int sA, int sB,
                                         int64_t ksoff, int64_t voff, int64_t vsoff, int lane,
                                         QStage<KT, HD> &S)
{
    typedef QStage<KT, HD> Q;
    constexpr int KK = Q::KK, NL = Q::NLOAD;
    const PoolLayout &L = a.L;
    const int P = L.page_tokens;
    const uint8_t *gA = a.base + pA * L.page_bytes, *gB = a.base + pB * L.page_bytes;
    // Both scale planes in one 16-byte load of 32 lanes: lane c < 16 fills
    // ks bytes 16c .. 16c+15, lane 16 + c fills vs bytes 16c .. 16c+15.  The
    // texture unit spends about as long on a load of 4-byte lanes as on one
    // of 16-byte lanes, so one wide load replaces two narrow ones.  (Some
    // lane of the first 16 always takes part, so the wave always issues it.)
    {
        const int c = lane & 15, h = c >> 3;
        const uint8_t *pg = h ? gB : gA;
        const int slot = h ? sB : sA;
        // K: 16 tokens x KK halves = 32*KK bytes per half; V: block db of a
        // half is 16 tokens = 32 bytes, two lanes.  Offsets inside a page
        // fit 32 bits.
        const int o = 16 * (c & 7), db = (c >> 1) & 3, part = c & 1;
        const uint32_t koffs = (uint32_t)ksoff + (uint32_t)(slot * KK * 2 + o);
        const uint32_t voffs = (uint32_t)vsoff + (uint32_t)((db * P + slot + 8 * part) * 2);
        const uint8_t *src = pg + (lane < 16 ? koffs : voffs);
        const bool use = lane < 16 ? o < 32 * KK : db < KK;
        if (lane < 32 && use)
            __builtin_amdgcn_global_load_lds(src, (lds_ptr)&S.ks[0], 16, 0, AUX);
    }
    const uint8_t *vA = gA + voff + sA, *vB = gB + voff + sB;
#pragma unroll
    for (int q = 0; q < NL; q++) {
        // half h, code row r of it
        const bool h = NL >= 2 ? q >= NL / 2 : lane >= 32;
        const int r = NL >= 2 ? 64 * (q % (NL / 2)) + lane : (lane & 31);
        const uint8_t *src = (h ? vB : vA) + (uint32_t)(r * P);
        __builtin_amdgcn_global_load_lds(src, (lds_ptr)&S.v[1024 * q], 16, 0, AUX);
    }
}

// s_waitcnt immediate for vmcnt(n), the other counters left alone.
constexpr int vmcnt_imm(int n)
{
    return 0x0F70 | (n & 15) | ((n >> 4) << 14);
}

// K codes and K scales of the staged block into operand registers.
template <int KT, int HD, bool SPLIT>
__device__ __forceinline__ void read_qk(const QStage<KT, HD> &S, int j, int g, QBlock<KT, HD, SPLIT> &B)
{
    typedef QStage<KT, HD> Q;
    constexpr int KK = Q::KK, RB = Q::RB;
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            // token row of tile t, lane j; the 8 codes of k-step kk for lane
            // group g: q4_0 piece kk (g >= 2 take its high nibbles), q8_0
            // piece 2kk + g/2
            const int tk = 8 * (j >> 2) + (j & 3) + 4 * t;
            const int pc = KT == KV_Q4_0 ? kk : 2 * kk + (g >> 1);
            const int off = tk * RB + 16 * (pc ^ qk_swz<KT, RB / 16>(tk)) + 8 * (g & 1);
            const u2 c = *reinterpret_cast<const u2 *>(&S.k[off]);
            if (t)
                B.k1[kk] = c;
            else
                B.k0[kk] = c;
        }
    // 2*KK bytes per token; SPLIT: lanes j >= 8 start 4 tokens on
    const int ko = 128 * (g >> 1) + 16 * KK * (g & 1) + (SPLIT && j >= 8 ? 8 * KK : 0);
#pragma unroll
    for (int i = 0; i < (SPLIT ? KK / 2 : KK); i++)
        B.ks[i] = *reinterpret_cast<const u4 *>(&S.ks[ko + 16 * i]);
}

// V codes and V scales of the staged block into operand registers.
template <int KT, int HD, bool SPLIT>
__device__ __forceinline__ void read_qv(const QStage<KT, HD> &S, int j, int g, QBlock<KT, HD, SPLIT> &B)
{
    constexpr int KK = QStage<KT, HD>::KK, HB = QStage<KT, HD>::CODE_BYTES / 2;
#pragma unroll
    for (int r = 0; r < (KT == KV_Q4_0 ? KK : 2 * KK); r++)
        B.v[r] = *reinterpret_cast<const u2 *>(&S.v[HB * (g >> 1) + 16 * (r * 16 + j) + 8 * (g & 1)]);
    typedef typename QBlock<KT, HD, SPLIT>::VS VS;
    const int vo = 128 * (g >> 1) + 16 * (g & 1) + (SPLIT && j >= 8 ? 8 : 0);
#pragma unroll
    for (int db = 0; db < KK; db++)
        B.vs[db] = *reinterpret_cast<const VS *>(&S.vs[vo + 32 * db]);
}

// One wave's staging area for a block of an f32 page, filled by 16-byte
// direct global->LDS loads.  With x(j) = (j >> 1) & 7:
//   k: slot ((kk*2 + t)*16 + j)*8 + (c ^ x(j)) holds token row tk_t(j),
//      dimensions 32*kk + 4*c .. + 3;
//   v: slot (nb*16 + j)*8 + (c ^ x(j)) holds dimension 16*nb + j, block
//      tokens 4*c .. 4*c + 3.
// A quarter-wave of a load fetches two whole 128-byte K rows (V: two
// dimensions' 64-byte runs of both pages), and the swizzle spreads the
// 16-byte operand reads of 16 lanes over all banks.
template <int HD>
struct F32Stage {
    static constexpr int BYTES = 32 * HD * 4, NLOAD = BYTES / 1024;
    uint8_t k[BYTES];
    uint8_t v[BYTES];
};

// Per-lane parts of the f32 staging addresses, fixed for the kernel.  Load q
// of K reads page (q & 1) only (rows of tokens 16 (q & 1) ..); each V lane
// keeps to one page per parity of q.  So a load is a per-block base, the
// lane's offset and a constant.
struct F32Lanes {
    uint32_t k[2], v[2]; // byte offsets for even / odd loads
    bool vb[2];          // V lane on page B
};

template <int HD>
__device__ __forceinline__ F32Lanes f32_lanes(int lane, int P)
{
    F32Lanes n;
    const int jl = lane >> 3;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int c = (lane & 7) ^ ((4 * p + (lane >> 4)) & 7);
        n.k[p] = (uint32_t)((8 * (jl >> 2) + (jl & 3)) * HD * 4 + 16 * c);
        n.v[p] = (uint32_t)(16 * c + jl * P * 4);
        n.vb[p] = c >= 4;
    }
    return n;
}

template <int HD, int AUX>
__device__ __forceinline__ void issue_f32(const DecodeArgs &a, int64_t pA, int64_t pB, int sA, int sB,
                                          int64_t koff, int64_t voff, const F32Lanes &ln, F32Stage<HD> &S)
{
    const PoolLayout &L = a.L;
    const int P = L.page_tokens;
    const uint8_t *gA = a.base + pA * L.page_bytes, *gB = a.base + pB * L.page_bytes;
    // K: slot 64q + lane holds token row 16 (q & 1) + 8 (jl >> 2) + (jl & 3)
    // + 4 ((q >> 1) & 1), dimensions 32 (q >> 2) + 4c .. + 3
    const uint8_t *kA = gA + (int64_t)sA * HD * 4 + koff, *kB = gB + (int64_t)sB * HD * 4 + koff;
#pragma unroll
    for (int q = 0; q < F32Stage<HD>::NLOAD; q++) {
        const int p = q & 1;
        const uint8_t *src = (p ? kB : kA) + ln.k[p] + (4 * ((q >> 1) & 1) * HD * 4 + 128 * (q >> 2));
        __builtin_amdgcn_global_load_lds(src, (lds_ptr)&S.k[1024 * q], 16, 0, AUX);
    }
    // V: slot 64q + lane holds dimension 16 (q >> 1) + 8 (q & 1) + jl, block
    // tokens 4c .. 4c + 3 (page A for c < 4)
    const uint8_t *vA = gA + voff + (int64_t)sA * 4, *vB = gB + voff + (int64_t)(sB - 16) * 4;
    const uint8_t *vbase[2] = {ln.vb[0] ? vB : vA, ln.vb[1] ? vB : vA};
#pragma unroll
    for (int q = 0; q < F32Stage<HD>::NLOAD; q++) {
        const int p = q & 1;
        const uint8_t *src = vbase[p] + ln.v[p] + (int64_t)(16 * (q >> 1) + 8 * p) * P * 4;
        __builtin_amdgcn_global_load_lds(src, (lds_ptr)&S.v[1024 * q], 16, 0, AUX);
    }
}

// fp16 K staged through LDS (one-round grids, head_dim 128).  Loaded
// straight into operand registers, a K load touches 16 token rows, 64 bytes
// of each, and one workgroup streams about 31 GB/s however many blocks it
// keeps in flight; a probe of the same pages streams 35 GB/s with that
// shape and 60 GB/s when each K load reads 1 KiB in one run (V's register
// loads, 16 dimensions' rows on each page, are already such runs).  The
// longest sequences of a ragged one-round batch stream at that rate, so
// there K goes through LDS: every direct global->LDS load reads four whole
// 256-byte token rows, and the operands read back are the bytes the
// register loads would hold.  With sw(r) = ((r >> 1) & 12) | (r & 3), the
// 16-byte slot 16r + (c ^ sw(r)) holds block token r, bytes 16c .. of its
// row, so that the operand reads of 16 lanes fall on all 64 banks.
struct F16KStage {
    static constexpr int BYTES = 32 * 128 * 2, NLOAD = BYTES / 1024;
    uint8_t k[BYTES];
};

__device__ __forceinline__ int f16_kswz(int r) { return ((r >> 1) & 12) | (r & 3); }

__device__ __forceinline__ void issue_k_f16(const DecodeArgs &a, int64_t pA, int64_t pB, int sA, int sB,
                                            int64_t koff, int lane, F16KStage &S)
{
    const PoolLayout &L = a.L;
    const uint8_t *gA = a.base + pA * L.page_bytes + koff, *gB = a.base + pB * L.page_bytes + koff;
    // load q reads block rows 4q .. 4q + 3 (tokens 0-15 on page A)
#pragma unroll
    for (int q = 0; q < F16KStage::NLOAD; q++) {
        const int r = 4 * q + (lane >> 4);
        const uint8_t *row = q < 4 ? gA + (int64_t)(sA + r) * 256 : gB + (int64_t)(sB + r - 16) * 256;
        __builtin_amdgcn_global_load_lds(row + 16 * ((lane & 15) ^ f16_kswz(r)), (lds_ptr)&S.k[1024 * q], 16, 0,
                                         kDecodeF16KAux);
    }
}

// The operands load_k would hold, from the stage.
__device__ __forceinline__ void read_k_f16(const F16KStage &S, int j, int g, h8 *k0, h8 *k1)
{
    const int tk0 = 8 * (j >> 2) + (j & 3), tk1 = tk0 + 4;
    const int x0 = f16_kswz(tk0), x1 = f16_kswz(tk1);
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
        k0[kk] = *reinterpret_cast<const h8 *>(&S.k[(16 * tk0 + ((4 * kk + g) ^ x0)) * 16]);
        k1[kk] = *reinterpret_cast<const h8 *>(&S.k[(16 * tk1 + ((4 * kk + g) ^ x1)) * 16]);
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x)
{
    // (an update of 0 with in-row patterns: folds into the instruction using it)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Maximum of a non-negative value over the wave, wave-uniform: DPP within
// each 16-lane row, then the four row results (non-negative floats order
// like their bit patterns).
__device__ __forceinline__ float wave_max_nonneg(float x)
{
    x = fmaxf(x, dpp_f<0xB1>(x));  // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_f<0x4E>(x));  // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_f<0x141>(x)); // row_half_mirror
    x = fmaxf(x, dpp_f<0x140>(x)); // row_mirror
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const uint32_t m = max(max(__builtin_amdgcn_readlane(b, 0), __builtin_amdgcn_readlane(b, 16)),
                           max(__builtin_amdgcn_readlane(b, 32), __builtin_amdgcn_readlane(b, 48)));
    return __builtin_bit_cast(float, m);
}

// Power-of-two operand scale of one block with largest magnitude m: the
// running scale `run` is kept while m*run lies in [2^-2, 2^15) (fp16 hi
// halves below 65504, lo halves normal down to 2^-22 of the maximum);
// otherwise the scale puts m in [2^14, 2^15).  The first block (run == 0)
// keeps 1 when it may, so that ordinary data needs no multiply.
__device__ __forceinline__ float block_scale(float m, float run)
{
    const float r = run == 0.0f ? 1.0f : run;
    const float ms = m * r;
    if (m == 0.0f || (ms >= 0.25f && ms < 32768.0f))
        return r;
    int k = 14 - ((int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xFF) - 127);
    k = min(max(k, -126), 127);
    return __builtin_bit_cast(float, (uint32_t)(k + 127) << 23);
}

// 1 / x for a power of two x in [2^-126, 2^126]: exact exponent arithmetic.
__device__ __forceinline__ float pow2_recip(float x)
{
    return __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, x));
}

// Reads one f32 block from the staging area and turns it into hi/lo fp16
// operands.  Tokens past t1 (or the whole block on a rejected page) are
// zeroed first, so that stale slots take no part in the scales.  K is scaled
// by ksc and V by vsc (running powers of two, updated here); when vsc changes
// the accumulators are rescaled to the new one.
template <int HD>
__device__ __forceinline__ void read_f32(const F32Stage<HD> &Sf, int j, int g, int base, int ok, int t1,
                                         h8 *kh0, h8 *kh1, h8 *kl0, h8 *kl1, h8 *vh, h8 *vl, float &ksc,
                                         float &vsc, State<HD> &S, float neg1)
{
    constexpr int KK = HD / 32, NB = HD / 16;
    const int x = (j >> 1) & 7;
    float kf[2][KK][8], vf[NB][8];
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float4 w = *reinterpret_cast<const float4 *>(
                    &Sf.k[((((kk * 2 + t) * 16 + j) * 8) + ((2 * g + h) ^ x)) * 16]);
                kf[t][kk][4 * h] = w.x;
                kf[t][kk][4 * h + 1] = w.y;
                kf[t][kk][4 * h + 2] = w.z;
                kf[t][kk][4 * h + 3] = w.w;
            }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 w =
                *reinterpret_cast<const float4 *>(&Sf.v[(((nb * 16 + j) * 8) + ((2 * g + h) ^ x)) * 16]);
            vf[nb][4 * h] = w.x;
            vf[nb][4 * h + 1] = w.y;
            vf[nb][4 * h + 2] = w.z;
            vf[nb][4 * h + 3] = w.w;
        }
    if (base + 32 > t1 || ok != 3) {
        const int tk0 = 8 * (j >> 2) + (j & 3);
        const bool okk = (ok >> (j >> 3)) & 1; // K rows: tokens 16-31 in lanes j >= 8
        const bool okv = (ok >> (g >> 1)) & 1; // V rows: tokens 8g .. 8g+7
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const bool live = okk && base + tk0 + 4 * t < t1;
#pragma unroll
            for (int kk = 0; kk < KK; kk++)
#pragma unroll
                for (int i = 0; i < 8; i++)
                    kf[t][kk][i] = live ? kf[t][kk][i] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool live = okv && base + 8 * g + i < t1;
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                vf[nb][i] = live ? vf[nb][i] : 0.0f;
        }
    }
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int i = 0; i < 8; i++)
            mk = fmaxf(mk, fmaxf(fabsf(kf[0][kk][i]), fabsf(kf[1][kk][i])));
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int i = 0; i < 8; i++)
            mv = fmaxf(mv, fabsf(vf[nb][i]));
    mk = wave_max_nonneg(mk);
    mv = wave_max_nonneg(mv);
    ksc = block_scale(mk, ksc);
    const float vnew = block_scale(mv, vsc);
    if (vsc != 0.0f && vnew != vsc) {
        const float f = vnew * pow2_recip(vsc);
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
            S.o[nb] *= f;
    }
    vsc = vnew;
    if (ksc != 1.0f) {
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                kf[0][kk][i] *= ksc;
                kf[1][kk][i] *= ksc;
            }
    }
    if (vsc != 1.0f) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
            for (int i = 0; i < 8; i++)
                vf[nb][i] *= vsc;
    }
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        u4 h0, l0, h1, l1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t a0, b0, a1, b1;
            split_pair(kf[0][kk][2 * k], kf[0][kk][2 * k + 1], a0, b0, neg1);
            split_pair(kf[1][kk][2 * k], kf[1][kk][2 * k + 1], a1, b1, neg1);
            h0[k] = a0;
            l0[k] = b0;
            h1[k] = a1;
            l1[k] = b1;
        }
        kh0[kk] = __builtin_bit_cast(h8, h0);
        kl0[kk] = __builtin_bit_cast(h8, l0);
        kh1[kk] = __builtin_bit_cast(h8, h1);
        kl1[kk] = __builtin_bit_cast(h8, l1);
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        u4 hh, ll;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t a0, b0;
            split_pair(vf[nb][2 * k], vf[nb][2 * k + 1], a0, b0, neg1);
            hh[k] = a0;
            ll[k] = b0;
        }
        vh[nb] = __builtin_bit_cast(h8, hh);
        vl[nb] = __builtin_bit_cast(h8, ll);
    }
}

// Scores of one block from quantised K: per k-step a fresh product of the
// codes, scaled by the K block scale of its row's token, then the packed
// hi/lo columns are completed with the lane mirror.  The codes enter as fp16
// subnormals (code + offset) * 2^-24 (q4_0: n = code + 8, its high nibbles
// in place as 16n; q8_0: code + 128); each product starts from qz[kk], minus
// the offset times 2^-24 times its column's query sum over the k-step, so it
// ends at 2^-24 times the product of the codes themselves (the 2^24 is in
// the scores' factor).
template <int KT, int HD, int GP>
__device__ __forceinline__ void qk_q(const QBlock<KT, HD> &B, const h8 *qh, const f4 *qz, int g, f4 &s0, f4 &s1)
{
    constexpr int KK = HD / 32;
    s0 = f4{0.0f, 0.0f, 0.0f, 0.0f};
    s1 = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // q4_0: lanes g >= 2 take the high nibbles in place (16n); their query
    // elements carry 1/16
    const uint32_t km = (g & 2) ? 0x00F000F0u : 0x000F000Fu;
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        const h8 a0 = KT == KV_Q4_0 ? u4x8_sub_to_h8(B.k0[kk], km) : i8x8_sub_to_h8(B.k0[kk]);
        const h8 a1 = KT == KV_Q4_0 ? u4x8_sub_to_h8(B.k1[kk], km) : i8x8_sub_to_h8(B.k1[kk]);
        const f4 z0 = mfma(a0, qh[kk], qz[kk]);
        const f4 z1 = mfma(a1, qh[kk], qz[kk]);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            // output row 4g + r of tile 0 is token 8g + r, of tile 1 8g + 4 + r
            s0[r] = fmaf(z0[r], half_at(B.ks, r * KK + kk), s0[r]);
            s1[r] = fmaf(z1[r], half_at(B.ks, (4 + r) * KK + kk), s1[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        s0[r] += mirror<GP>(s0[r]);
        s1[r] += mirror<GP>(s1[r]);
    }
}

// qk_q for four heads per kv head: tile 0 goes through query columns 0-7
// (qh, zero in 8-15) and tile 1 through columns 8-15 (qh1, the same query
// moved up 8 columns), into one accumulator per k-step.  Lanes j < 8 then
// hold tokens 8g .. 8g+3 of column j, lanes j >= 8 tokens 8g+4 .. 8g+7 of
// column j - 8: every lane's four outputs are scores in use, so the K
// scales cost four multiply-adds per k-step instead of eight, and the
// softmax finds its tokens where it needs them.  qz holds each column's
// start value in both halves.
template <int KT, int HD>
__device__ __forceinline__ void qk_q_split(const QBlock<KT, HD, true> &B, const h8 *qh, const h8 *qh1,
                                           const f4 *qz, int g, f4 &s)
{
    constexpr int KK = HD / 32;
    s = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t km = (g & 2) ? 0x00F000F0u : 0x000F000Fu;
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        const h8 a0 = KT == KV_Q4_0 ? u4x8_sub_to_h8(B.k0[kk], km) : i8x8_sub_to_h8(B.k0[kk]);
        const h8 a1 = KT == KV_Q4_0 ? u4x8_sub_to_h8(B.k1[kk], km) : i8x8_sub_to_h8(B.k1[kk]);
        f4 z = mfma(a0, qh[kk], qz[kk]);
        z = mfma(a1, qh1[kk], z);
#pragma unroll
        for (int r = 0; r < 4; r++)
            s[r] = fmaf(z[r], half_at(B.ks, r * KK + kk), s[r]);
    }
#pragma unroll
    for (int r = 0; r < 4; r++)
        s[r] += mirror<4>(s[r]);
}

template <int HD, int GP>
__device__ __forceinline__ void qk(const h8 *k0, const h8 *k1, const h8 *qh, const h8 *ql, f4 &s0,
                                   f4 &s1)
{
    s0 = f4{0.0f, 0.0f, 0.0f, 0.0f};
    s1 = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) {
        s0 = mfma(k0[kk], qh[kk], s0);
        s1 = mfma(k1[kk], qh[kk], s1);
        if (GP == 0) {
            s0 = mfma(k0[kk], ql[kk], s0);
            s1 = mfma(k1[kk], ql[kk], s1);
        }
    }
    if (GP != 0) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            s0[r] += mirror<GP>(s0[r]);
            s1[r] += mirror<GP>(s1[r]);
        }
    }
}

// Online-softmax update and P*V for one block whose scores are s0/s1.
// Unpacked: P rows are heads, hi and lo halves in two products.  Packed: row
// j < G carries p_hi of head j and row 2G-1-j p_lo of head j (the lane of
// that column already holds the head's full score), one product; the two
// output rows of a head are added in the final merge.
template <int HD, int GP, bool VLO = false>
__device__ __forceinline__ void softmax_pv(f4 s0, f4 s1, h8 *v, int base, int ok, int t1, int j,
                                           int g, float c, State<HD> &S, h8 *vl = nullptr)
{
    constexpr int NB = HD / 16;
    float sc[8];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sc[r] = s0[r] * c;
        sc[4 + r] = s1[r] * c;
    }
    if (base + 32 > t1 || ok != 3) {
        // Tokens past the end (or on a rejected page) get weight 0, and
        // their V values -- whatever the slot holds -- are zeroed so they
        // cannot turn 0 * V into NaN.
        const bool okg = (ok >> (g >> 1)) & 1; // this lane's tokens 8g .. 8g+7
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!(base + 8 * g + i < t1 && okg)) {
                sc[i] = -INFINITY;
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    v[nb][i] = (_Float16)0.0f;
                    if (VLO)
                        vl[nb][i] = (_Float16)0.0f;
                }
            }
        }
    }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; i++)
        mx = fmaxf(mx, sc[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(S.m2, mx);
    // every score so far masked (a rejected first page): a finite reference
    // keeps alpha and p at 0 instead of exp2(-inf + inf)
    const float mref = mnew == -INFINITY ? 0.0f : mnew;
    // the bare exponential instruction: results below 2^-126 (flushed to
    // zero) weigh nothing beside the block maximum's 2^14
    const float alpha = __builtin_amdgcn_exp2f(S.m2 - mref);
    S.m2 = mnew;
    // p carries a factor 2^14 (its lo half stays a normal fp16); the running
    // sum carries the same factor, which cancels in the final division.
    const float msub = mref - 14.0f;
    float ps = 0.0f;
    h8 ph, pl;
    const bool lo_row = GP != 0 && j >= GP;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float p = __builtin_amdgcn_exp2f(sc[i] - msub);
        ps += p;
        const _Float16 hi = (_Float16)p;
        const _Float16 lo = (_Float16)(p - (float)hi);
        if (GP == 0) {
            ph[i] = hi;
            pl[i] = lo;
        } else {
            ph[i] = lo_row ? lo : hi;
        }
    }
    S.lsum = S.lsum * alpha + ps;
    // Output rows of this lane are 4g + r; their factor is the alpha of the
    // head of column 4g + r.  Skipped when no running max moved (a multiply
    // by exactly 1).
    if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * g + r);
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                S.o[nb][r] *= ar;
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        S.o[nb] = mfma(ph, v[nb], S.o[nb]);
        if (GP == 0)
            S.o[nb] = mfma(pl, v[nb], S.o[nb]);
        if (VLO)
            S.o[nb] = mfma(ph, vl[nb], S.o[nb]);
    }
}

// P*V of one output tile from quantised V.  The codes enter as exact fp16
// values code - offset (q4_0: n - 8 of dimension tile h of the byte row,
// the high nibbles in place as 16 (n - 8), so tile 2db+1 accumulates 16 O).
// (Codes taken as subnormals with the offset taken out by a second product
// lose accuracy: the two sums cancel when the output is small beside the
// weights, 9e-5 against 6e-6 relative at batch 256 x 8192.)
template <int KT>
__device__ __forceinline__ void pv_q(const h8 &pw8, u2 codes, int h, f4 &o)
{
    const h8 vv = KT == KV_Q4_0 ? u4x8_masked_to_h8(codes, h ? 0xF0F0F0F0u : 0x0F0F0F0Fu,
                                                    h ? h2{(_Float16)1152.0f, (_Float16)1152.0f}
                                                      : h2{(_Float16)1032.0f, (_Float16)1032.0f})
                                : i8x8_to_h8(codes);
    o = mfma(pw8, vv, o);
}

// Lane j ^ 8 of the same 16-lane row (an update of 0: folds into its user).
__device__ __forceinline__ float xor8(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t xor8u(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, true);
}

// softmax_pv_q for four heads per kv head (packed columns 0-3 hi, 4-7 lo),
// on the scores of qk_q_split: lane j < 8 holds tokens 8g .. 8g+3 of column
// j, lane j + 8 tokens 8g+4 .. 8g+7 of it, so the softmax and the V-scale
// fold run on 4 tokens per lane instead of 8.  The folded P pairs then go
// back to the lanes of their operand rows (lanes 8-15 feed P rows 8-15,
// whose output rows are never read).  A column's running sum is split over
// lanes j and j + 8; the merge adds them.
template <int KT, int HD>
__device__ __forceinline__ void softmax_pv_q4(f4 s, QBlock<KT, HD, true> &B, int base, int ok, int t1, int j,
                                              int g, float c, State<HD> &S, float &vnorm)
{
    constexpr int KK = HD / 32, GP = 4;
    const bool upper = j >= 8;
    const int t_0 = 8 * g + (upper ? 4 : 0); // block-local token of sc[0]
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; r++)
        sc[r] = s[r] * c;
    if (base + 32 > t1 || ok != 3) {
        const bool okg = (ok >> (g >> 1)) & 1; // tokens 8g .. 8g+7
        // dead tokens: score -inf and V scale 0, as in softmax_pv_q
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (!(base + t_0 + r < t1 && okg)) {
                sc[r] = -INFINITY;
                const uint32_t keep = (r & 1) ? 0x0000FFFFu : 0xFFFF0000u;
#pragma unroll
                for (int db = 0; db < KK; db++)
                    B.vs[db][r >> 1] &= keep;
            }
    }
    uint32_t mw = 0;
#pragma unroll
    for (int db = 0; db < KK; db++)
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t e = B.vs[db][k];
            mw = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(us2, mw),
                                                                         __builtin_bit_cast(us2, e)));
        }
    uint32_t mh = max(mw & 0xFFFFu, mw >> 16);
    mh = max(mh, xor8u(mh));
    mh = max(mh, (uint32_t)__shfl_xor((int)mh, 16));
    mh = max(mh, (uint32_t)__shfl_xor((int)mh, 32));
    float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mx = fmaxf(mx, xor8(mx));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(S.m2, mx);
    const float mref = mnew == -INFINITY ? 0.0f : mnew; // as in softmax_pv
    const float alpha = __builtin_amdgcn_exp2f(S.m2 - mref);
    S.m2 = mnew;
    const float msub = mref - 14.0f;
    float p[4], ps = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        p[r] = __builtin_amdgcn_exp2f(sc[r] - msub);
        ps += p[r];
    }
    S.lsum = S.lsum * alpha + ps;
    uint32_t bits = __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)mh));
    if (bits & 0x7FFFFFu)
        bits = (bits & 0xFF800000u) + 0x800000u;
    const float pw = __builtin_bit_cast(float, bits);
    const bool grow = pw > vnorm;
    const float f = grow ? vnorm * __builtin_bit_cast(float, 0x7F000000u - bits) : 1.0f;
    if (grow)
        vnorm = pw;
    if (__any(alpha != 1.0f) || grow) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * g + r) * f;
#pragma unroll
            for (int nb = 0; nb < 2 * KK; nb++)
                S.o[nb][r] *= ar;
        }
    }
    // the column this lane works for is j & 7: lo rows are 4..7
    const bool lo_row = (j & 7) >= GP;
    const float inv = vnorm > 0.0f ? __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, vnorm)) *
                                         (lo_row ? 2048.0f : 1.0f)
                                   : 0.0f;
    const uint32_t cut = lo_row ? 0xFFFFE000u : 0u;
    float pp[4];
#pragma unroll
    for (int r = 0; r < 4; r++)
        pp[r] = p[r] * inv;
#pragma unroll
    for (int db = 0; db < KK; db++) {
        // the scale words of this lane's 4 tokens (copied out before the
        // bit casts)
        const uint32_t w0 = B.vs[db][0], w1 = B.vs[db][1];
        const h2 v01 = __builtin_bit_cast(h2, w0), v23 = __builtin_bit_cast(h2, w1);
        const float x0 = fmaf(pp[0], (float)v01[0], 0.0f), x1 = fmaf(pp[1], (float)v01[1], 0.0f);
        const float x2 = fmaf(pp[2], (float)v23[0], 0.0f), x3 = fmaf(pp[3], (float)v23[1], 0.0f);
        const float y0 = x0 - __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x0) & cut);
        const float y1 = x1 - __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x1) & cut);
        const float y2 = x2 - __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x2) & cut);
        const float y3 = x3 - __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x3) & cut);
        const uint32_t pa = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(y0, y1));
        const uint32_t pb = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(y2, y3));
        // lanes j < 8: own tokens 0-3, then lane j+8's tokens 4-7
        const h8 pw8 = __builtin_bit_cast(h8, u4{pa, pb, xor8u(pa), xor8u(pb)});
#pragma unroll
        for (int h = 0; h < 2; h++)
            pv_q<KT>(pw8, B.v[KT == KV_Q4_0 ? db : 2 * db + h], h, S.o[2 * db + h]);
    }
}

// Online softmax and P*V for one block of a quantised page.  Rows of P are
// packed as in softmax_pv (row j < G: hi half of head j, row 2G-1-j: lo half
// times 2^11).  For V block db the rows carry w = p * vscale / vnorm, vnorm
// being the wave's running power-of-two cap over every V scale it has seen
// (one cap for all blocks: the lo rows' extra 2^11 keeps 22 significant
// bits for any scale within 2^10 of the cap).  Tokens past the end or on a
// rejected page get score -inf and scale 0, so whatever their slots hold
// takes no part in w or in the cap.
template <int KT, int HD, int GP>
__device__ __forceinline__ void softmax_pv_q(f4 s0, f4 s1, QBlock<KT, HD> &B, int base, int ok, int t1, int j,
                                             int g, float c, State<HD> &S, float &vnorm)
{
    constexpr int KK = HD / 32;
    float sc[8];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sc[r] = s0[r] * c;
        sc[4 + r] = s1[r] * c;
    }
    if (base + 32 > t1 || ok != 3) {
        const bool okg = (ok >> (g >> 1)) & 1; // tokens 8g .. 8g+7
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!(base + 8 * g + i < t1 && okg)) {
                sc[i] = -INFINITY;
                const uint32_t keep = (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
#pragma unroll
                for (int db = 0; db < KK; db++)
                    B.vs[db][i >> 1] &= keep;
            }
        }
    }
    // cap: the largest V scale of the block.  Scales are non-negative
    // halves, whose bit patterns order like the values.
    // (each word is copied out before the bit cast: hipcc's __builtin_bit_cast
    // of an ext_vector element reads element 0 whatever the index)
    uint32_t mw = 0;
#pragma unroll
    for (int db = 0; db < KK; db++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t e = B.vs[db][k];
            mw = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(us2, mw),
                                                                         __builtin_bit_cast(us2, e)));
        }
    uint32_t mh = max(mw & 0xFFFFu, mw >> 16);
    mh = max(mh, (uint32_t)__shfl_xor((int)mh, 16));
    mh = max(mh, (uint32_t)__shfl_xor((int)mh, 32));
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; i++)
        mx = fmaxf(mx, sc[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(S.m2, mx);
    const float mref = mnew == -INFINITY ? 0.0f : mnew; // as in softmax_pv
    const float alpha = __builtin_amdgcn_exp2f(S.m2 - mref);
    S.m2 = mnew;
    const float msub = mref - 14.0f;
    float p[8], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        p[i] = __builtin_amdgcn_exp2f(sc[i] - msub);
        ps += p[i];
    }
    S.lsum = S.lsum * alpha + ps;
    // smallest power of two >= the largest scale (never NaN: scales come
    // from the append's truncation, which maps NaN away)
    uint32_t bits = __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)mh));
    if (bits & 0x7FFFFFu)
        bits = (bits & 0xFF800000u) + 0x800000u;
    const float pw = __builtin_bit_cast(float, bits);
    const bool grow = pw > vnorm; // uniform across the wave
    // vnorm and pw are 0 or powers of two in [2^-24, 2^16]: their quotient
    // and reciprocal are exact exponent arithmetic
    const float f = grow ? vnorm * __builtin_bit_cast(float, 0x7F000000u - bits) : 1.0f;
    if (grow)
        vnorm = pw;
    if (__any(alpha != 1.0f) || grow) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * g + r) * f;
#pragma unroll
            for (int nb = 0; nb < 2 * KK; nb++)
                S.o[nb][r] *= ar;
        }
    }
    const bool lo_row = j >= GP;
    // lo rows carry 2^11 from the start: x = 2^11 w there, and its lo half is
    // x minus x cut to 11 significant bits (the value its hi half
    // round-toward-zero converts to), exact in float32
    const float inv = vnorm > 0.0f ? __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, vnorm)) *
                                         (lo_row ? 2048.0f : 1.0f)
                                   : 0.0f;
    const uint32_t cut = lo_row ? 0xFFFFE000u : 0u;
    float pp[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        pp[i] = p[i] * inv;
#pragma unroll
    for (int db = 0; db < KK; db++) {
        const h8 vh = __builtin_bit_cast(h8, B.vs[db]);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // x = p / vnorm * vscale (times 2^11 on lo rows), the scale read
            // as a half by the mixed-precision multiply-add (exact widening)
            const float x = fmaf(pp[i], (float)vh[i], 0.0f);
            // hi rows: x itself; lo rows: x - trunc11(x)
            y[i] = x - __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & cut);
        }
        uint32_t pk[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            pk[k] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(y[2 * k], y[2 * k + 1]));
        const h8 pw8 = __builtin_bit_cast(h8, u4{pk[0], pk[1], pk[2], pk[3]});
#pragma unroll
        for (int h = 0; h < 2; h++)
            pv_q<KT>(pw8, B.v[KT == KV_Q4_0 ? db : 2 * db + h], h, S.o[2 * db + h]);
    }
}

// Body of the decode kernels.  KT: KV_F16, or KV_Q8_0 / KV_Q4_0 (packed GP
// only).  STG: fp16 pages with K staged through LDS (F16KStage).
template <int KT, int HD, int GP, bool NT, bool PREFETCH, int NW, bool STG = false>
__device__ __forceinline__ void decode_body(const DecodeArgs &a)
{
    static_assert(!STG || (KT == KV_F16 && HD == 128), "staged fp16 pages at head_dim 128");
    constexpr int KK = HD / 32, NB = HD / 16;
    constexpr bool QUANT = KT == KV_Q8_0 || KT == KV_Q4_0;
    constexpr bool F32 = KT == KV_F32;
    constexpr int kStageAux = stage_aux<NW>(); // quantised and f32 stages
    // quantised pages, four heads per kv head: the two token tiles of a block
    // share one score accumulator (qk_q_split)
    constexpr bool SPLIT = QUANT && GP == 4;
    static_assert(!(QUANT || F32) || GP != 0, "quantised and f32 pages use the packed hi/lo form");
    const PoolLayout &L = a.L;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int H = a.num_heads, KVH = L.num_kv_heads, G = H / KVH, P = L.page_tokens;
    const int h0 = kvh * G;
    int len = a.seq_lens[b];
    if (len > a.max_blocks * P || len < 0) {
        // more tokens than the block table maps (read what it maps), or a
        // negative length (nothing to read)
        if (threadIdx.x == 0 && split == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_SLOT);
        len = len < 0 ? 0 : a.max_blocks * P;
    }
    // the last split runs to the end of the sequence, so that a length
    // beyond the one the plan was sized for is still attended in full
    const int t0 = split * a.split_tokens;
    const int t1 = split == a.num_splits - 1 ? len : min(len, t0 + a.split_tokens);
    const int64_t qrow = (int64_t)b * H + h0;

    // Decode step (gi_paged_decode_step): the new token (position
    // seq_lens[b] - 1) is stored before it is attended, as Forward stores
    // before it attends (forward.go:236-267), by the workgroup whose token
    // range holds it, for its own kv head.  With pages of up to 32 tokens
    // every cache line of a page belongs to one 32-token block, which one
    // wave reads (wave w reads blocks t0 + 32w + 32*NW*i): that wave stores the
    // token, after issuing its first block's loads unless that is the
    // token's block (the stores wait for the loads of the token's values,
    // which should not hold up the block's loads), and waits for the stores
    // to complete only before it issues the token's block.  The other waves
    // never wait.  Wider pages share lines between the blocks of two waves,
    // so there every thread joins the store and a barrier follows.  No other
    // workgroup reads that token's bytes (other kv heads are other bytes,
    // split ranges are whole pages).  A length the tables cannot hold is
    // flagged, as the separate append does, and nothing is stored.
    int sblk = -1;          // the token's block, in the wave that stores it
    int64_t st_page = 0;    // and where the token goes
    int st_slot = 0;
    if (a.new_k) {
        const int raw = a.seq_lens[b], pos = raw - 1;
        if (pos < 0 && threadIdx.x == 0 && split == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_SLOT);
        if (raw == len && t0 <= pos && pos < t1) {
            const int64_t pg = a.block_tables[(int64_t)b * a.max_blocks + pos / P];
            const bool okp = pg >= 0 && pg < L.num_pages;
            if (!okp && threadIdx.x == 0 && a.status)
                atomicOr(a.status, FLAG_BAD_PAGE);
            if (P <= 32) {
                if (okp && w == ((pos - t0) >> 5) % NW) {
                    sblk = __builtin_amdgcn_readfirstlane(t0 + ((pos - t0) & ~31));
                    st_page = pg;
                    st_slot = pos % P;
                }
            } else {
                const int64_t e = ((int64_t)b * L.num_kv_heads + kvh) * HD + threadIdx.x;
                if (okp && threadIdx.x < HD)
                    store_token_elem<KT>(L, a.append_base + pg * L.page_bytes, pos % P, kvh, threadIdx.x,
                                         a.new_k[e], a.new_v[e], true);
                __syncthreads();
            }
        }
    }
    auto store_token = [&]() {
        const int64_t e0 = ((int64_t)b * L.num_kv_heads + kvh) * HD;
#pragma unroll
        for (int d = lane; d < HD; d += 64)
            store_token_elem<KT>(L, a.append_base + st_page * L.page_bytes, st_slot, kvh, d, a.new_k[e0 + d],
                                 a.new_v[e0 + d], true);
    };

    // The per-wave staging areas of the block loop (quantised and f32 pages,
    // and fp16 K) and, after it, the cross-wave merge share one LDS
    // allocation.  (fp16 V loads straight into registers: staging V as well
    // measured slower.)
    constexpr int STAGE_BYTES = QUANT ? NW * (int)sizeof(QStage<QUANT ? KT : KV_Q8_0, HD>)
                                : F32 ? NW * (int)sizeof(F32Stage<HD>)
                                : STG ? NW * (int)sizeof(F16KStage) : 0;
    constexpr int MERGE_BYTES = NW * 16 * HD * (int)sizeof(float);
    __shared__ __align__(16) uint8_t s_stage[STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES];
    float(*s_o)[16][HD] = reinterpret_cast<float(*)[16][HD]>(s_stage);
    __shared__ float s_m[NW][16], s_l[NW][16];

    float *wsp = nullptr;
    if (a.num_splits > 1)
        wsp = a.ws + (((int64_t)b * KVH + kvh) * a.num_splits + split) * (G * (HD + 2));

    if (t0 >= t1) {
        for (int e = threadIdx.x; e < G * HD; e += 64 * NW) {
            if (wsp)
                wsp[e] = 0.0f;
            else
                a.out[qrow * HD + e] = 0.0f;
        }
        if (wsp && threadIdx.x < G) {
            wsp[G * HD + 2 * threadIdx.x] = -INFINITY;
            wsp[G * HD + 2 * threadIdx.x + 1] = 0.0f;
        }
        return;
    }

    // Q^T operand: column j = head h0 + j (zero beyond the group), k-slot
    // (g, v) of step kk = dimension 32*kk + 8*g + v.
    // Packed: column j < G is q_hi of head j, column 2G-1-j is q_lo of head j.
    // SPLIT: lanes j >= 8 take the query of column j - 8 (qh1, the operand
    // of the second token tile), so that their scores and scale factor are
    // those of column j - 8.
    const int jq = SPLIT ? (j & 7) : j;
    const int qhead = GP == 0 ? jq : (jq < G ? jq : 2 * G - 1 - jq);
    const bool qvalid = GP == 0 ? jq < G : jq < 2 * G;
    const bool qlo = GP != 0 && jq >= G;
    // Each head's query is scaled by 2^qe (from its largest |q|) so both fp16
    // halves stay normal, and the scores are scaled back through c.  The hi
    // and lo columns of a head see the same values, so they pick the same qe.
    // (Loaded by load_q once the wave's first block is in flight, so that the
    // two memory round trips overlap.)
    h8 qh[KK], ql[KK], qh1[KK];
    f4 qz[KK]; // quantised pages: the initial value of each k-step's product
    float c = 0.0f;
    auto load_q = [&]() {
        float qv[KK][8];
        float mq = 0.0f;
        const float *qp = a.q + (qrow + qhead) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            const float4 x0 = qvalid ? *reinterpret_cast<const float4 *>(qp + 32 * kk) : float4{};
            const float4 x1 = qvalid ? *reinterpret_cast<const float4 *>(qp + 32 * kk + 4) : float4{};
            qv[kk][0] = x0.x;
            qv[kk][1] = x0.y;
            qv[kk][2] = x0.z;
            qv[kk][3] = x0.w;
            qv[kk][4] = x1.x;
            qv[kk][5] = x1.y;
            qv[kk][6] = x1.z;
            qv[kk][7] = x1.w;
#pragma unroll
            for (int v = 0; v < 8; v++)
                mq = fmaxf(mq, fabsf(qv[kk][v]));
        }
        mq = fmaxf(mq, __shfl_xor(mq, 16));
        mq = fmaxf(mq, __shfl_xor(mq, 32));
        const int qe = pow2_exponent_for(mq);
        // q4_0 pages: dimensions 16..31 of each block (lanes g >= 2) meet
        // high nibbles that carry 16
        const float up = ldexpf(KT == KV_Q4_0 && (g & 2) ? 0.0625f : 1.0f, qe);
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int v = 0; v < 8; v++) {
                // q4_0 pages: operand slot v holds dimension 8g + sv, in the
                // order the nibble conversion yields (0, 2, 1, 3, 4, 6, 5, 7)
                const int sv = KT == KV_Q4_0 ? (v & 4) | ((v & 1) << 1) | ((v >> 1) & 1) : v;
                const float x = qv[kk][sv] * up;
                _Float16 hi = (_Float16)x;
                _Float16 lo = (_Float16)(x - (float)hi);
                const _Float16 q = qlo ? lo : hi;
                qh[kk][v] = SPLIT && j >= 8 ? (_Float16)0.0f : q;
                qh1[kk][v] = j >= 8 ? q : (_Float16)0.0f;
                ql[kk][v] = lo;
            }
        c = a.scale * kLog2e * ldexpf(1.0f, -qe);
        if constexpr (QUANT) {
            // codes enter the products as (code + off) * 2^-24: start each
            // product at -off * 2^-24 times its column's query sum (the
            // values of the operand itself; q4_0 high-nibble slots count 16
            // times), and take 2^24 out through c
            const float off = KT == KV_Q4_0 ? 8.0f : 128.0f;
            const float fac = KT == KV_Q4_0 && (g & 2) ? 16.0f : 1.0f;
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                float t = 0.0f;
#pragma unroll
                for (int v = 0; v < 8; v++)
                    t += (float)(SPLIT && j >= 8 ? qh1[kk][v] : qh[kk][v]);
                t *= fac;
                t += __shfl_xor(t, 16);
                t += __shfl_xor(t, 32);
                const float z = t * (-off * 0x1p-24f);
                qz[kk] = f4{z, z, z, z};
            }
            c *= 0x1p24f;
        }
    };
    State<HD> S;
    S.m2 = -INFINITY;
    S.lsum = 0.0f;
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
        S.o[nb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float ksc = 0.0f, vsc = 0.0f; // f32 pages: running K / V operand scales
    const float neg1 = mfma_ops::opaque_neg1(); // f32 pages: for split_pair
    float vnorm = 0.0f; // quantised pages: running power-of-two cap of the V scales

    // bytes per stored element: fp16 2, q8_0 1, q4_0 1/2
    constexpr int EB_NUM = F32 ? 4 : KT == KV_F16 ? 2 : 1, EB_DEN = KT == KV_Q4_0 ? 2 : 1;
    const int64_t koff = L.k_off + (int64_t)kvh * P * HD * EB_NUM / EB_DEN;
    const int64_t voff = L.v_off + (int64_t)kvh * HD * P * EB_NUM / EB_DEN;
    const int32_t *bt = a.block_tables + (int64_t)b * a.max_blocks;
    const int stride = 32 * NW;

    // Block starts are wave-uniform (scalar registers), so the loop test is a
    // scalar branch.  Every block but the last runs inside the loop, where
    // the next block's loads are issued unconditionally (K once this block's
    // scores exist, V once its P*V has consumed the V registers): the wait
    // counters then see one pattern of loads in flight on every path, and a
    // wait for this block's V never waits for the next block's K.
    int base = __builtin_amdgcn_readfirstlane(t0 + 32 * w);
    // before the loads of block x are issued: the decode step's token stores
    // of this wave have completed if x holds the token (the memory clobber
    // keeps the compiler from moving loads or stores across the wait)
    auto store_done = [&](int x) {
        if (x == sblk)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    // the token's stores: before the first block's loads if that block holds
    // it, otherwise right after them (store_late)
    const bool store_late = sblk >= 0 && sblk != base;
    if (sblk >= 0 && !store_late)
        store_token();
    if constexpr (QUANT) {
        const int64_t ksoff = L.ks_off + (int64_t)kvh * P * KK * 2;
        const int64_t vsoff = L.vs_off + (int64_t)kvh * KK * P * 2;
        if (base < t1) {
            QStage<KT, HD> &Sq = reinterpret_cast<QStage<KT, HD> *>(s_stage)[w];
            int64_t pA, pB;
            int sA, sB;
            int ok;
            store_done(base);
            block_pages(a, bt, base, t1, pA, pB, sA, sB, ok);
            issue_qk<KT, HD, kStageAux>(a, pA, pB, sA, sB, koff, lane, Sq);
            issue_qv<KT, HD, kStageAux>(a, pA, pB, sA, sB, ksoff, voff, vsoff, lane, Sq);
            load_q();
            if (store_late)
                store_token();
            // Loads go out in the order K codes, scales, V codes of one
            // block, K codes of the next, ...: the K half of a block is read
            // (and the next block's K refills its slots) before the scores,
            // the V half after them, so neither half's registers live
            // through the other's work.
            constexpr int NL = QStage<KT, HD>::NLOAD;
            for (;;) {
                QBlock<KT, HD, SPLIT> B;
                // this block's K codes and scales have arrived (its V codes,
                // the last NL loads issued, may still be in flight)
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(NL));
                read_qk<KT, HD, SPLIT>(Sq, j, g, B);
                const int next = base + stride;
                const bool more = next < t1;
                int64_t nA = pA, nB = pB;
                int nsA = sA, nsB = sB;
                int nok = ok;
                if (more) {
                    store_done(next);
                    block_pages(a, bt, next, t1, nA, nB, nsA, nsB, nok);
                    // every read of this block's K half has returned before
                    // its slots are refilled
                    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
                    issue_qk<KT, HD, kStageAux>(a, nA, nB, nsA, nsB, koff, lane, Sq);
                }
                f4 s0, s1;
                if constexpr (SPLIT)
                    qk_q_split<KT, HD>(B, qh, qh1, qz, g, s0);
                else
                    qk_q<KT, HD, GP>(B, qh, qz, g, s0, s1);
                // this block's V codes have arrived (the next block's K
                // codes, issued after them, may still be in flight)
                if (more)
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(NL));
                else
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                read_qv<KT, HD, SPLIT>(Sq, j, g, B);
                if (more) {
                    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
                    issue_qv<KT, HD, kStageAux>(a, nA, nB, nsA, nsB, ksoff, voff, vsoff, lane, Sq);
                }
                if constexpr (SPLIT)
                    softmax_pv_q4<KT, HD>(s0, B, base, ok, t1, j, g, c, S, vnorm);
                else
                    softmax_pv_q<KT, HD, GP>(s0, s1, B, base, ok, t1, j, g, c, S, vnorm);
                if (!more)
                    break;
                pA = nA;
                pB = nB;
                sA = nsA;
                sB = nsB;
                ok = nok;
                base = next;
            }
        }
    } else if constexpr (F32) {
        if (base < t1) {
            F32Stage<HD> &Sf = reinterpret_cast<F32Stage<HD> *>(s_stage)[w];
            const F32Lanes fl = f32_lanes<HD>(lane, P);
            int64_t pA, pB;
            int sA, sB;
            int ok;
            store_done(base);
            block_pages(a, bt, base, t1, pA, pB, sA, sB, ok);
            issue_f32<HD, kStageAux>(a, pA, pB, sA, sB, koff, voff, fl, Sf);
            load_q();
            if (store_late)
                store_token();
            for (;;) {
                h8 kh0[KK], kh1[KK], kl0[KK], kl1[KK], vh[NB], vl[NB];
                // the only vector loads in flight are this block's
                __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
                read_f32<HD>(Sf, j, g, base, ok, t1, kh0, kh1, kl0, kl1, vh, vl, ksc, vsc, S, neg1);
                const int next = base + stride;
                const bool more = next < t1;
                int64_t nA = pA, nB = pB;
                int nsA = sA, nsB = sB;
                int nok = ok;
                if (more) {
                    store_done(next);
                    block_pages(a, bt, next, t1, nA, nB, nsA, nsB, nok);
                    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): this block's reads returned
                    issue_f32<HD, kStageAux>(a, nA, nB, nsA, nsB, koff, voff, fl, Sf);
                }
                // S = (kh + kl) . (q_hi | q_lo): two products per k-step
                f4 s0 = f4{0.0f, 0.0f, 0.0f, 0.0f}, s1 = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    s0 = mfma(kh0[kk], qh[kk], s0);
                    s1 = mfma(kh1[kk], qh[kk], s1);
                    s0 = mfma(kl0[kk], qh[kk], s0);
                    s1 = mfma(kl1[kk], qh[kk], s1);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    s0[r] += mirror<GP>(s0[r]);
                    s1[r] += mirror<GP>(s1[r]);
                }
                softmax_pv<HD, GP, true>(s0, s1, vh, base, ok, t1, j, g, c * pow2_recip(ksc), S, vl);
                if (!more)
                    break;
                pA = nA;
                pB = nB;
                sA = nsA;
                sB = nsB;
                ok = nok;
                base = next;
            }
        }
    } else if constexpr (STG) {
        if (base < t1) {
            // Per block n: wait for K (n) in the stage, read its operands,
            // issue K (n + 1) into the stage; scores; wait for V (n) (issued
            // after P V (n - 1), before K (n + 1)); softmax and P V; issue V
            // (n + 1) into registers.  In flight at the top of block n + 1:
            // K (n + 1), then V (n + 1), so vmcnt(NLOAD) waits for K alone.
            F16KStage &Sk = reinterpret_cast<F16KStage *>(s_stage)[w];
            h8 v[NB];
            int64_t pA, pB;
            int sA, sB;
            int ok;
            store_done(base);
            block_pages(a, bt, base, t1, pA, pB, sA, sB, ok);
            issue_k_f16(a, pA, pB, sA, sB, koff, lane, Sk);
            load_v<HD, NT>(a, pA, pB, sA, sB, voff, j, g, v);
            load_q();
            if (store_late)
                store_token();
            // the first block: everything issued so far
            __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
            for (;;) {
                h8 k0[KK], k1[KK];
                read_k_f16(Sk, j, g, k0, k1);
                const int next = base + stride;
                const bool more = next < t1;
                int64_t nA = pA, nB = pB;
                int nsA = sA, nsB = sB;
                int nok = ok;
                if (more) {
                    store_done(next);
                    block_pages(a, bt, next, t1, nA, nB, nsA, nsB, nok);
                    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): this block's K reads returned
                    issue_k_f16(a, nA, nB, nsA, nsB, koff, lane, Sk);
                }
                f4 s0, s1;
                qk<HD, GP>(k0, k1, qh, ql, s0, s1);
                softmax_pv<HD, GP>(s0, s1, v, base, ok, t1, j, g, c, S);
                if (!more)
                    break;
                __builtin_amdgcn_sched_barrier(0);
                load_v<HD, NT>(a, nA, nB, nsA, nsB, voff, j, g, v);
                pA = nA;
                pB = nB;
                sA = nsA;
                sB = nsB;
                ok = nok;
                base = next;
                // K of the next block has arrived (its V, issued after it, may still be in flight)
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(F16KStage::NLOAD));
            }
        }
    } else if (base < t1) {
        h8 k0[KK], k1[KK], v[NB];
        int64_t pA, pB;
        int sA, sB;
        int ok;
        store_done(base);
        block_pages(a, bt, base, t1, pA, pB, sA, sB, ok);
        load_k<HD, NT>(a, pA, pB, sA, sB, koff, j, g, k0, k1);
        load_v<HD, NT>(a, pA, pB, sA, sB, voff, j, g, v);
        load_q();
        if (store_late)
            store_token();
        f4 s0, s1;
        for (;;) {
            qk<HD, GP>(k0, k1, qh, ql, s0, s1);
            const int next = base + stride;
            if (next >= t1)
                break;
            int64_t nA, nB;
            int nsA, nsB;
            int nok;
            store_done(next);
            block_pages(a, bt, next, t1, nA, nB, nsA, nsB, nok);
            if (PREFETCH)
                load_k<HD, NT>(a, nA, nB, nsA, nsB, koff, j, g, k0, k1);
            softmax_pv<HD, GP>(s0, s1, v, base, ok, t1, j, g, c, S);
            if (!PREFETCH)
                load_k<HD, NT>(a, nA, nB, nsA, nsB, koff, j, g, k0, k1);
            __builtin_amdgcn_sched_barrier(0);
            load_v<HD, NT>(a, nA, nB, nsA, nsB, voff, j, g, v);
            pA = nA;
            pB = nB;
            sA = nsA;
            sB = nsB;
            ok = nok;
            base = next;
        }
        softmax_pv<HD, GP>(s0, s1, v, base, ok, t1, j, g, c, S);
    }

    // every wave is done with its staging area before the merge reuses it
    __syncthreads();
    // wave totals -> LDS
    float lt = S.lsum;
    if constexpr (QUANT && GP == 4)
        lt += xor8(lt); // the compact softmax splits a column over lanes j, j + 8
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    if (g == 0) {
        s_m[w][j] = S.m2;
        s_l[w][j] = lt;
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float o = S.o[nb][r];
            if constexpr (QUANT) {
                // rows G .. 2G-1 hold lo halves carrying 2^11; every row
                // holds O / vnorm of its dimension block
                const int row = 4 * g + r;
                o *= vnorm * (row >= G && row < 2 * G ? 1.0f / 2048.0f : 1.0f) *
                     (KT == KV_Q4_0 && (nb & 1) ? 0.0625f : 1.0f);
            }
            if constexpr (F32) {
                // the accumulators hold O times the wave's V scale
                if (vsc != 0.0f)
                    o *= pow2_recip(vsc);
            }
            s_o[w][4 * g + r][16 * nb + j] = o;
        }
    __syncthreads();

    for (int e = threadIdx.x; e < G * HD; e += 64 * NW) {
        const int hh = e / HD, d = e - hh * HD;
        float M = s_m[0][hh];
#pragma unroll
        for (int x = 1; x < NW; x++)
            M = fmaxf(M, s_m[x][hh]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int x = 0; x < NW; x++) {
            const float mx2 = s_m[x][hh];
            const float f = mx2 == -INFINITY ? 0.0f : exp2f(mx2 - M);
            float o = s_o[x][hh][d];
            if (GP != 0)
                o += s_o[x][2 * G - 1 - hh][d];
            num = fmaf(o, f, num);
            den = fmaf(s_l[x][hh], f, den);
        }
        if (wsp) {
            wsp[hh * HD + d] = num;
            if (d == 0) {
                wsp[G * HD + 2 * hh] = M * (1.0f / kLog2e);
                wsp[G * HD + 2 * hh + 1] = den;
            }
        } else {
            a.out[(qrow + hh) * HD + d] = den > 0.0f ? num / den : 0.0f;
        }
    }
}

// GP: 0 for any group size up to 16 (hi/lo halves in separate products),
// or the group size G in {1, 2, 4, 8} for the packed form.  NT:
// non-temporal (streaming) loads of K/V.  PREFETCH: the next block's loads
// are issued as soon as this block's K (then V) registers are consumed.
// OCC: minimum waves per SIMD requested from the register allocator.  NW:
// waves per workgroup (DecodeArgs.waves).
template <int HD, int GP, bool NT, bool PREFETCH, int OCC, int NW = 4, bool STG = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC))) void attn_mfma_f16(DecodeArgs a)
{
    decode_body<KV_F16, HD, GP, NT, PREFETCH, NW, STG>(a);
}

// f32 pages, packed form (GP = G in {1, 2, 4, 8}).  NW: waves per
// workgroup, 4, or 8 at head dimension 64 (DecodeArgs.waves).
template <int HD, int GP, bool NT, bool PREFETCH, int OCC, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC))) void attn_mfma_f32(DecodeArgs a)
{
    decode_body<KV_F32, HD, GP, NT, PREFETCH, NW>(a);
}

// q8_0 / q4_0 pages, packed form (GP = G in {1, 2, 4, 8}).
template <int KT, int HD, int GP, bool NT, bool PREFETCH, int OCC, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC))) void attn_mfma_q(DecodeArgs a)
{
    decode_body<KT, HD, GP, NT, PREFETCH, NW>(a);
}

} // namespace mfma_decode

bool mfma_decode_supported(const PoolLayout &L, int num_heads)
{
    if (L.page_tokens % 16 != 0)
        return false;
    if (L.head_dim != 64 && L.head_dim != 128)
        return false;
    if (num_heads % L.num_kv_heads)
        return false;
    const int G = num_heads / L.num_kv_heads;
    if (L.kv_type == KV_F16)
        return G >= 1 && G <= 16;
    if (L.kv_type == KV_Q8_0 || L.kv_type == KV_Q4_0 || L.kv_type == KV_F32)
        return G == 1 || G == 2 || G == 4 || G == 8;
    return false;
}

// Launch choices of the decode kernels, as measured best on MI355X:
// non-temporal K/V loads (read once), the next block's loads issued as soon as
// registers free up, at least one wave per SIMD asked of the register
// allocator, and the packed hi/lo query layout for groups of up to 8 heads.
constexpr bool kDecodeNt = true;
constexpr bool kDecodePrefetch = true;
constexpr int kDecodeOcc = 1;
constexpr bool kDecodePack = true;

// K staged through LDS (F16KStage) for head_dim 128 and pages of 16 or 32
// tokens: in four-wave workgroups (grids of several rounds), and in
// eight-wave ones (one round) whose splits hold at most kDecodeStgTokens
// tokens, where one workgroup's streaming rate sets the launch's length.
// Same box: batch 256 x 8192 (page 16) 1.273-1.275 against 1.286 ms per
// launch; batch 32 x U[512, 4096] (page 16) 0.0638-0.0646 against
// 0.0723-0.0750; but 8 x 32768 in eight-wave splits of 8192 (page 32), where
// every CU streams until the end, 0.1751 against 0.1652, so those keep the
// register loads.
constexpr int kDecodeStgTokens = 4096;

template <int HD, int GP>
static void launch_mfma_hd(const DecodeArgs &a, dim3 grid, hipStream_t st)
{
    const int P = a.L.page_tokens;
    const bool stg = HD == 128 && GP != 0 && (P == 16 || P == 32);
    constexpr bool STG = HD == 128 && GP != 0;
    if (a.waves == 8) {
        if (stg && a.split_tokens <= kDecodeStgTokens)
            hipLaunchKernelGGL((mfma_decode::attn_mfma_f16<HD, GP, kDecodeNt, kDecodePrefetch, kDecodeOcc, 8, STG>),
                               grid, dim3(512), 0, st, a);
        else
            hipLaunchKernelGGL((mfma_decode::attn_mfma_f16<HD, GP, kDecodeNt, kDecodePrefetch, kDecodeOcc, 8>),
                               grid, dim3(512), 0, st, a);
    } else if (stg) {
        hipLaunchKernelGGL((mfma_decode::attn_mfma_f16<HD, GP, kDecodeNt, kDecodePrefetch, kDecodeOcc, 4, STG>),
                           grid, dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((mfma_decode::attn_mfma_f16<HD, GP, kDecodeNt, kDecodePrefetch, kDecodeOcc, 4>),
                           grid, dim3(256), 0, st, a);
    }
}

// q4_0 pages are bound by the vector ALU: three waves per SIMD (the
// register allocator then keeps the kernel at 168 VGPRs, unspilled) measured
// 0.487 against 0.522 ms per launch at batch 256 x 8192.  q8_0 pages are
// bound by the texture path, where a third wave costs (0.855 against 0.78).
template <int KT>
constexpr int kDecodeOccQ = KT == KV_Q4_0 ? 3 : kDecodeOcc;

template <int KT, int HD>
static void launch_mfma_q(const DecodeArgs &a, dim3 grid, hipStream_t st)
{
#define GI_Q(GPv)                                                                                        \
    if (a.waves == 8)                                                                                    \
        hipLaunchKernelGGL((mfma_decode::attn_mfma_q<KT, HD, GPv, kDecodeNt, kDecodePrefetch,             \
                                                     kDecodeOccQ<KT>, 8>),                              \
                           grid, dim3(512), 0, st, a);                                                  \
    else                                                                                                 \
        hipLaunchKernelGGL((mfma_decode::attn_mfma_q<KT, HD, GPv, kDecodeNt, kDecodePrefetch,             \
                                                     kDecodeOccQ<KT>, 4>),                              \
                           grid, dim3(256), 0, st, a)
    switch (a.num_heads / a.L.num_kv_heads) {
    case 1: GI_Q(1); break;
    case 2: GI_Q(2); break;
    case 4: GI_Q(4); break;
    default: GI_Q(8); break;
    }
#undef GI_Q
}

template <int HD>
static void launch_mfma_f32(const DecodeArgs &a, dim3 grid, hipStream_t st)
{
    // eight waves (decode_waves) only at head dimension 64: 8 x 16 KiB stages
    constexpr int NW8 = HD == 64 ? 8 : 4;
#define GI_F(GPv)                                                                                 \
    if (a.waves == 8)                                                                             \
        hipLaunchKernelGGL((mfma_decode::attn_mfma_f32<HD, GPv, kDecodeNt, kDecodePrefetch,       \
                                                       kDecodeOcc, NW8>),                         \
                           grid, dim3(64 * NW8), 0, st, a);                                       \
    else                                                                                          \
        hipLaunchKernelGGL((mfma_decode::attn_mfma_f32<HD, GPv, kDecodeNt, kDecodePrefetch,       \
                                                       kDecodeOcc>),                              \
                           grid, dim3(256), 0, st, a)
    switch (a.num_heads / a.L.num_kv_heads) {
    case 1: GI_F(1); break;
    case 2: GI_F(2); break;
    case 4: GI_F(4); break;
    default: GI_F(8); break;
    }
#undef GI_F
}

template <int HD>
static void launch_mfma_g(const DecodeArgs &a, dim3 grid, hipStream_t st)
{
    switch (a.num_heads / a.L.num_kv_heads) {
    case 1: launch_mfma_hd<HD, kDecodePack ? 1 : 0>(a, grid, st); break;
    case 2: launch_mfma_hd<HD, kDecodePack ? 2 : 0>(a, grid, st); break;
    case 4: launch_mfma_hd<HD, kDecodePack ? 4 : 0>(a, grid, st); break;
    case 8: launch_mfma_hd<HD, kDecodePack ? 8 : 0>(a, grid, st); break;
    default: launch_mfma_hd<HD, 0>(a, grid, st); break;
    }
}

hipError_t launch_decode_mfma(const DecodeArgs &a, hipStream_t st)
{
    dim3 grid(a.num_splits, a.L.num_kv_heads, a.batch);
    const bool h128 = a.L.head_dim == 128;
    switch (a.L.kv_type) {
    case KV_Q8_0:
        if (h128)
            launch_mfma_q<KV_Q8_0, 128>(a, grid, st);
        else
            launch_mfma_q<KV_Q8_0, 64>(a, grid, st);
        break;
    case KV_Q4_0:
        if (h128)
            launch_mfma_q<KV_Q4_0, 128>(a, grid, st);
        else
            launch_mfma_q<KV_Q4_0, 64>(a, grid, st);
        break;
    case KV_F32:
        if (h128)
            launch_mfma_f32<128>(a, grid, st);
        else
            launch_mfma_f32<64>(a, grid, st);
        break;
    default:
        if (h128)
            launch_mfma_g<128>(a, grid, st);
        else
            launch_mfma_g<64>(a, grid, st);
        break;
    }
    return hipGetLastError();
}

} // namespace gi
