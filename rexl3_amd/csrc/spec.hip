// Speculative verification by rejection sampling, exact in integer masses (no reference counterpart: REXL3 accepts a
// draft by equality with its keyed sample, crates/spec/src/lib.rs:30-35; this is the extended pipeline's verifier).
//
// p and q are the softmax of the target and draft rows at the row's temperature, as integer masses relative to each
// row's maximum (gbs_modeu.hpp). Draft j of a sequence is accepted iff u_j * q(x) < p(x), i.e.
// floor(u_j * Eq_x * Zp) < Ep_x * Zq exactly. At the first rejection the token is drawn from max(p - q, 0), i.e. from the
// integer weights max(Ep_i * Zq - Eq_i * Zp, 0), with t = floor(u * R) and the first id (ascending) whose running weight
// exceeds t; after `width` acceptances the bonus token is drawn from p of the last row the same way. Temperature 0:
// p is the argmax (ties to the lowest id).
//
// Every row is read once. The row pass takes the maxima (order keys, so the argmax ties to the lowest id), the NaN
// flags and float bounds on the mass sums, which decide nearly every draft: spec_rows_k with one block per row when the
// rows fill the chip, else spec_split_k over (chunks, rows). The block that completes a sequence decides what the
// bounds allow. spec_exact_k then sums the exact masses of the rows that still need them (each drawing sequence's
// draw row, and any row whose test the bounds left open), prepares the draw's weights in the same sweep and draws;
// spec_draw_k draws only what that pass leaves (its fallbacks) and otherwise returns at once.
#include <cfloat>

#include "gbs_modeu.hpp"

using namespace gbs;
using namespace gbs::modeu;

namespace {

#ifndef GBS_SPEC_NT
#define GBS_SPEC_NT 256
#endif
#ifndef GBS_SPEC_BLOCKS
#define GBS_SPEC_BLOCKS 1024
#endif
#ifndef GBS_SPEC_U
#define GBS_SPEC_U 2  // 4-element groups in flight per thread (config 5: 2 -> 127 us, 4 -> 130.5 us, 6 -> 195 us)
#endif
#ifndef GBS_SPEC_AUX_FWD
#define GBS_SPEC_AUX_FWD 2  // cache policy of the forward sweeps' loads (2: non-temporal)
#endif
#ifndef GBS_SPEC_AUX_REV
#define GBS_SPEC_AUX_REV 2
#endif
#ifndef GBS_SPEC_PIPE
#define GBS_SPEC_PIPE 1
#endif
constexpr int NT = GBS_SPEC_NT;
constexpr int TARGET_BLOCKS = GBS_SPEC_BLOCKS;
constexpr int MIN_CHUNK = 2048;
constexpr int U = GBS_SPEC_U;        // 4-element groups per thread in flight, per row
constexpr int DU = 4;                // the draw: 4-element groups per thread per tile
constexpr int TILE = NT * 4 * DU;    // the draw: elements per tile
constexpr int NWD = NT / WAVE;       // the draw: waves per block (one partial sum per wave and tile)
constexpr int SUB = WAVE * 4 * DU;   // the draw: elements of a sub-tile (a wave's part of a tile)
constexpr int DRAW_BLOCKS = 768;     // the draw: blocks in all (one round on the chip)
#ifndef GBS_SPEC_ROWS_MIN
#define GBS_SPEC_ROWS_MIN 192
#endif
constexpr int ROWS_KERNEL_MIN = GBS_SPEC_ROWS_MIN;  // rows from which one block per row fills the chip

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int splits_for(int rows, int vocab) {
    int s = (TARGET_BLOCKS + rows - 1) / rows;
    const int by_size = (vocab + MIN_CHUNK - 1) / MIN_CHUNK;
    if (s > by_size) s = by_size;
    return s < 1 ? 1 : s;
}

// chunk of a split: whole 4-element groups, so that 16-byte loads stay inside one split
int chunk_for(int vocab, int S) {
    const int c = (vocab + S - 1) / S;
    return (c + 3) / 4 * 4;
}

struct RowInfo {
    u64 tkey, dkey;  // row maxima as order keys (0 = no finite-or-inf element; the draft's carries no index)
    unsigned nan;
    unsigned state;  // the draft's test by the float sums, ACC_YES / ACC_NO / ACC_OPEN
    float fp, fq;    // float sums of 2^((l - M) c2) over the target and the draft row
    u64 ep, eq;      // the draft token's masses (a draft row at T > 0 whose test ran)
    unsigned check;  // the row block's own check (row_check), when the row kernel made it
};

// the test of a draft from float bounds on the mass sums
constexpr unsigned ACC_YES = 0, ACC_NO = 1, ACC_OPEN = 2;

struct SeqInfo {
    int status, accepted, row, mode;  // mode 0: token fixed; 1: residual draw; 2: bonus draw
    int token, argmax;                // argmax: the draw row's target argmax (the draw of a zero total)
    float Mp, Mq, c2;                 // the draw row's maxima and 1/T scale
    float fp;                         // the draw row's float sums (fq below)
    u64 zp, zq;                       // the draw row's mass sums
    int j0, j1, pending;              // rows j0..j1 of the sequence need exact sums (pending)
    float fq;
};

// the exact pass, per sub-tile of a draw row: sums of the masses of the tokens whose residual weight is
// certainly Ep Zq - Eq Zp (A: Ep, B: Eq; the bonus draw: A alone)
struct SubRec {
    u64 A, B;
};
// and per block, its undecided tokens: masses and sub-tile
struct AmbRec {
    u64 ep, eq;
    u32 p, pad;
};
constexpr int AMB_CAP = 128;       // undecided tokens a block of the exact pass keeps
constexpr int AMB_SEQ_CAP = 1024;  // and a sequence's list holds (beyond either, the draw kernel draws)

struct SpecWs {
    unsigned* row_counters;  // [R]
    unsigned* seq_counters;  // [n_seq] (launch 2)
    unsigned* draw_counters; // [n_seq] (launch 3)
    u64* maxparts;           // [R][S][2]
    unsigned* nanparts;      // [R][S]
    u64* sumparts;           // [R][S][2]
    RowInfo* rows;           // [R]
    SeqInfo* seqs;           // [n_seq]
    u128* wparts;            // [n_seq][tiles][NWD]: the draw's sub-tile weights
    u64* zparts;             // [R][SZ][2]: the exact sums, per block of the exact pass (or per row block)
    SubRec* subrecs;         // [n_seq][tiles][NWD]: the exact pass's sub-tile sums for the draw
    AmbRec* ambs;            // [n_seq][AMB_SEQ_CAP]: its undecided tokens (counted in draw_counters, zero after)
    unsigned* fstate;        // [n_seq]: whether the row blocks swept the draw row themselves (FS_*; zero after)
};

// The row kernel's blocks of a sequence sweep its draw row themselves once the sequence is decided, instead of the exact
// pass's grid: the deciding block publishes FS_GO or FS_NO, and a block that waits past its time limit claims
// FS_GIVEN_UP, after which the exact pass does the sweep. Whoever moves the word from FS_OPEN first decides, so the
// sequence's blocks all sweep or none do.
constexpr unsigned FS_OPEN = 0, FS_GO = 1, FS_NO = 2, FS_GIVEN_UP = 3;
constexpr int FAMB_CAP = 256;  // undecided tokens a row block keeps while it sweeps

// The counters that must be zero between launches sit at fixed offsets in the first SPEC_CTL_BYTES (room for 65535
// rows and sequences, whatever this launch's shape); every launch leaves them zero. The rest is written before it is
// read, so a workspace cleared once serves launches of any shape.
constexpr size_t SPEC_CTL_BYTES = 4 * (size_t)65536 * 4;

struct Plan {
    int R, S, S3, tpb, SZ, F;  // F: blocks of the row pass per sequence
    size_t bytes;
};

Plan plan(int n_seq, int width, int vocab) {
    Plan p;
    p.R = n_seq * (width + 1);
    p.S = splits_for(p.R, vocab);
    // the draw: tiles per block (tpb), then the blocks per sequence that cover every tile
    const int tiles = (vocab + TILE - 1) / TILE;
    int want = (DRAW_BLOCKS + n_seq - 1) / n_seq;
    want = want < 1 ? 1 : (want > tiles ? tiles : want);
    p.tpb = (tiles + want - 1) / want;
    p.S3 = (tiles + p.tpb - 1) / p.tpb;
    // per-block exact sums per row: one per block of the exact pass's grid, or per row of a sequence (the row blocks')
    p.F = (p.R >= ROWS_KERNEL_MIN ? 1 : p.S) * (width + 1);
    p.SZ = p.S3 > p.F ? p.S3 : p.F;
    p.bytes = SPEC_CTL_BYTES + align256((size_t)p.R * p.S * 16) + align256((size_t)p.R * p.S * 4) + align256((size_t)p.R * p.S * 16) +
              align256((size_t)p.R * sizeof(RowInfo)) + align256((size_t)n_seq * sizeof(SeqInfo)) +
              align256((size_t)n_seq * tiles * NWD * 16) + align256((size_t)p.R * p.SZ * 16) +
              align256((size_t)n_seq * tiles * NWD * sizeof(SubRec)) + align256((size_t)n_seq * AMB_SEQ_CAP * sizeof(AmbRec));
    return p;
}

SpecWs carve(void* ws, int n_seq, int vocab, const Plan& p) {
    char* c = (char*)ws;
    SpecWs w;
    w.row_counters = (unsigned*)c; c += (size_t)65536 * 4;
    w.seq_counters = (unsigned*)c; c += (size_t)65536 * 4;
    w.draw_counters = (unsigned*)c; c += (size_t)65536 * 4;
    w.fstate = (unsigned*)c; c += (size_t)65536 * 4;
    w.maxparts = (u64*)c; c += align256((size_t)p.R * p.S * 16);
    w.nanparts = (unsigned*)c; c += align256((size_t)p.R * p.S * 4);
    w.sumparts = (u64*)c; c += align256((size_t)p.R * p.S * 16);
    w.rows = (RowInfo*)c; c += align256((size_t)p.R * sizeof(RowInfo));
    w.seqs = (SeqInfo*)c; c += align256((size_t)n_seq * sizeof(SeqInfo));
    w.wparts = (u128*)c; c += align256((size_t)n_seq * ((vocab + TILE - 1) / TILE) * NWD * 16);
    w.zparts = (u64*)c; c += align256((size_t)p.R * p.SZ * 16);
    w.subrecs = (SubRec*)c; c += align256((size_t)n_seq * ((vocab + TILE - 1) / TILE) * NWD * sizeof(SubRec));
    w.ambs = (AmbRec*)c;
    return w;
}

// Buffer resource over `bytes` bytes at `base`: a load at or past the end returns zeros and touches no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, u32 bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Streams elements [lo, hi) of a target row (and of the draft row when `two`) through f(t, d, i), each element once,
// in ascending index order per thread (descending when REV). Elements a thread is handed past `hi` arrive as -inf,
// which no pass counts. vec: rows are 16-byte aligned and lo is a multiple of 4, so a thread reads 4-element groups
// by 16-byte non-temporal loads, U groups of each row in flight; otherwise it reads single elements.
template <bool REV, int NTH = NT, class F>
__device__ __forceinline__ void stream_rows(const float* tr, const float* dr, bool two, int vocab, int lo, int hi, bool vec, F&& f) {
    constexpr int GSTEP = NTH * 4, ISTEP = GSTEP * U;
    const int tid = (int)threadIdx.x;
    if (!vec) {
        for (int i = lo + tid; i < hi; i += NTH) f(tr[i], two ? dr[i] : -INFINITY, i);
        return;
    }
    const __amdgpu_buffer_rsrc_t rt = rsrc(tr, (u32)vocab * 4u), rd = rsrc(two ? dr : tr, (u32)vocab * 4u);
    const int nit = (hi - lo + ISTEP - 1) / ISTEP;
    auto base_of = [&](int k) { return lo + (REV ? nit - 1 - k : k) * ISTEP + tid * 4; };
    auto issue = [&](int base, u32x4 (&t)[U], u32x4 (&d)[U]) {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const u32 off = (u32)(base + j * GSTEP) * 4u;
            t[j] = __builtin_amdgcn_raw_buffer_load_b128(rt, off, 0, REV ? GBS_SPEC_AUX_REV : GBS_SPEC_AUX_FWD);
            if (two) d[j] = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, REV ? GBS_SPEC_AUX_REV : GBS_SPEC_AUX_FWD);
        }
    };
#if GBS_SPEC_PIPE
    u32x4 tn[U], dn[U];
    if (nit > 0) issue(base_of(0), tn, dn);
#endif
    for (int k = 0; k < nit; ++k) {
        const int base = base_of(k);
        u32x4 t[U], d[U];
#if GBS_SPEC_PIPE
#pragma unroll
        for (int j = 0; j < U; ++j) {
            t[j] = tn[j];
            d[j] = dn[j];
        }
        if (k + 1 < nit) issue(base_of(k + 1), tn, dn);
#else
        issue(base, t, d);
#endif
#pragma unroll
        for (int jj = 0; jj < U; ++jj) {
            const int j = REV ? U - 1 - jj : jj;
            const int e = base + j * GSTEP;
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int q = REV ? 3 - qq : qq;
                const bool in = e + q < hi;
                const float tv = in ? __uint_as_float(t[j][q]) : -INFINITY;
                const float dv = (two && in) ? __uint_as_float(d[j][q]) : -INFINITY;
                f(tv, dv, e + q);
            }
        }
    }
}

__device__ __forceinline__ u64 max_key(float v, int i) { return (v != v || v == -INFINITY) ? 0ull : make_key(okey_f32(v), (u32)i); }

__device__ __forceinline__ RowInfo load_row(const RowInfo* rows, int r) {
    RowInfo ri;
    ri.tkey = ld_agent(&rows[r].tkey);
    ri.dkey = ld_agent(&rows[r].dkey);
    ri.nan = ld_agent(&rows[r].nan);
    return ri;
}

__device__ __forceinline__ void store_seq(SeqInfo* seqs, int s, const SeqInfo& v) {
    st_agent(&seqs[s].status, v.status);
    st_agent(&seqs[s].accepted, v.accepted);
    st_agent(&seqs[s].row, v.row);
    st_agent(&seqs[s].mode, v.mode);
    st_agent(&seqs[s].token, v.token);
    st_agent(&seqs[s].argmax, v.argmax);
    st_agent((u32*)&seqs[s].Mp, __float_as_uint(v.Mp));
    st_agent((u32*)&seqs[s].Mq, __float_as_uint(v.Mq));
    st_agent((u32*)&seqs[s].c2, __float_as_uint(v.c2));
    st_agent(&seqs[s].zp, v.zp);
    st_agent(&seqs[s].zq, v.zq);
}

// a value every lane of the wave holds, moved to a scalar register (so that buffer resources and branches built from it
// are uniform)
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ unsigned uni(unsigned v) { return (unsigned)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ u64 uni(u64 v) { return ((u64)uni((unsigned)(v >> 32)) << 32) | uni((unsigned)v); }

// the row's record, read by every thread of a block and held in scalar registers
__device__ __forceinline__ RowInfo load_row_uniform(const RowInfo* rows, int r) {
    RowInfo ri = load_row(rows, r);
    ri.tkey = uni(ri.tkey);
    ri.dkey = uni(ri.dkey);
    ri.nan = uni(ri.nan);
    return ri;
}

__device__ __forceinline__ SeqInfo load_seq(const SeqInfo* seqs, int s) {
    SeqInfo v{};
    v.status = uni(ld_agent(&seqs[s].status));
    v.accepted = uni(ld_agent(&seqs[s].accepted));
    v.row = uni(ld_agent(&seqs[s].row));
    v.mode = uni(ld_agent(&seqs[s].mode));
    v.token = uni(ld_agent(&seqs[s].token));
    v.argmax = uni(ld_agent(&seqs[s].argmax));
    v.Mp = __uint_as_float(uni(ld_agent((const u32*)&seqs[s].Mp)));
    v.Mq = __uint_as_float(uni(ld_agent((const u32*)&seqs[s].Mq)));
    v.c2 = __uint_as_float(uni(ld_agent((const u32*)&seqs[s].c2)));
    v.fp = __uint_as_float(uni(ld_agent((const u32*)&seqs[s].fp)));
    v.fq = __uint_as_float(uni(ld_agent((const u32*)&seqs[s].fq)));
    v.zp = uni(ld_agent(&seqs[s].zp));
    v.zq = uni(ld_agent(&seqs[s].zq));
    return v;
}

__device__ __forceinline__ u128 load_u128(const u128* p) {
    const u64 lo = ld_agent((const u64*)p), hi = ld_agent((const u64*)p + 1);
    return ((u128)hi << 64) | lo;
}

__device__ __forceinline__ bool temp_ok(float t) { return isfinite(t) && t >= 0.0f; }

// floor(u * a) < b, exactly
__device__ __forceinline__ bool accept_test(float u, u128 a, u128 b) { return mul_floor(u, a, nullptr) < b; }

__device__ __forceinline__ float key_value(u64 k) { return okey_to_f32(key_ok(k)); }

// the mass of a token of logit l in a row of maximum M; FAST: mass_fast's preconditions hold for the row
template <bool FAST>
__device__ __forceinline__ u64 row_mass(float l, float M, float c2) {
    if (FAST) return mass_fast(l, M, c2);
    return l > -INFINITY ? mass(l, M, c2) : 0ull;
}

// residual (mode 1) or bonus (mode 2) weight of a token of target logit t and draft logit d
template <bool FAST = false>
__device__ __forceinline__ u128 pair_weight(int mode, float t, float d, float Mp, float Mq, float c2, u64 zp, u64 zq) {
    const u64 ep = row_mass<FAST>(t, Mp, c2);
    if (mode == 2) return (u128)ep;
    const u64 eq = row_mass<FAST>(d, Mq, c2);
    const u128 a = (u128)ep * zq, b = (u128)eq * zp;
    return a > b ? a - b : (u128)0;
}


// sum of a u128 over the wave, in every lane (cross-lane moves by DPP and permlane swaps)
__device__ __forceinline__ u128 wave_sum_u128(u128 v) {
    u64 lo = (u64)v, hi = (u64)(v >> 64);
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) {
        const u64 olo = xor_lane64(lo, m), ohi = xor_lane64(hi, m);
        const u64 s = lo + olo;
        hi = hi + ohi + (s < lo ? 1ull : 0ull);
        lo = s;
    }
    return ((u128)hi << 64) | lo;
}

// ---- the row pass, for many rows: one block per row ----
// The block reads its target and draft row once. Besides the maxima and the NaN flag it sums 2^((l - M) c2) in float
// (per thread against a running maximum, rescaled to the row's maximum at the end). That float sum F bounds the exact
// mass sum: Z = sum of mass(l) with mass(l) = floor(2^44 2^y) for y the float (l - M) c2 (n <= -52 or y < -64 give 0),
// so 2^44 F (1 - e) - V <= Z <= 2^44 F (1 + e) + V, where e bounds the relative error of F against the exact
// sum of 2^y (the exponent's rounding, 2^-23 |y| per element, the exponential's, each rescaling's and each addition's,
// in all below 2^-14 for rows of up to 2^18 elements) and V (one unit of truncation per element) the truncations.
// The test of a draft decides from these bounds when they do not straddle the boundary floor(u Eq Zp) < Ep Zq;
// otherwise (and where the bounds need finite M and c2) it is left open. The block that completes a sequence's last
// row decides what it can: a first rejection or the bonus row without an open test before it is final; the rows from
// the first open test to the first certain rejection (or the bonus row) get exact sums from spec_exact_k, which
// then decides the sequence. The draw needs its row's exact sums in every case, so a sequence drawing at T > 0 always
// has one row in the exact pass.
#ifndef GBS_SPEC_RNT
#define GBS_SPEC_RNT 1024
#endif
constexpr int RNT = GBS_SPEC_RNT;  // threads of the one-block-per-row kernel
constexpr double ACC_REL = 1.0 / 2048.0;  // e above: eight times the largest relative error of the float sums

template <int NTH>
__device__ __forceinline__ u64 block_max_u64(u64 v, u64* s) {
    const int w = (int)threadIdx.x / WAVE, l = lane_id();
    v = wave_max_u64(v);
    if (l == 0) s[w] = v;
    __syncthreads();
    u64 r = 0;
#pragma unroll
    for (int k = 0; k < NTH / WAVE; ++k) r = s[k] > r ? s[k] : r;
    __syncthreads();
    return r;
}

template <int NTH>
__device__ __forceinline__ u64 block_sum_u64(u64 v, u64* s) {
    const int w = (int)threadIdx.x / WAVE, l = lane_id();
    v = wave_sum_u64(v);
    if (l == 0) s[w] = v;
    __syncthreads();
    u64 r = 0;
#pragma unroll
    for (int k = 0; k < NTH / WAVE; ++k) r += s[k];
    __syncthreads();
    return r;
}

template <int NTH>
__device__ __forceinline__ float block_sum_f32(float v, float* s) {
    const int w = (int)threadIdx.x / WAVE, l = lane_id();
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) v += __uint_as_float(xor_lane(__float_as_uint(v), m));
    if (l == 0) s[w] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int k = 0; k < NTH / WAVE; ++k) r += s[k];
    __syncthreads();
    return r;
}

// The draft's test from float sums Fp, Fq of the rows (ACC_YES: floor(u Eq Zp) < Ep Zq for every Zp, Zq the bounds
// allow; ACC_NO: for none; else ACC_OPEN). Ep = 0 always rejects and Eq = 0 (with Ep > 0) always accepts, since Zq >= 2^44.
__device__ __forceinline__ unsigned accept_bounds(float u, u64 ep, u64 eq, float fp, float fq, int vocab) {
    if (ep == 0ull) return ACC_NO;
    if (eq == 0ull) return ACC_YES;
    if (!(isfinite(fp) && isfinite(fq) && fp >= 1.0f && fq >= 1.0f)) return ACC_OPEN;
    const double one = 17592186044416.0;  // 2^44: the maximum's mass, and a lower bound of every sum
    const double V = (double)vocab;
    const double hp = (double)fp * one * (1.0 + ACC_REL) + V, hq = (double)fq * one * (1.0 + ACC_REL) + V;
    const double lp = fmax((double)fp * one * (1.0 - ACC_REL) - V, one), lq = fmax((double)fq * one * (1.0 - ACC_REL) - V, one);
    const double ud = (double)u, epd = (double)ep, eqd = (double)eq;
    constexpr double R = 1.0 / 1099511627776.0;  // 2^-40, over the doubles' rounding
    // floor(u Eq Zp) <= u Eq Zp <= u Eq hp < Ep lq <= Ep Zq
    if (ud * eqd * hp * (1.0 + R) < epd * lq * (1.0 - R)) return ACC_YES;
    // floor(u Eq Zp) >= floor(u Eq lp) >= Ep hq + 1 > Ep Zq when u Eq lp - 1 >= Ep hq
    if (ud * eqd * lp * (1.0 - R) - 1.0 >= epd * hq * (1.0 + R)) return ACC_NO;
    return ACC_OPEN;
}

// The draw row's float sums bound its exact mass sums (as accept_bounds takes them) when both are finite and >= 1
__device__ __forceinline__ bool ratio_bounds_ok(float fp, float fq) { return isfinite(fp) && isfinite(fq) && fp >= 1.0f && fq >= 1.0f; }

// Bounds on Zp / Zq from those sums: a token with Ep / Eq >= hi has the residual weight Ep Zq - Eq Zp, one with
// Ep / Eq <= lo has none
__device__ __forceinline__ void ratio_bounds(float fp, float fq, int vocab, float& hi, float& lo) {
    const double one = 17592186044416.0, V = (double)vocab;
    const double hp = (double)fp * one * (1.0 + ACC_REL) + V, hq = (double)fq * one * (1.0 + ACC_REL) + V;
    const double lp = fmax((double)fp * one * (1.0 - ACC_REL) - V, one), lq = fmax((double)fq * one * (1.0 - ACC_REL) - V, one);
    hi = (float)(hp / lq);
    lo = (float)(lp / hq);
}

// A row's inputs to its check: its temperature, and for a draft row its uniform, token and the two logits of the token
struct RowArgs {
    float T, u, tx, dx;
    int x;
    bool ures_ok;  // the sequence's resampling uniform is in [0, 1) (checked with row 0)
};

__device__ __forceinline__ RowArgs row_args(int seq, int j, int width, int vocab, long long stride, const float* __restrict__ target,
                                            const float* __restrict__ draft, const int* __restrict__ draft_ids, const float* __restrict__ temps,
                                            const float* __restrict__ u_accept, const float* __restrict__ u_resample) {
    const int r = seq * (width + 1) + j;
    RowArgs a;
    a.T = temps[r];
    a.ures_ok = true;
    if (j == 0) {
        const float ur = u_resample[seq];
        a.ures_ok = ur >= 0.0f && ur < 1.0f;
    }
    a.u = 0.0f;
    a.x = 0;
    a.tx = a.dx = -INFINITY;
    if (j < width) {
        a.u = u_accept[(size_t)seq * width + j];
        a.x = draft_ids[(size_t)seq * width + j];
        if (a.x >= 0 && a.x < vocab) {
            a.tx = target[(size_t)r * (size_t)stride + a.x];
            a.dx = draft[(size_t)r * (size_t)stride + a.x];
        }
    }
    return a;
}

// Row r (row j of its sequence): its parameters and flags, and for a draft the test by the float bounds (its state and
// the token's masses are stored in the row's record). Returns state | flags << 4 (flags: 1 invalid parameter, 2 NaN,
// 4 no candidate).
__device__ __forceinline__ unsigned row_check(int r, int j, int width, int vocab, const RowArgs& a, const RowInfo& ri, float fp, float fq,
                                              SpecWs ws) {
    const float Tj = a.T;
    bool bad = !temp_ok(Tj) || !a.ures_ok;
    unsigned state = ACC_NO;
    if (j < width) {
        const float u = a.u;
        const int x = a.x;
        bad |= !(u >= 0.0f && u < 1.0f) || x < 0 || x >= vocab;
        if (!bad && !ri.nan && ri.tkey != 0ull && ri.dkey != 0ull) {
            if (Tj == 0.0f) state = x == (int)key_id(ri.tkey) ? ACC_YES : ACC_NO;
            else {
                const float cj = temp_scale(Tj);
                const float Mp = key_value(ri.tkey), Mq = key_value(ri.dkey);
                const u64 ep = a.tx > -INFINITY ? mass(a.tx, Mp, cj) : 0ull;
                const u64 eq = a.dx > -INFINITY ? mass(a.dx, Mq, cj) : 0ull;
                state = (mass_fast_ok(Mp, cj) && mass_fast_ok(Mq, cj)) ? accept_bounds(u, ep, eq, fp, fq, vocab) : ACC_OPEN;
                st_agent(&ws.rows[r].ep, ep);
                st_agent(&ws.rows[r].eq, eq);
            }
        }
        st_agent(&ws.rows[r].state, state);
    }
    unsigned f = bad ? 1u : 0u;
    f |= ri.nan != 0u ? 2u : 0u;
    f |= (ri.tkey == 0ull || (j < width && ri.dkey == 0ull)) ? 4u : 0u;
    return state | f << 4;
}

// The sequence's decisions, by the block that completes the sequence's last row. Thread j checks row j (its
// parameters, flags and the draft's bounded test; pretested: the row block checked it already). The first row whose
// test is not ACC_YES is j0, the first ACC_NO (or the bonus row) j1. With j0 == j1 the accepted count is final; the draw then needs row j1's exact sums
// (pending), unless its temperature is 0. With j0 < j1 the tests from j0 on wait for exact sums (pending).
// Returns, on thread 0, whether the draw row's sweep can run in the exact pass's one-read form with the fast masses
// (the row blocks may then sweep it themselves).
__device__ bool decide_rows(int seq, int width, int vocab, long long stride, const float* __restrict__ target, const float* __restrict__ draft,
                            const int* __restrict__ draft_ids, const float* __restrict__ temps, const float* __restrict__ u_accept,
                            const float* __restrict__ u_resample, SpecWs ws, bool pretested) {
    const int W1 = width + 1;
    __shared__ int s_all, s_first, s_rej;
    if (threadIdx.x == 0) {
        s_all = 0;
        s_first = width;
        s_rej = width;
    }
    __syncthreads();
    const int r0 = seq * W1;
    for (int j = (int)threadIdx.x; j <= width; j += (int)blockDim.x) {
        unsigned c;
        if (pretested) {
            c = ld_agent(&ws.rows[r0 + j].check);
        } else {
            const RowArgs a = row_args(seq, j, width, vocab, stride, target, draft, draft_ids, temps, u_accept, u_resample);
            const float fp = ld_agent((const float*)&ws.rows[r0 + j].fp), fq = ld_agent((const float*)&ws.rows[r0 + j].fq);
            c = row_check(r0 + j, j, width, vocab, a, load_row(ws.rows, r0 + j), fp, fq, ws);
        }
        const unsigned state = c & 15u;
        const int f = (int)(c >> 4);
        if (j < width) {
            if (state != ACC_YES) atomicMin(&s_first, j);
            if (state == ACC_NO) atomicMin(&s_rej, j);
        }
        if (f) atomicOr(&s_all, f);
    }
    __syncthreads();
    if (threadIdx.x != 0) return false;
    SeqInfo si{};
    si.status = GBS_ROW_OK;
    const int all = s_all;
    if (all & 1) si.status = GBS_ROW_INVALID_PARAMS;
    else if (all & 2) si.status = GBS_ROW_NAN_LOGIT;
    else if (all & 4) si.status = GBS_ROW_NO_CANDIDATES;
    if (si.status == GBS_ROW_OK) {
        si.j0 = s_first;
        si.j1 = s_rej;
        const int k = si.j0;
        const RowInfo ri = load_row(ws.rows, r0 + k);
        const float Tk = temps[r0 + k];
        if (si.j0 == si.j1) {  // the accepted count is final: row k's record, without its sums at T > 0
            si.accepted = k;
            si.row = r0 + k;
            si.argmax = (int)key_id(ri.tkey);
            si.mode = Tk == 0.0f ? 0 : (k < width ? 1 : 2);
            si.token = Tk == 0.0f ? si.argmax : -1;
            if (Tk != 0.0f) {
                si.Mp = key_value(ri.tkey);
                si.Mq = k < width ? key_value(ri.dkey) : si.Mp;
                si.c2 = temp_scale(Tk);
                si.fp = ld_agent((const float*)&ws.rows[r0 + k].fp);
                si.fq = ld_agent((const float*)&ws.rows[r0 + k].fq);
            }
        }
        si.pending = (si.j0 != si.j1 || Tk != 0.0f) ? 1 : 0;
    }
    store_seq(ws.seqs, seq, si);
    st_agent(&ws.seqs[seq].j0, si.j0);
    st_agent(&ws.seqs[seq].j1, si.j1);
    st_agent(&ws.seqs[seq].pending, si.pending);
    st_agent((u32*)&ws.seqs[seq].fp, __float_as_uint(si.fp));
    st_agent((u32*)&ws.seqs[seq].fq, __float_as_uint(si.fq));
    if (si.status != GBS_ROW_OK || si.pending == 0 || si.j0 != si.j1 || si.mode == 0) return false;
    const bool fast = mass_fast_ok(si.Mp, si.c2) && mass_fast_ok(si.Mq, si.c2);
    return fast && (si.mode == 2 || ratio_bounds_ok(si.fp, si.fq));
}

// Streams elements [lo, hi) of a target row (and of the draft row when `two`) through g(t, d, i0) by 4-element groups
// t[q], d[q] of elements i0 + q, each element once and each thread's groups in ascending index order; elements past
// `hi` arrive as -inf. vec as for stream_rows; otherwise each element is a group of its own (the rest -inf).
template <int NTH, class G>
__device__ __forceinline__ void stream_groups(const float* tr, const float* dr, bool two, int vocab, int lo, int hi, bool vec, G&& g) {
    constexpr int GSTEP = NTH * 4, ISTEP = GSTEP * U;
    const int tid = (int)threadIdx.x;
    if (!vec) {
        for (int i = lo + tid; i < hi; i += NTH) {
            const float t[4] = {tr[i], -INFINITY, -INFINITY, -INFINITY};
            const float d[4] = {two ? dr[i] : -INFINITY, -INFINITY, -INFINITY, -INFINITY};
            g(t, d, i);
        }
        return;
    }
    const __amdgpu_buffer_rsrc_t rt = rsrc(tr, (u32)vocab * 4u), rd = rsrc(two ? dr : tr, (u32)vocab * 4u);
    const int nit = (hi - lo + ISTEP - 1) / ISTEP;
    auto issue = [&](int base, u32x4 (&t)[U], u32x4 (&d)[U]) {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const u32 off = (u32)(base + j * GSTEP) * 4u;
            t[j] = __builtin_amdgcn_raw_buffer_load_b128(rt, off, 0, GBS_SPEC_AUX_FWD);
            if (two) d[j] = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, GBS_SPEC_AUX_FWD);
        }
    };
    u32x4 tn[U], dn[U];
    if (nit > 0) issue(lo + tid * 4, tn, dn);
    for (int k = 0; k < nit; ++k) {
        const int base = lo + k * ISTEP + tid * 4;
        u32x4 t[U], d[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            t[j] = tn[j];
            d[j] = dn[j];
        }
        if (k + 1 < nit) issue(base + ISTEP, tn, dn);
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int e = base + j * GSTEP;
            float tv[4], dv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool in = e + q < hi;
                tv[q] = in ? __uint_as_float(t[j][q]) : -INFINITY;
                dv[q] = (two && in) ? __uint_as_float(d[j][q]) : -INFINITY;
            }
            g(tv, dv, e);
        }
    }
}

// The row pass of one thread: the target's largest value and its first index (a strict > over ascending indices keeps
// the first of equal values, -0 and +0 included; NaN and -inf never replace -inf), the draft's largest value, the NaN
// flag and, when DRAW, the float sums of 2^((v - m) c2) against running maxima m (starting at -FLT_MAX, so that -inf
// adds exp2(-inf) = 0). A group whose largest value exceeds a running maximum (rare past a row's first groups) takes a
// wave-uniform branch that updates the maxima element by element and rescales the sums by 2^((m_old - m_new) c2);
// then every term's exponent is <= 0.
template <bool DRAW, int NTH>
__device__ __forceinline__ void rows_sweep(const float* tr, const float* dr, bool has_draft, int vocab, int lo, int hi, bool vec, float c2,
                                           float& tm, int& ti, float& dm, bool& nanf, float& om_t, float& s_t, float& om_d, float& s_d) {
    stream_groups<NTH>(tr, dr, has_draft, vocab, lo, hi, vec, [&](const float (&t)[4], const float (&d)[4], int i0) {
        bool un = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) un |= __builtin_isunordered(t[q], d[q]);
        nanf |= un;
        const float gt = fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]));
        const float gd = fmaxf(fmaxf(d[0], d[1]), fmaxf(d[2], d[3]));
        dm = fmaxf(dm, gd);
        const bool up = gt > tm || (DRAW && (gt > om_t || gd > om_d));
        if (ballot(up) != 0ull) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                ti = t[q] > tm ? i0 + q : ti;
                tm = t[q] > tm ? t[q] : tm;
            }
            if (DRAW) {
                const float nt = fmaxf(om_t, gt), nd = fmaxf(om_d, gd);
                s_t = nt > om_t ? s_t * __builtin_amdgcn_exp2f((om_t - nt) * c2) : s_t;
                s_d = nd > om_d ? s_d * __builtin_amdgcn_exp2f((om_d - nd) * c2) : s_d;
                om_t = nt;
                om_d = nd;
            }
        }
        if (DRAW) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                s_t += __builtin_amdgcn_exp2f((t[q] - om_t) * c2);
                s_d += __builtin_amdgcn_exp2f((d[q] - om_d) * c2);
            }
        }
    });
}

template <int MODE, bool FAST, int CAP, bool PRE = true>
__device__ __forceinline__ void exact_subtiles(const float* tr, const float* dr, int vocab, int p0, int step, int p1, bool vec, float Mp, float Mq,
                                               float c2, float rho_hi, float rho_lo, SubRec* recs, AmbRec* s_amb, unsigned* s_namb, u64& zp,
                                               u64& zq);

constexpr long long FUSE_WAIT_TICKS = 10000;  // a row block's wait for its sequence's decision: 100 us of the 100 MHz clock
long long g_fuse_wait = FUSE_WAIT_TICKS;     // the limit the launches pass (gbs_spec_set_fuse_wait)

// The sequence's sweep of its draw row by the row pass's own blocks, once the sequence is decided (every block of the
// launch resident at once): block blk of the sequence's nblk takes its share of the draw row's sub-tiles, one per wave
// at a time, and writes the exact pass's per-block sums at [row][blk] of zparts (sz per row), the sub-tile sums and
// the list of undecided tokens. The decider publishes the sequence's state word (FS_GO when go), the other blocks wait
// for it at most wait_ticks, and give up past that; whoever moves the word from FS_OPEN first decides.
template <int NTH>
__device__ void coop_sweep(bool decider, bool go, int seq, int blk, int nblk, int vocab, long long stride, bool vec, const float* target,
                           const float* draft, SpecWs ws, int sz, long long wait_ticks) {
    __shared__ u64 s_red[NTH / WAVE];
    __shared__ unsigned s_flag, s_go, s_namb;
    __shared__ AmbRec s_amb[FAMB_CAP];
    if (threadIdx.x == 0) {
        unsigned* word = &ws.fstate[seq];
        unsigned v;
        if (decider) {
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);  // the sequence's record has been stored
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            unsigned expect = FS_OPEN;
            const bool set = __hip_atomic_compare_exchange_strong(word, &expect, go ? FS_GO : FS_NO, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                                  __HIP_MEMORY_SCOPE_AGENT);
            v = set ? (go ? FS_GO : FS_NO) : expect;
        } else {
            const long long t_end = (long long)wall_clock64() + wait_ticks;
            while ((v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == FS_OPEN) {
                if ((long long)wall_clock64() > t_end) {
                    unsigned expect = FS_OPEN;
                    const bool set = __hip_atomic_compare_exchange_strong(word, &expect, FS_GIVEN_UP, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                                          __HIP_MEMORY_SCOPE_AGENT);
                    v = set ? FS_GIVEN_UP : expect;
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
        }
        s_go = v == FS_GO ? 1u : 0u;
        s_namb = 0u;
    }
    __syncthreads();
    if (!s_go) return;
    // this block's share of the draw row's sub-tiles, one per wave at a time
    const SeqInfo si = load_seq(ws.seqs, seq);
    const int nsub = (vocab + TILE - 1) / TILE * NWD;
    const int per = (nsub + nblk - 1) / nblk;
    const int pb = min(nsub, blk * per), pe = min(nsub, pb + per);
    const int p0 = pb + (int)threadIdx.x / WAVE;
    const float* tq = target + (size_t)si.row * (size_t)stride;
    const float* dq = draft + (size_t)si.row * (size_t)stride;
    SubRec* recs = ws.subrecs + (size_t)seq * nsub;
    u64 zp = 0, zq = 0;
    if (si.mode == 1) {
        float hi, lo;
        ratio_bounds(si.fp, si.fq, vocab, hi, lo);
        exact_subtiles<1, true, FAMB_CAP, (NTH > NT)>(tq, dq, vocab, p0, NTH / WAVE, pe, vec, si.Mp, si.Mq, si.c2, hi, lo, recs, s_amb, &s_namb, zp, zq);
    } else {
        exact_subtiles<2, true, FAMB_CAP, (NTH > NT)>(tq, dq, vocab, p0, NTH / WAVE, pe, vec, si.Mp, si.Mq, si.c2, 0.0f, 0.0f, recs, s_amb, &s_namb, zp, zq);
    }
    zp = block_sum_u64<NTH>(zp, s_red);  // (its barriers also publish s_namb and s_amb)
    zq = block_sum_u64<NTH>(zq, s_red);
    const unsigned nb = s_namb < (unsigned)FAMB_CAP ? s_namb : (unsigned)FAMB_CAP;
    if (threadIdx.x == 0) {
        st_agent(&ws.zparts[((size_t)si.row * sz + blk) * 2], zp);
        st_agent(&ws.zparts[((size_t)si.row * sz + blk) * 2 + 1], zq);
        s_flag = s_namb != 0u ? atomicAdd(&ws.draw_counters[seq], s_namb > (unsigned)FAMB_CAP ? (unsigned)AMB_SEQ_CAP + 1u : s_namb) : 0u;
    }
    __syncthreads();
    AmbRec* list = ws.ambs + (size_t)seq * AMB_SEQ_CAP;
    for (unsigned i = threadIdx.x; i < nb; i += NTH) {
        if (s_flag + i < (unsigned)AMB_SEQ_CAP) {
            st_agent(&list[s_flag + i].ep, s_amb[i].ep);
            st_agent(&list[s_flag + i].eq, s_amb[i].eq);
            st_agent(&list[s_flag + i].p, s_amb[i].p);
        }
    }
}

// fuse: the row blocks sweep their sequence's draw row once it is decided (coop_sweep)
__global__ void __launch_bounds__(RNT) spec_rows_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab, long long stride,
                                                   bool vec, const int* __restrict__ draft_ids, const float* __restrict__ temps,
                                                   const float* __restrict__ u_accept, const float* __restrict__ u_resample, SpecWs ws,
                                                   bool fuse, int sz, long long wait_ticks) {
    __shared__ u64 s_red[RNT / WAVE];
    __shared__ float s_redf[RNT / WAVE];
    __shared__ unsigned s_flag;
    const int r = blockIdx.x;
    const int W1 = width + 1;
    const int seq = r / W1;
    const bool has_draft = (r % W1) < width;
    const float* tr = target + (size_t)r * (size_t)stride;
    const float* dr = draft + (size_t)r * (size_t)stride;
    const float T = temps[r];
    const bool draw = temp_ok(T) && T > 0.0f;
    const float c2 = draw ? temp_scale(T) : 0.0f;
    // per thread: the largest value and its first index (elements arrive in ascending index order per thread, and a
    // strict > keeps the first of equal values, -0 and +0 included; NaN and -inf never replace -inf), and at T > 0 the
    // float sums against running maxima
    float tm = -INFINITY, dm = -INFINITY, om_t = -FLT_MAX, om_d = -FLT_MAX, s_t = 0.0f, s_d = 0.0f;
    int ti = 0;
    bool nanf = false;
    if (draw) rows_sweep<true, RNT>(tr, dr, has_draft, vocab, 0, vocab, vec, c2, tm, ti, dm, nanf, om_t, s_t, om_d, s_d);
    else rows_sweep<false, RNT>(tr, dr, has_draft, vocab, 0, vocab, vec, c2, tm, ti, dm, nanf, om_t, s_t, om_d, s_d);
    // the row's own check: its inputs are loaded while the block reduces
    const int j = r - seq * W1;
    RowArgs ra{};
    if (threadIdx.x == 0) ra = row_args(seq, j, width, vocab, stride, target, draft, draft_ids, temps, u_accept, u_resample);
    // the draft's key carries no index (only its maximum's value is used)
    const u64 tkey = block_max_u64<RNT>(tm == -INFINITY ? 0ull : make_key(okey_f32(tm), (u32)ti), s_red);
    const u64 dkey = block_max_u64<RNT>(dm == -INFINITY ? 0ull : make_key(okey_f32(dm), 0u), s_red);
    const bool nan = block_max_u64<RNT>(nanf ? 1ull : 0ull, s_red) != 0ull;
    float fp = 0.0f, fq = 0.0f;
    if (draw && tkey != 0ull && !nan) {
        // each thread's sum rescaled to the row's maximum (a thread that saw no finite value holds 0)
        const float Mp = key_value(tkey), Mq = dkey != 0ull ? key_value(dkey) : Mp;
        fp = block_sum_f32<RNT>(s_t > 0.0f ? s_t * __builtin_amdgcn_exp2f((om_t - Mp) * c2) : 0.0f, s_redf);
        fq = block_sum_f32<RNT>(s_d > 0.0f ? s_d * __builtin_amdgcn_exp2f((om_d - Mq) * c2) : 0.0f, s_redf);
    }
    if (threadIdx.x == 0) {
        st_agent(&ws.rows[r].tkey, tkey);
        st_agent(&ws.rows[r].dkey, dkey);
        st_agent(&ws.rows[r].nan, nan ? 1u : 0u);
        st_agent((u32*)&ws.rows[r].fp, __float_as_uint(fp));
        st_agent((u32*)&ws.rows[r].fq, __float_as_uint(fq));
        RowInfo ri{};
        ri.tkey = tkey;
        ri.dkey = dkey;
        ri.nan = nan ? 1u : 0u;
        st_agent(&ws.rows[r].check, row_check(r, j, width, vocab, ra, ri, fp, fq, ws));
    }
    const bool last = arrive_last(&ws.seq_counters[seq], (unsigned)W1, &s_flag);
    const bool go = last && decide_rows(seq, width, vocab, stride, target, draft, draft_ids, temps, u_accept, u_resample, ws, true);
    if (fuse) coop_sweep<RNT>(last, go, seq, r - seq * W1, W1, vocab, stride, vec, target, draft, ws, sz, wait_ticks);
}

// inclusive prefix sum of a u128 over the wave
__device__ __forceinline__ u128 wave_scan_u128(u128 v) {
    const int l = lane_id();
    u64 lo = (u64)v, hi = (u64)(v >> 64);
#pragma unroll
    for (int m = 1; m < WAVE; m <<= 1) {
        const int src = l >= m ? l - m : l;
        const u64 olo = shfl64(lo, src), ohi = shfl64(hi, src);
        if (l >= m) {
            const u64 s = lo + olo;
            hi = hi + ohi + (s < lo ? 1ull : 0ull);
            lo = s;
        }
    }
    return ((u128)hi << 64) | lo;
}

// exclusive prefix sum of a u128 over the block (thread order) and the block's total; all threads call it.
// s_wt: NT / WAVE entries of LDS, free on entry; free again on return.
__device__ __forceinline__ u128 block_scan_u128(u128 v, u128& total, u128* s_wt) {
    const int w = (int)threadIdx.x / WAVE, l = lane_id();
    const u128 inc = wave_scan_u128(v);
    if (l == WAVE - 1) s_wt[w] = inc;
    __syncthreads();
    u128 off = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < NT / WAVE; ++k) {
        const u128 x = s_wt[k];
        off += k < w ? x : (u128)0;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return off + inc - v;
}

// ---- launch 3: the draw ----
// Grid (blocks per sequence, n_seq). The row that a sequence draws from (its first rejected row: the residual; or its
// last row: the bonus from p) is cut into tiles of TILE elements; block b takes tiles [b * tpb, (b + 1) * tpb), the
// next tile's loads in flight while one is summed. Wave w covers the SUB = 256 DU contiguous elements [w SUB, (w + 1)
// SUB) of a tile (group j of a lane at j * 256 + 4 lane), so the wave sums of (tile, wave) are the weights of
// consecutive SUB-element sub-tiles: sub-tile p = tile * NWD + wave holds elements [SUB p, SUB (p + 1)). The
// sequence's last block finds the sub-tile that holds t = floor(u * total) by a block scan over them, then the element
// by a block scan over the sub-tile (DU elements per thread).
template <int MODE, bool FAST>
__device__ __forceinline__ void draw_tiles(const float* tr, const float* dr, int vocab, int t0, int t1, bool vec, float Mp, float Mq,
                                           float c2, u64 zp, u64 zq, u128* wparts) {
    const int tid = (int)threadIdx.x, w = tid / WAVE, l = lane_id();
    const __amdgpu_buffer_rsrc_t rt = rsrc(tr, (u32)vocab * 4u), rd = rsrc(MODE == 1 ? dr : tr, (u32)vocab * 4u);
    auto issue = [&](int tile, float (&t)[DU * 4], float (&d)[DU * 4]) {
#pragma unroll
        for (int j = 0; j < DU; ++j) {
            const int e = tile * TILE + w * SUB + j * (WAVE * 4) + l * 4;
            if (vec) {
                const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rt, (u32)e * 4u, 0, 2);
                u32x4 b = {0u, 0u, 0u, 0u};
                if (MODE == 1) b = __builtin_amdgcn_raw_buffer_load_b128(rd, (u32)e * 4u, 0, 2);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    t[j * 4 + q] = __uint_as_float(a[q]);
                    d[j * 4 + q] = __uint_as_float(b[q]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    t[j * 4 + q] = e + q < vocab ? tr[e + q] : -INFINITY;
                    d[j * 4 + q] = (MODE == 1 && e + q < vocab) ? dr[e + q] : -INFINITY;
                }
            }
        }
    };
    float tn[DU * 4], dn[DU * 4];
    if (t0 < t1) issue(t0, tn, dn);
    for (int tile = t0; tile < t1; ++tile) {
        float t[DU * 4], d[DU * 4];
#pragma unroll
        for (int i = 0; i < DU * 4; ++i) {
            t[i] = tn[i];
            d[i] = dn[i];
        }
        if (tile + 1 < t1) issue(tile + 1, tn, dn);
        u128 part = 0;
#pragma unroll
        for (int j = 0; j < DU; ++j) {
            const int e = tile * TILE + w * SUB + j * (WAVE * 4) + l * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool in = e + q < vocab;  // buffer loads past the row's end return 0, not -inf
                part += pair_weight<FAST>(MODE, in ? t[j * 4 + q] : -INFINITY, in ? d[j * 4 + q] : -INFINITY, Mp, Mq, c2, zp, zq);
            }
        }
        part = wave_sum_u128(part);
        if (l == 0) {
            u64* o = (u64*)&wparts[(size_t)tile * NWD + w];
            st_agent(o, (u64)part);
            st_agent(o + 1, (u64)(part >> 64));
        }
    }
}

// a sequence's outputs: status, accepted count, the accepted drafts, then the drawn token and -1 after it
__device__ void write_outputs(int seq, const SeqInfo& si, int token, int width, const int* __restrict__ draft_ids, int* __restrict__ out_accepted,
                              int* __restrict__ out_tokens, int* __restrict__ out_status) {
    const int W1 = width + 1;
    if (out_status) out_status[seq] = si.status;
    out_accepted[seq] = si.status == GBS_ROW_OK ? si.accepted : 0;
    for (int j = 0; j < W1; ++j) {
        int v = -1;
        if (si.status == GBS_ROW_OK) {
            if (j < si.accepted) v = draft_ids[(size_t)seq * width + j];
            else if (j == si.accepted) v = token;
        }
        out_tokens[(size_t)seq * W1 + j] = v;
    }
}

// The draw from sub-tile weights: thread k holds the weights of sub-tiles [k SPT, (k + 1) SPT) in sub. A block scan
// finds the sub-tile that holds t = floor(u * total), then a block scan over that sub-tile's elements (DU per thread,
// exact weights) the element. A zero total draws the target's argmax. All threads call it and get the token.
template <int SPT>
__device__ int pick_token(const u128 (&sub)[SPT], int nsub, int vocab, float u, const SeqInfo& si, const float* tr, const float* dr, bool fast,
                          u128* s_wt, u128* s_rem_p, unsigned* s_flag_p, int* s_tok_p) {
    static_assert(NT == WAVE * 4, "a sub-tile (256 elements) is one element per thread");
    u128& s_rem = *s_rem_p;
    unsigned& s_flag = *s_flag_p;
    int& s_tok = *s_tok_p;
    const int tid = (int)threadIdx.x;
    if (tid == 0) {
        s_flag = (unsigned)nsub;  // a zero total selects no sub-tile
        s_tok = si.argmax;        // and draws the target's argmax
    }
    u128 v = 0;
#pragma unroll
    for (int k = 0; k < SPT; ++k) v += sub[k];
    u128 total;
    const u128 ex = block_scan_u128(v, total, s_wt);
    const u128 t = mul_floor(u, total, nullptr);
    if (v != 0 && ex <= t && t - ex < v) {  // this thread's sub-tiles hold t: find which
        u128 before = ex;
        int kk = -1;
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            if (kk < 0) {
                if (t - before < sub[k]) kk = k;
                else before += sub[k];
            }
        }
        s_flag = (unsigned)(tid * SPT + kk);
        s_rem = t - before;
    }
    __syncthreads();
    const int p = (int)s_flag;
    const u128 rem = s_rem;
    // sub-tile p: DU consecutive elements per thread; a block scan of the threads' sums; the element whose range holds
    // rem (selections, no indexing)
    static_assert(SUB == NT * DU, "a sub-tile is DU elements per thread");
    const int e0 = p * SUB + tid * DU;
    u128 we[DU], wsum = 0;
#pragma unroll
    for (int q = 0; q < DU; ++q) {
        const int e = e0 + q;
        const bool in = p < nsub && e < vocab;
        const float te = in ? tr[e] : -INFINITY;
        const float de = (in && si.mode == 1) ? dr[e] : -INFINITY;
        we[q] = fast ? pair_weight<true>(si.mode, te, de, si.Mp, si.Mq, si.c2, si.zp, si.zq)
                     : pair_weight(si.mode, te, de, si.Mp, si.Mq, si.c2, si.zp, si.zq);
        wsum += we[q];
    }
    u128 sub_total;
    const u128 before = block_scan_u128(wsum, sub_total, s_wt);
    if (p < nsub && wsum != 0 && before <= rem && rem - before < wsum) {
        u128 acc = before;
        int qf = -1;
#pragma unroll
        for (int q = 0; q < DU; ++q) {
            const bool hit = qf < 0 && rem - acc < we[q];
            qf = hit ? q : qf;
            acc += qf < 0 ? we[q] : (u128)0;
        }
        s_tok = e0 + qf;
    }
    __syncthreads();
    return s_tok;
}

// ---- the row pass for fewer rows: (splits, rows) ----
// Block sp takes chunk sp of row r: its part of the row pass (maxima, NaN flag and, at T > 0, float sums rescaled to
// the chunk's maximum). The row's last block rescales the chunks' sums to the row's maximum (one more rescaling of
// each term, inside the bound's margin) and writes the row's record; the block that completes a sequence's last row
// decides it as spec_rows_k's does.
__global__ void __launch_bounds__(NT) spec_split_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab,
                                                   long long stride, int chunk, bool vec, const int* __restrict__ draft_ids,
                                                   const float* __restrict__ temps, const float* __restrict__ u_accept,
                                                   const float* __restrict__ u_resample, SpecWs ws, bool fuse, int sz,
                                                   long long wait_ticks) {
    __shared__ u64 s_red[NT / WAVE];
    __shared__ float s_redf[NT / WAVE];
    __shared__ unsigned s_flag;
    const int S = gridDim.x, sp = blockIdx.x, r = blockIdx.y;
    const int W1 = width + 1;
    const int seq = r / W1;
    const bool has_draft = (r % W1) < width;
    const float* tr = target + (size_t)r * (size_t)stride;
    const float* dr = draft + (size_t)r * (size_t)stride;
    const int lo = min(vocab, sp * chunk), hi = min(vocab, lo + chunk);
    const float T = temps[r];
    const bool draw = temp_ok(T) && T > 0.0f;
    const float c2 = draw ? temp_scale(T) : 0.0f;
    float tm = -INFINITY, dm = -INFINITY, om_t = -FLT_MAX, om_d = -FLT_MAX, s_t = 0.0f, s_d = 0.0f;
    int ti = 0;
    bool nanf = false;
    if (draw) rows_sweep<true, NT>(tr, dr, has_draft, vocab, lo, hi, vec, c2, tm, ti, dm, nanf, om_t, s_t, om_d, s_d);
    else rows_sweep<false, NT>(tr, dr, has_draft, vocab, lo, hi, vec, c2, tm, ti, dm, nanf, om_t, s_t, om_d, s_d);
    const u64 tk = block_max_u64<NT>(tm == -INFINITY ? 0ull : make_key(okey_f32(tm), (u32)ti), s_red);
    const u64 dk = block_max_u64<NT>(dm == -INFINITY ? 0ull : make_key(okey_f32(dm), 0u), s_red);
    const bool bn = block_max_u64<NT>(nanf ? 1ull : 0ull, s_red) != 0ull;
    float fp = 0.0f, fq = 0.0f;
    if (draw) {  // the chunk's sums against its own maxima (an empty side sums to 0)
        const float Mp = tk != 0ull ? key_value(tk) : 0.0f, Mq = dk != 0ull ? key_value(dk) : 0.0f;
        fp = block_sum_f32<NT>((tk != 0ull && s_t > 0.0f) ? s_t * __builtin_amdgcn_exp2f((om_t - Mp) * c2) : 0.0f, s_redf);
        fq = block_sum_f32<NT>((dk != 0ull && s_d > 0.0f) ? s_d * __builtin_amdgcn_exp2f((om_d - Mq) * c2) : 0.0f, s_redf);
    }
    if (threadIdx.x == 0) {
        st_agent(&ws.maxparts[((size_t)r * S + sp) * 2], tk);
        st_agent(&ws.maxparts[((size_t)r * S + sp) * 2 + 1], dk);
        st_agent(&ws.nanparts[(size_t)r * S + sp], bn ? 1u : 0u);
        st_agent(&ws.sumparts[((size_t)r * S + sp) * 2], (u64)__float_as_uint(fp));
        st_agent(&ws.sumparts[((size_t)r * S + sp) * 2 + 1], (u64)__float_as_uint(fq));
    }
    const bool row_last = arrive_last(&ws.row_counters[r], (unsigned)S, &s_flag);
    bool seq_last = false, go = false;
    if (row_last) {
        // the row: maxima over the chunks, then each chunk's sums rescaled to them (thread o takes chunks o, o + NT, ...)
        u64 a = 0, b = 0, n = 0;
        for (int o = (int)threadIdx.x; o < S; o += NT) {
            const u64 x = ld_agent(&ws.maxparts[((size_t)r * S + o) * 2]), y = ld_agent(&ws.maxparts[((size_t)r * S + o) * 2 + 1]);
            a = x > a ? x : a;
            b = y > b ? y : b;
            n |= ld_agent(&ws.nanparts[(size_t)r * S + o]);
        }
        a = block_max_u64<NT>(a, s_red);
        b = block_max_u64<NT>(b, s_red);
        n = block_max_u64<NT>(n, s_red);
        if (draw && a != 0ull && n == 0ull) {
            const float Mp = key_value(a), Mq = b != 0ull ? key_value(b) : Mp;
            float xp = 0.0f, xq = 0.0f;
            for (int o = (int)threadIdx.x; o < S; o += NT) {
                const u64 x = ld_agent(&ws.maxparts[((size_t)r * S + o) * 2]), y = ld_agent(&ws.maxparts[((size_t)r * S + o) * 2 + 1]);
                const float gp = __uint_as_float((u32)ld_agent(&ws.sumparts[((size_t)r * S + o) * 2]));
                const float gq = __uint_as_float((u32)ld_agent(&ws.sumparts[((size_t)r * S + o) * 2 + 1]));
                xp += (x != 0ull && gp > 0.0f) ? gp * __builtin_amdgcn_exp2f((key_value(x) - Mp) * c2) : 0.0f;
                xq += (y != 0ull && gq > 0.0f) ? gq * __builtin_amdgcn_exp2f((key_value(y) - Mq) * c2) : 0.0f;
            }
            fp = block_sum_f32<NT>(xp, s_redf);
            fq = block_sum_f32<NT>(xq, s_redf);
        }
        if (threadIdx.x == 0) {
            st_agent(&ws.rows[r].tkey, a);
            st_agent(&ws.rows[r].dkey, b);
            st_agent(&ws.rows[r].nan, (unsigned)n);
            st_agent((u32*)&ws.rows[r].fp, __float_as_uint(fp));
            st_agent((u32*)&ws.rows[r].fq, __float_as_uint(fq));
        }
        seq_last = arrive_last(&ws.seq_counters[seq], (unsigned)W1, &s_flag);
        go = seq_last && decide_rows(seq, width, vocab, stride, target, draft, draft_ids, temps, u_accept, u_resample, ws, false);
    }
    // every chunk block of the sequence sweeps its share of the draw row
    if (fuse) coop_sweep<NT>(seq_last, go, seq, (r - seq * W1) * S + sp, W1 * S, vocab, stride, vec, target, draft, ws, sz, wait_ticks);
}

// ---- the exact pass ----
// Grid (S3, n_seq), the draw's grid. A pending sequence whose accepted count is final (j0 == j1) has one row left,
// the row it draws from; block b takes that row's tiles [b tpb, (b + 1) tpb) in the draw's layout (sub-tile p = tile
// NWD + wave holds elements [SUB p, SUB (p + 1))) and sums its exact masses, Zp and Zq. In the same sweep it prepares
// the draw's sub-tile weights, which need Zp and Zq: the bonus draw's weight is Ep alone (a sub-tile's sum A of Ep);
// the residual's, max(Ep Zq - Eq Zp, 0), is Ep Zq - Eq Zp for a token with Ep / Eq >= Hp / Lq (A and B sum its Ep and Eq)
// and 0 for one with Ep / Eq <= Lp / Hq, where [Lp, Hp] and [Lq, Hq] bound Zp and Zq (the row's float sums). The few
// tokens in between keep their (Ep, Eq, sub-tile) in the block's LDS list, flushed at the block's end to the
// sequence's list (one atomic per block for its place). The sequence's last block adds the sums up, weights each
// sub-tile exactly as A Zq - B Zp plus its listed tokens' weights, draws, writes the outputs and leaves the draw kernel
// nothing to do. Rows whose bounds are unusable, lists that overflow, and sequences with open tests before the draw
// row (j0 < j1: exact sums for rows j0..j1, in chunks of tpb tiles, then the tests in order) leave the draw to the
// draw kernel, with the draw row's exact sums.

// a mass (< 2^46) as a float, within 2^-23 of it: two exact conversions and one rounding fused multiply-add
__device__ __forceinline__ float to_float(u64 v) { return fmaf((float)(u32)(v >> 32), 4294967296.0f, (float)(u32)v); }

// Sub-tiles p0, p0 + step, ... below p1 (a sub-tile is one wave's SUB elements; sub-tile p starts at element p SUB),
// each summed by the calling wave; undecided tokens go to s_amb (CAP entries, *s_namb counts them all).
template <int MODE, bool FAST, int CAP, bool PRE>
__device__ __forceinline__ void exact_subtiles(const float* tr, const float* dr, int vocab, int p0, int step, int p1, bool vec, float Mp, float Mq,
                                               float c2, float rho_hi, float rho_lo, SubRec* recs, AmbRec* s_amb, unsigned* s_namb, u64& zp,
                                               u64& zq) {
    const int l = lane_id();
    const __amdgpu_buffer_rsrc_t rt = rsrc(tr, (u32)vocab * 4u), rd = rsrc(MODE == 1 ? dr : tr, (u32)vocab * 4u);
    auto issue = [&](int p, float (&t)[DU * 4], float (&d)[DU * 4]) {
#pragma unroll
        for (int j = 0; j < DU; ++j) {
            const int e = p * SUB + j * (WAVE * 4) + l * 4;
            if (vec) {
                const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rt, (u32)e * 4u, 0, 2);
                u32x4 b = {0u, 0u, 0u, 0u};
                if (MODE == 1) b = __builtin_amdgcn_raw_buffer_load_b128(rd, (u32)e * 4u, 0, 2);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    t[j * 4 + q] = __uint_as_float(a[q]);
                    d[j * 4 + q] = __uint_as_float(b[q]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    t[j * 4 + q] = e + q < vocab ? tr[e + q] : -INFINITY;
                    d[j * 4 + q] = (MODE == 1 && e + q < vocab) ? dr[e + q] : -INFINITY;
                }
            }
        }
    };
    constexpr float LO = 1.0f - 1.0f / 524288.0f, HI = 1.0f + 1.0f / 524288.0f;  // 1 -+ 2^-19, over the float roundings
    // PRE: the next sub-tile's loads go out before this one is summed (twice the registers)
    float tn[DU * 4], dn[DU * 4];
    if (PRE && p0 < p1) issue(p0, tn, dn);
    for (int p = p0; p < p1; p += step) {
        float t[DU * 4], d[DU * 4];
        if (PRE) {
#pragma unroll
            for (int i = 0; i < DU * 4; ++i) {
                t[i] = tn[i];
                d[i] = dn[i];
            }
            if (p + step < p1) issue(p + step, tn, dn);
        } else {
            issue(p, t, d);
        }
        u64 A = 0, B = 0;
#pragma unroll
        for (int j = 0; j < DU; ++j) {
            const int e = p * SUB + j * (WAVE * 4) + l * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool in = e + q < vocab;  // buffer loads past the row's end return 0, not -inf
                const u64 ep = row_mass<FAST>(in ? t[j * 4 + q] : -INFINITY, Mp, c2);
                zp += ep;
                if (MODE == 2) {
                    A += ep;
                } else {
                    const u64 eq = row_mass<FAST>(in ? d[j * 4 + q] : -INFINITY, Mq, c2);
                    zq += eq;
                    const float a = to_float(ep), b = to_float(eq);
                    const bool pos = a * LO >= b * rho_hi;
                    const bool neg = a * HI <= b * rho_lo;
                    A += pos ? ep : 0ull;
                    B += pos ? eq : 0ull;
                    const bool amb = !pos && !neg;
                    if (ballot(amb) != 0ull && amb) {
                        const unsigned slot = atomicAdd(s_namb, 1u);
                        if (slot < (unsigned)CAP) s_amb[slot] = AmbRec{ep, eq, (u32)p, 0u};
                    }
                }
            }
        }
        A = wave_sum_u64(A);
        B = wave_sum_u64(B);
        if (l == 0) {
            st_agent(&recs[p].A, A);
            st_agent(&recs[p].B, B);
        }
    }
}

__global__ void __launch_bounds__(NT) spec_exact_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab,
                                                   long long stride, int tpb, int zs, int fparts, bool vec, const int* __restrict__ draft_ids,
                                                   const float* __restrict__ temps, const float* __restrict__ u_accept,
                                                   const float* __restrict__ u_resample, SpecWs ws, int* __restrict__ out_accepted,
                                                   int* __restrict__ out_tokens, int* __restrict__ out_status) {
    __shared__ u64 s_red[NT / WAVE];
    __shared__ u128 s_wt[NT / WAVE];
    __shared__ u128 s_rem;
    __shared__ unsigned s_flag;
    __shared__ int s_done, s_tok;
    __shared__ unsigned s_namb;
    __shared__ AmbRec s_amb[AMB_CAP];
    __shared__ u64 s_wlo[(GBS_MAX_VOCAB + TILE - 1) / TILE * NWD], s_whi[(GBS_MAX_VOCAB + TILE - 1) / TILE * NWD];
    const int S = gridDim.x, sp = blockIdx.x, seq = blockIdx.y;
    const int W1 = width + 1, r0 = seq * W1;
    const int tiles = (vocab + TILE - 1) / TILE;
    const int nsub = tiles * NWD;
    // swept: the row pass's blocks summed the draw row (their sums are parts 0..fparts - 1 of zparts); block 0 finishes
    const bool swept = uni(ld_agent(&ws.fstate[seq])) == FS_GO;
    if (swept && sp != 0) return;
    const SeqInfo si = load_seq(ws.seqs, seq);
    const int pending = uni(ld_agent(&ws.seqs[seq].pending));
    const int j0 = uni(ld_agent(&ws.seqs[seq].j0)), j1 = uni(ld_agent(&ws.seqs[seq].j1));
    const bool work = si.status == GBS_ROW_OK && pending != 0;
    if (work && j0 == j1) {
        const int mode = si.mode;
        const float* tr = target + (size_t)si.row * (size_t)stride;
        const float* dr = draft + (size_t)si.row * (size_t)stride;
        const float Mp = si.Mp, Mq = si.Mq, c2 = si.c2;
        const bool fast = mass_fast_ok(Mp, c2) && mass_fast_ok(Mq, c2);
        // the ratio bounds from the row's float sums (as accept_bounds takes them)
        const float fp = si.fp, fq = si.fq;
        const bool bounds = fast && ratio_bounds_ok(fp, fq);
        const bool fused = mode == 2 || bounds;
        float rho_hi = 0.0f, rho_lo = 0.0f;
        if (mode == 1 && bounds) ratio_bounds(fp, fq, vocab, rho_hi, rho_lo);
        SubRec* recs = ws.subrecs + (size_t)seq * nsub;
        AmbRec* list = ws.ambs + (size_t)seq * AMB_SEQ_CAP;
        if (!swept) {
            const int t0 = sp * tpb, t1 = min(tiles, t0 + tpb);
            u64 zp = 0, zq = 0;
            if (threadIdx.x == 0) s_namb = 0;
            __syncthreads();
            if (fused) {
                // the block's tiles, sub-tile w of each to wave w
                const int w = (int)threadIdx.x / WAVE, p0 = t0 * NWD + w, p1 = t1 * NWD;
                if (mode == 1)
                    exact_subtiles<1, true, AMB_CAP>(tr, dr, vocab, p0, NWD, p1, vec, Mp, Mq, c2, rho_hi, rho_lo, recs, s_amb, &s_namb, zp, zq);
                else if (fast)
                    exact_subtiles<2, true, AMB_CAP>(tr, dr, vocab, p0, NWD, p1, vec, Mp, Mq, c2, 0.0f, 0.0f, recs, s_amb, &s_namb, zp, zq);
                else
                    exact_subtiles<2, false, AMB_CAP>(tr, dr, vocab, p0, NWD, p1, vec, Mp, Mq, c2, 0.0f, 0.0f, recs, s_amb, &s_namb, zp, zq);
            } else {
                const int lo = min(vocab, t0 * TILE), hi = min(vocab, t1 * TILE);
                stream_rows<false>(tr, dr, mode == 1, vocab, lo, hi, vec, [&](float t, float d, int) {
                    zp += t > -INFINITY ? mass(t, Mp, c2) : 0ull;
                    zq += d > -INFINITY ? mass(d, Mq, c2) : 0ull;
                });
            }
            zp = block_sum_u64<NT>(zp, s_red);  // (its barriers also publish s_namb and s_amb)
            zq = block_sum_u64<NT>(zq, s_red);
            // the block's undecided tokens go to the sequence's list, at a place taken by one atomic (the block's count is
            // added even past the list's end, so that the last block sees the overflow)
            const unsigned nb = s_namb < (unsigned)AMB_CAP ? s_namb : (unsigned)AMB_CAP;
            if (threadIdx.x == 0) {
                st_agent(&ws.zparts[((size_t)si.row * zs + sp) * 2], zp);
                st_agent(&ws.zparts[((size_t)si.row * zs + sp) * 2 + 1], zq);
                s_flag = s_namb != 0u ? atomicAdd(&ws.draw_counters[seq], s_namb > (unsigned)AMB_CAP ? (unsigned)AMB_SEQ_CAP + 1u : s_namb) : 0u;
            }
            __syncthreads();
            const unsigned base = s_flag;
            for (unsigned i = threadIdx.x; i < nb; i += NT) {
                if (base + i < (unsigned)AMB_SEQ_CAP) {
                    st_agent(&list[base + i].ep, s_amb[i].ep);
                    st_agent(&list[base + i].eq, s_amb[i].eq);
                    st_agent(&list[base + i].p, s_amb[i].p);
                }
            }
            if (!arrive_last(&ws.row_counters[seq], (unsigned)S, &s_flag)) return;
        }
        // the last block: every load at once (the blocks' sums, the sub-tile sums, the list's length and its first
        // 2 NT entries), then the exact sums, the sub-tile weights and the draw
        u64 a = 0, b = 0;
        const int parts = swept ? fparts : S;
        for (int o = (int)threadIdx.x; o < parts; o += NT) {
            a += ld_agent(&ws.zparts[((size_t)si.row * zs + o) * 2]);
            b += ld_agent(&ws.zparts[((size_t)si.row * zs + o) * 2 + 1]);
        }
        constexpr int PPT = (GBS_MAX_VOCAB + TILE - 1) / TILE * NWD / NT;  // sub-tiles per thread at the largest vocabulary
        u64 A[PPT], B[PPT];
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int p = (int)threadIdx.x + k * NT;
            A[k] = (fused && p < nsub) ? ld_agent(&recs[p].A) : 0ull;
            B[k] = (fused && mode == 1 && p < nsub) ? ld_agent(&recs[p].B) : 0ull;
        }
        const unsigned total = uni(ld_agent(&ws.draw_counters[seq]));
        AmbRec e[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int g = (int)threadIdx.x + k * NT;
            e[k].ep = ld_agent(&list[g].ep);
            e[k].eq = ld_agent(&list[g].eq);
            e[k].p = ld_agent(&list[g].p);
        }
        a = block_sum_u64<NT>(a, s_red);
        b = block_sum_u64<NT>(b, s_red);
        if (threadIdx.x == 0) st_agent(&ws.draw_counters[seq], 0u);  // the list's counter, zero again for the next launch
        SeqInfo sx = si;
        sx.zp = a;
        sx.zq = b;
        if (!fused || total > (unsigned)AMB_SEQ_CAP) {  // the draw kernel draws, with the exact sums
            if (threadIdx.x == 0) {
                st_agent(&ws.seqs[seq].zp, a);
                st_agent(&ws.seqs[seq].zq, b);
            }
            return;
        }
        // the sub-tile weights in LDS: A Zq - B Zp (the bonus draw: A), then each undecided token's exact weight
        // max(Ep Zq - Eq Zp, 0) added to its sub-tile's (64-bit LDS atomics, the carry into the high half)
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int p = (int)threadIdx.x + k * NT;
            if (p < nsub) {
                const u128 wgt = mode == 2 ? (u128)A[k] : (u128)A[k] * b - (u128)B[k] * a;
                s_wlo[p] = (u64)wgt;
                s_whi[p] = (u64)(wgt >> 64);
            }
        }
        __syncthreads();
        auto add_token = [&](const AmbRec& r) {
            const u128 x = (u128)r.ep * b, y = (u128)r.eq * a;
            if (x > y) {
                const u128 d = x - y;
                const u64 lo = (u64)d;
                const u64 old = atomicAdd((unsigned long long*)&s_wlo[r.p], (unsigned long long)lo);
                const u64 carry = old + lo < old ? 1ull : 0ull;
                atomicAdd((unsigned long long*)&s_whi[r.p], (unsigned long long)((u64)(d >> 64) + carry));
            }
        };
#pragma unroll
        for (int k = 0; k < 2; ++k)
            if ((unsigned)threadIdx.x + (unsigned)(k * NT) < total) add_token(e[k]);
        for (unsigned g = threadIdx.x + 2u * NT; g < total; g += NT) {
            AmbRec r;
            r.ep = ld_agent(&list[g].ep);
            r.eq = ld_agent(&list[g].eq);
            r.p = ld_agent(&list[g].p);
            add_token(r);
        }
        __syncthreads();
        constexpr int SPT = ((GBS_MAX_VOCAB + TILE - 1) / TILE * NWD + NT - 1) / NT;
        u128 sub[SPT];
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int p = (int)threadIdx.x * SPT + k;
            sub[k] = p < nsub ? (((u128)s_whi[p] << 64) | s_wlo[p]) : (u128)0;
        }
        const int token = pick_token(sub, nsub, vocab, u_resample[seq], sx, tr, dr, fast, s_wt, &s_rem, &s_flag, &s_tok);
        if (threadIdx.x == 0) {
            sx.mode = 0;
            sx.token = token;
            store_seq(ws.seqs, seq, sx);
            write_outputs(seq, sx, token, width, draft_ids, out_accepted, out_tokens, out_status);
        }
        return;
    }
    if (work) {
        const int lo = min(vocab, sp * tpb * TILE), hi = min(vocab, lo + tpb * TILE);
        for (int j = j0; j <= j1; ++j) {
            const int r = r0 + j;
            const float T = temps[r];
            if (T == 0.0f) continue;
            const RowInfo info = load_row_uniform(ws.rows, r);
            const bool two = j < width;
            const float Mp = key_value(info.tkey), Mq = two ? key_value(info.dkey) : Mp;
            const float c2 = temp_scale(T);
            const float* tr = target + (size_t)r * (size_t)stride;
            const float* dr = draft + (size_t)r * (size_t)stride;
            u64 zp = 0, zq = 0;
            if (mass_fast_ok(Mp, c2) && mass_fast_ok(Mq, c2))
                stream_rows<false>(tr, dr, two, vocab, lo, hi, vec, [&](float t, float d, int) {
                    zp += mass_fast(t, Mp, c2);
                    zq += mass_fast(d, Mq, c2);
                });
            else
                stream_rows<false>(tr, dr, two, vocab, lo, hi, vec, [&](float t, float d, int) {
                    zp += t > -INFINITY ? mass(t, Mp, c2) : 0ull;
                    zq += d > -INFINITY ? mass(d, Mq, c2) : 0ull;
                });
            zp = block_sum_u64<NT>(zp, s_red);
            zq = block_sum_u64<NT>(zq, s_red);
            if (threadIdx.x == 0) {
                st_agent(&ws.zparts[((size_t)r * zs + sp) * 2], zp);
                st_agent(&ws.zparts[((size_t)r * zs + sp) * 2 + 1], zq);
            }
        }
    }
    if (!arrive_last(&ws.row_counters[seq], (unsigned)S, &s_flag)) return;
    if (!work) {  // final since the row pass: an error status, or a greedy draw row
        if (threadIdx.x == 0) write_outputs(seq, si, si.token, width, draft_ids, out_accepted, out_tokens, out_status);
        return;
    }
    if (threadIdx.x == 0) s_done = 0;
    __syncthreads();
    for (int j = j0; j <= j1; ++j) {
        const int r = r0 + j;
        const float T = temps[r];
        u64 a = 0, b = 0;
        if (T != 0.0f) {
            for (int o = (int)threadIdx.x; o < S; o += NT) {
                a += ld_agent(&ws.zparts[((size_t)r * zs + o) * 2]);
                b += ld_agent(&ws.zparts[((size_t)r * zs + o) * 2 + 1]);
            }
            a = block_sum_u64<NT>(a, s_red);
            b = block_sum_u64<NT>(b, s_red);
        }
        if (threadIdx.x == 0) {
            bool acc = false;
            if (j < width) {
                const unsigned state = ld_agent(&ws.rows[r].state);
                acc = state == ACC_YES;
                if (state == ACC_OPEN) {
                    const u64 ep = ld_agent(&ws.rows[r].ep), eq = ld_agent(&ws.rows[r].eq);
                    acc = accept_test(u_accept[(size_t)seq * width + j], (u128)eq * a, (u128)ep * b);
                }
            }
            if (!acc) {
                const RowInfo ri = load_row(ws.rows, r);
                SeqInfo si{};
                si.status = GBS_ROW_OK;
                si.accepted = j;
                si.row = r;
                si.argmax = (int)key_id(ri.tkey);
                if (T == 0.0f) {
                    si.mode = 0;
                    si.token = si.argmax;
                } else {
                    si.mode = j < width ? 1 : 2;
                    si.token = -1;
                    si.Mp = key_value(ri.tkey);
                    si.Mq = key_value(ri.dkey);
                    si.c2 = temp_scale(T);
                    si.zp = a;
                    si.zq = b;
                }
                store_seq(ws.seqs, seq, si);
                if (si.mode == 0) write_outputs(seq, si, si.token, width, draft_ids, out_accepted, out_tokens, out_status);
                s_done = 1;
            }
        }
        __syncthreads();
        if (s_done) break;
    }
}



__global__ void __launch_bounds__(NT) spec_draw_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab, long long stride,
                                                  int tpb, bool vec, const int* __restrict__ draft_ids, const float* __restrict__ u_resample,
                                                  SpecWs ws, int* __restrict__ out_accepted, int* __restrict__ out_tokens,
                                                  int* __restrict__ out_status, bool final_written) {
    __shared__ u128 s_rem;
    __shared__ u128 s_wt[NT / WAVE];
    __shared__ unsigned s_flag;
    __shared__ int s_tok;
    const int S = gridDim.x, sp = blockIdx.x, seq = blockIdx.y;
    const int tiles = (vocab + TILE - 1) / TILE;
    const int nsub = tiles * NWD;
    if (sp == 0 && threadIdx.x == 0) st_agent(&ws.fstate[seq], FS_OPEN);  // read for the last time by the exact pass
    const bool drawing = uni(ld_agent(&ws.seqs[seq].status)) == GBS_ROW_OK && uni(ld_agent(&ws.seqs[seq].mode)) != 0;
    if (final_written && !drawing) return;  // the exact pass wrote this sequence's outputs
    const SeqInfo si = load_seq(ws.seqs, seq);
    const float* tr = target + (size_t)si.row * (size_t)stride;
    const float* dr = draft + (size_t)si.row * (size_t)stride;
    u128* wp = ws.wparts + (size_t)seq * nsub;
    const bool fast = mass_fast_ok(si.Mp, si.c2) && (si.mode == 2 || mass_fast_ok(si.Mq, si.c2));
    if (drawing) {
        const int t0 = sp * tpb, t1 = min(tiles, t0 + tpb);
        if (si.mode == 1 && fast) draw_tiles<1, true>(tr, dr, vocab, t0, t1, vec, si.Mp, si.Mq, si.c2, si.zp, si.zq, wp);
        else if (si.mode == 1) draw_tiles<1, false>(tr, dr, vocab, t0, t1, vec, si.Mp, si.Mq, si.c2, si.zp, si.zq, wp);
        else if (fast) draw_tiles<2, true>(tr, dr, vocab, t0, t1, vec, si.Mp, si.Mq, si.c2, si.zp, si.zq, wp);
        else draw_tiles<2, false>(tr, dr, vocab, t0, t1, vec, si.Mp, si.Mq, si.c2, si.zp, si.zq, wp);
    }
    if (!arrive_last(&ws.draw_counters[seq], (unsigned)S, &s_flag)) return;
    int token = si.token;
    if (drawing) {
        constexpr int SPT = ((GBS_MAX_VOCAB + TILE - 1) / TILE * NWD + NT - 1) / NT;
        u128 sub[SPT];
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int p = (int)threadIdx.x * SPT + k;
            sub[k] = p < nsub ? load_u128(&wp[p]) : (u128)0;
        }
        token = pick_token(sub, nsub, vocab, u_resample[seq], si, tr, dr, fast, s_wt, &s_rem, &s_flag, &s_tok);
    }
    if (threadIdx.x == 0) write_outputs(seq, si, token, width, draft_ids, out_accepted, out_tokens, out_status);
}

// compute units of the current device (0 when the query fails: the row blocks then never sweep the draw rows)
int cu_count() {
    static int counts[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (counts[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        counts[dev] = n;
    }
    return counts[dev];
}

// blocks of spec_split_k the current device holds at once (0 when a query fails: its blocks then never sweep)
int split_resident() {
    static int counts[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (counts[dev] == 0) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, spec_split_k, NT, 0) != hipSuccess) return 0;
        counts[dev] = per_cu * cu_count();
    }
    return counts[dev];
}

}  // namespace

GBS_EXPORT int64_t gbs_spec_set_fuse_wait(int64_t ticks) {
    const long long prev = g_fuse_wait;
    if (ticks >= 0) g_fuse_wait = ticks;
    return prev;
}

GBS_EXPORT size_t gbs_spec_verify_workspace_bytes(int n_seq, int width, int vocab) {
    if (n_seq <= 0 || width < 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB) return 0;
    return plan(n_seq, width, vocab).bytes;
}

GBS_EXPORT int gbs_spec_verify(const float* target, const float* draft, int n_seq, int width, int vocab, int stride,
                               const int* draft_ids, const float* temperatures, const float* u_accept, const float* u_resample,
                               int* out_accepted, int* out_tokens, int* out_status, void* ws, size_t ws_bytes, void* stream) {
    if (n_seq < 0 || width < 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB || stride < vocab) return GBS_ERR_INVALID;
    if (n_seq == 0) return 0;
    if (!target || !temperatures || !u_resample || !out_accepted || !out_tokens || !ws || !aligned(ws, 256)) return GBS_ERR_INVALID;
    if (width > 0 && (!draft || !draft_ids || !u_accept)) return GBS_ERR_INVALID;
    const Plan p = plan(n_seq, width, vocab);
    if (p.R > 65535 || ws_bytes < p.bytes) return GBS_ERR_INVALID;
    const SpecWs w = carve(ws, n_seq, vocab, p);
    const hipStream_t st = to_stream(stream);
    const int chunk = chunk_for(vocab, p.S);
    const float* dr = width > 0 ? draft : target;
    const bool vec = vocab % 4 == 0 && stride % 4 == 0 && aligned(target, 16) && aligned(dr, 16);
    const long long ld = stride;
    int rc;
    if (p.R >= ROWS_KERNEL_MIN) {
        // the row blocks sweep the draw rows only when all of them are resident at once (one per CU) and the exact
        // pass's per-block sums have room for one per row of a sequence
        const bool fuse = p.R <= cu_count();
        hipLaunchKernelGGL(spec_rows_k, dim3(p.R), dim3(RNT), 0, st, target, dr, width, vocab, ld, vec, draft_ids, temperatures, u_accept,
                           u_resample, w, fuse, p.SZ, g_fuse_wait);
        rc = launch_status();
        if (rc) return rc;
    } else {
        // the same sweep when the whole grid is resident at once
        const bool fuse = (long long)p.S * p.R <= (long long)split_resident();
        hipLaunchKernelGGL(spec_split_k, dim3(p.S, p.R), dim3(NT), 0, st, target, dr, width, vocab, ld, chunk, vec, draft_ids, temperatures,
                           u_accept, u_resample, w, fuse, p.SZ, g_fuse_wait);
        rc = launch_status();
        if (rc) return rc;
    }
    hipLaunchKernelGGL(spec_exact_k, dim3(p.S3, n_seq), dim3(NT), 0, st, target, dr, width, vocab, ld, p.tpb, p.SZ, p.F, vec, draft_ids, temperatures,
                       u_accept, u_resample, w, out_accepted, out_tokens, out_status);
    rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(spec_draw_k, dim3(p.S3, n_seq), dim3(NT), 0, st, target, dr, width, vocab, ld, p.tpb, vec, draft_ids, u_resample, w,
                       out_accepted, out_tokens, out_status, true);
    return launch_status();
}
