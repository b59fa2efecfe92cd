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
// Three launches, each (splits, rows) with a last-block hand-off:
//   1. row maxima (order keys, so the argmax ties to the lowest id) and NaN flags of target and draft rows;
//   2. the rows' integer mass sums; the last row of a sequence to finish decides the sequence's acceptances;
//   3. the residual (or bonus) weights of the one row per sequence that needs a draw, per chunk; the last block finds the
//      chunk that holds the draw and scans it.
#include "gbs_modeu.hpp"

using namespace gbs;
using namespace gbs::modeu;

namespace {

constexpr int NT = 256;
constexpr int TARGET_BLOCKS = 1024;
constexpr int MIN_CHUNK = 2048;

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int splits_for(int rows, int vocab) {
    int s = (TARGET_BLOCKS + rows - 1) / rows;
    const int by_size = (vocab + MIN_CHUNK - 1) / MIN_CHUNK;
    if (s > by_size) s = by_size;
    return s < 1 ? 1 : s;
}

struct RowInfo {
    u64 tkey, dkey;  // row maxima as order keys (0 = no finite-or-inf element)
    u64 zp, zq;      // integer mass sums
    unsigned nan;
    unsigned pad[3];
};

struct SeqInfo {
    int status, accepted, row, mode;  // mode 0: token fixed; 1: residual draw; 2: bonus draw
    int token, pad[3];
};

struct SpecWs {
    unsigned* row_counters;  // [R]
    unsigned* seq_counters;  // [n_seq] (launch 2)
    unsigned* draw_counters; // [n_seq] (launch 3)
    u64* maxparts;           // [R][S][2]
    unsigned* nanparts;      // [R][S]
    u64* sumparts;           // [R][S][2]
    RowInfo* rows;           // [R]
    SeqInfo* seqs;           // [n_seq]
    u128* wparts;            // [n_seq][S3]
};

// The counters that must be zero between launches sit at fixed offsets in the first SPEC_CTL_BYTES (room for 65535
// rows and sequences, whatever this launch's shape); every launch leaves them zero. The rest is written before it is
// read, so a workspace cleared once serves launches of any shape.
constexpr size_t SPEC_CTL_BYTES = 3 * (size_t)65536 * 4;

struct Plan {
    int R, S, S3;
    size_t bytes;
};

Plan plan(int n_seq, int width, int vocab) {
    Plan p;
    p.R = n_seq * (width + 1);
    p.S = splits_for(p.R, vocab);
    p.S3 = splits_for(n_seq, vocab);
    p.bytes = SPEC_CTL_BYTES + align256((size_t)p.R * p.S * 16) + align256((size_t)p.R * p.S * 4) + align256((size_t)p.R * p.S * 16) +
              align256((size_t)p.R * sizeof(RowInfo)) + align256((size_t)n_seq * sizeof(SeqInfo)) +
              align256((size_t)n_seq * p.S3 * 16);
    return p;
}

SpecWs carve(void* ws, int n_seq, const Plan& p) {
    char* c = (char*)ws;
    SpecWs w;
    w.row_counters = (unsigned*)c; c += (size_t)65536 * 4;
    w.seq_counters = (unsigned*)c; c += (size_t)65536 * 4;
    w.draw_counters = (unsigned*)c; c += (size_t)65536 * 4;
    w.maxparts = (u64*)c; c += align256((size_t)p.R * p.S * 16);
    w.nanparts = (unsigned*)c; c += align256((size_t)p.R * p.S * 4);
    w.sumparts = (u64*)c; c += align256((size_t)p.R * p.S * 16);
    w.rows = (RowInfo*)c; c += align256((size_t)p.R * sizeof(RowInfo));
    w.seqs = (SeqInfo*)c; c += align256((size_t)n_seq * sizeof(SeqInfo));
    w.wparts = (u128*)c;
    return w;
}

__device__ __forceinline__ u64 max_key(float v, int i) { return (v != v || v == -INFINITY) ? 0ull : make_key(okey_f32(v), (u32)i); }

template <typename T>
__device__ __forceinline__ T block_reduce_max(T v, T* s) {
    s[threadIdx.x] = v;
    __syncthreads();
    for (int h = NT / 2; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) s[threadIdx.x] = s[threadIdx.x] > s[threadIdx.x + h] ? s[threadIdx.x] : s[threadIdx.x + h];
        __syncthreads();
    }
    const T r = s[0];
    __syncthreads();
    return r;
}

template <typename T>
__device__ __forceinline__ T block_reduce_sum(T v, T* s) {
    s[threadIdx.x] = v;
    __syncthreads();
    for (int h = NT / 2; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) s[threadIdx.x] = s[threadIdx.x] + s[threadIdx.x + h];
        __syncthreads();
    }
    const T r = s[0];
    __syncthreads();
    return r;
}

__device__ __forceinline__ RowInfo load_row(const RowInfo* rows, int r) {
    RowInfo ri;
    ri.tkey = ld_agent(&rows[r].tkey);
    ri.dkey = ld_agent(&rows[r].dkey);
    ri.zp = ld_agent(&rows[r].zp);
    ri.zq = ld_agent(&rows[r].zq);
    ri.nan = ld_agent(&rows[r].nan);
    return ri;
}

__device__ __forceinline__ void store_seq(SeqInfo* seqs, int s, const SeqInfo& v) {
    st_agent(&seqs[s].status, v.status);
    st_agent(&seqs[s].accepted, v.accepted);
    st_agent(&seqs[s].row, v.row);
    st_agent(&seqs[s].mode, v.mode);
    st_agent(&seqs[s].token, v.token);
}

__device__ __forceinline__ SeqInfo load_seq(const SeqInfo* seqs, int s) {
    SeqInfo v{};
    v.status = ld_agent(&seqs[s].status);
    v.accepted = ld_agent(&seqs[s].accepted);
    v.row = ld_agent(&seqs[s].row);
    v.mode = ld_agent(&seqs[s].mode);
    v.token = ld_agent(&seqs[s].token);
    return v;
}

__device__ __forceinline__ u128 load_u128(const u128* p) {
    const u64 lo = ld_agent((const u64*)p), hi = ld_agent((const u64*)p + 1);
    return ((u128)hi << 64) | lo;
}

// ---- launch 1: maxima ----
__global__ void __launch_bounds__(NT) spec_max_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab,
                                                 int chunk, SpecWs ws) {
    __shared__ u64 s_red[NT];
    __shared__ unsigned s_flag;
    const int S = gridDim.x, sp = blockIdx.x, r = blockIdx.y;
    const bool has_draft = (r % (width + 1)) < width;
    const float* tr = target + (size_t)r * vocab;
    const float* dr = draft + (size_t)r * vocab;
    const int lo = sp * chunk, hi = min(vocab, lo + chunk);
    u64 tk = 0, dk = 0;
    bool nan = false;
    for (int i = lo + (int)threadIdx.x; i < hi; i += NT) {
        const float t = tr[i];
        nan |= t != t;
        const u64 k = max_key(t, i);
        tk = k > tk ? k : tk;
        if (has_draft) {
            const float d = dr[i];
            nan |= d != d;
            const u64 kd = max_key(d, i);
            dk = kd > dk ? kd : dk;
        }
    }
    tk = block_reduce_max(tk, s_red);
    dk = block_reduce_max(dk, s_red);
    const unsigned bn = block_reduce_max((u64)(nan ? 1 : 0), s_red) != 0ull;
    if (threadIdx.x == 0) {
        st_agent(&ws.maxparts[((size_t)r * S + sp) * 2], tk);
        st_agent(&ws.maxparts[((size_t)r * S + sp) * 2 + 1], dk);
        st_agent(&ws.nanparts[(size_t)r * S + sp], bn);
    }
    if (!arrive_last(&ws.row_counters[r], (unsigned)S, &s_flag)) return;
    if (threadIdx.x == 0) {
        u64 a = 0, b = 0;
        unsigned n = 0;
        for (int o = 0; o < S; ++o) {
            const u64 x = ld_agent(&ws.maxparts[((size_t)r * S + o) * 2]), y = ld_agent(&ws.maxparts[((size_t)r * S + o) * 2 + 1]);
            a = x > a ? x : a;
            b = y > b ? y : b;
            n |= ld_agent(&ws.nanparts[(size_t)r * S + o]);
        }
        st_agent(&ws.rows[r].tkey, a);
        st_agent(&ws.rows[r].dkey, b);
        st_agent(&ws.rows[r].nan, n);
    }
}

__device__ __forceinline__ bool temp_ok(float t) { return isfinite(t) && t >= 0.0f; }

// floor(u * a) < b, exactly
__device__ __forceinline__ bool accept_test(float u, u128 a, u128 b) { return mul_floor(u, a, nullptr) < b; }

__device__ __forceinline__ float key_value(u64 k) { return okey_to_f32(key_ok(k)); }

// ---- launch 2: mass sums, then the sequence's acceptances ----
__global__ void __launch_bounds__(NT) spec_mass_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab,
                                                  int chunk, const int* __restrict__ draft_ids, const float* __restrict__ temps,
                                                  const float* __restrict__ u_accept, const float* __restrict__ u_resample, SpecWs ws) {
    __shared__ u64 s_red[NT];
    __shared__ unsigned s_flag;
    const int S = gridDim.x, sp = blockIdx.x, r = blockIdx.y;
    const int W1 = width + 1;
    const int seq = r / W1;
    const bool has_draft = (r % W1) < width;
    const float T = temps[r];
    const bool draw = temp_ok(T) && T > 0.0f;
    const RowInfo info = load_row(ws.rows, r);
    const float Mp = key_value(info.tkey), Mq = key_value(info.dkey);
    const float c2 = draw ? temp_scale(T) : 0.0f;
    const float* tr = target + (size_t)r * vocab;
    const float* dr = draft + (size_t)r * vocab;
    const int lo = sp * chunk, hi = min(vocab, lo + chunk);
    u64 zp = 0, zq = 0;
    if (draw && info.tkey != 0ull && !info.nan) {
        for (int i = lo + (int)threadIdx.x; i < hi; i += NT) {
            const float t = tr[i];
            if (t > -INFINITY) zp += mass(t, Mp, c2);
            if (has_draft && info.dkey != 0ull) {
                const float d = dr[i];
                if (d > -INFINITY) zq += mass(d, Mq, c2);
            }
        }
    }
    zp = block_reduce_sum(zp, s_red);
    zq = block_reduce_sum(zq, s_red);
    if (threadIdx.x == 0) {
        st_agent(&ws.sumparts[((size_t)r * S + sp) * 2], zp);
        st_agent(&ws.sumparts[((size_t)r * S + sp) * 2 + 1], zq);
    }
    if (!arrive_last(&ws.row_counters[r], (unsigned)S, &s_flag)) return;
    if (threadIdx.x == 0) {
        u64 a = 0, b = 0;
        for (int o = 0; o < S; ++o) {
            a += ld_agent(&ws.sumparts[((size_t)r * S + o) * 2]);
            b += ld_agent(&ws.sumparts[((size_t)r * S + o) * 2 + 1]);
        }
        st_agent(&ws.rows[r].zp, a);
        st_agent(&ws.rows[r].zq, b);
    }
    if (!arrive_last(&ws.seq_counters[seq], (unsigned)W1, &s_flag)) return;
    if (threadIdx.x != 0) return;
    // the sequence's decisions (one thread; width is small)
    SeqInfo si{};
    si.status = GBS_ROW_OK;
    const int r0 = seq * W1;
    bool bad = !(u_resample[seq] >= 0.0f && u_resample[seq] < 1.0f);
    for (int j = 0; j <= width; ++j) bad |= !temp_ok(temps[r0 + j]);
    for (int j = 0; j < width; ++j) {
        const float u = u_accept[(size_t)seq * width + j];
        const int x = draft_ids[(size_t)seq * width + j];
        bad |= !(u >= 0.0f && u < 1.0f) || x < 0 || x >= vocab;
    }
    bool nan = false, empty = false;
    for (int j = 0; j <= width; ++j) {
        const RowInfo ri = load_row(ws.rows, r0 + j);
        nan |= ri.nan != 0u;
        empty |= ri.tkey == 0ull || (j < width && ri.dkey == 0ull);
    }
    if (bad) si.status = GBS_ROW_INVALID_PARAMS;
    else if (nan) si.status = GBS_ROW_NAN_LOGIT;
    else if (empty) si.status = GBS_ROW_NO_CANDIDATES;
    if (si.status == GBS_ROW_OK) {
        int j = 0;
        for (; j < width; ++j) {
            const RowInfo ri = load_row(ws.rows, r0 + j);
            const float Tj = temps[r0 + j];
            const int x = draft_ids[(size_t)seq * width + j];
            bool acc;
            if (Tj == 0.0f) acc = x == (int)key_id(ri.tkey);
            else {
                const float cj = temp_scale(Tj);
                const float tx = target[(size_t)(r0 + j) * vocab + x], dx = draft[(size_t)(r0 + j) * vocab + x];
                const u64 ep = tx > -INFINITY ? mass(tx, key_value(ri.tkey), cj) : 0ull;
                const u64 eq = dx > -INFINITY ? mass(dx, key_value(ri.dkey), cj) : 0ull;
                acc = accept_test(u_accept[(size_t)seq * width + j], (u128)eq * ri.zp, (u128)ep * ri.zq);
            }
            if (!acc) break;
        }
        si.accepted = j;
        si.row = r0 + j;
        const float Tj = temps[r0 + j];
        if (Tj == 0.0f) {
            si.mode = 0;
            si.token = (int)key_id(ld_agent(&ws.rows[r0 + j].tkey));
        } else {
            si.mode = j < width ? 1 : 2;
            si.token = -1;
        }
    }
    store_seq(ws.seqs, seq, si);
}

// residual (mode 1) or bonus (mode 2) weight of element i of the sequence's draw row
__device__ __forceinline__ u128 draw_weight(int mode, const float* tr, const float* dr, int i, float Mp, float Mq, float c2, u64 zp, u64 zq) {
    const float t = tr[i];
    const u64 ep = t > -INFINITY ? mass(t, Mp, c2) : 0ull;
    if (mode == 2) return (u128)ep;
    const float d = dr[i];
    const u64 eq = d > -INFINITY ? mass(d, Mq, c2) : 0ull;
    const u128 a = (u128)ep * zq, b = (u128)eq * zp;
    return a > b ? a - b : (u128)0;
}

// ---- launch 3: the draw ----
__global__ void __launch_bounds__(NT) spec_draw_k(const float* __restrict__ target, const float* __restrict__ draft, int width, int vocab,
                                                  int chunk, const int* __restrict__ draft_ids, const float* __restrict__ temps,
                                                  const float* __restrict__ u_resample, SpecWs ws, int* __restrict__ out_accepted,
                                                  int* __restrict__ out_tokens, int* __restrict__ out_status) {
    __shared__ u128 s_red[NT];
    __shared__ unsigned s_flag;
    __shared__ int s_tok;
    const int S = gridDim.x, sp = blockIdx.x, seq = blockIdx.y;
    const SeqInfo si = load_seq(ws.seqs, seq);
    const bool drawing = si.status == GBS_ROW_OK && si.mode != 0;
    const int lo = sp * chunk, hi = min(vocab, lo + chunk);
    float Mp = 0.f, Mq = 0.f, c2 = 0.f;
    u64 zp = 0, zq = 0;
    const float* tr = target;
    const float* dr = draft;
    if (drawing) {
        const RowInfo ri = load_row(ws.rows, si.row);
        Mp = key_value(ri.tkey);
        Mq = key_value(ri.dkey);
        zp = ri.zp;
        zq = ri.zq;
        c2 = temp_scale(temps[si.row]);
        tr = target + (size_t)si.row * vocab;
        dr = draft + (size_t)si.row * vocab;
    }
    u128 part = 0;
    if (drawing)
        for (int i = lo + (int)threadIdx.x; i < hi; i += NT) part += draw_weight(si.mode, tr, dr, i, Mp, Mq, c2, zp, zq);
    part = block_reduce_sum(part, s_red);
    if (threadIdx.x == 0) {
        st_agent((u64*)&ws.wparts[(size_t)seq * S + sp], (u64)part);
        st_agent((u64*)&ws.wparts[(size_t)seq * S + sp] + 1, (u64)(part >> 64));
    }
    if (!arrive_last(&ws.draw_counters[seq], (unsigned)S, &s_flag)) return;
    int token = si.token;
    if (drawing) {
        if (threadIdx.x == 0) {
            u128 total = 0;
            for (int o = 0; o < S; ++o) total += load_u128(&ws.wparts[(size_t)seq * S + o]);
            const u128 t = mul_floor(u_resample[seq], total, nullptr);
            u128 before = 0;
            int c = 0;
            for (; c < S; ++c) {
                const u128 w = load_u128(&ws.wparts[(size_t)seq * S + c]);
                if (before + w > t) break;
                before += w;
            }
            s_red[0] = t - before;  // target within chunk c
            s_flag = (unsigned)c;
        }
        __syncthreads();
        const u128 tc = s_red[0];
        const int c = (int)s_flag;
        __syncthreads();
        // chunk c, split into NT contiguous ranges; thread sums, then the owning range is scanned
        const int clo = c * chunk, chi = min(vocab, clo + chunk);
        const int per = (chi - clo + NT - 1) / NT;
        const int a = clo + (int)threadIdx.x * per, b = min(chi, a + per);
        u128 mine = 0;
        for (int i = a; i < b; ++i) mine += draw_weight(si.mode, tr, dr, i, Mp, Mq, c2, zp, zq);
        s_red[threadIdx.x] = mine;
        __syncthreads();
        if (threadIdx.x == 0) {
            u128 before = 0;
            int owner = NT - 1;
            for (int k = 0; k < NT; ++k) {
                if (before + s_red[k] > tc) {
                    owner = k;
                    break;
                }
                before += s_red[k];
            }
            s_red[NT - 1] = tc - before;  // reuse: the owner's remaining target (its own slot is read below first)
            s_flag = (unsigned)owner;
        }
        __syncthreads();
        const int owner = (int)s_flag;
        const u128 to = s_red[NT - 1];
        if ((int)threadIdx.x == owner) {
            u128 acc = 0;
            int tok = b > a ? b - 1 : a;
            for (int i = a; i < b; ++i) {
                acc += draw_weight(si.mode, tr, dr, i, Mp, Mq, c2, zp, zq);
                if (acc > to) {
                    tok = i;
                    break;
                }
            }
            s_tok = tok;
        }
        __syncthreads();
        token = s_tok;
    }
    if (threadIdx.x == 0) {
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
}

}  // namespace

GBS_EXPORT size_t gbs_spec_verify_workspace_bytes(int n_seq, int width, int vocab) {
    if (n_seq <= 0 || width < 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB) return 0;
    return plan(n_seq, width, vocab).bytes;
}

GBS_EXPORT int gbs_spec_verify(const float* target, const float* draft, int n_seq, int width, int vocab, const int* draft_ids,
                               const float* temperatures, const float* u_accept, const float* u_resample, int* out_accepted,
                               int* out_tokens, int* out_status, void* ws, size_t ws_bytes, void* stream) {
    if (n_seq < 0 || width < 0 || vocab <= 0 || vocab > GBS_MAX_VOCAB) return GBS_ERR_INVALID;
    if (n_seq == 0) return 0;
    if (!target || !temperatures || !u_resample || !out_accepted || !out_tokens || !ws || !aligned(ws, 256)) return GBS_ERR_INVALID;
    if (width > 0 && (!draft || !draft_ids || !u_accept)) return GBS_ERR_INVALID;
    const Plan p = plan(n_seq, width, vocab);
    if (p.R > 65535 || ws_bytes < p.bytes) return GBS_ERR_INVALID;
    const SpecWs w = carve(ws, n_seq, p);
    const hipStream_t st = to_stream(stream);
    const int chunk = (vocab + p.S - 1) / p.S;
    const int chunk3 = (vocab + p.S3 - 1) / p.S3;
    const float* dr = width > 0 ? draft : target;
    hipLaunchKernelGGL(spec_max_k, dim3(p.S, p.R), dim3(NT), 0, st, target, dr, width, vocab, chunk, w);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(spec_mass_k, dim3(p.S, p.R), dim3(NT), 0, st, target, dr, width, vocab, chunk, draft_ids, temperatures, u_accept,
                       u_resample, w);
    rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(spec_draw_k, dim3(p.S3, n_seq), dim3(NT), 0, st, target, dr, width, vocab, chunk3, draft_ids, temperatures,
                       u_resample, w, out_accepted, out_tokens, out_status);
    return launch_status();
}
