// Exact per-row top-`count` (count <= 64) by (value desc, id asc): the drop-ins for REXL3's gb_topk / gb_topk_valid
// (crates/cuda/csrc/glue.cu:509-711, 1076-1106), gb_nemo_glue_topk (crates/cuda/csrc/nemotron_glue.cu:184-525) and
// gb_glm_topk_f16 (crates/cuda/csrc/glm_glue.cu:270-315).
//
// Two launches, so that a caller workspace of any prior contents works:
//   stage 1, grid (chunks, rows) x 256 threads: each wave streams its share of the chunk (16-byte loads, one 4-element
//     group per lane per step, the next step's loads issued before the current group is ranked) through a gated wave
//     list; the block's four lists are merged by wave 0 and the best `count` keys of the chunk go to the workspace.
//   stage 2, grid (rows) x 256 threads: the row's chunk lists are merged the same way; ids and values are written.
// The chunk split never changes a result: the keys are distinct and the merge keeps exactly the largest.
#include "gbs_select.hpp"

using namespace gbs;

namespace {

constexpr int REF_CHUNK = 16384;  // the bf16/f16 workspace plan: ceil(valid / 16384) lists per row (glue.cu:1079)
using namespace gbs::sel;

template <int DT>
__global__ void __launch_bounds__(NT) topk_stage1_k(const void* logits, long long stride, int valid, int chunk, int nchunks,
                                                    int count, int pitch, u64* ws) {
    __shared__ u64 s_buf[NW][BUF];
    __shared__ u64 s_list[NW][WAVE];
    const int c = blockIdx.x, r = blockIdx.y;
    const size_t esz = DT == DT_F32 ? 4 : 2;
    const void* row = (const char*)logits + (size_t)r * (size_t)stride * esz;
    const int lo = c * chunk;
    const int hi = min(valid, lo + chunk);
    const bool vec = (stride % 4 == 0) && aligned(logits, DT == DT_F32 ? 16 : 8);
    WaveTop<BUF> wt;
    wt.init(s_buf[threadIdx.x / WAVE], count, 0ull);
    block_select<DT>(row, lo, hi, vec, count, wt, s_list);
    if (threadIdx.x < pitch) ws[((size_t)r * nchunks + c) * pitch + threadIdx.x] = wt.list;
}

// merge the row's nchunks lists (pitch keys each, sorted, best first), write ids / values
template <int DT>
__global__ void __launch_bounds__(NT) topk_stage2_k(const void* logits, long long stride, const u64* ws, int nchunks, int pitch,
                                                    int count, int* ids, float* vals) {
    __shared__ u64 s_list[NW][WAVE];
    const int r = blockIdx.x;
    const int w = threadIdx.x / WAVE, l = lane_id();
    const u64* lists = ws + (size_t)r * nchunks * pitch;
    u64 list = 0;
    for (int c = w; c < nchunks; c += NW) {
        const u64 g = l < pitch ? lists[(size_t)c * pitch + l] : 0ull;
        list = wave_merge_desc(list, g);
    }
    list = block_tree_merge<NW>(list, s_list);
    if (w == 0) {
        if (l < count) {
            int id = -1;
            float v = -INFINITY;
            if (list != 0ull) {
                id = (int)key_id(list);
                if (DT == DT_F32) v = ((const float*)logits)[(size_t)r * (size_t)stride + (size_t)id];  // as stored
                else v = okey16_to_f32<DT == DT_F16>(key_ok(list));
            }
            ids[(size_t)r * count + l] = id;
            vals[(size_t)r * count + l] = v;
        }
    }
}

// Stage 1 and stage 2 in ONE launch: every chunk block writes its list to the workspace (agent-scope stores) and counts
// its arrival; the row's last block merges the row's lists (agent-scope loads) and writes ids / values, as stage 2 does.
// The arrival counter of row r is counters[r]; the last block resets it to 0.
template <int DT>
__global__ void __launch_bounds__(NT) topk_fused_k(const void* logits, long long stride, int valid, int chunk, int nchunks, int count,
                                                   int pitch, unsigned* counters, u64* ws, int* ids, float* vals) {
    __shared__ u64 s_buf[NW][BUF];
    __shared__ u64 s_list[NW][WAVE];
    __shared__ unsigned s_flag;
    const int c = blockIdx.x, r = blockIdx.y;
    const int w = threadIdx.x / WAVE, l = lane_id();
    const size_t esz = DT == DT_F32 ? 4 : 2;
    const void* row = (const char*)logits + (size_t)r * (size_t)stride * esz;
    const int lo = c * chunk;
    const int hi = min(valid, lo + chunk);
    const bool vec = (stride % 4 == 0) && aligned(logits, DT == DT_F32 ? 16 : 8);
    WaveTop<BUF> wt;
    wt.init(s_buf[w], count, 0ull);
    block_select<DT>(row, lo, hi, vec, count, wt, s_list);
    u64* lists = ws + (size_t)r * nchunks * pitch;
    if ((int)threadIdx.x < pitch) st_agent(&lists[(size_t)c * pitch + threadIdx.x], wt.list);
    if (!arrive_last(&counters[r], (unsigned)nchunks, &s_flag)) return;
    u64 list = 0;
    for (int o = w; o < nchunks; o += NW) {
        const u64 g = l < pitch ? ld_agent(&lists[(size_t)o * pitch + l]) : 0ull;
        list = wave_merge_desc(list, g);
    }
    __syncthreads();
    list = block_tree_merge<NW>(list, s_list);
    if (w == 0 && l < count) {
        int id = -1;
        float v = -INFINITY;
        if (list != 0ull) {
            id = (int)key_id(list);
            if (DT == DT_F32) v = ((const float*)logits)[(size_t)r * (size_t)stride + (size_t)id];  // as stored
            else v = okey16_to_f32<DT == DT_F16>(key_ok(list));
        }
        ids[(size_t)r * count + l] = id;
        vals[(size_t)r * count + l] = v;
    }
}

template <int DT>
int launch_topk(const void* logits, int rows, long long stride, int valid, int count, int chunk, int nchunks, int pitch, int* ids,
                float* vals, u64* ws, void* stream) {
    hipLaunchKernelGGL(topk_stage1_k<DT>, dim3(nchunks, rows), dim3(NT), 0, to_stream(stream), logits, stride, valid, chunk,
                       nchunks, count, pitch, ws);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(topk_stage2_k<DT>, dim3(rows), dim3(NT), 0, to_stream(stream), logits, stride, (const u64*)ws, nchunks,
                       pitch, count, ids, vals);
    return launch_status();
}

int ref_pitch(int count) { return count <= 16 ? 16 : count <= 32 ? 32 : 64; }
size_t ref_nchunks(int valid) { return ((size_t)valid + REF_CHUNK - 1) / REF_CHUNK; }

size_t topk16_ws_bytes(int rows, int valid, int count) {
    if (rows <= 0 || valid <= 0 || count <= 0 || count > GBS_MAX_COUNT) return 0;
    return (size_t)rows * ref_nchunks(valid) * (size_t)ref_pitch(count) * sizeof(u64);
}

template <int DT>
int topk16(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals, void* workspace, size_t ws_bytes,
           void* stream) {
    if (rows < 0 || stride <= 0 || valid <= 0 || valid > stride || count < 1 || count > GBS_MAX_COUNT || count > valid)
        return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    if (rows > 65535 || !logits || !ids || !vals || !workspace || !aligned(workspace, 16)) return GBS_ERR_INVALID;
    if (ws_bytes < topk16_ws_bytes(rows, valid, count)) return GBS_ERR_INVALID;
    return launch_topk<DT>(logits, rows, stride, valid, count, REF_CHUNK, (int)ref_nchunks(valid), ref_pitch(count), ids, vals,
                           (u64*)workspace, stream);
}

}  // namespace

GBS_EXPORT size_t gb_topk_valid_workspace_bytes(int rows, int valid, int count) { return topk16_ws_bytes(rows, valid, count); }
GBS_EXPORT size_t gb_topk_workspace_bytes(int rows, int vocab, int count) { return topk16_ws_bytes(rows, vocab, count); }

GBS_EXPORT int gb_topk_valid(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals, void* workspace,
                             size_t ws_bytes, void* stream) {
    return topk16<DT_BF16>(logits, rows, stride, valid, count, ids, vals, workspace, ws_bytes, stream);
}

GBS_EXPORT int gb_topk(const void* logits, int rows, int vocab, int count, int* ids, float* vals, void* workspace, size_t ws_bytes,
                       void* stream) {
    return gb_topk_valid(logits, rows, vocab, vocab, count, ids, vals, workspace, ws_bytes, stream);
}

GBS_EXPORT size_t gb_glm_topk_f16_workspace_bytes(int rows, int valid, int count) { return topk16_ws_bytes(rows, valid, count); }

GBS_EXPORT int gb_glm_topk_f16(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals,
                               void* workspace, size_t ws_bytes, void* stream) {
    if (valid < 1 || valid > stride) return GBS_ERR_INVALID;
    return topk16<DT_F16>(logits, rows, stride, valid, count, ids, vals, workspace, ws_bytes, stream);
}

// The workspace of the reference's plan holds rows * blocks * 8 lists of `count` keys (nemotron_glue.cu:507-510); this
// implementation cuts each row into up to blocks * 8 chunks of at least 1024 elements and keeps one list per chunk.
GBS_EXPORT int gb_nemo_glue_topk(const void* logits, int rows, int vocab, int count, int blocks, void* ws, size_t ws_bytes,
                                 void* ids, void* vals, void* stream) {
    if (rows < 0 || vocab < 0 || count < 0 || blocks < 0) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    if (count < 1 || count > GBS_MAX_COUNT || count > vocab || blocks < 1 || rows > 65535) return GBS_ERR_INVALID;
    const size_t need = (size_t)rows * (size_t)blocks * 8 * (size_t)count * sizeof(u64);
    if (!logits || !ws || !ids || !vals || ws_bytes < need || !aligned(ws, 8) || !aligned(logits, 4) || !aligned(ids, 4) ||
        !aligned(vals, 4))
        return GBS_ERR_INVALID;
    const long long max_chunks = (long long)blocks * 8;
    long long chunk = ((long long)vocab + max_chunks - 1) / max_chunks;
    if (chunk < 1024) chunk = 1024;
    chunk = (chunk + 3) / 4 * 4;
    const int nchunks = (int)(((long long)vocab + chunk - 1) / chunk);
    return launch_topk<DT_F32>(logits, rows, vocab, vocab, count, (int)chunk, nchunks, count, (int*)ids, (float*)vals, (u64*)ws,
                               stream);
}

// The single-launch fp16 variant (crates/cuda/csrc/ling_kda_proj_fused.cu:2735-2764): bytes [0, 256) of the workspace
// hold the per-row arrival counters (64 rows; zero before the first call, every call leaves them zero), then the
// lists of the gb_glm_topk_f16 plan. Results are gb_glm_topk_f16's.
constexpr int LING_ROWS_MAX = 64;
constexpr size_t LING_CTL_BYTES = 256;

GBS_EXPORT size_t gb_ling_topk_f16_workspace_bytes(int rows, int valid, int count) {
    if (rows <= 0 || valid <= 0 || count <= 0 || count > GBS_MAX_COUNT) return 0;
    return LING_CTL_BYTES + topk16_ws_bytes(rows, valid, count);
}

GBS_EXPORT int gb_ling_topk_f16(const void* logits, int rows, int stride, int valid, int count, int* ids, float* vals, void* workspace,
                                size_t ws_bytes, void* stream) {
    if (rows < 0 || valid < 1 || valid > stride || count < 1 || count > GBS_MAX_COUNT || count > valid) return GBS_ERR_INVALID;
    if (rows == 0) return 0;
    // the counter region holds 64 rows: more would put counters where the lists are
    if (rows > LING_ROWS_MAX || !logits || !ids || !vals || !workspace || !aligned(workspace, 16)) return GBS_ERR_INVALID;
    if (ws_bytes < gb_ling_topk_f16_workspace_bytes(rows, valid, count)) return GBS_ERR_INVALID;
    const int nchunks = (int)ref_nchunks(valid);
    hipLaunchKernelGGL(topk_fused_k<DT_F16>, dim3(nchunks, rows), dim3(NT), 0, to_stream(stream), logits, (long long)stride, valid,
                       REF_CHUNK, nchunks, count, ref_pitch(count), (unsigned*)workspace,
                       (u64*)((char*)workspace + LING_CTL_BYTES), ids, vals);
    return launch_status();
}
