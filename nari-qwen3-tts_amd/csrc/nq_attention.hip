// Paged GQA attention over the talker's paged KV cache, and the code
// predictor's dense short-cache attention.
//
// Decode rows (one query) use a stream decomposition: the plan lists every
// 16-token key block of every decode row (page id, first slot, token count,
// row and query) and the (kv head, block) units are split into equal
// contiguous spans, one span per wave.  A wave fetches its span's block
// descriptors with one coalesced load, then streams K and V with 128-bit loads
// (D/8 lanes cover one 256-byte row, so one load instruction moves 1 KiB).
// Every kv head's block list is cut into the same spans and wave i takes span
// i / Hkv of head i % Hkv, so the waves of one span read the head slices of
// the same pages at the same time (whole 2 KiB token rows per page).  Register
// use stays at 128 so four waves per SIMD are resident and the launch's 4096
// waves cover the chip in one round.  A wave
// keeps one online softmax per (query, kv head) it touches and writes either
// the final output (when it saw all of that row's keys) or an fp32 partial;
// a second launch merges the partials, so no device-wide fence is needed
// inside the streaming kernel and every wave moves the same number of bytes
// whatever the length mix of the batch.
//
// Causal prefill rows (several queries) are split per query into key chunks
// of 64..1024 tokens and run by a workgroup-per-chunk kernel with the same
// inner loop and its own merge.
//
// Semantics follow FlashInfer's paged decode/prefill as bound in
// executor/talker_kv.py:140-306 (scale 1/sqrt(D), fp32 softmax and
// accumulation, bf16 output), the bottom-right causal rule of
// BatchPrefillWithPagedKVCacheWrapper(causal=True) (talker_kv.py:218) and the
// short-cache kernel of model/kernels.py:408-463.
#include <mutex>
#include <type_traits>

#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kWaves = kAttnThreads / kWave;
constexpr int kBlockTok = 16;          // tokens per key block
constexpr int kStreamWaves = 4096;     // upper bound on stream workers per launch
constexpr bool kStreamDoubleBuffer = false;
constexpr int kMinBlocksPerWave = 4;   // smaller spans would make merging dominate
constexpr int kTargetItems = 8192;     // preferred upper bound on prefill chunk items
constexpr int kMinChunkTokens = 64;
constexpr int kMaxChunkTokens = 1024;  // also the LDS page-id capacity (page size >= 1)
constexpr int kPlanThreads = 1024;     // rows per plan launch (largest bucket)
constexpr int kPlanGrid = 8;

enum MetaSlot {
    kMetaChunks = 0, kMetaChunkTok = 1, kMetaStatus = 2, kMetaQueries = 3,
    kMetaDecRows = 4, kMetaBlocks = 5, kMetaPTiles = 6, kMetaPieces = 7, kMetaBinSlots = 8,
    kMetaSplitRows = 9, kMetaPItems = 10, kMetaPWide = 11, kMetaCount = 16
};

// Decode bins: the fused decode kernel runs kBinWgs workgroups (one per CU);
// workgroup (bin, kv head) owns whole (decode row, kv head) items.  Its waves
// (at most 128 VGPRs each) are kBinWavesSmall for launches of up to
// kBinSmallRows rows and kBinWavesLarge above: on the batch-64 step eight
// waves measured 55.5-55.8 us per launch against 56.3-57.7 for sixteen (12:
// 56.8-57.3, 4: 58.9-59.7), while the 112 decode rows of the mixed batch took
// 133.5-135.5 us with eight and 104.8-105.9 with sixteen.  A launch that runs
// beside the prefill part of its batch (NQ_ATTN_BESIDE_PREFILL) takes
// kBinWavesShared above kBinSmallRows: with twelve waves the mixed batch's layer
// took 128.1-128.9 us against 132.7-135.3 with sixteen (its decode rows alone
// 104.4-105.3 against 103.7-103.8).
constexpr int kBinWgs = 256;
constexpr int kBinWavesSmall = 8;
constexpr int kBinWavesLarge = 16;
constexpr int kBinWavesShared = 12;
constexpr int kBinSmallRows = 64;
constexpr int kBinMaxSlots = 40;   // pieces per bin (LDS q capacity)
constexpr int kBinSortCap = 2048;  // pieces the plan can sort
constexpr bool kDecodeBins = true;  // decode rows of general batches through the bins (else stream + merge)

// Shortest piece a decode row is cut into, in 16-token blocks: a bin's average load below this (a
// small batch) would cut every row into pieces that each wave of a bin covers in under a block and
// that then pay the cross-workgroup merge.  8 rows with KV U{16..512}: 19.5 us per launch cutting
// to the average load, 14.7 with 16-block pieces, 13.9 with 32 or 64 (whole rows).  Batches whose
// average bin load is longer (more than 32 x 16 tokens x 32 bins of decode tokens at 8 KV heads, the
// batch-64 step among them) are dealt as before.
constexpr int kBinMinPieceBlocks = 32;

__host__ __device__ inline int bins_per_head(int num_kv_heads) {
    const int nb = kBinWgs / num_kv_heads;
    return nb < 1 ? 1 : nb;
}

// Prefill MFMA tiles against 64-key tiles, in one of two shapes chosen per
// batch by the plan: narrow tiles of kPrefQ queries of one row (a wave: 16
// queries of one query head, two register sets of K/V in flight) when the
// batch has prefill rows only, wide tiles of kPrefQWide queries (a wave: 16
// queries in both query heads of the kv head, each K/V operand read feeding
// two MFMAs; one register set in flight) when it also has decode rows, whose
// launch then runs beside it.  On the mixed batch of 16 prompt chunks and 112
// decode rows the wide tiles took the layer to 124.3-126.8 us against
// 128.9-132.3 with narrow ones (four alternations on one box: 328 instead of
// 608 tile workgroups share the CUs with the decode bins), while the prefill
// rows alone took 38.0-38.1 us against 35.2-35.3 with narrow tiles (a longer
// chain per key tile on the longest tiles' critical path).
constexpr int kPrefQ = 32;
constexpr int kPrefQWide = 64;
constexpr int kPrefK = 64;
constexpr int kPrefPages = 1024;  // page ids of one prefill item kept in LDS
// A tile whose causal key range spans more than kPrefPieceTiles 64-key tiles is
// cut into up to kPrefMaxPieces pieces of whole key tiles, one workgroup each;
// the last piece to finish merges them.  Cutting shorter tiles measured slower:
// with the mixed batch's wide tiles cut to fill the 512 resident workgroups
// (pieces of at most 5 key tiles) the prefill rows took 74.5-74.8 us (58.8 with
// a relaxed arrival count in a timing copy), against 38 us uncut.
constexpr int kPrefPieceTiles = 16;
constexpr int kPrefMaxPieces = 4;

// Prefill chunk descriptor.
struct alignas(16) ChunkDesc {
    int query;       // query token index (row of q / out)
    int page_start;  // index into kv_indices of the chunk's first page
    int tok_begin;   // first key position of the chunk
    int tok_end;     // one past its last key position
    int n_chunks;    // chunks of this query
    int first_chunk; // index of the query's first chunk
    int pad0, pad1;
};

// Decode block descriptor (int4): {page (a kv_indices offset when the page
// size is below 16), first slot | token count << 24, decode row, query}.
// Decode row descriptor (int4): {row, query, first block, block count}.

struct PlanLayout {
    int64_t meta, chunk_indptr, desc, part_ml, part_o;
    int64_t dec_rows, blocks, spart_ml, spart_o, pitems, pieces, bins, piece_ml, piece_o, arrivals, tile_arrivals;
    int64_t total;
    int64_t max_chunks, max_blocks, max_slots, max_ptiles, max_pitems, max_pieces;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

__host__ __device__ inline PlanLayout plan_layout(int T, int max_pages, int page_size, int Hq, int Hkv,
                                                  int D) {
    PlanLayout L;
    const int G = Hq / Hkv;
    L.max_chunks = 2 * static_cast<int64_t>(T) + kTargetItems / Hkv +
                   static_cast<int64_t>(max_pages) * page_size / kMaxChunkTokens + 64;
    L.max_blocks = static_cast<int64_t>(max_pages) * (page_size > kBlockTok ? page_size / kBlockTok : 1) + T;
    L.max_slots = kStreamWaves + static_cast<int64_t>(Hkv) * T;
    L.max_ptiles = (static_cast<int64_t>(T) + kPrefQ - 1) / kPrefQ + kPlanThreads;
    L.max_pitems = L.max_ptiles * kPrefMaxPieces;
    L.max_pieces = static_cast<int64_t>(T) + bins_per_head(Hkv);
    // the chunk kernel's per-chunk partials, or (head dim 128, two query heads per
    // kv head) the prefill tiles' per-(query, piece) partials, whichever is larger
    const int64_t part_rows = L.max_chunks > static_cast<int64_t>(T) * kPrefMaxPieces
                                  ? L.max_chunks : static_cast<int64_t>(T) * kPrefMaxPieces;
    int64_t off = 0;
    L.meta = off;         off = align256(off + kMetaCount * 4);
    L.chunk_indptr = off; off = align256(off + (static_cast<int64_t>(T) + 1) * 4);
    L.desc = off;         off = align256(off + L.max_chunks * static_cast<int64_t>(sizeof(ChunkDesc)));
    L.part_ml = off;      off = align256(off + part_rows * Hq * 2 * 4);
    L.part_o = off;       off = align256(off + part_rows * Hq * D * 4);
    L.dec_rows = off;     off = align256(off + static_cast<int64_t>(T) * 16);
    L.blocks = off;       off = align256(off + L.max_blocks * 16);
    L.spart_ml = off;     off = align256(off + L.max_slots * G * 2 * 4);
    L.spart_o = off;      off = align256(off + L.max_slots * G * D * 4);
    L.pitems = off;       off = align256(off + L.max_pitems * 32);
    L.pieces = off;       off = align256(off + L.max_pieces * 16);
    L.bins = off;         off = align256(off + static_cast<int64_t>(bins_per_head(Hkv)) * kBinMaxSlots * 48);
    L.piece_ml = off;     off = align256(off + L.max_pieces * Hq * 2 * 4);
    L.piece_o = off;      off = align256(off + L.max_pieces * Hq * D * 4);
    L.arrivals = off;     off = align256(off + static_cast<int64_t>(T) * Hkv * 4);
    L.tile_arrivals = off; off = align256(off + L.max_ptiles * Hkv * 4);
    L.total = off;
    return L;
}

// Prefill tile t (of qt queries) of a row with kv_len keys and qo_len queries
// covers keys [0, kv_len - qo_len + qt t + nq) (bottom-right causal); its
// 64-key tiles, and the pieces they are cut into.
__device__ __forceinline__ int pref_tile_keys(int kv_len, int qo_len, int t, int qt) {
    const int nq = qo_len - t * qt < qt ? qo_len - t * qt : qt;
    const int n_keys = kv_len - qo_len + t * qt + nq;
    return n_keys > 0 ? n_keys : 0;
}

// Pieces of a tile over n_keys keys.  Every piece spans at least two key
// tiles, so the first key of the last piece lies below the tile's first query
// limit (the limits of a tile's queries lie within 64 keys of each other):
// each piece's first key tile holds a key every query attends to.
__device__ __forceinline__ int pref_pieces(int n_keys) {
    const int n_kt = (n_keys + kPrefK - 1) / kPrefK;
    int k = (n_kt + kPrefPieceTiles - 1) / kPrefPieceTiles;
    k = k > n_kt / 2 ? n_kt / 2 : k;
    return k < 1 ? 1 : (k > kPrefMaxPieces ? kPrefMaxPieces : k);
}

__device__ int plan_block_scan(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int incl = wave_incl_scan(v);
    if (lane == kWave - 1) tmp[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const int nw = blockDim.x / kWave;
        const int w = lane < nw ? tmp[lane] : 0;
        const int wi = wave_incl_scan(w);
        if (lane < nw) tmp[lane] = wi - w;
        if (lane == nw - 1) tmp[kWave] = wi;
    }
    __syncthreads();
    const int res = tmp[wave] + incl - v;
    *total = tmp[kWave];
    __syncthreads();
    return res;
}

// Largest r in [0, n) with off[r] <= x (off non-decreasing, off[0] == 0).
__device__ __forceinline__ int find_le(const int *off, int n, int x) {
    int lo = 0, hi = n;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= x) lo = mid; else hi = mid;
    }
    return lo;
}

// Every workgroup scans the rows into LDS; workgroup 0 writes the per-row and
// prefill-chunk tables, all workgroups fill the decode block table.
__global__ void __launch_bounds__(kPlanThreads)
attention_plan_kernel(const int32_t *__restrict__ qo_indptr, const int32_t *__restrict__ kv_indptr,
                      const int32_t *__restrict__ last_page_len,
                      const int32_t *__restrict__ kv_indices, const int64_t *__restrict__ position_ids,
                      const int64_t *__restrict__ write_pages, const int64_t *__restrict__ write_offsets,
                      int n_rows, int max_queries, int index_limit, int page_size, int num_kv_heads,
                      char *__restrict__ ws, PlanLayout L, int decode_as_prefill) {
    __shared__ int s_qo[kPlanThreads + 1];
    __shared__ int s_kvlen[kPlanThreads];
    __shared__ int s_base[kPlanThreads];
    __shared__ int s_boff[kPlanThreads];
    __shared__ int s_dec[kPlanThreads];
    __shared__ unsigned long long s_cand[8];
    __shared__ int s_tmp[6 * (kWave + 1)];
    __shared__ __attribute__((aligned(16))) unsigned s_keys[kBinSortCap];
    __shared__ unsigned s_sorted[kBinSortCap];
    __shared__ int4 s_pa[kBinSortCap], s_pb[kBinSortCap];

    int32_t *meta = reinterpret_cast<int32_t *>(ws + L.meta);
    int32_t *chunk_indptr = reinterpret_cast<int32_t *>(ws + L.chunk_indptr);
    ChunkDesc *desc = reinterpret_cast<ChunkDesc *>(ws + L.desc);
    int4 *dec_rows = reinterpret_cast<int4 *>(ws + L.dec_rows);
    int4 *blocks = reinterpret_cast<int4 *>(ws + L.blocks);

    const int tid = threadIdx.x;
    const bool lead = blockIdx.x == 0;
    int ps_log2 = 0;
    while ((1 << ps_log2) < page_size) ++ps_log2;
    // Without packed queries row r's query token is r: the lead issues its
    // position / write-slot loads now, with the row loads, rather than after
    // the scans.
    const bool early_pos = lead && !qo_indptr && position_ids && write_pages && write_offsets && tid < n_rows;
    int64_t e_pos = 0, e_pg = 0, e_off = 0;
    if (early_pos) {
        e_pos = position_ids[tid];
        e_pg = write_pages[tid];
        e_off = write_offsets[tid];
    }
    if (tid < n_rows) {
        const int np = kv_indptr[tid + 1] - kv_indptr[tid];
        int last = last_page_len[tid];
        last = last < 1 ? 1 : (last > page_size ? page_size : last);  // keys stay inside the row's pages
        s_kvlen[tid] = np > 0 ? (np - 1) * page_size + last : 0;
        s_base[tid] = kv_indptr[tid];
        s_qo[tid] = qo_indptr ? qo_indptr[tid] : tid;
    }
    if (tid == 0) s_qo[n_rows] = qo_indptr ? qo_indptr[n_rows] : n_rows;
    if (tid < 8) s_cand[tid] = 0;
    __syncthreads();
    const int T = s_qo[n_rows];
    auto fail = [&](int code) {
        if (lead && tid == 0) {
            meta[kMetaChunks] = 0;
            meta[kMetaChunkTok] = kMinChunkTokens;
            meta[kMetaStatus] = code;
            meta[kMetaQueries] = 0;
            meta[kMetaDecRows] = 0;
            meta[kMetaBlocks] = 0;
            meta[kMetaPTiles] = 0;
            meta[kMetaPieces] = 0;
            meta[kMetaBinSlots] = 0;
            meta[kMetaSplitRows] = 0;
            meta[kMetaPItems] = 0;
        }
    };
    if (T < 0 || T > max_queries) {
        fail(NQ_ERR_INVALID_ARGUMENT);
        return;
    }

    // Decode rows and their key blocks, and prefill rows' tiles and pieces in
    // both tile shapes, in one scan; the shape follows whether the batch has
    // decode rows.  With decode_as_prefill (no decode launch will run) a
    // one-query row is planned as a prefill row.
    int is_dec = 0, nblk = 0, nt_n = 0, np_n = 0, nt_w = 0, np_w = 0;
    if (tid < n_rows) {
        const int qo_len = s_qo[tid + 1] - s_qo[tid];
        if (qo_len == 1 && !decode_as_prefill) {
            is_dec = 1;
            nblk = (s_kvlen[tid] + kBlockTok - 1) / kBlockTok;
            nblk = nblk < 1 ? 1 : nblk;
        } else if (qo_len >= 1) {
            nt_n = (qo_len + kPrefQ - 1) / kPrefQ;
            for (int t = 0; t < nt_n; ++t) np_n += pref_pieces(pref_tile_keys(s_kvlen[tid], qo_len, t, kPrefQ));
            nt_w = (qo_len + kPrefQWide - 1) / kPrefQWide;
            for (int t = 0; t < nt_w; ++t) np_w += pref_pieces(pref_tile_keys(s_kvlen[tid], qo_len, t, kPrefQWide));
        }
    }
    int sc_excl[6], sc_total[6];
    block_exclusive_scan_n<6>({is_dec, nblk, nt_n, np_n, nt_w, np_w}, s_tmp, sc_excl, sc_total);
    const int dec_idx = sc_excl[0], boff = sc_excl[1];
    const int n_dec = sc_total[0], n_blocks = sc_total[1];
    const bool wide = n_dec > 0;
    const int qt = wide ? kPrefQWide : kPrefQ;
    const int nt = wide ? nt_w : nt_n;
    const int t0_tiles = wide ? sc_excl[4] : sc_excl[2], p0_items = wide ? sc_excl[5] : sc_excl[3];
    const int n_ptiles = wide ? sc_total[4] : sc_total[2], n_pitems = wide ? sc_total[5] : sc_total[3];
    s_dec[tid] = dec_idx;
    s_boff[tid] = boff;
    __syncthreads();
    if (n_blocks > L.max_blocks) {
        fail(NQ_ERR_CAPACITY);
        return;
    }
    if (lead && is_dec) dec_rows[dec_idx] = make_int4(tid, s_qo[tid], boff, nblk);

    // Decode bins (lead workgroup): rows longer than a bin's average load C (at
    // least kBinMinPieceBlocks) are cut into k = ceil(blocks / C) near-equal pieces; pieces are sorted by size
    // (descending, then piece id) and dealt to the bins in snake order
    // (0, 1, .., NB-1, NB-1, .., 0, ..), which evens the bins' loads.  Piece
    // descriptor: {decode row, first block, block count, (first piece << 9) | k
    // for a split row, else -1}.  Bin table [NB][kBinMaxSlots] of three int4
    // each: the piece, {query token, position, write page, write offset |
    // (last piece of its row) << 31} (what the fused decode kernel's q/k
    // RoPE and K/V write need, so its prologue reads one row of this table
    // instead of chasing ids), and {piece id or -1 for an empty slot}.  A
    // missing or out-of-range position / write slot stores write page -1,
    // which the fused kernel reports.  The split rows' arrival counters
    // (decode row x kv head) start at zero.
    if (lead) {
        const int NB = bins_per_head(num_kv_heads);
        int C = n_blocks > 0 ? (n_blocks + NB - 1) / NB : 1;
        C = C < kBinMinPieceBlocks ? kBinMinPieceBlocks : C;
        const int k = is_dec ? (nblk + C - 1) / C : 0;
        int pc_excl[2], pc_total[2];
        block_exclusive_scan_n<2>({k, k > 1 ? 1 : 0}, s_tmp, pc_excl, pc_total);
        const int p0 = pc_excl[0], P = pc_total[0], n_split = pc_total[1];
        const int slots = (P + NB - 1) / NB;
        if (P > L.max_pieces || P > kBinSortCap || NB + 1 > 511) {
            fail(NQ_ERR_CAPACITY);
            return;
        }
        int32_t *arrivals = reinterpret_cast<int32_t *>(ws + L.arrivals);
        for (int i = tid; i < n_dec * num_kv_heads; i += blockDim.x) arrivals[i] = 0;
        int4 *pieces = reinterpret_cast<int4 *>(ws + L.pieces);
        int4 rope = make_int4(0, 0, -1, 0);
        if (k > 0) {
            const int tok = s_qo[tid];
            rope.x = tok;
            if (position_ids && write_pages && write_offsets) {
                const int64_t pos = early_pos ? e_pos : position_ids[tok];
                const int64_t pg = early_pos ? e_pg : write_pages[tok];
                const int64_t off = early_pos ? e_off : write_offsets[tok];
                const bool ok = pos >= 0 && pos <= 0x7fffffff && pg >= 0 && pg <= 0x7fffffff && off >= 0 &&
                                off <= 0x7fffffff;
                rope = make_int4(tok, ok ? static_cast<int>(pos) : 0, ok ? static_cast<int>(pg) : -1,
                                 ok ? static_cast<int>(off) : 0);
            }
        }
        // piece i covers blocks [i * nblk / k, (i + 1) * nblk / k); 32-bit
        // arithmetic where the product fits (an inlined 64-bit division is slow)
        const bool narrow = nblk < (1 << 20) && k <= (1 << 11);
        auto cut = [&](int i) {
            return narrow ? static_cast<int>(static_cast<unsigned>(i) * static_cast<unsigned>(nblk) /
                                             static_cast<unsigned>(k))
                          : static_cast<int>(static_cast<int64_t>(i) * nblk / k);
        };
        for (int i = 0; i < k; ++i) {
            const int first = boff + cut(i);
            const int last = boff + cut(i + 1);
            const int4 pc = make_int4(dec_idx, first, last - first, k > 1 ? (p0 << 9) | k : -1);
            pieces[p0 + i] = pc;
            s_pa[p0 + i] = pc;  // p0 + i < P <= kBinSortCap (checked above)
            s_pb[p0 + i] = make_int4(rope.x, rope.y, rope.z,
                                     static_cast<int>(static_cast<unsigned>(rope.w) | (i == k - 1 ? 0x80000000u : 0u)));
            const unsigned cnt = static_cast<unsigned>(last - first) > 0xFFFFu ? 0xFFFFu : static_cast<unsigned>(last - first);
            s_keys[p0 + i] = ((0xFFFFu - cnt) << 16) | static_cast<unsigned>(p0 + i);
        }
        int np2 = 1;
        while (np2 < P) np2 <<= 1;
        for (int i = P + tid; i < np2; i += blockDim.x) s_keys[i] = 0xFFFFFFFFu;
        const unsigned *sorted = s_keys;
        if (np2 > kWave) {
            // more than 64 pieces: each key's place is the count of smaller keys
            // (the keys are distinct: the low half is the piece id), one pass
            // with one barrier instead of a log^2 network of them
            __syncthreads();
            // (four keys per LDS read; the padding keys up to np2 are all ones,
            // never below a piece key)
            const uint4 *keys4 = reinterpret_cast<const uint4 *>(s_keys);
            for (int i = tid; i < P; i += blockDim.x) {
                const unsigned key = s_keys[i];
                int rank = 0;
                for (int j = 0; j < np2 / 4; ++j) {
                    const uint4 q = keys4[j];
                    rank += (q.x < key ? 1 : 0) + (q.y < key ? 1 : 0) + (q.z < key ? 1 : 0) + (q.w < key ? 1 : 0);
                }
                s_sorted[rank] = key;
            }
            sorted = s_sorted;
            np2 = 1;  // the LDS network below has nothing left to do
        } else {
            // up to 64 pieces: one wave sorts them in registers (lane i holds key i), no barriers
            __syncthreads();
            if (tid < kWave) {
                unsigned key = tid < np2 ? s_keys[tid] : 0xFFFFFFFFu;
                for (int size = 2; size <= np2; size <<= 1) {
                    for (int stride = size >> 1; stride > 0; stride >>= 1) {
                        const unsigned other = __shfl_xor(key, stride, kWave);
                        const bool low = (tid & stride) == 0;       // the lower index of the pair
                        const bool asc = (tid & size) == 0;         // the pair's direction
                        const unsigned lo = key < other ? key : other, hi = key < other ? other : key;
                        key = (low == asc) ? lo : hi;
                    }
                }
                if (tid < np2) s_keys[tid] = key;
            }
            np2 = 1;  // the LDS network below has nothing left to do
        }
        for (int size = 2; size <= np2; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                __syncthreads();
                for (int i = tid; i < np2 / 2; i += blockDim.x) {
                    const int lo = 2 * i - (i & (stride - 1));
                    const int hi = lo + stride;
                    const unsigned a = s_keys[lo], b = s_keys[hi];
                    if ((a > b) == ((lo & size) == 0)) {
                        s_keys[lo] = b;
                        s_keys[hi] = a;
                    }
                }
            }
        }
        __syncthreads();
        int4 *table = reinterpret_cast<int4 *>(ws + L.bins);
        for (int e = tid; e < NB * kBinMaxSlots; e += blockDim.x) {
            const int bin = e / kBinMaxSlots, round = e % kBinMaxSlots;
            const int i = round * NB + ((round & 1) ? NB - 1 - bin : bin);
            const int pid = round < slots && i < P ? static_cast<int>(sorted[i] & 0xFFFFu) : -1;
            table[3 * e] = pid >= 0 ? s_pa[pid] : make_int4(-1, 0, 0, -1);
            table[3 * e + 1] = pid >= 0 ? s_pb[pid] : make_int4(0, 0, -1, 0);
            table[3 * e + 2] = make_int4(pid, 0, 0, 0);
        }
        if (tid == 0) {
            meta[kMetaPieces] = P;
            meta[kMetaBinSlots] = slots;
            meta[kMetaSplitRows] = n_split;
        }
        // no barrier here: nothing below reads the sort's LDS, and a barrier
        // would wait for the table's stores to complete
    }

    // the block table: the other workgroups when there are any (the lead has
    // the bins and the row tables to write)
    const int fillers = gridDim.x > 1 ? gridDim.x - 1 : 1;
    const int filler = gridDim.x > 1 ? static_cast<int>(blockIdx.x) - 1 : 0;
    const int gstride = fillers * blockDim.x;
    for (int b = filler * blockDim.x + tid; filler >= 0 && b < n_blocks; b += gstride) {
        const int r = find_le(s_boff, n_rows, b);
        const int tok0 = (b - s_boff[r]) * kBlockTok;
        int ntok = s_kvlen[r] - tok0;
        ntok = ntok < 0 ? 0 : (ntok > kBlockTok ? kBlockTok : ntok);
        int page, slot0;
        if (page_size >= kBlockTok) {
            const int at = s_base[r] + (tok0 >> ps_log2);
            page = (ntok > 0 && at < index_limit) ? kv_indices[at] : -1;
            slot0 = tok0 & (page_size - 1);
        } else {
            page = s_base[r] + (tok0 >> ps_log2);  // kv_indices offset; pages looked up per token
            slot0 = 0;
        }
        blocks[b] = make_int4(page, slot0 | (ntok << 24), s_dec[r], s_qo[r]);
    }
    if (!lead) return;

    // Prefill rows: tiles of qt queries, each cut into pieces of whole 64-key tiles.
    // Item = two int4: the tile {first query, queries, first page offset, key
    // limit of the first query (bottom-right causal)} and the piece {first key,
    // end key, (piece << 8) | pieces, tile index}.  The tiles' arrival
    // counters (tile x kv head) start at zero.
    {
        if (n_ptiles > L.max_ptiles || n_pitems > L.max_pitems) {
            fail(NQ_ERR_CAPACITY);
            return;
        }
        int4 *pitems = reinterpret_cast<int4 *>(ws + L.pitems);
        int32_t *tile_arrivals = reinterpret_cast<int32_t *>(ws + L.tile_arrivals);
        for (int i = tid; i < n_ptiles * num_kv_heads; i += blockDim.x) tile_arrivals[i] = 0;
        const int qo_len = s_qo[tid + 1] - s_qo[tid];
        int it = p0_items;
        for (int t = 0; t < nt; ++t) {
            const int4 td = make_int4(s_qo[tid] + t * qt, min(qt, qo_len - t * qt), s_base[tid],
                                      s_kvlen[tid] - qo_len + t * qt + 1);
            const int n_keys = pref_tile_keys(s_kvlen[tid], qo_len, t, qt);
            const int n_kt = (n_keys + kPrefK - 1) / kPrefK;
            const int k = pref_pieces(n_keys);
            for (int p = 0; p < k; ++p, ++it) {
                const int kb = kPrefK * (p * n_kt / k);
                const int ke = p == k - 1 ? n_keys : kPrefK * ((p + 1) * n_kt / k);
                pitems[2 * it] = td;
                pitems[2 * it + 1] = make_int4(kb, ke, (p << 8) | k, t0_tiles + t);
            }
        }
        if (tid == 0) {
            meta[kMetaPTiles] = n_ptiles;
            meta[kMetaPItems] = n_pitems;
            meta[kMetaPWide] = wide ? 1 : 0;
        }
    }
    if (n_ptiles == 0) {
        // no prefill rows: no query has key chunks, so every chunk offset is 0
        // and the chunk size is the smallest candidate (what the general path
        // below computes for such a batch, without its scans)
        for (int q = tid; q <= T; q += blockDim.x) chunk_indptr[q] = 0;
        if (tid == 0) {
            meta[kMetaChunks] = 0;
            meta[kMetaChunkTok] = kMinChunkTokens < page_size ? page_size : kMinChunkTokens;
            meta[kMetaQueries] = T;
            meta[kMetaDecRows] = n_dec;
            meta[kMetaBlocks] = n_blocks;
            meta[kMetaStatus] = NQ_OK;
        }
        return;
    }

    // Prefill queries: key chunks per query.
    auto query_keys = [&](int q, int *row_out) {
        const int lo = find_le(s_qo, n_rows, q);
        const int qo_len = s_qo[lo + 1] - s_qo[lo];
        int kvlen = s_kvlen[lo] - qo_len + (q - s_qo[lo]) + 1;
        kvlen = kvlen < 0 ? 0 : (kvlen > s_kvlen[lo] ? s_kvlen[lo] : kvlen);
        *row_out = lo;
        // -1: a decode query, served by the stream kernel
        return qo_len > 1 || (qo_len == 1 && decode_as_prefill) ? kvlen : -1;
    };
    const int n_cand = 5;  // 64 .. 1024 tokens
    unsigned long long cand[n_cand];
#pragma unroll
    for (int c = 0; c < n_cand; ++c) cand[c] = 0;
    for (int q = tid; q < T; q += blockDim.x) {
        int row;
        const int kvlen = query_keys(q, &row);
        if (kvlen < 0) continue;
#pragma unroll
        for (int c = 0; c < n_cand; ++c) {
            int ct = kMinChunkTokens << c;
            ct = ct < page_size ? page_size : ct;
            const int n = (kvlen + ct - 1) / ct;
            cand[c] += n > 0 ? n : 1;
        }
    }
    // wave sums first, then one LDS atomic per wave and candidate (and none for a zero sum: a
    // decode-only batch adds nothing) -- per-thread 64-bit atomics on five addresses serialize
#pragma unroll
    for (int c = 0; c < n_cand; ++c) {
        unsigned lo = static_cast<unsigned>(cand[c]), hi = static_cast<unsigned>(cand[c] >> 32);
        unsigned long long v = cand[c];
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            lo = __shfl_xor(static_cast<unsigned>(v), m, kWave);
            hi = __shfl_xor(static_cast<unsigned>(v >> 32), m, kWave);
            v += (static_cast<unsigned long long>(hi) << 32) | lo;
        }
        if ((tid & (kWave - 1)) == 0 && v != 0) atomicAdd(&s_cand[c], v);
    }
    __syncthreads();
    int chosen = -1;
    for (int c = 0; c < n_cand; ++c)
        if (s_cand[c] * num_kv_heads <= kTargetItems) { chosen = c; break; }
    if (chosen < 0)
        for (int c = 0; c < n_cand; ++c)
            if (s_cand[c] <= static_cast<unsigned long long>(L.max_chunks)) { chosen = c; break; }
    if (chosen < 0) {
        fail(NQ_ERR_CAPACITY);
        return;
    }
    int chunk_tok = kMinChunkTokens << chosen;
    chunk_tok = chunk_tok < page_size ? page_size : chunk_tok;
    const int chunk_pages = chunk_tok / page_size;

    int carry = 0;
    for (int base = 0; base < T; base += blockDim.x) {
        const int q = base + tid;
        int n = 0, row = 0, kvlen = -1;
        if (q < T) {
            kvlen = query_keys(q, &row);
            if (kvlen >= 0) {
                n = (kvlen + chunk_tok - 1) / chunk_tok;
                if (n < 1) n = 1;
            }
        }
        int total;
        const int excl = plan_block_scan(n, s_tmp, &total);
        if (q < T) {
            const int c0 = carry + excl;
            chunk_indptr[q] = c0;
            for (int k = 0; k < n; ++k) {
                ChunkDesc d;
                d.query = q;
                d.page_start = s_base[row] + k * chunk_pages;
                d.tok_begin = k * chunk_tok;
                d.tok_end = min(kvlen, (k + 1) * chunk_tok);
                d.n_chunks = n;
                d.first_chunk = c0;
                d.pad0 = d.pad1 = 0;
                desc[c0 + k] = d;
            }
        }
        carry += total;
    }
    if (tid == 0) {
        chunk_indptr[T] = carry;
        meta[kMetaChunks] = carry;
        meta[kMetaChunkTok] = chunk_tok;
        meta[kMetaQueries] = T;
        meta[kMetaDecRows] = n_dec;
        meta[kMetaBlocks] = n_blocks;
        meta[kMetaStatus] = NQ_OK;
    }
}

// ---------------------------------------------------------------------------
// Shared lane layout: D/8 lanes hold one 256/128-byte K or V row (8 bf16 each),
// so a wave covers TPL = 64/(D/8) tokens per 128-bit load instruction.

template <int D, int G>
struct Lanes {
    static constexpr int LPT = D / 8;
    static constexpr int TPL = kWave / LPT;
    static constexpr int NL = kBlockTok / TPL;  // loads per 16-token block per K or V
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b),
                                           c, false);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v;
    v.x = static_cast<__bf16>(lo);
    v.y = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int w) {
    return w == 0 ? v.x : (w == 1 ? v.y : (w == 2 ? v.z : v.w));
}

// Online softmax of G query heads over 16-token blocks.  q stays in bf16 and
// both products run on v_dot2_f32_bf16 with fp32 accumulation: q.k as four
// dot2 per 8 elements, and P.V pairs two tokens per dot2 (the weights are
// rounded to bf16 for the product and for the normaliser alike, as a bf16
// tensor-core P.V would).  With kFp32P the weights stay fp32 and P.V is fp32
// multiply-adds on the widened V (the short-cache attention of the code
// predictor, whose reference kernel keeps P in fp32, model/kernels.py:452-461).
template <int D, int G, bool kFp32P = false>
struct SoftmaxState {
    uint32_t qb[G][4];
    float scale;
    float m[G], l[G], acc[G][8];

    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            m[j] = -INFINITY;
            l[j] = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
        }
    }

    __device__ __forceinline__ void load_q(const uint16_t *qptr, int64_t q_s1, int h, int sub,
                                           float scale_log2) {
        scale = scale_log2;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const uint4 p = *reinterpret_cast<const uint4 *>(qptr + (h * G + j) * q_s1 + sub * 8);
            qb[j][0] = p.x;
            qb[j][1] = p.y;
            qb[j][2] = p.z;
            qb[j][3] = p.w;
        }
    }

    // One 16-token block already in registers.
    __device__ __forceinline__ void consume(const uint4 (&kr)[Lanes<D, G>::NL],
                                            const uint4 (&vr)[Lanes<D, G>::NL],
                                            const bool (&valid)[Lanes<D, G>::NL]) {
        float s[Lanes<D, G>::NL][G];
        scores(kr, valid, s);
        accumulate(vr, s);
    }

    // The block's scaled scores (log2 domain), -inf for masked tokens.
    __device__ __forceinline__ void scores(const uint4 (&kr)[Lanes<D, G>::NL],
                                           const bool (&valid)[Lanes<D, G>::NL],
                                           float (&s)[Lanes<D, G>::NL][G]) const {
        constexpr int NL = Lanes<D, G>::NL;
        constexpr int LPT = Lanes<D, G>::LPT;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                float part = dot2_bf16(qb[j][0], kr[i].x, 0.f);
                part = dot2_bf16(qb[j][1], kr[i].y, part);
                part = dot2_bf16(qb[j][2], kr[i].z, part);
                part = dot2_bf16(qb[j][3], kr[i].w, part);
                part = group_sum<LPT>(part) * scale;
                s[i][j] = valid[i] ? part : -INFINITY;
            }
        }
    }

    // Online-softmax update with the block's scores and its V rows.
    __device__ __forceinline__ void accumulate(const uint4 (&vr)[Lanes<D, G>::NL],
                                               const float (&s)[Lanes<D, G>::NL][G]) {
        constexpr int NL = Lanes<D, G>::NL;
        if constexpr (kFp32P) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                float mb = s[0][j];
#pragma unroll
                for (int i = 1; i < NL; ++i) mb = fmaxf(mb, s[i][j]);
                const float mn = fmaxf(m[j], mb);
                const bool live = mn != -INFINITY;
                const float alpha = live ? exp2f(m[j] - mn) : 1.f;
                m[j] = live ? mn : m[j];
                float lsum = 0.f;
                float o[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
                for (int i = 0; i < NL; ++i) {
                    const float pw = live && s[i][j] != -INFINITY ? exp2f(s[i][j] - mn) : 0.f;
                    float v[8];
                    unpack8(vr[i], v);
                    lsum += pw;
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[e] = fmaf(pw, v[e], o[e]);
                }
                l[j] = l[j] * alpha + lsum;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[j][e] = acc[j][e] * alpha + o[e];
            }
            return;
        }
        static_assert(NL % 2 == 0, "tokens are paired for P.V");
        // softmax of each query head first: P packed as bf16 token pairs, the old sums rescaled
        uint32_t pp[G][NL / 2];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            float mb = s[0][j];
#pragma unroll
            for (int i = 1; i < NL; ++i) mb = fmaxf(mb, s[i][j]);
            const float mn = fmaxf(m[j], mb);
            const bool live = mn != -INFINITY;  // else nothing seen yet: P = 0, state unchanged
            const float alpha = live ? exp2f(m[j] - mn) : 1.f;
            m[j] = live ? mn : m[j];
            float lsum = 0.f;
#pragma unroll
            for (int u = 0; u < NL / 2; ++u) {
                pp[j][u] = live ? pack_bf16x2(exp2f(s[2 * u][j] - mn), exp2f(s[2 * u + 1][j] - mn)) : 0u;
                lsum += __uint_as_float(pp[j][u] << 16) + __uint_as_float(pp[j][u] & 0xffff0000u);
            }
            l[j] = l[j] * alpha + lsum;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[j][e] *= alpha;
        }
        // then P.V over V words of token pairs (2u, 2u+1) interleaved as (v_a[e], v_b[e]), each
        // pair built just before its use so only one is live at a time
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int u = 0; u < NL / 2; ++u) {
                const uint32_t a = word(vr[2 * u], w), b = word(vr[2 * u + 1], w);
                const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05040100u);
                const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07060302u);
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    acc[j][2 * w] = dot2_bf16(pp[j][u], lo, acc[j][2 * w]);
                    acc[j][2 * w + 1] = dot2_bf16(pp[j][u], hi, acc[j][2 * w + 1]);
                }
            }
        }
    }

    // Fold the lane groups of the wave together (result valid in every lane).
    __device__ __forceinline__ void combine_lane_groups() {
        constexpr int LPT = Lanes<D, G>::LPT;
#pragma unroll
        for (int mask = LPT; mask < kWave; mask <<= 1) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float mo = __shfl_xor(m[j], mask, kWave);
                const float lo = __shfl_xor(l[j], mask, kWave);
                const float mn = fmaxf(m[j], mo);
                const float a = m[j] == -INFINITY ? 0.f : exp2f(m[j] - mn);
                const float bsc = mo == -INFINITY ? 0.f : exp2f(mo - mn);
                l[j] = l[j] * a + lo * bsc;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float ao = __shfl_xor(acc[j][e], mask, kWave);
                    acc[j][e] = acc[j][e] * a + ao * bsc;
                }
                m[j] = mn;
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Stream kernel for decode rows.

// Loads of one 16-token block, straight-line: tokens past the block's count
// or on an invalid page read slot 0 of a valid page and are masked, so all
// 2*NL loads are in flight together.  kSmallPages (page size < 16) looks each
// token's page up in kv_indices first.
template <int D, int G, bool kSmallPages>
__device__ __forceinline__ void stream_issue(const int4 &dsc, int h, const uint16_t *__restrict__ cache,
                                             int64_t c_page, int64_t c_kind, int64_t c_slot,
                                             int64_t c_head, int num_pages, int ps_log2,
                                             const int32_t *__restrict__ kv_indices, int index_limit,
                                             int g, int sub, uint4 (&kr)[Lanes<D, G>::NL],
                                             uint4 (&vr)[Lanes<D, G>::NL],
                                             bool (&valid)[Lanes<D, G>::NL], bool *bad) {
    constexpr int NL = Lanes<D, G>::NL;
    constexpr int TPL = Lanes<D, G>::TPL;
    const int ntok = static_cast<int>(static_cast<unsigned>(dsc.y) >> 24);
    const int slot0 = dsc.y & 0xffffff;
    const uint16_t *head_base = cache + h * c_head + sub * 8;
    int page[NL], slot[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int t = i * TPL + g;
        if constexpr (kSmallPages) {
            const int at = dsc.x + (t >> ps_log2);
            page[i] = (t < ntok && at < index_limit) ? kv_indices[at] : 0;
            slot[i] = t & ((1 << ps_log2) - 1);
        } else {
            page[i] = dsc.x;
            slot[i] = slot0 + t;
        }
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int t = i * TPL + g;
        const bool page_ok = static_cast<unsigned>(page[i]) < static_cast<unsigned>(num_pages);
        const bool in_block = t < ntok;
        if (in_block && !page_ok) *bad = true;
        valid[i] = in_block && page_ok;
        const int64_t off = static_cast<int64_t>(page_ok ? page[i] : 0) * c_page +
                            static_cast<int64_t>(valid[i] ? slot[i] : 0) * c_slot;
        kr[i] = *reinterpret_cast<const uint4 *>(head_base + off);
        vr[i] = *reinterpret_cast<const uint4 *>(head_base + off + c_kind);
    }
}

// stream_issue in two halves, so the K and V loads of a block can be issued at different times.
// BlockRef holds what the loads of one block need: for page sizes >= 16 a block lies in one page
// and the wave's tokens i*TPL + g sit at a fixed slot stride from one base offset (every slot of
// the page is a valid address, tokens past the block's count are masked); smaller pages keep one
// offset per token.
template <int D, int G, bool kSmallPages>
struct BlockRef {
    static constexpr int NL = Lanes<D, G>::NL;
    static constexpr int TPL = Lanes<D, G>::TPL;
    int64_t off[kSmallPages ? NL : 1];
    unsigned valid;  // bit i: token i*TPL + g is a real key

    __device__ __forceinline__ void make(const int4 &dsc, int64_t c_page, int64_t c_slot, int num_pages, int ps_log2,
                                         const int32_t *__restrict__ kv_indices, int index_limit, int g, bool *bad) {
        const int ntok = static_cast<int>(static_cast<unsigned>(dsc.y) >> 24);
        const int slot0 = dsc.y & 0xffffff;
        valid = 0;
        if constexpr (kSmallPages) {
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                const int t = i * TPL + g;
                const int at = dsc.x + (t >> ps_log2);
                const int page = (t < ntok && at < index_limit) ? kv_indices[at] : 0;
                const bool page_ok = static_cast<unsigned>(page) < static_cast<unsigned>(num_pages);
                if (t < ntok && !page_ok) *bad = true;
                const bool ok = t < ntok && page_ok;
                valid |= ok ? 1u << i : 0u;
                off[i] = static_cast<int64_t>(page_ok ? page : 0) * c_page +
                         static_cast<int64_t>(ok ? (t & ((1 << ps_log2) - 1)) : 0) * c_slot;
            }
        } else {
            const bool page_ok = static_cast<unsigned>(dsc.x) < static_cast<unsigned>(num_pages);
#pragma unroll
            for (int i = 0; i < NL; ++i) valid |= (i * TPL + g < ntok && page_ok) ? 1u << i : 0u;
            if (ntok > 0 && !page_ok) *bad = true;
            off[0] = static_cast<int64_t>(page_ok ? dsc.x : 0) * c_page + static_cast<int64_t>(slot0 + g) * c_slot;
        }
    }

    __device__ __forceinline__ void load(const uint16_t *__restrict__ base, int64_t c_slot, uint4 (&r)[NL]) const {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int64_t o = kSmallPages ? off[kSmallPages ? i : 0] : off[0] + static_cast<int64_t>(i * TPL) * c_slot;
            r[i] = *reinterpret_cast<const uint4 *>(base + o);
        }
    }

    __device__ __forceinline__ void flags(bool (&ok)[NL]) const {
#pragma unroll
        for (int i = 0; i < NL; ++i) ok[i] = (valid >> i) & 1u;
    }
};

__device__ __forceinline__ int4 shfl_int4(const int4 &v, int src) {
    return make_int4(__shfl(v.x, src, kWave), __shfl(v.y, src, kWave), __shfl(v.z, src, kWave),
                     __shfl(v.w, src, kWave));
}

__host__ __device__ __forceinline__ int span_start(int s, int n_blocks, int n_spans) {
    return static_cast<int>(static_cast<int64_t>(s) * n_blocks / n_spans);
}

// Spans per kv head: every head's block list is cut at the same places, so the
// Hkv waves of one span read the Hkv head slices of the same pages together.
__host__ __device__ __forceinline__ int stream_spans(int n_blocks, int span_cap) {
    int S = n_blocks / kMinBlocksPerWave;
    return S < 1 ? 1 : (S > span_cap ? span_cap : S);
}

// Span holding block b (largest s with span_start(s) <= b).
__device__ __forceinline__ int span_of(int b, int n_blocks, int n_spans) {
    int s = static_cast<int>(static_cast<int64_t>(b) * n_spans / n_blocks);
    while (s + 1 < n_spans && span_start(s + 1, n_blocks, n_spans) <= b) ++s;
    while (s > 0 && span_start(s, n_blocks, n_spans) > b) --s;
    return s;
}

template <int D, int G, bool kSmallPages>
__device__ __forceinline__ void
stream_body(const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1,
            const uint16_t *__restrict__ cache, int64_t c_page, int64_t c_kind, int64_t c_slot,
            int64_t c_head, int num_pages, const int32_t *__restrict__ kv_indices, int index_limit,
            int num_kv_heads, int ps_log2, float scale_log2, uint16_t *__restrict__ out,
            int64_t o_s0, int64_t o_s1, char *__restrict__ ws, const PlanLayout &L, int32_t *status) {
    using LN = Lanes<D, G>;
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    if (meta[kMetaStatus] != NQ_OK) {
        if (blockIdx.x == 0 && threadIdx.x == 0 && status) atomicExch(status, meta[kMetaStatus]);
        return;
    }
    const int n_dec = meta[kMetaDecRows];
    const int NBT = meta[kMetaBlocks];
    const int S = stream_spans(NBT, gridDim.x * kWaves / num_kv_heads);
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = blockIdx.x * kWaves + threadIdx.x / kWave;
    if (NBT == 0 || wid >= S * num_kv_heads) return;  // whole waves leave; no barriers below
    const int h_span = wid % num_kv_heads;
    const int span = wid / num_kv_heads;
    const int s0 = span_start(span, NBT, S);
    const int s1 = span_start(span + 1, NBT, S);
    const int4 *blocks = reinterpret_cast<const int4 *>(ws + L.blocks);
    const int4 *dec_rows = reinterpret_cast<const int4 *>(ws + L.dec_rows);
    float *part_ml = reinterpret_cast<float *>(ws + L.spart_ml);
    float *part_o = reinterpret_cast<float *>(ws + L.spart_o);
    const int g = lane / LN::LPT;
    const int sub = lane % LN::LPT;

    // Block descriptors of the span, 64 at a time, one per lane; (h, b) walk
    // the span without divisions.
    int win = s0;
    int4 dwin = make_int4(-1, 0, 0, 0);
    if (s0 + lane < s1) dwin = blocks[s0 + lane];

    SoftmaxState<D, G> st;
    st.reset();
    int cur_pair = -1, cur_query = 0, cur_h = 0, pair_lo = 0, pair_hi = 0;
    bool bad = false;

    const int h_cur = h_span;
    bool done = false;
    // Flush the finished (row, kv head) on a row change or at the span end:
    // final output if this wave saw all of its blocks, else an fp32 partial.
    auto enter = [&](int w, const int4 &dsc) {
        const int pair = w < s1 ? dsc.z : -2;  // decode row; the head is fixed per wave
        if (pair == cur_pair) return;
        if (cur_pair >= 0) {
            st.combine_lane_groups();
            if (g == 0) {
                if (pair_lo >= s0 && pair_hi <= s1) {
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        const float inv = st.l[j] > 0.f ? 1.0f / st.l[j] : 0.f;
                        uint4 o;
                        o.x = pack2_bf16(st.acc[j][0] * inv, st.acc[j][1] * inv);
                        o.y = pack2_bf16(st.acc[j][2] * inv, st.acc[j][3] * inv);
                        o.z = pack2_bf16(st.acc[j][4] * inv, st.acc[j][5] * inv);
                        o.w = pack2_bf16(st.acc[j][6] * inv, st.acc[j][7] * inv);
                        *reinterpret_cast<uint4 *>(out + cur_query * o_s0 + (cur_h * G + j) * o_s1 + sub * 8) = o;
                    }
                } else {
                    const int64_t slot = static_cast<int64_t>(span + cur_pair) * num_kv_heads + cur_h;
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        float *po = part_o + (slot * G + j) * D + sub * 8;
                        *reinterpret_cast<float4 *>(po) =
                            make_float4(st.acc[j][0], st.acc[j][1], st.acc[j][2], st.acc[j][3]);
                        *reinterpret_cast<float4 *>(po + 4) =
                            make_float4(st.acc[j][4], st.acc[j][5], st.acc[j][6], st.acc[j][7]);
                        if (sub == 0) {
                            part_ml[(slot * G + j) * 2] = st.m[j];
                            part_ml[(slot * G + j) * 2 + 1] = st.l[j];
                        }
                    }
                }
            }
        }
        if (w == s1) {
            done = true;
            return;
        }
        cur_pair = pair;
        cur_query = dsc.w;
        cur_h = h_cur;
        const int4 dr = dec_rows[dsc.z];
        pair_lo = dr.z;
        pair_hi = pair_lo + dr.w;
        st.reset();
        st.load_q(q + cur_query * q_s0, q_s1, h_cur, sub, scale_log2);
    };
    auto desc_of = [&](int w) {
        if (w - win >= kWave) {
            win += kWave;
            dwin = win + lane < s1 ? blocks[win + lane] : make_int4(-1, 0, 0, 0);
        }
        return shfl_int4(dwin, w - win);
    };
    if constexpr (!kStreamDoubleBuffer) {
        uint4 kc[LN::NL], vc[LN::NL];
        bool okc[LN::NL];
        for (int w = s0;; ++w) {
            const int4 dc = w < s1 ? desc_of(w) : make_int4(-1, 0, 0, 0);
            enter(w, dc);
            if (done) break;
            stream_issue<D, G, kSmallPages>(dc, h_cur, cache, c_page, c_kind, c_slot, c_head, num_pages,
                                            ps_log2, kv_indices, index_limit, g, sub, kc, vc, okc, &bad);
            st.consume(kc, vc, okc);
        }
        if (bad && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
        return;
    }
    // Two register buffers alternate: while one block is consumed the loads of
    // the next are in flight.
    uint4 ka[LN::NL], va[LN::NL], kb[LN::NL], vb[LN::NL];
    bool oka[LN::NL], okb[LN::NL];
    int4 da = desc_of(s0), db = make_int4(-1, 0, 0, 0);
    stream_issue<D, G, kSmallPages>(da, h_cur, cache, c_page, c_kind, c_slot, c_head, num_pages, ps_log2,
                                    kv_indices, index_limit, g, sub, ka, va, oka, &bad);
    for (int w = s0;; w += 2) {
        if (w + 1 < s1) {
            db = desc_of(w + 1);
            stream_issue<D, G, kSmallPages>(db, h_cur, cache, c_page, c_kind, c_slot, c_head, num_pages,
                                            ps_log2, kv_indices, index_limit, g, sub, kb, vb, okb, &bad);
        }
        enter(w, da);
        if (done) break;
        st.consume(ka, va, oka);
        if (w + 2 < s1) {
            da = desc_of(w + 2);
            stream_issue<D, G, kSmallPages>(da, h_cur, cache, c_page, c_kind, c_slot, c_head, num_pages,
                                            ps_log2, kv_indices, index_limit, g, sub, ka, va, oka, &bad);
        }
        enter(w + 1, db);
        if (done) break;
        st.consume(kb, vb, okb);
    }
    if (bad && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
}

#define NQ_STREAM_ARGS                                                                            \
    const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1, const uint16_t *__restrict__ cache, \
        int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head, int num_pages,             \
        const int32_t *__restrict__ kv_indices, int index_limit, int num_kv_heads, int ps_log2,     \
        float scale_log2, uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1,                   \
        char *__restrict__ ws, PlanLayout L, int32_t *status
#define NQ_STREAM_PASS                                                                             \
    q, q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices, index_limit,      \
        num_kv_heads, ps_log2, scale_log2, out, o_s0, o_s1, ws, L, status

// Up to two query heads per kv head the state fits 128 VGPRs: four waves per
// SIMD stay resident, so the 4096 waves of a launch run in a single round.
template <int D, int G, bool kSmallPages>
__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
paged_stream_kernel_occ4(NQ_STREAM_ARGS) {
    stream_body<D, G, kSmallPages>(NQ_STREAM_PASS);
}

template <int D, int G, bool kSmallPages>
__global__ void __launch_bounds__(kAttnThreads) paged_stream_kernel(NQ_STREAM_ARGS) {
    stream_body<D, G, kSmallPages>(NQ_STREAM_PASS);
}

// Merge the stream partials of each (decode row, kv head) pair that more than
// one wave touched: one workgroup per pair, one thread per output element.
template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
merge_stream_kernel(const char *__restrict__ ws, PlanLayout L, int num_kv_heads, int worker_cap, int max_rows,
                    uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1) {
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    const int4 *dec_rows = reinterpret_cast<const int4 *>(ws + L.dec_rows);
    const float *part_ml = reinterpret_cast<const float *>(ws + L.spart_ml);
    const float *part_o = reinterpret_cast<const float *>(ws + L.spart_o);
    // pair p = (decode row j, kv head h) with j = p / Hkv: the row descriptor load does not wait
    // for the plan's counters
    for (int p = blockIdx.x; p < max_rows * num_kv_heads; p += gridDim.x) {
        const int j = p / num_kv_heads, h = p - j * num_kv_heads;
        const int4 dr = dec_rows[j];
        if (meta[kMetaStatus] != NQ_OK) return;
        const int n_dec = meta[kMetaDecRows];
        const int NBT = meta[kMetaBlocks];
        if (j >= n_dec || NBT == 0) return;  // pairs only grow with p
        const int S = stream_spans(NBT, worker_cap / num_kv_heads);
        const int i0 = span_of(dr.z, NBT, S);
        const int i1 = span_of(dr.z + dr.w - 1, NBT, S);
        if (i0 == i1) continue;  // one wave saw the whole row and wrote it
        for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
            const int jj = t / D, d = t % D;
            // up to 16 contributors per round: all their (m, l, o) loads in flight together
            constexpr int kR = 16;
            float mx = -INFINITY, ls = 0.f, os = 0.f;
            for (int c0 = i0; c0 <= i1; c0 += kR) {
                float mk[kR], lk[kR], ok[kR];
#pragma unroll
                for (int u = 0; u < kR; ++u) {
                    mk[u] = -INFINITY;
                    lk[u] = 0.f;
                    ok[u] = 0.f;
                    if (c0 + u <= i1) {
                        const int64_t slot = static_cast<int64_t>(c0 + u + j) * num_kv_heads + h;
                        mk[u] = part_ml[(slot * G + jj) * 2];
                        lk[u] = part_ml[(slot * G + jj) * 2 + 1];
                        ok[u] = part_o[(slot * G + jj) * D + d];
                    }
                }
                float cm = mx;
#pragma unroll
                for (int u = 0; u < kR; ++u) cm = fmaxf(cm, mk[u]);
                if (cm == -INFINITY) continue;
                const float keep = mx == -INFINITY ? 0.f : exp2f(mx - cm);
                ls *= keep;
                os *= keep;
#pragma unroll
                for (int u = 0; u < kR; ++u) {
                    const float sc = mk[u] == -INFINITY ? 0.f : exp2f(mk[u] - cm);
                    ls += lk[u] * sc;
                    os += ok[u] * sc;
                }
                mx = cm;
            }
            out[dr.y * o_s0 + (h * G + jj) * o_s1 + d] = f32_to_bf16(ls > 0.f ? os / ls : 0.f);
        }
    }
}

// ---------------------------------------------------------------------------
// Fused decode kernel over bins, for batches of decode rows.
//
// Workgroup (bin b, kv head h) = blockIdx b * Hkv + h, W waves.  Prologue:
// for every piece of the bin the G query heads of kv head h of its row are
// normalised and rotated from the packed QKV projection's split-K planes into
// LDS, and the piece holding the row's last block also writes the new token's
// K (normalised, rotated) and V into its cache slot -- the q/k norm + RoPE +
// KV write of nq_qkv_partials_norm_rope_kv_write, through the same
// norm_rope_pair arithmetic.  After a barrier the bin's blocks (its pieces'
// blocks in slot order) are cut into W equal spans, one per wave, and
// streamed as in the stream kernel.  A piece wholly inside a span is finished
// in registers; the (at most two) boundary pieces of a span leave their
// (m, l, acc) in LDS and are merged in wave order after a second barrier.  A
// finished piece of an unsplit row is that row's output (bf16).  A row split
// across bins (only rows longer than a bin's share) leaves fp32 piece
// partials, written and read with agent-scope relaxed atomics (coherent across
// the XCDs' L2s without a cache flush) and ordered by waiting for the stores
// before an arrival count on the (row, kv head) counter; the piece that
// completes the count merges all pieces in piece order and resets the counter.
// No workgroup waits for another, and unsplit rows pay nothing for this.

struct RopeSrc {
    const float *partials;  // [splits][tokens][(Hq + 2 Hkv) D] fp32 planes
    int splits, tokens;
    int64_t plane, row;
    const uint16_t *q_weight, *k_weight;
    const int64_t *positions, *write_pages, *write_offsets;
    float eps, log_theta;
    int round_to_input;
    // bf16 query [tokens, Hq, D] already rotated (the kernel's q-input mode: no
    // planes, no norm / RoPE, no K/V write -- the caller's rope kernel did them)
    const uint16_t *q;
    int64_t q_s0, q_s1;
};

template <int D, int G>
struct BinPart {
    static constexpr int kFloats = G * D + 2 * G;  // acc [G][D], then (m, l) per head
};

// Finished piece from a merge-layout lane (elements e0 .. e0 + V of the G*D
// outputs): bf16 output of an unsplit row, else the piece's fp32 partial.
template <int D, int G, int V>
__device__ __forceinline__ void bin_store(const float (&os)[V], float mx, float ls, int e0, bool split, int pid, int h,
                                          int query, int Hq, uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1,
                                          float *__restrict__ piece_ml, float *__restrict__ piece_o) {
    const int jj = e0 / D, d0 = e0 - jj * D;
    const int qh = h * G + jj;
    if (!split) {
        const float inv = ls > 0.f ? 1.0f / ls : 0.f;
        uint16_t *op = out + query * o_s0 + qh * o_s1 + d0;
#pragma unroll
        for (int v = 0; v < V; ++v) op[v] = f32_to_bf16(os[v] * inv);
        return;
    }
    float *po = piece_o + (static_cast<int64_t>(pid) * Hq + qh) * D + d0;
#pragma unroll
    for (int v = 0; v < V; ++v) __hip_atomic_store(po + v, os[v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d0 == 0) {
        __hip_atomic_store(piece_ml + (static_cast<int64_t>(pid) * Hq + qh) * 2, mx, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(piece_ml + (static_cast<int64_t>(pid) * Hq + qh) * 2 + 1, ls, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wave that has stored its piece of a split row counts the arrival; the
// piece completing the count merges the row's pieces (whole wave, G*D outputs).
template <int D, int G>
__device__ __forceinline__ void bin_arrive(int4 pc, int h, int num_kv_heads, int query, int lane,
                                           int32_t *__restrict__ arrivals, const float *__restrict__ piece_ml,
                                           const float *__restrict__ piece_o, uint16_t *__restrict__ out,
                                           int64_t o_s0, int64_t o_s1) {
    // The arrival count is an agent-scope acquire-release operation: it publishes this piece's
    // stores (release) and, for the piece that completes the count, makes every other piece's
    // stores visible to the merge below (acquire).
    int32_t *counter = arrivals + pc.x * num_kv_heads + h;
    int before = 0;
    if (lane == 0) before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    before = __shfl(before, 0, kWave);
    const int p0 = pc.w >> 9, k = pc.w & 511;
    if (before != k - 1) return;
    const int Hq = num_kv_heads * G;
    for (int t = lane; t < G * D; t += kWave) {
        const int jj = t / D, d = t - jj * D;
        const int qh = h * G + jj;
        float mx = -INFINITY, ls = 0.f, os = 0.f;
        for (int q = p0; q < p0 + k; ++q) {
            const float mk = coherent_load(piece_ml + (static_cast<int64_t>(q) * Hq + qh) * 2);
            const float lk = coherent_load(piece_ml + (static_cast<int64_t>(q) * Hq + qh) * 2 + 1);
            const float ok = coherent_load(piece_o + (static_cast<int64_t>(q) * Hq + qh) * D + d);
            if (mk == -INFINITY) continue;
            const float cm = fmaxf(mx, mk);
            const float keep = mx == -INFINITY ? 0.f : exp2f(mx - cm);
            const float sc = exp2f(mk - cm);
            ls = ls * keep + lk * sc;
            os = os * keep + ok * sc;
            mx = cm;
        }
        out[query * o_s0 + qh * o_s1 + d] = f32_to_bf16(ls > 0.f ? os / ls : 0.f);
    }
    if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int G, bool kSmallPages, bool kQIn, int W>
__global__ void __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(4, 8)))
bin_decode_kernel(RopeSrc rs, uint16_t *__restrict__ cache, int64_t c_page, int64_t c_kind, int64_t c_slot,
                  int64_t c_head, int num_pages, const int32_t *__restrict__ kv_indices, int index_limit,
                  int num_kv_heads, int ps_log2, float scale_log2, uint16_t *__restrict__ out, int64_t o_s0,
                  int64_t o_s1, char *__restrict__ ws, PlanLayout L, int32_t *status) {
    using LN = Lanes<D, G>;
    constexpr int kPart = BinPart<D, G>::kFloats;
    constexpr int HALF = D / 2;
    __shared__ int4 s_piece[kBinMaxSlots];
    __shared__ int4 s_rope[kBinMaxSlots];  // {query token, position, write page, write offset | last << 31}
    __shared__ int s_pid[kBinMaxSlots];
    __shared__ int s_start[kBinMaxSlots + 1];
    __shared__ int s_n;
    __shared__ __attribute__((aligned(16))) uint16_t s_q[kBinMaxSlots * G * D];
    __shared__ __attribute__((aligned(16))) float s_part[W * 2 * kPart];
    __shared__ int s_wsp[W + 1];  // wave span starts

    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    const int NB = bins_per_head(num_kv_heads);
    const int bin = blockIdx.x / num_kv_heads, h = blockIdx.x - (blockIdx.x / num_kv_heads) * num_kv_heads;
    if (bin >= NB) return;
    // one round trip: the plan's status and slot count, and this bin's table row
    // (fixed stride, so its address does not wait for either)
    const int4 *table = reinterpret_cast<const int4 *>(ws + L.bins) + static_cast<int64_t>(bin) * kBinMaxSlots * 3;
    int4 t_piece = make_int4(-1, 0, 0, -1), t_rope = make_int4(0, 0, -1, 0), t_id = make_int4(-1, 0, 0, 0);
    if (threadIdx.x < kBinMaxSlots) {
        t_piece = table[3 * threadIdx.x];
        t_rope = table[3 * threadIdx.x + 1];
        t_id = table[3 * threadIdx.x + 2];
    }
    const int plan_status = meta[kMetaStatus], slots = meta[kMetaBinSlots];
    if (plan_status != NQ_OK) {
        if (blockIdx.x == 0 && threadIdx.x == 0 && status) atomicExch(status, plan_status);
        return;
    }
    if (slots <= 0) return;
    if (slots > kBinMaxSlots) {
        if (threadIdx.x == 0 && status) atomicExch(status, NQ_ERR_CAPACITY);
        return;
    }
    const int4 *blocks = reinterpret_cast<const int4 *>(ws + L.blocks);
    float *piece_ml = reinterpret_cast<float *>(ws + L.piece_ml);
    float *piece_o = reinterpret_cast<float *>(ws + L.piece_o);
    int32_t *arrivals = reinterpret_cast<int32_t *>(ws + L.arrivals);
    const int Hq = num_kv_heads * G;

    // the bin's pieces (empty slots come last) and their block offsets
    if (threadIdx.x < slots) {
        s_pid[threadIdx.x] = t_id.x;
        s_piece[threadIdx.x] = t_piece;
        s_rope[threadIdx.x] = t_rope;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0, n = 0;
        for (int i = 0; i < slots; ++i) {
            s_start[i] = acc;
            if (s_pid[i] >= 0) {
                acc += s_piece[i].z;
                n = i + 1;
            }
        }
        s_start[slots] = acc;
        for (int i = n; i <= slots; ++i) s_start[i] = acc;
        s_n = n;
    }
    __syncthreads();
    const int nslots = s_n;
    const int NBB = s_start[nslots];
    if (NBB == 0) return;
    if (threadIdx.x <= W) s_wsp[threadIdx.x] = span_start(threadIdx.x, NBB, W);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    bool bad = false;

    // the wave's span of the bin's blocks and its first 64 block descriptors
    // (one per lane: lane -> bin-local block -> global block), fetched now so
    // that they arrive during the RoPE work below
    const int s0 = span_start(wave, NBB, W);
    const int s1 = span_start(wave + 1, NBB, W);
    auto global_block = [&](int lb) {
        int sl = 0;
        while (sl + 1 < nslots && s_start[sl + 1] <= lb) ++sl;
        return s_piece[sl].y + lb - s_start[sl];
    };
    int win = s0;
    int4 dwin = make_int4(-1, 0, 0, 0);
    if (s0 + lane < s1) dwin = blocks[global_block(s0 + lane)];

    const int g = lane / LN::LPT;
    const int sub = lane % LN::LPT;
    const uint16_t *head_base = cache + h * c_head + sub * 8;

    // 1. q/k norm + RoPE + K/V write for the bin's rows (one wave per head unit);
    // the norm weights are in registers before the first unit's planes arrive
    float qw1 = 0.f, qw2 = 0.f, kw1 = 0.f, kw2 = 0.f;
    if (lane < HALF) {
        qw1 = bf16_to_f32(rs.q_weight[lane]);
        qw2 = bf16_to_f32(rs.q_weight[lane + HALF]);
        kw1 = bf16_to_f32(rs.k_weight[lane]);
        kw2 = bf16_to_f32(rs.k_weight[lane + HALF]);
    }
    if constexpr (kQIn) {
        // q-input mode: the bin's rotated query heads into LDS, one wave per (piece, head)
        for (int u = wave; u < nslots * G; u += W) {
            const int sl = u / G, j = u - sl * G;
            const int64_t tok = s_rope[sl].x;
            if (tok >= rs.tokens) {
                bad = true;
                continue;
            }
            const uint16_t *qh = rs.q + tok * rs.q_s0 + (h * G + j) * rs.q_s1;
            for (int d = lane; d < D; d += kWave) s_q[(sl * G + j) * D + d] = qh[d];
        }
    }
    for (int u = wave; u < (kQIn ? 0 : nslots * (G + 2)); u += W) {
        const int sl = u / (G + 2), kind = u - sl * (G + 2);
        const int4 rp = s_rope[sl];
        const bool row_last = rp.w < 0;
        if (kind >= G && !row_last) continue;  // the row's new K/V belong to its last piece
        const int64_t tok = rp.x;
        if (tok >= rs.tokens) {  // a query beyond the projection's rows
            bad = true;
            continue;
        }
        const int col = kind < G ? (h * G + kind) * D : (kind == G ? Hq + h : Hq + num_kv_heads + h) * D;
        const bool on = lane < HALF;
        float x1 = 0.f, x2 = 0.f;
        if (on) {
            // the split-K planes four at a time (all loads in flight together),
            // added in plane order
            const float *e = rs.partials + tok * rs.row + col + lane;
            for (int i0 = 0; i0 < rs.splits; i0 += 4) {
                float a[4], c[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const bool ok = i0 + v < rs.splits;
                    a[v] = ok ? e[(i0 + v) * rs.plane] : 0.f;
                    c[v] = ok ? e[(i0 + v) * rs.plane + HALF] : 0.f;
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (i0 + v < rs.splits) {
                        x1 += a[v];
                        x2 += c[v];
                    }
                }
            }
            x1 = bf16_to_f32(f32_to_bf16(x1));
            x2 = bf16_to_f32(f32_to_bf16(x2));
        }
        const int64_t page = rp.z, woff = rp.w & 0x7fffffff;
        const bool slot_ok = static_cast<uint64_t>(page) < static_cast<uint64_t>(num_pages) &&
                             static_cast<uint64_t>(woff) < (static_cast<uint64_t>(1) << ps_log2);
        if (kind >= G && !slot_ok) {
            bad = true;
            continue;
        }
        uint16_t *cslot = cache + page * c_page + woff * c_slot + h * c_head;
        if (kind == G + 1) {
            if (on) {
                cslot[c_kind + lane] = f32_to_bf16(x1);
                cslot[c_kind + lane + HALF] = f32_to_bf16(x2);
            }
            continue;
        }
        uint16_t o1 = 0, o2 = 0;
        norm_rope_pair<D>(x1, x2, on, kind < G ? qw1 : kw1, kind < G ? qw2 : kw2, lane, rs.eps, rs.log_theta,
                          static_cast<float>(rp.y), rs.round_to_input, o1, o2);
        if (!on) continue;
        if (kind < G) {
            s_q[(sl * G + kind) * D + lane] = o1;
            s_q[(sl * G + kind) * D + lane + HALF] = o2;
        } else {
            cslot[lane] = o1;
            cslot[lane + HALF] = o2;
        }
    }
    // the span's first block goes in flight as soon as the wave's RoPE units are done (at once for
    // the waves without any), under the other waves' RoPE work and the barrier, unless it is the
    // block that receives a row's new K/V (written by this workgroup before the barrier)
    uint4 kc[LN::NL], vc[LN::NL];
    BlockRef<D, G, kSmallPages> ref;
    bool issued = false;
    if (s0 < s1) {
        int sl0 = 0;
        while (sl0 + 1 < nslots && s_start[sl0 + 1] <= s0) ++sl0;
        const bool write_block = !kQIn && s_rope[sl0].w < 0 && s0 == s_start[sl0 + 1] - 1;
        if (!write_block) {
            ref.make(shfl_int4(dwin, 0), c_page, c_slot, num_pages, ps_log2, kv_indices, index_limit, g, &bad);
            ref.load(head_base, c_slot, kc);
            ref.load(head_base + c_kind, c_slot, vc);
            issued = true;
        }
    }
    __syncthreads();  // rotated q in LDS, the new K/V in the cache for every wave of the workgroup

    // 2. stream the wave's span of the bin's blocks
    if (s0 < s1) {
        // further descriptors of the span, 64 at a time
        auto desc_of = [&](int w) {
            if (w - win >= kWave) {
                win += kWave;
                dwin = win + lane < s1 ? blocks[global_block(win + lane)] : make_int4(-1, 0, 0, 0);
            }
            return shfl_int4(dwin, w - win);
        };
        SoftmaxState<D, G> st;
        int cur = -1;
        while (s_start[cur + 1] <= s0) ++cur;  // slot of the span's first block
        st.reset();
        st.load_q(s_q + cur * G * D, D, 0, sub, scale_log2);
        // finish slot sl's part of this span: whole pieces go out, boundary ones to LDS
        auto flush = [&](int sl) {
            st.combine_lane_groups();
            const bool whole = s_start[sl] >= s0 && s_start[sl + 1] <= s1;
            if (whole) {
                const int4 pc = s_piece[sl];
                const int query = s_rope[sl].x;
                if (g == 0) {
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        float os[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) os[e] = st.acc[j][e];
                        bin_store<D, G, 8>(os, st.m[j], st.l[j], j * D + sub * 8, pc.w >= 0, s_pid[sl], h, query, Hq,
                                           out, o_s0, o_s1, piece_ml, piece_o);
                    }
                }
                if (pc.w >= 0)
                    bin_arrive<D, G>(pc, h, num_kv_heads, query, lane, arrivals, piece_ml, piece_o, out, o_s0, o_s1);
            } else if (g == 0) {
                float *pp = s_part + (wave * 2 + (s_start[sl] > s0 ? 1 : 0)) * kPart;
#pragma unroll
                for (int j = 0; j < G; ++j) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) pp[j * D + sub * 8 + e] = st.acc[j][e];
                    if (sub == 0) {
                        pp[G * D + 2 * j] = st.m[j];
                        pp[G * D + 2 * j + 1] = st.l[j];
                    }
                }
            }
        };
        for (int w = s0; w < s1; ++w) {
            if (w == s_start[cur + 1]) {
                flush(cur);
                ++cur;
                st.reset();
                st.load_q(s_q + cur * G * D, D, 0, sub, scale_log2);
            }
            if (w != s0 || !issued) {
                ref.make(desc_of(w), c_page, c_slot, num_pages, ps_log2, kv_indices, index_limit, g, &bad);
                ref.load(head_base, c_slot, kc);
                ref.load(head_base + c_kind, c_slot, vc);
            }
            bool ok[LN::NL];
            ref.flags(ok);
            st.consume(kc, vc, ok);
        }
        flush(cur);
    }
    if (bad && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
    __syncthreads();

    // 3. pieces shared by several waves: merge their LDS partials.  All
    // contributors' maxima are read at once and the row maximum taken first,
    // then every (l, o) is read independently and added with its scale in
    // wave order, so the merge costs a few LDS round trips instead of one
    // chain per contributor (and stays deterministic).  The work is dealt to
    // every wave as (piece, 64 outputs) units, one output per lane; a split
    // piece (partial to global memory, then its arrival counted) stays one
    // unit of a whole wave.  Each output's arithmetic is the same either way.
    constexpr int EPL = G * D / kWave;  // outputs per lane for a whole piece; also 64-output units per piece
    constexpr int V = EPL < 4 ? EPL : 4;
    constexpr int NG = EPL / V;
    // wave span starts in registers; the wave whose span holds bin-local block b
    // is the number of later span starts <= b (they never decrease)
    int wsp[W + 1];
#pragma unroll
    for (int w = 0; w <= W; ++w) wsp[w] = s_wsp[w];
    auto wave_of = [&](int b) {
        int w = 0;
#pragma unroll
        for (int i = 1; i < W; ++i) w += wsp[i] <= b ? 1 : 0;
        return w;
    };
    // merge VV consecutive outputs from e0 of the piece in bin-local blocks [a, b) held by waves w0..w1
    auto merge = [&](auto vtag, int sl, int a, int w0, int w1, int e0) {
        constexpr int VV = decltype(vtag)::value;
        const int jj = e0 / D;
        // wave w contributes when w0 <= w <= w1 and its span is not empty (bins
        // of < 16 blocks); its partial of this piece is its first slot when the
        // piece starts in its span, else its second.  Every slot read stays
        // inside s_part; a non-contributor's value (its slot may never have
        // been written) is dropped by a select, never multiplied in.
        float mk[W];
        int base[W];
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const bool on = w >= w0 && w <= w1 && wsp[w] != wsp[w + 1];
            base[w] = (w * 2 + (a > wsp[w] ? 1 : 0)) * kPart;
            const float m = s_part[base[w] + G * D + 2 * jj];
            mk[w] = on ? m : -INFINITY;
            mx = fmaxf(mx, mk[w]);
        }
        float ls = 0.f, os[VV];
#pragma unroll
        for (int v = 0; v < VV; ++v) os[v] = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const bool on = mk[w] != -INFINITY;
            const float sc = on ? exp2f(mk[w] - mx) : 0.f;
            const float *pp = s_part + base[w];
            const float lk = pp[G * D + 2 * jj + 1];
            ls += on ? lk * sc : 0.f;
#pragma unroll
            for (int v = 0; v < VV; ++v) {
                const float ov = pp[e0 + v];
                os[v] += on ? ov * sc : 0.f;
            }
        }
        bin_store<D, G, VV>(os, mx, ls, e0, s_piece[sl].w >= 0, s_pid[sl], h, s_rope[sl].x, Hq, out, o_s0, o_s1,
                            piece_ml, piece_o);
    };
    for (int u = wave; u < nslots * EPL; u += W) {
        const int sl = u / EPL, unit = u - sl * EPL;
        const int a = s_start[sl], b = s_start[sl + 1];
        if (a == b) continue;
        const int w0 = wave_of(a), w1 = wave_of(b - 1);
        if (w0 == w1) continue;  // finished by its wave
        const int4 pc = s_piece[sl];
        if (pc.w < 0) {
            merge(std::integral_constant<int, 1>(), sl, a, w0, w1, unit * kWave + lane);
            continue;
        }
        if (unit != 0) continue;
        for (int grp = 0; grp < NG; ++grp) merge(std::integral_constant<int, V>(), sl, a, w0, w1, (grp * kWave + lane) * V);
        bin_arrive<D, G>(pc, h, num_kv_heads, s_rope[sl].x, lane, arrivals, piece_ml, piece_o, out, o_s0, o_s1);
    }
}

// ---------------------------------------------------------------------------
// Chunk kernel for causal prefill queries and the dense short-cache kernel:
// a workgroup per (query, chunk, kv head); waves split the chunk's blocks.

struct Smem {
    float m[kWaves][8];
    float l[kWaves][8];
    float acc[kWaves][8][128];
    int pages[kMaxChunkTokens];
};

// Attend G query heads of kv head h to `ntok` keys; key position `rel` lives in
// page page_of(rel) at slot slot_of(rel).  Leaves per-wave states in `sm`.
template <int D, int G, bool kFp32P = false, typename PageOf, typename SlotOf>
__device__ __forceinline__ void attend_chunk(const uint16_t *__restrict__ qptr, int64_t q_s1,
                                             const uint16_t *__restrict__ cache, int64_t c_page,
                                             int64_t c_kind, int64_t c_slot, int64_t c_head, int h,
                                             int ntok, int page_limit, float scale_log2,
                                             PageOf page_of, SlotOf slot_of, Smem &sm, bool *bad) {
    using LN = Lanes<D, G>;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int g = lane / LN::LPT;
    const int sub = lane % LN::LPT;
    SoftmaxState<D, G, kFp32P> st;
    st.reset();
    st.load_q(qptr, q_s1, h, sub, scale_log2);
    const uint16_t *head_base = cache + h * c_head + sub * 8;
    const int nblk = ntok > 0 ? (ntok + kBlockTok - 1) / kBlockTok : 0;
    for (int b = wave; b < nblk; b += kWaves) {
        uint4 kr[LN::NL], vr[LN::NL];
        bool valid[LN::NL];
        int page[LN::NL];
#pragma unroll
        for (int i = 0; i < LN::NL; ++i) {
            const int rel = b * kBlockTok + i * LN::TPL + g;
            page[i] = rel < ntok ? page_of(rel) : 0;
        }
#pragma unroll
        for (int i = 0; i < LN::NL; ++i) {
            const int rel = b * kBlockTok + i * LN::TPL + g;
            const bool page_ok = static_cast<unsigned>(page[i]) < static_cast<unsigned>(page_limit);
            const bool in_range = rel < ntok;
            if (in_range && !page_ok) *bad = true;
            valid[i] = in_range && page_ok;
            const int64_t off = static_cast<int64_t>(page_ok ? page[i] : 0) * c_page +
                                static_cast<int64_t>(valid[i] ? slot_of(rel) : 0) * c_slot;
            kr[i] = *reinterpret_cast<const uint4 *>(head_base + off);
            vr[i] = *reinterpret_cast<const uint4 *>(head_base + off + c_kind);
        }
        st.consume(kr, vr, valid);
    }
    st.combine_lane_groups();
    if (g == 0) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (sub == 0) {
                sm.m[wave][j] = st.m[j];
                sm.l[wave][j] = st.l[j];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) sm.acc[wave][j][sub * 8 + e] = st.acc[j][e];
        }
    }
    __syncthreads();
}

template <int D>
__device__ __forceinline__ void wave_combine(const Smem &sm, int t, float *M, float *Lsum, float *O) {
    const int j = t / D, d = t % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sm.m[w][j]);
    float ls = 0.f, os = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = sm.m[w][j];
            const float sc = mw == -INFINITY ? 0.f : exp2f(mw - mx);
            ls += sm.l[w][j] * sc;
            os += sm.acc[w][j][d] * sc;
        }
    }
    *M = mx;
    *Lsum = ls;
    *O = os;
}

template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
paged_chunk_kernel(const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1,
                   const uint16_t *__restrict__ cache, int64_t c_page, int64_t c_kind,
                   int64_t c_slot, int64_t c_head, int num_pages,
                   const int32_t *__restrict__ kv_indices, int index_limit, int num_kv_heads,
                   int ps_log2, float scale_log2, uint16_t *__restrict__ out, int64_t o_s0,
                   int64_t o_s1, char *__restrict__ ws, PlanLayout L, int32_t *status) {
    __shared__ Smem sm;
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    const ChunkDesc *desc = reinterpret_cast<const ChunkDesc *>(ws + L.desc);
    float *part_ml = reinterpret_cast<float *>(ws + L.part_ml);
    float *part_o = reinterpret_cast<float *>(ws + L.part_o);
    if (meta[kMetaStatus] != NQ_OK) return;
    const int n_chunks = meta[kMetaChunks];
    const int Hq = num_kv_heads * G;
    const int64_t n_items = static_cast<int64_t>(n_chunks) * num_kv_heads;
    const int ps = 1 << ps_log2;
    bool bad = false;
    for (int64_t w = blockIdx.x; w < n_items; w += gridDim.x) {
        const int c = static_cast<int>(w / num_kv_heads);
        const int h = static_cast<int>(w - static_cast<int64_t>(c) * num_kv_heads);
        const ChunkDesc d = desc[c];
        const int ntok = d.tok_end - d.tok_begin;
        const int npg = (ntok + ps - 1) >> ps_log2;
        for (int t = threadIdx.x; t < npg; t += kAttnThreads) {
            const int at = d.page_start + t;
            sm.pages[t] = at < index_limit ? kv_indices[at] : -1;
        }
        __syncthreads();
        attend_chunk<D, G>(
            q + d.query * q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, h, ntok, num_pages,
            scale_log2, [&](int rel) { return sm.pages[rel >> ps_log2]; },
            [&](int rel) { return rel & (ps - 1); }, sm, &bad);
        for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
            float M, Ls, O;
            wave_combine<D>(sm, t, &M, &Ls, &O);
            const int j = t / D, dd = t % D;
            if (d.n_chunks == 1) {
                out[d.query * o_s0 + (h * G + j) * o_s1 + dd] = f32_to_bf16(Ls > 0.f ? O / Ls : 0.f);
            } else {
                const int64_t hh = static_cast<int64_t>(c) * Hq + h * G + j;
                part_o[hh * D + dd] = O;
                if (dd == 0) {
                    part_ml[hh * 2] = M;
                    part_ml[hh * 2 + 1] = Ls;
                }
            }
        }
        __syncthreads();
    }
    if (bad && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
}

template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
merge_chunks_kernel(const char *__restrict__ ws, PlanLayout L, int num_kv_heads,
                    uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1) {
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    if (meta[kMetaStatus] != NQ_OK) return;
    const int T = meta[kMetaQueries];
    const int32_t *chunk_indptr = reinterpret_cast<const int32_t *>(ws + L.chunk_indptr);
    const float *part_ml = reinterpret_cast<const float *>(ws + L.part_ml);
    const float *part_o = reinterpret_cast<const float *>(ws + L.part_o);
    const int Hq = num_kv_heads * G;
    const int64_t n_items = static_cast<int64_t>(T) * num_kv_heads;
    for (int64_t w = blockIdx.x; w < n_items; w += gridDim.x) {
        const int qi = static_cast<int>(w / num_kv_heads);
        const int h = static_cast<int>(w - static_cast<int64_t>(qi) * num_kv_heads);
        const int c0 = chunk_indptr[qi];
        const int nk = chunk_indptr[qi + 1] - c0;
        if (nk <= 1) continue;
        for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
            const int j = t / D, dd = t % D;
            float mx = -INFINITY;
            for (int k = 0; k < nk; ++k)
                mx = fmaxf(mx, part_ml[(static_cast<int64_t>(c0 + k) * Hq + h * G + j) * 2]);
            float ls = 0.f, os = 0.f;
            if (mx != -INFINITY) {
#pragma unroll 4
                for (int k = 0; k < nk; ++k) {
                    const int64_t hh = static_cast<int64_t>(c0 + k) * Hq + h * G + j;
                    const float mk = part_ml[hh * 2];
                    const float sc = mk == -INFINITY ? 0.f : exp2f(mk - mx);
                    ls += part_ml[hh * 2 + 1] * sc;
                    os += part_o[hh * D + dd] * sc;
                }
            }
            out[qi * o_s0 + (h * G + j) * o_s1 + dd] = f32_to_bf16(ls > 0.f ? os / ls : 0.f);
        }
    }
}

template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
dense_short_kernel(const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1,
                   const uint16_t *__restrict__ cache, int64_t c_row, int64_t c_kind, int64_t c_pos,
                   int64_t c_head, int rows, int valid_length, int num_kv_heads, float scale_log2,
                   uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1) {
    __shared__ Smem sm;
    const int64_t n_items = static_cast<int64_t>(rows) * num_kv_heads;
    bool bad = false;
    for (int64_t w = blockIdx.x; w < n_items; w += gridDim.x) {
        const int row = static_cast<int>(w / num_kv_heads);
        const int h = static_cast<int>(w - static_cast<int64_t>(row) * num_kv_heads);
        attend_chunk<D, G, true>(
            q + row * q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, h, valid_length, rows,
            scale_log2, [&](int) { return row; }, [&](int rel) { return rel; }, sm, &bad);
        for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
            float M, Ls, O;
            wave_combine<D>(sm, t, &M, &Ls, &O);
            const int j = t / D, d = t % D;
            out[row * o_s0 + (h * G + j) * o_s1 + d] = f32_to_bf16(Ls > 0.f ? O / Ls : 0.f);
        }
        __syncthreads();
    }
}

// Code-predictor layer attention with the q/k norm + RoPE + K/V write fused
// in.  Workgroup (row, kv head h): waves 0 .. G-1 normalise and rotate query
// heads h G + j from the packed QKV projection's split-K planes (summed in
// plane order and rounded to bf16) and store them to q_out, wave G does the
// same for key head h and writes it into the dense cache at cache_position,
// wave G + 1 copies value head h there -- the arithmetic of
// nq_qkv_partials_norm_rope_kv_write, so the same bits -- and after a barrier
// the workgroup attends over positions [0, cache_position] exactly as
// dense_short_kernel does.  One launch instead of two per layer.
template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
dense_rope_short_kernel(const float *__restrict__ partials, int splits, int64_t plane, int64_t prow,
                        const uint16_t *__restrict__ q_weight, const uint16_t *__restrict__ k_weight,
                        const int64_t *__restrict__ positions, int64_t pos_stride, float eps, float log_theta,
                        int round_to_input, uint16_t *__restrict__ q_out, int64_t q_s0, int64_t q_s1,
                        uint16_t *__restrict__ cache, int64_t c_row, int64_t c_kind, int64_t c_pos,
                        int64_t c_head, int rows, int cache_position, int num_kv_heads, float scale_log2,
                        uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1) {
    constexpr int HALF = D / 2;
    __shared__ Smem sm;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int Hq = num_kv_heads * G;
    const int64_t n_items = static_cast<int64_t>(rows) * num_kv_heads;
    bool bad = false;
    for (int64_t w = blockIdx.x; w < n_items; w += gridDim.x) {
        const int row = static_cast<int>(w / num_kv_heads);
        const int h = static_cast<int>(w - static_cast<int64_t>(row) * num_kv_heads);
        uint16_t *slot = cache + row * c_row + cache_position * c_pos + h * c_head;
        for (int u = wave; u < G + 2; u += kWaves) {
            const int col = (u < G ? h * G + u : u == G ? Hq + h : Hq + num_kv_heads + h) * D;
            const float *e = partials + row * prow + col;
            // the planes four at a time (all loads in flight together), added in plane order,
            // rounded to bf16
            auto load = [&](int d) {
                float sum = 0.f;
                for (int i0 = 0; i0 < splits; i0 += 4) {
                    float a[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) a[v] = i0 + v < splits ? e[(i0 + v) * plane + d] : 0.f;
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (i0 + v < splits) sum += a[v];
                }
                return bf16_to_f32(f32_to_bf16(sum));
            };
            if (u == G + 1) {
                for (int d = lane; d < D; d += kWave) slot[c_kind + d] = f32_to_bf16(load(d));
                continue;
            }
            const bool on = lane < HALF;
            float x1 = 0.f, x2 = 0.f, w1 = 0.f, w2 = 0.f;
            if (on) {
                const uint16_t *wt = u < G ? q_weight : k_weight;
                w1 = bf16_to_f32(wt[lane]);
                w2 = bf16_to_f32(wt[lane + HALF]);
                x1 = load(lane);
                x2 = load(lane + HALF);
            }
            uint16_t o1 = 0, o2 = 0;
            norm_rope_pair<D>(x1, x2, on, w1, w2, lane, eps, log_theta,
                              static_cast<float>(positions[row * pos_stride]), round_to_input, o1, o2);
            if (!on) continue;
            uint16_t *dst = u < G ? q_out + row * q_s0 + (h * G + u) * q_s1 : slot;
            dst[lane] = o1;
            dst[lane + HALF] = o2;
        }
        __syncthreads();  // the rotated q and the new K/V are visible to every wave of the workgroup
        attend_chunk<D, G, true>(
            q_out + row * q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, h, cache_position + 1, rows,
            scale_log2, [&](int) { return row; }, [&](int rel) { return rel; }, sm, &bad);
        for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
            float M, Ls, O;
            wave_combine<D>(sm, t, &M, &Ls, &O);
            const int j = t / D, d = t % D;
            out[row * o_s0 + (h * G + j) * o_s1 + d] = f32_to_bf16(Ls > 0.f ? O / Ls : 0.f);
        }
        __syncthreads();
    }
}

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Prefill rows on MFMA (head dim 128, two query heads per kv head).  A
// workgroup takes one piece (a range of whole 64-key tiles) of one 64-query
// tile of a row and one kv head h; wave w owns queries 16 w .. 16 w + 15 in
// both query heads 2h and 2h + 1, so every K and V operand it reads from LDS
// feeds two MFMAs.  Per 64-key tile the workgroup stages K and V as they sit
// in the cache ([key][d], 16-byte stores) and each wave computes the
// transposed scores S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (K from LDS as
// the A operand, Q held in registers as the B operand), so a lane holds 16
// scores of ONE query (lane & 15) per head for keys 16 nt + 4 (lane >> 4) + e.
// The online softmax is then per lane (the four lanes of a query agree on the
// running maximum through two cross-lane exchanges, and keep partial row sums
// that are added once at the end), the probabilities are packed to bf16 in
// registers and used directly as the B operand of O^T += V^T P^T, whose A
// operand (V^T: 8 keys of one column per lane, in the same key order as the
// lane's probabilities) comes from gfx950's transposing LDS read
// (ds_read_b64_tr_b16).  P never goes through LDS.  Keys past the piece's end
// are never loaded; the causal mask is applied only on tiles that reach a
// query's limit.  A tile's pieces merge as described at the piece stores.

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 pf_bf16x2 __attribute__((ext_vector_type(2)));
typedef float pf_floatx2 __attribute__((ext_vector_type(2)));
typedef float pf_floatx4 __attribute__((ext_vector_type(4)));
typedef short pf_v4i16 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ pf_bf16x8 pf_as_bf16x8(const uint4 &v) {
    pf_bf16x8 r;
    __builtin_memcpy(&r, &v, sizeof(r));
    return r;
}

// round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pf_pack_bf16(float a, float b) {
    const pf_bf16x2 r = __builtin_convertvector((pf_floatx2){a, b}, pf_bf16x2);
    uint32_t u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}

// One workgroup's prefill items in the tile shape kWide (see kPrefQ); ks, vs
// and pages are the launch's LDS arrays, s_arrived its arrival flag.
template <int D, bool kWide>
__device__ __forceinline__ void prefill_tiles(
    const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1, const uint16_t *__restrict__ cache, int64_t c_page,
    int64_t c_kind, int64_t c_slot, int64_t c_head, int num_pages, const int32_t *__restrict__ kv_indices,
    int index_limit, int num_kv_heads, int ps_log2, float scale_log2, uint16_t *__restrict__ out, int64_t o_s0,
    int64_t o_s1, char *__restrict__ ws, const PlanLayout &L, int32_t *status, uint16_t *ks, uint16_t *vs,
    int *pages, int *s_arrived) {
    // K and V row pitch (bf16): rows 288 bytes apart, the 32-byte row offset at which gfx950 serves
    // 16-byte LDS reads of consecutive rows without bank conflicts (272-byte rows measured 0.6 us
    // slower per layer of the mixed batch)
    constexpr int KP = D + 16;
    constexpr int DT = D / 16;         // 16-wide output column tiles
    constexpr int KK = D / 32;         // 32-deep k steps of S^T
    constexpr int NH = kWide ? 2 : 1;  // query heads per wave
    constexpr int kDepth = kWide ? 1 : 2;  // 64-key tiles whose K/V loads are in flight
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    const int4 *pitems = reinterpret_cast<const int4 *>(ws + L.pitems);
    float *part_ml = reinterpret_cast<float *>(ws + L.part_ml);
    float *part_o = reinterpret_cast<float *>(ws + L.part_o);
    int32_t *tile_arrivals = reinterpret_cast<int32_t *>(ws + L.tile_arrivals);
    const int Hq = 2 * num_kv_heads;
    const int64_t n_items = static_cast<int64_t>(meta[kMetaPItems]) * num_kv_heads;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15, kq = lane >> 4;
    const int ps_mask = (1 << ps_log2) - 1;
    // V^T operand reads: lane r16 of lane group kq points at key 4 kq + r16 / 4 (+ 16, + 32 kh),
    // columns 16 dt + 4 (r16 % 4) .. + 3; ds_read_b64_tr_b16 then hands lane j the four keys
    // 4 kq .. 4 kq + 3 of column 16 dt + j
    const uint16_t *vrow = vs + (kq * 4 + (r16 >> 2)) * KP + 4 * (r16 & 3);
    const bool out_vec = (reinterpret_cast<uintptr_t>(out) & 7) == 0 && (o_s0 & 3) == 0 && (o_s1 & 3) == 0;
    // the wave's queries within a tile, and its query head a of kv head h: wide waves take 16
    // queries each in both heads, narrow ones 16 queries (wave & 1) of head 2h + (wave >> 1)
    const int qsub = kWide ? wave * 16 : (wave & 1) * 16;
    auto head_of = [&](int h, int a) { return kWide ? 2 * h + a : 2 * h + (wave >> 1); };
    bool bad = false;
    for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int pi = static_cast<int>(item / num_kv_heads);
        const int h = static_cast<int>(item - static_cast<int64_t>(pi) * num_kv_heads);
        const int4 td = pitems[2 * pi], pd = pitems[2 * pi + 1];
        const int q0 = td.x, nq = td.y, page_start = td.z, lim0 = td.w;
        const int kb = pd.x, ke = pd.y, piece = pd.z >> 8, n_pieces = pd.z & 255;
        const int qj = qsub + r16;              // the lane's query within the tile
        const int limit = lim0 + qj;            // its keys are [0, limit) (lanes past nq compute on zeros)
        uint4 qa[NH][KK];
        {
            const bool ok = qj < nq;
#pragma unroll
            for (int a = 0; a < NH; ++a) {
                const uint16_t *qp = q + static_cast<int64_t>(q0 + qj) * q_s0 + head_of(h, a) * q_s1 + kq * 8;
#pragma unroll
                for (int kk = 0; kk < KK; ++kk)
                    qa[a][kk] = ok ? *reinterpret_cast<const uint4 *>(qp + kk * 32) : make_uint4(0, 0, 0, 0);
            }
        }
        // per head: raw-score maximum, this lane's part of the row sum
        float m_run[NH], l_run[NH];
        pf_floatx4 acc[NH][DT];  // acc[a][dt][e] = O[query qj][head a][16 dt + 4 kq + e] (unnormalised)
#pragma unroll
        for (int a = 0; a < NH; ++a) {
            m_run[a] = -INFINITY;
            l_run[a] = 0.f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[a][dt] = pf_floatx4{0.f, 0.f, 0.f, 0.f};
        }
        // K/V of the next kDepth 64-key tiles are loaded into registers (one set per tile in
        // flight) while the current tile is computed; each thread owns kStageVec (key, 8-channel)
        // pieces of a tile.
        constexpr int kStageVec = kPrefK * (D / 8) / kAttnThreads;
        uint4 kr[kDepth][kStageVec], vr[kDepth][kStageVec];
        // the piece's page list goes to LDS once (when it fits), so a tile's K/V loads do not wait
        // for an index load
        const int pg0 = kb >> ps_log2;
        const int n_pg = ke > kb ? ((ke - 1) >> ps_log2) - pg0 + 1 : 0;
        const bool lds_pages = n_pg <= kPrefPages;
        __syncthreads();  // the previous item's page reads are done
        if (lds_pages) {
            for (int t = threadIdx.x; t < n_pg; t += kAttnThreads) {
                const int at = page_start + pg0 + t;
                const int pg = at < index_limit ? kv_indices[at] : -1;
                if (static_cast<unsigned>(pg) >= static_cast<unsigned>(num_pages)) bad = true;
                pages[t] = pg;
            }
        }
        __syncthreads();
        auto issue = [&](int kt, auto set) {
            constexpr int S = decltype(set)::value;
            int pg[kStageVec];
#pragma unroll
            for (int v = 0; v < kStageVec; ++v) {
                const int e = threadIdx.x + v * kAttnThreads;
                const int kk = kt + e / (D / 8);
                if (lds_pages) {
                    pg[v] = kk < ke ? pages[(kk >> ps_log2) - pg0] : -1;
                } else {
                    const int at = page_start + (kk >> ps_log2);
                    pg[v] = (kk < ke && at < index_limit) ? kv_indices[at] : -1;
                    if (kk < ke && static_cast<unsigned>(pg[v]) >= static_cast<unsigned>(num_pages)) bad = true;
                }
            }
#pragma unroll
            for (int v = 0; v < kStageVec; ++v) {
                const int e = threadIdx.x + v * kAttnThreads;
                const int key = e / (D / 8), c8 = e - key * (D / 8);
                kr[S][v] = make_uint4(0, 0, 0, 0);
                vr[S][v] = make_uint4(0, 0, 0, 0);
                if (static_cast<unsigned>(pg[v]) < static_cast<unsigned>(num_pages)) {
                    const int64_t off = static_cast<int64_t>(pg[v]) * c_page +
                                        static_cast<int64_t>((kt + key) & ps_mask) * c_slot + h * c_head + c8 * 8;
                    kr[S][v] = *reinterpret_cast<const uint4 *>(cache + off);
                    vr[S][v] = *reinterpret_cast<const uint4 *>(cache + off + c_kind);
                }
            }
        };
        // one 64-key tile from register set S, whose loads were issued kDepth tiles ago
        auto step = [&](int kt0, auto set) {
            constexpr int S = decltype(set)::value;
            __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
            for (int v = 0; v < kStageVec; ++v) {
                const int e = threadIdx.x + v * kAttnThreads;
                const int key = e / (D / 8), c8 = e - key * (D / 8);
                *reinterpret_cast<uint4 *>(ks + key * KP + c8 * 8) = kr[S][v];
                *reinterpret_cast<uint4 *>(vs + key * KP + c8 * 8) = vr[S][v];
            }
            __syncthreads();
            if (kt0 + kDepth * kPrefK < ke) issue(kt0 + kDepth * kPrefK, set);
            // S^T = K Q^T over 4 key subtiles, each K operand read once for the wave's heads:
            // sc[a][nt][e] = S[head a][query qj][key kt0 + 16 nt + 4 kq + e]
            pf_floatx4 sc[NH][4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
                for (int a = 0; a < NH; ++a) sc[a][nt] = pf_floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    const uint4 kv = *reinterpret_cast<const uint4 *>(ks + (nt * 16 + r16) * KP + kk * 32 + kq * 8);
#pragma unroll
                    for (int a = 0; a < NH; ++a)
                        sc[a][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf_as_bf16x8(kv), pf_as_bf16x8(qa[a][kk]),
                                                                             sc[a][nt], 0, 0, 0);
                }
            }
            // causal mask, only where the tile reaches past the wave's first query limit
            if (kt0 + kPrefK > lim0 + qsub) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (kt0 + nt * 16 + kq * 4 + e >= limit) {
#pragma unroll
                            for (int a = 0; a < NH; ++a) sc[a][nt][e] = -INFINITY;
                        }
            }
            // every piece's first tile holds a key below each lane's limit (the piece's first key is
            // below the tile's first limit), so the new maximum is finite and m_run = -inf gives
            // alpha = 0
            uint32_t pk[NH][8];  // bf16 probabilities: pk[a][2 nt + e / 2] holds keys 16 nt + 4 kq + e, e + 1
            bool rescale = false;
            float alpha[NH];
#pragma unroll
            for (int a = 0; a < NH; ++a) {
                float mx = fmaxf(fmaxf(sc[a][0][0], sc[a][0][1]), fmaxf(sc[a][0][2], sc[a][0][3]));
#pragma unroll
                for (int nt = 1; nt < 4; ++nt)
                    mx = fmaxf(mx, fmaxf(fmaxf(sc[a][nt][0], sc[a][nt][1]), fmaxf(sc[a][nt][2], sc[a][nt][3])));
                mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
                mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
                const float mn = fmaxf(m_run[a], mx);
                alpha[a] = __builtin_amdgcn_exp2f((m_run[a] - mn) * scale_log2);
                rescale = rescale || alpha[a] != 1.f;
                const float nb = -mn * scale_log2;
                float rs = 0.f;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    float p[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        p[e] = __builtin_amdgcn_exp2f(fmaf(sc[a][nt][e], scale_log2, nb));
                        rs += p[e];
                    }
                    pk[a][2 * nt] = pf_pack_bf16(p[0], p[1]);
                    pk[a][2 * nt + 1] = pf_pack_bf16(p[2], p[3]);
                }
                l_run[a] = l_run[a] * alpha[a] + rs;
                m_run[a] = mn;
            }
            if (__any(rescale)) {
#pragma unroll
                for (int a = 0; a < NH; ++a)
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[a][dt][e] *= alpha[a];
            }
            // O^T += V^T P^T, each V^T operand read once for the wave's heads: k slot s of lane group
            // kq is key 32 kh + 16 (s / 4) + 4 kq + s % 4 in both operands
#pragma unroll
            for (int kh = 0; kh < kPrefK / 32; ++kh) {
                uint4 pu[NH];
#pragma unroll
                for (int a = 0; a < NH; ++a)
                    pu[a] = make_uint4(pk[a][4 * kh], pk[a][4 * kh + 1], pk[a][4 * kh + 2], pk[a][4 * kh + 3]);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const uint16_t *vp = vrow + kh * 32 * KP + dt * 16;
                    const pf_v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (pf_v4i16 __attribute__((address_space(3))) *)(vp));
                    const pf_v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (pf_v4i16 __attribute__((address_space(3))) *)(vp + 16 * KP));
                    pf_bf16x8 va;
                    __builtin_memcpy(&va, &lo, 8);
                    __builtin_memcpy(reinterpret_cast<char *>(&va) + 8, &hi, 8);
#pragma unroll
                    for (int a = 0; a < NH; ++a)
                        acc[a][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf_as_bf16x8(pu[a]), acc[a][dt], 0, 0, 0);
                }
            }
        };
        using Set0 = std::integral_constant<int, 0>;
        using Set1 = std::integral_constant<int, kDepth - 1>;
        if (kb < ke) issue(kb, Set0{});
        if constexpr (kDepth == 2) {
            if (kb + kPrefK < ke) issue(kb + kPrefK, Set1{});
        }
        for (int kt0 = kb; kt0 < ke; kt0 += kDepth * kPrefK) {
            step(kt0, Set0{});
            if constexpr (kDepth == 2) {
                if (kt0 + kPrefK < ke) step(kt0 + kPrefK, Set1{});
            }
        }
        float lt[NH];
#pragma unroll
        for (int a = 0; a < NH; ++a) {
            lt[a] = l_run[a] + __shfl_xor(l_run[a], 16, kWave);
            lt[a] += __shfl_xor(lt[a], 32, kWave);
        }
        if (n_pieces == 1) {
            if (qj < nq) {
#pragma unroll
                for (int a = 0; a < NH; ++a) {
                    const float inv = lt[a] > 0.f ? 1.0f / lt[a] : 0.f;
                    uint16_t *op = out + static_cast<int64_t>(q0 + qj) * o_s0 + head_of(h, a) * o_s1 + 4 * kq;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) {
                        const uint32_t w0 = pf_pack_bf16(acc[a][dt][0] * inv, acc[a][dt][1] * inv);
                        const uint32_t w1 = pf_pack_bf16(acc[a][dt][2] * inv, acc[a][dt][3] * inv);
                        if (out_vec) {
                            *reinterpret_cast<uint2 *>(op + dt * 16) = make_uint2(w0, w1);
                        } else {
                            op[dt * 16] = static_cast<uint16_t>(w0);
                            op[dt * 16 + 1] = static_cast<uint16_t>(w0 >> 16);
                            op[dt * 16 + 2] = static_cast<uint16_t>(w1);
                            op[dt * 16 + 3] = static_cast<uint16_t>(w1 >> 16);
                        }
                    }
                }
            }
            continue;
        }
        // A piece of a split tile leaves its unnormalised (m, l, acc) per (query, piece, query
        // head), m in the exp2 domain, with agent-scope stores (coherent across the XCDs' L2s),
        // waits for them, then counts its arrival on the (tile, kv head) counter; the piece that
        // completes the count merges the tile's pieces in piece order.
        if (qj < nq) {
#pragma unroll
            for (int a = 0; a < NH; ++a) {
                const int64_t pr = (static_cast<int64_t>(q0 + qj) * kPrefMaxPieces + piece) * Hq + head_of(h, a);
                // columns 16 dt + 4 kq + e as pairs (e = 0, 1 and 2, 3): 8-byte words 8 dt and 8 dt + 1
                uint64_t *po = reinterpret_cast<uint64_t *>(part_o + pr * D + 4 * kq);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                    for (int e = 0; e < 4; e += 2) {
                        const uint64_t w = static_cast<uint64_t>(__float_as_uint(acc[a][dt][e])) |
                                           (static_cast<uint64_t>(__float_as_uint(acc[a][dt][e + 1])) << 32);
                        __hip_atomic_store(po + dt * 8 + e / 2, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
                if (kq == 0) {
                    __hip_atomic_store(part_ml + pr * 2, m_run[a] * scale_log2, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(part_ml + pr * 2 + 1, lt[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        // every wave's partial stores happen before thread 0's arrival count (workgroup barrier),
        // which is an agent-scope acquire-release operation: it publishes the workgroup's stores
        // and, for the piece that completes the count, makes the other pieces' stores visible to
        // the merge below (the barrier after it carries that to every wave of the workgroup)
        __syncthreads();
        int32_t *counter = tile_arrivals + static_cast<int64_t>(pd.w) * num_kv_heads + h;
        if (threadIdx.x == 0) *s_arrived = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*s_arrived != n_pieces - 1) continue;
        // merge: thread = (row, quarter of D), a row being (query, query head): wide tiles give a
        // thread one query in both heads, narrow ones one (query, head) pair.  A row's (m, l) and
        // its first two pieces' partial rows are loaded together (one memory round trip), then
        // pieces are added two at a time, weighted by 2^(m_p - max) / sum_p 2^(m_p - max) l_p
        {
            constexpr int kQuarter = D / 4;   // columns per thread and row
            constexpr int kWords = kQuarter / 2;
            const int quarter = threadIdx.x & 3;
            const int mq = kWide ? threadIdx.x >> 2 : threadIdx.x >> 3;
            if (mq < nq) {
#pragma unroll
                for (int a = 0; a < NH; ++a) {
                    const int hh = kWide ? 2 * h + a : 2 * h + ((threadIdx.x >> 2) & 1);
                    // row of (query, piece p, head hh): pr0 + p Hq
                    const int64_t pr0 = static_cast<int64_t>(q0 + mq) * kPrefMaxPieces * Hq + hh;
                    float mk[kPrefMaxPieces], lk[kPrefMaxPieces];
#pragma unroll
                    for (int p = 0; p < kPrefMaxPieces; ++p) {
                        mk[p] = -INFINITY;
                        lk[p] = 0.f;
                        if (p < n_pieces) {
                            mk[p] = coherent_load(part_ml + (pr0 + p * Hq) * 2);
                            lk[p] = coherent_load(part_ml + (pr0 + p * Hq) * 2 + 1);
                        }
                    }
                    // u[s][w]: columns 2w, 2w + 1 of the quarter, piece p + s (the last piece again,
                    // with weight 0, past the end)
                    uint64_t u[2][kWords];
                    auto load_pair = [&](int p) {
#pragma unroll
                        for (int s = 0; s < 2; ++s) {
                            const int pp = p + s < n_pieces ? p + s : p;
                            uint64_t *src =
                                reinterpret_cast<uint64_t *>(part_o + (pr0 + pp * Hq) * D + quarter * kQuarter);
#pragma unroll
                            for (int w = 0; w < kWords; ++w)
                                u[s][w] = __hip_atomic_load(src + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    };
                    load_pair(0);
                    float wt[kPrefMaxPieces];
                    float mx = -INFINITY;
#pragma unroll
                    for (int p = 0; p < kPrefMaxPieces; ++p) mx = fmaxf(mx, mk[p]);
                    float ls = 0.f;
#pragma unroll
                    for (int p = 0; p < kPrefMaxPieces; ++p) {
                        wt[p] = mk[p] == -INFINITY ? 0.f : exp2f(mk[p] - mx);  // the piece's weight
                        ls += wt[p] * lk[p];
                    }
                    const float inv = ls > 0.f ? 1.0f / ls : 0.f;
#pragma unroll
                    for (int p = 0; p < kPrefMaxPieces; ++p) wt[p] = p < n_pieces ? wt[p] * inv : 0.f;
                    float o[kQuarter];
#pragma unroll
                    for (int c = 0; c < kQuarter; ++c) o[c] = 0.f;
#pragma unroll
                    for (int p = 0; p < kPrefMaxPieces; p += 2) {
                        if (p >= n_pieces) break;
                        if (p > 0) load_pair(p);
                        const float w0 = wt[p], w1 = wt[p + 1];
#pragma unroll
                        for (int w = 0; w < kWords; ++w) {
                            o[2 * w] += w0 * __uint_as_float(static_cast<uint32_t>(u[0][w])) +
                                        w1 * __uint_as_float(static_cast<uint32_t>(u[1][w]));
                            o[2 * w + 1] += w0 * __uint_as_float(static_cast<uint32_t>(u[0][w] >> 32)) +
                                            w1 * __uint_as_float(static_cast<uint32_t>(u[1][w] >> 32));
                        }
                    }
                    uint16_t *op = out + static_cast<int64_t>(q0 + mq) * o_s0 + hh * o_s1 + quarter * kQuarter;
                    const bool vec = (reinterpret_cast<uintptr_t>(op) & 15) == 0;
#pragma unroll
                    for (int c = 0; c < kQuarter; c += 8) {
                        if (vec) {
                            *reinterpret_cast<uint4 *>(op + c) =
                                make_uint4(pf_pack_bf16(o[c], o[c + 1]), pf_pack_bf16(o[c + 2], o[c + 3]),
                                           pf_pack_bf16(o[c + 4], o[c + 5]), pf_pack_bf16(o[c + 6], o[c + 7]));
                        } else {
#pragma unroll
                            for (int v = 0; v < 8; ++v) op[c + v] = f32_to_bf16(o[c + v]);
                        }
                    }
                }
            }
        }
        if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (bad && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
}

// Two waves per SIMD: the narrow shape keeps two register sets of K/V in flight, the wide shape
// one set and both heads' scores and accumulators (at most 256 VGPRs either way).
template <int D>
__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
prefill_tile_kernel(const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1,
                    const uint16_t *__restrict__ cache, int64_t c_page, int64_t c_kind, int64_t c_slot,
                    int64_t c_head, int num_pages, const int32_t *__restrict__ kv_indices, int index_limit,
                    int num_kv_heads, int ps_log2, float scale_log2, uint16_t *__restrict__ out,
                    int64_t o_s0, int64_t o_s1, char *__restrict__ ws, PlanLayout L, int32_t *status) {
    constexpr int KP = D + 16;
    __shared__ __attribute__((aligned(16))) uint16_t ks[kPrefK * KP];
    __shared__ __attribute__((aligned(16))) uint16_t vs[kPrefK * KP];
    __shared__ int pages[kPrefPages];
    __shared__ int s_arrived;
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    if (meta[kMetaStatus] != NQ_OK) return;
    if (meta[kMetaPWide])
        prefill_tiles<D, true>(q, q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices,
                               index_limit, num_kv_heads, ps_log2, scale_log2, out, o_s0, o_s1, ws, L, status, ks, vs,
                               pages, &s_arrived);
    else
        prefill_tiles<D, false>(q, q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices,
                                index_limit, num_kv_heads, ps_log2, scale_log2, out, o_s0, o_s1, ws, L, status, ks,
                                vs, pages, &s_arrived);
}

template <int D, int G>
int launch_paged(const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                 int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head, int num_pages,
                 const int32_t *kv_indices, int index_limit, int Hkv, int ps_log2, float scale,
                 uint16_t *out, int64_t o_s0, int64_t o_s1, char *ws, const PlanLayout &L,
                 int max_queries, int parts, int32_t *status, hipStream_t stream) {
    const int sgrid = kStreamWaves / kWaves;
    bool decode_done = false;
    if constexpr (D == 128 && G <= 2) {
        // decode rows through the bins (whole rows per workgroup, split rows merged by their last
        // piece: no merge launch), with the rotated q read from `q`; a plan holds at most
        // kPlanThreads rows, so its bins fit kBinMaxSlots whenever this bound does
        const int NB = bins_per_head(Hkv);
        const int rows_bound = max_queries < kPlanThreads ? max_queries : kPlanThreads;
        if (kDecodeBins && (parts & NQ_ATTN_DECODE) && Hkv <= kBinWgs && (rows_bound + NB - 1) / NB + 1 <= kBinMaxSlots) {
            RopeSrc rs{};
            rs.tokens = max_queries;
            rs.q = q;
            rs.q_s0 = q_s0;
            rs.q_s1 = q_s1;
            const dim3 grid(static_cast<unsigned>(NB * Hkv));
            uint16_t *kv = const_cast<uint16_t *>(cache);  // q-input mode writes no K/V
#define NQ_BIN_QIN(SMALL, W)                                                                                   \
    hipLaunchKernelGGL((bin_decode_kernel<D, G, SMALL, true, W>), grid, dim3(W * kWave), 0, stream, rs, kv, c_page, \
                       c_kind, c_slot, c_head, num_pages, kv_indices, index_limit, Hkv, ps_log2, scale * kLog2e, out, \
                       o_s0, o_s1, ws, L, status)
            const bool few_rows = rows_bound <= kBinSmallRows;
            const bool beside = (parts & NQ_ATTN_BESIDE_PREFILL) != 0;
            if (ps_log2 < 4) {
                if (few_rows) NQ_BIN_QIN(true, kBinWavesSmall);
                else if (beside) NQ_BIN_QIN(true, kBinWavesShared);
                else NQ_BIN_QIN(true, kBinWavesLarge);
            } else {
                if (few_rows) NQ_BIN_QIN(false, kBinWavesSmall);
                else if (beside) NQ_BIN_QIN(false, kBinWavesShared);
                else NQ_BIN_QIN(false, kBinWavesLarge);
            }
#undef NQ_BIN_QIN
            if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
            decode_done = true;
        }
    }
    if ((parts & NQ_ATTN_DECODE) && !decode_done) {
#define NQ_LAUNCH_STREAM(KERNEL, SMALL)                                                          \
    hipLaunchKernelGGL((KERNEL<D, G, SMALL>), dim3(sgrid), dim3(kAttnThreads), 0, stream, q, q_s0, \
                       q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices,         \
                       index_limit, Hkv, ps_log2, scale * kLog2e, out, o_s0, o_s1, ws, L, status)
    const bool small_pages = ps_log2 < 4;
    if constexpr (G <= 2) {
        if (small_pages) NQ_LAUNCH_STREAM(paged_stream_kernel_occ4, true);
        else NQ_LAUNCH_STREAM(paged_stream_kernel_occ4, false);
    } else {
        if (small_pages) NQ_LAUNCH_STREAM(paged_stream_kernel, true);
        else NQ_LAUNCH_STREAM(paged_stream_kernel, false);
    }
#undef NQ_LAUNCH_STREAM
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    const int64_t pairs = static_cast<int64_t>(max_queries) * Hkv;
    const int mgrid = static_cast<int>(pairs < 2048 ? pairs : 2048);
    hipLaunchKernelGGL((merge_stream_kernel<D, G>), dim3(mgrid), dim3(kAttnThreads), 0, stream, ws,
                       L, Hkv, sgrid * kWaves, max_queries, out, o_s0, o_s1);
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    }
    if (!(parts & NQ_ATTN_PREFILL)) return NQ_OK;
    if constexpr (D == 128 && G == 2) {
        const int64_t titems = L.max_pitems * Hkv;
        const int tgrid = static_cast<int>(titems < 4096 ? titems : 4096);
        hipLaunchKernelGGL((prefill_tile_kernel<D>), dim3(tgrid), dim3(kAttnThreads), 0, stream, q, q_s0, q_s1,
                           cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices, index_limit, Hkv, ps_log2,
                           scale * kLog2e, out, o_s0, o_s1, ws, L, status);
        return NQ_LAUNCH_STATUS();
    }
    const int64_t items = L.max_chunks * Hkv;
    const int grid = static_cast<int>(items < 8192 ? items : 8192);
    hipLaunchKernelGGL((paged_chunk_kernel<D, G>), dim3(grid), dim3(kAttnThreads), 0, stream, q,
                       q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices,
                       index_limit, Hkv, ps_log2, scale * kLog2e, out, o_s0, o_s1, ws, L, status);
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    const int64_t merges = static_cast<int64_t>(max_queries) * Hkv;
    const int cgrid = static_cast<int>(merges < 4096 ? merges : 4096);
    hipLaunchKernelGGL((merge_chunks_kernel<D, G>), dim3(cgrid), dim3(kAttnThreads), 0, stream, ws,
                       L, Hkv, out, o_s0, o_s1);
    return NQ_LAUNCH_STATUS();
}

template <int D, int G>
int launch_dense(const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                 int64_t c_row, int64_t c_kind, int64_t c_pos, int64_t c_head, int rows,
                 int valid_length, int Hkv, float scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                 hipStream_t stream) {
    int64_t items = static_cast<int64_t>(rows) * Hkv;
    int grid = static_cast<int>(items < 8192 ? items : 8192);
    hipLaunchKernelGGL((dense_short_kernel<D, G>), dim3(grid), dim3(kAttnThreads), 0, stream, q,
                       q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, rows, valid_length, Hkv,
                       scale * kLog2e, out, o_s0, o_s1);
    return NQ_LAUNCH_STATUS();
}

template <int D, int G>
int launch_dense_rope(const float *partials, int splits, int rows, const uint16_t *q_weight, const uint16_t *k_weight,
                      const int64_t *positions, int64_t pos_stride, float eps, float rope_theta, int round_to_input,
                      uint16_t *q_out, int64_t q_s0, int64_t q_s1, uint16_t *cache, int64_t c_row, int64_t c_kind,
                      int64_t c_pos, int64_t c_head, int cache_position, int Hkv, float scale, uint16_t *out,
                      int64_t o_s0, int64_t o_s1, hipStream_t stream) {
    const int64_t prow = static_cast<int64_t>(Hkv * G + 2 * Hkv) * D;
    const int64_t items = static_cast<int64_t>(rows) * Hkv;
    const int grid = static_cast<int>(items < 8192 ? items : 8192);
    hipLaunchKernelGGL((dense_rope_short_kernel<D, G>), dim3(grid), dim3(kAttnThreads), 0, stream, partials, splits,
                       static_cast<int64_t>(rows) * prow, prow, q_weight, k_weight, positions, pos_stride, eps,
                       logf(rope_theta), round_to_input, q_out, q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head,
                       rows, cache_position, Hkv, scale * kLog2e, out, o_s0, o_s1);
    return NQ_LAUNCH_STATUS();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace nq

using nq::PlanLayout;

extern "C" int64_t nq_attention_workspace_bytes(int max_query_tokens, int max_pages, int page_size,
                                                int num_qo_heads, int num_kv_heads, int head_dim) {
    if (max_query_tokens < 1 || max_pages < 1 || page_size < 1 || num_kv_heads < 1 ||
        num_qo_heads < num_kv_heads || head_dim < 8)
        return NQ_ERR_INVALID_ARGUMENT;
    return nq::plan_layout(max_query_tokens, max_pages, page_size, num_qo_heads, num_kv_heads, head_dim)
        .total;
}

extern "C" int nq_attention_plan_parts(const int32_t *qo_indptr, const int32_t *kv_indptr,
                                       const int32_t *last_page_len, const int32_t *kv_indices,
                                       const int64_t *position_ids, const int64_t *write_pages,
                                       const int64_t *write_offsets, int n_rows, int max_query_tokens,
                                       int max_pages, int page_size, int num_qo_heads, int num_kv_heads,
                                       int head_dim, int parts, void *workspace, int64_t workspace_bytes,
                                       void *stream) {
    NQ_CHECK_ARG((parts & (NQ_ATTN_DECODE | NQ_ATTN_PREFILL)) != 0 &&
                 (parts & ~(NQ_ATTN_DECODE | NQ_ATTN_PREFILL | NQ_ATTN_BESIDE_PREFILL)) == 0);
    NQ_CHECK_ARG(!(parts & NQ_ATTN_BESIDE_PREFILL) || (parts & NQ_ATTN_DECODE));
    NQ_CHECK_ARG(n_rows >= 1 && max_query_tokens >= 1 && max_pages >= 1);
    if (n_rows > nq::kPlanThreads) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    NQ_CHECK_ARG(kv_indptr && last_page_len && kv_indices && workspace);
    NQ_CHECK_ARG(qo_indptr || n_rows <= max_query_tokens);
    const PlanLayout L =
        nq::plan_layout(max_query_tokens, max_pages, page_size, num_qo_heads, num_kv_heads, head_dim);
    NQ_CHECK_ARG(workspace_bytes >= L.total);
    hipLaunchKernelGGL(nq::attention_plan_kernel, dim3(nq::kPlanGrid), dim3(nq::kPlanThreads), 0,
                       static_cast<hipStream_t>(stream), qo_indptr, kv_indptr, last_page_len,
                       kv_indices, position_ids, write_pages, write_offsets, n_rows, max_query_tokens,
                       max_pages, page_size, num_kv_heads, static_cast<char *>(workspace), L,
                       (parts & NQ_ATTN_DECODE) ? 0 : 1);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_attention_plan(const int32_t *qo_indptr, const int32_t *kv_indptr,
                                 const int32_t *last_page_len, const int32_t *kv_indices,
                                 const int64_t *position_ids, const int64_t *write_pages,
                                 const int64_t *write_offsets,
                                 int n_rows, int max_query_tokens, int max_pages, int page_size,
                                 int num_qo_heads, int num_kv_heads, int head_dim, void *workspace,
                                 int64_t workspace_bytes, void *stream) {
    return nq_attention_plan_parts(qo_indptr, kv_indptr, last_page_len, kv_indices, position_ids, write_pages,
                                   write_offsets, n_rows, max_query_tokens, max_pages, page_size, num_qo_heads,
                                   num_kv_heads, head_dim, NQ_ATTN_DECODE | NQ_ATTN_PREFILL, workspace,
                                   workspace_bytes, stream);
}

extern "C" int nq_paged_attention(const uint16_t *q, int64_t q_s0, int64_t q_s1,
                                  const uint16_t *cache, int64_t c_page, int64_t c_kind,
                                  int64_t c_slot, int64_t c_head, int num_pages,
                                  const int32_t *kv_indices, int page_size, int num_qo_heads,
                                  int num_kv_heads, int head_dim, float sm_scale, uint16_t *out,
                                  int64_t o_s0, int64_t o_s1, int max_query_tokens, int max_pages,
                                  int parts, void *workspace, int64_t workspace_bytes,
                                  int32_t *status, void *stream) {
    NQ_CHECK_ARG(q && cache && kv_indices && out && workspace);
    NQ_CHECK_ARG((parts & (NQ_ATTN_DECODE | NQ_ATTN_PREFILL)) != 0 &&
                 (parts & ~(NQ_ATTN_DECODE | NQ_ATTN_PREFILL | NQ_ATTN_BESIDE_PREFILL)) == 0);
    NQ_CHECK_ARG(!(parts & NQ_ATTN_BESIDE_PREFILL) || (parts & NQ_ATTN_DECODE));
    NQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0 && num_pages >= 1);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    NQ_CHECK_ARG(max_query_tokens >= 1 && max_pages >= 1);
    if (!nq::aligned16(q) || !nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((q_s0 | q_s1 | c_page | c_kind | c_slot | c_head | o_s0 | o_s1) & 7) return NQ_ERR_UNSUPPORTED;
    const PlanLayout L =
        nq::plan_layout(max_query_tokens, max_pages, page_size, num_qo_heads, num_kv_heads, head_dim);
    NQ_CHECK_ARG(workspace_bytes >= L.total);
    int ps_log2 = 0;
    while ((1 << ps_log2) < page_size) ++ps_log2;
    const int G = num_qo_heads / num_kv_heads;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
#define NQ_PAGED(DD, GG)                                                                          \
    if (head_dim == DD && G == GG)                                                                \
        return nq::launch_paged<DD, GG>(q, q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head,     \
                                        num_pages, kv_indices, max_pages, num_kv_heads, ps_log2,  \
                                        sm_scale, out, o_s0, o_s1, ws, L, max_query_tokens,       \
                                        parts, status, s);
    NQ_PAGED(128, 1) NQ_PAGED(128, 2) NQ_PAGED(128, 4) NQ_PAGED(128, 8)
    NQ_PAGED(64, 1) NQ_PAGED(64, 2) NQ_PAGED(64, 4) NQ_PAGED(64, 8)
#undef NQ_PAGED
    return NQ_ERR_UNSUPPORTED;
}

extern "C" int nq_cp_short_attention(const uint16_t *q, int64_t q_s0, int64_t q_s1,
                                     const uint16_t *cache, int64_t c_row, int64_t c_kind,
                                     int64_t c_pos, int64_t c_head, int rows, int valid_length,
                                     int num_qo_heads, int num_kv_heads, int head_dim,
                                     float sm_scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                                     void *stream) {
    NQ_CHECK_ARG(q && cache && out && rows >= 1 && valid_length >= 1);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    if (!nq::aligned16(q) || !nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((q_s0 | q_s1 | c_row | c_kind | c_pos | c_head) & 7) return NQ_ERR_UNSUPPORTED;
    const int G = num_qo_heads / num_kv_heads;
    hipStream_t s = static_cast<hipStream_t>(stream);
#define NQ_DENSE(DD, GG)                                                                         \
    if (head_dim == DD && G == GG)                                                               \
        return nq::launch_dense<DD, GG>(q, q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, rows, \
                                        valid_length, num_kv_heads, sm_scale, out, o_s0, o_s1, s);
    NQ_DENSE(128, 1) NQ_DENSE(128, 2) NQ_DENSE(128, 4) NQ_DENSE(128, 8)
    NQ_DENSE(64, 1) NQ_DENSE(64, 2) NQ_DENSE(64, 4) NQ_DENSE(64, 8)
#undef NQ_DENSE
    return NQ_ERR_UNSUPPORTED;
}

extern "C" int nq_cp_rope_short_attention(const float *partials, int splits, int rows, const uint16_t *q_weight,
                                          const uint16_t *k_weight, const int64_t *positions, int64_t pos_stride,
                                          float eps, float rope_theta, int round_to_input, uint16_t *q_out,
                                          int64_t q_s0, int64_t q_s1, uint16_t *cache, int64_t c_row, int64_t c_kind,
                                          int64_t c_pos, int64_t c_head, int cache_position, int num_qo_heads,
                                          int num_kv_heads, int head_dim, float sm_scale, uint16_t *out,
                                          int64_t o_s0, int64_t o_s1, void *stream) {
    NQ_CHECK_ARG(partials && splits >= 1 && q_weight && k_weight && positions && q_out && cache && out);
    NQ_CHECK_ARG(rows >= 1 && cache_position >= 0 && rope_theta > 0.f);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    if (!nq::aligned16(q_out) || !nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((q_s0 | q_s1 | c_row | c_kind | c_pos | c_head) & 7) return NQ_ERR_UNSUPPORTED;
    const int G = num_qo_heads / num_kv_heads;
    hipStream_t s = static_cast<hipStream_t>(stream);
#define NQ_DENSE_ROPE(DD, GG)                                                                                    \
    if (head_dim == DD && G == GG)                                                                               \
        return nq::launch_dense_rope<DD, GG>(partials, splits, rows, q_weight, k_weight, positions, pos_stride,   \
                                             eps, rope_theta, round_to_input, q_out, q_s0, q_s1, cache, c_row,   \
                                             c_kind, c_pos, c_head, cache_position, num_kv_heads, sm_scale, out, \
                                             o_s0, o_s1, s);
    NQ_DENSE_ROPE(128, 1) NQ_DENSE_ROPE(128, 2) NQ_DENSE_ROPE(64, 1) NQ_DENSE_ROPE(64, 2)
#undef NQ_DENSE_ROPE
    return NQ_ERR_UNSUPPORTED;
}

extern "C" int nq_paged_decode_rope_attention(const float *partials, int splits, int tokens, const uint16_t *q_weight,
                                              const uint16_t *k_weight, const int64_t *positions, float eps,
                                              float rope_theta, int round_to_input, uint16_t *cache, int64_t c_page,
                                              int64_t c_kind, int64_t c_slot, int64_t c_head, int num_pages,
                                              const int64_t *write_pages, const int64_t *write_offsets,
                                              const int32_t *kv_indices, int page_size, int num_qo_heads,
                                              int num_kv_heads, int head_dim, float sm_scale, uint16_t *out,
                                              int64_t o_s0, int64_t o_s1, int max_query_tokens, int max_pages,
                                              void *workspace, int64_t workspace_bytes, int32_t *status,
                                              void *stream) {
    NQ_CHECK_ARG(partials && splits >= 1 && tokens >= 1 && q_weight && k_weight && positions && cache);
    NQ_CHECK_ARG(write_pages && write_offsets && kv_indices && out && workspace);
    NQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0 && num_pages >= 1 && rope_theta > 0.f);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    NQ_CHECK_ARG(max_query_tokens >= 1 && max_pages >= 1 && tokens <= max_query_tokens);
    const int G = num_qo_heads / num_kv_heads;
    const int NB = nq::bins_per_head(num_kv_heads);
    // shapes the fused kernel does not take: the caller runs the rope and attention kernels instead
    if (head_dim != 128 || (G != 1 && G != 2) || num_kv_heads > nq::kBinWgs ||
        (max_query_tokens + NB - 1) / NB + 1 > nq::kBinMaxSlots)
        return NQ_ERR_UNSUPPORTED;
    if (!nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((c_page | c_kind | c_slot | c_head | o_s0 | o_s1) & 7) return NQ_ERR_UNSUPPORTED;
    const PlanLayout L =
        nq::plan_layout(max_query_tokens, max_pages, page_size, num_qo_heads, num_kv_heads, head_dim);
    NQ_CHECK_ARG(workspace_bytes >= L.total);
    int ps_log2 = 0;
    while ((1 << ps_log2) < page_size) ++ps_log2;
    const int64_t row = static_cast<int64_t>(num_qo_heads + 2 * num_kv_heads) * head_dim;
    const nq::RopeSrc rs{partials, splits, tokens, static_cast<int64_t>(tokens) * row, row, q_weight, k_weight,
                         positions, write_pages, write_offsets, eps, logf(rope_theta), round_to_input};
    hipStream_t st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    const float scale_log2 = sm_scale * nq::kLog2e;
    const dim3 grid(static_cast<unsigned>(NB * num_kv_heads));
#define NQ_BIN(GG, SMALL, W)                                                                                   \
    hipLaunchKernelGGL((nq::bin_decode_kernel<128, GG, SMALL, false, W>), grid, dim3(W * nq::kWave), 0, st, rs,   \
                       cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices, max_pages, num_kv_heads, ps_log2, \
                       scale_log2, out, o_s0, o_s1, ws, L, status)
#define NQ_BIN_W(GG, SMALL)                                                 \
    do {                                                                    \
        if (max_query_tokens <= nq::kBinSmallRows) NQ_BIN(GG, SMALL, nq::kBinWavesSmall); \
        else NQ_BIN(GG, SMALL, nq::kBinWavesLarge);                         \
    } while (0)
    const bool small_pages = ps_log2 < 4;
    if (G == 2) {
        if (small_pages) NQ_BIN_W(2, true);
        else NQ_BIN_W(2, false);
    } else {
        if (small_pages) NQ_BIN_W(1, true);
        else NQ_BIN_W(1, false);
    }
#undef NQ_BIN_W
#undef NQ_BIN
    return NQ_LAUNCH_STATUS();
}

// ---------------------------------------------------------------------------
// No-allocation variant of nq_attention_plan + nq_paged_attention.
//
// The plan and the partial results live in `scratch`, a file-scope device
// array (one copy per GPU, held until the process ends).  In host code the
// name `scratch` is only a host-side stand-in: its device address is fetched
// once per device with hipGetSymbolAddress and only that pointer is passed to
// the kernels.  The plan kernel writes every counter the attention kernels
// read (and zeroes the split-row arrival counts), so nothing is cleared on
// the host.  Calls that overlap on one GPU share the array and race.

static __device__ __align__(256) char scratch[NQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
char *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call there).
int scratch_on_current_device(char **out) {
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return NQ_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return NQ_ERR_LAUNCH;
        g_scratch_ptr[device] = static_cast<char *>(ptr);
    }
    *out = g_scratch_ptr[device];
    return NQ_OK;
}

}  // namespace

extern "C" int nq_paged_attention_noalloc(const int32_t *qo_indptr, const int32_t *kv_indptr,
                                          const int32_t *last_page_len, const int32_t *kv_indices, int n_rows,
                                          const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                                          int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head,
                                          int num_pages, int page_size, int num_qo_heads, int num_kv_heads,
                                          int head_dim, float sm_scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                                          int max_query_tokens, int max_pages, int parts, int32_t *status,
                                          void *stream) {
    // every check of the two entry points it stands for, before anything is launched
    NQ_CHECK_ARG(n_rows >= 1 && max_query_tokens >= 1 && max_pages >= 1);
    if (n_rows > nq::kPlanThreads) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(q && cache && kv_indptr && last_page_len && kv_indices && out);
    NQ_CHECK_ARG(qo_indptr || n_rows <= max_query_tokens);
    NQ_CHECK_ARG((parts & (NQ_ATTN_DECODE | NQ_ATTN_PREFILL)) != 0 &&
                 (parts & ~(NQ_ATTN_DECODE | NQ_ATTN_PREFILL | NQ_ATTN_BESIDE_PREFILL)) == 0);
    NQ_CHECK_ARG(!(parts & NQ_ATTN_BESIDE_PREFILL) || (parts & NQ_ATTN_DECODE));
    NQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0 && num_pages >= 1);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    if (!nq::aligned16(q) || !nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((q_s0 | q_s1 | c_page | c_kind | c_slot | c_head | o_s0 | o_s1) & 7) return NQ_ERR_UNSUPPORTED;
    const int G = num_qo_heads / num_kv_heads;
    if ((head_dim != 64 && head_dim != 128) || (G != 1 && G != 2 && G != 4 && G != 8)) return NQ_ERR_UNSUPPORTED;
    const PlanLayout L =
        nq::plan_layout(max_query_tokens, max_pages, page_size, num_qo_heads, num_kv_heads, head_dim);
    if (L.total > NQ_NOALLOC_SCRATCH_BYTES) return NQ_ERR_INVALID_ARGUMENT;  // beyond the static scratch
    char *ws = nullptr;
    const int rc = scratch_on_current_device(&ws);
    if (rc != NQ_OK) return rc;
    const int planned = nq_attention_plan(qo_indptr, kv_indptr, last_page_len, kv_indices, nullptr, nullptr,
                                          nullptr, n_rows, max_query_tokens, max_pages, page_size, num_qo_heads,
                                          num_kv_heads, head_dim, ws, NQ_NOALLOC_SCRATCH_BYTES, stream);
    if (planned != NQ_OK) return planned;
    return nq_paged_attention(q, q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indices,
                              page_size, num_qo_heads, num_kv_heads, head_dim, sm_scale, out, o_s0, o_s1,
                              max_query_tokens, max_pages, parts, ws, NQ_NOALLOC_SCRATCH_BYTES, status, stream);
}
