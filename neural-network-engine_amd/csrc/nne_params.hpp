// Launch-parameter structs of the attention kernels, in plain C++ (no HIP
// types), so host-only code -- the split-K launch planner and its tests --
// can use them without the HIP toolchain.
//
// Layout conventions (all f32):
//   Q/O  [B, Hq,  T_q, d]  and  K/V [B, Hkv, T_k, d], each a strided view
//   (element strides for batch, head, row, dim).  Query head hq reads KV head
//   hq / G with G = Hq / Hkv, the repeat-KV mapping of the reference's
//   GroupedQueryAttention (src/models/llama.rs:256-266).
//   A key c is visible to query row r iff c <= r + q_offset (causal) -- the
//   reference's flash path uses q_offset = 0 (src/nn/flash_attention.rs:113),
//   its cached GQA/MHA paths use q_offset = start_pos (llama.rs:280-283,
//   attention.rs:104-108).
#pragma once

#include <stdint.h>

namespace nne {

struct View4 {
    const float* p;
    int64_t sb, sh, st, sd;
};

struct OutView4 {
    float* p;
    int64_t sb, sh, st, sd;
};

// Prefill (MFMA) kernel parameters.  One workgroup = 4 waves; each wave owns
// one "unit" = 32 query rows of one query head.  Units of one KV head are
// numbered u = row_block * G + g, and workgroup w of that KV head takes units
// 4w .. 4w+3, so the G query heads of a group share every K/V tile the
// workgroup stages in LDS.
constexpr int kMaxSplitItems = 256;   // work items per KV head of a key-split launch

struct PrefillParams {
    View4 q, k, v;
    OutView4 o;
    int B, Hq, Hkv, G, Tq, Tk, d;
    int q_offset;
    float qscale;   // softmax scale * log2(e), folded into Q
    int n_rb;       // ceil(Tq / 32)
    int n_units;    // G * n_rb
    int n_wg;       // ceil(n_units / 4) work items (4 units each) per KV head
    int total;      // B * Hkv * n_wg work items
    // Persistent schedule: a work item is the 4 units of one workgroup-sized
    // step of a KV head.  With `pairing`, items of ranks r and n_wg-1-r of a
    // head form one super-item (equal causal work); n_pairs super-items per
    // head, n_super in all, per_xcd of them per XCD.
    int pairing;
    int n_pairs;
    int n_super;
    int per_xcd;
    // One item per workgroup (hardware dispatch) of a causal problem whose
    // XCDs hold whole KV heads: items are taken longest first across the
    // XCD's order_hpx heads, and while the XCD's items fit two per CU
    // (order_cu CUs per XCD) the two workgroups of a CU get complementary
    // lengths.  order_cu = 0: items in head-major rank order.
    int order_cu;
    int order_hpx;
    // Key split for problems too small to fill the chip (n_chunks > 1): the
    // key tiles of every work item are cut into chunks of chunk_tiles tiles,
    // one workgroup per (item, chunk); each leaves a partial (max, sum, O)
    // record in ws and counts itself in cnt[item] (zeroed, left zeroed), and
    // the last to arrive merges the item's records and writes O.
    int n_chunks;       // largest chunk count of an item
    int chunk_tiles;
    float* ws;
    uint32_t* cnt;
    // Workgroup w of a KV head runs chunk w - part_prefix[i] of item i, where
    // part_prefix[i] <= w < part_prefix[i + 1] (items of a head in rank order,
    // empty items one chunk); part_prefix[n_wg] workgroups per head.
    uint16_t part_prefix[kMaxSplitItems + 1];
};

// Head dims above 256 (deep.hip), prefill, cross-attention and decode alike,
// and prefill at 129-256 dims the wave-pair kernel does not take.  The G * Tq
// query rows of a KV head are flattened (row r: query head kvh * G + r / Tq,
// position r % Tq) and cut into 32-row units; a workgroup serves one unit and
// one kDeepChunk-dim chunk of the output dims (256 dims on the 2-wave form,
// which runs unsplit).  Sequence
// b has lens[b] keys when lens != null (a KV cache), else Tk; with `causal`,
// key c is visible to position t iff c <= t + q_offset.
constexpr int kDeepChunk = 512;
constexpr int kDeepMaxHeads = 512;   // (sequence, KV head) pairs of a ragged key split
constexpr int kDeepMaxSplit = 8;     // key parts per unit of a key split

struct DeepParams {
    View4 q, k, v;
    OutView4 o;
    const int32_t* lens;
    int B, Hq, Hkv, G, Tq, Tk, d;
    int q_offset;
    float qscale;    // softmax scale * log2(e), folded into Q
    int n_units;     // ceil(G * Tq / 32) per KV head
    int n_oc;        // output chunks per unit
    int total;       // B * Hkv * n_units * n_oc * n_split workgroups
    int per_xcd;     // ceil(total / 8)
    // Causal launches over whole KV heads per XCD (B * Hkv % 8 == 0):
    // order_hpx heads per XCD, units taken longest first across them.
    int order_hpx;
    // Key split (n_split > 1, up to 8 parts; problems with too few units to
    // fill the device): workgroup s of a (unit, chunk) streams the unit's key tiles
    // [s * split_tiles, (s + 1) * split_tiles) and leaves a partial record in
    // ws -- (max, sum) of its rpu rows, then their unnormalised O over the
    // chunk -- at record ((head * n_units + unit) * n_oc + chunk) * n_split + s;
    // the combine kernel merges the records of each (unit, chunk).
    int n_split;
    int split_tiles;
    int rpu;         // rows per record: min(32, G * Tq)
    float* ws;
    // Ragged key split (decode over ragged lengths, one unit and one chunk per
    // (sequence, KV head) pair h): pair h takes workgroups and records
    // part_prefix[h] .. part_prefix[h + 1] - 1, each split_tiles tiles of its
    // keys, so long sequences get more parts than short ones.
    int ragged;
    uint16_t part_prefix[kDeepMaxHeads + 1];
};

// Fused decode prologue (qkv.hip): rows m < M of x [M, C] (row stride x_rs,
// unit column stride) times the packed q/k/v weights (n_tiles tiles of 64
// output columns, C split into S slices of kc_per_slice 64-wide chunks), plus
// bias[j] (j = q, k, v; [H_j * d] or null); q and k rotated at position
// pos[m] with tables cos/sin [max_seq_len, d] (no rotation when cos is null);
// row m, head h, dim i written to
// out[j] + m * o_sb[j] + h * o_sh[j] + i.  With S > 1, ws holds the partial
// tiles ([n_tiles][S][64][64]) and cnt[n_tiles] the zeroed arrival counters.
struct QkvParams {
    const float* x;
    int64_t x_rs;
    const float* wp;
    const float* bias[3];
    const float* cos;
    const float* sin;
    const int32_t* pos;
    float* out[3];
    int64_t o_sb[3], o_sh[3];
    int M, C, Hq, Hkv, d;
    int n_tiles, S, kc_per_slice;
    float* ws;
    uint32_t* cnt;
};

// Split-K few-query kernel parameters (decode and cross-attention).  Each KV
// head serves G * Tq query rows; a launch takes R of them starting at row0,
// and its row rr maps to query head kvh*G + (row0+rr)/Tq and query position
// (row0+rr) % Tq.  Every row sees every key of its sequence.
// Sequences whose flattened prefix travels in the kernel arguments.
constexpr int kKeyBlock = 16;    // keys per split-K block (one 16x16x4 MFMA tile of keys)
constexpr int kArgSeqs = 128;
constexpr int kMaxPackWg = 512;   // workgroups of a whole-head packed launch
constexpr int kMaxCutWg = 256;    // workgroups of a launch with cut chunks (chunk_end)

struct SplitKParams {
    View4 q;
    const float* k;
    const float* v;
    int64_t ksb, ksh, kst;   // K strides (dim stride 1)
    int64_t vsb, vsh, vst;   // V strides (dim stride 1)
    const int32_t* lens;     // per-sequence key counts (device), or null
    int tk;                  // key count when lens == null
    int max_keys;            // host-validated upper bound on every key count
    OutView4 o;
    int B, Hq, Hkv, G, Tq, d, R;
    int row0;                // first of this launch's rows (row passes of many-row heads)
    float qscale;            // softmax scale * log2(e)
    // Causal rows (masked != 0): query t sees keys c <= q_off + t only.
    int masked;
    int q_off;
    int n_wg;                // workgroups of the split kernel
    int packed;              // whole-head packing (groups in pack_head, below)
    int chunk;               // flattened keys per workgroup (cut == 0)
    int cut;                 // chunks cut by the host (chunk_end, below)
    // decode step only (k_new != null): the new row [B, Hkv, 1, d] is attended
    // as key lens[b] and stored into the cache; lens_w[b] is advanced.
    const float* k_new;
    const float* v_new;
    int64_t kn_sb, kn_sh, vn_sb, vn_sh;
    int32_t* lens_w;
    // Flattened start of each sequence, pref[b] = Hkv * sum_{b' < b} L_b',
    // computed by the host when B <= kArgSeqs (arg_pref valid), else by the
    // split kernel from lens into ws_pref.
    int arg_pref_valid;
    int arg_pref[kArgSeqs + 1];
    // Fused combine (arg_pref_valid launches): the last workgroup to finish a
    // split head merges its partial records; ws_cnt[head] counts arrivals and
    // is left at zero.  max_parts bounds the workgroups sharing one head.
    int fused;
    int max_parts;
    uint32_t* ws_cnt;        // [B*Hkv] arrival counters, zero between launches
    // workspace
    int32_t* ws_pref;        // [B+1] flattened start of each sequence (this launch)
    float* ws_ml;            // [slots][R][2] partial (max, sum); slot = workgroup + head
    float* ws_o;             // [slots][R][D] unnormalised partial O
    // Whole-head packing (packed != 0, arg_pref_valid launches): workgroup w
    // streams the heads pack_head[w] .. pack_head[w+1]-1 (flattened order
    // b * Hkv + kvh) whole, so no head is split and no records exist.  With
    // packed == 2 (paired), workgroup w streams head pack_head[2w], then head
    // pack_head[2w+1] unless that is 0xFFFF.
    union {
    uint16_t pack_head[kMaxPackWg + 1];
    // Cut chunks (cut != 0, fused launches): workgroup w streams the
    // flattened keys [chunk_end[w-1], chunk_end[w]) (chunk_end[-1] = 0,
    // chunk_end[n_wg-1] = every key), cut so that a workgroup's keys plus a
    // fixed cost for each segment after its first are about equal.
    int chunk_end[kMaxCutWg];
    };
};

}  // namespace nne
