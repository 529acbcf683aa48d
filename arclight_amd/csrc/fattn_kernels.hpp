// Kernel-side parameter block and launchers of the attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "norm_rope.hpp"

// Everything a flash-attention kernel needs, resolved on the host from the
// al_fattn_args descriptors. Byte strides; pointers are device pointers.
struct FattnParams {
    const char * q;     int64_t q_nb1, q_nb2, q_nb3;     // f32 [D, T, Hq, B]
    uint32_t q_bytes;                                    // bytes of one q stream slice, clamped
    const char * k;     int64_t k_nb1, k_nb2, k_nb3;     // f16 [D, n_kv, Hkv, Bk]
    const char * v;     int64_t v_nb1, v_nb2, v_nb3;     // f16 [D, n_kv, Hkv, Bv]
    const char * mask;  int64_t m_nb1, m_nb2, m_nb3;     // f16 [m_ne0, rows, m_ne2, m_ne3] or null
    int32_t m_ne0, m_ne2, m_ne3;
    uint32_t m_slice_bytes;                              // bytes of one mask stream slice (dims 0..2), clamped
    const float * sinks;                                 // f32 [Hq] or null
    char * dst;         int64_t dst_nb1;                 // f32 rows (i3*T + i1)*Hq + i2

    int32_t T, Hq, Hkv, G, B, R;    // R = T*G query rows per kv head
    uint32_t g_magic;               // ceil(2^32 / G) (0 for G = 1): r / G = umulhi(r, g_magic) for r G < 2^32
    uint32_t split_magic;           // prefill: ceil(2^32 / (n_split * in-workgroup splits)) (0 for 1)
    uint32_t tiles_magic;           // prefill: ceil(2^32 / n_row_tiles) (0 for 1)
    int32_t rk3, rv3;               // q streams per k / v stream
    int32_t n_kv;                   // cells addressable in k/v
    int32_t kv_hi;                  // cells >= kv_hi are masked for all rows
    int64_t causal_pos0;            // < 0: off
    float   scale;                  // already divided by softcap when softcap != 0
    float   softcap;
    float   max_bias, m0, m1;
    uint32_t n_head_log2;

    int32_t n_row_tiles;
    int32_t n_split;
    int32_t cells_per_split;        // multiple of 32
    int32_t interleave;             // decode kernel: splits take every n_split-th 16-cell stage
    int32_t merge_rows;             // decode kernel: query rows per merging workgroup
    int32_t mask_pre;               // decode kernel: each wave's mask values preloaded into LDS
    int32_t mask_rows;              //   distinct mask rows of a workgroup (32-byte items per stage)
    int32_t mask_wave_bytes;        //   LDS bytes per wave (whole 1 KiB DMA blocks)
    int32_t one_pass;               // decode kernel, 2 waves: the waves' states merged in one pass
    float *    part;                // split-KV merge records: [units][n_split][rows per tile][record stride]
    unsigned * counters;            // [units] in the fixed counter region, zero between calls
    int *      err;                 // device error flags (al_device_errors): [0, 1] set_rows, [2] a merge gave up waiting
    const int32_t * dyn;            // decode kernel: device {kv_len, causal_pos0} read at run time, or null
};

// Split-KV kernel: rows per tile for R query rows per kv head (16, 32 or 64).
int fattn_splitkv_rows_per_tile(int R);
// Wavefronts per workgroup of the split-KV kernel for a rows-per-tile value.
int fattn_splitkv_waves(int rows_per_tile);
hipError_t fattn_splitkv_launch(const FattnParams & p, int rows_per_tile, hipStream_t stream);

// Prefill kernel: row tiles of rows_per_tile = 128 or 64 query rows (64:
// two cell splits within the workgroup), n_split workgroups per (kv head,
// row tile, stream) (1..kFattnPrefillMaxSplit; with more than one, merge
// records of rows_per_tile rows and arrival counters in the workspace);
// needs fattn_prefill_lds_bytes() of LDS. Masking: the length / causal rule
// and an explicit mask tensor (rows 16-byte aligned), whose rows the kernel
// scans for their visible extent; a mask that is not a run of zeros then
// -inf in every row of a tile is applied value by value in that tile.
hipError_t fattn_prefill_launch(const FattnParams & p, int rows_per_tile, hipStream_t stream);
size_t fattn_prefill_lds_bytes();
constexpr int kFattnPrefillRows = 128;          // query rows per workgroup (at most)
constexpr int kFattnPrefillMaxSplit = 4;        // workgroups sharing one row tile

// Decode kernel: up to 32 query rows per kv head (17..32 as two row blocks,
// 8 x 2 only), one kv head per workgroup, `waves` wavefronts each streaming
// 16-cell stages of K/V through a private ring of `stages` LDS buffers;
// fattn_decode_config_ok tells which combinations exist. At most
// kFattnMaxSplit splits per (stream, kv head); with more than one, merge
// records in the workspace and split flags in its counter region
// (kFattnDecodeFlagWords per stream x kv head, at most
// kFattnDecodeFlagUnits of them); min(splits, rows / merge_rows) splits of a
// unit merge.
bool fattn_decode_config_ok(int waves, int stages);

// The attention inputs of one layer folded into the decode kernel
// (al_fattn_f16_with_inputs), for one new token: every workgroup brings its
// kv head's query rows through RMSNorm, the weight and the rotation itself,
// and the token's K (normed, rotated) and V rows, rounded to f16, replace
// the cache's copy of its cell in the stage that holds it; split 0 writes
// those rows into the cache and, when asked, the query rows into q_out.
struct DecodeInputs {
    const char * q_w;                           // f32 [128] or null (ATTN_Q_NORM)
    const char * k;  int64_t k_nb1, k_nb2;      // f32 rows (kv head, token)
    const char * k_w;                           // f32 [128] or null (ATTN_K_NORM)
    const char * v;  int64_t v_nb1;             // f32 [Hkv * 128, T]: token stride
    const int32_t * pos;                        // [T] positions (rotation)
    const char * rows; int64_t rows_nb0;        // [T] cache row of each token, i64 or i32
    int32_t rows64;
    int32_t T;                                  // 1
    char * q_out; int64_t qo_nb1, qo_nb2;       // f32 rows (head, token), or null
    char * k_cache; int64_t kc_nb1;             // f16 rows of Hkv * 128
    char * v_cache; int64_t vc_nb1;
    int64_t n_rows;                             // cache rows
    float eps;
    RopeConsts rope;
};
// mode: the rotation (0 none, 1 pairs (2i, 2i + 1), 2 NEOX); only
// fattn_decode_fused_ok shapes, no mask tensor, one stream, one token.
bool fattn_decode_fused_ok(int waves, int stages);
// The checks of al_attn_inputs_f32 and the fused prologue's limits (prologue.hip).
int attn_inputs_decode(const struct al_attn_inputs_args * a, DecodeInputs * out, int * mode);
hipError_t fattn_decode_launch_fused(const FattnParams & p, const DecodeInputs & in, int mode, int waves, int stages,
                                     hipStream_t stream);
size_t fattn_decode_lds_bytes(int waves, int stages, bool mask, bool mask_pre);
// LDS for the preloaded mask values of a decode workgroup (all its waves).
constexpr int kDecodeMaskPreBytes = 16384;
hipError_t fattn_decode_launch(const FattnParams & p, int waves, int stages, hipStream_t stream);

// Floats of one split-KV merge record row (O[128], m, l, pad).
constexpr int kFattnRecordStride = 132;
// Bytes per query row of a decode split's record (O[128] as a block of rows,
// then the rows' (m, l) pairs): 16 RB rows make a whole number of 128-byte
// lines.
constexpr int kDecodeRecRow = 520;
// At most kFattnMaxSplit splits per row tile; one merge level.
constexpr int kFattnMaxSplit = 32;
// Every workspace starts with a fixed arrival-counter region (one counter
// per row tile or kv head), so that no call's merge records ever overlap
// another call's counters; kernels leave it zeroed. Records follow it.
constexpr size_t kFattnCounterBytes = 256u << 10;
// Arrival counters use the lower half of that region, which stays zero
// between calls.
constexpr int kFattnCounterWords = (int) (kFattnCounterBytes / 8);
// The upper half holds the decode kernel's split flags, kFattnDecodeFlagWords
// per (stream, kv head): a flag word per split and the unit's epoch (word
// 32). These words carry epochs from call to call and are never cleared.
constexpr int kFattnDecodeFlagWords = 64;
constexpr int kFattnDecodeFlagUnits = (int) (kFattnCounterBytes / 8) / kFattnDecodeFlagWords;
