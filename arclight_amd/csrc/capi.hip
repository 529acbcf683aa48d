// Host side of the C ABI: operand validation (the reference's asserts),
// kernel selection, split-KV sizing, workspace management and launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/arclight_fattn.h"
#include "../../include/arclight_prologue.h"
#include "fattn_kernels.hpp"
#include "kv_write.hpp"
#include "runtime.hpp"

namespace {

thread_local std::string g_last_error;

}  // namespace

int al_fail(int code, const char * fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int al_hip_fail(hipError_t e, const char * what) {
    return al_fail(AL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

void al_clear_error() { g_last_error.clear(); }

// ---------------------------------------------------------------------------
// per-device state
// ---------------------------------------------------------------------------

namespace {

// Library-owned split-KV workspace of one stream.
struct Workspace {
    void * ptr = nullptr;
    size_t bytes = 0;
};

struct DeviceState {
    bool       init = false;
    int        n_cu = 0;
    int        lds_per_block = 0;
    std::map<void *, Workspace> ws;     // per stream (nullptr: the default stream)
    int *      err = nullptr;       // kernel-recorded errors: this device's copy of g_err_flags
    void *     noalloc = nullptr;   // this device's copy of `scratch` (al_fattn_f16_noalloc), once set up
};

std::mutex g_mu;
std::vector<DeviceState> g_dev;

}  // namespace

// Kernel-recorded error flags (al_device_errors), one copy per GPU.
static __device__ __align__(256) int g_err_flags[64];

static int device_state(int * dev_out, DeviceState ** st_out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return al_hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_mu);
    if ((int) g_dev.size() <= dev) g_dev.resize(dev + 1);
    DeviceState & st = g_dev[dev];
    if (!st.init) {
        e = hipDeviceGetAttribute(&st.n_cu, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return al_hip_fail(e, "hipDeviceGetAttribute");
        e = hipDeviceGetAttribute(&st.lds_per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (e != hipSuccess) return al_hip_fail(e, "hipDeviceGetAttribute");
        e = hipGetSymbolAddress((void **) &st.err, HIP_SYMBOL(g_err_flags));
        if (e != hipSuccess) return al_hip_fail(e, "hipGetSymbolAddress(error flags)");
        e = hipMemset(st.err, 0, sizeof(g_err_flags));
        if (e != hipSuccess) return al_hip_fail(e, "hipMemset(error flags)");
        st.init = true;
    }
    *dev_out = dev;
    *st_out = &st;
    return AL_OK;
}

int al_device_error_flag(int ** flag) {
    int dev;
    DeviceState * st;
    const int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    *flag = st->err;
    return AL_OK;
}

int al_device_cu_count(int * n_cu) {
    int dev;
    DeviceState * st;
    const int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    *n_cu = st->n_cu;
    return AL_OK;
}

int al_device_lds_per_block(int * bytes) {
    int dev;
    DeviceState * st;
    const int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    *bytes = st->lds_per_block;
    return AL_OK;
}

// Library-owned workspace of (current device, stream), zero-filled when
// (re)allocated. The kernels leave the counter region zeroed after every
// call. One workspace per stream: calls on one stream are ordered, so they
// can share counters and records; calls on different streams never do.
static int library_workspace(size_t bytes, void * stream, void ** ptr) {
    int dev;
    DeviceState * st;
    const int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace & w = st->ws[stream];
    if (w.bytes < bytes) {
        if (w.ptr) {
            hipError_t e = hipDeviceSynchronize();   // also graphs replayed from a capture on this stream
            if (e != hipSuccess) return al_hip_fail(e, "hipDeviceSynchronize");
            e = hipFree(w.ptr);
            if (e != hipSuccess) return al_hip_fail(e, "hipFree(workspace)");
            w.ptr = nullptr;
            w.bytes = 0;
        }
        const size_t sz = std::max(bytes, (size_t) 4 << 20);
        hipError_t e = hipMalloc(&w.ptr, sz);
        if (e != hipSuccess) return al_fail(AL_ERR_HIP, "hipMalloc(workspace %zu bytes): %s", sz, hipGetErrorString(e));
        e = hipMemset(w.ptr, 0, sz);
        if (e != hipSuccess) return al_hip_fail(e, "hipMemset(workspace)");
        e = hipDeviceSynchronize();               // zeroed before the stream's kernels use it
        if (e != hipSuccess) return al_hip_fail(e, "hipDeviceSynchronize");
        w.bytes = sz;
    }
    *ptr = w.ptr;
    return AL_OK;
}

extern "C" int al_fattn_release_stream(void * stream) {
    int dev;
    DeviceState * st;
    const int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = st->ws.find(stream);
    if (it == st->ws.end()) return AL_OK;
    if (it->second.ptr) {
        // the stream's kernels (and graphs replayed on it) may still use it
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return al_hip_fail(e, "hipDeviceSynchronize");
        e = hipFree(it->second.ptr);
        if (e != hipSuccess) return al_hip_fail(e, "hipFree(workspace)");
    }
    st->ws.erase(it);
    return AL_OK;
}

// ---------------------------------------------------------------------------
// flash attention
// ---------------------------------------------------------------------------

namespace {

enum Kernel { kSplitKV, kPrefill, kDecode };

struct Plan {
    FattnParams p;
    Kernel kernel = kSplitKV;
    int waves = 2;                  // decode kernel: wavefronts per workgroup
    int stages = 2;                 // decode kernel: LDS stage buffers
    int rows_per_tile = 16;
    size_t part_offset = 0;         // merge records: workspace offset and bytes (0: none)
    size_t part_bytes = 0;
    size_t workspace_bytes() const { return part_bytes ? part_offset + part_bytes : 0; }
};

bool aligned16(const void * ptr) { return ((uintptr_t) ptr & 15u) == 0; }

// ceil(2^32 / d) for d >= 2, 0 for d <= 1: x / d = umulhi(x, magic) when x d < 2^32
uint32_t magic_u32(const int64_t d) {
    return d > 1 ? (uint32_t) (((1ull << 32) + (uint64_t) d - 1) / (uint64_t) d) : 0u;
}

// AL_FATTN_PREFILL=0 keeps many-row calls on the split-KV kernel.
bool prefer_prefill() {
    static bool v = [] {
        const char * s = getenv("AL_FATTN_PREFILL");
        return !(s && s[0] == '0');
    }();
    return v;
}

int env_int(const char * name, int dflt) {
    const char * s = getenv(name);
    const int x = s ? atoi(s) : 0;
    return x > 0 ? x : dflt;
}

// Fewest query rows per kv head that go to the prefill kernel
// (AL_PREFILL_MIN_ROWS); fewer take the decode or split-KV kernel.
int prefill_min_rows() {
    static int v = env_int("AL_PREFILL_MIN_ROWS", 256);
    return v;
}

// Rows per prefill row tile forced by AL_PREFILL_ROWS (64 or 128); 0: by shape.
int prefill_rows_forced() {
    static int v = [] {
        const int x = env_int("AL_PREFILL_ROWS", 0);
        return x == 64 || x == 128 ? x : 0;
    }();
    return v;
}

// Prefill workgroup splits: at most AL_PREFILL_MAX_SPLIT per row tile, and a
// split only when each workgroup keeps at least AL_PREFILL_SPLIT_TILES 64-cell
// tiles per in-workgroup split.
int prefill_max_split() {
    static int v = std::min(env_int("AL_PREFILL_MAX_SPLIT", kFattnPrefillMaxSplit), kFattnPrefillMaxSplit);
    return v;
}
int prefill_split_tiles() {
    static int v = env_int("AL_PREFILL_SPLIT_TILES", 4);
    return v;
}

int wgs_per_cu() {
    static int v = env_int("AL_SPLITKV_WGS_PER_CU", 2);
    return v;
}

// AL_FATTN_DECODE=0 keeps decode calls on the split-KV kernel.
bool prefer_decode() {
    static bool v = [] {
        const char * s = getenv("AL_FATTN_DECODE");
        return !(s && s[0] == '0');
    }();
    return v;
}

// Decode kernel sizing: workgroups per CU to aim for, and the fewest 16-cell
// stages a split may hold.
int decode_wgs_per_cu() {
    static int v = env_int("AL_DECODE_WGS_PER_CU", 4);
    return v;
}
// Decode kernel shape: wavefronts per workgroup (AL_DECODE_WAVES) and LDS
// stage buffers per wave (AL_DECODE_STAGES); combinations without a kernel
// fall back to 2 x 3. Unset: 2 x 3 for up to 8 query rows per kv head
// (decode and 2-draft verify; fewer, deeper streams per CU beat more of
// them), 8 x 2 for more (verify of 4 or more drafts, whose final merge of
// 16- or 32-row records is bound by the lanes the last workgroup brings to
// it: 16 rows at 4096 / 16384 / 32768 cells take 21.8 / 28.9 / 37.7 us with
// 2 x 3 and 15.0 / 25.7 / 37.5 us with 8 x 2).
int decode_waves(int rows) {
    static int v = env_int("AL_DECODE_WAVES", 0);
    return v > 0 ? v : (rows <= 8 ? 2 : 8);
}
int decode_stages(int rows) {
    static int v = env_int("AL_DECODE_STAGES", 0);
    return v > 0 ? v : (rows <= 8 ? 3 : 2);
}
// AL_DECODE_INTERLEAVE=0: each split takes a contiguous cell range.
bool decode_interleave() {
    static bool v = [] {
        const char * s = getenv("AL_DECODE_INTERLEAVE");
        return !(s && s[0] == '0');
    }();
    return v;
}
int decode_min_stages() {
    static int v = env_int("AL_DECODE_MIN_STAGES", 2);
    return v;
}
// Query rows each merging workgroup of a split decode call takes
// (AL_DECODE_MERGE_ROWS overrides). A merger is bound by the record bytes
// its CU loads (32 splits x 520 bytes per row), but every merger polls the
// same flag line, so few of them. Up to 8 rows per kv head (one token, the
// 2-wave shape): 2 rows each (4K decode 10.07 -> 9.62 us per layer, the
// decode block 34.05 -> 33.53, 32K unchanged); more rows (verify, the 8-wave
// shape): 8 rows each (4-draft verify 2 mergers, 8-draft 4: 21.7 -> 16.7 us
// per layer at 8K cells; 2 rows each 15.2 against 14.2 for 4 drafts).
int decode_merge_rows(int rows) {
    static int v = env_int("AL_DECODE_MERGE_ROWS", 0);
    return v > 0 ? v : (rows <= 8 ? 2 : 8);
}
// Splits of up to this many cells (AL_DECODE_ONE_PASS_CELLS, 0: never; read
// on every call, so that one process can compare the two forms) merge the
// 2 x 3 shape's two waves in one pass with all threads, which shortens the
// tail of short splits (4K / 8K / 16K decode 9.5 / 11.5 / 16.4 -> 9.1 / 11.2
// / 16.1 us per layer, 2-draft verify at 8K 12.9 -> 12.5); with 1024 cells
// per split (32K) the tree merge is faster (25.8 against 26.7 us).
int decode_one_pass_cells() {
    const char * s = getenv("AL_DECODE_ONE_PASS_CELLS");
    return s && s[0] ? atoi(s) : 512;
}
// AL_DECODE_MASK_PRE=0: decode loads the mask rows with every stage, never
// preloaded (read on every call that has a mask tensor, so that one process
// can compare the two forms).
bool decode_mask_pre() {
    const char * s = getenv("AL_DECODE_MASK_PRE");
    return !(s && s[0] == '0');
}
// Most splits per (stream, kv head) (AL_DECODE_MAX_SPLIT, at most kFattnMaxSplit).
int decode_max_split() {
    static int v = std::min(env_int("AL_DECODE_MAX_SPLIT", kFattnMaxSplit), kFattnMaxSplit);
    return v;
}

// Mirrors the asserts of nnml_flash_attn_ext (nnml/src/tensor.cpp:1292-1320)
// and nnml_compute_forward_flash_attn_ext_f16 (arm.cpp:2213-2245), then the
// limits of this path.
int make_plan(const al_fattn_args * a, int n_cu, int lds_per_block, Plan * out) {
    if (!a) return al_fail(AL_ERR_INVALID, "fattn: null arguments");
    const al_tensor &q = a->q, &k = a->k, &v = a->v, &m = a->mask, &s = a->sinks, &d = a->dst;
    if (!q.data || !k.data || !v.data || !d.data) return al_fail(AL_ERR_INVALID, "fattn: q, k, v and dst are required");
    if (a->prec != AL_PREC_DEFAULT && a->prec != AL_PREC_F32)
        return al_fail(AL_ERR_INVALID, "fattn: prec %d is not DEFAULT or F32 (ops.cpp:1441-1443)", a->prec);
    const int64_t D = k.ne[0], DV = v.ne[0], T = q.ne[1], Hq = q.ne[2], B = q.ne[3];
    const int64_t n_kv = k.ne[1], Hkv = k.ne[2];
    // nnml_can_mul_mat(k, q) (tensor.cpp:1294)
    if (q.ne[0] != D) return al_fail(AL_ERR_INVALID, "fattn: q ne0 %lld != k ne0 %lld", (long long) q.ne[0], (long long) D);
    if (Hkv <= 0 || Hq % Hkv != 0 || k.ne[3] <= 0 || B % k.ne[3] != 0)
        return al_fail(AL_ERR_INVALID, "fattn: q heads/streams (%lld, %lld) do not broadcast over k (%lld, %lld)",
                       (long long) Hq, (long long) B, (long long) Hkv, (long long) k.ne[3]);
    if (v.ne[1] != n_kv) return al_fail(AL_ERR_INVALID, "fattn: v cells %lld != k cells %lld", (long long) v.ne[1], (long long) n_kv);
    if (v.ne[2] <= 0 || Hq % v.ne[2] != 0 || v.ne[3] <= 0 || B % v.ne[3] != 0)
        return al_fail(AL_ERR_INVALID, "fattn: q heads/streams do not broadcast over v");
    // rows contiguous (arm.cpp:2224-2226)
    if (q.nb[0] != 4 || k.nb[0] != 2 || v.nb[0] != 2) return al_fail(AL_ERR_INVALID, "fattn: q/k/v rows must be contiguous");
    // dst not permuted (arm.cpp:2219-2238)
    if (d.ne[0] != DV || d.ne[1] != Hq || d.ne[2] != T || d.ne[3] != B)
        return al_fail(AL_ERR_INVALID, "fattn: dst must be [DV, Hq, T, B]");
    if (d.nb[0] != 4 || d.nb[0] > d.nb[1] || d.nb[1] > d.nb[2] || d.nb[2] > d.nb[3])
        return al_fail(AL_ERR_INVALID, "fattn: dst cannot be transposed or permuted");
    if (m.data) {
        const int64_t tpad = (T + 63) / 64 * 64;
        if (m.ne[1] < tpad) return al_fail(AL_ERR_INVALID, "fattn: mask has %lld rows, needs >= PAD(T,64) = %lld (tensor.cpp:1300-1301)",
                                           (long long) m.ne[1], (long long) tpad);
        if (m.ne[0] < n_kv) return al_fail(AL_ERR_INVALID, "fattn: mask has %lld columns < n_kv %lld", (long long) m.ne[0], (long long) n_kv);
        if (m.ne[2] <= 0 || m.ne[3] <= 0 || Hq % m.ne[2] != 0 || B % m.ne[3] != 0)
            return al_fail(AL_ERR_INVALID, "fattn: mask dims 2/3 do not broadcast (tensor.cpp:1302-1303)");
        if (m.nb[0] != 2) return al_fail(AL_ERR_INVALID, "fattn: mask must be contiguous (tensor.cpp:1298)");
    } else if (a->max_bias > 0.0f) {
        return al_fail(AL_ERR_INVALID, "fattn: max_bias > 0 requires a mask (tensor.cpp:1305-1307)");
    }
    if (s.data && (s.type != AL_TYPE_F32 || s.ne[0] != Hq))
        return al_fail(AL_ERR_INVALID, "fattn: sinks must be f32 [Hq] (tensor.cpp:1328-1329)");

    // limits of this path
    if (q.type != AL_TYPE_F32) return al_fail(AL_ERR_UNSUPPORTED, "fattn: q type %d (f32 only)", q.type);
    if (k.type != AL_TYPE_F16 || v.type != AL_TYPE_F16)
        return al_fail(AL_ERR_UNSUPPORTED, "fattn: k/v types %d/%d (f16 K/V cache only)", k.type, v.type);
    if (d.type != AL_TYPE_F32) return al_fail(AL_ERR_UNSUPPORTED, "fattn: dst type %d (f32 only)", d.type);
    if (m.data && m.type != AL_TYPE_F16) return al_fail(AL_ERR_UNSUPPORTED, "fattn: mask type %d (f16 only)", m.type);
    if (D != 128 || DV != 128) return al_fail(AL_ERR_UNSUPPORTED, "fattn: head dim %lld/%lld (128 only)", (long long) D, (long long) DV);
    if (v.ne[2] != Hkv || v.ne[3] != k.ne[3]) return al_fail(AL_ERR_UNSUPPORTED, "fattn: k and v must have the same heads and streams");
    if (!aligned16(q.data) || !aligned16(k.data) || !aligned16(v.data) || !aligned16(d.data) ||
        q.nb[1] % 16 || q.nb[2] % 16 || q.nb[3] % 16 || k.nb[1] % 16 || k.nb[2] % 16 || k.nb[3] % 16 ||
        v.nb[1] % 16 || v.nb[2] % 16 || v.nb[3] % 16 || d.nb[1] % 16)
        return al_fail(AL_ERR_UNSUPPORTED, "fattn: operands must be 16-byte aligned with 16-byte multiple strides");
    if (n_kv <= 0 || n_kv > INT32_MAX / 2 || T <= 0 || T > (1 << 24) || B > 65535 || Hq * T > INT32_MAX / 2)
        return al_fail(AL_ERR_UNSUPPORTED, "fattn: sizes out of range");
    // K/V of one (stream, head) are addressed with 32-bit buffer offsets
    if ((uint64_t) (n_kv - 1) * k.nb[1] + 256 > (uint64_t) INT32_MAX || (uint64_t) (n_kv - 1) * v.nb[1] + 256 > (uint64_t) INT32_MAX)
        return al_fail(AL_ERR_UNSUPPORTED, "fattn: one head's K/V view spans more than 2 GiB");

    Plan pl;
    FattnParams & p = pl.p;
    memset(&p, 0, sizeof(p));
    p.q = (const char *) q.data; p.q_nb1 = q.nb[1]; p.q_nb2 = q.nb[2]; p.q_nb3 = q.nb[3];
    const uint64_t q_slice = (uint64_t) (T - 1) * q.nb[1] + (uint64_t) (Hq - 1) * q.nb[2] + (uint64_t) D * 4;
    p.q_bytes = (uint32_t) std::min<uint64_t>(q_slice, INT32_MAX);
    p.k = (const char *) k.data; p.k_nb1 = k.nb[1]; p.k_nb2 = k.nb[2]; p.k_nb3 = k.nb[3];
    p.v = (const char *) v.data; p.v_nb1 = v.nb[1]; p.v_nb2 = v.nb[2]; p.v_nb3 = v.nb[3];
    if (m.data) {
        p.mask = (const char *) m.data; p.m_nb1 = m.nb[1]; p.m_nb2 = m.nb[2]; p.m_nb3 = m.nb[3];
        p.m_ne0 = (int32_t) std::min<int64_t>(m.ne[0], INT32_MAX); p.m_ne2 = (int32_t) m.ne[2]; p.m_ne3 = (int32_t) m.ne[3];
        const uint64_t slice = (uint64_t) (m.ne[2] - 1) * m.nb[2] + (uint64_t) (m.ne[1] - 1) * m.nb[1] + (uint64_t) m.ne[0] * 2;
        p.m_slice_bytes = (uint32_t) std::min<uint64_t>(slice, INT32_MAX);
    }
    p.sinks = (const float *) s.data;
    p.dst = (char *) d.data; p.dst_nb1 = d.nb[1];
    p.T = (int32_t) T; p.Hq = (int32_t) Hq; p.Hkv = (int32_t) Hkv; p.G = (int32_t) (Hq / Hkv); p.B = (int32_t) B;
    p.R = p.T * p.G;
    p.g_magic = magic_u32(p.G);
    p.rk3 = (int32_t) (B / k.ne[3]); p.rv3 = (int32_t) (B / v.ne[3]);
    p.n_kv = (int32_t) n_kv;
    p.kv_hi = (int32_t) ((a->kv_len <= 0 || a->kv_len > n_kv) ? n_kv : a->kv_len);
    p.causal_pos0 = a->causal_pos0 < 0 ? -1 : a->causal_pos0;
    p.dyn = a->dyn_len;
    if (p.dyn && m.data) return al_fail(AL_ERR_UNSUPPORTED, "fattn: dyn_len needs implicit masking (no mask tensor)");
    p.softcap = a->logit_softcap;
    p.scale = a->scale;
    if (p.softcap != 0.0f) p.scale /= p.softcap;                        // arm.cpp:2267-2269
    p.max_bias = a->max_bias;
    p.n_head_log2 = 1u << (uint32_t) floor(log2((double) Hq));          // arm.cpp:2271-2274
    p.m0 = powf(2.0f, -(p.max_bias) / p.n_head_log2);
    p.m1 = powf(2.0f, -(p.max_bias / 2.0f) / p.n_head_log2);

    // Many query rows: the prefill kernel, one workgroup per row tile of 128
    // rows, or of 64 rows (two cell splits inside the workgroup) when
    // 128-row tiles leave CUs idle; n_split workgroups per tile (each taking
    // every n_split-th share of the 64-cell tiles of the visible range) when
    // the row tiles alone still do not fill the device. It keeps the running
    // max on scores as computed, so it needs scale > 0 unless softcapped.
    const int64_t big_units = (p.R + kFattnPrefillRows - 1) / kFattnPrefillRows * Hkv * B;
    const int prefill_rows = prefill_rows_forced() ? prefill_rows_forced()
                             : big_units >= n_cu ? kFattnPrefillRows : kFattnPrefillRows / 2;
    const int in_wg_split = kFattnPrefillRows / prefill_rows;
    const int64_t prefill_tiles = (p.R + prefill_rows - 1) / prefill_rows;
    const int64_t prefill_units = prefill_tiles * Hkv * B;
    int64_t prefill_split = 1;
    {
        int64_t extent = p.kv_hi;
        if (p.causal_pos0 >= 0) extent = std::min<int64_t>(extent, p.causal_pos0 + T);
        const int64_t cell_tiles = std::max<int64_t>(1, (extent + 63) / 64);
        while (prefill_split < prefill_max_split() && prefill_units * prefill_split < n_cu &&
               cell_tiles >= prefill_split_tiles() * in_wg_split * (prefill_split + 1))
            ++prefill_split;
    }
    // (an explicit mask: the prefill kernel reads its rows 16 bytes at a time)
    const bool mask_rows16 = !m.data || (aligned16(m.data) && m.nb[1] % 16 == 0 && m.nb[2] % 16 == 0 && m.nb[3] % 16 == 0);
    const bool prefill_shape = !p.dyn && p.R >= prefill_min_rows() && prefill_units <= kFattnCounterWords &&
                               (uint64_t) p.R * (uint64_t) p.G < (1ull << 32) && prefill_tiles * B <= 65535 &&
                               (uint64_t) (n_kv + 64) * k.nb[1] + 256 <= (uint64_t) UINT32_MAX &&
                               (uint64_t) (n_kv + 64) * v.nb[1] + 256 <= (uint64_t) UINT32_MAX && mask_rows16 &&
                               lds_per_block >= (int64_t) fattn_prefill_lds_bytes() && q_slice < INT32_MAX &&
                               (p.softcap != 0.0f || p.scale > 0.0f) && prefer_prefill();
    const size_t prefill_part = prefill_split > 1 ? (size_t) prefill_units * prefill_split * prefill_rows *
                                                        kFattnRecordStride * sizeof(float)
                                                  : 0;
    if (prefill_shape) {
        pl.kernel = kPrefill;
        pl.rows_per_tile = prefill_rows;
        p.n_row_tiles = (int32_t) prefill_tiles;
        p.n_split = (int32_t) prefill_split;
        p.cells_per_split = 0;
        p.split_magic = magic_u32(prefill_split * in_wg_split);
        p.tiles_magic = magic_u32(prefill_tiles);
        if (prefill_split > 1) {
            pl.part_offset = kFattnCounterBytes;
            pl.part_bytes = prefill_part;
        }
        *out = pl;
        return AL_OK;
    }

    // Up to 16 rows per kv head (32 with implicit masks): the decode kernel,
    // when its LDS rings fit and a head's K/V view is addressable with 32-bit
    // offsets.
    int dwaves = decode_waves(p.R), stages = decode_stages(p.R);
    if (!fattn_decode_config_ok(dwaves, stages)) {
        dwaves = 2;
        stages = 3;
    }
    // 17..32 rows (two row blocks) exist as 8 x 2
    const bool two_blocks = p.R > 16;
    if (two_blocks) {
        dwaves = 8;
        stages = 2;
    }
    const size_t decode_lds = fattn_decode_lds_bytes(dwaves, stages, m.data != nullptr, false);
    const bool mask_ok = !m.data || (p.m_slice_bytes < INT32_MAX && aligned16(m.data) && m.nb[1] % 16 == 0 &&
                                     m.nb[2] % 16 == 0 && m.nb[3] % 16 == 0);
    const int64_t decode_units = Hkv * B;
    const size_t decode_q_lds = two_blocks ? 16384 : 8192;                 // the query rows, f32
    if (p.R <= 32 && prefer_decode() && (size_t) lds_per_block >= decode_lds + decode_q_lds &&
        mask_ok &&
        q_slice < INT32_MAX &&
        decode_units <= kFattnCounterWords &&
        (uint64_t) (n_kv + 16) * k.nb[1] + 256 <= (uint64_t) UINT32_MAX &&
        (uint64_t) (n_kv + 16) * v.nb[1] + 256 <= (uint64_t) UINT32_MAX) {
        pl.kernel = kDecode;
        pl.waves = dwaves;
        pl.stages = stages;
        pl.rows_per_tile = two_blocks ? 32 : 16;
        p.n_row_tiles = 1;
        int64_t extent = p.kv_hi;                                       // with dyn_len: the bound
        if (p.causal_pos0 >= 0 && !p.dyn) extent = std::min<int64_t>(extent, p.causal_pos0 + T);
        extent = std::max<int64_t>(extent, 0);
        const int64_t nst = std::max<int64_t>(1, (extent + 15) / 16);   // 16-cell stages
        // workgroups resident per CU by LDS (160 KiB per CU on gfx950)
        const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(4, (int64_t) (160 << 10) / (int64_t) decode_lds));
        const int64_t target = (int64_t) n_cu * std::min<int64_t>(per_cu, decode_wgs_per_cu());
        int64_t n_split = (target + decode_units - 1) / decode_units;
        // every wave of a split gets at least decode_min_stages() stages
        n_split = std::min<int64_t>(n_split, std::max<int64_t>(1, nst / (dwaves * decode_min_stages())));
        n_split = std::max<int64_t>(1, std::min<int64_t>(n_split, decode_max_split()));
        // split flags: kFattnDecodeFlagWords counter words per unit
        if (decode_units > kFattnDecodeFlagUnits) n_split = 1;
        const int64_t cps = (nst + n_split - 1) / n_split;
        p.cells_per_split = (int32_t) (cps * 16);
        p.n_split = (int32_t) ((nst + cps - 1) / cps);
        p.interleave = decode_interleave() ? 1 : 0;
        p.merge_rows = decode_merge_rows((int) std::min<int64_t>(p.R, pl.rows_per_tile));
        p.one_pass = dwaves == 2 && stages == 3 && cps * 16 <= decode_one_pass_cells() ? 1 : 0;
        // A mask tensor: each wave's mask values go into LDS before its first
        // stage when the workgroup's share fits kDecodeMaskPreBytes (32 bytes
        // per stage and distinct mask row: the tokens when the heads share
        // the mask rows, else the query rows; AL_DECODE_MASK_PRE=0: with
        // every stage instead)
        if (m.data && decode_mask_pre()) {
            const int64_t rows_here = std::min<int64_t>(pl.rows_per_tile, p.R);
            const int64_t D = m.ne[2] == 1 ? (rows_here - 1) / p.G + 1 : rows_here;
            const int64_t per_wave = p.interleave ? (nst + (int64_t) dwaves * p.n_split - 1) / ((int64_t) dwaves * p.n_split)
                                                  : (cps + dwaves - 1) / dwaves;
            const int64_t wave_bytes = (per_wave * D + 31) / 32 * 1024;
            if (wave_bytes * dwaves <= kDecodeMaskPreBytes &&
                (size_t) lds_per_block >= fattn_decode_lds_bytes(dwaves, stages, true, true) + decode_q_lds) {
                p.mask_pre = 1;
                p.mask_rows = (int32_t) D;
                p.mask_wave_bytes = (int32_t) wave_bytes;
            }
        }
        if (p.n_split > 1) {
            pl.part_offset = kFattnCounterBytes;
            pl.part_bytes = (size_t) decode_units * p.n_split * pl.rows_per_tile * kDecodeRecRow;
        }
        *out = pl;
        return AL_OK;
    }

    if (p.dyn)
        return al_fail(AL_ERR_UNSUPPORTED, "fattn: dyn_len needs the decode kernel (up to 32 query rows per kv head)");

    // split-KV sizing
    pl.rows_per_tile = fattn_splitkv_rows_per_tile(std::min(p.R, 64));
    p.n_row_tiles = (p.R + pl.rows_per_tile - 1) / pl.rows_per_tile;
    int64_t extent = p.kv_hi;
    if (p.causal_pos0 >= 0) extent = std::min<int64_t>(extent, p.causal_pos0 + T);
    extent = std::max<int64_t>(extent, 0);
    const int64_t tiles = (extent + 31) / 32;
    const int64_t units = (int64_t) Hkv * p.n_row_tiles * B;
    const int64_t waves = fattn_splitkv_waves(pl.rows_per_tile);
    const int64_t target = (int64_t) n_cu * wgs_per_cu();
    int64_t n_split = (target + units - 1) / units;
    // every wave of a split gets at least one 32-cell tile
    n_split = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(n_split, (tiles + waves - 1) / waves), kFattnMaxSplit));
    int64_t cps_tiles = std::max<int64_t>(1, (tiles + n_split - 1) / n_split);
    p.cells_per_split = (int32_t) (cps_tiles * 32);
    n_split = std::max<int64_t>(1, (extent + p.cells_per_split - 1) / p.cells_per_split);
    if (units > kFattnCounterWords) n_split = 1;
    if (n_split == 1) p.cells_per_split = (int32_t) std::max<int64_t>(32, (extent + 31) / 32 * 32);
    p.n_split = (int32_t) n_split;
    if (p.n_split > 1) {
        pl.part_offset = kFattnCounterBytes;
        pl.part_bytes = (size_t) units * p.n_split * pl.rows_per_tile * kFattnRecordStride * sizeof(float);
    }
    *out = pl;
    return AL_OK;
}

}  // namespace

extern "C" uint64_t al_fattn_workspace_bytes(const al_fattn_args * a) {
    int n_cu = 0, lds = 0;
    if (al_device_cu_count(&n_cu) != AL_OK || al_device_lds_per_block(&lds) != AL_OK) return 0;
    Plan pl;
    if (make_plan(a, n_cu, lds, &pl) != AL_OK) return 0;
    return pl.workspace_bytes();
}

// One call with the plan's workspace: the caller's, else the library's for
// the stream (library_workspace), or with noalloc_ws set the no-allocation
// entry's device array, which is never grown.
// fused: the attention inputs folded into the decode kernel (fmode: their
// rotation); AL_ERR_UNSUPPORTED before any launch when the plan is not the
// decode kernel in a shape that takes them.
static int fattn_run(const al_fattn_args * a, void * noalloc_ws, size_t noalloc_bytes,
                     const DecodeInputs * fused = nullptr, int fmode = 0) {
    int n_cu = 0, lds = 0;
    int rc = al_device_cu_count(&n_cu);
    if (rc == AL_OK) rc = al_device_lds_per_block(&lds);
    if (rc != AL_OK) return rc;
    Plan pl;
    rc = make_plan(a, n_cu, lds, &pl);
    if (rc != AL_OK) return rc;
    if (fused && (pl.kernel != kDecode || !fattn_decode_fused_ok(pl.waves, pl.stages) || pl.p.R > 16 ||
                  pl.p.B != 1 || pl.p.mask))
        return al_fail(AL_ERR_UNSUPPORTED, "fattn_with_inputs: the call does not run on the decode kernel "
                       "(up to 16 rows per kv head, one stream, no mask tensor)");
    const size_t need = pl.workspace_bytes();
    if (need) {
        void * ws = noalloc_ws ? noalloc_ws : a->workspace;
        if (noalloc_ws) {
            if (noalloc_bytes < need)
                return al_fail(AL_ERR_WORKSPACE, "fattn (no allocation): the call needs %zu bytes of scratch, "
                               "more than the %zu-byte device array", need, noalloc_bytes);
        } else if (ws) {
            if (a->workspace_bytes < need)
                return al_fail(AL_ERR_WORKSPACE, "fattn: workspace %llu bytes < %zu needed",
                               (unsigned long long) a->workspace_bytes, need);
        } else {
            rc = library_workspace(need, a->stream, &ws);
            if (rc != AL_OK) return rc;
        }
        pl.p.counters = (unsigned *) ws;
        pl.p.part = (float *) ((char *) ws + pl.part_offset);
    }
    rc = al_device_error_flag(&pl.p.err);
    if (rc != AL_OK) return rc;
    hipError_t e;
    switch (pl.kernel) {
        case kPrefill: e = fattn_prefill_launch(pl.p, pl.rows_per_tile, (hipStream_t) a->stream); break;
        case kDecode:
            e = fused ? fattn_decode_launch_fused(pl.p, *fused, fmode, pl.waves, pl.stages, (hipStream_t) a->stream)
                      : fattn_decode_launch(pl.p, pl.waves, pl.stages, (hipStream_t) a->stream);
            break;
        default:       e = fattn_splitkv_launch(pl.p, pl.rows_per_tile, (hipStream_t) a->stream); break;
    }
    if (e != hipSuccess) return al_hip_fail(e, "fattn: kernel launch");
    return AL_OK;
}

extern "C" int al_fattn_f16(const al_fattn_args * a) { return fattn_run(a, nullptr, 0); }

extern "C" int al_fattn_apply_node_hints(al_fattn_args * a, const int32_t * op_params) {
    if (!a || !op_params || op_params[4] != (int32_t) AL_FATTN_HINT_TAG) return 0;
    a->kv_len = op_params[5];
    a->causal_pos0 = op_params[6] < 0 ? -1 : op_params[6];
    a->mask = al_tensor{};
    return 1;
}

// Byte range [lo, hi) an operand's elements span (esz bytes each).
static void tensor_span(const al_tensor & t, uint64_t esz, uintptr_t * lo, uintptr_t * hi) {
    uint64_t last = 0;
    for (int i = 0; i < 4; ++i)
        if (t.ne[i] > 0) last += (uint64_t) (t.ne[i] - 1) * t.nb[i];
    *lo = (uintptr_t) t.data;
    *hi = (uintptr_t) t.data + last + esz;
}

static bool spans_overlap(const al_tensor & a, uint64_t ea, const al_tensor & b, uint64_t eb) {
    if (!a.data || !b.data) return false;
    uintptr_t alo, ahi, blo, bhi;
    tensor_span(a, ea, &alo, &ahi);
    tensor_span(b, eb, &blo, &bhi);
    return alo < bhi && blo < ahi;
}

extern "C" int al_fattn_f16_with_inputs(const al_attn_inputs_args * in, const al_fattn_args * a) {
    if (!in || !a) return al_fail(AL_ERR_INVALID, "fattn_with_inputs: null arguments");
    DecodeInputs di;
    int mode = 0;
    int rc = attn_inputs_decode(in, &di, &mode);
    if (rc != AL_OK) return rc;
    // Every workgroup reads the raw inputs while the first split writes
    // q_out and the new cache rows, so no input may share memory with those
    // outputs (the pair of calls allows an in-place Q; this launch does not).
    const al_tensor * inputs[] = {&in->q, &in->q_w, &in->k, &in->k_w, &in->v, &in->pos, &in->rows};
    const uint64_t in_esz[] = {4, 4, 4, 4, 4, 4, in->rows.type == AL_TYPE_I64 ? 8u : 4u};
    for (int i = 0; i < 7; ++i)
        if (spans_overlap(*inputs[i], in_esz[i], in->q_out, 4) || spans_overlap(*inputs[i], in_esz[i], in->k_cache, 2) ||
            spans_overlap(*inputs[i], in_esz[i], in->v_cache, 2))
            return al_fail(AL_ERR_UNSUPPORTED, "fattn_with_inputs: an input shares memory with q_out or the caches "
                           "(in-place operands need al_attn_inputs_f32 then al_fattn_f16)");
    // the attention's query operand is q_out (al_fattn q axes [D, T, Hq, B]),
    // read here from the inputs' raw rows, which the kernel normalizes
    const al_tensor & q = a->q, & qo = in->q_out;
    if (q.data != qo.data || q.ne[0] != 128 || q.ne[1] != qo.ne[2] || q.ne[2] != qo.ne[1] || q.ne[3] != 1 ||
        q.nb[1] != qo.nb[2] || q.nb[2] != qo.nb[1])
        return al_fail(AL_ERR_INVALID, "fattn_with_inputs: the attention's q must view the inputs' q_out");
    // the new tokens' cache rows are the attention's cells: the K / V views
    // start at the caches with their row strides and 128-half heads
    const al_tensor & k = a->k, & v = a->v;
    if (k.data != in->k_cache.data || k.nb[1] != in->k_cache.nb[1] || k.nb[2] != 256 || k.ne[2] * 128 != in->k_cache.ne[0] ||
        v.data != in->v_cache.data || v.nb[1] != in->v_cache.nb[1] || v.nb[2] != 256 || v.ne[2] * 128 != in->v_cache.ne[0])
        return al_fail(AL_ERR_UNSUPPORTED, "fattn_with_inputs: the K / V views are not the caches the inputs write");
    al_fattn_args aa = *a;
    aa.q.data = in->q.data;
    aa.q.nb[1] = in->q.nb[2];
    aa.q.nb[2] = in->q.nb[1];
    aa.q.nb[3] = in->q.nb[3];
    return fattn_run(&aa, nullptr, 0, &di, mode);
}

extern "C" int al_fattn_f16_worker(const al_fattn_args * a, int ith, int nth) {
    if (nth < 1 || ith < 0 || ith >= nth) return al_fail(AL_ERR_INVALID, "fattn: worker %d of %d", ith, nth);
    if (ith != 0) return AL_OK;                        // one launch per node
    const int rc = fattn_run(a, nullptr, 0);
    if (rc != AL_OK) return rc;
    const hipError_t e = hipStreamSynchronize((hipStream_t) a->stream);
    if (e != hipSuccess) return al_hip_fail(e, "fattn: hipStreamSynchronize");
    // errors the kernels recorded (a merge that gave up waiting writes NaN
    // rows and sets one), reported here as the reference's asserts would stop
    return al_device_errors();
}

// ---------------------------------------------------------------------------
// no-allocation entry point
// ---------------------------------------------------------------------------

// The scratch of al_fattn_f16_noalloc: arrival counters, decode split flags
// and merge records, laid out as a caller workspace. One copy per GPU,
// held until the process ends; every call on that GPU shares it.
static __device__ __align__(256) unsigned char scratch[AL_FATTN_NOALLOC_SCRATCH_BYTES];

__global__ void zero_words_kernel(unsigned * p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

extern "C" int al_fattn_noalloc_init(void) {
    int dev;
    DeviceState * st;
    int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if (st->noalloc) return AL_OK;
    void * ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return al_hip_fail(e, "hipGetSymbolAddress(scratch)");
    // the counter region must start at zero (every call leaves it so)
    const int words = (int) (kFattnCounterBytes / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, nullptr, (unsigned *) ptr, words);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return al_hip_fail(e, "clearing the scratch counters");
    st->noalloc = ptr;
    return AL_OK;
}

extern "C" int al_fattn_f16_noalloc(const al_fattn_args * a) {
    int dev;
    DeviceState * st;
    int rc = device_state(&dev, &st);
    if (rc != AL_OK) return rc;
    void * scratch_ptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        scratch_ptr = st->noalloc;
    }
    if (!scratch_ptr) {
        rc = al_fattn_noalloc_init();
        if (rc != AL_OK) return rc;
        std::lock_guard<std::mutex> lk(g_mu);
        scratch_ptr = st->noalloc;
    }
    return fattn_run(a, scratch_ptr, AL_FATTN_NOALLOC_SCRATCH_BYTES);
}

extern "C" const char * al_last_error(void) { return g_last_error.c_str(); }

extern "C" const char * al_version(void) { return "arclight_amd fattn 0.1 (gfx950)"; }

extern "C" int al_device_errors(void) {
    int * flag = nullptr;
    int rc = al_device_error_flag(&flag);
    if (rc != AL_OK) return rc;
    int h[4] = {0, 0, 0, 0};
    hipError_t e = hipMemcpy(h, flag, sizeof(h), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return al_hip_fail(e, "hipMemcpy(error flag)");
    if (h[0] || h[2]) {
        e = hipMemset(flag, 0, sizeof(h));
        if (e != hipSuccess) return al_hip_fail(e, "hipMemset(error flag)");
        if (h[0]) return al_fail(AL_ERR_INVALID, "set_rows: row index %d out of range (ops.cpp:171)", h[1]);
        return al_fail(AL_ERR_HIP, "fattn: a merging workgroup gave up waiting for the other splits' records");
    }
    return AL_OK;
}
