// C ABI of libmtlattn_hip.so (declared in include/mtlattn_capi.h): argument
// validation, kernel-family routing and workspace sizing. Replaces the host
// dispatcher of the reference (src/ext.mm:293-773) minus everything torch- or
// Metal-specific; it never allocates device memory and never syncs the host.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/mtlattn_capi.h"
#include "kernels.h"

using namespace mtlattn;

// Scratch of mtlattn_varlen_fwd_noalloc: the split-KV partials live in this
// file-scope device array instead of a caller's workspace. Each GPU the
// library runs on holds its own copy (MTLATTN_NOALLOC_SCRATCH_BYTES) from the
// first call on that GPU until the process ends. In host code `scratch` is
// only a symbol handle: its device address comes from hipGetSymbolAddress,
// once per device (device_scratch below), and only that address is ever
// passed to kernels.
static __device__ __align__(256) char scratch[MTLATTN_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return MTLATTN_OK;
}

int launch_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    return fail(MTLATTN_ERR_LAUNCH, "mtlattn: %s launch failed: %s", what, hipGetErrorString(e));
}

bool env_set(const char* name) {
    const char* v = std::getenv(name);
    return v != nullptr && v[0] != '\0' && std::strcmp(v, "0") != 0;
}

// Force the portable VALU kernels (MTLATTN_NO_MPP keeps the reference's name
// for "skip the fast path", src/ext.mm:396).
bool force_generic() { return env_set("MTLATTN_NO_MPP") || env_set("MTLATTN_NO_MFMA"); }

bool is16(int dtype) { return dtype == MTLATTN_DTYPE_F16 || dtype == MTLATTN_DTYPE_BF16; }

int elem_size(int dtype) { return dtype == MTLATTN_DTYPE_F32 ? 4 : 2; }

bool aligned16(const void* ptr, int64_t row_stride, int dtype) {
    return ((uintptr_t)ptr & 15u) == 0 && (row_stride * elem_size(dtype)) % 16 == 0;
}

// The matrix-core kernels address a staged 64-row tile with 32-bit per-lane
// byte offsets: row strides below 2^25 elements (the reference passes row
// strides as uint32, src/ext.mm:48-51). Larger strides take the portable
// kernels.
bool tile_stride_ok(int64_t row_stride) { return row_stride >= 0 && row_stride < (int64_t(1) << 25); }

// Shape/flag checks shared by every entry (src/ext.mm:306-331).
int check_problem(const mtlattn_problem* p) {
    if (p == nullptr) return fail(MTLATTN_ERR_INVALID, "mtlattn: null problem descriptor");
    if (p->dtype != MTLATTN_DTYPE_F32 && p->dtype != MTLATTN_DTYPE_F16 && p->dtype != MTLATTN_DTYPE_BF16)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: unsupported dtype code %d", p->dtype);
    if (p->num_seqs < 1) return fail(MTLATTN_ERR_INVALID, "mtlattn: cu_seqlens_q/kv must both be [B+1]");
    if (p->total_q < 0 || p->total_kv < 0) return fail(MTLATTN_ERR_INVALID, "mtlattn: negative token count");
    if (p->total_q > 0x7fffffffLL || p->total_kv > 0x7fffffffLL)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: more than 2^31 tokens is unsupported");
    if (p->head_dim < 1 || p->head_dim > 256)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: head_dim %d unsupported (expected 1..256)", p->head_dim);
    if (p->num_heads_kv <= 0 || p->num_heads_q <= 0 || p->num_heads_q % p->num_heads_kv != 0)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: query heads (%d) must be a multiple of kv heads (%d)",
                    p->num_heads_q, p->num_heads_kv);
    if (p->cu_seqlens_q == nullptr || p->cu_seqlens_kv == nullptr)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: cu_seqlens must be device int32 pointers");
    if (p->bias != nullptr) {
        if (p->bias_q_stride < 0 || p->bias_h_stride < 0 || p->bias_kv_cols < 0 ||
            (p->bias_seq_local != 0 && (p->bias_seq_stride < 0 || p->bias_seq_rows < 1)))
            return fail(MTLATTN_ERR_INVALID, "mtlattn: attn_mask strides must be non-negative");
    }
    return MTLATTN_OK;
}

Geometry make_geo(const mtlattn_problem* p) {
    Geometry g;
    g.cu_q = p->cu_seqlens_q;
    g.cu_kv = p->cu_seqlens_kv;
    g.total_q = p->total_q;
    g.total_kv = p->total_kv;
    g.num_seqs = p->num_seqs;
    g.hq = p->num_heads_q;
    g.hkv = p->num_heads_kv;
    g.g = p->num_heads_q / p->num_heads_kv;
    g.d = p->head_dim;
    g.scale = p->scale;
    g.causal = p->causal ? 1 : 0;
    g.window = p->window > 0 ? p->window : 0;
    // a bias with no columns reads as 0 everywhere: the same as none
    g.bias = p->bias_kv_cols > 0 ? p->bias : nullptr;
    g.bias_qs = p->bias_q_stride;
    g.bias_hs = p->bias_h_stride;
    g.bias_cols = p->bias_kv_cols;
    g.bias_ss = p->bias_seq_local != 0 ? p->bias_seq_stride : -1;
    g.bias_rows = p->bias_seq_local != 0 ? p->bias_seq_rows : 0;
    return g;
}

int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// Heads per 16-row decode group (largest divisor of g with heads * max_q <= 16).
int decode_heads_per_group(int g, int max_q) {
    int hpb = 16 / (max_q > 0 ? max_q : 1);
    if (hpb > g) hpb = g;
    if (hpb < 1) hpb = 1;
    while (g % hpb != 0) --hpb;
    return hpb;
}

// Split-KV applicability without the routing heuristics (kernel limits).
bool splitkv_supported(const mtlattn_problem* p) {
    return is16(p->dtype) && decode_head_dim(p->head_dim) && p->max_seqlen_q >= 1 && p->max_seqlen_q <= 16;
}

// Partial rows of the split-KV workspace for ns equal splits per sequence
// (chunk == 0) or fixed KV chunks of `chunk` keys.
int64_t splitkv_rows(const mtlattn_problem* p, int ns, int chunk) {
    const int g = p->num_heads_q / p->num_heads_kv;
    const int n_hg = g / decode_heads_per_group(g, p->max_seqlen_q);
    return decode_workspace_rows(p->total_kv, p->num_seqs, p->num_heads_kv, n_hg, chunk, ns);
}

size_t splitkv_bytes(const mtlattn_problem* p, int ns, int chunk) {
    const size_t rows = (size_t)splitkv_rows(p, ns, chunk);
    const size_t o = rows * (size_t)p->head_dim * sizeof(float);
    return ((o + 255) & ~(size_t)255) + rows * sizeof(float);
}

struct PagedKV {
    const int32_t* block_table;
    int64_t bt_stride, num_pages;
    int page_size;
};

int run_splitkv(const mtlattn_problem* p, const void* q, int64_t qrs, const void* k, int64_t krs, const void* v,
                int64_t vrs, void* out, float* lse, int ns, int chunk, void* ws, size_t ws_bytes, hipStream_t st,
                const PagedKV* paged = nullptr) {
    const size_t need = splitkv_bytes(p, ns, chunk);
    if (ws_bytes < need || (ws == nullptr && need > 0))
        return fail(MTLATTN_ERR_WORKSPACE, "mtlattn: split-KV workspace too small (%zu < %zu bytes)", ws_bytes,
                    need);
    DecodeArgs a;
    a.geo = make_geo(p);
    a.q = q; a.q_rs = qrs; a.k = k; a.k_rs = krs; a.v = v; a.v_rs = vrs;
    a.o = out; a.lse = lse;
    const size_t obytes = (size_t)splitkv_rows(p, ns, chunk) * (size_t)p->head_dim * sizeof(float);
    a.o_part = (float*)ws;
    a.lse_part = (float*)((char*)ws + ((obytes + 255) & ~(size_t)255));
    a.num_splits = ns;
    a.chunk = chunk;
    a.max_q = p->max_seqlen_q;
    if (paged != nullptr) {
        a.block_table = paged->block_table;
        a.bt_stride = paged->bt_stride;
        a.page_size = paged->page_size;
        a.num_pages = (int)paged->num_pages;
    }
    return launch_status(launch_decode(p->dtype, a, st), "split-KV decode");
}

// Work split of the automatic decode path (reference gate src/ext.mm:372-376:
// few queries and long KV; here also with a window or a bias, which the
// reference keeps off its split path). Without a window every sequence's KV
// is cut into fixed chunks of `chunk` keys (a multiple of 256), sized so that
// about 18 work items per CU exist (measured on MI355X: fewer leave a ragged
// last round, more add per-item start-up and partial-row traffic), so every
// wave streams the same number of bytes whatever the spread of KV lengths.
// With a window only the last W + q_len - 1 keys of a sequence can be seen:
// each sequence gets `ns` equal splits of that band instead (chunk == 0), so
// the work items and the workspace scale with the band, not the KV length.
constexpr int64_t kItemsPerCu = 18;

struct DecodePlan {
    int chunk = 0;    // > 0: fixed KV chunks of this many keys
    int ns = 0;       // > 0: equal splits per sequence over the window band
    bool routed() const { return chunk > 0 || ns > 0; }
};

// Chunk length (keys, a multiple of 256 in [256, 8192]) for `work` keys of
// work per (kv head, head group).
int64_t plan_chunk(const mtlattn_problem* p, int64_t work) {
    const int g = p->num_heads_q / p->num_heads_kv;
    const int64_t groups = (int64_t)p->num_heads_kv * (g / decode_heads_per_group(g, p->max_seqlen_q));
    const int64_t items = (int64_t)device_cus() * kItemsPerCu;
    int64_t c = (work * groups + items - 1) / items;
    if (const char* e = std::getenv("MTLATTN_DECODE_CHUNK")) {   // tuning override (keys)
        const long v = std::strtol(e, nullptr, 10);
        if (v > 0) c = v;
    }
    c = (c + 128) / 256 * 256;      // nearest multiple of 256 keys
    if (c < 256) c = 256;
    if (c > 8192) c = 8192;
    return c;
}

// Keys a sequence of `kv` keys lets its rows see: the window band (W +
// q_len - 1, plus up to 31 below it for the tile-aligned start) or all.
int64_t band_keys(const mtlattn_problem* p, int64_t kv) {
    if (p->window <= 0) return kv;
    const int64_t band = (int64_t)p->window + p->max_seqlen_q - 1 + 31;
    return kv < band ? kv : band;
}

DecodePlan decode_plan(const mtlattn_problem* p) {
    DecodePlan plan;
    if (check_problem(p) != MTLATTN_OK) return plan;
    if (p->total_q <= 0 || env_set("MTLATTN_NO_SPLITKV") || force_generic() || !splitkv_supported(p)) return plan;
    const int64_t avg_kv = p->total_kv / (p->num_seqs > 0 ? p->num_seqs : 1);
    // keys a sequence's rows see on average (the window band at most)
    const int64_t band = (int64_t)p->window + p->max_seqlen_q - 1;
    const int64_t eff = p->window > 0 && avg_kv > band ? band : avg_kv;
    if (eff < 2048) return plan;
    if (p->window <= 0) {
        plan.chunk = (int)plan_chunk(p, p->total_kv);
    } else {
        // the splits must cover the longest band: W + q_len - 1 keys plus up
        // to 31 below its tile-aligned start
        const int64_t c = plan_chunk(p, eff * p->num_seqs);
        plan.ns = (int)((band + 31 + c - 1) / c);
    }
    return plan;
}

// Paged decode: the logical KV total is device data, p->total_kv bounds it.
// Without a window, fixed chunks as on the contiguous path (slots for the
// bound; chunks past a sequence's end exit at once); with one, equal splits
// of the band sized for num_seqs bands of work.
DecodePlan paged_plan(const mtlattn_problem* p, int64_t max_seqlen_kv) {
    DecodePlan plan;
    if (p->window <= 0) {
        plan.chunk = (int)plan_chunk(p, p->total_kv > 0 ? p->total_kv : 1);
        return plan;
    }
    const int64_t span = band_keys(p, max_seqlen_kv > 0 ? max_seqlen_kv : 1);
    const int64_t c = plan_chunk(p, span * p->num_seqs);
    plan.ns = (int)((span + c - 1) / c);
    return plan;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch (set up on the first call
// on that device), or nullptr with the error recorded.
void* device_scratch(int* code) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *code = fail(MTLATTN_ERR_LAUNCH, "mtlattn: no current HIP device for the static scratch (%s)",
                     hipGetErrorString(e));
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            *code = fail(MTLATTN_ERR_LAUNCH, "mtlattn: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                         hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int mtlattn_abi_version(void) { return MTLATTN_ABI_VERSION; }

const char* mtlattn_last_error(void) { return g_last_error.c_str(); }

int mtlattn_gpu_core_count(int device) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
        fail(MTLATTN_ERR_INVALID, "mtlattn: no HIP device %d", device);
        return 0;
    }
    return n;
}

int32_t mtlattn_decode_num_splits(const mtlattn_problem* p) {
    const DecodePlan plan = decode_plan(p);
    if (!plan.routed()) return 0;
    const int64_t slots = plan.chunk > 0 ? p->total_kv / plan.chunk + p->num_seqs + 1
                                         : (int64_t)p->num_seqs * plan.ns;
    return slots > 0x7fffffff ? 0x7fffffff : (int32_t)slots;
}

namespace {

// Splits of the fp32 matrix-core forward over its key tiles: when its grid
// (one workgroup per 128 query rows and head) holds fewer than two
// workgroups per CU, up to 8 splits, no more than the key tiles, and few
// enough that the partials fit the no-allocation scratch, so that
// mtlattn_varlen_fwd_noalloc splits alike and stays bitwise equal.
int f32_fwd_splits(const mtlattn_problem* p) {
    if (p->dtype != MTLATTN_DTYPE_F32 || !f32_mfma_head_dim(p->head_dim) || force_generic() || p->total_q <= 0 ||
        p->total_kv <= 0)
        return 1;
    const int64_t tiles = std::max<int64_t>((p->total_q + 127) / 128, p->num_seqs);
    const int64_t wgs = tiles * p->num_heads_q, want = 2 * (int64_t)device_cus();
    if (wgs >= want) return 1;
    int64_t ns = std::min<int64_t>(std::min<int64_t>((want + wgs - 1) / wgs, 8), (p->total_kv + 31) / 32);
    const int64_t per_split = (int64_t)p->total_q * p->num_heads_q * (p->head_dim + 1) * (int64_t)sizeof(float);
    ns = std::min<int64_t>(ns, (int64_t)MTLATTN_NOALLOC_SCRATCH_BYTES / std::max<int64_t>(per_split, 1));
    return ns >= 2 ? (int)ns : 1;
}

size_t fwd_part_bytes(const mtlattn_problem* p, int splits) {
    return (size_t)f32_fwd_part_floats(splits, p->total_q, p->num_heads_q, p->head_dim) * sizeof(float);
}

}  // namespace

size_t mtlattn_varlen_fwd_workspace_size(const mtlattn_problem* p) {
    const DecodePlan plan = decode_plan(p);
    if (plan.routed()) return splitkv_bytes(p, plan.ns, plan.chunk);
    if (check_problem(p) != MTLATTN_OK) return 0;
    return fwd_part_bytes(p, f32_fwd_splits(p));
}

int mtlattn_varlen_fwd(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k,
                       int64_t k_row_stride, const void* v, int64_t v_row_stride, void* out, float* lse,
                       void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (p->total_q == 0) return ok();
    if (q == nullptr || out == nullptr || (p->total_kv > 0 && (k == nullptr || v == nullptr)))
        return fail(MTLATTN_ERR_INVALID, "mtlattn: null q/k/v/out pointer");
    hipStream_t st = (hipStream_t)stream;
    const DecodePlan plan = decode_plan(p);
    const bool vec_ok = aligned16(q, q_row_stride, p->dtype) && aligned16(k, k_row_stride, p->dtype) &&
                        aligned16(v, v_row_stride, p->dtype) && ((uintptr_t)out & 15u) == 0;
    if (plan.routed() && vec_ok)
        return run_splitkv(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, out, lse, plan.ns, plan.chunk,
                           workspace, workspace_bytes, st);
    FwdArgs a;
    a.geo = make_geo(p);
    a.q = q; a.q_rs = q_row_stride; a.k = k; a.k_rs = k_row_stride; a.v = v; a.v_rs = v_row_stride;
    a.o = out; a.lse = lse;
    if (is16(p->dtype) && mfma_head_dim(p->head_dim) && vec_ok && tile_stride_ok(k_row_stride) &&
        tile_stride_ok(v_row_stride) && !force_generic())
        return launch_status(launch_fwd_mfma(p->dtype, a, st), "flash forward");
    if (p->dtype == MTLATTN_DTYPE_F32 && f32_mfma_head_dim(p->head_dim) && vec_ok && !force_generic()) {
        // split partials in the workspace when it holds them (the size query
        // counts them); a smaller workspace runs unsplit
        const int splits = f32_fwd_splits(p);
        if (splits > 1 && workspace != nullptr && ((uintptr_t)workspace & 15u) == 0 &&
            workspace_bytes >= fwd_part_bytes(p, splits)) {
            a.f32_part = (float*)workspace;
            a.f32_splits = splits;
        }
        return launch_status(launch_fwd_f32mfma(a, st), "fp32 flash forward");
    }
    return launch_status(launch_fwd_generic(p->dtype, a, st), "generic forward");
}

int mtlattn_varlen_fwd_noalloc(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k,
                               int64_t k_row_stride, const void* v, int64_t v_row_stride, void* out, float* lse,
                               void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (p->total_q == 0) return ok();
    // the workspace mtlattn_varlen_fwd would need: split-KV partials when the
    // call is routed to decode, the key-split partials of an fp32 forward on a
    // small grid (f32_fwd_splits caps their count so that they fit the static
    // scratch), nothing for the 16-bit flash forward
    const size_t need = mtlattn_varlen_fwd_workspace_size(p);
    if (need == 0)
        return mtlattn_varlen_fwd(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, out, lse, nullptr, 0, stream);
    if (need > (size_t)MTLATTN_NOALLOC_SCRATCH_BYTES)
        return fail(MTLATTN_ERR_WORKSPACE,
                    "mtlattn: varlen_fwd_noalloc: this call needs %zu bytes of split-KV scratch, more than the "
                    "static %lld bytes; use mtlattn_varlen_fwd with a workspace",
                    need, (long long)MTLATTN_NOALLOC_SCRATCH_BYTES);
    void* ws = device_scratch(&rc);
    if (ws == nullptr) return rc;
    return mtlattn_varlen_fwd(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, out, lse, ws, need, stream);
}

namespace {

size_t bwd_delta_bytes(const mtlattn_problem* p) { return (size_t)p->total_q * (size_t)p->num_heads_q * sizeof(float); }
// offset of the fp32 dK/dV partials in the backward workspace
size_t bwd_part_offset(const mtlattn_problem* p) { return (bwd_delta_bytes(p) + 255) / 256 * 256; }

// Splits of the fp32 matrix-core dK/dV: its grid has one workgroup per 128
// keys and kv head, which leaves CUs idle on small problems and few kv heads;
// split each workgroup's (query head, query tile) iterations until there are
// about two workgroups per CU, at most 8 splits and no more than the
// iterations of the longest sequence.
int f32_dkv_splits(const mtlattn_problem* p) {
    if (p->dtype != MTLATTN_DTYPE_F32 || !f32_mfma_head_dim(p->head_dim) || force_generic() || p->total_q <= 0 ||
        p->total_kv <= 0)
        return 1;
    const int64_t tiles = std::max<int64_t>((p->total_kv + 127) / 128, p->num_seqs);
    const int64_t wgs = tiles * p->num_heads_kv, want = 2 * (int64_t)device_cus();
    if (wgs >= want) return 1;
    const int64_t iters = (int64_t)(p->num_heads_q / p->num_heads_kv) * ((std::max<int64_t>(p->max_seqlen_q, 1) + 31) / 32);
    const int64_t ns = std::min<int64_t>(std::min<int64_t>((want + wgs - 1) / wgs, 8), iters);
    return (int)std::max<int64_t>(ns, 1);
}

// Splits of the fp32 matrix-core dQ over its key tiles, by the same rule
// (one workgroup per 128 query rows and head; the key tiles of a workgroup
// bounded by total_kv).
int f32_dq_splits(const mtlattn_problem* p) {
    if (p->dtype != MTLATTN_DTYPE_F32 || !f32_mfma_head_dim(p->head_dim) || force_generic() || p->total_q <= 0 ||
        p->total_kv <= 0)
        return 1;
    const int64_t tiles = std::max<int64_t>((p->total_q + 127) / 128, p->num_seqs);
    const int64_t wgs = tiles * p->num_heads_q, want = 2 * (int64_t)device_cus();
    if (wgs >= want) return 1;
    const int64_t ns = std::min<int64_t>(std::min<int64_t>((want + wgs - 1) / wgs, 8), (p->total_kv + 31) / 32);
    return (int)std::max<int64_t>(ns, 1);
}

// fp32 partial bytes after delta: dQ's, then (in the same space, after the
// dQ splits are summed) dK/dV's
size_t bwd_part_bytes(const mtlattn_problem* p) {
    const int64_t fq = f32_dq_part_floats(f32_dq_splits(p), p->total_q, p->num_heads_q, p->head_dim);
    const int64_t fk = f32_dkv_part_floats(f32_dkv_splits(p), p->total_kv, p->num_heads_kv, p->head_dim);
    return (size_t)std::max<int64_t>(fq, fk) * sizeof(float);
}

}  // namespace

size_t mtlattn_varlen_bwd_workspace_size(const mtlattn_problem* p) {
    if (check_problem(p) != MTLATTN_OK) return 0;
    const size_t part = bwd_part_bytes(p);
    if (part > 0) return bwd_part_offset(p) + part;
    return bwd_delta_bytes(p);
}

int mtlattn_bwd_preprocess(const mtlattn_problem* p, const void* out, int64_t out_row_stride, const void* dout,
                           int64_t dout_row_stride, float* delta, void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (p->total_q == 0) return ok();
    if (out == nullptr || dout == nullptr || delta == nullptr)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: null out/dout/delta pointer");
    const Geometry g = make_geo(p);
    return launch_status(launch_bwd_preprocess(p->dtype, g, out, out_row_stride, dout, dout_row_stride, delta,
                                               (hipStream_t)stream),
                         "delta preprocess");
}

namespace {

BwdArgs make_bwd(const mtlattn_problem* p, const void* q, int64_t qrs, const void* k, int64_t krs, const void* v,
                 int64_t vrs, const void* dout, int64_t dors, const float* lse, const float* delta) {
    BwdArgs a;
    a.geo = make_geo(p);
    a.q = q; a.q_rs = qrs; a.k = k; a.k_rs = krs; a.v = v; a.v_rs = vrs; a.dout = dout; a.do_rs = dors;
    a.lse = lse; a.delta = delta;
    a.dq = nullptr; a.dk = nullptr; a.dv = nullptr; a.out_f32 = 0;
    return a;
}

bool bwd_mfma_ok(const mtlattn_problem* p, const void* q, int64_t qrs, const void* k, int64_t krs, const void* v,
                 int64_t vrs, const void* dout, int64_t dors) {
    return is16(p->dtype) && mfma_head_dim(p->head_dim) && !force_generic() && aligned16(q, qrs, p->dtype) &&
           aligned16(k, krs, p->dtype) && aligned16(v, vrs, p->dtype) && aligned16(dout, dors, p->dtype) &&
           tile_stride_ok(qrs) && tile_stride_ok(krs) && tile_stride_ok(vrs) && tile_stride_ok(dors);
}

// fp32 inputs on the fp32 matrix-core kernels (16-byte aligned operand rows
// and output rows)
bool bwd_f32_ok(const mtlattn_problem* p, const void* q, int64_t qrs, const void* k, int64_t krs, const void* v,
                int64_t vrs, const void* dout, int64_t dors) {
    return p->dtype == MTLATTN_DTYPE_F32 && f32_mfma_head_dim(p->head_dim) && !force_generic() &&
           aligned16(q, qrs, p->dtype) && aligned16(k, krs, p->dtype) && aligned16(v, vrs, p->dtype) &&
           aligned16(dout, dors, p->dtype);
}

}  // namespace

int mtlattn_bwd_dq(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k,
                   int64_t k_row_stride, const void* v, int64_t v_row_stride, const void* dout,
                   int64_t dout_row_stride, const float* lse, const float* delta, void* dq, int32_t dq_dtype,
                   void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (dq_dtype != MTLATTN_DTYPE_F32 && dq_dtype != p->dtype)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: dq dtype must be fp32 or the input dtype");
    if (p->total_q == 0) return ok();
    if (q == nullptr || dout == nullptr || lse == nullptr || delta == nullptr || dq == nullptr ||
        (p->total_kv > 0 && (k == nullptr || v == nullptr)))
        return fail(MTLATTN_ERR_INVALID, "mtlattn: null pointer argument");
    BwdArgs a = make_bwd(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse, delta);
    a.dq = dq;
    a.out_f32 = dq_dtype == MTLATTN_DTYPE_F32 ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    if (bwd_mfma_ok(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride))
        return launch_status(launch_bwd_dq_mfma(p->dtype, a, st), "dQ");
    if (bwd_f32_ok(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride) &&
        ((uintptr_t)dq & 15u) == 0)
        return launch_status(launch_bwd_dq_f32mfma(a, st), "fp32 dQ");
    return launch_status(launch_bwd_dq_generic(p->dtype, a, st), "generic dQ");
}

namespace {

// mtlattn_bwd_dkv, with fp32 dK/dV partials for `splits` splits in `part`
// (fp32 matrix-core path only; splits == 1: none)
int bwd_dkv(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
            const void* v, int64_t v_row_stride, const void* dout, int64_t dout_row_stride, const float* lse,
            const float* delta, void* dk, void* dv, int32_t dkv_dtype, void* stream, float* part, int splits) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (dkv_dtype != MTLATTN_DTYPE_F32 && dkv_dtype != p->dtype)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: dk/dv dtype must be fp32 or the input dtype");
    if (p->total_kv == 0) return ok();
    if (k == nullptr || v == nullptr || dk == nullptr || dv == nullptr ||
        (p->total_q > 0 && (q == nullptr || dout == nullptr || lse == nullptr || delta == nullptr)))
        return fail(MTLATTN_ERR_INVALID, "mtlattn: null pointer argument");
    BwdArgs a = make_bwd(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse, delta);
    a.dk = dk;
    a.dv = dv;
    a.out_f32 = dkv_dtype == MTLATTN_DTYPE_F32 ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    if (bwd_mfma_ok(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride))
        return launch_status(launch_bwd_dkv_mfma(p->dtype, a, st), "dK/dV");
    if (bwd_f32_ok(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride) &&
        ((uintptr_t)dk & 15u) == 0 && ((uintptr_t)dv & 15u) == 0) {
        a.f32_part = part;
        a.f32_splits = part != nullptr ? splits : 1;
        return launch_status(launch_bwd_dkv_f32mfma(a, st), "fp32 dK/dV");
    }
    return launch_status(launch_bwd_dkv_generic(p->dtype, a, st), "generic dK/dV");
}

}  // namespace

int mtlattn_bwd_dkv(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k,
                    int64_t k_row_stride, const void* v, int64_t v_row_stride, const void* dout,
                    int64_t dout_row_stride, const float* lse, const float* delta, void* dk, void* dv,
                    int32_t dkv_dtype, void* stream) {
    return bwd_dkv(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse, delta, dk, dv,
                   dkv_dtype, stream, nullptr, 1);
}

int mtlattn_varlen_bwd(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k,
                       int64_t k_row_stride, const void* v, int64_t v_row_stride, const void* out,
                       int64_t out_row_stride, const void* dout, int64_t dout_row_stride, const float* lse,
                       void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    // delta is required; the fp32 dK/dV partials after it are used when the
    // workspace holds them (mtlattn_varlen_bwd_workspace_size), else dK/dV
    // runs unsplit
    const size_t need = bwd_delta_bytes(p);
    if (workspace_bytes < need || (need > 0 && workspace == nullptr))
        return fail(MTLATTN_ERR_WORKSPACE, "mtlattn: backward workspace too small (%zu < %zu bytes)",
                    workspace_bytes, need);
    float* delta = (float*)workspace;
    int splits = f32_dkv_splits(p), dq_splits = f32_dq_splits(p);
    float* part = nullptr;
    const size_t part_bytes = bwd_part_bytes(p);
    if (part_bytes > 0 && workspace != nullptr && ((uintptr_t)workspace & 15u) == 0 &&
        workspace_bytes >= bwd_part_offset(p) + part_bytes)
        part = (float*)((char*)workspace + bwd_part_offset(p));
    else
        splits = dq_splits = 1;
    // Head dims 64 and 128 on the matrix-core path: the dQ kernel computes
    // delta from O and dO itself (bitwise equal to the preprocess) and leaves
    // it in the workspace for dK/dV, which saves the preprocess's pass over dO.
    const bool fuse_delta = p->total_q > 0 && (p->head_dim == 64 || p->head_dim == 128) &&
                            bwd_mfma_ok(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout,
                                        dout_row_stride) &&
                            ((uintptr_t)out & 15u) == 0 && out_row_stride % 8 == 0;
    const bool fuse_delta_f32 = p->total_q > 0 && out != nullptr && dout != nullptr &&
                                bwd_f32_ok(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout,
                                           dout_row_stride) &&
                                aligned16(out, out_row_stride, p->dtype) && ((uintptr_t)dq & 15u) == 0;
    if (fuse_delta) {
        if (q == nullptr || out == nullptr || dout == nullptr || lse == nullptr || dq == nullptr ||
            (p->total_kv > 0 && (k == nullptr || v == nullptr)))
            return fail(MTLATTN_ERR_INVALID, "mtlattn: null pointer argument");
        BwdArgs a = make_bwd(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse, delta);
        a.dq = dq;
        a.o = out;
        a.o_rs = out_row_stride;
        a.delta_out = delta;
        rc = launch_status(launch_bwd_dq_mfma(p->dtype, a, (hipStream_t)stream), "dQ");
        if (rc != MTLATTN_OK) return rc;
    } else if (fuse_delta_f32) {
        // fp32 matrix cores: the dQ kernel computes delta from O and dO (equal
        // to the preprocess up to fp32 rounding) and leaves it in the workspace
        if (q == nullptr || lse == nullptr || dq == nullptr || (p->total_kv > 0 && (k == nullptr || v == nullptr)))
            return fail(MTLATTN_ERR_INVALID, "mtlattn: null pointer argument");
        BwdArgs a = make_bwd(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse, delta);
        a.dq = dq;
        a.out_f32 = 1;
        a.o = out;
        a.o_rs = out_row_stride;
        a.delta_out = delta;
        a.f32_part = part;
        a.f32_splits = part != nullptr ? dq_splits : 1;
        rc = launch_status(launch_bwd_dq_f32mfma(a, (hipStream_t)stream), "fp32 dQ");
        if (rc != MTLATTN_OK) return rc;
    } else if (p->total_q > 0) {
        rc = mtlattn_bwd_preprocess(p, out, out_row_stride, dout, dout_row_stride, delta, stream);
        if (rc != MTLATTN_OK) return rc;
        rc = mtlattn_bwd_dq(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse,
                            delta, dq, p->dtype, stream);
        if (rc != MTLATTN_OK) return rc;
    }
    rc = bwd_dkv(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, dout, dout_row_stride, lse, delta, dk, dv,
                 p->dtype, stream, part, splits);
    if (rc != MTLATTN_OK) return rc;
    // Rows outside every sequence take no part in the forward: zero gradient.
    hipStream_t st = (hipStream_t)stream;
    const int64_t es = elem_size(p->dtype);
    const int64_t qrow = (int64_t)p->num_heads_q * p->head_dim * es, krow = (int64_t)p->num_heads_kv * p->head_dim * es;
    const ZeroFill fills[3] = {{dq, qrow, p->total_q, p->cu_seqlens_q},
                               {dk, krow, p->total_kv, p->cu_seqlens_kv},
                               {dv, krow, p->total_kv, p->cu_seqlens_kv}};
    return launch_status(launch_zero_outside(fills, 3, p->num_seqs, st), "gradient tail fill");
}

size_t mtlattn_attn_splitkv_workspace_size(const mtlattn_problem* p, int32_t num_splits) {
    if (check_problem(p) != MTLATTN_OK || num_splits < 1) return 0;
    return splitkv_bytes(p, num_splits, 0);
}

int mtlattn_attn_splitkv(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k,
                         int64_t k_row_stride, const void* v, int64_t v_row_stride, void* out, float* lse,
                         int32_t num_splits, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (!is16(p->dtype)) return fail(MTLATTN_ERR_UNSUPPORTED, "splitkv: half/bf16");
    if (!decode_head_dim(p->head_dim)) return fail(MTLATTN_ERR_UNSUPPORTED, "splitkv: D in {64,128}");
    if (p->max_seqlen_q < 1 || p->max_seqlen_q > 16)
        return fail(MTLATTN_ERR_UNSUPPORTED, "splitkv: max_seqlen_q must be in [1, 16]");
    if (num_splits < 1 || num_splits > 4096) return fail(MTLATTN_ERR_INVALID, "splitkv: num_splits in [1, 4096]");
    if (p->total_q == 0) return ok();
    if (q == nullptr || out == nullptr || (p->total_kv > 0 && (k == nullptr || v == nullptr)))
        return fail(MTLATTN_ERR_INVALID, "mtlattn: null q/k/v/out pointer");
    if (!aligned16(q, q_row_stride, p->dtype) || !aligned16(k, k_row_stride, p->dtype) ||
        !aligned16(v, v_row_stride, p->dtype) || ((uintptr_t)out & 15u) != 0)
        return fail(MTLATTN_ERR_UNSUPPORTED, "splitkv: q/k/v rows must be 16-byte aligned");
    return run_splitkv(p, q, q_row_stride, k, k_row_stride, v, v_row_stride, out, lse, num_splits, 0, workspace,
                       workspace_bytes, (hipStream_t)stream);
}

size_t mtlattn_paged_decode_workspace_size(const mtlattn_problem* p, int64_t max_seqlen_kv) {
    if (check_problem(p) != MTLATTN_OK || !splitkv_supported(p)) return 0;
    const DecodePlan plan = paged_plan(p, max_seqlen_kv);
    return splitkv_bytes(p, plan.ns, plan.chunk);
}

int mtlattn_paged_decode(const mtlattn_problem* p, const void* q, int64_t q_row_stride, const void* k_cache,
                         int64_t k_row_stride, const void* v_cache, int64_t v_row_stride, int32_t page_size,
                         int64_t num_pages, const int32_t* block_table, int64_t block_table_stride,
                         int64_t max_seqlen_kv, void* out, float* lse, void* workspace, size_t workspace_bytes,
                         void* stream) {
    int rc = check_problem(p);
    if (rc != MTLATTN_OK) return rc;
    if (!is16(p->dtype)) return fail(MTLATTN_ERR_UNSUPPORTED, "paged_decode: half/bf16");
    if (!decode_head_dim(p->head_dim)) return fail(MTLATTN_ERR_UNSUPPORTED, "paged_decode: D in {64,128}");
    if (p->max_seqlen_q < 1 || p->max_seqlen_q > 16)
        return fail(MTLATTN_ERR_UNSUPPORTED, "paged_decode: max_seqlen_q must be in [1, 16]");
    if (page_size < 16 || page_size % 16 != 0)
        return fail(MTLATTN_ERR_INVALID, "paged_decode: page_size must be a positive multiple of 16 (got %d)",
                    page_size);
    if (num_pages < 1 || num_pages > 0x7fffffffLL || num_pages * (int64_t)page_size > 0x7fffffffLL)
        return fail(MTLATTN_ERR_INVALID, "paged_decode: num_pages * page_size must be in [1, 2^31)");
    if (block_table_stride < 1) return fail(MTLATTN_ERR_INVALID, "paged_decode: block_table_stride must be >= 1");
    if (max_seqlen_kv < 0) return fail(MTLATTN_ERR_INVALID, "paged_decode: negative max_seqlen_kv");
    if (p->total_q == 0) return ok();
    if (q == nullptr || out == nullptr || k_cache == nullptr || v_cache == nullptr || block_table == nullptr)
        return fail(MTLATTN_ERR_INVALID, "paged_decode: null q/k_cache/v_cache/block_table/out pointer");
    if (!aligned16(q, q_row_stride, p->dtype) || !aligned16(k_cache, k_row_stride, p->dtype) ||
        !aligned16(v_cache, v_row_stride, p->dtype) || ((uintptr_t)out & 15u) != 0)
        return fail(MTLATTN_ERR_UNSUPPORTED, "paged_decode: q/k/v rows must be 16-byte aligned");
    const DecodePlan plan = paged_plan(p, max_seqlen_kv);
    const PagedKV pk{block_table, block_table_stride, num_pages, page_size};
    return run_splitkv(p, q, q_row_stride, k_cache, k_row_stride, v_cache, v_row_stride, out, lse, plan.ns,
                       plan.chunk, workspace, workspace_bytes, (hipStream_t)stream, &pk);
}


int mtlattn_pack_padded(int32_t dtype, int32_t B, int32_t N, int32_t H, int32_t D, const void* src, int64_t sb,
                        int64_t sh, int64_t sn, const int32_t* lens, int32_t* cu_out, void* dst, void* stream) {
    if (dtype != MTLATTN_DTYPE_F32 && dtype != MTLATTN_DTYPE_F16 && dtype != MTLATTN_DTYPE_BF16)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: unsupported dtype %d", dtype);
    if (B < 0 || N < 0 || H <= 0 || D <= 0 || sb < 0 || sh < 0 || sn < 0)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: pack_padded: bad shape or strides");
    if (B == 0) return MTLATTN_OK;
    if (src == nullptr || lens == nullptr || cu_out == nullptr || dst == nullptr)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: pack_padded: null pointer");
    const int es = dtype == MTLATTN_DTYPE_F32 ? 4 : 2;
    return launch_status(launch_pad_pack(es, B, N, H, D, src, sb, sh, sn, lens, cu_out, dst, (hipStream_t)stream),
                         "pack_padded");
}

int mtlattn_unpack_padded(int32_t dtype, int32_t B, int32_t N, int32_t H, int32_t D, const void* src,
                          const int32_t* lens, const int32_t* cu, void* dst, int64_t sb, int64_t sh, int64_t sn,
                          void* stream) {
    if (dtype != MTLATTN_DTYPE_F32 && dtype != MTLATTN_DTYPE_F16 && dtype != MTLATTN_DTYPE_BF16)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: unsupported dtype %d", dtype);
    if (B < 0 || N < 0 || H <= 0 || D <= 0 || sb < 0 || sh < 0 || sn < 0)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: unpack_padded: bad shape or strides");
    if (B == 0) return MTLATTN_OK;
    if (src == nullptr || lens == nullptr || cu == nullptr || dst == nullptr)
        return fail(MTLATTN_ERR_INVALID, "mtlattn: unpack_padded: null pointer");
    const int es = dtype == MTLATTN_DTYPE_F32 ? 4 : 2;
    return launch_status(launch_pad_unpack(es, B, N, H, D, src, lens, cu, dst, sb, sh, sn, (hipStream_t)stream),
                         "unpack_padded");
}

}  // extern "C"
