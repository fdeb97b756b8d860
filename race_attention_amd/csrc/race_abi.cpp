// extern "C" entry points of librace_amd.so (declared in include/race_attention.h):
// argument validation, kernel-variant selection, workspace layout and launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/race_attention.h"
#include "race_decode.h"
#include "race_launch.h"
#include "race_noncausal.h"
#include "race_softhash.h"

using namespace race;

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_check(hipError_t e, const char *what)
{
    if (e != hipSuccess)
        return fail(RACE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return RACE_OK;
}

#define RACE_TRY(expr)            \
    do {                          \
        const int _rc = (expr);   \
        if (_rc != RACE_OK)       \
            return _rc;           \
    } while (0)

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t rup(int64_t a, int64_t b) { return cdiv(a, b) * b; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Tokens per workgroup: `req` rounded to the sub-chunk, or (req = 0) about `target`
// workgroups per launch with at least 4 sub-chunks each.
int64_t resolve_block(int64_t T, int64_t streams, int C, int64_t req, int64_t target)
{
    int64_t cb;
    if (req > 0) {
        cb = rup(req, C);
    } else {
        const int64_t nb = std::max<int64_t>(1, cdiv(target, std::max<int64_t>(1, streams)));
        cb = std::max<int64_t>(4 * C, rup(cdiv(T, nb), C));
    }
    return std::min(cb, rup(T, C));
}

// ------------------------------------------------------------------ geometry
struct Geo {
    int ST, DP, C, n_st, S_pad;
    // fused layer with n_st > 1: the kernels that write outputs run one launch per bucket tile,
    // each adding the earlier tiles' fp32 sum in its store (no partial-sum reduction pass)
    bool seq = false;
    int64_t CB, NB;
    int64_t Z;               // kv streams
    size_t state_elems_B;    // per workspace array
    size_t state_elems_A;
};

void fill_ws_sizes(Geo &g)
{
    g.state_elems_B = (size_t)g.Z * (g.NB + 1) * g.S_pad * g.DP;
    g.state_elems_A = (size_t)g.Z * (g.NB + 1) * g.S_pad;
}

int op_geometry(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block, Geo &g)
{
    if (N <= 0 || T <= 0 || S <= 0 || D <= 0)
        return fail(RACE_ERR_INVALID, "race_op: N, T, S, D must be positive (got %lld, %lld, %lld, %lld)",
                    (long long)N, (long long)T, (long long)S, (long long)D);
    if (N > 65535)
        return fail(RACE_ERR_UNSUPPORTED, "race_op: N = %lld streams exceeds 65535", (long long)N);
    if (T > (int64_t)1 << 30 || S > 4096)
        return fail(RACE_ERR_UNSUPPORTED, "race_op: T <= 2^30 and S <= 4096 required");
    if (D > 256)
        return fail(RACE_ERR_UNSUPPORTED, "race_op: head dim D = %lld > 256 is not compiled", (long long)D);
    g.DP = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
    // bucket tiles of at most 64 (the largest measured fastest at D = 32 and 64 for S = 64 and 128;
    // 128-wide tiles at D = 32 are slower)
    const int st_max = std::min(64, 4096 / g.DP);
    g.ST = st_max;
    for (int st : {16, 32, 64, 128})
        if (st <= st_max && st >= S) {
            g.ST = st;
            break;
        }
    if (!op_variant_exists(g.ST, g.DP))
        return fail(RACE_ERR_UNSUPPORTED, "race_op: no kernel for tile (%d, %d)", g.ST, g.DP);
    g.C = OP_C;
    g.n_st = (int)cdiv(S, g.ST);
    g.S_pad = g.n_st * g.ST;
    g.Z = N;
    g.CB = resolve_block(T, N * g.n_st, g.C, block, 2048);
    g.NB = cdiv(T, g.CB);
    fill_ws_sizes(g);
    return RACE_OK;
}

int qkv_geometry(const race_qkv_shape *sh, Geo &g)
{
    if (!sh)
        return fail(RACE_ERR_INVALID, "race_qkv: null shape");
    if (sh->B <= 0 || sh->Hq <= 0 || sh->Hkv <= 0 || sh->T <= 0 || sh->L <= 0)
        return fail(RACE_ERR_INVALID, "race_qkv: B, Hq, Hkv, T, L must be positive");
    if (sh->T > (1 << 30))  // token indices and sub-chunk look-ahead stay in 32-bit range
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: T = %d tokens, at most 2^30 are supported", sh->T);
    if (sh->Hq % sh->Hkv)
        return fail(RACE_ERR_INVALID, "race_qkv: Hq = %d is not a multiple of Hkv = %d", sh->Hq, sh->Hkv);
    if (sh->K < 1 || sh->K > 4)
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: K = %d bits, the fused path supports 1..4", sh->K);
    if (sh->D != 64 && sh->D != 128)
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: head dim %d, the fused path supports 64 and 128", sh->D);
    if (!(sh->eps > 0.0f) || !(sh->scale > 0.0f))
        return fail(RACE_ERR_INVALID, "race_qkv: eps and scale must be positive");
    if ((int64_t)sh->Hq * sh->D > (1 << 20))
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: Hq*D = %lld too large", (long long)sh->Hq * sh->D);
    const int R = 1 << sh->K;
    const int64_t S = (int64_t)sh->L * R;
    if (S > 4096)
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: S = %lld buckets > 4096", (long long)S);
    g.DP = sh->D;
    const int st_max = g.DP == 64 ? 128 : 64;
    g.ST = st_max;
    for (int st : {32, 64, 128})
        if (st <= st_max && st >= S) {
            g.ST = st;
            break;
        }
    if (!qkv_variant_exists(g.ST, g.DP))
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: no kernel for tile (%d, %d)", g.ST, g.DP);
    g.C = QKV_C;
    g.n_st = (int)cdiv(S, g.ST);
    g.S_pad = g.n_st * g.ST;
    g.Z = (int64_t)sh->B * sh->Hkv;
    if (g.Z > 65535)
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv: B*Hkv = %lld exceeds 65535", (long long)g.Z);
    // ~768 workgroups per launch: whole rounds on MI355X's 256 CUs both for the backward kernels
    // (one workgroup per CU: 3 rounds) and for the bf16 readout (three per CU: 1 round), with
    // few enough blocks to keep the block-state traffic and per-block set-up low
    g.seq = g.n_st > 1 && fused_variant_exists(g.ST, g.DP, sh->K);
    g.CB = resolve_block(sh->T, g.Z * (g.seq ? 1 : g.n_st), g.C, sh->block, 768);
    g.NB = cdiv(sh->T, g.CB);
    fill_ws_sizes(g);
    return RACE_OK;
}

// Carve a workspace into 256-byte aligned pieces.
struct Carver {
    char *base;
    size_t used = 0, cap;
    Carver(void *p, size_t c) : base((char *)p), cap(c) {}
    float *take(size_t elems)
    {
        float *p = (float *)(base ? base + used : nullptr);
        used += align256(elems * sizeof(float));
        return p;
    }
};

int check_view(const race_tensor &t, const char *name, bool bf16_vec)
{
    if (!t.data)
        return fail(RACE_ERR_INVALID, "%s: null data pointer", name);
    if (t.stride_b < 0 || t.stride_h < 0 || t.stride_t < 0)
        return fail(RACE_ERR_INVALID, "%s: negative stride", name);
    if (bf16_vec) {
        if (((uintptr_t)t.data & 15) || (t.stride_b & 7) || (t.stride_h & 7) || (t.stride_t & 7))
            return fail(RACE_ERR_INVALID,
                        "%s: bf16 rows must be 16-byte aligned (pointer %% 16 == 0, strides %% 8 == 0)", name);
        // the row movers form in-sub-chunk row offsets with 24-bit multiplies (row < 32)
        if (t.stride_t >= ((int64_t)1 << 24))
            return fail(RACE_ERR_UNSUPPORTED, "%s: token stride %lld too large (at most 2^24 - 1 elements)", name,
                        (long long)t.stride_t);
    }
    return RACE_OK;
}

View to_view(const race_tensor &t) { return View{t.data, t.stride_b, t.stride_h, t.stride_t}; }
OutView to_out(const race_tensor &t, int f32) { return OutView{t.data, t.stride_b, t.stride_h, t.stride_t, 0, f32}; }

hipStream_t hs(race_stream s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ kernel timing
// When enabled, every launch is bracketed by a pair of HIP events recorded on the
// launch stream; race_profile_read resolves them into per-kernel totals.
struct EventPair {
    hipEvent_t a, b;
};
struct Profiler {
    std::mutex mu;
    bool on = false;
    std::vector<EventPair> pending[RACE_PROF_KERNELS];
    double total_ms[RACE_PROF_KERNELS] = {};
    int64_t count[RACE_PROF_KERNELS] = {};
};
Profiler &prof()
{
    static Profiler p;
    return p;
}

struct ProfScope {
    int id;
    hipStream_t s;
    EventPair ev{nullptr, nullptr};
    ProfScope(int id_, hipStream_t s_) : id(id_), s(s_)
    {
        Profiler &p = prof();
        std::lock_guard<std::mutex> g(p.mu);
        if (!p.on)
            return;
        if (hipEventCreate(&ev.a) != hipSuccess || hipEventCreate(&ev.b) != hipSuccess) {
            ev = EventPair{nullptr, nullptr};
            return;
        }
        (void)hipEventRecord(ev.a, s);
    }
    ~ProfScope()
    {
        if (!ev.a)
            return;
        (void)hipEventRecord(ev.b, s);
        Profiler &p = prof();
        std::lock_guard<std::mutex> g(p.mu);
        p.pending[id].push_back(ev);
    }
};

hipError_t prof_block_scan(float *wsB, int64_t elemsB, float *wsA, int64_t elemsA, int NB, int Z, int rev,
                           hipStream_t s, float *loB = nullptr, float *loA = nullptr)
{
    ProfScope ps(RACE_PROF_BLOCK_SCAN, s);
    return launch_block_scan(wsB, elemsB, wsA, elemsA, NB, Z, rev, s, loB, loA);
}
hipError_t prof_reduce(const float *part, int n_st, int64_t tile, const OutView &out, int B, int H, int T, int D,
                       hipStream_t s)
{
    ProfScope ps(RACE_PROF_REDUCE, s);
    return launch_reduce_partials(part, n_st, tile, out, B, H, T, D, s);
}
hipError_t prof_softhash(const SoftHashParams &P, int bf16, int bwd, hipStream_t s)
{
    ProfScope ps(bwd ? RACE_PROF_SOFTHASH_BWD : RACE_PROF_SOFTHASH_FWD, s);
    return launch_softhash(P, bf16, bwd, s);
}
hipError_t prof_decode(const DecodeParams &P, int bf16, hipStream_t s)
{
    ProfScope ps(RACE_PROF_DECODE, s);
    return launch_decode(P, bf16, s);
}

}  // namespace

extern "C" {

int race_abi_version(void) { return RACE_ABI_VERSION; }

const char *race_last_error(void) { return g_err.c_str(); }

// ============================================================================ soft-hash
static int hash_common(const race_hash_shape *sh, const race_tensor &x, int x_dtype,
                       const float *planes_T, SoftHashParams &P)
{
    if (!sh)
        return fail(RACE_ERR_INVALID, "race_soft_hash: null shape");
    if (sh->B <= 0 || sh->H <= 0 || sh->T <= 0 || sh->D <= 0 || sh->L <= 0 || sh->M <= 0)
        return fail(RACE_ERR_INVALID, "race_soft_hash: B, H, T, D, L, M must be positive");
    if (sh->T > (1 << 30))  // token indices stay in 32-bit range
        return fail(RACE_ERR_UNSUPPORTED, "race_soft_hash: T = %d tokens, at most 2^30 are supported", sh->T);
    if (sh->K < 1 || sh->K > 8)
        return fail(RACE_ERR_UNSUPPORTED, "race_soft_hash: K = %d, supported 1..8", sh->K);
    if (x_dtype != RACE_F32 && x_dtype != RACE_BF16)
        return fail(RACE_ERR_INVALID, "race_soft_hash: dtype must be RACE_F32 or RACE_BF16");
    if (sh->D > 256 || (int64_t)sh->D * sh->L * sh->K > 16384)
        return fail(RACE_ERR_UNSUPPORTED, "race_soft_hash: D <= 256 and D*L*K <= 16384 required");
    if (!(sh->scale > 0.0f))
        return fail(RACE_ERR_INVALID, "race_soft_hash: scale must be positive");
    if (!planes_T)
        return fail(RACE_ERR_INVALID, "race_soft_hash: null planes");
    RACE_TRY(check_view(x, "race_soft_hash: x", false));
    std::memset(&P, 0, sizeof(P));
    P.x = to_view(x);
    P.planes = planes_T;
    P.B = sh->B;
    P.H = sh->H;
    P.T = sh->T;
    P.D = sh->D;
    P.L = sh->L;
    P.K = sh->K;
    P.LK = sh->L * sh->K;
    P.M = sh->M;
    P.unshared = sh->unshared ? 1 : 0;
    P.plane_stride = (int64_t)sh->D * P.LK;
    P.round_planes = x_dtype == RACE_BF16;
    P.scale = sh->scale;
    P.inv_scale = 1.0f / sh->scale;
    return hip_check(softhash_prepare(P.D, P.LK), "race_soft_hash: set shared memory");
}

int race_soft_hash_fwd(const race_hash_shape *sh, race_tensor x, int x_dtype, const float *planes_T,
                       float *probs, race_stream stream)
{
    SoftHashParams P;
    RACE_TRY(hash_common(sh, x, x_dtype, planes_T, P));
    if (!probs)
        return fail(RACE_ERR_INVALID, "race_soft_hash_fwd: null probs");
    P.probs = probs;
    return hip_check(prof_softhash(P, x_dtype == RACE_BF16, 0, hs(stream)), "race_soft_hash_fwd");
}

int race_soft_hash_bwd(const race_hash_shape *sh, race_tensor x, int x_dtype, const float *planes_T,
                       const float *gprobs, race_tensor dx, race_stream stream)
{
    SoftHashParams P;
    RACE_TRY(hash_common(sh, x, x_dtype, planes_T, P));
    if (!gprobs)
        return fail(RACE_ERR_INVALID, "race_soft_hash_bwd: null gprobs");
    RACE_TRY(check_view(dx, "race_soft_hash_bwd: dx", false));
    P.gprobs = gprobs;
    P.dx = to_view(dx);
    return hip_check(prof_softhash(P, x_dtype == RACE_BF16, 1, hs(stream)), "race_soft_hash_bwd");
}

int race_soft_hash_bwd_partials(const race_hash_shape *sh)
{
    if (!sh || sh->T <= 0 || sh->B <= 0 || sh->H <= 0)
        return 0;
    const bool mf = softhash_mfma_ok(sh->D, sh->L, sh->K, sh->M, 1);
    return softhash_grid_x(sh->T, sh->B, sh->H, mf) * sh->B * sh->H;
}

int race_soft_hash_bwd_scale(const race_hash_shape *sh, race_tensor x, int x_dtype, const float *planes_T,
                             const float *gprobs, race_tensor dx, float *gscale_partials, race_stream stream)
{
    SoftHashParams P;
    RACE_TRY(hash_common(sh, x, x_dtype, planes_T, P));
    if (!gprobs || !gscale_partials)
        return fail(RACE_ERR_INVALID, "race_soft_hash_bwd_scale: null gprobs or partials");
    RACE_TRY(check_view(dx, "race_soft_hash_bwd_scale: dx", false));
    P.gprobs = gprobs;
    P.dx = to_view(dx);
    P.gscale = gscale_partials;
    return hip_check(prof_softhash(P, x_dtype == RACE_BF16, 1, hs(stream)), "race_soft_hash_bwd_scale");
}

// The same two calls with the scale read on the device (BatchedACE's learnable temperature,
// scaling/benchmark_time.py:104,111, which the reference keeps as a device tensor): sh->scale is
// not used. scale_dev must point to one fp32 > 0 that stays unchanged until the kernels have run.
int race_soft_hash_fwd_dscale(const race_hash_shape *sh, race_tensor x, int x_dtype, const float *planes_T,
                              const float *scale_dev, float *probs, race_stream stream)
{
    if (!scale_dev)
        return fail(RACE_ERR_INVALID, "race_soft_hash_fwd_dscale: null scale");
    race_hash_shape s1 = sh ? *sh : race_hash_shape{};
    s1.scale = 1.0f;  // checked on the device side by its producer (a clamp), not here
    SoftHashParams P;
    RACE_TRY(hash_common(sh ? &s1 : nullptr, x, x_dtype, planes_T, P));
    if (!probs)
        return fail(RACE_ERR_INVALID, "race_soft_hash_fwd_dscale: null probs");
    P.probs = probs;
    P.scale_dev = scale_dev;
    return hip_check(prof_softhash(P, x_dtype == RACE_BF16, 0, hs(stream)), "race_soft_hash_fwd_dscale");
}

int race_soft_hash_bwd_dscale(const race_hash_shape *sh, race_tensor x, int x_dtype, const float *planes_T,
                              const float *scale_dev, const float *gprobs, race_tensor dx, float *gscale_partials,
                              float *dscale, race_stream stream)
{
    if (!scale_dev)
        return fail(RACE_ERR_INVALID, "race_soft_hash_bwd_dscale: null scale");
    race_hash_shape s1 = sh ? *sh : race_hash_shape{};
    s1.scale = 1.0f;
    SoftHashParams P;
    RACE_TRY(hash_common(sh ? &s1 : nullptr, x, x_dtype, planes_T, P));
    if (!gprobs || !gscale_partials || !dscale)
        return fail(RACE_ERR_INVALID, "race_soft_hash_bwd_dscale: null gprobs, partials or dscale");
    RACE_TRY(check_view(dx, "race_soft_hash_bwd_dscale: dx", false));
    P.gprobs = gprobs;
    P.dx = to_view(dx);
    P.gscale = gscale_partials;
    P.scale_dev = scale_dev;
    hipStream_t st = hs(stream);
    RACE_TRY(hip_check(prof_softhash(P, x_dtype == RACE_BF16, 1, st), "race_soft_hash_bwd_dscale"));
    return hip_check(launch_scale_grad(gscale_partials, race_soft_hash_bwd_partials(&s1), scale_dev, dscale, st),
                     "race_soft_hash_bwd_dscale: scale gradient");
}

// ============================================================================ op-level scan
static size_t op_bytes(const Geo &g, int64_t T, int64_t D, int backward)
{
    size_t b = align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4);
    if (backward)  // the backward suffix states as double-floats (hi and lo arrays)
        b += 2 * (align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4));
    if (g.n_st > 1)
        b += align256((size_t)g.n_st * g.Z * T * D * 4);
    return b;
}

size_t race_op_workspace_bytes(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block, int backward)
{
    Geo g;
    if (op_geometry(N, T, S, D, block, g) != RACE_OK)
        return 0;
    return op_bytes(g, T, D, backward);
}

static ScanParams op_params(const Geo &g, int64_t T, int64_t S, int64_t D, float eps)
{
    ScanParams P;
    std::memset(&P, 0, sizeof(P));
    P.T = (int)T;
    P.S = (int)S;
    P.D = (int)D;
    P.L = 1;
    P.K = 0;
    P.R = 1;
    P.G = 1;
    P.Hkv = 1;
    P.CB = (int)g.CB;
    P.NB = (int)g.NB;
    P.n_st = g.n_st;
    P.S_pad = g.S_pad;
    P.DPw = g.DP;
    P.eps = eps;
    P.scale = 1.0f;
    P.inv_scale = 1.0f;
    P.v = View{nullptr, T * D, 0, D};  // contiguous [N][T][D] values / grads
    P.go = P.v;
    P.zH = 1;
    return P;
}

static int run_scan_op(ScanKernel k, const Geo &g, const ScanParams &P, hipStream_t s)
{
    ProfScope ps(RACE_PROF_OP_FWD_TOTALS + (int)k, s);
    const dim3 grid((unsigned)g.NB, (unsigned)g.n_st, (unsigned)g.Z);
    return hip_check(launch_scan_op(k, g.ST, g.DP, P, grid, s), "race_op kernel launch");
}

static int op_check(const float *pK, const float *pQ, const float *V, float eps, void *ws,
                    size_t ws_bytes, size_t need, const char *who)
{
    if (!pK || !pQ || !V)
        return fail(RACE_ERR_INVALID, "%s: null input pointer", who);
    if (!(eps >= 0.0f))
        return fail(RACE_ERR_INVALID, "%s: eps must be >= 0", who);
    if (!ws || ws_bytes < need)
        return fail(RACE_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", who, need, ws ? ws_bytes : 0);
    return RACE_OK;
}

// A kept-state buffer: present, 256-byte aligned and at least race_op_state_bytes of this call's
// own geometry (a buffer sized for another shape or block would be overrun by the kernels).
static int kept_state_check(const void *state, size_t state_bytes, int64_t N, int64_t T, int64_t S, int64_t D,
                            int64_t block, const char *who)
{
    if (!state || (reinterpret_cast<uintptr_t>(state) & 255))
        return fail(RACE_ERR_INVALID, "%s: state must be a 256-byte aligned buffer", who);
    Geo g;
    RACE_TRY(op_geometry(N, T, S, D, block, g));
    const size_t need = align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4);
    if (state_bytes < need)
        return fail(RACE_ERR_WORKSPACE, "%s: state of %zu bytes needed for this shape and block, got %zu", who, need,
                    state_bytes);
    return RACE_OK;
}

// forward block states [wsB | wsA] inside a caller's state buffer (race_op_state_bytes)
static void state_views(const Geo &g, const float *state, float *&wsB, float *&wsA)
{
    wsB = const_cast<float *>(state);
    wsA = wsB + align256(g.state_elems_B * 4) / 4;
}

static int op_fwd_impl(const float *pK, const float *pQ, const float *V, float *out, int64_t N, int64_t T,
                       int64_t S, int64_t D, float eps, int64_t block, void *workspace, size_t workspace_bytes,
                       race_stream stream, int linear, const char *who, float *state = nullptr)
{
    Geo g;
    RACE_TRY(op_geometry(N, T, S, D, block, g));
    RACE_TRY(op_check(pK, pQ, V, eps, workspace, workspace_bytes, op_bytes(g, T, D, 0), who));
    if (!out)
        return fail(RACE_ERR_INVALID, "%s: null out", who);
    Carver cv(workspace, workspace_bytes);
    ScanParams P = op_params(g, T, S, D, eps);
    P.linear = linear;
    P.pK = pK;
    P.pQ = pQ;
    P.V = V;
    P.wsB = cv.take(g.state_elems_B);
    P.wsA = cv.take(g.state_elems_A);
    if (state)
        state_views(g, state, P.wsB, P.wsA);
    float *part = g.n_st > 1 ? cv.take((size_t)g.n_st * N * T * D) : nullptr;
    P.out = part ? OutView{part, T * D, 0, D, N * T * D, 1} : OutView{out, T * D, 0, D, 0, 1};
    const hipStream_t s = hs(stream);
    RACE_TRY(run_scan_op(K_FWD_TOTALS, g, P, s));
    RACE_TRY(hip_check(prof_block_scan(P.wsB, (int64_t)g.S_pad * g.DP, P.wsA, g.S_pad, (int)g.NB, (int)g.Z, 0, s), "block scan"));
    RACE_TRY(run_scan_op(K_FWD_READOUT, g, P, s));
    if (part)
        RACE_TRY(hip_check(prof_reduce(part, g.n_st, N * T * D, OutView{out, T * D, 0, D, 0, 1},
                                                  (int)N, 1, (int)T, (int)D, s), "reduce partials"));
    return RACE_OK;
}

int race_op_fwd(const float *pK, const float *pQ, const float *V, float *out, int64_t N, int64_t T,
                int64_t S, int64_t D, float eps, int64_t block, void *workspace, size_t workspace_bytes,
                race_stream stream)
{
    return op_fwd_impl(pK, pQ, V, out, N, T, S, D, eps, block, workspace, workspace_bytes, stream, 0,
                       "race_op_fwd");
}

static int op_bwd_impl(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK, float *gpQ,
                       float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps, int64_t block,
                       void *workspace, size_t workspace_bytes, race_stream stream, int linear, const char *who,
                       const float *state = nullptr)
{
    Geo g;
    RACE_TRY(op_geometry(N, T, S, D, block, g));
    RACE_TRY(op_check(pK, pQ, V, eps, workspace, workspace_bytes, op_bytes(g, T, D, 1), who));
    if (!gO || !gpK || !gpQ || !gV)
        return fail(RACE_ERR_INVALID, "%s: null gradient pointer", who);
    Carver cv(workspace, workspace_bytes);
    ScanParams P = op_params(g, T, S, D, eps);
    P.linear = linear;
    P.pK = pK;
    P.pQ = pQ;
    P.V = V;
    P.gO = gO;
    P.gpK = gpK;
    P.gpQ = gpQ;
    P.wsB = cv.take(g.state_elems_B);
    P.wsA = cv.take(g.state_elems_A);
    P.ws2B = cv.take(g.state_elems_B);
    P.ws2A = cv.take(g.state_elems_A);
    P.ws3B = cv.take(g.state_elems_B);
    P.ws3A = cv.take(g.state_elems_A);
    float *part = g.n_st > 1 ? cv.take((size_t)g.n_st * N * T * D) : nullptr;
    P.dv = part ? OutView{part, T * D, 0, D, N * T * D, 1} : OutView{gV, T * D, 0, D, 0, 1};
    const hipStream_t s = hs(stream);
    if (state) {  // forward block states kept by race_op_fwd_keep (only read from here on)
        state_views(g, state, P.wsB, P.wsA);
    } else {  // recomputed: nothing is saved between calls
        RACE_TRY(run_scan_op(K_FWD_TOTALS, g, P, s));
        RACE_TRY(hip_check(prof_block_scan(P.wsB, (int64_t)g.S_pad * g.DP, P.wsA, g.S_pad, (int)g.NB, (int)g.Z, 0, s),
                           "block scan"));
    }
    RACE_TRY(run_scan_op(K_BWD_TOTALS, g, P, s));
    RACE_TRY(hip_check(prof_block_scan(P.ws2B, (int64_t)g.S_pad * g.DP, P.ws2A, g.S_pad, (int)g.NB, (int)g.Z, 1, s,
                                       P.ws3B, P.ws3A),
                       "block scan"));
    RACE_TRY(run_scan_op(K_BWD_MAIN, g, P, s));
    if (part)
        RACE_TRY(hip_check(prof_reduce(part, g.n_st, N * T * D, OutView{gV, T * D, 0, D, 0, 1},
                                                  (int)N, 1, (int)T, (int)D, s), "reduce partials"));
    return RACE_OK;
}

size_t race_op_state_bytes(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block)
{
    Geo g;
    if (op_geometry(N, T, S, D, block, g) != RACE_OK)
        return 0;
    return align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4);
}

int race_op_fwd_keep(const float *pK, const float *pQ, const float *V, float *out, int64_t N, int64_t T,
                     int64_t S, int64_t D, float eps, int64_t block, void *workspace, size_t workspace_bytes,
                     float *state, size_t state_bytes, race_stream stream)
{
    RACE_TRY(kept_state_check(state, state_bytes, N, T, S, D, block, "race_op_fwd_keep"));
    return op_fwd_impl(pK, pQ, V, out, N, T, S, D, eps, block, workspace, workspace_bytes, stream, 0,
                       "race_op_fwd_keep", state);
}

int race_op_bwd_kept(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK, float *gpQ,
                     float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps, int64_t block,
                     void *workspace, size_t workspace_bytes, const float *state, size_t state_bytes,
                     race_stream stream)
{
    RACE_TRY(kept_state_check(state, state_bytes, N, T, S, D, block, "race_op_bwd_kept"));
    return op_bwd_impl(pK, pQ, V, gO, gpK, gpQ, gV, N, T, S, D, eps, block, workspace, workspace_bytes, stream, 0,
                       "race_op_bwd_kept", state);
}

int race_op_bwd(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK, float *gpQ,
                float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps, int64_t block,
                void *workspace, size_t workspace_bytes, race_stream stream)
{
    return op_bwd_impl(pK, pQ, V, gO, gpK, gpQ, gV, N, T, S, D, eps, block, workspace, workspace_bytes, stream, 0,
                       "race_op_bwd");
}

// ============================================================================ causal linear attention
// Unnormalised causal linear attention on the same chunked scan (W = Q, no 1/(A+eps)).
int race_causal_dot_product(const float *Q, const float *K, const float *V, float *out, int64_t N, int64_t L,
                            int64_t E, int64_t M, int64_t block, void *workspace, size_t workspace_bytes,
                            race_stream stream)
{
    return op_fwd_impl(K, Q, V, out, N, L, E, M, 0.0f, block, workspace, workspace_bytes, stream, 1,
                       "race_causal_dot_product");
}

int race_causal_dot_backward(const float *Q, const float *K, const float *V, const float *gO, float *gQ,
                             float *gK, float *gV, int64_t N, int64_t L, int64_t E, int64_t M, int64_t block,
                             void *workspace, size_t workspace_bytes, race_stream stream)
{
    return op_bwd_impl(K, Q, V, gO, gK, gQ, gV, N, L, E, M, 0.0f, block, workspace, workspace_bytes, stream, 1,
                       "race_causal_dot_backward");
}

int race_causal_dot_product_keep(const float *Q, const float *K, const float *V, float *out, int64_t N, int64_t L,
                                 int64_t E, int64_t M, int64_t block, void *workspace, size_t workspace_bytes,
                                 float *state, size_t state_bytes, race_stream stream)
{
    RACE_TRY(kept_state_check(state, state_bytes, N, L, E, M, block, "race_causal_dot_product_keep"));
    return op_fwd_impl(K, Q, V, out, N, L, E, M, 0.0f, block, workspace, workspace_bytes, stream, 1,
                       "race_causal_dot_product_keep", state);
}

int race_causal_dot_backward_kept(const float *Q, const float *K, const float *V, const float *gO, float *gQ,
                                  float *gK, float *gV, int64_t N, int64_t L, int64_t E, int64_t M, int64_t block,
                                  void *workspace, size_t workspace_bytes, const float *state, size_t state_bytes,
                                  race_stream stream)
{
    RACE_TRY(kept_state_check(state, state_bytes, N, L, E, M, block, "race_causal_dot_backward_kept"));
    return op_bwd_impl(K, Q, V, gO, gK, gQ, gV, N, L, E, M, 0.0f, block, workspace, workspace_bytes, stream, 1,
                       "race_causal_dot_backward_kept", state);
}

// ============================================================================ non-causal op
static size_t nc_bytes(const Geo &g, int backward)
{
    return (backward ? 2 : 1) * (align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4));
}

size_t race_nc_op_workspace_bytes(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block, int backward)
{
    Geo g;
    if (op_geometry(N, T, S, D, block, g) != RACE_OK)
        return 0;
    return nc_bytes(g, backward);
}

// whole-sequence totals of (w, x): per-block sums then the forward block scan (slot NB); x rows
// through the view xv of a [Z / zH][zH][T][D] layout
static int nc_totals(const Geo &g, ScanParams P, const float *w, const View &xv, int zH, float *wsB, float *wsA,
                     hipStream_t s)
{
    P.pK = w;
    P.V = static_cast<const float *>(xv.p);
    P.v = xv;
    P.zH = zH;
    P.wsB = wsB;
    P.wsA = wsA;
    RACE_TRY(run_scan_op(K_FWD_TOTALS, g, P, s));
    return hip_check(prof_block_scan(wsB, (int64_t)g.S_pad * g.DP, wsA, g.S_pad, (int)g.NB, (int)g.Z, 0, s), "block scan");
}

static NcParams nc_params(const Geo &g, int64_t T, int64_t S, int64_t D, float eps, int zH)
{
    NcParams Q;
    std::memset(&Q, 0, sizeof(Q));
    Q.T = (int)T;
    Q.S = (int)S;
    Q.D = (int)D;
    Q.NB = (int)g.NB;
    Q.S_pad = g.S_pad;
    Q.DPw = g.DP;
    Q.eps = eps;
    Q.zH = zH;
    return Q;
}

static NcRows nc_rows(const View &v) { return NcRows{v.sb, v.sh, v.st}; }

// every row of the views starts 16-byte aligned and D % 4 == 0: rows move as 16-byte runs
static int nc_vec(int64_t D, std::initializer_list<const View *> vs)
{
    if (D & 3)
        return 0;
    for (const View *v : vs)
        if ((reinterpret_cast<uintptr_t>(v->p) & 15) || (v->sb & 3) || (v->sh & 3) || (v->st & 3))
            return 0;
    return 1;
}

// the contiguous [N][T][D] layout of the race_nc_op_* entry points as a view (zH = 1)
static View nc_flat(const float *p, int64_t T, int64_t D) { return View{p, T * D, 0, D}; }

// A [Bz][H][T][D] view of the view entry points. Inputs may share rows between streams (a zero
// stream or head stride reads one row set for all of them); an output must give every
// (stream, head, token) row its own D elements, or concurrent workgroups would write the same
// memory: sorted by stride, each dimension of extent > 1 must step past everything the smaller
// ones span.
static int nc_view_check(const View &v, int64_t Bz, int64_t H, int64_t T, int64_t D, bool output, const char *name,
                         const char *who)
{
    if (!v.p)
        return fail(RACE_ERR_INVALID, "%s: null %s", who, name);
    if (v.sb < 0 || v.sh < 0 || v.st < D || v.st >= ((int64_t)1 << 31))
        return fail(RACE_ERR_INVALID, "%s: %s strides must be >= 0 with D <= token stride < 2^31", who, name);
    if (output) {
        int64_t st[3] = {v.sb, v.sh, v.st}, n[3] = {Bz, H, T};
        for (int i = 0; i < 3; ++i)  // sort the three dimensions by stride
            for (int j = i + 1; j < 3; ++j)
                if (st[j] < st[i]) {
                    std::swap(st[i], st[j]);
                    std::swap(n[i], n[j]);
                }
        int64_t span = D;  // elements covered by the dimensions taken so far
        for (int i = 0; i < 3; ++i) {
            if (n[i] <= 1)
                continue;
            if (st[i] < span)
                return fail(RACE_ERR_INVALID, "%s: output %s has overlapping rows (strides %lld, %lld, %lld)", who,
                            name, (long long)v.sb, (long long)v.sh, (long long)v.st);
            span = st[i] * (n[i] - 1) + span;
        }
    }
    return RACE_OK;
}

// streams n = b * H + h of the [B*H][T][S] probabilities; V / out rows through views
static int nc_fwd_impl(const float *pK, const float *pQ, const View &V, const View &out, int64_t Bz, int64_t H,
                       int64_t T, int64_t S, int64_t D, float eps, int64_t block, void *workspace,
                       size_t workspace_bytes, race_stream stream, float *state, const char *who)
{
    if (Bz <= 0 || H <= 0 || Bz * H > INT32_MAX)
        return fail(RACE_ERR_INVALID, "%s: B and H must be positive", who);
    const int64_t N = Bz * H;
    Geo g;
    RACE_TRY(op_geometry(N, T, S, D, block, g));
    RACE_TRY(op_check(pK, pQ, static_cast<const float *>(V.p), eps, workspace, workspace_bytes, nc_bytes(g, 0), who));
    RACE_TRY(nc_view_check(V, Bz, H, T, D, false, "V", who));
    RACE_TRY(nc_view_check(out, Bz, H, T, D, true, "out", who));
    Carver cv(workspace, workspace_bytes);
    float *wsB = cv.take(g.state_elems_B), *wsA = cv.take(g.state_elems_A);
    if (state)  // the totals are kept for the backward
        state_views(g, state, wsB, wsA);
    const hipStream_t s = hs(stream);
    RACE_TRY(nc_totals(g, op_params(g, T, S, D, eps), pK, V, (int)H, wsB, wsA, s));
    NcParams Q = nc_params(g, T, S, D, eps, (int)H);
    Q.pQ = pQ;
    Q.out = static_cast<float *>(const_cast<void *>(out.p));
    Q.rO = nc_rows(out);
    Q.vec = nc_vec(D, {&out});
    Q.totB = wsB;
    Q.totA = wsA;
    ProfScope ps(RACE_PROF_NC_FWD, s);
    return hip_check(launch_noncausal(0, g.DP, Q, (int)N, s), "race_nc readout");
}

static int nc_bwd_impl(const float *pK, const float *pQ, const View &V, const View &gO, float *gpK, float *gpQ,
                       const View &gV, int64_t Bz, int64_t H, int64_t T, int64_t S, int64_t D, float eps,
                       int64_t block, void *workspace, size_t workspace_bytes, race_stream stream,
                       const float *state, const char *who)
{
    if (Bz <= 0 || H <= 0 || Bz * H > INT32_MAX)
        return fail(RACE_ERR_INVALID, "%s: B and H must be positive", who);
    const int64_t N = Bz * H;
    Geo g;
    RACE_TRY(op_geometry(N, T, S, D, block, g));
    RACE_TRY(op_check(pK, pQ, static_cast<const float *>(V.p), eps, workspace, workspace_bytes, nc_bytes(g, 1), who));
    if (!gpK || !gpQ)
        return fail(RACE_ERR_INVALID, "%s: null gradient pointer", who);
    RACE_TRY(nc_view_check(V, Bz, H, T, D, false, "V", who));
    RACE_TRY(nc_view_check(gO, Bz, H, T, D, false, "gO", who));
    RACE_TRY(nc_view_check(gV, Bz, H, T, D, true, "gV", who));
    Carver cv(workspace, workspace_bytes);
    float *wsB = cv.take(g.state_elems_B), *wsA = cv.take(g.state_elems_A);
    float *ws2B = cv.take(g.state_elems_B), *ws2A = cv.take(g.state_elems_A);
    const hipStream_t s = hs(stream);
    const ScanParams P = op_params(g, T, S, D, eps);
    if (state)  // the forward's totals, kept by the forward
        state_views(g, state, wsB, wsA);
    else
        RACE_TRY(nc_totals(g, P, pK, V, (int)H, wsB, wsA, s));
    RACE_TRY(nc_totals(g, P, pQ, gO, (int)H, ws2B, ws2A, s));
    NcParams Q = nc_params(g, T, S, D, eps, (int)H);
    Q.pK = pK;
    Q.V = static_cast<const float *>(V.p);
    Q.gO = static_cast<const float *>(gO.p);
    Q.gpK = gpK;
    Q.gpQ = gpQ;
    Q.gV = static_cast<float *>(const_cast<void *>(gV.p));
    Q.rV = nc_rows(V);
    Q.rG = nc_rows(gO);
    Q.rGV = nc_rows(gV);
    Q.vec = nc_vec(D, {&V, &gO, &gV});
    Q.totB = wsB;
    Q.totA = wsA;
    Q.totGE = ws2B;
    ProfScope ps(RACE_PROF_NC_BWD, s);
    return hip_check(launch_noncausal(1, g.DP, Q, (int)N, s), "race_nc backward");
}

int race_nc_op_fwd(const float *pK, const float *pQ, const float *V, float *out, int64_t N, int64_t T, int64_t S,
                   int64_t D, float eps, int64_t block, void *workspace, size_t workspace_bytes, race_stream stream)
{
    if (!out)
        return fail(RACE_ERR_INVALID, "race_nc_op_fwd: null out");
    return nc_fwd_impl(pK, pQ, nc_flat(V, T, D), nc_flat(out, T, D), N, 1, T, S, D, eps, block, workspace,
                       workspace_bytes, stream, nullptr, "race_nc_op_fwd");
}

int race_nc_op_bwd(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK, float *gpQ,
                   float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps, int64_t block,
                   void *workspace, size_t workspace_bytes, race_stream stream)
{
    if (!gO || !gV)
        return fail(RACE_ERR_INVALID, "race_nc_op_bwd: null gradient pointer");
    return nc_bwd_impl(pK, pQ, nc_flat(V, T, D), nc_flat(gO, T, D), gpK, gpQ, nc_flat(gV, T, D), N, 1, T, S, D, eps,
                       block, workspace, workspace_bytes, stream, nullptr, "race_nc_op_bwd");
}

int race_nc_op_fwd_keep(const float *pK, const float *pQ, const float *V, float *out, int64_t N, int64_t T,
                        int64_t S, int64_t D, float eps, int64_t block, void *workspace, size_t workspace_bytes,
                        float *state, size_t state_bytes, race_stream stream)
{
    RACE_TRY(kept_state_check(state, state_bytes, N, T, S, D, block, "race_nc_op_fwd_keep"));
    if (!out)
        return fail(RACE_ERR_INVALID, "race_nc_op_fwd_keep: null out");
    return nc_fwd_impl(pK, pQ, nc_flat(V, T, D), nc_flat(out, T, D), N, 1, T, S, D, eps, block, workspace,
                       workspace_bytes, stream, state, "race_nc_op_fwd_keep");
}

int race_nc_op_bwd_kept(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK, float *gpQ,
                        float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps, int64_t block,
                        void *workspace, size_t workspace_bytes, const float *state, size_t state_bytes,
                        race_stream stream)
{
    RACE_TRY(kept_state_check(state, state_bytes, N, T, S, D, block, "race_nc_op_bwd_kept"));
    if (!gO || !gV)
        return fail(RACE_ERR_INVALID, "race_nc_op_bwd_kept: null gradient pointer");
    return nc_bwd_impl(pK, pQ, nc_flat(V, T, D), nc_flat(gO, T, D), gpK, gpQ, nc_flat(gV, T, D), N, 1, T, S, D, eps,
                       block, workspace, workspace_bytes, stream, state, "race_nc_op_bwd_kept");
}

int race_nc_fwd_view(const float *pK, const float *pQ, race_tensor V, race_tensor out, int64_t B, int64_t H,
                     int64_t T, int64_t S, int64_t D, float eps, int64_t block, void *workspace,
                     size_t workspace_bytes, float *state, size_t state_bytes, race_stream stream)
{
    if (state)
        RACE_TRY(kept_state_check(state, state_bytes, B * H, T, S, D, block, "race_nc_fwd_view"));
    return nc_fwd_impl(pK, pQ, to_view(V), to_view(out), B, H, T, S, D, eps, block, workspace, workspace_bytes,
                       stream, state, "race_nc_fwd_view");
}

int race_nc_bwd_view(const float *pK, const float *pQ, race_tensor V, race_tensor gO, float *gpK, float *gpQ,
                     race_tensor gV, int64_t B, int64_t H, int64_t T, int64_t S, int64_t D, float eps,
                     int64_t block, void *workspace, size_t workspace_bytes, const float *state,
                     size_t state_bytes, race_stream stream)
{
    if (state)
        RACE_TRY(kept_state_check(state, state_bytes, B * H, T, S, D, block, "race_nc_bwd_view"));
    return nc_bwd_impl(pK, pQ, to_view(V), to_view(gO), gpK, gpQ, to_view(gV), B, H, T, S, D, eps, block,
                       workspace, workspace_bytes, stream, state, "race_nc_bwd_view");
}

// ============================================================================ fused layer
size_t race_qkv_state_bytes(const race_qkv_shape *sh)
{
    Geo g;
    if (qkv_geometry(sh, g) != RACE_OK)
        return 0;
    return align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4);
}

// The fused kernels (race_fused.h) carry the backward suffix states in fp32; the generic ones
// (race_scan_kernels.h, hash bits or tiles the fused set does not compile) as double-floats,
// whose low parts need a second pair of arrays.
static bool qkv_generic(const race_qkv_shape *sh, const Geo &g) { return !fused_variant_exists(g.ST, g.DP, sh->K); }

static size_t qkv_scratch(const race_qkv_shape *sh, const Geo &g, int backward)
{
    const size_t q_elems = (size_t)sh->B * sh->Hq * sh->T * sh->D;
    const size_t kv_elems = (size_t)sh->B * sh->Hkv * sh->T * sh->D;
    size_t b = 0;
    if (backward)
        b += (qkv_generic(sh, g) ? 2 : 1) * (align256(g.state_elems_B * 4) + align256(g.state_elems_A * 4));
    if (g.n_st > 1) {  // fp32 partial sums: one per tile, or one running sum (seq)
        const size_t m = g.seq ? 1 : g.n_st;
        b += align256(m * q_elems * 4);
        if (backward)
            b += 2 * align256(m * kv_elems * 4);
    }
    return b;
}

size_t race_qkv_scratch_bytes(const race_qkv_shape *sh, int backward)
{
    Geo g;
    if (qkv_geometry(sh, g) != RACE_OK)
        return 0;
    return qkv_scratch(sh, g, backward);
}

static ScanParams qkv_params(const race_qkv_shape *sh, const Geo &g)
{
    ScanParams P;
    std::memset(&P, 0, sizeof(P));
    P.T = sh->T;
    P.R = 1 << sh->K;
    P.S = sh->L * P.R;
    P.D = sh->D;
    P.L = sh->L;
    P.K = sh->K;
    P.G = sh->Hq / sh->Hkv;
    P.Hkv = sh->Hkv;
    P.CB = (int)g.CB;
    P.NB = (int)g.NB;
    P.n_st = g.n_st;
    P.S_pad = g.S_pad;
    P.DPw = g.DP;
    P.eps = sh->eps;
    P.scale = sh->scale;
    P.inv_scale = 1.0f / sh->scale;
    return P;
}

// Output view of bucket tile j of n when the tiles run one launch after another: every tile but
// the last writes the fp32 running sum `run` (contiguous [B][H][T][D]); every tile but the first
// adds the running sum in its store; the last writes the caller's output.
static OutView tile_out(int j, int n, float *run, const OutView &final_out, int H, int64_t T, int64_t D)
{
    OutView o = j == n - 1 ? final_out : OutView{run, H * T * D, T * D, D, 0, 1};
    o.acc = j > 0 ? run : nullptr;
    o.acc_sb = H * T * D;
    o.acc_sh = T * D;
    o.acc_st = D;
    o.stage_f32 = 1;
    return o;
}

static int run_scan_qkv(ScanKernel k, const Geo &g, const ScanParams &P, hipStream_t s)
{
    ProfScope ps(RACE_PROF_QKV_FWD_TOTALS + (int)k, s);
    // (seq) the output kernels cover the one bucket tile P.st_base per launch
    const unsigned tiles = g.seq && k != K_FWD_TOTALS ? 1u : (unsigned)g.n_st;
    const dim3 grid((unsigned)g.NB, tiles, (unsigned)g.Z);
    // kernels specialised on the hash bits where compiled (K = 2..4), generic ones otherwise
    if (fused_variant_exists(g.ST, g.DP, P.K))
        return hip_check(launch_fused(k, g.ST, g.DP, P.K, P, grid, s), "race_qkv fused kernel launch");
    return hip_check(launch_scan_qkv(k, g.ST, g.DP, P, grid, s), "race_qkv kernel launch");
}

static int qkv_inputs(const race_qkv_shape *sh, const race_tensor &q, const race_tensor &k,
                      const race_tensor &v, const float *planes_T, const char *who)
{
    (void)sh;
    RACE_TRY(check_view(q, who, true));
    RACE_TRY(check_view(k, who, true));
    RACE_TRY(check_view(v, who, true));
    if (!planes_T)
        return fail(RACE_ERR_INVALID, "%s: null planes", who);
    return RACE_OK;
}

int race_qkv_fwd(const race_qkv_shape *sh, race_tensor q, race_tensor k, race_tensor v, const float *planes_T,
                 race_tensor out, int out_dtype, void *state, size_t state_bytes, void *scratch_buf,
                 size_t scratch_bytes, race_stream stream)
{
    Geo g;
    RACE_TRY(qkv_geometry(sh, g));
    RACE_TRY(qkv_inputs(sh, q, k, v, planes_T, "race_qkv_fwd"));
    if (out_dtype != RACE_F32 && out_dtype != RACE_BF16)
        return fail(RACE_ERR_INVALID, "race_qkv_fwd: out_dtype must be RACE_F32 or RACE_BF16");
    RACE_TRY(check_view(out, "race_qkv_fwd: out", false));
    const size_t need_state = race_qkv_state_bytes(sh), need_scr = qkv_scratch(sh, g, 0);
    if (!state || state_bytes < need_state)
        return fail(RACE_ERR_WORKSPACE, "race_qkv_fwd: state of %zu bytes needed, got %zu", need_state,
                    state ? state_bytes : 0);
    if (need_scr && (!scratch_buf || scratch_bytes < need_scr))
        return fail(RACE_ERR_WORKSPACE, "race_qkv_fwd: scratch of %zu bytes needed, got %zu", need_scr,
                    scratch_buf ? scratch_bytes : 0);
    ScanParams P = qkv_params(sh, g);
    P.q = to_view(q);
    P.k = to_view(k);
    P.v = to_view(v);
    P.planes = planes_T;
    Carver cs(state, state_bytes);
    P.wsB = cs.take(g.state_elems_B);
    P.wsA = cs.take(g.state_elems_A);
    const int64_t T = sh->T, D = sh->D;
    const int64_t q_elems = (int64_t)sh->B * sh->Hq * T * D;
    float *part = nullptr;
    if (g.n_st > 1) {
        Carver cw(scratch_buf, scratch_bytes);
        part = cw.take((size_t)(g.seq ? 1 : g.n_st) * q_elems);
        P.out = OutView{part, (int64_t)sh->Hq * T * D, T * D, D, q_elems, 1};
    } else {
        P.out = to_out(out, out_dtype == RACE_F32);
    }
    const hipStream_t s = hs(stream);
    RACE_TRY(run_scan_qkv(K_FWD_TOTALS, g, P, s));
    RACE_TRY(hip_check(prof_block_scan(P.wsB, (int64_t)g.S_pad * g.DP, P.wsA, g.S_pad, (int)g.NB, (int)g.Z, 0, s), "block scan"));
    if (g.seq) {
        for (int j = 0; j < g.n_st; ++j) {
            P.st_base = j;
            P.out = tile_out(j, g.n_st, part, to_out(out, out_dtype == RACE_F32), sh->Hq, T, D);
            RACE_TRY(run_scan_qkv(K_FWD_READOUT, g, P, s));
        }
        return RACE_OK;
    }
    RACE_TRY(run_scan_qkv(K_FWD_READOUT, g, P, s));
    if (part)
        RACE_TRY(hip_check(prof_reduce(part, g.n_st, q_elems, to_out(out, out_dtype == RACE_F32), sh->B,
                                                  sh->Hq, sh->T, sh->D, s), "reduce partials"));
    return RACE_OK;
}

// Everything of race_qkv_bwd after its argument checks; `scr` holds qkv_scratch(sh, g, 1) bytes.
static int qkv_bwd_run(const race_qkv_shape *sh, const Geo &g, race_tensor q, race_tensor k, race_tensor v,
                       race_tensor go, const float *planes_T, const void *state, size_t state_bytes, race_tensor dq,
                       race_tensor dk, race_tensor dv, void *scr, size_t scr_bytes, race_stream stream);

static int qkv_bwd_checks(const race_qkv_shape *sh, Geo &g, race_tensor q, race_tensor k, race_tensor v,
                          race_tensor go, const float *planes_T, const void *state, size_t state_bytes,
                          race_tensor dq, race_tensor dk, race_tensor dv, const char *who)
{
    RACE_TRY(qkv_geometry(sh, g));
    RACE_TRY(qkv_inputs(sh, q, k, v, planes_T, who));
    RACE_TRY(check_view(go, "race_qkv_bwd: go", true));
    RACE_TRY(check_view(dq, "race_qkv_bwd: dq", false));
    RACE_TRY(check_view(dk, "race_qkv_bwd: dk", false));
    RACE_TRY(check_view(dv, "race_qkv_bwd: dv", false));
    const size_t need_state = race_qkv_state_bytes(sh);
    if (!state || state_bytes < need_state)
        return fail(RACE_ERR_WORKSPACE, "%s: state of %zu bytes needed, got %zu", who, need_state,
                    state ? state_bytes : 0);
    return RACE_OK;
}

int race_qkv_bwd(const race_qkv_shape *sh, race_tensor q, race_tensor k, race_tensor v, race_tensor go,
                 const float *planes_T, const void *state, size_t state_bytes, race_tensor dq, race_tensor dk,
                 race_tensor dv, void *scratch_buf, size_t scratch_bytes, race_stream stream)
{
    Geo g;
    RACE_TRY(qkv_bwd_checks(sh, g, q, k, v, go, planes_T, state, state_bytes, dq, dk, dv, "race_qkv_bwd"));
    const size_t need_scr = qkv_scratch(sh, g, 1);
    if (!scratch_buf || scratch_bytes < need_scr)
        return fail(RACE_ERR_WORKSPACE, "race_qkv_bwd: scratch of %zu bytes needed, got %zu", need_scr,
                    scratch_buf ? scratch_bytes : 0);
    return qkv_bwd_run(sh, g, q, k, v, go, planes_T, state, state_bytes, dq, dk, dv, scratch_buf, scratch_bytes,
                       stream);
}

static int qkv_bwd_run(const race_qkv_shape *sh, const Geo &g, race_tensor q, race_tensor k, race_tensor v,
                       race_tensor go, const float *planes_T, const void *state, size_t state_bytes, race_tensor dq,
                       race_tensor dk, race_tensor dv, void *scr, size_t scr_bytes, race_stream stream)
{
    ScanParams P = qkv_params(sh, g);
    P.q = to_view(q);
    P.k = to_view(k);
    P.v = to_view(v);
    P.go = to_view(go);
    P.planes = planes_T;
    Carver cs(const_cast<void *>(state), state_bytes);
    P.wsB = cs.take(g.state_elems_B);
    P.wsA = cs.take(g.state_elems_A);
    Carver cw(scr, scr_bytes);
    P.ws2B = cw.take(g.state_elems_B);
    P.ws2A = cw.take(g.state_elems_A);
    const bool generic = qkv_generic(sh, g);
    if (generic) {
        P.ws3B = cw.take(g.state_elems_B);
        P.ws3A = cw.take(g.state_elems_A);
    }
    const int64_t T = sh->T, D = sh->D;
    const int64_t q_elems = (int64_t)sh->B * sh->Hq * T * D, kv_elems = (int64_t)sh->B * sh->Hkv * T * D;
    float *pq = nullptr, *pk = nullptr, *pv = nullptr;
    if (g.seq) {
        pq = cw.take(q_elems);
        pk = cw.take(kv_elems);
        pv = cw.take(kv_elems);
        const hipStream_t s = hs(stream);
        for (int j = 0; j < g.n_st; ++j) {
            P.st_base = j;
            P.dq = tile_out(j, g.n_st, pq, to_out(dq, 0), sh->Hq, T, D);
            RACE_TRY(run_scan_qkv(K_BWD_TOTALS, g, P, s));
        }
        P.st_base = 0;
        RACE_TRY(hip_check(prof_block_scan(P.ws2B, (int64_t)g.S_pad * g.DP, P.ws2A, g.S_pad, (int)g.NB, (int)g.Z, 1,
                                           s),
                           "block scan"));
        for (int j = 0; j < g.n_st; ++j) {
            P.st_base = j;
            P.dk = tile_out(j, g.n_st, pk, to_out(dk, 0), sh->Hkv, T, D);
            P.dv = tile_out(j, g.n_st, pv, to_out(dv, 0), sh->Hkv, T, D);
            RACE_TRY(run_scan_qkv(K_BWD_MAIN, g, P, s));
        }
        return RACE_OK;
    }
    if (g.n_st > 1) {
        pq = cw.take((size_t)g.n_st * q_elems);
        pk = cw.take((size_t)g.n_st * kv_elems);
        pv = cw.take((size_t)g.n_st * kv_elems);
        P.dq = OutView{pq, (int64_t)sh->Hq * T * D, T * D, D, q_elems, 1};
        P.dk = OutView{pk, (int64_t)sh->Hkv * T * D, T * D, D, kv_elems, 1};
        P.dv = OutView{pv, (int64_t)sh->Hkv * T * D, T * D, D, kv_elems, 1};
    } else {
        P.dq = to_out(dq, 0);
        P.dk = to_out(dk, 0);
        P.dv = to_out(dv, 0);
    }
    const hipStream_t s = hs(stream);
    RACE_TRY(run_scan_qkv(K_BWD_TOTALS, g, P, s));
    RACE_TRY(hip_check(prof_block_scan(P.ws2B, (int64_t)g.S_pad * g.DP, P.ws2A, g.S_pad, (int)g.NB, (int)g.Z, 1, s,
                                       generic ? P.ws3B : nullptr, generic ? P.ws3A : nullptr),
                       "block scan"));
    RACE_TRY(run_scan_qkv(K_BWD_MAIN, g, P, s));
    if (g.n_st > 1) {
        RACE_TRY(hip_check(prof_reduce(pq, g.n_st, q_elems, to_out(dq, 0), sh->B, sh->Hq, sh->T, sh->D, s),
                           "reduce partials"));
        RACE_TRY(hip_check(prof_reduce(pk, g.n_st, kv_elems, to_out(dk, 0), sh->B, sh->Hkv, sh->T, sh->D, s),
                           "reduce partials"));
        RACE_TRY(hip_check(prof_reduce(pv, g.n_st, kv_elems, to_out(dv, 0), sh->B, sh->Hkv, sh->T, sh->D, s),
                           "reduce partials"));
    }
    return RACE_OK;
}

int race_qkv_final_state(const race_qkv_shape *sh, const void *state, size_t state_bytes, float *A, float *Bs,
                         race_stream stream)
{
    Geo g;
    RACE_TRY(qkv_geometry(sh, g));
    const size_t need = race_qkv_state_bytes(sh);
    if (!state || state_bytes < need)
        return fail(RACE_ERR_WORKSPACE, "race_qkv_final_state: state of %zu bytes needed", need);
    if (!A || !Bs)
        return fail(RACE_ERR_INVALID, "race_qkv_final_state: null output");
    Carver cs(const_cast<void *>(state), state_bytes);
    const float *wsB = cs.take(g.state_elems_B);
    const float *wsA = cs.take(g.state_elems_A);
    const int S = sh->L << sh->K;
    return hip_check(launch_state_extract(wsB, wsA, (int)g.NB, g.S_pad, g.DP, (int)g.Z, S, sh->D, A, Bs, hs(stream)),
                     "race_qkv_final_state");
}

// ============================================================================ backward without a workspace
// race_qkv_bwd_static: race_qkv_bwd with its scratch (the suffix-state block sums of the
// backward) in a file-scope device array instead of a caller's buffer, for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops). The array lives on
// every GPU the library runs on until the process ends; its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and only that address reaches the
// kernels. Calls on one GPU share the array, so calls that overlap on one GPU (other streams,
// other threads) race; every element a call reads it has first written in the same call, so
// nothing needs clearing between calls.
static __device__ __align__(256) char scratch[RACE_STATIC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_addr[MAX_DEVICES] = {};

// Device address of `scratch` on the device that runs `stream` (the current device for the null
// stream), looked up on the first call for that device.
int static_scratch(race_stream stream, void **out)
{
    int cur = 0;
    RACE_TRY(hip_check(hipGetDevice(&cur), "race_qkv_bwd_static: hipGetDevice"));
    int dev = cur;
    if (stream)
        RACE_TRY(hip_check(hipStreamGetDevice(hs(stream), &dev), "race_qkv_bwd_static: hipStreamGetDevice"));
    if (dev < 0 || dev >= MAX_DEVICES)
        return fail(RACE_ERR_UNSUPPORTED, "race_qkv_bwd_static: device %d beyond %d", dev, MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        if (dev != cur)
            RACE_TRY(hip_check(hipSetDevice(dev), "race_qkv_bwd_static: hipSetDevice"));
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur)
            (void)hipSetDevice(cur);
        RACE_TRY(hip_check(e, "race_qkv_bwd_static: hipGetSymbolAddress"));
        if (!p)
            return fail(RACE_ERR_HIP, "race_qkv_bwd_static: no device address for the scratch array");
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return RACE_OK;
}
}  // namespace

size_t race_static_scratch_bytes(void) { return RACE_STATIC_SCRATCH_BYTES; }

int race_qkv_bwd_static(const race_qkv_shape *sh, race_tensor q, race_tensor k, race_tensor v, race_tensor go,
                        const float *planes_T, const void *state, size_t state_bytes, race_tensor dq, race_tensor dk,
                        race_tensor dv, race_stream stream)
{
    Geo g;
    RACE_TRY(qkv_bwd_checks(sh, g, q, k, v, go, planes_T, state, state_bytes, dq, dk, dv, "race_qkv_bwd_static"));
    const size_t need = qkv_scratch(sh, g, 1);
    if (need > RACE_STATIC_SCRATCH_BYTES)
        return fail(RACE_ERR_WORKSPACE,
                    "race_qkv_bwd_static: this shape needs %zu bytes of scratch, beyond the static %zu (use "
                    "race_qkv_bwd with a workspace)",
                    need, (size_t)RACE_STATIC_SCRATCH_BYTES);
    void *p = nullptr;
    RACE_TRY(static_scratch(stream, &p));
    return qkv_bwd_run(sh, g, q, k, v, go, planes_T, state, state_bytes, dq, dk, dv, p, RACE_STATIC_SCRATCH_BYTES,
                       stream);
}

// ============================================================================ decode
int race_decode_step(const race_decode_shape *sh, const void *q, const void *k, const void *v, int dtype,
                     const float *planes_T, float *A, float *Bs, void *out, race_stream stream)
{
    if (!sh)
        return fail(RACE_ERR_INVALID, "race_decode_step: null shape");
    if (sh->B <= 0 || sh->Hq <= 0 || sh->Hkv <= 0 || sh->L <= 0)
        return fail(RACE_ERR_INVALID, "race_decode_step: B, Hq, Hkv, L must be positive");
    if (sh->Hq % sh->Hkv || sh->Hq / sh->Hkv > DEC_GMAX)
        return fail(RACE_ERR_UNSUPPORTED, "race_decode_step: Hq/Hkv must be an integer <= %d", DEC_GMAX);
    if (sh->D != 64 && sh->D != 128)
        return fail(RACE_ERR_UNSUPPORTED, "race_decode_step: head dim %d, supported 64 and 128", sh->D);
    if (sh->K < 1 || sh->K > 4 || sh->L * sh->K > DEC_LKMAX || (sh->L << sh->K) > DEC_SMAX)
        return fail(RACE_ERR_UNSUPPORTED, "race_decode_step: K <= 4, L*K <= %d, L*2^K <= %d required", DEC_LKMAX,
                    DEC_SMAX);
    if (dtype != RACE_F32 && dtype != RACE_BF16)
        return fail(RACE_ERR_INVALID, "race_decode_step: dtype must be RACE_F32 or RACE_BF16");
    if (!q || !k || !v || !out || !A || !Bs || !planes_T)
        return fail(RACE_ERR_INVALID, "race_decode_step: null pointer");
    if (((uintptr_t)Bs & 15))
        return fail(RACE_ERR_INVALID, "race_decode_step: state Bs must be 16-byte aligned");
    if (!(sh->eps > 0.0f) || !(sh->scale > 0.0f))
        return fail(RACE_ERR_INVALID, "race_decode_step: eps and scale must be positive");
    DecodeParams P;
    std::memset(&P, 0, sizeof(P));
    P.q = q;
    P.k = k;
    P.v = v;
    P.out = out;
    P.A = A;
    P.Bs = Bs;
    P.planes = planes_T;
    P.B = sh->B;
    P.Hkv = sh->Hkv;
    P.G = sh->Hq / sh->Hkv;
    P.D = sh->D;
    P.L = sh->L;
    P.K = sh->K;
    P.round_planes = dtype == RACE_BF16;
    P.eps = sh->eps;
    P.inv_scale = 1.0f / sh->scale;
    return hip_check(prof_decode(P, dtype == RACE_BF16, hs(stream)), "race_decode_step");
}

// ============================================================================ kernel timing
int race_profile_enable(int on)
{
    Profiler &p = prof();
    std::lock_guard<std::mutex> g(p.mu);
    p.on = on != 0;
    return RACE_OK;
}

int race_profile_read(int kernel, double *total_ms, int64_t *launches)
{
    if (kernel < 0 || kernel >= RACE_PROF_KERNELS || !total_ms || !launches)
        return fail(RACE_ERR_INVALID, "race_profile_read: bad kernel id or null output");
    Profiler &p = prof();
    std::vector<EventPair> evs;
    {
        std::lock_guard<std::mutex> g(p.mu);
        evs.swap(p.pending[kernel]);
    }
    double add = 0.0;
    int rc = RACE_OK;
    for (const EventPair &e : evs) {
        float ms = 0.0f;
        if (rc == RACE_OK) {
            hipError_t err = hipEventSynchronize(e.b);
            if (err == hipSuccess)
                err = hipEventElapsedTime(&ms, e.a, e.b);
            if (err != hipSuccess)
                rc = hip_check(err, "race_profile_read");
        }
        add += ms;
        (void)hipEventDestroy(e.a);
        (void)hipEventDestroy(e.b);
    }
    std::lock_guard<std::mutex> g(p.mu);
    p.total_ms[kernel] += add;
    p.count[kernel] += (int64_t)evs.size();
    *total_ms = p.total_ms[kernel];
    *launches = p.count[kernel];
    return rc;
}

int race_profile_reset(void)
{
    Profiler &p = prof();
    std::vector<EventPair> evs;
    {
        std::lock_guard<std::mutex> g(p.mu);
        for (int k = 0; k < RACE_PROF_KERNELS; ++k) {
            evs.insert(evs.end(), p.pending[k].begin(), p.pending[k].end());
            p.pending[k].clear();
            p.total_ms[k] = 0.0;
            p.count[k] = 0;
        }
    }
    for (const EventPair &e : evs) {
        (void)hipEventSynchronize(e.b);
        (void)hipEventDestroy(e.a);
        (void)hipEventDestroy(e.b);
    }
    return RACE_OK;
}

}  // extern "C"
