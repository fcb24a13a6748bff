// C ABI of the scoring path (include/chimera_hip.h): context, index upload,
// the batched search pipeline, traces and graph capture.
#include "chimera_hip.h"
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

using namespace chimera;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

#define CK_HIP(expr, what)                                                                              \
    do {                                                                                                \
        const hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess) return fail(CHIMERA_ERR_HIP, std::string(what) + " failed: " + hipGetErrorString(e_)); \
    } while (0)

#define CK(expr)                    \
    do {                            \
        const int r_ = (expr);      \
        if (r_ != CHIMERA_OK) return r_; \
    } while (0)

}  // namespace

// Workspace of chimera_search_device_noalloc: one array per device, held
// until the process ends and shared by every such call on that device. Host
// code uses only the address hipGetSymbolAddress returns for it.
constexpr size_t kStaticScratchBytes = size_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

std::mutex g_scratch_mu;
std::vector<unsigned char*> g_scratch_ptr;  // device ordinal -> address of scratch on that device

// Address of the static workspace on `device`, which must be current; looked
// up once per device.
int scratch_address(int device, unsigned char** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr.size() <= static_cast<size_t>(device)) g_scratch_ptr.resize(static_cast<size_t>(device) + 1, nullptr);
    if (!g_scratch_ptr[static_cast<size_t>(device)]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return fail(CHIMERA_ERR_HIP, std::string("hipGetSymbolAddress of the static workspace failed: ") +
                                             hipGetErrorString(e));
        g_scratch_ptr[static_cast<size_t>(device)] = static_cast<unsigned char*>(p);
    }
    *out = g_scratch_ptr[static_cast<size_t>(device)];
    return CHIMERA_OK;
}

}  // namespace

// Per-batch device buffers of the search pipeline, carved from one block:
// the context's workspace (allocated at upload) or the static workspace of
// chimera_search_device_noalloc.
struct Workspace {
    float* queries = nullptr;     // [B * 32 * dim] query staging (host entry points)
    float* rot = nullptr;         // [B * 32 * 128]
    float* cb1 = nullptr;         // [B * 32]
    float* cbex = nullptr;        // [B * 32]
    float* lut = nullptr;         // [B * kLutPerQuery]
    uint32_t* labels = nullptr;   // [B * 32 * nprobe]
    uint32_t* vcnt = nullptr;     // [qs][nbk][32] visit counts, then offsets (see CandidateArgs)
    uint32_t* vtot = nullptr;     // [qs]
    uint2* rec = nullptr;         // [qs][vcap] visit records, then candidates
    uint32_t* tcount = nullptr;   // [qs][nbk] candidates per bucket
    float2* gstat = nullptr;      // [qs][nbk][groups_per_bucket(blog)]
    uint2* gsec = nullptr;        // [qs][nbk][groups_per_bucket(blog)]
    uint16_t* gkey = nullptr;     // [qs][nbk][groups_per_bucket(blog)]
    int32_t* ccount = nullptr;    // [qs] candidates per query
    int32_t* rcount = nullptr;    // [B]
    int32_t* rids = nullptr;      // [B * k_refine]
    float* rscore = nullptr;      // [B * k_refine]
    float* s1 = nullptr;          // [B * k_refine]
    int32_t* fcount = nullptr;    // [B]
    int32_t* fids = nullptr;      // [B * fb_cap]
    float* fscores = nullptr;     // [B * fb_cap]
    uint32_t* err = nullptr;      // status word
    int32_t* out_counts = nullptr;  // [B] (host entry points)
    int qs = 0;                   // queries of candidate state
};

struct WorkspaceShape {
    size_t batch, qs, dim, nprobe, nbk, vcap, k_refine, fb_cap;
    bool staging;  // query staging and result counts of the host entry points
    int blog;      // documents per candidate bucket = 2^blog
};

// Bytes of a workspace of this shape (arrays at 256-byte boundaries); with a
// base, also the pointers into it.
size_t carve_workspace(const WorkspaceShape& sh, unsigned char* base, Workspace* w) {
    size_t off = 0;
    auto take = [&](auto*& p, size_t count) {
        using T = std::remove_reference_t<decltype(*p)>;
        off = (off + 255) / 256 * 256;
        if (base) p = reinterpret_cast<T*>(base + off);
        off += std::max<size_t>(count, 1) * sizeof(T);
    };
    Workspace tmp;
    Workspace& x = w ? *w : tmp;
    const size_t B = sh.batch, QS = sh.qs;
    if (sh.staging) take(x.queries, B * kQ * sh.dim);
    take(x.rot, B * kQ * kDim);
    take(x.cb1, B * kQ);
    take(x.cbex, B * kQ);
    take(x.lut, B * kLutPerQuery);
    take(x.labels, B * kQ * sh.nprobe);
    take(x.vcnt, QS * sh.nbk * kQ);
    take(x.vtot, QS);
    take(x.rec, QS * sh.vcap);
    take(x.tcount, QS * sh.nbk);
    take(x.gstat, QS * sh.nbk * static_cast<size_t>(groups_per_bucket(sh.blog)));
    take(x.gsec, QS * sh.nbk * static_cast<size_t>(groups_per_bucket(sh.blog)));
    take(x.gkey, QS * sh.nbk * static_cast<size_t>(groups_per_bucket(sh.blog)));
    take(x.ccount, QS);
    take(x.rcount, B);
    take(x.rids, B * sh.k_refine);
    take(x.rscore, B * sh.k_refine);
    take(x.s1, B * sh.k_refine);
    take(x.fcount, B);
    take(x.fids, B * sh.fb_cap);
    take(x.fscores, B * sh.fb_cap);
    take(x.err, 1);
    if (sh.staging) take(x.out_counts, B);
    x.qs = static_cast<int>(QS);
    return (off + 255) / 256 * 256;
}

struct chimera_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void*> index_allocs;
    std::vector<void*> ws_allocs;
    uint64_t bytes = 0;

    bool has_index = false;
    int64_t n = 0, dim = 0, n_clusters = 0, ex_bits = 0, num_docs = 0;
    int32_t* doc_ptrs = nullptr;
    uint64_t* cluster_pos = nullptr;
    uint8_t* codes_clu = nullptr;
    float* f1_clu = nullptr;
    int32_t* doc_clu = nullptr;
    uint8_t* codes_tok = nullptr;
    float* f1_tok = nullptr;
    uint8_t* full_codes = nullptr;
    float* full_factors = nullptr;
    float* centroids = nullptr;
    float* norms = nullptr;
    uint8_t* flips = nullptr;
    uint32_t* inv = nullptr;  // cluster position -> token (device-built indexes)

    chimera_search_options opt{};
    int max_batch = 0;
    int qs = 0;           // candidate-stage sub-batch
    int qs_cap = 0;       // queries the candidate workspace holds
    int64_t vcap = 0;     // visit records per query (candidate stage)
    int nbk = 0;          // document buckets per query
    int blog = kMaxBucketLog2;  // documents per bucket = 2^blog
    int held = 8;               // visit records per reduce thread kept in registers
    int fb_cap = 0;       // full-bit documents per query

    Workspace ws;                 // per-batch buffers, one allocation
    // Results of the host entry points, laid out per call as [ids (nq k)]
    // [scores (nq k)] [counts (nq)] [status word] in one device region, so
    // that one copy brings them back into the pinned staging buffer (which
    // also carries the query batch up).
    unsigned char* w_out = nullptr;
    size_t w_out_bytes = 0;
    int64_t* w_out_ids = nullptr;
    float* w_out_scores = nullptr;
    int32_t* w_out_counts = nullptr;
    uint32_t* w_out_status = nullptr;
    size_t w_out_used = 0;             // bytes of the region the last call laid out
    unsigned char* h_stage = nullptr;  // pinned host memory (hipHostMalloc)
    size_t h_stage_bytes = 0;
    uint32_t* noalloc_status = nullptr;  // status word of the last chimera_search_device_noalloc (own allocation)
    bool noalloc_pending = false;        // that word has not been read by chimera_synchronize

    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    bool capturing = false;
    bool exact_scoring = false;
    int probe_mode = 0;
    int num_cus = 256;
    // matrix-core probe
    uint16_t* cbf = nullptr;
    float* cnh = nullptr;  // -|c|^2/2
    float cmax = 0.f;   // >= max |c| over the centroids
    float ecmax = 0.f;  // >= max |c - bf16(c)|
    uint32_t* p_err = nullptr;    // device word: bits of max |c - bf16(c)|
    uint32_t* p_ncand = nullptr;  // [rows] filtered candidates per row of the last matrix-core probe
    float* p_gm = nullptr;
    float* p_thr = nullptr;
    uint32_t* p_rval = nullptr;  // probe records: 16 fp16 values (8 words) each
    uint32_t* p_rtile = nullptr;  // probe records: tile
    uint32_t* p_cnt = nullptr;
    uint32_t* p_flag = nullptr;
    ExactFallback p_xfb;  // exact recomputation of flagged probe rows
    bool probe_mfma_ready = false;

    // per-stage event timing
    bool profiling = false;
    double stage_ms[CHIMERA_STAGES] = {};
    int64_t stage_n[CHIMERA_STAGES] = {};
    struct Pending {
        int stage;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
    hipEvent_t open_event = nullptr;
    int open_stage = -1;
};

namespace {

template <typename T>
int dev_alloc(chimera_ctx* c, std::vector<void*>& list, T** p, size_t count, const char* what) {
    *p = nullptr;
    if (count == 0) count = 1;
    void* ptr = nullptr;
    const hipError_t e = hipMalloc(&ptr, count * sizeof(T));
    if (e != hipSuccess) {
        return fail(CHIMERA_ERR_HIP, std::string("hipMalloc of ") + what + " (" + std::to_string(count * sizeof(T)) +
                                         " bytes) failed: " + hipGetErrorString(e));
    }
    list.push_back(ptr);
    c->bytes += count * sizeof(T);
    *p = static_cast<T*>(ptr);
    return CHIMERA_OK;
}

void free_list(std::vector<void*>& list) {
    for (void* p : list) (void)hipFree(p);
    list.clear();
}

void release_index(chimera_ctx* c) {
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->graph_exec = nullptr;
    c->graph = nullptr;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    free_list(c->ws_allocs);
    free_list(c->index_allocs);
    c->bytes = 0;
    c->has_index = false;
    c->w_out = nullptr;
    c->w_out_bytes = 0;
    c->ws = Workspace{};
    c->noalloc_status = nullptr;
    c->noalloc_pending = false;
    c->probe_mfma_ready = false;
    c->inv = nullptr;
    c->cbf = nullptr;
    c->cnh = nullptr;
    c->p_err = nullptr;
    c->p_ncand = nullptr;
    c->p_xfb = ExactFallback{};
}

int set_device(chimera_ctx* c) {
    CK_HIP(hipSetDevice(c->device), "hipSetDevice");
    return CHIMERA_OK;
}

}  // namespace

namespace chimera {

int api_fail(int code, const std::string& msg) { return fail(code, msg); }

int api_enter(chimera_ctx* c, hipStream_t* stream) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    CK(set_device(c));
    *stream = c->stream;
    return CHIMERA_OK;
}

}  // namespace chimera

namespace {
hipEvent_t take_event(chimera_ctx* c);
}  // namespace

namespace chimera {

void stage_begin(chimera_ctx* c, int stage) {
    if (!c->profiling || c->capturing) return;
    c->open_event = take_event(c);
    c->open_stage = stage;
    if (c->open_event) (void)hipEventRecord(c->open_event, c->stream);
}

void stage_end(chimera_ctx* c) {
    if (!c->profiling || c->capturing || !c->open_event) return;
    hipEvent_t b = take_event(c);
    if (!b) return;
    (void)hipEventRecord(b, c->stream);
    c->pending.push_back({c->open_stage, c->open_event, b});
    c->open_event = nullptr;
}

}  // namespace chimera

namespace {

hipEvent_t take_event(chimera_ctx* c) {
    if (!c->pool.empty()) {
        hipEvent_t e = c->pool.back();
        c->pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

int collect_stage_times(chimera_ctx* c) {
    for (auto& p : c->pending) {
        CK_HIP(hipEventSynchronize(p.b), "hipEventSynchronize");
        float ms = 0.f;
        CK_HIP(hipEventElapsedTime(&ms, p.a, p.b), "hipEventElapsedTime");
        c->stage_ms[p.stage] += ms;
        c->stage_n[p.stage] += 1;
        c->pool.push_back(p.a);
        c->pool.push_back(p.b);
    }
    c->pending.clear();
    return CHIMERA_OK;
}

#define STAGE(c, id, expr, what) \
    do {                          \
        stage_begin(c, id);       \
        CK_HIP(expr, what);       \
        stage_end(c);             \
    } while (0)

// Device buffers that live for one call; freed after the stream drains.
struct TempBuffers {
    hipStream_t stream = nullptr;
    std::vector<void*> ptrs;
    ~TempBuffers() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <typename T>
    int alloc(T** p, size_t count, const char* what) {
        *p = nullptr;
        if (count == 0) count = 1;
        void* ptr = nullptr;
        const hipError_t e = hipMalloc(&ptr, count * sizeof(T));
        if (e != hipSuccess) {
            return fail(CHIMERA_ERR_HIP, std::string("hipMalloc of ") + what + " (" +
                                             std::to_string(count * sizeof(T)) + " bytes) failed: " +
                                             hipGetErrorString(e));
        }
        ptrs.push_back(ptr);
        *p = static_cast<T*>(ptr);
        return CHIMERA_OK;
    }
    void release(void* p) {
        auto it = std::find(ptrs.begin(), ptrs.end(), p);
        if (it == ptrs.end()) return;
        if (stream) (void)hipStreamSynchronize(stream);
        (void)hipFree(p);
        ptrs.erase(it);
    }
};

template <typename T>
int upload(chimera_ctx* c, T** dst, const T* src, size_t count, const char* what) {
    CK(dev_alloc(c, c->index_allocs, dst, count, what));
    if (count) CK_HIP(hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice), what);
    return CHIMERA_OK;
}

// count elements from src followed by pad zeros
template <typename T>
int upload_padded(chimera_ctx* c, T** dst, const T* src, size_t count, size_t pad, const char* what) {
    CK(dev_alloc(c, c->index_allocs, dst, count + pad, what));
    if (count) CK_HIP(hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice), what);
    CK_HIP(hipMemset(*dst + count, 0, pad * sizeof(T)), what);
    return CHIMERA_OK;
}

}  // namespace

namespace chimera {

__global__ void gather_token_order_kernel(const uint8_t* __restrict__ codes_clu, const float* __restrict__ f1_clu,
                                          const uint32_t* __restrict__ tok2pos, int64_t n,
                                          uint8_t* __restrict__ codes_tok, float* __restrict__ f1_tok) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const uint32_t p = tok2pos[t];
    reinterpret_cast<uint4*>(codes_tok)[t] = reinterpret_cast<const uint4*>(codes_clu)[p];
    f1_tok[t] = f1_clu[p];
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < n;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x)
        p[t] = v;
}

hipError_t launch_gather_token_order(hipStream_t s, const uint8_t* codes_clu, const float* f1_clu,
                                     const uint32_t* tok2pos, int64_t n, uint8_t* codes_tok, float* f1_tok) {
    hipLaunchKernelGGL(gather_token_order_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                       codes_clu, f1_clu, tok2pos, n, codes_tok, f1_tok);
    return hipGetLastError();
}

__global__ void copy_u32_kernel(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src, int64_t n) {
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < n;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x)
        dst[t] = src[t];
}

hipError_t launch_copy_u32(hipStream_t s, uint32_t* dst, const uint32_t* src, int64_t n) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(copy_u32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, dst, src, n);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, int64_t n, uint32_t v) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace chimera

namespace {

// Capacity of the union of chunk selections (search_impl.cu:426-459): at
// most sum_c floor(F (c+1) / n_ch) <= F (n_ch + 1) / 2 documents, and never
// more than k_refine.
// The candidate stage keeps one LDS counter per document bucket (at most
// 16,384 buckets of at most 8,192 documents).
constexpr int64_t kMaxDocs = int64_t{16384} * kMaxBucketDocs;

int fullbit_capacity(const chimera_search_options& o) {
    const int64_t f = o.k_full_bit;
    const int64_t nch = o.num_chunks;
    int64_t sum = 0;
    for (int64_t c = 0; c < nch && sum < o.k_refine; ++c) sum += std::min<int64_t>(f * (c + 1) / nch, f);
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(sum, o.k_refine)));
}

int validate_options(const chimera_search_options& o, int64_t n_clusters) {
    if (o.nprobe <= 0 || o.k_refine <= 0 || o.k_full_bit <= 0 || o.cagra_itopk_size <= 0 || o.num_chunks <= 0) {
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "All Chimera search options must be positive");
    }
    if (o.k_full_bit > o.k_refine) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "k_full_bit must not exceed k_refine");
    if (n_clusters > 0 && o.nprobe > n_clusters) {
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nprobe must not exceed the number of clusters");
    }
    if (o.nprobe > 2048) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nprobe must not exceed 2048");
    if (o.k_refine > 16384) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "k_refine must not exceed 16384");
    return CHIMERA_OK;
}

int status_errors(chimera_ctx* c, uint32_t err) {
    if (err & kErrCandOverflow)
        return fail(CHIMERA_ERR_CAPACITY, "Candidate visits exceeded workspace bound " + std::to_string(c->vcap));
    if (err & kErrFullbitCap)
        return fail(CHIMERA_ERR_CAPACITY, "Full-bit candidate count exceeded workspace bound " + std::to_string(c->fb_cap));
    return CHIMERA_OK;
}

int check_errors(chimera_ctx* c, const uint32_t* word) {
    uint32_t err = 0;
    CK_HIP(hipMemcpy(&err, word, sizeof(err), hipMemcpyDeviceToHost), "reading search status");
    return status_errors(c, err);
}

int check_search_args(chimera_ctx* c, int32_t nq, int32_t k) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    if (!c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot search an empty Chimera index");
    if (k <= 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "k must be positive");
    if (nq < 0 || nq > c->max_batch) {
        return fail(CHIMERA_ERR_INVALID_ARGUMENT,
                    "batch of " + std::to_string(nq) + " queries exceeds the workspace bound of " + std::to_string(c->max_batch));
    }
    return CHIMERA_OK;
}

CandidateArgs candidate_args(chimera_ctx* c, const Workspace& w) {
    CandidateArgs a{};
    a.labels = w.labels;
    a.nprobe = c->opt.nprobe;
    a.cluster_pos = c->cluster_pos;
    a.codes_clu = c->codes_clu;
    a.f1_clu = c->f1_clu;
    a.doc_clu = c->doc_clu;
    a.n_clusters = c->n_clusters;
    a.num_docs = c->num_docs;
    a.lut = w.lut;
    a.cb1 = w.cb1;
    a.blog = c->blog;
    a.held = c->held;
    a.nbk = c->nbk;
    a.vcnt = w.vcnt;
    a.vtot = w.vtot;
    a.rec = w.rec;
    a.vcap = c->vcap;
    a.tcount = w.tcount;
    a.gstat = w.gstat;
    a.gsec = w.gsec;
    a.gkey = w.gkey;
    a.k_refine = c->opt.k_refine;
    a.ccount = w.ccount;
    a.rcount = w.rcount;
    a.rids = w.rids;
    a.rscore = w.rscore;
    a.err = w.err;
    a.num_cus = c->num_cus;
    a.wqs = w.qs;
    return a;
}

// Candidate stage + refinement selection for queries [qb, qb + qn), in
// sub-batches of at most min(c->qs, w.qs) queries (the candidate state of
// the workspace holds w.qs).
int run_candidates(chimera_ctx* c, const Workspace& w, hipStream_t s, int qb, int qn) {
    const CandidateArgs a = candidate_args(c, w);
    const int sub = std::min(c->qs, w.qs);
    for (int q0 = qb; q0 < qb + qn; q0 += sub) {
        const int n = std::min(sub, qb + qn - q0);
        STAGE(c, 4, launch_candidates(s, a, q0, n, 0), "candidate count kernel");
        STAGE(c, 5, launch_candidates(s, a, q0, n, 1), "candidate offsets kernel");
        STAGE(c, 6, launch_candidates(s, a, q0, n, 2), "candidate emit kernel");
        STAGE(c, 7, launch_candidates(s, a, q0, n, 3), "candidate reduce kernel");
        STAGE(c, 8, launch_candidates(s, a, q0, n, 4), "refine selection kernel");
    }
    return CHIMERA_OK;
}

// Rotation, LUT and probe of queries [qb, qb + nq) (d_queries is the whole
// batch). The matrix-core probe runs at every batch size (one query at docs2m:
// 0.19 ms against 52 ms for the exact vector kernel, whose 8-row blocks leave
// the GPU idle); its buffers belong to the context, allocated at upload.
int run_front(chimera_ctx* c, const Workspace& w, hipStream_t s, const float* d_queries, int32_t qb, int32_t nq) {
    const size_t q0 = static_cast<size_t>(qb);
    float* rot = w.rot + q0 * kQ * kDim;
    uint32_t* labels = w.labels + q0 * kQ * static_cast<size_t>(c->opt.nprobe);
    STAGE(c, 0, launch_rotate_lut(s, d_queries + q0 * kQ * static_cast<size_t>(c->dim), nq, static_cast<int>(c->dim),
                                  c->flips, static_cast<int>(c->ex_bits), rot, w.cb1 + q0 * kQ,
                                  w.cbex + q0 * kQ, w.lut + q0 * kLutPerQuery),
          "rotation kernel");
    const int nrows = nq * kQ;
    const ProbePlan plan = plan_probe_mfma(nrows, c->n_clusters, c->opt.nprobe, c->num_cus);
    const bool use_mfma = c->probe_mfma_ready && plan.usable && c->probe_mode != 1;
    if (use_mfma) {
        static const char* const what[3] = {"matrix-core probe (sampled pass)", "matrix-core probe (filtered pass)",
                                            "probe rerank"};
        for (int part = 0; part < 3; ++part)
            STAGE(c, 1 + part,
                  launch_probe_mfma(s, plan, rot, nrows, c->cbf, c->cnh, c->centroids, c->norms, c->n_clusters,
                                    c->cmax, c->ecmax, c->opt.nprobe, c->p_gm, c->p_thr, c->p_rval, c->p_rtile, c->p_cnt,
                                    c->p_flag, c->p_ncand, labels, c->p_xfb, part, c->probe_mode == 3),
                  what[part]);
    } else {
        STAGE(c, 2, launch_probe_exact(s, rot, nrows, c->centroids, c->norms, c->n_clusters, c->opt.nprobe, labels),
              "probe kernel");
    }
    return CHIMERA_OK;
}

// One-bit refine, chunked selection, full-bit scoring and top-k of queries
// [qb, qb + nq); d_ids / d_scores / d_counts are the whole batch's outputs.
int run_back(chimera_ctx* c, const Workspace& w, hipStream_t s, int32_t qb, int32_t nq, int32_t k, int64_t* d_ids,
             float* d_scores, int32_t* d_counts) {
    const chimera_search_options& o = c->opt;
    const size_t q0 = static_cast<size_t>(qb);
    const size_t kr = static_cast<size_t>(o.k_refine), fb = static_cast<size_t>(c->fb_cap);
    const float* rot = w.rot + q0 * kQ * kDim;
    const float* cb1 = w.cb1 + q0 * kQ;
    const float* cbex = w.cbex + q0 * kQ;
    const int32_t* rcount = w.rcount + q0;
    const int32_t* rids = w.rids + q0 * kr;
    float* s1 = w.s1 + q0 * kr;
    int32_t* fcount = w.fcount + q0;
    int32_t* fids = w.fids + q0 * fb;
    float* fscores = w.fscores + q0 * fb;
    if (c->exact_scoring) {
        STAGE(c, 9, launch_refine_lut(s, nq, o.k_refine, w.lut + q0 * kLutPerQuery, cb1, rcount, rids, c->doc_ptrs,
                                      c->codes_tok, c->f1_tok, s1),
              "refine kernel");
    } else {
        STAGE(c, 9, launch_refine_mfma(s, nq, o.k_refine, rot, cb1, rcount, rids, c->doc_ptrs, c->codes_tok, c->f1_tok,
                                       s1, c->num_cus),
              "refine kernel");
    }
    STAGE(c, 10, launch_chunk_select(s, nq, s1, rcount, rids, o.k_refine, o.k_full_bit, o.num_chunks, c->fb_cap, fcount,
                                     fids, w.err),
          "full-bit selection kernel");
    if (c->exact_scoring) {
        STAGE(c, 11, launch_fullbit(s, nq, rot, cbex, fcount, fids, c->fb_cap, c->doc_ptrs, c->full_codes,
                                    c->full_factors, static_cast<int>(1 + c->ex_bits), fscores),
              "full-bit kernel");
    } else {
        STAGE(c, 11, launch_fullbit_mfma(s, nq, rot, cbex, fcount, fids, c->fb_cap, c->doc_ptrs, c->full_codes,
                                         c->full_factors, static_cast<int>(1 + c->ex_bits), fscores, c->num_cus),
              "full-bit kernel");
    }
    STAGE(c, 12, launch_final_topk(s, nq, fcount, fids, fscores, c->fb_cap, k, d_ids + q0 * static_cast<size_t>(k),
                                   d_scores ? d_scores + q0 * static_cast<size_t>(k) : nullptr, d_counts + q0),
          "top-k kernel");
    return CHIMERA_OK;
}

int run_pipeline(chimera_ctx* c, const Workspace& w, const float* d_queries, int32_t nq, int32_t k, int64_t* d_ids,
                 float* d_scores, int32_t* d_counts) {
    if (nq == 0) return CHIMERA_OK;
    hipStream_t s = c->stream;
    CK_HIP(launch_fill_u32(s, w.err, 1, 0u), "clearing status");
    CK(run_front(c, w, s, d_queries, 0, nq));
    CK(run_candidates(c, w, s, 0, nq));
    return run_back(c, w, s, 0, nq, k, d_ids, d_scores, d_counts);
}

// Lays out the result region of a host call of nq queries and k results
// (growing it, and the pinned staging buffer to hold it or host_bytes of
// input, when needed).
int ensure_out(chimera_ctx* c, int32_t nq, int32_t k, size_t host_bytes) {
    const size_t m = static_cast<size_t>(nq) * static_cast<size_t>(k);
    const size_t used = m * 12 + static_cast<size_t>(nq) * 4 + 4;
    if (used > c->w_out_bytes) {
        CK_HIP(hipStreamSynchronize(c->stream), "synchronising before output growth");
        // the region lives with the workspace; the old one leaves the list
        if (c->w_out) {
            auto it = std::find(c->ws_allocs.begin(), c->ws_allocs.end(), static_cast<void*>(c->w_out));
            if (it != c->ws_allocs.end()) c->ws_allocs.erase(it);
            (void)hipFree(c->w_out);
            c->bytes -= c->w_out_bytes;
            c->w_out = nullptr;
            c->w_out_bytes = 0;
        }
        const size_t bytes = (used + 255) / 256 * 256;
        CK(dev_alloc(c, c->ws_allocs, &c->w_out, bytes, "search results"));
        c->w_out_bytes = bytes;
    }
    const size_t host = std::max(used, host_bytes);
    if (host > c->h_stage_bytes) {
        CK_HIP(hipStreamSynchronize(c->stream), "synchronising before staging growth");
        if (c->h_stage) (void)hipHostFree(c->h_stage);
        c->h_stage = nullptr;
        c->h_stage_bytes = 0;
        const size_t bytes = (host + 4095) / 4096 * 4096;
        void* p = nullptr;
        CK_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault), "pinned staging buffer");
        c->h_stage = static_cast<unsigned char*>(p);
        c->h_stage_bytes = bytes;
    }
    c->w_out_ids = reinterpret_cast<int64_t*>(c->w_out);
    c->w_out_scores = reinterpret_cast<float*>(c->w_out + m * 8);
    c->w_out_counts = reinterpret_cast<int32_t*>(c->w_out + m * 12);
    c->w_out_status = reinterpret_cast<uint32_t*>(c->w_out + m * 12 + static_cast<size_t>(nq) * 4);
    c->w_out_used = used;
    return CHIMERA_OK;
}


// Search-side state shared by index upload and device build: centroid norms
// bound, matrix-core probe buffers, candidate bounds and the workspace. The
// index arrays, centroid norms and n/dim/n_clusters/ex_bits/num_docs are set.
int finish_setup(chimera_ctx* c, const chimera_search_options& o, int32_t max_batch) {
    c->opt = o;
    c->max_batch = max_batch;
    const chimera_search_options* opt = &c->opt;
    {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device) == hipSuccess && cus > 0)
            c->num_cus = cus;
        std::vector<float> nrm(static_cast<size_t>(c->n_clusters));
        CK_HIP(hipMemcpy(nrm.data(), c->norms, nrm.size() * sizeof(float), hipMemcpyDeviceToHost), "centroid norms");
        float mx = 0.0f;
        for (float v : nrm) mx = std::max(mx, v);
        // the fp32 sum of 128 squares is within 1e-5 of |c|^2
        c->cmax = static_cast<float>(std::sqrt(static_cast<double>(mx)) * (1.0 + 1e-4));
        const ProbePlan plan = plan_probe_mfma(max_batch * kQ, c->n_clusters, opt->nprobe, c->num_cus);
        if (plan.usable) {
            const size_t rows = static_cast<size_t>(max_batch) * kQ;
            CK(dev_alloc(c, c->index_allocs, &c->cbf, static_cast<size_t>(c->n_clusters) * kDim, "bf16 centroids"));
            CK(dev_alloc(c, c->index_allocs, &c->cnh, static_cast<size_t>(c->n_clusters), "probe initial values"));
            CK(dev_alloc(c, c->index_allocs, &c->p_err, 1, "centroid rounding bound"));
            CK_HIP(launch_probe_centroids(c->stream, c->centroids, c->norms, c->n_clusters, c->cbf, c->cnh, c->p_err),
                   "bf16 centroids");
            uint32_t eb = 0;
            CK_HIP(hipMemcpyAsync(&eb, c->p_err, sizeof(eb), hipMemcpyDeviceToHost, c->stream), "centroid rounding bound");
            CK_HIP(hipStreamSynchronize(c->stream), "centroid rounding bound");
            float ef = 0.0f;
            std::memcpy(&ef, &eb, sizeof(ef));
            // the fp32 sum of 128 squares is within 1e-5 of |c - c_b|^2
            c->ecmax = static_cast<float>(static_cast<double>(ef) * (1.0 + 1e-4));
            CK(dev_alloc(c, c->index_allocs, &c->p_gm, static_cast<size_t>(plan.n_sampled) * rows, "probe tile minima"));
            CK(dev_alloc(c, c->index_allocs, &c->p_thr, rows, "probe thresholds"));
            const size_t sub_rows = probe_sublist_rows(max_batch * kQ, c->num_cus);
            const size_t nrec = sub_rows * 2 * static_cast<size_t>(plan.lane_cap);
            CK(dev_alloc(c, c->index_allocs, &c->p_rval, nrec * 8, "probe records"));
            CK(dev_alloc(c, c->index_allocs, &c->p_rtile, nrec, "probe record tiles"));
            CK(dev_alloc(c, c->index_allocs, &c->p_cnt, sub_rows * 2, "probe counts"));
            CK(dev_alloc(c, c->index_allocs, &c->p_flag, rows, "probe flags"));
            CK(dev_alloc(c, c->index_allocs, &c->p_ncand, rows, "probe candidate counts"));
            CK_HIP(launch_fill_u32(c->stream, c->p_ncand, static_cast<int64_t>(rows), 0u), "probe candidate counts");
            c->p_xfb.list_cap = kExactFallbackRows;
            CK(dev_alloc(c, c->index_allocs, &c->p_xfb.list, kExactFallbackRows, "flagged probe rows"));
            CK(dev_alloc(c, c->index_allocs, &c->p_xfb.nflag, 1, "flagged probe row count"));
            CK(dev_alloc(c, c->index_allocs, &c->p_xfb.partial,
                         static_cast<size_t>(kExactFallbackRows) * kExactPartialKeys, "flagged probe row keys"));
            c->probe_mfma_ready = true;
        }
    }

    // Workspace bounds (utils.cu:217-264,299-456): visit records per query
    // <= 32 * (sum of the nprobe largest cluster sizes).
    {
        std::vector<uint64_t> cpos(static_cast<size_t>(c->n_clusters) + 1);
        CK_HIP(hipMemcpy(cpos.data(), c->cluster_pos, cpos.size() * sizeof(uint64_t), hipMemcpyDeviceToHost),
               "cluster positions");
        int64_t bound = 0;
        CK(chimera_visit_bound(cpos.data(), static_cast<uint64_t>(c->n_clusters), opt->nprobe, &bound));
        c->vcap = std::max<int64_t>(1, bound);
    }
    c->nbk = cand_buckets(c->num_docs, c->blog);
    c->fb_cap = fullbit_capacity(*opt);
    const int64_t per_query =
        c->vcap * 8 + static_cast<int64_t>(c->nbk) * (kQ * 4 + 4 + groups_per_bucket(c->blog) * 18) + 16;
    // per-query candidate state for as many queries as half of the free HBM
    // allows (at most 64 GiB): a 1,024-query batch over 2M documents runs as
    // one sub-batch
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) free_b = size_t{8} << 30;
    const int64_t budget = std::max<int64_t>(int64_t{1} << 30, std::min<int64_t>(int64_t{64} << 30,
                                                                                 static_cast<int64_t>(free_b / 2)));
    int qs = static_cast<int>(std::max<int64_t>(8, std::min<int64_t>(budget / std::max<int64_t>(per_query, 1), 4096)));
    qs = qs / 8 * 8;
    const int maxb8 = (max_batch + 7) / 8 * 8;
    c->qs = std::min(qs, maxb8);
    c->qs_cap = c->qs;

    const WorkspaceShape sh{static_cast<size_t>(max_batch), static_cast<size_t>(c->qs), static_cast<size_t>(c->dim),
                            static_cast<size_t>(opt->nprobe), static_cast<size_t>(c->nbk), static_cast<size_t>(c->vcap),
                            static_cast<size_t>(opt->k_refine), static_cast<size_t>(c->fb_cap), true, c->blog};
    unsigned char* block = nullptr;
    CK(dev_alloc(c, c->ws_allocs, &block, carve_workspace(sh, nullptr, nullptr), "search workspace"));
    carve_workspace(sh, block, &c->ws);
    CK_HIP(launch_fill_u32(c->stream, reinterpret_cast<uint32_t*>(c->ws.rcount), max_batch, 0u), "clearing refined counts");
    CK_HIP(launch_fill_u32(c->stream, c->ws.err, 1, 0u), "clearing status");
    CK(dev_alloc(c, c->ws_allocs, &c->noalloc_status, 1, "no-allocation search status"));
    CK_HIP(launch_fill_u32(c->stream, c->noalloc_status, 1, 0u), "clearing status");
    CK_HIP(hipStreamSynchronize(c->stream), "workspace setup");
    c->has_index = true;
    return CHIMERA_OK;
}


// Index build on the device (build_index.cu:394-501 with the CAGRA
// assignment replaced by the exact matrix-core nearest-centroid search).
int build_on_device(chimera_ctx* c, const float* d_emb, uint64_t n_, uint64_t dim_, const int32_t* doc_lens,
                    uint64_t m_, uint64_t k_, uint64_t ex_bits_, const int64_t* centroid_ids,
                    const uint8_t* flips, const chimera_search_options* opt, int32_t max_batch) {
    // validate_build_inputs (build_index.cu:75-126)
    if (dim_ < 64 || dim_ > static_cast<uint64_t>(kDim))
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Embedding dimension must be in [64, 128]");
    if (n_ == 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Embedding storage must contain a non-empty whole number of vectors");
    if (n_ > 0x7FFFFFFFull) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Embedding count exceeds the int32 index format limit");
    if (k_ == 0 || k_ > n_)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "n_clusters must be between 1 and the number of embeddings");
    if (ex_bits_ < 1 || ex_bits_ > 7)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "ex_bits must be in [1, 7] so full codes fit in 2-8 bits per dimension");
    if (m_ == 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "doc_lens must not be empty");
    if (m_ > static_cast<uint64_t>(kMaxDocs))
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "indexes of more than 134,217,728 documents are not supported");
    std::vector<int32_t> ptrs(m_ + 1, 0);
    {
        uint64_t tokens = 0;
        for (uint64_t d = 0; d < m_; ++d) {
            if (doc_lens[d] <= 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Every document length must be positive");
            const uint64_t l = static_cast<uint64_t>(doc_lens[d]);
            if (tokens > n_ || l > n_ - tokens)
                return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Document lengths exceed the number of embeddings");
            tokens += l;
            ptrs[d + 1] = static_cast<int32_t>(tokens);
        }
        if (tokens != n_) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Document lengths do not sum to the number of embeddings");
    }
    for (uint64_t i = 0; i < k_; ++i)
        if (centroid_ids[i] < 0 || static_cast<uint64_t>(centroid_ids[i]) >= n_)
            return fail(CHIMERA_ERR_INVALID_ARGUMENT, "centroid id out of range");
    CK(validate_options(*opt, static_cast<int64_t>(k_)));
    if (max_batch <= 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "max_batch must be positive");
    CK(set_device(c));
    release_index(c);
    const CandShape shape = cand_shape(static_cast<int64_t>(m_), static_cast<int64_t>(n_), static_cast<int64_t>(k_),
                                       opt->nprobe);
    CK_HIP(configure_kernels(cand_buckets(static_cast<int64_t>(m_), shape.blog), opt->nprobe, opt->k_refine,
                             fullbit_capacity(*opt)),
           "configuring kernel LDS limits");
    c->blog = shape.blog;
    c->held = shape.held;
    {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device) == hipSuccess && cus > 0)
            c->num_cus = cus;
    }
    c->n = static_cast<int64_t>(n_);
    c->dim = static_cast<int64_t>(dim_);
    c->n_clusters = static_cast<int64_t>(k_);
    c->ex_bits = static_cast<int64_t>(ex_bits_);
    c->num_docs = static_cast<int64_t>(m_);
    const size_t n = static_cast<size_t>(n_);
    const size_t K = static_cast<size_t>(k_);
    const int dim = static_cast<int>(dim_);
    const int ex_bits = static_cast<int>(ex_bits_);
    const size_t width = static_cast<size_t>(1 + ex_bits);
    hipStream_t s = c->stream;
    TempBuffers tmp;
    tmp.stream = s;

    CK(upload(c, &c->doc_ptrs, ptrs.data(), m_ + 1, "doc_ptrs"));
    CK(upload(c, &c->flips, flips, 4 * kDim / 8, "rotator flips"));
    CK(dev_alloc(c, c->index_allocs, &c->codes_tok, (n + kRefinePadTokens) * kCodeBytes, "token-order codes"));
    CK(dev_alloc(c, c->index_allocs, &c->f1_tok, n + kRefinePadTokens, "token-order factors"));
    CK_HIP(hipMemsetAsync(c->codes_tok + n * kCodeBytes, 0, kRefinePadTokens * kCodeBytes, s), "code padding");
    CK_HIP(hipMemsetAsync(c->f1_tok + n, 0, kRefinePadTokens * sizeof(float), s), "factor padding");
    CK(dev_alloc(c, c->index_allocs, &c->full_codes, (n + kFullbitPadTokens) * 16 * width, "full codes"));
    CK(dev_alloc(c, c->index_allocs, &c->full_factors, n + kFullbitPadTokens, "full factors"));
    CK_HIP(hipMemsetAsync(c->full_codes + n * 16 * width, 0, kFullbitPadTokens * 16 * width, s), "full code padding");
    CK_HIP(hipMemsetAsync(c->full_factors + n, 0, kFullbitPadTokens * sizeof(float), s), "full factor padding");
    uint32_t* status = nullptr;
    CK(tmp.alloc(&status, 1, "build status"));
    CK_HIP(launch_fill_u32(s, status, 1, 0u), "clearing build status");

    // encode every token (build_index.cu:258-303)
    CK_HIP(launch_encode_tokens(s, d_emb, c->n, dim, c->flips, ex_bits, c->num_cus, c->codes_tok, c->f1_tok,
                                c->full_codes, c->full_factors, status),
           "token encoding");

    // rotated centroids (build_index.cu:221-238)
    int64_t* d_ids = nullptr;
    CK(tmp.alloc(&d_ids, K, "centroid ids"));
    CK_HIP(hipMemcpyAsync(d_ids, centroid_ids, K * sizeof(int64_t), hipMemcpyHostToDevice, s), "centroid ids");
    CK(dev_alloc(c, c->index_allocs, &c->centroids, K * kDim, "centroids"));
    CK(dev_alloc(c, c->index_allocs, &c->norms, K, "centroid norms"));
    CK_HIP(launch_gather_rows(s, d_emb, dim, d_ids, c->n_clusters, c->flips, true, c->centroids), "centroid rotation");
    CK_HIP(launch_centroid_norms(s, c->centroids, c->n_clusters, c->norms), "centroid norms");

    // nearest-centroid assignment in the input space (build_index.cu:186-219)
    uint32_t* labels = nullptr;
    CK(tmp.alloc(&labels, n, "assignments"));
    {
        float* cu = nullptr;
        float* nu = nullptr;
        float* nhu = nullptr;
        uint16_t* cbu = nullptr;
        uint32_t* ebu = nullptr;
        CK(tmp.alloc(&cu, K * kDim, "assignment centroids"));
        CK(tmp.alloc(&nu, K, "assignment centroid norms"));
        CK(tmp.alloc(&nhu, K, "assignment probe initial values"));
        CK(tmp.alloc(&cbu, K * kDim, "assignment bf16 centroids"));
        CK(tmp.alloc(&ebu, 1, "assignment centroid rounding bound"));
        CK_HIP(launch_gather_rows(s, d_emb, dim, d_ids, c->n_clusters, nullptr, false, cu), "centroid gather");
        CK_HIP(launch_centroid_norms(s, cu, c->n_clusters, nu), "centroid norms");
        CK_HIP(launch_probe_centroids(s, cu, nu, c->n_clusters, cbu, nhu, ebu), "bf16 centroids");
        std::vector<float> hn(K);
        uint32_t eb = 0;
        CK_HIP(hipMemcpyAsync(hn.data(), nu, K * sizeof(float), hipMemcpyDeviceToHost, s), "centroid norms");
        CK_HIP(hipMemcpyAsync(&eb, ebu, sizeof(eb), hipMemcpyDeviceToHost, s), "centroid rounding bound");
        CK_HIP(hipStreamSynchronize(s), "centroid norms");
        float mx = 0.0f;
        for (float v : hn) mx = std::max(mx, v);
        const float cmax = static_cast<float>(std::sqrt(static_cast<double>(mx)) * (1.0 + 1e-4));
        float ef = 0.0f;
        std::memcpy(&ef, &eb, sizeof(ef));
        const float ecmax = static_cast<float>(static_cast<double>(ef) * (1.0 + 1e-4));
        const int64_t batch = std::min<int64_t>(c->n, int64_t{1} << 20);
        const ProbePlan full_plan = plan_assign_top1(static_cast<int>(batch), c->n_clusters, c->num_cus);
        uint32_t *ukey = nullptr, *cnt = nullptr, *flag = nullptr;
        uint2* buf = nullptr;
        CK(tmp.alloc(&ukey, static_cast<size_t>(batch), "assignment keys"));
        const size_t sub_rows = probe_sublist_rows(static_cast<int>(batch), c->num_cus);
        CK(tmp.alloc(&cnt, sub_rows * 2, "assignment counts"));
        CK(tmp.alloc(&flag, static_cast<size_t>(batch), "assignment flags"));
        CK(tmp.alloc(&buf, sub_rows * 2 * static_cast<size_t>(full_plan.lane_cap), "assignment candidates"));
        ExactFallback xfb;
        xfb.list_cap = kExactFallbackRows;
        CK(tmp.alloc(&xfb.list, static_cast<size_t>(kExactFallbackRows), "flagged assignment rows"));
        CK(tmp.alloc(&xfb.nflag, 1, "flagged assignment row count"));
        CK(tmp.alloc(&xfb.partial, static_cast<size_t>(kExactFallbackRows) * kExactPartialKeys,
                     "flagged assignment keys"));
        float* padded = nullptr;
        if (dim < kDim) CK(tmp.alloc(&padded, static_cast<size_t>(batch) * kDim, "padded rows"));
        for (int64_t start = 0; start < c->n; start += batch) {
            const int nb = static_cast<int>(std::min<int64_t>(batch, c->n - start));
            const float* rows = d_emb + static_cast<size_t>(start) * dim;
            if (dim < kDim) {
                CK_HIP(launch_gather_rows(s, rows, dim, nullptr, nb, nullptr, false, padded), "row padding");
                rows = padded;
            }
            const ProbePlan plan = plan_assign_top1(nb, c->n_clusters, c->num_cus);
            CK_HIP(launch_assign_top1(s, plan, rows, nb, cbu, nhu, cu, nu, c->n_clusters, cmax, ecmax, ukey, buf, cnt,
                                      flag, labels + start, xfb),
                   "centroid assignment");
        }
        CK_HIP(hipStreamSynchronize(s), "centroid assignment");
        for (void* p : {static_cast<void*>(cu), static_cast<void*>(nu), static_cast<void*>(nhu), static_cast<void*>(cbu),
                        static_cast<void*>(ebu), static_cast<void*>(ukey), static_cast<void*>(cnt), static_cast<void*>(flag),
                        static_cast<void*>(buf), static_cast<void*>(padded), static_cast<void*>(xfb.list),
                        static_cast<void*>(xfb.nflag), static_cast<void*>(xfb.partial)})
            if (p) tmp.release(p);
    }

    // IVF lists and the cluster-ordered arrays (ivf_pg.cpp:110-126,
    // build_index.cu:328-363)
    {
        uint32_t *keys_out = nullptr, *vals_in = nullptr, *token_doc_u = nullptr, *runs_d = nullptr;
        CK(tmp.alloc(&keys_out, n, "sorted assignments"));
        CK(tmp.alloc(&vals_in, n, "token ids"));
        CK(dev_alloc(c, c->index_allocs, &c->inv, n, "IVF lists"));
        size_t temp_bytes = 0;
        CK_HIP(launch_sort_assignments(s, labels, c->n, c->n_clusters, keys_out, vals_in, c->inv, nullptr,
                                       &temp_bytes),
               "sort sizing");
        unsigned char* sort_tmp = nullptr;
        CK(tmp.alloc(&sort_tmp, temp_bytes, "sort scratch"));
        CK_HIP(launch_sort_assignments(s, labels, c->n, c->n_clusters, keys_out, vals_in, c->inv, sort_tmp,
                                       &temp_bytes),
               "assignment sort");
        CK(dev_alloc(c, c->index_allocs, &c->cluster_pos, K + 1, "cluster_pos"));
        CK(dev_alloc(c, c->index_allocs, &c->codes_clu, n * kCodeBytes, "clustered codes"));
        CK(dev_alloc(c, c->index_allocs, &c->f1_clu, n, "clustered factors"));
        CK(dev_alloc(c, c->index_allocs, &c->doc_clu, n, "clustered doc ids"));
        CK(tmp.alloc(&token_doc_u, n, "token documents"));
        CK(tmp.alloc(&runs_d, K, "cluster runs"));
        CK_HIP(launch_layout(s, keys_out, c->inv, c->n, c->n_clusters, c->doc_ptrs, c->num_docs, c->codes_tok,
                             c->f1_tok, reinterpret_cast<int32_t*>(token_doc_u), c->cluster_pos, c->codes_clu,
                             c->f1_clu, c->doc_clu, runs_d),
               "index layout");
    }
    uint32_t st = 0;
    CK_HIP(hipMemcpyAsync(&st, status, sizeof(st), hipMemcpyDeviceToHost, s), "build status");
    CK_HIP(hipStreamSynchronize(s), "index build");
    if (st & 1u) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "Every embedding must be finite and non-zero");
    if (st & 2u) return fail(CHIMERA_ERR_RUNTIME, "Full-code rescale search exceeded its event bound");
    return finish_setup(c, *opt, max_batch);
}

}  // namespace

extern "C" {

const char* chimera_last_error(void) { return g_last_error.c_str(); }

int chimera_device_count(void) {
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        fail(CHIMERA_ERR_HIP, std::string("hipGetDeviceCount failed: ") + hipGetErrorString(e));
        return -1;
    }
    return n;
}

int chimera_create(chimera_ctx** out, int device) {
    if (!out) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    int count = 0;
    CK_HIP(hipGetDeviceCount(&count), "Querying HIP devices");
    if (count == 0) return fail(CHIMERA_ERR_RUNTIME, "No HIP device is available");
    if (device < 0 || device >= count) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "device ordinal out of range");
    auto* c = new chimera_ctx();
    c->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail(CHIMERA_ERR_HIP, std::string("creating the HIP stream failed: ") + hipGetErrorString(e));
    }
    // the static workspace's address on this device (once per device)
    unsigned char* sp = nullptr;
    const int r = scratch_address(device, &sp);
    if (r != CHIMERA_OK) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return r;
    }
    *out = c;
    return CHIMERA_OK;
}

void chimera_destroy(chimera_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    release_index(c);
    for (auto& p : c->pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    for (hipEvent_t e : c->pool) (void)hipEventDestroy(e);
    if (c->h_stage) (void)hipHostFree(c->h_stage);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int chimera_memory_usage(chimera_ctx* c, uint64_t* bytes) {
    if (!c || !bytes) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    *bytes = c->bytes;
    return CHIMERA_OK;
}

int chimera_device_memory_info(chimera_ctx* c, uint64_t* free_bytes, uint64_t* total_bytes) {
    if (!c || !free_bytes || !total_bytes) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    size_t f = 0, t = 0;
    CK_HIP(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    *free_bytes = f;
    *total_bytes = t;
    return CHIMERA_OK;
}

int chimera_stream(chimera_ctx* c, void** stream) {
    if (!c || !stream) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    *stream = c->stream;
    return CHIMERA_OK;
}

int chimera_upload_index(chimera_ctx* c, const chimera_index_desc* d, const chimera_search_options* opt,
                         int32_t max_batch) {
    if (!c || !d || !opt) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    release_index(c);
    if (d->num_embeddings == 0 || d->num_embeddings > 0x7FFFFFFFull || d->dimension < 64 || d->dimension > 128 ||
        d->num_clusters == 0 || d->num_clusters > d->num_embeddings || d->ex_bits < 1 || d->ex_bits > 7 ||
        d->num_docs == 0) {
        return fail(CHIMERA_ERR_RUNTIME, "Invalid Chimera index description");
    }
    if (d->num_docs > kMaxDocs)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "indexes of more than 134,217,728 documents are not supported");
    if (!d->doc_ptrs || !d->cluster_pos || !d->clustered_codes || !d->clustered_factors || !d->clustered_doc_ids ||
        !d->token_to_cluster_pos || !d->full_codes || !d->full_factors || !d->rotated_centroids || !d->rotator_flips) {
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "index description has a null array");
    }
    CK(validate_options(*opt, static_cast<int64_t>(d->num_clusters)));
    const CandShape shape = cand_shape(static_cast<int64_t>(d->num_docs), static_cast<int64_t>(d->num_embeddings),
                                       static_cast<int64_t>(d->num_clusters), opt->nprobe);
    CK_HIP(configure_kernels(cand_buckets(static_cast<int64_t>(d->num_docs), shape.blog), opt->nprobe, opt->k_refine,
                             fullbit_capacity(*opt)),
           "configuring kernel LDS limits");
    c->blog = shape.blog;
    c->held = shape.held;
    if (max_batch <= 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "max_batch must be positive");
    if (d->doc_ptrs[0] != 0 || static_cast<uint64_t>(d->doc_ptrs[d->num_docs]) != d->num_embeddings) {
        return fail(CHIMERA_ERR_RUNTIME, "Document lengths do not match the number of indexed embeddings");
    }
    if (d->cluster_pos[0] != 0 || d->cluster_pos[d->num_clusters] != d->num_embeddings) {
        return fail(CHIMERA_ERR_RUNTIME, "Invalid IVF cluster offsets");
    }
    // Every index the kernels follow must stay inside its array.
    for (uint64_t k = 0; k < d->num_clusters; ++k)
        if (d->cluster_pos[k + 1] < d->cluster_pos[k]) return fail(CHIMERA_ERR_RUNTIME, "Invalid IVF cluster offsets");
    for (uint64_t m = 0; m < d->num_docs; ++m)
        if (d->doc_ptrs[m + 1] <= d->doc_ptrs[m]) return fail(CHIMERA_ERR_RUNTIME, "Invalid document lengths in Chimera index");
    for (uint64_t t = 0; t < d->num_embeddings; ++t)
        if (d->token_to_cluster_pos[t] >= d->num_embeddings)
            return fail(CHIMERA_ERR_RUNTIME, "Invalid token-to-cluster position in Chimera index");
    c->n = static_cast<int64_t>(d->num_embeddings);
    c->dim = static_cast<int64_t>(d->dimension);
    c->n_clusters = static_cast<int64_t>(d->num_clusters);
    c->ex_bits = static_cast<int64_t>(d->ex_bits);
    c->num_docs = static_cast<int64_t>(d->num_docs);
    c->opt = *opt;
    c->max_batch = max_batch;
    const size_t n = static_cast<size_t>(c->n);
    const size_t width = static_cast<size_t>(1 + c->ex_bits);

    CK(upload(c, &c->doc_ptrs, d->doc_ptrs, static_cast<size_t>(c->num_docs) + 1, "doc_ptrs"));
    CK(upload(c, &c->cluster_pos, d->cluster_pos, static_cast<size_t>(c->n_clusters) + 1, "cluster_pos"));
    CK(upload(c, &c->codes_clu, d->clustered_codes, n * kCodeBytes, "clustered codes"));
    CK(upload(c, &c->f1_clu, d->clustered_factors, n, "clustered factors"));
    CK(upload(c, &c->doc_clu, d->clustered_doc_ids, n, "clustered doc ids"));
    CK(upload_padded(c, &c->full_codes, d->full_codes, n * 16 * width, kFullbitPadTokens * 16 * width, "full codes"));
    CK(upload_padded(c, &c->full_factors, d->full_factors, n, kFullbitPadTokens, "full factors"));
    CK(upload(c, &c->centroids, d->rotated_centroids, static_cast<size_t>(c->n_clusters) * kDim, "centroids"));
    CK(upload(c, &c->flips, d->rotator_flips, 4 * kDim / 8, "rotator flips"));
    uint32_t* tok2pos = nullptr;
    CK(upload(c, &tok2pos, d->token_to_cluster_pos, n, "token positions"));
    CK(dev_alloc(c, c->index_allocs, &c->codes_tok, (n + kRefinePadTokens) * kCodeBytes, "token-order codes"));
    CK(dev_alloc(c, c->index_allocs, &c->f1_tok, n + kRefinePadTokens, "token-order factors"));
    CK_HIP(hipMemsetAsync(c->codes_tok + n * kCodeBytes, 0, kRefinePadTokens * kCodeBytes, c->stream), "code padding");
    CK_HIP(hipMemsetAsync(c->f1_tok + n, 0, kRefinePadTokens * sizeof(float), c->stream), "factor padding");
    CK(dev_alloc(c, c->index_allocs, &c->norms, static_cast<size_t>(c->n_clusters), "centroid norms"));
    CK_HIP(launch_gather_token_order(c->stream, c->codes_clu, c->f1_clu, tok2pos, c->n, c->codes_tok, c->f1_tok),
           "token-order gather");
    CK_HIP(launch_centroid_norms(c->stream, c->centroids, c->n_clusters, c->norms), "centroid norms");
    CK_HIP(hipStreamSynchronize(c->stream), "index upload");
    {
        auto it = std::find(c->index_allocs.begin(), c->index_allocs.end(), static_cast<void*>(tok2pos));
        c->index_allocs.erase(it);
        c->bytes -= n * sizeof(uint32_t);
        (void)hipFree(tok2pos);
    }
    const int r = finish_setup(c, *opt, max_batch);
    if (r != CHIMERA_OK) {
        // a failed initialisation releases everything (chimera_index.cu:167-172)
        const std::string msg = g_last_error;
        release_index(c);
        g_last_error = msg;
    }
    return r;
}

int chimera_search_device(chimera_ctx* c, const float* d_queries, int32_t nq, int32_t k, int64_t* d_out_ids,
                          float* d_out_scores, int32_t* d_out_counts) {
    CK(check_search_args(c, nq, k));
    if (nq > 0 && (!d_queries || !d_out_ids || !d_out_counts)) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    return run_pipeline(c, c->ws, d_queries, nq, k, d_out_ids, d_out_scores, d_out_counts);
}

int chimera_search_device_noalloc(chimera_ctx* c, const float* d_queries, int32_t nq, int32_t k,
                                  int64_t* d_out_ids, float* d_out_scores, int32_t* d_out_counts) {
    CK(check_search_args(c, nq, k));
    if (nq > 0 && (!d_queries || !d_out_ids || !d_out_counts)) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    if (nq == 0) return CHIMERA_OK;
    // candidate state for one sub-batch: the candidate kernels take any
    // query count, so a small batch reserves records for its own queries only
    const size_t qs = static_cast<size_t>(std::min(nq, c->qs));
    const WorkspaceShape sh{static_cast<size_t>(nq), qs, static_cast<size_t>(c->dim),
                            static_cast<size_t>(c->opt.nprobe), static_cast<size_t>(c->nbk),
                            static_cast<size_t>(c->vcap), static_cast<size_t>(c->opt.k_refine),
                            static_cast<size_t>(c->fb_cap), false, c->blog};
    const size_t need = carve_workspace(sh, nullptr, nullptr);
    if (need > kStaticScratchBytes) {
        // the largest batch that fits, for the message
        int32_t fit = 0;
        for (int32_t b = 1; b < nq; ++b) {
            WorkspaceShape t = sh;
            t.batch = static_cast<size_t>(b);
            t.qs = static_cast<size_t>(std::min(b, c->qs));
            if (carve_workspace(t, nullptr, nullptr) > kStaticScratchBytes) break;
            fit = b;
        }
        return fail(CHIMERA_ERR_CAPACITY, "a batch of " + std::to_string(nq) + " queries needs " + std::to_string(need) +
                                              " bytes of workspace; the static workspace holds " +
                                              std::to_string(kStaticScratchBytes) + " (at most " + std::to_string(fit) +
                                              " queries of this index)");
    }
    unsigned char* base = nullptr;
    CK(scratch_address(c->device, &base));
    Workspace w;
    carve_workspace(sh, base, &w);
    // no events either: stage timing is off for this call
    const bool prof = c->profiling;
    c->profiling = false;
    int r = CHIMERA_OK;
    const hipError_t e = launch_fill_u32(c->stream, reinterpret_cast<uint32_t*>(w.rcount), nq, 0u);
    if (e != hipSuccess) r = fail(CHIMERA_ERR_HIP, std::string("clearing refined counts failed: ") + hipGetErrorString(e));
    if (r == CHIMERA_OK) r = run_pipeline(c, w, d_queries, nq, k, d_out_ids, d_out_scores, d_out_counts);
    // the status word moves out of the shared array into the context's own
    // word, so a later call on another context cannot overwrite it before
    // chimera_synchronize reads it
    if (r == CHIMERA_OK) {
        const hipError_t ce = launch_copy_u32(c->stream, c->noalloc_status, w.err, 1);
        if (ce != hipSuccess) r = fail(CHIMERA_ERR_HIP, std::string("status copy failed: ") + hipGetErrorString(ce));
    }
    c->profiling = prof;
    if (r == CHIMERA_OK) c->noalloc_pending = true;
    return r;
}

int chimera_synchronize(chimera_ctx* c) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    CK(set_device(c));
    CK_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->has_index) CK(check_errors(c, c->ws.err));
    if (c->noalloc_pending) {
        c->noalloc_pending = false;
        CK(check_errors(c, c->noalloc_status));
    }
    return CHIMERA_OK;
}

int chimera_search(chimera_ctx* c, const float* queries, int32_t nq, int32_t k, int64_t* out_ids, float* out_scores,
                   int32_t* out_counts) {
    CK(check_search_args(c, nq, k));
    if (nq == 0) return CHIMERA_OK;
    if (!queries || !out_ids || !out_counts) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    const size_t qbytes = static_cast<size_t>(nq) * kQ * static_cast<size_t>(c->dim) * sizeof(float);
    CK(ensure_out(c, nq, k, qbytes));
    // the batch goes up, and the results and status word come back, through
    // the pinned staging buffer: one DMA copy each way
    std::memcpy(c->h_stage, queries, qbytes);
    CK_HIP(hipMemcpyAsync(c->ws.queries, c->h_stage, qbytes, hipMemcpyHostToDevice, c->stream), "query upload");
    CK(run_pipeline(c, c->ws, c->ws.queries, nq, k, c->w_out_ids, c->w_out_scores, c->w_out_counts));
    CK_HIP(launch_copy_u32(c->stream, c->w_out_status, c->ws.err, 1), "search status");
    CK_HIP(hipMemcpyAsync(c->h_stage, c->w_out, c->w_out_used, hipMemcpyDeviceToHost, c->stream), "result copy");
    CK_HIP(hipStreamSynchronize(c->stream), "search");
    const size_t m = static_cast<size_t>(nq) * k;
    std::memcpy(out_ids, c->h_stage, m * sizeof(int64_t));
    if (out_scores) std::memcpy(out_scores, c->h_stage + m * 8, m * sizeof(float));
    std::memcpy(out_counts, c->h_stage + m * 12, static_cast<size_t>(nq) * sizeof(int32_t));
    uint32_t err = 0;
    std::memcpy(&err, c->h_stage + m * 12 + static_cast<size_t>(nq) * 4, sizeof(err));
    return status_errors(c, err);
}

int chimera_search_trace(chimera_ctx* c, const float* queries, int32_t nq, int32_t k, int64_t* out_ids,
                         float* out_scores, int32_t* out_counts, chimera_trace* tr) {
    CK(check_search_args(c, nq, k));
    if (nq == 0) return CHIMERA_OK;
    if (!queries || !out_ids || !out_counts || !tr) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    hipStream_t s = c->stream;
    const size_t qbytes = static_cast<size_t>(nq) * kQ * static_cast<size_t>(c->dim) * sizeof(float);
    CK(ensure_out(c, nq, k, 0));
    const Workspace& w = c->ws;
    CK_HIP(hipMemcpyAsync(w.queries, queries, qbytes, hipMemcpyHostToDevice, s), "query upload");
    CK_HIP(launch_fill_u32(s, w.err, 1, 0u), "clearing status");
    CK(run_front(c, w, s, w.queries, 0, nq));
    const size_t NQ = static_cast<size_t>(nq);
    auto d2h = [&](void* dst, const void* src, size_t bytes) -> int {
        if (dst && bytes) CK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "trace copy");
        return CHIMERA_OK;
    };
    CK(d2h(tr->rotated, w.rot, NQ * kQ * kDim * 4));
    CK(d2h(tr->cb1_sumq, w.cb1, NQ * kQ * 4));
    CK(d2h(tr->cbex_sumq, w.cbex, NQ * kQ * 4));
    CK(d2h(tr->labels, w.labels, NQ * kQ * static_cast<size_t>(c->opt.nprobe) * 4));
    std::vector<int32_t> counts(static_cast<size_t>(c->qs));
    // dense candidate lists of a sub-batch, compacted on the device
    const int64_t tcap = std::max<int64_t>(1, std::min<int64_t>(tr->cand_capacity, c->num_docs));
    TempBuffers tmp;
    tmp.stream = s;
    int32_t* d_cand = nullptr;
    float* d_score = nullptr;
    if (tr->candidates || tr->candidate_scores) {
        CK(tmp.alloc(&d_cand, static_cast<size_t>(c->qs) * static_cast<size_t>(tcap), "trace candidates"));
        CK(tmp.alloc(&d_score, static_cast<size_t>(c->qs) * static_cast<size_t>(tcap), "trace candidate scores"));
    }
    for (int qb = 0; qb < nq; qb += c->qs) {
        const int qn = std::min(c->qs, nq - qb);
        CK(run_candidates(c, w, s, qb, qn));
        if (d_cand) CK_HIP(launch_cand_compact(s, candidate_args(c, w), qn, tcap, d_cand, d_score), "candidate compaction");
        CK_HIP(hipMemcpyAsync(counts.data(), w.ccount, static_cast<size_t>(qn) * 4, hipMemcpyDeviceToHost, s),
               "trace copy");
        CK_HIP(hipStreamSynchronize(s), "trace");
        for (int j = 0; j < qn; ++j) {
            const int q = qb + j;
            if (tr->candidate_count) tr->candidate_count[q] = counts[static_cast<size_t>(j)];
            const int64_t m = std::min<int64_t>({counts[static_cast<size_t>(j)], tr->cand_capacity, tcap});
            if (m > 0 && d_cand) {
                CK(d2h(tr->candidates ? tr->candidates + static_cast<size_t>(q) * tr->cand_capacity : nullptr,
                       d_cand + static_cast<size_t>(j) * tcap, static_cast<size_t>(m) * 4));
                CK(d2h(tr->candidate_scores ? tr->candidate_scores + static_cast<size_t>(q) * tr->cand_capacity : nullptr,
                       d_score + static_cast<size_t>(j) * tcap, static_cast<size_t>(m) * 4));
            }
        }
        CK_HIP(hipStreamSynchronize(s), "trace");
    }
    CK(run_back(c, w, s, 0, nq, k, c->w_out_ids, c->w_out_scores, w.out_counts));
    const size_t kr = static_cast<size_t>(c->opt.k_refine);
    CK(d2h(tr->refined_count, w.rcount, NQ * 4));
    CK(d2h(tr->refined_ids, w.rids, NQ * kr * 4));
    CK(d2h(tr->refined_scores, w.s1, NQ * kr * 4));
    CK(d2h(tr->fullbit_count, w.fcount, NQ * 4));
    if (tr->fullbit_ids || tr->fullbit_scores) {
        const size_t fc = static_cast<size_t>(c->fb_cap);
        std::vector<int32_t> ids(NQ * fc);
        std::vector<float> sc(NQ * fc);
        CK(d2h(ids.data(), w.fids, NQ * fc * 4));
        CK(d2h(sc.data(), w.fscores, NQ * fc * 4));
        CK_HIP(hipStreamSynchronize(s), "trace");
        const size_t cap = static_cast<size_t>(std::max<int64_t>(0, tr->fullbit_capacity));
        for (size_t q = 0; q < NQ; ++q)
            for (size_t j = 0; j < std::min(cap, fc); ++j) {
                if (tr->fullbit_ids) tr->fullbit_ids[q * cap + j] = ids[q * fc + j];
                if (tr->fullbit_scores) tr->fullbit_scores[q * cap + j] = sc[q * fc + j];
            }
    }
    const size_t m = NQ * static_cast<size_t>(k);
    CK(d2h(out_ids, c->w_out_ids, m * 8));
    CK(d2h(out_scores, c->w_out_scores, m * 4));
    CK(d2h(out_counts, w.out_counts, NQ * 4));
    CK_HIP(hipStreamSynchronize(s), "trace");
    return check_errors(c, w.err);
}

int chimera_graph_capture(chimera_ctx* c, const float* d_queries, int32_t nq, int32_t k, int64_t* d_out_ids,
                          float* d_out_scores, int32_t* d_out_counts) {
    CK(check_search_args(c, nq, k));
    CK(set_device(c));
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->graph_exec = nullptr;
    c->graph = nullptr;
    CK_HIP(hipStreamSynchronize(c->stream), "pre-capture sync");
    CK_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    c->capturing = true;
    const int r = run_pipeline(c, c->ws, d_queries, nq, k, d_out_ids, d_out_scores, d_out_counts);
    c->capturing = false;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (r != CHIMERA_OK) {
        if (g) (void)hipGraphDestroy(g);
        return r;
    }
    CK_HIP(e, "hipStreamEndCapture");
    c->graph = g;
    CK_HIP(hipGraphInstantiate(&c->graph_exec, c->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    return CHIMERA_OK;
}

int chimera_graph_launch(chimera_ctx* c) {
    if (!c || !c->graph_exec) return fail(CHIMERA_ERR_RUNTIME, "no captured search graph");
    CK(set_device(c));
    CK_HIP(hipGraphLaunch(c->graph_exec, c->stream), "hipGraphLaunch");
    return CHIMERA_OK;
}

int chimera_set_probe_mode(chimera_ctx* c, int mode) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    if (mode < 0 || mode > 3) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "probe mode must be 0, 1, 2 or 3");
    c->probe_mode = mode;
    return CHIMERA_OK;
}

int chimera_set_candidate_batch(chimera_ctx* c, int32_t queries) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    if (!c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot size the candidate batch of an empty Chimera index");
    int qs = queries <= 0 ? c->qs_cap : std::min(c->qs_cap, std::max(8, queries / 8 * 8));
    c->qs = qs;
    return CHIMERA_OK;
}

int chimera_set_exact_scoring(chimera_ctx* c, int mode) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    if (mode != 0 && mode != 1) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "scoring mode must be 0 or 1");
    c->exact_scoring = mode == 1;
    return CHIMERA_OK;
}

int chimera_device_alloc(chimera_ctx* c, void** ptr, size_t bytes) {
    if (!c || !ptr) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    *ptr = nullptr;
    CK_HIP(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
    return CHIMERA_OK;
}

int chimera_device_free(chimera_ctx* c, void* ptr) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    CK(set_device(c));
    if (ptr) CK_HIP(hipFree(ptr), "hipFree");
    return CHIMERA_OK;
}

int chimera_copy_to_device(chimera_ctx* c, void* dst, const void* src, size_t bytes) {
    if (!c || (!dst && bytes) || (!src && bytes)) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    if (bytes) CK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "copy to device");
    CK_HIP(hipStreamSynchronize(c->stream), "copy to device");
    return CHIMERA_OK;
}

int chimera_copy_to_host(chimera_ctx* c, void* dst, const void* src, size_t bytes) {
    if (!c || (!dst && bytes) || (!src && bytes)) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    if (bytes) CK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "copy to host");
    CK_HIP(hipStreamSynchronize(c->stream), "copy to host");
    return CHIMERA_OK;
}

int chimera_set_profiling(chimera_ctx* c, int enable) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    CK(set_device(c));
    CK(collect_stage_times(c));
    c->profiling = enable != 0;
    for (int i = 0; i < CHIMERA_STAGES; ++i) {
        c->stage_ms[i] = 0.0;
        c->stage_n[i] = 0;
    }
    return CHIMERA_OK;
}

int chimera_stage_times(chimera_ctx* c, double* ms, int64_t* launches) {
    if (!c || !ms || !launches) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    CK(set_device(c));
    CK(collect_stage_times(c));
    for (int i = 0; i < CHIMERA_STAGES; ++i) {
        ms[i] = c->stage_ms[i];
        launches[i] = c->stage_n[i];
    }
    return CHIMERA_OK;
}

int chimera_graph_time(chimera_ctx* c, int32_t iters, float* ms) {
    if (!c || !ms) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    if (!c->graph_exec) return fail(CHIMERA_ERR_RUNTIME, "no captured search graph");
    if (iters <= 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "iters must be positive");
    CK(set_device(c));
    hipEvent_t a = nullptr, b = nullptr;
    CK_HIP(hipEventCreate(&a), "hipEventCreate");
    CK_HIP(hipEventCreate(&b), "hipEventCreate");
    hipError_t e = hipEventRecord(a, c->stream);
    for (int32_t i = 0; i < iters && e == hipSuccess; ++i) e = hipGraphLaunch(c->graph_exec, c->stream);
    if (e == hipSuccess) e = hipEventRecord(b, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    CK_HIP(e, "timed graph replay");
    return check_errors(c, c->ws.err);
}

int chimera_rotate_lut_device(chimera_ctx* c, const float* d_queries, int32_t nq, float* d_rotated, float* d_cb1,
                              float* d_cbex, float* d_lut) {
    if (!c || !c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot search an empty Chimera index");
    if (nq < 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nq must be non-negative");
    if (nq == 0) return CHIMERA_OK;
    CK(set_device(c));
    CK_HIP(launch_rotate_lut(c->stream, d_queries, nq, static_cast<int>(c->dim), c->flips,
                             static_cast<int>(c->ex_bits), d_rotated, d_cb1, d_cbex, d_lut),
           "rotation kernel");
    return CHIMERA_OK;
}

int chimera_probe_device(chimera_ctx* c, const float* d_rotated, int32_t nrows, int32_t nprobe, uint32_t* d_labels) {
    if (!c || !c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot search an empty Chimera index");
    if (nprobe <= 0 || nprobe > c->n_clusters || nprobe > 2048)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nprobe must be in [1, min(n_clusters, 2048)]");
    if (nrows < 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nrows must be non-negative");
    if (nrows == 0) return CHIMERA_OK;
    CK(set_device(c));
    const ProbePlan plan = plan_probe_mfma(nrows, c->n_clusters, nprobe, c->num_cus);
    const bool fits = static_cast<int64_t>(nrows) <= static_cast<int64_t>(c->max_batch) * kQ && nprobe == c->opt.nprobe;
    if (c->probe_mfma_ready && plan.usable && fits && c->probe_mode != 1) {
        for (int part = 0; part < 3; ++part)
            STAGE(c, 1 + part,
                  launch_probe_mfma(c->stream, plan, d_rotated, nrows, c->cbf, c->cnh, c->centroids, c->norms,
                                    c->n_clusters, c->cmax, c->ecmax, nprobe, c->p_gm, c->p_thr, c->p_rval, c->p_rtile,
                                    c->p_cnt, c->p_flag, c->p_ncand, d_labels, c->p_xfb, part, c->probe_mode == 3),
                  "matrix-core probe");
    } else {
        STAGE(c, 2, launch_probe_exact(c->stream, d_rotated, nrows, c->centroids, c->norms, c->n_clusters, nprobe,
                                       d_labels),
              "probe kernel");
    }
    return CHIMERA_OK;
}

float chimera_probe_margin(float qn, float eq, float cmax, float ecmax) { return probe_delta(qn, eq, cmax, ecmax); }

int chimera_visit_bound(const uint64_t* cluster_pos, uint64_t n_clusters, int32_t nprobe, int64_t* visits) {
    if (!cluster_pos || !visits) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    if (nprobe <= 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nprobe must be positive");
    try {
        // the nprobe largest cluster sizes in a min-heap of at most nprobe
        const size_t np = static_cast<size_t>(std::min<uint64_t>(n_clusters, static_cast<uint64_t>(nprobe)));
        std::vector<uint64_t> heap;
        heap.reserve(np);
        for (uint64_t k = 0; k < n_clusters; ++k) {
            if (cluster_pos[k + 1] < cluster_pos[k]) return fail(CHIMERA_ERR_RUNTIME, "Invalid IVF cluster offsets");
            const uint64_t size = cluster_pos[k + 1] - cluster_pos[k];
            if (heap.size() < np) {
                heap.push_back(size);
                std::push_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
            } else if (np > 0 && size > heap.front()) {
                std::pop_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
                heap.back() = size;
                std::push_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
            }
        }
        uint64_t top = 0;
        for (uint64_t v : heap) top += v;
        // per-query visit offsets are scanned and stored as 32-bit integers
        if (top > static_cast<uint64_t>(INT32_MAX) / kQ)
            return fail(CHIMERA_ERR_CAPACITY, "The " + std::to_string(np) + " largest IVF clusters hold " +
                                                  std::to_string(top) +
                                                  " tokens: a query's candidate visits would exceed the 32-bit "
                                                  "workspace offsets; lower nprobe or use more clusters");
        *visits = static_cast<int64_t>(top) * kQ;
        return CHIMERA_OK;
    } catch (const std::exception& ex) {
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, std::string("visit bound: ") + ex.what());
    }
}

int chimera_probe_bounds(chimera_ctx* c, float* cmax, float* ecmax) {
    if (!c || !cmax || !ecmax) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    if (!c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot search an empty Chimera index");
    *cmax = c->cmax;
    *ecmax = c->probe_mfma_ready ? c->ecmax : 0.0f;
    return CHIMERA_OK;
}

int chimera_probe_stats(chimera_ctx* c, int32_t nrows, uint32_t* candidates) {
    if (!c || !candidates) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    if (!c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot search an empty Chimera index");
    if (!c->probe_mfma_ready) return fail(CHIMERA_ERR_RUNTIME, "the matrix-core probe is not set up for this index");
    if (nrows < 0 || static_cast<int64_t>(nrows) > static_cast<int64_t>(c->max_batch) * kQ)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "nrows exceeds the probe workspace");
    CK(set_device(c));
    if (nrows > 0)
        CK_HIP(hipMemcpyAsync(candidates, c->p_ncand, static_cast<size_t>(nrows) * sizeof(uint32_t),
                              hipMemcpyDeviceToHost, c->stream),
               "probe statistics");
    CK_HIP(hipStreamSynchronize(c->stream), "probe statistics");
    return CHIMERA_OK;
}

int chimera_unpack_codes_device(chimera_ctx* c, int32_t width, const uint8_t* d_packed, int64_t n, uint8_t* d_raw) {
    if (!c) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null context");
    if (width < 1 || width > 8) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "width must be in [1, 8]");
    if (n < 0) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "n must be non-negative");
    CK(set_device(c));
    CK_HIP(launch_unpack_codes(c->stream, width, d_packed, n, d_raw), "unpack kernel");
    return CHIMERA_OK;
}

int chimera_build_index_device(chimera_ctx* c, const float* d_embeddings, uint64_t num_embeddings,
                               uint64_t dimension, const int32_t* doc_lens, uint64_t num_docs, uint64_t num_clusters,
                               uint64_t ex_bits, const int64_t* centroid_ids, const uint8_t* rotator_flips,
                               const chimera_search_options* opt, int32_t max_batch) {
    if (!c || !d_embeddings || !doc_lens || !centroid_ids || !rotator_flips || !opt)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    const int r = build_on_device(c, d_embeddings, num_embeddings, dimension, doc_lens, num_docs, num_clusters, ex_bits,
                                  centroid_ids, rotator_flips, opt, max_batch);
    if (r != CHIMERA_OK) {
        const std::string msg = g_last_error;
        (void)set_device(c);
        release_index(c);
        g_last_error = msg;
    }
    return r;
}

int chimera_download_index(chimera_ctx* c, chimera_index_host* h) {
    if (!c || !h) return fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    if (!c->has_index) return fail(CHIMERA_ERR_RUNTIME, "Cannot download an empty Chimera index");
    if ((h->inv_list || h->token_to_cluster_pos) && !c->inv)
        return fail(CHIMERA_ERR_INVALID_ARGUMENT, "IVF lists are kept only for indexes built on the device");
    CK(set_device(c));
    const size_t n = static_cast<size_t>(c->n);
    const size_t K = static_cast<size_t>(c->n_clusters);
    const size_t width = static_cast<size_t>(1 + c->ex_bits);
    auto get = [&](void* dst, const void* src, size_t bytes, const char* what) -> int {
        if (!dst) return CHIMERA_OK;
        CK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), what);
        return CHIMERA_OK;
    };
    CK(get(h->cluster_pos, c->cluster_pos, (K + 1) * sizeof(uint64_t), "cluster_pos download"));
    CK(get(h->one_bit_codes, c->codes_tok, n * kCodeBytes, "one-bit codes download"));
    CK(get(h->one_bit_factors, c->f1_tok, n * sizeof(float), "one-bit factors download"));
    CK(get(h->full_codes, c->full_codes, n * 16 * width, "full codes download"));
    CK(get(h->full_factors, c->full_factors, n * sizeof(float), "full factors download"));
    CK(get(h->clustered_codes, c->codes_clu, n * kCodeBytes, "clustered codes download"));
    CK(get(h->clustered_factors, c->f1_clu, n * sizeof(float), "clustered factors download"));
    CK(get(h->clustered_doc_ids, c->doc_clu, n * sizeof(int32_t), "clustered doc ids download"));
    CK(get(h->rotated_centroids, c->centroids, K * kDim * sizeof(float), "centroid download"));
    if (h->inv_list || h->token_to_cluster_pos) {
        std::vector<uint32_t> local;
        uint32_t* inv = h->inv_list;
        if (!inv) {
            local.resize(n);
            inv = local.data();
        }
        CK(get(inv, c->inv, n * sizeof(uint32_t), "IVF list download"));
        if (h->token_to_cluster_pos)
            for (size_t p = 0; p < n; ++p) h->token_to_cluster_pos[inv[p]] = static_cast<uint32_t>(p);
    }
    return CHIMERA_OK;
}

}  // extern "C"
