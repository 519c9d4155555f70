// relm_mp_ops.so - torch.library binding of the relational message-passing ops.
//
// Registers TORCH_LIBRARY(relm_mp) with the reference's schema strings
// (maichmueller/relmo src/_ops/mp/mp_ops.cpp:3754-3838) and the same
// CompositeImplicitAutograd dispatch key (mp_ops.cpp:3840-3848).  Each op
// validates its arguments with the reference's messages, then:
//   * GPU tensors (float32 / float64): the HIP kernels of librelm_mp_hip.so,
//     called through its C ABI (include/relm_mp.h) on the current stream;
//   * CPU tensors (float32 / float64): sequential per-edge loops with the
//     reference CPU lane's semantics (mp_ops.cpp:2815-2911) and its ATen
//     logsumexp sequences (mp_ops.cpp:2981-3036);
//   * other dtypes: the reference's ATen index_select / index_add_ sequences
//     (mp_ops.cpp:2913-3003).
// GPU tensors never take the CPU lane.
#include <ATen/ATen.h>
#include <ATen/hip/HIPContext.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <c10/util/intrusive_ptr.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <torch/custom_class.h>
#include <torch/library.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "relm_mp.h"

#ifndef RELM_MP_BUILD_TORCH_VERSION
#define RELM_MP_BUILD_TORCH_VERSION "unknown"
#endif

namespace relm_amd {

using at::Tensor;

constexpr int64_t kModeSum = 0;
constexpr int64_t kModeLogSumExp = 1;

// ---- validation (mp_ops.cpp:28-72) ----------------------------------------

bool is_fastpath_dtype(at::ScalarType dtype) {
    return dtype == at::kFloat || dtype == at::kDouble;
}

void check_rank(const Tensor& t, int64_t expected, const char* name) {
    TORCH_CHECK(t.dim() == expected, name, " must be rank ", expected, ", got rank ", t.dim(), ".");
}

void check_int64_index(const Tensor& t, const char* name) {
    check_rank(t, 1, name);
    TORCH_CHECK(t.scalar_type() == at::kLong, name, " must have dtype torch.int64.");
}

void check_in_bounds(int64_t idx, int64_t size, const char* name) {
    TORCH_CHECK(idx >= 0 && idx < size, name, " index out of bounds: ", idx, " not in [0, ", size,
                ").");
}

Tensor contiguous(const Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

bool all_gpu(std::initializer_list<const Tensor*> ts) {
    for (const Tensor* t : ts)
        if (!t->is_cuda()) return false;
    return true;
}

bool all_cpu(std::initializer_list<const Tensor*> ts) {
    for (const Tensor* t : ts)
        if (!t->is_cpu()) return false;
    return true;
}

void check_same_gpu(const Tensor& a, const Tensor& b, const char* an, const char* bn) {
    TORCH_CHECK(a.get_device() == b.get_device(), an, " and ", bn,
                " must be on the same CUDA device.");
}

int dtype_code(const Tensor& t) { return t.scalar_type() == at::kDouble ? RELM_MP_F64 : RELM_MP_F32; }

void raise_if(int rc) {
    if (rc == RELM_MP_OK) return;
    const std::string msg = relm_mp_last_error();
    if (rc == RELM_MP_ERR_UNSUPPORTED_MODE) throw std::invalid_argument(msg);
    TORCH_CHECK(false, msg);
}

hipStream_t current_stream(const Tensor& t) {
    return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

Tensor byte_buffer(size_t bytes, const Tensor& like) {
    return at::empty({static_cast<int64_t>(bytes == 0 ? 1 : bytes)},
                     like.options().dtype(at::kByte));
}

// ---- index plans and their cache ---------------------------------------------
//
// A plan (relm_mp.h) lives in a byte tensor on the device together with a
// snapshot of the indices it was built from.  PlanRef holds it with the
// stream that built it, so that work on another stream can wait for the plan.
//
// The cache keeps recent plans.  A plan is served to a later call only when
// that call's index arrays equal the plan's snapshot: one device pass compares
// them with up to RELM_MP_MAX_MATCH candidates of the same role, device,
// length and bounds, so an index tensor written after the build - in place,
// through .data, through a raw pointer - leads to a new plan, never to a stale
// one.  Candidates last used with the same tensor objects are compared first.
// The autograd functions of the facade hand a forward's plan to its backward
// directly (fanin_reduce_planned and the *_planned backward ops).
// RELM_MP_PLAN_CACHE=0 disables the cache; RELM_MP_PLAN_CACHE=identity
// compares only with plans last used with the same tensor objects;
// RELM_MP_PLAN_CACHE_MB bounds the plan memory the cache keeps (default 2048).

enum PlanRole : int {
    kRoleInverse = 1,
    kRoleCsr = 2,
    kRoleCsrRows = 3,  // CSR plan whose gathered rows are the edges themselves
};

void check_hip(hipError_t e, const char* what) {
    TORCH_CHECK(e == hipSuccess, "relm_mp: ", what, ": ", hipGetErrorString(e));
}

struct PlanRef : torch::CustomClassHolder {
    relm_mp_plan plan{};
    Tensor mem;
    int role = 0;
    int device = -1;
    int64_t key_bound = 0;
    int64_t gather_bound = 0;
    hipStream_t stream = nullptr;  // the stream the plan was built on
    // CSR plans of a fanin forward: the inverse map of their gathered indices
    // (flat_src), built by the first backward that needs it
    // (relm_mp_plan_fanin_backward_by_src) and kept for later backward calls
    // on the same stream with the same row count; inv_rows < 0: none.
    // inv_collide_rows: the row count for which flat_src was found not to be
    // injective (the plan's indices do not change, so neither does that
    // answer); later backward calls go straight to the inverse plan.
    std::mutex inv_mu;
    Tensor inv_mem;
    int64_t inv_rows = -1;
    hipStream_t inv_stream = nullptr;
    int64_t inv_collide_rows = -1;

    PlanRef() = default;
    PlanRef(const PlanRef&) = delete;
    PlanRef& operator=(const PlanRef&) = delete;

    bool defined() const { return plan.kind != 0; }

    // Work enqueued on `s` from now on waits for the build, and the plan
    // memory is not handed out again before that work has finished.  The
    // wait is on an event recorded on the build stream now, behind the
    // build and whatever followed it there (no event is recorded at build
    // time: a marker between the build and its own stream's next kernel
    // would stall that stream).
    void use_on(hipStream_t s) const {
        if (s == stream || !mem.defined()) return;
        hipEvent_t ev = nullptr;
        check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "plan event");
        hipError_t err = hipEventRecord(ev, stream);
        if (err == hipSuccess) err = hipStreamWaitEvent(s, ev, 0);
        (void)hipEventDestroy(ev);  // released once the wait has been resolved
        if (err != hipSuccess) {
            // the build stream is gone: everything it ran has finished
            (void)hipGetLastError();
            check_hip(hipDeviceSynchronize(), "plan stream sync");
        }
        c10::hip::HIPCachingAllocator::recordStream(
            mem.storage().data_ptr(), c10::hip::getStreamFromExternal(s, device));
    }
};

using PlanPtr = c10::intrusive_ptr<PlanRef>;

class PlanCache {
   public:
    static PlanCache& get() {
        static PlanCache cache;
        return cache;
    }

    bool enabled() const { return enabled_; }

    // A cached plan of `role` built from indices equal to (key, gather) under
    // the same bounds (gather_bound < 0: any gather bound), ready for use on
    // `s`; null if there is none.  gather null: only the keys are compared.
    PlanPtr lookup(int role, const Tensor& key, const Tensor* gather, int64_t key_bound,
                   int64_t gather_bound, hipStream_t s) {
        if (!enabled_) return PlanPtr();
        if (PlanPtr t = trusted(role, key, gather, key_bound, gather_bound)) {
            t->use_on(s);
            return t;
        }
        struct Cand {
            PlanPtr ref;
            bool same;
            uint64_t stamp;
        };
        std::vector<Cand> cand;
        {
            std::lock_guard<std::mutex> lock(mu_);
            for (const Entry& e : entries_) {
                const PlanRef& r = *e.ref;
                if (r.role != role || r.device != key.get_device() ||
                    r.plan.num_edges != key.numel() || r.key_bound != key_bound ||
                    (gather_bound >= 0 && r.gather_bound != gather_bound))
                    continue;
                const bool same = e.key_impl == key.unsafeGetTensorImpl() &&
                                  e.key_ver == version(key) &&
                                  (gather == nullptr ||
                                   (e.gather_impl == gather->unsafeGetTensorImpl() &&
                                    e.gather_ver == version(*gather)));
                if (identity_only_ && !same) continue;
                cand.push_back({e.ref, same, e.stamp});
            }
            if (cand.empty()) {
                ++misses_;
                return PlanPtr();
            }
        }
        std::sort(cand.begin(), cand.end(), [](const Cand& a, const Cand& b) {
            return a.same != b.same ? a.same : a.stamp > b.stamp;
        });
        if (cand.size() > RELM_MP_MAX_MATCH) cand.resize(RELM_MP_MAX_MATCH);
        std::vector<const relm_mp_plan*> plans;
        for (const Cand& c : cand) {
            c.ref->use_on(s);  // the comparison reads the snapshot the build wrote
            plans.push_back(&c.ref->plan);
        }
        std::vector<int32_t> match(cand.size(), 0);
        Tensor ws = byte_buffer(relm_mp_plan_match_workspace_size(), key);
        raise_if(relm_mp_plan_match(key.data_ptr<int64_t>(),
                                    gather != nullptr ? gather->data_ptr<int64_t>() : nullptr,
                                    key.numel(), plans.data(), static_cast<int32_t>(plans.size()),
                                    match.data(), ws.data_ptr(), static_cast<size_t>(ws.numel()), s));
        std::lock_guard<std::mutex> lock(mu_);
        for (size_t j = 0; j < cand.size(); ++j) {
            if (!match[j]) continue;
            for (Entry& e : entries_) {
                if (e.ref.get() != cand[j].ref.get()) continue;
                e.stamp = ++clock_;
                note_tensors(e, key, gather);
            }
            ++(cand[j].same ? same_hits_ : other_hits_);
            remember(cand[j].ref, key, gather);
            return cand[j].ref;
        }
        ++misses_;
        return PlanPtr();
    }

    // Keeps `ref` (a completed build of `key` / `gather`), evicting the least
    // recently used plans beyond the memory bound.
    void insert(const PlanPtr& ref, const Tensor& key, const Tensor* gather) {
        if (!enabled_) return;
        const size_t bytes = static_cast<size_t>(ref->mem.numel());
        if (bytes > limit_) return;
        std::lock_guard<std::mutex> lock(mu_);
        remember(ref, key, gather);
        Entry e;
        e.ref = ref;
        e.bytes = bytes;
        e.stamp = ++clock_;
        note_tensors(e, key, gather);
        total_ += bytes;
        entries_.push_back(std::move(e));
        while ((total_ > limit_ || entries_.size() > kMaxEntries) && entries_.size() > 1) {
            size_t victim = 0;
            for (size_t i = 1; i < entries_.size(); ++i)
                if (entries_[i].stamp < entries_[victim].stamp) victim = i;
            total_ -= entries_[victim].bytes;
            entries_.erase(entries_.begin() + static_cast<std::ptrdiff_t>(victim));
        }
        peak_ = std::max(peak_, total_);
    }

    void clear() {
        std::lock_guard<std::mutex> lock(mu_);
        entries_.clear();
        trusted_.clear();
        total_ = 0;
    }

    // Trust scopes (plan_trust_enter / plan_trust_exit, nestable, process
    // wide): while one is open, the caller promises that no index tensor is
    // written, so a plan built or compared equal in the scope is served again
    // for the very same tensors (same TensorImpl, version, data pointer and
    // size) without comparing them.  Closing the outermost scope forgets
    // those tensors.
    void trust_enter() {
        std::lock_guard<std::mutex> lock(mu_);
        ++trust_depth_;
    }

    void trust_exit() {
        std::lock_guard<std::mutex> lock(mu_);
        if (trust_depth_ > 0 && --trust_depth_ == 0) trusted_.clear();
    }

    // entries, hits with the same tensors, hits with other tensors of equal
    // content, misses (lookups that found no equal plan), bytes kept, peak
    // bytes, plans served in trust scopes without a comparison
    std::vector<int64_t> stats() {
        std::lock_guard<std::mutex> lock(mu_);
        return {static_cast<int64_t>(entries_.size()), same_hits_, other_hits_, misses_,
                static_cast<int64_t>(total_), static_cast<int64_t>(peak_), trusted_hits_};
    }

    int64_t size() {
        std::lock_guard<std::mutex> lock(mu_);
        return static_cast<int64_t>(entries_.size());
    }

   private:
    static constexpr size_t kMaxEntries = 64;
    static constexpr size_t kMaxTrusted = 64;

    // A plan and the tensors it was built or verified for in the open trust
    // scope; the references keep the TensorImpl addresses from being reused.
    struct Trusted {
        PlanPtr ref;
        Tensor key;
        Tensor gather;
        uint32_t key_ver = 0;
        uint32_t gather_ver = 0;
    };

    static bool same_tensor(const Tensor& held, uint32_t ver, const Tensor& t) {
        return held.unsafeGetTensorImpl() == t.unsafeGetTensorImpl() && version(t) == ver &&
               held.data_ptr() == t.data_ptr() && held.numel() == t.numel();
    }

    PlanPtr trusted(int role, const Tensor& key, const Tensor* gather, int64_t key_bound,
                    int64_t gather_bound) {
        std::lock_guard<std::mutex> lock(mu_);
        if (trust_depth_ == 0) return PlanPtr();
        for (const Trusted& t : trusted_) {
            const PlanRef& r = *t.ref;
            if (r.role != role || r.key_bound != key_bound ||
                (gather_bound >= 0 && r.gather_bound != gather_bound) ||
                !same_tensor(t.key, t.key_ver, key) || t.gather.defined() != (gather != nullptr) ||
                (gather != nullptr && !same_tensor(t.gather, t.gather_ver, *gather)))
                continue;
            ++trusted_hits_;
            return t.ref;
        }
        return PlanPtr();
    }

    // Records (ref, key, gather) for the open trust scope; mu_ held.
    void remember(const PlanPtr& ref, const Tensor& key, const Tensor* gather) {
        if (trust_depth_ == 0) return;
        if (trusted_.size() >= kMaxTrusted) trusted_.erase(trusted_.begin());
        Trusted t;
        t.ref = ref;
        t.key = key;
        t.key_ver = version(key);
        if (gather != nullptr) {
            t.gather = *gather;
            t.gather_ver = version(*gather);
        }
        trusted_.push_back(std::move(t));
    }


    // The tensors a plan was last used with, kept only as a hint for ordering
    // the candidates: the address may belong to a later tensor by now, which
    // costs nothing because every candidate's content is compared.
    struct Entry {
        PlanPtr ref;
        const c10::TensorImpl* key_impl = nullptr;
        const c10::TensorImpl* gather_impl = nullptr;
        uint32_t key_ver = 0;
        uint32_t gather_ver = 0;
        size_t bytes = 0;
        uint64_t stamp = 0;
    };

    PlanCache() {
        const char* flag = std::getenv("RELM_MP_PLAN_CACHE");
        if (flag != nullptr) {
            std::string v(flag);
            for (char& c : v) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
            enabled_ = !(v == "0" || v == "false" || v == "no" || v == "off");
            identity_only_ = v == "identity";
        }
        const char* mb = std::getenv("RELM_MP_PLAN_CACHE_MB");
        if (mb != nullptr) limit_ = static_cast<size_t>(std::strtoull(mb, nullptr, 10)) << 20;
    }

    // Inference tensors keep no version counter (reading it throws); the
    // version is only an ordering hint here, every candidate's content is
    // compared.
    static uint32_t version(const Tensor& t) {
        return t.is_inference() ? 0u : t.unsafeGetTensorImpl()->version_counter().current_version();
    }

    static void note_tensors(Entry& e, const Tensor& key, const Tensor* gather) {
        e.key_impl = key.unsafeGetTensorImpl();
        e.key_ver = version(key);
        e.gather_impl = gather != nullptr ? gather->unsafeGetTensorImpl() : nullptr;
        e.gather_ver = gather != nullptr ? version(*gather) : 0;
    }

    std::mutex mu_;
    std::vector<Entry> entries_;
    size_t total_ = 0;
    size_t peak_ = 0;
    size_t limit_ = size_t(2048) << 20;
    uint64_t clock_ = 0;
    int64_t same_hits_ = 0;
    int64_t other_hits_ = 0;
    int64_t misses_ = 0;
    int64_t trusted_hits_ = 0;
    int trust_depth_ = 0;
    std::vector<Trusted> trusted_;
    bool enabled_ = true;
    bool identity_only_ = false;
};

PlanPtr new_plan(int role, const Tensor& like, int64_t key_bound, int64_t gather_bound,
                 size_t bytes, hipStream_t s) {
    PlanPtr r = c10::make_intrusive<PlanRef>();
    r->mem = byte_buffer(bytes, like);
    r->role = role;
    r->device = like.get_device();
    r->key_bound = key_bound;
    r->gather_bound = gather_bound;
    r->stream = s;
    return r;
}

int inverse_flags() { return PlanCache::get().enabled() ? RELM_MP_PLAN_SNAPSHOT : 0; }

PlanPtr inverse_plan(const Tensor& key, int64_t key_bound, const char* key_name,
                     const Tensor& gather, int64_t gather_bound, const char* gather_name,
                     bool gather_first, hipStream_t s) {
    PlanCache& cache = PlanCache::get();
    if (PlanPtr hit = cache.lookup(kRoleInverse, key, &gather, key_bound, gather_bound, s)) return hit;
    const int flags = inverse_flags();
    PlanPtr r = new_plan(kRoleInverse, key, key_bound, gather_bound,
                         relm_mp_inv_plan_bytes(key_bound, key.numel(), flags), s);
    raise_if(relm_mp_inv_plan_build(key.data_ptr<int64_t>(), key_bound, key_name,
                                    gather.data_ptr<int64_t>(), gather_bound, gather_name,
                                    gather_first ? 1 : 0, key.numel(), flags, r->mem.data_ptr(),
                                    static_cast<size_t>(r->mem.numel()), &r->plan, s));
    cache.insert(r, key, &gather);
    return r;
}

// CSR plan keyed by `key` gathering `gather` (null: message e reads row e).
PlanPtr csr_build(int role, const Tensor& key, int64_t key_bound, const char* key_name,
                  const Tensor* gather, int64_t gather_bound, const char* gather_name,
                  bool gather_first, hipStream_t s) {
    const int64_t n = key.numel();
    PlanPtr r = new_plan(role, key, key_bound, gather_bound, relm_mp_csr_plan_bytes(key_bound, n), s);
    Tensor scratch = byte_buffer(relm_mp_csr_plan_scratch_bytes(key_bound, n), key);
    // returns once the indices are validated; the build's remaining kernels
    // and the caller's compute stay queued on the stream
    raise_if(relm_mp_csr_plan_build_async(
        key.data_ptr<int64_t>(), key_bound, key_name,
        gather != nullptr ? gather->data_ptr<int64_t>() : nullptr, gather_bound, gather_name,
        gather_first ? 1 : 0, n, r->mem.data_ptr(), static_cast<size_t>(r->mem.numel()),
        scratch.data_ptr(), static_cast<size_t>(scratch.numel()), &r->plan, s));
    PlanCache::get().insert(r, key, gather);
    return r;
}

PlanPtr csr_plan(const Tensor& key, int64_t key_bound, const char* key_name, const Tensor& gather,
                 int64_t gather_bound, const char* gather_name, bool gather_first, hipStream_t s) {
    if (PlanPtr hit = PlanCache::get().lookup(kRoleCsr, key, &gather, key_bound, gather_bound, s))
        return hit;
    return csr_build(kRoleCsr, key, key_bound, key_name, &gather, gather_bound, gather_name,
                     gather_first, s);
}

// CSR plan keyed by `key` whose message e reads row e (no gather array).
PlanPtr csr_plan_rows(const Tensor& key, int64_t key_bound, const char* key_name, hipStream_t s) {
    const int64_t n = key.numel();
    if (PlanPtr hit = PlanCache::get().lookup(kRoleCsrRows, key, nullptr, key_bound, n, s))
        return hit;
    return csr_build(kRoleCsrRows, key, key_bound, key_name, nullptr, n, "", false, s);
}

Tensor compute_scratch(const relm_mp_plan& plan, int64_t emb, int dtype, int64_t mode,
                       const Tensor& like) {
    const size_t bytes = relm_mp_plan_compute_scratch_bytes(&plan, emb, dtype, mode);
    return byte_buffer(bytes, like);
}

// ---- GPU lane ----------------------------------------------------------------

// Inverse plan keyed by flat_dst gathering src_global_idx, with `gather`
// (the plan's first compute step, which reads the gathered rows through the
// plan) enqueued before the host waits for the index check: its kernels stay
// in bounds on bad indices and the result is discarded then.
template <class Gather>
void fanout_inverse(const Tensor& d_idx, int64_t out_rows, const Tensor& s_idx, int64_t x_rows,
                    hipStream_t stream, Gather&& gather) {
    PlanCache& cache = PlanCache::get();
    if (PlanPtr hit = cache.lookup(kRoleInverse, d_idx, &s_idx, out_rows, x_rows, stream)) {
        raise_if(gather(hit->plan));
        return;
    }
    const int flags = inverse_flags();
    PlanPtr r = new_plan(kRoleInverse, d_idx, out_rows, x_rows,
                         relm_mp_inv_plan_bytes(out_rows, d_idx.numel(), flags), stream);
    raise_if(relm_mp_inv_plan_build_async(d_idx.data_ptr<int64_t>(), out_rows, "flat_dst",
                                          s_idx.data_ptr<int64_t>(), x_rows, "src_global_idx", 1,
                                          d_idx.numel(), flags, r->mem.data_ptr(),
                                          static_cast<size_t>(r->mem.numel()), &r->plan, stream));
    const int rc = gather(r->plan);
    raise_if(relm_mp_plan_validate(&r->plan));
    raise_if(rc);
    cache.insert(r, d_idx, &s_idx);
}

Tensor fanout_scatter_gpu(const Tensor& x_cat, const Tensor& src, const Tensor& dst,
                          int64_t out_rows) {
    c10::OptionalDeviceGuard guard(x_cat.device());
    check_same_gpu(x_cat, src, "x_cat", "src_global_idx");
    check_same_gpu(x_cat, dst, "x_cat", "flat_dst");
    const int64_t emb = x_cat.size(1);
    if (src.numel() == 0 || out_rows == 0 || emb == 0)
        return at::zeros({out_rows, emb}, x_cat.options());
    const Tensor x = contiguous(x_cat);
    const Tensor s_idx = contiguous(src);
    const Tensor d_idx = contiguous(dst);
    hipStream_t stream = current_stream(x);
    Tensor out = at::empty({out_rows, emb}, x_cat.options());
    fanout_inverse(d_idx, out_rows, s_idx, x.size(0), stream, [&](const relm_mp_plan& plan) {
        return relm_mp_plan_gather_last(dtype_code(x), &plan, s_idx.data_ptr<int64_t>(),
                                        x.data_ptr(), emb, out.data_ptr(), stream);
    });
    return out;
}

Tensor fanout_scatter_backward_gpu(const Tensor& grad_out, const Tensor& src, const Tensor& dst,
                                   int64_t x_rows) {
    c10::OptionalDeviceGuard guard(grad_out.device());
    check_same_gpu(grad_out, src, "grad_out", "src_global_idx");
    check_same_gpu(grad_out, dst, "grad_out", "flat_dst");
    const int64_t emb = grad_out.size(1);
    if (src.numel() == 0 || x_rows == 0 || emb == 0)
        return at::zeros({x_rows, emb}, grad_out.options());
    const Tensor g = contiguous(grad_out);
    const Tensor s_idx = contiguous(src);
    const Tensor d_idx = contiguous(dst);
    hipStream_t stream = current_stream(g);
    PlanPtr gp = csr_plan(s_idx, x_rows, "src_global_idx", d_idx, g.size(0), "flat_dst", false,
                          stream);
    Tensor grad_x = at::empty({x_rows, emb}, grad_out.options());
    Tensor scratch = compute_scratch(gp->plan, emb, dtype_code(g), kModeSum, g);
    raise_if(relm_mp_plan_segment_reduce(dtype_code(g), &gp->plan, nullptr, g.data_ptr(), emb,
                                         kModeSum, grad_x.data_ptr(), scratch.data_ptr(),
                                         static_cast<size_t>(scratch.numel()), stream));
    return grad_x;
}

// Fanout rows written into / read from `slots` argument slots of emb columns
// per line of a wider matrix (relm_mp.h, grouped row layout): line n, slot s
// holds fanout row n * slots + s at columns [col_offset + s * emb, + emb).
// `mat` has unit column stride and non-overlapping lines.
bool grouped_gpu_ok(const Tensor& mat) {
    return mat.stride(1) == 1 && (mat.size(0) <= 1 || mat.stride(0) >= mat.size(1));
}

int64_t line_stride(const Tensor& mat) { return mat.size(0) <= 1 ? mat.size(1) : mat.stride(0); }

void fanout_scatter_into_gpu(const Tensor& x_cat, const Tensor& src, const Tensor& dst,
                             const Tensor& out, int64_t col_offset, int64_t slots) {
    c10::OptionalDeviceGuard guard(x_cat.device());
    check_same_gpu(x_cat, src, "x_cat", "src_global_idx");
    check_same_gpu(x_cat, dst, "x_cat", "flat_dst");
    check_same_gpu(x_cat, out, "x_cat", "out");
    const int64_t emb = x_cat.size(1);
    const int64_t out_rows = out.size(0) * slots;
    const Tensor x = contiguous(x_cat);
    const Tensor s_idx = contiguous(src);
    const Tensor d_idx = contiguous(dst);
    hipStream_t stream = current_stream(x);
    char* base = static_cast<char*>(out.data_ptr()) + col_offset * out.element_size();
    const int64_t stride = line_stride(out);
    fanout_inverse(d_idx, out_rows, s_idx, x.size(0), stream, [&](const relm_mp_plan& plan) {
        return relm_mp_plan_gather_last_grouped(dtype_code(x), &plan, s_idx.data_ptr<int64_t>(),
                                                x.data_ptr(), emb, slots, stride, base, stream);
    });
}

Tensor fanout_scatter_backward_from_gpu(const Tensor& grad, const Tensor& src, const Tensor& dst,
                                        int64_t x_rows, int64_t col_offset, int64_t slots,
                                        int64_t emb) {
    c10::OptionalDeviceGuard guard(grad.device());
    check_same_gpu(grad, src, "grad", "src_global_idx");
    check_same_gpu(grad, dst, "grad", "flat_dst");
    const Tensor g = grouped_gpu_ok(grad) ? grad : grad.contiguous();
    const Tensor s_idx = contiguous(src);
    const Tensor d_idx = contiguous(dst);
    const int64_t rows = g.size(0) * slots;
    hipStream_t stream = current_stream(g);
    PlanPtr gp = csr_plan(s_idx, x_rows, "src_global_idx", d_idx, rows, "flat_dst", false, stream);
    Tensor grad_x = at::empty({x_rows, emb}, grad.options());
    Tensor scratch = compute_scratch(gp->plan, emb, dtype_code(g), kModeSum, g);
    const char* base = static_cast<const char*>(g.data_ptr()) + col_offset * g.element_size();
    raise_if(relm_mp_plan_segment_sum_grouped(dtype_code(g), &gp->plan, base, rows, emb, slots,
                                              line_stride(g), grad_x.data_ptr(), scratch.data_ptr(),
                                              static_cast<size_t>(scratch.numel()), stream));
    return grad_x;
}

// fanin_reduce on the GPU; *plan_out (if given) receives the forward's CSR
// plan (keys dst_idx, gathers flat_src) for the backward.
// The reference's CPU lane computes logsumexp with ATen calls
// (mp_ops.cpp:2981-3035), so an index out of range raises ATen's errors, in
// the order of those calls: index_select raises IndexError "index out of
// range in self"; scatter_reduce_ and index_add_ raise "index i is out of
// bounds for dimension 0 with size n" for the first bad index in edge order.
// The GPU lane validates on the device; when a logsumexp op's plan build
// reports a bad index, these restate the reference's error for it.
bool any_outside(const Tensor& idx, int64_t size) {
    return ((idx < 0) | (idx >= size)).any().item<bool>();
}

void raise_first_outside(const Tensor& idx, int64_t size) {
    const Tensor bad = ((idx < 0) | (idx >= size)).nonzero();
    if (bad.numel() == 0) return;
    const int64_t v = idx[bad[0][0].item<int64_t>()].item<int64_t>();
    TORCH_CHECK(false, "index ", v, " is out of bounds for dimension 0 with size ", size);
}

// mp_ops.cpp:3019-3035: rel_flat.index_select(flat_src), then scatter_reduce_ over dst_idx.
void raise_lse_forward_index_error(const Tensor& s_idx, int64_t rel_rows, const Tensor& d_idx,
                                   int64_t dim_size) {
    TORCH_CHECK_INDEX(!any_outside(s_idx, rel_rows), "index out of range in self");
    raise_first_outside(d_idx, dim_size);
}

// mp_ops.cpp:2981-3003: rel_flat / out / grad_out index_select, then index_add_ into
// the rel_rows gradient rows.
void raise_lse_backward_index_error(const Tensor& s_idx, int64_t rel_flat_rows, const Tensor& d_idx,
                                    int64_t out_rows, int64_t rel_rows) {
    TORCH_CHECK_INDEX(!any_outside(s_idx, rel_flat_rows), "index out of range in self");
    TORCH_CHECK_INDEX(!any_outside(d_idx, out_rows), "index out of range in self");
    raise_first_outside(s_idx, rel_rows);
}

Tensor fanin_reduce_gpu(const Tensor& rel_flat, const Tensor& flat_src, const Tensor& dst_idx,
                        int64_t dim_size, int64_t mode, PlanPtr* plan_out = nullptr) {
    c10::OptionalDeviceGuard guard(rel_flat.device());
    check_same_gpu(rel_flat, flat_src, "rel_flat", "flat_src");
    check_same_gpu(rel_flat, dst_idx, "rel_flat", "dst_idx");
    const int64_t emb = rel_flat.size(1);
    if (flat_src.numel() == 0 || dim_size == 0 || emb == 0) {
        if (mode == kModeSum) return at::zeros({dim_size, emb}, rel_flat.options());
        return at::full({dim_size, emb}, -std::numeric_limits<double>::infinity(),
                        rel_flat.options());
    }
    const Tensor rel = contiguous(rel_flat);
    const Tensor s_idx = contiguous(flat_src);
    const Tensor d_idx = contiguous(dst_idx);
    hipStream_t stream = current_stream(rel);
    PlanPtr gp;
    try {
        gp = csr_plan(d_idx, dim_size, "dst_idx", s_idx, rel.size(0), "flat_src", true, stream);
    } catch (const c10::Error&) {
        if (mode == kModeLogSumExp) raise_lse_forward_index_error(s_idx, rel.size(0), d_idx, dim_size);
        throw;
    }
    Tensor out = at::empty({dim_size, emb}, rel_flat.options());
    Tensor scratch = compute_scratch(gp->plan, emb, dtype_code(rel), mode, rel);
    raise_if(relm_mp_plan_segment_reduce(dtype_code(rel), &gp->plan, nullptr, rel.data_ptr(), emb,
                                         mode, out.data_ptr(), scratch.data_ptr(),
                                         static_cast<size_t>(scratch.numel()), stream));
    if (plan_out != nullptr) *plan_out = gp;
    return out;
}

// The forward's CSR plan for a fanin backward: the plan handed over by the
// autograd function when it fits these indices (a handoff within one call's
// graph: not compared again), else a cached plan of equal indices.  Null if
// neither exists.
PlanPtr fanin_forward_plan(const PlanRef* handoff, const Tensor& d_idx, const Tensor& s_idx,
                           int64_t dim_size, hipStream_t stream) {
    if (handoff != nullptr && handoff->defined() && handoff->role == kRoleCsr &&
        handoff->device == d_idx.get_device() && handoff->plan.num_edges == d_idx.numel() &&
        handoff->key_bound == dim_size) {
        handoff->use_on(stream);
        return PlanPtr::reclaim_copy(const_cast<PlanRef*>(handoff));
    }
    return PlanCache::get().lookup(kRoleCsr, d_idx, &s_idx, dim_size, -1, stream);
}

// The backward through the forward's CSR plan when flat_src is injective but
// not the identity (the callers' layout): the inverse map of flat_src comes
// from the plan's snapshot of it without atomics, and the kernel is queued
// before the host learns whether flat_src repeats.  False (nothing to use)
// when there is no such plan or flat_src repeats: the caller then builds its
// own plans.  Rows [0, rows) of grad_rel are written.
bool backward_by_src(const PlanPtr& fwd, int64_t mode, const Tensor& g, const void* out,
                     const void* rel, int64_t emb, Tensor& grad_rel, int64_t rows, hipStream_t stream) {
    if (!fwd || fwd->plan.gather_identity != 0 || fwd->plan.snap_gathers == nullptr ||
        rows < fwd->plan.num_gather)
        return false;
    PlanRef& ref = *fwd;
    std::lock_guard<std::mutex> lock(ref.inv_mu);
    if (ref.inv_collide_rows == rows)
        return false;
    const bool ready = ref.inv_rows == rows && ref.inv_stream == stream && ref.inv_mem.defined();
    Tensor mem = ready ? ref.inv_mem : byte_buffer(relm_mp_inv_plan_bytes(rows, fwd->plan.num_edges, 0), g);
    int64_t collisions = 0;
    raise_if(relm_mp_plan_fanin_backward_by_src(dtype_code(g), &fwd->plan, mode, g.data_ptr(), out, rel, emb,
                                                grad_rel.data_ptr(), rows, mem.data_ptr(),
                                                static_cast<size_t>(mem.numel()), ready ? 1 : 0, &collisions,
                                                stream));
    if (!ready && collisions == 0) {
        ref.inv_mem = mem;
        ref.inv_rows = rows;
        ref.inv_stream = stream;
    }
    if (collisions != 0)
        ref.inv_collide_rows = rows;
    return collisions == 0;
}

Tensor fanin_reduce_sum_backward_gpu(const Tensor& grad_out, const Tensor& flat_src,
                                     const Tensor& dst_idx, int64_t rel_rows,
                                     const PlanRef* handoff = nullptr) {
    c10::OptionalDeviceGuard guard(grad_out.device());
    check_same_gpu(grad_out, flat_src, "grad_out", "flat_src");
    check_same_gpu(grad_out, dst_idx, "grad_out", "dst_idx");
    const int64_t emb = grad_out.size(1);
    if (flat_src.numel() == 0 || rel_rows == 0 || emb == 0)
        return at::zeros({rel_rows, emb}, grad_out.options());
    const Tensor g = contiguous(grad_out);
    const Tensor s_idx = contiguous(flat_src);
    const Tensor d_idx = contiguous(dst_idx);
    hipStream_t stream = current_stream(g);
    Tensor grad_rel = at::empty({rel_rows, emb}, grad_out.options());
    // The forward's plan (keys dst_idx, gathers flat_src, validated) serves
    // directly when flat_src is the identity.
    const PlanPtr fwd = fanin_forward_plan(handoff, d_idx, s_idx, g.size(0), stream);
    if (fwd && fwd->plan.gather_identity != 0 && fwd->plan.num_edges <= rel_rows) {
        raise_if(relm_mp_plan_fanin_backward_by_dst(dtype_code(g), &fwd->plan,
                                                    d_idx.data_ptr<int64_t>(), kModeSum,
                                                    g.data_ptr(), nullptr, nullptr, emb,
                                                    grad_rel.data_ptr(), rel_rows, stream));
        return grad_rel;
    }
    if (backward_by_src(fwd, kModeSum, g, nullptr, nullptr, emb, grad_rel, rel_rows, stream))
        return grad_rel;
    PlanPtr inv = inverse_plan(s_idx, rel_rows, "flat_src", d_idx, g.size(0), "dst_idx", false,
                               stream);
    if (inv->plan.collisions == 0) {
        raise_if(relm_mp_plan_gather_last(dtype_code(g), &inv->plan, d_idx.data_ptr<int64_t>(),
                                          g.data_ptr(), emb, grad_rel.data_ptr(), stream));
        return grad_rel;
    }
    PlanPtr gp = csr_plan(s_idx, rel_rows, "flat_src", d_idx, g.size(0), "dst_idx", false, stream);
    Tensor scratch = compute_scratch(gp->plan, emb, dtype_code(g), kModeSum, g);
    raise_if(relm_mp_plan_segment_reduce(dtype_code(g), &gp->plan, nullptr, g.data_ptr(), emb,
                                         kModeSum, grad_rel.data_ptr(), scratch.data_ptr(),
                                         static_cast<size_t>(scratch.numel()), stream));
    return grad_rel;
}

Tensor fanin_reduce_logsumexp_backward_gpu(const Tensor& grad_out, const Tensor& rel_flat,
                                           const Tensor& flat_src, const Tensor& dst_idx,
                                           const Tensor& out, int64_t rel_rows,
                                           const PlanRef* handoff = nullptr) {
    c10::OptionalDeviceGuard guard(grad_out.device());
    check_same_gpu(grad_out, rel_flat, "grad_out", "rel_flat");
    check_same_gpu(grad_out, flat_src, "grad_out", "flat_src");
    check_same_gpu(grad_out, dst_idx, "grad_out", "dst_idx");
    check_same_gpu(grad_out, out, "grad_out", "out");
    TORCH_CHECK(grad_out.scalar_type() == rel_flat.scalar_type() &&
                    grad_out.scalar_type() == out.scalar_type(),
                "grad_out, rel_flat, and out must share dtype.");
    const int64_t emb = grad_out.size(1);
    if (flat_src.numel() == 0 || rel_rows == 0 || emb == 0)
        return at::zeros({rel_rows, emb}, rel_flat.options());
    const Tensor g = contiguous(grad_out);
    const Tensor rel = contiguous(rel_flat);
    const Tensor o = contiguous(out);
    const Tensor s_idx = contiguous(flat_src);
    const Tensor d_idx = contiguous(dst_idx);
    hipStream_t stream = current_stream(g);
    // A message row is read from rel_flat and written to grad_rel, so flat_src
    // must index both; rows beyond rel_flat cannot receive a gradient.
    const int64_t key_bound = std::min<int64_t>(rel_rows, rel.size(0));
    Tensor grad_rel = at::empty({rel_rows, emb}, rel_flat.options());
    const int dt = dtype_code(rel);
    const PlanPtr fwd = fanin_forward_plan(handoff, d_idx, s_idx, g.size(0), stream);
    if (fwd && fwd->plan.gather_identity != 0 && fwd->plan.num_edges <= key_bound) {
        raise_if(relm_mp_plan_fanin_backward_by_dst(dt, &fwd->plan, d_idx.data_ptr<int64_t>(),
                                                    kModeLogSumExp, g.data_ptr(), o.data_ptr(),
                                                    rel.data_ptr(), emb, grad_rel.data_ptr(),
                                                    rel_rows, stream));
        return grad_rel;
    }
    if (key_bound < rel_rows) grad_rel.narrow(0, key_bound, rel_rows - key_bound).zero_();
    if (backward_by_src(fwd, kModeLogSumExp, g, o.data_ptr(), rel.data_ptr(), emb, grad_rel, key_bound,
                        stream))
        return grad_rel;
    const auto reference_error = [&]() {
        raise_lse_backward_index_error(s_idx, rel.size(0), d_idx, o.size(0), rel_rows);
    };
    PlanPtr inv;
    try {
        inv = inverse_plan(s_idx, key_bound, "flat_src", d_idx, g.size(0), "dst_idx", true, stream);
    } catch (const c10::Error&) {
        reference_error();
        throw;
    }
    if (inv->plan.collisions == 0) {
        raise_if(relm_mp_plan_logsumexp_backward(dt, &inv->plan, d_idx.data_ptr<int64_t>(),
                                                 g.data_ptr(), o.data_ptr(), rel.data_ptr(), emb,
                                                 grad_rel.data_ptr(), nullptr, 0, stream));
        return grad_rel;
    }
    PlanPtr gp;
    try {
        gp = csr_plan(s_idx, key_bound, "flat_src", d_idx, g.size(0), "dst_idx", true, stream);
    } catch (const c10::Error&) {
        reference_error();
        throw;
    }
    Tensor scratch = compute_scratch(gp->plan, emb, dt, kModeSum, g);
    raise_if(relm_mp_plan_logsumexp_backward(dt, &gp->plan, nullptr, g.data_ptr(), o.data_ptr(),
                                             rel.data_ptr(), emb, grad_rel.data_ptr(),
                                             scratch.data_ptr(),
                                             static_cast<size_t>(scratch.numel()), stream));
    return grad_rel;
}

// ---- CPU lane (mp_ops.cpp:2815-2911) -------------------------------------------

template <typename scalar_t>
void cpu_scatter_rows(const scalar_t* in, const int64_t* read_idx, int64_t read_rows,
                      const char* read_name, const int64_t* write_idx, int64_t write_rows,
                      const char* write_name, bool read_checked_first, int64_t n, int64_t emb,
                      scalar_t* out, bool accumulate) {
    for (int64_t e = 0; e < n; ++e) {
        const int64_t r = read_idx[e];
        const int64_t w = write_idx[e];
        if (read_checked_first) {
            check_in_bounds(r, read_rows, read_name);
            check_in_bounds(w, write_rows, write_name);
        } else {
            check_in_bounds(w, write_rows, write_name);
            check_in_bounds(r, read_rows, read_name);
        }
        const scalar_t* src_row = in + r * emb;
        scalar_t* dst_row = out + w * emb;
        if (accumulate) {
            for (int64_t k = 0; k < emb; ++k) dst_row[k] += src_row[k];
        } else {
            std::memcpy(dst_row, src_row, static_cast<size_t>(emb) * sizeof(scalar_t));
        }
    }
}

// Runs out[write[e]] (+)= in[read[e]] over all edges for f32 / f64 CPU tensors.
void cpu_lane(const Tensor& in, const Tensor& read_idx, const char* read_name,
              const Tensor& write_idx, const char* write_name, bool read_checked_first,
              Tensor& out, bool accumulate) {
    const Tensor x = contiguous(in);
    const Tensor ri = contiguous(read_idx);
    const Tensor wi = contiguous(write_idx);
    const int64_t emb = out.size(1);
    if (x.scalar_type() == at::kFloat) {
        cpu_scatter_rows<float>(x.data_ptr<float>(), ri.data_ptr<int64_t>(), x.size(0), read_name,
                                wi.data_ptr<int64_t>(), out.size(0), write_name,
                                read_checked_first, ri.numel(), emb, out.data_ptr<float>(),
                                accumulate);
    } else {
        cpu_scatter_rows<double>(x.data_ptr<double>(), ri.data_ptr<int64_t>(), x.size(0),
                                 read_name, wi.data_ptr<int64_t>(), out.size(0), write_name,
                                 read_checked_first, ri.numel(), emb, out.data_ptr<double>(),
                                 accumulate);
    }
}

// ---- ATen sequences (mp_ops.cpp:2913-3036) -------------------------------------

Tensor fanin_logsumexp_aten(const Tensor& rel_flat, const Tensor& flat_src, const Tensor& dst_idx,
                            int64_t dim_size) {
    const int64_t emb = rel_flat.size(1);
    Tensor max_vals =
        at::full({dim_size, emb}, -std::numeric_limits<double>::infinity(), rel_flat.options());
    if (flat_src.numel() == 0 || dim_size == 0) return max_vals;
    Tensor msgs = rel_flat.index_select(0, flat_src);
    Tensor index = dst_idx.unsqueeze(1).expand({dst_idx.size(0), emb});
    max_vals.scatter_reduce_(0, index, msgs, "amax", true);
    Tensor max_offsets = max_vals.index_select(0, dst_idx);
    Tensor exps = (msgs - max_offsets).exp();
    Tensor exps_sum = at::zeros({dim_size, emb}, rel_flat.options());
    exps_sum.scatter_add_(0, index, exps);
    return exps_sum.log() + max_vals;
}

Tensor fanin_logsumexp_backward_aten(const Tensor& grad_out, const Tensor& rel_flat,
                                     const Tensor& flat_src, const Tensor& dst_idx,
                                     const Tensor& out, int64_t rel_rows) {
    const int64_t emb = grad_out.size(1);
    Tensor grad_rel = at::zeros({rel_rows, emb}, rel_flat.options());
    if (flat_src.numel() == 0 || rel_rows == 0) return grad_rel;
    Tensor msgs = rel_flat.index_select(0, flat_src);
    Tensor out_sel = out.index_select(0, dst_idx);
    Tensor grad_sel = grad_out.index_select(0, dst_idx);
    Tensor weights = (msgs - out_sel).exp();
    grad_rel.index_add_(0, flat_src, grad_sel * weights);
    return grad_rel;
}

// ---- ops -------------------------------------------------------------------------

Tensor fanout_scatter(const Tensor& x_cat, const Tensor& src_global_idx, const Tensor& flat_dst,
                      int64_t out_rows) {
    check_rank(x_cat, 2, "x_cat");
    check_int64_index(src_global_idx, "src_global_idx");
    check_int64_index(flat_dst, "flat_dst");
    TORCH_CHECK(src_global_idx.size(0) == flat_dst.size(0),
                "src_global_idx and flat_dst must have equal length.");
    TORCH_CHECK(out_rows >= 0, "out_rows must be >= 0.");
    const int64_t emb = x_cat.size(1);
    if (src_global_idx.numel() == 0 || out_rows == 0)
        return at::zeros({out_rows, emb}, x_cat.options());
    if (all_gpu({&x_cat, &src_global_idx, &flat_dst}) && is_fastpath_dtype(x_cat.scalar_type()))
        return fanout_scatter_gpu(x_cat, src_global_idx, flat_dst, out_rows);
    Tensor out = at::zeros({out_rows, emb}, x_cat.options());
    if (all_cpu({&x_cat, &src_global_idx, &flat_dst}) && is_fastpath_dtype(x_cat.scalar_type())) {
        cpu_lane(x_cat, src_global_idx, "src_global_idx", flat_dst, "flat_dst", true, out, false);
        return out;
    }
    out.index_copy_(0, flat_dst, x_cat.index_select(0, src_global_idx));
    return out;
}

Tensor fanout_scatter_backward(const Tensor& grad_out, const Tensor& src_global_idx,
                               const Tensor& flat_dst, int64_t x_rows) {
    check_rank(grad_out, 2, "grad_out");
    check_int64_index(src_global_idx, "src_global_idx");
    check_int64_index(flat_dst, "flat_dst");
    TORCH_CHECK(src_global_idx.size(0) == flat_dst.size(0),
                "src_global_idx and flat_dst must have equal length.");
    TORCH_CHECK(x_rows >= 0, "x_rows must be >= 0.");
    const int64_t emb = grad_out.size(1);
    if (src_global_idx.numel() == 0 || x_rows == 0)
        return at::zeros({x_rows, emb}, grad_out.options());
    if (all_gpu({&grad_out, &src_global_idx, &flat_dst}) &&
        is_fastpath_dtype(grad_out.scalar_type()))
        return fanout_scatter_backward_gpu(grad_out, src_global_idx, flat_dst, x_rows);
    Tensor grad_x = at::zeros({x_rows, emb}, grad_out.options());
    if (all_cpu({&grad_out, &src_global_idx, &flat_dst}) &&
        is_fastpath_dtype(grad_out.scalar_type())) {
        // mp_ops.cpp:2838-2861: src (write side) is checked before flat_dst.
        cpu_lane(grad_out, flat_dst, "flat_dst", src_global_idx, "src_global_idx", false, grad_x,
                 true);
        return grad_x;
    }
    grad_x.index_add_(0, src_global_idx, grad_out.index_select(0, flat_dst));
    return grad_x;
}

// No counterpart in the reference: fanout_scatter written straight into the
// argument columns of the central input matrix, and its backward reading the
// gradient from there (fused.py:299-375 fans out into args_flat
// [nodes * max_arity, emb], reshapes it and copies it into all_inputs).
// out[n, col_offset + s * emb + c] = fanout_scatter(x_cat, src_global_idx,
// flat_dst, out.size(0) * slots)[n * slots + s, c]; the other columns of out
// keep their values.
void check_slot_columns(int64_t width, int64_t col_offset, int64_t slots, int64_t emb) {
    TORCH_CHECK(slots >= 1, "slots must be >= 1.");
    TORCH_CHECK(col_offset >= 0, "col_offset must be >= 0.");
    TORCH_CHECK(emb >= 0, "emb must be >= 0.");
    TORCH_CHECK(col_offset + slots * emb <= width,
                "the argument slots [col_offset, col_offset + slots * emb) exceed the ", width,
                " columns.");
}

void fanout_scatter_into(const Tensor& x_cat, const Tensor& src_global_idx, const Tensor& flat_dst,
                         const Tensor& out, int64_t col_offset, int64_t slots) {
    check_rank(x_cat, 2, "x_cat");
    check_rank(out, 2, "out");
    check_int64_index(src_global_idx, "src_global_idx");
    check_int64_index(flat_dst, "flat_dst");
    TORCH_CHECK(src_global_idx.size(0) == flat_dst.size(0),
                "src_global_idx and flat_dst must have equal length.");
    const int64_t emb = x_cat.size(1);
    check_slot_columns(out.size(1), col_offset, slots, emb);
    TORCH_CHECK(out.scalar_type() == x_cat.scalar_type(), "out must have the dtype of x_cat.");
    TORCH_CHECK(out.device() == x_cat.device(), "out must be on the device of x_cat.");
    const int64_t rows = out.size(0) * slots;
    if (rows == 0 || emb == 0) return;
    if (src_global_idx.numel() > 0 && all_gpu({&x_cat, &src_global_idx, &flat_dst}) &&
        is_fastpath_dtype(x_cat.scalar_type()) && grouped_gpu_ok(out)) {
        fanout_scatter_into_gpu(x_cat, src_global_idx, flat_dst, out, col_offset, slots);
        // written through its pointer: count it as an in-place change, as
        // the ATen path's copy_ does
        out.unsafeGetTensorImpl()->bump_version();
        return;
    }
    const Tensor res = fanout_scatter(x_cat, src_global_idx, flat_dst, rows);
    out.narrow(1, col_offset, slots * emb).copy_(res.view({out.size(0), slots * emb}));
}

Tensor fanout_scatter_backward_from(const Tensor& grad, const Tensor& src_global_idx,
                                    const Tensor& flat_dst, int64_t x_rows, int64_t col_offset,
                                    int64_t slots, int64_t emb) {
    check_rank(grad, 2, "grad");
    check_int64_index(src_global_idx, "src_global_idx");
    check_int64_index(flat_dst, "flat_dst");
    TORCH_CHECK(src_global_idx.size(0) == flat_dst.size(0),
                "src_global_idx and flat_dst must have equal length.");
    TORCH_CHECK(x_rows >= 0, "x_rows must be >= 0.");
    check_slot_columns(grad.size(1), col_offset, slots, emb);
    if (src_global_idx.numel() == 0 || x_rows == 0 || emb == 0)
        return at::zeros({x_rows, emb}, grad.options());
    if (all_gpu({&grad, &src_global_idx, &flat_dst}) && is_fastpath_dtype(grad.scalar_type()))
        return fanout_scatter_backward_from_gpu(grad, src_global_idx, flat_dst, x_rows, col_offset,
                                                slots, emb);
    const Tensor slice = grad.narrow(1, col_offset, slots * emb).reshape({grad.size(0) * slots, emb});
    return fanout_scatter_backward(slice, src_global_idx, flat_dst, x_rows);
}

Tensor fanin_reduce_sum(const Tensor& rel_flat, const Tensor& flat_src, const Tensor& dst_idx,
                        int64_t dim_size, PlanPtr* plan_out) {
    const int64_t emb = rel_flat.size(1);
    if (flat_src.numel() == 0 || dim_size == 0)
        return at::zeros({dim_size, emb}, rel_flat.options());
    if (all_gpu({&rel_flat, &flat_src, &dst_idx}) && is_fastpath_dtype(rel_flat.scalar_type()))
        return fanin_reduce_gpu(rel_flat, flat_src, dst_idx, dim_size, kModeSum, plan_out);
    Tensor out = at::zeros({dim_size, emb}, rel_flat.options());
    if (all_cpu({&rel_flat, &flat_src, &dst_idx}) && is_fastpath_dtype(rel_flat.scalar_type())) {
        cpu_lane(rel_flat, flat_src, "flat_src", dst_idx, "dst_idx", true, out, true);
        return out;
    }
    out.index_add_(0, dst_idx, rel_flat.index_select(0, flat_src));
    return out;
}

Tensor fanin_reduce_logsumexp(const Tensor& rel_flat, const Tensor& flat_src,
                              const Tensor& dst_idx, int64_t dim_size, PlanPtr* plan_out) {
    if (all_gpu({&rel_flat, &flat_src, &dst_idx}) && is_fastpath_dtype(rel_flat.scalar_type()))
        return fanin_reduce_gpu(rel_flat, flat_src, dst_idx, dim_size, kModeLogSumExp, plan_out);
    return fanin_logsumexp_aten(rel_flat, flat_src, dst_idx, dim_size);
}

Tensor fanin_reduce_impl(const Tensor& rel_flat, const Tensor& flat_src, const Tensor& dst_idx,
                         int64_t dim_size, int64_t mode, PlanPtr* plan_out) {
    check_rank(rel_flat, 2, "rel_flat");
    check_int64_index(flat_src, "flat_src");
    check_int64_index(dst_idx, "dst_idx");
    TORCH_CHECK(flat_src.size(0) == dst_idx.size(0), "flat_src and dst_idx must have equal length.");
    TORCH_CHECK(dim_size >= 0, "dim_size must be >= 0.");
    if (mode == kModeSum) return fanin_reduce_sum(rel_flat, flat_src, dst_idx, dim_size, plan_out);
    if (mode == kModeLogSumExp)
        return fanin_reduce_logsumexp(rel_flat, flat_src, dst_idx, dim_size, plan_out);
    throw std::invalid_argument("Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.");
}

Tensor fanin_reduce(const Tensor& rel_flat, const Tensor& flat_src, const Tensor& dst_idx,
                    int64_t dim_size, int64_t mode) {
    return fanin_reduce_impl(rel_flat, flat_src, dst_idx, dim_size, mode, nullptr);
}

Tensor fanin_reduce_sum_backward_impl(const Tensor& grad_out, const Tensor& flat_src,
                                      const Tensor& dst_idx, int64_t rel_rows,
                                      const PlanRef* handoff) {
    check_rank(grad_out, 2, "grad_out");
    check_int64_index(flat_src, "flat_src");
    check_int64_index(dst_idx, "dst_idx");
    TORCH_CHECK(flat_src.size(0) == dst_idx.size(0), "flat_src and dst_idx must have equal length.");
    TORCH_CHECK(rel_rows >= 0, "rel_rows must be >= 0.");
    const int64_t emb = grad_out.size(1);
    if (flat_src.numel() == 0 || rel_rows == 0)
        return at::zeros({rel_rows, emb}, grad_out.options());
    if (all_gpu({&grad_out, &flat_src, &dst_idx}) && is_fastpath_dtype(grad_out.scalar_type()))
        return fanin_reduce_sum_backward_gpu(grad_out, flat_src, dst_idx, rel_rows, handoff);
    Tensor grad_rel = at::zeros({rel_rows, emb}, grad_out.options());
    if (all_cpu({&grad_out, &flat_src, &dst_idx}) && is_fastpath_dtype(grad_out.scalar_type())) {
        // mp_ops.cpp:2888-2911: flat_src (write side) is checked before dst_idx.
        cpu_lane(grad_out, dst_idx, "dst_idx", flat_src, "flat_src", false, grad_rel, true);
        return grad_rel;
    }
    grad_rel.index_add_(0, flat_src, grad_out.index_select(0, dst_idx));
    return grad_rel;
}

Tensor fanin_reduce_logsumexp_backward_impl(const Tensor& grad_out, const Tensor& rel_flat,
                                            const Tensor& flat_src, const Tensor& dst_idx,
                                            const Tensor& out, int64_t rel_rows,
                                            const PlanRef* handoff) {
    check_rank(grad_out, 2, "grad_out");
    check_rank(rel_flat, 2, "rel_flat");
    check_int64_index(flat_src, "flat_src");
    check_int64_index(dst_idx, "dst_idx");
    check_rank(out, 2, "out");
    TORCH_CHECK(flat_src.size(0) == dst_idx.size(0), "flat_src and dst_idx must have equal length.");
    TORCH_CHECK(rel_flat.size(1) == grad_out.size(1),
                "rel_flat and grad_out must share embedding dim.");
    TORCH_CHECK(out.size(0) == grad_out.size(0), "out and grad_out must share dim_size.");
    TORCH_CHECK(out.size(1) == grad_out.size(1), "out and grad_out must share embedding dim.");
    TORCH_CHECK(rel_rows >= 0, "rel_rows must be >= 0.");
    const int64_t emb = grad_out.size(1);
    if (flat_src.numel() == 0 || rel_rows == 0)
        return at::zeros({rel_rows, emb}, rel_flat.options());
    if (all_gpu({&grad_out, &rel_flat, &flat_src, &dst_idx, &out}) &&
        is_fastpath_dtype(grad_out.scalar_type()))
        return fanin_reduce_logsumexp_backward_gpu(grad_out, rel_flat, flat_src, dst_idx, out,
                                                   rel_rows, handoff);
    return fanin_logsumexp_backward_aten(grad_out, rel_flat, flat_src, dst_idx, out, rel_rows);
}

Tensor fanin_reduce_sum_backward(const Tensor& grad_out, const Tensor& flat_src,
                                 const Tensor& dst_idx, int64_t rel_rows) {
    return fanin_reduce_sum_backward_impl(grad_out, flat_src, dst_idx, rel_rows, nullptr);
}

Tensor fanin_reduce_logsumexp_backward(const Tensor& grad_out, const Tensor& rel_flat,
                                       const Tensor& flat_src, const Tensor& dst_idx,
                                       const Tensor& out, int64_t rel_rows) {
    return fanin_reduce_logsumexp_backward_impl(grad_out, rel_flat, flat_src, dst_idx, out,
                                                rel_rows, nullptr);
}

// No reference counterpart: fanin_reduce together with the index plan it ran
// on (an empty PlanRef on the CPU lanes), and the backward ops taking that
// plan, so that the autograd function of the facade hands the forward's plan
// to the backward of the same call without a cache lookup.
std::tuple<Tensor, PlanPtr> fanin_reduce_planned(const Tensor& rel_flat, const Tensor& flat_src,
                                                 const Tensor& dst_idx, int64_t dim_size,
                                                 int64_t mode) {
    PlanPtr plan;
    Tensor out = fanin_reduce_impl(rel_flat, flat_src, dst_idx, dim_size, mode, &plan);
    if (!plan) plan = c10::make_intrusive<PlanRef>();
    return std::make_tuple(out, plan);
}

Tensor fanin_reduce_sum_backward_planned(const Tensor& grad_out, const Tensor& flat_src,
                                         const Tensor& dst_idx, int64_t rel_rows,
                                         const PlanPtr& plan) {
    return fanin_reduce_sum_backward_impl(grad_out, flat_src, dst_idx, rel_rows, plan.get());
}

Tensor fanin_reduce_logsumexp_backward_planned(const Tensor& grad_out, const Tensor& rel_flat,
                                               const Tensor& flat_src, const Tensor& dst_idx,
                                               const Tensor& out, int64_t rel_rows,
                                               const PlanPtr& plan) {
    return fanin_reduce_logsumexp_backward_impl(grad_out, rel_flat, flat_src, dst_idx, out,
                                                rel_rows, plan.get());
}

// ---- pack ops (mp_ops.cpp:412-570, 2511-2772) --------------------------------
//
// Values are concatenated with at::cat (differentiable; a single part is
// returned as is), the index outputs by one pass over all parts: pair e of part
// i becomes (a[e] * a_mul + a_add, b[e] * b_mul + b_add).  The reference
// always returns a new tensor for the first index output and returns the
// second index tensor of a single part unchanged where it applies no
// arithmetic to it; `alias_single_b` keeps that.

struct IndexPart {
    Tensor a;
    Tensor b;
    int64_t a_mul, a_add, b_mul, b_add;
};

void pack_parts_cpu(const std::vector<IndexPart>& parts, int64_t* out_a, int64_t* out_b) {
    int64_t pos = 0;
    for (const IndexPart& p : parts) {
        const Tensor a = contiguous(p.a);
        const int64_t* pa = a.data_ptr<int64_t>();
        const int64_t n = a.numel();
        const uint64_t am = static_cast<uint64_t>(p.a_mul), aa = static_cast<uint64_t>(p.a_add);
        for (int64_t e = 0; e < n; ++e)
            out_a[pos + e] = static_cast<int64_t>(static_cast<uint64_t>(pa[e]) * am + aa);
        if (out_b != nullptr) {
            const Tensor b = contiguous(p.b);
            const int64_t* pb = b.data_ptr<int64_t>();
            const uint64_t bm = static_cast<uint64_t>(p.b_mul), ba = static_cast<uint64_t>(p.b_add);
            for (int64_t e = 0; e < n; ++e)
                out_b[pos + e] = static_cast<int64_t>(static_cast<uint64_t>(pb[e]) * bm + ba);
        }
        pos += n;
    }
}

void pack_parts_gpu(const std::vector<IndexPart>& parts, int64_t* out_a, int64_t* out_b,
                    const Tensor& like) {
    std::vector<Tensor> keep;
    std::vector<relm_mp_index_part> desc;
    keep.reserve(2 * parts.size());
    desc.reserve(parts.size());
    for (const IndexPart& p : parts) {
        keep.push_back(contiguous(p.a));
        const int64_t* pa = keep.back().data_ptr<int64_t>();
        const int64_t* pb = nullptr;
        if (out_b != nullptr) {
            keep.push_back(contiguous(p.b));
            pb = keep.back().data_ptr<int64_t>();
        }
        desc.push_back({pa, pb, p.a.numel(), p.a_mul, p.a_add, p.b_mul, p.b_add});
    }
    // Contiguous copies made here are released to the caching allocator after
    // the launch is enqueued on the same stream, so their memory is reused in
    // stream order only.
    raise_if(relm_mp_pack_index(desc.data(), static_cast<int32_t>(desc.size()), out_a, out_b,
                                current_stream(like)));
}

std::tuple<Tensor, Tensor> pack_index_parts(const std::vector<IndexPart>& parts,
                                            bool alias_single_b, const Tensor& like) {
    int64_t total = 0;
    for (const IndexPart& p : parts) total += p.a.numel();
    const auto opts = like.options().dtype(at::kLong);
    const bool b_alias = alias_single_b && parts.size() == 1;
    Tensor out_a = at::empty({total}, opts);
    Tensor out_b = b_alias ? parts.front().b : at::empty({total}, opts);
    if (total == 0) return std::make_tuple(out_a, out_b);
    int64_t* pb = b_alias ? nullptr : out_b.data_ptr<int64_t>();
    if (like.is_cuda()) {
        c10::DeviceGuard guard(like.device());
        pack_parts_gpu(parts, out_a.data_ptr<int64_t>(), pb, like);
    } else {
        pack_parts_cpu(parts, out_a.data_ptr<int64_t>(), pb);
    }
    return std::make_tuple(out_a, out_b);
}

// Checks of one value part shared by the four ops (mp_ops.cpp:443-466, 2543-2569).
void check_value_part(const Tensor& t, size_t i, const c10::Device& device, at::ScalarType dtype,
                      int64_t emb, const char* op, const char* part_name, const char* what) {
    check_rank(t, 2, what);
    TORCH_CHECK(t.device() == device, op, " expects all ", part_name,
                " on the same device. Mismatch at part ", i, ".");
    TORCH_CHECK(t.scalar_type() == dtype, op, " expects all ", part_name,
                " with the same dtype. Mismatch at part ", i, ".");
    TORCH_CHECK(t.size(1) == emb, op, " expects matching embedding dim across ", part_name,
                ". Part ", i, " has emb=", t.size(1), ", expected ", emb, ".");
}

Tensor cat_values(const std::vector<Tensor>& parts) {
    return parts.size() == 1 ? parts.front() : at::cat(parts, 0);
}

std::tuple<Tensor, Tensor, Tensor> pack_multi(const char* op, const char* value_name,
                                              const char* first_name, const char* second_name,
                                              const std::vector<Tensor>& values,
                                              const std::vector<Tensor>& first,
                                              const std::vector<Tensor>& second) {
    const Tensor& ref = values.front();
    check_rank(ref, 2, (std::string(value_name) + "[0]").c_str());
    const int64_t emb = ref.size(1);
    std::vector<IndexPart> parts;
    parts.reserve(values.size());
    int64_t row_offset = 0;
    const std::string vname = std::string(value_name) + "[i]";
    const std::string fname = std::string(first_name) + "_parts[i]";
    const std::string sname = std::string(second_name) + "_parts[i]";
    for (size_t i = 0; i < values.size(); ++i) {
        check_rank(values[i], 2, vname.c_str());
        check_int64_index(first[i], fname.c_str());
        check_int64_index(second[i], sname.c_str());
        check_value_part(values[i], i, ref.device(), ref.scalar_type(), emb, op, value_name,
                         vname.c_str());
        TORCH_CHECK(first[i].device() == ref.device() && second[i].device() == ref.device(), op,
                    " expects all index tensors on the same device as ", value_name, ".");
        TORCH_CHECK(first[i].size(0) == second[i].size(0), op, " expects ", first_name, " and ",
                    second_name, " lengths to match for part ", i, ".");
        parts.push_back({first[i], second[i], 1, row_offset, 1, 0});
        row_offset += values[i].size(0);
    }
    auto [a, b] = pack_index_parts(parts, /*alias_single_b=*/true, ref);
    return std::make_tuple(cat_values(values), a, b);
}

std::tuple<Tensor, Tensor, Tensor> fanout_pack_multi(const std::vector<Tensor>& x_parts,
                                                     const std::vector<Tensor>& src_idx_parts,
                                                     const std::vector<Tensor>& flat_dst_parts) {
    TORCH_CHECK(!x_parts.empty(), "fanout_pack_multi requires at least one source tensor.");
    TORCH_CHECK(x_parts.size() == src_idx_parts.size() && x_parts.size() == flat_dst_parts.size(),
                "fanout_pack_multi expects x_parts, src_idx_parts, and flat_dst_parts with equal "
                "lengths.");
    return pack_multi("fanout_pack_multi", "x_parts", "src_idx", "flat_dst", x_parts,
                      src_idx_parts, flat_dst_parts);
}

std::tuple<Tensor, Tensor, Tensor> fanin_pack_multi(const std::vector<Tensor>& rel_parts,
                                                    const std::vector<Tensor>& flat_src_parts,
                                                    const std::vector<Tensor>& dst_idx_parts) {
    TORCH_CHECK(!rel_parts.empty(), "fanin_pack_multi requires at least one relation tensor.");
    TORCH_CHECK(rel_parts.size() == flat_src_parts.size() && rel_parts.size() == dst_idx_parts.size(),
                "fanin_pack_multi expects rel_parts, flat_src_parts, and dst_idx_parts with equal "
                "lengths.");
    return pack_multi("fanin_pack_multi", "rel_parts", "flat_src", "dst_idx", rel_parts,
                      flat_src_parts, dst_idx_parts);
}

// Row offset of each value part (mp_ops.cpp:2540-2572, 2672-2704).
std::vector<int64_t> value_offsets(const char* op, const char* value_name,
                                   const std::vector<Tensor>& values) {
    const Tensor& ref = values.front();
    check_rank(ref, 2, (std::string(value_name) + "[0]").c_str());
    const std::string vname = std::string(value_name) + "[i]";
    std::vector<int64_t> offsets(values.size(), 0);
    int64_t row_offset = 0;
    for (size_t i = 0; i < values.size(); ++i) {
        check_value_part(values[i], i, ref.device(), ref.scalar_type(), ref.size(1), op,
                         value_name, vname.c_str());
        offsets[i] = row_offset;
        row_offset += values[i].size(0);
    }
    return offsets;
}

void check_edge_part(const char* op, const char* value_name, const Tensor& src, const Tensor& dst,
                     const c10::Device& device, int64_t i) {
    check_int64_index(src, "edge_src_parts[i]");
    check_int64_index(dst, "edge_dst_parts[i]");
    TORCH_CHECK(src.device() == device && dst.device() == device, op,
                " expects all edge index tensors on the same device as ", value_name, ".");
    TORCH_CHECK(src.size(0) == dst.size(0), op, " expects edge src/dst lengths to match for part ",
                i, ".");
}

std::tuple<Tensor, Tensor, Tensor> empty_edge_pack(const Tensor& values_cat, const Tensor& ref) {
    Tensor empty_idx = at::empty({0}, ref.options().dtype(at::kLong));
    return std::make_tuple(values_cat, empty_idx, empty_idx.clone());
}

std::tuple<Tensor, Tensor, Tensor> fanout_pack_from_edges(
    const std::vector<Tensor>& x_parts, const std::vector<Tensor>& edge_src_parts,
    const std::vector<Tensor>& edge_dst_parts, const std::vector<int64_t>& src_part_ids,
    const std::vector<int64_t>& arity_parts, const std::vector<int64_t>& pos_parts,
    const std::vector<int64_t>& slot_offset_parts) {
    const char* op = "fanout_pack_from_edges";
    TORCH_CHECK(!x_parts.empty(), "fanout_pack_from_edges requires at least one source tensor.");
    const size_t n_edge = edge_src_parts.size();
    TORCH_CHECK(edge_dst_parts.size() == n_edge,
                "fanout_pack_from_edges expects edge_src_parts and edge_dst_parts with equal "
                "lengths.");
    TORCH_CHECK(src_part_ids.size() == n_edge && arity_parts.size() == n_edge &&
                    pos_parts.size() == n_edge && slot_offset_parts.size() == n_edge,
                "fanout_pack_from_edges expects metadata arrays to match number of edge parts.");
    const std::vector<int64_t> offsets = value_offsets(op, "x_parts", x_parts);
    const Tensor& ref = x_parts.front();
    const Tensor x_cat = cat_values(x_parts);
    if (n_edge == 0) return empty_edge_pack(x_cat, ref);
    std::vector<IndexPart> parts;
    parts.reserve(n_edge);
    for (size_t i = 0; i < n_edge; ++i) {
        check_edge_part(op, "x_parts", edge_src_parts[i], edge_dst_parts[i], ref.device(),
                        static_cast<int64_t>(i));
        const int64_t src_part = src_part_ids[i];
        TORCH_CHECK(src_part >= 0 && src_part < static_cast<int64_t>(x_parts.size()),
                    "fanout_pack_from_edges src_part_ids[", i, "] out of range: ", src_part, ".");
        const int64_t arity = arity_parts[i], pos = pos_parts[i];
        TORCH_CHECK(arity > 0, "fanout_pack_from_edges requires arity > 0 for edge part ", i, ".");
        TORCH_CHECK(pos >= 0 && pos < arity, "fanout_pack_from_edges pos out of range for edge part ",
                    i, ": pos=", pos, " arity=", arity, ".");
        // flat_dst = slot_offset + dst * arity + pos, sums wrapping as int64 does.
        const int64_t b_add = static_cast<int64_t>(static_cast<uint64_t>(slot_offset_parts[i]) +
                                                   static_cast<uint64_t>(pos));
        parts.push_back({edge_src_parts[i], edge_dst_parts[i], 1, offsets[src_part], arity, b_add});
    }
    auto [src_global, flat_dst] = pack_index_parts(parts, /*alias_single_b=*/false, ref);
    return std::make_tuple(x_cat, src_global, flat_dst);
}

std::tuple<Tensor, Tensor, Tensor> fanin_pack_from_edges(
    const std::vector<Tensor>& rel_parts, const std::vector<Tensor>& edge_src_parts,
    const std::vector<Tensor>& edge_dst_parts, const std::vector<int64_t>& rel_part_ids,
    const std::vector<int64_t>& arity_parts, const std::vector<int64_t>& pos_parts, int64_t mode) {
    const char* op = "fanin_pack_from_edges";
    TORCH_CHECK(!rel_parts.empty(), "fanin_pack_from_edges requires at least one relation tensor.");
    TORCH_CHECK(mode == 0 || mode == 1,
                "fanin_pack_from_edges mode must be 0 (relation) or 1 (label), got ", mode, ".");
    const size_t n_edge = edge_src_parts.size();
    TORCH_CHECK(edge_dst_parts.size() == n_edge,
                "fanin_pack_from_edges expects edge_src_parts and edge_dst_parts with equal "
                "lengths.");
    TORCH_CHECK(rel_part_ids.size() == n_edge && arity_parts.size() == n_edge &&
                    pos_parts.size() == n_edge,
                "fanin_pack_from_edges expects metadata arrays to match number of edge parts.");
    const std::vector<int64_t> offsets = value_offsets(op, "rel_parts", rel_parts);
    const Tensor& ref = rel_parts.front();
    const Tensor rel_cat = cat_values(rel_parts);
    if (n_edge == 0) return empty_edge_pack(rel_cat, ref);
    std::vector<IndexPart> parts;
    parts.reserve(n_edge);
    for (size_t i = 0; i < n_edge; ++i) {
        check_edge_part(op, "rel_parts", edge_src_parts[i], edge_dst_parts[i], ref.device(),
                        static_cast<int64_t>(i));
        const int64_t rel_part = rel_part_ids[i];
        TORCH_CHECK(rel_part >= 0 && rel_part < static_cast<int64_t>(rel_parts.size()),
                    "fanin_pack_from_edges rel_part_ids[", i, "] out of range: ", rel_part, ".");
        int64_t a_mul = 1, a_add = offsets[rel_part];
        if (mode == 0) {
            const int64_t arity = arity_parts[i], pos = pos_parts[i];
            TORCH_CHECK(arity > 0,
                        "fanin_pack_from_edges requires arity > 0 in relation mode for edge part ",
                        i, ".");
            TORCH_CHECK(pos >= 0 && pos < arity,
                        "fanin_pack_from_edges pos out of range for edge part ", i, ": pos=", pos,
                        " arity=", arity, ".");
            // flat_src = (src * arity + pos) + rel_offset.
            a_mul = arity;
            a_add = static_cast<int64_t>(static_cast<uint64_t>(pos) +
                                         static_cast<uint64_t>(offsets[rel_part]));
        }
        parts.push_back({edge_src_parts[i], edge_dst_parts[i], a_mul, a_add, 1, 0});
    }
    auto [flat_src, dst_idx] = pack_index_parts(parts, /*alias_single_b=*/true, ref);
    return std::make_tuple(rel_cat, flat_src, dst_idx);
}

// ---- LGAN indexed reductions (mp_ops.cpp:3350-3743) ---------------------------
//
// Relation instances pool their slots (sum / arity), take one residual
// aggregation step over relation-relation edges and aggregate onto entities
// over two edge sets (tn, nn); sum (0) or mean (2) per destination.  GPU lane
// (float32 / float64 CUDA tensors of one dtype): every aggregation is one CSR
// segment sum (edge order inside each destination) whose result rows are
// finished as they are stored (relm_mp_plan_segment_sum_scaled: division by
// the count or arity, residual addition); the backward runs the transposed
// sums over plans keyed by the sources, with the mean's per-message division
// applied to each gathered gradient row as it is loaded
// (relm_mp_plan_segment_sum_msgdiv).  Other
// tensors: the reference's tensor sequence.

constexpr int64_t kModeMean = 2;

void check_int32_or_int64_index(const Tensor& t, const char* name) {
    check_rank(t, 1, name);
    TORCH_CHECK(t.scalar_type() == at::kLong || t.scalar_type() == at::kInt, name,
                " must have dtype torch.int64 or torch.int32.");
}

bool same_device(const Tensor& ref, std::initializer_list<const Tensor*> ts) {
    for (const Tensor* t : ts)
        if (t->device() != ref.device()) return false;
    return true;
}

// Sum (mean) of src_rows[s[e]] onto rows t[e] of a [dim, emb] result.
Tensor lgan_aggregate_aten(const Tensor& src_rows, const Tensor& s, const Tensor& t, int64_t dim,
                           int64_t mode) {
    Tensor out = at::zeros({dim, src_rows.size(1)}, src_rows.options());
    if (s.numel() == 0 || t.numel() == 0 || dim == 0) return out;
    out.index_add_(0, t, src_rows.index_select(0, s));
    if (mode == kModeMean) {
        Tensor count = at::zeros({dim, 1}, src_rows.options());
        count.index_add_(0, t, at::ones({t.size(0), 1}, src_rows.options()));
        out = out / count.clamp_min_(1.0);
    }
    return out;
}

// Transpose of lgan_aggregate_aten: rows s[e] of a [src_rows, emb] result
// receive grad[t[e]] (divided by the messages into t[e] in mean mode).
Tensor lgan_reverse_aten(const Tensor& grad, const Tensor& s, const Tensor& t, int64_t src_rows,
                         int64_t mode) {
    Tensor out = at::zeros({src_rows, grad.size(1)}, grad.options());
    if (s.numel() == 0 || t.numel() == 0 || src_rows == 0) return out;
    Tensor msgs = grad.index_select(0, t);
    if (mode == kModeMean) {
        Tensor count = at::zeros({grad.size(0), 1}, grad.options());
        count.index_add_(0, t, at::ones({t.size(0), 1}, grad.options()));
        msgs = msgs / count.index_select(0, t).clamp_min_(1.0);
    }
    out.index_add_(0, s, msgs);
    return out;
}

Tensor index64(const Tensor& t) {
    return contiguous(t.scalar_type() == at::kLong ? t : t.to(at::kLong));
}

bool lgan_gpu_lane(std::initializer_list<const Tensor*> values) {
    const Tensor& ref = **values.begin();
    if (!ref.is_cuda() || !is_fastpath_dtype(ref.scalar_type())) return false;
    for (const Tensor* v : values)
        if (v->scalar_type() != ref.scalar_type() || v->size(1) != ref.size(1)) return false;
    return true;
}

const void* ptr_or_null(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// base + (sum or mean of src_rows[s[e]] onto rows t[e]); base may be undefined.
Tensor lgan_aggregate_gpu(const Tensor& src_rows, const Tensor& s, const Tensor& t, int64_t dim,
                          int64_t mode, const Tensor& base, const char* s_name, const char* t_name,
                          hipStream_t st) {
    const int64_t D = src_rows.size(1);
    const int dt = dtype_code(src_rows);
    Tensor out = at::empty({dim, D}, src_rows.options());
    if (dim == 0 || D == 0) return out;
    if (s.numel() == 0 || t.numel() == 0) {
        raise_if(relm_mp_rows_scale(dt, nullptr, nullptr, RELM_MP_DIV_NONE, nullptr, nullptr,
                                    ptr_or_null(base), dim, D, out.data_ptr(), st));
        return out;
    }
    PlanPtr gp = csr_plan(t, dim, t_name, s, src_rows.size(0), s_name, true, st);
    Tensor scratch = compute_scratch(gp->plan, D, dt, kModeSum, src_rows);
    raise_if(relm_mp_plan_segment_sum_scaled(
        dt, &gp->plan, src_rows.data_ptr(), D,
        mode == kModeMean ? RELM_MP_DIV_SEGMENT : RELM_MP_DIV_NONE, nullptr, ptr_or_null(base),
        out.data_ptr(), scratch.data_ptr(), static_cast<size_t>(scratch.numel()), st));
    return out;
}

// base + transpose of the aggregation (s, t): rows s[e] of [src_rows, emb]
// receive grad[t[e]] (divided by the messages into t[e] in mean mode).
Tensor lgan_reverse_gpu(const Tensor& grad, const Tensor& s, const Tensor& t, int64_t src_rows,
                        int64_t mode, const Tensor& base, const char* s_name, const char* t_name,
                        hipStream_t st) {
    const int64_t D = grad.size(1);
    const int dt = dtype_code(grad);
    Tensor out = at::empty({src_rows, D}, grad.options());
    if (src_rows == 0 || D == 0) return out;
    if (s.numel() == 0 || t.numel() == 0) {
        raise_if(relm_mp_rows_scale(dt, nullptr, nullptr, RELM_MP_DIV_NONE, nullptr, nullptr,
                                    ptr_or_null(base), src_rows, D, out.data_ptr(), st));
        return out;
    }
    PlanPtr gp = csr_plan(s, src_rows, s_name, t, grad.size(0), t_name, false, st);
    Tensor scratch = compute_scratch(gp->plan, D, dt, kModeSum, grad);
    if (mode == kModeMean) {
        // each message's grad row divided by the messages into its row - the
        // segment sizes of the forward's plan - as it is loaded
        PlanPtr fwd = csr_plan(t, grad.size(0), t_name, s, src_rows, s_name, true, st);
        raise_if(relm_mp_plan_segment_sum_msgdiv(dt, &gp->plan, grad.data_ptr(), D, fwd->plan.offsets,
                                                 ptr_or_null(base), out.data_ptr(), scratch.data_ptr(),
                                                 static_cast<size_t>(scratch.numel()), st));
        return out;
    }
    raise_if(relm_mp_plan_segment_sum_scaled(dt, &gp->plan, grad.data_ptr(), D, RELM_MP_DIV_NONE,
                                             nullptr, ptr_or_null(base), out.data_ptr(),
                                             scratch.data_ptr(),
                                             static_cast<size_t>(scratch.numel()), st));
    return out;
}

struct LganEdges {
    Tensor rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent;
};

LganEdges lgan_edges64(const Tensor& rr_src, const Tensor& rr_dst, const Tensor& tn_rel,
                       const Tensor& tn_ent, const Tensor& nn_rel, const Tensor& nn_ent) {
    return {index64(rr_src), index64(rr_dst), index64(tn_rel),
            index64(tn_ent), index64(nn_rel), index64(nn_ent)};
}

std::tuple<Tensor, Tensor, Tensor> lgan_step_gpu(const Tensor& x, const LganEdges& g,
                                                 int64_t entity_dim_size, int64_t mode,
                                                 hipStream_t st) {
    const int64_t K = x.size(0);
    Tensor upd = lgan_aggregate_gpu(x, g.rr_src, g.rr_dst, K, mode, x, "rr_src", "rr_dst", st);
    Tensor tn = lgan_aggregate_gpu(upd, g.tn_rel, g.tn_ent, entity_dim_size, mode, Tensor(),
                                   "tn_rel", "tn_ent", st);
    Tensor nn = lgan_aggregate_gpu(upd, g.nn_rel, g.nn_ent, entity_dim_size, mode, Tensor(),
                                   "nn_rel", "nn_ent", st);
    return std::make_tuple(upd, tn, nn);
}

Tensor lgan_step_backward_gpu(const Tensor& g, const Tensor& g_tn, const Tensor& g_nn,
                              const LganEdges& e, int64_t K, int64_t mode, hipStream_t st) {
    Tensor g1 = lgan_reverse_gpu(g_tn, e.tn_rel, e.tn_ent, K, mode, g, "tn_rel", "tn_ent", st);
    g1 = lgan_reverse_gpu(g_nn, e.nn_rel, e.nn_ent, K, mode, g1, "nn_rel", "nn_ent", st);
    return lgan_reverse_gpu(g1, e.rr_src, e.rr_dst, K, mode, g1, "rr_src", "rr_dst", st);
}

void check_lgan_edges(const Tensor& rr_src, const Tensor& rr_dst, const Tensor& tn_rel,
                      const Tensor& tn_ent, const Tensor& nn_rel, const Tensor& nn_ent) {
    check_int32_or_int64_index(rr_src, "rr_src");
    check_int32_or_int64_index(rr_dst, "rr_dst");
    check_int32_or_int64_index(tn_rel, "tn_rel");
    check_int32_or_int64_index(tn_ent, "tn_ent");
    check_int32_or_int64_index(nn_rel, "nn_rel");
    check_int32_or_int64_index(nn_ent, "nn_ent");
}

std::tuple<Tensor, Tensor, Tensor> lgan_pool_reduce(
    const Tensor& slot_messages, const Tensor& slot_to_relation_instance,
    const Tensor& relation_instance_arities, const Tensor& rr_src, const Tensor& rr_dst,
    const Tensor& tn_rel, const Tensor& tn_ent, const Tensor& nn_rel, const Tensor& nn_ent,
    int64_t entity_dim_size, int64_t mode) {
    check_rank(slot_messages, 2, "slot_messages");
    check_int32_or_int64_index(slot_to_relation_instance, "slot_to_relation_instance");
    check_int64_index(relation_instance_arities, "relation_instance_arities");
    check_lgan_edges(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent);
    TORCH_CHECK(same_device(slot_messages, {&slot_to_relation_instance, &relation_instance_arities,
                                            &rr_src, &rr_dst, &tn_rel, &tn_ent, &nn_rel, &nn_ent}),
                "lgan_pool_reduce expects all tensors on the same device.");
    TORCH_CHECK(entity_dim_size >= 0, "entity_dim_size must be >= 0.");
    TORCH_CHECK(slot_to_relation_instance.size(0) == slot_messages.size(0),
                "slot_to_relation_instance length must match slot_messages rows.");
    TORCH_CHECK(tn_rel.size(0) == tn_ent.size(0), "tn_rel and tn_ent must have equal length.");
    TORCH_CHECK(nn_rel.size(0) == nn_ent.size(0), "nn_rel and nn_ent must have equal length.");
    TORCH_CHECK(rr_src.size(0) == rr_dst.size(0), "rr_src and rr_dst must have equal length.");
    TORCH_CHECK(mode == kModeSum || mode == kModeMean,
                "lgan_pool_reduce supports only mode 0=sum or 2=mean.");
    const int64_t K = relation_instance_arities.size(0);
    const int64_t D = slot_messages.size(1);
    if (lgan_gpu_lane({&slot_messages})) {
        c10::OptionalDeviceGuard guard(slot_messages.device());
        hipStream_t st = current_stream(slot_messages);
        const Tensor slot = contiguous(slot_messages);
        if (slot.numel() > 0 && K == 0)  // every slot's relation instance is out of range
            check_in_bounds(index64(slot_to_relation_instance)[0].item<int64_t>(), 0,
                            "slot_to_relation_instance");
        const bool pooled = slot.numel() > 0 && K > 0;
        Tensor rpx = pooled ? at::empty({K, D}, slot.options()) : at::zeros({K, D}, slot.options());
        if (pooled) {
            const Tensor s2r = index64(slot_to_relation_instance);
            PlanPtr gp = csr_plan_rows(s2r, K, "slot_to_relation_instance", st);
            const int dt = dtype_code(slot);
            Tensor scratch = compute_scratch(gp->plan, D, dt, kModeSum, slot);
            const Tensor arity = contiguous(relation_instance_arities);
            raise_if(relm_mp_plan_segment_sum_scaled(
                dt, &gp->plan, slot.data_ptr(), D, RELM_MP_DIV_VALUES, arity.data_ptr<int64_t>(),
                nullptr, rpx.data_ptr(), scratch.data_ptr(), static_cast<size_t>(scratch.numel()),
                st));
        }
        return lgan_step_gpu(rpx, lgan_edges64(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent),
                             entity_dim_size, mode, st);
    }
    Tensor rpx = slot_messages.new_zeros({K, D});
    if (slot_messages.numel() > 0) {
        rpx.index_add_(0, slot_to_relation_instance, slot_messages);
        rpx = rpx / relation_instance_arities.to(slot_messages.scalar_type()).view({K, 1}).clamp_min_(1.0);
    }
    rpx = rpx + lgan_aggregate_aten(rpx, rr_src, rr_dst, K, mode);
    return std::make_tuple(rpx, lgan_aggregate_aten(rpx, tn_rel, tn_ent, entity_dim_size, mode),
                           lgan_aggregate_aten(rpx, nn_rel, nn_ent, entity_dim_size, mode));
}

std::tuple<Tensor, Tensor, Tensor> lgan_relation_graph_step(
    const Tensor& relation_pair_x, const Tensor& rr_src, const Tensor& rr_dst,
    const Tensor& tn_rel, const Tensor& tn_ent, const Tensor& nn_rel, const Tensor& nn_ent,
    int64_t entity_dim_size, int64_t mode) {
    check_rank(relation_pair_x, 2, "relation_pair_x");
    check_lgan_edges(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent);
    TORCH_CHECK(same_device(relation_pair_x, {&rr_src, &rr_dst, &tn_rel, &tn_ent, &nn_rel, &nn_ent}),
                "lgan_relation_graph_step expects all tensors on the same device.");
    TORCH_CHECK(entity_dim_size >= 0, "entity_dim_size must be >= 0.");
    TORCH_CHECK(rr_src.size(0) == rr_dst.size(0), "rr_src and rr_dst must have equal length.");
    TORCH_CHECK(tn_rel.size(0) == tn_ent.size(0), "tn_rel and tn_ent must have equal length.");
    TORCH_CHECK(nn_rel.size(0) == nn_ent.size(0), "nn_rel and nn_ent must have equal length.");
    TORCH_CHECK(mode == kModeSum || mode == kModeMean,
                "lgan_relation_graph_step supports only mode 0=sum or 2=mean.");
    if (lgan_gpu_lane({&relation_pair_x})) {
        c10::OptionalDeviceGuard guard(relation_pair_x.device());
        return lgan_step_gpu(contiguous(relation_pair_x),
                             lgan_edges64(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent),
                             entity_dim_size, mode, current_stream(relation_pair_x));
    }
    const int64_t K = relation_pair_x.size(0);
    Tensor upd = relation_pair_x + lgan_aggregate_aten(relation_pair_x, rr_src, rr_dst, K, mode);
    return std::make_tuple(upd, lgan_aggregate_aten(upd, tn_rel, tn_ent, entity_dim_size, mode),
                           lgan_aggregate_aten(upd, nn_rel, nn_ent, entity_dim_size, mode));
}

Tensor lgan_relation_graph_step_backward(const Tensor& grad_relation_pair_x,
                                         const Tensor& grad_tn_msgs, const Tensor& grad_nn_msgs,
                                         const Tensor& rr_src, const Tensor& rr_dst,
                                         const Tensor& tn_rel, const Tensor& tn_ent,
                                         const Tensor& nn_rel, const Tensor& nn_ent,
                                         int64_t relation_count, int64_t mode) {
    check_rank(grad_relation_pair_x, 2, "grad_relation_pair_x");
    check_rank(grad_tn_msgs, 2, "grad_tn_msgs");
    check_rank(grad_nn_msgs, 2, "grad_nn_msgs");
    check_lgan_edges(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent);
    TORCH_CHECK(same_device(grad_relation_pair_x, {&grad_tn_msgs, &grad_nn_msgs, &rr_src, &rr_dst,
                                                   &tn_rel, &tn_ent, &nn_rel, &nn_ent}),
                "lgan_relation_graph_step_backward expects all tensors on the same device.");
    TORCH_CHECK(relation_count >= 0, "relation_count must be >= 0.");
    TORCH_CHECK(mode == kModeSum || mode == kModeMean,
                "lgan_relation_graph_step_backward supports only mode 0=sum or 2=mean.");
    if (lgan_gpu_lane({&grad_relation_pair_x, &grad_tn_msgs, &grad_nn_msgs}) &&
        grad_relation_pair_x.size(0) == relation_count) {
        c10::OptionalDeviceGuard guard(grad_relation_pair_x.device());
        return lgan_step_backward_gpu(contiguous(grad_relation_pair_x), contiguous(grad_tn_msgs),
                                      contiguous(grad_nn_msgs),
                                      lgan_edges64(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent),
                                      relation_count, mode, current_stream(grad_relation_pair_x));
    }
    Tensor g = grad_relation_pair_x + lgan_reverse_aten(grad_tn_msgs, tn_rel, tn_ent, relation_count, mode) +
               lgan_reverse_aten(grad_nn_msgs, nn_rel, nn_ent, relation_count, mode);
    return g + lgan_reverse_aten(g, rr_src, rr_dst, relation_count, mode);
}

Tensor lgan_pool_reduce_backward(const Tensor& grad_relation_pair_x, const Tensor& grad_tn_msgs,
                                 const Tensor& grad_nn_msgs,
                                 const Tensor& slot_to_relation_instance,
                                 const Tensor& relation_instance_arities, const Tensor& rr_src,
                                 const Tensor& rr_dst, const Tensor& tn_rel, const Tensor& tn_ent,
                                 const Tensor& nn_rel, const Tensor& nn_ent,
                                 int64_t relation_count, int64_t mode) {
    check_rank(grad_relation_pair_x, 2, "grad_relation_pair_x");
    check_rank(grad_tn_msgs, 2, "grad_tn_msgs");
    check_rank(grad_nn_msgs, 2, "grad_nn_msgs");
    check_int32_or_int64_index(slot_to_relation_instance, "slot_to_relation_instance");
    check_int64_index(relation_instance_arities, "relation_instance_arities");
    check_lgan_edges(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent);
    TORCH_CHECK(same_device(grad_relation_pair_x,
                            {&grad_tn_msgs, &grad_nn_msgs, &slot_to_relation_instance,
                             &relation_instance_arities, &rr_src, &rr_dst, &tn_rel, &tn_ent,
                             &nn_rel, &nn_ent}),
                "lgan_pool_reduce_backward expects all tensors on the same device.");
    TORCH_CHECK(mode == kModeSum || mode == kModeMean,
                "lgan_pool_reduce_backward supports only mode 0=sum or 2=mean.");
    TORCH_CHECK(relation_count >= 0, "relation_count must be >= 0.");
    if (lgan_gpu_lane({&grad_relation_pair_x, &grad_tn_msgs, &grad_nn_msgs}) &&
        grad_relation_pair_x.size(0) == relation_count) {
        c10::OptionalDeviceGuard guard(grad_relation_pair_x.device());
        hipStream_t st = current_stream(grad_relation_pair_x);
        Tensor g = lgan_step_backward_gpu(contiguous(grad_relation_pair_x), contiguous(grad_tn_msgs),
                                          contiguous(grad_nn_msgs),
                                          lgan_edges64(rr_src, rr_dst, tn_rel, tn_ent, nn_rel, nn_ent),
                                          relation_count, mode, st);
        const Tensor s2r = index64(slot_to_relation_instance);
        const int64_t E = s2r.numel(), D = g.size(1);
        Tensor grad_slot = at::empty({E, D}, g.options());
        if (E > 0) {
            // each slot reads its relation instance's row and arity
            const int64_t bound = std::min<int64_t>(relation_count, relation_instance_arities.numel());
            const auto mm = at::aminmax(s2r);
            const int64_t lo = std::get<0>(mm).item<int64_t>(), hi = std::get<1>(mm).item<int64_t>();
            if (lo < 0) check_in_bounds(lo, bound, "slot_to_relation_instance");
            check_in_bounds(hi, bound, "slot_to_relation_instance");
        }
        if (E > 0 && D > 0) {
            const Tensor arity = contiguous(relation_instance_arities);
            raise_if(relm_mp_rows_scale(dtype_code(g), g.data_ptr(), s2r.data_ptr<int64_t>(),
                                        RELM_MP_DIV_VALUES, nullptr, arity.data_ptr<int64_t>(),
                                        nullptr, E, D, grad_slot.data_ptr(), st));
        }
        return grad_slot;
    }
    Tensor g = grad_relation_pair_x + lgan_reverse_aten(grad_tn_msgs, tn_rel, tn_ent, relation_count, mode) +
               lgan_reverse_aten(grad_nn_msgs, nn_rel, nn_ent, relation_count, mode);
    g = g + lgan_reverse_aten(g, rr_src, rr_dst, relation_count, mode);
    Tensor grad_slot = g.index_select(0, slot_to_relation_instance);
    Tensor counts = relation_instance_arities.to(grad_slot.scalar_type())
                        .index_select(0, slot_to_relation_instance.to(at::kLong))
                        .view({slot_to_relation_instance.size(0), 1})
                        .clamp_min_(1.0);
    return grad_slot / counts;
}

std::string build_info() {
    return std::string("build_torch=") + RELM_MP_BUILD_TORCH_VERSION +
           ";build_cuda_tag=cpu;abi_target=rocm-gfx950;abi_lane=nonstable;" + relm_mp_build_info();
}

void plan_cache_clear() { PlanCache::get().clear(); }

int64_t plan_cache_size() { return PlanCache::get().size(); }

std::vector<int64_t> plan_cache_stats() { return PlanCache::get().stats(); }

void plan_trust_enter() { PlanCache::get().trust_enter(); }

void plan_trust_exit() { PlanCache::get().trust_exit(); }

// ---- fused FiLM step with Mish (no counterpart in the reference) ---------------
//
// y = mish(beta[k] + gamma[k] * (s + add[k])) over row ranges k of s (one
// range per predicate in a central layer); float32 GPU tensors, the tables
// [ranges, width].  The backward returns (ds, dgamma, dbeta): the gradient of
// add is gamma * dbeta.

namespace {

struct FilmArgs {
    Tensor s, gamma, beta, add;
    std::vector<int64_t> starts;
};

FilmArgs film_args(const Tensor& s, at::IntArrayRef range_start, const Tensor& gamma, const Tensor& beta,
                   const std::optional<Tensor>& add) {
    TORCH_CHECK(s.dim() == 2 && s.is_cuda() && s.scalar_type() == at::kFloat,
                "film_mish: s must be a 2-D float32 GPU tensor.");
    const int64_t k = static_cast<int64_t>(range_start.size()) - 1;
    TORCH_CHECK(k >= 1 && k <= RELM_MP_FILM_MAX_RANGES, "film_mish: 1 to ", RELM_MP_FILM_MAX_RANGES,
                " row ranges expected.");
    for (const Tensor* t : {&gamma, &beta}) {
        TORCH_CHECK(t->dim() == 2 && t->size(0) == k && t->size(1) == s.size(1) &&
                        t->scalar_type() == at::kFloat && t->device() == s.device(),
                    "film_mish: gamma and beta must be float32 [ranges, width] on the device of s.");
    }
    FilmArgs a{contiguous(s), contiguous(gamma), contiguous(beta), Tensor(),
               std::vector<int64_t>(range_start.begin(), range_start.end())};
    if (add.has_value() && add->defined()) {
        TORCH_CHECK(add->sizes() == gamma.sizes() && add->scalar_type() == at::kFloat &&
                        add->device() == s.device(),
                    "film_mish: add must be float32 [ranges, width] on the device of s.");
        a.add = contiguous(*add);
    }
    return a;
}

const float* fptr(const Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }

}  // namespace

Tensor film_mish(const Tensor& s, at::IntArrayRef range_start, const Tensor& gamma, const Tensor& beta,
                 const std::optional<Tensor>& add) {
    const FilmArgs a = film_args(s, range_start, gamma, beta, add);
    c10::OptionalDeviceGuard guard(s.device());
    Tensor y = at::empty_like(a.s);
    raise_if(relm_mp_film_mish(fptr(a.s), a.s.size(0), a.s.size(1), a.starts.data(),
                               static_cast<int32_t>(a.starts.size() - 1), fptr(a.gamma), fptr(a.beta),
                               fptr(a.add), y.data_ptr<float>(), current_stream(a.s)));
    return y;
}

std::tuple<Tensor, Tensor, Tensor> film_mish_backward(const Tensor& grad, const Tensor& s,
                                                      at::IntArrayRef range_start, const Tensor& gamma,
                                                      const Tensor& beta,
                                                      const std::optional<Tensor>& add) {
    const FilmArgs a = film_args(s, range_start, gamma, beta, add);
    TORCH_CHECK(grad.sizes() == s.sizes() && grad.scalar_type() == at::kFloat &&
                    grad.device() == s.device(),
                "film_mish_backward: grad must match s.");
    c10::OptionalDeviceGuard guard(s.device());
    const Tensor g = contiguous(grad);
    const int32_t k = static_cast<int32_t>(a.starts.size() - 1);
    const int64_t width = a.s.size(1);
    const int64_t blocks = relm_mp_film_mish_blocks(a.starts.data(), k);
    TORCH_CHECK(blocks >= 0, "film_mish_backward: bad row ranges.");
    Tensor ds = at::empty_like(a.s);
    Tensor partial = at::empty({std::max<int64_t>(blocks, 1), 2, width}, a.s.options().dtype(at::kDouble));
    raise_if(relm_mp_film_mish_backward(fptr(a.s), g.data_ptr<float>(), a.s.size(0), width,
                                        a.starts.data(), k, fptr(a.gamma), fptr(a.beta), fptr(a.add),
                                        ds.data_ptr<float>(), partial.data_ptr<double>(), blocks,
                                        current_stream(a.s)));
    // per range, the sums of its blocks (consecutive, RELM_MP_FILM_ROWS_PER_BLOCK
    // rows each) in fp64, rounded to fp32 once
    if (k == 1 && blocks > 0) {
        const Tensor sum = partial.sum(0).to(at::kFloat);  // [2, width]
        return {ds, sum.narrow(0, 0, 1), sum.narrow(0, 1, 1)};
    }
    Tensor sums = at::zeros({k, 2, width}, partial.options());
    int64_t b0 = 0;
    for (int32_t r = 0; r < k; ++r) {
        const int64_t rows = a.starts[r + 1] - a.starts[r];
        const int64_t nb = rows <= 0 ? 0 : (rows + RELM_MP_FILM_ROWS_PER_BLOCK - 1) / RELM_MP_FILM_ROWS_PER_BLOCK;
        if (nb > 0) sums[r].copy_(partial.narrow(0, b0, nb).sum(0));
        b0 += nb;
    }
    const Tensor sums32 = sums.to(at::kFloat);
    return {ds, sums32.select(1, 0), sums32.select(1, 1)};
}

// ---- a @ b^T for the models' narrow Linears (no counterpart in the reference) ----
//
// a [M, K], b [N, K], float32 on one GPU, unit column strides: a @ b^T as a
// new [M, N] tensor, through hipBLAS (rocBLAS) on torch's handle for the
// current stream.  For the tall, narrow products of the relation MLPs (M in
// the hundreds of thousands, K and N of 64 to 128) rocBLAS streams at about
// the HBM rate where the library GEMM torch picks (hipBLASLt) runs 2-3x
// slower; the caller chooses which shapes come here.
Tensor mm_nt(const Tensor& a, const Tensor& b) {
    TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && a.size(1) == b.size(1),
                "mm_nt: a [M, K] and b [N, K] expected.");
    TORCH_CHECK(a.is_cuda() && b.device() == a.device() && a.scalar_type() == at::kFloat &&
                    b.scalar_type() == at::kFloat,
                "mm_nt: float32 tensors on one GPU expected.");
    const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
    const int64_t lim = std::numeric_limits<int>::max();
    TORCH_CHECK(M <= lim && N <= lim && K <= lim, "mm_nt: sizes must fit 32 bits.");
    const Tensor A = (a.stride(1) == 1 && a.stride(0) >= std::max<int64_t>(K, 1)) ? a : a.contiguous();
    const Tensor B = (b.stride(1) == 1 && b.stride(0) >= std::max<int64_t>(K, 1)) ? b : b.contiguous();
    TORCH_CHECK(A.stride(0) <= lim && B.stride(0) <= lim, "mm_nt: row strides must fit 32 bits.");
    c10::OptionalDeviceGuard guard(a.device());
    Tensor out = at::empty({M, N}, a.options());
    if (M == 0 || N == 0) return out;
    if (K == 0) return out.zero_();
    // column-major view: out^T [N, M] = op(B) [N, K] x A^T [K, M], with B read
    // as a K x N column-major matrix (ld = its row stride) and transposed
    const float one = 1.0f, zero = 0.0f;
    hipblasHandle_t handle = at::cuda::getCurrentCUDABlasHandle();
    const hipblasStatus_t st =
        hipblasSgemm(handle, HIPBLAS_OP_T, HIPBLAS_OP_N, static_cast<int>(N), static_cast<int>(M),
                     static_cast<int>(K), &one, B.data_ptr<float>(), static_cast<int>(B.stride(0)),
                     A.data_ptr<float>(), static_cast<int>(A.stride(0)), &zero, out.data_ptr<float>(),
                     static_cast<int>(N));
    TORCH_CHECK(st == HIPBLAS_STATUS_SUCCESS, "mm_nt: hipblasSgemm failed (status ", static_cast<int>(st),
                ").");
    return out;
}

}  // namespace relm_amd

TORCH_LIBRARY(relm_mp, m) {
    m.def("fanout_scatter(Tensor x_cat, Tensor src_global_idx, Tensor flat_dst, int out_rows) -> Tensor");
    m.def("fanout_scatter_backward(Tensor grad_out, Tensor src_global_idx, Tensor flat_dst, int x_rows) -> Tensor");
    m.def("fanin_reduce(Tensor rel_flat, Tensor flat_src, Tensor dst_idx, int dim_size, int mode) -> Tensor");
    m.def("fanin_reduce_sum_backward(Tensor grad_out, Tensor flat_src, Tensor dst_idx, int rel_rows) -> Tensor");
    m.def("fanin_reduce_logsumexp_backward(Tensor grad_out, Tensor rel_flat, Tensor flat_src, Tensor dst_idx, Tensor out, int rel_rows) -> Tensor");
    m.def("fanout_pack_multi(Tensor[] x_parts, Tensor[] src_idx_parts, Tensor[] flat_dst_parts) -> (Tensor, Tensor, Tensor)");
    m.def("fanin_pack_multi(Tensor[] rel_parts, Tensor[] flat_src_parts, Tensor[] dst_idx_parts) -> (Tensor, Tensor, Tensor)");
    m.def("fanout_pack_from_edges(Tensor[] x_parts, Tensor[] edge_src_parts, Tensor[] edge_dst_parts, int[] src_part_ids, int[] arity_parts, int[] pos_parts, int[] slot_offset_parts) -> (Tensor, Tensor, Tensor)");
    m.def("fanin_pack_from_edges(Tensor[] rel_parts, Tensor[] edge_src_parts, Tensor[] edge_dst_parts, int[] rel_part_ids, int[] arity_parts, int[] pos_parts, int mode) -> (Tensor, Tensor, Tensor)");
    m.def("lgan_pool_reduce(Tensor slot_messages, Tensor slot_to_relation_instance, Tensor relation_instance_arities, Tensor rr_src, Tensor rr_dst, Tensor tn_rel, Tensor tn_ent, Tensor nn_rel, Tensor nn_ent, int entity_dim_size, int mode) -> (Tensor, Tensor, Tensor)");
    m.def("lgan_pool_reduce_backward(Tensor grad_relation_pair_x, Tensor grad_tn_msgs, Tensor grad_nn_msgs, Tensor slot_to_relation_instance, Tensor relation_instance_arities, Tensor rr_src, Tensor rr_dst, Tensor tn_rel, Tensor tn_ent, Tensor nn_rel, Tensor nn_ent, int relation_count, int mode) -> Tensor");
    m.def("lgan_relation_graph_step(Tensor relation_pair_x, Tensor rr_src, Tensor rr_dst, Tensor tn_rel, Tensor tn_ent, Tensor nn_rel, Tensor nn_ent, int entity_dim_size, int mode) -> (Tensor, Tensor, Tensor)");
    m.def("lgan_relation_graph_step_backward(Tensor grad_relation_pair_x, Tensor grad_tn_msgs, Tensor grad_nn_msgs, Tensor rr_src, Tensor rr_dst, Tensor tn_rel, Tensor tn_ent, Tensor nn_rel, Tensor nn_ent, int relation_count, int mode) -> Tensor");
    m.def("fanout_scatter_into(Tensor x_cat, Tensor src_global_idx, Tensor flat_dst, Tensor(a!) out, int col_offset, int slots) -> ()");
    m.def("fanout_scatter_backward_from(Tensor grad, Tensor src_global_idx, Tensor flat_dst, int x_rows, int col_offset, int slots, int emb) -> Tensor");
    m.def("build_info() -> str");
    // No reference counterpart: the forward's index plan handed to the backward.
    m.class_<relm_amd::PlanRef>("PlanRef");
    m.def("fanin_reduce_planned(Tensor rel_flat, Tensor flat_src, Tensor dst_idx, int dim_size, int mode) -> (Tensor, __torch__.torch.classes.relm_mp.PlanRef)");
    m.def("fanin_reduce_sum_backward_planned(Tensor grad_out, Tensor flat_src, Tensor dst_idx, int rel_rows, __torch__.torch.classes.relm_mp.PlanRef plan) -> Tensor");
    m.def("fanin_reduce_logsumexp_backward_planned(Tensor grad_out, Tensor rel_flat, Tensor flat_src, Tensor dst_idx, Tensor out, int rel_rows, __torch__.torch.classes.relm_mp.PlanRef plan) -> Tensor");
    // No reference counterpart: control of the index-plan cache.
    m.def("plan_cache_clear() -> ()");
    m.def("plan_cache_size() -> int");
    m.def("plan_cache_stats() -> int[]");
    m.def("plan_trust_enter() -> ()");
    m.def("plan_trust_exit() -> ()");
    m.def("film_mish(Tensor s, int[] range_start, Tensor gamma, Tensor beta, Tensor? add) -> Tensor");
    m.def("film_mish_backward(Tensor grad, Tensor s, int[] range_start, Tensor gamma, Tensor beta, Tensor? add) -> (Tensor, Tensor, Tensor)");
    m.def("mm_nt(Tensor a, Tensor b) -> Tensor");
}

TORCH_LIBRARY_IMPL(relm_mp, CompositeImplicitAutograd, m) {
    m.impl("fanout_scatter", relm_amd::fanout_scatter);
    m.impl("fanout_scatter_backward", relm_amd::fanout_scatter_backward);
    m.impl("fanin_reduce", relm_amd::fanin_reduce);
    m.impl("fanin_reduce_sum_backward", relm_amd::fanin_reduce_sum_backward);
    m.impl("fanin_reduce_logsumexp_backward", relm_amd::fanin_reduce_logsumexp_backward);
    m.impl("fanout_pack_multi", relm_amd::fanout_pack_multi);
    m.impl("fanin_pack_multi", relm_amd::fanin_pack_multi);
    m.impl("fanout_pack_from_edges", relm_amd::fanout_pack_from_edges);
    m.impl("fanin_pack_from_edges", relm_amd::fanin_pack_from_edges);
    m.impl("lgan_pool_reduce", relm_amd::lgan_pool_reduce);
    m.impl("lgan_pool_reduce_backward", relm_amd::lgan_pool_reduce_backward);
    m.impl("lgan_relation_graph_step", relm_amd::lgan_relation_graph_step);
    m.impl("lgan_relation_graph_step_backward", relm_amd::lgan_relation_graph_step_backward);
    m.impl("fanout_scatter_into", relm_amd::fanout_scatter_into);
    m.impl("fanout_scatter_backward_from", relm_amd::fanout_scatter_backward_from);
    m.impl("build_info", relm_amd::build_info);
    m.impl("fanin_reduce_planned", relm_amd::fanin_reduce_planned);
    m.impl("fanin_reduce_sum_backward_planned", relm_amd::fanin_reduce_sum_backward_planned);
    m.impl("fanin_reduce_logsumexp_backward_planned",
           relm_amd::fanin_reduce_logsumexp_backward_planned);
    m.impl("plan_cache_clear", relm_amd::plan_cache_clear);
    m.impl("plan_cache_size", relm_amd::plan_cache_size);
    m.impl("plan_cache_stats", relm_amd::plan_cache_stats);
    m.impl("plan_trust_enter", relm_amd::plan_trust_enter);
    m.impl("plan_trust_exit", relm_amd::plan_trust_exit);
    m.impl("film_mish", relm_amd::film_mish);
    m.impl("film_mish_backward", relm_amd::film_mish_backward);
    m.impl("mm_nt", relm_amd::mm_nt);
}
