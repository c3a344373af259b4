// MI355XBackend: DeviceBackend over libpxk_gfx950 (include/pxk.h).
#include "pulsatrix/mi355x_backend.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iterator>
#include <new>
#include <stdexcept>
#include <string>

namespace pulsatrix {

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

void* raw_alloc(size_t bytes) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();  // clear the sticky out-of-memory status before a retry
        throw std::bad_alloc();
    }
    hip_check(e, "MI355XBackend::allocate (hipMalloc)");
    return p;
}

void raw_free(void* p) { (void)hipFree(p); }

pxk_operand op(const float* p, int64_t ld) { return pxk_operand{p, ld, 0, 0, 0, 0}; }

constexpr size_t kReduceFloats = 1024 + 64;

}  // namespace

// ---- MI355XBackend -------------------------------------------------------------------------------

MI355XBackend::MI355XBackend(int device_index) : device_(device_index) {
    int count = 0;
    hip_check(hipGetDeviceCount(&count), "MI355XBackend: hipGetDeviceCount");
    if (device_index < 0 || device_index >= count)
        throw std::runtime_error("MI355XBackend: no HIP device " + std::to_string(device_index));
    hip_check(hipSetDevice(device_index), "MI355XBackend: hipSetDevice");
    hipStream_t s = nullptr;
    hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "MI355XBackend: hipStreamCreate");
    stream_ = s;
    size_t budget = 0;
    if (const char* mb = std::getenv("PULSATRIX_HIP_MEMORY_BUDGET_MB")) budget = std::strtoull(mb, nullptr, 10) << 20;
    const char* debug = std::getenv("PULSATRIX_HIP_SYNC_DEBUG");
    sync_debug_ = debug != nullptr && std::string(debug) == "1";
    allocator_ = std::make_unique<CachingAllocator>(
        raw_alloc, raw_free, [this] { hip_check(hipStreamSynchronize(S(stream_)), "MI355XBackend (allocator)"); },
        budget);
    reduce_ = static_cast<float*>(allocator_->allocate(kReduceFloats * sizeof(float)));
}

MI355XBackend::~MI355XBackend() {
    if (stream_) (void)hipStreamSynchronize(S(stream_));
    allocator_.reset();  // synchronizes, then returns every block, before the stream goes away
    if (stream_) (void)hipStreamDestroy(S(stream_));
}

void MI355XBackend::check(int rc, const char* what) {
    if (rc == PXK_OK) return;
    const std::string msg = std::string(what) + ": " + pxk_last_error();
    if (rc == PXK_ERR_INVALID) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void MI355XBackend::synchronize() { hip_check(hipStreamSynchronize(S(stream_)), "MI355XBackend::synchronize"); }

void* MI355XBackend::allocate(size_t bytes) {
    if (bytes == 0) return nullptr;
    void* p = nullptr;
    try {
        p = allocator_->allocate(bytes);
    } catch (const std::bad_alloc&) {
        throw std::runtime_error("MI355XBackend::allocate: failed to allocate " + std::to_string(bytes) + " bytes");
    }
    return track(p, owner_);
}

void MI355XBackend::free(void* ptr) noexcept {
    if (ptr == nullptr) return;
    untrack(ptr);
    // Kernels queued on the stream may still read the block; the allocator only recycles it to
    // later work on the same in-order stream, so no wait is needed.
    allocator_->free(ptr);
}

void* MI355XBackend::track(void* p, uint64_t owner) {
    try {
        blocks_.emplace(p, Block{++allocations_, owner});
    } catch (...) {
        allocator_->free(p);
        throw;
    }
    return p;
}

void MI355XBackend::untrack(void* p) noexcept {
    const auto it = blocks_.find(p);
    if (it == blocks_.end()) return;
    const Block b = it->second;
    blocks_.erase(it);
    if (capturing_) ++frees_in_capture_;
    if (b.owner == kSharedOwner) {
        if (b.serial <= shared_captured_serial_) ++shared_retired_;
        return;
    }
    const auto o = owners_.find(b.owner);
    if (o != owners_.end() && b.serial <= o->second.captured_serial) ++o->second.retired;
}

void MI355XBackend::snapshot(uint64_t owner, uint64_t& owner_retired, uint64_t& shared_retired) {
    OwnerState& st = owners_[owner];
    st.captured_serial = allocations_;
    shared_captured_serial_ = allocations_;
    owner_retired = st.retired;
    shared_retired = shared_retired_;
}

bool MI355XBackend::unchanged(uint64_t owner, uint64_t owner_retired, uint64_t shared_retired) const noexcept {
    const auto o = owners_.find(owner);
    return o != owners_.end() && o->second.retired == owner_retired && shared_retired_ == shared_retired;
}

void MI355XBackend::forget_owner(uint64_t owner) {
    owners_.erase(owner);
    if (owner_ == owner) owner_ = 0;
}

void MI355XBackend::copy(void* dst, const void* src, size_t bytes, CopyDirection dir) {
    if (bytes == 0) return;
    hipMemcpyKind kind = hipMemcpyDeviceToDevice;
    switch (dir) {
        case CopyDirection::HostToDevice: kind = hipMemcpyHostToDevice; break;
        case CopyDirection::DeviceToHost: kind = hipMemcpyDeviceToHost; break;
        case CopyDirection::DeviceToDevice: kind = hipMemcpyDeviceToDevice; break;
        case CopyDirection::HostToHost: std::memcpy(dst, src, bytes); return;
    }
    const bool word_aligned = reinterpret_cast<uintptr_t>(dst) % sizeof(float) == 0 &&
                              reinterpret_cast<uintptr_t>(src) % sizeof(float) == 0;
    if (kind == hipMemcpyDeviceToDevice && bytes % sizeof(float) == 0 && word_aligned) {
        // A copy kernel rather than an SDMA copy: it stays inside a captured graph.
        check(pxk_copy_2d(static_cast<float*>(dst), 0, static_cast<const float*>(src), 0, 1,
                          static_cast<int64_t>(bytes / sizeof(float)), stream_),
              "MI355XBackend::copy");
        return;
    }
    hip_check(hipMemcpyAsync(dst, src, bytes, kind, S(stream_)), "MI355XBackend::copy");
    if (kind != hipMemcpyDeviceToDevice) synchronize();  // host copies synchronize (hip_backend.hip:102-110)
}

void MI355XBackend::fill(void* ptr, float value, size_t n) {
    check(pxk_fill(static_cast<float*>(ptr), value, static_cast<int64_t>(n), stream_), "MI355XBackend::fill");
}

float* MI355XBackend::workspace(size_t bytes) {
    if (bytes > ws_bytes_) {
        if (ws_ && logging_) {
            retired_ws_.push_back(ws_);  // a logged GEMM still points at it
        } else if (ws_) {
            untrack(ws_);
            allocator_->free(ws_);
        }
        ws_ = nullptr;
        ws_bytes_ = std::max(bytes, ws_bytes_ * 2);
        ws_ = static_cast<float*>(track(allocator_->allocate(ws_bytes_), kSharedOwner));
    }
    return ws_;
}

void MI355XBackend::run_gemm(pxk_gemm_desc& d) {
    const size_t need = pxk_gemm_workspace(&d);
    if (need > 0) {
        d.workspace = workspace(need);
        d.workspace_bytes = ws_bytes_;
    }
    check(pxk_gemm(&d, stream_), "MI355XBackend gemm");
    if (logging_) {
        int32_t tile = 0, splits = 0;
        check(pxk_gemm_plan(&d, &tile, &splits), "MI355XBackend gemm (plan)");
        static const char* const kTile[] = {"auto",   "128x128", "64x64",  "32x64",  "32x32",
                                            "32x64d", "32x32d",  "skinny", "32x48d", "32x48"};
        char name[96];
        std::snprintf(name, sizeof(name), "gemm %s %s%s pro%d epi%d split%d", kTile[tile >= 0 && tile <= 9 ? tile : 0],
                      d.trans_a ? "T" : "N", d.trans_b ? "T" : "N", d.prologue, d.epilogue, splits);
        // Algorithmic bytes: every operand once (A, B, the prologue's denominators, the
        // epilogue's inputs and outputs), none of the split-K partials or re-reads.
        const double bt = static_cast<double>(d.batch), g = static_cast<double>(d.kgroups);
        const double mn = static_cast<double>(d.m) * d.n * bt, mk = static_cast<double>(d.m) * d.k * g * bt;
        const double kn = static_cast<double>(d.k) * d.n * g * (d.b.batch_stride || d.b.inner_stride ? bt : 1.0);
        double floats = mk + kn + (d.z.ptr && d.prologue != PXK_PRO_NONE ? mk : 0.0);
        for (const pxk_operand* o : {&d.c, &d.c2, &d.c3, &d.x, &d.y, &d.w, &d.z2, &d.z3, &d.c2_den})
            if (o->ptr) floats += mn;
        if (d.z.ptr && d.prologue == PXK_PRO_NONE) floats += mn;  // the RoPE / value rules read Z like C
        if (d.epilogue == PXK_EPI_STORE && d.beta != 0.0f) floats += mn;  // C read back
        if (d.x_rms) floats += static_cast<double>(d.m) * bt;                // the rows' rms
        if (d.x_gamma) floats += static_cast<double>(d.n);                  // the norm's gains
        if (d.row_rms) floats += static_cast<double>(d.m) * bt;              // rms written out
        const pxk_gemm_desc copy = d;
        if (owner_ != 0) log_owner_ = owner_;
        log_.push_back(LaunchRecord{name, "gemm", 2.0 * d.m * d.n * d.k * d.batch * d.kgroups, 4.0 * floats,
                                    [copy](void* st) { return pxk_gemm(&copy, st); }});
    }
    if (sync_debug_) synchronize();
}

void MI355XBackend::start_launch_log() {
    log_.clear();
    for (float* w : retired_ws_) {
        untrack(w);
        allocator_->free(w);
    }
    retired_ws_.clear();
    logging_ = true;
    log_owner_ = owner_;
}

void MI355XBackend::stop_launch_log() {
    if (!logging_) return;
    logging_ = false;
    snapshot(log_owner_, log_owner_retired_, log_shared_retired_);
}

void MI355XBackend::time_launch_log(int reps, std::vector<double>& seconds) {
    const size_t n = log_.size();
    seconds.assign(n, 0.0);
    if (n == 0 || reps <= 0) return;
    if (logging_) throw std::logic_error("MI355XBackend::time_launch_log: the launch log is still open");
    if (!unchanged(log_owner_, log_owner_retired_, log_shared_retired_))
        throw std::logic_error("MI355XBackend::time_launch_log: device memory the logged launches address was "
                               "freed since the log closed; record the pass again");
    for (const auto& r : log_) check(r.run(stream_), "MI355XBackend::time_launch_log (warm-up)");
    // Each dispatch records its own start and end (pxk_timing_*), so a launch's time is its kernels'
    // durations as the GPU ran them, in the order and cache state of the recorded pass.
    const int capacity = static_cast<int>(8 * n + 64);
    std::vector<int> first(n + 1);
    std::vector<float> ms(static_cast<size_t>(capacity));
    for (int rep = 0; rep < reps; ++rep) {
        check(pxk_timing_begin(capacity), "MI355XBackend::time_launch_log");
        try {
            for (size_t i = 0; i < n; ++i) {
                first[i] = pxk_timing_count();
                check(log_[i].run(stream_), "MI355XBackend::time_launch_log");
            }
        } catch (...) {
            (void)pxk_timing_end(ms.data(), capacity);
            throw;
        }
        first[n] = pxk_timing_count();
        check(pxk_timing_end(ms.data(), capacity), "MI355XBackend::time_launch_log");
        if (first[n] >= capacity) throw std::runtime_error("MI355XBackend::time_launch_log: timing window too small");
        for (size_t i = 0; i < n; ++i) {
            for (int k = first[i]; k < first[i + 1]; ++k) seconds[i] += 1e-3 * ms[static_cast<size_t>(k)] / reps;
            log_[i].dispatches = first[i + 1] - first[i];
        }
    }
}

void MI355XBackend::gemm(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) {
    gemm_ex(a, false, b, false, out, m, k, n, 0.0f);
}

void MI355XBackend::gemm_ex(const float* a, bool ta, const float* b, bool tb, float* out, size_t m, size_t k,
                            size_t n, float beta) {
    if (m == 0 || n == 0) return;
    pxk_gemm_desc d{};
    d.m = static_cast<int64_t>(m);
    d.n = static_cast<int64_t>(n);
    d.k = static_cast<int64_t>(k);
    d.batch = d.inner = d.kgroups = 1;
    d.trans_a = ta;
    d.trans_b = tb;
    d.epilogue = PXK_EPI_STORE;
    d.beta = beta;
    d.a = op(a, ta ? d.m : d.k);
    d.b = op(b, tb ? d.k : d.n);
    d.c = op(out, d.n);
    run_gemm(d);
}

void MI355XBackend::gemm_strided_batched(const float* a, bool ta, size_t stride_a, const float* b, bool tb,
                                         size_t stride_b, float* out, size_t stride_out, size_t m, size_t k, size_t n,
                                         size_t batch, float beta) {
    if (m == 0 || n == 0 || batch == 0) return;
    pxk_gemm_desc d{};
    d.m = static_cast<int64_t>(m);
    d.n = static_cast<int64_t>(n);
    d.k = static_cast<int64_t>(k);
    d.batch = static_cast<int64_t>(batch);
    d.inner = d.kgroups = 1;
    d.trans_a = ta;
    d.trans_b = tb;
    d.epilogue = PXK_EPI_STORE;
    d.beta = beta;
    d.a = pxk_operand{a, ta ? d.m : d.k, static_cast<int64_t>(stride_a), 0, 0, 0};
    d.b = pxk_operand{b, tb ? d.k : d.n, static_cast<int64_t>(stride_b), 0, 0, 0};
    d.c = pxk_operand{out, d.n, static_cast<int64_t>(stride_out), 0, 0, 0};
    run_gemm(d);
}

void MI355XBackend::elementwise(ElementwiseOp o, const float* in, float* out, size_t n) {
    check(pxk_elementwise(static_cast<int>(o), in, out, static_cast<int64_t>(n), stream_), "MI355XBackend::elementwise");
}

void MI355XBackend::add(const float* a, const float* b, float* out, size_t n) {
    check(pxk_add(a, b, out, static_cast<int64_t>(n), stream_), "MI355XBackend::add");
}

void MI355XBackend::mul(const float* a, const float* b, float* out, size_t n) {
    check(pxk_mul(a, b, out, static_cast<int64_t>(n), stream_), "MI355XBackend::mul");
}

void MI355XBackend::column_sums(const float* in, float* out, size_t rows, size_t cols, float beta) {
    check(pxk_column_sums(in, out, static_cast<int64_t>(rows), static_cast<int64_t>(cols), beta, stream_),
          "MI355XBackend::column_sums");
}

void MI355XBackend::add_row_vector(const float* in, const float* row, float* out, size_t rows, size_t cols) {
    check(pxk_add_row_vector(in, row, out, static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::add_row_vector");
}

void MI355XBackend::axpby(float alpha, const float* x, float beta, const float* y, float* out, size_t n) {
    check(pxk_axpby(alpha, x, beta, y, out, static_cast<int64_t>(n), stream_), "MI355XBackend::axpby");
}

float MI355XBackend::dot(const float* a, const float* b, size_t n) {
    check(pxk_dot(a, b, static_cast<int64_t>(n), reduce_ + 1024, reduce_, stream_), "MI355XBackend::dot");
    float out = 0.0f;
    hip_check(hipMemcpyAsync(&out, reduce_ + 1024, sizeof(float), hipMemcpyDeviceToHost, S(stream_)),
              "MI355XBackend::dot");
    synchronize();
    return out;
}

void MI355XBackend::dot_into(const float* a, const float* b, size_t n, float* out) {
    float* partials = static_cast<float*>(allocator_->allocate(pxk_reduce_partials(static_cast<int64_t>(n))));
    check(pxk_dot(a, b, static_cast<int64_t>(n), out, partials, stream_), "MI355XBackend::dot_into");
    allocator_->free(partials);
}

float MI355XBackend::sum(const float* in, size_t n) {
    check(pxk_sum(in, static_cast<int64_t>(n), reduce_ + 1024, reduce_, stream_), "MI355XBackend::sum");
    float out = 0.0f;
    hip_check(hipMemcpyAsync(&out, reduce_ + 1024, sizeof(float), hipMemcpyDeviceToHost, S(stream_)),
              "MI355XBackend::sum");
    synchronize();
    return out;
}

void MI355XBackend::softmax_rows(const float* in, float* out, size_t rows, size_t cols) {
    check(pxk_softmax_rows(in, out, static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::softmax_rows");
}

void MI355XBackend::rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, size_t rows,
                                     size_t cols, float eps) {
    check(pxk_rms_norm_forward(in, gamma, out, row_rms, static_cast<int64_t>(rows), static_cast<int64_t>(cols), eps,
                               stream_),
          "MI355XBackend::rms_norm_forward");
}

void MI355XBackend::rope_rotate(const float* in, const float* cos_table, const float* sin_table, float* out,
                                size_t num_slices, size_t seq_len, size_t head_dim, bool inverse, bool rotate_half) {
    check(pxk_rope_rotate(in, cos_table, sin_table, out, static_cast<int64_t>(num_slices),
                          static_cast<int64_t>(seq_len), static_cast<int64_t>(head_dim), inverse, rotate_half,
                          stream_),
          "MI355XBackend::rope_rotate");
}

void MI355XBackend::permute_0213(const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3) {
    check(pxk_permute_0213(in, out, static_cast<int64_t>(d0), static_cast<int64_t>(d1), static_cast<int64_t>(d2),
                           static_cast<int64_t>(d3), stream_),
          "MI355XBackend::permute_0213");
}

void MI355XBackend::attention_mask_fill(float* scores, const float* key_keep, size_t batch, size_t heads,
                                        size_t q_len, size_t k_len, bool causal, size_t q_offset, size_t window,
                                        float value) {
    check(pxk_attention_mask_fill(scores, key_keep, static_cast<int64_t>(batch), static_cast<int64_t>(heads),
                                  static_cast<int64_t>(q_len), static_cast<int64_t>(k_len), causal,
                                  static_cast<int64_t>(q_offset), static_cast<int64_t>(window), value, stream_),
          "MI355XBackend::attention_mask_fill");
}

void MI355XBackend::gather_rows(const float* table, const float* indices, float* out, size_t count, size_t dim) {
    check(pxk_gather_rows(table, indices, out, static_cast<int64_t>(count), static_cast<int64_t>(dim), stream_),
          "MI355XBackend::gather_rows");
}

void MI355XBackend::lrp_linear(const float* x, const float* w, const float* z, const float* r, float* r_in,
                               size_t rows, size_t in_features, size_t out_features, float eps) {
    // r_in = x * ((r / stab(z)) W^T): the per-term divide of lrp_math.hpp:21-30 factored out of
    // the sum, one fused MFMA GEMM (DIV_STAB prologue, MUL_X epilogue).
    if (rows == 0 || in_features == 0) return;
    pxk_gemm_desc d{};
    d.m = static_cast<int64_t>(rows);
    d.n = static_cast<int64_t>(in_features);
    d.k = static_cast<int64_t>(out_features);
    d.batch = d.inner = d.kgroups = 1;
    d.trans_b = 1;
    d.prologue = PXK_PRO_DIV_STAB;
    d.epilogue = PXK_EPI_MUL_X;
    d.eps = eps;
    d.a = op(r, d.k);
    d.z = op(z, d.k);
    d.b = op(w, d.k);
    d.c = op(r_in, d.n);
    d.x = op(x, d.n);
    run_gemm(d);
}

void MI355XBackend::lrp_residual_split(const float* a, const float* b, const float* r, float* r_a, float* r_b,
                                       size_t n, float eps) {
    check(pxk_lrp_residual_split(a, b, r, r_a, r_b, static_cast<int64_t>(n), eps, stream_),
          "MI355XBackend::lrp_residual_split");
}

void MI355XBackend::lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* r_out, size_t n,
                                             float eps) {
    check(pxk_lrp_bilinear_elementwise(a, b, r, r_out, static_cast<int64_t>(n), eps, stream_),
          "MI355XBackend::lrp_bilinear_elementwise");
}

void MI355XBackend::lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a,
                                        float* r_b, size_t slices, size_t m, size_t p, size_t q, float eps,
                                        bool b_transposed) {
    // GEMM form of Eq. 15 (lrp_math.hpp:57-86): s = R / (2 O + eps sign O);
    // r_a = A * (s B^T); r_b = B * (A^T s) (or B^T * (s^T A) when B is stored transposed).
    if (slices == 0 || m == 0 || p == 0 || q == 0) return;
    const int64_t M = static_cast<int64_t>(m), P = static_cast<int64_t>(p), Q = static_cast<int64_t>(q);
    const int64_t B = static_cast<int64_t>(slices);
    float* s = static_cast<float*>(allocate(static_cast<size_t>(B * M * Q) * sizeof(float)));
    check(pxk_lrp_bilinear_scale(r_o, o, s, B * M * Q, eps, stream_), "MI355XBackend::lrp_bilinear_matmul");
    pxk_gemm_desc d{};
    d.batch = B;
    d.inner = d.kgroups = 1;
    d.epilogue = PXK_EPI_MUL_X;
    // r_a (M x P) = A (M x P) * [s (M x Q) @ B^T (Q x P)]
    d.m = M;
    d.n = P;
    d.k = Q;
    d.trans_b = b_transposed ? 0 : 1;
    d.a = pxk_operand{s, Q, M * Q, 0, 0, 0};
    d.b = pxk_operand{b, P, P * Q, 0, 0, 0};  // stored (P x Q) read as N x K, or (Q x P) as K x N
    if (!b_transposed) d.b.ld = Q;
    d.c = pxk_operand{r_a, P, M * P, 0, 0, 0};
    d.x = pxk_operand{a, P, M * P, 0, 0, 0};
    run_gemm(d);
    // r_b, in B's stored layout
    pxk_gemm_desc e{};
    e.batch = B;
    e.inner = e.kgroups = 1;
    e.epilogue = PXK_EPI_MUL_X;
    e.trans_a = 1;
    e.k = M;
    if (!b_transposed) {  // (P x Q) = B * (A^T s)
        e.m = P;
        e.n = Q;
        e.a = pxk_operand{a, P, M * P, 0, 0, 0};
        e.b = pxk_operand{s, Q, M * Q, 0, 0, 0};
        e.c = pxk_operand{r_b, Q, P * Q, 0, 0, 0};
        e.x = pxk_operand{b, Q, P * Q, 0, 0, 0};
    } else {  // (Q x P) = B^T * (s^T A)
        e.m = Q;
        e.n = P;
        e.a = pxk_operand{s, Q, M * Q, 0, 0, 0};
        e.b = pxk_operand{a, P, M * P, 0, 0, 0};
        e.c = pxk_operand{r_b, P, P * Q, 0, 0, 0};
        e.x = pxk_operand{b, P, P * Q, 0, 0, 0};
    }
    run_gemm(e);
    free(s);
}

void MI355XBackend::lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, size_t rows,
                                     size_t cols) {
    check(pxk_lrp_softmax_rows(x, y, r, r_in, static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::lrp_softmax_rows");
}

void MI355XBackend::lrp_rope(const float* x, const float* y, const float* r, const float* cos_table,
                             const float* sin_table, float* r_in, size_t slices, size_t seq_len, size_t head_dim,
                             float eps, bool rotate_half) {
    check(pxk_lrp_rope(x, y, r, cos_table, sin_table, r_in, static_cast<int64_t>(slices), static_cast<int64_t>(seq_len),
                       static_cast<int64_t>(head_dim), eps, rotate_half, stream_),
          "MI355XBackend::lrp_rope");
}

void MI355XBackend::lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, size_t n,
                                          float eps, LrpGate gate_mode) {
    check(pxk_lrp_stabilized_divide(r, denom, gate, out, static_cast<int64_t>(n), eps, static_cast<int>(gate_mode),
                                    stream_),
          "MI355XBackend::lrp_stabilized_divide");
}

void MI355XBackend::copy_2d(float* dst, size_t dst_stride, const float* src, size_t src_stride, size_t rows,
                            size_t cols) {
    check(pxk_copy_2d(dst, static_cast<int64_t>(dst_stride), src, static_cast<int64_t>(src_stride),
                      static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::copy_2d");
}

void MI355XBackend::accumulate_rows(const float* in, float* out, size_t rows, size_t cols) {
    check(pxk_accumulate_rows(in, out, static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::accumulate_rows");
}

// ---- graphs ------------------------------------------------------------------------------------

std::unique_ptr<CapturedGraph> MI355XBackend::capture(uint64_t owner, const std::function<void()>& work) {
    if (owner == 0) throw std::invalid_argument("MI355XBackend::capture: no owner");
    if (capturing_) throw std::logic_error("MI355XBackend::capture: a capture is already in progress");
    const uint64_t prev_owner = set_owner(owner);
    hip_check(hipStreamBeginCapture(S(stream_), hipStreamCaptureModeThreadLocal), "MI355XBackend::capture");
    capturing_ = true;
    frees_in_capture_ = 0;
    hipGraph_t g = nullptr;
    try {
        work();
    } catch (...) {
        capturing_ = false;
        (void)hipStreamEndCapture(S(stream_), &g);
        if (g) (void)hipGraphDestroy(g);
        // A runtime call the capture refused leaves its status behind as the thread's last error;
        // clear it, or the next launch would report it.
        (void)hipGetLastError();
        set_owner(prev_owner);
        throw;
    }
    capturing_ = false;
    set_owner(prev_owner);
    hip_check(hipStreamEndCapture(S(stream_), &g), "MI355XBackend::capture (end)");
    if (frees_in_capture_ != 0) {
        (void)hipGraphDestroy(g);
        throw std::logic_error("MI355XBackend::capture: the captured work freed " + std::to_string(frees_in_capture_) +
                               " device block(s) that its launches may address; run it once eagerly at the same "
                               "shapes before capturing");
    }
    hipGraphExec_t e = nullptr;
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip_check(rc, "MI355XBackend::capture (instantiate)");
    std::unique_ptr<CapturedGraph> out(new CapturedGraph());
    out->be_ = this;
    out->exec_ = e;
    out->owner_ = owner;
    snapshot(owner, out->owner_retired_, out->shared_retired_);
    return out;
}

CapturedGraph::~CapturedGraph() {
    if (exec_) {
        (void)hipStreamSynchronize(S(be_->stream()));  // a replay may still be running
        (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec_));
    }
}

bool CapturedGraph::valid() const noexcept { return be_->unchanged(owner_, owner_retired_, shared_retired_); }

void CapturedGraph::replay() {
    if (!valid())
        throw std::logic_error("replay: device memory the captured graph addresses was freed or reallocated since "
                               "the capture (a longer pass regrew a buffer, or the split-K pool grew); capture again");
    hip_check(hipGraphLaunch(static_cast<hipGraphExec_t>(exec_), S(be_->stream())), "replay");
}

// ---- outside the path ---------------------------------------------------------------------------

void MI355XBackend::elementwise_backward(ElementwiseOp o, const float* x, const float* grad_out, float* grad_in,
                                         size_t n) {
    check(pxk_elementwise_backward(static_cast<int>(o), x, grad_out, grad_in, static_cast<int64_t>(n), stream_),
          "MI355XBackend::elementwise_backward");
}
void MI355XBackend::softmax_rows_backward(const float* y, const float* dy, float* dx, size_t rows, size_t cols) {
    check(pxk_softmax_rows_backward(y, dy, dx, static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::softmax_rows_backward");
}
void MI355XBackend::logsumexp_rows(const float* in, float* out, size_t rows, size_t cols) {
    check(pxk_logsumexp_rows(in, out, static_cast<int64_t>(rows), static_cast<int64_t>(cols), stream_),
          "MI355XBackend::logsumexp_rows");
}
void MI355XBackend::adam_step(float* param, const float* grad, float* m, float* v, size_t n, float lr, float beta1,
                              float beta2, float eps, float bias_correction1, float bias_correction2) {
    check(pxk_adam_step(param, grad, m, v, static_cast<int64_t>(n), lr, beta1, beta2, eps, bias_correction1,
                        bias_correction2, stream_),
          "MI355XBackend::adam_step");
}
void MI355XBackend::dropout_forward(const float* in, float* out, float* mask, size_t n, float p, float scale,
                                    uint64_t seed, uint64_t offset) {
    check(pxk_dropout_forward(in, out, mask, static_cast<int64_t>(n), p, scale, seed, offset, stream_),
          "MI355XBackend::dropout_forward");
}
void MI355XBackend::bce_with_logits(const float* logits, const float* target, float* out, size_t n) {
    check(pxk_bce_with_logits(logits, target, out, static_cast<int64_t>(n), 0, 1.0f, stream_),
          "MI355XBackend::bce_with_logits");
}
void MI355XBackend::bce_with_logits_grad(const float* logits, const float* target, float* grad, size_t n, float scale) {
    check(pxk_bce_with_logits(logits, target, grad, static_cast<int64_t>(n), 1, scale, stream_),
          "MI355XBackend::bce_with_logits_grad");
}
void MI355XBackend::layer_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                                       float* row_std, size_t rows, size_t cols, float eps) {
    check(pxk_layer_norm_forward(in, gamma, beta, xhat, out, row_std, static_cast<int64_t>(rows),
                                 static_cast<int64_t>(cols), eps, stream_),
          "MI355XBackend::layer_norm_forward");
}
void MI355XBackend::layer_norm_backward(const float* grad_out, const float* gamma, const float* xhat,
                                        const float* row_std, float* grad_in, size_t rows, size_t cols) {
    check(pxk_layer_norm_backward(grad_out, gamma, xhat, row_std, grad_in, static_cast<int64_t>(rows),
                                  static_cast<int64_t>(cols), stream_),
          "MI355XBackend::layer_norm_backward");
}
void MI355XBackend::rms_norm_backward(const float* grad_out, const float* gamma, const float* in, const float* row_rms,
                                      float* grad_in, float* gamma_terms, size_t rows, size_t cols) {
    check(pxk_rms_norm_backward(grad_out, gamma, in, row_rms, grad_in, gamma_terms, static_cast<int64_t>(rows),
                                static_cast<int64_t>(cols), stream_),
          "MI355XBackend::rms_norm_backward");
}
void MI355XBackend::scatter_add_rows(const float* src, const float* indices, float* table, size_t count, size_t dim) {
    check(pxk_scatter_add_rows(src, indices, table, static_cast<int64_t>(count), static_cast<int64_t>(dim), stream_),
          "MI355XBackend::scatter_add_rows");
}
void MI355XBackend::tanh_gaussian_forward(const float* mean, const float* log_std, const float* eps, float* action,
                                          float* std_cache, float* log_prob, size_t rows, size_t cols,
                                          float stabilizer, double half_log_two_pi) {
    check(pxk_tanh_gaussian_forward(mean, log_std, eps, action, std_cache, log_prob, static_cast<int64_t>(rows),
                                    static_cast<int64_t>(cols), stabilizer, half_log_two_pi, stream_),
          "MI355XBackend::tanh_gaussian_forward");
}
void MI355XBackend::tanh_gaussian_backward(const float* action, const float* std_cache, const float* eps,
                                           const float* grad_action, const float* grad_log_prob, float* grad_mean,
                                           float* grad_log_std, size_t n, float stabilizer) {
    check(pxk_tanh_gaussian_backward(action, std_cache, eps, grad_action, grad_log_prob, grad_mean, grad_log_std,
                                     static_cast<int64_t>(n), stabilizer, stream_),
          "MI355XBackend::tanh_gaussian_backward");
}
void MI355XBackend::logic_pointwise(LogicOp op, int norm, const float* a, const float* b, const float* g_or_r,
                                    const float* y, float* out_a, float* out_b, size_t n, float eps) {
    check(pxk_logic_pointwise(static_cast<int>(op), norm, a, b, g_or_r, y, out_a, out_b, static_cast<int64_t>(n), eps,
                              stream_),
          "MI355XBackend::logic_pointwise");
}
void MI355XBackend::aggregator_forward(const float* x, float* mean_pow, float* out, size_t n, size_t cols, float p) {
    check(pxk_aggregator_forward(x, mean_pow, out, static_cast<int64_t>(n), static_cast<int64_t>(cols), p, stream_),
          "MI355XBackend::aggregator_forward");
}
void MI355XBackend::aggregator_backward(const float* x, const float* mean_pow, const float* grad_out, float* grad_in,
                                        size_t n, size_t cols, float p) {
    check(pxk_aggregator_backward(x, mean_pow, grad_out, grad_in, static_cast<int64_t>(n), static_cast<int64_t>(cols), p,
                                  stream_),
          "MI355XBackend::aggregator_backward");
}
void MI355XBackend::aggregator_lrp(const float* x, const float* mean_pow, const float* r_out, float* r_in, size_t n,
                                   size_t cols, float p, float eps) {
    check(pxk_aggregator_lrp(x, mean_pow, r_out, r_in, static_cast<int64_t>(n), static_cast<int64_t>(cols), p, eps,
                             stream_),
          "MI355XBackend::aggregator_lrp");
}

namespace {
pxk_conv_geometry geometry(const ConvGeometry& g) {
    return pxk_conv_geometry{static_cast<int64_t>(g.kh),       static_cast<int64_t>(g.kw),
                             static_cast<int64_t>(g.stride_h), static_cast<int64_t>(g.stride_w),
                             static_cast<int64_t>(g.pad_h),    static_cast<int64_t>(g.pad_w)};
}
int64_t i64(size_t v) { return static_cast<int64_t>(v); }
}  // namespace

void MI355XBackend::im2col(const float* in, float* col, size_t n, size_t c, size_t h, size_t w,
                           const ConvGeometry& geometry_) {
    const pxk_conv_geometry g = geometry(geometry_);
    check(pxk_im2col(in, col, i64(n), i64(c), i64(h), i64(w), &g, stream_), "MI355XBackend::im2col");
}
void MI355XBackend::col2im_add(const float* col, float* out, size_t n, size_t c, size_t h, size_t w,
                               const ConvGeometry& geometry_) {
    const pxk_conv_geometry g = geometry(geometry_);
    check(pxk_col2im_add(col, out, i64(n), i64(c), i64(h), i64(w), &g, stream_), "MI355XBackend::col2im_add");
}
void MI355XBackend::add_channel_vector(const float* in, const float* vec, float* out, size_t n, size_t c, size_t inner) {
    check(pxk_add_channel_vector(in, vec, out, i64(n), i64(c), i64(inner), stream_), "MI355XBackend::add_channel_vector");
}
void MI355XBackend::lrp_conv(const float* col, const float* kernel, const float* pre_bias, const float* r, float* r_col,
                             size_t n, size_t out_channels, size_t p, size_t q, float eps) {
    check(pxk_lrp_conv(col, kernel, pre_bias, r, r_col, i64(n), i64(out_channels), i64(p), i64(q), eps, stream_),
          "MI355XBackend::lrp_conv");
}
void MI355XBackend::max_pool_forward(const float* in, float* out, float* argmax, size_t planes, size_t h, size_t w,
                                     size_t kh, size_t kw, size_t sh, size_t sw, size_t ph, size_t pw) {
    check(pxk_max_pool_forward(in, out, argmax, i64(planes), i64(h), i64(w), i64(kh), i64(kw), i64(sh), i64(sw), i64(ph),
                               i64(pw), stream_),
          "MI355XBackend::max_pool_forward");
}
void MI355XBackend::max_unpool(const float* src, const float* argmax, float* dst, size_t planes, size_t h, size_t w,
                               size_t kh, size_t kw, size_t sh, size_t sw, size_t ph, size_t pw) {
    check(pxk_max_unpool(src, argmax, dst, i64(planes), i64(h), i64(w), i64(kh), i64(kw), i64(sh), i64(sw), i64(ph),
                         i64(pw), stream_),
          "MI355XBackend::max_unpool");
}
void MI355XBackend::avg_pool_forward(const float* in, float* out, size_t planes, size_t h, size_t w, size_t kh,
                                     size_t kw) {
    check(pxk_avg_pool_forward(in, out, i64(planes), i64(h), i64(w), i64(kh), i64(kw), stream_),
          "MI355XBackend::avg_pool_forward");
}
void MI355XBackend::avg_pool_backward(const float* grad_out, float* grad_in, size_t planes, size_t h, size_t w,
                                      size_t kh, size_t kw) {
    check(pxk_avg_pool_backward(grad_out, grad_in, i64(planes), i64(h), i64(w), i64(kh), i64(kw), stream_),
          "MI355XBackend::avg_pool_backward");
}
void MI355XBackend::lrp_avg_pool(const float* x, const float* r, float* r_in, size_t planes, size_t h, size_t w,
                                 size_t kh, size_t kw, float eps) {
    check(pxk_lrp_avg_pool(x, r, r_in, i64(planes), i64(h), i64(w), i64(kh), i64(kw), eps, stream_),
          "MI355XBackend::lrp_avg_pool");
}
void MI355XBackend::batch_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                                       float* channel_std, size_t n, size_t c, size_t spatial, float eps) {
    check(pxk_batch_norm_forward(in, gamma, beta, xhat, out, channel_std, i64(n), i64(c), i64(spatial), eps, stream_),
          "MI355XBackend::batch_norm_forward");
}
void MI355XBackend::batch_norm_backward(const float* grad_out, const float* gamma, const float* xhat,
                                        const float* channel_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                        size_t n, size_t c, size_t spatial) {
    check(pxk_batch_norm_backward(grad_out, gamma, xhat, channel_std, grad_in, gamma_grad, beta_grad, i64(n), i64(c),
                                  i64(spatial), stream_),
          "MI355XBackend::batch_norm_backward");
}
void MI355XBackend::batch_norm_update_running(const float* in, float* running_mean, float* running_var, size_t n,
                                              size_t c, size_t spatial, float momentum) {
    check(pxk_batch_norm_update_running(in, running_mean, running_var, i64(n), i64(c), i64(spatial), momentum, stream_),
          "MI355XBackend::batch_norm_update_running");
}
void MI355XBackend::batch_norm_eval_forward(const float* in, const float* gamma, const float* beta,
                                            const float* running_mean, const float* running_var, float* xhat,
                                            float* out, float* channel_std, size_t n, size_t c, size_t spatial,
                                            float eps) {
    check(pxk_batch_norm_eval_forward(in, gamma, beta, running_mean, running_var, xhat, out, channel_std, i64(n), i64(c),
                                      i64(spatial), eps, stream_),
          "MI355XBackend::batch_norm_eval_forward");
}
void MI355XBackend::batch_norm_eval_backward(const float* grad_out, const float* gamma, const float* xhat,
                                             const float* channel_std, float* grad_in, float* gamma_grad,
                                             float* beta_grad, size_t n, size_t c, size_t spatial) {
    check(pxk_batch_norm_eval_backward(grad_out, gamma, xhat, channel_std, grad_in, gamma_grad, beta_grad, i64(n), i64(c),
                                       i64(spatial), stream_),
          "MI355XBackend::batch_norm_eval_backward");
}
void MI355XBackend::group_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                                       float* group_std, size_t n, size_t c, size_t spatial, size_t num_groups,
                                       float eps) {
    check(pxk_group_norm_forward(in, gamma, beta, xhat, out, group_std, i64(n), i64(c), i64(spatial), i64(num_groups),
                                 eps, stream_),
          "MI355XBackend::group_norm_forward");
}
void MI355XBackend::group_norm_backward(const float* grad_out, const float* gamma, const float* xhat,
                                        const float* group_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                        size_t n, size_t c, size_t spatial, size_t num_groups) {
    check(pxk_group_norm_backward(grad_out, gamma, xhat, group_std, grad_in, gamma_grad, beta_grad, i64(n), i64(c),
                                  i64(spatial), i64(num_groups), stream_),
          "MI355XBackend::group_norm_backward");
}
void MI355XBackend::recurrent_cell(RecurrentCellOp op, const RecurrentCellArgs& args, size_t n) {
    pxk_recurrent_args a{};
    std::copy(std::begin(args.in), std::end(args.in), a.in);
    std::copy(std::begin(args.out), std::end(args.out), a.out);
    a.eps = args.eps;
    check(pxk_recurrent_cell(static_cast<int>(op), &a, i64(n), stream_), "MI355XBackend::recurrent_cell");
}
void MI355XBackend::gru_lrp_hprev(const float* h_prev, const float* w_hn, const float* hn, const float* r_term_b,
                                  const float* direct, float* r_hprev, size_t rows, size_t hidden, float eps) {
    check(pxk_gru_lrp_hprev(h_prev, w_hn, hn, r_term_b, direct, r_hprev, i64(rows), i64(hidden), eps, stream_),
          "MI355XBackend::gru_lrp_hprev");
}
void MI355XBackend::ssm_pass(SsmPassOp op, const SsmPassArgs& args) {
    pxk_ssm_args a{};
    std::copy(std::begin(args.in), std::end(args.in), a.in);
    std::copy(std::begin(args.out), std::end(args.out), a.out);
    a.n = args.n;
    a.l = args.l;
    a.d = args.d;
    a.s = args.s;
    a.eps = args.eps;
    a.gamma = args.gamma;
    check(pxk_ssm_pass(static_cast<int>(op), &a, stream_), "MI355XBackend::ssm_pass");
}
void MI355XBackend::rl_rows(RlRowOp op, const RlRowArgs& args) {
    pxk_rl_args a{};
    std::copy(std::begin(args.in), std::end(args.in), a.in);
    std::copy(std::begin(args.out), std::end(args.out), a.out);
    a.rows = args.rows;
    a.cols = args.cols;
    a.scale = args.scale;
    a.lower = args.lower;
    a.upper = args.upper;
    a.gamma = args.gamma;
    a.tau = args.tau;
    a.ignore_index = args.ignore_index;
    check(pxk_rl_rows(static_cast<int>(op), &a, stream_), "MI355XBackend::rl_rows");
}
void MI355XBackend::top_k_rows(const float* in, float* values, float* indices, size_t rows, size_t cols, size_t k,
                               bool largest) {
    check(pxk_top_k_rows(in, values, indices, static_cast<int64_t>(rows), static_cast<int64_t>(cols),
                         static_cast<int64_t>(k), largest, stream_),
          "MI355XBackend::top_k_rows");
}

}  // namespace pulsatrix
