// The ROCm backend: MI355X (gfx950) devices behind mensurflow's Backend/Buffer/Stream interface
// (src/backends/backend.hpp), with kernel adapters for the fp32 BLAS hot path. It reaches HIP
// only through the C ABI of include/mfr_rocm.h (libmfr_rocm.so): no HIP header is included
// here. Patterned on the reference's GPU backends: errors become exceptions carrying the
// runtime's message (src/backends/cuda/backend.cpp:22-34), one stream per device created lazily
// under a mutex (:222-229), zero devices when the runtime is missing (:200-220).
//
// Kernel adapters read tensor strides directly, so transposed, sliced and broadcast views reach
// the GPU without a host round trip; an operand without a unit stride is first packed on the
// device (OpId::StridedCopy).
#include "backends/backend.hpp"
#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "core/tensor_access.hpp"
#include "mfr_rocm.h"

#include <algorithm>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace mensurflow::detail {

namespace {

// Status -> the exception the reference throws for the same failure.
void check(int status) {
    if (status == MFR_OK) {
        return;
    }
    const std::string message = mfr_last_error();
    if (status == MFR_E_INVALID) {
        throw std::invalid_argument(message);
    }
    if (status == MFR_E_UNSUPPORTED) {
        throw NotImplemented(message);
    }
    throw std::runtime_error(message);
}

// Device memory blocks of one device kept for reuse. Every kernel and copy of a device runs on
// that device's one stream (RocmBackend::stream), in order, so a block a Buffer releases can serve
// the next allocation at once: work on the new tensor is queued after the work that used the old
// one. Without the pool each released tensor would reach hipFree, which waits for the whole
// device, so dropping a temporary would stall the host until the GPU is idle.
// Blocks come in size classes (powers of two below 1 MiB, at least 512 B; multiples of 2 MiB
// above). Idle blocks are kept up to 1/8 of the device's memory; past that a released block is
// freed. An allocation that fails frees every idle block and tries again.
class BlockPool {
  public:
    explicit BlockPool(int device) : device_(device) {
        std::size_t bytes = 0;
        if (mfr_get_device_info(device, nullptr, 0, &bytes, nullptr, nullptr) == MFR_OK) {
            limit_ = std::max<std::size_t>(bytes / 8, std::size_t{1} << 30);
        }
    }
    ~BlockPool() { release_idle(); }
    BlockPool(const BlockPool&) = delete;
    BlockPool& operator=(const BlockPool&) = delete;

    static std::size_t size_class(std::size_t bytes) {
        constexpr std::size_t kSmall = std::size_t{1} << 20;
        constexpr std::size_t kLargeStep = std::size_t{2} << 20;
        if (bytes >= kSmall) {
            return (bytes + kLargeStep - 1) / kLargeStep * kLargeStep;
        }
        std::size_t size = 512;
        while (size < bytes) {
            size *= 2;
        }
        return size;
    }

    // A block of `size` bytes (a size class): an idle one, else a new allocation.
    void* take(std::size_t size) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            auto found = idle_.find(size);
            if (found != idle_.end() && !found->second.empty()) {
                void* block = found->second.back();
                found->second.pop_back();
                idle_bytes_ -= size;
                return block;
            }
        }
        void* block = nullptr;
        if (mfr_malloc(device_, size, &block) != MFR_OK) {
            release_idle();
            check(mfr_malloc(device_, size, &block));
        }
        return block;
    }

    void give(std::size_t size, void* block) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            if (idle_bytes_ + size <= limit_) {
                idle_[size].push_back(block);
                idle_bytes_ += size;
                return;
            }
        }
        (void)mfr_free(device_, block); // errors ignored, as the reference's buffer destructor
    }

    void release_idle() {
        std::unordered_map<std::size_t, std::vector<void*>> blocks;
        {
            std::lock_guard<std::mutex> lock(mutex_);
            blocks.swap(idle_);
            idle_bytes_ = 0;
        }
        for (auto& [size, list] : blocks) {
            for (void* block : list) {
                (void)mfr_free(device_, block);
            }
        }
    }

  private:
    int device_;
    std::size_t limit_ = std::size_t{1} << 30;
    std::mutex mutex_;
    std::unordered_map<std::size_t, std::vector<void*>> idle_;
    std::size_t idle_bytes_ = 0;
};

// A tensor's device memory: a pool block (a zero-byte buffer has none and a null pointer).
class RocmBuffer final : public Buffer {
  public:
    RocmBuffer(std::shared_ptr<BlockPool> pool, std::size_t bytes)
        : pool_(std::move(pool)), size_(bytes) {
        if (bytes > 0) {
            block_ = BlockPool::size_class(bytes);
            data_ = pool_->take(block_);
        }
    }
    ~RocmBuffer() override {
        if (data_ != nullptr) {
            pool_->give(block_, data_);
        }
    }
    RocmBuffer(const RocmBuffer&) = delete;
    RocmBuffer& operator=(const RocmBuffer&) = delete;
    std::size_t size() const override { return size_; }
    void* native() const override { return data_; }

  private:
    std::shared_ptr<BlockPool> pool_; // outlives every buffer taken from it
    std::size_t size_;
    std::size_t block_ = 0;
    void* data_ = nullptr;
};

std::byte* bytes_of(const Buffer& buffer) { return static_cast<std::byte*>(buffer.native()); }

class RocmStream final : public Stream {
  public:
    explicit RocmStream(int device) { check(mfr_stream_create(device, &stream_)); }
    ~RocmStream() override { (void)mfr_stream_destroy(stream_); }
    RocmStream(const RocmStream&) = delete;
    RocmStream& operator=(const RocmStream&) = delete;

    void copy_h2d(Buffer& dst, std::size_t offset, const void* src, std::size_t bytes) override {
        check(mfr_memcpy_h2d(stream_, bytes_of(dst) + offset, src, bytes));
    }
    void copy_d2h(void* dst, const Buffer& src, std::size_t offset, std::size_t bytes) override {
        check(mfr_memcpy_d2h(stream_, dst, bytes_of(src) + offset, bytes));
    }
    void copy_d2d(Buffer& dst, std::size_t dst_offset, const Buffer& src, std::size_t src_offset,
                  std::size_t bytes) override {
        check(mfr_memcpy_d2d(stream_, bytes_of(dst) + dst_offset, bytes_of(src) + src_offset,
                             bytes));
    }
    void synchronize() override { check(mfr_stream_sync(stream_)); }

    mfr_stream_t handle() const { return stream_; }

  private:
    mfr_stream_t stream_ = nullptr;
};

mfr_stream_t handle(Stream& stream) { return static_cast<RocmStream&>(stream).handle(); }

template <typename T> T* ptr(const Tensor& t) { return TensorAccess::data<T>(t); }

// The address of a tensor's first element whatever its dtype (TensorAccess::data<T> counts the
// offset in sizeof(T) steps, so a byte pointer needs the element size here).
std::byte* first_byte(const Tensor& t) {
    return static_cast<std::byte*>(TensorAccess::buffer(t).native()) +
           static_cast<std::size_t>(t.offset()) * t.itemsize();
}

// ---- GEMM family -------------------------------------------------------------------------------

// A matrix operand the GEMM kernel can read: a unit stride in one of its two dimensions (or an
// extent of 1 there). Otherwise a packed copy on the device.
Tensor readable_matrix(const Tensor& t) {
    const int nd = t.dim();
    const auto& s = t.strides();
    const bool rows_unit = s[nd - 2] == 1 || t.size(-2) == 1;
    const bool cols_unit = s[nd - 1] == 1 || t.size(-1) == 1;
    return rows_unit || cols_unit ? t : t.contiguous();
}

void fill_matrix(mfr_gemm_desc& d, const Tensor& a, const Tensor& b, const Tensor& out) {
    d.m = out.size(-2);
    d.n = out.size(-1);
    d.k = a.size(-1);
    d.a = ptr<float>(a);
    d.a_rs = a.strides()[a.dim() - 2];
    d.a_cs = a.strides()[a.dim() - 1];
    d.b = ptr<float>(b);
    d.b_rs = b.strides()[b.dim() - 2];
    d.b_cs = b.strides()[b.dim() - 1];
    d.c = ptr<float>(out);
    d.c_rs = out.size(-1);
    d.alpha = 1.0f;
    d.beta = 0.0f;
    d.act = MFR_ACT_NONE;
}

// The tuner's choice for this call (TunableKernel params "tile", "stage", "splits"; none =
// AUTO).
void apply_tuning(mfr_gemm_desc& d, const TuningConfig& tuning) {
    if (tuning.size >= 3) {
        d.tile = static_cast<std::int32_t>(tuning.values[0]);
        d.stage = static_cast<std::int32_t>(tuning.values[1]);
        d.splits = static_cast<std::int32_t>(tuning.values[2]);
    }
}

// OpId::Matmul: op(a) [m,k] and op(b) [k,n] as views; out contiguous [m,n].
// OpId::Gemm: the same, then c0 [m,n] when beta != 0, then bias [n] when has_bias.
// `a` and `b` are the readable forms of inputs[0] and inputs[1].
mfr_gemm_desc matrix_desc(OpId op, const OpArgs& args, const Tensor& a, const Tensor& b) {
    const Tensor& out = args.outputs[0];
    mfr_gemm_desc d{};
    fill_matrix(d, a, b, out);
    if (op == OpId::Gemm) {
        d.alpha = args.alpha;
        d.beta = args.beta;
        std::size_t next = 2;
        if (args.beta != 0.0f) {
            d.c0 = ptr<float>(args.inputs[next++]);
            d.c0_rs = out.size(-1);
        }
        if (args.has_bias) {
            d.bias = ptr<float>(args.inputs[next]);
        }
        d.act = args.activation;
    }
    apply_tuning(d, args.tuning);
    return d;
}

void matmul_kernel(const OpArgs& args, Stream& stream) {
    const Tensor a = readable_matrix(args.inputs[0]);
    const Tensor b = readable_matrix(args.inputs[1]);
    const mfr_gemm_desc d = matrix_desc(OpId::Matmul, args, a, b);
    check(mfr_sgemm(handle(stream), &d));
}

void gemm_kernel(const OpArgs& args, Stream& stream) {
    const Tensor a = readable_matrix(args.inputs[0]);
    const Tensor b = readable_matrix(args.inputs[1]);
    const mfr_gemm_desc d = matrix_desc(OpId::Gemm, args, a, b);
    check(mfr_sgemm(handle(stream), &d));
}

// OpId::GemmBatched: a [batch..., m, k] and b [batch..., k, n] as views with the full batch shape
// (stride 0 on broadcast dimensions), out contiguous, and c0 (contiguous, out's shape) when
// beta != 0. Batch dimensions that step through memory together are merged, size-1 dimensions
// dropped; the innermost MFR_MAX_BATCH_DIMS go into one launch's descriptor, any left are
// walked on the host, one launch per index (`outer`).
struct BatchDim {
    std::int64_t size, a, b, c, c0;
};

struct BatchedCall {
    mfr_gemm_desc desc{};
    std::vector<BatchDim> outer;
};

BatchedCall batched_desc(const OpArgs& args, const Tensor& a, const Tensor& b) {
    const Tensor& out = args.outputs[0];
    const bool with_c0 = args.inputs.size() > 2;
    const Tensor* c0 = with_c0 ? &args.inputs[2] : nullptr;
    const int batch_dims = out.dim() - 2;
    std::vector<BatchDim> dims;
    for (int d = 0; d < batch_dims; ++d) {
        const auto du = static_cast<std::size_t>(d);
        const BatchDim dim{out.size(d), a.strides()[du], b.strides()[du], out.strides()[du],
                           c0 != nullptr ? c0->strides()[du] : 0};
        if (dim.size == 1) {
            continue;
        }
        if (!dims.empty()) {
            BatchDim& prev = dims.back();
            if (prev.a == dim.size * dim.a && prev.b == dim.size * dim.b &&
                prev.c == dim.size * dim.c && prev.c0 == dim.size * dim.c0) {
                prev.size *= dim.size;
                prev.a = dim.a;
                prev.b = dim.b;
                prev.c = dim.c;
                prev.c0 = dim.c0;
                continue;
            }
        }
        dims.push_back(dim);
    }
    BatchedCall call;
    mfr_gemm_desc& d = call.desc;
    fill_matrix(d, a, b, out);
    d.alpha = args.alpha;
    d.beta = with_c0 ? args.beta : 0.0f;
    if (with_c0) {
        d.c0 = ptr<float>(*c0);
        d.c0_rs = out.size(-1);
    }
    const std::size_t inner = std::min<std::size_t>(dims.size(), MFR_MAX_BATCH_DIMS);
    const std::size_t outer = dims.size() - inner;
    d.batch_dims = static_cast<std::int32_t>(inner);
    for (std::size_t i = 0; i < inner; ++i) {
        const BatchDim& dim = dims[outer + i];
        d.batch[i] = dim.size;
        d.a_bs[i] = dim.a;
        d.b_bs[i] = dim.b;
        d.c_bs[i] = dim.c;
        d.c0_bs[i] = dim.c0;
    }
    call.outer.assign(dims.begin(), dims.begin() + static_cast<std::ptrdiff_t>(outer));
    d.flags = args.causal ? MFR_GEMM_CAUSAL : 0;
    apply_tuning(d, args.tuning);
    return call;
}

void gemm_batched_kernel(const OpArgs& args, Stream& stream) {
    const Tensor a = readable_matrix(args.inputs[0]);
    const Tensor b = readable_matrix(args.inputs[1]);
    BatchedCall call = batched_desc(args, a, b);
    mfr_gemm_desc& d = call.desc;
    std::int64_t launches = 1;
    for (const BatchDim& dim : call.outer) {
        launches *= dim.size;
    }
    const float* a0 = d.a;
    const float* b0 = d.b;
    float* c_base = d.c;
    const float* c0_base = d.c0;
    for (std::int64_t l = 0; l < launches; ++l) {
        std::int64_t rest = l, oa = 0, ob = 0, oc = 0, oc0 = 0;
        for (std::size_t i = call.outer.size(); i-- > 0;) {
            const std::int64_t idx = rest % call.outer[i].size;
            rest /= call.outer[i].size;
            oa += idx * call.outer[i].a;
            ob += idx * call.outer[i].b;
            oc += idx * call.outer[i].c;
            oc0 += idx * call.outer[i].c0;
        }
        d.a = a0 + oa;
        d.b = b0 + ob;
        d.c = c_base + oc;
        d.c0 = c0_base != nullptr ? c0_base + oc0 : nullptr;
        check(mfr_sgemm(handle(stream), &d));
    }
}

// ---- tuning ------------------------------------------------------------------------------------
//
// The GEMM kernels' settings a tuner may choose (the reference's TunableKernel,
// src/core/dispatcher.hpp:226-239, registered as the Metal matmul is,
// src/backends/metal/backend.mm:231-289): params {"tile", "stage", "splits"} = the workgroup
// tile (MFR_TILE_*, the thin path included), operand staging (MFR_STAGE_NEVER /
// MFR_STAGE_ALWAYS) and the depth ranges of split-K (1 = none). The defaults {0, 0, 0} leave all
// three to the kernel (AUTO). The space is one region whose start is what AUTO picks for the
// call (mfr_sgemm_plan), with the tiles ordered by area (the thin path first) and the split
// counts by size, so neighbours on an axis are neighbours in effect; a point is allowed when
// mfr_sgemm_plan accepts it and runs that many ranges (a count the depth is too short for runs
// fewer, the same as a smaller point; the thin path only where it takes the product, unsplit).

// The descriptor the kernel for `op` would launch with for these args.
mfr_gemm_desc planned_desc(OpId op, const OpArgs& args) {
    const Tensor a = readable_matrix(args.inputs[0]);
    const Tensor b = readable_matrix(args.inputs[1]);
    return op == OpId::GemmBatched ? batched_desc(args, a, b).desc : matrix_desc(op, args, a, b);
}

TuningConfig tuning_of(std::int64_t tile, std::int64_t stage, std::int64_t splits) {
    TuningConfig config;
    config.values[0] = tile;
    config.values[1] = stage;
    config.values[2] = splits;
    config.size = 3;
    return config;
}

template <OpId Op> std::vector<std::int64_t> gemm_key(const OpArgs& args) {
    const Tensor& out = args.outputs[0];
    std::int64_t batch = 1;
    for (int d = 0; d + 2 < out.dim(); ++d) {
        batch *= out.size(d);
    }
    const std::int64_t m = out.size(-2), n = out.size(-1), k = args.inputs[0].size(-1);
    if (Op == OpId::GemmBatched) {
        return {batch, m, n, k};
    }
    return {m, n, k};
}

template <OpId Op> std::vector<SearchRegion> gemm_space(const OpArgs& args) {
    mfr_gemm_desc d = planned_desc(Op, args);
    d.tile = MFR_TILE_AUTO;
    d.stage = MFR_STAGE_AUTO;
    d.splits = 0;
    std::int32_t tile = 0, stage = 0, splits = 0, regions = 0;
    check(mfr_sgemm_plan(args.outputs[0].device().index, &d, &tile, &stage, &splits, &regions));
    if (tile == MFR_TILE_AUTO) {
        return {}; // nothing to compute: nothing to tune
    }
    SearchRegion region;
    region.name = "mfma";
    region.start = tuning_of(tile, stage, splits);
    region.axes = {{0, {MFR_TILE_THIN, MFR_TILE_64x64, MFR_TILE_128x64, MFR_TILE_64x128,
                        MFR_TILE_128x128, MFR_TILE_256x256, MFR_TILE_PANEL}},
                   {1, {MFR_STAGE_NEVER, MFR_STAGE_ALWAYS}},
                   {2, {1, 2, 4, 8, 16, 32}}};
    return {region};
}

template <OpId Op> bool gemm_allowed(const OpArgs& args, const TuningConfig& config) {
    if (config.size != 3 || config.values[0] <= MFR_TILE_AUTO ||
        config.values[0] >= MFR_TILE_COUNT ||
        (config.values[1] != MFR_STAGE_NEVER && config.values[1] != MFR_STAGE_ALWAYS) ||
        config.values[2] < 1 || config.values[2] > MFR_MAX_SPLITS) {
        return false;
    }
    OpArgs tuned = args;
    tuned.tuning = config;
    const mfr_gemm_desc d = planned_desc(Op, tuned);
    std::int32_t tile = 0, stage = 0, splits = 0, regions = 0;
    return mfr_sgemm_plan(args.outputs[0].device().index, &d, &tile, &stage, &splits,
                          &regions) == MFR_OK &&
           splits == config.values[2];
}

template <OpId Op> TunableKernel gemm_tunable(const char* name) {
    TunableKernel t;
    t.name = name;
    t.version = 2;
    t.key_names = Op == OpId::GemmBatched ? std::vector<std::string>{"batch", "m", "n", "k"}
                                          : std::vector<std::string>{"m", "n", "k"};
    t.key = gemm_key<Op>;
    t.params = {"tile", "stage", "splits"};
    t.defaults = [] { return tuning_of(MFR_TILE_AUTO, MFR_STAGE_AUTO, 0); };
    t.space = gemm_space<Op>;
    t.allowed = gemm_allowed<Op>;
    return t;
}

// ---- attention ---------------------------------------------------------------------------------

// OpId::Attention: q [batch..., lq, d], k and v [batch..., lk, dv] as views with the full batch
// shape (stride 0 on broadcast dimensions), then the Bool mask [batch..., lq, lk] when has_mask;
// out contiguous [batch..., lq, dv]; alpha is the scale. Batch dimensions of extent 1 are
// dropped. A layout the fused kernel does not take throws NotImplemented, and the op composes.
void attention_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& q = args.inputs[0];
    const Tensor& k = args.inputs[1];
    const Tensor& v = args.inputs[2];
    const Tensor* mask = args.has_mask ? &args.inputs[3] : nullptr;
    const Tensor& out = args.outputs[0];
    const int nd = out.dim();
    const auto row = static_cast<std::size_t>(nd - 2);
    const auto col = static_cast<std::size_t>(nd - 1);
    if (v.size(-1) != q.size(-1)) {
        throw NotImplemented("attention: fused kernel needs v's width equal to d");
    }
    for (const Tensor* t : {&q, &k, &v}) {
        if (t->strides()[col] != 1 && t->size(-1) != 1) {
            throw NotImplemented("attention: fused kernel needs unit stride along d");
        }
    }
    mfr_attention_desc d{};
    d.lq = q.size(-2);
    d.lk = k.size(-2);
    d.d = q.size(-1);
    int dims = 0;
    for (std::size_t i = 0; i < row; ++i) {
        if (out.shape()[i] == 1) {
            continue;
        }
        if (dims == MFR_MAX_BATCH_DIMS) {
            throw NotImplemented("attention: more than " + std::to_string(MFR_MAX_BATCH_DIMS) +
                                 " batch dimensions for the fused kernel");
        }
        d.batch[dims] = out.shape()[i];
        d.q_bs[dims] = q.strides()[i];
        d.k_bs[dims] = k.strides()[i];
        d.v_bs[dims] = v.strides()[i];
        d.out_bs[dims] = out.strides()[i];
        d.mask_bs[dims] = mask != nullptr ? mask->strides()[i] : 0;
        ++dims;
    }
    d.batch_dims = dims;
    d.q = ptr<float>(q);
    d.q_rs = q.strides()[row];
    d.k = ptr<float>(k);
    d.k_rs = k.strides()[row];
    d.v = ptr<float>(v);
    d.v_rs = v.strides()[row];
    d.out = ptr<float>(out);
    d.out_rs = out.strides()[row];
    if (mask != nullptr) {
        d.mask = ptr<std::uint8_t>(*mask);
        d.mask_rs = mask->strides()[row];
        d.mask_cs = mask->strides()[col];
    }
    d.causal = args.causal ? 1 : 0;
    d.scale = args.alpha;
    check(mfr_attention(handle(stream), &d));
}

// ---- GEMV --------------------------------------------------------------------------------------

// Inputs: a contiguous [rows, cols], x, and y0 when given; args.transpose = A^T.
void gemv_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& a = args.inputs[0];
    const float* y0 = args.inputs.size() > 2 ? ptr<float>(args.inputs[2]) : nullptr;
    check(mfr_sgemv(handle(stream), args.transpose ? 1 : 0, a.size(0), a.size(1), args.alpha,
                    ptr<float>(a), a.size(1), ptr<float>(args.inputs[1]), y0 ? args.beta : 0.0f,
                    y0, ptr<float>(args.outputs[0])));
}

void matvec_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& a = args.inputs[0];
    check(mfr_smatvec(handle(stream), a.size(0), a.size(1), ptr<float>(a), a.size(1),
                      ptr<float>(args.inputs[1]), ptr<float>(args.outputs[0])));
}

// ---- elementwise, softmax, argmax, layout ------------------------------------------------------

void bias_add_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& out = args.outputs[0];
    check(mfr_bias_act(handle(stream), ptr<float>(args.inputs[0]), ptr<float>(args.inputs[1]),
                       ptr<float>(out), out.size(0), out.size(1), MFR_ACT_NONE));
}

void gelu_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& out = args.outputs[0];
    check(mfr_bias_act(handle(stream), ptr<float>(args.inputs[0]), nullptr, ptr<float>(out), 1,
                       out.numel(), args.approximate ? MFR_ACT_GELU_TANH : MFR_ACT_GELU_ERF));
}

// Inputs: x, y, condition (values first: the dispatch key is their dtype), each a view of out's
// shape, expanded (stride 0) where it broadcasts; mfr_where_nd reads them through their strides.
void where_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& out = args.outputs[0];
    const Tensor& x = args.inputs[0];
    const Tensor& y = args.inputs[1];
    const Tensor& cond = args.inputs[2];
    if (x.is_contiguous() && y.is_contiguous() && cond.is_contiguous()) {
        check(mfr_where(handle(stream), ptr<std::uint8_t>(cond), ptr<float>(x), ptr<float>(y),
                        ptr<float>(out), out.numel()));
        return;
    }
    if (out.dim() > MFR_MAX_COPY_DIMS) {
        const Tensor px = x.contiguous(), py = y.contiguous(), pc = cond.contiguous();
        check(mfr_where(handle(stream), ptr<std::uint8_t>(pc), ptr<float>(px), ptr<float>(py),
                        ptr<float>(out), out.numel()));
        return;
    }
    check(mfr_where_nd(handle(stream), out.dim(), out.shape().data(), ptr<std::uint8_t>(cond),
                       cond.strides().data(), ptr<float>(x), x.strides().data(), ptr<float>(y),
                       y.strides().data(), ptr<float>(out)));
}

void softmax_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& x = args.inputs[0];
    std::int64_t outer = 1, length = 1, inner = 1;
    for (int d = 0; d < x.dim(); ++d) {
        if (d < args.axis) {
            outer *= x.size(d);
        } else if (d == args.axis) {
            length = x.size(d);
        } else {
            inner *= x.size(d);
        }
    }
    check(mfr_softmax(handle(stream), ptr<float>(x), ptr<float>(args.outputs[0]), outer, length,
                      inner));
}

void argmax_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& x = args.inputs[0];
    const std::int64_t width = x.size(x.dim() - 1);
    check(mfr_argmax(handle(stream), ptr<float>(x), ptr<std::int64_t>(args.outputs[0]),
                     x.numel() / width, width));
}

template <int Op> void binary_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& out = args.outputs[0];
    const float* b = Op == MFR_EW_SCAL ? nullptr : ptr<float>(args.inputs[1]);
    check(mfr_elementwise(handle(stream), Op, ptr<float>(args.inputs[0]), b, args.alpha,
                          ptr<float>(out), out.numel()));
}

// OpId::Dot: two unit-stride vectors of one length (the op checks them), a 0-d output.
void dot_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& x = args.inputs[0];
    check(mfr_sdot(handle(stream), x.numel(), ptr<float>(x), ptr<float>(args.inputs[1]),
                   ptr<float>(args.outputs[0])));
}

// Packs a strided view (any dtype) into the contiguous output on the device.
void strided_copy_kernel(const OpArgs& args, Stream& stream) {
    const Tensor& x = args.inputs[0];
    if (x.dim() > MFR_MAX_COPY_DIMS) {
        throw NotImplemented("strided_copy: more than " + std::to_string(MFR_MAX_COPY_DIMS) +
                             " dimensions on rocm");
    }
    check(mfr_strided_copy(handle(stream), first_byte(x), first_byte(args.outputs[0]),
                           static_cast<std::int32_t>(x.itemsize()), x.dim(), x.shape().data(),
                           x.strides().data()));
}

class RocmBackend final : public Backend {
  public:
    RocmBackend() {
        int count = 0;
        if (mfr_get_device_count(&count) == MFR_OK) {
            count_ = count;
        }
        streams_.resize(static_cast<std::size_t>(count_));
        for (int i = 0; i < count_; ++i) {
            pools_.push_back(std::make_shared<BlockPool>(i));
        }
    }

    DeviceType type() const override { return DeviceType::ROCm; }
    int device_count() const override { return count_; }

    DeviceInfo info(int index) const override {
        char name[256] = {0};
        std::size_t bytes = 0;
        check(mfr_get_device_info(index, name, sizeof(name), &bytes, nullptr, nullptr));
        return {name, bytes};
    }

    std::shared_ptr<Buffer> allocate(int index, std::size_t bytes) override {
        return std::make_shared<RocmBuffer>(pools_.at(static_cast<std::size_t>(index)), bytes);
    }

    Stream& stream(int index) override {
        std::lock_guard<std::mutex> lock(mutex_);
        auto& slot = streams_.at(static_cast<std::size_t>(index));
        if (!slot) {
            slot = std::make_unique<RocmStream>(index);
        }
        return *slot;
    }

    void register_kernels(Dispatcher& dispatcher) override {
        auto add = [&dispatcher](OpId op, KernelFn kernel) {
            dispatcher.register_kernel({op, DeviceType::ROCm, DType::F32}, kernel);
        };
        add(OpId::Matmul, matmul_kernel);
        add(OpId::Gemm, gemm_kernel);
        add(OpId::Attention, attention_kernel);
        add(OpId::GemmBatched, gemm_batched_kernel);
        add(OpId::Gemv, gemv_kernel);
        add(OpId::Matvec, matvec_kernel);
        add(OpId::BiasAdd, bias_add_kernel);
        add(OpId::Gelu, gelu_kernel);
        add(OpId::Where, where_kernel);
        add(OpId::Softmax, softmax_kernel);
        add(OpId::Argmax, argmax_kernel);
        add(OpId::Add, binary_kernel<MFR_EW_ADD>);
        add(OpId::Mul, binary_kernel<MFR_EW_MUL>);
        add(OpId::Sub, binary_kernel<MFR_EW_SUB>);
        add(OpId::Dot, dot_kernel);
        add(OpId::Scal, binary_kernel<MFR_EW_SCAL>);
        dispatcher.register_tunable({OpId::Matmul, DeviceType::ROCm, DType::F32},
                                    gemm_tunable<OpId::Matmul>("matmul"));
        dispatcher.register_tunable({OpId::Gemm, DeviceType::ROCm, DType::F32},
                                    gemm_tunable<OpId::Gemm>("gemm"));
        dispatcher.register_tunable({OpId::GemmBatched, DeviceType::ROCm, DType::F32},
                                    gemm_tunable<OpId::GemmBatched>("gemm_strided_batched"));
        for (DType type : {DType::F32, DType::I32, DType::I64, DType::U8, DType::Bool,
                           DType::F16, DType::BF16}) {
            dispatcher.register_kernel({OpId::StridedCopy, DeviceType::ROCm, type},
                                       strided_copy_kernel);
        }
    }

  private:
    int count_ = 0;
    std::mutex mutex_;
    std::vector<std::unique_ptr<RocmStream>> streams_;
    std::vector<std::shared_ptr<BlockPool>> pools_;
};

} // namespace

void register_rocm_backend(Registry& registry) { registry.add(std::make_unique<RocmBackend>()); }

} // namespace mensurflow::detail
