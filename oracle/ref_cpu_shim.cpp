// C entry point over nnops' own CPU MatMul (the AVX-512-VNNI int8 route that
// the reference ships as its CPU backend), for the CPU baseline of bench.py
// and a parity cross-check of the oracle. Test infrastructure only: compiled
// by oracle/Makefile (target `ref`) against the nnops sources where they lie,
// into oracle/_ref/. Nothing from the reference is copied here; this file
// builds the reference's TensorViews and calls
//   nnops::MatMul::create / compute   include/nnops/ops/matmul.hpp:88-135
// with a ComputeContext whose CpuBackend hooks (include/nnops/core/
// parallel_for.hpp:60-110) run on a small std::thread pool defined below.
#include "nnops/ops/linear.hpp"
#include "nnops/ops/matmul.hpp"
#include "nnops/ops/quant_linear.hpp"

#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <cstdint>
#include <functional>
#include <mutex>
#include <span>
#include <thread>
#include <vector>

using namespace nnops;

namespace nnops::backend::cpu {
// the CPU backend's Linear (src/backend/cpu/matmul/linear.cpp:199)
Status linear_cpu(const LinearAttributes& attrs, TensorView& output, std::span<const TensorView> inputs,
                  const ComputeContext& ctx, void* workspace);
}  // namespace nnops::backend::cpu

namespace {

// Fixed worker pool: parallel_for hands out indices through one atomic
// counter; the caller's thread takes part as worker 0.
class Pool {
public:
    explicit Pool(int n) : n_(n < 1 ? 1 : n)
    {
        for (int i = 1; i < n_; ++i) {
            th_.emplace_back([this, i] { loop(i); });
        }
    }
    ~Pool()
    {
        {
            std::lock_guard<std::mutex> g(m_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : th_) {
            t.join();
        }
    }
    int size() const { return n_; }
    static int& tid()
    {
        thread_local int id = 0;
        return id;
    }
    void run(int64_t begin, int64_t end, const ParallelForBody& body)
    {
        {
            std::lock_guard<std::mutex> g(m_);
            body_ = &body;
            next_.store(begin);
            end_ = end;
            busy_ = n_ - 1;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> l(m_);
        done_.wait(l, [this] { return busy_ == 0; });
    }

private:
    void work()
    {
        for (;;) {
            const int64_t i = next_.fetch_add(1);
            if (i >= end_) {
                return;
            }
            (*body_)(i);
        }
    }
    void loop(int id)
    {
        tid() = id;
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> l(m_);
                cv_.wait(l, [&] { return gen_ != seen; });
                seen = gen_;
                if (stop_) {
                    return;
                }
            }
            work();
            std::lock_guard<std::mutex> g(m_);
            if (--busy_ == 0) {
                done_.notify_one();
            }
        }
    }
    int n_;
    std::vector<std::thread> th_;
    std::mutex m_;
    std::condition_variable cv_, done_;
    uint64_t gen_ = 0;
    bool stop_ = false;
    const ParallelForBody* body_ = nullptr;
    std::atomic<int64_t> next_{0};
    int64_t end_ = 0;
    int busy_ = 0;
};

Pool* pool_of(int threads)
{
    static std::mutex pm;
    static std::unique_ptr<Pool> pool;
    std::lock_guard<std::mutex> g(pm);
    if (!pool || pool->size() != threads) {
        pool.reset();
        pool = std::make_unique<Pool>(threads);
    }
    return pool.get();
}

ComputeContext context_on(Pool* p)
{
    ComputeContext ctx{};
    ctx.cpu.parallel_for = [p](int64_t b, int64_t e, const ParallelForBody& body) { p->run(b, e, body); };
    ctx.cpu.num_threads = [p] { return p->size(); };
    ctx.cpu.thread_id = [] { return Pool::tid(); };
    return ctx;
}

}  // namespace

extern "C" {

// s8 A [M,K] x s8 W ([N,K] with trans_b, else [K,N]) -> s32 (out_s8 = 0) or
// s8 C [M,N]: per-tensor A scale, per-channel W scales (or s_b = NULL: 1),
// int32 bias (or NULL), Relu, per-tensor output scale and zero point (nnops'
// requant, half away from zero). `threads` workers.
int ref_cpu_matmul_i8(const int8_t* a, const int8_t* w, const int32_t* bias, void* c, int64_t M, int64_t N,
                      int64_t K, int trans_b, int out_s8, float s_a, const float* s_b, float s_out, int32_t zp_out,
                      int relu, int threads)
{
    Pool* p = pool_of(threads);
    QuantParams qa;
    qa.scale = s_a;
    QuantParams qb;
    if (s_b != nullptr) {
        qb.granularity = QuantGranularity::PerChannel;
        qb.scale_data = s_b;
        qb.num_scales = N;
    }
    QuantParams qc;
    qc.scale = s_out;
    qc.zero_point = zp_out;
    const int64_t ashape[] = {M, K}, wshape_t[] = {N, K}, wshape[] = {K, N}, cshape[] = {M, N}, bshape[] = {N};
    TensorView av(ashape, DataType::s8, const_cast<int8_t*>(a), TensorLayout::Dense, qa);
    TensorView wv(trans_b ? std::span<const int64_t>(wshape_t) : std::span<const int64_t>(wshape), DataType::s8,
                  const_cast<int8_t*>(w), TensorLayout::Dense, qb);
    TensorView bv(bshape, DataType::s32, const_cast<int32_t*>(bias));
    const DataType odt = out_s8 ? DataType::s8 : DataType::s32;
    TensorView cv(cshape, odt, c, TensorLayout::Dense, out_s8 ? qc : QuantParams{});

    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    attrs.output_dtype = odt;
    if (relu) {
        attrs.epilogue.type = EpilogueActivateType::Relu;
    }
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {av, wv, bv};
    TensorView outs[] = {cv};
    const Status st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, bias ? 3 : 2), ctx);
    return static_cast<int>(st);
}

int ref_cpu_matmul_s8(const int8_t* a, const int8_t* w, const int32_t* bias, int8_t* c, int64_t M, int64_t N,
                      int64_t K, float s_a, const float* s_b, float s_out, int32_t zp_out, int relu, int threads)
{
    return ref_cpu_matmul_i8(a, w, bias, c, M, N, K, 1, 1, s_a, s_b, s_out, zp_out, relu, threads);
}

// f16 A [M,K] x q4_1 W -> f16 C [M,N] (nnops' fp x q4_1 route: the output
// dtype follows A; matmul_qblock_fused for small M, src/ops/matmul.cpp:49-58).
// W is [N][ceil(K/32)] blocks with trans_b (the Linear/GGUF form), else
// [K][ceil(N/32)] blocks.
int ref_cpu_matmul_q4_1(const uint16_t* a, const uint8_t* w, uint16_t* c, int64_t M, int64_t N, int64_t K,
                        int trans_b, int threads)
{
    Pool* p = pool_of(threads);
    const int64_t ashape[] = {M, K}, wshape_t[] = {N, K}, wshape[] = {K, N}, cshape[] = {M, N};
    TensorView av(ashape, DataType::f16, const_cast<uint16_t*>(a));
    TensorView wv(trans_b ? std::span<const int64_t>(wshape_t) : std::span<const int64_t>(wshape), DataType::q4_1,
                  const_cast<uint8_t*>(w));
    TensorView cv(cshape, DataType::f16, c);
    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {av, wv};
    TensorView outs[] = {cv};
    const Status st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, 2), ctx);
    return static_cast<int>(st);
}

// nnops' fp x q4_1 MatMul with the full fp epilogue: f32 / f16 A [M, K]
// (a_f16), W [N][K/32] blocks (trans_b) or [K][N/32], bias of A's type [N] or
// NULL, C of A's type [M, N] (its contents are old C when beta != 0 or
// residual_pre): C = act(clip(alpha A W + bias + beta C_old)), through
// MatMul::create / compute (include/nnops/ops/matmul.hpp:5-11,33-65).
int ref_cpu_matmul_q4_1_ep(const void* a, int a_f16, const uint8_t* w, const void* bias, void* c, int64_t M,
                           int64_t N, int64_t K, int trans_b, float alpha, float beta, int residual_pre, int act,
                           float act_alpha, float act_beta, float min_clip, float max_clip, int threads)
{
    Pool* p = pool_of(threads);
    const DataType dt = a_f16 ? DataType::f16 : DataType::f32;
    const int64_t ashape[] = {M, K}, wshape_t[] = {N, K}, wshape[] = {K, N}, cshape[] = {M, N}, bshape[] = {N};
    TensorView av(ashape, dt, const_cast<void*>(a));
    TensorView wv(trans_b ? std::span<const int64_t>(wshape_t) : std::span<const int64_t>(wshape), DataType::q4_1,
                  const_cast<uint8_t*>(w));
    TensorView bv(bshape, dt, const_cast<void*>(bias));
    TensorView cv(cshape, dt, c);
    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    attrs.alpha = alpha;
    attrs.beta = beta;
    attrs.residual_pre_activation = residual_pre != 0;
    attrs.epilogue.type = static_cast<EpilogueActivateType>(act);
    attrs.epilogue.alpha = act_alpha;
    attrs.epilogue.beta = act_beta;
    attrs.epilogue.min_clip = min_clip;
    attrs.epilogue.max_clip = max_clip;
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {av, wv, bv};
    TensorView outs[] = {cv};
    const Status st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, bias ? 3 : 2), ctx);
    return static_cast<int>(st);
}

// nnops' Linear over a q4_1 weight [N2, K] (blocks along K): f32 / f16 X
// [M, K] (x_f16), bias of X's type [N2] or NULL, output C of X's type [M, N]
// (N = N2 / 2 when gated, else N2; its current contents are the residual when
// add_to). Calls the CPU backend's linear_cpu (src/backend/cpu/matmul/
// linear.cpp:199-309) directly: the operator's validate admits the gated form
// for fp weights of X's type only (src/ops/linear.cpp:92), and this is the
// reference's own combine over the q4_1 GEMM for the HIP extension's parity.
static int linear_any(const void* x, int x_f16, const void* w, bool w_q4_1, const void* bias, void* c, int64_t M,
                      int64_t N2, int64_t K, int act, float act_alpha, float act_beta, float min_clip,
                      float max_clip, int add_to, int residual_pre, int gated, int gate_act, float gate_alpha,
                      float gate_beta, float gate_limit, int threads)
{
    Pool* p = pool_of(threads);
    const DataType dt = x_f16 ? DataType::f16 : DataType::f32;
    const int64_t N = gated ? N2 / 2 : N2;
    const int64_t xshape[] = {M, K}, wshape[] = {N2, K}, bshape[] = {N2}, cshape[] = {M, N};
    TensorView xv(xshape, dt, const_cast<void*>(x));
    TensorView wv(wshape, w_q4_1 ? DataType::q4_1 : dt, const_cast<void*>(w));
    TensorView bv(bshape, dt, const_cast<void*>(bias));
    TensorView cv(cshape, dt, c);
    LinearAttributes attrs{};
    attrs.epilogue.type = static_cast<EpilogueActivateType>(act);
    attrs.epilogue.alpha = act_alpha;
    attrs.epilogue.beta = act_beta;
    attrs.epilogue.min_clip = min_clip;
    attrs.epilogue.max_clip = max_clip;
    attrs.add_to = add_to != 0;
    attrs.residual_pre_activation = residual_pre != 0;
    attrs.gated = gated != 0;
    attrs.gate_activation = static_cast<EpilogueActivateType>(gate_act);
    attrs.gate_alpha = gate_alpha;
    attrs.gate_beta = gate_beta;
    attrs.gate_limit = gate_limit;
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {xv, wv, bv};
    const Status st = backend::cpu::linear_cpu(attrs, cv, std::span<const TensorView>(ins, bias ? 3 : 2), ctx,
                                               nullptr);
    return static_cast<int>(st);
}

int ref_cpu_linear_q4_1(const void* x, int x_f16, const uint8_t* w, const void* bias, void* c, int64_t M,
                        int64_t N2, int64_t K, int act, float act_alpha, float act_beta, float min_clip,
                        float max_clip, int add_to, int residual_pre, int gated, int gate_act, float gate_alpha,
                        float gate_beta, float gate_limit, int threads)
{
    return linear_any(x, x_f16, w, true, bias, c, M, N2, K, act, act_alpha, act_beta, min_clip, max_clip, add_to,
                      residual_pre, gated, gate_act, gate_alpha, gate_beta, gate_limit, threads);
}

// The same Linear over a dense weight of X's type [N2, K] (nnops' own gated
// route: src/ops/linear.cpp:92, linear_cpu's fp GEMM plus the combine).
int ref_cpu_linear_fp(const void* x, int x_f16, const void* w, const void* bias, void* c, int64_t M, int64_t N2,
                      int64_t K, int act, float act_alpha, float act_beta, float min_clip, float max_clip, int add_to,
                      int residual_pre, int gated, int gate_act, float gate_alpha, float gate_beta, float gate_limit,
                      int threads)
{
    return linear_any(x, x_f16, w, false, bias, c, M, N2, K, act, act_alpha, act_beta, min_clip, max_clip, add_to,
                      residual_pre, gated, gate_act, gate_alpha, gate_beta, gate_limit, threads);
}

// nnops' dense float MatMul: f32 x f32 or f16 x f16 (f16), A [M, K], B
// [N, K] (trans_b) or [K, N], C [M, N] of A's type (MatMul::create /
// compute; matmul_small_fp or FpRoute<T> by shape).
int ref_cpu_matmul_fp(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K, int trans_b, int f16,
                      int threads)
{
    Pool* p = pool_of(threads);
    const DataType dt = f16 ? DataType::f16 : DataType::f32;
    const int64_t ashape[] = {M, K}, bshape_t[] = {N, K}, bshape[] = {K, N}, cshape[] = {M, N};
    TensorView av(ashape, dt, const_cast<void*>(a));
    TensorView bv(trans_b ? std::span<const int64_t>(bshape_t) : std::span<const int64_t>(bshape), dt,
                  const_cast<void*>(b));
    TensorView cv(cshape, dt, c);
    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {av, bv};
    TensorView outs[] = {cv};
    const Status st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, 2), ctx);
    return static_cast<int>(st);
}

// nnops' two-step prepackWeights of an s8 weight for the integer route
// (src/ops/matmul.cpp:96-141: the query for the packed descriptor, then the
// fill), kept in a heap blob; the handle is freed by ref_cpu_packed_free.
struct PackedI8 {
    void* blob = nullptr;
    int64_t shape[2] = {0, 0};
    int64_t pitch = 0;
    DataType dtype = DataType::s8;
    TensorLayout layout = TensorLayout::Dense;
    int trans_b = 0, out_s8 = 0;
};

void* ref_cpu_prepack_i8(const int8_t* w, int64_t N, int64_t K, int trans_b, int out_s8, const float* s_b,
                         int threads)
{
    Pool* p = pool_of(threads);
    QuantParams qb;
    if (s_b != nullptr) {
        qb.granularity = QuantGranularity::PerChannel;
        qb.scale_data = s_b;
        qb.num_scales = N;
    }
    const int64_t wshape_t[] = {N, K}, wshape[] = {K, N};
    TensorView wv(trans_b ? std::span<const int64_t>(wshape_t) : std::span<const int64_t>(wshape), DataType::s8,
                  const_cast<int8_t*>(w), TensorLayout::Dense, qb);
    MatMulAttributes attrs{};
    attrs.transpose_b = trans_b != 0;
    attrs.output_dtype = out_s8 ? DataType::s8 : DataType::s32;
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView bq[] = {wv};
    TensorView q;
    TensorView oq[] = {q};
    op->prepackWeights(bq, oq, ctx);
    if (oq[0].rank() != 2) {
        return nullptr;     // no packed form
    }
    auto* h = new PackedI8;
    h->shape[0] = oq[0].shape(0);
    h->shape[1] = oq[0].shape(1);
    h->pitch = oq[0].pitch();
    h->dtype = oq[0].data_type();
    h->layout = oq[0].layout();
    h->trans_b = trans_b;
    h->out_s8 = out_s8;
    const size_t bytes = (size_t)h->pitch * (size_t)h->shape[0];
    h->blob = std::aligned_alloc(64, (bytes + 63) / 64 * 64);
    TensorView fill(std::span<const int64_t>(h->shape, 2), h->dtype, h->blob, h->pitch, h->layout, qb);
    TensorView oq2[] = {fill};
    op->prepackWeights(bq, oq2, ctx);
    return h;
}

void ref_cpu_packed_free(void* handle)
{
    auto* h = static_cast<PackedI8*>(handle);
    if (h != nullptr) {
        std::free(h->blob);
        delete h;
    }
}

// The int8 MatMul of ref_cpu_matmul_i8 over a prepacked weight.
int ref_cpu_matmul_i8_packed(const int8_t* a, const void* handle, const int32_t* bias, void* c, int64_t M,
                             int64_t N, int64_t K, float s_a, const float* s_b, float s_out, int32_t zp_out,
                             int relu, int threads)
{
    const auto* h = static_cast<const PackedI8*>(handle);
    Pool* p = pool_of(threads);
    QuantParams qa;
    qa.scale = s_a;
    QuantParams qb;
    if (s_b != nullptr) {
        qb.granularity = QuantGranularity::PerChannel;
        qb.scale_data = s_b;
        qb.num_scales = N;
    }
    QuantParams qc;
    qc.scale = s_out;
    qc.zero_point = zp_out;
    const int64_t ashape[] = {M, K}, cshape[] = {M, N}, bshape[] = {N};
    TensorView av(ashape, DataType::s8, const_cast<int8_t*>(a), TensorLayout::Dense, qa);
    TensorView wv(std::span<const int64_t>(h->shape, 2), h->dtype, h->blob, h->pitch, h->layout, qb);
    TensorView bv(bshape, DataType::s32, const_cast<int32_t*>(bias));
    const DataType odt = h->out_s8 ? DataType::s8 : DataType::s32;
    TensorView cv(cshape, odt, c, TensorLayout::Dense, h->out_s8 ? qc : QuantParams{});
    MatMulAttributes attrs{};
    attrs.transpose_b = h->trans_b != 0;
    attrs.output_dtype = odt;
    if (relu) {
        attrs.epilogue.type = EpilogueActivateType::Relu;
    }
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {av, wv, bv};
    TensorView outs[] = {cv};
    const Status st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, bias ? 3 : 2), ctx);
    return static_cast<int>(st);
}

// The int8 pair with a dequantizing f16 destination (nnops' DqRoute): s8 A
// [M,K] with per-token scales (or an f16 A with per-token QuantParams,
// quantized by nnops' matmul_dq_from_fp when a_f16), s8 W [N,K] with
// per-channel scales, f16 bias [N] or NULL, Relu, f16 C [M,N].
int ref_cpu_matmul_dq_f16(const void* a, int a_f16, const float* s_a_rows, const int8_t* w, const float* s_b,
                          const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K, int relu,
                          int threads)
{
    Pool* p = pool_of(threads);
    QuantParams qa;
    qa.granularity = QuantGranularity::PerToken;
    qa.scale_data = s_a_rows;
    qa.num_scales = M;
    QuantParams qb;
    qb.granularity = QuantGranularity::PerChannel;
    qb.scale_data = s_b;
    qb.num_scales = N;
    const int64_t ashape[] = {M, K}, wshape[] = {N, K}, cshape[] = {M, N}, bshape[] = {N};
    TensorView av(ashape, a_f16 ? DataType::f16 : DataType::s8, const_cast<void*>(a), TensorLayout::Dense, qa);
    TensorView wv(wshape, DataType::s8, const_cast<int8_t*>(w), TensorLayout::Dense, qb);
    TensorView bv(bshape, DataType::f16, const_cast<uint16_t*>(bias));
    TensorView cv(cshape, DataType::f16, c);
    MatMulAttributes attrs{};
    attrs.transpose_b = true;
    attrs.output_dtype = DataType::f16;
    if (relu) {
        attrs.epilogue.type = EpilogueActivateType::Relu;
    }
    auto op = MatMul::create(attrs, Backend::CPU);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {av, wv, bv};
    TensorView outs[] = {cv};
    const Status st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, bias ? 3 : 2), ctx);
    return static_cast<int>(st);
}

// nnops' QuantizeLinear (f16 x [R,C] -> s8) or DequantizeLinear (s8 -> f16)
// with per-token scales and s8 zero points (axis -1), through
// QuantizeLinear / DequantizeLinear::create / compute
// (include/nnops/ops/quant_linear.hpp:47-122).
int ref_cpu_qdq_f16(const void* x, const float* scale, const int8_t* zp, void* y, int64_t R, int64_t Cc,
                    int dequant, int threads)
{
    Pool* p = pool_of(threads);
    const int64_t shape[] = {R, Cc}, pshape[] = {R};
    QuantLinearAttributes attrs{};
    attrs.axis = -1;
    attrs.output_dtype = dequant ? DataType::f16 : DataType::s8;
    TensorView xv(shape, dequant ? DataType::s8 : DataType::f16, const_cast<void*>(x));
    TensorView sv(pshape, DataType::f32, const_cast<float*>(scale));
    TensorView zv(pshape, DataType::s8, const_cast<int8_t*>(zp));
    TensorView yv(shape, dequant ? DataType::f16 : DataType::s8, y);
    const ComputeContext ctx = context_on(p);
    const TensorView ins[] = {xv, sv, zv};
    TensorView outs[] = {yv};
    Status st;
    if (dequant) {
        auto op = DequantizeLinear::create(attrs, Backend::CPU);
        st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, 3), ctx);
    } else {
        auto op = QuantizeLinear::create(attrs, Backend::CPU);
        st = op->compute(std::span<TensorView>(outs), std::span<const TensorView>(ins, 3), ctx);
    }
    return static_cast<int>(st);
}

}  // extern "C"
