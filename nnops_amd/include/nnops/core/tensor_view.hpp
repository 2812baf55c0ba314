#pragma once
/// @file tensor_view.hpp
/// @brief TensorDesc / TensorView — non-owning, pitched tensor views.
///
/// The same model as nnops (include/nnops/core/tensor_view.hpp:38-365): the
/// innermost dimension is a row, `pitch` is the byte distance between rows and
/// may exceed the row's bytes; outer dimensions are dense over rows. The view
/// never owns memory; on the HIP backend the data pointers are device pointers.
/// Only the Dense layout is carried here (the path has no channel-last tensors).

#include "nnops/core/data_type.hpp"
#include "nnops/core/quant_params.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <span>

namespace nnops {

/// Layout tags. Values follow nnops' append-only numbering
/// (include/nnops/core/tensor_layout.hpp:27-129).
enum class TensorLayout : uint8_t {
    PackedB = 10,
    Dense = 12,
    /// The HIP backend's prepacked matmul B (MatMul / Linear ::prepackWeights):
    /// an s8 weight as [N][kp] k-contiguous rows (kp = K rounded up to 128,
    /// zero padded) followed by its int32 column sums. Shape [N, ceil(bytes/N)]
    /// like nnops' PackedB; appended after nnops' last tag (17).
    PackedBHip = 18,
};

struct TensorDesc {
    static constexpr int64_t kMaxRank = 8;
    std::array<int64_t, kMaxRank> dims{};
    int64_t rank = 0;
    DataType dtype = DataType::f32;
    TensorLayout layout = TensorLayout::Dense;
    /// Row stride in units of data_type_stride_unit(); 0 = compact.
    int64_t row_stride_elems = 0;

    int64_t numel() const noexcept
    {
        int64_t n = 1;
        for (int64_t i = 0; i < rank; ++i) {
            n *= dims[static_cast<size_t>(i)];
        }
        return n;
    }
    int64_t rows() const noexcept
    {
        int64_t r = 1;
        for (int64_t i = 0; i + 1 < rank; ++i) {
            r *= dims[static_cast<size_t>(i)];
        }
        return r;
    }
    int64_t cols() const noexcept { return rank > 0 ? dims[static_cast<size_t>(rank - 1)] : 1; }
};

class TensorView {
public:
    static constexpr int64_t kMaxRank = 8;

    TensorView() = default;

    /// Dense view: pitch is one row's bytes.
    TensorView(std::span<const int64_t> shape, DataType dtype, void* data,
               TensorLayout layout = TensorLayout::Dense, QuantParams qp = {})
        : data_(data), dtype_(dtype), layout_(layout), qp_(qp)
    {
        set_shape(shape);
        pitch_ = rank_ >= 1 ? static_cast<int64_t>(data_type_row_bytes(dtype, shape_[rank_ - 1]))
                            : 0;
    }

    /// Pitched view: `pitch` bytes between consecutive rows.
    TensorView(std::span<const int64_t> shape, DataType dtype, void* data, int64_t pitch,
               TensorLayout layout = TensorLayout::Dense, QuantParams qp = {})
        : data_(data), pitch_(pitch), dtype_(dtype), layout_(layout), qp_(qp)
    {
        set_shape(shape);
    }

    int64_t rank() const noexcept { return rank_; }
    int64_t shape(int64_t d) const noexcept { return shape_[static_cast<size_t>(d)]; }
    std::span<const int64_t> shape_span() const noexcept
    {
        return {shape_.data(), static_cast<size_t>(rank_)};
    }
    int64_t pitch() const noexcept { return pitch_; }
    DataType data_type() const noexcept { return dtype_; }
    TensorLayout layout() const noexcept { return layout_; }
    const QuantParams& quant_params() const noexcept { return qp_; }
    bool is_empty() const noexcept { return data_ == nullptr; }

    template <typename T>
    T* ptr() const noexcept { return static_cast<T*>(data_); }

    int64_t numel() const noexcept
    {
        if (rank_ == 0) {
            return data_ != nullptr ? 1 : 0;
        }
        int64_t n = 1;
        for (int64_t i = 0; i < rank_; ++i) {
            n *= shape_[static_cast<size_t>(i)];
        }
        return n;
    }

    /// Rows of the innermost dimension (product of the outer dims).
    int64_t total_rows() const noexcept
    {
        int64_t r = 1;
        for (int64_t i = 0; i + 1 < rank_; ++i) {
            r *= shape_[static_cast<size_t>(i)];
        }
        return r;
    }

    /// Row stride in element (or block) units; 1 for rank < 2.
    int64_t row_stride_elems() const noexcept
    {
        if (rank_ < 2) {
            return 1;
        }
        const int64_t unit = static_cast<int64_t>(data_type_stride_unit(dtype_));
        return unit > 0 ? pitch_ / unit : 0;
    }

    TensorDesc desc() const noexcept
    {
        TensorDesc d;
        d.rank = rank_;
        d.dims = shape_;
        d.dtype = dtype_;
        d.layout = layout_;
        d.row_stride_elems = rank_ >= 2 ? row_stride_elems() : 0;
        return d;
    }

private:
    void set_shape(std::span<const int64_t> shape) noexcept
    {
        rank_ = static_cast<int64_t>(shape.size() <= kMaxRank ? shape.size() : kMaxRank);
        for (int64_t i = 0; i < rank_; ++i) {
            shape_[static_cast<size_t>(i)] = shape[static_cast<size_t>(i)];
        }
    }

    std::array<int64_t, kMaxRank> shape_{};
    int64_t rank_ = 0;
    void* data_ = nullptr;
    int64_t pitch_ = 0;
    DataType dtype_ = DataType::f32;
    TensorLayout layout_ = TensorLayout::Dense;
    QuantParams qp_{};
};

}  // namespace nnops
