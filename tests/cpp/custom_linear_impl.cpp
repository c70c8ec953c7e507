// A linear implementation written against the reference's LinearLayer::LinearImpl
// interface (src/layers/linear.h:131-153: impl_id, supports(ctx, weight_set), prepare and
// forward taking the owning layer, the op context, the weight set, input, output, the
// stream and the cached descriptors). tests/test_operator_dispatch.py compiles it against
// edge-fm-x_amd/host (syntax only): an impl ported from the reference changes its stream
// type and its kernel calls, nothing else.
#include "engine.hpp"
#include "operators.hpp"

namespace edge_fm {

class ExampleLinearImpl final : public LinearLayer::LinearImpl {
public:
    std::string impl_id() const override { return "example_linear"; }

    bool supports(const LinearLayer::LinearOpContext& ctx, const LinearLayer::WeightSet& weight_set) const override {
        return weight_set.quant_type_ == LinearLayer::QuantType::FP16_BF16 && weight_set.weight_ != nullptr &&
               ctx.shape.input_dtype == DType::BFloat16 && ctx.shape.output_dtype == DType::BFloat16 &&
               ctx.shape.in_features % 32 == 0;
    }

    void prepare(LinearLayer& owner, const LinearLayer::LinearOpContext& ctx, const LinearLayer::WeightSet& weight_set,
                 const Tensor& input, Tensor& output, hipStream_t stream,
                 LinearLayer::CachedDescriptors& cached) override {
        (void)owner, (void)weight_set, (void)input, (void)output, (void)stream;
        if (cached.prepared_) return;
        cached.selected_impl_id_ = impl_id();
        cached.workspace_bytes_ = efm_linear_workspace_bytes(ctx.shape.m, ctx.shape.in_features, ctx.shape.out_features);
        cached.prepared_ = true;
    }

    void forward(LinearLayer& owner, const LinearLayer::LinearOpContext& ctx, const LinearLayer::WeightSet& weight_set,
                 const Tensor& input, Tensor& output, hipStream_t stream,
                 LinearLayer::CachedDescriptors& cached) override {
        prepare(owner, ctx, weight_set, input, output, stream, cached);
        efm_check(efm_linear(ctx.shape.m, ctx.shape.in_features, ctx.shape.out_features, input.data_ptr(),
                             weight_set.weight_->data_ptr(), weight_set.bias_ ? weight_set.bias_->data_ptr() : nullptr,
                             output.data_ptr(), EFM_DTYPE_BF16, stream),
                  "example_linear " + owner.layer_prefix());
    }
};

}  // namespace edge_fm
