// sdpa_ops.cc -- TensorFlow op definitions of Sdpa (attention forward) and
// SdpaGrad (its backward) for the MI355X build.
//
// The interface is the reference's, unchanged, so that graphs, checkpoints
// and the Python wrapper keep working: same op names, input names, types and
// order, attribute names, defaults and order, outputs and shape functions
// (sdpa/sdpa_ops.cc:7-63).  Kernels are registered in sdpa_kernels.cc.
#include "tensorflow/core/framework/op.h"
#include "tensorflow/core/framework/shape_inference.h"

namespace tensorflow {

using shape_inference::DimensionHandle;
using shape_inference::InferenceContext;
using shape_inference::ShapeHandle;

namespace {

// o [B, S_q, D_v] and stats [B, S_q] from q [B, S_q, D_qk] and v [B, S_kv, D_v].
Status SdpaShape(InferenceContext* c) {
    ShapeHandle q, k, v;
    TF_RETURN_IF_ERROR(c->WithRank(c->input(0), 3, &q));
    TF_RETURN_IF_ERROR(c->WithRank(c->input(1), 3, &k));
    TF_RETURN_IF_ERROR(c->WithRank(c->input(2), 3, &v));
    const DimensionHandle batch = c->Dim(q, 0), rows = c->Dim(q, 1), width = c->Dim(v, 2);
    c->set_output(0, c->MakeShape({batch, rows, width}));
    c->set_output(1, c->MakeShape({batch, rows}));
    return OkStatus();
}

// dq, dk, dv have the shapes of q, k, v.
Status SdpaGradShape(InferenceContext* c) {
    for (int i = 0; i < 3; ++i) {
        ShapeHandle s;
        TF_RETURN_IF_ERROR(c->WithRank(c->input(i), 3, &s));
        c->set_output(i, s);
    }
    return OkStatus();
}

}  // namespace

REGISTER_OP("Sdpa")
    .Input("q: T")           // [B, S_q, D_qk]
    .Input("k: T")           // [B, S_kv, D_qk]
    .Input("v: T")           // [B, S_kv, D_v]
    .Input("seed: uint64")   // scalar
    .Input("offset: uint64") // scalar
    .Attr("scale: float = 1.0")
    .Attr("dropout: float = 0.0")
    .Attr("causal_mask: bool = false")
    .Attr("T: {half, float}")
    .Output("output: T")     // [B, S_q, D_v]
    .Output("stats: float")  // [B, S_q], m + log(l + 1e-6)
    .SetShapeFn(SdpaShape);

REGISTER_OP("SdpaGrad")
    .Input("q: T")
    .Input("k: T")
    .Input("v: T")
    .Input("out: T")         // the forward's output
    .Input("stats: float")   // the forward's stats
    .Input("do: T")          // gradient of the output
    .Input("seed: uint64")
    .Input("offset: uint64")
    .Output("dq: T")
    .Output("dk: T")
    .Output("dv: T")
    .Attr("dropout: float = 0.0")
    .Attr("scale: float = 1.0")
    .Attr("causal_mask: bool = false")
    .Attr("T: {half, float}")
    .SetShapeFn(SdpaGradShape);

}  // namespace tensorflow
