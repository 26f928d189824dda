"""Copy the ONNX 1.18 node-test models of the ops on this path, with their test_data_set_0
input / output tensors, from the reference's vendored conformance data
(tests/conformance_data/onnx-1.18/node/<test>/) into tests/golden/onnx_node/<test>/.
These are data files (protobuf ModelProto / TensorProto), committed as fixtures; the GPU
tests parse and execute them with iconnx_amd.onnx and GpuGraphExecutor.

    python tests/golden/copy_onnx_models.py [/root/reference]
"""
import os
import shutil
import sys

TESTS = [
    "test_dynamicquantizelinear", "test_dynamicquantizelinear_max_adjusted",
    "test_dynamicquantizelinear_min_adjusted", "test_matmulinteger", "test_dequantizelinear",
    "test_dequantizelinear_axis", "test_mul", "test_mul_bcast", "test_add", "test_add_bcast",
    "test_div", "test_div_bcast", "test_sub", "test_sub_bcast",
    "test_layer_normalization_2d_axis_negative_1",
    "test_layer_normalization_3d_axis_negative_1_epsilon", "test_softmax_axis_2",
    "test_softmax_example", "test_erf", "test_transpose_default",
    "test_transpose_all_permutations_0", "test_matmul_2d", "test_matmul_3d",
    # Gather (the UINT8 embedding table of DistilBERT-INT8 goes through it)
    "test_gather_0", "test_gather_1", "test_gather_2d_indices", "test_gather_negative_indices",
    # the LayerNorm of an export below opset 17, node by node: ReduceMean, Pow, Sqrt
    "test_reduce_mean_default_axes_keepdims_example", "test_reduce_mean_default_axes_keepdims_random",
    "test_reduce_mean_do_not_keepdims_example", "test_reduce_mean_do_not_keepdims_random",
    "test_reduce_mean_keepdims_example", "test_reduce_mean_keepdims_random",
    "test_reduce_mean_negative_axes_keepdims_example", "test_reduce_mean_negative_axes_keepdims_random",
    "test_pow", "test_pow_bcast_array", "test_pow_bcast_scalar", "test_pow_example",
    "test_sqrt", "test_sqrt_example",
    # the shape / mask plumbing of an exported encoder: reshape targets from Shape, position
    # ids by Slice, the attention mask by Equal / Unsqueeze / Expand / Where
    "test_shape", "test_shape_example", "test_shape_start_1", "test_shape_end_1",
    "test_shape_start_negative_1", "test_shape_end_negative_1", "test_shape_start_1_end_2",
    "test_shape_start_1_end_negative_1", "test_shape_clip_start", "test_shape_clip_end",
    "test_unsqueeze_axis_0", "test_unsqueeze_axis_1", "test_unsqueeze_axis_2",
    "test_unsqueeze_negative_axes", "test_unsqueeze_three_axes", "test_unsqueeze_two_axes",
    "test_unsqueeze_unsorted_axes", "test_squeeze", "test_squeeze_negative_axes",
    "test_concat_1d_axis_0", "test_concat_1d_axis_negative_1", "test_concat_2d_axis_0",
    "test_concat_2d_axis_1", "test_concat_2d_axis_negative_1", "test_concat_2d_axis_negative_2",
    "test_concat_3d_axis_0", "test_concat_3d_axis_1", "test_concat_3d_axis_2",
    "test_concat_3d_axis_negative_1", "test_concat_3d_axis_negative_2",
    "test_concat_3d_axis_negative_3",
    "test_slice", "test_slice_default_axes", "test_slice_default_steps",
    "test_slice_end_out_of_bounds", "test_slice_neg", "test_slice_neg_steps",
    "test_slice_negative_axes", "test_slice_start_out_of_bounds",
    "test_expand_dim_changed", "test_expand_dim_unchanged", "test_equal", "test_equal_bcast",
    "test_where_example", "test_where_long_example",
]


def main(ref):
    src_root = os.path.join(ref, "tests", "conformance_data", "onnx-1.18", "node")
    dst_root = os.path.join(os.path.dirname(os.path.abspath(__file__)), "onnx_node")
    for t in TESTS:
        src, dst = os.path.join(src_root, t), os.path.join(dst_root, t)
        os.makedirs(os.path.join(dst, "test_data_set_0"), exist_ok=True)
        shutil.copyfile(os.path.join(src, "model.onnx"), os.path.join(dst, "model.onnx"))
        for f in sorted(os.listdir(os.path.join(src, "test_data_set_0"))):
            if f.endswith(".pb"):
                shutil.copyfile(os.path.join(src, "test_data_set_0", f),
                                os.path.join(dst, "test_data_set_0", f))
    print("copied %d models to %s" % (len(TESTS), dst_root))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
