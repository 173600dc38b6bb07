// ggml_rows.hpp -- a ggml tensor seen as rows of ne[0] values, for the
// backend's node kernels (ggml_backend.hip) and the reference-arithmetic
// row kernels they call (decode_ref.hip).
//
// Row r of a node is (i1, i2, i3) = (r % ne1, r / ne1 % ne2, r / (ne1 * ne2))
// of the node's own shape.  An operand whose shape equals the node's, or is
// repeated over it as ggml broadcasts (each of its ne1..ne3 divides the
// node's), holds that row at byte offset
//   (i1 % ne1) * nb1 + (i2 % ne2) * nb2 + (i3 % ne3) * nb3
// of its own ne / nb.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ane {

struct NodeRows {
    uint64_t ne1, ne2, ne3;
    uint64_t nb1, nb2, nb3;
};

struct RowIdx {
    uint64_t i1, i2, i3;
};

__host__ __device__ inline RowIdx row_index(const NodeRows& d, uint64_t r) {
    const uint64_t q = r / d.ne1;
    return RowIdx{r - q * d.ne1, q % d.ne2, q / d.ne2};
}

__host__ __device__ inline uint64_t row_offset(const NodeRows& m, const RowIdx& i) {
    return (i.i1 % m.ne1) * m.nb1 + (i.i2 % m.ne2) * m.nb2 + (i.i3 % m.ne3) * m.nb3;
}

// Row kernels in the reference handlers' arithmetic (decode_ref.hip), one
// launch over `rows` rows of `dim` floats; every operand's innermost stride
// is 4 bytes and its row offsets come from its NodeRows.
//   rms_norm_node_launch: out = rms_norm_fp32(in) with unit weights;
//   softmax_node_launch:  out = softmax_fp32(fl(fl(in * scale) + mask)),
//       mask optional (nullptr: fl(in * scale)); an element whose
//       x - max is -inf contributes exactly 0;
//   rope_node_launch:     out = rope_fp32(in) at theta, the row's position
//       pos[i2] (int32), adjacent pairs over all dim values.
int rms_norm_node_launch(uint32_t dim, uint64_t rows, float eps, const uint8_t* in, const NodeRows& src,
                         uint8_t* out, const NodeRows& dst, hipStream_t s);
int softmax_node_launch(uint32_t dim, uint64_t rows, float scale, const uint8_t* in, const NodeRows& src,
                        const uint8_t* mask, const NodeRows& msk, uint8_t* out, const NodeRows& dst, hipStream_t s);
int rope_node_launch(uint32_t dim, uint64_t rows, float theta, const int32_t* pos, const uint8_t* in,
                     const NodeRows& src, uint8_t* out, const NodeRows& dst, hipStream_t s);

}  // namespace ane
