// gemv_chain.hip -- a decode step's INT4 GEMVs from one call.
//
// kc_gemv_int4_bf16_chain launches a list of kc_gemv_int4_bf16 GEMVs back to
// back on one stream, so that an op may read what earlier ops wrote (its x
// may be an earlier op's y) and a caller crosses the FFI boundary once per
// decode step instead of once per projection.  The reference's decode loop
// calls launch_gemv_int4 once per projection (quant_int4.cu:221-234).
//
// A single persistent launch with a device-wide barrier between the ops was
// built and measured first: on this runtime a cooperative launch alone costs
// about 19 us and each barrier 5-18 us (one arrival counter polled by every
// workgroup), against about 2 us of ramp-up and tail per GEMV, so successive
// launches are faster.
#include "kc_common.hpp"

extern "C" int kc_gemv_int4_bf16_chain(const kc_gemv_op* ops, int n_ops, kc_stream_t stream) {
    const char* fn = "kc_gemv_int4_bf16_chain";
    if (n_ops < 0 || n_ops > KC_GEMV_CHAIN_MAX_OPS || (n_ops > 0 && !ops))
        return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: n_ops=%d (at most %d, ops non-null)",
                             fn, n_ops, KC_GEMV_CHAIN_MAX_OPS);
    // validate every op before launching any
    for (int i = 0; i < n_ops; ++i) {
        const kc_gemv_op& o = ops[i];
        if (o.rows < 0 || o.cols < 0 || o.group_size <= 0 || o.cols % 2 != 0 ||
            (o.cols > 0 && o.cols % o.group_size != 0))
            return kc::set_error(KC_ERR_INVALID_ARGUMENT,
                                 "%s: op %d: rows=%d cols=%d group_size=%d", fn, i, o.rows,
                                 o.cols, o.group_size);
        if (o.rows > 0 && (!o.y || (o.cols > 0 && (!o.packed || !o.scales || !o.zeros || !o.x))))
            return kc::set_error(KC_ERR_INVALID_ARGUMENT, "%s: op %d: null device pointer", fn, i);
    }
    for (int i = 0; i < n_ops; ++i) {
        const kc_gemv_op& o = ops[i];
        const int st = kc_gemv_int4_bf16(o.packed, o.scales, o.zeros, o.x, o.y, o.rows, o.cols,
                                         o.group_size, stream);
        if (st != KC_SUCCESS) return st;
    }
    return KC_SUCCESS;
}
