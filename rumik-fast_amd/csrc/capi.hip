// Exported C ABI (include/rumik_hip.h): host-side validation and dispatch. Kernels live in the other files.
#include "internal.h"

extern "C" {

int rk_abi_version(void) { return 5; }

const char* rk_status_string(int status) {
    switch (status) {
        case RK_OK: return "ok";
        case RK_ERR_SHAPE: return "shape";
        case RK_ERR_BLOCK: return "unsupported block shape";
        case RK_ERR_DTYPE: return "unsupported dtype";
        case RK_ERR_NULL: return "null pointer";
        case RK_ERR_ALIGN: return "misaligned pointer (16-byte alignment required)";
        case RK_ERR_LAUNCH: return "kernel launch failed";
        case RK_ERR_SCRATCH: return "workspace larger than the library's fixed scratch (RK_MM_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

int rk_gemv_int4_g128(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale, const uint16_t* min,
                      void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream) {
    // Path per shape, from measurements on MI355X (hipGraph-timed, weights rotated past the 256 MB MALL):
    // many short rows (N >= 8192, K <= 4096: the fused q/k/v/gate/up projection) run faster on the matrix
    // cores; long rows (K = 11008) and small N run faster on the VALU kernel.
    if (N >= 8192 && K <= 4096) {
        if (rows && !(rows == 1 || rows == 2 || rows == 4 || rows == 8)) return RK_ERR_BLOCK;
        return gemv_int4_mfma_launch(x, x_dtype, q, scale, min, y, y_dtype, N, K, waves, stream);
    }
    return gemv_int4_valu_launch(x, x_dtype, q, scale, min, y, y_dtype, N, K, waves, rows, stream);
}

// The MFMA kernel for every shape (16-row tile per wave; `rows` validated, unused).
int rk_gemv_int4_g128_mfma(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                           const uint16_t* min, void* y, int y_dtype, int N, int K, int waves, int rows,
                           rk_stream_t stream) {
    if (rows && !(rows == 1 || rows == 2 || rows == 4 || rows == 8)) return RK_ERR_BLOCK;
    return gemv_int4_mfma_launch(x, x_dtype, q, scale, min, y, y_dtype, N, K, waves, stream);
}

// The same GEMV with the multiply-adds on the VALU (v_dot2_f32_f16, exact 1024-magic dequant, transposed DPP
// row reduction): R rows per wave, the reference's (warps, rows) knobs map to (waves per block, rows per wave).
int rk_gemv_int4_g128_valu(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                           const uint16_t* min, void* y, int y_dtype, int N, int K, int waves, int rows,
                           rk_stream_t stream) {
    return gemv_int4_valu_launch(x, x_dtype, q, scale, min, y, y_dtype, N, K, waves, rows, stream);
}

// Two independent int4 GEMVs (y1 = W1 x1, y2 = W2 x2) in one launch: the layer's o and down projections.
int rk_gemv_int4_g128_pair(const void* x1, int x1_dtype, const uint8_t* q1, const uint16_t* s1, const uint16_t* m1,
                           void* y1, int y1_dtype, int N1, int K1, const void* x2, int x2_dtype, const uint8_t* q2,
                           const uint16_t* s2, const uint16_t* m2, void* y2, int y2_dtype, int N2, int K2,
                           rk_stream_t stream) {
    return gemv_int4_pair_launch(x1, x1_dtype, q1, s1, m1, y1, y1_dtype, N1, K1, x2, x2_dtype, q2, s2, m2, y2,
                                 y2_dtype, N2, K2, stream);
}

int rk_gemv_int8_rows(const void* x, int x_dtype, const void* q, int q_kind, const void* scale, int s_dtype,
                      void* y, int y_dtype, int N, int K, rk_stream_t stream) {
    return gemv_int8_rows_launch(x, x_dtype, q, q_kind, scale, s_dtype, y, y_dtype, N, K, 0, 0, stream);
}

// Block-shape-explicit int8 GEMV (waves per block, rows per wave; 0 = default), for tuning sweeps.
int rk_gemv_int8_rows_ex(const void* x, int x_dtype, const void* q, int q_kind, const void* scale, int s_dtype,
                         void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream) {
    return gemv_int8_rows_launch(x, x_dtype, q, q_kind, scale, s_dtype, y, y_dtype, N, K, waves, rows, stream);
}

}  // extern "C"
