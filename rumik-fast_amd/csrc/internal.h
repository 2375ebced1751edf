// Launchers shared between the library's translation units. Not part of the C ABI: the library is built with
// hidden visibility and only include/rumik_hip.h is exported.
#pragma once
#include "common.h"

int gemv_int4_valu_launch(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale, const uint16_t* min,
                          void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream);
int gemv_int4_mfma_launch(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale, const uint16_t* min,
                          void* y, int y_dtype, int N, int K, int waves, rk_stream_t stream);
int gemv_int4_pair_launch(const void* x1, int x1_dtype, const uint8_t* q1, const uint16_t* s1, const uint16_t* m1,
                          void* y1, int y1_dtype, int N1, int K1, const void* x2, int x2_dtype, const uint8_t* q2,
                          const uint16_t* s2, const uint16_t* m2, void* y2, int y2_dtype, int N2, int K2,
                          rk_stream_t stream);
int gemv_int8_rows_launch(const void* x, int x_dtype, const void* q, int q_kind, const void* scale, int s_dtype,
                          void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream);
