/* internal.h — helpers shared by the Mamba and RWKV-7 parts of the CPU oracle (test
 * infrastructure only; not exported through oracle.h). */
#ifndef REDUKT_ORACLE_INTERNAL_H
#define REDUKT_ORACLE_INTERNAL_H

#include <stdint.h>
#include <stdio.h>

/* A weight matrix as the reference holds it: F32, or int8 with f32 scales per group of
 * `group` columns (Q8wMatrix, src/domain/gemv.rs:244-273). */
typedef struct {
    int rows, cols, group; /* group: 0 = F32 */
    int fma;               /* GEMV in numeric contract 2 (fma-v1) instead of 1 */
    float* f;              /* F32 data (NULL for Q8) */
    int8_t* q;
    float* sc;
} Mat;

/* Takes ownership of `data` (kept for F32, quantized and freed for Q8). */
int mat_make(Mat* m, float* data, int rows, int cols, int quant, int group);
void mat_free(Mat* m);
void mat_row(const Mat* m, int row, float* out);
/* Rows [r0, r1) of out = M·v in the reference order (f32_rows / q8w_rows). */
void mat_rows(const Mat* m, int r0, int r1, const float* v, float* out);
float* read_f32(FILE* f, size_t count);
float orc_lane_sigmoidf(float x);

#endif
