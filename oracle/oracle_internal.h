/* Test infrastructure only: internals shared by the oracle's C files. */
#ifndef FURNACE_ORACLE_INTERNAL_H
#define FURNACE_ORACLE_INTERNAL_H
#include <stdint.h>
void orc_set_error(const char* fmt, ...);
void orc_dequant_block_q5_0(const uint8_t* b, float* out);
void orc_dequant_block_q4_k(const uint8_t* b, float* out);
void orc_dequant_block_q6_k(const uint8_t* b, float* out);
#endif
