/* Qwen3-0.6B: 28 layers, grouped-query attention 16 query / 8 KV heads of 128.
 * Dimensions as in TD/models/qwen3_06b.h:6-19 of the reference.  The reference training
 * step has no QK-norm and RoPE base 10000 (TD/mil_dynamic.h:737, TD/cpu_ops.h:466); these
 * defaults keep that behaviour, and --qk-norm / --rope-theta select Qwen3's own values. */
#pragma once
#define MODEL_NAME "Qwen3-0.6B"
#define DIM 1024
#define HIDDEN 3072
#define HEADS 16
#define KV_HEADS 8
#define HD 128
#define SEQ 256
#define NLAYERS 28
#define VOCAB 151936
#define ROPE_THETA 10000.0f
#define QK_NORM 0
#define CKPT_PATH "ane_qwen3_06b_dyn_ckpt.bin"
#define DEFAULT_DATA_PATH "../tinystories_data00.bin"
