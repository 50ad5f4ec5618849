/* Stories110M: Llama-2-shaped, 12 layers, multi-head attention (12 heads of 64).
 * Dimensions as in TD/models/stories110m.h:6-19 of the reference; RoPE base and the
 * absence of QK-norm as in the reference training step (TD/cpu_ops.h:466). */
#pragma once
#define MODEL_NAME "Stories110M"
#define DIM 768
#define HIDDEN 2048
#define HEADS 12
#define KV_HEADS 12
#define HD 64
#define SEQ 256
#define NLAYERS 12
#define VOCAB 32000
#define ROPE_THETA 10000.0f
#define QK_NORM 0
#define CKPT_PATH "ane_stories110M_dyn_ckpt.bin"
#define DEFAULT_DATA_PATH "../tinystories_data00.bin"
