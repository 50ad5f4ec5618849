/* Qwen3-0.6B at sequence length 512 (TD/models/qwen3_06b_seq512.h of the reference). */
#pragma once
#define MODEL_NAME "Qwen3-0.6B-seq512"
#define DIM 1024
#define HIDDEN 3072
#define HEADS 16
#define KV_HEADS 8
#define HD 128
#define SEQ 512
#define NLAYERS 28
#define VOCAB 151936
#define ROPE_THETA 10000.0f
#define QK_NORM 0
#define CKPT_PATH "ane_qwen3_dyn_seq512_ckpt.bin"
#define DEFAULT_DATA_PATH "../tinystories_data00.bin"
