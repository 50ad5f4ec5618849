/* A small GQA model for tests of the CLI: 2 layers, 4 query / 2 KV heads of 64. */
#pragma once
#define MODEL_NAME "Tiny-GQA"
#define DIM 128
#define HIDDEN 256
#define HEADS 4
#define KV_HEADS 2
#define HD 64
#define SEQ 64
#define NLAYERS 2
#define VOCAB 512
#define ROPE_THETA 10000.0f
#define QK_NORM 0
#define CKPT_PATH "ane_tiny_dyn_ckpt.bin"
#define DEFAULT_DATA_PATH "../tinystories_data00.bin"
