// Paged decode-attention kernels with bf16 KV pages.
#define HELM_TKV helm::bf16_t
#define HELM_TKV_IS_16BIT 1
#define HELM_LAUNCH_NAME launch_attn_bf16
#include "attn_dispatch.h"
