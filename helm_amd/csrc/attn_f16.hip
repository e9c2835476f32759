// Paged decode-attention kernels with f16 KV pages.
#define HELM_TKV helm::f16_t
#define HELM_TKV_IS_16BIT 1
#define HELM_LAUNCH_NAME launch_attn_f16
#include "attn_dispatch.h"
