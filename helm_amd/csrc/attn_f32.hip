// Paged decode-attention kernels with f32 KV pages.
#define HELM_TKV float
#define HELM_TKV_IS_16BIT 0
#define HELM_LAUNCH_NAME launch_attn_f32
#include "attn_dispatch.h"
