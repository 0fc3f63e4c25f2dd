"""burn_dragon_amd: MI355X (gfx950) HIP implementation of burn_dragon's
recurrent linear-attention forward path (chunked bf16-MFMA prefill with fused
RoPE, sparse bandwidth-bound decode), behind the reference's custom-op
surface.  The compute lives in libbdh_hip.so (C ABI: include/bdh_hip.h)."""
from .recurrent import (CompiledRecurrentAttentionPlan, KernelProfileSnapshot,  # noqa: F401
                        RecurrentAttentionOutput, RecurrentProfileSnapshot, alibi_decay,
                        default_alibi_slopes,
                        recurrent_profile_enable, recurrent_profile_reset,
                        recurrent_profile_snapshot, release_stream_scratch, supports_backend,
                        supports_recurrent_backend, try_fused_recurrent_attention,
                        try_fused_recurrent_attention_rope,
                        try_fused_recurrent_attention_wgpu,
                        try_fused_recurrent_attention_wgpu_with_plan,
                        try_fused_recurrent_attention_with_plan)
from .attention import (CompiledDenseCausalAttentionPlan,  # noqa: F401
                        supports_dense_causal_attention_backend,
                        try_fused_dense_causal_attention,
                        try_fused_dense_causal_attention_wgpu,
                        try_fused_dense_causal_attention_with_plan)
from .backward import (DenseCausalAttentionVjp, RecurrentAttentionGrads,  # noqa: F401
                       dense_causal_attention_vjp, dense_causal_attention_vjp_with_initial_rho,
                       recurrent_attention_vjp)
from .decode import DecodeOutput, decode_step  # noqa: F401
from .layer import LowRankLayerOutput, LowRankWeights, lowrank_layer_forward  # noqa: F401
from .model import (BdhModelState, BdhModelWeights, load_model_state, model_forward_logits,  # noqa: F401
                    new_model_state, pack_model, save_model_state)
