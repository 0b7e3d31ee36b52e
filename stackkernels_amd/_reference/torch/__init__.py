from stackkernels_amd._reference.torch.attention import attention_reference, repeat_kv

__all__ = ["attention_reference", "repeat_kv"]
