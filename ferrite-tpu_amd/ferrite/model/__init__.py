from ferrite.model.gpt import GPTConfig, forward, init_params, loss_fn, param_count

__all__ = ["GPTConfig", "forward", "init_params", "loss_fn", "param_count"]
