from natten_mps_amd.autograd._factory import (
    create_na_autograd_fn,
    create_na_av_autograd_fn,
    create_na_global_autograd_fn,
    create_na_lse_autograd_fn,
    create_na_qk_autograd_fn,
)

NeighborhoodAttention1DFunction = create_na_autograd_fn(1)
NeighborhoodAttention1DLSEFunction = create_na_lse_autograd_fn(1)
NeighborhoodAttention1DGlobalFunction = create_na_global_autograd_fn(1)
NA1DQKFunction = create_na_qk_autograd_fn(1)
NA1DAVFunction = create_na_av_autograd_fn(1)
