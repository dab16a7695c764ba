from natten_mps_amd.autograd._factory import (
    create_na_autograd_fn,
    create_na_av_autograd_fn,
    create_na_global_autograd_fn,
    create_na_lse_autograd_fn,
    create_na_qk_autograd_fn,
)

NeighborhoodAttention3DFunction = create_na_autograd_fn(3)
NeighborhoodAttention3DLSEFunction = create_na_lse_autograd_fn(3)
NeighborhoodAttention3DGlobalFunction = create_na_global_autograd_fn(3)
NA3DQKFunction = create_na_qk_autograd_fn(3)
NA3DAVFunction = create_na_av_autograd_fn(3)
