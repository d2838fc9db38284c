"""What the batch-1 kernel's fp16 exchange of the cross-XCD partial sums costs, on the CPU.

tests/pi05_rounding.py restates the batch-1 loop in float64 with the kernel's roundings (bf16 MFMA
operands, chunked attention, fp16 partial sums with the parity bit). Run once with the partial sums
exchanged exactly and once as the kernel exchanges them, the two distances to the fp32 oracle isolate
the exchange's share. On the hardest case (18 layers, one Euler step of dt = -1, every residual gate 1,
all 32 action dims integrated) the fp16 exchange adds 3.8 % to the error of the bf16 operands alone
(mean-abs 6.46e-3 -> 6.70e-3); 2.5 % on the benchmark shape (18 layers x 10 steps, Lp = 968, Tv = 50) (3.09e-4 -> 3.16e-4). The reference keeps
the partial sums in fp32 (src/pi05/mk6.cu:63, 147). The restatement's own planted mistake (a dropped
exchange rounding would leave the two runs equal) is ruled out by requiring them to differ.
"""
from tests import pi05_case as P
from tests import pi05_rounding as R


def test_fp16_exchange_share_of_the_error_on_the_hard_case():
    c = R.unit_gates(P.make_case(NL=18, Lp=968, Tv=50, S=1, seed=11))
    ref = P.run_oracle(c)[0]
    e32 = P.parity(R.denoise(c, "fp32"), ref)
    e16 = P.parity(R.denoise(c, "fp16"), ref)
    ratio = e16["mean_abs"] / e32["mean_abs"]
    print(f"hard case: bf16 operands alone {e32}, with the fp16 exchange {e16}, ratio {ratio:.3f}", flush=True)
    assert e16["mean_abs"] != e32["mean_abs"]
    assert ratio <= 1.10, (e32, e16)
