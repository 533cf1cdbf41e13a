"""MI355X-native per-matrix quantization hot path of LookAtMyQuant (Hessian, damped Cholesky, block LDLQ with
Lloyd-Max or bitshift-trellis Viterbi, KL sensitivity) behind the reference's Python entry points."""
