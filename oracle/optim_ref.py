"""Test infrastructure only (never imported by the product): a float32 numpy restatement of
ExponentiatedAdam.update_step (v1_model_utils/optimizers.py:268-376, dense branch :354-376), and
SignedConstraint (v1_model_utils/models.py:419-427), in TF's operation order."""
import numpy as np

f32 = np.float32


def alpha(lr, beta_1, beta_2, step):
    """optimizers.py:273-283: lr * sqrt(1 - beta_2^t) / (1 - beta_1^t), fp32, t = step."""
    t = f32(step)
    b1p, b2p = np.power(f32(beta_1), t), np.power(f32(beta_2), t)
    return f32(f32(lr) * np.sqrt(f32(1) - b2p)) / (f32(1) - b1p)


def exp_adam_step(w, m, v, g, a, beta_1=0.9, beta_2=0.999, eps=1e-7, vhat=None, positive=None):
    """One step in place on float32 arrays (optimizers.py:354-376, then the constraint)."""
    one_m_b1, one_m_b2 = f32(1) - f32(beta_1), f32(1) - f32(beta_2)
    m += (g - m) * one_m_b1                                   # :356
    v += (g * g - v) * one_m_b2                               # :358
    u = v
    if vhat is not None:                                      # :360-364 AMSGrad
        np.maximum(vhat, v, out=vhat)
        u = vhat
    ag = m / (np.sqrt(u) + f32(eps))                          # :368
    s = np.sign(w)                                            # :371-372, sign(0) = +1
    s[s == 0] = 1
    w *= np.exp((-a * ag) * s).astype(f32)                    # :374-376
    if positive is not None:                                  # models.py:425-427
        w[...] = np.where(positive, np.maximum(w, 0), -np.maximum(-w, 0))
    return w
