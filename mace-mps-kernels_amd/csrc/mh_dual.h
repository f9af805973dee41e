// mh_dual.h — forward-mode dual numbers for the second-order kernels (prepended to their generated source only).
//
// A value x + e d with e^2 = 0: running a function's own statements on duals gives, in the d part, its derivative
// along the direction placed in the inputs' d parts.  The kernels behind a double backward are the first-order
// kernels' statements with `float` replaced by `mh_dual`: the forward's d part is the Jacobian-vector product, the
// backward's d part (incoming gradient held real) the directional derivative of the gradient, a Hessian-vector
// product.  The value parts repeat the first-order arithmetic exactly.  Kept free of #includes (hipRTC); the
// functions are host-callable too so that the same statements can be checked on the CPU.
#pragma once

#ifndef MH_HD
#define MH_HD __host__ __device__
#endif

struct mh_dual {
    float v, d;
    MH_HD mh_dual() : v(0.f), d(0.f) {}
    MH_HD mh_dual(float a) : v(a), d(0.f) {}                 // constants carry no derivative
    MH_HD mh_dual(float a, float b) : v(a), d(b) {}
};

MH_HD inline mh_dual operator+(mh_dual a, mh_dual b) { return mh_dual(a.v + b.v, a.d + b.d); }
MH_HD inline mh_dual operator-(mh_dual a, mh_dual b) { return mh_dual(a.v - b.v, a.d - b.d); }
MH_HD inline mh_dual operator-(mh_dual a) { return mh_dual(-a.v, -a.d); }
MH_HD inline mh_dual operator*(mh_dual a, mh_dual b) { return mh_dual(a.v * b.v, a.d * b.v + a.v * b.d); }
MH_HD inline mh_dual operator/(mh_dual a, mh_dual b) {
    const float q = a.v / b.v;
    return mh_dual(q, (a.d - q * b.d) / b.v);
}
MH_HD inline mh_dual& operator+=(mh_dual& a, mh_dual b) { return a = a + b; }
MH_HD inline mh_dual& operator-=(mh_dual& a, mh_dual b) { return a = a - b; }
MH_HD inline mh_dual& operator*=(mh_dual& a, mh_dual b) { return a = a * b; }
MH_HD inline bool operator<(mh_dual a, float c) { return a.v < c; }
MH_HD inline bool operator>=(mh_dual a, float c) { return a.v >= c; }

// sqrt: derivative d / (2 sqrt v), taken as 0 at v == 0 (where callers clamp the result anyway)
MH_HD inline mh_dual sqrtf(mh_dual a) {
    const float s = sqrtf(a.v);
    return mh_dual(s, s > 0.f ? a.d / (2.f * s) : 0.f);
}
// max with a constant, the derivative passed where the value is kept (torch's clamp_min convention at equality)
MH_HD inline mh_dual fmaxf(mh_dual a, float c) { return a.v >= c ? a : mh_dual(c); }
MH_HD inline mh_dual sinf(mh_dual a) { return mh_dual(sinf(a.v), cosf(a.v) * a.d); }
MH_HD inline mh_dual cosf(mh_dual a) { return mh_dual(cosf(a.v), -sinf(a.v) * a.d); }
MH_HD inline mh_dual expf(mh_dual a) { const float e = expf(a.v); return mh_dual(e, e * a.d); }
