/*
 * Host build of the sampler's correctly rounded math (gemma4.pas_amd/csrc/
 * g4s_crmath.h) for CPU tests: the same header the gfx950 kernels include,
 * compiled by g++ with -ffp-contract=off, so its results can be checked
 * against long double and mpmath references without a GPU.
 */
#include "../../gemma4.pas_amd/csrc/g4s_crmath.h"

using namespace g4s::cr;

extern "C" {
float t_exp_cr32(double xh, double xl) { return exp_cr32(xh, xl); }
float t_exp_diff_cr32(float a, float b) { return exp_diff_cr32(a, b); }
int t_exp_diff_cr32_try(float a, float b, float* r) { return exp_diff_cr32_try(a, b, r) ? 1 : 0; }
int t_exp_cr32_try(double xh, double xl, float* r) { return exp_cr32_try(xh, xl, r) ? 1 : 0; }
/* n pairs: ok[i] = 1 when the try path settled pair i, out_try[i] its value,
 * out_ref[i] = exp_diff_cr32(a[i], b[i]) */
void t_exp_diff_try_bulk(const float* a, const float* b, float* out_try, float* out_ref, int* ok, long n)
{
    for (long i = 0; i < n; ++i) {
        ok[i] = exp_diff_cr32_try(a[i], b[i], &out_try[i]) ? 1 : 0;
        out_ref[i] = exp_diff_cr32(a[i], b[i]);
    }
}
double t_exp_fast_d(double x) { return exp_fast_d(x); }
void t_exp_dd(double xh, double xl, double* out) { dd r = exp_dd(xh, xl); out[0] = r.hi; out[1] = r.lo; }
double t_tanh_fast_d(double w) { return tanh_fast_d(w); }
void t_tanh_dd(double wh, double wl, double* out) { dd r = tanh_dd(dd{wh, wl}); out[0] = r.hi; out[1] = r.lo; }
float t_softcap_topk_cr32(float x, float cap) { return softcap_topk_cr32(x, cap); }
float t_softcap_full_cr32(float x, float inv_cap, float cap) { return softcap_full_cr32(x, inv_cap, cap); }
float t_mul_u_p_cr32(double u, float p) { return mul_u_p_cr32(u, p); }
float t_round_dd_f32(double hi, double lo) { return round_dd_f32(hi, lo); }
int t_rounding_safe(double y, int tol, double eps) { return rounding_safe(y, tol, eps) ? 1 : 0; }
/* bulk helpers: n elements */
void t_exp_diff_bulk(const float* a, const float* b, float* out, long n) { for (long i = 0; i < n; ++i) out[i] = exp_diff_cr32(a[i], b[i]); }
void t_softcap_topk_bulk(const float* x, float cap, float* out, long n) { for (long i = 0; i < n; ++i) out[i] = softcap_topk_cr32(x[i], cap); }
void t_softcap_full_bulk(const float* x, float inv_cap, float cap, float* out, long n) { for (long i = 0; i < n; ++i) out[i] = softcap_full_cr32(x[i], inv_cap, cap); }
}
