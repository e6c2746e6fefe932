/*
 * libstade_hip -- MI355X (gfx950) execution of STADE-generated derivative code.
 *
 * Each `stade_hip_<k>_<mode>` entry point replaces one generated host function of
 * `stade_amdgpu_file` (/root/reference/src/STADE.jl:18604-18605): `<k>_b_amdgpu` (adjoint),
 * `<k>_d_amdgpu` (tangent) or `<k>_hv_amdgpu` (Hessian-vector product), for the kernel text
 * `stade.jl_amd/corpus/<k>.jl` and its generated `_b/_d/_hv` texts.
 *
 * Conventions, shared by every entry point:
 *   - Arguments follow the generated function's own order (`agen_signature_args`
 *     /root/reference/src/STADE.jl:3455-3464: each float argument followed by its shadow,
 *     Int64 arguments once, then the stacks; `tgen_signature_args` 3306-3315; `hvp_emit`
 *     6750-6756: the adjoint list, then (xd, xbd) per float argument, then the stacks).
 *   - Arrays are device pointers to the caller's column-major, densely packed Julia arrays
 *     (the pointer of a ROCArray).  Indices keep Julia's meaning: element (i, j) of an
 *     (m, n) array is at offset (i-1) + (j-1)*m.  Element alignment is enough: a view into a
 *     larger array is accepted (16-byte vector paths check alignment and fall back).
 *   - Outputs are mutated in place exactly as the generated code does: primal outputs are
 *     overwritten, shadows are accumulated (not overwritten), statement resets zero the
 *     shadows the generated code zeroes, stacks are written by the forward sweep.
 *   - A float scalar argument is passed by value; its shadow is a host pointer that holds
 *     the seed on entry and the generated function's returned value on exit (the adjoint
 *     returns scalar shadows, 3672; the HVP returns (xb, xbd) pairs, 6772-6779).  An entry
 *     point with such outputs synchronises `stream` once before returning; the others only
 *     enqueue work on `stream` (NULL = the default stream).
 *   - Return value: 0 on success; a positive hipError_t code or a negative STADE_HIP_E*
 *     code on failure, with a message in stade_hip_last_error().  Argument errors are
 *     reported before any work is enqueued.
 *   - Calls on one device share a library workspace (reduction partials, device scalars and
 *     scratch).  Calls are serialised per device: a host thread holds the device's lock while
 *     it enqueues, and a call on a stream other than the previous call's first waits
 *     (hipStreamWaitEvent) for the event that call recorded at its end, so calls on different
 *     streams run one after the other instead of racing.
 *   - Graph capture: a call on a capturing stream takes no dependency outside the capture, and
 *     the workspace does not grow under capture (STADE_HIP_ESTATE): make one eager call of the
 *     largest size first.  Replays are not ordered against eager calls on other streams (the
 *     caller orders them, as any graph); they share the workspace with those calls.  A scratch
 *     buffer that a captured graph may hold is never freed: a later, larger eager call retires
 *     it and allocates another, so earlier graphs stay valid.
 */
#ifndef STADE_HIP_H
#define STADE_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STADE_HIP_OK 0
#define STADE_HIP_EINVAL (-1)
#define STADE_HIP_ENOMEM (-2)
#define STADE_HIP_ERANGE (-3)
#define STADE_HIP_ESTATE (-4)   /* not possible in the library's current state (e.g. workspace growth under graph capture) */

/* ---- library ------------------------------------------------------------------------ */
const char* stade_hip_last_error(void);
const char* stade_hip_version(void);
int32_t stade_hip_free(void* p);
int32_t stade_hip_synchronize(hipStream_t stream);
/* Device-side input error (an index the generated code would reject with a BoundsError,
 * such as a label outside 1..i_out): 1 if raised since the last read, then cleared.
 * Synchronous. */
int32_t stade_hip_device_error(int32_t* flag);

/* Library workspace of the current device (no counterpart in the reference: the generated
 * code allocates per call): the bytes of scratch held, and the number of scratch buffers
 * retired because a captured graph may still use them (kept until the process ends). */
int32_t stade_hip_workspace_info(int64_t* scratch_bytes, int64_t* retired);

/* ---- kernel timing (no counterpart in the reference; its timings come from an external
 * bench kit, /root/reference/claude/manual-stade-dev.md:2040).  While enabled, every kernel
 * launch is bracketed by HIP events on the launch's stream; read() waits for the pending
 * events and returns the summed elapsed time and launch count of one kernel name. */
int32_t stade_hip_profile_start(void);
int32_t stade_hip_profile_stop(void);
int32_t stade_hip_profile_read(const char* kernel, double* total_ms, int64_t* launches);

/* ---- inputs: STADE's stable seed and Julia's Random.Xoshiro scalar stream -------------
 * stade_hip_stable_seed  = `val_stable_seed` (FNV-1a64), /root/reference/src/STADE.jl:16619-16625
 * stade_hip_rng_seed     = `Random.Xoshiro(seed)` state (Julia 1.10 seeding)
 * stade_hip_rng_normal_f64 = n draws of `val_normal(rng)`, 16628-16637
 * stade_hip_rng_uniform_f64 = n draws of `lo + (hi - lo) * rand(rng)`
 * stade_hip_rng_int_range = n draws of lo + floor(rand(rng) * (hi - lo + 1))
 * Host memory; no device work. */
uint64_t stade_hip_stable_seed(const char* name);
int32_t stade_hip_rng_seed(uint64_t seed, uint64_t state[4]);
int32_t stade_hip_rng_normal_f64(uint64_t state[4], double* out, int64_t n);
int32_t stade_hip_rng_uniform_f64(uint64_t state[4], double* out, int64_t n, double lo, double hi);
int32_t stade_hip_rng_int_range(uint64_t state[4], int64_t* out, int64_t n, int64_t lo, int64_t hi);

/* ---- config 1: affine_lsq(loss, w, x, b, t, r, i_m, i_n) -------------------------------
 * loss += 0.5 * sum((w * x + b - t) .^ 2), w (i_m, i_n) Float64.
 * replaces affine_lsq_b_amdgpu / _d_amdgpu / _hv_amdgpu (corpus/affine_lsq_{b,d,hv}.jl) */
int32_t stade_hip_affine_lsq_b(double* loss, const double* lossb, const double* w, double* wb, const double* x, double* xb,
                               const double* b, double* bb, const double* t, double* tb, double* r, double* rb,
                               int64_t i_m, int64_t i_n, hipStream_t stream);
int32_t stade_hip_affine_lsq_d(double* loss, double* lossd, const double* w, const double* wd, const double* x, const double* xd,
                               const double* b, const double* bd, const double* t, const double* td, double* r, double* rd,
                               int64_t i_m, int64_t i_n, hipStream_t stream);
int32_t stade_hip_affine_lsq_hv(double* loss, const double* lossb, const double* w, double* wb, const double* x, double* xb,
                                const double* b, double* bb, const double* t, double* tb, double* r, double* rb,
                                int64_t i_m, int64_t i_n, double* lossd, const double* lossbd, const double* wd, double* wbd,
                                const double* xd, double* xbd, const double* bd, double* bbd, const double* td, double* tbd,
                                double* rd, double* rbd, hipStream_t stream);

/* ---- config 2: diffusion2d(loss, u, un, n) ---------------------------------------------
 * one periodic 5-point step un = u + 0.1 * lap(u) on n x n, then loss += sum(un .^ 2).
 * replaces diffusion2d_b_amdgpu / _d_amdgpu / _hv_amdgpu (corpus/diffusion2d_{b,d,hv}.jl);
 * the adjoint scatter is the owner-computes gather of `cgen_gather_periodic_inverse`
 * (/root/reference/src/STADE.jl:7343-7529).  n <= 46340. */
int32_t stade_hip_diffusion2d_b(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                int64_t n, hipStream_t stream);
int32_t stade_hip_diffusion2d_d(double* loss, double* lossd, const double* u, const double* ud, double* un, double* und,
                                int64_t n, hipStream_t stream);
int32_t stade_hip_diffusion2d_hv(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                 int64_t n, double* lossd, const double* lossbd, const double* ud, double* ubd, double* und,
                                 double* unbd, hipStream_t stream);
/* No counterpart in the reference: stade_hip_diffusion2d_b for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same arguments, effects and kernels; the pass-1 loss partials live in a static device array
 * of 131072 doubles (1 MiB per GPU, held until the process ends) instead of the library
 * workspace, and the call makes no allocation.  A grid needing more partials than that
 * (n above 23168 in the worst case; 32768 when n is a multiple of 128 and the arrays are
 * 16-byte aligned) is refused with STADE_HIP_ERANGE before any work.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (different streams or threads) race. */
int32_t stade_hip_diffusion2d_b_noalloc(double* loss, const double* lossb, const double* u, double* ub, double* un,
                                        double* unb, int64_t n, hipStream_t stream);

/* ---- config 5: burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps) ------------------------
 * explicit viscous Burgers on n periodic cells, at most nsteps steps, each taken while the
 * elapsed time is below tend (a counted loop with a guard), then loss += sum(u .^ 2).
 * replaces initstacks_burgers1d_b / burgers1d_b_amdgpu / _d_amdgpu / _hv_amdgpu
 * (corpus/burgers1d_{b,d,hv}.jl).  Stacks: branch_stack Int64[nsteps] (1 = step taken),
 * u_stack Float64[nsteps * n] with u_stack[(x-1) + (t-1)*n + 1] = state at the start of step t
 * (`agen_local_position` /root/reference/src/STADE.jl:4867-4881).  The HVP's shadow tape
 * (`u_stack_d`, allocated inside the generated _hv, 6864-6866) is library scratch. */
int32_t stade_hip_burgers1d_stack_lengths(int64_t n, int64_t nsteps, int64_t lengths[2]);
int32_t stade_hip_initstacks_burgers1d_b(int64_t n, int64_t nsteps, int64_t** branch_stack, double** u_stack);
int32_t stade_hip_burgers1d_b(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                              double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                              int64_t n, int64_t nsteps, int64_t* branch_stack, double* u_stack, hipStream_t stream);
int32_t stade_hip_burgers1d_d(double* loss, double* lossd, double* u, double* ud, double* un, double* und, double nu, double nud,
                              double dt, double dtd, double dx, double dxd, double tend, double tendd, int64_t n, int64_t nsteps,
                              hipStream_t stream);
int32_t stade_hip_burgers1d_hv(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                               double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                               int64_t n, int64_t nsteps, double* lossd, const double* lossbd, const double* ud, double* ubd,
                               double* und, double* unbd, double nud, double* nubd, double dtd, double* dtbd, double dxd,
                               double* dxbd, double tendd, double* tendbd, int64_t* branch_stack, double* u_stack,
                               hipStream_t stream);

/* Tape policy: checkpoints and segment recompute.  The generated functions keep the state of
 * every step (u_stack, nsteps * n values; the HVP's u_stack_d as many again).  Under this
 * policy the caller passes u_ckpt instead, the state at the start of every `every`-th step
 * (ceil(nsteps / every) * n values, stade_hip_burgers1d_ckpt_lengths); the reverse sweep
 * recomputes each segment of `every` steps from its checkpoint into an `every`-row tape in
 * library scratch and sweeps it back.  Every other output (loss, ub, un, unb, branch_stack,
 * the scalar shadows, and for the HVP their tangents) is that of stade_hip_burgers1d_b / _hv;
 * u_ckpt row k equals u_stack row k * every.  The reference's counterpart is a generator
 * policy, not an ABI: its `ii_` recompute planning (/root/reference/src/STADE.jl:19314-20273)
 * and rematerialised restores (`agen_remat_*` 5687-5899) rewrite the generated text so that
 * values are recomputed in the reverse sweep instead of stored. */
int32_t stade_hip_burgers1d_ckpt_lengths(int64_t n, int64_t nsteps, int64_t every, int64_t lengths[2]);
int32_t stade_hip_burgers1d_b_ckpt(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                   double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend,
                                   double* tendb, int64_t n, int64_t nsteps, int64_t* branch_stack, double* u_ckpt, int64_t every,
                                   hipStream_t stream);
int32_t stade_hip_burgers1d_hv_ckpt(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                    double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                                    int64_t n, int64_t nsteps, double* lossd, const double* lossbd, const double* ud, double* ubd,
                                    double* und, double* unbd, double nud, double* nubd, double dtd, double* dtbd, double dxd,
                                    double* dxbd, double tendd, double* tendbd, int64_t* branch_stack, double* u_ckpt, int64_t every,
                                    hipStream_t stream);

/* ---- config 3: mlp2_ce(loss, x, lab, w1, b1, w2, b2, h1, z, i_b, i_in, i_h, i_out) --------
 * tanh hidden layer, softmax cross-entropy summed over the batch, Float32 arrays (STADE's
 * precision=Float32, `cgen_convert_precision` /root/reference/src/STADE.jl:15351-15365),
 * Int64 labels 1..i_out.  x (i_in, i_b), w1 (i_h, i_in), w2 (i_out, i_h), h1 (i_h, i_b),
 * z (i_out, i_b), column-major.  replaces mlp2_ce_b_amdgpu / _d_amdgpu / _hv_amdgpu
 * (corpus/mlp2_ce_{b,d,hv}.jl).  i_out <= 16, i_h <= 2048.  A label outside 1..i_out
 * contributes no term (the generated code would raise a BoundsError) and sets the device
 * error flag read by stade_hip_device_error. */
int32_t stade_hip_mlp2_ce_b(float* loss, const float* lossb, const float* x, float* xb, const int64_t* lab, const float* w1,
                            float* w1b, const float* b1, float* b1b, const float* w2, float* w2b, const float* b2, float* b2b,
                            float* h1, float* h1b, float* z, float* zb, int64_t i_b, int64_t i_in, int64_t i_h, int64_t i_out,
                            hipStream_t stream);
int32_t stade_hip_mlp2_ce_d(float* loss, float* lossd, const float* x, const float* xd, const int64_t* lab, const float* w1,
                            const float* w1d, const float* b1, const float* b1d, const float* w2, const float* w2d,
                            const float* b2, const float* b2d, float* h1, float* h1d, float* z, float* zd, int64_t i_b,
                            int64_t i_in, int64_t i_h, int64_t i_out, hipStream_t stream);
int32_t stade_hip_mlp2_ce_hv(float* loss, const float* lossb, const float* x, float* xb, const int64_t* lab, const float* w1,
                             float* w1b, const float* b1, float* b1b, const float* w2, float* w2b, const float* b2, float* b2b,
                             float* h1, float* h1b, float* z, float* zb, int64_t i_b, int64_t i_in, int64_t i_h, int64_t i_out,
                             float* lossd, const float* lossbd, const float* xd, float* xbd, const float* w1d, float* w1bd,
                             const float* b1d, float* b1bd, const float* w2d, float* w2bd, const float* b2d, float* b2bd,
                             float* h1d, float* h1bd, float* zd, float* zbd, hipStream_t stream);

/* ---- config 4: conv3x3(loss, xp, w, out, i_nb, i_c, i_k, i_h, i_w) ----------------------
 * 3 x 3 cross-correlation, stride 1, zero padding held in the input, then
 * loss += 0.5 * sum(out .^ 2); Float32.  xp (i_w+2, i_h+2, i_c, i_nb), w (3, 3, i_c, i_k),
 * out (i_w, i_h, i_k, i_nb), column-major.  replaces conv3x3_b_amdgpu / _d_amdgpu /
 * _hv_amdgpu (corpus/conv3x3_{b,d,hv}.jl).  xpb covers the padded frame too: taps that read
 * the padding accumulate their adjoint there, as the generated scatter does. */
int32_t stade_hip_conv3x3_b(float* loss, const float* lossb, const float* xp, float* xpb, const float* w, float* wb,
                            float* out, float* outb, int64_t i_nb, int64_t i_c, int64_t i_k, int64_t i_h, int64_t i_w,
                            hipStream_t stream);
int32_t stade_hip_conv3x3_d(float* loss, float* lossd, const float* xp, const float* xpd, const float* w, const float* wd,
                            float* out, float* outd, int64_t i_nb, int64_t i_c, int64_t i_k, int64_t i_h, int64_t i_w,
                            hipStream_t stream);
int32_t stade_hip_conv3x3_hv(float* loss, const float* lossb, const float* xp, float* xpb, const float* w, float* wb,
                             float* out, float* outb, int64_t i_nb, int64_t i_c, int64_t i_k, int64_t i_h, int64_t i_w,
                             float* lossd, const float* lossbd, const float* xpd, float* xpbd, const float* wd, float* wbd,
                             float* outd, float* outbd, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* STADE_HIP_H */
