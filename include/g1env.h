/* g1env.h -- C ABI of libg1env.so, the MI355X (gfx950) build of g1.cu's G1 environment and fused
 * rollout. The first block is the reference's own surface (Infatoshi/g1.cu src/g1_env.cu:361-476):
 * same symbol names, argument meaning, ownership and synchronisation. Errors print to stderr and
 * exit(1), as the reference's CK macro does (src/g1_env.cu:33-34).
 *
 * Ownership: the library owns the per-world device state (created by g1_env_create, freed by
 * g1_env_destroy). Pointers marked DEVICE are caller-owned device buffers (torch tensors'
 * data_ptr(), contiguous fp32); pointers marked HOST are host memory.
 * Streams: every launch goes to the null stream, which torch's default stream serialises with.
 */
#ifndef G1ENV_H
#define G1ENV_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the reference surface --------------------------------------------------------------- */

/* Allocate N worlds; substeps physics steps per control step; pgs_iters PGS sweeps; seed keys the
 * library's counter-based RNG (replaces curand_init). Blocks.  (src/g1_env.cu:405-422) */
void* g1_env_create(int N, int substeps, int pgs_iters, unsigned long seed);

/* Stand pose + 0.02*U(-1,1) on the 29 actuated joints, zero velocity and previous action; obs_out
 * HOST [N*100]. Blocks.  (src/g1_env.cu:424-429, k_reset :97-111) */
void g1_env_reset(void* h, float* obs_out);

/* One control step from HOST actions act [N*29]; writes HOST obs [N*100], rew [N], done [N]
 * (0/1 floats). Auto-resets finished worlds. Blocks.  (src/g1_env.cu:431-441, k_step :245-268) */
void g1_env_step(void* h, const float* act, float* obs, float* rew, float* done);

/* Fused rollout of H control steps. All pointers DEVICE: W packed policy (torch order W0,b0,W1,b1,
 * Wmu,bmu,Wv,bv,log_std), mean/var [100] frozen obs stats; outputs O [H*N*100] (raw obs),
 * A [H*N*29], LP/V/R/D [H*N], Vlast [N]. Asynchronous on the null stream. H <= 0 runs no control
 * step and writes only Vlast, as the reference's loop does. A work-queue error of the rollout
 * (see g1_env_check) stops the process at the caller's next call into the library.
 * (src/g1_env.cu:446-453, k_rollout :278-338) */
void g1_rollout(void* h, int H, const float* W, const float* mean, const float* var, float* O, float* A,
                float* LP, float* V, float* R, float* D, float* Vlast);

/* World 0's qpos to HOST out [36].  (src/g1_env.cu:457-460) */
void g1_env_qpos(void* h, float* out);

/* All worlds' qpos to HOST out [N*36].  (src/g1_env.cu:464-467) */
void g1_env_qpos_all(void* h, float* out);

/* K control steps of zero-action physics (reward/termination/auto-reset included). Blocks; K <= 0
 * does nothing.  (src/g1_env.cu:385-389, k_phys_bench :343-359) */
void g1_env_bench_phys(void* h, int K);

/* Print registers, scratch, LDS and occupancy of the kernels.  (src/g1_env.cu:365-382) */
void g1_occupancy_report(void);

int g1_env_obs_dim(void); /* 100  (src/g1_env.cu:391) */
int g1_env_act_dim(void); /* 29   (src/g1_env.cu:392) */

void g1_env_destroy(void* h); /* (src/g1_env.cu:469-474) */

/* ---- additive exports: no counterpart in the reference ABI ---------------------------------
 * For parity tests, benchmarks and the scaled policy configuration. Existing symbols above are
 * unchanged by them. */

/* g1_rollout with pre-generated noise: act_noise DEVICE [H*N*29] N(0,1) action noise and
 * reset_noise DEVICE [H*N*29] U(-1,1) auto-reset noise (either may be NULL: library RNG). */
void g1_rollout_ex(void* h, int H, const float* W, const float* mean, const float* var, float* O, float* A,
                   float* LP, float* V, float* R, float* D, float* Vlast, const float* act_noise,
                   const float* reset_noise);

/* g1_rollout_ex that allocates nothing: no counterpart in the reference. For callers that cannot
 * allocate device memory during the call (tight serving loops, harnesses that forbid allocation).
 * g1_rollout packs the policy weights into a buffer it grows with hipMalloc; this entry point packs
 * them into a fixed device array of the library (640 Ki floats, 2.5 MiB per GPU, held until the
 * process ends), which fits every shape g1_env_set_policy accepts. Returns 0, or -1 (message on
 * stderr) when no env was created on the current device or the packed policy exceeds the array.
 * All calls on one GPU share the array; the library orders its launches on the null stream, so
 * successive calls do not overlap, and callers must not run two of them concurrently on other
 * streams. Asynchronous, like g1_rollout; no profiling events are recorded. Not for HIP graph
 * capture: its launches and its closing error-word copy go to the null stream, and it reads the
 * previous rollout's error word from host memory on entry. */
int g1_rollout_noalloc(void* h, int H, const float* W, const float* mean, const float* var, float* O, float* A,
                       float* LP, float* V, float* R, float* D, float* Vlast, const float* act_noise,
                       const float* reset_noise);

/* Bytes of device memory the env holds: its state, work-queue and staging buffers from
 * g1_env_create, plus the packed-policy buffers that g1_rollout and g1_rollout_ex grow on demand
 * (g1_rollout_noalloc never does). Not the library's file-scope device arrays. */
long g1_env_device_bytes(void* h);

/* HOST state get/set: qp [N*36], qv [N*35], pa [N*29] previous action, steps [N]. Blocks. */
void g1_env_set_state(void* h, const float* qp, const float* qv, const float* pa, const int* steps);
void g1_env_get_state(void* h, float* qp, float* qv, float* pa, int* steps);

/* Policy shape used by g1_rollout: nlayers hidden layers of widths hidden[] (<= 512, 1..3 layers),
 * activation 0 = tanh (the reference's AC), 1 = ELU; heads mu (29) and value (1); packing extends
 * the reference order. Returns 0, or -1 (message on stderr) for an unsupported shape. */
int g1_env_set_policy(void* h, int nlayers, const int* hidden, int activation);
long g1_env_policy_params(void* h);

/* Friction coefficient of the foot contacts (model value 0.6) and PGS sweep count. */
void g1_env_set_contact(void* h, float mu, int pgs_iters);

/* Copy the per-substep contact-count histogram (ncon 0..8) to HOST out9 (may be NULL), clear it,
 * and enable (1) or disable (0) further accumulation. Blocks. */
void g1_env_ncon_hist(void* h, int enable, unsigned long long* out9);

/* Per-launch timing of the rollout's kernels with HIP events on the null stream. enable != 0
 * clears the record and starts recording; g1_env_profile_read syncs and writes HOST out4 =
 * {physics ms total, physics launches, policy ms total, policy launches}. */
void g1_env_profile(void* h, int enable);
void g1_env_profile_read(void* h, double* out4);

/* Wait for the device and return the physics work queue's error word: 0 = no error, 1 = a
 * dependency wait between work items exceeded its bound, 2 = a block ran off the XCD its queue was
 * placed on. Results of the launches since the error are undefined. Does not exit. */
int g1_env_check(void* h);

/* State hand-over between the physics work items: fences = 0 hands a world pair's state over in
 * the L2 of its queue's XCD (the default; needs the round-robin block placement verified at
 * creation), fences = 1 uses agent-scope release/acquire fences (correct on any placement,
 * slower). Returns 0, or -1 when the mode is unavailable. */
int g1_env_set_handover(void* h, int fences);

/* Rollout form: on = 1 (the default) runs g1_rollout as one persistent launch that interleaves the
 * policy of 16-world tiles with the physics work items; on = 0 launches the policy and the physics
 * once per control step. The one-launch form covers every shape g1_env_set_policy accepts (two
 * hidden layers of at most 256 units on a register-resident tile, other shapes on a tile that
 * stages its activations in library-allocated device memory); g1_rollout_noalloc runs the latter
 * shapes in the per-step form. Returns 0, 1 when on = 1 but the current policy shape takes the
 * per-step form, or -1 for an invalid argument. */
int g1_env_set_fused(void* h, int on);

/* Parity probes running the same device code as the rollout on caller states (all DEVICE,
 * asynchronous): n worlds, qpos [n*36], qvel [n*35], qacc out [n*35], ncon out [n].
 * g1_probe_qacc: tau [n*35] on the hinge dofs; damped folds dt*kd into the factor (the env's
 * implicit PD); contact toggles the foot contacts. g1_probe_substep: nsub env substeps from PD
 * targets [n*29] (damped, contact, velocity guard, integration), qpos/qvel updated in place. */
void g1_probe_qacc(int n, float* qpos, float* qvel, const float* tau, int damped, int contact, int pgs, float mu,
                   float* qacc, int* ncon);
void g1_probe_substep(int n, float* qpos, float* qvel, const float* target, int nsub, int pgs, float mu,
                      float* qacc, int* ncon);

/* Policy MLP on normalised observations obs_norm DEVICE [n*100]: mu_out [n*29], v_out [n].
 * Blocks. Returns 0, or -1 for an unsupported shape. */
int g1_probe_policy(int n, int nlayers, const int* hidden, int activation, const float* W, const float* obs_norm,
                    float* mu_out, float* v_out);

/* nsub semi-implicit Euler substeps of n worlds (DEVICE qpos [n][36], qvel [n][35], updated in
 * place) driven by a generalized force on the hinge dofs (DEVICE tau [n][35], base entries
 * ignored); contact on/off, damped (M + dt kd) or plain factor, the env's velocity guard (NaN -> 0,
 * clamp +-50) on/off, pgs sweeps, friction mu. qacc [n][35] and ncon [n] (DEVICE) receive the last
 * substep's values. Asynchronous
 * on the null stream. Additive (no reference symbol): the batched smooth-dynamics benchmark (no
 * contact, plain factor, tau held over substeps; reference standalone bench src/sim_aba.cu:19-58)
 * and the contact-solve benchmark on fixed contact states run on it. */
void g1_dynamics_bench(int n, float* qpos, float* qvel, const float* tau, int nsub, int contact, int damped, int guard,
                       int pgs, float mu, float* qacc, int* ncon);

/* The physics kernel's reciprocal and quotient helpers on n DEVICE operand pairs: rcp[i] = 1/b[i],
 * quot[i] = a[i]/b[i] (both correctly rounded for positive normal b). */
void g1_probe_divide(int n, const float* a, const float* b, float* rcp, float* quot);

/* The physics kernel's square root of the Cholesky pivots on n DEVICE arguments: out[i] =
 * sqrt(x[i]) correctly rounded for x[i] >= 2^-96, +0 and +inf. */
void g1_probe_sqrt(int n, const float* x, float* out);

/* The physics kernel's sine/cosine of the free joint's half rotation angle on n DEVICE arguments:
 * sn[i] = sin(x[i]), cs[i] = cos(x[i]) rounded to float. */
void g1_probe_sincos(int n, const float* x, float* sn, float* cs);

/* The physics kernel's sine/cosine of the hinge half-angles (forward kinematics) on n DEVICE
 * arguments: sn[i] = sin(x[i]), cs[i] = cos(x[i]) rounded to float. */
void g1_probe_sincos_hinge(int n, const float* x, float* sn, float* cs);

/* Philox4x32-10 of n DEVICE counters ctr [n*4] with key (k0, k1) into out [n*4]. */
void g1_probe_philox(int n, const unsigned* ctr, unsigned* out, unsigned k0, unsigned k1);

#ifdef __cplusplus
}
#endif
#endif /* G1ENV_H */
