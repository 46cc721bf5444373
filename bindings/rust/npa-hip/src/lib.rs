//! Safe wrapper over `npa-hip-sys` with the shapes of the reference's operator surface (the
//! `burn_automata_kernels` exports, crates/burn_automata_kernels/src/lib.rs:40-66): a host-slice
//! context for `build_hashgrid` (crates/burn_automata_kernels/src/hashgrid.rs:16-69),
//! `perceive_with_options` (reference/forward.rs:26-143), `euler_step` (reference/step.rs:4-55),
//! `decode_gaussians_3d` (gaussian.rs:53-100), `splat_particles_2d` (splat.rs:30-93) and
//! `NpaModel::step_cpu` (crates/burn_automata/src/model.rs:768-858), and a device-resident rollout
//! state for the GPU executor (`create_state*` / `step_state_many` / `read_state` /
//! `update_state_model`, crates/burn_automata/src/gpu/executor/). Status codes map onto the
//! reference's `KernelError` variants (crates/burn_automata_kernels/src/config.rs:101-137).
use std::ffi::CStr;
use std::fmt;
use std::ptr;

pub use npa_hip_sys as sys;

/// The library's status codes, named after the reference's error variants.
#[derive(Clone, Debug, PartialEq, Eq)]
pub enum NpaError {
    InvalidDim,
    InvalidEps,
    InvalidGridSize,
    ParticleModeRequiresPowerOfTwo,
    PositionShape,
    StateShape,
    OutputShape,
    InvalidArgument,
    InvalidModel,
    Io,
    Json,
    InvalidFormat,
    Device,
    OutOfMemory,
    CoordOverflow,
    Other(i32),
}

/// A failed call: the status and the context's last error message.
#[derive(Clone, Debug)]
pub struct Error {
    pub kind: NpaError,
    pub message: String,
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "{:?}: {}", self.kind, self.message)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

fn kind_of(status: sys::npa_status) -> NpaError {
    match status {
        sys::NPA_ERR_INVALID_DIM => NpaError::InvalidDim,
        sys::NPA_ERR_INVALID_EPS => NpaError::InvalidEps,
        sys::NPA_ERR_INVALID_GRID_SIZE => NpaError::InvalidGridSize,
        sys::NPA_ERR_PARTICLE_MODE_POW2 => NpaError::ParticleModeRequiresPowerOfTwo,
        sys::NPA_ERR_POSITION_SHAPE => NpaError::PositionShape,
        sys::NPA_ERR_STATE_SHAPE => NpaError::StateShape,
        sys::NPA_ERR_OUTPUT_SHAPE => NpaError::OutputShape,
        sys::NPA_ERR_INVALID_ARGUMENT => NpaError::InvalidArgument,
        sys::NPA_ERR_INVALID_MODEL => NpaError::InvalidModel,
        sys::NPA_ERR_IO => NpaError::Io,
        sys::NPA_ERR_JSON => NpaError::Json,
        sys::NPA_ERR_INVALID_FORMAT => NpaError::InvalidFormat,
        sys::NPA_ERR_DEVICE => NpaError::Device,
        sys::NPA_ERR_OUT_OF_MEMORY => NpaError::OutOfMemory,
        sys::NPA_ERR_COORD_OVERFLOW => NpaError::CoordOverflow,
        other => NpaError::Other(other),
    }
}

/// Hashgrid snapshot with the reference's fields (`HashGridSnapshot`, hashgrid.rs:3-14).
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct HashGridSnapshot {
    pub batch_size: usize,
    pub particle_count: usize,
    pub cell_count: usize,
    pub bin_offsets: Vec<usize>,
    pub permutation: Vec<usize>,
    pub inverse_permutation: Vec<usize>,
}

/// `PerceptionOutput` (reference/types.rs:33-41): features [B*N][F], density [B*N], blurred state
/// [B*N][S], state gradient [B*N][S*d] (empty without the state gradient), density gradient [B*N][d]
/// (empty without the density gradient).
#[derive(Clone, Debug)]
pub struct PerceptionOutput {
    pub features: Vec<f32>,
    pub density: Vec<f32>,
    pub blurred_state: Vec<f32>,
    pub state_gradient: Vec<f32>,
    pub density_gradient: Vec<f32>,
    pub feature_dims: usize,
}

/// `Gaussian3d` (gaussian.rs:5-11): one decoded Gaussian with (sh_degree + 1)^2 coefficient triples
/// in oriented mode and one otherwise.
#[derive(Clone, Debug, PartialEq)]
pub struct Gaussian3d {
    pub position_visibility: [f32; 4],
    pub spherical_harmonic: Vec<[f32; 3]>,
    pub rotation: [f32; 4],
    pub scale_opacity: [f32; 4],
}

/// One step's outputs (`StepOutput`): next positions [B*N][4], next states [B*N][S], density [B*N].
#[derive(Clone, Debug)]
pub struct StepOutput {
    pub next_positions: Vec<[f32; 4]>,
    pub next_states: Vec<f32>,
    pub density: Vec<f32>,
}

/// Model weights in the reference's row-major layout: w1 [H][F], b1 [H], w2 [O][H], b2 [O].
pub struct Weights<'a> {
    pub w1: &'a [f32],
    pub b1: &'a [f32],
    pub w2: &'a [f32],
    pub b2: &'a [f32],
}

impl Weights<'_> {
    fn raw(&self) -> sys::npa_weights {
        sys::npa_weights { w1: self.w1.as_ptr(), b1: self.b1.as_ptr(), w2: self.w2.as_ptr(), b2: self.b2.as_ptr() }
    }
}

/// A library context on one GPU in host-I/O mode: every call takes host slices, copies them to the
/// device, runs, copies the results back and synchronises.
pub struct Context {
    raw: *mut sys::npa_context,
}

impl Context {
    /// Context on `device` (HIP ordinal) with the library's own stream, in host-I/O mode.
    pub fn new(device: i32) -> Result<Self> {
        let mut raw = ptr::null_mut();
        let st = unsafe { sys::npa_context_create(device, ptr::null_mut(), &mut raw) };
        if st != sys::NPA_OK {
            return Err(Error { kind: kind_of(st), message: "npa_context_create failed".into() });
        }
        let ctx = Context { raw };
        ctx.check(unsafe { sys::npa_context_set_host_io(raw, 1) })?;
        Ok(ctx)
    }

    pub fn as_raw(&self) -> *mut sys::npa_context {
        self.raw
    }

    fn check(&self, status: sys::npa_status) -> Result<()> {
        if status == sys::NPA_OK {
            return Ok(());
        }
        let msg = unsafe { sys::npa_last_error(self.raw) };
        let message = if msg.is_null() { String::new() } else { unsafe { CStr::from_ptr(msg) }.to_string_lossy().into_owned() };
        Err(Error { kind: kind_of(status), message })
    }

    /// `build_hashgrid` (hashgrid.rs:16-69).
    pub fn build_hashgrid(&self, positions: &[[f32; 4]], batch_size: usize, particle_count: usize,
                          cfg: &sys::npa_grid_cfg) -> Result<HashGridSnapshot> {
        let cells: usize = cfg.grid_size[..cfg.dim as usize].iter().map(|&v| v as usize).product();
        let total = batch_size * particle_count;
        let mut offsets = vec![0u32; batch_size * cells + 1];
        let mut perm = vec![0u32; total];
        let mut inv = vec![0u32; total];
        self.check(unsafe {
            sys::npa_build_hashgrid(self.raw, positions.as_ptr() as *const f32, batch_size as u32,
                                    particle_count as u32, cfg, offsets.as_mut_ptr(), offsets.len(),
                                    perm.as_mut_ptr(), inv.as_mut_ptr(), total)
        })?;
        let widen = |v: Vec<u32>| v.into_iter().map(|x| x as usize).collect::<Vec<_>>();
        Ok(HashGridSnapshot { batch_size, particle_count, cell_count: cells, bin_offsets: widen(offsets),
                              permutation: widen(perm), inverse_permutation: widen(inv) })
    }

    /// `perceive_with_options` (reference/forward.rs:26-143): density, blurred state, moment-corrected
    /// and normalised gradients and the feature rows of every particle.
    #[allow(clippy::too_many_arguments)]
    pub fn perceive_with_options(&self, positions: &[[f32; 4]], states: &[f32], batch_size: usize,
                                 particle_count: usize, state_dims: usize, cfg: &sys::npa_grid_cfg,
                                 options: &sys::npa_perception_opts) -> Result<PerceptionOutput> {
        let total = batch_size * particle_count;
        let d = cfg.dim as usize;
        let feature_dims = state_dims * 2 + if options.state_grad != 0 { state_dims * d } else { 0 }
            + if options.density_grad != 0 { d } else { 0 } + if options.position_features != 0 { d } else { 0 };
        let mut out = PerceptionOutput {
            features: vec![0.0; total * feature_dims],
            density: vec![0.0; total],
            blurred_state: vec![0.0; total * state_dims],
            state_gradient: if options.state_grad != 0 { vec![0.0; total * state_dims * d] } else { Vec::new() },
            density_gradient: if options.density_grad != 0 { vec![0.0; total * d] } else { Vec::new() },
            feature_dims,
        };
        let mut f = 0u32;
        let sg = if out.state_gradient.is_empty() { ptr::null_mut() } else { out.state_gradient.as_mut_ptr() };
        let dg = if out.density_gradient.is_empty() { ptr::null_mut() } else { out.density_gradient.as_mut_ptr() };
        self.check(unsafe {
            sys::npa_perceive(self.raw, positions.as_ptr() as *const f32, states.as_ptr(), batch_size as u32,
                              particle_count as u32, state_dims as u32, cfg, options, out.features.as_mut_ptr(),
                              out.features.len(), out.density.as_mut_ptr(), out.blurred_state.as_mut_ptr(), sg, dg,
                              &mut f)
        })?;
        out.feature_dims = f as usize;
        Ok(out)
    }

    /// `euler_step` (reference/step.rs:4-55): positions += dt dx m over the spatial memory axes
    /// (wrapped on periodic grids), states += dt ds m (3D opacity logits clamped); returns the new
    /// positions and states.
    #[allow(clippy::too_many_arguments)]
    pub fn euler_step(&self, positions: &[[f32; 4]], states: &[f32], dx: &[[f32; 4]], ds: &[f32],
                      batch_size: usize, particle_count: usize, state_dims: usize, cfg: &sys::npa_grid_cfg,
                      dt: f32, update_mask: Option<&[f32]>) -> Result<(Vec<[f32; 4]>, Vec<f32>)> {
        let total = batch_size * particle_count;
        let mut next_positions = vec![[0.0f32; 4]; total];
        let mut next_states = vec![0.0f32; total * state_dims];
        self.check(unsafe {
            sys::npa_euler_step(self.raw, positions.as_ptr() as *const f32, states.as_ptr(),
                                dx.as_ptr() as *const f32, ds.as_ptr(), batch_size as u32, particle_count as u32,
                                state_dims as u32, cfg, dt, update_mask.map_or(ptr::null(), |m| m.as_ptr()),
                                next_positions.as_mut_ptr() as *mut f32, next_states.as_mut_ptr())
        })?;
        Ok((next_positions, next_states))
    }

    /// `decode_gaussians_3d` (gaussian.rs:53-100). The reference asserts its layout checks; here a
    /// state width too small for the mode is an `InvalidArgument` error.
    pub fn decode_gaussians_3d(&self, positions: &[[f32; 4]], states: &[f32], state_dims: usize,
                               cfg: &sys::npa_gaussian_decode_cfg) -> Result<Vec<Gaussian3d>> {
        let n = positions.len();
        let k = if cfg.mode == sys::NPA_DECODE_SH0_ORIENTED {
            ((cfg.sh_degree + 1) * (cfg.sh_degree + 1)) as usize
        } else {
            1
        };
        let mut pv = vec![[0.0f32; 4]; n];
        let mut sh = vec![[0.0f32; 3]; n * k];
        let mut rot = vec![[0.0f32; 4]; n];
        let mut so = vec![[0.0f32; 4]; n];
        self.check(unsafe {
            sys::npa_decode_gaussians_3d(self.raw, positions.as_ptr() as *const f32, states.as_ptr(), n as u32,
                                         state_dims as u32, cfg, pv.as_mut_ptr() as *mut f32,
                                         sh.as_mut_ptr() as *mut f32, rot.as_mut_ptr() as *mut f32,
                                         so.as_mut_ptr() as *mut f32)
        })?;
        Ok((0..n)
            .map(|i| Gaussian3d { position_visibility: pv[i], spherical_harmonic: sh[i * k..(i + 1) * k].to_vec(),
                                  rotation: rot[i], scale_opacity: so[i] })
            .collect())
    }

    /// `splat_particles_2d` (splat.rs:30-93): the additive RGBA image [size * size][4].
    pub fn splat_particles_2d(&self, positions: &[[f32; 4]], colors: &[[f32; 3]], cfg: &sys::npa_splat2d_cfg)
                              -> Result<Vec<[f32; 4]>> {
        if positions.len() != colors.len() {
            return Err(Error { kind: NpaError::InvalidArgument,
                               message: format!("{} positions but {} colors", positions.len(), colors.len()) });
        }
        let size = cfg.image_size as usize;
        let mut image = vec![[0.0f32; 4]; size * size];
        self.check(unsafe {
            sys::npa_splat_2d(self.raw, positions.as_ptr() as *const f32, colors.as_ptr() as *const f32,
                              positions.len() as u32, cfg, image.as_mut_ptr() as *mut f32)
        })?;
        Ok(image)
    }

    /// `NpaModel::step_cpu` (model.rs:768-858): hashgrid, perception, update MLP, masked Euler step.
    #[allow(clippy::too_many_arguments)]
    pub fn step(&self, model: &sys::npa_model_cfg, weights: &Weights<'_>, positions: &[[f32; 4]], states: &[f32],
                batch_size: usize, particle_count: usize, grid: &sys::npa_grid_cfg, dt: f32,
                update_mask: Option<&[f32]>) -> Result<StepOutput> {
        let total = batch_size * particle_count;
        let mut out = StepOutput { next_positions: vec![[0.0; 4]; total],
                                   next_states: vec![0.0; total * model.state_dims as usize],
                                   density: vec![0.0; total] };
        let w = weights.raw();
        self.check(unsafe {
            sys::npa_step(self.raw, positions.as_ptr() as *const f32, states.as_ptr(), batch_size as u32,
                          particle_count as u32, grid, model, &w, dt,
                          update_mask.map_or(ptr::null(), |m| m.as_ptr()),
                          out.next_positions.as_mut_ptr() as *mut f32, out.next_states.as_mut_ptr(),
                          out.density.as_mut_ptr())
        })?;
        Ok(out)
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        unsafe { sys::npa_context_destroy(self.raw) }
    }
}

/// A device-resident rollout state (ping-pong positions and states, the device hash update mask),
/// the twin of `WgpuAutomataState`. It holds device memory until dropped.
pub struct State<'c> {
    raw: *mut sys::npa_state,
    ctx: &'c Context,
}

impl<'c> State<'c> {
    /// `create_state_with_update_prob`: the model, grid and initial particles (host slices).
    #[allow(clippy::too_many_arguments)]
    pub fn new(ctx: &'c Context, model: &sys::npa_model_cfg, weights: &Weights<'_>, grid: &sys::npa_grid_cfg,
               positions: &[[f32; 4]], states: &[f32], batch_size: usize, particle_count: usize, dt: f32,
               update_prob: f32, seed: u64) -> Result<Self> {
        let mut raw = ptr::null_mut();
        let w = weights.raw();
        ctx.check(unsafe {
            sys::npa_state_create(ctx.raw, model, &w, grid, positions.as_ptr() as *const f32, states.as_ptr(),
                                  batch_size as u32, particle_count as u32, dt, update_prob, seed, &mut raw)
        })?;
        Ok(State { raw, ctx })
    }

    /// `step_state_many`: `steps` rollout steps on the device, no host synchronisation.
    pub fn step(&mut self, steps: u32) -> Result<()> {
        self.ctx.check(unsafe { sys::npa_state_step(self.raw, steps) })
    }

    /// `read_state`: current positions, states and densities into host slices.
    pub fn read(&self, positions: &mut [[f32; 4]], states: &mut [f32], density: Option<&mut [f32]>) -> Result<()> {
        self.ctx.check(unsafe {
            sys::npa_state_read(self.raw, positions.as_mut_ptr() as *mut f32, states.as_mut_ptr(),
                                density.map_or(ptr::null_mut(), |d| d.as_mut_ptr()))
        })
    }

    /// `update_state_model`: new weights for the following steps.
    pub fn update_model(&mut self, weights: &Weights<'_>) -> Result<()> {
        let w = weights.raw();
        self.ctx.check(unsafe { sys::npa_state_update_model(self.raw, &w) })
    }

    pub fn step_index(&self) -> Result<u64> {
        let mut k = 0u64;
        self.ctx.check(unsafe { sys::npa_state_step_index(self.raw, &mut k) })?;
        Ok(k)
    }

    pub fn as_raw(&self) -> *mut sys::npa_state {
        self.raw
    }
}

impl Drop for State<'_> {
    fn drop(&mut self) {
        unsafe { sys::npa_state_destroy(self.raw) }
    }
}
