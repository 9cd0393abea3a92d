//! Backend selection with the HIP arm: the replacement for
//! src/runtime.rs:143-200 in a DiskMule build with the cargo feature `hip`.
//!
//! The GPU variant keeps its name, `Metal { residency }`, so every match in
//! `architecture::load` (src/architecture.rs:155-176) and the graphs compile
//! unchanged: under the feature the graphs' `MetalContext` is `crate::hip`'s.
//! `DISKMULE_BACKEND` takes `hip` beside `auto`, `metal` and `cpu`:
//!   - `hip` selects the GPU backend when the crate was built with `hip`, and
//!     is an InvalidConfiguration otherwise;
//!   - `auto` selects it on macOS (Metal) and in a `hip` build; elsewhere the
//!     CPU, as before;
//!   - `metal` keeps requiring macOS.
//! The residency (mapped experts, or N streamed slots per layer) comes from
//! the reference's own `expert_residency_from_environment`.
//!
//! Not compiled in the repository that holds it (no Rust toolchain in its
//! build image).

#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum BackendSelection {
    Cpu,
    #[cfg(any(target_os = "macos", feature = "hip"))]
    Metal { residency: ExpertResidency },
}

impl BackendSelection {
    pub fn from_environment() -> Result<Self, RuntimeError> {
        let requested = env::var("DISKMULE_BACKEND").unwrap_or_else(|_| "auto".to_owned());
        match requested.as_str() {
            "cpu" => Ok(Self::Cpu),
            "auto" => {
                #[cfg(any(target_os = "macos", feature = "hip"))]
                {
                    Ok(Self::Metal {
                        residency: expert_residency_from_environment()?,
                    })
                }
                #[cfg(not(any(target_os = "macos", feature = "hip")))]
                {
                    Ok(Self::Cpu)
                }
            }
            "hip" => {
                #[cfg(feature = "hip")]
                {
                    Ok(Self::Metal {
                        residency: expert_residency_from_environment()?,
                    })
                }
                #[cfg(not(feature = "hip"))]
                {
                    Err(RuntimeError::InvalidConfiguration(
                        "DISKMULE_BACKEND=hip requires a build with the hip feature".to_owned(),
                    ))
                }
            }
            "metal" => {
                #[cfg(target_os = "macos")]
                {
                    Ok(Self::Metal {
                        residency: expert_residency_from_environment()?,
                    })
                }
                #[cfg(not(target_os = "macos"))]
                {
                    Err(RuntimeError::InvalidConfiguration(
                        "DISKMULE_BACKEND=metal requires macOS".to_owned(),
                    ))
                }
            }
            _ => Err(RuntimeError::InvalidConfiguration(
                "DISKMULE_BACKEND must be auto, metal, hip, or cpu".to_owned(),
            )),
        }
    }

    pub fn label(self) -> String {
        // "Metal" on macOS, "HIP" in a hip build on another system
        let device = if cfg!(target_os = "macos") { "Metal" } else { "HIP" };
        match self {
            Self::Cpu => "CPU".to_owned(),
            #[cfg(any(target_os = "macos", feature = "hip"))]
            Self::Metal {
                residency: ExpertResidency::Mapped,
            } => device.to_owned(),
            #[cfg(any(target_os = "macos", feature = "hip"))]
            Self::Metal {
                residency: ExpertResidency::Streamed { slots_per_layer },
            } => format!("{device} streamed ({slots_per_layer} expert slots/layer)"),
        }
    }
}
