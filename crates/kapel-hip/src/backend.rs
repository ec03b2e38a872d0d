//! The backend proper (feature `hip`): device memory, transfers, the two
//! products on the device and the host for the rest.

use std::any::Any;
use std::ffi::{CStr, c_void};
use std::sync::{Arc, Mutex, Weak};

use kapel_core::{DType, Device, Error, Layout, Result, Storage, Tensor};
use kapel_cpu::Cpu;
use kapel_ops::{
    AdamWStep, Affine, ArgMax, Attention, Binary, Cast, Concat, Contiguous, CrossEntropy,
    ExpertMatmul, GatherColumns, GatherRows, Glu, HeadLayout, LayerNorm, LogSoftmax, Matmul, Max,
    Mean, Moments8, Operation, PagedAttention, QuantizedMatmul, Record, Recording, Recurrent,
    RmsNorm, Rope, Run, ScatterAddRows, Softmax, Sum, TopK, Transfer, Unary, Update, Write,
};

use crate::abi::{self, KhWeight};
use crate::hip;
use crate::{float_code, format_code};

/// Bytes of device memory of one allocation, freed when the last tensor that
/// holds it is dropped.
#[derive(Debug)]
pub struct HipStorage {
    ptr: *mut c_void,
    len: usize,
    ordinal: u32,
}

// The pointer is a device address: no host data is shared through it.
unsafe impl Send for HipStorage {}
unsafe impl Sync for HipStorage {}

impl HipStorage {
    fn new(ordinal: u32, len: usize, zeroed: bool) -> Result<Self> {
        let op = "HipStorage::new";
        let mut ptr = std::ptr::null_mut();
        // SAFETY: plain runtime calls on this process's device `ordinal`.
        unsafe {
            check(op, hip::hipSetDevice(ordinal as i32))?;
            if len > 0 {
                check(op, hip::hipMalloc(&mut ptr, len))?;
                if zeroed {
                    check(op, hip::hipMemset(ptr, 0, len))?;
                }
            }
        }
        Ok(Self { ptr, len, ordinal })
    }

    /// The device address of byte `offset`.
    pub fn ptr(&self, offset: usize) -> *mut c_void {
        self.ptr.wrapping_byte_add(offset)
    }
}

impl Drop for HipStorage {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            // SAFETY: the pointer came from hipMalloc on this device.
            unsafe {
                hip::hipSetDevice(self.ordinal as i32);
                hip::hipFree(self.ptr);
            }
        }
    }
}

impl Storage for HipStorage {
    fn device(&self) -> Device {
        Device::Hip(self.ordinal)
    }

    fn len(&self) -> usize {
        self.len
    }

    fn as_any(&self) -> &dyn Any {
        self
    }

    fn as_any_mut(&mut self) -> Option<&mut dyn Any> {
        Some(self)
    }
}

fn check(op: &'static str, status: hip::HipError) -> Result<()> {
    if status == hip::HIP_SUCCESS {
        return Ok(());
    }
    // SAFETY: the runtime returns a static NUL-terminated string.
    let text = unsafe { CStr::from_ptr(hip::hipGetErrorString(status)) };
    Err(Error::Device {
        op,
        message: text.to_string_lossy().into_owned(),
    })
}

/// A library status as a Kapel error (the mapping of `include/kapel_hip.h`).
fn status(op: &'static str, code: i32) -> Result<()> {
    if code == abi::KH_OK {
        return Ok(());
    }
    // SAFETY: the library returns a static NUL-terminated string.
    let text = unsafe { CStr::from_ptr(abi::kh_error_string(code)) };
    let message = text.to_string_lossy().into_owned();
    Err(match code {
        abi::KH_ERR_OVERFLOW => Error::Overflow { op },
        abi::KH_ERR_SHAPE | abi::KH_ERR_NULL | abi::KH_ERR_DTYPE | abi::KH_ERR_MISALIGNED
        | abi::KH_ERR_ARITY => Error::InvalidArgument { op, message },
        _ => Error::Device { op, message },
    })
}

struct Inner {
    ordinal: u32,
    stream: *mut c_void,
    /// Zero-filled at allocation; every call leaves it as the next accepts.
    workspace: Mutex<Option<Arc<HipStorage>>>,
    cpu: Cpu,
    byte_activations: bool,
}

// The stream is used by one call at a time (the workspace's lock).
unsafe impl Send for Inner {}
unsafe impl Sync for Inner {}

impl Drop for Inner {
    fn drop(&mut self) {
        // SAFETY: the stream was created by this backend.
        unsafe {
            hip::hipSetDevice(self.ordinal as i32);
            hip::hipStreamSynchronize(self.stream);
            hip::hipStreamDestroy(self.stream);
        }
    }
}

static BACKENDS: Mutex<Vec<(u32, Weak<Inner>)>> = Mutex::new(Vec::new());

/// The HIP backend of one device. Cloning shares its stream and workspace.
#[derive(Clone)]
pub struct Hip {
    inner: Arc<Inner>,
}

impl Hip {
    /// The backend of device `ordinal`: the one alive in the process, or a
    /// new one with its own stream.
    ///
    /// # Errors
    ///
    /// If there is no such device.
    pub fn new(ordinal: u32) -> Result<Self> {
        let op = "Hip::new";
        let mut backends = BACKENDS.lock().expect("not poisoned");
        backends.retain(|(_, b)| b.strong_count() > 0);
        if let Some(inner) = backends.iter().filter(|(o, _)| *o == ordinal).find_map(|(_, b)| b.upgrade()) {
            return Ok(Self { inner });
        }
        let mut stream = std::ptr::null_mut();
        // SAFETY: plain runtime calls.
        unsafe {
            let mut count = 0;
            check(op, hip::hipGetDeviceCount(&mut count))?;
            if ordinal as i32 >= count {
                return Err(Error::Device {
                    op,
                    message: format!("no device {ordinal} ({count} found)"),
                });
            }
            check(op, hip::hipSetDevice(ordinal as i32))?;
            check(op, hip::hipStreamCreate(&mut stream))?;
        }
        let inner = Arc::new(Inner {
            ordinal,
            stream,
            workspace: Mutex::new(None),
            cpu: Cpu::new(),
            byte_activations: false,
        });
        backends.push((ordinal, Arc::downgrade(&inner)));
        Ok(Self { inner })
    }

    /// Activations quantized to bytes in the products by quantized weights,
    /// for up to 16 rows, as `Cpu::with_byte_activations`
    /// (crates/kapel-cpu/src/backend.rs:71-81, matmul.rs:292-306).
    pub fn with_byte_activations(self, on: bool) -> Self {
        let inner = &self.inner;
        Self {
            inner: Arc::new(Inner {
                ordinal: inner.ordinal,
                stream: {
                    let mut stream = std::ptr::null_mut();
                    // SAFETY: a new stream for the new backend value.
                    unsafe {
                        hip::hipSetDevice(inner.ordinal as i32);
                        hip::hipStreamCreate(&mut stream);
                    }
                    stream
                },
                workspace: Mutex::new(None),
                cpu: Cpu::new().with_byte_activations(on),
                byte_activations: on,
            }),
        }
    }

    /// The device of this backend.
    pub fn device(&self) -> Device {
        Device::Hip(self.inner.ordinal)
    }

    /// Waits for the work queued on the backend's stream.
    ///
    /// # Errors
    ///
    /// Those of the device.
    pub fn synchronize(&self) -> Result<()> {
        // SAFETY: the backend's own stream.
        unsafe { check("Hip::synchronize", hip::hipStreamSynchronize(self.inner.stream)) }
    }

    fn storage_of<'a>(&self, op: &'static str, t: &'a Tensor) -> Result<&'a HipStorage> {
        if t.device() != self.device() {
            return Err(Error::WrongDevice {
                op,
                expected: self.device(),
                got: t.device(),
            });
        }
        t.storage().as_any().downcast_ref::<HipStorage>().ok_or_else(|| Error::Device {
            op,
            message: "a tensor of this device without device storage".into(),
        })
    }

    /// The device address of a contiguous tensor's first element.
    fn address(&self, op: &'static str, t: &Tensor) -> Result<*mut c_void> {
        let storage = self.storage_of(op, t)?;
        Ok(storage.ptr(t.dtype().storage_bytes(t.layout().offset())?))
    }

    fn empty(&self, dtype: DType, shape: &[usize], zeroed: bool) -> Result<Tensor> {
        let layout = Layout::contiguous(shape)?;
        let bytes = dtype.storage_bytes(layout.numel())?;
        let storage = HipStorage::new(self.inner.ordinal, bytes, zeroed)?;
        Tensor::from_storage(Arc::new(storage), layout, dtype)
    }

    /// The workspace, at least `bytes` (256-byte aligned by hipMalloc).
    fn workspace(&self, bytes: u64) -> Result<Arc<HipStorage>> {
        let mut slot = self.inner.workspace.lock().expect("not poisoned");
        if let Some(ws) = slot.as_ref()
            && ws.len as u64 >= bytes
        {
            return Ok(ws.clone());
        }
        // The old one is freed once the stream no longer uses it.
        self.synchronize()?;
        let ws = Arc::new(HipStorage::new(self.inner.ordinal, bytes.max(256) as usize, true)?);
        *slot = Some(ws.clone());
        Ok(ws)
    }

    fn weight(&self, op: &'static str, w: &Tensor) -> Result<Option<KhWeight>> {
        let Some((format, group)) = format_code(w.dtype()) else {
            return Ok(None);
        };
        Ok(Some(KhWeight {
            format,
            group,
            data: self.address(op, w)?,
            bytes: w.dtype().storage_bytes(w.numel())? as u64,
            n: w.shape()[0] as u64,
        }))
    }

    /// An operation on the host: inputs downloaded, `Cpu` run, outputs uploaded.
    fn host_forward<O: Operation>(&self, op: &O, inputs: &[&Tensor]) -> Result<Tensor>
    where
        Cpu: Run<O>,
    {
        let host: Vec<Tensor> = inputs.iter().map(|t| self.download(t)).collect::<Result<_>>()?;
        let refs: Vec<&Tensor> = host.iter().collect();
        let y = self.inner.cpu.forward(op, &refs)?;
        self.upload(&y)
    }

    fn host_backward<O: Operation>(
        &self,
        op: &O,
        inputs: &[&Tensor],
        grad: &Tensor,
    ) -> Result<Vec<Option<Tensor>>>
    where
        Cpu: Run<O>,
    {
        let host: Vec<Tensor> = inputs.iter().map(|t| self.download(t)).collect::<Result<_>>()?;
        let refs: Vec<&Tensor> = host.iter().collect();
        let g = self.download(grad)?;
        self.inner
            .cpu
            .backward(op, &refs, &g)?
            .into_iter()
            .map(|t| t.map(|t| self.upload(&t)).transpose())
            .collect()
    }

    /// Writes a host tensor's bytes over a device tensor's storage, in place.
    fn write_back(&self, op: &'static str, target: &mut Tensor, host: &Tensor) -> Result<()> {
        let host = host.contiguous()?;
        let bytes = host.storage().host_bytes().ok_or(Error::WrongDevice {
            op,
            expected: Device::Cpu,
            got: host.device(),
        })?;
        let start = host.dtype().storage_bytes(host.layout().offset())?;
        let size = host.dtype().storage_bytes(host.numel())?;
        let offset = target.dtype().storage_bytes(target.layout().offset())?;
        let storage = target
            .storage_mut()
            .and_then(|s| s.as_any_mut())
            .and_then(|s| s.downcast_mut::<HipStorage>())
            .ok_or_else(|| Error::InvalidArgument {
                op,
                message: "the target is shared or not on this device".into(),
            })?;
        // SAFETY: `size` bytes from the host buffer into the storage at the
        // target's offset, within it (same shape and type).
        unsafe {
            check(op, hip::hipStreamSynchronize(self.inner.stream))?;
            check(
                op,
                hip::hipMemcpy(storage.ptr(offset), bytes[start..].as_ptr().cast(), size, hip::HOST_TO_DEVICE),
            )
        }
    }

    /// A device tensor's values as a host tensor, updated on the host by
    /// `f`, then written back.
    fn in_place<R>(
        &self,
        op: &'static str,
        target: &mut Tensor,
        f: impl FnOnce(&mut Tensor) -> Result<R>,
    ) -> Result<R> {
        let mut host = self.download(target)?.contiguous()?;
        let r = f(&mut host)?;
        self.write_back(op, target, &host)?;
        Ok(r)
    }
}

impl Transfer for Hip {
    fn upload(&self, tensor: &Tensor) -> Result<Tensor> {
        let op = "Hip::upload";
        if tensor.device() == self.device() {
            return Ok(tensor.clone());
        }
        let host = if tensor.device() == Device::Cpu { tensor.contiguous()? } else {
            return Err(Error::WrongDevice { op, expected: Device::Cpu, got: tensor.device() });
        };
        let bytes = host.storage().host_bytes().ok_or(Error::WrongDevice {
            op,
            expected: Device::Cpu,
            got: host.device(),
        })?;
        let start = host.dtype().storage_bytes(host.layout().offset())?;
        let size = host.dtype().storage_bytes(host.numel())?;
        let out = self.empty(host.dtype(), host.shape(), false)?;
        let dst = self.address(op, &out)?;
        // SAFETY: `size` bytes into a fresh allocation of `size` bytes.
        unsafe { check(op, hip::hipMemcpy(dst, bytes[start..].as_ptr().cast(), size, hip::HOST_TO_DEVICE))? };
        Ok(out)
    }

    fn download(&self, tensor: &Tensor) -> Result<Tensor> {
        let op = "Hip::download";
        if tensor.device() == Device::Cpu {
            return Ok(tensor.clone());
        }
        let storage = self.storage_of(op, tensor)?;
        let mut bytes = vec![0u8; storage.len];
        self.synchronize()?;
        // SAFETY: the whole storage into a host buffer of its size.
        unsafe {
            check(op, hip::hipMemcpy(bytes.as_mut_ptr().cast(), storage.ptr(0), storage.len, hip::DEVICE_TO_HOST))?;
        }
        // The same layout over a host copy of the storage.
        let elements = storage.len / tensor.dtype().storage_bytes(1).unwrap_or(1).max(1);
        let flat = if tensor.dtype().is_quantized() {
            let per = tensor.dtype().block_len();
            Tensor::from_bytes(tensor.dtype(), &[storage.len / tensor.dtype().block_bytes() * per], &bytes)?
        } else {
            Tensor::from_bytes(tensor.dtype(), &[elements], &bytes)?
        };
        Tensor::from_storage(flat.storage().clone(), tensor.layout().clone(), tensor.dtype())
    }
}

impl Run<QuantizedMatmul> for Hip {
    /// On the device for the formats of libkapel_hip, with f32, bf16 or f16
    /// activations; on the host otherwise.
    fn forward(&self, op: &QuantizedMatmul, inputs: &[&Tensor]) -> Result<Tensor> {
        let name = QuantizedMatmul::NAME;
        let signature = op.infer(inputs)?;
        let x = inputs[0];
        let mut weights = Vec::with_capacity(inputs.len() - 1);
        for w in &inputs[1..] {
            match self.weight(name, w)? {
                Some(kw) => weights.push(kw),
                None => return self.host_forward(op, inputs),
            }
        }
        let (Some(x_kind), Some(out_kind)) = (float_code(x.dtype()), float_code(signature.dtype)) else {
            return self.host_forward(op, inputs);
        };
        let x = if x.is_contiguous() { x.clone() } else { self.host_forward(&Contiguous, &[x])? };
        let k = inputs[1].shape()[1] as u64;
        let rows: usize = x.shape()[..x.rank().saturating_sub(1)].iter().product();
        let out = self.empty(signature.dtype, &signature.shape, false)?;
        let flags = if self.inner.byte_activations { abi::KH_BYTE_ACTIVATIONS } else { 0 };
        // SAFETY: the weights, x and out are device buffers of the sizes the
        // signature gives; the workspace is at least what the library asks.
        unsafe {
            let need = abi::kh_qmatmul_workspace(weights.as_ptr(), weights.len() as u32, k, rows as u64, flags);
            let ws = self.workspace(need)?;
            status(
                name,
                abi::kh_qmatmul(
                    weights.as_ptr(),
                    weights.len() as u32,
                    k,
                    x_kind,
                    self.address(name, &x)?,
                    rows as u64,
                    out_kind,
                    self.address(name, &out)?,
                    flags,
                    ws.ptr(0),
                    ws.len as u64,
                    self.inner.stream,
                ),
            )?;
        }
        Ok(out)
    }

    /// Only x has a gradient (crates/kapel-ops/src/matmul.rs:152-156): on the
    /// host, as kapel-cuda computes it through dequantized weights.
    fn backward(&self, op: &QuantizedMatmul, inputs: &[&Tensor], grad: &Tensor) -> Result<Vec<Option<Tensor>>> {
        op.infer_backward(inputs, grad)?;
        self.host_backward(op, inputs, grad)
    }
}

impl Run<ExpertMatmul> for Hip {
    /// On the device for the formats of libkapel_hip; the indices are read
    /// and checked first, as every backend does (crates/kapel-ops/src/experts.rs:149-163).
    fn forward(&self, op: &ExpertMatmul, inputs: &[&Tensor]) -> Result<Tensor> {
        let name = ExpertMatmul::NAME;
        let signature = op.infer(inputs)?;
        let (x, w, idx) = (inputs[0], inputs[1], inputs[2]);
        let (Some(weight), Some(x_kind), Some(out_kind)) =
            (self.weight(name, w)?, float_code(x.dtype()), float_code(signature.dtype))
        else {
            return self.host_forward(op, inputs);
        };
        let host_idx = self.download(idx)?.contiguous()?;
        let values: Vec<usize> = match idx.dtype() {
            DType::U32 => host_idx.to_vec::<u32>()?.into_iter().map(|v| v as usize).collect(),
            _ => host_idx.to_vec::<i32>()?.into_iter().map(|v| if v < 0 { usize::MAX } else { v as usize }).collect(),
        };
        op.check(&values)?;
        let as_u32: Vec<u32> = values.iter().map(|&v| v as u32).collect();
        let idx_dev = self.upload(&Tensor::from_slice(&as_u32, idx.shape())?)?;
        let x = if x.is_contiguous() { x.clone() } else { self.host_forward(&Contiguous, &[x])? };
        let (tokens, topk) = (idx.shape()[0] as u64, idx.shape()[1] as u32);
        let per_route = u32::from(x.rank() == 3);
        let k = w.shape()[1] as u64;
        let experts = op.experts as u32;
        let out = self.empty(signature.dtype, &signature.shape, false)?;
        let flags = if self.inner.byte_activations { abi::KH_BYTE_ACTIVATIONS } else { 0 };
        // SAFETY: device buffers of the signature's sizes; indices checked.
        unsafe {
            let need = abi::kh_expert_matmul_workspace(&weight, experts, k, tokens, topk, per_route, x_kind, flags);
            let ws = self.workspace(need)?;
            status(
                name,
                abi::kh_expert_matmul(
                    &weight,
                    experts,
                    k,
                    x_kind,
                    self.address(name, &x)?,
                    tokens,
                    topk,
                    per_route,
                    self.address(name, &idx_dev)?.cast(),
                    out_kind,
                    self.address(name, &out)?,
                    flags,
                    ws.ptr(0),
                    ws.len as u64,
                    self.inner.stream,
                ),
            )?;
        }
        Ok(out)
    }

    fn backward(&self, op: &ExpertMatmul, inputs: &[&Tensor], grad: &Tensor) -> Result<Vec<Option<Tensor>>> {
        op.infer_backward(inputs, grad)?;
        self.host_backward(op, inputs, grad)
    }
}

/// The operations run on the host.
macro_rules! on_the_host {
    ($($op:ty),* $(,)?) => {$(
        impl Run<$op> for Hip {
            fn forward(&self, op: &$op, inputs: &[&Tensor]) -> Result<Tensor> {
                op.infer(inputs)?;
                self.host_forward(op, inputs)
            }

            fn backward(&self, op: &$op, inputs: &[&Tensor], grad: &Tensor) -> Result<Vec<Option<Tensor>>> {
                op.infer_backward(inputs, grad)?;
                self.host_backward(op, inputs, grad)
            }
        }
    )*};
}

on_the_host!(
    Unary, Glu, Binary, Affine, Cast, Contiguous, Concat, Matmul, Sum, Mean, Max, ArgMax, Softmax,
    LogSoftmax, CrossEntropy, LayerNorm, RmsNorm, Attention, PagedAttention, Rope, GatherRows,
    ScatterAddRows, TopK, GatherColumns,
);

impl Write for Hip {
    fn zeros(&self, shape: &[usize], dtype: DType) -> Result<Tensor> {
        self.empty(dtype, shape, true)
    }

    fn write_rows(&self, table: &mut Tensor, index: &Tensor, rows: &Tensor) -> Result<()> {
        let (index, rows) = (self.download(index)?, self.download(rows)?);
        self.in_place(kapel_ops::WRITE_ROWS, table, |t| self.inner.cpu.write_rows(t, &index, &rows))
    }

    fn copy_from_host(&self, target: &mut Tensor, values: &Tensor) -> Result<()> {
        kapel_ops::check_copy(target, values)?;
        self.write_back(kapel_ops::COPY_FROM_HOST, target, values)
    }
}

impl Record for Hip {
    /// Each operation is queued as it is called: nothing to record.
    fn records(&self) -> bool {
        false
    }

    fn record(&self, _pass: &mut dyn FnMut() -> Result<Tensor>) -> Result<Option<Recording>> {
        Ok(None)
    }
}

impl Recurrent for Hip {
    fn causal_conv(&self, state: &mut Tensor, x: &Tensor, weight: &Tensor, slots: &Tensor) -> Result<Tensor> {
        let (x, weight, slots) = (self.download(x)?, self.download(weight)?, self.download(slots)?);
        let y = self.in_place(kapel_ops::CAUSAL_CONV, state, |s| self.inner.cpu.causal_conv(s, &x, &weight, &slots))?;
        self.upload(&y)
    }

    fn delta_rule(
        &self,
        state: &mut Tensor,
        q: &Tensor,
        k: &Tensor,
        v: &Tensor,
        g: &Tensor,
        beta: &Tensor,
        slots: &Tensor,
        layout: HeadLayout,
    ) -> Result<Tensor> {
        let host: Vec<Tensor> = [q, k, v, g, beta, slots].iter().map(|t| self.download(t)).collect::<Result<_>>()?;
        let y = self.in_place(kapel_ops::DELTA_RULE, state, |s| {
            self.inner.cpu.delta_rule(s, &host[0], &host[1], &host[2], &host[3], &host[4], &host[5], layout)
        })?;
        self.upload(&y)
    }
}

impl Update for Hip {
    fn adamw(&self, param: &mut Tensor, m: &mut Tensor, v: &mut Tensor, grad: &Tensor, step: &AdamWStep) -> Result<()> {
        let op = kapel_ops::ADAMW;
        let g = self.download(grad)?;
        let (mut hp, mut hm, mut hv) = (
            self.download(param)?.contiguous()?,
            self.download(m)?.contiguous()?,
            self.download(v)?.contiguous()?,
        );
        self.inner.cpu.adamw(&mut hp, &mut hm, &mut hv, &g, step)?;
        self.write_back(op, param, &hp)?;
        self.write_back(op, m, &hm)?;
        self.write_back(op, v, &hv)
    }

    fn adamw8bit(
        &self,
        param: &mut Tensor,
        moments: &mut Moments8,
        grad: &Tensor,
        maps: &Tensor,
        step: &AdamWStep,
    ) -> Result<()> {
        let op = kapel_ops::ADAMW8;
        let (g, maps) = (self.download(grad)?, self.download(maps)?);
        let mut hp = self.download(param)?.contiguous()?;
        let mut hm = Moments8 {
            m: self.download(&moments.m)?.contiguous()?,
            v: self.download(&moments.v)?.contiguous()?,
            m_scale: self.download(&moments.m_scale)?.contiguous()?,
            v_scale: self.download(&moments.v_scale)?.contiguous()?,
        };
        self.inner.cpu.adamw8bit(&mut hp, &mut hm, &g, &maps, step)?;
        self.write_back(op, param, &hp)?;
        self.write_back(op, &mut moments.m, &hm.m)?;
        self.write_back(op, &mut moments.v, &hm.v)?;
        self.write_back(op, &mut moments.m_scale, &hm.m_scale)?;
        self.write_back(op, &mut moments.v_scale, &hm.v_scale)
    }
}

/// `Hip` runs the whole catalogue.
#[allow(dead_code)]
fn runs_the_catalogue() {
    fn is_backend<B: kapel_ops::Backend>() {}
    is_backend::<Hip>();
}
