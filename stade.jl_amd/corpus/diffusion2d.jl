# diffusion2d(loss, u, un, n)
#
# One explicit step of 2-D periodic diffusion on an n x n grid followed by the
# squared-norm loss of the new state:
#   un = u + 0.1 * (u[i-1,j] + u[i+1,j] + u[i,j-1] + u[i,j+1] - 4 u[i,j])
#   loss += sum(un .^ 2)
#
# The (i, j) nest is rectangular and independent, so it is one flattened loop
# (rule 2); i is the fastest coordinate (column-major).  Periodic neighbours
# come from mod.
#
# loss: length-1 output array, accumulated in place
# u: field of length n * n, column-major (i fastest)
# un: new field of length n * n, overwritten
# n: grid points per side
function diffusion2d(loss, u, un, n)
    # periodic 5-point update, one cell per iteration
    for idx = 1:n * n
        i = mod(idx - 1, n) + 1
        j = div(idx - 1, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        un[idx] = u[idx] + 0.1 * (u[(j - 1) * n + im] + u[(j - 1) * n + ip] + u[(jm - 1) * n + i] + u[(jp - 1) * n + i] - 4.0 * u[idx])
    end
    # squared norm of the new state
    for k = 1:n * n
        loss[1] = loss[1] + un[k] ^ 2
    end
    return nothing
end
